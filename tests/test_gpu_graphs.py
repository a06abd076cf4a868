"""The nine kernel_fns captured in HIP graphs (torch.cuda.CUDAGraph on ROCm).

Every entry point takes torch's current stream, never synchronises and never allocates (outputs and
workspaces come from torch's allocator, which draws from the graph's private pool during capture),
and no kernel path issues hipMemsetAsync. So each op, and a chain of them, can be captured once and
replayed. Each graph is replayed several times, with unrelated eager work of the same ops on other
data and a device synchronisation between the replays, and every replay must equal the eager result
bit for bit (the kernels are deterministic)."""
import pytest
import torch

from autokernel_amd import kernels

pytestmark = pytest.mark.gpu
K = kernels.get


def _inputs(dev, seed):
    g = torch.Generator().manual_seed(seed)

    def rn(*shape, dt=torch.float16, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(dt).to(dev)

    pos = torch.arange(256, dtype=torch.float32)[:, None] * (10000.0 ** (-torch.arange(0, 128, 2) / 128.0))[None]
    return {
        "rmsnorm": {"x": rn(512, 1024), "weight": rn(1024, scale=0.02) + 1},
        "layernorm": {"x": rn(512, 1024), "weight": rn(1024), "bias": rn(1024)},
        "softmax": {"x": rn(512, 4096, scale=3.0)},
        "rotary_embedding": {"x": rn(1, 8, 256, 128), "cos": pos.cos().half().to(dev), "sin": pos.sin().half().to(dev)},
        "cross_entropy": {"logits": rn(512, 32000), "targets": torch.randint(0, 32000, (512,), generator=g).to(dev)},
        "reduce": {"x": rn(512, 4096)},
        "matmul": {"A": rn(512, 1024, dt=torch.bfloat16, scale=1 / 32), "B": rn(768, 1024, dt=torch.bfloat16).t()},
        # 16 output tiles over K = 8192: split-K (fp32 slices in a torch-allocated workspace, then a
        # fixed-order sum), two launches in the graph
        "matmul_splitk": {"A": rn(512, 8192, scale=1 / 90), "B": rn(8192, 512)},
        "fused_mlp": {"x": rn(256, 512, dt=torch.bfloat16), "w_gate": rn(1024, 512, dt=torch.bfloat16, scale=0.02),
                      "w_up": rn(1024, 512, dt=torch.bfloat16, scale=0.02),
                      "w_down": rn(512, 1024, dt=torch.bfloat16, scale=0.02)},
        "flash_attention": {"Q": rn(1, 8, 512, 128), "K": rn(1, 8, 512, 128), "V": rn(1, 8, 512, 128)},
    }


def _capture(fn):
    """Warm up on a side stream (torch's recommended order), then capture one call."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _replays(g, out, expected, eager_other, what, n=4):
    for r in range(n):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected), f"{what}: replay {r} differs from the eager result"
        eager_other()  # the same op eagerly on other data between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("op", ["rmsnorm", "layernorm", "softmax", "rotary_embedding", "cross_entropy", "reduce",
                                "matmul", "matmul_splitk", "fused_mlp", "flash_attention"])
def test_op_in_graph(gpu, op):
    ins = _inputs(gpu, 1)[op]
    other = _inputs(gpu, 2)[op]
    fn = K(op.split("_splitk")[0])
    if op == "matmul_splitk":  # the case must take the split-K path (a nonzero fp32 workspace)
        from autokernel_amd.kernels import _ops
        assert _ops.gemm_workspace_bytes(1, 512, 512, 8192, 8192, 512, 512, False) > 0
    expected = fn(**ins).clone()
    torch.cuda.synchronize()
    g, out = _capture(lambda: fn(**ins))
    print(f"graph {op}: captured, {tuple(out.shape)} {out.dtype}", flush=True)
    _replays(g, out, expected, lambda: fn(**other), op)


def test_chain_in_graph(gpu):
    """rmsnorm -> Q projection (nn.Linear layout) -> RoPE -> causal attention -> output projection,
    one graph."""
    gen = torch.Generator().manual_seed(3)
    T, D, H, HD = 256, 1024, 8, 128
    x = torch.randn(T, D, generator=gen).half().to(gpu)
    w = (torch.randn(D, generator=gen) * 0.02 + 1).half().to(gpu)
    wq, wk, wv, wo = ((torch.randn(D, D, generator=gen) / D ** 0.5).half().to(gpu) for _ in range(4))
    pos = torch.arange(T, dtype=torch.float32)[:, None] * (10000.0 ** (-torch.arange(0, HD, 2) / HD))[None]
    cos, sin = pos.cos().half().to(gpu), pos.sin().half().to(gpu)

    def chain():
        h = K("rmsnorm")(x, w)
        heads = lambda t: t.view(1, T, H, HD).transpose(1, 2)  # noqa: E731  [1, H, T, HD] strided view
        q = K("rotary_embedding")(heads(K("matmul")(h, wq.t())).contiguous(), cos, sin)
        k = K("rotary_embedding")(heads(K("matmul")(h, wk.t())).contiguous(), cos, sin)
        v = heads(K("matmul")(h, wv.t()))
        o = K("flash_attention")(q, k, v, causal=True)
        return K("matmul")(o.transpose(1, 2).reshape(T, D), wo.t())

    expected = chain().clone()
    torch.cuda.synchronize()
    g, out = _capture(chain)
    x_other = torch.randn(T, D, generator=gen).half().to(gpu)
    _replays(g, out, expected, lambda: K("rmsnorm")(x_other, w), "chain")

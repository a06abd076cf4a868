"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Cases follow the reference harness's stages (bench.py:641-966): every test size x dtype of the
op table, the edge sizes, the five adversarial transforms with its NaN / Inf rule and 10x
relaxed tolerance, and bitwise determinism over three runs; plus the BASELINE workloads, the
golden fixtures and the layouts the model plug-in relies on. Inputs are generated on the CPU
with a fixed seed and copied to the GPU, so the oracle sees the same bits.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from autokernel_amd import kernels, spec
from autokernel_amd.kernels import flash_attention as fa_mod
from autokernel_amd.kernels import reduce as reduce_mod
from oracle import reference_ops as R

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def to_dev(inputs, dev):
    return {k: v.to(dev) if isinstance(v, torch.Tensor) else v for k, v in inputs.items()}


def has_nan_inf(t):
    t = t.float()
    return bool(torch.isnan(t).any() or torch.isinf(t).any())


def assert_close(out, exp, atol, rtol, what=""):
    out_f, exp_f = out.detach().float().cpu(), exp.detach().float().cpu()
    assert out_f.shape == exp_f.shape, f"{what}: shape {tuple(out_f.shape)} vs {tuple(exp_f.shape)}"
    diff = (out_f - exp_f).abs()
    ok = torch.allclose(out_f, exp_f, atol=atol, rtol=rtol)
    assert ok, f"{what}: max_abs_err={diff.max().item():.3e} (atol={atol}, rtol={rtol})"


def sweep_cases():
    cases = []
    for op, cfg in spec.KERNEL_CONFIGS.items():
        for label, size in cfg["test_sizes"]:
            for dt in cfg["test_dtypes"]:
                cases.append(pytest.param(op, label, size, dt, id=f"{op}-{label}-{str(dt)[6:]}"))
        for label, size in cfg["edge_sizes"]:
            dt = cfg["test_dtypes"][0]
            cases.append(pytest.param(op, label, size, dt, id=f"{op}-{label}-{str(dt)[6:]}"))
    return cases


@pytest.mark.parametrize("op,label,size,dtype", sweep_cases())
def test_sweep(gpu, op, label, size, dtype):
    cfg = spec.KERNEL_CONFIGS[op]
    inputs = cfg["input_generator"](size, dtype, "cpu", seed=42)
    expected = R.REFERENCE[op](inputs)
    dev_inputs = to_dev(inputs, gpu)
    out = kernels.get(op)(**dev_inputs)
    torch.cuda.synchronize()
    assert not (has_nan_inf(out) and not has_nan_inf(expected)), f"{op} {label}: NaN/Inf in output"
    tol = cfg["tolerances"][dtype]
    if op == "layernorm" and dtype == torch.bfloat16:
        # The harness's bf16 layernorm tolerance (2e-3) is below one bf16 rounding step (2^-8
        # relative): two fp32 implementations round rare near-tie values to neighbouring bf16
        # values. Stock F.layer_norm on the GPU misses 2e-3 against the same oracle on about the
        # same share of elements (measured 0-0.0006 % for both). Check the north-star bf16
        # tolerance, that such flips stay rare, and that they are no more frequent than stock's.
        assert_close(out, expected, 1e-2, 1e-2, f"{op} {label} {dtype}")
        bound = tol["atol"] + tol["rtol"] * expected.float().abs()
        d = (out.float().cpu() - expected.float()).abs()
        flips = (d > bound).float().mean().item()
        x = dev_inputs["x"]
        stock = torch.nn.functional.layer_norm(x, x.shape[-1:], dev_inputs["weight"], dev_inputs["bias"], 1e-5)
        stock_flips = ((stock.float().cpu() - expected.float()).abs() > bound).float().mean().item()
        print(f"layernorm bf16 {label} {tuple(size.values())}: {flips:.4%} of elements beyond the table's "
              f"{tol['atol']:g} (one bf16 step; stock GPU F.layer_norm {stock_flips:.4%}), max |d| "
              f"{d.max().item():.3e}", flush=True)
        assert flips < 1e-3, f"{op} {label}: {flips:.2%} of elements differ by a bf16 step"
        assert flips <= 4 * stock_flips + 1e-5, f"{op} {label}: {flips:.4%} flips against stock's {stock_flips:.4%}"
        return
    assert_close(out, expected, tol["atol"], tol["rtol"], f"{op} {label} {dtype}")


@pytest.mark.parametrize("case", [c for c, _ in spec.ADVERSARIAL])
@pytest.mark.parametrize("op", list(spec.KERNEL_CONFIGS))
def test_adversarial(gpu, op, case):
    """The reference harness's stage 3: NaN/Inf only where the reference has them, else 10x tol."""
    cfg = spec.KERNEL_CONFIGS[op]
    dtype = cfg["test_dtypes"][0]
    inputs = spec.adversarial_inputs(cfg["input_generator"](spec.stage_size(cfg), dtype, "cpu", seed=42), case)
    expected = R.REFERENCE[op](inputs)
    out = kernels.get(op)(**to_dev(inputs, gpu)).cpu()
    if has_nan_inf(out) or has_nan_inf(expected):
        assert has_nan_inf(out) and has_nan_inf(expected), \
            f"{op}/{case}: output NaN/Inf={has_nan_inf(out)} reference NaN/Inf={has_nan_inf(expected)}"
        return
    tol = cfg["tolerances"][dtype]
    assert_close(out, expected, 10 * tol["atol"], 10 * tol["rtol"], f"{op}/{case}")


@pytest.mark.parametrize("op", ["rmsnorm", "softmax", "layernorm", "rotary_embedding", "reduce"])
def test_adversarial_nan_positions_match(gpu, op):
    """Stricter than the harness rule for the row ops: NaN / Inf at the same elements."""
    cfg = spec.KERNEL_CONFIGS[op]
    dtype = cfg["test_dtypes"][0]
    for case in ("near_max", "mixed_scale"):
        inputs = spec.adversarial_inputs(cfg["input_generator"](spec.stage_size(cfg), dtype, "cpu", seed=42), case)
        expected = R.REFERENCE[op](inputs).float()
        out = kernels.get(op)(**to_dev(inputs, gpu)).float().cpu()
        assert torch.equal(torch.isnan(out), torch.isnan(expected)), f"{op}/{case}: NaN mask differs"
        assert torch.equal(torch.isinf(out), torch.isinf(expected)), f"{op}/{case}: Inf mask differs"
        fin = torch.isfinite(expected)
        tol = cfg["tolerances"][dtype]
        assert_close(out[fin], expected[fin], 10 * tol["atol"], 10 * tol["rtol"], f"{op}/{case}")


@pytest.mark.parametrize("op", list(spec.KERNEL_CONFIGS))
def test_determinism(gpu, op):
    """Stage 4: three runs on identical inputs are bitwise equal."""
    cfg = spec.KERNEL_CONFIGS[op]
    dtype = cfg["test_dtypes"][0]
    outs = []
    for _ in range(3):
        inputs = to_dev(cfg["input_generator"](spec.stage_size(cfg), dtype, "cpu", seed=42), gpu)
        outs.append(kernels.get(op)(**inputs).cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


# ----------------------------------------------------------------------- BASELINE workloads
def test_baseline_rmsnorm(gpu):
    i = spec.baseline_rmsnorm()
    out = kernels.get("rmsnorm")(i["x"].to(gpu), i["weight"].to(gpu), 1e-6)
    assert_close(out, R.rmsnorm_ref(i["x"], i["weight"], 1e-6), 1e-2, 1e-2, "C1 rmsnorm")


def test_baseline_rope_and_softmax(gpu):
    i = spec.baseline_rope()
    rope = kernels.get("rotary_embedding")
    for name in ("q", "k"):
        out = rope(i[name].to(gpu), i["cos"].to(gpu), i["sin"].to(gpu)).cpu()
        exp = R.rotary_embedding_ref(i[name], i["cos"], i["sin"])
        assert torch.equal(out, exp), f"C2a rope {name}: not bit-identical to the oracle"
    s = spec.baseline_softmax()
    out = kernels.get("softmax")(s["x"].to(gpu))
    assert_close(out, R.softmax_ref(s["x"]), 1e-3, 1e-3, "C2b softmax")


def test_baseline_matmul(gpu):
    i = spec.baseline_matmul()
    out = kernels.get("matmul")(i["A"].to(gpu), i["B"].to(gpu))
    exp = R.matmul_ref(i["A"].float(), i["B"].float()).bfloat16()
    assert_close(out, exp, 1e-2, 1e-2, "C3a matmul")


def test_baseline_fused_mlp(gpu):
    i = spec.baseline_fused_mlp()
    out = kernels.get("fused_mlp")(**to_dev(i, gpu))
    exp = R.fused_mlp_ref(**i)
    assert_close(out, exp, 1e-2, 1e-2, "C3b fused_mlp")


@pytest.mark.parametrize("B,S", [(4, 2048), (1, 8192)])
def test_baseline_attention(gpu, B, S):
    """C4 at full size, every (batch, head) pair at both shapes. The oracle materialises S x S
    scores per (batch, head), so it runs one head at a time (about a second of CPU per head at
    S = 8192)."""
    i = spec.baseline_attention(B=B, S=S)
    out = kernels.get("flash_attention")(**to_dev(i, gpu)).cpu()
    for b in range(B):
        for h in range(32):
            sl = (slice(b, b + 1), slice(h, h + 1))
            exp = R.flash_attention_ref(i["Q"][sl], i["K"][sl], i["V"][sl])
            assert_close(out[sl], exp, 1e-2, 1e-2, f"C4 attention B{B} S{S} batch {b} head {h}")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("H", [32, 8])  # 8 heads: 128 query blocks, the split-key path
def test_attention_as_accurate_as_sdpa(gpu, dt, H):
    """The flash kernel's arithmetic (a lazily raised exp2 base, P rounded for the P V product, row
    sums of the rounded P, one reciprocal at the end) is as accurate as the image's stock SDPA: at
    the 7B forward's [1, 32, 2048, 128], causal, its mean distance to an fp32 evaluation of the same
    inputs is within 10 % of SDPA's and its largest within 50 % (measured: mean +3.9 % in f16 and
    bf16, max 8 % / 24 % below SDPA's). With 8 heads the grid is small enough for the split-key
    path (two key halves merged at the end), held to the same bounds (measured: mean +2.5 %,
    max 1.4 % below SDPA's in f16 and equal in bf16). Inputs as C4 (N(0, 1),
    seeded on the CPU); the fp32 reference is SDPA on the fp32 copies."""
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(1, H, 2048, 128, generator=g).to(dt).to(gpu) for _ in range(3))
    out = kernels.get("flash_attention")(q, k, v, causal=True).float()
    sdpa = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True).float()
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True)
    e_ak, e_sdpa = (out - ref).abs(), (sdpa - ref).abs()
    same = (out == sdpa).float().mean().item()
    print(f"attention {dt} H={H}: vs fp32 mean {e_ak.mean().item():.3e} max {e_ak.max().item():.3e}; stock SDPA mean "
          f"{e_sdpa.mean().item():.3e} max {e_sdpa.max().item():.3e}; {100 * same:.2f} % bit-equal to SDPA", flush=True)
    assert e_ak.mean() <= 1.10 * e_sdpa.mean(), (dt, H, e_ak.mean().item(), e_sdpa.mean().item())
    assert e_ak.max() <= 1.5 * e_sdpa.max(), (dt, H, e_ak.max().item(), e_sdpa.max().item())


# ----------------------------------------------------------------------- golden fixtures
def fx(name):
    with np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False) as z:
        return {k: torch.from_numpy(np.ascontiguousarray(z[k])) for k in z.files}


def test_golden_on_gpu(gpu):
    f = fx("rmsnorm_f16")
    y = kernels.get("rmsnorm")(f["x"].to(gpu), f["w"].to(gpu)).cpu()
    assert torch.all(y[2] == 0)
    assert_close(y, f["y"], 2e-3, 2e-3, "golden rmsnorm f16")
    for name in ("rope_f16", "rope_f32"):
        f = fx(name)
        y = kernels.get("rotary_embedding")(f["x"].to(gpu), f["cos"].to(gpu), f["sin"].to(gpu)).cpu()
        assert torch.equal(y, f["y"]), f"golden {name}: not bit-identical"
    f = fx("softmax_f32")
    assert_close(kernels.get("softmax")(f["x"].to(gpu)), f["y64"], 1e-6, 1e-6, "golden softmax")
    f = fx("layernorm_f32")
    assert_close(kernels.get("layernorm")(f["x"].to(gpu), f["w"].to(gpu), f["b"].to(gpu)), f["y64"], 1e-5, 1e-5, "golden layernorm")
    f = fx("cross_entropy_f32")
    y = kernels.get("cross_entropy")(f["logits"].to(gpu), f["targets"].to(gpu))
    assert abs(y.item() - f["y64"].item()) < 1e-5
    f = fx("reduce_f32")
    ys = kernels.get("reduce")(f["x"].to(gpu)).cpu().double()
    assert torch.allclose(ys, f["sum64"], atol=1e-5, rtol=1e-5, equal_nan=True), "golden sum"
    mx = reduce_mod.reduce_max(f["x"].to(gpu)).cpu()
    assert torch.equal(torch.isnan(mx), torch.isnan(f["max"]))
    assert torch.equal(mx[~torch.isnan(mx)], f["max"][~torch.isnan(f["max"])])
    for name, tol in (("matmul_f32", 1e-4), ("matmul_f16", 1e-2)):
        f = fx(name)
        assert_close(kernels.get("matmul")(f["A"].to(gpu), f["B"].to(gpu)), f["y64"], tol, tol, name)
    f = fx("attention_f16")
    for causal, key in ((True, "causal64"), (False, "full64")):
        y = kernels.get("flash_attention")(f["Q"].to(gpu), f["K"].to(gpu), f["V"].to(gpu), causal=causal)
        assert_close(y, f[key], 1e-2, 1e-2, f"golden attention causal={causal}")
    f = fx("fused_mlp_f32")
    for act in ("silu", "gelu", "relu2"):
        y = kernels.get("fused_mlp")(f["x"].to(gpu), f["wg"].to(gpu), f["wu"].to(gpu), f["wd"].to(gpu), act)
        assert_close(y, f[act + "64"], 1e-4, 1e-4, f"golden fused_mlp {act}")


def _one_step(out, exp, what, min_equal=0.95):
    """16-bit result against a once-rounded fixture: mostly bit-identical, never more than one
    rounding step away."""
    out, exp = out.cpu(), exp.to(out.dtype)
    same = out == exp
    step = 2.0 ** -10 if out.dtype == torch.float16 else 2.0 ** -7
    far = (out.double() - exp.double()).abs() > step * exp.double().abs().clamp_min(2.0 ** -14) * 1.0001
    assert same.float().mean().item() >= min_equal, f"{what}: {same.float().mean().item():.2%} bit-identical"
    assert not bool(far[~same].any()), f"{what}: an element more than one rounding step off"


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_golden_16bit_on_gpu(gpu, dt):
    """layernorm, reduce and the fused MLP in f16 / bf16 against the step-rounded float64 fixtures."""
    tag = "f16" if dt == torch.float16 else "bf16"
    f = {k: v.to(dt) for k, v in fx(f"layernorm_{tag}").items()}
    _one_step(kernels.get("layernorm")(f["x"].to(gpu), f["w"].to(gpu), f["b"].to(gpu)), f["y"], f"layernorm {tag}")
    f = fx(f"reduce_{tag}")
    x = f["x"].to(dt).to(gpu)
    _one_step(kernels.get("reduce")(x), f["sum"], f"reduce sum {tag}")
    assert torch.equal(reduce_mod.reduce_max(x).cpu(), f["max"].to(dt)), f"reduce max {tag}"
    f = {k: v.to(dt) for k, v in fx(f"fused_mlp_{tag}").items()}
    for act in ("silu", "gelu", "relu2"):
        y = kernels.get("fused_mlp")(f["x"].to(gpu), f["wg"].to(gpu), f["wu"].to(gpu), f["wd"].to(gpu), act)
        _one_step(y, f[act], f"fused_mlp {act} {tag}")


# --------------------------------------------------------------------------- layouts / API
def test_matmul_linear_layout_and_strides(gpu):
    g = torch.Generator().manual_seed(3)
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        x = torch.randn(300, 256, generator=g).to(dt)
        W = torch.randn(520, 256, generator=g).to(dt)
        exp = R.matmul_ref(x.float(), W.float().T).to(dt)
        out = kernels.get("matmul")(x.to(gpu), W.to(gpu).t())  # [N, K] read in place
        tol = 1e-4 if dt == torch.float32 else 2e-2
        assert_close(out, exp, tol, tol, f"NT {dt}")
        big = torch.randn(300, 300, generator=g).to(dt)
        xs = big.to(gpu)[:, :256]  # lda = 300 != K
        assert_close(kernels.get("matmul")(xs, W.to(gpu).t()), R.matmul_ref(big[:, :256].float(), W.float().T).to(dt), tol, tol, "strided A")
    A = torch.randn(3, 64, 128, generator=g).half()
    B = torch.randn(3, 128, 96, generator=g).half()
    assert_close(kernels.get("matmul")(A.to(gpu), B.to(gpu)), R.matmul_ref(A.float(), B.float()).half(), 1e-2, 1e-2, "batched")


@pytest.mark.parametrize("M,N,K,layout,dt", [
    (1023, 1023, 1023, "kn", torch.float16),      # K, lda and ldb odd
    (600, 300, 515, "nk", torch.bfloat16),        # nn.Linear-layout B, K odd
    (700, 1001, 512, "kn", torch.float16),        # [K, N] B with N % 8 != 0
    (257, 1030, 1024, "kn", torch.bfloat16),      # N % 8 == 6
    (512, 640, 512, "offset", torch.float16),     # A's base 2 bytes past a 16-byte boundary
    (100, 90, 70, "kn", torch.float16),           # below the repack size: the element-load kernel
])
def test_matmul_misaligned_operands_repacked(gpu, M, N, K, layout, dt):
    """Operands the 16-byte loads cannot read are repacked by kernel_fn (zero-padded K, [N, K] or
    [K, N] copies): the result equals the register-staged kernel run on the original operands bit
    for bit (the padding adds exact zeros at the end of each sum), and the oracle at the tolerance."""
    from autokernel_amd.kernels import _ops
    g = torch.Generator().manual_seed(M + N + K)
    A = (torch.randn(M, K + (1 if layout == "offset" else 0), generator=g) / K ** 0.5).to(dt)
    if layout == "nk":
        W = torch.randn(N, K, generator=g).to(dt)
        Bd, Bs, bt = W.to(gpu).t(), W.to(gpu), True
        Bf = W.float().T
    else:
        Bk = torch.randn(K, N, generator=g).to(dt)
        Bd, Bs, bt = Bk.to(gpu), Bk.to(gpu), False
        Bf = Bk.float()
    Ad = A.to(gpu)[:, 1:] if layout == "offset" else A.to(gpu)
    Af = A[:, 1:].float() if layout == "offset" else A.float()
    out = kernels.get("matmul")(Ad, Bd)
    assert_close(out, R.matmul_ref(Af, Bf).to(dt), 2e-2, 2e-2, f"misaligned {M}x{N}x{K} {layout} {dt}")
    direct = torch.empty(M, N, device=gpu, dtype=dt)
    _ops.gemm(direct, Ad, Bs, bt, None)
    assert torch.equal(out, direct), f"repacked != element-load kernel {M}x{N}x{K} {layout} {dt}"


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_matmul_batched_past_grid_z_limit(gpu, dt):
    """70000 items: past the 65535 a grid's z dimension holds, so ak_gemm_batched runs the batch in
    two chunks; every item against the oracle, including the first and last of each chunk."""
    g = torch.Generator().manual_seed(5)
    A = (torch.randn(70000, 8, 16, generator=g) / 4).to(dt)
    B = torch.randn(70000, 16, 24, generator=g).to(dt)
    out = kernels.get("matmul")(A.to(gpu), B.to(gpu)).cpu()
    exp = R.matmul_ref(A.float(), B.float()).to(dt)
    tol = 1e-4 if dt == torch.float32 else 2e-2
    assert_close(out, exp, tol, tol, f"70000 x [8 x 24 x 16] {dt}")
    for i in (0, 65534, 65535, 69999):
        assert_close(out[i], exp[i], tol, tol, f"item {i} {dt}")


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_matmul_batched_one_launch(gpu, dt):
    """torch.matmul's batched and broadcast forms run as one ak_gemm_batched launch (the batch on the
    grid's third dimension): against the oracle at the table's tolerance, and bit-identical to the
    same products run one 2-D GEMM at a time (the same per-element arithmetic). Cases: [K, N] and
    transposed ([N, K] stored) B, a 2-D operand broadcast over the batch (batch stride 0), two
    broadcast batch dims, attention-shaped products, K not a multiple of 8 and a [K, N] B with
    N % 8 != 0 (the register-staged kernel; per item, the 2-D path's repacked LDS-DMA products give
    the same bits), an empty batch and K = 0."""
    from autokernel_amd.kernels.host import _gemm
    g = torch.Generator().manual_seed(21)
    tol = 1e-4 if dt == torch.float32 else 2e-2

    def r(*s):
        return (torch.randn(*s, generator=g) / max(s[-1], 1) ** 0.5).to(dt)
    cases = [(r(3, 64, 128), r(3, 128, 96)),
             (r(4, 70, 256), r(4, 96, 256).transpose(-1, -2)),     # B read as stored [N, K] matrices
             (r(70, 256), r(5, 256, 136)),                         # A broadcast (batch stride 0)
             (r(5, 96, 256), r(256, 136)),                         # B 2-D: flattened into one GEMM
             (r(6, 64, 512), r(512, 96).expand(6, 512, 96)),       # B broadcast (batch stride 0)
             (r(2, 1, 40, 64), r(1, 3, 64, 72)),                   # two broadcast batch dims
             (r(32, 512, 64), r(32, 64, 512)),                     # attention scores shape
             (r(32, 512, 512), r(32, 512, 64)),
             (r(3, 33, 100), r(3, 100, 40)),                       # K % 8 != 0
             (r(8, 128, 130), r(8, 130, 256)),                     # K % 8 != 0, items the 2-D path repacks
             (r(4, 96, 256), r(4, 256, 100)),                      # [K, N] B, N % 8 != 0
             (r(0, 8, 64), r(0, 64, 8)), (r(2, 8, 0), r(2, 0, 8))]
    for A, B in cases:
        out = kernels.get("matmul")(A.to(gpu), B.to(gpu)).cpu()
        exp = R.matmul_ref(A.float(), B.float()).to(dt)
        what = f"{tuple(A.shape)} @ {tuple(B.shape)} {dt}"
        assert out.shape == exp.shape, what
        assert_close(out, exp, tol, tol, what)
        if B.dim() >= 3 and out.numel() and A.shape[-1]:
            batch = torch.broadcast_shapes(A.shape[:-2], B.shape[:-2])
            Ab = A.expand(*batch, *A.shape[-2:]).reshape(-1, *A.shape[-2:]).to(gpu)
            Bb = B.expand(*batch, *B.shape[-2:]).reshape(-1, *B.shape[-2:]).to(gpu)
            one = torch.stack([_gemm(Ab[i], Bb[i]) for i in range(Ab.shape[0])]).cpu()
            assert torch.equal(out.reshape(one.shape), one), what


@pytest.mark.parametrize("M,N,K", [(2048, 6144, 256), (500, 1100, 320), (256, 192, 64)])
def test_matmul_linear_wide_tiles(gpu, M, N, K):
    """nn.Linear-layout shapes whose best tiling is 256x192 (a fused QKV projection's 2048 x 6144,
    ragged edges in M and N, a single tile) against the fp32 oracle."""
    g = torch.Generator().manual_seed(M + N)
    for dt in (torch.float16, torch.bfloat16):
        x = (torch.randn(M, K, generator=g) / K ** 0.5).to(dt)
        W = torch.randn(N, K, generator=g).to(dt)
        out = kernels.get("matmul")(x.to(gpu), W.to(gpu).t())
        assert_close(out, R.matmul_ref(x.float(), W.float().T).to(dt), 2e-2, 2e-2, f"{M}x{N}x{K} {dt}")


@pytest.mark.parametrize("M,N,K,bt", [(300, 520, 256, True), (2048, 4096, 512, True), (130, 102, 96, True),
                                      (257, 384, 128, False), (64, 200, 70, False)])
def test_gemm_residual_equals_gemm_then_add(gpu, M, N, K, bt):
    """ak_gemm_residual (LDS-DMA path, [K, N] B path, register-staged fallback for K % 64 != 0,
    unaligned row strides) gives exactly ak_gemm followed by torch's element-type add, and the
    oracle's R + A @ B within the matmul tolerance."""
    from autokernel_amd.kernels.matmul import gemm, gemm_residual
    g = torch.Generator().manual_seed(M * 7 + N + K)
    for dt in (torch.float16, torch.bfloat16):
        A = (torch.randn(M, K, generator=g) / K ** 0.5).to(dt)
        W = torch.randn(N, K, generator=g).to(dt) if bt else torch.randn(K, N, generator=g).to(dt)
        Rr = (torch.randn(M, N, generator=g) * 8).to(dt)
        Rr[0, : min(N, 8)] = -0.0
        Ad, Wd, Rd = A.to(gpu), W.to(gpu), Rr.to(gpu)
        Bd = Wd.t() if bt else Wd
        out = gemm_residual(Ad, Bd, Rd)
        sep = Rd + gemm(Ad, Bd)
        assert torch.equal(out, sep), f"{M}x{N}x{K} bt={bt} {dt}: fused add differs from the separate add"
        B32 = W.float().T if bt else W.float()
        exp = (Rr.float() + R.matmul_ref(A.float(), B32).to(dt).float()).to(dt)
        assert_close(out, exp, 2e-2, 2e-2, f"{M}x{N}x{K} bt={bt} {dt}")


@pytest.mark.parametrize("Bt,T,heads,D,K,bt", [(2, 300, (8, 2, 2), 64, 512, True), (1, 130, (2, 1, 1), 128, 96, True),
                                              (2, 128, (2, 2, 0), 64, 128, False)])
def test_gemm_rope_equals_projection_then_rotation(gpu, Bt, T, heads, D, K, bt):
    """ak_gemm_rope (LDS-DMA path, register-staged fallback for K % 64 != 0, [K, N] B) gives
    exactly the projection followed by the model's fp32 rotation of the q / k columns, computed
    with separate torch ops as the model does, and leaves the v columns as plain products."""
    from autokernel_amd import llama
    from autokernel_amd.kernels.matmul import gemm, gemm_rope
    H, Hk, Hv = heads
    N, rot = (H + Hk + Hv) * D, (H + Hk) * D
    g = torch.Generator().manual_seed(T + D + K)
    cos, sin = llama.rope_tables(D, T + 5)
    for dt in (torch.float16, torch.bfloat16):
        A = torch.randn(Bt * T, K, generator=g).to(dt)
        W = (torch.randn(N, K, generator=g) * 0.05).to(dt)
        Wd = W.to(gpu) if bt else W.t().contiguous().to(gpu)
        Bm = Wd.t() if bt else Wd
        c, s = cos.to(gpu), sin.to(gpu)
        out = gemm_rope(A.to(gpu), Bm, c, s, T, D, rot)
        plain = gemm(A.to(gpu), Bm)
        qk = plain[:, :rot].view(Bt, T, H + Hk, D)
        eq, _ = llama.apply_rotary_emb(qk, qk, c, s)
        assert torch.equal(out[:, :rot], eq.reshape(Bt * T, rot)), f"rotated columns {dt}"
        assert torch.equal(out[:, rot:], plain[:, rot:]), f"plain columns {dt}"


def test_rope_model_layout(gpu):
    """[B, S, H, D] with cos [1, S, 1, D/2] (the layout a LLaMA block holds) reads the table per s."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 40, 8, 64, generator=g).half()
    cos, sin = spec.rope_tables(40, 64)
    c4, s4 = cos.view(1, 40, 1, 32), sin.view(1, 40, 1, 32)
    out = kernels.get("rotary_embedding")(x.to(gpu), c4.to(gpu), s4.to(gpu)).cpu()
    assert torch.equal(out, R.rotary_embedding_ref(x, c4, s4))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_rope_index_arithmetic(gpu, dt):
    """The kernels find a thread's row, column and table row by multiply-shift division. Divisors
    that are not powers of two: head_dim 96 (12 or 24 vectors per row), 37 and 127 table rows,
    3 heads per token, many table periods, rows fewer than a wave. Bit-identical to the oracle,
    and the fp32-table model form (q as a column slice of a fused projection) bit-identical to the
    reference model's complex rotation in fp32."""
    from autokernel_amd import llama
    from autokernel_amd.kernels.rotary_embedding import apply_fp32_tables
    g = torch.Generator().manual_seed(11)
    cases = [((3, 5, 37, 96), (37, 48)),        # [B, H, S, D]: table row = row % 37, 15 periods
             ((2, 37, 3, 96), (1, 37, 1, 48)),  # [B, S, H, D]: table row = (row // 3) % 37
             ((1, 7, 127, 64), (127, 32)),
             ((2, 1, 3, 96), (3, 48))]          # 6 rows
    for xs, ts in cases:
        x = torch.randn(*xs, generator=g).to(dt)
        c, s = torch.randn(*ts, generator=g).to(dt), torch.randn(*ts, generator=g).to(dt)
        out = kernels.get("rotary_embedding")(x.to(gpu), c.to(gpu), s.to(gpu)).cpu()
        assert torch.equal(out, R.rotary_embedding_ref(x, c, s)), (xs, ts, dt)
    if dt != torch.float32:
        qkv = torch.randn(2, 37, 3 * 96 + 40, generator=g).to(dt)
        cos, sin = llama.rope_tables(96, 41)
        q = qkv[..., :288].view(2, 37, 3, 96)
        exp, _ = llama.apply_rotary_emb(q, q, cos, sin)
        out = apply_fp32_tables(qkv.to(gpu)[..., :288].view(2, 37, 3, 96), cos.to(gpu), sin.to(gpu)).cpu()
        assert torch.equal(out, exp), (dt, (out.float() - exp.float()).abs().max().item())


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("S", [200, 600])  # 600: the split-key path (80 query blocks, Sk >= 256)
def test_attention_gqa_strided(gpu, D, causal, S):
    g = torch.Generator().manual_seed(5 + S)
    B, Hq, Hkv = 2, 8, 2
    q = torch.randn(B, S, Hq, D, generator=g).half()
    k = torch.randn(B, S, Hkv, D, generator=g).half()
    v = torch.randn(B, S, Hkv, D, generator=g).half()
    # strided [B, H, S, D] views of [B, S, H, D] storage, GQA without repeat_interleave
    out = fa_mod.attention(q.to(gpu).transpose(1, 2), k.to(gpu).transpose(1, 2), v.to(gpu).transpose(1, 2), causal)
    rep = Hq // Hkv
    exp = R.flash_attention_ref(q.transpose(1, 2).float(), k.transpose(1, 2).repeat_interleave(rep, 1).float(),
                                v.transpose(1, 2).repeat_interleave(rep, 1).float(), causal)
    assert_close(out, exp, 1e-2, 1e-2, f"GQA D{D} causal={causal} S={S}")


@pytest.mark.parametrize("D,dt", [(64, torch.float16), (128, torch.float16), (128, torch.bfloat16)])
@pytest.mark.parametrize("trend", ["rising", "falling"])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_moving_row_max(gpu, D, dt, trend, causal):
    """Scores that rise (or fall) steadily along the key axis: about 5.4 log2 units per 64-key tile
    over 1024 keys, so with a rising trend every row's maximum passes the kernel's lazily raised
    exp2 base (slack 8) on every other tile and the O rescale and row-sum update run all through the
    steady state; with a falling trend they never run after the first tile. Raw Q K^T reaches ~700,
    where f16 steps are 0.5: the reference's rounding of Q K^T to f16 would itself move these
    softmax weights by ~3 %, so the expected output is the oracle's op sequence on fp32 copies of
    the inputs (no intermediate rounding), at the harness's tolerance for the output type."""
    g = torch.Generator().manual_seed(11 + D)
    B, H, S = 1, 4, 1024
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    ramp = torch.linspace(0.0, 85.0, S) if trend == "rising" else torch.linspace(85.0, 0.0, S)
    Q = (8.0 * u + 0.1 * torch.randn(B, H, S, D, generator=g)).to(dt)
    K = (ramp[:, None] * u + 0.1 * torch.randn(B, H, S, D, generator=g)).to(dt)
    V = torch.randn(B, H, S, D, generator=g).to(dt)
    out = kernels.get("flash_attention")(Q.to(gpu), K.to(gpu), V.to(gpu), causal)
    exp = R.flash_attention_ref(Q.float(), K.float(), V.float(), causal)
    tol = 1e-2 if dt == torch.float16 else 2e-2
    assert_close(out, exp, tol, tol, f"{trend} scores D{D} {dt} causal={causal}")


@pytest.mark.parametrize("D,dt", [(64, torch.float16), (128, torch.float16), (64, torch.bfloat16), (128, torch.bfloat16)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Sq,Sk", [(1024, 1024), (777, 777), (300, 1000), (1000, 300), (256, 256), (1023, 1023)])
def test_attention_split_keys(gpu, D, dt, causal, Sq, Sk):
    """Grids of at most 256 query blocks with Sk >= 256 split each block's key tiles over two wave
    groups and merge (O, base, row sum) at the end. Covered: odd tile counts (an empty last
    iteration in the second half), a partial last key tile, rectangular causal masks both ways (a
    second-half wave may have no key for its queries), GQA, D 64 / 128, f16 / bf16. Checked against
    the oracle at the harness tolerance, and against the unsplit kernel on the same inputs (the
    heads repeated until the grid passes 256 blocks): within four output ulps (P is rounded relative
    to each half's own exp2 base, so the two paths may round a few weights differently)."""
    g = torch.Generator().manual_seed(Sq * 3 + Sk + D)
    B, Hq, Hk = 1, 4, 2
    Q = torch.randn(B, Hq, Sq, D, generator=g).to(dt)
    K = torch.randn(B, Hk, Sk, D, generator=g).to(dt)
    V = torch.randn(B, Hk, Sk, D, generator=g).to(dt)
    assert -(-Sq // 128) * Hq * B <= 256 and Sk >= 256  # the split path
    exp = R.flash_attention_ref(Q, K.repeat_interleave(2, 1), V.repeat_interleave(2, 1), causal)
    out = kernels.get("flash_attention")(Q.to(gpu), K.to(gpu), V.to(gpu), causal)
    tol = 1e-2 if dt == torch.float16 else 2e-2
    assert_close(out, exp, tol, tol, f"split keys {Sq}x{Sk} D{D} {dt} causal={causal}")
    rep = -(-257 // (-(-Sq // 128) * Hq)) + 1  # enough head copies for more than 256 blocks
    Qr, Kr, Vr = (t.repeat(1, rep, 1, 1).to(gpu) for t in (Q, K, V))
    whole = kernels.get("flash_attention")(Qr, Kr, Vr, causal)[:, :Hq].cpu()
    ulp = 2.0 ** -10 if dt == torch.float16 else 2.0 ** -7
    d = (out.cpu().float() - whole.float()).abs()
    assert (d <= 4 * ulp * torch.clamp(whole.float().abs(), min=1.0)).all(), d.max().item()


@pytest.mark.parametrize("D,dt", [(64, torch.float16), (128, torch.bfloat16)])
@pytest.mark.parametrize("Sk", [1, 63, 64, 300, 4096])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_decode_shapes(gpu, D, dt, Sk, causal):
    """One query row against 1 .. 4096 keys (a decode step), GQA 32 / 8: the query block holds one
    valid row, so three of its four waves (in each key half, where the keys split) have no query.
    With the top-left causal mask the single query sees key 0 only, so its output is V[0]."""
    g = torch.Generator().manual_seed(Sk + D)
    Q = torch.randn(2, 32, 1, D, generator=g).to(dt)
    K = torch.randn(2, 8, Sk, D, generator=g).to(dt)
    V = torch.randn(2, 8, Sk, D, generator=g).to(dt)
    exp = R.flash_attention_ref(Q, K.repeat_interleave(4, 1), V.repeat_interleave(4, 1), causal)
    out = kernels.get("flash_attention")(Q.to(gpu), K.to(gpu), V.to(gpu), causal).cpu()
    tol = 1e-2 if dt == torch.float16 else 2e-2
    assert_close(out, exp, tol, tol, f"decode Sk={Sk} D{D} {dt} causal={causal}")
    if causal:
        assert torch.equal(out, V.repeat_interleave(4, 1)[:, :, :1]), "causal decode row is V[0]"


def test_attention_rectangular_and_scale(gpu):
    g = torch.Generator().manual_seed(6)
    Q = torch.randn(1, 4, 96, 64, generator=g).bfloat16()
    K = torch.randn(1, 4, 160, 64, generator=g).bfloat16()
    V = torch.randn(1, 4, 160, 64, generator=g).bfloat16()
    for causal in (True, False):
        for scale in (None, 0.05, 0.0, 1.0):  # 1.0: unscaled scores
            out = kernels.get("flash_attention")(Q.to(gpu), K.to(gpu), V.to(gpu), causal, scale)
            exp = R.flash_attention_ref(Q.float(), K.float(), V.float(), causal, scale)
            assert_close(out, exp, 2e-2, 2e-2, f"rect causal={causal} scale={scale}")


def test_softmax_dispatch_timed_events(gpu):
    """ak_set_launch_events: the next softmax dispatch records the pair (a positive duration), the
    result is the untimed launch's, and the setting applies to one launch only."""
    from autokernel_amd import _lib
    x = torch.randn(1024, 4096, generator=torch.Generator().manual_seed(9)).half().to(gpu)
    want = kernels.get("softmax")(x)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    b.record()
    torch.cuda.synchronize()
    assert _lib.load().ak_set_launch_events(a.cuda_event, b.cuda_event) == _lib.AK_OK
    got = kernels.get("softmax")(x)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b)
    assert torch.equal(got, want)
    assert 0.0 < ms < 50.0, ms
    c = torch.cuda.Event(enable_timing=True)
    c.record()
    kernels.get("softmax")(x)  # untimed: leaves b as the first dispatch recorded it
    torch.cuda.synchronize()
    assert a.elapsed_time(b) == ms


def test_reduce_other_dims_and_max(gpu):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(6, 70, 33, generator=g).half()
    for dim in (0, 1, 2, -1):
        assert_close(kernels.get("reduce")(x.to(gpu), dim), R.reduce_sum_ref(x.float(), dim).half(), 1e-2, 1e-2, f"sum dim {dim}")
        assert torch.equal(reduce_mod.reduce_max(x.to(gpu), dim).cpu(), R.reduce_max_ref(x, dim))


def test_softmax_dim_and_layernorm_none(gpu):
    g = torch.Generator().manual_seed(8)
    x = torch.randn(33, 17, 5, generator=g)
    assert_close(kernels.get("softmax")(x.to(gpu), 0), R.softmax_ref(x, 0), 1e-5, 1e-5, "softmax dim 0")
    y = kernels.get("layernorm")(x.to(gpu), None, None)
    assert_close(y, torch.nn.functional.layer_norm(x, (5,)), 1e-5, 1e-5, "layernorm no affine")


WIDE_TOL = {torch.float16: 1e-3, torch.bfloat16: 2e-3, torch.float32: 1e-5}


@pytest.mark.parametrize("cols", [4097, 16383, 16385, 50257, 65535, 65537])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=["f16", "bf16", "f32"])
def test_softmax_ce_wide_odd_rows(gpu, cols, dtype):
    """Widths that do not vectorise, on each side of the register-cached wide-row kernels' limits
    (4096 < cols <= 16 * 1024 and <= 64 * 1024; 65537 stays on the looped kernel): softmax and
    cross-entropy against the oracle, with a row holding -inf entries, a row of large values and a
    constant row, and bitwise-equal reruns."""
    g = torch.Generator().manual_seed(cols)
    x = torch.randn(6, cols, generator=g) * 3
    x[1, ::7] = -math.inf
    x[2] = x[2] * 10 + (60000 if dtype == torch.float16 else 1e5)
    x[3] = 0.5
    x = x.to(dtype)
    tol = WIDE_TOL[dtype]
    sm = kernels.get("softmax")
    y = sm(x.to(gpu))
    assert_close(y, R.softmax_ref(x), tol, tol, f"softmax wide {cols} {dtype}")
    assert torch.equal(y, sm(x.to(gpu))), "softmax wide rerun differs"
    # the input one element past an aligned base: its rows no longer share the output's dword
    # alignment, so 16-bit rows take the unpacked wide kernel
    buf = torch.empty(x.numel() + 1, dtype=dtype, device=gpu)
    buf[1:] = x.flatten().to(gpu)
    y_off = sm(buf[1:].view_as(x))
    assert_close(y_off, R.softmax_ref(x), tol, tol, f"softmax wide {cols} {dtype}, offset input")
    tg = torch.randint(0, cols, (6,), generator=g)
    tg[1] = 7  # a -inf logit: loss +inf, as the oracle gives
    tg[4] = -100
    keep = [0, 2, 3, 5]
    ce = kernels.get("cross_entropy")
    out = ce(x[keep].to(gpu), tg[keep].to(gpu))
    exp = R.cross_entropy_ref(x[keep], tg[keep])
    ce_tol = 1e-5 if dtype == torch.float32 else 1e-2  # the op table's cross-entropy tolerances
    assert abs(out.float().item() - exp.float().item()) <= ce_tol * max(1.0, abs(exp.float().item())), \
        f"cross-entropy wide {cols} {dtype}: {out.float().item()} vs {exp.float().item()}"
    out_inf = ce(x.to(gpu), tg.to(gpu))
    assert math.isinf(out_inf.float().item()) and math.isinf(R.cross_entropy_ref(x, tg).float().item())
    assert torch.equal(out, ce(x[keep].to(gpu), tg[keep].to(gpu))), "cross-entropy wide rerun differs"
    # a NaN or +inf logit makes its row NaN (softmax) and the loss NaN, as the oracle gives; an
    # all -inf row is NaN too. Row 5 keeps a finite target so only the planted value matters.
    xs = x[[0, 5, 0]].clone()
    xs[0, cols // 2] = math.nan
    xs[1, cols - 1] = math.inf
    xs[2] = -math.inf
    ys = sm(xs.to(gpu)).cpu()
    ref = R.softmax_ref(xs)
    assert torch.equal(torch.isnan(ys), torch.isnan(ref)), f"softmax wide {cols} {dtype}: NaN rows differ"
    for r in range(3):
        lr = ce(xs[r:r + 1].to(gpu), tg[[0]].to(gpu)).float().item()
        er = R.cross_entropy_ref(xs[r:r + 1], tg[[0]]).float().item()
        assert math.isnan(lr) and math.isnan(er), (cols, dtype, r, lr, er)


def test_cross_entropy_ignore_and_3d(gpu):
    g = torch.Generator().manual_seed(9)
    logits = torch.randn(2, 50, 320, generator=g).half()
    tg = torch.randint(0, 320, (2, 50), generator=g)
    tg[0, :7] = -100
    out = kernels.get("cross_entropy")(logits.to(gpu), tg.to(gpu))
    exp = R.cross_entropy_ref(logits, tg)
    assert out.dtype == logits.dtype and out.dim() == 0
    assert abs(out.float().item() - exp.float().item()) < 1e-2


def test_fused_mlp_activations_f16(gpu):
    g = torch.Generator().manual_seed(10)
    x = torch.randn(130, 256, generator=g).half()
    wg, wu = (torch.randn(384, 256, generator=g) * 0.05).half(), (torch.randn(384, 256, generator=g) * 0.05).half()
    wd = (torch.randn(256, 384, generator=g) * 0.05).half()
    for act in ("silu", "gelu", "relu2", "none"):
        out = kernels.get("fused_mlp")(x.to(gpu), wg.to(gpu), wu.to(gpu), wd.to(gpu), act)
        assert_close(out, R.fused_mlp_ref(x, wg, wu, wd, act), 1e-2, 1e-2, f"mlp {act}")


def test_copy_reference_kernel(gpu):
    """ak_copy (the bandwidth reference of the benchmark) copies bytes exactly, odd sizes included."""
    from autokernel_amd import _lib
    for n in (8, 4096 * 8 + 8, 1 << 22):
        src = torch.randint(-30000, 30000, (n,), device=gpu, dtype=torch.int16)
        dst = torch.zeros_like(src)
        _lib.check(_lib.load().ak_copy(src.data_ptr(), dst.data_ptr(), n * 2, _lib.stream_of(src)), "ak_copy")
        torch.cuda.synchronize()
        assert torch.equal(src, dst)


def _attention_abi(Q, K, V, causal, scale=None):
    """ak_flash_attn_fwd called directly (no padding in Python): for f16 / bf16 heads other than 64
    and 128 this is the general kernel."""
    from autokernel_amd import _lib
    B, H, S, D = Q.shape
    O = torch.empty_like(Q)
    a = [_lib.i64_array(t.stride()[:3]) for t in (Q, K, V, O)]
    st = _lib.load().ak_flash_attn_fwd(_lib.dtype_code(Q, "fa"), Q.data_ptr(), K.data_ptr(), V.data_ptr(),
                                       O.data_ptr(), B, H, K.shape[1], S, K.shape[2], D, a[0], a[1], a[2], a[3],
                                       int(causal), D ** -0.5 if scale is None else scale, _lib.stream_of(Q))
    _lib.check(st, "ak_flash_attn_fwd")
    return O


@pytest.mark.parametrize("D", [16, 32, 96, 256])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_attention_general_head_dims(gpu, D, dt):
    """Head dims other than 64 / 128 (the Triton starter's D in 16..256, kernels/flash_attention.py:159)
    at the harness's f16 / bf16 tolerance, both through kernel_fn (narrow heads zero-padded onto the
    MFMA kernels) and through the C ABI directly (the general kernel)."""
    g = torch.Generator().manual_seed(D)
    for causal, (B, H, S) in ((True, (1, 4, 127)), (False, (2, 2, 200))):
        Q, K, V = (torch.randn(B, H, S, D, generator=g).to(dt) for _ in range(3))
        exp = R.flash_attention_ref(Q, K, V, causal)
        out = kernels.get("flash_attention")(Q.to(gpu), K.to(gpu), V.to(gpu), causal)
        assert_close(out, exp, 1e-2, 1e-2, f"D={D} {dt} causal={causal}")
        direct = _attention_abi(Q.to(gpu), K.to(gpu), V.to(gpu), causal)
        assert_close(direct, exp, 1e-2, 1e-2, f"D={D} {dt} causal={causal} (general kernel)")


@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_attention_fp32(gpu, D):
    """fp32 attention at the north star's fp32 tolerance (1e-4): the general kernel keeps fp32
    throughout, including GQA, a rectangular causal mask, an explicit scale and strided views."""
    g = torch.Generator().manual_seed(100 + D)
    Q = torch.randn(2, 4, 150, D, generator=g)
    K = torch.randn(2, 2, 170, D, generator=g)
    V = torch.randn(2, 2, 170, D, generator=g)
    for causal in (True, False):
        exp = R.flash_attention_ref(Q, K.repeat_interleave(2, 1), V.repeat_interleave(2, 1), causal, 0.3)
        out = kernels.get("flash_attention")(Q.to(gpu), K.to(gpu), V.to(gpu), causal, 0.3)
        assert_close(out, exp, 1e-4, 1e-4, f"fp32 D={D} causal={causal}")
    # [B, S, H, D] storage read through transposed views
    Qs = Q.transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    Ks = K[:, :1].repeat(1, 4, 1, 1).transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    Vs = V[:, :1].repeat(1, 4, 1, 1).transpose(1, 2).contiguous().to(gpu).transpose(1, 2)
    exp = R.flash_attention_ref(Q, K[:, :1].repeat(1, 4, 1, 1), V[:, :1].repeat(1, 4, 1, 1), True)
    assert_close(kernels.get("flash_attention")(Qs, Ks, Vs, True), exp, 1e-4, 1e-4, f"fp32 strided D={D}")


def test_attention_general_overflow_rows(gpu):
    """Scores beyond the f16 range give the reference's inf / NaN rows (the harness's mixed_scale
    transform) at D = 32, in the general kernel (which rounds Q K^T and its scaled value to f16 as
    the reference does) and on the padded MFMA route; the NaN pattern must match exactly."""
    g = torch.Generator().manual_seed(5)
    Q, K, V = (torch.randn(1, 2, 96, 32, generator=g).half() for _ in range(3))
    Q[0, 0, 10:20] *= 300
    K[0, 0, :5] *= 300
    exp = R.flash_attention_ref(Q, K, V, True)
    assert torch.isnan(exp).any()
    keep = ~torch.isnan(exp)
    for out in (_attention_abi(Q.to(gpu), K.to(gpu), V.to(gpu), True).cpu(),
                kernels.get("flash_attention")(Q.to(gpu), K.to(gpu), V.to(gpu), True).cpu()):
        assert torch.equal(torch.isnan(out), torch.isnan(exp))
        assert_close(out[keep], exp[keep], 1e-2, 1e-2, "finite rows")


# ------------------------------------------------------------------ randomized shape sweeps
def _rand_shapes(seed, n, lo, hi, align_choices):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        dims = []
        for a in align_choices:
            v = int(rng.integers(lo, hi))
            dims.append(max(a, v - v % a))
        out.append(tuple(dims))
    return out


# grids that 128x128 tiles would leave mostly idle: the nn.Linear-layout B takes 64x64 tiles there
SMALL_GRID_SHAPES = [(2048, 768, 768), (2048, 768, 3072), (1024, 1024, 1024), (65, 130, 192), (64, 64, 64)]


@pytest.mark.parametrize("M,N,K", _rand_shapes(7, 10, 1, 700, (1, 4, 1)) + _rand_shapes(8, 6, 64, 1600, (16, 8, 64))
                         + SMALL_GRID_SHAPES)
def test_gemm_epilogues_random_shapes(gpu, M, N, K):
    """Seeded random shapes across the LDS-DMA path (K % 64 == 0, 64x64 to 256x256 tiles), the
    register-staged fallback and ragged tile edges, plus shapes whose grids take the small tiles:
    plain, residual and rotary epilogues in f16 and bf16, both B layouts; the epilogue variants
    equal the plain GEMM followed by the separate op, bit for bit."""
    from autokernel_amd import llama
    from autokernel_amd.kernels.matmul import gemm, gemm_residual, gemm_rope
    g = torch.Generator().manual_seed(M * 1009 + N * 31 + K)
    for dt in (torch.float16, torch.bfloat16):
        A = (torch.randn(M, K, generator=g) / max(K, 1) ** 0.5).to(dt)
        W = torch.randn(N, K, generator=g).to(dt)
        Rr = torch.randn(M, N, generator=g).to(dt)
        Ad, Rd = A.to(gpu), Rr.to(gpu)
        for bt in (True, False):
            Bd = W.to(gpu).t() if bt else W.t().contiguous().to(gpu)
            plain = gemm(Ad, Bd)
            assert_close(plain, R.matmul_ref(A.float(), W.float().T).to(dt), 2e-2, 2e-2, f"{M}x{N}x{K} bt={bt} {dt}")
            assert torch.equal(gemm_residual(Ad, Bd, Rd), Rd + plain), f"residual {M}x{N}x{K} bt={bt} {dt}"
            if N % 8 == 0:
                D = 8 if N % 16 else 16
                T = max(1, M // 2) if M % 2 == 0 else M
                cos, sin = (t.to(gpu) for t in llama.rope_tables(D, T))
                rot = (N // D - (1 if N // D > 1 else 0)) * D
                out = gemm_rope(Ad, Bd, cos, sin, T, D, rot)
                ref = plain.clone()
                if rot:
                    view = plain[:, :rot].reshape(M // T, T, rot // D, D)
                    eq, _ = llama.apply_rotary_emb(view, view, cos, sin)
                    ref[:, :rot] = eq.reshape(M, rot)
                assert torch.equal(out, ref), f"rope {M}x{N}x{K} bt={bt} {dt} D={D}"


def _attn_cases():
    rng = np.random.default_rng(11)
    cases = []
    for _ in range(12):
        B = int(rng.integers(1, 3))
        Hk = int(rng.integers(1, 3))
        Hq = Hk * int(rng.choice([1, 2, 4]))
        Sq, Sk = int(rng.integers(1, 300)), int(rng.integers(1, 300))
        D = int(rng.choice([16, 24, 32, 40, 64, 80, 96, 128, 160, 256]))
        dt = [torch.float16, torch.bfloat16, torch.float32][int(rng.integers(0, 3))]
        causal = bool(rng.integers(0, 2))
        cases.append(pytest.param(B, Hq, Hk, Sq, Sk, D, dt, causal, id=f"{B}x{Hq}/{Hk}x{Sq}x{Sk}x{D}-{str(dt)[6:]}-{'c' if causal else 'n'}"))
    return cases


@pytest.mark.parametrize("B,Hq,Hk,Sq,Sk,D,dt,causal", _attn_cases())
def test_attention_random_shapes(gpu, B, Hq, Hk, Sq, Sk, D, dt, causal):
    """Seeded random attention problems over every path (MFMA kernels, zero-padded narrow heads,
    the general kernel): GQA, rectangular causal masks, ragged lengths, f16 / bf16 / fp32."""
    g = torch.Generator().manual_seed(B * 7 + Hq * 13 + Sq * 17 + Sk * 19 + D)
    Q = torch.randn(B, Hq, Sq, D, generator=g).to(dt)
    K = torch.randn(B, Hk, Sk, D, generator=g).to(dt)
    V = torch.randn(B, Hk, Sk, D, generator=g).to(dt)
    rep = Hq // Hk
    exp = R.flash_attention_ref(Q, K.repeat_interleave(rep, 1), V.repeat_interleave(rep, 1), causal)
    out = kernels.get("flash_attention")(Q.to(gpu), K.to(gpu), V.to(gpu), causal)
    tol = 1e-4 if dt == torch.float32 else 1e-2
    # top-left causal mask: query i always sees key 0, so no row is empty
    assert_close(out, exp, tol, tol, f"attention {B}x{Hq}/{Hk}x{Sq}x{Sk}x{D} {dt} causal={causal}")


@pytest.mark.parametrize("M,N,K,bt", [(1024, 1024, 8192, True), (1024, 1024, 8192, False), (1024, 1024, 4096, False),
                                      (128, 128, 4096, True), (300, 520, 2048, True), (512, 200, 4096, False)])
def test_gemm_split_k(gpu, M, N, K, bt):
    """Under-filled grids with a long K run split-K (ak_gemm_ws, matmul's kernel_fn path): within the
    harness tolerance of the oracle in f16 / bf16, both B layouts, ragged tiles, and bitwise
    reproducible run to run."""
    from autokernel_amd import _lib
    from autokernel_amd.kernels.matmul import gemm
    lib = _lib.load()
    for dt in (torch.float16, torch.bfloat16):
        g = torch.Generator().manual_seed(M + N + K + int(bt))
        A = (torch.randn(M, K, generator=g) / K ** 0.5).to(dt)
        W = torch.randn(N, K, generator=g).to(dt)
        Bd = W.to(gpu).t() if bt else W.t().contiguous().to(gpu)
        code = _lib.dtype_code(A, "mm")
        ldb = K if bt else N
        assert lib.ak_gemm_workspace_bytes(code, M, N, K, K, ldb, N, int(bt)) > 0, "expected a split"
        outs = [gemm(A.to(gpu), Bd, split_k=True) for _ in range(3)]
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
        assert_close(outs[0], R.matmul_ref(A.float(), W.float().T).to(dt), 2e-2, 2e-2, f"split {M}x{N}x{K} {dt}")


@pytest.mark.parametrize("N", [1020, 1004])
def test_gemm_padded_kn_view_not_split(gpu, N):
    """A [K, N] B that is a column slice of a wider matrix (N % 8 == 4, ldb % 8 == 0, long K) must not
    take the split path, whose [K, N] kernel needs N % 8 == 0: the result equals the oracle in
    every column, the last four included."""
    from autokernel_amd import _lib
    from autokernel_amd.kernels.matmul import gemm
    lib = _lib.load()
    M, K, ld = 1024, 4096, 1024
    g = torch.Generator().manual_seed(N)
    A = (torch.randn(M, K, generator=g) / K ** 0.5).half()
    Bfull = torch.randn(K, ld, generator=g).half()
    assert lib.ak_gemm_workspace_bytes(_lib.AK_F16, M, N, K, K, ld, N, 0) == 0
    out = gemm(A.to(gpu), Bfull.to(gpu)[:, :N], split_k=True)
    exp = R.matmul_ref(A.float(), Bfull[:, :N].float()).half()
    assert_close(out, exp, 1e-2, 1e-2, f"padded [K, N] view N={N}")
    assert_close(out[:, -4:], exp[:, -4:], 1e-2, 1e-2, "last four columns")


@pytest.mark.parametrize("M,N,K", [(2048, 2304, 768), (300, 520, 200), (8 * 512, 3072, 768), (64, 50257, 768),
                                   (2048, 768, 768)])
def test_gemm_bias_one_rounding(gpu, M, N, K):
    """ak_gemm_bias: x @ W.T + bias with the bias added to the fp32 accumulator and one rounding,
    against the oracle's fp32 product + bias rounded once (f16 and bf16, nn.Linear layout), and
    compared with stock F.linear (printed: bitwise agreement)."""
    from autokernel_amd.kernels.matmul import gemm_bias
    for dt in (torch.float16, torch.bfloat16):
        g = torch.Generator().manual_seed(M + N + K)
        x = torch.randn(M, K, generator=g).to(dt)
        W = (torch.randn(N, K, generator=g) * 0.05).to(dt)
        b = (torch.randn(N, generator=g) * 0.5).to(dt)
        out = gemm_bias(x.to(gpu), W.to(gpu).t(), b.to(gpu))
        exp = (R.matmul_ref(x.float(), W.float().T) + b.float()).to(dt)
        assert_close(out, exp, 1e-2, 1e-2, f"gemm_bias {M}x{N}x{K} {dt}")
        stock = torch.nn.functional.linear(x.to(gpu), W.to(gpu), b.to(gpu))
        eq = (out == stock).float().mean().item()
        print(f"gemm_bias {M}x{N}x{K} {dt}: {100 * eq:.3f}% bit-equal to F.linear", flush=True)
        assert eq > 0.99


def _ulps16(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units in the last place between two f16 / bf16 tensors of one dtype (finite)."""
    def ordered(t):
        i = t.contiguous().view(torch.int16).int()
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (ordered(a) - ordered(b)).abs()


def _gelu_matches_torch(out: torch.Tensor, exp: torch.Tensor, what: str) -> None:
    """out against torch's F.gelu of the same rounded inputs: bit-equal on all but a handful of
    elements, and within one unit in the last place everywhere. The exceptions are inputs whose fp32
    GELU lies within a few fp32 ulps of a rounding tie of the element type (f16 x = -1.4853515625:
    exact GELU -0.1020813206, the f16 midpoint -0.1020812988); 1 + erf(x / sqrt 2) cancels there, and
    torch's own F.gelu on the GPU lands on either side of the tie depending on the element's
    position in its vectorised loop."""
    ulps = _ulps16(out, exp)
    n_diff = int((ulps != 0).sum())
    print(f"{what}: {n_diff} of {out.numel()} elements differ from torch (max {int(ulps.max())} ulp)", flush=True)
    assert int(ulps.max()) <= 1, what
    assert n_diff <= max(4, out.numel() // 100000), what


def test_gate_up_activation_every_value(gpu):
    """Every finite f16 / bf16 value through ak_mlp_gate_up's SiLU and GELU (the epilogue's lookup
    tables): with x the [256, 256] identity, gate[m, n] = W_gate[n, m] exactly and up = 1 (W_up all
    ones), so h holds act(value) rounded once. Against torch's own F.silu / F.gelu of the same
    values on the GPU under _gelu_matches_torch's rule."""
    from autokernel_amd.kernels.fused_mlp import gate_up
    F = torch.nn.functional
    for dt in (torch.float16, torch.bfloat16):
        vals = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(dt)
        vals = vals[torch.isfinite(vals)]
        N = vals.numel() // 256
        W = vals.view(N, 256).to(gpu)
        x = torch.eye(256, dtype=dt, device=gpu)
        ones = torch.ones(N, 256, dtype=dt, device=gpu)
        Wt = W.t().contiguous()
        for act, ref in (("silu", F.silu), ("gelu", F.gelu)):
            h = gate_up(x, W, ones, act)
            _gelu_matches_torch(h, ref(Wt), f"every {dt} value through the gate/up {act}")


@pytest.mark.parametrize("M,N,K", [(2048, 3072, 768), (8 * 512, 768, 3072), (300, 520, 200), (257, 77, 96),
                                   (2048, 768, 3072)])
def test_gemm_bias_gelu_and_residual_epilogues(gpu, M, N, K):
    """ak_gemm_bias_gelu and ak_gemm_bias_residual (GPT-2 / BERT MLP and output-projection shapes, an
    unaligned N that takes the register-staged path), f16 and bf16: ak_gemm_bias followed by torch's
    own F.gelu on the GPU to within the rounding-tie rule of _gelu_matches_torch, the residual form
    bit-equal to ak_gemm_bias plus torch's add (the rounding points of a biased nn.Linear, nn.GELU
    and `x + y`), and the GELU form within the harness's matmul tolerance (f16 1e-2, bf16 2e-2,
    bench.py:330-337) of the oracle's fp32 product + bias, rounded, through exact GELU in fp32."""
    from autokernel_amd.kernels.matmul import gemm_bias, gemm_bias_gelu, gemm_bias_residual
    F = torch.nn.functional
    for dt in (torch.float16, torch.bfloat16):
        g = torch.Generator().manual_seed(M * 3 + N + K)
        x = torch.randn(M, K, generator=g).to(dt)
        W = (torch.randn(N, K, generator=g) * 0.05).to(dt)
        b = (torch.randn(N, generator=g) * 0.5).to(dt)
        r = torch.randn(M, N, generator=g).to(dt)
        xd, Wd, bd, rd = x.to(gpu), W.to(gpu), b.to(gpu), r.to(gpu)
        lin = gemm_bias(xd, Wd.t(), bd)
        out = gemm_bias_gelu(xd, Wd.t(), bd)
        _gelu_matches_torch(out, F.gelu(lin), f"gelu epilogue {M}x{N}x{K} {dt}")
        exp = F.gelu((R.matmul_ref(x.float(), W.float().T) + b.float()).to(dt).float()).to(dt)
        tol = spec.KERNEL_CONFIGS["matmul"]["tolerances"][dt]
        assert_close(out, exp, tol["atol"], tol["rtol"], f"gemm_bias_gelu vs oracle {M}x{N}x{K} {dt}")
        res = gemm_bias_residual(xd, Wd.t(), bd, rd)
        assert torch.equal(res, rd + lin), f"residual epilogue {M}x{N}x{K} {dt}"
        print(f"gemm bias+residual {M}x{N}x{K} {dt}: bit-equal", flush=True)


def test_gemm_bias_gelu_every_value(gpu):
    """Every finite f16 / bf16 value through ak_gemm_bias_gelu once: with A the [256, 256] identity
    and a zero bias, C[m, n] = W[n, m] exactly, so W [N, 256] holding all finite values feeds each
    to the epilogue. Matches F.gelu of the same values under _gelu_matches_torch's rule: the fp32
    GELU is rounded like torch's (fp32 first, then the element type, never once from the exact
    product), which keeps every value whose fp32 GELU is not within a few ulps of a tie bit-equal."""
    from autokernel_amd.kernels.matmul import gemm_bias_gelu
    for dt in (torch.float16, torch.bfloat16):
        vals = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).view(dt)
        vals = vals[torch.isfinite(vals)]
        N = vals.numel() // 256
        assert N * 256 == vals.numel(), (dt, vals.numel())
        W = vals.view(N, 256).to(gpu)
        A = torch.eye(256, dtype=dt, device=gpu)
        out = gemm_bias_gelu(A, W.t(), torch.zeros(N, dtype=dt, device=gpu))
        exp = torch.nn.functional.gelu(W.t().contiguous())
        _gelu_matches_torch(out, exp, f"every {dt} value through the GELU epilogue")

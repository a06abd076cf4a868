"""Op specification table: sizes, dtypes, tolerances, work counts and seeded input generators.

Restates the reference harness's KERNEL_CONFIGS (bench.py:330-597) and gen_* generators
(bench.py:203-276) so the harness, tests and benchmark share one table, plus the BASELINE
workload configurations. Inputs are generated on the CPU with a seeded torch.Generator and then
moved to the target device, so a CPU check and the GPU kernel see identical bits (the reference
seeds the device RNG instead; distributions and shapes are the same).
"""
from __future__ import annotations

import math
from typing import Any, Callable, Dict, List, Tuple

import torch

Size = Dict[str, int]


def _bytes(dt: torch.dtype) -> int:
    return torch.tensor([], dtype=dt).element_size()


def _randn(shape, dtype, gen, device, scale: float = 1.0, mean: float = 0.0) -> torch.Tensor:
    t = torch.randn(*shape, generator=gen, dtype=torch.float32)
    if scale != 1.0:
        t = t * scale
    if mean != 0.0:
        t = t + mean
    return t.to(dtype).to(device)


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


# ---------------------------------------------------------------- generators (bench.py:203-276)
def gen_matmul(size: Size, dtype, device="cpu", seed=42) -> dict:
    g = _gen(seed)
    return {"A": _randn((size["M"], size["K"]), dtype, g, device),
            "B": _randn((size["K"], size["N"]), dtype, g, device)}


def gen_softmax(size: Size, dtype, device="cpu", seed=42) -> dict:
    return {"x": _randn((size["rows"], size["cols"]), dtype, _gen(seed), device)}


def gen_layernorm(size: Size, dtype, device="cpu", seed=42) -> dict:
    b, d = size["batch"], size["dim"]
    return {"x": _randn((b, d), dtype, _gen(seed), device),
            "weight": torch.ones(d, dtype=dtype, device=device),
            "bias": torch.zeros(d, dtype=dtype, device=device)}


def gen_flash_attention(size: Size, dtype, device="cpu", seed=42) -> dict:
    g = _gen(seed)
    shp = (size["batch"], size["heads"], size["seq_len"], size["head_dim"])
    return {"Q": _randn(shp, dtype, g, device), "K": _randn(shp, dtype, g, device),
            "V": _randn(shp, dtype, g, device)}


def gen_fused_mlp(size: Size, dtype, device="cpu", seed=42) -> dict:
    g = _gen(seed)
    b, d, h = size["batch"], size["dim"], size["hidden"]
    return {"x": _randn((b, d), dtype, g, device),
            "w_gate": _randn((h, d), dtype, g, device, 0.02),
            "w_up": _randn((h, d), dtype, g, device, 0.02),
            "w_down": _randn((d, h), dtype, g, device, 0.02)}


def gen_cross_entropy(size: Size, dtype, device="cpu", seed=42) -> dict:
    g = _gen(seed)
    b, v = size["batch"], size["vocab"]
    logits = _randn((b, v), dtype, g, device)
    targets = torch.randint(0, v, (b,), generator=g, dtype=torch.long).to(device)
    return {"logits": logits, "targets": targets}


def gen_rotary_embedding(size: Size, dtype, device="cpu", seed=42) -> dict:
    g = _gen(seed)
    b, h, s, d = size["batch"], size["heads"], size["seq_len"], size["head_dim"]
    return {"x": _randn((b, h, s, d), dtype, g, device),
            "cos": _randn((s, d // 2), dtype, g, device),
            "sin": _randn((s, d // 2), dtype, g, device)}


def gen_rmsnorm(size: Size, dtype, device="cpu", seed=42) -> dict:
    g = _gen(seed)
    return {"x": _randn((size["M"], size["N"]), dtype, g, device),
            "weight": _randn((size["N"],), dtype, g, device)}


def gen_reduce(size: Size, dtype, device="cpu", seed=42) -> dict:
    return {"x": _randn((size["M"], size["N"]), dtype, _gen(seed), device)}


F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


def _tol(f16, bf16, f32=None):
    t = {F16: {"atol": f16, "rtol": f16}, BF16: {"atol": bf16[0], "rtol": bf16[1]}}
    if f32 is not None:
        t[F32] = {"atol": f32, "rtol": f32}
    return t


# ------------------------------------------------------------ KERNEL_CONFIGS (bench.py:330-597)
KERNEL_CONFIGS: Dict[str, Dict[str, Any]] = {
    "matmul": {
        "test_sizes": [("tiny", {"M": 128, "N": 128, "K": 128}), ("small", {"M": 512, "N": 512, "K": 512}),
                       ("medium", {"M": 1024, "N": 1024, "K": 1024}), ("large", {"M": 2048, "N": 2048, "K": 2048}),
                       ("xlarge", {"M": 4096, "N": 4096, "K": 4096}), ("tall", {"M": 8192, "N": 1024, "K": 1024}),
                       ("wide", {"M": 1024, "N": 8192, "K": 1024}), ("deep_k", {"M": 1024, "N": 1024, "K": 8192}),
                       ("llm_qkv", {"M": 4096, "N": 4096, "K": 512}), ("llm_mlp", {"M": 4096, "N": 11008, "K": 4096})],
        "test_dtypes": [F16, BF16, F32],
        "tolerances": _tol(1e-2, (2e-2, 2e-2), 1e-4),
        "flops_fn": lambda s: 2 * s["M"] * s["N"] * s["K"],
        "bytes_fn": lambda s, dt: (s["M"] * s["K"] + s["K"] * s["N"] + s["M"] * s["N"]) * _bytes(dt),
        "input_generator": gen_matmul,
        "edge_sizes": [("edge_1023", {"M": 1023, "N": 1023, "K": 1023}), ("edge_4097", {"M": 4097, "N": 4097, "K": 512}),
                       ("edge_1537", {"M": 1537, "N": 1537, "K": 1537})],
        "bound": "mfma",
    },
    "softmax": {
        "test_sizes": [("tiny", {"rows": 32, "cols": 128}), ("small", {"rows": 256, "cols": 512}),
                       ("medium", {"rows": 1024, "cols": 1024}), ("large", {"rows": 4096, "cols": 4096}),
                       ("xlarge", {"rows": 8192, "cols": 8192}), ("wide", {"rows": 1024, "cols": 32768}),
                       ("narrow", {"rows": 32768, "cols": 128}), ("vocab", {"rows": 4096, "cols": 50257})],
        "test_dtypes": [F16, BF16, F32],
        "tolerances": _tol(1e-3, (2e-3, 2e-3), 1e-5),
        "flops_fn": lambda s: 5 * s["rows"] * s["cols"],
        "bytes_fn": lambda s, dt: 2 * s["rows"] * s["cols"] * _bytes(dt),
        "input_generator": gen_softmax,
        "edge_sizes": [("edge_1023", {"rows": 1023, "cols": 1023}), ("edge_4097", {"rows": 4097, "cols": 4097}),
                       ("edge_50257", {"rows": 1024, "cols": 50257})],
        "bound": "hbm",
    },
    "layernorm": {
        "test_sizes": [("tiny", {"batch": 32, "dim": 128}), ("small", {"batch": 256, "dim": 512}),
                       ("medium", {"batch": 1024, "dim": 1024}), ("large", {"batch": 4096, "dim": 2048}),
                       ("xlarge", {"batch": 8192, "dim": 4096}), ("wide", {"batch": 1024, "dim": 8192}),
                       ("llm_7b", {"batch": 4096, "dim": 4096}), ("llm_13b", {"batch": 4096, "dim": 5120})],
        "test_dtypes": [F16, BF16, F32],
        "tolerances": _tol(1e-3, (2e-3, 2e-3), 1e-5),
        "flops_fn": lambda s: 8 * s["batch"] * s["dim"],
        "bytes_fn": lambda s, dt: (2 * s["batch"] * s["dim"] + 2 * s["dim"]) * _bytes(dt),
        "input_generator": gen_layernorm,
        "edge_sizes": [("edge_1023", {"batch": 1023, "dim": 1023}), ("edge_4097", {"batch": 4097, "dim": 4097})],
        "bound": "hbm",
    },
    "flash_attention": {
        "test_sizes": [("tiny", {"batch": 1, "heads": 4, "seq_len": 64, "head_dim": 64}),
                       ("small", {"batch": 2, "heads": 8, "seq_len": 256, "head_dim": 64}),
                       ("medium", {"batch": 2, "heads": 16, "seq_len": 512, "head_dim": 64}),
                       ("large", {"batch": 2, "heads": 32, "seq_len": 1024, "head_dim": 64}),
                       ("xlarge", {"batch": 2, "heads": 32, "seq_len": 2048, "head_dim": 64}),
                       ("long", {"batch": 1, "heads": 32, "seq_len": 4096, "head_dim": 64}),
                       ("gqa", {"batch": 2, "heads": 32, "seq_len": 1024, "head_dim": 128}),
                       ("llm_7b", {"batch": 1, "heads": 32, "seq_len": 2048, "head_dim": 128})],
        "test_dtypes": [F16, BF16],
        "tolerances": _tol(1e-2, (2e-2, 2e-2), 1e-4),
        # the reference's nominal count (bench.py:446): 4*B*H*S^2*D, i.e. the non-causal work
        "flops_fn": lambda s: 4 * s["batch"] * s["heads"] * s["seq_len"] ** 2 * s["head_dim"],
        "bytes_fn": lambda s, dt: 4 * s["batch"] * s["heads"] * s["seq_len"] * s["head_dim"] * _bytes(dt),
        "input_generator": gen_flash_attention,
        "edge_sizes": [("edge_127", {"batch": 1, "heads": 8, "seq_len": 127, "head_dim": 64}),
                       ("edge_1023", {"batch": 1, "heads": 8, "seq_len": 1023, "head_dim": 64})],
        "bound": "mfma",
    },
    "fused_mlp": {
        "test_sizes": [("tiny", {"batch": 32, "dim": 128, "hidden": 256}),
                       ("small", {"batch": 256, "dim": 512, "hidden": 1024}),
                       ("medium", {"batch": 1024, "dim": 1024, "hidden": 2048}),
                       ("large", {"batch": 2048, "dim": 2048, "hidden": 5504}),
                       ("xlarge", {"batch": 4096, "dim": 4096, "hidden": 11008}),
                       ("llm_7b", {"batch": 2048, "dim": 4096, "hidden": 11008}),
                       ("llm_13b", {"batch": 2048, "dim": 5120, "hidden": 13824})],
        "test_dtypes": [F16, BF16, F32],
        "tolerances": _tol(1e-2, (2e-2, 2e-2), 1e-4),
        "flops_fn": lambda s: 2 * s["batch"] * s["dim"] * s["hidden"] * 3,
        "bytes_fn": lambda s, dt: (2 * s["batch"] * s["dim"] + 3 * s["hidden"] * s["dim"]) * _bytes(dt),
        "input_generator": gen_fused_mlp,
        "edge_sizes": [("edge_1023", {"batch": 1023, "dim": 1024, "hidden": 2048}),
                       ("edge_4097", {"batch": 4097, "dim": 512, "hidden": 1024})],
        "bound": "mfma",
    },
    "cross_entropy": {
        "test_sizes": [("tiny", {"batch": 32, "vocab": 256}), ("small", {"batch": 256, "vocab": 1024}),
                       ("medium", {"batch": 1024, "vocab": 4096}), ("large", {"batch": 4096, "vocab": 32000}),
                       ("xlarge", {"batch": 8192, "vocab": 50257}), ("llama", {"batch": 4096, "vocab": 32000}),
                       ("gpt2", {"batch": 4096, "vocab": 50257})],
        "test_dtypes": [F16, BF16, F32],
        "tolerances": _tol(1e-2, (2e-2, 2e-2), 1e-5),
        "flops_fn": lambda s: 4 * s["batch"] * s["vocab"],
        "bytes_fn": lambda s, dt: (s["batch"] * s["vocab"] + s["batch"]) * _bytes(dt),
        "input_generator": gen_cross_entropy,
        "edge_sizes": [("edge_1023", {"batch": 1023, "vocab": 32000}), ("edge_50257", {"batch": 4096, "vocab": 50257})],
        "bound": "hbm",
    },
    "rotary_embedding": {
        "test_sizes": [("tiny", {"batch": 1, "heads": 4, "seq_len": 64, "head_dim": 64}),
                       ("small", {"batch": 2, "heads": 8, "seq_len": 256, "head_dim": 64}),
                       ("medium", {"batch": 2, "heads": 16, "seq_len": 512, "head_dim": 64}),
                       ("large", {"batch": 2, "heads": 32, "seq_len": 1024, "head_dim": 128}),
                       ("xlarge", {"batch": 2, "heads": 32, "seq_len": 2048, "head_dim": 128}),
                       ("llm_7b", {"batch": 1, "heads": 32, "seq_len": 2048, "head_dim": 128}),
                       ("llm_13b", {"batch": 1, "heads": 40, "seq_len": 2048, "head_dim": 128})],
        "test_dtypes": [F16, BF16, F32],
        "tolerances": _tol(1e-3, (2e-3, 2e-3), 1e-5),
        "flops_fn": lambda s: 6 * s["batch"] * s["heads"] * s["seq_len"] * s["head_dim"],
        "bytes_fn": lambda s, dt: (2 * s["batch"] * s["heads"] * s["seq_len"] * s["head_dim"]
                                   + s["seq_len"] * s["head_dim"]) * _bytes(dt),
        "input_generator": gen_rotary_embedding,
        "edge_sizes": [("edge_127", {"batch": 1, "heads": 8, "seq_len": 127, "head_dim": 64}),
                       ("edge_1023", {"batch": 1, "heads": 8, "seq_len": 1023, "head_dim": 128})],
        "bound": "hbm",
    },
    "rmsnorm": {
        "test_sizes": [("small", {"M": 1024, "N": 768}), ("medium", {"M": 4096, "N": 1024}),
                       ("large", {"M": 4096, "N": 4096}), ("llama", {"M": 2048, "N": 4096})],
        "test_dtypes": [F16, BF16],
        "tolerances": _tol(1e-2, (1e-1, 5e-2)),
        "flops_fn": lambda s: 6 * s["M"] * s["N"],
        "bytes_fn": lambda s, dt: (2 * s["M"] * s["N"] + s["N"]) * _bytes(dt),
        "input_generator": gen_rmsnorm,
        "edge_sizes": [("edge_1023", {"M": 1023, "N": 768}), ("edge_4097", {"M": 4097, "N": 1024})],
        "bound": "hbm",
    },
    "reduce": {
        "test_sizes": [("small", {"M": 1024, "N": 1024}), ("medium", {"M": 4096, "N": 4096}),
                       ("large", {"M": 8192, "N": 8192}), ("wide", {"M": 1024, "N": 32768})],
        "test_dtypes": [F16, BF16],
        "tolerances": _tol(1e-2, (1e-1, 5e-2)),
        "flops_fn": lambda s: s["M"] * s["N"],
        "bytes_fn": lambda s, dt: (s["M"] * s["N"] + s["M"]) * _bytes(dt),
        "input_generator": gen_reduce,
        "edge_sizes": [("edge_1023", {"M": 1023, "N": 1024}), ("edge_4097", {"M": 4096, "N": 4097})],
        "bound": "hbm",
    },
}

# kwargs each kernel_fn is called with (keys of the generator dicts, bench.py:672)
ADVERSARIAL = [  # bench.py:808-816, applied to every floating-point input tensor
    ("near_max", lambda t, g: t * 60000.0 if t.dtype == torch.float16 else t * 1e30),
    ("near_zero", lambda t, g: t * 1e-6),
    ("mixed_scale", lambda t, g: t * torch.where(
        torch.rand(t.shape, generator=g).to(t.dtype).to(t.device) > 0.5,
        torch.tensor(1e3, dtype=t.dtype, device=t.device), torch.tensor(1e-3, dtype=t.dtype, device=t.device))),
    ("all_zeros", lambda t, g: torch.zeros_like(t)),
    ("all_same", lambda t, g: torch.ones_like(t) * 0.5),
]


def adversarial_inputs(inputs: dict, case: str, seed: int = 7) -> dict:
    """Apply one of the reference's stage-3 transforms to every float tensor of `inputs`."""
    fn = dict(ADVERSARIAL)[case]
    g = _gen(seed)
    return {k: (fn(v, g) if isinstance(v, torch.Tensor) and v.is_floating_point() else v)
            for k, v in inputs.items()}


def stage_size(cfg: dict) -> Size:
    """The 'small' size (or sizes[1]) used by the reference's stages 3 and 4 (bench.py:798-805)."""
    for label, sz in cfg["test_sizes"]:
        if label == "small":
            return sz
    return cfg["test_sizes"][min(1, len(cfg["test_sizes"]) - 1)][1]


def primary_size(cfg: dict) -> Tuple[str, Size]:
    """The 'large' size, else the last one (bench.py:1032-1041)."""
    for label, sz in cfg["test_sizes"]:
        if label == "large":
            return label, sz
    return cfg["test_sizes"][-1]


# ------------------------------------------------------------------------- BASELINE workloads
def rope_tables(seq: int, head_dim: int, theta: float = 10000.0, dtype=F16, device="cpu"):
    """cos / sin [seq, head_dim/2] for positions 0..seq-1, computed in fp32 then cast."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ang = torch.outer(torch.arange(seq, dtype=torch.float32), inv)
    return ang.cos().to(dtype).to(device), ang.sin().to(dtype).to(device)


def baseline_rmsnorm(device="cpu", seed=0, M=4096, N=4096) -> dict:
    """C1: x f16 [4096, 4096] ~N(0,1), weight ~N(1, 0.02), eps 1e-6, seed 0."""
    g = _gen(seed)
    return {"x": _randn((M, N), F16, g, device), "weight": _randn((N,), F16, g, device, 0.02, 1.0)}


def baseline_rope(device="cpu", seed=0, B=1, H=32, S=2048, D=128) -> dict:
    """C2a: q, k f16 [1, 32, 2048, 128] ~N(0,1), cos / sin from theta 10000 at positions 0..2047."""
    g = _gen(seed)
    cos, sin = rope_tables(S, D, device=device)
    return {"q": _randn((B, H, S, D), F16, g, device), "k": _randn((B, H, S, D), F16, g, device),
            "cos": cos, "sin": sin}


def baseline_softmax(device="cpu", seed=0, R=8192, C=8192) -> dict:
    """C2b: x f16 [8192, 8192] ~N(0, 3) (standard deviation 3)."""
    return {"x": _randn((R, C), F16, _gen(seed), device, 3.0)}


def baseline_matmul(device="cpu", seed=0, M=4096, N=4096, K=4096) -> dict:
    """C3a: A, B bf16 [4096, 4096] ~N(0,1)/sqrt(K)."""
    g = _gen(seed)
    s = 1.0 / math.sqrt(K)
    return {"A": _randn((M, K), BF16, g, device, s), "B": _randn((K, N), BF16, g, device, s)}


def baseline_fused_mlp(device="cpu", seed=0, M=2048, D=4096, H=11008) -> dict:
    """C3b: x bf16 [2048, 4096] ~N(0,1); w_gate, w_up [11008, 4096], w_down [4096, 11008] ~N(0, 0.02)
    (nn.Linear layout, the transposes of the shapes BASELINE.json lists)."""
    g = _gen(seed)
    return {"x": _randn((M, D), BF16, g, device), "w_gate": _randn((H, D), BF16, g, device, 0.02),
            "w_up": _randn((H, D), BF16, g, device, 0.02), "w_down": _randn((D, H), BF16, g, device, 0.02)}


def baseline_attention(device="cpu", seed=0, B=4, H=32, S=2048, D=128) -> dict:
    """C4: Q, K, V f16 [4, 32, 2048, 128] (or [1, 32, 8192, 128]) ~N(0,1), causal, scale D^-0.5."""
    g = _gen(seed)
    return {k: _randn((B, H, S, D), F16, g, device) for k in ("Q", "K", "V")}


def attention_causal_flops(B: int, H: int, S: int, D: int) -> int:
    """Algorithmic flops of causal attention: 2 GEMMs over the S(S+1)/2 visible pairs."""
    return 2 * 2 * B * H * D * (S * (S + 1) // 2)

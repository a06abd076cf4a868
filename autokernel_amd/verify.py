"""Model plug-in verifier: the role of the reference's verify.py.

    python -m autokernel_amd.verify [--model 7b|small|path/to/model.py --class-name C]
        [--input-shape 1,2048] [--dtype float16] [--kernels all|matmul,rmsnorm,...]
        [--workspace DIR | --kernel-module path/to/kernel_x.py ...]
        [--atol 1e-2 --rtol 1e-2] [--diagnose] [--json out.json]

--workspace / --kernel-module plug in any module that defines kernel_fn (and KERNEL_TYPE), found
the reference's way (verify.py:322-405): DIR/orchestration_state.json first, else every
DIR/kernel_<type>_<rank>_optimized.py; each is imported by path and its kernel_fn replaces the
matching modules (verify.py:510-641).

Runs the stock forward, swaps modules for libak355-backed wrappers, reruns, compares the outputs
(verify.py:687-765 semantics) and times both (10 warm-up, 50 timed, median; verify.py:258-307).

Replacement strategies (the reference has matmul, layernorm and rmsnorm, verify.py:557-637;
rotary embedding, attention and the SwiGLU MLP are added here):
  matmul            every nn.Linear -> x @ W.T through ak_gemm reading W in place (no per-call
                    weight.t().contiguous() copy, verify.py:429); inside attention one fused
                    QKV GEMM
  layernorm         nn.LayerNorm -> ak_layernorm
  rmsnorm           RMSNorm-like modules (by class name, or weight + eps, no bias, "...norm") ->
                    ak_rmsnorm_rsqrt for class RMSNorm (the model's rsqrt form), else ak_rmsnorm
  rotary_embedding  inside attention: RoPE through ak_rope_f32_tables, or (with matmul, f16 / bf16)
                    in the epilogue of the fused QKV GEMM (ak_gemm_rope)
  flash_attention   attention modules (wq / wk / wv / wo, n_heads, n_kv_heads) -> GQA-native
                    ak_flash_attn_fwd on strided [B, T, H, D] views (no repeat_interleave, no
                    transpose copies); encoder attention (query / key / value / out_proj,
                    num_heads: BERT) -> the non-causal kernel when no attention_mask is given;
                    fused-QKV causal attention (c_attn / c_proj, n_head, a tril mask: GPT-2)
                    -> the causal kernel on column slices of the c_attn output
  fused_mlp         SwiGLU feed-forward modules (w1 gate, w3 up, w2 down) -> ak_mlp_gate_up + ak_gemm
  (with matmul)     pre-norm blocks (attention, feed_forward, attention_norm, ffn_norm) whose
                    attention and feed-forward are swapped: each residual add runs in the epilogue
                    of the GEMM that ends its branch (ak_gemm_residual), f16 / bf16
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
from dataclasses import dataclass
from typing import Any, Callable, Dict, Iterable, List, Optional, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels
from .kernels import flash_attention as fa_mod
from .kernels import rotary_embedding as rope_mod
from .kernels.fused_mlp import gate_up
from .kernels.matmul import gemm, gemm_bias, gemm_bias_gelu, gemm_bias_residual, gemm_residual, gemm_rope
from .kernels.rmsnorm import rms_norm_rsqrt

ALL_KERNELS = ("matmul", "rmsnorm", "layernorm", "rotary_embedding", "flash_attention", "fused_mlp")
WARMUP_RUNS = 10
TIMED_RUNS = 50
DEFAULT_TOLERANCES = {  # verify.py:51-55 (the north star asks 1e-2 for f16 / bf16 end to end)
    torch.float16: {"atol": 1e-3, "rtol": 1e-3},
    torch.bfloat16: {"atol": 2e-3, "rtol": 2e-3},
    torch.float32: {"atol": 1e-5, "rtol": 1e-5},
}
RMSNORM_NAMES = {"RMSNorm", "LlamaRMSNorm", "T5LayerNorm", "GemmaRMSNorm"}


# ------------------------------------------------------------------ external kernel modules
@dataclass
class KernelReplacement:
    """One kernel module to plug in (verify.py:62-69): its op type, profiling rank, measured
    speedup, the .py path, and, once loaded, its kernel_fn."""
    kernel_type: str
    rank: int = 0
    speedup: float = 0.0
    optimized_path: str = ""
    module_fn: Optional[Callable] = None


def discover_optimized_kernels(workspace: str) -> List[KernelReplacement]:
    """Kernel modules under `workspace`, found as verify.py:322-395 finds them.

    1. workspace/orchestration_state.json: each entry of "kernels" (op_type or type, rank, speedup
       or best_speedup) names optimized_path, else <stem of its "file">_optimized.py, else
       kernel_<type>_<rank>_optimized.py; kept when the file exists and the speedup is above 1.
    2. Otherwise every kernel_<type>_<rank>_optimized.py, sorted by name; the type may contain
       underscores (flash_attention) and the rank is its last all-digit part (speedup unknown: 0).
    """
    found: List[KernelReplacement] = []
    state_path = os.path.join(workspace, "orchestration_state.json")
    if os.path.exists(state_path):
        with open(state_path) as f:
            state = json.load(f)
        if isinstance(state, dict) and "kernels" in state:
            for k in state["kernels"]:
                ktype = k.get("op_type", k.get("type", "unknown"))
                rank = int(k.get("rank", 0))
                speedup = float(k.get("speedup", k.get("best_speedup", 1.0)))
                path = k.get("optimized_path", "")
                if not path:
                    base = k.get("file", "")
                    stem = os.path.splitext(os.path.basename(base))[0] if base else f"kernel_{ktype}_{rank}"
                    path = os.path.join(workspace, f"{stem}_optimized.py")
                if os.path.exists(path) and speedup > 1.0:
                    found.append(KernelReplacement(ktype, rank, speedup, path))
            return found
    if not os.path.isdir(workspace):
        return found
    for fname in sorted(os.listdir(workspace)):
        if not (fname.startswith("kernel_") and fname.endswith("_optimized.py")):
            continue
        parts = fname[: -len("_optimized.py")].split("_")
        if len(parts) < 3:
            continue
        rank, cut = 0, len(parts)
        for i in range(len(parts) - 1, 0, -1):
            if parts[i].isdigit():
                rank, cut = int(parts[i]), i
                break
        ktype = "_".join(parts[1:cut]) if cut > 1 else parts[1]
        found.append(KernelReplacement(ktype, rank, 0.0, os.path.join(workspace, fname)))
    return found


def load_kernel_module(path: str):
    """Import a kernel .py file by path (verify.py:398-405); it must define kernel_fn."""
    path = os.path.abspath(path)
    name = "ak_user_kernel_" + os.path.splitext(os.path.basename(path))[0]
    spec_ = importlib.util.spec_from_file_location(name, path)
    if spec_ is None or spec_.loader is None:
        raise ImportError(f"cannot load a kernel module from {path}")
    mod = importlib.util.module_from_spec(spec_)
    spec_.loader.exec_module(mod)
    if not callable(getattr(mod, "kernel_fn", None)):
        raise ImportError(f"{path} defines no kernel_fn")
    return mod


def replacement_from_module(path: str) -> KernelReplacement:
    """A replacement for one module file: its KERNEL_TYPE, else the type in its file name."""
    mod = load_kernel_module(path)
    ktype = getattr(mod, "KERNEL_TYPE", None)
    if not ktype:
        found = discover_optimized_kernels(os.path.dirname(os.path.abspath(path)))
        match = [r for r in found if os.path.samefile(r.optimized_path, path)]
        if not match:
            raise ValueError(f"{path}: no KERNEL_TYPE and no kernel_<type>_<rank>_optimized.py name")
        ktype = match[0].kernel_type
    return KernelReplacement(ktype, 0, 0.0, os.path.abspath(path), mod.kernel_fn)


class ModuleLinearWrapper(nn.Module):
    """nn.Linear through an external matmul kernel_fn called as the reference calls it
    (verify.py:408-438): kernel_fn(x_2d, weight.t().contiguous()), then + bias."""

    def __init__(self, original: nn.Linear, fn: Callable):
        super().__init__()
        self.original, self.kernel_fn = original, fn
        self.weight, self.bias = original.weight, original.bias

    def forward(self, x):
        x2 = x.reshape(-1, x.shape[-1])
        out = self.kernel_fn(x2, self.weight.t().contiguous())
        if self.bias is not None:
            out = out + self.bias
        return out.reshape(*x.shape[:-1], out.shape[-1])


class ModuleLayerNormWrapper(nn.Module):
    """nn.LayerNorm through an external kernel_fn: (x, w, b, eps), else (x, w, b), else (x) on
    TypeError (verify.py:441-474)."""

    def __init__(self, original: nn.LayerNorm, fn: Callable):
        super().__init__()
        self.original, self.kernel_fn = original, fn
        self.weight, self.bias, self.eps = original.weight, original.bias, original.eps

    def forward(self, x):
        x2 = x.reshape(-1, x.shape[-1])
        try:
            out = self.kernel_fn(x2, self.weight, self.bias, self.eps)
        except TypeError:
            try:
                out = self.kernel_fn(x2, self.weight, self.bias)
            except TypeError:
                out = self.kernel_fn(x2)
        return out.reshape(x.shape)


class ModuleRMSNormWrapper(nn.Module):
    """RMSNorm-like module through an external kernel_fn: (x, w, eps), else (x, w) on TypeError;
    (x) when the module has no weight (verify.py:477-507)."""

    def __init__(self, original: nn.Module, fn: Callable):
        super().__init__()
        self.original, self.kernel_fn = original, fn
        self.weight = getattr(original, "weight", None)
        self.eps = getattr(original, "eps", 1e-6)

    def forward(self, x):
        x2 = x.reshape(-1, x.shape[-1])
        if self.weight is None:
            out = self.kernel_fn(x2)
        else:
            try:
                out = self.kernel_fn(x2, self.weight, self.eps)
            except TypeError:
                out = self.kernel_fn(x2, self.weight)
        return out.reshape(x.shape)


MODULE_WRAPPERS = {"matmul": ModuleLinearWrapper, "layernorm": ModuleLayerNormWrapper,
                   "rmsnorm": ModuleRMSNormWrapper}


# ------------------------------------------------------------------------------ wrappers
def _linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x @ W.T (+ bias) with W read in place; an f16 / bf16 bias is fused into the GEMM and
    rounded once with the product, as stock nn.Linear (addmm) rounds it."""
    x2 = x.reshape(-1, x.shape[-1])
    if bias is not None and bias.dtype == x.dtype and x.dtype in (torch.float16, torch.bfloat16):
        out = gemm_bias(x2, weight.t(), bias)
    else:
        out = gemm(x2, weight.t())
        if bias is not None:
            out = out + bias
    return out.view(*x.shape[:-1], weight.shape[0])


class LinearWrapper(nn.Module):
    """nn.Linear -> ak_gemm with the [out, in] weight read in place (b_trans = 1)."""

    def __init__(self, original: nn.Linear):
        super().__init__()
        self.original = original
        self.weight = original.weight
        self.bias = original.bias

    def forward(self, x):
        return _linear(x, self.weight, self.bias)


class LayerNormWrapper(nn.Module):
    def __init__(self, original: nn.LayerNorm):
        super().__init__()
        self.original = original
        self.weight, self.bias, self.eps = original.weight, original.bias, original.eps

    def forward(self, x):
        return kernels.get("layernorm")(x, self.weight, self.bias, self.eps)


class RMSNormWrapper(nn.Module):
    """RMSNorm-like module -> libak355. A module of class `RMSNorm` computes
    x * rsqrt(mean(x^2) + eps) * w (the reference's models/llama_7b.py:28-30 and llama.py), which
    ak_rmsnorm_rsqrt reproduces op for op; other classes get reference.py's form (kernel_fn)."""

    def __init__(self, original: nn.Module):
        super().__init__()
        self.original = original
        self.weight = getattr(original, "weight", None)
        self.eps = getattr(original, "eps", 1e-6)
        self.model_form = type(original).__name__ == "RMSNorm"

    def forward(self, x):
        w = self.weight if self.weight is not None else torch.ones(x.shape[-1], device=x.device, dtype=x.dtype)
        if self.model_form:
            return rms_norm_rsqrt(x, w, self.eps)
        return kernels.get("rmsnorm")(x, w, self.eps)


class FeedForwardWrapper(nn.Module):
    """w2(silu(w1 x) * w3 x) -> fused gate/up kernel + down GEMM."""

    def __init__(self, original: nn.Module, gate: nn.Linear, up: nn.Linear, down: nn.Linear):
        super().__init__()
        self.original = original
        self.gate, self.up, self.down = gate, up, down

    def forward(self, x, residual: Optional[torch.Tensor] = None):
        if residual is None or not _fusable(residual):
            y = kernels.get("fused_mlp")(x, self.gate.weight, self.up.weight, self.down.weight, "silu")
            return y if residual is None else residual + y
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        h = gate_up(x2, self.gate.weight, self.up.weight, "silu")
        y = gemm_residual(h, self.down.weight.t(), residual.reshape(-1, residual.shape[-1]))
        return y.view(residual.shape)


def _fusable(residual: torch.Tensor) -> bool:
    """ak_gemm_residual serves f16 / bf16 (fp32 keeps the separate add)."""
    return residual.dtype in (torch.float16, torch.bfloat16)


def _identity_dropout(d) -> bool:
    """A missing dropout, or one that passes its input through (eval mode or p = 0)."""
    return not isinstance(d, nn.Dropout) or not d.training or d.p == 0


def _bias_fusable(lin: nn.Linear, x: torch.Tensor) -> bool:
    """The biased-GEMM epilogues serve an f16 / bf16 Linear whose bias has the input's dtype."""
    return _fusable(x) and lin.bias is not None and lin.bias.dtype == x.dtype and lin.weight.dtype == x.dtype


def _linear_residual(x: torch.Tensor, lin: nn.Linear, residual: Optional[torch.Tensor]) -> torch.Tensor:
    """residual + lin(x), the add carried by the GEMM's epilogue where the dtypes allow: the
    product (+ bias) is rounded, then the sum, as the separate add rounds it."""
    if residual is None:
        return _linear(x, lin.weight, lin.bias)
    x2 = x.reshape(-1, x.shape[-1])
    r2 = residual.reshape(-1, residual.shape[-1])
    if _bias_fusable(lin, x):
        return gemm_bias_residual(x2, lin.weight.t(), lin.bias, r2).view(residual.shape)
    if lin.bias is None and _fusable(x):
        return gemm_residual(x2, lin.weight.t(), r2).view(residual.shape)
    return residual + _linear(x, lin.weight, lin.bias)


class GeluMLPWrapper(nn.Module):
    """proj(gelu(fc(x))) (+ dropout), the two-Linear GELU MLP of the reference's GPT-2 (c_fc / c_proj,
    models/gpt2.py:55-68) and BERT (dense1 / dense2, models/bert_base.py:43-53), in two GEMM launches:
    fc's bias and the exact (erf) GELU in the first GEMM's epilogue, proj's bias (and a caller's
    residual) in the second's. Each intermediate is rounded where the stock modules round it, so the
    output matches them bit for bit. Other dtypes, a tanh GELU or an active dropout take the
    unfused path (libak355 GEMMs, the module's own GELU and dropout)."""

    def __init__(self, original: nn.Module, fc: nn.Linear, gelu: nn.GELU, proj: nn.Linear):
        super().__init__()
        self.original = original
        self.fc, self.gelu, self.proj = fc, gelu, proj
        drops = [c for c in original.children() if isinstance(c, nn.Dropout)]
        self.drop = drops[0] if drops else None

    def forward(self, x, residual: Optional[torch.Tensor] = None):
        fc, proj = self.fc, self.proj
        if not (_bias_fusable(fc, x) and self.gelu.approximate == "none" and _identity_dropout(self.drop)):
            y = _linear(self.gelu(_linear(x, fc.weight, fc.bias)), proj.weight, proj.bias)
            y = self.drop(y) if self.drop is not None else y
            return y if residual is None else residual + y
        h = gemm_bias_gelu(x.reshape(-1, x.shape[-1]), fc.weight.t(), fc.bias)
        return _linear_residual(h.view(*x.shape[:-1], -1), proj, residual)


def _rope_tables_from(args) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos / sin from either (cos, sin) tensors or one complex freqs_cis tensor."""
    if len(args) >= 2 and not torch.is_complex(args[0]):
        return args[0], args[1]
    f = args[0]
    return f.real.float(), f.imag.float()


class AttentionWrapper(nn.Module):
    """GQA attention block (wq / wk / wv / wo) with libak355 RoPE and flash attention.

    use_rope / use_fa select which of the two replace the stock steps; the projections use
    ak_gemm when use_matmul is set.
    """

    def __init__(self, original: nn.Module, use_rope: bool, use_fa: bool, use_matmul: bool):
        super().__init__()
        self.original = original
        self.use_rope, self.use_fa, self.use_matmul = use_rope, use_fa, use_matmul
        o = original
        self.n_heads, self.n_kv_heads, self.head_dim = o.n_heads, o.n_kv_heads, o.head_dim
        # One [H*D + 2*Hk*D, dim] weight for the three projections: one GEMM instead of three, and
        # q / k / v are column slices of its output. It is a copy, rebuilt whenever a source weight
        # changes (in-place update, optimizer step, load_state_dict: tracked by version and storage).
        self.fused_qkv = use_matmul and all(getattr(o, n).bias is None for n in ("wq", "wk", "wv"))
        self._qkv_key = None
        self._w_qkv = None

    def _qkv_weight(self) -> Optional[torch.Tensor]:
        if not self.fused_qkv:
            return None
        o = self.original
        ws = (o.wq.weight, o.wk.weight, o.wv.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype, tuple(w.shape)) for w in ws)
        if key != self._qkv_key:
            with torch.no_grad():
                self._w_qkv = torch.cat(ws, 0).contiguous()
            self._qkv_key = key
        return self._w_qkv

    @property
    def w_qkv(self) -> Optional[torch.Tensor]:
        return self._qkv_weight()

    def _proj(self, lin: nn.Linear, x):
        return _linear(x, lin.weight, lin.bias) if self.use_matmul else lin(x)

    def _fp32_tables(self, cos: torch.Tensor, sin: torch.Tensor, T: int):
        """Contiguous fp32 cos / sin [T, D/2], converted once per source table and length (the
        model passes the same buffers to every layer and every call)."""
        key = (cos.data_ptr(), cos._version, sin.data_ptr(), sin._version, cos.dtype, T)
        cached = getattr(self, "_tab", None)
        if cached is None or cached[0] != key:
            self._tab = (key, cos[:T].float().contiguous(), sin[:T].float().contiguous())
        return self._tab[1], self._tab[2]

    def forward(self, x, *rope_args, residual: Optional[torch.Tensor] = None):
        o = self.original
        B, T, _ = x.shape
        H, Hk, D = self.n_heads, self.n_kv_heads, self.head_dim
        cos, sin = _rope_tables_from(rope_args)
        rotated = False
        w_qkv = self._qkv_weight()
        if w_qkv is not None:
            if self.use_rope and x.dtype in (torch.float16, torch.bfloat16) and D % 4 == 0:
                # q and k heads rotated in the projection's epilogue: no RoPE launch of their own
                c32, s32 = self._fp32_tables(cos, sin, T)
                qkv = gemm_rope(x.reshape(B * T, -1), w_qkv.t(), c32, s32, T, D, (H + Hk) * D)
                rotated = True
            else:
                qkv = gemm(x.reshape(B * T, -1), w_qkv.t())
            q = qkv[:, : H * D].view(B, T, H, D)
            k = qkv[:, H * D: (H + Hk) * D].view(B, T, Hk, D)
            v = qkv[:, (H + Hk) * D:].view(B, T, Hk, D)
        else:
            q = self._proj(o.wq, x).view(B, T, H, D)
            k = self._proj(o.wk, x).view(B, T, Hk, D)
            v = self._proj(o.wv, x).view(B, T, Hk, D)
        if self.use_rope and not rotated:
            c32, s32 = self._fp32_tables(cos, sin, T)
            if w_qkv is not None:
                # q and k heads are adjacent in each token's row of the fused output: one launch
                # rotates all H + Hk of them (the same per-element arithmetic as two calls)
                qk = rope_mod.apply_fp32_tables(qkv[:, : (H + Hk) * D].view(B, T, H + Hk, D), c32, s32)
                q, k = qk[:, :, :H], qk[:, :, H:]
            else:
                q = rope_mod.apply_fp32_tables(q, c32, s32)
                k = rope_mod.apply_fp32_tables(k, c32, s32)
        elif not self.use_rope:
            c, s = cos[:T].view(1, T, 1, -1), sin[:T].view(1, T, 1, -1)

            def rot(t):
                tf = t.float()
                a, b = tf[..., 0::2], tf[..., 1::2]
                return torch.stack((a * c - b * s, a * s + b * c), -1).flatten(-2).type_as(t)
            q, k = rot(q), rot(k)
        if self.use_fa:
            y = torch.empty((B, T, H, D), device=x.device, dtype=x.dtype)
            fa_mod.attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), True, None,
                             out=y.transpose(1, 2))
            y = y.view(B, T, H * D)
        else:
            qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
            if H != Hk:
                kh = kh.repeat_interleave(H // Hk, dim=1)
                vh = vh.repeat_interleave(H // Hk, dim=1)
            y = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True).transpose(1, 2).reshape(B, T, H * D)
        if residual is None:
            return self._proj(o.wo, y)
        if self.use_matmul and o.wo.bias is None and _fusable(residual):
            out = gemm_residual(y.reshape(B * T, H * D), o.wo.weight.t(), residual.reshape(B * T, -1))
            return out.view(residual.shape)
        return residual + self._proj(o.wo, y)


class EncoderAttentionWrapper(nn.Module):
    """Bidirectional self-attention with separate query / key / value / out_proj Linears and
    num_heads (the reference's BERT, models/bert_base.py:16-40): the projections through ak_gemm when
    matmul is swapped, attention through the non-causal flash-attention kernel on strided
    [B, T, H, D] views. A call with an attention_mask goes to the original module (the kernel takes
    no arbitrary mask)."""

    def __init__(self, original: nn.Module, use_matmul: bool):
        super().__init__()
        self.original = original
        self.use_matmul = use_matmul
        # query / key / value as one GEMM over a concatenated [3C, C] weight (and bias): q, k and v
        # are column slices of its output, read in place by the attention kernel. Each output
        # element is the same dot product in the same order as in three separate GEMMs. The copy
        # is rebuilt whenever a source weight or bias changes (tracked by version and storage).
        lins = (original.query, original.key, original.value)
        self.fused_qkv = use_matmul and len({l.bias is None for l in lins}) == 1
        self._qkv_key = None
        self._w_qkv = self._b_qkv = None

    def _qkv_params(self):
        o = self.original
        ps = [t for l in (o.query, o.key, o.value) for t in (l.weight, l.bias) if t is not None]
        key = tuple((t.data_ptr(), t._version, t.dtype, tuple(t.shape)) for t in ps)
        if key != self._qkv_key:
            with torch.no_grad():
                self._w_qkv = torch.cat([o.query.weight, o.key.weight, o.value.weight], 0).contiguous()
                self._b_qkv = None if o.query.bias is None else torch.cat(
                    [o.query.bias, o.key.bias, o.value.bias], 0).contiguous()
            self._qkv_key = key
        return self._w_qkv, self._b_qkv

    def forward(self, x, attention_mask=None, residual: Optional[torch.Tensor] = None):
        o = self.original
        if attention_mask is not None:
            out = o(x, attention_mask)
            return out if residual is None else residual + out
        B, T, C = x.shape
        H = o.num_heads
        D = C // H

        def proj(lin, t):
            return _linear(t, lin.weight, lin.bias) if self.use_matmul else lin(t)
        if self.fused_qkv:
            qkv = _linear(x, *self._qkv_params())
            q, k, v = (qkv[..., i * C:(i + 1) * C].view(B, T, H, D) for i in range(3))
        else:
            q, k, v = (proj(lin, x).view(B, T, H, D) for lin in (o.query, o.key, o.value))
        y = torch.empty((B, T, H, D), device=x.device, dtype=x.dtype)  # written in place, no transpose copy
        fa_mod.attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), False, None, out=y.transpose(1, 2))
        y = y.view(B, T, C)
        drop = getattr(o, "dropout", None)
        if residual is not None and self.use_matmul and _identity_dropout(drop):
            return _linear_residual(y, o.out_proj, residual)
        out = proj(o.out_proj, y)
        out = drop(out) if isinstance(drop, nn.Module) else out
        return out if residual is None else residual + out


class FusedQKVAttentionWrapper(nn.Module):
    """Causal self-attention with one fused c_attn Linear (3 * n_embd outputs) and a lower-triangular
    mask buffer (the reference's GPT-2, models/gpt2.py:18-54): c_attn and c_proj through ak_gemm when
    matmul is swapped; q, k and v read in place as column slices of the c_attn output by the causal
    flash-attention kernel (no split copies, no materialised T x T scores)."""

    def __init__(self, original: nn.Module, use_matmul: bool):
        super().__init__()
        self.original = original
        self.use_matmul = use_matmul

    def forward(self, x, residual: Optional[torch.Tensor] = None):
        o = self.original
        B, T, C = x.shape
        H = o.n_head
        D = C // H

        def proj(lin, t):
            return _linear(t, lin.weight, lin.bias) if self.use_matmul else lin(t)
        qkv = proj(o.c_attn, x)
        q, k, v = (qkv[..., i * C:(i + 1) * C].view(B, T, H, D).transpose(1, 2) for i in range(3))
        y = torch.empty((B, T, H, D), device=x.device, dtype=x.dtype)  # written in place, no transpose copy
        fa_mod.attention(q, k, v, True, None, out=y.transpose(1, 2))
        y = y.view(B, T, C)
        drop = getattr(o, "resid_dropout", None)
        if residual is not None and self.use_matmul and _identity_dropout(drop):
            return _linear_residual(y, o.c_proj, residual)
        out = proj(o.c_proj, y)
        out = drop(out) if isinstance(drop, nn.Module) else out
        return out if residual is None else residual + out


class ResidualBlockWrapper(nn.Module):
    """Pre-norm block x = x + attention(attention_norm(x)); x = x + feed_forward(ffn_norm(x))
    (models/llama_7b.py:109-112) whose attention and feed-forward are libak355 wrappers: each
    residual add is handed to the GEMM that ends its branch (the output projection, the down
    projection), so it costs no launch of its own and gives the same bits as the separate add."""

    def __init__(self, original: nn.Module):
        super().__init__()
        self.original = original

    def forward(self, x, *args):
        b = self.original
        h = b.attention(b.attention_norm(x), *args, residual=x)
        return b.feed_forward(b.ffn_norm(h), residual=h)


class GPT2BlockWrapper(nn.Module):
    """Pre-norm block x = x + attn(ln_1(x)); x = x + mlp(ln_2(x)) (models/gpt2.py:71-82) whose attn
    and mlp are libak355 wrappers: each residual add is carried by the epilogue of the GEMM that
    ends its branch (c_proj of the attention, c_proj of the MLP), bit for bit the separate add."""

    def __init__(self, original: nn.Module):
        super().__init__()
        self.original = original

    def forward(self, x):
        b = self.original
        h = b.attn(b.ln_1(x), residual=x)
        return b.mlp(b.ln_2(h), residual=h)


class PostNormBlockWrapper(nn.Module):
    """Post-norm block x = norm1(x + attention(x)); x = norm2(x + mlp(x)) (models/bert_base.py:56-66)
    whose attention and mlp are libak355 wrappers: each residual add is carried by the epilogue of
    the GEMM that ends its branch (out_proj, dense2), the norms by the layernorm strategy or stock."""

    def __init__(self, original: nn.Module):
        super().__init__()
        self.original = original

    def forward(self, x):
        b = self.original
        h = b.norm1(b.attention(x, residual=x))
        return b.norm2(b.mlp(h, residual=h))


def _is_prenorm_block(m: nn.Module) -> bool:
    return all(isinstance(getattr(m, n, None), nn.Module)
               for n in ("attention", "feed_forward", "attention_norm", "ffn_norm"))


def _is_gpt2_block(m: nn.Module) -> bool:
    return (all(isinstance(getattr(m, n, None), nn.Module) for n in ("ln_1", "attn", "ln_2", "mlp"))
            and isinstance(m.attn, FusedQKVAttentionWrapper) and m.attn.use_matmul
            and isinstance(m.mlp, GeluMLPWrapper))


def _is_postnorm_block(m: nn.Module) -> bool:
    return (all(isinstance(getattr(m, n, None), nn.Module) for n in ("attention", "norm1", "mlp", "norm2"))
            and not hasattr(m, "feed_forward") and isinstance(m.attention, EncoderAttentionWrapper)
            and m.attention.use_matmul and isinstance(m.mlp, GeluMLPWrapper))


def _gelu_mlp_parts(m: nn.Module):
    """(fc, gelu, proj) of a Linear -> GELU -> Linear MLP named as GPT-2's (c_fc, c_proj) or BERT's
    (dense1, dense2) with one nn.GELU child; None for anything else."""
    gelus = [c for c in m.children() if isinstance(c, nn.GELU)]
    if len(gelus) != 1:
        return None
    for a, b in (("c_fc", "c_proj"), ("dense1", "dense2")):
        fc, proj = getattr(m, a, None), getattr(m, b, None)
        if (isinstance(fc, nn.Linear) and isinstance(proj, nn.Linear) and fc.out_features == proj.in_features
                and fc.in_features == proj.out_features):
            return fc, gelus[0], proj
    return None


# ------------------------------------------------------------------------- module swapping
def _is_rmsnorm(m: nn.Module) -> bool:
    name = type(m).__name__
    return name in RMSNORM_NAMES or (hasattr(m, "weight") and hasattr(m, "eps") and not hasattr(m, "bias")
                                     and name.lower().endswith("norm") and not isinstance(m, nn.LayerNorm))


def _is_attention(m: nn.Module) -> bool:
    return all(hasattr(m, a) for a in ("wq", "wk", "wv", "wo", "n_heads", "n_kv_heads", "head_dim"))


def _is_fused_qkv_causal_attention(m: nn.Module) -> bool:
    """c_attn [3 C, C] / c_proj Linears, n_head, n_embd and a causal (lower-triangular ones) mask."""
    c_attn, c_proj = getattr(m, "c_attn", None), getattr(m, "c_proj", None)
    n_head, n_embd = getattr(m, "n_head", None), getattr(m, "n_embd", None)
    mask = getattr(m, "bias", None)
    if not (isinstance(c_attn, nn.Linear) and isinstance(c_proj, nn.Linear) and isinstance(n_head, int)
            and isinstance(n_embd, int) and isinstance(mask, torch.Tensor) and mask.dim() >= 2):
        return False
    if c_attn.out_features != 3 * n_embd or n_embd % n_head:
        return False
    sq = mask.reshape(-1, *mask.shape[-2:])[0]
    return sq.shape[0] == sq.shape[1] and bool(torch.equal(sq != 0, torch.ones_like(sq, dtype=torch.bool).tril()))


def _is_encoder_attention(m: nn.Module) -> bool:
    return (all(isinstance(getattr(m, a, None), nn.Linear) for a in ("query", "key", "value", "out_proj"))
            and isinstance(getattr(m, "num_heads", None), int))


def _swiglu_parts(m: nn.Module):
    for g, u, d in (("w1", "w3", "w2"), ("gate_proj", "up_proj", "down_proj")):
        if all(isinstance(getattr(m, a, None), nn.Linear) for a in (g, u, d)):
            return getattr(m, g), getattr(m, u), getattr(m, d)
    return None


class OptimizedModelContext:
    """Swap modules for libak355 wrappers on enter, restore them on exit (verify.py:510-641).

    kernel_types holds libak355 strategy names (ALL_KERNELS) and / or KernelReplacement entries
    (external kernel modules, e.g. from discover_optimized_kernels). An external module's
    kernel_fn replaces the modules of its type with the reference's call conventions (matmul,
    layernorm, rmsnorm, verify.py:557-637) and takes precedence over a libak355 strategy of the
    same type; other external types are skipped with a note, as the reference does."""

    def __init__(self, model: nn.Module, kernel_types: Iterable[Union[str, KernelReplacement]]):
        self.model = model
        items = list(kernel_types)
        self.external: Dict[str, KernelReplacement] = {}
        self.notes: List[str] = []
        for r in items:
            if not isinstance(r, KernelReplacement):
                continue
            if r.kernel_type not in MODULE_WRAPPERS:
                self.notes.append(f"no replacement strategy for kernel type '{r.kernel_type}' "
                                  f"({r.optimized_path}); supported for modules: {sorted(MODULE_WRAPPERS)}")
            elif r.kernel_type in self.external:
                self.notes.append(f"{r.optimized_path}: a {r.kernel_type} module is already plugged in, skipped")
            else:
                self.external[r.kernel_type] = r
        self.kinds = {k for k in items if isinstance(k, str)} - set(self.external)
        unknown = self.kinds - set(ALL_KERNELS)
        if unknown:
            raise ValueError(f"no replacement strategy for {sorted(unknown)}; known: {ALL_KERNELS}")
        self._orig: Dict[str, nn.Module] = {}
        self.applied: Dict[str, int] = {}

    def _load_external(self) -> None:
        for t, r in list(self.external.items()):
            if r.module_fn is None:
                try:
                    r.module_fn = load_kernel_module(r.optimized_path).kernel_fn
                except Exception as e:  # noqa: BLE001 - a broken module is skipped, as the reference does
                    self.notes.append(f"failed to load {r.optimized_path}: {type(e).__name__}: {e}")
                    del self.external[t]

    def _set(self, name: str, new: nn.Module) -> None:
        parent = self.model
        parts = name.split(".")
        for p in parts[:-1]:
            parent = getattr(parent, p)
        self._orig[name] = getattr(parent, parts[-1])
        setattr(parent, parts[-1], new)

    def _count(self, kind):
        self.applied[kind] = self.applied.get(kind, 0) + 1

    def __enter__(self) -> nn.Module:
        self._load_external()
        k = self.kinds
        ext = self.external
        taken = set()
        modules = list(self.model.named_modules())
        # composite blocks first: their Linears are driven by the block wrapper
        for name, m in modules:
            if not name:
                continue
            if _is_attention(m) and (k & {"rotary_embedding", "flash_attention"}):
                self._set(name, AttentionWrapper(m, "rotary_embedding" in k, "flash_attention" in k, "matmul" in k))
                taken.update(n for n, _ in m.named_modules(prefix=name))
                self._count("attention")
            elif _is_encoder_attention(m) and "flash_attention" in k:
                self._set(name, EncoderAttentionWrapper(m, "matmul" in k))
                taken.update(n for n, _ in m.named_modules(prefix=name))
                self._count("attention")
            elif _is_fused_qkv_causal_attention(m) and "flash_attention" in k:
                self._set(name, FusedQKVAttentionWrapper(m, "matmul" in k))
                taken.update(n for n, _ in m.named_modules(prefix=name))
                self._count("attention")
            elif "fused_mlp" in k and _swiglu_parts(m) is not None and not isinstance(m, nn.Linear):
                self._set(name, FeedForwardWrapper(m, *_swiglu_parts(m)))
                taken.update(n for n, _ in m.named_modules(prefix=name))
                self._count("fused_mlp")
            elif "matmul" in k and _gelu_mlp_parts(m) is not None:
                self._set(name, GeluMLPWrapper(m, *_gelu_mlp_parts(m)))
                taken.update(n for n, _ in m.named_modules(prefix=name))
                self._count("gelu_mlp")
        for name, m in modules:
            if not name or name in taken or any(name.startswith(t + ".") for t in taken):
                continue
            kind = ("matmul" if isinstance(m, nn.Linear) else "layernorm" if isinstance(m, nn.LayerNorm)
                    else "rmsnorm" if _is_rmsnorm(m) else None)
            if kind in ext:
                self._set(name, MODULE_WRAPPERS[kind](m, ext[kind].module_fn))
                self._count(kind)
            elif "matmul" in k and isinstance(m, nn.Linear):
                self._set(name, LinearWrapper(m))
                self._count("matmul")
            elif "layernorm" in k and isinstance(m, nn.LayerNorm):
                self._set(name, LayerNormWrapper(m))
                self._count("layernorm")
            elif "rmsnorm" in k and _is_rmsnorm(m):
                self._set(name, RMSNormWrapper(m))
                self._count("rmsnorm")
        # blocks last: they call the (already swapped) submodules with their residuals
        if "matmul" in k:
            for name, m in modules:
                if (name and _is_prenorm_block(m) and isinstance(m.attention, AttentionWrapper)
                        and m.attention.use_matmul and isinstance(m.feed_forward, FeedForwardWrapper)):
                    self._set(name, ResidualBlockWrapper(m))
                    self._count("residual_block")
                elif name and _is_gpt2_block(m):
                    self._set(name, GPT2BlockWrapper(m))
                    self._count("residual_block")
                elif name and _is_postnorm_block(m):
                    self._set(name, PostNormBlockWrapper(m))
                    self._count("residual_block")
        return self.model

    def __exit__(self, *exc):
        # newest swap first: a block wrapper goes before the submodules swapped inside its block,
        # so each path below resolves through the original modules
        for name in reversed(list(self._orig)):
            parent = self.model
            parts = name.split(".")
            for p in parts[:-1]:
                parent = getattr(parent, p)
            setattr(parent, parts[-1], self._orig[name])
        self._orig.clear()
        return False


# ---------------------------------------------------------------------- compare / timing
def compare_outputs(ref: torch.Tensor, opt: torch.Tensor, dtype: torch.dtype,
                    atol: Optional[float] = None, rtol: Optional[float] = None) -> Dict[str, Any]:
    """verify.py:687-765: shape check, NaN / Inf asymmetry fails, allclose on the non-NaN part."""
    r: Dict[str, Any] = {"shapes_match": ref.shape == opt.shape}
    if not r["shapes_match"]:
        r.update(correctness="FAIL", reason=f"shape mismatch {tuple(ref.shape)} vs {tuple(opt.shape)}")
        return r
    rf, of = ref.float(), opt.float()
    r["ref_has_nan"], r["opt_has_nan"] = bool(torch.isnan(rf).any()), bool(torch.isnan(of).any())
    r["ref_has_inf"], r["opt_has_inf"] = bool(torch.isinf(rf).any()), bool(torch.isinf(of).any())
    if r["opt_has_nan"] and not r["ref_has_nan"]:
        r.update(correctness="FAIL", reason="optimized output has NaN where the reference does not")
        return r
    if r["opt_has_inf"] and not r["ref_has_inf"]:
        r.update(correctness="FAIL", reason="optimized output has Inf where the reference does not")
        return r
    valid = ~(torch.isnan(rf) & torch.isnan(of))
    d = (rf - of).abs()[valid]
    r["max_abs_error"] = float(d.max()) if d.numel() else 0.0
    r["mean_abs_error"] = float(d.mean()) if d.numel() else 0.0
    tol = DEFAULT_TOLERANCES.get(dtype, {"atol": 1e-4, "rtol": 1e-4})
    atol = tol["atol"] if atol is None else atol
    rtol = tol["rtol"] if rtol is None else rtol
    ok = bool(torch.allclose(rf[valid], of[valid], atol=atol, rtol=rtol)) if valid.any() else True
    r.update(correctness="PASS" if ok else "FAIL", atol=atol, rtol=rtol)
    if not ok:
        r["reason"] = f"values exceed tolerance (atol={atol}, rtol={rtol}); max_abs_error={r['max_abs_error']:.6e}"
    return r


def make_token_ids(model: nn.Module, shape: Tuple[int, ...], device, seed: int = 42) -> torch.Tensor:
    """Token ids uniform in [0, vocab) from a seeded CPU generator (verify.py:230-251 draws 32000)."""
    vocab = 32000
    for m in model.modules():
        if isinstance(m, nn.Embedding):
            vocab = m.num_embeddings
            break
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, shape, generator=g, dtype=torch.long).to(device)


@torch.no_grad()
def benchmark_model(model: nn.Module, inp, warmup: int = WARMUP_RUNS, timed: int = TIMED_RUNS):
    """(output, median ms) over `timed` event-timed forwards after `warmup` (verify.py:258-307)."""
    run = (lambda: model(**inp)) if isinstance(inp, dict) else (lambda: model(inp))
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    st = [torch.cuda.Event(enable_timing=True) for _ in range(timed)]
    en = [torch.cuda.Event(enable_timing=True) for _ in range(timed)]
    for i in range(timed):
        st[i].record()
        run()
        en[i].record()
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) for a, b in zip(st, en))
    out = run()
    torch.cuda.synchronize()
    if not isinstance(out, torch.Tensor):
        out = out[0] if isinstance(out, (tuple, list)) else out
    return out, t[len(t) // 2]


def diagnose(model, inp, ref_out, kinds: List[str], dtype, atol=None, rtol=None) -> List[dict]:
    """Apply one kernel type at a time to find which one breaks the comparison (verify.py:772-828)."""
    rows = []
    for kind in kinds:
        with OptimizedModelContext(model, [kind]) as m, torch.no_grad():
            out = m(inp)
        torch.cuda.synchronize()
        c = compare_outputs(ref_out, out, dtype, atol, rtol)
        label = kind.kernel_type + " (module)" if isinstance(kind, KernelReplacement) else kind
        rows.append({"kernel_type": label, "correctness": c["correctness"], "max_abs_error": c.get("max_abs_error")})
    return rows


def _load_model(args, dtype, device) -> nn.Module:
    from . import llama
    if args.model in ("7b", "small"):
        return llama.build(args.model, dtype, device, seed=args.seed, n_layers=args.layers)
    spec_ = importlib.util.spec_from_file_location("user_model", os.path.abspath(args.model))
    mod = importlib.util.module_from_spec(spec_)
    spec_.loader.exec_module(mod)
    with torch.device(device):
        model = getattr(mod, args.class_name)().to(dtype)
    return model.eval()


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="libak355 model plug-in verifier")
    ap.add_argument("--model", default="7b", help="7b, small, or a model .py file")
    ap.add_argument("--class-name", default="LlamaModel7B")
    ap.add_argument("--input-shape", default="1,2048")
    ap.add_argument("--dtype", default="float16", choices=["float16", "bfloat16", "float32"])
    ap.add_argument("--kernels", default=None,
                    help="libak355 strategies: all (default without kernel modules), none, or a list")
    ap.add_argument("--workspace", default=None,
                    help="plug in the kernel modules found here (orchestration_state.json or "
                         "kernel_<type>_<rank>_optimized.py)")
    ap.add_argument("--kernel-module", action="append", default=[],
                    help="plug in this kernel .py (KERNEL_TYPE + kernel_fn); repeatable")
    ap.add_argument("--layers", type=int, default=None, help="override the layer count (7b / small)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--atol", type=float, default=None)
    ap.add_argument("--rtol", type=float, default=None)
    ap.add_argument("--warmup", type=int, default=WARMUP_RUNS)
    ap.add_argument("--timed", type=int, default=TIMED_RUNS)
    ap.add_argument("--diagnose", action="store_true")
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    dtype = getattr(torch, args.dtype)
    dev = torch.device("cuda:0")
    external = discover_optimized_kernels(args.workspace) if args.workspace else []
    external += [replacement_from_module(p) for p in args.kernel_module]
    spec_k = args.kernels or ("none" if external else "all")
    kinds: List[Any] = (list(ALL_KERNELS) if spec_k == "all" else [] if spec_k == "none"
                        else [s.strip() for s in spec_k.split(",")])
    kinds += external
    for r in external:
        print(f"kernel module: {r.kernel_type} (rank {r.rank}, speedup {r.speedup:g}) <- {r.optimized_path}")
    model = _load_model(args, dtype, dev)
    shape = tuple(int(s) for s in args.input_shape.split(","))
    inp = make_token_ids(model, shape, dev)
    print(f"model: {type(model).__name__}, params {sum(p.numel() for p in model.parameters()) / 1e9:.2f} B, "
          f"input {list(shape)}, dtype {args.dtype}")
    ref_out, ref_ms = benchmark_model(model, inp, args.warmup, args.timed)
    ctx = OptimizedModelContext(model, kinds)
    with ctx as m:
        opt_out, opt_ms = benchmark_model(m, inp, args.warmup, args.timed)
        applied = dict(ctx.applied)
    for note in ctx.notes:
        print(f"NOTE: {note}")
    cmp = compare_outputs(ref_out, opt_out, dtype, args.atol, args.rtol)
    res = {"model": type(model).__name__, "input_shape": list(shape), "dtype": args.dtype, "kernels": kinds,
           "replaced": applied, "ref_latency_ms": ref_ms, "opt_latency_ms": opt_ms,
           "end_to_end_speedup": ref_ms / opt_ms, **{k: v for k, v in cmp.items()}}
    if args.diagnose and cmp["correctness"] != "PASS":
        res["diagnosis"] = diagnose(model, inp, ref_out, kinds, dtype, args.atol, args.rtol)
    for k in ("replaced", "ref_latency_ms", "opt_latency_ms", "end_to_end_speedup", "max_abs_error",
              "mean_abs_error", "correctness"):
        print(f"{k}: {res.get(k)}")
    if "diagnosis" in res:
        for d in res["diagnosis"]:
            print(f"  {d}")
    if args.json:
        with open(args.json, "w") as f:
            json.dump(res, f, indent=2, default=str)
    return 0 if cmp["correctness"] == "PASS" else 1


if __name__ == "__main__":
    sys.exit(main())

"""The C ABI: libak355.so loads without a GPU and exports every entry point of include/ak355.h
(CPU only; calls here are rejected by host-side argument checks before any HIP call)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ak355.h")


def declared_functions() -> list[str]:
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(ak_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    from autokernel_amd import _lib
    return _lib.load()


def test_header_declares_the_suite():
    names = declared_functions()
    for op in ("ak_rmsnorm", "ak_layernorm", "ak_softmax", "ak_rope", "ak_cross_entropy", "ak_reduce_sum",
               "ak_reduce_max", "ak_gemm", "ak_mlp_gate_up", "ak_flash_attn_fwd", "ak_version"):
        assert op in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"libak355.so does not export {name}"


def test_python_binding_covers_header():
    from autokernel_amd import _lib
    bound = set(_lib.SIGNATURES) | set(_lib._STR_FUNCS)
    assert set(declared_functions()) <= bound


def test_version_and_status_strings(lib):
    from autokernel_amd import _lib
    assert "gfx950" in _lib.version()
    assert lib.ak_status_string(0) == b"ok"
    assert lib.ak_status_string(1) == b"invalid argument"
    assert lib.ak_status_string(99) == b"unknown status"


def test_invalid_arguments_rejected_on_host(lib):
    from autokernel_amd import _lib
    x = ctypes.c_void_p(16)
    assert lib.ak_rmsnorm(1, x, x, x, -1, 8, 1e-6, None) == _lib.AK_EINVAL
    assert lib.ak_rmsnorm(1, None, x, x, 4, 8, 1e-6, None) == _lib.AK_EINVAL
    assert lib.ak_rmsnorm(7, x, x, x, 4, 8, 1e-6, None) == _lib.AK_EINVAL  # bad dtype code
    assert lib.ak_rmsnorm(1, x, x, x, 0, 8, 1e-6, None) == _lib.AK_OK      # empty: nothing to do
    assert lib.ak_softmax(1, x, x, 3, -2, None) == _lib.AK_EINVAL
    assert lib.ak_copy(x, x, -16, None) == _lib.AK_EINVAL
    assert lib.ak_copy(x, x, 24, None) == _lib.AK_EUNSUPPORTED          # not a multiple of 16 bytes
    assert lib.ak_copy(ctypes.c_void_p(8), x, 16, None) == _lib.AK_EUNSUPPORTED  # misaligned
    assert lib.ak_copy(x, x, 0, None) == _lib.AK_OK
    assert lib.ak_set_launch_events(None, None) == _lib.AK_OK  # clears this thread's slot
    assert lib.ak_rope(1, x, x, x, x, 4, 7, 4, 1, None) == _lib.AK_EINVAL   # odd head_dim
    assert lib.ak_gemm(1, x, x, x, 4, 4, 4, 2, 4, 4, 0, None) == _lib.AK_EINVAL  # lda < K
    y = ctypes.c_void_p(4096)
    assert lib.ak_gemm_residual(1, x, x, x, x, 4, 4, 4, 4, 4, 4, 0, None) == _lib.AK_EINVAL  # R is C
    assert lib.ak_gemm_residual(1, x, x, ctypes.c_void_p(40), x, 4, 4, 4, 4, 4, 4, 0, None) == _lib.AK_EINVAL
    assert lib.ak_gemm_residual(1, x, x, None, y, 4, 4, 4, 4, 4, 4, 0, None) == _lib.AK_EINVAL
    assert lib.ak_gemm_residual(0, x, x, x, y, 4, 4, 4, 4, 4, 4, 0, None) == _lib.AK_EUNSUPPORTED  # fp32
    assert lib.ak_gemm_residual(1, x, x, x, y, 0, 4, 4, 4, 4, 4, 0, None) == _lib.AK_OK  # empty
    assert lib.ak_gemm_bias_gelu(1, x, x, None, y, 4, 4, 4, 4, 4, 4, 1, None) == _lib.AK_EINVAL  # no bias
    assert lib.ak_gemm_bias_gelu(1, x, x, x, y, 4, 4, 4, 4, 4, 2, 1, None) == _lib.AK_EINVAL     # ldc < N
    assert lib.ak_gemm_bias_gelu(0, x, x, x, y, 4, 4, 4, 4, 4, 4, 1, None) == _lib.AK_EUNSUPPORTED  # fp32
    assert lib.ak_gemm_bias_gelu(1, x, x, x, y, 4, 0, 4, 4, 4, 4, 1, None) == _lib.AK_OK         # empty
    assert lib.ak_gemm_bias_residual(1, x, x, x, x, x, 4, 4, 4, 4, 4, 4, 1, None) == _lib.AK_EINVAL  # R is C
    assert lib.ak_gemm_bias_residual(1, x, x, x, None, y, 4, 4, 4, 4, 4, 4, 1, None) == _lib.AK_EINVAL
    assert lib.ak_gemm_bias_residual(1, x, x, None, x, y, 4, 4, 4, 4, 4, 4, 1, None) == _lib.AK_EINVAL
    assert lib.ak_gemm_bias_residual(0, x, x, x, x, y, 4, 4, 4, 4, 4, 4, 1, None) == _lib.AK_EUNSUPPORTED
    assert lib.ak_gemm_bias_residual(1, x, x, x, x, y, 0, 4, 4, 4, 4, 4, 1, None) == _lib.AK_OK  # empty
    assert lib.ak_gemm_workspace_bytes(1, 1024, 1024, 8192, 8192, 8192, 1024, 1) == 4 * 1024 * 1024 * 4
    assert lib.ak_gemm_workspace_bytes(1, 1024, 1024, 4096, 4096, 1024, 1024, 0) == 4 * 1024 * 1024 * 4
    assert lib.ak_gemm_workspace_bytes(1, 1024, 1024, 1024, 1024, 1024, 1024, 0) == 0   # slices < 1024 deep
    assert lib.ak_gemm_workspace_bytes(0, 1024, 1024, 8192, 8192, 8192, 1024, 1) == 0   # fp32: no split
    assert lib.ak_gemm_workspace_bytes(1, 4096, 4096, 4096, 4096, 4096, 4096, 1) == 0   # fills the GPU
    assert lib.ak_gemm_workspace_bytes(1, 1024, 1024, 8192, 8192, 8192, 1022, 1) == 0   # ldc % 4
    # [K, N] B with N % 8 == 4 (a padded column slice): the [K, N] split kernel needs N % 8 == 0
    assert lib.ak_gemm_workspace_bytes(1, 1024, 1020, 4096, 4096, 1024, 1020, 0) == 0
    assert lib.ak_gemm_workspace_bytes(1, 1024, 1020, 4096, 4096, 4096, 1020, 1) > 0   # [N, K] B splits
    # the no-alloc cross-entropy refuses more rows than its device array holds, before any HIP call
    big = _lib.CE_NOALLOC_MAX_ROWS + 1
    assert lib.ak_cross_entropy_noalloc(1, x, x, x, big, 8, -100, None) == _lib.AK_EINVAL
    assert lib.ak_cross_entropy_noalloc(1, x, x, None, 4, 8, -100, None) == _lib.AK_EINVAL   # no output
    assert lib.ak_cross_entropy_noalloc(7, x, x, x, 4, 8, -100, None) == _lib.AK_EINVAL      # bad dtype
    assert lib.ak_gemm_ws(1, x, x, x, 0, 4, 4, 4, 4, 4, 1, None, 0, None) == _lib.AK_OK  # empty -> ak_gemm
    bat = lib.ak_gemm_batched  # (dtype, A, B, C, batch, M, N, K, lda, ldb, ldc, sa, sb, sc, b_trans, stream)
    assert bat(1, x, x, y, -1, 4, 4, 4, 4, 4, 4, 16, 16, 16, 0, None) == _lib.AK_EINVAL   # negative batch
    assert bat(1, x, x, y, 0, 4, 4, 4, 4, 4, 4, 16, 16, 16, 0, None) == _lib.AK_OK        # empty batch
    assert bat(1, x, x, y, 2, 4, 4, 4, 4, 4, 4, 16, 16, 8, 0, None) == _lib.AK_EINVAL     # C items overlap
    assert bat(1, x, x, y, 2, 4, 4, 4, 4, 4, 4, -16, 16, 16, 0, None) == _lib.AK_EINVAL   # negative stride
    assert bat(1, x, x, y, 2, 4, 4, 4, 2, 4, 4, 16, 16, 16, 0, None) == _lib.AK_EINVAL    # lda < K
    assert bat(7, x, x, y, 2, 4, 4, 4, 4, 4, 4, 16, 16, 16, 0, None) == _lib.AK_EINVAL    # bad dtype code
    rope = lib.ak_gemm_rope
    assert rope(1, x, x, y, 4, 8, 4, 4, 4, 8, 1, x, x, 4, 6, 6, None) == _lib.AK_EINVAL  # head_dim % 4
    assert rope(1, x, x, y, 4, 8, 4, 4, 4, 8, 1, x, x, 4, 4, 6, None) == _lib.AK_EINVAL  # rot_cols % head_dim
    assert rope(1, x, x, y, 4, 8, 4, 4, 4, 8, 1, x, x, 4, 4, 12, None) == _lib.AK_EINVAL  # rot_cols > N
    assert rope(1, x, x, y, 4, 8, 4, 4, 4, 8, 1, None, x, 4, 4, 8, None) == _lib.AK_EINVAL  # no table
    assert rope(1, x, x, y, 4, 8, 4, 4, 4, 8, 1, x, x, 0, 4, 8, None) == _lib.AK_EINVAL  # seq_len
    assert rope(0, x, x, y, 4, 8, 4, 4, 4, 8, 1, x, x, 4, 4, 8, None) == _lib.AK_EUNSUPPORTED  # fp32
    assert rope(1, x, x, y, 0, 8, 4, 4, 4, 8, 1, x, x, 4, 4, 8, None) == _lib.AK_OK  # empty
    assert lib.ak_mlp_gate_up(1, x, x, x, x, 4, 4, 4, 9, None) == _lib.AK_EINVAL  # activation code
    assert lib.ak_reduce_max(1, x, x, 2, 0, 1, None) == _lib.AK_EINVAL      # max of nothing
    s = _lib.i64_array([8, 8, 8])
    assert lib.ak_flash_attn_fwd(1, x, x, x, x, 1, 4, 3, 8, 8, 64, s, s, s, s, 1, 1.0, None) == _lib.AK_EINVAL
    assert lib.ak_flash_attn_fwd(1, x, x, x, x, 1, 4, 4, 8, 8, 320, s, s, s, s, 1, 1.0, None) == _lib.AK_EUNSUPPORTED
    assert lib.ak_flash_attn_fwd(7, x, x, x, x, 1, 4, 4, 8, 8, 64, s, s, s, s, 1, 1.0, None) == _lib.AK_EINVAL
    assert lib.ak_flash_attn_fwd(0, x, x, x, x, 1, 4, 4, 8, 0, 64, s, s, s, s, 1, 1.0, None) == _lib.AK_EUNSUPPORTED


def test_kernel_fn_refuses_cpu_tensors():
    import torch
    from autokernel_amd import kernels
    with pytest.raises(RuntimeError, match="no CPU path"):
        kernels.get("softmax")(torch.randn(4, 8))
    with pytest.raises(RuntimeError, match="no CPU path"):
        kernels.get("matmul")(torch.randn(4, 8), torch.randn(8, 4))


def test_kernel_modules_keep_reference_signatures():
    import inspect

    from autokernel_amd import kernels
    expect = {
        "matmul": ["A", "B"], "softmax": ["x", "dim"], "layernorm": ["x", "weight", "bias", "eps"],
        "rmsnorm": ["x", "weight", "eps"], "flash_attention": ["Q", "K", "V", "causal", "sm_scale"],
        "fused_mlp": ["x", "w_gate", "w_up", "w_down", "activation"], "cross_entropy": ["logits", "targets"],
        "rotary_embedding": ["x", "cos", "sin"], "reduce": ["x", "dim"],
    }
    defaults = {("rmsnorm", "eps"): 1e-6, ("layernorm", "eps"): 1e-5, ("flash_attention", "causal"): True,
                ("flash_attention", "sm_scale"): None, ("fused_mlp", "activation"): "silu",
                ("softmax", "dim"): -1, ("reduce", "dim"): -1}
    for name, params in expect.items():
        sig = inspect.signature(kernels.get(name))
        assert list(sig.parameters) == params, name
        for (op, p), d in defaults.items():
            if op == name:
                assert sig.parameters[p].default == d

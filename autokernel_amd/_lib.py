"""ctypes binding of libak355.so (declared in include/ak355.h).

The library is loaded after torch so that it binds to the HIP runtime torch already mapped
(both carry the soname libamdhip64.so.7); kernels then run on torch's streams and memory.
There is no fallback: if the library is missing or a launch fails, the caller gets an error.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("AK355_LIB") or Path(__file__).resolve().with_name("libak355.so"))

AK_F32, AK_F16, AK_BF16 = 0, 1, 2
DTYPE_CODE = {torch.float32: AK_F32, torch.float16: AK_F16, torch.bfloat16: AK_BF16}

AK_OK, AK_EINVAL, AK_EUNSUPPORTED, AK_EHIP = 0, 1, 2, 3
ACTIVATIONS = {"silu": 0, "gelu": 1, "relu2": 2}
ACT_NONE = 3
CE_NOALLOC_MAX_ROWS = 1 << 20  # AK_CE_NOALLOC_MAX_ROWS (include/ak355.h)

_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_p = ctypes.c_void_p
_pi64 = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes (restype is int unless listed in _STR_FUNCS)
SIGNATURES: dict[str, list] = {
    "ak_rmsnorm": [_i, _p, _p, _p, _i64, _i64, _f, _p],
    "ak_layernorm": [_i, _p, _p, _p, _p, _i64, _i64, _f, _p],
    "ak_softmax": [_i, _p, _p, _i64, _i64, _p],
    "ak_rope": [_i, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "ak_rope_f32_tables": [_i, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p],
    "ak_rmsnorm_rsqrt": [_i, _p, _p, _p, _i64, _i64, _f, _p],
    "ak_cross_entropy": [_i, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "ak_cross_entropy_noalloc": [_i, _p, _p, _p, _i64, _i64, _i64, _p],
    "ak_reduce_sum": [_i, _p, _p, _i64, _i64, _i64, _p],
    "ak_reduce_max": [_i, _p, _p, _i64, _i64, _i64, _p],
    "ak_gemm": [_i, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p],
    "ak_gemm_batched": [_i, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p],
    "ak_gemm_residual": [_i, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p],
    "ak_gemm_bias": [_i, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p],
    "ak_gemm_bias_gelu": [_i, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p],
    "ak_gemm_bias_residual": [_i, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p],
    "ak_gemm_workspace_bytes": [_i, _i64, _i64, _i64, _i64, _i64, _i64, _i],
    "ak_gemm_ws": [_i, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p, _i64, _p],
    "ak_gemm_rope": [_i, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p, _p, _i64, _i64, _i64, _p],
    "ak_mlp_gate_up": [_i, _p, _p, _p, _p, _i64, _i64, _i64, _i, _p],
    "ak_copy": [_p, _p, _i64, _p],
    "ak_set_launch_events": [_p, _p],
    "ak_flash_attn_fwd": [_i, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                          _pi64, _pi64, _pi64, _pi64, _i, _f, _p],
}
_STR_FUNCS = ("ak_version", "ak_status_string", "ak_last_hip_error_string")
_I64_FUNCS = ("ak_gemm_workspace_bytes",)  # return int64_t instead of a status

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class AkError(RuntimeError):
    """A libak355 entry point returned an error status."""


def load() -> ctypes.CDLL:
    """Load libak355.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m autokernel_amd.build` "
                    "(autokernel_amd has no non-HIP fallback)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = ctypes.c_int64 if name in _I64_FUNCS else ctypes.c_int
            for name in _STR_FUNCS:
                fn = getattr(lib, name)
                fn.restype = ctypes.c_char_p
            lib.ak_status_string.argtypes = [ctypes.c_int]
            _lib = lib
    return _lib


def version() -> str:
    return load().ak_version().decode()


def check(status: int, op: str, **info) -> None:
    if status == AK_OK:
        return
    lib = load()
    msg = lib.ak_status_string(status).decode()
    if status == AK_EHIP:
        msg += ": " + lib.ak_last_hip_error_string().decode()
    detail = ", ".join(f"{k}={v}" for k, v in info.items())
    raise AkError(f"{op}: {msg} ({detail})")


def dtype_code(t: torch.Tensor, op: str) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"{op}: unsupported dtype {t.dtype} (float32, float16, bfloat16)") from None


def require_gpu(op: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{op}: expected GPU tensors, got a tensor on {t.device} "
                               "(autokernel_amd has no CPU path)")


# The raw handle of a device's current stream: the value of torch.cuda.current_stream(d).cuda_stream
# without building a Stream object (1.8 us per call -> 0.07 us; torch's compiled kernels launch the
# same way)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def i64_array(vals) -> ctypes.Array:
    return (ctypes.c_int64 * len(vals))(*vals)

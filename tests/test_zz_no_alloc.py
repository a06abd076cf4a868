"""ak_cross_entropy_noalloc (the entry point that allocates nothing) against ak_cross_entropy.

Both are called through the C ABI on the same inputs; the results must be bit-identical. Two
calls in a row, the second with fewer rows (and a different vocabulary, with ignored rows), so the
device array that holds the per-row losses is reused with stale contents past the second call's
rows.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ce_pair(lib, logits, targets, ignore_index=-100):
    from autokernel_amd import _lib
    rows, vocab = logits.shape
    code = _lib.DTYPE_CODE[logits.dtype]
    stream = _lib.stream_of(logits)
    ws = torch.empty(max(rows, 1), device=logits.device, dtype=torch.float32)
    ref = torch.empty((), device=logits.device, dtype=logits.dtype)
    out = torch.full((), float("nan"), device=logits.device, dtype=logits.dtype)
    _lib.check(lib.ak_cross_entropy(code, logits.data_ptr(), targets.data_ptr(), ws.data_ptr(), ref.data_ptr(),
                                    rows, vocab, ignore_index, stream), "ak_cross_entropy")
    _lib.check(lib.ak_cross_entropy_noalloc(code, logits.data_ptr(), targets.data_ptr(), out.data_ptr(),
                                            rows, vocab, ignore_index, stream), "ak_cross_entropy_noalloc")
    torch.cuda.synchronize()
    return ref, out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(gpu, dtype):
    from autokernel_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(7)
    # call 1: the harness's large size; call 2: fewer rows, a wide odd vocabulary, ignored rows
    for rows, vocab in ((4096, 32000), (1000, 50257)):
        print(f"noalloc ce {dtype} rows={rows} vocab={vocab}", flush=True)
        logits = (torch.randn(rows, vocab, generator=g) * 3).to(dtype).to(gpu)
        targets = torch.randint(0, vocab, (rows,), generator=g)
        if rows == 1000:
            targets[::7] = -100
        targets = targets.to(gpu)
        ref, out = _ce_pair(lib, logits, targets)
        assert torch.isfinite(ref.float())
        assert torch.equal(out.view(torch.int16 if dtype != torch.float32 else torch.int32),
                           ref.view(torch.int16 if dtype != torch.float32 else torch.int32)), (rows, vocab, out, ref)


def test_noalloc_rejects_rows_above_the_maximum(gpu):
    from autokernel_amd import _lib
    lib = _lib.load()
    x = torch.empty(16, device=gpu, dtype=torch.float16)
    st = lib.ak_cross_entropy_noalloc(_lib.AK_F16, x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                      _lib.CE_NOALLOC_MAX_ROWS + 1, 8, -100, _lib.stream_of(x))
    assert st == _lib.AK_EINVAL
    # no rows: the mean over nothing is NaN, as torch gives
    out = torch.zeros((), device=gpu, dtype=torch.float16)
    st = lib.ak_cross_entropy_noalloc(_lib.AK_F16, None, None, ctypes.c_void_p(out.data_ptr()), 0, 8, -100,
                                      _lib.stream_of(out))
    assert st == _lib.AK_OK
    torch.cuda.synchronize()
    assert torch.isnan(out.float())

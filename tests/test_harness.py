"""The harness's verdict logic with fake kernel_fns on the CPU (no GPU needed).

Each fake forces one failure the reference harness handles (bench.py:641-966): wrong values,
NaN, a timeout, out-of-memory (a SKIP, not a FAIL), a shape mismatch, and run-to-run noise.
"""
from __future__ import annotations

import time

import pytest
import torch

from autokernel_amd import baseline_torch, harness, spec


def tiny_softmax_config():
    cfg = dict(spec.KERNEL_CONFIGS["softmax"])
    cfg["test_sizes"] = [("tiny", {"rows": 4, "cols": 16}), ("small", {"rows": 8, "cols": 32}),
                         ("big", {"rows": 16, "cols": 64})]
    cfg["edge_sizes"] = [("edge_odd", {"rows": 3, "cols": 7})]
    cfg["test_dtypes"] = [torch.float32, torch.float16]
    cfg["reference_fn"] = baseline_torch.BASELINE["softmax"]
    return cfg


def run(fn, **kw):
    return harness.run_correctness(fn, tiny_softmax_config(), device="cpu", log=lambda *a: None, **kw)


def test_good_kernel_passes_all_stages():
    r = run(lambda x: torch.softmax(x.float(), -1).to(x.dtype))
    assert r["correctness"] == "PASS"
    for k in ("smoke_test", "numerical_stability", "determinism", "edge_cases"):
        assert r[k] == "PASS", (k, r[k])
    assert r["shape_sweep"].startswith("PASS (6 configs")


def test_wrong_values_fail_smoke_and_abort():
    r = run(lambda x: torch.softmax(x, -1) * 1.1)
    assert r["smoke_test"] == "FAIL" and r["correctness"] == "FAIL"
    assert r["shape_sweep"] == "SKIP"  # smoke failure aborts the remaining stages


def test_nan_output_fails():
    def nan_kernel(x):
        y = torch.softmax(x, -1)
        y[0, 0] = float("nan")
        return y
    assert run(nan_kernel)["smoke_test"] == "FAIL"


def test_timeout_is_a_failure():
    calls = {"n": 0}

    def slow(x):
        calls["n"] += 1
        if calls["n"] > 1:
            time.sleep(3)
        return torch.softmax(x, -1)
    r = run(slow, timeout_s=1, quick=True)
    assert r["smoke_test"] == "PASS"
    assert r["shape_sweep"].startswith("FAIL")
    assert any("TIMEOUT" in d for d in r["details"])


def test_oom_is_a_skip_not_a_failure():
    def oom_on_big(x):
        if x.shape[0] >= 16:
            raise torch.cuda.OutOfMemoryError("out of memory (forced)")
        return torch.softmax(x.float(), -1).to(x.dtype)
    r = run(oom_on_big, quick=True)
    assert r["correctness"] == "PASS"
    assert r["shape_sweep"].startswith("PASS (6 configs")


def test_shape_mismatch_fails():
    r = run(lambda x: torch.softmax(x, -1).T.contiguous() if x.shape[0] == 8 else torch.softmax(x.float(), -1).to(x.dtype), quick=True)
    assert r["shape_sweep"].startswith("FAIL")
    assert any("shape mismatch" in d for d in r["details"])


def test_nondeterminism_fails_stage4():
    def noisy(x):
        y = torch.softmax(x.float(), -1)
        return (y + torch.rand_like(y) * 1e-7).to(x.dtype)
    r = run(noisy)
    assert r["determinism"] == "FAIL"


def test_nan_where_reference_is_clean_fails_stage3():
    def nan_on_zero_input(x):
        if torch.all(x == 0):
            return torch.full_like(x, float("nan"))
        return torch.softmax(x.float(), -1).to(x.dtype)
    r = run(nan_on_zero_input)
    assert r["numerical_stability"] == "FAIL"
    assert any("reference is clean" in d for d in r["details"])


def test_compare_matches_reference_semantics():
    a = torch.tensor([1.0, 2.0, 3.0])
    c = harness.compare(a, a + 1e-3, atol=1e-2, rtol=0)
    assert c["match"] and c["pct_within_tol"] == 100.0
    c = harness.compare(a, a + 1.0, atol=1e-2, rtol=1e-2)
    assert not c["match"] and "exceeds tol" in c["reason"]
    assert not harness.compare(a, a[:2], 1, 1)["match"]


def test_roofline_classification():
    g = harness.GPUSpec(peak_tflops_fp16=2516.6, peak_tflops_fp32=157.3, peak_bandwidth_gb_s=8000.0)
    r = harness.roofline(flops=2 * 4096 ** 3, nbytes=3 * 4096 ** 2 * 2, ms=0.1, gpu=g)
    assert r["bottleneck"] == "compute_bound" and abs(r["throughput_tflops"] - 1374.4) < 1
    r = harness.roofline(flops=5 * 8192 ** 2, nbytes=2 * 8192 ** 2 * 2, ms=0.05, gpu=g)
    assert r["bottleneck"] == "memory_bound" and abs(r["pct_peak_bandwidth"] - 67.1) < 0.1

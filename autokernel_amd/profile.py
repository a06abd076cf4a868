"""ROCm-aware model profiler: the role of the reference's profile.py on MI355X.

    python -m autokernel_amd.profile [--model 7b|small|path/to/model.py --class-name C]
        [--input-shape 1,2048] [--dtype float16] [--kernels none|all|matmul,rmsnorm,...]
        [--trace kernel_trace.csv | kernel_stats.csv] [--output profile_report.json]

Ranks a model's GPU kernels by time and maps each to an AutoKernel op type, so the ops worth a
libak355 kernel come first (Amdahl ordering). Kernel times come from one of two sources:
  live   torch.profiler (roctracer on ROCm) around PROFILE_ITERS forwards after WARMUP_ITERS
         warm-up forwards (profile.py:529-652), device events only (the reference also counts the
         host op that launched each kernel, so such kernels count twice there); --kernels swaps
         ops to libak355 first, through the verify plug-in, to profile the optimized model;
  trace  a rocprofv3 --kernel-trace CSV (Kernel_Name, Start_Timestamp, End_Timestamp per launch)
         or its --stats summary (Name, Calls, TotalDurationNs), for any program.
The reference classifies kernels by vendor-name fragments (profile.py:44-55, :449-465), and ROCm's
library kernels do not carry them: hipBLASLt / Tensile GEMMs are `Cijk_...`, aotriton attention is
`attn_fwd`. The rules here add those names and libak355's own kernels ahead of the reference's
rules, which still apply unchanged after them. The report has the layout of the reference's
profile_report.json (profile.py:664-745), plus a per-op-type summary.
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import re
import sys
from collections import defaultdict
from dataclasses import dataclass
from typing import Dict, Iterable, List, Optional, Tuple

WARMUP_ITERS = 5    # profile.py:37
PROFILE_ITERS = 10  # profile.py:38

# libak355's kernels (exact names from this library), checked first. gemm_dma / gemm_mfma with
# two B matrices (the sixth template argument, NB = 2) are the fused MLP's gate / up projection.
_AK_FUSED_MLP = re.compile(r"ak::gemm_(?:dma|mfma)<[^,>]+(?:,\s*[^,>]+){4},\s*2,")
_AK_RULES: List[Tuple[str, str]] = [
    ("ak::fa_fwd", "flash_attention"),
    ("ak::gate_up", "fused_mlp"),
    ("ak::gemm", "matmul"),
    ("ak::transpose", "matmul"),
    ("ak::rope", "rotary_embedding"),
    ("ak::rmsnorm", "rmsnorm"),
    ("ak::layernorm", "layernorm"),
    ("ak::softmax", "softmax"),
    ("ak::ce_", "cross_entropy"),
    ("ak::reduce", "reduce"),
]
# Kernel names of ROCm's libraries and of PyTorch-ROCm's native kernels, checked next.
_ROCM_RULES: List[Tuple[List[str], str]] = [
    (["attn_fwd", "fmha_fwd", "fmha_bwd", "flash_fwd", "aotriton"], "flash_attention"),
    (["cijk_", "rocblas", "hipblaslt", "tensile", "devicegemm", "device_gemm", "gemm_xdl",
      "gemm_universal"], "matmul"),
    (["rowwisemoments", "vectorized_layer_norm", "layer_norm_kernel"], "layernorm"),
    (["log_softmax", "nll_loss"], "cross_entropy"),
]
# The reference's rules (profile.py:44-55), in its order; first match wins.
_REFERENCE_RULES: List[Tuple[List[str], str]] = [
    (["flash", "fmha"], "flash_attention"),
    (["attention"], "flash_attention"),
    (["gemm", "matmul", "cublas"], "matmul"),
    (["softmax"], "softmax"),
    (["layer_norm", "layernorm"], "layernorm"),
    (["rms_norm", "rmsnorm"], "rmsnorm"),
    (["gelu", "silu", "mlp"], "fused_mlp"),
    (["cross_entropy", "nll"], "cross_entropy"),
    (["rotary", "rope"], "rotary_embedding"),
    (["reduce", "all_reduce"], "reduce"),
]
_MM_WORD = re.compile(r"(?:^|[^a-z])mm(?:$|[^a-z])")  # profile.py:459-463

SUPPORTED_OP_TYPES = ("matmul", "softmax", "layernorm", "rmsnorm", "flash_attention", "fused_mlp",
                      "cross_entropy", "rotary_embedding", "reduce")
COMPUTE_BOUND = {"matmul", "flash_attention"}                     # profile.py:484
MEMORY_BOUND = {"softmax", "layernorm", "rmsnorm", "reduce", "rotary_embedding", "fused_mlp",
                "cross_entropy"}                                  # profile.py:485-486


def classify_kernel(kernel_name: str) -> str:
    """Map a kernel name (ROCm, libak355 or the reference's vendor names) to an op type."""
    if _AK_FUSED_MLP.search(kernel_name):
        return "fused_mlp"
    for frag, op in _AK_RULES:
        if frag in kernel_name:
            return op
    low = kernel_name.lower()
    for rules in (_ROCM_RULES, _REFERENCE_RULES):
        for frags, op in rules:
            if any(f in low for f in frags):
                return op
    if "mm" in low and _MM_WORD.search(low):
        return "matmul"
    return "other"


def roofline_position(op_type: str, gpu_time_us: float) -> str:
    """The reference's heuristic (profile.py:477-501)."""
    if op_type in COMPUTE_BOUND:
        return "compute-bound"
    if op_type in MEMORY_BOUND:
        return "memory-bound"
    return "likely compute-bound" if gpu_time_us > 100.0 else "likely memory-bound"


def priority_label(pct: float) -> str:
    """profile.py:655-661."""
    return "HIGH" if pct >= 10.0 else "MEDIUM" if pct >= 3.0 else "LOW"


@dataclass
class KernelRecord:
    """Aggregated time of one kernel name (and input shapes, when the source has them)."""
    name: str
    op_type: str
    gpu_time_us: float
    call_count: int
    input_shapes: str = ""


def records_from_times(times: Dict[Tuple[str, str], List[float]]) -> List[KernelRecord]:
    """{(name, shapes): [per-call microseconds]} -> records sorted by total time, descending."""
    recs = [KernelRecord(n, classify_kernel(n), sum(v), len(v), s) for (n, s), v in times.items() if sum(v) > 0]
    recs.sort(key=lambda r: r.gpu_time_us, reverse=True)
    return recs


def read_rocprof_csv(path: str) -> List[KernelRecord]:
    """Records from a rocprofv3 kernel-trace CSV (one row per launch) or its stats CSV."""
    times: Dict[Tuple[str, str], List[float]] = defaultdict(list)
    with open(path, newline="") as f:
        rows = list(csv.DictReader(f))
    if not rows:
        return []
    cols = set(rows[0])
    if {"Kernel_Name", "Start_Timestamp", "End_Timestamp"} <= cols:
        for r in rows:
            times[(r["Kernel_Name"], "")].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        return records_from_times(times)
    if {"Name", "Calls", "TotalDurationNs"} <= cols:
        recs = [KernelRecord(r["Name"], classify_kernel(r["Name"]), float(r["TotalDurationNs"]) / 1e3,
                             int(r["Calls"])) for r in rows]
        recs.sort(key=lambda r: r.gpu_time_us, reverse=True)
        return recs
    raise ValueError(f"{path}: not a rocprofv3 kernel trace or kernel stats CSV (columns {sorted(cols)})")


def profile_live(model, inputs, warmup: int = WARMUP_ITERS, iters: int = PROFILE_ITERS) -> List[KernelRecord]:
    """Device kernel times of `iters` forwards under torch.profiler (profile.py:544-648)."""
    import torch
    with torch.no_grad():
        for _ in range(warmup):
            model(inputs)
        torch.cuda.synchronize()
        acts = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
        with torch.profiler.profile(activities=acts, record_shapes=True) as prof:
            for _ in range(iters):
                model(inputs)
                torch.cuda.synchronize()
    times: Dict[Tuple[str, str], List[float]] = defaultdict(list)
    cpu = torch.autograd.DeviceType.CPU
    for evt in prof.key_averages(group_by_input_shape=True):
        # Host events (aten::add, hipLaunchKernel) also carry the device time of the kernels they
        # launched; counting them as well would count those kernels twice. Keep device events.
        if getattr(evt, "device_type", None) == cpu:
            continue
        us = getattr(evt, "self_device_time_total", None) or getattr(evt, "self_cuda_time_total", 0)
        if us > 0:
            times[(evt.key, str(evt.input_shapes) if evt.input_shapes else "")] += [us / evt.count] * evt.count
    return records_from_times(times)


def build_report(records: List[KernelRecord], meta: dict, gpu, iters: int,
                 supported: Iterable[str] = SUPPORTED_OP_TYPES, speedup_per_kernel: float = 3.0) -> dict:
    """profile_report.json (profile.py:664-745): ranked kernels, cumulative share, roofline side,
    support, priority, and an Amdahl estimate with supported kernels `speedup_per_kernel` faster."""
    supported = set(supported)
    total = sum(r.gpu_time_us for r in records)
    top, cum, by_op = [], 0.0, defaultdict(float)
    for i, r in enumerate(records):
        pct = 100.0 * r.gpu_time_us / total if total > 0 else 0.0
        cum += pct
        by_op[r.op_type] += r.gpu_time_us
        top.append({
            "rank": i + 1, "name": r.name, "op_type": r.op_type, "shape_info": r.input_shapes,
            "gpu_time_ms": round(r.gpu_time_us / 1e3, 3), "call_count": r.call_count,
            "avg_time_us": round(r.gpu_time_us / max(r.call_count, 1), 2), "pct_total": round(pct, 1),
            "cumulative_pct": round(cum, 1), "roofline": roofline_position(r.op_type, r.gpu_time_us),
            "autokernel_supported": r.op_type in supported, "optimization_priority": priority_label(pct)})
    sup = sum(r.gpu_time_us for r in records if r.op_type in supported)
    f = sup / total if total > 0 else 0.0
    amdahl = 1.0 / ((1.0 - f) + f / speedup_per_kernel) if f > 0 else 1.0
    top5 = sum(r.gpu_time_us for r in records[:5])
    return {
        **meta,
        "gpu_name": gpu.name, "gpu_peak_tflops_fp16": gpu.peak_tflops_fp16,
        "gpu_peak_bandwidth_gb_s": gpu.peak_bandwidth_gb_s,
        "total_gpu_time_ms": round(total / 1e3, 3), "total_kernels": len(records), "profile_iters": iters,
        "top_kernels": top,
        "optimization_summary": {
            "supported_kernels_pct": round(100.0 * f, 1),
            "top5_pct": round(100.0 * top5 / total, 1) if total > 0 else 0.0,
            "estimated_max_speedup": f"{amdahl:.1f}x (Amdahl's law, f={f:.0%} supported, "
                                     f"{speedup_per_kernel:.0f}x per-kernel)"},
        "op_type_summary": {op: {"gpu_time_ms": round(t / 1e3, 3), "pct_total": round(100.0 * t / total, 1)}
                            for op, t in sorted(by_op.items(), key=lambda kv: -kv[1])} if total > 0 else {},
    }


def print_report(report: dict, limit: int = 20) -> None:
    print("=" * 72)
    print("  libak355 profiler (ROCm)")
    print("=" * 72)
    print(f"  Model: {report.get('model')}  input {report.get('input_shape')}  dtype {report.get('dtype')}")
    print(f"  GPU:   {report['gpu_name']}   total kernel time {report['total_gpu_time_ms']} ms")
    print(f"  {'rank':>4} {'op type':17s} {'ms':>9} {'%':>6} {'cum%':>6}  kernel")
    for k in report["top_kernels"][:limit]:
        print(f"  {k['rank']:4d} {k['op_type']:17s} {k['gpu_time_ms']:9.3f} {k['pct_total']:6.1f} "
              f"{k['cumulative_pct']:6.1f}  {k['name'][:70]}")
    s = report["optimization_summary"]
    print(f"  supported: {s['supported_kernels_pct']}%  top-5: {s['top5_pct']}%  estimate: {s['estimated_max_speedup']}")


def main(argv: Optional[List[str]] = None) -> int:
    ap = argparse.ArgumentParser(description="Rank a model's GPU kernels by time (ROCm-aware)")
    ap.add_argument("--model", default="small", help="7b, small, or a model .py file")
    ap.add_argument("--class-name", default=None)
    ap.add_argument("--input-shape", default="1,2048")
    ap.add_argument("--dtype", default="float16", choices=["float16", "bfloat16", "float32"])
    ap.add_argument("--kernels", default="none", help="none, all, or a comma list of ops to swap first")
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--trace", default=None, help="rocprofv3 kernel_trace.csv / kernel_stats.csv instead of a live run")
    ap.add_argument("--output", default="profile_report.json")
    args = ap.parse_args(argv)
    from .harness import GPUSpec, detect_gpu
    if args.trace:
        records = read_rocprof_csv(args.trace)
        meta = {"model": None, "class_name": None, "input_shape": None, "dtype": None, "source": args.trace}
        gpu, iters = detect_gpu() if _gpu_visible() else GPUSpec(), None
    else:
        import torch
        from . import verify
        if not torch.cuda.is_available():
            print("profile: no GPU visible (use --trace for a rocprofv3 CSV)", file=sys.stderr)
            return 1
        dtype = getattr(torch, args.dtype)
        dev = torch.device("cuda")
        model = verify._load_model(args, dtype, dev)
        shape = tuple(int(s) for s in args.input_shape.split(","))
        ids = verify.make_token_ids(model, shape, dev)
        kinds = () if args.kernels == "none" else (verify.ALL_KERNELS if args.kernels == "all"
                                                   else tuple(args.kernels.split(",")))
        with verify.OptimizedModelContext(model, kinds) as m:
            records = profile_live(m, ids)
        meta = {"model": args.model, "class_name": args.class_name, "input_shape": list(shape),
                "dtype": args.dtype, "kernels_swapped": list(kinds), "source": "torch.profiler"}
        gpu, iters = detect_gpu(), PROFILE_ITERS
    report = build_report(records, meta, gpu, iters)
    with open(args.output, "w") as f:
        json.dump(report, f, indent=2)
    print_report(report)
    print(f"  report: {os.path.abspath(args.output)}")
    return 0


def _gpu_visible() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001 - no torch / no runtime: report without GPU facts
        return False


if __name__ == "__main__":
    sys.exit(main())

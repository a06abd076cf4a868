"""Counter evidence for the roofline claims (run under rocprofv3 --pmc).

HBM traffic of the bandwidth-bound kernels (`run` / `summarize`) and MFMA / LDS activity of the
matrix kernels (`run_mfma` / `summarize_mfma`):

    rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE \
        --kernel-trace -d DIR -o mfma_a --output-format csv -- python -m autokernel_amd.roofline_probe run_mfma
    rocprofv3 --pmc SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS SQ_WAVE_CYCLES \
        -d DIR -o mfma_b --output-format csv -- python -m autokernel_amd.roofline_probe run_mfma
    python -m autokernel_amd.roofline_probe summarize_mfma DIR

HBM traffic of the bandwidth-bound kernels:

    rocprofv3 --pmc FETCH_SIZE -d DIR -o fetch --output-format csv -- python -m autokernel_amd.roofline_probe run
    rocprofv3 --pmc WRITE_SIZE -d DIR -o write --output-format csv -- python -m autokernel_amd.roofline_probe run
    python -m autokernel_amd.roofline_probe summarize DIR > profiles/hbm_traffic_row_ops.md

`run` launches a plain device copy of a known size (calibration: FETCH_SIZE / WRITE_SIZE of a
copy that must move exactly its buffer size gives the counters' scale) and then each HBM-bound
kernel at its BASELINE / harness-primary shape, three times each, with the Infinity Cache
flushed before every launch. `summarize` averages the counters per dispatch, scales them by the
copy calibration, and writes profiles/traffic.json (HBM bytes per launch) next to the markdown.
"""
from __future__ import annotations

import csv
import glob
import json
import os
import sys
from collections import defaultdict

COPY_BYTES = 512 * 2 ** 20
PROBES = {  # kernel-name fragment -> (key, algorithmic bytes per launch)
    "softmax_rows": ("softmax_f16_8192x8192", 2 * 8192 * 8192 * 2),
    "rmsnorm_rows": ("rmsnorm_f16_4096x4096", (2 * 4096 * 4096 + 4096) * 2),
    "rope_vec": ("rope_f16_1x32x2048x128", (2 * 32 * 2048 * 128 + 2048 * 128) * 2),
    "layernorm_rows": ("layernorm_f16_4096x2048", (2 * 4096 * 2048 + 2 * 2048) * 2),
    "ce_rows": ("cross_entropy_f16_4096x32000", (4096 * 32000 + 4096) * 2),
    "reduce_rows": ("reduce_f16_8192x8192", (8192 * 8192 + 8192) * 2),
}


def run() -> None:
    import torch

    from . import kernels, spec
    dev = torch.device("cuda:0")
    flush = torch.empty(512 * 2 ** 20, dtype=torch.uint8, device=dev)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    calls = []
    s = spec.baseline_softmax(device=dev)
    calls.append(lambda: kernels.get("softmax")(s["x"]))
    r = spec.baseline_rmsnorm(device=dev)
    calls.append(lambda: kernels.get("rmsnorm")(r["x"], r["weight"]))
    q = spec.baseline_rope(device=dev)
    calls.append(lambda: kernels.get("rotary_embedding")(q["q"], q["cos"], q["sin"]))
    x = torch.randn(4096, 2048, device=dev, dtype=torch.float16)
    w, b = torch.ones(2048, device=dev, dtype=torch.float16), torch.zeros(2048, device=dev, dtype=torch.float16)
    calls.append(lambda: kernels.get("layernorm")(x, w, b))
    ce = spec.gen_cross_entropy({"batch": 4096, "vocab": 32000}, torch.float16, dev)
    calls.append(lambda: kernels.get("cross_entropy")(**ce))
    xr = spec.gen_reduce({"M": 8192, "N": 8192}, torch.float16, dev)["x"]
    calls.append(lambda: kernels.get("reduce")(xr))
    for _ in range(3):
        flush.zero_()
        dst.copy_(src)
    for c in calls:
        for _ in range(3):
            flush.zero_()
            c()
    torch.cuda.synchronize()
    print("roofline_probe: done", flush=True)


SPEC_CLOCK_GHZ = 2.4  # MI355X peak engine clock, the clock the 2516.6 TFLOP/s dense figure assumes
PEAK_TFLOPS = 2516.6
# (kernel-name fragment, label, flops per launch, the call that launches it); each probe runs
# three times in this order, so dispatches are assigned to probes by order and name
MFMA_PROBES = [
    ("gemm_dma<ak::TBF16, 256, 256, 2, 4, 1, 0, 64, 2, true", "matmul bf16 4096^3 (NN: [K, N] B, LDS-DMA)",
     2 * 4096 ** 3, "matmul4k"),
    ("gemm_dma<ak::TBF16, 256, 256, 2, 4, 1, 0, 64, 2, false", "matmul bf16 8192^3 (NT: nn.Linear B, LDS-DMA)",
     2 * 8192 ** 3, "matmul8k"),
    ("gemm_dma<ak::TBF16, 256, 128, 2, 4, 2, 1", "fused_mlp gate/up bf16 2048x4096 H=11008",
     2 * 2048 * 4096 * 11008 * 2, "mlp"),
    ("gemm_dma<ak::TBF16, 256, 128, 4, 2, 1, 0", "fused_mlp down bf16 2048x4096 K=11008", 2 * 2048 * 4096 * 11008,
     "mlp"),
    ("fa_fwd2<ak::TF16, 128, 1>", "flash_attention f16 causal [4,32,2048,128]", 2 * 2 * 4 * 32 * 128 * (2048 * 2049 // 2),
     "fa2k"),
    ("fa_fwd2<ak::TF16, 128, 1>", "flash_attention f16 causal [1,32,8192,128]", 2 * 2 * 32 * 128 * (8192 * 8193 // 2),
     "fa8k"),
    ("gemm_dma<ak::TBF16, 256, 256, 2, 4, 1, 0, 64, 2, false", "matmul bf16 4096^3 (NT: nn.Linear B, LDS-DMA)",
     2 * 4096 ** 3, "matmul4knt"),
    # stock torch.matmul on the same operands (the hipBLASLt kernels this image's library picks)
    ("Cijk_Ailk_Bljk_BBS_BH_Bias_HA_S_SAV_UserArgs_MT256x256x64", "stock hipBLASLt: matmul bf16 4096^3 NN",
     2 * 4096 ** 3, "blas4k"),
    ("Custom_Cijk_Alik_Bljk_BBS_BH_Bias_HA_S_SAV_NTD_SK3_UserArgs_MT256x256x64", "stock hipBLASLt: matmul bf16 4096^3 NT",
     2 * 4096 ** 3, "blas4knt"),
    ("Custom_Cijk_Alik_Bljk_BBS_BH_MT256x256x64_MI16x16x1_UserArgs", "stock hipBLASLt: matmul bf16 8192^3 NT",
     2 * 8192 ** 3, "blas8k"),
]


def run_mfma() -> None:
    import torch

    from . import kernels, spec
    dev = torch.device("cuda:0")
    flush = torch.empty(512 * 2 ** 20, dtype=torch.uint8, device=dev)
    # the calibration copy of `run` (FETCH_SIZE / WRITE_SIZE scale), before the matrix kernels
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        flush.zero_()
        dst.copy_(src)
    del src, dst
    m = spec.baseline_matmul(device=dev)
    g = torch.Generator(device=dev).manual_seed(0)
    a8 = (torch.randn(8192, 8192, device=dev, generator=g) / 8192 ** 0.5).bfloat16()
    w8 = torch.randn(8192, 8192, device=dev, generator=g).bfloat16()
    f = spec.baseline_fused_mlp(device=dev)
    a = spec.baseline_attention(device=dev)
    a_long = spec.baseline_attention(device=dev, B=1, S=8192)
    w4 = torch.randn(4096, 4096, device=dev, generator=g).bfloat16()
    calls = {"matmul4k": lambda: kernels.get("matmul")(m["A"], m["B"]),
             "matmul4knt": lambda: kernels.get("matmul")(m["A"], w4.t()),
             "blas4k": lambda: torch.matmul(m["A"], m["B"]),
             "blas4knt": lambda: torch.matmul(m["A"], w4.t()),
             "blas8k": lambda: torch.matmul(a8, w8.t()),
             "matmul8k": lambda: kernels.get("matmul")(a8, w8.t()),
             "mlp": lambda: kernels.get("fused_mlp")(**f),
             "fa2k": lambda: kernels.get("flash_attention")(**a),
             "fa8k": lambda: kernels.get("flash_attention")(**a_long)}
    for key in dict.fromkeys(p[3] for p in MFMA_PROBES):
        for _ in range(3):
            flush.zero_()
            calls[key]()
    torch.cuda.synchronize()
    print("roofline_probe: done", flush=True)


def _dispatches(dirpath: str):
    """[(dispatch id, kernel name, {counter: value}, duration ns or None)] in dispatch order, from
    the counter_collection CSVs and, where the pass also ran --kernel-trace, its kernel_trace CSV."""
    out = []
    for path in glob.glob(os.path.join(dirpath, "**", "*counter_collection*.csv"), recursive=True):
        dur = {}
        kt = path.replace("counter_collection", "kernel_trace")
        if os.path.exists(kt):
            with open(kt) as f:
                for row in csv.DictReader(f):
                    dur[row["Dispatch_Id"]] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
        per = {}
        with open(path) as f:
            for row in csv.DictReader(f):
                d = per.setdefault(row["Dispatch_Id"], (row["Kernel_Name"], defaultdict(float)))
                d[1][row["Counter_Name"]] += float(row["Counter_Value"])
        out.append([(int(i), n, dict(c), dur.get(i)) for i, (n, c) in per.items()])
    return [sorted(o) for o in out]


def summarize_mfma(dirpath: str) -> None:
    passes = _dispatches(dirpath)
    # per probe: counters summed over the passes, durations from the pass that traced kernels
    rows = []
    for pi, (frag, label, flops, _) in enumerate(MFMA_PROBES):
        ctr, durs = defaultdict(list), []
        for disp in passes:
            # probes with the same fragment take consecutive groups of three launches, in order
            same = [x for x in disp if frag in x[1]]
            k = sum(1 for q in MFMA_PROBES[:pi] if q[0] == frag)
            for _, name, c, d in same[3 * k:3 * k + 3]:
                for n, v in c.items():
                    ctr[n].append(v)
                if d:
                    durs.append(d)
        if not ctr:
            continue
        rows.append((frag, label, flops, {n: sum(v) / len(v) for n, v in ctr.items()},
                     sum(durs) / len(durs) if durs else None))

    lines = ["# MFMA and LDS activity of the matrix kernels (rocprofv3 PMC)", "",
             "Commands (two counter passes, the first with the kernel trace, then the summary):", "",
             "    rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE --kernel-trace -d DIR -o mfma_a --output-format csv -- python -m autokernel_amd.roofline_probe run_mfma",
             "    rocprofv3 --pmc SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS SQ_WAVE_CYCLES -d DIR -o mfma_b --output-format csv -- python -m autokernel_amd.roofline_probe run_mfma",
             "    python -m autokernel_amd.roofline_probe summarize_mfma DIR", "",
             "* MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 256 CUs x 4 SIMDs).",
             "* Sustained clock = GRBM_GUI_ACTIVE / 8 / kernel duration (same launch, profiled).",
             f"* Clock-scaled peak = {PEAK_TFLOPS} TFLOP/s x clock / {SPEC_CLOCK_GHZ} GHz: what 100 % MFMA busy would give at",
             "  the clock the kernel actually ran at. TFLOP/s here are from the profiled durations (counter",
             "  collection slows kernels by a few percent; bench.py's figures are the unprofiled ones).",
             "* LDS bank-conflict rate = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE (the rocprof-compute",
             "  definition). Averages over three launches per workload, caches flushed before each.", "",
             "| kernel | workload | TFLOP/s (profiled) | % of spec peak | sustained clock | MFMA busy | % of clock-scaled peak | LDS bank-conflict rate | VALU active / wave-cycle | LDS active / wave-cycle | LDS wait / wave-cycle |",
             "|---|---|---|---|---|---|---|---|---|---|---|"]
    for frag, label, flops, c, dur in rows:
        grbm = c.get("GRBM_GUI_ACTIVE", float("nan")) / 8  # summed over the 8 XCDs
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", float("nan")) / (grbm * 256 * 4)
        conf = c.get("SQ_LDS_BANK_CONFLICT", 0.0) / max(c.get("SQ_LDS_IDX_ACTIVE", 0.0), 1.0)
        wc = max(c.get("SQ_WAVE_CYCLES", 0.0), 1.0)
        if dur:
            tf = flops / (dur * 1e-9) / 1e12
            clk = grbm / (dur * 1e-9) / 1e9
            perf = f"{tf:.0f} | {100 * tf / PEAK_TFLOPS:.1f}% | {clk:.2f} GHz"
            scaled = f"{100 * tf / (PEAK_TFLOPS * clk / SPEC_CLOCK_GHZ):.1f}%"
        else:
            perf, scaled = "n/a | n/a | n/a", "n/a"
        lines.append(f"| {frag.split('(')[0]} | {label} | {perf} | {100 * busy:.1f}% | {scaled} | {100 * conf:.1f}% | "
                     f"{c.get('SQ_ACTIVE_INST_VALU', 0.0) / wc:.3f} | {c.get('SQ_ACTIVE_INST_LDS', 0.0) / wc:.3f} | "
                     f"{c.get('SQ_WAIT_INST_LDS', 0.0) / wc:.3f} |")
    print("\n".join(lines))


STALL_PASSES = (
    "SQ_VALU_MFMA_BUSY_CYCLES SQ_VALU_MFMA_COEXEC_CYCLES SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_VALU2 SQ_INSTS_VALU "
    "SQ_INSTS_MFMA SQ_WAVE_CYCLES SQ_BUSY_CYCLES GRBM_GUI_ACTIVE",
    "SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY SQ_ACTIVE_INST_LDS SQ_LDS_DATA_FIFO_FULL SQ_LDS_CMD_FIFO_FULL "
    "SQ_INSTS_LDS_LOAD_BANDWIDTH SQ_WAVE_CYCLES GRBM_GUI_ACTIVE",
)


def summarize_mfma_stall(dirpath: str) -> None:
    """Where the matrix kernels' SIMD cycles go: MFMA busy, VALU issued beside a busy MFMA unit,
    time waves spend in s_waitcnt / s_barrier or ready but not issued, LDS pressure."""
    passes = _dispatches(dirpath)
    lines = ["# Issue and stall counters of the matrix kernels (rocprofv3 PMC)", "",
             "Commands (two counter passes of eight SQ counters each, then the summary):", ""]
    lines += [f"    rocprofv3 --pmc {p} -d DIR -o stall_{'ab'[i]} --output-format csv -- "
              "python -m autokernel_amd.roofline_probe run_mfma" for i, p in enumerate(STALL_PASSES)]
    lines += ["    python -m autokernel_amd.roofline_probe summarize_mfma_stall DIR", "",
              "* SIMD-cycles = GRBM_GUI_ACTIVE / 8 XCDs x 256 CUs x 4 SIMDs. MFMA busy and MFMA + VALU co-issue",
              "  (SQ_VALU_MFMA_COEXEC_CYCLES: a VALU instruction issued while the MFMA unit was busy) are per",
              "  SIMD-cycle.",
              "* Wave-time shares are per SQ_WAVE_CYCLES: VALU active (SQ_ACTIVE_INST_VALU), waiting in",
              "  s_waitcnt / s_barrier (SQ_WAIT_ANY), ready but not issued because the unit or port it needs",
              "  was taken (SQ_WAIT_INST_ANY; with two waves per SIMD this includes the other wave's MFMAs).",
              "* LDS command FIFO full: SQ_LDS_CMD_FIFO_FULL per shader engine (32) per kernel cycle.",
              "* LDS bytes per MFMA: SQ_INSTS_LDS_LOAD_BANDWIDTH x 64 / SQ_INSTS_MFMA (16x16x32 MFMAs in the",
              "  GEMMs, 32x32x16 in attention, 16 and 32 KFLOP each). Three launches per workload.", "",
              "| kernel | workload | MFMA busy | MFMA + VALU co-issue | VALU instr. per MFMA | VALU active | "
              "in s_waitcnt / s_barrier | ready, not issued | LDS cmd FIFO full | LDS bytes per MFMA |",
              "|---|---|---|---|---|---|---|---|---|---|"]
    for pi, (frag, label, _flops, _) in enumerate(MFMA_PROBES):
        k = sum(1 for q in MFMA_PROBES[:pi] if q[0] == frag)
        ctr = defaultdict(list)
        for disp in passes:
            same = [x for x in disp if frag in x[1]]
            for _, _name, c, _d in same[3 * k:3 * k + 3]:
                for n, v in c.items():
                    ctr[n].append(v)
        if not ctr:
            continue
        c = {n: sum(v) / len(v) for n, v in ctr.items()}
        nan = float("nan")
        grbm = c.get("GRBM_GUI_ACTIVE", nan) / 8
        simd = grbm * 256 * 4
        wc = c.get("SQ_WAVE_CYCLES", nan)
        mfma = c.get("SQ_INSTS_MFMA", nan)
        lines.append(
            f"| {frag.split('(')[0]} | {label} | {100 * c.get('SQ_VALU_MFMA_BUSY_CYCLES', nan) / simd:.1f}% | "
            f"{100 * c.get('SQ_VALU_MFMA_COEXEC_CYCLES', nan) / simd:.1f}% | "
            f"{(c.get('SQ_INSTS_VALU', nan) - mfma) / mfma:.1f} | {100 * c.get('SQ_ACTIVE_INST_VALU', nan) / wc:.0f}% | "
            f"{100 * c.get('SQ_WAIT_ANY', nan) / wc:.0f}% | {100 * c.get('SQ_WAIT_INST_ANY', nan) / wc:.0f}% | "
            f"{100 * c.get('SQ_LDS_CMD_FIFO_FULL', nan) / 32 / grbm:.1f}% | "
            f"{64 * c.get('SQ_INSTS_LDS_LOAD_BANDWIDTH', nan) / mfma:.0f} |")
    print("\n".join(lines))


# unique bytes each matrix workload must move at least once (inputs read, output written)
MFMA_IDEAL_BYTES = {
    "matmul4k": 3 * 4096 * 4096 * 2,
    "matmul8k": 3 * 8192 * 8192 * 2,
    "mlp_gateup": (2048 * 4096 + 2 * 11008 * 4096 + 2048 * 11008) * 2,
    "mlp_down": (2048 * 11008 + 4096 * 11008 + 2048 * 4096) * 2,
    "fa2k": 4 * 4 * 32 * 2048 * 128 * 2,
    "fa8k": 4 * 32 * 8192 * 128 * 2,
    "matmul4knt": 3 * 4096 * 4096 * 2,
    "blas4k": 3 * 4096 * 4096 * 2,
    "blas4knt": 3 * 4096 * 4096 * 2,
    "blas8k": 3 * 8192 * 8192 * 2,
}


def summarize_mfma_traffic(dirpath: str) -> None:
    """Traffic past L2 (FETCH_SIZE / WRITE_SIZE, calibrated on the copy) and the L2 hit rate of each
    matrix kernel against the unique bytes its workload must move, per GFLOP."""
    passes = _dispatches(dirpath)
    allrows = [x for disp in passes for x in disp]
    cal = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        vals = [c[ctr] for _, n, c, _ in allrows if ctr in c and ("copy" in n.lower() or "elementwise" in n.lower())
                and c[ctr] * 1024 > COPY_BYTES / 4]
        cal[ctr] = COPY_BYTES / (1024 * sum(vals) / len(vals)) if vals else 1.0
    keys = ["matmul4k", "matmul8k", "mlp_gateup", "mlp_down", "fa2k", "fa8k", "matmul4knt", "blas4k", "blas4knt", "blas8k"]
    lines = ["# Traffic past L2 of the matrix kernels (rocprofv3 PMC)", "",
             "Commands (one counter group per run):", "",
             "    rocprofv3 --pmc FETCH_SIZE -d DIR -o fetch --output-format csv -- python -m autokernel_amd.roofline_probe run_mfma",
             "    rocprofv3 --pmc WRITE_SIZE -d DIR -o write --output-format csv -- python -m autokernel_amd.roofline_probe run_mfma",
             "    rocprofv3 --pmc TCC_HIT_sum TCC_MISS_sum -d DIR -o l2 --output-format csv -- python -m autokernel_amd.roofline_probe run_mfma",
             "    python -m autokernel_amd.roofline_probe summarize_mfma_traffic DIR", "",
             f"FETCH / WRITE_SIZE count bytes leaving the L2s for the fabric (Infinity Cache or HBM), scaled by a "
             f"{COPY_BYTES >> 20} MiB copy: FETCH x{cal['FETCH_SIZE']:.3f}, WRITE x{cal['WRITE_SIZE']:.3f}. Unique = the "
             "bytes the workload must move at least once. Three launches each, caches flushed before every launch.", "",
             "| kernel | workload | GFLOP | unique MB | fetched MB | written MB | fetched / unique | bytes past L2 per FLOP | L2 hit rate |",
             "|---|---|---|---|---|---|---|---|---|"]
    for pi, (frag, label, flops, _) in enumerate(MFMA_PROBES):
        k = sum(1 for q in MFMA_PROBES[:pi] if q[0] == frag)
        ctr = defaultdict(list)
        for disp in passes:
            same = [x for x in disp if frag in x[1]]
            for _, name, c, _d in same[3 * k:3 * k + 3]:
                for n, v in c.items():
                    ctr[n].append(v)
        if not ctr:
            continue
        c = {n: sum(v) / len(v) for n, v in ctr.items()}
        fetch = c.get("FETCH_SIZE", float("nan")) * 1024 * cal["FETCH_SIZE"]
        write = c.get("WRITE_SIZE", float("nan")) * 1024 * cal["WRITE_SIZE"]
        hit = c.get("TCC_HIT_sum", float("nan")) / max(c.get("TCC_HIT_sum", 0.0) + c.get("TCC_MISS_sum", 0.0), 1.0)
        uniq = MFMA_IDEAL_BYTES[keys[pi]]
        lines.append(f"| {frag.split('(')[0]} | {label} | {flops / 1e9:.1f} | {uniq / 1e6:.1f} | {fetch / 1e6:.1f} | "
                     f"{write / 1e6:.1f} | {fetch / uniq:.2f} | {(fetch + write) / flops:.4f} | {100 * hit:.1f}% |")
    print("\n".join(lines))


def _read(dirpath: str):
    """{kernel name: {counter: [values per dispatch]}} from rocprofv3 counter_collection CSVs."""
    out = defaultdict(lambda: defaultdict(list))
    for path in glob.glob(os.path.join(dirpath, "**", "*counter_collection*.csv"), recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                out[row["Kernel_Name"]][row["Counter_Name"]].append(float(row["Counter_Value"]))
    return out


def summarize(dirpath: str) -> None:
    data = _read(dirpath)
    copy = [v for k, v in data.items() if "copy" in k.lower() or "elementwise" in k.lower() and "fill" not in k.lower()]
    cal = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        vals = [x for d in copy for x in d.get(ctr, [])]
        big = [x for x in vals if x * 1024 > COPY_BYTES / 4]  # the 512 MiB copy, not small fills
        cal[ctr] = (COPY_BYTES / (1024 * sum(big) / len(big))) if big else None
    lines = ["# HBM traffic of the bandwidth-bound kernels (rocprofv3 PMC)", "",
             "Command (each counter in its own run):", "",
             "    rocprofv3 --pmc FETCH_SIZE -d DIR -o fetch --output-format csv -- python -m autokernel_amd.roofline_probe run",
             "    rocprofv3 --pmc WRITE_SIZE -d DIR -o write --output-format csv -- python -m autokernel_amd.roofline_probe run",
             "    python -m autokernel_amd.roofline_probe summarize DIR", "",
             f"Calibration: a {COPY_BYTES >> 20} MiB device copy reads and writes exactly {COPY_BYTES >> 20} MiB; "
             f"scale FETCH x{cal['FETCH_SIZE']:.3f}, WRITE x{cal['WRITE_SIZE']:.3f} (counter KiB -> bytes)." if all(cal.values())
             else "Calibration copy not found: raw KiB x 1024 used.", "",
             "| kernel | shape | algorithmic bytes | FETCH bytes | WRITE bytes | traffic / algorithmic |",
             "|---|---|---|---|---|---|"]
    traffic = {}
    for frag, (key, alg) in PROBES.items():
        rows = [(k, v) for k, v in data.items() if frag in k]
        if not rows:
            continue
        name, d = rows[0]
        fetch = sum(d.get("FETCH_SIZE", [0])) / max(len(d.get("FETCH_SIZE", [])), 1) * 1024 * (cal["FETCH_SIZE"] or 1)
        write = sum(d.get("WRITE_SIZE", [0])) / max(len(d.get("WRITE_SIZE", [])), 1) * 1024 * (cal["WRITE_SIZE"] or 1)
        traffic[key] = {"hbm_bytes_per_launch": int(fetch + write), "fetch_bytes": int(fetch), "write_bytes": int(write),
                        "algorithmic_bytes": alg}
        lines.append(f"| {name[:60]} | {key} | {alg} | {int(fetch)} | {int(write)} | {(fetch + write) / alg:.3f} |")
    print("\n".join(lines))
    here = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    with open(os.path.join(here, "profiles", "traffic.json"), "w") as f:
        json.dump(traffic, f, indent=1)


if __name__ == "__main__":
    cmd = sys.argv[1] if len(sys.argv) > 1 else "run"
    if cmd == "summarize":
        summarize(sys.argv[2])
    elif cmd == "summarize_mfma":
        summarize_mfma(sys.argv[2])
    elif cmd == "summarize_mfma_traffic":
        summarize_mfma_traffic(sys.argv[2])
    elif cmd == "summarize_mfma_stall":
        summarize_mfma_stall(sys.argv[2])
    elif cmd == "run_mfma":
        run_mfma()
    else:
        run()

"""HBM traffic evidence for the bandwidth-bound kernels (run under rocprofv3 --pmc).

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
    if len(sys.argv) > 1 and sys.argv[1] == "summarize":
        summarize(sys.argv[2])
    else:
        run()

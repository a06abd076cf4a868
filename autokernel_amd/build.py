"""Build libak355.so (the gfx950 kernels and their C ABI) in-tree with hipcc.

    python -m autokernel_amd.build            # compile every source, link autokernel_amd/libak355.so

Each ``csrc/*.hip`` compiles to an object under ``autokernel_amd/_build/`` in parallel, then one
``hipcc -shared`` links them. No CMake, no JIT cache: the library sits next to this file so it
travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libak355.so"
ARCH = "gfx950"

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in generated code. The host pass warns that it
# does not know the feature; that warning is expected.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found: set HIPCC or install ROCm (/opt/rocm/bin/hipcc)")
    return cand


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, extra: list[str]) -> tuple[Path, str]:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    # keep only real diagnostics (drop the expected host-pass feature warning)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (proc.stderr or "").splitlines() if noise not in l)
    # inline assembly must not write a register the compiler reserves (M0 is an asm input bound with
    # "{m0}" instead): such a clobber is not preserved and its value may be live across the statement
    if "clobber list contains reserved registers" in msgs:
        raise RuntimeError(f"{src.name}: inline asm clobbers a reserved register:\n{msgs[:2000]}")
    return obj, msgs


def build(verbose: bool = True, jobs: int | None = None, extra_flags: list[str] | None = None,
          out: Path | None = None, build_dir: Path | None = None) -> Path:
    """Compile every HIP source for gfx950 and link ``libak355.so``. Always rebuilds.

    extra_flags / out / build_dir produce a variant library elsewhere (tuning builds)."""
    global BUILD_DIR
    t0 = time.time()
    lib_path = Path(out) if out else LIB_PATH
    saved = BUILD_DIR
    if build_dir:
        BUILD_DIR = Path(build_dir)
    try:
        return _build(verbose, jobs, extra_flags, lib_path, t0)
    finally:
        BUILD_DIR = saved


def _build(verbose, jobs, extra_flags, lib_path: Path, t0: float) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    extra = list(extra_flags or [])
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    objs: list[Path] = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = {ex.submit(_compile, s, extra): s for s in srcs}
        for fut in cf.as_completed(futs):
            obj, msgs = fut.result()
            objs.append(obj)
            if verbose and msgs.strip():
                print(msgs, file=sys.stderr)
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, sorted(objs))]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path} from {len(srcs)} sources in {time.time() - t0:.1f}s")
    return lib_path


if __name__ == "__main__":
    build()

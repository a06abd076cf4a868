"""Export libak355 as a HuggingFace Kernels project for the ROCm backend (gfx950).

Counterpart of the reference's export_hf.py, which packages one CUDA or Triton kernel file for
the CUDA backend: build.toml (export_hf.py:269-326), a TORCH_LIBRARY_EXPAND binding
(:367-418), flake.nix for kernel-builder (:423-444), the module's __init__.py (:450-489) and
the export_kernel / CLI flow (:674-864). Here the kernels are libak355's hand-written HIP sources
and its C ABI, so the project holds:

    <name>/build.toml                    backends = ["rocm"], rocm-archs = ["gfx950"], the HIP flags
    <name>/flake.nix                     kernel-builder entry (same role as the reference's)
    <name>/README.md
    <name>/include/ak355.h               the C ABI
    <name>/<name>_rocm/csrc/*            libak355's HIP sources and headers, unchanged
    <name>/torch-ext/torch_binding.cpp   one torch op per C entry point (TORCH_LIBRARY_EXPAND)
    <name>/torch-ext/torch_binding.h
    <name>/torch-ext/<name>/__init__.py  kernel_fn of the chosen op type (or every op), KERNEL_TYPE
    <name>/torch-ext/<name>/_host.py     the reference kernel_fn semantics over the torch ops: the
                                         in-tree autokernel_amd/kernels/host.py, copied unchanged

The op type comes from --op, else from the KERNEL_TYPE line of the kernel file (the reference's
detect_kernel_type, export_hf.py:87-92); "all" exports every op as a named function.

    python -m autokernel_amd.export_hf --name ak_rmsnorm --op rmsnorm --repo-id me/ak-rmsnorm
"""
from __future__ import annotations

import argparse
import os
import re
import shutil
import subprocess
import sys
import textwrap
from pathlib import Path

from . import build as _build

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
TEMPLATE_DIR = PKG_DIR / "hf_export"
HEADER = REPO_ROOT / "include" / "ak355.h"
# the kernel_fn shape / dtype layer, shared with the in-tree package and shipped unchanged
HOST_LAYER = PKG_DIR / "kernels" / "host.py"
DEFAULT_KERNEL_PATH = REPO_ROOT / "kernel.py"
DEFAULT_OUTPUT_DIR = REPO_ROOT / "workspace" / "hf_export"
ROCM_ARCHS = (_build.ARCH,)
# every flag of build.HIP_FLAGS except the arch (rocm-archs carries it)
HIP_FLAGS = tuple(f for f in _build.HIP_FLAGS if not f.startswith("--offload-arch"))

OP_TYPES = ("rmsnorm", "layernorm", "softmax", "rotary_embedding", "cross_entropy", "reduce",
            "matmul", "fused_mlp", "flash_attention")
# torch ops (torch_binding.cpp) each op type's kernel_fn calls
OP_BINDINGS = {
    "rmsnorm": ("rmsnorm",),
    "layernorm": ("layernorm",),
    "softmax": ("softmax",),
    "rotary_embedding": ("rope",),
    "cross_entropy": ("cross_entropy",),
    "reduce": ("reduce_sum", "reduce_max"),
    "matmul": ("gemm", "gemm_batched", "gemm_workspace_bytes"),
    "fused_mlp": ("mlp_gate_up", "gemm"),
    "flash_attention": ("flash_attn_fwd",),
}


def detect_kernel_type(source: str) -> str | None:
    """The KERNEL_TYPE declared at module level of a kernel file, if any."""
    m = re.search(r'^KERNEL_TYPE\s*=\s*["\'](\w+)["\']', source, re.MULTILINE)
    return m.group(1) if m else None


def kernel_sources() -> list[Path]:
    """libak355's HIP sources and headers, sorted (the library is one unit: every op ships all)."""
    return sorted(p for p in _build.CSRC.iterdir() if p.suffix in (".hip", ".h"))


def _toml_list(items, indent: str = "  ") -> str:
    return "[\n" + "".join(f'{indent}"{i}",\n' for i in items) + "]"


def generate_build_toml(name: str, repo_id: str, src: list[str]) -> str:
    return (
        "[general]\n"
        f'name = "{name}"\n'
        'license = "Apache-2.0"\n'
        "version = 1\n"
        'backends = ["rocm"]\n'
        "\n"
        "[general.hub]\n"
        f'repo-id = "{repo_id}"\n'
        "\n"
        "[torch]\n"
        f"src = {_toml_list(['torch-ext/torch_binding.cpp', 'torch-ext/torch_binding.h'])}\n"
        "\n"
        f"[kernel.{name}]\n"
        'backend = "rocm"\n'
        f"rocm-archs = {_toml_list(ROCM_ARCHS)}\n"
        'depends = ["torch"]\n'
        'include = ["include"]\n'
        "# packed fp32 VALU forms stay off; -O3, C++17 (the flags libak355 is validated with)\n"
        f"hip-flags = {_toml_list(HIP_FLAGS)}\n"
        f"src = {_toml_list(src)}\n"
    )


def generate_flake_nix(name: str) -> str:
    return textwrap.dedent(f"""\
        {{
          description = "Flake for the {name} ROCm kernels (libak355, gfx950)";

          inputs = {{
            kernel-builder.url = "github:huggingface/kernels";
          }};

          outputs =
            {{
              self,
              kernel-builder,
            }}:
            kernel-builder.lib.genKernelFlakeOutputs {{
              inherit self;
              path = ./.;
            }};
        }}
    """)


def generate_init_py(name: str, repo_id: str, op: str) -> str:
    funcs = ", ".join(OP_TYPES) + ", reduce_max"
    if op == "all":
        tail = "KERNEL_TYPE = None\nKERNEL_FNS = _host.KERNEL_FNS\n"
        use = "module.rmsnorm(x, weight)"
    else:
        tail = f'KERNEL_TYPE = "{op}"\nkernel_fn = _host.KERNEL_FNS[KERNEL_TYPE]\n'
        use = "module.kernel_fn(...)"
    return (
        f'"""{name}: AutoKernel ops on hand-written HIP kernels for MI355X (gfx950), libak355.\n'
        "\n"
        "Usage:\n"
        "    from kernels import get_kernel\n"
        f'    module = get_kernel("{repo_id}")\n'
        f"    result = {use}\n"
        '"""\n'
        "from ._ops import ops\n"
        "from . import _host\n"
        "\n"
        "_host.bind(ops)\n"
        f"from ._host import {funcs}  # noqa: E402,F401\n"
        "\n"
        + tail
    )


def generate_readme(name: str, repo_id: str, op: str) -> str:
    ops_line = "every op of the suite" if op == "all" else f"`{op}` (kernel_fn)"
    return textwrap.dedent(f"""\
        # {name}

        AutoKernel's kernel suite on hand-written HIP kernels for AMD Instinct MI355X (gfx950):
        libak355. Exports {ops_line} with the signature and semantics of the reference's
        `kernel_fn` (reference.py). The torch ops are thin wrappers over libak355's C ABI
        (`include/ak355.h`); `_host.py` does the shape handling.

        ## Build

        `build.toml` targets the ROCm backend for gfx950 only. The HIP sources must be compiled
        with the flags under `hip-flags` (packed fp32 VALU forms disabled).

            nix flake lock
            nix run -L .#build-and-copy

        ## Use

        ```python
        from kernels import get_kernel
        module = get_kernel("{repo_id}")
        ```

        ## Requirements

        - PyTorch built for ROCm
        - AMD Instinct MI355X (gfx950)
    """)


def export_kernel(name: str, output_dir: str | Path = DEFAULT_OUTPUT_DIR, repo_id: str | None = None,
                  op: str | None = None, kernel_path: str | Path | None = None, verbose: bool = True) -> Path:
    """Write the project to output_dir/name and return its path. ValueError on a bad name or op."""
    if not name.isidentifier():
        raise ValueError(f"'{name}' is not a valid Python identifier (try e.g. 'ak_matmul')")
    if op is None:
        kp = Path(kernel_path or DEFAULT_KERNEL_PATH)
        if not kp.is_file():
            raise ValueError(f"kernel file not found: {kp}")
        op = detect_kernel_type(kp.read_text(encoding="utf-8"))
        if op is None:
            raise ValueError(f"{kp} declares no KERNEL_TYPE; pass --op")
    if op != "all" and op not in OP_TYPES:
        raise ValueError(f"unknown op type {op!r} (one of {', '.join(OP_TYPES)}, or 'all')")
    repo_id = repo_id or f"your-username/{name}"

    project = Path(output_dir) / name
    src_dir = project / f"{name}_rocm" / "csrc"
    inc_dir = project / "include"
    ext_dir = project / "torch-ext"
    mod_dir = ext_dir / name
    for d in (src_dir, inc_dir, mod_dir):
        d.mkdir(parents=True, exist_ok=True)

    src = []
    for p in kernel_sources():
        shutil.copyfile(p, src_dir / p.name)
        src.append(f"{name}_rocm/csrc/{p.name}")
    shutil.copyfile(HEADER, inc_dir / HEADER.name)
    src.insert(0, f"include/{HEADER.name}")
    for f in ("torch_binding.cpp", "torch_binding.h"):
        shutil.copyfile(TEMPLATE_DIR / f, ext_dir / f)
    shutil.copyfile(HOST_LAYER, mod_dir / "_host.py")
    files = {
        project / "build.toml": generate_build_toml(name, repo_id, src),
        project / "flake.nix": generate_flake_nix(name),
        project / "README.md": generate_readme(name, repo_id, op),
        mod_dir / "__init__.py": generate_init_py(name, repo_id, op),
    }
    for path, text in files.items():
        path.write_text(text, encoding="utf-8")
    if verbose:
        print(f"exported {op} as {project}")
        for p in sorted(project.rglob("*")):
            if p.is_file():
                print(f"  {p.relative_to(project)}")
        ops = sorted({o for t in (OP_TYPES if op == "all" else (op,)) for o in OP_BINDINGS[t]})
        print(f"torch ops used: {', '.join(ops)}")
        print("next: nix flake lock && nix run -L .#build-and-copy   (in the project directory)")
    return project


LOCAL_OPS_NAME = "ak355_hf"
LOCAL_OPS_LIB = TEMPLATE_DIR / "libak355_torch_ops.so"
# kernel-builder supplies registration.h at build time; this stand-in serves the local build only
# (ops registered with torch, no Python module init: the library is loaded with
# torch.ops.load_library)
_LOCAL_REGISTRATION_H = """\
#pragma once
#include <torch/library.h>
#define TORCH_LIBRARY_EXPAND(NAME, MODULE) TORCH_LIBRARY(NAME, MODULE)
#define REGISTER_EXTENSION(NAME)
"""


def build_local_ops(verbose: bool = True) -> Path:
    """Export every op to autokernel_amd/_build/hf and compile its torch binding with g++ against
    torch's headers and the in-tree libak355.so, as autokernel_amd/hf_export/libak355_torch_ops.so
    (torch op namespace ak355_hf). Checks the exported project builds and lets the GPU tests run
    its ops; kernel-builder is not needed."""
    import torch

    out_dir = _build.BUILD_DIR / "hf"
    if out_dir.exists():
        shutil.rmtree(out_dir)
    project = export_kernel(LOCAL_OPS_NAME, out_dir, op="all", verbose=False)
    reg = out_dir / "registration"
    reg.mkdir(parents=True, exist_ok=True)
    (reg / "registration.h").write_text(_LOCAL_REGISTRATION_H, encoding="utf-8")
    troot = Path(torch.__file__).resolve().parent
    tmp = LOCAL_OPS_LIB.with_suffix(".so.tmp")
    cmd = [
        shutil.which("g++") or "g++", "-std=c++17", "-O2", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch.compiled_with_cxx11_abi())}",
        f"-DTORCH_EXTENSION_NAME={LOCAL_OPS_NAME}",
        f"-I{troot / 'include'}", f"-I{troot / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
        "-I/opt/rocm/include", f"-I{reg}",
        str(project / "torch-ext" / "torch_binding.cpp"),
        f"-L{troot / 'lib'}", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip",
        f"-L{_build.PKG_DIR}", "-lak355", "-Wl,-rpath,$ORIGIN/..",
        "-o", str(tmp),
    ]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"torch binding build failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LOCAL_OPS_LIB)
    if verbose:
        print(f"built {LOCAL_OPS_LIB} (torch ops {LOCAL_OPS_NAME}::*)")
    return LOCAL_OPS_LIB


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description="Export libak355 as a HuggingFace Kernels ROCm project.")
    ap.add_argument("--name", required=True, help="project / module name (a Python identifier)")
    ap.add_argument("--kernel", default=str(DEFAULT_KERNEL_PATH),
                    help="kernel file whose KERNEL_TYPE picks the op (default: kernel.py)")
    ap.add_argument("--op", default=None, help=f"op type ({', '.join(OP_TYPES)}, or 'all'); overrides --kernel")
    ap.add_argument("--output", default=str(DEFAULT_OUTPUT_DIR), help="output directory")
    ap.add_argument("--repo-id", default=None, help="HuggingFace repo id for the hub section")
    a = ap.parse_args(argv)
    try:
        export_kernel(a.name, a.output, a.repo_id, a.op, a.kernel)
    except ValueError as e:
        print(f"ERROR: {e}", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Build the gfx950 decode kernels in-tree.

Produces, inside ``mega_kernel_qwen36/``:

* ``libmkq.so``  -- the HIP kernels and their C ABI (``include/mkq.h``), built
  with ``hipcc --offload-arch=gfx950``; no CUDA, no hipify;
* ``_C.<ext>``   -- the thin PyTorch-ROCm binding (pybind11) over that ABI,
  built with the host compiler against torch's headers and linked to
  ``libmkq.so`` through ``$ORIGIN``.

Usage: ``python mega-kernel-3.6_amd/build.py [--lib-only] [-j N]``.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys
import sysconfig

HERE = pathlib.Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
PKG = HERE / "mega_kernel_qwen36"
BUILD = HERE / "_build"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed FP32 VALU ops are disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{REPO / 'include'}",
]

LIB_NAME = "libmkq.so"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")
    if out.strip():
        sys.stderr.write(out + "\n")


def hip_sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


def build_lib(jobs: int) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in hip_sources():
        obj = BUILD / (src.stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    out = PKG / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          "-Wl,-soname," + LIB_NAME])
    os.replace(tmp, out)
    return out


def build_glue() -> pathlib.Path:
    import torch
    import torch.utils.cpp_extension as cpp_ext

    ext_suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = PKG / ("_C" + ext_suffix)
    tmp = out.with_name(out.name + ".tmp")
    cxx = os.environ.get("CXX", "g++")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [*cpp_ext.include_paths(), sysconfig.get_paths()["include"], os.path.join(ROCM, "include"), str(REPO / "include")]
    torch_lib = cpp_ext.library_paths()[0]
    cmd = [
        cxx, "-shared", "-fPIC", "-O2", "-std=c++17", "-fvisibility=hidden",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_C",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{p}" for p in incs],
        str(CSRC / "torch_glue.cpp"),
        "-o", str(tmp),
        f"-L{PKG}", "-lmkq", "-Wl,-rpath,$ORIGIN",
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        f"-Wl,-rpath,{torch_lib}",
        f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=min(8, os.cpu_count() or 1))
    args = ap.parse_args(argv)
    lib = build_lib(args.jobs)
    print(f"built {lib}")
    if not args.lib_only:
        glue = build_glue()
        print(f"built {glue}")


if __name__ == "__main__":
    main()

"""Build recipe for the native parts of oxitorch_amd.

`build_liboxihip()` compiles the gfx950 HIP kernels and the C-ABI into
`oxitorch_amd/liboxihip.so` (hipcc, one object per source, in parallel).
`build_native()` compiles the C++ host core (tensor storage, dispatch,
autograd graph, Python bindings) into `oxitorch_amd/_native*.so`.

Both run on a machine without a GPU: hipcc cross-compiles for gfx950.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
INCLUDE = ROOT / "include"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # every product and sum rounds on its own, as in the reference's
    # one-op-per-pass evaluation (no fused multiply-add contraction)
    "-ffp-contract=off",
    # no packed FP32 instructions: some of their forms have given wrong
    # results now and then on MI355X, with no error
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

HIP_SOURCES = ["runtime.hip", "elementwise.hip", "norm.hip", "norm_bwd_none.hip", "norm_bwd_gelu.hip", "norm_bwd_silu.hip", "norm_bwd_softmax.hip", "softmax.hip", "reduce.hip", "embedding.hip", "indexing.hip", "optim.hip", "transfer.hip"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def build_liboxihip(jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link liboxihip.so."""
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc(), *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    jobs = jobs or min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for fut in [ex.submit(_run, c) for c in cmds]:
            fut.result()
    out = PKG / "liboxihip.so"
    tmp = PKG / "liboxihip.so.tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


def native_ext_name() -> str:
    return "_native" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so")


def build_native() -> Path:
    """Compile the C++ host core + pybind11 bindings against liboxihip.so."""
    import pybind11

    BUILD.mkdir(exist_ok=True)
    srcs = sorted((CSRC / "host").glob("*.cpp"))
    if not srcs:
        raise RuntimeError("no host sources found")
    out = PKG / native_ext_name()
    tmp = out.with_suffix(".tmp")
    cmd = [
        "g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
        "-ffp-contract=off",
        f"-I{INCLUDE}", f"-I{CSRC / 'host'}", f"-I{pybind11.get_include()}",
        f"-I{sysconfig.get_paths()['include']}",
        *map(str, srcs),
        f"-L{PKG}", "-loxihip", "-Wl,-rpath,$ORIGIN",
        "-o", str(tmp),
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_liboxihip()
    if (CSRC / "host").is_dir():
        build_native()


if __name__ == "__main__":
    what = sys.argv[1:] or ["all"]
    if "all" in what:
        build_all()
    else:
        if "lib" in what:
            build_liboxihip()
        if "native" in what:
            build_native()
    print("built", ", ".join(what))

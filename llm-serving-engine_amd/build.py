"""Builds the gfx950 libraries in-tree (no JIT cache, no hipify, no torch build system).

    python llm-serving-engine_amd/build.py [--incremental] [-v]

Outputs, next to the Python package so that they travel with the source tree:
  llmserve/_lib/libllmserve_hip.so    HIP kernels + the C ABI of include/llmserve_hip.h
  llmserve/_lib/libllmserve_torch.so  torch.ops.llmserve_hip.* over that C ABI

Every HIP source is compiled with hipcc for gfx950 only, with correctly rounded fp32
division/sqrt (the quantizers are bit-exact with torch's CPU ops) and without packed-fp32
instructions.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shlex
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO / "include"
LIB_DIR = PKG_ROOT / "llmserve" / "_lib"
OBJ_DIR = REPO / "_build"

HIP_LIB = LIB_DIR / "libllmserve_hip.so"
TORCH_LIB = LIB_DIR / "libllmserve_torch.so"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3",
    "-std=c++20",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    f"-I{INCLUDE}",
]

HIP_SOURCES = [
    "errors.hip",
    "quant_pack.hip",
    "gemv.hip",
    "gemm_prefill.hip",
    "gemm_int4.hip",
    "fused_ops.hip",
    "sampling.hip",
    "paged_decode.hip",
    "attn_meta.hip",
    "decode_chain.hip",
    "lm_head.hip",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def _torch_paths() -> tuple[list[str], list[str]]:
    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths(device_type="cuda")
    lib = str(Path(torch.__file__).parent / "lib")
    return inc, [lib]


def _includes(path: Path, seen: set[Path]) -> set[Path]:
    """The in-tree headers `path` includes, transitively."""
    import re

    for name in re.findall(r'^#include "([^"]+)"', path.read_text(), re.M):
        for d in (CSRC, INCLUDE):
            h = d / name
            if h.is_file() and h not in seen:
                seen.add(h)
                _includes(h, seen)
    return seen


def _stale(src: Path, obj: Path) -> bool:
    """True when obj is missing or older than its source or a header it includes."""
    if not obj.is_file():
        return True
    deps = [src, *_includes(src, set()), Path(__file__)]
    return max(d.stat().st_mtime for d in deps) > obj.stat().st_mtime


def build(verbose: bool = False, jobs: int | None = None,
          incremental: bool = False) -> tuple[Path, Path]:
    """Compile the HIP sources and link both libraries. Rebuilds everything unless
    ``incremental`` (then only objects older than their sources or the headers)."""
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 1)
    objs = [OBJ_DIR / (Path(s).stem + ".o") for s in HIP_SOURCES]
    todo = [(s, o) for s, o in zip(HIP_SOURCES, objs)
            if not incremental or _stale(CSRC / s, o)]
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [
            ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", str(CSRC / s), "-o", str(o)], verbose)
            for s, o in todo
        ]
        for f in futs:
            f.result()
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, HIP_LIB)

    inc, libdirs = _torch_paths()
    tmp = TORCH_LIB.with_suffix(".so.tmp")
    cmd = [
        "g++",
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-D_GLIBCXX_USE_CXX11_ABI=1",
        f"-I{INCLUDE}",
        *[f"-I{p}" for p in inc],
        str(CSRC / "torch_ops.cpp"),
        "-o",
        str(tmp),
        f"-L{LIB_DIR}",
        "-lllmserve_hip",
        *[f"-L{p}" for p in libdirs],
        "-lc10",
        "-lc10_hip",
        "-ltorch_cpu",
        "-ltorch",
        "-Wl,-rpath,$ORIGIN",
        *[f"-Wl,-rpath,{p}" for p in libdirs],
    ]
    _run(cmd, verbose)
    os.replace(tmp, TORCH_LIB)
    return HIP_LIB, TORCH_LIB


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv):
        print(p)

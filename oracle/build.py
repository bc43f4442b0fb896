"""ORACLE (test infrastructure only) — build recipe for the CPU checker libraries.

    python oracle/build.py

1. ``oracle/lib/<isa>/liboracle_cpu.so`` from ``oracle/cpu_kernels.c``.
2. When ``/root/reference`` is present: the reference's own kernel sources
   ``src/llmserve/kernels/csrc/int8_gemv.cpp``, ``paged_attention.cpp`` and ``fused_ops.cpp``
   compiled where
   they lie, as PyTorch CPU extension modules, into ``oracle/_ref/<isa>/`` — the same
   sources and flags the reference's JIT loader uses (kernels/__init__.py:58-72), with
   g++ called directly instead of torch's build system. Nothing from the reference is
   copied into this repository; ``oracle/_ref`` is git-ignored.

Both are built for two ISA levels, because the GPU box's host CPU is not this one:
``x86-64-v4`` (AVX-512, which turns on the reference's AVX-512 branch) and ``x86-64-v3``.
``oracle.cpu`` picks the one the running CPU supports; the reference's ``-march=native``
becomes the explicit ISA level.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

HERE = Path(__file__).resolve().parent
REFERENCE = Path("/root/reference")
REF_CSRC = REFERENCE / "src" / "llmserve" / "kernels" / "csrc"
ISAS = ("x86-64-v4", "x86-64-v3")
REF_FLAGS = ["-O3", "-fopenmp", "-ffast-math"]  # + -march=<isa>


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{r.stderr[-4000:]}")


def cpu_lib_path(isa: str) -> Path:
    return HERE / "lib" / isa / "liboracle_cpu.so"


def ref_module_path(isa: str, name: str) -> Path:
    return HERE / "_ref" / isa / f"{name}.so"


def build_cpu() -> list[Path]:
    out = []
    for isa in ISAS:
        p = cpu_lib_path(isa)
        p.parent.mkdir(parents=True, exist_ok=True)
        _run(["gcc", *REF_FLAGS, f"-march={isa}", "-std=c11", "-fPIC", "-shared",
              str(HERE / "cpu_kernels.c"), "-o", str(p), "-lm"])
        out.append(p)
    return out


def _torch_ext_cmd(src: Path, name: str, isa: str, extra_ld: list[str]) -> list[str]:
    import torch
    from torch.utils import cpp_extension

    tdir = Path(torch.__file__).parent
    incs = [tdir / "include", tdir / "include" / "torch" / "csrc" / "api" / "include"]
    abi = [f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}"]
    pyb = []
    for k in ("PYBIND11_COMPILER_TYPE", "PYBIND11_STDLIB", "PYBIND11_BUILD_ABI"):
        v = getattr(torch._C, f"_{k}", None)
        if v is not None:
            pyb.append(f'-D{k}="{v}"')
    out = ref_module_path(isa, name)
    return [
        "g++", *REF_FLAGS, f"-march={isa}", "-std=c++17", "-fPIC", "-shared",
        "-DTORCH_API_INCLUDE_EXTENSION_H", f"-DTORCH_EXTENSION_NAME={name}", *abi, *pyb,
        *[f"-isystem{p}" for p in incs], f"-isystem{sysconfig.get_paths()['include']}",
        str(src), "-o", str(out),
        f"-L{tdir / 'lib'}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        f"-Wl,-rpath,{tdir / 'lib'}", "-fopenmp", *extra_ld,
    ]


def build_ref(jobs: int = 4) -> list[Path]:
    """Compile the reference's kernels, or return [] when the reference is not mounted."""
    if not REF_CSRC.is_dir():
        return []
    specs = [("int8_gemv.cpp", "llmserve_int8_gemv", []),
             ("paged_attention.cpp", "llmserve_paged_attention", ["-lmvec"]),
             ("fused_ops.cpp", "llmserve_fused_ops", [])]
    cmds, outs = [], []
    for isa in ISAS:
        (HERE / "_ref" / isa).mkdir(parents=True, exist_ok=True)
        for src, name, ld in specs:
            cmds.append(_torch_ext_cmd(REF_CSRC / src, name, isa, ld))
            outs.append(ref_module_path(isa, name))
    with cf.ThreadPoolExecutor(jobs) as ex:
        for f in [ex.submit(_run, c) for c in cmds]:
            f.result()
    return outs


if __name__ == "__main__":
    for p in build_cpu() + (build_ref() if "--no-ref" not in sys.argv else []):
        print(p)

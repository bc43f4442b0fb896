"""ORACLE — test infrastructure only.

A CPU restatement of the reference's quantized decode path (Buland-Choudhary/
llm-serving-engine, src/llmserve/): the quantizers in numpy (``oracle.quant``), the three CPU
kernels in C (``oracle/cpu_kernels.c`` via ``oracle.cpu``) and float64 references of the same
mathematics (``oracle.math_ref``). ``oracle/build.py`` additionally compiles the
reference's own C++ kernel sources into ``oracle/_ref/`` when ``/root/reference`` is present.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
anything from here, and only as the checker or the timed CPU baseline — never as the thing
measured on the GPU or shipped. The product (``llm-serving-engine_amd/llmserve``) never imports
this package.

Pinning (each function's docstring names its checks):
  * quantizers: bit-exact against torch-CPU golden vectors (tests/golden/), hand-built ties,
    zero/constant rows and the round-trip bound |deq - w| <= scale / 2;
  * C kernels: against the float64 mathematics at the reference tests' tolerances and, when
    oracle/_ref is built, against the reference's compiled kernels;
  * float64 references: brute force on tiny cases, SDPA and closed forms.
"""

"""Benchmark of the quantized decode path on one MI355X (BASELINE config 2 as the headline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

One step = one decode token (M = 1) through the weight-only int4 (group 128, AWQ-scaled)
linears of all 28 Qwen3-0.6B layers: fused qkv 1024->4096, o 2048->1024, gate_up 1024->6144,
down 3072->1024 — 112 GEMV launches with distinct weights, replayed from a HIP graph. Four
distinct copies of the model's quantized linears (4 x 250 MB) rotate between steps, so the
weights stream from HBM and not from the 256 MB Infinity Cache. Inputs are resident in HBM
before the timed region; weights are random N(0, 0.02), activations N(0, 1) with 1% of the
input channels x20; each layer shape's AWQ scale comes from the reference's grid search
(quant.py:154-170) on 512 such rows and that shape's first weight.

`value` = algorithmic bytes per step (packed weights + group scales/zeros + inv_act_scale +
x + y) x steps / wall time of the K timed steps. `roofline` is for the dominant kernel: of the
four GEMVs of a step (each launched 28 times) the one with the longest duration on the
profiler's clock, i.e. the median End - Start of its dispatches in the committed rocprofv3
kernel trace of `bench.py --only gemv` (profiles/gemv_kernel_trace.md); `frac` is its
algorithmic bytes over that median, and every other fraction that names a profile
(`extra.c1_int8_gemv`, `extra.c4_int8kv_paged_decode`: decode + merge) is computed the same
way from the file's rows. Measured live in this run and carried beside each of them:
`pipelined_*`, the per-dispatch interval of back-to-back launches over distinct inputs in a
HIP graph replay (HIP events on the kernels' stream), where one dispatch's ramp overlaps the
previous one's drain, and the same interval for a one-element fill kernel
(`empty_kernel_pipelined_us`, the floor of that measurement).
`cpu_baseline` times the reference's own CPU kernels (oracle/_ref, built from the reference
sources) — or the oracle's C restatement where that build is absent — on the host cores, on
the same quantized weights: config 2 on one thread per physical core of the GPU's NUMA node;
`extra.cpu` adds configs 1 and 4 and a 4-thread run of all three, with the CPU model and its
AVX-512 flag (about 25 s in all).
Extra fields report M = 4 / 16 steps (the kernel Int4Linear runs at that batch: the GEMV up
to 4 rows, the matrix-core kernel on the packed weight above, one launch per linear up to 16
rows), rows at the reference's own published benchmark shapes (`extra.reference_shapes`) and configs 1 (int8 GEMV), 3
(prefill int8 GEMM on the bf16 matrix cores, x conversion included), 4 (int8-KV decode) and
5 (the full greedy decode step of a random-init int4-AWQ Qwen3-0.6B at batch 64 over the int8
KV cache, one HIP graph replay per step: tokens/s, with the fp32 and the int4 LM head, and
per-op times; the same model at batch 1 and 4, with the persistent per-layer chain and
without).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "llm-serving-engine_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_TFLOPS = 2500.0  # MI355X dense bf16
LAYERS = 28
SHAPES = {"qkv": (4096, 1024), "o": (1024, 2048), "gate_up": (6144, 1024), "down": (1024, 3072)}
GROUP = 128
COPIES = 4
METRIC = "quantized GEMV GB/s & % HBM peak (Qwen3-0.6B shapes); quantized decode tok/s"


def int4_bytes(N: int, K: int, M: int) -> int:
    """Algorithmic bytes of one int4 GEMV: nibbles + fp32 scale/zero per group +
    inv_act_scale + x + y."""
    return N * K // 2 + 8 * N * (K // GROUP) + 4 * K + 4 * M * K + 4 * M * N


def int8_bytes(N: int, K: int, M: int) -> int:
    return N * K + 4 * N + 4 * M * K + 4 * M * N


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_weights(torch, dev, seed: int = 0):
    """COPIES x LAYERS x 4 int4 AWQ linears, quantized on the GPU. The AWQ scale of each
    layer shape comes from the reference's grid search on that shape's first weight and the
    calibration rows (reused by the other layers of the shape)."""
    from llmserve.kernels import load_quant
    from llmserve.quant import _search_awq_scale

    g = torch.Generator(device=dev).manual_seed(seed)
    calib, scales = {}, {}
    for name, (N, K) in SHAPES.items():
        x = torch.randn(512, K, device=dev, generator=g)
        outl = torch.randperm(K, device=dev, generator=g)[: K // 100]
        x[:, outl] *= 20.0
        calib[name] = x
        scales[name] = _search_awq_scale(torch.randn(N, K, device=dev, generator=g) * 0.02, x, GROUP)
    model = []
    for c in range(COPIES):
        layers = []
        for layer in range(LAYERS):
            lin = {}
            for name, (N, K) in SHAPES.items():
                w = torch.randn(N, K, device=dev, generator=g) * 0.02
                lin[name] = load_quant().int4_quantize(w, GROUP, scales[name])
                del w
            layers.append(lin)
        model.append(layers)
    log(f"[bench] quantized {COPIES} copies x {LAYERS} layers x {len(SHAPES)} linears")
    return model, calib


def make_inputs(torch, dev, calib, M: int):
    return {name: calib[name][:M].contiguous() for name in SHAPES}


GEMV_ROWS = 4  # Int4Linear.gemv_max_rows: the GEMV up to 4 rows, the matrix-core kernel above


def pack_all(torch, model, gemv):
    """The packed copy of every weight (Int4Linear keeps one for its matrix-core kernel)."""
    return [[{n: gemv.int4_gemm_pack(*lin[n][:3], GROUP) for n in SHAPES} for lin in layers]
            for layers in model]


def capture_steps(torch, model, xs, gemv, packed=None):
    """One HIP graph per weight copy, each holding the 112 launches of one step: the int4 GEMV
    (M <= GEMV_ROWS) or, given the packed weights, the matrix-core kernel with its split pass,
    as Int4Linear runs them."""
    def launch(lin, pk, name):
        nib, gs, gz, inv = lin[name]
        if pk is None:
            return gemv.int4_linear(xs[name], nib, gs, gz, GROUP, inv)
        return gemv.int4_linear_gemm_packed(xs[name], pk[name], SHAPES[name][0], GROUP, inv)

    graphs, outs = [], []
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the op (allocator) outside capture
        for name in SHAPES:
            launch(model[0][0], None if packed is None else packed[0][0], name)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for c, layers in enumerate(model):
        g = torch.cuda.CUDAGraph()
        ys = []
        with torch.cuda.graph(g):
            for li, lin in enumerate(layers):
                for name in SHAPES:
                    ys.append(launch(lin, None if packed is None else packed[c][li], name))
        graphs.append(g)
        outs.append(ys)
    torch.cuda.synchronize()
    return graphs, outs


def time_graphs(torch, graphs, steps: int, warmup: int) -> tuple[float, float]:
    """(wall seconds, GPU event seconds) for `steps` replays after `warmup`."""
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return t1 - t0, e0.elapsed_time(e1) / 1e3


def kernel_avg_us(torch, launch, n: int, reps: int = 20) -> float:
    """Average duration of one `launch(i)` call when the calls run back to back: n calls
    (distinct inputs) are captured in a HIP graph, the graph is replayed `reps` times between
    two HIP events recorded on the stream the kernels run on, and the interval is divided by
    n * reps. This is the per-dispatch interval a kernel-trace profiler reports for the same
    replays (profiles/bench_kernel_trace.md); no host launch overhead is inside it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm the ops (allocator, LDS attributes) outside capture
        for i in range(min(n, 3)):
            launch(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            launch(i)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) * 1e3 / (n * reps)


# rocprofv3 rows (kernel, workgroups) of the kernels the BENCH line's fractions name, in the
# committed kernel-trace summaries: the GEMVs Int4Linear runs at M = 1 for the four shapes and
# config 1's int8 GEMV (profiles/gemv_kernel_trace.md, `bench.py --only gemv`), config 4's
# decode and merge (profiles/attention_kernel_trace.md, `bench.py --only attention`).
PROFILE_ROWS = {
    "qkv": ("gemv_kernel_trace.md", "gemv_lat<1, 32, 1, 4, true, 1>", "512 x 1"),
    "o": ("gemv_kernel_trace.md", "gemv_lat<1, 64, 1, 4, true, 1>", "256 x 1"),
    "gate_up": ("gemv_kernel_trace.md", "gemv_lat<1, 32, 1, 4, true, 1>", "768 x 1"),
    "down": ("gemv_kernel_trace.md", "gemv_lat<1, 32, 1, 6, true, 3>", "256 x 1"),
    "c1": ("gemv_kernel_trace.md", "gemv_lat<1, 64, 1, 4, false, 1>", "1536 x 1"),
    "c4_decode": ("attention_kernel_trace.md", "paged_decode_kernel<signed char, 128, 2, true, true>",
                  "256 x 1"),
    "c4_merge": ("attention_kernel_trace.md", "paged_decode_merge_kernel<128>", "128 x 1"),
}


def read_profile(key: str) -> dict | None:
    """avg / median us of a kernel from a committed kernel-trace summary: the markdown row
    `| `kernel` | workgroups (x, y) x threads | dispatches | avg us | median us | min us |`."""
    fname, kernel, wgs = PROFILE_ROWS[key]
    p = REPO / "profiles" / fname
    if not p.is_file():
        return None
    for line in p.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == f"`{kernel}`" and cells[1].startswith(wgs + ","):
            try:
                return {"file": f"profiles/{fname}", "kernel": kernel, "workgroups": wgs,
                        "dispatches": int(cells[2]), "avg_us": float(cells[3]),
                        "median_us": float(cells[4])}
            except ValueError:
                return None
    return None


def read_traffic(kernel: str) -> dict | None:
    """HBM bytes per launch from the committed PMC summary (profiles/roofline_traffic.md):
    a markdown table row `| kernel | fetch_bytes | write_bytes | ... |`."""
    p = REPO / "profiles" / "roofline_traffic.md"
    if not p.is_file():
        return None
    for line in p.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0] == kernel:
            try:
                return {"fetch": float(cells[1]), "write": float(cells[2])}
            except ValueError:
                return None
    return None


def host_info(torch) -> dict:
    """The host cores this process may run on: CPU model, AVX-512, the allowed logical CPUs,
    their physical cores (one logical CPU per core) by NUMA node, and the GPU's NUMA node
    (from the PCI device of cuda:0 when the driver exposes it)."""
    info = {"model": None, "avx512f": False, "allowed_cpus": sorted(os.sched_getaffinity(0))}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name") and info["model"] is None:
                info["model"] = line.split(":", 1)[1].strip()
            if line.startswith("flags") and " avx512f" in line:
                info["avx512f"] = True
    except OSError:
        pass
    cores = {}  # (node, package, core) -> first allowed logical CPU
    for c in info["allowed_cpus"]:
        base = Path(f"/sys/devices/system/cpu/cpu{c}")
        try:
            pkg = int((base / "topology/physical_package_id").read_text())
            core = int((base / "topology/core_id").read_text())
        except (OSError, ValueError):
            pkg, core = 0, c
        nodes = sorted(base.glob("node[0-9]*"))
        node = int(nodes[0].name[4:]) if nodes else 0
        cores.setdefault((node, pkg, core), c)
    by_node = {}
    for (node, _, _), c in sorted(cores.items()):
        by_node.setdefault(node, []).append(c)
    info["physical_cores_by_node"] = {str(n): v for n, v in by_node.items()}
    gpu_node = None
    try:
        pr = torch.cuda.get_device_properties(0)
        dom, bus, dv = (getattr(pr, "pci_domain_id", 0), getattr(pr, "pci_bus_id", None),
                        getattr(pr, "pci_device_id", None))
        if bus is not None and dv is not None:
            f = Path(f"/sys/bus/pci/devices/{dom:04x}:{bus:02x}:{dv:02x}.0/numa_node")
            gpu_node = int(f.read_text())
    except Exception:  # pragma: no cover - depends on the box
        gpu_node = None
    info["gpu_numa_node"] = gpu_node
    return info


def cpu_baseline(torch, model, calib, dev, budget_s: float = 4.0) -> tuple[dict, dict]:
    """The reference's own CPU kernels (oracle/_ref, compiled from its sources; the oracle's C
    restatement where that build is absent) on the host cores, for configs 1 (int8_linear,
    6144 x 1024, M = 1), 2 (int4_linear over the 112 Qwen3-0.6B linears, M = 1, x * inv first
    as Int4Linear.forward does) and 4 (paged_attention_decode_int8 over config 4's cache, q
    pre-multiplied by the smoothing vector as attention.py does): each for about `budget_s`
    seconds, once with one thread per physical core of the GPU's NUMA node (of the cores this
    process may use; the node with most of them when the GPU's is unknown) and once with 4
    threads, the threads pinned to those cores. Returns (the config-2 line on the node's
    cores, all runs)."""
    import numpy as np

    from oracle import cpu as ocpu

    info = host_info(torch)
    by_node = info["physical_cores_by_node"]
    node = str(info["gpu_numa_node"]) if str(info["gpu_numa_node"]) in by_node else \
        max(by_node, key=lambda n: len(by_node[n]))
    node_cores = by_node[node]
    kind = "reference" if ocpu.ref_available() else "port"
    if kind == "reference":
        gm, pm = ocpu.ref_module("llmserve_int8_gemv"), ocpu.ref_module("llmserve_paged_attention")
    else:
        log("[bench] reference CPU kernels unavailable; timing the C restatement")

    # config 2: one copy of the 112 linears
    host = [{n: tuple(t.cpu() for t in lin[n]) for n in SHAPES} for lin in model[0]]
    xs = {n: calib[n][:1].cpu().contiguous() for n in SHAPES}

    def c2():
        for lin in host:
            for n in SHAPES:
                nib, gs, gz, inv = lin[n]
                if kind == "reference":
                    gm.int4_linear((xs[n] * inv).contiguous(), nib, gs, gz, GROUP)
                else:
                    ocpu.int4_linear(xs[n].numpy(), nib.numpy(), gs.numpy(), gz.numpy(), GROUP,
                                     inv.numpy())
    c2_bytes = LAYERS * sum(int4_bytes(N, K, 1) for N, K in SHAPES.values())

    # config 1: 6144 x 1024 int8 weights, 64 copies (400 MB: past the last-level cache)
    from llmserve.kernels import load_quant

    g = torch.Generator(device=dev).manual_seed(11)
    q1 = [tuple(t.cpu() for t in load_quant().int8_quantize(
        torch.randn(6144, 1024, device=dev, generator=g) * 0.02)) for _ in range(64)]
    x1 = torch.randn(1, 1024)
    it1 = [0]

    def c1():
        w, sc = q1[it1[0] % len(q1)]
        it1[0] += 1
        if kind == "reference":
            gm.int8_linear(x1, w, sc)
        else:
            ocpu.int8_linear(x1.numpy(), w.numpy(), sc.numpy())
    c1_bytes = int8_bytes(6144, 1024, 1)

    # config 4: one copy of its cache
    copies, q, cl, qm, bs, D, c4_bytes = c4_inputs(torch, dev, ncopies=1)
    kq, vq, ks, vs, bt = (t.cpu() for t in copies[0])
    qh, clh = (q * qm).cpu(), cl.cpu()
    del copies

    def c4():
        if kind == "reference":
            pm.paged_attention_decode_int8(qh, kq, vq, ks, vs, bt, clh, bs, D ** -0.5, 0)
        else:
            ocpu.paged_decode_int8(qh.numpy(), kq.numpy(), vq.numpy(), ks.numpy(), vs.numpy(),
                                   bt.numpy(), clh.numpy(), bs, D ** -0.5, 0)

    def timed(fn, nbytes):
        fn()  # warm-up
        n, t0, best = 0, time.perf_counter(), float("inf")
        while time.perf_counter() - t0 < budget_s:
            t = time.perf_counter()
            fn()
            best = min(best, time.perf_counter() - t)
            n += 1
        el = time.perf_counter() - t0
        return {"GBps": round(nbytes * n / el / 1e9, 3), "calls": n, "s": round(el, 2),
                "best_ms": round(best * 1e3, 3)}

    saved_aff, saved_threads = os.sched_getaffinity(0), torch.get_num_threads()
    runs = {}
    try:
        for label, cores in (("node_physical_cores", node_cores), ("4_threads", node_cores[:4])):
            os.sched_setaffinity(0, cores)
            torch.set_num_threads(len(cores))
            ocpu.set_threads(len(cores))
            runs[label] = {"threads": len(cores), "cpus": cores,
                           "c1_int8_gemv": timed(c1, c1_bytes),
                           "c2_int4_112_gemvs": timed(c2, c2_bytes),
                           "c4_int8kv_paged_decode": timed(c4, c4_bytes)}
            log(f"[bench] cpu {label}: {runs[label]}")
    finally:
        os.sched_setaffinity(0, saved_aff)
        torch.set_num_threads(saved_threads)
    main_run = runs["node_physical_cores"]
    line = {
        "value": main_run["c2_int4_112_gemvs"]["GBps"],
        "unit": "GB/s",
        "cores": main_run["threads"],
        "kind": kind,
        "sample": (f"{main_run['c2_int4_112_gemvs']['calls']} steps x 112 int4 g128 GEMVs (M=1, "
                   f"all 28 Qwen3-0.6B layers, one 250 MB weight copy) in "
                   f"{main_run['c2_int4_112_gemvs']['s']} s, one thread per physical core of "
                   f"NUMA node {node} ({info['model']}, AVX-512 "
                   f"{'yes' if info['avx512f'] else 'no'}); 4-thread and configs 1 / 4 runs in "
                   f"extra.cpu"),
    }
    return line, {"host": info, "numa_node": node, "kind": kind, "runs": runs}


def extra_configs(torch, dev) -> dict:
    """Kernel-level GB/s for BASELINE configs 1 (int8 GEMV) and 4 (int8-KV paged decode)."""
    import numpy as np

    from llmserve.kernels import load_int8_gemv, load_paged_attention, load_quant

    out = {}
    g = torch.Generator(device=dev).manual_seed(1)
    N, K = 6144, 1024
    qs = [load_quant().int8_quantize(torch.randn(N, K, device=dev, generator=g) * 0.02)
          for _ in range(160)]  # 1 GB of int8 weights
    x = torch.randn(1, K, device=dev, generator=g)
    gemv = load_int8_gemv()
    us = kernel_avg_us(torch, lambda i: gemv.int8_linear(x, *qs[i % len(qs)]), 200)
    b = int8_bytes(N, K, 1)
    out["c1_int8_gemv"] = with_profile(
        {"pipelined_us": round(us, 2), "pipelined_GBps": round(b / us / 1e3, 1),
         "pipelined_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": b}, b, ["c1"])
    del qs
    # config 3: prefill-sized int8 GEMMs (M = 2048) on the bf16 matrix cores
    c3 = {}
    for name, (N3, K3) in {"qkv": (6144, 2048), "gate_up": (16384, 2048), "down": (2048, 8192)}.items():
        x3 = torch.randn(2048, K3, device=dev, generator=g)
        ws3 = [load_quant().int8_quantize(torch.randn(N3, K3, device=dev, generator=g) * 0.02)
               for _ in range(2)]
        us3 = kernel_avg_us(torch, lambda i: gemv.int8_linear_prefill(x3, *ws3[i % 2]), 20)
        fl = 2.0 * 2048 * N3 * K3
        c3[name] = {"us": round(us3, 2), "TFLOPs": round(fl / us3 / 1e6, 1),
                    "mfma_frac": round(fl / us3 / 1e6 / MFMA_BF16_TFLOPS, 4), "flops": fl}
        del x3, ws3
    out["c3_int8_prefill_gemm_bf16"] = c3
    # config 4
    copies, q, cl, qm, bs, D, b = c4_inputs(torch, dev)
    pa = load_paged_attention()

    def launch(i):
        kq, vq, ks, vs, bt = copies[i % len(copies)]
        pa.paged_attention_decode_int8(q, kq, vq, ks, vs, bt, cl, bs, D ** -0.5, 0, qm)

    us = kernel_avg_us(torch, launch, 40)
    out["c4_int8kv_paged_decode"] = with_profile(
        {"pipelined_us": round(us, 2), "pipelined_GBps": round(b / us / 1e3, 1),
         "pipelined_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": b}, b,
        ["c4_decode", "c4_merge"])
    del copies
    out["reference_shapes"] = reference_shapes(torch, dev)
    return out


def with_profile(row: dict, nbytes: int, keys: list[str]) -> dict:
    """Adds the committed kernel-trace medians of `keys` (the kernels of one call, summed:
    decode + merge) and `frac` = bytes / that sum; without the profile rows `frac` is the
    in-process per-dispatch interval's."""
    profs = [read_profile(k) for k in keys]
    if all(p is not None for p in profs):
        us = sum(p["median_us"] for p in profs)
        row.update({"profile_us": round(us, 3), "profile": profs,
                    "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                    "GBps": round(nbytes / us / 1e3, 1)})
    else:
        row.update({"frac": row["pipelined_frac"], "GBps": row["pipelined_GBps"],
                    "profile": None})
    return row


def reference_shapes(torch, dev) -> dict:
    """The reference's own published CPU benchmark shapes (4-vCPU Xeon, its results files),
    run here on the same kernels, beside its figures: the int8-KV decode at Qwen3-0.6B
    attention geometry, block 16, batch 16 x ctx 1024 / 4096 and batch 1 x ctx 256 / 1024 /
    4096 (results/microbench/attention.json, docs/report.md:277-278: 2941 / 14555 and 40 / 264
    / 1082 us), and the int4 group-64 gate_up GEMV 1024 -> 6144 at M = 1 / 4 / 16
    (results/m8/kernels.md:8-10: 0.51 / 2.96 / 8.12 ms). GPU times are per-dispatch intervals
    of back-to-back launches over rotating copies (HIP events around graph replays)."""
    from llmserve.kernels import load_int8_gemv, load_paged_attention, load_quant

    out = {"attention_int8kv": {}, "int4_g64_gate_up": {}}
    pa = load_paged_attention()
    Hq, Hk, D, bs = 16, 8, 128, 16
    g = torch.Generator(device=dev).manual_seed(77)
    ref_attn = {(16, 1024): 2941.0, (16, 4096): 14555.0, (1, 256): 40.0, (1, 1024): 264.0,
                (1, 4096): 1082.0}
    for (B, ctx), ref_us in ref_attn.items():
        nblk = -(-ctx // bs)
        slots = B * nblk * bs
        copies = []
        for _ in range(max(2, min(16, (1 << 30) // (2 * slots * Hk * (D + 4))))):
            perm = torch.randperm(B * nblk, generator=g, device=dev)
            kq = torch.randint(-127, 128, (slots, Hk, D), dtype=torch.int8, device=dev, generator=g)
            vq = torch.randint(-127, 128, (slots, Hk, D), dtype=torch.int8, device=dev, generator=g)
            ks = torch.rand(slots, Hk, device=dev, generator=g) * 0.05
            vs = torch.rand(slots, Hk, device=dev, generator=g) * 0.05
            copies.append((kq, vq, ks, vs, perm.view(B, nblk).contiguous()))
        q = torch.randn(B, Hq, D, device=dev, generator=g)
        cl = torch.full((B,), ctx, dtype=torch.long, device=dev)

        def launch(i, copies=copies, q=q, cl=cl):
            kq, vq, ks, vs, bt = copies[i % len(copies)]
            pa.paged_attention_decode_int8(q, kq, vq, ks, vs, bt, cl, bs, D ** -0.5, 0, None)

        us = kernel_avg_us(torch, launch, 4 * len(copies))
        nbytes = B * ctx * Hk * (2 * D + 8)
        out["attention_int8kv"][f"B={B} ctx={ctx}"] = {
            "us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "reference_cpu_us": ref_us,
            "speedup": round(ref_us / us, 1)}
        del copies
    gemv = load_int8_gemv()
    N, K, G = 6144, 1024, 64
    lins = [load_quant().int4_quantize(torch.randn(N, K, device=dev, generator=g) * 0.02, G,
                                       torch.rand(K, device=dev, generator=g) + 0.5)
            for _ in range(64)]  # 64 x 3.5 MB
    for M, ref_ms in ((1, 0.51), (4, 2.96), (16, 8.12)):
        x = torch.randn(M, K, device=dev, generator=g)

        def launch(i, x=x):
            nib, gs, gz, inv = lins[i % len(lins)]
            gemv.int4_linear(x, nib, gs, gz, G, inv)

        us = kernel_avg_us(torch, launch, 128)
        nbytes = N * K // 2 + 8 * N * (K // G) + 4 * K + 4 * M * K + 4 * M * N
        out["int4_g64_gate_up"][f"M={M}"] = {
            "us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "reference_cpu_us": ref_ms * 1e3,
            "speedup": round(ref_ms * 1e3 / us, 1)}
    return out


def c5_decode(torch, dev, steps: int, warmup: int, profile: bool = False) -> dict:
    """Config 5: greedy decode of 64 sequences through a random-init int4-AWQ Qwen3-0.6B (28
    layers, g128, AWQ scales searched on synthetic activations) over an int8 KV cache with key
    smoothing; contexts ~ U[1024, 4096], block tables a random permutation of the physical
    blocks, cache contents random int8 with random scales (the state after a prefill). Each
    step is one graph replay of the whole step (embedding to greedy token, context lengths
    advanced on the device). tok/s = 64 x steps / wall time; also the same with the LM head
    quantized (quantize_lm_head), and per-op times at the step's shapes. profile: the fp32-head
    replays only (for a kernel trace of the step)."""
    import numpy as np

    from llmserve.kv_cache import KVCache
    from llmserve.model_runner import DecodeRunner
    from llmserve.quant import Int4Linear
    from llmserve.transformer import QWEN3_0_6B, QuantCausalLM

    cfg = QWEN3_0_6B
    B, bs = 64, 16
    nq, nk, D, H = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.hidden_size
    rng = np.random.default_rng(55)
    ctx = rng.integers(1024, 4097, B).astype(np.int64)
    grow = 2 * (warmup + steps) + 4  # two runs (fp32 and int4 LM head) plus capture steps
    nblk = -(-(ctx + grow) // bs)
    width, total = int(nblk.max()), int(nblk.sum())
    perm = rng.permutation(total)
    bt = np.zeros((B, width), np.int64)
    used = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[used:used + n]
        used += n
    t0 = time.perf_counter()
    model = QuantCausalLM(cfg, GROUP, seed=5, device=dev)
    lm4 = Int4Linear(nn_linear(torch, model.embed), GROUP, None, device=dev)
    log(f"[bench] c5 model built in {time.perf_counter() - t0:.1f} s")
    cache = KVCache(cfg, total, bs, device=dev, kv_dtype="int8")
    g = torch.Generator(device=dev).manual_seed(56)
    for k, v in cache.layers:
        for t in (k, v):
            t.data.random_(-127, 128, generator=g)
            t.scale.uniform_(0.005, 0.05, generator=g)
        s = torch.rand(nk, D, device=dev, generator=g) * 1.5 + 0.5
        k.set_smoothing(s / s.mean(-1, keepdim=True), nq)
    ids = torch.from_numpy(rng.integers(0, cfg.vocab_size, B)).to(dev)
    runner = DecodeRunner(model, cache, ids, torch.from_numpy(ctx), torch.from_numpy(bt))
    out = {"batch": B, "layers": cfg.num_hidden_layers, "context": "U[1024,4096]",
           "kv_cache_GB": round(cache.nbytes() / 1e9, 2)}
    for head in ("fp32", "int4"):
        model.lm_head = lm4 if head == "int4" else None
        runner.capture(keep_state=False)
        for _ in range(warmup):
            runner.replay()
        torch.cuda.synchronize()
        ctx0 = runner.context_lens.clone()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            runner.replay()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        gpu_ms = e0.elapsed_time(e1)
        ctx_mid = (ctx0.double() + (steps - 1) / 2).cpu().numpy()
        kv_read = int(cfg.num_hidden_layers * nk * (2 * D + 8) * ctx_mid.sum())
        wb = model.weight_bytes(B)
        lin, lm = wb["linears"], wb["lm_head"]
        step_bytes = lin + lm + kv_read
        ms = wall / steps * 1e3
        out[f"lm_head_{head}"] = {
            "tok_per_s": round(B * steps / wall, 1), "ms_per_step": round(ms, 4),
            "gpu_ms_per_step": round(gpu_ms / steps, 4), "steps": steps,
            "bytes_per_step": step_bytes, "kv_read_bytes": kv_read, "weight_bytes": lin + lm,
            "hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"[bench] c5 lm_head {head}: {out[f'lm_head_{head}']}")
        runner.graph = None
        if profile:
            return out
    model.lm_head = None
    out["per_op"] = c5_per_op(torch, dev, model, lm4, cache, runner)
    del runner, cache
    out["small_batch"] = {str(b): small_batch_decode(torch, dev, model, b, steps)
                          for b in (1, 4)}
    return out


def small_batch_decode(torch, dev, model, B: int, steps: int) -> dict:
    """The config-5 model's greedy decode step at batch B (1 or 4), contexts ~ U[1024, 4096],
    one graph replay per step; at 1 and 2 rows the step runs one persistent launch per layer
    for the linear chain (QuantCausalLM.chain_max_rows), compared here with the launch-per-op
    step (use_chain False). tok/s = B x steps / wall time."""
    import numpy as np

    from llmserve.kv_cache import KVCache
    from llmserve.model_runner import DecodeRunner

    cfg = model.cfg
    bs = 16
    rng = np.random.default_rng(60 + B)
    ctx = rng.integers(1024, 4097, B).astype(np.int64)
    nblk = -(-(ctx + 2 * steps + 16) // bs)
    width, total = int(nblk.max()), int(nblk.sum())
    perm = rng.permutation(total)
    bt = np.zeros((B, width), np.int64)
    used = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[used:used + n]
        used += n
    cache = KVCache(cfg, total, bs, device=dev, kv_dtype="int8")
    g = torch.Generator(device=dev).manual_seed(61)
    for k, v in cache.layers:
        for t in (k, v):
            t.data.random_(-127, 128, generator=g)
            t.scale.uniform_(0.005, 0.05, generator=g)
    ids = torch.from_numpy(rng.integers(0, cfg.vocab_size, B)).to(dev)
    runner = DecodeRunner(model, cache, ids, torch.from_numpy(ctx), torch.from_numpy(bt))
    res = {}
    for mode in ("chain", "per_op"):
        model.use_chain = mode == "chain"
        if mode == "chain" and not (model._chain_ok(B) and B <= model.chain_max_rows):
            continue
        runner.capture(keep_state=False)
        for _ in range(3):
            runner.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps // 2):
            runner.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        n = steps // 2
        res[mode] = {"tok_per_s": round(B * n / wall, 1), "us_per_step": round(wall / n * 1e6, 1)}
        runner.graph = None
    model.use_chain = True
    log(f"[bench] c5 model at batch {B}: {res}")
    return res


def nn_linear(torch, w):
    """A bias-free nn.Linear view of an existing [out, in] weight (for Int4Linear)."""
    lin = torch.nn.Linear(w.shape[1], w.shape[0], bias=False, device="meta")
    lin.weight = torch.nn.Parameter(w, requires_grad=False)
    return lin


def c5_per_op(torch, dev, model, lm4, cache, runner) -> dict:
    """Average time of each op of the config-5 step at its shapes (64 rows), launched
    back to back over the 28 layers' distinct weights and caches, with its algorithmic bytes
    (and flops for the linears) as fractions of the HBM and bf16-MFMA peaks."""
    from llmserve.kernels import load_fused_ops, load_paged_attention

    cfg = model.cfg
    fo, pa = load_fused_ops(), load_paged_attention()
    nq, nk, D, H, I = (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                       cfg.hidden_size, cfg.intermediate_size)
    B, L, eps = runner.ids.numel(), cfg.num_hidden_layers, cfg.rms_norm_eps
    g = torch.Generator(device=dev).manual_seed(57)
    x = {K: torch.randn(B, K, device=dev, generator=g) for K in (H, nq * D, I)}
    resid = torch.randn(B, H, device=dev, generator=g)
    qkv = torch.randn(B, (nq + 2 * nk) * D, device=dev, generator=g)
    gu = torch.randn(B, 2 * I, device=dev, generator=g)
    q = torch.randn(B, nq, D, device=dev, generator=g)
    logits = torch.randn(B, cfg.vocab_size, device=dev, generator=g)
    ctx, bt, bs = runner.context_lens, runner.block_tables, runner.block_size
    kv_read = int(nk * (2 * D + 8) * ctx.double().sum().item())
    lay = model.layers

    kc0, vc0 = cache.layers[0]
    frags = {H: fo.add_rmsnorm_xfrag_(resid.clone(), x[H], lay[0].input_layernorm, None, eps),
             I: fo.silu_mul_xfrag(gu, None),
             nq * D: pa.paged_attention_decode_int8_xfrag(
                 q, kc0.data, vc0.data, kc0.scale, vc0.scale, bt, ctx, bs, D ** -0.5, 0,
                 kc0._q_mult, None)[1]}

    def frag_gemm(name, lin_of, N, K, per_step=L, planes=False):
        """the step's GEMM on activation fragments (their producer timed on its own); planes:
        the K-split form the step uses before a residual norm (output planes)"""
        xf = frags[K]
        P = fo.int4_xfrag_splits(B, N, K) if planes else 1

        def launch(i):
            if P > 1:
                fo.int4_linear_gemm_xfrag_split(xf, lin_of(i).gemm_packed, B, N, K, GROUP, P)
            else:
                fo.int4_linear_gemm_xfrag(xf, lin_of(i).gemm_packed, B, N, K, GROUP)
        if P > 1:
            name = f"{name[:-1]}, K split in {P} planes)"
        return name, launch, int4_bytes(N, K, B) + 4 * B * N * (P - 1), 2.0 * B * N * K, per_step

    def lin(attr):
        return lambda i: getattr(lay[i % L], attr)

    def attn(i):
        kc, vc = cache.layers[i % L]
        pa.paged_attention_decode_int8_xfrag(q, kc.data, vc.data, kc.scale, vc.scale, bt, ctx, bs,
                                             D ** -0.5, 0, kc._q_mult,
                                             lay[i % L].o_proj.inv_act_scale)

    def qkv_kv(i):
        kc, vc = cache.layers[i % L]
        fo.decode_qkv_kv(qkv, model.rope_cos, model.rope_sin, ctx, bt, bs, lay[i % L].q_norm,
                         lay[i % L].k_norm, eps, kc.smooth, kc.data, vc.data, kc.scale, vc.scale,
                         nq, nk, D)

    ctx_save = ctx.clone()
    norm_bytes = 4 * B * H * 3 + 4 * B * H  # x read + written, r read, fragments (hi + lo)
    entries = [
        frag_gemm("qkv_proj (int4 GEMM on fragments, 1024->4096)", lin("qkv_proj"),
                  (nq + 2 * nk) * D, H),
        ("decode_qkv_kv (norm + RoPE + KV write)", qkv_kv, 4 * B * (nq + 2 * nk) * D + 4 * B * nq * D
         + 2 * B * nk * (D + 4), 0.0, L),
        ("paged_attention_decode_int8_xfrag (+ merge writing o_proj's fragments)", attn,
         kv_read + 8 * B * nq * D + 4 * B * nq * D, 0.0, L),
        frag_gemm("o_proj (int4 GEMM on fragments, 2048->1024)", lin("o_proj"), H, nq * D,
                  planes=True),
        ("add_rmsnorm_xfrag_ (residual + norm + next split)",
         lambda i: fo.add_rmsnorm_xfrag_(resid, x[H], lay[i % L].input_layernorm,
                                         lay[i % L].gate_up_proj.inv_act_scale, eps),
         norm_bytes, 0.0, 2 * L),
        frag_gemm("gate_up_proj (int4 GEMM on fragments, 1024->6144)", lin("gate_up_proj"),
                  2 * I, H),
        ("silu_mul_xfrag (silu * up + down's split)",
         lambda i: fo.silu_mul_xfrag(gu, lay[i % L].down_proj.inv_act_scale), 4 * B * 3 * I, 0.0, L),
        frag_gemm("down_proj (int4 GEMM on fragments, 3072->1024)", lin("down_proj"), H, I,
                  planes=True),
        ("lm_head fp32 (hipBLASLt, torch.mm)", lambda i: torch.mm(x[H], model.lm_weight.t()),
         model.embed.numel() * 4 + 4 * B * (H + cfg.vocab_size), 2.0 * B * cfg.vocab_size * H, 1),
        ("lm_head fp32 (split-bf16 matrix cores on fragments: the step's)",
         lambda i: fo.lm_head_f32_xfrag(frags[H], model.lm_weight, B),
         model.embed.numel() * 4 + 4 * B * (H + cfg.vocab_size), 2.0 * B * cfg.vocab_size * H, 1),
        frag_gemm("lm_head int4 (GEMM on fragments, 1024->151936)", lambda i: lm4,
                  cfg.vocab_size, H, 1),
        ("argmax_advance", lambda i: fo.argmax_advance(logits, ctx), 4 * B * cfg.vocab_size, 0.0, 1),
    ]
    res = {}
    for name, launch, nbytes, flops, per_step in entries:
        us = kernel_avg_us(torch, launch, 56 if per_step > 1 else 8)
        r = {"us": round(us, 2), "per_step": per_step, "GBps": round(nbytes / us / 1e3, 1),
             "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
        if flops:
            r["TFLOPs"] = round(flops / us / 1e6, 2)
            r["mfma_frac"] = round(flops / us / 1e6 / MFMA_BF16_TFLOPS, 4)
        res[name] = r
    ctx.copy_(ctx_save)
    return res


def c4_inputs(torch, dev, ncopies: int = 4):
    """Config 4: `ncopies` copies (~280 MB each) of an int8 KV cache for 32 sequences, ctx ~
    U[512, 8192], block tables a random permutation of the physical blocks."""
    import numpy as np

    rng = np.random.default_rng(2024)
    B, Hq, Hk, D, bs = 32, 16, 8, 128, 16
    ctx = rng.integers(512, 8193, B)
    nblk = -(-ctx // bs)
    total = int(nblk.sum())
    width = int(nblk.max())
    copies = []
    for _ in range(ncopies):
        perm = rng.permutation(total)
        bt = np.zeros((B, width), np.int64)
        used = 0
        for i, n in enumerate(nblk):
            bt[i, :n] = perm[used:used + n]
            used += n
        kq = torch.randint(-127, 128, (total * bs, Hk, D), dtype=torch.int8, device=dev)
        vq = torch.randint(-127, 128, (total * bs, Hk, D), dtype=torch.int8, device=dev)
        ks = torch.rand(total * bs, Hk, device=dev) * 0.05
        vs = torch.rand(total * bs, Hk, device=dev) * 0.05
        copies.append((kq, vq, ks, vs, torch.from_numpy(bt).to(dev)))
    q = torch.randn(B, Hq, D, device=dev)
    cl = torch.from_numpy(ctx.astype(np.int64)).to(dev)
    qm = torch.rand(Hq, D, device=dev) + 0.5
    nbytes = int(ctx.sum()) * Hk * (2 * D + 8) + 8 * B * Hq * D + 8 * int(nblk.sum()) + 4 * Hq * D
    return copies, q, cl, qm, bs, D, nbytes


def profile_only(torch, dev, what: str) -> int:
    """64 launches of one kernel, for rocprofv3 counter runs (no timing output)."""
    from llmserve.kernels import load_int8_gemv, load_paged_attention, load_quant

    if what in ("gemv", "gemv4"):  # the four int4 g128 GEMV shapes at M = 1 (4), then config
        # 1's int8 GEMV
        g = torch.Generator(device=dev).manual_seed(3)
        gemv = load_int8_gemv()
        rows = 4 if what == "gemv4" else 1
        for name, (N, K) in SHAPES.items():  # 64 distinct weights each (~0.6 GB in all)
            lins = [load_quant().int4_quantize(torch.randn(N, K, device=dev, generator=g) * 0.02,
                                               GROUP, torch.rand(K, device=dev, generator=g) + 0.5)
                    for _ in range(64)]
            x = torch.randn(rows, K, device=dev, generator=g)
            for i in range(64):
                nib, gs, gz, inv = lins[i]
                gemv.int4_linear(x, nib, gs, gz, GROUP, inv)
            del lins
        N, K = 6144, 1024
        qs = [load_quant().int8_quantize(torch.randn(N, K, device=dev, generator=g) * 0.02)
              for _ in range(64)]
        x = torch.randn(rows, K, device=dev, generator=g)
        for i in range(64):
            gemv.int8_linear(x, *qs[i])
    elif what == "prefill":  # config 3 gate_up: M = 2048, 2048 -> 16384
        g = torch.Generator(device=dev).manual_seed(4)
        x = torch.randn(2048, 2048, device=dev, generator=g)
        qs = [load_quant().int8_quantize(torch.randn(16384, 2048, device=dev, generator=g) * 0.02)
              for _ in range(2)]
        gemv = load_int8_gemv()
        for i in range(16):
            gemv.int8_linear_prefill(x, *qs[i % 2])
    elif what == "prefill3":  # config 3's three GEMMs (qkv, gate_up, down), M = 2048, 16 each
        g = torch.Generator(device=dev).manual_seed(4)
        gemv = load_int8_gemv()
        for N, K in ((6144, 2048), (16384, 2048), (2048, 8192)):
            x = torch.randn(2048, K, device=dev, generator=g)
            qs = [load_quant().int8_quantize(torch.randn(N, K, device=dev, generator=g) * 0.02)
                  for _ in range(2)]
            for i in range(16):
                gemv.int8_linear_prefill(x, *qs[i % 2])
            del x, qs
    elif what == "gemm4":  # config 5's batched int4 linear: qkv 1024->4096 at 64 rows, packed
        N, K = SHAPES["qkv"]
        g = torch.Generator(device=dev).manual_seed(5)
        gemv = load_int8_gemv()
        packed = []
        for _ in range(64):
            nib, gs, gz, inv = load_quant().int4_quantize(
                torch.randn(N, K, device=dev, generator=g) * 0.02, GROUP,
                torch.rand(K, device=dev, generator=g) + 0.5)
            packed.append((gemv.int4_gemm_pack(nib, gs, gz, GROUP), inv))
        x = torch.randn(64, K, device=dev, generator=g)
        for i in range(64):
            pk, inv = packed[i]
            gemv.int4_linear_gemm_packed(x, pk, N, GROUP, inv)
    elif what == "gemm16":  # config 2 at 16 rows: the four shapes, packed weights, one launch
        g = torch.Generator(device=dev).manual_seed(6)
        gemv = load_int8_gemv()
        for name, (N, K) in SHAPES.items():  # 32 distinct weights each
            lins = []
            for _ in range(32):
                nib, gs, gz, inv = load_quant().int4_quantize(
                    torch.randn(N, K, device=dev, generator=g) * 0.02, GROUP,
                    torch.rand(K, device=dev, generator=g) + 0.5)
                lins.append((gemv.int4_gemm_pack(nib, gs, gz, GROUP), inv))
            x = torch.randn(16, K, device=dev, generator=g)
            for i in range(64):
                pk, inv = lins[i % 32]
                gemv.int4_linear_gemm_packed(x, pk, N, GROUP, inv)
            del lins
    elif what == "c5step":  # config 5's decode step: 2 + 10 graph replays, fp32 LM head
        c5_decode(torch, dev, 10, 2, profile=True)
    elif what == "c5step1":  # the config-5 model at batch 1: the per-layer chain, then per-op
        from llmserve.transformer import QWEN3_0_6B, QuantCausalLM

        small_batch_decode(torch, dev, QuantCausalLM(QWEN3_0_6B, GROUP, seed=5, device=dev), 1, 20)
    elif what == "attention":
        copies, q, cl, qm, bs, D, _ = c4_inputs(torch, dev)
        pa = load_paged_attention()
        for i in range(64):
            kq, vq, ks, vs, bt = copies[i % len(copies)]
            pa.paged_attention_decode_int8(q, kq, vq, ks, vs, bt, cl, bs, D ** -0.5, 0, qm)
    elif what == "lmhead":  # config 5's fp32 LM head 1024 -> 151936 at 64 rows, 2 weight copies
        from llmserve.kernels import load_fused_ops

        fo = load_fused_ops()
        V, H, B = 151936, 1024, 64
        g = torch.Generator(device=dev).manual_seed(6)
        ws = [torch.randn(V, H, device=dev, generator=g) * 0.02 for _ in range(2)]
        r = torch.randn(B, H, device=dev, generator=g)
        xf = fo.add_rmsnorm_xfrag_(torch.randn(B, H, device=dev, generator=g), r,
                                   torch.ones(H, device=dev), None, 1e-6)
        for i in range(32):
            fo.lm_head_f32_xfrag(xf, ws[i % 2], B)
    else:  # copy of 256 MiB: the reference for scaling FETCH_SIZE / WRITE_SIZE
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).random_(0, 255)
        dst = torch.empty_like(src)
        for _ in range(64):
            dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] profile run done: {what}")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip configs 1, 3, 4 and 5")
    ap.add_argument("--only", choices=["gemv", "gemv4", "gemm4", "gemm16", "attention", "prefill",
                                       "prefill3", "lmhead", "copy",
                                       "c5step", "c5step1"],
                    help="profiling run: only launch that kernel (64 times) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run --gpus 1)",
              file=sys.stderr)
        return 2
    import torch

    from llmserve.kernels import load_int8_gemv

    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    if args.only:
        return profile_only(torch, dev, args.only)
    log("[bench] quantizing 4 copies of the Qwen3-0.6B linears (int4 g128 AWQ)")
    model, calib = build_weights(torch, dev)
    gemv = load_int8_gemv()

    by_rows = {}
    headline = None
    spread = None
    packed = None
    for M in (1, 4, 16):
        xs = make_inputs(torch, dev, calib, M)
        if M > GEMV_ROWS and packed is None:
            packed = pack_all(torch, model, gemv)
        graphs, _ = capture_steps(torch, model, xs, gemv, packed if M > GEMV_ROWS else None)
        steps = args.steps if M == 1 else max(20, args.steps // 4)
        wall, gpu = time_graphs(torch, graphs, steps, args.warmup)
        step_bytes = LAYERS * sum(int4_bytes(N, K, M) for N, K in SHAPES.values())
        gbs = step_bytes * steps / wall / 1e9
        by_rows[str(M)] = {"kernel": ("gemv" if M <= GEMV_ROWS else
                                      "matrix-core on packed weight, fragments built in the kernel (one launch)"),
                           "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                           "ms_per_step": round(wall / steps * 1e3, 4),
                           "gpu_ms_per_step": round(gpu / steps * 1e3, 4), "bytes": step_bytes}
        if M == 1:
            headline = (gbs, wall / steps * 1e3, steps, step_bytes)
            # spread: five more timed windows of at least 200 steps (outside the headline's)
            n = max(steps, 200)
            runs = sorted(step_bytes * n / time_graphs(torch, graphs, n, 0)[0] / 1e9
                          for _ in range(5))
            spread = {"windows": 5, "steps_per_window": n, "GBps_min": round(runs[0], 1),
                      "GBps_median": round(runs[2], 1), "GBps_max": round(runs[-1], 1)}
        del graphs
        log(f"[bench] M={M}: {by_rows[str(M)]}")
    del packed

    # dominant kernel: of the four GEMV shapes at M = 1 (each launched 28 times per step), the
    # one with the most time per step on the profiler's clock (the committed kernel trace of
    # `bench.py --only gemv`: each dispatch's own start-to-end interval); `frac` is its
    # algorithmic bytes over that median. Measured live here, beside it: the per-dispatch
    # interval of 224 back-to-back launches in a graph replay (HIP events on the kernels'
    # stream), where each dispatch's ramp overlaps the previous one's drain.
    xs = make_inputs(torch, dev, calib, 1)
    order = [(c, l) for l in range(LAYERS) for c in range(COPIES)]

    def shape_launch(name):
        def launch(i):
            c, l = order[i % len(order)]
            nib, gs, gz, inv = model[c][l][name]
            gemv.int4_linear(xs[name], nib, gs, gz, GROUP, inv)
        return launch

    per_shape = {}
    for name, (N, K) in SHAPES.items():
        kb = int4_bytes(N, K, 1)
        live = kernel_avg_us(torch, shape_launch(name), 224)
        prof = read_profile(name)
        per_shape[name] = {"N": N, "K": K, "bytes": kb, "pipelined_us": round(live, 3),
                           "pipelined_frac": round(kb / live / 1e3 / HBM_PEAK_GBS, 4)}
        if prof is not None:
            per_shape[name].update({"profile_median_us": prof["median_us"],
                                    "profile_frac": round(kb / prof["median_us"] / 1e3 / HBM_PEAK_GBS, 4)})
    have_prof = all("profile_median_us" in v for v in per_shape.values())
    clock = "profile_median_us" if have_prof else "pipelined_us"
    dom = max(per_shape, key=lambda n: per_shape[n][clock])
    N, K = SHAPES[dom]
    kb = per_shape[dom]["bytes"]
    dur = per_shape[dom][clock]
    # the per-dispatch floor of the pipelined measurement: a one-element fill kernel
    tiny = [torch.zeros(1, device=dev) for _ in range(8)]
    empty_us = kernel_avg_us(torch, lambda i: tiny[i % 8].fill_(float(i)), 224)
    achieved = kb / dur / 1e3
    traffic = read_traffic(f"gemv_lat int4 {dom} M=1")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": None if traffic is None else int(traffic["fetch"] + traffic["write"]),
                "kernel": f"gemv_lat int4 ({dom} {K}->{N}, M=1)",
                "duration_us": dur,
                "clock": ("rocprofv3 kernel trace median (profiles/gemv_kernel_trace.md, "
                          "`bench.py --only gemv`)" if have_prof else
                          "in-process per-dispatch interval (no committed profile found)"),
                "bytes_per_launch": kb,
                "pipelined_interval_us": per_shape[dom]["pipelined_us"],
                "pipelined_GBps": round(kb / per_shape[dom]["pipelined_us"] / 1e3, 1),
                "empty_kernel_pipelined_us": round(empty_us, 3),
                "per_shape": per_shape}
    log(f"[bench] roofline: {roofline}")

    extra = {} if args.no_extra else extra_configs(torch, dev)
    if not args.no_extra:
        extra["c5_decode_step"] = c5_decode(torch, dev, max(20, args.steps // 4), 5)
    if extra:
        log(f"[bench] extra: {extra}")
    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baselines (about 25 s)")
        cpu, extra["cpu"] = cpu_baseline(torch, model, calib, dev)
        log(f"[bench] cpu: {cpu}")

    gbs, ms, steps, step_bytes = headline
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": ("config 2: int4 g128 AWQ weight-only GEMV through all 28 Qwen3-0.6B "
                         "layers (qkv 1024->4096, o 2048->1024, gate_up 1024->6144, down "
                         "3072->1024), M=1, 4 rotating weight copies, HIP graph per step"),
            "model_shapes": "Qwen3-0.6B",
            "group_size": GROUP,
            "rows": 1,
            "bytes_per_step": step_bytes,
            "parallelism": "single GPU",
        },
        "spread": spread,
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "by_rows": by_rows,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

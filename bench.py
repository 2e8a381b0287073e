"""W4A16 benchmark on one MI355X.

Headline workload: the Llama-3-8B decode sweep,
M in {1, 4, 8, 16} x {qkv 4096x6144, o 4096x4096, gate_up 4096x28672,
down 14336x4096}, symmetric int4, group 128, fp16 scales, fp16 activations.
One "step" is one pass over the 16 (layer, M) GEMMs, each launched R times
on distinct weight copies.  Inputs are resident in HBM before timing starts.

Timing.  The whole step -- the 16 shapes' R launches each, weight copies
rotated -- is captured once into one HIP graph, the way a graph-captured
decode step runs its linears: launches run back-to-back on the GPU without
host launch gaps.  The timed region replays it K times.
  value    = algorithmic bytes of every timed launch / wall time of the
             timed region (GB/s, whole job, the GPU's gaps between
             back-to-back launches included).
  decode   = per shape, a graph of that shape's R launches, HIP events
             around each replay (graph launch cost included, spread over R).
  roofline = the decode kernel: algorithmic bytes / the kernel's own mean
             duration, from HIP events around single launches on the launch
             stream (the graph period above adds the gap between
             back-to-back launches), vs 8 TB/s HBM3E.
Algorithmic bytes per GEMM: N*K/2 (int4) + N*(K/G)*2 (fp16 scales) +
M*K*2 (x) + M*N*2 (y).

MALL.  MI355X's 256 MB Infinity Cache would hold any one decode layer, so
each layer has C distinct weight copies holding >= 512 MB (8 for gate_up,
60 for o).  In the graphs (R = 4) a copy is reused only after ~850 MB of other
weights have streamed through; the roofline's single launches walk each
layer's copies in turn, so every launch reads its weights from HBM.

Also reported:
  reference_api = the same sweep through the reference's API
                  (gemm_w4a16_marlin with fp32 scale_marlin from repack_w4a16);
  decode_bf16   = the same sweep with bf16 activations (the reference
                  engine's dtype): step-graph value and kernel durations;
  prefill       = M in {256, 1024, 4096} over the same layers (BASELINE
                  configs[2]), TFLOP/s = 2*M*N*K / mean launch time, vs
                  2516.6 TFLOP/s fp16 MFMA;
  prefill_bf16  = the same with bf16 activations (the reference engine's
                  dtype; 2516.6 TFLOP/s bf16 MFMA);
  stack         = the 32-layer Llama-3-8B linear stack (q, k, v, o, gate, up,
                  down per layer) replayed as one HIP graph
                  per step at M = 1 and M = 32: linear-layer time per decode
                  step and its HBM GB/s;
  act_order_70b = the Llama-3-70B layers with asymmetric int4 and act-order
                  at M = 1, 16 (GB/s) and 2048 (TFLOP/s);
  cpu_baseline  = the reference CPU path (dequantize to fp32, fp32 GEMM --
                  the reference test oracle restated in oracle/) on this
                  host's cores over bounded samples of every config;
  roofline.copy_ceiling / read_ceiling = a 512 MiB device copy and 1 GiB
                  read-only reductions: what HBM gives a simple stream;
  roofline.read_floor = per layer, a plain streaming read of the layer's
                  decode bytes (the kernel's own duration): frac_of_read_floor
                  is that time over the decode kernel's, per shape and mean;
  prefill_dense_fp16_yardstick = the dense fp16 library GEMM (hipBLASLt
                  through torch) at every prefill shape; prefill_vs_dense is
                  its time over the W4A16 call's, from events around each call
                  ("call") and from back-to-back calls in one graph ("graph");
  repack        = repack_w4a16 per layer, GB/s of words and scales moved over
                  the kernels' own interval (and the whole call's time);
  gptq_repack   = repack_w4a16_gptq of the Llama-3-8B and -70B layers, in natural
                  order and through an act-order permutation: the repack
                  kernel's own interval and GB/s of words read and written.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--no-prefill] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2516.6

LLAMA8B = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 28672), ("down", 14336, 4096)]
LLAMA70B = [("qkv", 8192, 10240), ("gate_up", 8192, 57344), ("down", 28672, 8192)]
ACT_ORDER_M = [1, 16, 2048]
DECODE_M = [1, 4, 8, 16]
PREFILL_M = [256, 1024, 4096]
STACK_LAYERS = 32
STACK_M = [1, 32]
G = 128
COPIES = 8          # at least this many weight copies per layer
MALL_SAFE_BYTES = 512 << 20  # ... and enough that one layer's copies hold this much (the MALL is 256 MB)
REPS = 4


def copies_for(k: int, n: int) -> int:
    """Weight copies of one layer: rotating over them, a launch's weights were last
    read >= 512 MB of that layer's own traffic earlier, so they come from HBM."""
    return max(COPIES, -(-MALL_SAFE_BYTES // decode_bytes(1, k, n)))


def decode_bytes(m: int, k: int, n: int, g: int = G) -> int:
    return n * k // 2 + n * (k // g) * 2 + m * k * 2 + m * n * 2


def make_weights(k: int, n: int, copies: int, dev):
    """`copies` independent random int4 weights: (MARLIN words, fp32 [K/G,N] scales, fp16 [K/G,N] scales)."""
    import torch

    import pulsar_amd

    out = []
    for _ in range(copies):
        packed = torch.randint(-(2 ** 31), 2 ** 31, (n, k // 8), dtype=torch.int32, device=dev)
        scale = (torch.randn(n, k // G, device=dev) * 0.02).abs_().add_(1e-3).half()
        wm, sm = pulsar_amd.ops.repack_w4a16(packed, scale, G)
        out.append((wm, sm, sm.half()))
        del packed
    return out


def _median_time(fn, reps: int) -> float:
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def graph_period_us(torch, fn, calls: int, replays: int = 3) -> float:
    """Device time per call of `calls` back-to-back calls fn(0), fn(1), ... captured in one
    HIP graph (no host work between them): the best of `replays` replays, in us."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(calls):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) * 1e3 / calls)
    del graph
    return best


def cpu_baseline() -> dict:
    """The reference CPU path timed on this host: the reference test oracle
    (pulsar/tests/test_w4a16_gemm.py:56-62), i.e. dequantize the whole weight
    to fp32, then an fp32 GEMM, per call.  Dequant: oracle/w4a16_oracle.c
    (OpenMP); GEMM: numpy's BLAS sgemm (oracle.gemm_f32_blas).  A call's time is
    its dequant's plus its GEMM's, each timed on its own: every dequant is
    timed before the first BLAS call, because BLAS worker threads keep spinning
    for a while after a GEMM and would take the cores from the OpenMP dequant
    (an artefact of two thread pools in one process, not part of the path).
    Bounded samples of every BASELINE config:
      value  - configs[1], the 16 decode-sweep GEMMs: bytes over the summed
               per-call times (dequant and GEMM each a median of 5), GB/s;
      config1_m1_k4096_n4096 - configs[0], its two phases apart (median of 5);
      prefill - configs[2]: GEMM at M = 256, 1024 and 4096 (median of 3 /
                once / once), plus the layer's dequant;
      act_order_70b - configs[3]: the asymmetric act-order dequant of each 70B
                layer (once), GEMM at M = 1, 16 (median of 3) and at M = 2048
                (once);
      stack  - configs[4]: one Llama-3-8B layer's seven linears at M = 1 and
               32 (median of 3 each phase) times 32 layers (the layers have
               the same shapes), per decode token."""
    import numpy as np

    from oracle import oracle as O
    from pulsar_amd.stack import LLAMA3_8B_LINEARS

    t_start = time.perf_counter()
    rng = np.random.default_rng(0)

    def ct_weight(k, n, seed):
        u = O.uint4(seed, 2, (n, k))
        return O.pack_ct((u.astype(np.int16) - 8).astype(np.int8)), O.abs_normal(seed, 3, (n, k // G))

    # ---- phase 1: every dequant, before any BLAS call -------------------------------------
    def dq_ct(packed, scale):
        w = np.empty((packed.shape[0], packed.shape[1] * 8), dtype=np.float32)
        O.dequant_ct(packed, scale, G, out=w)
        return w, _median_time(lambda: O.dequant_ct(packed, scale, G, out=w), 5)

    l8 = {}
    for i, (name, k, n) in enumerate(LLAMA8B):
        l8[name] = dq_ct(*ct_weight(k, n, 10 + i))
    w1, dq1 = dq_ct(*ct_weight(4096, 4096, 20))
    l70 = {}
    for i, (name, k, n) in enumerate(LLAMA70B):
        p = O.make_problem(1, n, k, G, seed=30 + i, symmetric=False, act_order=True)
        qw, qz, s_kn, g_idx = p.qweight(), p.qzeros(), p.scale_kn, p.g_idx
        del p
        t0 = time.perf_counter()
        w = O.dequant_gptq(qw, s_kn, qz, g_idx, G)
        l70[name] = (w, time.perf_counter() - t0)
        del qw, qz
    layer = []
    for j, (_, k, n) in enumerate(LLAMA3_8B_LINEARS):
        w, dq = dq_ct(*ct_weight(k, n, 40 + j))
        layer.append((k, n, w, dq))

    # ---- phase 2: the GEMMs ---------------------------------------------------------------
    def gemm_time(w, rows, reps):
        xm = rng.standard_normal((rows, w.shape[1])).astype(np.float32)
        O.gemm_f32_blas(xm, w)
        return _median_time(lambda: O.gemm_f32_blas(xm, w), reps)

    tot_bytes = tot_time = 0.0
    decode = {}
    for m in DECODE_M:
        for name, k, n in LLAMA8B:
            w, dq = l8[name]
            t = dq + gemm_time(w, m, 5)
            decode[f"{name}_m{m}"] = round(t * 1e3, 3)
            tot_bytes += decode_bytes(m, k, n)
            tot_time += t
    gm1 = gemm_time(w1, 1, 5)
    config1 = {"dequant_ms": round(dq1 * 1e3, 3), "gemm_ms": round(gm1 * 1e3, 3),
               "total_ms": round((dq1 + gm1) * 1e3, 3),
               "GB/s": round(decode_bytes(1, 4096, 4096) / (dq1 + gm1) / 1e9, 3)}
    prefill = {}
    for name, k, n in LLAMA8B:
        w, dq = l8[name]
        for m, rows, reps in ((256, 256, 3), (1024, 1024, 1), (4096, 4096, 1)):
            gm = gemm_time(w, rows, reps) * (m // rows)
            prefill[f"{name}_m{m}"] = {"dequant_ms": round(dq * 1e3, 2), "gemm_ms": round(gm * 1e3, 2),
                                       "total_ms": round((dq + gm) * 1e3, 2),
                                       "TFLOP/s": round(2.0 * m * n * k / (dq + gm) / 1e12, 4),
                                       **({"gemm_rows_timed": rows} if rows != m else {})}
    act = {}
    for name, k, n in LLAMA70B:
        w, dq = l70[name]
        res = {"dequant_ms": round(dq * 1e3, 1)}
        for m, rows, reps in ((1, 1, 3), (16, 16, 3), (2048, 2048, 1)):
            gm = gemm_time(w, rows, reps) * (m // rows)
            r = {"gemm_ms": round(gm * 1e3, 2), "total_ms": round((dq + gm) * 1e3, 1)}
            if m <= 16:
                r["GB/s"] = round(act_order_bytes(m, k, n) / (dq + gm) / 1e9, 3)
            else:
                r["TFLOP/s"] = round(2.0 * m * n * k / (dq + gm) / 1e12, 4)
            res[f"m{m}"] = r
        act[name] = res
    del l70
    stack = {}
    for m in STACK_M:
        t = sum(dq + gemm_time(w, m, 3) for _, _, w, dq in layer)
        nbytes = STACK_LAYERS * sum(decode_bytes(m, k, n) for k, n, _, _ in layer)
        stack[f"m{m}"] = {"layer_ms": round(t * 1e3, 2), "ms_per_token": round(t * STACK_LAYERS * 1e3, 1),
                          "bytes_per_token": nbytes, "GB/s": round(nbytes / (t * STACK_LAYERS) / 1e9, 3)}

    return {
        "value": round(tot_bytes / tot_time / 1e9, 3),
        "unit": "GB/s",
        "cores": O.num_threads(),
        "blas_threads": O.blas_threads(),
        "kind": "port",
        "sample": "value: the 16 decode-sweep GEMMs once each, a call = full dequantize to fp32 (oracle/"
                  "w4a16_oracle.c, OpenMP) + fp32 BLAS GEMM, each phase a median of 5; prefill, act_order_70b "
                  "and stack as in their notes",
        "decode_ms": decode,
        "config1_m1_k4096_n4096": config1,
        "prefill": prefill,
        "act_order_70b": act,
        "stack": stack,
        "notes": {"prefill": "per layer: dequant median of 5; GEMM M=256 median of 3, M=1024 and M=4096 once",
                  "act_order_70b": "asymmetric act-order dequant (zero points, g_idx) once per layer; GEMM M=1, 16 "
                                   "median of 3, M=2048 once",
                  "stack": "one layer's 7 linears (dequant median of 5, GEMM median of 3) x 32 layers"},
        "cpu_seconds": round(time.perf_counter() - t_start, 1),
    }


def device_info(torch, dev) -> dict:
    """Name, compute units and, where rocm-smi answers, the current clocks (taken right after
    the timed decode sweep, so under load or just after it)."""
    import subprocess

    props = torch.cuda.get_device_properties(dev)
    info = {"name": torch.cuda.get_device_name(dev), "arch": getattr(props, "gcnArchName", None),
            "compute_units": props.multi_processor_count, "clocks": None}
    try:
        r = subprocess.run(["rocm-smi", "--showclocks", "--json"], capture_output=True, text=True, timeout=10)
        if r.returncode == 0:
            card = next(iter(json.loads(r.stdout).values()))
            info["clocks"] = {k: v for k, v in card.items() if "clock" in k.lower() and ("sclk" in k or "mclk" in k)}
    except (OSError, ValueError, StopIteration, AttributeError, subprocess.SubprocessError):
        pass
    return info


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def build_graphs(torch, shapes, weights, xs, fn, stream):
    """One graph per (layer, M): REPS launches on rotating weight copies."""
    graphs = []
    for mi, (m, name, k, n) in enumerate(shapes):
        copies = weights[name]
        first = (DECODE_M.index(m) % 2) * REPS  # M values alternate between copy halves
        idx = [(first + r) % len(copies) for r in range(REPS)]
        with torch.cuda.stream(stream):
            for i in idx:  # eager warm-up on the capture stream (workspace, code objects)
                fn(xs[(m, k)], copies[i])
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            outs = [fn(xs[(m, k)], copies[i]) for i in idx]
        graphs.append((g, outs))
    return graphs


def build_step_graph(torch, shapes, weights, xs, fn, stream):
    """One graph for a whole step: every shape's REPS launches on the same rotating weight
    copies as the per-shape graphs, in sweep order (16 shapes x REPS launches), the way a
    graph-captured decode step runs its linears."""
    plan = []
    for m, name, k, n in shapes:
        copies = weights[name]
        first = (DECODE_M.index(m) % 2) * REPS
        plan += [(xs[(m, k)], copies[(first + r) % len(copies)]) for r in range(REPS)]
    with torch.cuda.stream(stream):
        for x, w in plan:  # eager warm-up on the capture stream (workspace, code objects)
            fn(x, w)
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        outs = [fn(x, w) for x, w in plan]
    return g, outs


def time_step_graph(torch, graph, steps, warmup, stream) -> float:
    """Wall time of exactly `steps` replays, synchronized on both sides."""
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for _ in range(steps):
            graph.replay()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def time_graphs(torch, graphs, shapes, steps, warmup, stream):
    for _ in range(warmup):
        for g, _ in graphs:
            g.replay()
    torch.cuda.synchronize()
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in graphs]
           for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for s in range(steps):
            for i, (g, _) in enumerate(graphs):
                evs[s][i][0].record(stream)
                g.replay()
                evs[s][i][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_shape = []
    for i in range(len(graphs)):
        ms = sum(evs[s][i][0].elapsed_time(evs[s][i][1]) for s in range(steps)) / steps / REPS
        per_shape.append(ms)
    return wall, per_shape


COPY_BYTES = 512 << 20


def summarize_traffic(fetch_csv: str, write_csv: str) -> int:
    """HBM bytes per decode launch from two rocprofv3 --pmc runs of --pmc-workload.

    FETCH_SIZE and WRITE_SIZE are KiB per dispatch.  Each is scaled by the
    factor that makes the 512 MiB copy read (write) exactly 512 MiB, then the
    decode launches are averaged and set against their algorithmic bytes."""
    import csv

    def per_dispatch(path, counter):
        rows = {}
        for r in csv.DictReader(open(path)):
            if r.get("Counter_Name") != counter:
                continue
            key = r["Dispatch_Id"]
            rows[key] = (r["Kernel_Name"], rows.get(key, ("", 0.0))[1] + float(r["Counter_Value"]))
        return list(rows.values())

    out = {}
    for label, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"), ("write", write_csv, "WRITE_SIZE")):
        rows = per_dispatch(path, counter)
        copy = [v for name, v in rows if "copy" in name.lower()]
        dec = [v for name, v in rows if "decode_kernel" in name]
        if not copy or not dec:
            print(f"{path}: no copy or no decode dispatches for {counter}", file=sys.stderr)
            return 1
        factor = (COPY_BYTES / 1024.0) / max(copy)
        out[label] = {"counter": counter, "copy_kib": max(copy), "calibration_factor": round(factor, 4),
                      "decode_dispatches": len(dec), "decode_mean_kib": sum(dec) / len(dec),
                      "decode_mean_bytes_calibrated": sum(dec) / len(dec) * 1024.0 * factor}
    shapes = [(m, name, k, n) for m in DECODE_M for name, k, n in LLAMA8B]
    alg = sum(decode_bytes(m, k, n) for m, _, k, n in shapes) / len(shapes)
    traffic = out["fetch"]["decode_mean_bytes_calibrated"] + out["write"]["decode_mean_bytes_calibrated"]
    # the workload issues the shapes in sweep order, REPS launches each
    per_shape = {}
    dec = {label: [v for name, v in per_dispatch(path, counter) if "decode_kernel" in name]
           for label, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"), ("write", write_csv, "WRITE_SIZE"))}
    if all(len(v) == len(shapes) * REPS for v in dec.values()):
        for i, (m, name, k, n) in enumerate(shapes):
            b = sum(sum(dec[label][i * REPS:(i + 1) * REPS]) / REPS * 1024.0 * out[label]["calibration_factor"]
                    for label in ("fetch", "write"))
            per_shape[f"{name}_m{m}"] = {"bytes": round(b), "algorithmic": decode_bytes(m, k, n),
                                         "ratio": round(b / decode_bytes(m, k, n), 4)}
    res = {"bytes_per_launch": round(traffic), "algorithmic_bytes_per_launch": round(alg),
           "traffic_over_algorithmic": round(traffic / alg, 4), "launches": "the 16 decode-sweep shapes x "
           f"{REPS} launches each, fp16 scales", **out, "per_shape": per_shape}
    path = os.path.join(ROOT, "profiles", "decode_traffic.json")
    with open(path, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res))
    return 0


def summarize_trace(trace_csv: str, steps: int) -> int:
    """Recompute `roofline` from a rocprofv3 --kernel-trace CSV of this bench.

    The roofline leg runs last among the fp16-activation decode launches (the
    bf16 sweep, when it runs, comes after it): per shape, in the sweep order,
    steps*REPS unarmed calls, then as many armed ones.  So the trace's last
    16 * 2 * steps * REPS decode_kernel dispatches with fp16 activations (the
    kernel's first template argument false) are that leg; their mean duration
    per shape, and the algorithmic bytes over the mean of those means, give the
    figure the bench computes from its own events."""
    import csv

    def fp16_decode(name: str) -> bool:
        return "decode_kernelILb0E" in name or "decode_kernel<false" in name  # mangled or demangled

    rows = [r for r in csv.DictReader(open(trace_csv)) if fp16_decode(r["Kernel_Name"])]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    reps = steps * REPS
    shapes = [(m, name, k, n) for m in DECODE_M for name, k, n in LLAMA8B]
    need = len(shapes) * 2 * reps
    if len(rows) < need:
        print(f"{trace_csv}: {len(rows)} fp16 decode dispatches, the roofline leg needs {need}", file=sys.stderr)
        return 1
    leg = rows[-need:]
    per_shape, unarmed_all, armed_all = {}, [], []
    for i, (m, name, k, n) in enumerate(shapes):
        d = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in leg[i * 2 * reps:(i + 1) * 2 * reps]]
        un, ar = d[:reps], d[reps:]
        per_shape[f"{name}_m{m}"] = {"unarmed_us": round(sum(un) / reps, 3), "armed_us": round(sum(ar) / reps, 3)}
        unarmed_all.append(sum(un) / reps)
        armed_all.append(sum(ar) / reps)
    alg = sum(decode_bytes(m, k, n) for m, _, k, n in shapes) / len(shapes)
    res = {"fp16_decode_dispatches_in_trace": len(rows), "roofline_leg_dispatches": need,
           "mean_unarmed_us": round(sum(unarmed_all) / len(shapes), 3),
           "mean_armed_us": round(sum(armed_all) / len(shapes), 3),
           "algorithmic_bytes_per_launch": round(alg)}
    for tag in ("unarmed", "armed"):
        us = res[f"mean_{tag}_us"]
        res[f"achieved_{tag}_GB/s"] = round(alg / (us * 1e-6) / 1e9, 1)
        res[f"frac_{tag}"] = round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    res["per_shape"] = per_shape
    print(json.dumps(res))
    return 0


def stack_bench(torch, dev, steps: int, warmup: int) -> dict:
    """Config 5: the 32-layer linear stack as one graph per step, M = 1 and 32."""
    from pulsar_amd.stack import W4A16LinearStack, fuse_layers, random_layers

    rep: dict = {}
    layers = random_layers(STACK_LAYERS, device=dev, seed=0, stats=rep)
    out = {"layers": STACK_LAYERS, "linears_per_layer": len(layers[0]),
           "repack_at_load": {"linears": STACK_LAYERS * len(layers[0]), "ms": round(rep["repack_ms"], 2),
                              "call_ms": round(rep["repack_call_ms"], 2),
                              "bytes": rep["repack_bytes"],
                              "GB/s": round(rep["repack_bytes"] / (rep["repack_ms"] * 1e-3) / 1e9, 1),
                              "note": "GPTQ qweight -> MARLIN words, qweight read + words written; ms: the "
                                      "repack kernels' own intervals (pw4_time_next_kernel), call_ms: HIP events "
                                      "around each W4A16Linear.from_gptq, host time included"},
           "weight_bytes": sum(l.weight_marlin.numel() * 4 + l.scales.numel() * 2 for ly in layers for l in ly),
           "note": "m1/m32: the 7 linears per layer as 7 launches; fused_m1/fused_m32: q|k|v and gate|up "
                   "N-concatenated (4 launches per layer, same weights and outputs); gated_m1/gated_m32: "
                   "q|k|v fused and gate|up as one SiLU-gated GEMM whose silu(gate)*up output feeds down, "
                   "the model's MLP (4 launches per layer, no separate activation kernel)"}
    fused = fuse_layers(layers)
    gated = fuse_layers(layers, silu_gate=True)
    runs = ([(f"m{m}", layers, m) for m in STACK_M] + [(f"fused_m{m}", fused, m) for m in STACK_M] +
            [(f"gated_m{m}", gated, m) for m in STACK_M])
    for tag, ls, m in runs:
        st = W4A16LinearStack(ls, m, device=dev)
        st.capture()
        for _ in range(warmup):
            st.step()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        with torch.cuda.stream(st.stream):
            for a, b in ev:
                a.record(st.stream)
                st.step()
                b.record(st.stream)
        torch.cuda.synchronize()
        ms = sorted(a.elapsed_time(b) for a, b in ev)
        med = ms[len(ms) // 2]
        gbs = st.bytes_per_step() / (med * 1e-3) / 1e9
        out[tag] = {"us_per_step": round(med * 1e3, 1), "min_us": round(ms[0] * 1e3, 1),
                        "launches": st.launches_per_step(), "bytes_per_step": st.bytes_per_step(),
                        "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}
        del st
    del layers, fused, gated
    torch.cuda.empty_cache()
    return out


def act_order_bytes(m: int, k: int, n: int, g: int = G) -> int:
    """Algorithmic HBM bytes of one asymmetric act-order call: int4 weights,
    fp16 scales, int4 zero points, the int32 K permutation, x and y."""
    return n * k // 2 + n * (k // g) * 2 + n * (k // g) // 2 + k * 4 + m * k * 2 + m * n * 2


def act_order_bench(torch, dev, steps: int, warmup: int) -> dict:
    """Config 4: asymmetric int4 with act-order on the Llama-3-70B layers.

    Weights are GPTQ checkpoints (qweight [K/8,N], qzeros [K/G,N/8], fp16 scales
    [K/G,N], g_idx[p[i]] = i/G for a random permutation p) repacked with
    repack_w4a16_gptq.  Each layer has enough copies that R copies hold
    >= 512 MB, rotated per launch.  M = 1, 16: HBM GB/s of the graph period of
    back-to-back launches; M = 2048: TFLOP/s of event-bracketed launches."""
    import pulsar_amd

    out = {"workload": "llama3-70b qkv 8192x10240, gate_up 8192x57344, down 28672x8192; asymmetric int4 "
                       "G=128, fp16 scales, int4 zero points, act-order g_idx", "layers": {}}
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    for name, k, n in LLAMA70B:
        copies = max(2, -(-(512 << 20) // act_order_bytes(1, k, n)))
        ws = []
        for _ in range(copies):
            qweight = torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), dtype=torch.int32, device=dev, generator=gen)
            p = torch.randperm(k, device=dev, generator=gen)
            g_idx = torch.empty(k, dtype=torch.int32, device=dev)
            g_idx[p] = torch.arange(k, device=dev, dtype=torch.int32) // G
            wm, perm = pulsar_amd.ops.repack_w4a16_gptq(qweight, g_idx, G)
            qz = torch.randint(-(2 ** 31), 2 ** 31, (k // G, n // 8), dtype=torch.int32, device=dev, generator=gen)
            sc = (torch.randn(k // G, n, device=dev, generator=gen) * 0.02).abs_().add_(1e-3).half()
            ws.append((wm, sc, qz, perm))
            del qweight, p, g_idx
        stream = torch.cuda.Stream(device=dev)
        res = {"copies": copies}
        for m in ACT_ORDER_M:
            x = torch.randn(m, k, device=dev, generator=gen).half()

            def call(i, act=True):
                w = ws[i % copies]
                return pulsar_amd.ops.gemm_w4a16_gptq(x, w[0], w[1], w[2], w[3] if act else None, G)

            if m <= 16:
                def period(act):
                    with torch.cuda.stream(stream):
                        for i in range(copies):
                            call(i, act)
                    stream.synchronize()
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=stream):
                        outs = [call(i, act) for i in range(copies)]
                    for _ in range(warmup):
                        graph.replay()
                    torch.cuda.synchronize()
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    with torch.cuda.stream(stream):
                        a.record(stream)
                        for _ in range(steps):
                            graph.replay()
                        b.record(stream)
                    torch.cuda.synchronize()
                    del graph, outs
                    return a.elapsed_time(b) * 1e3 / (steps * copies)

                us = period(True)
                # the same weights, scales and zero points without the permutation: the
                # natural-order asymmetric call, so the ratio is what act-order costs
                nat = period(False)
                gbs = act_order_bytes(m, k, n) / (us * 1e-6) / 1e9
                res[f"m{m}"] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 3),
                                "natural_order_us": round(nat, 2), "over_natural_order": round(us / nat, 3)}
            else:
                for i in range(2):
                    call(i)
                ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                      for _ in range(max(steps, 4))]
                for i, (a, b) in enumerate(ev):
                    a.record()
                    call(i)
                    b.record()
                torch.cuda.synchronize()
                us = sum(a.elapsed_time(b) for a, b in ev) / len(ev) * 1e3
                tf = 2.0 * m * n * k / (us * 1e-6) / 1e12
                res[f"m{m}"] = {"us": round(us, 1), "TFLOP/s": round(tf, 1),
                                "frac_mfma": round(tf / FP16_PEAK_TFLOPS, 3)}
            del x
        out["layers"][name] = res
        del ws
        torch.cuda.empty_cache()
    return out


READ_BYTES = 1 << 30


def measure_read_ceiling(torch, dev) -> dict:
    """HBM read-only rate over 1 GiB (four times the MALL): the streaming-read probe
    (pulsar_amd/libpw4_probe.so, 16-byte loads, grid-stride, plain or non-temporal) at a
    few grid sizes, median of 5 each, the best reported; torch reductions over the same
    buffer alongside."""
    import ctypes

    import pulsar_amd

    t = torch.ones(READ_BYTES // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(1024, dtype=torch.int32, device=dev)

    def rate(fn):
        fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
        for a, b in ev:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        ms = sorted(a.elapsed_time(b) for a, b in ev)[2]
        return round(READ_BYTES / (ms * 1e-3) / 1e9, 1)

    probe = ctypes.CDLL(os.path.join(os.path.dirname(pulsar_amd.__file__), "libpw4_probe.so"))
    probe.pw4_probe_stream_read.restype = ctypes.c_int
    probe.pw4_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    stream = torch.cuda.current_stream().cuda_stream

    def read(blocks, nt):
        rc = probe.pw4_probe_stream_read(t.data_ptr(), READ_BYTES, blocks, nt, 0xDEADBEEF, sink.data_ptr(), stream)
        if rc != 0:
            raise RuntimeError(f"pw4_probe_stream_read failed: hipError {rc}")

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    probe_rates = {f"probe_{w}x{cus}_wg{'_nt' if nt else ''}": rate(lambda w=w, nt=nt: read(w * cus, nt))
                   for w in (1, 2, 4, 8, 16) for nt in (0, 1)}
    torch_rates = {"torch_amax_int32": rate(lambda: t.amax()), "torch_sum_f32": rate(lambda: t.view(torch.float32).sum())}
    del t, sink
    best = max(probe_rates, key=probe_rates.get)
    return {"GB/s": probe_rates[best], "op": best, "all": {**probe_rates, **torch_rates}, "bytes_read": READ_BYTES,
            "what": "streaming read of 1 GiB (16-byte loads, plain or non-temporal, grid-stride, workgroups of "
                    "256), median of 5, bytes read; the best grid and load kind of the probe"}


def measure_read_floor(torch, dev) -> dict:
    """Per Llama-3-8B layer: how long a plain streaming read of that layer's decode bytes
    (weights, scales, x and y at M = 1) takes -- the probe kernel's own duration, from HIP
    events that hipExtLaunchKernel fills with the dispatch's start and end, as for the
    decode kernel.  Each launch reads the next slice of a 1 GiB buffer (a slice recurs only
    after 1 GiB of other reads, so it comes from HBM, not the 256 MB MALL); 40 launches at
    1, 2 and 4 workgroups of 256 per CU, plain and non-temporal loads, the best one's mean
    reported."""
    import ctypes

    import pulsar_amd

    probe = ctypes.CDLL(os.path.join(os.path.dirname(pulsar_amd.__file__), "libpw4_probe.so"))
    probe.pw4_probe_stream_read_timed.restype = ctypes.c_int
    probe.pw4_probe_stream_read_timed.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                                  ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p,
                                                  ctypes.c_void_p, ctypes.c_void_p]
    t = torch.ones(READ_BYTES // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(1024, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    reps = 40
    out = {}
    for name, k, n in LLAMA8B:
        nb = decode_bytes(1, k, n) // 256 * 256
        slots = READ_BYTES // nb
        best = None
        for wpc in (1, 2, 4):
            for nt in (0, 1):
                ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                      for _ in range(reps)]
                for a, b in ev:  # create the events before handing them over
                    a.record(stream)
                    b.record(stream)
                for r in range(reps):
                    rc = probe.pw4_probe_stream_read_timed(t.data_ptr() + (r % slots) * nb, nb, wpc * cus, nt,
                                                           0xDEADBEEF, sink.data_ptr(), stream.cuda_stream, ev[r][0],
                                                           ev[r][1])
                    if rc != 0:
                        raise RuntimeError(f"pw4_probe_stream_read_timed failed: hipError {rc}")
                stream.synchronize()
                us = sum(a.elapsed_time(b) for a, b in ev) / reps * 1e3
                if best is None or us < best[0]:
                    best = (us, wpc, nt)
        out[name] = {"bytes": nb, "us": round(best[0], 2), "GB/s": round(nb / (best[0] * 1e-6) / 1e9, 1),
                     "workgroups_per_cu": best[1], "nontemporal": bool(best[2])}
    del t, sink
    return out


def repack_bench(torch, dev) -> dict:
    """repack_w4a16 (the reference's one-time CT -> MARLIN repack) per Llama-3-8B layer, on
    two copies in turn, median of 5.  Bytes: the CT words read and the MARLIN words
    written, plus the scales read (fp16) and written (fp32).
      us / GB/s / frac_hbm - the kernels' own interval: pw4_time_next_kernel armed for the
                 call, whose events take the word repack's start and the scale
                 transpose's end (the two dispatches, back to back on the stream);
      call_us  - HIP events recorded around the call, which also hold the host's launch
                 time of both kernels (a fixed ~10 us that dominates the small layers)."""
    import pulsar_amd

    lib = pulsar_amd.capi()
    out = {}
    for name, k, n in LLAMA8B:
        srcs = []
        for _ in range(2):
            packed = torch.randint(-(2 ** 31), 2 ** 31, (n, k // 8), dtype=torch.int32, device=dev)
            scale = (torch.randn(n, k // G, device=dev) * 0.02).abs_().add_(1e-3).half()
            srcs.append((packed, scale))
        pulsar_amd.ops.repack_w4a16(*srcs[0], G)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
        kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
        for a, b in kev:  # create the events before handing them over
            a.record()
            b.record()
        for i, (a, b) in enumerate(ev):
            a.record()
            pulsar_amd.ops.repack_w4a16(*srcs[i % 2], G)
            b.record()
        for i, (a, b) in enumerate(kev):
            if lib.pw4_time_next_kernel(a, b) != 0:
                raise RuntimeError("pw4_time_next_kernel failed")
            pulsar_amd.ops.repack_w4a16(*srcs[i % 2], G)
        torch.cuda.synchronize()
        call_ms = sorted(a.elapsed_time(b) for a, b in ev)[2]
        ms = sorted(a.elapsed_time(b) for a, b in kev)[2]
        if ms <= 0.0:  # the runtime left the events unset: the call's figure stands in
            ms = call_ms
        nbytes = n * k // 2 * 2 + n * (k // G) * (2 + 4)
        out[name] = {"us": round(ms * 1e3, 2), "call_us": round(call_ms * 1e3, 2), "bytes": nbytes,
                     "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
        del srcs
    return out


def gptq_repack_bench(torch, dev) -> dict:
    """repack_w4a16_gptq (GPTQ qweight [K/8, N] -> MARLIN) per Llama-3-8B and -70B linear
    (q, k, gate, down; 70B qkv, gate_up, down), in natural order and with act-order g_idx
    (a random permutation of the rows, G = 128).  us: the repack kernel's own interval
    (pw4_time_next_kernel armed for the call; the permutation's own kernel, which runs first,
    is not in it), median over 7 passes of rotating copies that hold >= 512 MB.  Bytes: the
    qweight words read plus the MARLIN words written (2 * N * K / 2)."""
    import pulsar_amd

    lib = pulsar_amd.capi()
    layers = [("8b_q", 4096, 4096), ("8b_k", 4096, 1024), ("8b_gate", 4096, 14336), ("8b_down", 14336, 4096)]
    layers += [("70b_" + name, k, n) for name, k, n in LLAMA70B]
    out = {}
    for name, k, n in layers:
        nbytes = n * k // 2 * 2
        copies = max(2, min(16, -(-(512 << 20) // nbytes)))
        qws = [torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), dtype=torch.int32, device=dev) for _ in range(copies)]
        g_idx = torch.empty(k, dtype=torch.int32, device=dev)
        g_idx[torch.randperm(k, device=dev)] = torch.arange(k, device=dev, dtype=torch.int32) // G
        r = {"bytes": nbytes}
        for label, gi in (("natural", None), ("act_order", g_idx)):
            pulsar_amd.ops.repack_w4a16_gptq(qws[0], gi, G)
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(7 * copies)]
            for a, b in ev:  # create the events before handing them over
                a.record()
                b.record()
            for i, (a, b) in enumerate(ev):
                if lib.pw4_time_next_kernel(a, b) != 0:
                    raise RuntimeError("pw4_time_next_kernel failed")
                pulsar_amd.ops.repack_w4a16_gptq(qws[i % copies], gi, G)
            torch.cuda.synchronize()
            us = sorted(a.elapsed_time(b) for a, b in ev)[len(ev) // 2] * 1e3
            r[label] = {"us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 3)}
        out[name] = r
        del qws, g_idx
        torch.cuda.empty_cache()
    return out


def dense_yardstick(torch, dev, reps: int) -> dict:
    """What the dense fp16 library GEMM (torch.nn.functional.linear -> hipBLASLt) does at
    the prefill shapes (every M of the sweep) with the same kind of data (x ~ N(0,1),
    weights ~ N(0,1)*0.02 in fp16): a measured ceiling for the W4A16 prefill next to the
    nameplate peak.  Timed like the W4A16 prefill sweep (events around each call), with the
    weights rotated over enough copies that each call reads them from HBM, as the W4A16
    calls do."""
    out = {}
    for name, k, n in LLAMA8B:
        copies = max(1, min(8, -(-(512 << 20) // (n * k * 2))))
        ws = [(torch.randn(n, k, device=dev) * 0.02).half() for _ in range(copies)]
        for m in PREFILL_M:
            x = torch.randn(m, k, device=dev).half()
            for i in range(2):
                torch.nn.functional.linear(x, ws[i % copies])
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
            for i, (a, b) in enumerate(ev):
                w = ws[i % copies]
                a.record()
                torch.nn.functional.linear(x, w)
                b.record()
            torch.cuda.synchronize()
            ms = sum(a.elapsed_time(b) for a, b in ev) / len(ev)
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            gus = graph_period_us(torch, lambda i: torch.nn.functional.linear(x, ws[i % copies]), max(copies, 4))
            out[f"{name}_m{m}"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
                                   "frac_mfma": round(tf / FP16_PEAK_TFLOPS, 3), "graph_us": round(gus, 1),
                                   "graph_TFLOP/s": round(2.0 * m * n * k / gus / 1e6, 1)}
            del x
        del ws
        torch.cuda.empty_cache()
    return out


def time_each_launch(torch, shapes, weights, xs, fn, stream, reps: int) -> tuple[list[float], list[float]]:
    """Per shape, the mean duration (ms) of single decode-kernel launches, each on the
    next of the layer's weight copies (>= 512 MB of them, so every launch streams its
    weights from HBM, not from the 256 MB MALL), two ways:
    * the kernel's own: each call arms pw4_time_next_kernel with a pair of HIP events,
      which the library passes to hipExtLaunchKernel; they take the dispatch's start and
      end timestamps, the interval rocprofv3's kernel trace reports;
    * the call's: HIP events recorded on the launch stream around unarmed calls, which
      also hold the queue latency in front of the kernel (about 2 us).
    Under rocprofv3 the armed events read several microseconds longer than the trace's
    durations of the same dispatches; run without the profiler for these figures."""
    from pulsar_amd import capi

    lib = capi()
    own, call = [], []
    with torch.cuda.stream(stream):
        for mi, (m, name, k, n) in enumerate(shapes):
            first = (DECODE_M.index(m) % 2) * REPS
            kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
            cev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
            for a, b in kev:  # create the events before handing them over
                a.record(stream)
                b.record(stream)
            ncp = len(weights[name])
            for r in range(reps):  # unarmed calls: a hooked launch costs the runtime more
                cev[r][0].record(stream)
                fn(xs[(m, k)], weights[name][(first + r) % ncp])
                cev[r][1].record(stream)
            for r in range(reps):
                if lib.pw4_time_next_kernel(kev[r][0], kev[r][1]) != 0:
                    raise RuntimeError("pw4_time_next_kernel failed")
                fn(xs[(m, k)], weights[name][(first + r) % ncp])
            stream.synchronize()
            ko = [a.elapsed_time(b) for a, b in kev]
            call.append(sum(a.elapsed_time(b) for a, b in cev) / reps)
            # events the runtime left unset read <= 0: then the call's figure stands in
            own.append(sum(ko) / reps if min(ko) > 0.0 else None)
    return own, call


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-reference-api", action="store_true")
    ap.add_argument("--no-decode-bf16", action="store_true")
    ap.add_argument("--prefill-reps", type=int, default=10)
    ap.add_argument("--no-stack", action="store_true")
    ap.add_argument("--no-act-order", action="store_true", help="skip the 70B act-order layers (configs[3])")
    ap.add_argument("--pmc-workload", choices=["decode", "prefill", "prefill-bf16"],
                    help="no timing: decode = the decode sweep's launches once each, then a 512 MiB copy (the "
                         "HBM counter calibration), for rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE; prefill = "
                         "one launch per layer at --pmc-m rows, for MFMA and traffic counters (prefill-bf16: "
                         "bf16 activations), then the same 512 MiB copy")
    ap.add_argument("--pmc-m", type=int, default=PREFILL_M[-1], help="rows of the prefill --pmc-workload")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode sweep (headline value null)")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise the two --pmc-workload counter CSVs into profiles/decode_traffic.json")
    ap.add_argument("--trace", metavar="KERNEL_TRACE_CSV",
                    help="recompute the roofline from a rocprofv3 --kernel-trace CSV of this bench run with "
                         "the same --steps")
    args = ap.parse_args()
    if args.traffic:
        return summarize_traffic(*args.traffic)
    if args.trace:
        return summarize_trace(args.trace, args.steps)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the W4A16 path has no multi-GPU component in this build "
              "(--gpus must be 1)", file=sys.stderr)
        return 2

    import torch

    import pulsar_amd

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    weights = {name: make_weights(k, n, copies_for(k, n), dev) for name, k, n in LLAMA8B}
    copy_counts = {name: len(w) for name, w in weights.items()}
    xs = {(m, k): torch.randn(m, k, device=dev).half() for m in DECODE_M for _, k, _ in LLAMA8B}
    shapes = [(m, name, k, n) for m in DECODE_M for name, k, n in LLAMA8B]
    stream = torch.cuda.Stream(device=dev)

    def gemm_fp16_scales(x, w):
        return pulsar_amd.ops.gemm_w4a16_gptq(x, w[0], w[2], None, None, G)

    def gemm_reference_api(x, w):
        return pulsar_amd.ops.gemm_w4a16_marlin(x, w[0], w[1], G)

    if args.pmc_workload in ("prefill", "prefill-bf16"):
        xdt = torch.bfloat16 if args.pmc_workload == "prefill-bf16" else torch.float16
        for name, k, n in LLAMA8B:
            x = torch.randn(args.pmc_m, k, device=dev).to(xdt)
            gemm_fp16_scales(x, weights[name][0])
        src = torch.empty(COPY_BYTES // 2, dtype=torch.float16, device=dev)
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        return 0
    if args.pmc_workload == "decode":
        with torch.cuda.stream(stream):
            for m, name, k, n in shapes:
                for r in range(REPS):
                    gemm_fp16_scales(xs[(m, k)], weights[name][r % len(weights[name])])
            src = torch.empty(COPY_BYTES // 2, dtype=torch.float16, device=dev)
            dst = torch.empty_like(src)
            dst.copy_(src)
        torch.cuda.synchronize()
        return 0

    value = achieved = wall = mean_launch_us = mean_call_us = None
    hook_ok = False
    per_gemm = {}
    launches = args.steps * REPS
    tot_bytes = sum(decode_bytes(m, k, n) for m, _, k, n in shapes) * launches
    if not args.no_decode:
        # the headline: one graph per step holding the whole sweep
        step_graph = build_step_graph(torch, shapes, weights, xs, gemm_fp16_scales, stream)
        wall = time_step_graph(torch, step_graph[0], args.steps, args.warmup, stream)
        value = tot_bytes / wall / 1e9
        del step_graph
        # per shape: a graph of that shape's REPS launches, HIP events around each replay
        graphs = build_graphs(torch, shapes, weights, xs, gemm_fp16_scales, stream)
        _, per_ms = time_graphs(torch, graphs, shapes, args.steps, args.warmup, stream)
        for (m, name, k, n), ms in zip(shapes, per_ms):
            gbs = decode_bytes(m, k, n) / (ms * 1e-3) / 1e9
            per_gemm[f"{name}_m{m}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                        "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}
        del graphs
        # the roofline: algorithmic bytes over the kernel's own duration
        each_ms, call_ms = time_each_launch(torch, shapes, weights, xs, gemm_fp16_scales, stream,
                                            args.steps * REPS)
        hook_ok = all(ms is not None for ms in each_ms)
        each_ms = [c if ms is None else ms for ms, c in zip(each_ms, call_ms)]
        for (m, name, k, n), ms, cms in zip(shapes, each_ms, call_ms):
            per_gemm[f"{name}_m{m}"]["kernel_us"] = round(ms * 1e3, 2)
            per_gemm[f"{name}_m{m}"]["call_us"] = round(cms * 1e3, 2)
        achieved = sum(decode_bytes(m, k, n) for m, _, k, n in shapes) / (sum(each_ms) * 1e-3) / 1e9
        mean_launch_us = sum(each_ms) / len(each_ms) * 1e3
        mean_call_us = sum(call_ms) / len(call_ms) * 1e3

    device = device_info(torch, dev)

    ref_api = None
    if not args.no_reference_api:
        sg2 = build_step_graph(torch, shapes, weights, xs, gemm_reference_api, stream)
        wall2 = time_step_graph(torch, sg2[0], args.steps, args.warmup, stream)
        del sg2
        g2 = build_graphs(torch, shapes, weights, xs, gemm_reference_api, stream)
        _, per2 = time_graphs(torch, g2, shapes, args.steps, args.warmup, stream)
        ref_api = {"value": round(tot_bytes / wall2 / 1e9, 2), "unit": "GB/s",
                   "per_gemm_us": {f"{name}_m{m}": round(ms * 1e3, 2) for (m, name, _, _), ms in zip(shapes, per2)}}
        del g2

    # the same sweep with bf16 activations (the reference engine's dtype): step-graph
    # value and the kernel's own duration per shape
    dec_bf16 = None
    if not args.no_decode and not args.no_decode_bf16:
        xb = {key: t.to(torch.bfloat16) for key, t in xs.items()}
        sgb = build_step_graph(torch, shapes, weights, xb, gemm_fp16_scales, stream)
        wallb = time_step_graph(torch, sgb[0], args.steps, args.warmup, stream)
        del sgb
        own_b, call_b = time_each_launch(torch, shapes, weights, xb, gemm_fp16_scales, stream, args.steps * REPS)
        own_b = [c if o is None else o for o, c in zip(own_b, call_b)]
        ach_b = sum(decode_bytes(m, k, n) for m, _, k, n in shapes) / (sum(own_b) * 1e-3) / 1e9
        dec_bf16 = {"value": round(tot_bytes / wallb / 1e9, 2), "unit": "GB/s",
                    "achieved": round(ach_b, 1), "frac": round(ach_b / HBM_PEAK_GBS, 4),
                    "mean_launch_us": round(sum(own_b) / len(own_b) * 1e3, 3),
                    "kernel_us": {f"{name}_m{m}": round(ms * 1e3, 2) for (m, name, _, _), ms in zip(shapes, own_b)},
                    "what": "the decode sweep with bf16 x (same weights, fp16 scales): value over the step graph, "
                            "achieved over the kernel's own mean duration, as the fp16 headline"}
        del xb

    # achievable-HBM context: a 512 MiB device-to-device copy (read + write bytes), and
    # read-only streams of 1 GiB (torch reductions: the weights of a decode GEMM are read,
    # never written)
    copy_ceiling = read_ceiling = read_floor = None
    if not args.no_decode:
        read_ceiling = measure_read_ceiling(torch, dev)
        read_floor = measure_read_floor(torch, dev)
        src = torch.empty(COPY_BYTES // 2, dtype=torch.float16, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
        for a, b in ev:
            a.record()
            dst.copy_(src)
            b.record()
        torch.cuda.synchronize()
        ms = sorted(a.elapsed_time(b) for a, b in ev)[2]
        copy_ceiling = {"GB/s": round(2 * COPY_BYTES / (ms * 1e-3) / 1e9, 1), "bytes_moved": 2 * COPY_BYTES,
                        "what": "torch copy_ of 512 MiB fp16 on the device, median of 5, read + write bytes"}
        del src, dst
    floor_frac = None
    if read_floor is not None and per_gemm and all("kernel_us" in v for v in per_gemm.values()):
        ratios = {key: read_floor[key.rsplit("_m", 1)[0]]["us"] / v["kernel_us"] for key, v in per_gemm.items()}
        floor_frac = {"mean": round(sum(ratios.values()) / len(ratios), 3),
                      "per_shape": {key: round(r, 3) for key, r in ratios.items()}}

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath)).get("bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    def prefill_sweep(xdtype):
        out = {}
        for pm in PREFILL_M:
            for name, k, n in LLAMA8B:
                x = torch.randn(pm, k, device=dev).to(xdtype)
                w = weights[name][0]
                for _ in range(2):
                    gemm_fp16_scales(x, w)
                ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                      for _ in range(args.prefill_reps)]
                for i, (a, b) in enumerate(ev):
                    w = weights[name][i % len(weights[name])]
                    a.record()
                    gemm_fp16_scales(x, w)
                    b.record()
                torch.cuda.synchronize()
                ms = sum(a.elapsed_time(b) for a, b in ev) / len(ev)
                tf = 2.0 * pm * n * k / (ms * 1e-3) / 1e12
                ws_ = weights[name]
                gus = graph_period_us(torch, lambda i: gemm_fp16_scales(x, ws_[i % len(ws_)]), len(ws_))
                out[f"{name}_m{pm}"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
                                        "frac_mfma": round(tf / FP16_PEAK_TFLOPS, 3), "graph_us": round(gus, 1),
                                        "graph_TFLOP/s": round(2.0 * pm * n * k / gus / 1e6, 1)}
                del x
        return out

    prefill = prefill_bf16 = None
    if not args.no_prefill:
        prefill = prefill_sweep(torch.float16)
        # bf16 activations (the reference engine's dtype), same weights and fp16 scales
        prefill_bf16 = prefill_sweep(torch.bfloat16)
    repack = None if args.no_prefill else repack_bench(torch, dev)
    dense = None if args.no_prefill else dense_yardstick(torch, dev, args.prefill_reps)
    del weights, xs
    torch.cuda.empty_cache()

    stack = None
    if not args.no_stack:
        stack = stack_bench(torch, dev, args.steps, args.warmup)

    act_order = None if args.no_act_order else act_order_bench(torch, dev, args.steps, args.warmup)
    gptq_repack = None if args.no_act_order else gptq_repack_bench(torch, dev)

    cpu = None if args.no_cpu else cpu_baseline()
    if cpu is not None:
        cpu["model"] = cpu_model()

    line = {
        "metric": "W4A16 GEMM HBM GB/s (M<=16) & TFLOP/s (M=4096), % of MI355X roofline",
        "value": None if value is None else round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None if wall is None else round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "device": device,
        "config": {
            "workload": "llama3-8b W4A16 decode sweep: M in {1,4,8,16} x {qkv 4096x6144, o 4096x4096, "
                        "gate_up 4096x28672, down 14336x4096}, symmetric int4 G=128 fp16 scales, MARLIN "
                        "layout, fp16 x",
            "launches_per_gemm_per_step": REPS,
            "weight_copies": copy_counts,
            "mall_safe": "each layer rotates over copies holding >= 512 MB (the MALL is 256 MB): in the "
                         "graphs a copy is reused after ~850 MB of other weights, and the roofline's single "
                         "launches walk each layer's copies in turn",
            "timing": "value: wall time of --steps replays of one HIP graph holding the whole sweep (16 shapes "
                      "x 4 launches, each on its layer's next weight copy), synchronized on both sides; "
                      "decode.*.us: a graph of each shape's 4 launches, HIP events around each replay",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": None if achieved is None else round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": None if achieved is None else round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": None if traffic is None else (
                "not measured in this run: bytes_per_launch of profiles/decode_traffic.json, the committed "
                "summary of two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE, calibrated against a "
                "512 MiB copy) of `bench.py --pmc-workload decode` (profiles/decode_traffic.md)"),
            "mean_launch_us": None if mean_launch_us is None else round(mean_launch_us, 3),
            "timing": None if achieved is None else (
                "achieved = mean algorithmic bytes / mean decode-kernel duration over single launches of "
                "the 16 shapes; each duration from a HIP event pair that hipExtLaunchKernel fills with "
                "the dispatch's own start and end (pw4_time_next_kernel), the interval rocprofv3's "
                "kernel trace reports" if hook_ok else
                "achieved = mean algorithmic bytes / mean duration of HIP events around single calls "
                "(the kernel timing events did not fire on this box; queue latency included)"),
            "mean_call_us": None if mean_call_us is None else round(mean_call_us, 3),
            "copy_ceiling": copy_ceiling,
            "read_ceiling": read_ceiling,
            "frac_of_read_ceiling": None if achieved is None or read_ceiling is None else
            round(achieved / read_ceiling["GB/s"], 4),
            "read_floor": read_floor,
            # per shape: the layer's streaming-read time over the decode kernel's own time
            "frac_of_read_floor": floor_frac,
        },
        "decode": per_gemm,
        "reference_api": ref_api,
        "decode_bf16": dec_bf16,
        "prefill": prefill,
        "prefill_bf16": prefill_bf16,
        "prefill_dense_fp16_yardstick": dense,
        # dense time / W4A16 time per shape: above 1 the W4A16 GEMM is the faster; "call"
        # from the events around each call (host time between them included), "graph"
        # from back-to-back calls in one graph (device time only)
        "prefill_vs_dense": None if not (prefill and dense) else {
            key: {"call": round(dense[key]["us"] / v["us"], 3), "graph": round(dense[key]["graph_us"] / v["graph_us"], 3)}
            for key, v in prefill.items() if key in dense},
        "repack": repack,
        "stack": stack,
        "act_order_70b": act_order,
        "gptq_repack": gptq_repack,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""W4A16 benchmark on one MI355X.

Workload of the headline line: the Llama-3-8B decode
sweep, M in {1, 4, 8, 16} x {qkv 4096x6144, o 4096x4096, gate_up 4096x28672,
down 14336x4096}, symmetric int4, group 128, fp16 activations.  One "step" is
one pass over the 16 GEMMs (repacked MARLIN weights, inputs resident in HBM).

MALL: MI355X's 256 MB Infinity Cache would hold any single decode shape, so
every layer has R distinct weight copies used round-robin; between two uses of
the same copy the sweep streams R x 109 MB >= 512 MB of other weights.

value     = algorithmic bytes of all timed GEMMs / wall time of the timed region
            (GB/s, whole job).  Algorithmic bytes per GEMM:
            N*K/2 (int4) + N*(K/G)*2 (fp16 scales) + M*K*2 + M*N*2.
roofline  = the decode kernel: bytes per launch / mean launch duration from HIP
            events recorded around each launch on the op's stream, vs 8 TB/s.
prefill   = the M=4096 prefill sweep (BASELINE configs[2] at its largest M),
            TFLOP/s = 2*M*N*K / mean launch time, vs 2516.6 TFLOP/s.
cpu_baseline = the reference CPU path (dequantize to fp32, fp32 GEMM: the
            reference test oracle restated in oracle/) on this host's cores,
            over one pass of the same decode sweep.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-prefill] [--no-cpu]
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
DECODE_M = [1, 4, 8, 16]
PREFILL_M = 4096
G = 128


def decode_bytes(m: int, k: int, n: int, g: int = G) -> int:
    return n * k // 2 + n * (k // g) * 2 + m * k * 2 + m * n * 2


def make_weights(k: int, n: int, copies: int, dev):
    import torch

    import pulsar_amd

    out = []
    for _ in range(copies):
        packed = torch.randint(-(2 ** 31), 2 ** 31, (n, k // 8), dtype=torch.int32, device=dev)
        scale = (torch.randn(n, k // G, device=dev) * 0.02).abs_().add_(1e-3).half()
        wm, sm = pulsar_amd.ops.repack_w4a16(packed, scale, G)
        out.append((wm, sm))
        del packed
    return out


def cpu_baseline(time_budget_s: float = 20.0) -> dict:
    """The reference CPU path timed on this host over one pass of the decode sweep."""
    import numpy as np

    from oracle import oracle as O

    tot_bytes, tot_time, shapes = 0, 0.0, 0
    t_start = time.perf_counter()
    rng = np.random.default_rng(0)
    for m in DECODE_M:
        for _, k, n in LLAMA8B:
            if time.perf_counter() - t_start > time_budget_s:
                break
            packed = rng.integers(-(2 ** 31), 2 ** 31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
            scale = (np.abs(rng.standard_normal((n, k // G))) * 0.02 + 1e-3).astype(np.float32)
            x = rng.standard_normal((m, k)).astype(np.float32)
            wbuf = np.empty((n, k), dtype=np.float32)
            t0 = time.perf_counter()
            O.w4a16_ct_forward(x, packed, scale, G, wbuf)
            tot_time += time.perf_counter() - t0
            tot_bytes += decode_bytes(m, k, n)
            shapes += 1
    return {
        "value": round(tot_bytes / tot_time / 1e9, 3),
        "unit": "GB/s",
        "cores": O.num_threads(),
        "kind": "port",
        "sample": f"one pass over {shapes} of the 16 decode-sweep GEMMs (dequantize to fp32 + OpenMP fp32 GEMM, "
                  f"oracle/w4a16_oracle.c), {tot_time:.1f} s of CPU work",
    }


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=6)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill-reps", type=int, default=10)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the W4A16 path has no multi-GPU component in this build "
              "(--gpus must be 1)", file=sys.stderr)
        return 2

    import torch

    import pulsar_amd

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    weights = {name: make_weights(k, n, args.copies, dev) for name, k, n in LLAMA8B}
    xs = {(m, k): torch.randn(m, k, device=dev).half() for m in DECODE_M for _, k, _ in LLAMA8B}
    plan = [(m, name, k, n) for m in DECODE_M for name, k, n in LLAMA8B]
    counter = [0]

    def run_gemm(m, name, k, n):
        wm, sm = weights[name][counter[0] % args.copies]
        counter[0] += 1
        return pulsar_amd.ops.gemm_w4a16_marlin(xs[(m, k)], wm, sm, G)

    for _ in range(args.warmup):
        for item in plan:
            run_gemm(*item)
    torch.cuda.synchronize()

    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in plan]
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        for i, item in enumerate(plan):
            evs[s][i][0].record()
            run_gemm(*item)
            evs[s][i][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    per_gemm = {}
    tot_bytes = 0
    tot_launch_ms = 0.0
    for i, (m, name, k, n) in enumerate(plan):
        ms = sum(evs[s][i][0].elapsed_time(evs[s][i][1]) for s in range(args.steps)) / args.steps
        b = decode_bytes(m, k, n)
        tot_bytes += b * args.steps
        tot_launch_ms += ms * args.steps
        per_gemm[f"{name}_m{m}"] = {"us": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                                    "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
    value = tot_bytes / wall / 1e9
    achieved = tot_bytes / (tot_launch_ms * 1e-3) / 1e9

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_traffic.json")
    if os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath)).get("bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    prefill = None
    if not args.no_prefill:
        prefill = {}
        for name, k, n in LLAMA8B:
            x = torch.randn(PREFILL_M, k, device=dev).half()
            wm, sm = weights[name][0]
            for _ in range(2):
                pulsar_amd.ops.gemm_w4a16_marlin(x, wm, sm, G)
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(args.prefill_reps)]
            for a, b in ev:
                a.record()
                pulsar_amd.ops.gemm_w4a16_marlin(x, wm, sm, G)
                b.record()
            torch.cuda.synchronize()
            ms = sum(a.elapsed_time(b) for a, b in ev) / len(ev)
            tf = 2.0 * PREFILL_M * n * k / (ms * 1e-3) / 1e12
            prefill[f"{name}_m{PREFILL_M}"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
                                               "frac_mfma": round(tf / FP16_PEAK_TFLOPS, 3)}

    cpu = None if args.no_cpu else cpu_baseline()
    if cpu is not None:
        cpu["model"] = cpu_model()

    line = {
        "metric": "W4A16 GEMM HBM GB/s (M<=16) & TFLOP/s (M=4096), % of MI355X roofline",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "llama3-8b W4A16 decode sweep: M in {1,4,8,16} x {qkv 4096x6144, o 4096x4096, "
                        "gate_up 4096x28672, down 14336x4096}, symmetric int4 G=128 MARLIN layout, fp16 x",
            "weight_copies": args.copies,
            "mall_safe": f"round-robin over {args.copies} weight copies per layer",
            "gemms_per_step": len(plan),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "decode": per_gemm,
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

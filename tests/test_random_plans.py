"""Seeded random shapes across the library's plan space, each against the fp32
oracle at the reference's bars (the same metrics as every parity test here).

The fixed-shape tests pin each plan at chosen shapes; these cases instead draw
M, N, K, the group size, the activation dtype, the weight format and the entry
point at random (from a fixed seed, so the list is the same on every run), so
that plan boundaries meet odd shapes: ragged N (not a multiple of 64), K tails
(not a multiple of 128), M on both sides of the decode/prefill switch and of
the decode kernel's 16- and 32-row tiles, forced K splits, zero points and
act-order.  Entry points, with the reference operator each one replaces:
  * gptq  -- repack_w4a16_gptq + gemm_w4a16_gptq (GPTQ ingestion; no reference
             counterpart, pinned by the oracle's dequantization)
  * ct    -- gemm_w4a16 on compressed-tensors words
             (pulsar-core/src/kernels/w4a16_gemm.cu:317-352)
  * split -- gemm_w4a16_split with a forced K-slice count
             (pulsar-core/src/kernels/w4a16_gemm.cu:355-489)
  * marlin -- repack_w4a16 + gemm_w4a16_marlin with fp32 scales
             (pulsar-core/src/kernels/w4a16_marlin.cu:354-551)
"""

import numpy as np
import pytest
import torch

from pulsar_amd import ops
from w4a16_case import baseline_case, check

pytestmark = pytest.mark.gpu

MAX_MACS = 60_000_000


def _draw_cases(n_cases: int, seed: int) -> list[dict]:
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n_cases:
        op = ["gptq", "gptq", "ct", "split", "marlin"][int(rng.integers(0, 5))]
        g = int(rng.choice([16, 32, 64, 128, 256]))
        k = g * int(rng.integers(1, max(2, 6144 // g)))
        # M: a third on the decode tiles' edges, a third log-uniform over the
        # decode range, a third over the prefill range
        r = rng.random()
        if r < 1 / 3:
            m = int(rng.choice([1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65]))
        elif r < 2 / 3:
            m = int(np.exp(rng.uniform(0, np.log(64))))
        else:
            m = int(rng.integers(65, 321))
        # N: a multiple of 8 up to 2048, within the oracle's budget
        n_max = min(2048, MAX_MACS // (m * k)) // 8 * 8
        if n_max < 8:
            continue
        n = 8 * int(rng.integers(1, n_max // 8 + 1))
        dtype = torch.bfloat16 if rng.random() < 0.4 else torch.float16
        sym = op in ("ct", "split", "marlin") or rng.random() < 0.4
        act = op == "gptq" and rng.random() < 0.5
        splits = int(rng.integers(1, 9)) if op == "split" else 0
        sdtype = torch.float16 if rng.random() < 0.5 else torch.float32
        cases.append(dict(op=op, m=m, n=n, k=k, g=g, dtype=dtype, sym=sym, act=act, splits=splits, sdtype=sdtype,
                          seed=int(rng.integers(0, 1 << 30))))
    return cases


CASES = _draw_cases(64, seed=20261202)


def _case_id(c: dict) -> str:
    dt = "bf16" if c["dtype"] == torch.bfloat16 else "f16"
    extra = ("" if c["sym"] else "-zp") + ("-act" if c["act"] else "") + (f"-s{c['splits']}" if c["splits"] else "")
    return f"{c['op']}-m{c['m']}-n{c['n']}-k{c['k']}-g{c['g']}-{dt}{extra}"


@pytest.mark.parametrize("c", CASES, ids=[_case_id(c) for c in CASES])
def test_random_plan(c):
    what = _case_id(c)
    print(what, flush=True)
    m, n, k, g, dtype = c["m"], c["n"], c["k"], c["g"], c["dtype"]
    case = baseline_case(m, n, k, g, dtype=dtype, seed=c["seed"], symmetric=c["sym"], act_order=c["act"])
    if c["op"] == "gptq":
        g_idx = torch.from_numpy(case.g_idx).cuda() if c["act"] else None
        wm, perm = ops.repack_w4a16_gptq(case.qweight(), g_idx, g)
        scales = torch.from_numpy(np.ascontiguousarray(case.scale_nk.T)).to(c["sdtype"]).cuda()
        qz = None if c["sym"] else case.qzeros()
        y = ops.gemm_w4a16_gptq(case.x, wm, scales, qz, perm if c["act"] else None, g)
    elif c["op"] == "ct":
        y = ops.gemm_w4a16(case.x, case.ct_packed(), case.scale(torch.float32), g)
    elif c["op"] == "split":
        y = ops.gemm_w4a16_split(case.x, case.ct_packed(), case.scale(torch.float32), g, c["splits"])
    else:
        wm, sm = ops.repack_w4a16(case.ct_packed(), case.scale(torch.float32), g)
        y = ops.gemm_w4a16_marlin(case.x, wm, sm, g)
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == dtype
    check(y, case.y_ref, dtype, what)

"""The accumulators before the cast to the output dtype, against an exact reference: the
third parity figure for a floating-point output (max-abs of the pre-cast fp32 accumulators,
bar 1e-2), beside the output's rel-L2 and its max-abs excess over half an ulp, which every
other GEMM test checks.  At K = 14336 and 28672 the fp16 output's own rounding (half an ulp is
0.0156 at |y| >= 32) exceeds 1e-2, so only the accumulators can be held to it.

The kernels have no fp32 output, but a forced K split leaves the accumulators in the open:
each K slice writes its fp32 partial tile into the caller's workspace, after the
PW4_ZERO_REGION_BYTES zero region, and the last arriving slice (decode) or the combine pass
(prefill) sums them in slice order and rounds once.  Read back after the call:
  * the fp16 output equals the slice-order fp32 sum of the partials, rounded to nearest even,
    bit for bit (which also pins the layouts read here: decode [N/64 units][slices][M][64],
    prefill [slices][M][N]);
  * the partials summed in float64 are the accumulators over the whole K, held to max-abs
    1e-2 against x @ dequant(W)^T in float64 (exact: the fp16 x and the dequantised weights
    (u - z) * s are fp32 values, and so are their products).
Reference counterparts: the split paths behind gemm_w4a16_split / gemm_w4a16_marlin
(pulsar-core/src/kernels/w4a16_gemm.cu:355-489, w4a16_common.cuh:94-120); the bar is the
north star's max-abs 1e-2.
"""

import numpy as np
import pytest

import pulsar_amd
from oracle import oracle as O
from pw4_capi import DTYPE_BF16, DTYPE_F16, DTYPE_F32, PW4_ZERO_REGION_BYTES, Hip, declare

pytestmark = pytest.mark.gpu

G = 128
MAX_ABS = 1e-2

# (plan, M, N, K, slices, bf16 x, act-order): the decode kernel's counter path and the
# 256-wide prefill kernel's split (exact scaling with fp16 x), at the long-K layers of
# Llama-3-8B and -70B; act-order is config 4's asymmetric int4 with a g_idx permutation
CASES = [
    ("decode", 16, 4096, 14336, 4, False, False),
    ("decode", 1, 2048, 28672, 8, False, False),
    ("decode", 8, 1024, 14336, 2, True, False),
    ("decode", 16, 1024, 28672, 8, False, True),
    ("prefill", 256, 2048, 14336, 4, False, False),
    ("prefill", 128, 1024, 28672, 8, False, False),
    ("prefill", 128, 1024, 28672, 4, False, True),
]


@pytest.fixture(scope="module")
def env():
    lib = declare(pulsar_amd.capi())
    hip = Hip()
    yield lib, hip
    hip.free_all()


@pytest.mark.parametrize("plan,m,n,k,slices,bf16,act", CASES)
def test_pre_cast_accumulators(env, plan, m, n, k, slices, bf16, act):
    lib, hip = env
    what = f"{plan} M={m} N={n} K={k} slices={slices} {'bf16' if bf16 else 'fp16'}{' act-order' if act else ''}"
    print(what, flush=True)
    p = O.make_problem(m, n, k, G, seed=m + n + k, bf16=bf16, symmetric=not act, act_order=act)
    wm = hip.malloc(lib.pw4_marlin_words(n, k) * 4)
    if act:
        # GPTQ words repacked in the permuted K order, fp16 [K/G, N] scales, int4 zero points
        gi = hip.upload(p.g_idx.astype(np.int32))
        perm = hip.malloc(k * 4)
        status = hip.malloc(4)
        assert lib.pw4_gidx_to_perm(gi, k, G, perm, status, None) == 0
        assert hip.download(status, (1,), np.int32)[0] == 0
        assert lib.pw4_repack_gptq(hip.upload(p.qweight()), perm, n, k, wm, None) == 0
        sm, sdt, qz = hip.upload(O.f32_to_f16_bits(p.scale_kn)), DTYPE_F16, hip.upload(p.qzeros())
    else:
        packed = hip.upload(p.ct_packed())
        sc = hip.upload(p.scale_nk.astype(np.float32))
        sm, sdt, qz, perm = hip.malloc(n * (k // G) * 4), DTYPE_F32, None, None
        assert lib.pw4_repack_w4a16(packed, sc, DTYPE_F32, n, k, G, wm, sm, None) == 0
    x = hip.upload(p.x16)
    y = hip.malloc(m * n * 2)
    ws_bytes = lib.pw4_gemm_w4a16_marlin_workspace_size(m, n, k, G, int(act), slices)
    assert ws_bytes >= PW4_ZERO_REGION_BYTES + slices * m * n * 4
    ws = hip.malloc(ws_bytes)
    hip.memset(ws, 0, ws_bytes)
    dt = DTYPE_BF16 if bf16 else DTYPE_F16
    rc = lib.pw4_gemm_w4a16_marlin(x, dt, wm, sm, sdt, qz, perm, y, m, n, k, G, slices, ws, ws_bytes, None)
    assert rc == 0, (what, lib.pw4_status_string(rc), lib.pw4_last_hip_error())
    raw = hip.download(ws, (ws_bytes // 4,), np.float32)[PW4_ZERO_REGION_BYTES // 4:]
    if plan == "decode":
        part = raw[:slices * m * n].reshape(n // 64, slices, m, 64).transpose(1, 2, 0, 3).reshape(slices, m, n)
    else:
        part = raw[:slices * m * n].reshape(slices, m, n)
    # the output is the slice-order fp32 sum, rounded once
    acc32 = part[0].copy()
    for s in range(1, slices):
        acc32 += part[s]
    out = hip.download(y, (m, n), np.uint16)
    want = O.f32_to_bf16_bits(acc32) if bf16 else O.f32_to_f16_bits(acc32)
    assert np.array_equal(out, want), f"{what}: output is not the rounded sum of the partials"
    # the accumulators against the exact product
    acc = part.astype(np.float64).sum(axis=0)
    ref = p.xf.astype(np.float64) @ p.dequant().astype(np.float64).T
    err = np.abs(acc - ref).max()
    print(f"{what}: accumulator max-abs {err:.3e}, max |y| {np.abs(ref).max():.1f}", flush=True)
    assert err <= MAX_ABS, f"{what}: accumulator max-abs {err:.3e} > {MAX_ABS}"


# The default plans (no forced split), whose accumulators never reach memory:
# pw4_observe_next_call arms the call to write the fp32 value each y element is
# rounded from.  (name, M, N, K, bf16 x, act-order, workspace expected)
DEFAULT_PLAN_CASES = [
    ("decode direct store", 4, 2048, 14336, False, False, False),
    ("decode direct store, act-order", 8, 1024, 8192, False, True, False),
    ("decode exchange tree", 16, 1024, 14336, False, False, True),
    ("decode exchange tree, bf16", 32, 1024, 4096, True, False, True),
    ("decode exchange tree, act-order", 16, 1024, 28672, False, True, True),
    ("prefill unsplit, exact scaling", 4096, 4096, 14336, False, False, False),
    ("prefill K slices + combine", 256, 4096, 14336, False, False, True),
]


@pytest.mark.parametrize("name,m,n,k,bf16,act,ws_expected", DEFAULT_PLAN_CASES)
def test_pre_cast_accumulators_default_plans(env, name, m, n, k, bf16, act, ws_expected):
    lib, hip = env
    what = f"{name}: M={m} N={n} K={k} {'bf16' if bf16 else 'fp16'}"
    print(what, flush=True)
    p = O.make_problem(m, n, k, G, seed=m + 3 * n + k, bf16=bf16, symmetric=not act, act_order=act)
    wm = hip.malloc(lib.pw4_marlin_words(n, k) * 4)
    if act:
        gi = hip.upload(p.g_idx.astype(np.int32))
        perm = hip.malloc(k * 4)
        status = hip.malloc(4)
        assert lib.pw4_gidx_to_perm(gi, k, G, perm, status, None) == 0
        assert lib.pw4_repack_gptq(hip.upload(p.qweight()), perm, n, k, wm, None) == 0
        sm, sdt, qz = hip.upload(O.f32_to_f16_bits(p.scale_kn)), DTYPE_F16, hip.upload(p.qzeros())
    else:
        packed = hip.upload(p.ct_packed())
        sc = hip.upload(p.scale_nk.astype(np.float32))
        sm, sdt, qz, perm = hip.malloc(n * (k // G) * 4), DTYPE_F32, None, None
        assert lib.pw4_repack_w4a16(packed, sc, DTYPE_F32, n, k, G, wm, sm, None) == 0
    x = hip.upload(p.x16)
    y = hip.malloc(m * n * 2)
    y32 = hip.malloc(m * n * 4)
    hip.memset(y32, 0xFF, m * n * 4)  # NaN everywhere: an element the call does not write fails below
    ws_bytes = lib.pw4_gemm_w4a16_marlin_workspace_size(m, n, k, G, int(act), 0)
    # the plan is the one named: the exchange tree and K slices use the workspace's zero region
    # and partials; the direct store and the unsplit prefill use none (act-order's copy of x
    # takes a workspace either way)
    if not act:
        assert (ws_bytes > 0) == ws_expected, (what, ws_bytes)
    ws = hip.malloc(max(ws_bytes, 1))
    hip.memset(ws, 0, max(ws_bytes, 1))
    dt = DTYPE_BF16 if bf16 else DTYPE_F16
    assert lib.pw4_observe_next_call(y32) == 0
    rc = lib.pw4_gemm_w4a16_marlin(x, dt, wm, sm, sdt, qz, perm, y, m, n, k, G, 0, ws, ws_bytes, None)
    assert rc == 0, (what, lib.pw4_status_string(rc), lib.pw4_last_hip_error())
    acc32 = hip.download(y32, (m, n), np.float32)
    out = hip.download(y, (m, n), np.uint16)
    assert np.isfinite(acc32).all(), f"{what}: some y element has no observed accumulator"
    want = O.f32_to_bf16_bits(acc32) if bf16 else O.f32_to_f16_bits(acc32)
    assert np.array_equal(out, want), f"{what}: output is not the rounded accumulator"
    rows = np.arange(m) if m <= 64 else np.unique(np.concatenate([np.arange(0, m, max(m // 24, 1)), [m - 1]]))
    ref = p.xf[rows].astype(np.float64) @ p.dequant().astype(np.float64).T
    err = np.abs(acc32[rows].astype(np.float64) - ref).max()
    print(f"{what}: accumulator max-abs {err:.3e} over {len(rows)} rows, max |y| {np.abs(ref).max():.1f}", flush=True)
    assert err <= MAX_ABS, f"{what}: accumulator max-abs {err:.3e} > {MAX_ABS}"

"""pw4_gemm_w4a16_marlin_noalloc, through the C ABI: the GEMM with no workspace
argument, whose scratch is a fixed device array in the library.  Each call's
output must equal pw4_gemm_w4a16_marlin's (same kernels, same plan, a
caller-owned workspace) bit for bit, on calls in a row that need the scratch
(exchange-tree slots and counters in its zero region, fp32 partials and the
act-order copy of x after it), each smaller than the one before; a call whose
plan needs more than PW4_NOALLOC_SCRATCH_BYTES is rejected before it launches."""

import numpy as np
import pytest

import pulsar_amd
from oracle import oracle as O
from pw4_capi import DTYPE_F16, DTYPE_F32, PW4_NOALLOC_SCRATCH_BYTES, Hip, declare

pytestmark = pytest.mark.gpu

G = 128


@pytest.fixture(scope="module")
def env():
    lib = declare(pulsar_amd.capi())
    hip = Hip()
    yield lib, hip
    hip.free_all()


def _operands(lib, hip, p):
    n, k = p.n, p.k
    wm = hip.malloc(lib.pw4_marlin_words(n, k) * 4)
    if p.g_idx is None:
        packed = hip.upload(p.ct_packed())
        sc = hip.upload(p.scale_nk.astype(np.float32))
        sm = hip.malloc(n * (k // G) * 4)
        assert lib.pw4_repack_w4a16(packed, sc, DTYPE_F32, n, k, G, wm, sm, None) == 0
        return wm, sm, DTYPE_F32, None, None
    gi = hip.upload(p.g_idx.astype(np.int32))
    perm = hip.malloc(k * 4)
    status = hip.malloc(4)
    assert lib.pw4_gidx_to_perm(gi, k, G, perm, status, None) == 0
    qw = hip.upload(p.qweight())
    assert lib.pw4_repack_gptq(qw, perm, n, k, wm, None) == 0
    return wm, hip.upload(O.f32_to_f16_bits(p.scale_kn)), DTYPE_F16, hip.upload(p.qzeros()), perm


# (M, N, K, num_splits, act_order), each call smaller than the one before
CALLS = [
    (300, 1040, 2048, 4, False),   # prefill K slices: partials in the scratch, combine
    (24, 2112, 28672, 0, False),   # decode, K windows (more slices than the tree takes; no scratch)
    (16, 2048, 14336, 0, False),   # decode, exchange-tree K slices in the zero region
    (8, 1024, 8192, 0, True),      # act-order: x[:, perm] gathered into the scratch
    (4, 512, 4096, 3, False),      # decode, forced K slices: counters + partials
    (1, 256, 1024, 0, False),      # decode, direct store (no scratch needed)
]


def test_noalloc_matches_workspace_entry_point(env):
    lib, hip = env
    for i, (m, n, k, splits, act) in enumerate(CALLS):
        p = O.make_problem(m, n, k, G, seed=90 + i, symmetric=not act, act_order=act)
        wm, sc, sdt, qz, perm = _operands(lib, hip, p)
        x = hip.upload(p.x16)
        need = lib.pw4_gemm_w4a16_marlin_workspace_size(m, n, k, G, int(act), splits)
        ws = hip.malloc(max(need, 1))
        hip.memset(ws, 0, max(need, 1))
        y_ws = hip.malloc(m * n * 2)
        y_na = hip.malloc(m * n * 2)
        hip.memset(y_na, 0xff, m * n * 2)
        assert lib.pw4_gemm_w4a16_marlin(x, DTYPE_F16, wm, sc, sdt, qz, perm, y_ws, m, n, k, G, splits, ws, need,
                                         None) == 0
        rc = lib.pw4_gemm_w4a16_marlin_noalloc(x, DTYPE_F16, wm, sc, sdt, qz, perm, y_na, m, n, k, G, splits, None)
        assert rc == 0, (lib.pw4_status_string(rc), lib.pw4_last_hip_error())
        a = hip.download(y_ws, (m, n), np.uint16)
        b = hip.download(y_na, (m, n), np.uint16)
        assert np.array_equal(a, b), f"call {i} (M={m} N={n} K={k}): noalloc differs from the workspace entry point"
        # and both meet the oracle
        ref = p.reference()
        got = b.view(np.float16).astype(np.float64)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-3


def test_noalloc_rejects_plans_beyond_the_scratch(env):
    lib, hip = env
    # act-order gathers x[:, perm] (M * K * 2 bytes) into the scratch: 4096 x 8192 is 64 MiB
    m, n, k = 4096, 256, 8192
    assert m * k * 2 > PW4_NOALLOC_SCRATCH_BYTES - (16 << 20)
    x = hip.malloc(m * k * 2)
    wm = hip.malloc(lib.pw4_marlin_words(n, k) * 4)
    sc = hip.malloc((k // G) * n * 2)
    perm = hip.upload(np.arange(k, dtype=np.int32))
    y = hip.malloc(m * n * 2)
    assert lib.pw4_gemm_w4a16_marlin_noalloc(x, DTYPE_F16, wm, sc, DTYPE_F16, None, perm, y, m, n, k, G, 0,
                                             None) == -3
    # forced K slices whose partials do not fit are rejected too (automatic plans run unsplit)
    assert lib.pw4_gemm_w4a16_marlin_noalloc(x, DTYPE_F16, wm, sc, DTYPE_F16, None, None, y, m, n, k, G, 16,
                                             None) == -3

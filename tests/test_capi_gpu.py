"""The drop-in boundary on the GPU, through the C ABI alone: ctypes calls into
libpulsar_w4a16.so on device memory from hipMalloc, no torch in the data path
(the way a non-ATen C++ caller of pulsar-core/inc/pulsar/ops.hpp:156-189 would
bind it).

One workspace, allocated once and cleared once, is shared by GEMM calls that
take different plans: the direct decode store, decode K slices reduced through
the exchange tree, decode K slices through fp32 partials and arrival counters,
prefill K slices with a combine, an act-order gather, and the CT layout
repacked per call.  Each result is checked against the fp32 oracle, and the
zero region at the start of the workspace must be zero after every call (the
contract in include/pulsar_w4a16.h).
"""

import numpy as np
import pytest
import torch

import pulsar_amd
from oracle import oracle as O
from pw4_capi import DTYPE_F16, DTYPE_F32, PW4_ZERO_REGION_BYTES, Hip, declare
from w4a16_case import check

pytestmark = pytest.mark.gpu

G = 128

# (name, M, N, K, num_splits, act_order): the plan each one takes is in the name
CASES = [
    ("decode_direct", 1, 4096, 4096, 0, False),
    ("decode_tree", 8, 1024, 14336, 0, False),
    ("decode_counter", 4, 512, 4096, 3, False),
    ("prefill_split", 300, 520, 2048, 4, False),
    ("prefill_exact", 260, 1024, 4096, 0, False),
    ("act_order_decode", 16, 512, 8192, 0, True),
    ("act_order_prefill", 200, 512, 2048, 0, True),
]


@pytest.fixture(scope="module")
def env():
    lib = declare(pulsar_amd.capi())
    hip = Hip()
    yield lib, hip
    hip.free_all()


def _marlin_weights(lib, hip, p):
    """Device MARLIN words and fp32 [K/G, N] scales from the reference's CT
    packing (pw4_repack_w4a16), or, with act-order, GPTQ words repacked in
    permuted order, fp16 scales, zero points and the permutation."""
    n, k = p.n, p.k
    words = lib.pw4_marlin_words(n, k)
    wm = hip.malloc(words * 4)
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
    assert hip.download(status, (1,), np.int32)[0] == 0
    qw = hip.upload(p.qweight())
    assert lib.pw4_repack_gptq(qw, perm, n, k, wm, None) == 0
    s16 = hip.upload(O.f32_to_f16_bits(p.scale_kn))
    qz = hip.upload(p.qzeros())
    return wm, s16, DTYPE_F16, qz, perm


def test_shared_workspace_across_plans(env):
    lib, hip = env
    problems = []
    for i, (name, m, n, k, splits, act) in enumerate(CASES):
        p = O.make_problem(m, n, k, G, seed=50 + i, symmetric=not act, act_order=act)
        problems.append((name, p, splits))
    ws_bytes = max(lib.pw4_gemm_w4a16_marlin_workspace_size(p.m, p.n, p.k, G, p.g_idx is not None, s)
                   for _, p, s in problems)
    ct_bytes = lib.pw4_gemm_w4a16_workspace_size(260, 1024, 4096, G, 0)
    ws_bytes = max(ws_bytes, ct_bytes)
    assert ws_bytes >= PW4_ZERO_REGION_BYTES
    ws = hip.malloc(ws_bytes)
    hip.memset(ws, 0, ws_bytes)  # cleared once
    for name, p, splits in problems:
        wm, sc, sdt, qz, perm = _marlin_weights(lib, hip, p)
        x = hip.upload(p.x16)
        y = hip.malloc(p.m * p.n * 2)
        rc = lib.pw4_gemm_w4a16_marlin(x, DTYPE_F16, wm, sc, sdt, qz, perm, y, p.m, p.n, p.k, G, splits, ws,
                                       ws_bytes, None)
        assert rc == 0, (name, lib.pw4_status_string(rc), lib.pw4_last_hip_error())
        out = hip.download(y, (p.m, p.n), np.uint16)
        check(torch.from_numpy(out.view(np.float16)), p.reference(), torch.float16, f"C ABI {name}")
        zero = hip.download(ws, (PW4_ZERO_REGION_BYTES,), np.uint8)
        assert not zero.any(), f"{name}: zero region left nonzero at byte {int(np.flatnonzero(zero)[0])}"
    # the reference's first op on the CT packing: repacked into the workspace per call
    p = O.make_problem(260, 1024, 4096, G, seed=70)
    x = hip.upload(p.x16)
    packed = hip.upload(p.ct_packed())
    sc = hip.upload(p.scale_nk.astype(np.float32))
    y = hip.malloc(p.m * p.n * 2)
    rc = lib.pw4_gemm_w4a16(x, DTYPE_F16, packed, sc, y, p.m, p.n, p.k, G, 0, ws, ws_bytes, None)
    assert rc == 0, lib.pw4_status_string(rc)
    out = hip.download(y, (p.m, p.n), np.uint16)
    check(torch.from_numpy(out.view(np.float16)), p.reference(), torch.float16, "C ABI gemm_w4a16 (CT)")
    assert not hip.download(ws, (PW4_ZERO_REGION_BYTES,), np.uint8).any()


def test_workspace_too_small_is_rejected(env):
    lib, hip = env
    p = O.make_problem(8, 1024, 14336, G, seed=80)
    need = lib.pw4_gemm_w4a16_marlin_workspace_size(p.m, p.n, p.k, G, 0, 0)
    assert need > 0
    wm, sc, sdt, qz, perm = _marlin_weights(lib, hip, p)
    x = hip.upload(p.x16)
    y = hip.malloc(p.m * p.n * 2)
    ws = hip.malloc(need)
    hip.memset(ws, 0, need)
    assert lib.pw4_gemm_w4a16_marlin(x, DTYPE_F16, wm, sc, sdt, qz, perm, y, p.m, p.n, p.k, G, 0, ws, need - 1,
                                     None) == -3
    assert lib.pw4_gemm_w4a16_marlin(x, DTYPE_F16, wm, sc, sdt, qz, perm, y, p.m, p.n, p.k, G, 0, None, 0,
                                     None) == -3
    assert lib.pw4_gemm_w4a16_marlin(x, DTYPE_F16, wm, sc, sdt, qz, perm, y, p.m, p.n, p.k, G, 0, ws, need,
                                     None) == 0
    out = hip.download(y, (p.m, p.n), np.uint16)
    check(torch.from_numpy(out.view(np.float16)), p.reference(), torch.float16, "C ABI exact workspace")


@pytest.mark.parametrize("k,g", [(18, 6), (4096, 128), (4100, 4), (8200, 8), (28672, 128)])
@pytest.mark.parametrize("offset", [0, 4])
def test_gidx_to_perm_alignments(k, g, offset):
    """pw4_gidx_to_perm on a 16-byte aligned g_idx and one 4 bytes past it, at K up to and past
    4096 (the entry-by-entry walk, and past 4096 the 16-byte loads where aligned), against
    numpy's stable argsort; then one row moved to another group must set the status word."""
    lib = declare(pulsar_amd.capi())
    hip = Hip()
    try:
        rng = np.random.default_rng(k + offset)
        g_idx = rng.permutation(np.arange(k, dtype=np.int32) // g).astype(np.int32)
        buf = np.concatenate([np.zeros(offset // 4, np.int32), g_idx])
        base = hip.upload(buf)
        perm = hip.malloc(k * 4)
        status = hip.malloc(4)
        assert lib.pw4_gidx_to_perm(base + offset, k, g, perm, status, None) == 0
        assert hip.download(status, (1,), np.int32)[0] == 0
        assert np.array_equal(hip.download(perm, (k,), np.int32), np.argsort(g_idx, kind="stable"))
        bad = g_idx.copy()
        bad[np.argmax(bad == 0)] = 1  # group 0 one row short, group 1 one row over
        base2 = hip.upload(np.concatenate([np.zeros(offset // 4, np.int32), bad]))
        assert lib.pw4_gidx_to_perm(base2 + offset, k, g, perm, status, None) == 0
        assert hip.download(status, (1,), np.int32)[0] != 0
    finally:
        hip.free_all()

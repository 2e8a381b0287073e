"""GPU parity of the GPTQ ingestion path (asymmetric zero points, act-order
g_idx): repack bit-exact vs the oracle, perm == stable argsort(g_idx), and the
GEMM vs the fp32 oracle of w = (u - z[g_idx[k]]) * s[g_idx[k]].  The reference
has no zero points and no act-order, so these are pinned by the oracle and by
invariants (symmetric GPTQ == compressed-tensors repack, bytewise)."""

import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsar_amd import ops
from w4a16_case import baseline_case, check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k", [(256, 512), (200, 2176), (1000, 4224)])
def test_symmetric_gptq_equals_reference_repack(n, k):
    c = baseline_case(1, n, k, 128)
    wm_ct, _ = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float32), 128)
    wm_gptq, perm = ops.repack_w4a16_gptq(c.qweight(), None, 128)
    assert perm.numel() == 0
    assert torch.equal(wm_ct, wm_gptq)


# The act-order repack stages a column block's source words and the permutation in LDS,
# 8 to 64 columns wide by K and N: the shapes below take every width (K up to 28672, where
# the permutation is read from global memory), ragged N and K tails; N % 4 != 0 (130, 66)
# takes the word-by-word staging path at 8 and 16 columns.
@pytest.mark.parametrize("n,k,g", [(256, 1024, 128), (136, 512, 64), (64, 256, 32), (128, 4096, 128),
                                   (200, 2112, 64), (14336, 4096, 128), (4096, 4096, 128),
                                   (1024, 4096, 128), (4096, 14336, 128), (512, 28672, 128), (16384, 4096, 128),
                                   (2048, 4096, 128), (130, 1024, 128), (66, 2048, 64)])
def test_act_order_repack_bit_exact(n, k, g):
    # (the repack moves qweight only; int4 zero points exist for N % 8 == 0)
    c = baseline_case(1, n, k, g, seed=3, symmetric=n % 8 != 0, act_order=True)
    g_idx = torch.from_numpy(c.g_idx).cuda()
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    want_perm = O.gidx_perm(c.g_idx, g)
    assert np.array_equal(perm.cpu().numpy(), want_perm)
    assert np.array_equal(perm.cpu().numpy(), np.argsort(c.g_idx, kind="stable"))
    want = O.repack_gptq_marlin(O.pack_gptq(c.u), want_perm)
    assert np.array_equal(wm.cpu().numpy(), want)


# Every column block width on ragged N, each with the workgroups walking several blocks
# (grid 1 and 3) and one block each: 32 and 64 columns take the strided column groups
# (columns g, g + NW, ...), 8 and 16 the adjacent ones; N = 130 the word-by-word loads.
@pytest.mark.parametrize("n,k", [(200, 1024), (130, 512)])
@pytest.mark.parametrize("cols", [8, 16, 32, 64])
@pytest.mark.parametrize("grid", [1, 3, 0])
def test_act_order_repack_widths_and_grids(n, k, cols, grid):
    c = baseline_case(1, n, k, 64, seed=5, symmetric=True, act_order=True)
    g_idx = torch.from_numpy(c.g_idx).cuda()
    want = O.repack_gptq_marlin(O.pack_gptq(c.u), O.gidx_perm(c.g_idx, 64))
    keys = ("PW4_REPACK_COLS", "PW4_REPACK_GRID")
    old = {key: os.environ.get(key) for key in keys}
    os.environ["PW4_REPACK_COLS"] = str(cols)
    os.environ["PW4_REPACK_GRID"] = str(grid)
    try:
        wm, _ = ops.repack_w4a16_gptq(c.qweight(), g_idx, 64)
    finally:
        for key, v in old.items():
            if v is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = v
    assert np.array_equal(wm.cpu().numpy(), want)


@pytest.mark.parametrize("k,g", [(256, 64), (4160, 64), (28672, 128)])
def test_bad_g_idx_rejected(k, g):
    """A group with one row too many (and another one short), and a group id out of range,
    at the first and the last row: each walk of the permutation kernel sees it."""
    g_idx = torch.arange(k, dtype=torch.int32, device="cuda") // g
    qw = torch.zeros(k // 8, 64, dtype=torch.int32, device="cuda")
    _, perm = ops.repack_w4a16_gptq(qw, g_idx, g)
    assert torch.equal(perm.cpu(), torch.arange(k, dtype=torch.int32))
    for row, value in ((0, 1), (k - 1, 0), (3, k // g + 5), (k - 2, -1)):
        bad = g_idx.clone()
        bad[row] = value
        with pytest.raises(RuntimeError, match="g_idx"):
            ops.repack_w4a16_gptq(qw, bad, g)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 5, 16, 32, 64, 65, 256])
@pytest.mark.parametrize("sym,act", [(False, True), (False, False), (True, True)])
@pytest.mark.parametrize("sdtype", [torch.float16, torch.float32])
def test_gptq_gemm(m, sym, act, dtype, sdtype):
    n, k, g = 512, 2048, 128
    c = baseline_case(m, n, k, g, dtype=dtype, seed=7, symmetric=sym, act_order=act)
    g_idx = torch.from_numpy(c.g_idx).cuda() if act else None
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).to(sdtype).cuda()
    qz = None if sym else c.qzeros()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, qz, perm if act else None, g)
    check(y, c.y_ref, dtype, f"gptq m={m} sym={sym} act={act} {dtype} scales={sdtype}")


@pytest.mark.parametrize("m", [1, 16, 100])
@pytest.mark.parametrize("g", [32, 64, 16])
def test_gptq_gemm_small_groups(m, g):
    n, k = 128, 512
    c = baseline_case(m, n, k, g, seed=8, symmetric=False, act_order=True)
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), torch.from_numpy(c.g_idx).cuda(), g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, c.qzeros(), perm, g)
    check(y, c.y_ref, torch.float16, f"gptq small groups m={m} g={g}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 5, 16, 32])
@pytest.mark.parametrize("g", [16, 32])
@pytest.mark.parametrize("sym,act", [(True, False), (False, False), (False, True)])
def test_decode_small_groups(m, g, sym, act, dtype):
    """Group sizes 16 and 32 at decode M run the decode kernel (four or eight quant groups
    per 128-K step, one masked MFMA per group, zero points per group): against the oracle at
    a size where K = 4096 spans 128-256 groups and 1000 columns leave a partial column block."""
    n, k = 1000, 4096
    c = baseline_case(m, n, k, g, dtype=dtype, seed=9 + g + m, symmetric=sym, act_order=act)
    g_idx = torch.from_numpy(c.g_idx).cuda() if act else None
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, None if sym else c.qzeros(), perm if act else None, g)
    check(y, c.y_ref, dtype, f"decode small groups m={m} g={g} sym={sym} act={act} {dtype}")


@pytest.mark.parametrize("m", [1, 8, 24])
@pytest.mark.parametrize("g", [16, 32])
def test_decode_small_groups_ct_layout(m, g):
    """The reference's gemm_w4a16 (compressed-tensors packing, read in place) with G = 16, 32."""
    n, k = 768, 2048
    c = baseline_case(m, n, k, g, seed=30 + g + m)
    y = ops.gemm_w4a16(c.x, c.ct_packed(), c.scale(torch.float32), g)
    check(y, c.y_ref, torch.float16, f"ct small groups m={m} g={g}")

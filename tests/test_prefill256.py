"""GPU parity of the 256-wide prefill kernel (MARLIN layout, fp16 and bf16 activations)
against the fp32 oracle, on ragged M / N, every group size it takes, symmetric
and asymmetric weights with act-order, and forced K splits.  The tile choice is
pinned through PW4_PREFILL_TILE so that small cases reach this kernel; the
same cases on the 128 x 128 kernel must agree with the oracle as well.

Counterpart of the reference's large-M cases, pulsar/tests/test_w4a16_marlin.py:16-208.
"""

import os

import numpy as np
import pytest
import torch

from pulsar_amd import ops
from w4a16_case import baseline_case, check, reference_case

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[256, 128], ids=["tile256", "tile128"])
def tile(request):
    old = os.environ.get("PW4_PREFILL_TILE")
    os.environ["PW4_PREFILL_TILE"] = str(request.param)
    yield request.param
    if old is None:
        del os.environ["PW4_PREFILL_TILE"]
    else:
        os.environ["PW4_PREFILL_TILE"] = old


@pytest.mark.parametrize("m,n,k,g", [(65, 64, 64, 64), (300, 200, 320, 64), (257, 520, 1024, 128),
                                     (512, 4104, 256, 128), (700, 1000, 2048, 64), (1024, 768, 1536, 1536),
                                     (96, 8, 128, 64)])
def test_prefill_marlin_ragged(tile, m, n, k, g):
    c = reference_case(m, n, k, g, torch.float16, seed=11)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), g)
    y = ops.gemm_w4a16_marlin(c.x, wm, sm, g)
    check(y, c.y_ref, torch.float16, f"tile={tile} m={m} n={n} k={k} g={g}")


@pytest.mark.parametrize("num_splits", [1, 2, 3, 7, 8, 11])
def test_prefill_marlin_split(tile, num_splits):
    """Forced K slices, fewer and more than the 8 the automatic plans use; fp32 partials
    summed in slice order by the combine pass."""
    m, n, k, g = 600, 384, 2048, 128
    c = reference_case(m, n, k, g, torch.float16, seed=12)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), g)
    y = ops.gemm_w4a16_marlin_split(c.x, wm, sm, g, num_splits)
    check(y, c.y_ref, torch.float16, f"tile={tile} split={num_splits}")


@pytest.mark.parametrize("sym,act", [(True, False), (False, False), (False, True)])
@pytest.mark.parametrize("sdtype", [torch.float16, torch.float32])
def test_prefill_gptq(tile, sym, act, sdtype):
    m, n, k, g = 520, 328, 1024, 64
    c = baseline_case(m, n, k, g, seed=13, symmetric=sym, act_order=act)
    g_idx = torch.from_numpy(c.g_idx).cuda() if act else None
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).to(sdtype).cuda()
    qz = None if sym else c.qzeros()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, qz, perm if act else None, g)
    check(y, c.y_ref, torch.float16, f"tile={tile} gptq sym={sym} act={act} scales={sdtype}")


@pytest.fixture
def plan_env():
    keys = ("PW4_PREFILL_ROWS", "PW4_PREFILL_SPLITS", "PW4_PREFILL_EXACT", "PW4_PREFILL_KHALVES")
    old = {k: os.environ.get(k) for k in keys}
    yield os.environ
    for k, v in old.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def test_prefill_tiles_agree():
    """Both prefill kernels accumulate in fp32 over the same dequantized fp16
    weights; their outputs agree to fp16 output rounding."""
    m, n, k, g = 1024, 1024, 2048, 128
    c = reference_case(m, n, k, g, torch.float16, seed=14)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), g)
    ys = {}
    for t in (128, 256):
        os.environ["PW4_PREFILL_TILE"] = str(t)
        try:
            ys[t] = ops.gemm_w4a16_marlin(c.x, wm, sm, g).float()
        finally:
            del os.environ["PW4_PREFILL_TILE"]
    diff = (ys[128] - ys[256]).abs().max().item()
    assert diff <= 2e-3 * ys[128].abs().max().item(), diff


def test_prefill_tail_split(plan_env):
    """288 tiles of 256 x 256 on 256 CUs: the last N-tile columns run as a
    second launch of 128-row tiles; every column must match the oracle."""
    plan_env["PW4_PREFILL_ROWS"] = "256"
    plan_env["PW4_PREFILL_SPLITS"] = "1"
    m, n, k, g = 1024, 18432, 512, 128
    c = reference_case(m, n, k, g, torch.float16, seed=15)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), g)
    y = ops.gemm_w4a16_marlin(c.x, wm, sm, g)
    check(y, c.y_ref, torch.float16, "tail split m=1024 n=18432")


@pytest.mark.parametrize("exact", ["1", "0"], ids=["exact", "rounded"])
@pytest.mark.parametrize("rows", [256, 128])
@pytest.mark.parametrize("splits", [1, 3, 8])
@pytest.mark.parametrize("m,n", [(300, 520), (129, 264)])
def test_prefill_plans_agree_with_oracle(plan_env, exact, rows, splits, m, n):
    """Every plan the 256-wide kernel can be given -- 256-row tiles (8 waves)
    or 128-row tiles (4 waves), unsplit (with 128-row tail tiles) or with K
    slices, exact scaling (the default for fp16 x) or the scale rounded into
    the fp16 B fragment -- computes the same GEMM: ragged M and N against the
    oracle, fp16 and fp32 scales."""
    k, g = 1024, 128
    plan_env["PW4_PREFILL_ROWS"] = str(rows)
    plan_env["PW4_PREFILL_SPLITS"] = str(splits)
    plan_env["PW4_PREFILL_EXACT"] = exact
    c = reference_case(m, n, k, g, torch.float16, seed=16)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), g)
    y32 = ops.gemm_w4a16_marlin(c.x, wm, sm, g)
    check(y32, c.y_ref, torch.float16, f"rows={rows} splits={splits} m={m} n={n} fp32 scales")
    y16 = ops.gemm_w4a16_gptq(c.x, wm, sm.half(), None, None, g)
    check(y16, c.y_ref, torch.float16, f"rows={rows} splits={splits} m={m} n={n} fp16 scales")


@pytest.mark.parametrize("m,n,k,g", [(65, 64, 64, 64), (300, 200, 320, 64), (257, 520, 1024, 128),
                                     (700, 1000, 2048, 64)])
@pytest.mark.parametrize("splits", [1, 3])
def test_prefill_bf16(plan_env, m, n, k, g, splits):
    """bf16 activations on the 256-wide kernel: splice into 128.0, one fp32 fma per value with
    the bf16-rounded scale, v_cvt_pk_bf16_f32, bf16 MFMA; against the oracle at the bf16
    tolerance, unsplit and with K slices."""
    plan_env["PW4_PREFILL_SPLITS"] = str(splits)
    c = reference_case(m, n, k, g, torch.bfloat16, seed=17)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float32), g)
    y = ops.gemm_w4a16_marlin(c.x, wm, sm, g)
    assert y.dtype == torch.bfloat16
    check(y, c.y_ref, torch.bfloat16, f"bf16 m={m} n={n} k={k} g={g} splits={splits}")


@pytest.mark.parametrize("sym,act", [(True, False), (False, True)])
def test_prefill_bf16_gptq(sym, act):
    m, n, k, g = 390, 328, 1024, 64
    c = baseline_case(m, n, k, g, dtype=torch.bfloat16, seed=18, symmetric=sym, act_order=act)
    g_idx = torch.from_numpy(c.g_idx).cuda() if act else None
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, None if sym else c.qzeros(), perm if act else None, g)
    check(y, c.y_ref, torch.bfloat16, f"bf16 gptq sym={sym} act={act}")


def test_prefill_bf16_kernels_agree():
    """The 256-wide and the 128 x 128 kernels build the same bf16 B fragments and sum in fp32:
    their outputs agree to bf16 output rounding."""
    m, n, k, g = 512, 1024, 2048, 128
    c = reference_case(m, n, k, g, torch.bfloat16, seed=19)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float32), g)
    ys = {}
    for t in (128, 256):
        os.environ["PW4_PREFILL_TILE"] = str(t)
        try:
            ys[t] = ops.gemm_w4a16_marlin(c.x, wm, sm, g).float()
        finally:
            del os.environ["PW4_PREFILL_TILE"]
    diff = (ys[128] - ys[256]).abs().max().item()
    assert diff <= 1e-2 * ys[128].abs().max().item(), diff


@pytest.mark.parametrize("dtype,exact", [(torch.float16, "1"), (torch.float16, "0"), (torch.bfloat16, "0")],
                         ids=["f16-exact", "f16-rounded", "bf16"])
@pytest.mark.parametrize("splits", [1, 2])
def test_prefill_tile_shapes_bit_identical(plan_env, dtype, exact, splits):
    """256-row tiles (8 waves, one 32-column tile each) and 128-row tiles (4
    waves, two column tiles each) feed every output element the same B fragments
    and A rows through the same MFMA sequence (and, in exact mode, the same
    rescale points): the outputs are bit-identical."""
    m, n, k, g = 700, 1032, 2048, 128
    c = reference_case(m, n, k, g, dtype, seed=20)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float32), g)
    plan_env["PW4_PREFILL_EXACT"] = exact
    plan_env["PW4_PREFILL_SPLITS"] = str(splits)
    ys = {}
    for rows in (128, 256):
        plan_env["PW4_PREFILL_ROWS"] = str(rows)
        ys[rows] = ops.gemm_w4a16_marlin(c.x, wm, sm, g)
    check(ys[128], c.y_ref, dtype, f"128-row tiles {dtype} exact={exact}")
    assert torch.equal(ys[256], ys[128]), (ys[256].float() - ys[128].float()).abs().max().item()


@pytest.mark.parametrize("rows", [128, 256])
def test_prefill_split_sum_repeated_calls(plan_env, rows):
    """K-slice plans of different tile and slice counts in a row on one stream, sharing the
    shim's workspace, then the first again: each matches the oracle, and the repeated call is
    bit-identical to the first (the fixed-order sum does not depend on what ran before)."""
    plan_env["PW4_PREFILL_ROWS"] = str(rows)
    g = 128
    cases = [(300, 520, 1024, 4), (700, 1032, 2048, 8), (129, 264, 1024, 2), (300, 520, 1024, 4)]
    first = None
    for i, (m, n, k, s) in enumerate(cases):
        plan_env["PW4_PREFILL_SPLITS"] = str(s)
        c = reference_case(m, n, k, g, torch.float16, seed=21 + (i % 3))
        wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), g)
        y = ops.gemm_w4a16_marlin(c.x, wm, sm, g)
        check(y, c.y_ref, torch.float16, f"rows={rows} m={m} n={n} splits={s} call {i}")
        if i == 0:
            first = y.clone()
        elif i == 3:
            assert torch.equal(y, first)


@pytest.mark.parametrize("dtype,exact", [(torch.float16, "1"), (torch.float16, "0"), (torch.bfloat16, "0")],
                         ids=["f16-exact", "f16-rounded", "bf16"])
@pytest.mark.parametrize("splits", [1, 2, 3])
@pytest.mark.parametrize("m,n,k,g", [(300, 520, 1024, 128), (129, 264, 1088, 64), (257, 200, 64, 64),
                                     (65, 1032, 192, 64)])
def test_prefill_k_halves_agree_with_oracle(plan_env, dtype, exact, splits, m, n, k, g):
    """128-row tiles whose 8-wave workgroup runs each K slice as two halves and sums them
    through LDS: against the oracle with K slices of an even, odd (17 chunks: the second
    half is one chunk short) and single chunk (the second half is empty), fp16 and fp32
    scales."""
    plan_env["PW4_PREFILL_ROWS"] = "128"
    plan_env["PW4_PREFILL_KHALVES"] = "2"
    plan_env["PW4_PREFILL_SPLITS"] = str(splits)
    plan_env["PW4_PREFILL_EXACT"] = exact
    c = reference_case(m, n, k, g, dtype, seed=23)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float32), g)
    what = f"k halves {dtype} exact={exact} splits={splits} m={m} n={n} k={k}"
    check(ops.gemm_w4a16_marlin(c.x, wm, sm, g), c.y_ref, dtype, what + " fp32 scales")
    check(ops.gemm_w4a16_gptq(c.x, wm, sm.half(), None, None, g), c.y_ref, dtype, what + " fp16 scales")


@pytest.mark.parametrize("dtype,exact", [(torch.float16, "1"), (torch.float16, "0"), (torch.bfloat16, "0")],
                         ids=["f16-exact", "f16-rounded", "bf16"])
@pytest.mark.parametrize("k", [2048, 2112])
def test_prefill_k_halves_equal_two_slices(plan_env, dtype, exact, k):
    """Unsplit in two K halves is the two-slice plan summed in the kernel: the same slice
    boundary (ceil(chunks / 2)), the same fp32 sum first slice + second, one rounding --
    bit-identical to the two-slice plan's combine pass."""
    m, n, g = 700, 1032, 64
    c = reference_case(m, n, k, g, dtype, seed=24)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float32), g)
    plan_env["PW4_PREFILL_ROWS"] = "128"
    plan_env["PW4_PREFILL_EXACT"] = exact
    ys = {}
    for kh, s in ((2, 1), (1, 2)):
        plan_env["PW4_PREFILL_KHALVES"] = str(kh)
        plan_env["PW4_PREFILL_SPLITS"] = str(s)
        ys[kh] = ops.gemm_w4a16_marlin(c.x, wm, sm, g)
    check(ys[2], c.y_ref, dtype, f"k halves {dtype} exact={exact} k={k}")
    assert torch.equal(ys[2], ys[1]), (ys[2].float() - ys[1].float()).abs().max().item()


@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_k_halves_gptq(plan_env, splits, dtype):
    """K halves with zero points and act-order (config 4's operators)."""
    plan_env["PW4_PREFILL_ROWS"] = "128"
    plan_env["PW4_PREFILL_KHALVES"] = "2"
    plan_env["PW4_PREFILL_SPLITS"] = str(splits)
    m, n, k, g = 390, 328, 1024, 64
    c = baseline_case(m, n, k, g, dtype=dtype, seed=25, symmetric=False, act_order=True)
    g_idx = torch.from_numpy(c.g_idx).cuda()
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, c.qzeros(), perm, g)
    check(y, c.y_ref, dtype, f"k halves gptq act-order {dtype} splits={splits}")

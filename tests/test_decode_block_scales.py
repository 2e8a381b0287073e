"""Decode block scales: one scale (and zero-point) load per four ring steps, handed between
lane groups with ds_bpermute, in place of one load per step.

The planner takes them on layers of 24 MiB of weights or more (MARLIN layout, quant groups
of 128 K or more, not windowed); PW4_DECODE_BLOCK_SCALES=1/0 forces them on or off where
they apply.  They change where a step's scale and zero point come from, not what is
computed: every output must be bit-identical with and without them, over the variants of
the decode kernel they reach -- 16- and 32-row tiles, the 4- and 8-step rings, the exchange
tree, partial last ring blocks (a wave's steps not a multiple of four), uneven K-wave splits,
fp16 and bf16 activations, fp32 and fp16 scales, zero points and act-order, G = 128 and 256
-- and match the oracle at the reference's bars (the reference's counterpart is the scale
fetch of w4a16_marlin.cu:197-304).
"""

import os

import numpy as np
import pytest
import torch

from pulsar_amd import ops
from w4a16_case import baseline_case, check

pytestmark = pytest.mark.gpu


@pytest.fixture
def bs_env():
    keys = ("PW4_DECODE_BLOCK_SCALES", "PW4_DECODE_SPLITS")
    old = {k: os.environ.get(k) for k in keys}
    yield os.environ
    for k, v in old.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def _run(c, g, sdtype, act, sym):
    g_idx = torch.from_numpy(c.g_idx).cuda() if act else None
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).to(sdtype).cuda()
    return ops.gemm_w4a16_gptq(c.x, wm, scales, None if sym else c.qzeros(), perm if act else None, g)


# (m, n, k, g, splits): splits 0 = the planner's (direct store or exchange tree)
CASES = [
    (1, 512, 4096, 128, 0),     # 4-step ring, one block per wave
    (3, 320, 14336, 128, 0),    # 14 steps per wave: a partial last block
    (5, 256, 14336, 128, 0),    # K slices through the exchange tree
    (16, 512, 4096, 256, 0),    # G = 256: two steps per group
    (12, 256, 8192, 128, 4),    # forced tree slices
    (24, 192, 4096, 128, 0),    # 32-row tiles, 8-step ring
    (2, 200, 2560, 128, 0),     # 20 steps: an uneven K-wave split, ragged N
]


@pytest.mark.parametrize("m,n,k,g,splits", CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("sym,act", [(True, False), (False, True)])
def test_block_scales_bit_identical(bs_env, m, n, k, g, splits, dtype, sym, act):
    if splits:
        bs_env["PW4_DECODE_SPLITS"] = str(splits)
    c = baseline_case(m, n, k, g, dtype=dtype, seed=m * 7 + n, symmetric=sym, act_order=act)
    ys = {}
    for bs in ("1", "0"):
        bs_env["PW4_DECODE_BLOCK_SCALES"] = bs
        ys[bs] = _run(c, g, torch.float16, act, sym)
    check(ys["1"], c.y_ref, dtype, f"block scales m={m} n={n} k={k} g={g} {dtype} sym={sym} act={act}")
    assert torch.equal(ys["1"], ys["0"]), (ys["1"].float() - ys["0"].float()).abs().max().item()


@pytest.mark.parametrize("m", [1, 16])
def test_block_scales_fp32_scales(bs_env, m):
    """fp32 scales (the reference API's scale_marlin) through the same exchange."""
    c = baseline_case(m, 384, 4096, 128, seed=31 + m)
    ys = {}
    for bs in ("1", "0"):
        bs_env["PW4_DECODE_BLOCK_SCALES"] = bs
        ys[bs] = _run(c, 128, torch.float32, False, True)
    check(ys["1"], c.y_ref, torch.float16, f"block scales fp32 scales m={m}")
    assert torch.equal(ys["1"], ys["0"])

"""GPU parity of repack_w4a16 (bit-exact vs the CPU restatement of the
reference packer) and gemm_w4a16_marlin (vs the fp32 oracle), mirroring
pulsar/tests/test_w4a16_marlin.py:16-208."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsar_amd import ops
from w4a16_case import check, reference_case

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]
NK_SHAPES = [(128, 128), (256, 512), (512, 4096), (4096, 4096)]
M_SIZES = [1, 4, 16, 64]
GROUP_SIZES = [64, 128]


# K % 32 != 0 (144, 48) takes the repack's word-by-word reads; K = 2112 (66 tiles) ends in a
# partial 16-tile workgroup; 28672 x 4096 is the gate_up layer.  Each workgroup also writes
# the scales of the groups that start in its 512-K range: G = 384 puts two groups in the
# first range, and G = 80 (with K % 32 != 0) starts groups at every offset within a range.
@pytest.mark.parametrize("n,k,g", [(128, 256, 64), (100, 144, 48), (4096, 4096, 128), (6144, 4096, 128),
                                   (72, 48, 16), (1000, 2048, 64), (64, 64, 64), (200, 2112, 64),
                                   (28672, 4096, 128), (130, 1536, 384), (96, 1040, 80)])
@pytest.mark.parametrize("sdtype", [torch.float32, torch.float16, torch.bfloat16])
def test_repack_bit_exact(n, k, g, sdtype):
    rng = np.random.default_rng(n + k)
    vals = rng.integers(-8, 8, size=(n, k)).astype(np.int8)
    scale = (rng.random((n, k // g)) * 0.04 + 0.01).astype(np.float32)
    packed = O.pack_ct(vals)
    wm, sm = ops.repack_w4a16(torch.from_numpy(packed).cuda(), torch.from_numpy(scale).to(sdtype).cuda(), g)
    want = O.repack_marlin(packed)
    assert wm.dtype == torch.int32 and wm.shape == (want.size,)
    assert np.array_equal(wm.cpu().numpy(), want), "weight_marlin differs from the reference packer"
    s_in = torch.from_numpy(scale).to(sdtype).float().numpy()
    assert sm.dtype == torch.float32 and np.array_equal(sm.cpu().numpy(), O.scale_transpose(s_in))


def test_repack_roundtrip():
    # The reference's round-trip case (test_w4a16_marlin.py:118-171): decoding
    # weight_marlin through the documented nibble map recovers the int4 weights.
    n, k, g = 128, 256, 64
    c = reference_case(1, n, k, g, torch.float16, seed=2)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float32), g)
    from test_oracle import reference_decode_marlin

    rec, pad = reference_decode_marlin(wm.cpu().numpy(), n, k)
    assert np.array_equal(rec, c.vals.astype(np.int16))
    assert torch.allclose(sm.cpu(), torch.from_numpy(c.scale_nk).t(), atol=1e-6)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("group_size", GROUP_SIZES)
@pytest.mark.parametrize("nk", NK_SHAPES)
@pytest.mark.parametrize("m", M_SIZES)
def test_gemm_w4a16_marlin(m, nk, group_size, dtype):
    n, k = nk
    c = reference_case(m, n, k, group_size, dtype)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(dtype), group_size)
    y = ops.gemm_w4a16_marlin(c.x, wm, sm, group_size)
    check(y, c.y_ref, dtype, f"marlin m={m} n={n} k={k} g={group_size} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("group_size", GROUP_SIZES)
@pytest.mark.parametrize("nk", [(256, 512), (512, 4096)])
@pytest.mark.parametrize("m", [1, 16, 64])
def test_marlin_matches_gemm_w4a16(m, nk, group_size, dtype):
    n, k = nk
    c = reference_case(m, n, k, group_size, dtype, seed=1)
    y_simple = ops.gemm_w4a16(c.x, c.ct_packed(), c.scale(dtype), group_size)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(dtype), group_size)
    y_marlin = ops.gemm_w4a16_marlin(c.x, wm, sm, group_size)
    denom = y_simple.float().abs().max().item()
    diff = (y_marlin.float() - y_simple.float()).abs().max().item()
    rel = diff / denom if denom > 0 else diff
    tol = 2e-2 if dtype == torch.bfloat16 else 5e-3
    assert rel <= tol, f"m={m} n={n} k={k} g={group_size} {dtype} marlin-vs-simple rel={rel:.3e}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m", [1, 16, 17, 64, 65, 200])
@pytest.mark.parametrize("num_splits", [1, 2, 3, 5, 16, 64])
def test_gemm_w4a16_marlin_split(num_splits, m, dtype):
    n, k, g = 256, 1024, 128
    c = reference_case(m, n, k, g, dtype, seed=4)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(dtype), g)
    y = ops.gemm_w4a16_marlin_split(c.x, wm, sm, g, num_splits)
    check(y, c.y_ref, dtype, f"marlin split={num_splits} m={m} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k,g", [(17, 100, 144, 48), (70, 72, 48, 16), (129, 1000, 2048, 64),
                                     (33, 64, 64, 64), (300, 200, 320, 32), (2, 4104, 256, 128)])
def test_gemm_w4a16_marlin_ragged(m, n, k, g, dtype):
    c = reference_case(m, n, k, g, dtype, seed=5)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(dtype), g)
    y = ops.gemm_w4a16_marlin(c.x, wm, sm, g)
    check(y, c.y_ref, dtype, f"marlin ragged m={m} n={n} k={k} g={g} {dtype}")


def test_gemm_w4a16_marlin_errors():
    c = reference_case(2, 128, 128, 64, torch.float16)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), 64)
    with pytest.raises(RuntimeError, match="wrong size"):
        ops.gemm_w4a16_marlin(c.x, wm[:-1], sm, 64)
    with pytest.raises(RuntimeError, match="fp32"):
        ops.gemm_w4a16_marlin(c.x, wm, sm.half(), 64)
    with pytest.raises(RuntimeError, match="K/G"):
        ops.gemm_w4a16_marlin(c.x, wm, sm[:1], 64)


_OPCHECK_UTILS = ("test_schema", "test_faketensor", "test_aot_dispatch_dynamic")


def test_opcheck_repack_w4a16():
    for dtype in DTYPES:
        c = reference_case(1, 128, 128, 64, dtype, seed=6)
        torch.library.opcheck(torch.ops.pulsar.repack_w4a16, (c.ct_packed(), c.scale(dtype), 64),
                              test_utils=_OPCHECK_UTILS)


def test_opcheck_gemm_w4a16_marlin():
    for dtype in DTYPES:
        c = reference_case(4, 128, 128, 64, dtype, seed=6)
        wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(dtype), 64)
        torch.library.opcheck(torch.ops.pulsar.gemm_w4a16_marlin, (c.x, wm, sm, 64), test_utils=_OPCHECK_UTILS)

"""GPU parity of gemm_w4a16 / gemm_w4a16_split (compressed-tensors packing)
against the fp32 CPU oracle: the reference's test grid
(pulsar/tests/test_w4a16_gemm.py:19-32,89-158) plus the decode/prefill
boundary and ragged shapes."""

import pytest
import torch

from pulsar_amd import ops
from w4a16_case import check, reference_case

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]
NK_SHAPES = [(128, 128), (256, 512), (512, 4096)]
M_SIZES = [1, 4, 16, 64]
GROUP_SIZES = [64, 128]
SPLIT_COUNTS = [1, 2, 3, 4, 8]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("group_size", GROUP_SIZES)
@pytest.mark.parametrize("nk", NK_SHAPES)
@pytest.mark.parametrize("m", M_SIZES)
def test_gemm_w4a16(m, nk, group_size, dtype):
    n, k = nk
    c = reference_case(m, n, k, group_size, dtype)
    y = ops.gemm_w4a16(c.x, c.ct_packed(), c.scale(dtype), group_size)
    assert y.dtype == dtype and y.shape == (m, n)
    check(y, c.y_ref, dtype, f"gemm_w4a16 m={m} n={n} k={k} g={group_size} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("group_size", GROUP_SIZES)
@pytest.mark.parametrize("nk", NK_SHAPES)
@pytest.mark.parametrize("m", M_SIZES)
@pytest.mark.parametrize("num_splits", SPLIT_COUNTS)
def test_gemm_w4a16_split(num_splits, m, nk, group_size, dtype):
    n, k = nk
    c = reference_case(m, n, k, group_size, dtype)
    y = ops.gemm_w4a16_split(c.x, c.ct_packed(), c.scale(dtype), group_size, num_splits)
    check(y, c.y_ref, dtype, f"split={num_splits} m={m} n={n} k={k} g={group_size} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k,g", [
    (17, 96, 256, 64), (33, 200, 512, 128), (65, 128, 256, 64), (130, 72, 384, 128),
    (3, 40, 48, 16), (70, 24, 80, 16), (129, 136, 1024, 32), (1, 8, 16, 16), (5, 1000, 2048, 256),
])
def test_gemm_w4a16_ragged(m, n, k, g, dtype):
    c = reference_case(m, n, k, g, dtype, seed=3)
    y = ops.gemm_w4a16(c.x, c.ct_packed(), c.scale(torch.float32), g)
    check(y, c.y_ref, dtype, f"ragged m={m} n={n} k={k} g={g} {dtype}")


def test_gemm_w4a16_empty_and_errors():
    x = torch.zeros(0, 128, dtype=torch.float16, device="cuda")
    wp = torch.zeros(64, 16, dtype=torch.int32, device="cuda")
    ws = torch.ones(64, 2, dtype=torch.float16, device="cuda")
    assert ops.gemm_w4a16(x, wp, ws, 64).shape == (0, 64)
    x = torch.zeros(2, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="group_size"):
        ops.gemm_w4a16(x, wp, ws, 24)
    with pytest.raises(RuntimeError, match="weight_scale"):
        ops.gemm_w4a16(x, wp, ws[:, :1], 64)
    with pytest.raises(RuntimeError, match="K/8"):
        ops.gemm_w4a16(x, wp[:, :8], ws, 64)
    with pytest.raises(RuntimeError, match="num_splits"):
        ops.gemm_w4a16_split(x, wp, ws, 64, 0)
    with pytest.raises(RuntimeError, match="fp16 or bf16"):
        ops.gemm_w4a16(x.float(), wp, ws, 64)


_OPCHECK_UTILS = ("test_schema", "test_faketensor", "test_aot_dispatch_dynamic")


def test_opcheck_gemm_w4a16():
    for dtype in DTYPES:
        c = reference_case(4, 128, 128, 64, dtype, seed=1)
        torch.library.opcheck(torch.ops.pulsar.gemm_w4a16, (c.x, c.ct_packed(), c.scale(dtype), 64),
                              test_utils=_OPCHECK_UTILS)


def test_opcheck_gemm_w4a16_split():
    for dtype in DTYPES:
        c = reference_case(4, 128, 128, 64, dtype, seed=1)
        for num_splits in (1, 2, 4):
            torch.library.opcheck(torch.ops.pulsar.gemm_w4a16_split,
                                  (c.x, c.ct_packed(), c.scale(dtype), 64, num_splits), test_utils=_OPCHECK_UTILS)

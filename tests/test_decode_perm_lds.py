"""Act-order x gathered in the decode kernel's LDS.

With act-order (GPTQ g_idx) the GEMM multiplies x[:, perm] by the repacked weights.  The
library either gathers x[:, perm] into the workspace with a separate launch, or -- where the
decode plan has one K slice and both x as given and the gathered slice fit in LDS -- lets the
decode kernel copy x into LDS and gather its slice there (PW4_DECODE_PERM_LDS=0 forces the
separate launch).  Both hand the same activations to the same MFMA sequence: outputs must be
bit-identical, and match the oracle at the reference's bars (the reference has no act-order;
its x load is a plain tile copy, pulsar-core/src/kernels/w4a16_common.cuh:36-45).
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import pulsar_amd
from pulsar_amd import ops
from pw4_capi import DTYPE_BF16, DTYPE_F16, declare
from w4a16_case import baseline_case, check

pytestmark = pytest.mark.gpu


@pytest.fixture
def px_env():
    keys = ("PW4_DECODE_PERM_LDS", "PW4_DECODE_BLOCK_SCALES")
    old = {k: os.environ.get(k) for k in keys}
    yield os.environ
    for k, v in old.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def _plan(m, n, k, g, dtype):
    lib = declare(pulsar_amd.capi())
    buf = ctypes.create_string_buffer(160)
    dt = DTYPE_BF16 if dtype == torch.bfloat16 else DTYPE_F16
    assert lib.pw4_plan_describe(1, dt, DTYPE_F16, 1, 1, 0, m, n, k, g, 0, buf, 160) == 0
    return buf.value.decode()


# (m, n, k): 70B-like K = 8192 and 28672, 8B-like K = 4096 at M up to 8, ragged N, K not a
# multiple of the 128-K step (its tail zero-filled), and one 16-byte column per thread or more
CASES = [(1, 512, 8192), (4, 320, 8192), (1, 256, 28672), (8, 200, 4096), (3, 264, 2176), (2, 128, 1024)]


@pytest.mark.parametrize("m,n,k", CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("sym", [True, False])
@pytest.mark.parametrize("bs", ["0", "1"])
def test_perm_in_lds_bit_identical(px_env, m, n, k, dtype, sym, bs):
    g = 128
    px_env["PW4_DECODE_BLOCK_SCALES"] = bs
    c = baseline_case(m, n, k, g, dtype=dtype, seed=m * 13 + k, symmetric=sym, act_order=True)
    g_idx = torch.from_numpy(c.g_idx).cuda()
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    qz = None if sym else c.qzeros()
    px_env.pop("PW4_DECODE_PERM_LDS", None)
    assert " px=0" not in _plan(m, n, k, g, dtype), _plan(m, n, k, g, dtype)
    y_lds = ops.gemm_w4a16_gptq(c.x, wm, scales, qz, perm, g)
    px_env["PW4_DECODE_PERM_LDS"] = "0"
    assert " px=0" in _plan(m, n, k, g, dtype)
    y_sep = ops.gemm_w4a16_gptq(c.x, wm, scales, qz, perm, g)
    check(y_lds, c.y_ref, dtype, f"act-order in LDS m={m} n={n} k={k} {dtype} sym={sym} bs={bs}")
    assert torch.equal(y_lds, y_sep), (y_lds.float() - y_sep.float()).abs().max().item()


def test_perm_in_lds_fp32_scales_and_misaligned_perm(px_env):
    """fp32 scales, and a permutation that is not 16-byte aligned: the call falls back to
    the gather launch and still matches."""
    m, n, k, g = 2, 256, 8192, 128
    c = baseline_case(m, n, k, g, seed=41, symmetric=False, act_order=True)
    g_idx = torch.from_numpy(c.g_idx).cuda()
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales32 = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).float().cuda()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales32, c.qzeros(), perm, g)
    check(y, c.y_ref, torch.float16, "act-order in LDS, fp32 scales")
    shifted = torch.empty(k + 1, dtype=torch.int32, device="cuda")[1:]
    shifted.copy_(perm)
    assert shifted.data_ptr() % 16 != 0
    y2 = ops.gemm_w4a16_gptq(c.x, wm, scales32, c.qzeros(), shifted, g)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("m,k", [(16, 8192), (2, 28672), (1, 65536)])
def test_perm_in_lds_not_taken(m, k):
    """Where x and its gathered slice would not both fit in LDS (or K is past the kernel's
    per-thread columns), the plan keeps the gather launch."""
    assert " px=0" in _plan(m, 256, k, 128, torch.float16) or not _plan(m, 256, k, 128, torch.float16).startswith(
        "decode")

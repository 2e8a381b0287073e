"""Maximum sizes: a prefill GEMM whose output holds more than 2^31 elements.

M = 75008 rows x N = 28672 columns (Llama-3-8B gate_up, K = 4096) is 2.15e9 outputs;
row 74898 straddles element 2^31, so every output and partial offset past it needs
64-bit arithmetic.  The reference has no case this large (its largest is M = 4096,
pulsar/tests/test_w4a16_marlin.py:16-208); the checks are:

* sampled rows (the first and last rows, the rows around element 2^31, random rows)
  against the fp32 oracle at the fp16 / bf16 tolerances of the other parity tests;
* with the plan pinned (256-row tiles, no K slices), a block of rows around the seam
  and the last 300 rows, computed again in a call of their own (M = 512 / 300, still
  past the decode range), are bit-identical: output rows are independent and every
  output is the same fp32 sum in the same K order, so a wrong row or column offset
  in a far tile shows up as a mismatch.
"""

import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsar_amd import ops
from w4a16_case import check

pytestmark = pytest.mark.gpu

M, N, K, G = 75008, 28672, 4096, 128
SEAM = (1 << 31) // N  # the row holding output element 2^31


@pytest.fixture(scope="module")
def layer():
    rng = np.random.default_rng(75008)
    u = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((K // G, N))) * 0.02 + 1e-3).astype(np.float16)
    wm, _ = ops.repack_w4a16_gptq(torch.from_numpy(O.pack_gptq(u)).cuda(), None, G)
    w = (u.astype(np.float32) - 8.0) * np.repeat(s.astype(np.float32).T, G, axis=1)  # [N, K]
    rows = np.unique(np.concatenate([[0, 1, 255, 256, M - 257, M - 256, M - 2, M - 1],
                                     np.arange(SEAM - 2, SEAM + 3),
                                     rng.choice(M, size=40, replace=False)]))
    return wm, torch.from_numpy(s).cuda(), w, rows


@pytest.fixture
def pinned_plan():
    keys = ("PW4_PREFILL_ROWS", "PW4_PREFILL_SPLITS")
    old = {k: os.environ.get(k) for k in keys}
    os.environ.update({"PW4_PREFILL_ROWS": "256", "PW4_PREFILL_SPLITS": "1"})
    yield
    for k, v in old.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def _x(dtype):
    g = torch.Generator(device="cuda:0").manual_seed(7)
    return torch.randn(M, K, device="cuda:0", generator=g).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_output_past_2_31_elements(layer, dtype):
    wm, s, w, rows = layer
    assert SEAM * N < (1 << 31) < (SEAM + 1) * N
    x = _x(dtype)
    y = ops.gemm_w4a16_gptq(x, wm, s, None, None, G)
    assert y.shape == (M, N) and y.dtype == dtype
    idx = torch.from_numpy(rows).cuda()
    y_rows = y.index_select(0, idx)
    del y
    x_rows = x.index_select(0, idx).float().cpu().numpy().astype(np.float64)
    y_ref = x_rows @ w.T.astype(np.float64)
    check(y_rows, y_ref, dtype, f"M={M} N={N} K={K} {dtype} rows {rows[:4]}..{rows[-2:]}")


@pytest.mark.parametrize("lo,hi", [(SEAM - 300, SEAM + 212), (M - 300, M)], ids=["seam", "last"])
def test_far_rows_equal_a_small_call(layer, pinned_plan, lo, hi):
    wm, s, _, _ = layer
    x = _x(torch.float16)
    y_big = ops.gemm_w4a16_gptq(x, wm, s, None, None, G)[lo:hi].clone()
    y_small = ops.gemm_w4a16_gptq(x[lo:hi].contiguous(), wm, s, None, None, G)
    assert torch.equal(y_big, y_small)

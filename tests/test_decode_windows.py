"""Windowed decode plans against the fp32 oracle, at the reference's bars.

Where the activations of the whole K range do not fit in LDS (M * K * 2 bytes
past ~150 KB), the decode kernel either cuts K into slices whose partial sums
meet across workgroups (the exchange tree, or the counter path past eight
slices), or -- the windowed plan -- keeps one slice and gives every workgroup
one unit over the whole K, staging the activations window by window into two
LDS buffers: copy waves copy window w + 1 while the eight compute waves work on
window w, and the waves meet at one barrier per window.  Either way the result
is the reference's gemm_w4a16_marlin
(pulsar-core/src/kernels/w4a16_marlin.cu:354-551) on the repacked weights.

The library takes the windowed plan by default where the slices would take the
counter path; PW4_DECODE_WIN=1 takes it wherever it applies, which is how the
cases below reach it.  Each case is one the planner sends to the windowed
kernel on a 256-CU MI355X (checked through the workspace query: a windowed plan
needs no workspace, the sliced plan it replaces needs the exchange tree's zero
region or the counter path's partials), and covers one of its variants: 16- and
32-row tiles, the 4- and 8-step weight rings, one or two reduction buffers,
16- and 32-column units, fp16 and bf16 activations, zero points, act-order,
64-wide quant groups, and the SiLU-gated output.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import pulsar_amd
from pulsar_amd import ops
from w4a16_case import baseline_case, check

pytestmark = pytest.mark.gpu


def _workspace(m, n, k, g, has_perm=0):
    f = pulsar_amd.capi().pw4_gemm_w4a16_marlin_workspace_size
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_int, ctypes.c_int64]
    return f(m, n, k, g, has_perm, 0)


@pytest.fixture
def win_env():
    old = os.environ.get("PW4_DECODE_WIN")
    yield os.environ
    if old is None:
        os.environ.pop("PW4_DECODE_WIN", None)
    else:
        os.environ["PW4_DECODE_WIN"] = old


def _silu_ref(y_full: np.ndarray) -> np.ndarray:
    m, n = y_full.shape
    t = y_full.astype(np.float64).reshape(m, n // 16, 2, 8)
    g, u = t[:, :, 0, :], t[:, :, 1, :]
    return (g / (1.0 + np.exp(-g)) * u).reshape(m, n // 2)


# (m, n, k, g, x dtype, symmetric, act-order, silu): what each case pins
CASES = [
    (16, 4096, 14336, 128, torch.float16, True, False, False),   # Llama-3-8B down, 8-step ring
    (8, 4096, 14336, 128, torch.bfloat16, False, False, False),  # 4-step ring, bf16, zero points
    (12, 4096, 14336, 128, torch.float16, False, True, False),   # act-order (gathered x), zero points
    (6, 4096, 14336, 64, torch.float16, True, False, False),     # two quant groups per 128-K step
    (32, 4096, 4096, 128, torch.float16, True, False, False),    # 32-row tiles, one reduction buffer
    (24, 6144, 4096, 128, torch.bfloat16, True, False, False),   # 32-column units (4 K waves)
    (4, 8192, 28672, 128, torch.float16, True, False, False),    # Llama-3-70B down shape, 32-column units
    (16, 4096, 14336, 128, torch.float16, False, False, True),   # SiLU-gated output (2F = 4096)
]


@pytest.mark.parametrize("m,n,k,g,dtype,sym,act,silu", CASES)
def test_windowed_plan_matches_oracle(win_env, m, n, k, g, dtype, sym, act, silu):
    what = f"windowed m={m} n={n} k={k} g={g} {dtype} sym={sym} act={act} silu={silu}"
    print(what, flush=True)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the cases are chosen for the windowed plans of a 256-CU device")
    win_env["PW4_DECODE_WIN"] = "0"
    assert _workspace(m, n, k, g) > 0  # the sliced plan: exchange-tree slots
    win_env["PW4_DECODE_WIN"] = "1"
    assert _workspace(m, n, k, g) == 0  # the windowed plan
    c = baseline_case(m, n, k, g, dtype=dtype, seed=m * 7 + n + k, symmetric=sym, act_order=act)
    g_idx = torch.from_numpy(c.g_idx).cuda() if act else None
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    qz = None if sym else c.qzeros()
    if silu:
        y = ops.gemm_w4a16_silu_mul(c.x, wm, scales, qz, perm if act else None, g)
        torch.cuda.synchronize()
        assert y.shape == (m, n // 2) and y.dtype == dtype
        check(y, _silu_ref(c.y_ref), dtype, what)
        return
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, qz, perm if act else None, g)
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == dtype
    check(y, c.y_ref, dtype, what)
    # the sliced plan on the same inputs meets the same bar
    win_env["PW4_DECODE_WIN"] = "0"
    y0 = ops.gemm_w4a16_gptq(c.x, wm, scales, qz, perm if act else None, g)
    torch.cuda.synchronize()
    check(y0, c.y_ref, dtype, what + " (K slices)")


def test_default_plan_windows_past_the_tree(win_env):
    """Without the override, M = 32 at K = 28672 (Llama-3-70B down's K) needs 13 slices, past the
    exchange tree's eight: the library takes the windowed plan instead of the counter path."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the case is chosen for the windowed plan of a 256-CU device")
    m, n, k, g = 32, 4096, 28672, 128
    win_env["PW4_DECODE_WIN"] = "0"
    assert _workspace(m, n, k, g) >= 13 * m * n * 4  # counter path: fp32 partials per slice
    win_env.pop("PW4_DECODE_WIN", None)
    assert _workspace(m, n, k, g) == 0
    c = baseline_case(m, n, k, g, seed=29)
    wm, _ = ops.repack_w4a16_gptq(c.qweight(), None, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, None, None, g)
    torch.cuda.synchronize()
    check(y, c.y_ref, torch.float16, f"default windowed m={m} n={n} k={k}")


def test_windowed_plan_repeats_bitwise(win_env):
    """Calls back to back on one stream, and a captured graph's replays, give the same bits:
    the windowed kernel keeps no state across calls (no workspace, no counters)."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the case is chosen for the windowed plan of a 256-CU device")
    win_env["PW4_DECODE_WIN"] = "1"
    m, n, k, g = 16, 4096, 14336, 128
    assert _workspace(m, n, k, g) == 0
    c = baseline_case(m, n, k, g, seed=11)
    wm, _ = ops.repack_w4a16_gptq(c.qweight(), None, g)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    first = ops.gemm_w4a16_gptq(c.x, wm, scales, None, None, g)
    for _ in range(5):
        assert torch.equal(ops.gemm_w4a16_gptq(c.x, wm, scales, None, None, g), first)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.gemm_w4a16_gptq(c.x, wm, scales, None, None, g)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = ops.gemm_w4a16_gptq(c.x, wm, scales, None, None, g)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)

"""GPU parity at the BASELINE.json shapes (Llama-3-8B / 70B layers), full size.

Decode shapes (M <= 16) are checked against the full fp32 oracle.  For the
prefill shapes only a seeded subset of output rows is recomputed on the CPU:
rows of y = x @ W^T are independent, so the subset check is exact for those
rows, and a checksum of the whole output (column sums of y against
(1^T x) @ W^T over the same oracle) covers every row.

Every case is held to all three fp16 bars of the north star (rel-L2 <= 1e-3,
max-abs <= 1e-2 beyond the fp16 output's own rounding, and the reference's
max-relative bar); the measured figures are printed for the record.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsar_amd import ops
from w4a16_case import baseline_case, check, metrics

pytestmark = pytest.mark.gpu

LLAMA8B = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 28672), "down": (14336, 4096)}
LLAMA70B = {"qkv": (8192, 10240), "gate_up": (8192, 57344), "down": (28672, 8192)}


@pytest.mark.parametrize("layer", list(LLAMA8B))
@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_decode_llama8b(layer, m):
    k, n = LLAMA8B[layer]
    c = baseline_case(m, n, k, 128, seed=0)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), 128)
    y = ops.gemm_w4a16_marlin(c.x, wm, sm, 128)
    r = check(y, c.y_ref, torch.float16, f"decode {layer} m={m}")
    print(f"decode {layer} m={m}: {r}")


@pytest.mark.parametrize("layer", list(LLAMA8B))
@pytest.mark.parametrize("m", [1, 16, 256])
def test_llama8b_bf16(layer, m):
    """bf16 activations (the reference engine's dtype) at the Llama-3-8B shapes, decode and a
    prefill size, at the reference's bf16 bar; prefill on a row subset."""
    k, n = LLAMA8B[layer]
    rows = None if m <= 16 else np.unique(np.concatenate([np.arange(0, m, 7), [m - 1]]))
    c = baseline_case(m, n, k, 128, dtype=torch.bfloat16, seed=2, rows=rows)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), 128)
    y = ops.gemm_w4a16_marlin(c.x, wm, sm, 128)
    assert y.dtype == torch.bfloat16
    if rows is not None:
        y = y[torch.from_numpy(rows).cuda()]
    r = check(y, c.y_ref, torch.bfloat16, f"bf16 {layer} m={m}")
    print(f"bf16 {layer} m={m}: {r}")


@pytest.mark.parametrize("layer", list(LLAMA8B))
@pytest.mark.parametrize("m", [256, 1024, 4096])
def test_prefill_llama8b_rows(layer, m):
    k, n = LLAMA8B[layer]
    rows = np.unique(np.concatenate([np.arange(0, m, max(m // 48, 1)), [m - 1]]))
    c = baseline_case(m, n, k, 128, seed=0, rows=rows)
    wm, sm = ops.repack_w4a16(c.ct_packed(), c.scale(torch.float16), 128)
    y = ops.gemm_w4a16_marlin(c.x, wm, sm, 128)
    r = check(y[torch.from_numpy(rows).cuda()], c.y_ref, torch.float16, f"prefill {layer} m={m}")
    print(f"prefill {layer} m={m}: {r}")


@pytest.mark.parametrize("layer", list(LLAMA70B))
@pytest.mark.parametrize("m", [1, 16, 2048])
def test_act_order_llama70b(layer, m):
    k, n = LLAMA70B[layer]
    rows = None if m <= 16 else np.arange(0, m, 97)
    c = baseline_case(m, n, k, 128, seed=1, symmetric=False, act_order=True, rows=rows)
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), torch.from_numpy(c.g_idx).cuda(), 128)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, c.qzeros(), perm, 128)
    if rows is not None:
        y = y[torch.from_numpy(rows).cuda()]
    r = check(y, c.y_ref, torch.float16, f"act-order {layer} m={m}")
    print(f"act-order 70B {layer} m={m}: {r}")


@pytest.mark.parametrize("layer", list(LLAMA70B))
@pytest.mark.parametrize("m", [1, 16, 2048])
def test_act_order_llama70b_bf16(layer, m):
    """Config 4 with bf16 activations (the reference engine's dtype): asymmetric int4,
    act-order, fp16 scales, at the reference's bf16 bar; M = 2048 on a row subset."""
    k, n = LLAMA70B[layer]
    rows = None if m <= 16 else np.arange(0, m, 97)
    c = baseline_case(m, n, k, 128, dtype=torch.bfloat16, seed=5, symmetric=False, act_order=True, rows=rows)
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), torch.from_numpy(c.g_idx).cuda(), 128)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    y = ops.gemm_w4a16_gptq(c.x, wm, scales, c.qzeros(), perm, 128)
    assert y.dtype == torch.bfloat16
    if rows is not None:
        y = y[torch.from_numpy(rows).cuda()]
    r = check(y, c.y_ref, torch.bfloat16, f"act-order bf16 {layer} m={m}")
    print(f"act-order 70B bf16 {layer} m={m}: {r}")


@pytest.mark.parametrize("layer", list(LLAMA8B))
def test_output_checksum_prefill(layer):
    """Column sums of y over ALL rows against the oracle: sum_m y[m, :] equals
    (sum_m x[m, :]) @ W^T up to fp16 output rounding of each term."""
    k, n = LLAMA8B[layer]
    m = 4096
    p = O.make_problem(m, n, k, 128, seed=2)
    w = p.dequant()
    colsum_ref = O.gemm_f32(np.ascontiguousarray(p.xf.sum(axis=0, keepdims=True)), w)[0]
    c_x = torch.from_numpy(p.x16.view(np.int16).copy()).view(torch.float16).cuda()
    packed = torch.from_numpy(p.ct_packed()).cuda()
    wm, sm = ops.repack_w4a16(packed, torch.from_numpy(p.scale_nk).half().cuda(), 128)
    y = ops.gemm_w4a16_marlin(c_x, wm, sm, 128)
    colsum = y.float().sum(dim=0).cpu().numpy()
    r = metrics(torch.from_numpy(colsum), colsum_ref)
    print(f"checksum {layer} m={m}: {r}")
    assert r["rel_l2"] < 1e-3, r

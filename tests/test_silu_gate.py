"""The SwiGLU gate in one GEMM: y = silu(x @ Wg^T) * (x @ Wu^T).

The reference runs two at::linear calls and at::silu(gate) * up
(pulsar-core/src/model/qwen3.cpp:116-118).  Here gate and up are one weight of
2F columns interleaved by 8 (fused columns 16j..16j+7 gate, 16j+8..16j+15 up).

* CPU: W4A16SiluGate.from_members regroups two repacked MARLIN weights; its
  words equal the oracle's repack of the column-interleaved weight bit for bit,
  and its scales and zero points interleave the same way.
* GPU: gemm_w4a16_silu_mul against silu(g) * u of the fp32 oracle GEMM, on
  every plan that produces it: decode without K slices (the kernel pairs the
  columns), decode with exchange-tree or counter K slices, the 256-wide prefill
  kernel unsplit (fp16 and bf16 x) and split (split-K combine), and the
  128 x 128 kernel (pinned through PW4_PREFILL_TILE) unsplit and split; the
  decode K-slice and unsplit 128 x 128 plans gate the GEMM output in a second
  pass.
"""

import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsar_amd import ops
from pulsar_amd.linear import W4A16Linear, W4A16SiluGate
from w4a16_case import baseline_case, check

G = 128


def _interleave_rows(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """[F, ...] gate and up -> [2F, ...] with rows 16j..16j+7 = a[8j..8j+7], 16j+8.. = b[8j..]."""
    f = a.shape[0]
    return np.stack([a.reshape(f // 8, 8, *a.shape[1:]), b.reshape(f // 8, 8, *b.shape[1:])], axis=1).reshape(
        2 * f, *a.shape[1:])


@pytest.mark.parametrize("f,k", [(64, 128), (192, 320), (256, 64)])
def test_interleave_matches_repack_of_interleaved_columns(f, k):
    rng = np.random.default_rng(f + k)
    g_vals = rng.integers(-8, 8, size=(f, k)).astype(np.int8)
    u_vals = rng.integers(-8, 8, size=(f, k)).astype(np.int8)
    gs = 64
    g_s = rng.random((k // gs, f)).astype(np.float32)
    u_s = rng.random((k // gs, f)).astype(np.float32)
    g_z = rng.integers(-2 ** 31, 2 ** 31, size=(k // gs, f // 8), dtype=np.int64).astype(np.int32)
    u_z = rng.integers(-2 ** 31, 2 ** 31, size=(k // gs, f // 8), dtype=np.int64).astype(np.int32)

    def lin(vals, s, z):
        wm = torch.from_numpy(O.repack_marlin(O.pack_ct(vals)))
        return W4A16Linear(wm, torch.from_numpy(s), gs, k, f, qzeros=torch.from_numpy(z))

    fused = W4A16SiluGate.from_members(lin(g_vals, g_s, g_z), lin(u_vals, u_s, u_z))
    want = O.repack_marlin(O.pack_ct(_interleave_rows(g_vals, u_vals)))
    assert np.array_equal(fused.weight_marlin.numpy(), want)
    assert np.array_equal(fused.scales.numpy(), _interleave_rows(g_s.T, u_s.T).T)
    assert np.array_equal(fused.qzeros.numpy(), np.stack([g_z, u_z], axis=2).reshape(k // gs, f // 4))
    assert (fused.in_features, fused.out_features, fused.intermediate) == (k, 2 * f, f)


def test_from_members_rejects_mismatches():
    wm = torch.zeros(64 * 128 // 8, dtype=torch.int32)
    a = W4A16Linear(wm, torch.ones(1, 64), 128, 128, 64)
    b = W4A16Linear(torch.zeros(128 * 128 // 8, dtype=torch.int32), torch.ones(1, 128), 128, 128, 128)
    with pytest.raises(ValueError):
        W4A16SiluGate.from_members(a, b)
    c = W4A16Linear(torch.zeros(64 * 128 // 8, dtype=torch.int32), torch.ones(1, 64).half(), 128, 128, 64)
    with pytest.raises(ValueError):
        W4A16SiluGate.from_members(a, c)


def _silu_ref(y_full: np.ndarray) -> np.ndarray:
    m, n = y_full.shape
    t = y_full.astype(np.float64).reshape(m, n // 16, 2, 8)
    g, u = t[:, :, 0, :], t[:, :, 1, :]
    return (g / (1.0 + np.exp(-g)) * u).reshape(m, n // 2)


@pytest.fixture
def plan_env():
    keys = ("PW4_PREFILL_ROWS", "PW4_PREFILL_SPLITS", "PW4_PREFILL_TILE", "PW4_PREFILL_KHALVES")
    old = {k: os.environ.get(k) for k in keys}
    yield os.environ
    for k, v in old.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


# (m, n = 2F, k, x dtype, plan overrides, absolute bound).  The absolute bound (max
# error within half an fp16 ulp + 1e-2) holds where both GEMM outputs are exact fp32 sums of
# exact (u - z) * s products and the gate is applied to them in fp32: the decode kernel's
# direct store, and the 256-wide prefill kernel with fp16 x (exact scaling) whether it gates in
# its epilogue or in the split-K combine.  The 128 x 128 kernel and the bf16 path round q * s to
# 16 bits in the B fragment (as the reference's MMA path does), gated-after plans round gate
# and up to fp16 first, and the product scales either error by the other factor; those cases
# are held to the relative bounds (rel-L2 1e-3, max 5e-3 of max |y|).
CASES = [
    (1, 512, 512, torch.float16, {}, True),      # decode, direct store
    (16, 1024, 1024, torch.float16, {}, True),
    (5, 4160, 256, torch.float16, {}, True),     # N past a 64-column block boundary
    (24, 512, 4096, torch.float16, {}, False),   # decode, exchange-tree K slices
    (32, 256, 28672, torch.float16, {"PW4_DECODE_WIN": "0"}, False),  # decode, counter K slices
    (32, 256, 28672, torch.float16, {}, False),  # decode, K windows where it would take the counter
    (48, 256, 4096, torch.float16, {}, False),   # 128-row prefill tile, then the SiLU pass (M > 32)
    (300, 1024, 512, torch.float16, {"PW4_PREFILL_SPLITS": "1"}, True),    # 256-wide prefill, unsplit
    (200, 1024, 512, torch.bfloat16, {"PW4_PREFILL_SPLITS": "1"}, False),  # the same, bf16 x
    (129, 512, 2048, torch.float16, {"PW4_PREFILL_SPLITS": "4"}, True),    # 256-wide, K slices -> combine
    (300, 1040, 1024, torch.bfloat16, {"PW4_PREFILL_SPLITS": "3", "PW4_PREFILL_ROWS": "256"}, False),  # 8 waves
    (129, 512, 2048, torch.float16, {"PW4_PREFILL_SPLITS": "12"}, True),   # 256-wide, 12 slices
    # 128-row tiles in two K halves (8 waves): gated in the epilogue, or in the combine
    (300, 1024, 512, torch.float16, {"PW4_PREFILL_SPLITS": "1", "PW4_PREFILL_KHALVES": "2"}, True),
    (200, 1024, 640, torch.bfloat16, {"PW4_PREFILL_SPLITS": "1", "PW4_PREFILL_KHALVES": "2", "PW4_PREFILL_ROWS": "128"},
     False),
    (129, 512, 2048, torch.float16, {"PW4_PREFILL_SPLITS": "2", "PW4_PREFILL_KHALVES": "2"}, True),
    (100, 512, 4096, torch.bfloat16, {"PW4_PREFILL_TILE": "128"}, False),  # 128 x 128 kernel, K slices
    (700, 1024, 256, torch.float16, {"PW4_PREFILL_TILE": "128"}, False),   # 128 x 128 kernel, unsplit
]


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,dtype,env,abs_bound", CASES)
@pytest.mark.parametrize("sym,act", [(True, False), (False, True)])
def test_silu_mul_matches_oracle(plan_env, m, n, k, dtype, env, abs_bound, sym, act):
    plan_env.update(env)
    c = baseline_case(m, n, k, G, dtype=dtype, seed=m + n, symmetric=sym, act_order=act)
    g_idx = torch.from_numpy(c.g_idx).cuda() if act else None
    wm, perm = ops.repack_w4a16_gptq(c.qweight(), g_idx, G)
    scales = torch.from_numpy(np.ascontiguousarray(c.scale_nk.T)).half().cuda()
    qz = None if sym else c.qzeros()
    y = ops.gemm_w4a16_silu_mul(c.x, wm, scales, qz, perm if act else None, G)
    assert y.shape == (m, n // 2) and y.dtype == dtype
    check(y, _silu_ref(c.y_ref), dtype, f"silu m={m} n={n} k={k} {dtype} sym={sym} act={act}",
          abs_excess=abs_bound)


@pytest.mark.gpu
def test_silu_gate_module_equals_separate_linears():
    """W4A16SiluGate.from_members on two repacked linears computes silu(gate(x)) * up(x) as the
    separate W4A16Linear calls do, up to the rounding of gate and up to fp16 there."""
    f, k = 1024, 2048
    rng = np.random.default_rng(3)
    lins = []
    for _ in range(2):
        u = rng.integers(0, 16, size=(f, k)).astype(np.uint8)
        s = (np.abs(rng.standard_normal((k // G, f))) * 0.02 + 1e-3).astype(np.float16)
        lins.append(W4A16Linear.from_gptq(torch.from_numpy(O.pack_gptq(u)).cuda(), torch.from_numpy(s).cuda(), G))
    fused = W4A16SiluGate.from_members(*lins)
    for shape in ((1, k), (3, 5, k), (300, k)):
        x = torch.randn(*shape, device="cuda:0").half()
        y = fused(x)
        assert y.shape == (*shape[:-1], f)
        g, u = lins[0](x).float(), lins[1](x).float()
        ref = torch.nn.functional.silu(g) * u
        torch.testing.assert_close(y.float(), ref, rtol=4e-3, atol=4e-3 * ref.abs().max().item())

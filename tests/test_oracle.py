"""Pins the CPU oracle (oracle/liborc.so) before anything is checked against it.

Each check is independent of the oracle's own code: a library routine (numpy
float16 rounding, numpy float64 matmul, numpy stable argsort), the reference's
own decoder for the MARLIN layout (pulsar/tests/test_w4a16_marlin.py:137-171,
restated below), hand-built known answers, and the committed golden fixtures.
"""

import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---- conversions -------------------------------------------------------------


def test_f16_rne_matches_numpy(orc):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10,
        rng.standard_normal(20000).astype(np.float32) * 1e-5,  # subnormal range
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 5.96e-8, 2.98e-8, 2.99e-8, np.inf, -np.inf],
                 dtype=np.float32),
    ])
    # halfway cases: odd and even mantissas + half ulp
    base = np.arange(1024, 2048, dtype=np.float32)
    vals = np.concatenate([vals, base + 0.5, -(base + 0.5)])
    got = orc.f32_to_f16_bits(vals)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = orc.f16_bits_to_f32(np.arange(0, 65536, dtype=np.uint16))
    want_back = np.arange(0, 65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(back), np.isnan(want_back))
    ok = ~np.isnan(want_back)
    assert np.array_equal(back[ok], want_back[ok])


def test_bf16_rne(orc):
    rng = np.random.default_rng(1)
    vals = rng.standard_normal(50000).astype(np.float32)
    got = orc.f32_to_bf16_bits(vals)
    # round to nearest even on the upper 16 bits, computed with float64 arithmetic
    u = vals.view(np.uint32).astype(np.uint64)
    lower = u & 0xFFFF
    upper = u >> 16
    round_up = (lower > 0x8000) | ((lower == 0x8000) & ((upper & 1) == 1))
    want = (upper + round_up).astype(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(orc.bf16_bits_to_f32(got), (got.astype(np.uint32) << 16).view(np.float32))


# ---- seeded generator ----------------------------------------------------------


def test_generator_deterministic_and_distributed(orc):
    a = orc.normal(0, 1, 200000)
    b = orc.normal(0, 1, 200000)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, orc.normal(1, 1, 200000))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    u = orc.uint4(0, 2, 160000)
    counts = np.bincount(u, minlength=16)
    assert counts.min() > 9000 and counts.max() < 11000
    s = orc.abs_normal(0, 3, 100000)
    assert s.min() >= 1e-3 and abs(s.mean() - (0.02 * np.sqrt(2 / np.pi) + 1e-3)) < 5e-4
    p = orc.perm(0, 5, 4096)
    assert np.array_equal(np.sort(p), np.arange(4096))


# ---- compressed-tensors packing (reference _pack_int4 convention) ------------------


def test_pack_ct_known_answers(orc):
    vals = np.zeros((2, 16), dtype=np.int8)
    vals[0, 0] = 1  # nibble 0 of word [0,0]
    vals[0, 9] = -1  # nibble 1 of word [0,1] = 0xF
    vals[1, 7] = -8  # nibble 7 of word [1,0] = 0x8
    vals[1, 12] = 7  # nibble 4 of word [1,1]
    p = orc.pack_ct(vals).view(np.uint32)
    assert p.shape == (2, 2)
    assert p[0, 0] == 0x00000001 and p[0, 1] == 0x000000F0
    assert p[1, 0] == 0x80000000 and p[1, 1] == 0x00070000
    rng = np.random.default_rng(3)
    v = rng.integers(-8, 8, size=(37, 64)).astype(np.int8)
    assert np.array_equal(orc.unpack_ct(orc.pack_ct(v)), v)


def test_gptq_packing(orc):
    rng = np.random.default_rng(4)
    u = rng.integers(0, 16, size=(24, 64)).astype(np.uint8)
    q = orc.pack_gptq(u)
    assert q.shape == (8, 24)
    # word [r, n] nibble j holds u[n, 8r + j]
    assert ((q.view(np.uint32)[2, 5] >> 12) & 0xF) == u[5, 19]
    assert np.array_equal(orc.unpack_gptq(q), u)
    z = rng.integers(0, 16, size=(4, 24)).astype(np.uint8)
    qz = orc.pack_gptq_zeros(z)
    assert ((qz.view(np.uint32)[1, 2] >> 4) & 0xF) == z[1, 17]
    assert np.array_equal(orc.unpack_gptq_zeros(qz), z)
    # compressed-tensors signed s  <->  GPTQ unsigned u = s + 8
    ct = orc.pack_ct((u.astype(np.int16) - 8).astype(np.int8))
    assert np.array_equal(orc.ct_to_gptq(ct), q)


# ---- MARLIN layout -----------------------------------------------------------------


def reference_decode_marlin(wm, n, k):
    """The decoder of the reference's test_repack_roundtrip
    (pulsar/tests/test_w4a16_marlin.py:137-171), restated with numpy: recovers
    the signed int4 value of every (col, k) from the MARLIN words."""
    block_n = block_k = 64
    k_tile, n_sub = 32, 8
    wm = wm.astype(np.int64) & 0xFFFFFFFF
    n_padded = -(-n // block_n) * block_n
    k_padded = -(-k // block_k) * block_k
    n_chunks = k_padded // block_k
    k_tiles_per_chunk = block_k // k_tile
    idx = np.arange(wm.size)
    lane = idx % 32
    sub_idx = (idx // 32) % n_sub
    k_tile_idx = (idx // (32 * n_sub)) % k_tiles_per_chunk
    k_chunk = (idx // (32 * n_sub * k_tiles_per_chunk)) % n_chunks
    col_block = idx // (32 * n_sub * k_tiles_per_chunk * n_chunks)
    col = (col_block * n_sub + sub_idx) * 8 + (lane >> 2)
    tg = lane & 3
    k_base = (k_chunk * k_tiles_per_chunk + k_tile_idx) * k_tile
    out = np.zeros((n, k), dtype=np.int16)
    pad = []
    for nib_idx in range(8):
        nib = (wm >> (4 * nib_idx)) & 0xF
        val = nib ^ 8
        val = np.where(val >= 8, val - 16, val)
        base = [0, 8, 16, 24, 0, 8, 16, 24][nib_idx]
        kk = k_base + base + tg * 2 + (1 if nib_idx >= 4 else 0)
        inside = (col < n) & (kk < k)
        out[col[inside], kk[inside]] = val[inside]
        pad.append(nib[~inside])
    assert wm.size == n_padded * k_padded // 8
    return out, np.concatenate(pad)


@pytest.mark.parametrize("n,k", [(128, 256), (64, 64), (100, 136), (8, 16), (200, 520)])
def test_marlin_forward_vs_reference_decoder(orc, n, k):
    vals = orc.uint4(2, 7, (n, k)).astype(np.int16) - 8
    wm = orc.repack_marlin(orc.pack_ct(vals.astype(np.int8)))
    rec, pad = reference_decode_marlin(wm, n, k)
    assert np.array_equal(rec, vals)
    assert np.all(pad == 8), "padding nibbles must be 8 (dequantize to 0)"


def test_marlin_known_answers(orc):
    n, k = 64, 64
    # all-zero signed weights -> every word 0x88888888
    wm = orc.repack_marlin(orc.pack_ct(np.zeros((n, k), dtype=np.int8)))
    assert np.all(wm.view(np.uint32) == 0x88888888)
    # a single 1 at (n=13, k=42): tile 1 (k 32..63), offset 10 = 8 + 2*tg + 0 with
    # tg = 1 -> nibble p = 1 (p%4 = 1, p/4 = 0); column 13 -> ns = 1, lane = 5*4 + 1
    vals = np.zeros((n, k), dtype=np.int8)
    vals[13, 42] = 1
    wm = orc.repack_marlin(orc.pack_ct(vals)).view(np.uint32)
    word = (1 * 8 + 1) * 32 + (5 * 4 + 1)
    assert wm[word] == (0x88888888 & ~(0xF << 4)) | (9 << 4)
    assert np.count_nonzero(wm != 0x88888888) == 1


def test_marlin_sources_agree(orc):
    u = orc.uint4(0, 9, (96, 192))
    a = orc.marlin_from_u(u)
    b = orc.repack_marlin(orc.pack_ct((u.astype(np.int16) - 8).astype(np.int8)))
    c = orc.repack_gptq_marlin(orc.pack_gptq(u))
    assert np.array_equal(a, b) and np.array_equal(a, c)
    assert np.array_equal(orc.marlin_to_u(a, 96, 192), u)


# ---- act-order -----------------------------------------------------------------------


def test_gidx_perm_is_stable_argsort(orc):
    k, g = 1024, 128
    p = orc.perm(7, 5, k)
    g_idx = np.empty(k, dtype=np.int32)
    g_idx[p] = np.arange(k, dtype=np.int32) // g
    perm = orc.gidx_perm(g_idx, g)
    assert np.array_equal(perm, np.argsort(g_idx, kind="stable").astype(np.int32))
    # identity grouping -> identity permutation
    assert np.array_equal(orc.gidx_perm(np.arange(k, dtype=np.int32) // g, g), np.arange(k))


def test_gidx_perm_rejects_bad_groupings(orc):
    g_idx = np.arange(256, dtype=np.int32) // 128
    bad = g_idx.copy()
    bad[0] = 1  # group 0 has 127 rows, group 1 has 129
    with pytest.raises(ValueError):
        orc.gidx_perm(bad, 128)
    bad = g_idx.copy()
    bad[5] = 2  # out of range
    with pytest.raises(ValueError):
        orc.gidx_perm(bad, 128)


def test_act_order_repack_gathers_rows(orc):
    n, k, g = 64, 256, 64
    u = orc.uint4(3, 2, (n, k))
    p = orc.perm(3, 5, k)
    g_idx = np.empty(k, dtype=np.int32)
    g_idx[p] = np.arange(k, dtype=np.int32) // g
    perm = orc.gidx_perm(g_idx, g)
    wm = orc.repack_gptq_marlin(orc.pack_gptq(u), perm)
    assert np.array_equal(orc.marlin_to_u(wm, n, k), u[:, perm])


# ---- dequant + GEMM ------------------------------------------------------------------


def test_dequant_known_answers(orc):
    vals = np.zeros((2, 32), dtype=np.int8)
    vals[0, 3] = -8
    vals[1, 31] = 7
    scale = np.array([[0.5, 2.0], [0.25, 3.0]], dtype=np.float32)  # G = 16
    w = orc.dequant_ct(orc.pack_ct(vals), scale, 16)
    assert w[0, 3] == -4.0 and w[1, 31] == 21.0
    assert np.count_nonzero(w) == 2
    # GPTQ: (u - z) * s with the group from g_idx
    u = np.full((8, 16), 8, dtype=np.uint8)
    u[5, 9] = 3
    z = np.full((2, 8), 8, dtype=np.uint8)
    z[1, 5] = 1
    s = np.ones((2, 8), dtype=np.float32)
    s[1, 5] = 0.5
    g_idx = (np.arange(16) // 8).astype(np.int32)
    w = orc.dequant_gptq(orc.pack_gptq(u), s, orc.pack_gptq_zeros(z), g_idx, 8)
    assert w[5, 9] == (3 - 1) * 0.5
    assert w[5, 8] == (8 - 1) * 0.5 and w[5, 7] == 0.0


def test_gemm_matches_float64(orc):
    rng = np.random.default_rng(5)
    for m, n, k in [(1, 64, 128), (5, 33, 136), (17, 96, 512), (64, 128, 1024)]:
        x = rng.standard_normal((m, k)).astype(np.float32)
        w = rng.standard_normal((n, k)).astype(np.float32)
        y = orc.gemm_f32(x, w)
        ref = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.abs(y - ref).max() <= 1e-5 * np.sqrt(k) * np.abs(ref).max() + 1e-5


def test_gemm_blas_matches_c_gemm(orc):
    """The BLAS GEMM the CPU baseline times computes what the C GEMM does."""
    rng = np.random.default_rng(7)
    for m, n, k in [(1, 64, 128), (16, 200, 1024), (300, 520, 4096)]:
        x = rng.standard_normal((m, k)).astype(np.float32)
        w = rng.standard_normal((n, k)).astype(np.float32)
        ref = x.astype(np.float64) @ w.astype(np.float64).T
        yb, yc = orc.gemm_f32_blas(x, w), orc.gemm_f32(x, w)
        assert yb.shape == (m, n) and yb.dtype == np.float32
        tol = 1e-5 * np.sqrt(k) * np.abs(ref).max() + 1e-5
        assert np.abs(yb - ref).max() <= tol and np.abs(yb - yc).max() <= 2 * tol


def test_gemm_split_semantics(orc):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 128)).astype(np.float32)  # 2 chunks of 64
    w = rng.standard_normal((32, 128)).astype(np.float32)
    y = orc.gemm_f32(x, w)
    for splits in (1, 2, 3, 4, 8):  # 3, 4, 8 exceed the chunk count: empty splits add 0
        assert np.allclose(orc.gemm_f32_split(x, w, splits), y, rtol=1e-5, atol=1e-5)
    # split 0 alone covers chunk 0: check against the first half of K
    y0 = orc.gemm_f32(np.ascontiguousarray(x[:, :64]), np.ascontiguousarray(w[:, :64]))
    y1 = orc.gemm_f32(np.ascontiguousarray(x[:, 64:]), np.ascontiguousarray(w[:, 64:]))
    assert np.allclose(orc.gemm_f32_split(x, w, 2), y0 + y1, rtol=1e-6, atol=1e-6)


def test_problem_reference_paths_agree(orc):
    p = orc.make_problem(3, 64, 256, 64, seed=11)
    y = p.reference()
    y_ct = orc.w4a16_ct_forward(p.xf, p.ct_packed(), p.scale_nk, 64)
    assert np.array_equal(y, y_ct)
    ref = p.xf.astype(np.float64) @ p.dequant().astype(np.float64).T
    assert np.abs(y - ref).max() < 1e-4
    pa = orc.make_problem(2, 64, 256, 64, seed=11, symmetric=False, act_order=True)
    w = pa.dequant()
    u = pa.u.astype(np.float64)
    g = pa.g_idx
    w_ref = (u - pa.z[g, :].T) * pa.scale_kn[g, :].T
    assert np.allclose(w, w_ref, rtol=0, atol=0)


# ---- committed golden fixtures ---------------------------------------------------------


def test_golden_fixtures(orc):
    path = os.path.join(GOLDEN, "w4a16_golden.npz")
    f = np.load(path, allow_pickle=False)
    # MARLIN repack of the reference round-trip shape (N=128, K=256, G=64)
    assert np.array_equal(orc.repack_marlin(f["rt_packed"]), f["rt_marlin"])
    assert np.array_equal(orc.scale_transpose(f["rt_scale"]), f["rt_scale_marlin"])
    # odd shape with padding
    assert np.array_equal(orc.repack_marlin(f["odd_packed"]), f["odd_marlin"])
    # GEMM on a small problem
    y = orc.w4a16_ct_forward(f["g_x"], f["g_packed"], f["g_scale"], int(f["g_group"]))
    assert np.allclose(y, f["g_y"], rtol=1e-6, atol=1e-5)
    # act-order asymmetric repack + dequant
    perm = orc.gidx_perm(f["ao_gidx"], int(f["ao_group"]))
    assert np.array_equal(perm, f["ao_perm"])
    assert np.array_equal(orc.repack_gptq_marlin(f["ao_qweight"], perm), f["ao_marlin"])
    w = orc.dequant_gptq(f["ao_qweight"], f["ao_scales"], f["ao_qzeros"], f["ao_gidx"], int(f["ao_group"]))
    assert np.array_equal(w, f["ao_w"])

"""ctypes bindings for the CPU oracle (oracle/liborc.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker.  The product library (pulsar_amd) never
imports it.  Every function restates a reference algorithm; the citations are
in oracle/w4a16_oracle.h.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liborc.so")
_lib = None

MARLIN_BN = 64
MARLIN_BK = 64


def build() -> str:
    """Compile liborc.so with the committed Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_F = ctypes.c_float


def _declare(L: ctypes.CDLL) -> None:
    sig = {
        "orc_f32_to_f16_n": (None, [_P, _P, _I64]),
        "orc_f16_to_f32_n": (None, [_P, _P, _I64]),
        "orc_f32_to_bf16_n": (None, [_P, _P, _I64]),
        "orc_bf16_to_f32_n": (None, [_P, _P, _I64]),
        "orc_fill_normal": (None, [_U64, _U64, _F, _F, _P, _I64]),
        "orc_fill_abs_normal": (None, [_U64, _U64, _F, _F, _P, _I64]),
        "orc_fill_uint4": (None, [_U64, _U64, _P, _I64]),
        "orc_fill_perm": (None, [_U64, _U64, _P, _I64]),
        "orc_pack_ct": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_unpack_ct": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_pack_gptq": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_unpack_gptq": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_pack_gptq_zeros": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_unpack_gptq_zeros": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_ct_to_gptq": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_marlin_words": (_I64, [_I64, _I64]),
        "orc_repack_marlin": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_marlin_from_u": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_marlin_to_u": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_scale_transpose": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_gidx_perm": (ctypes.c_int, [_P, _I64, _I64, _P]),
        "orc_repack_gptq_marlin": (ctypes.c_int, [_P, _P, _I64, _I64, _P]),
        "orc_dequant_ct": (ctypes.c_int, [_P, _P, _I64, _I64, _I64, _P]),
        "orc_dequant_gptq": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
        "orc_gemm_f32": (None, [_P, _P, _I64, _I64, _I64, _P]),
        "orc_gemm_f32_split": (None, [_P, _P, _I64, _I64, _I64, ctypes.c_int, _P]),
        "orc_w4a16_ct_forward": (None, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
        "orc_num_threads": (ctypes.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} failed with status {rc}")


# ---- conversions ---------------------------------------------------------


def f32_to_f16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_n(_p(a), _p(out), a.size)
    return out


def f16_bits_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_f16_to_f32_n(_p(a), _p(out), a.size)
    return out


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(_p(a), _p(out), a.size)
    return out


def bf16_bits_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_n(_p(a), _p(out), a.size)
    return out


# ---- seeded data -----------------------------------------------------------


def normal(seed: int, stream: int, shape, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_fill_normal(seed, stream, mean, std, _p(out), out.size)
    return out


def abs_normal(seed: int, stream: int, shape, std=0.02, offset=1e-3) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_fill_abs_normal(seed, stream, std, offset, _p(out), out.size)
    return out


def uint4(seed: int, stream: int, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint8)
    lib().orc_fill_uint4(seed, stream, _p(out), out.size)
    return out


def perm(seed: int, stream: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().orc_fill_perm(seed, stream, _p(out), n)
    return out


# ---- packing ---------------------------------------------------------------


def pack_ct(vals: np.ndarray) -> np.ndarray:
    vals = np.ascontiguousarray(vals, dtype=np.int8)
    n, k = vals.shape
    out = np.empty((n, k // 8), dtype=np.int32)
    _check(lib().orc_pack_ct(_p(vals), n, k, _p(out)), "pack_ct")
    return out


def unpack_ct(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    n, w = packed.shape
    out = np.empty((n, w * 8), dtype=np.int8)
    _check(lib().orc_unpack_ct(_p(packed), n, w * 8, _p(out)), "unpack_ct")
    return out


def pack_gptq(u: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(u, dtype=np.uint8)
    n, k = u.shape
    out = np.empty((k // 8, n), dtype=np.int32)
    _check(lib().orc_pack_gptq(_p(u), n, k, _p(out)), "pack_gptq")
    return out


def unpack_gptq(qweight: np.ndarray) -> np.ndarray:
    qweight = np.ascontiguousarray(qweight, dtype=np.int32)
    k8, n = qweight.shape
    out = np.empty((n, k8 * 8), dtype=np.uint8)
    _check(lib().orc_unpack_gptq(_p(qweight), n, k8 * 8, _p(out)), "unpack_gptq")
    return out


def pack_gptq_zeros(z: np.ndarray) -> np.ndarray:
    z = np.ascontiguousarray(z, dtype=np.uint8)
    kg, n = z.shape
    out = np.empty((kg, n // 8), dtype=np.int32)
    _check(lib().orc_pack_gptq_zeros(_p(z), kg, n, _p(out)), "pack_gptq_zeros")
    return out


def unpack_gptq_zeros(qzeros: np.ndarray) -> np.ndarray:
    qzeros = np.ascontiguousarray(qzeros, dtype=np.int32)
    kg, n8 = qzeros.shape
    out = np.empty((kg, n8 * 8), dtype=np.uint8)
    _check(lib().orc_unpack_gptq_zeros(_p(qzeros), kg, n8 * 8, _p(out)), "unpack_gptq_zeros")
    return out


def ct_to_gptq(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    n, w = packed.shape
    out = np.empty((w, n), dtype=np.int32)
    _check(lib().orc_ct_to_gptq(_p(packed), n, w * 8, _p(out)), "ct_to_gptq")
    return out


def marlin_words(n: int, k: int) -> int:
    return int(lib().orc_marlin_words(n, k))


def repack_marlin(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    n, w = packed.shape
    out = np.empty(marlin_words(n, w * 8), dtype=np.int32)
    _check(lib().orc_repack_marlin(_p(packed), n, w * 8, _p(out)), "repack_marlin")
    return out


def marlin_from_u(u: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(u, dtype=np.uint8)
    n, k = u.shape
    out = np.empty(marlin_words(n, k), dtype=np.int32)
    _check(lib().orc_marlin_from_u(_p(u), n, k, _p(out)), "marlin_from_u")
    return out


def marlin_to_u(wm: np.ndarray, n: int, k: int) -> np.ndarray:
    wm = np.ascontiguousarray(wm, dtype=np.int32)
    assert wm.size == marlin_words(n, k)
    out = np.zeros((n, k), dtype=np.uint8)
    _check(lib().orc_marlin_to_u(_p(wm), n, k, _p(out)), "marlin_to_u")
    return out


def scale_transpose(ws: np.ndarray) -> np.ndarray:
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    n, kg = ws.shape
    out = np.empty((kg, n), dtype=np.float32)
    _check(lib().orc_scale_transpose(_p(ws), n, kg, _p(out)), "scale_transpose")
    return out


def gidx_perm(g_idx: np.ndarray, group_size: int) -> np.ndarray:
    g_idx = np.ascontiguousarray(g_idx, dtype=np.int32)
    out = np.empty(g_idx.size, dtype=np.int32)
    _check(lib().orc_gidx_perm(_p(g_idx), g_idx.size, group_size, _p(out)), "gidx_perm")
    return out


def repack_gptq_marlin(qweight: np.ndarray, perm_: np.ndarray | None = None) -> np.ndarray:
    qweight = np.ascontiguousarray(qweight, dtype=np.int32)
    k8, n = qweight.shape
    if perm_ is not None:
        perm_ = np.ascontiguousarray(perm_, dtype=np.int32)
    out = np.empty(marlin_words(n, k8 * 8), dtype=np.int32)
    _check(lib().orc_repack_gptq_marlin(_p(qweight), _p(perm_), n, k8 * 8, _p(out)), "repack_gptq_marlin")
    return out


# ---- dequant / GEMM ------------------------------------------------------------


def dequant_ct(packed: np.ndarray, scale: np.ndarray, group_size: int, out: np.ndarray | None = None) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    n, w = packed.shape
    if out is None:
        out = np.empty((n, w * 8), dtype=np.float32)
    assert out.shape == (n, w * 8) and out.dtype == np.float32 and out.flags.c_contiguous
    _check(lib().orc_dequant_ct(_p(packed), _p(scale), n, w * 8, group_size, _p(out)), "dequant_ct")
    return out


def dequant_gptq(qweight, scales, qzeros, g_idx, group_size: int) -> np.ndarray:
    qweight = np.ascontiguousarray(qweight, dtype=np.int32)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    if qzeros is not None:
        qzeros = np.ascontiguousarray(qzeros, dtype=np.int32)
    if g_idx is not None:
        g_idx = np.ascontiguousarray(g_idx, dtype=np.int32)
    k8, n = qweight.shape
    out = np.empty((n, k8 * 8), dtype=np.float32)
    _check(
        lib().orc_dequant_gptq(_p(qweight), _p(scales), _p(qzeros), _p(g_idx), n, k8 * 8, group_size, _p(out)),
        "dequant_gptq",
    )
    return out


def gemm_f32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """y[M,N] = x[M,K] @ w[N,K]^T with fp32 accumulate."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n, k2 = w.shape
    assert k == k2
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_gemm_f32(_p(x), _p(w), m, n, k, _p(out))
    return out


def gemm_f32_blas(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """The same y[M,N] = x[M,K] @ w[N,K]^T in fp32 through numpy's BLAS sgemm:
    the reference oracle's `x.float() @ w_deq.t()` (pulsar/tests/
    test_w4a16_gemm.py:56-62) as a CPU library runs it.  Used for the timed CPU
    baseline, where the C loop nest above would understate the CPU; pinned
    against gemm_f32 and a float64 matmul."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    assert x.shape[1] == w.shape[1]
    return np.matmul(x, w.T)


def blas_threads() -> int | None:
    """Threads of the BLAS behind gemm_f32_blas (None when it cannot tell)."""
    try:
        from threadpoolctl import threadpool_info

        n = [i.get("num_threads") for i in threadpool_info() if i.get("user_api") == "blas"]
        return int(max(n)) if n else None
    except Exception:  # noqa: BLE001 -- informational only
        return None


def gemm_f32_split(x: np.ndarray, w: np.ndarray, splits: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_gemm_f32_split(_p(x), _p(w), m, n, k, splits, _p(out))
    return out


def w4a16_ct_forward(x: np.ndarray, packed: np.ndarray, scale: np.ndarray, group_size: int,
                     wbuf: np.ndarray | None = None) -> np.ndarray:
    """Reference CPU path: dequantize [N,K] to fp32, then fp32 GEMM."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    m, k = x.shape
    n = packed.shape[0]
    if wbuf is None:
        wbuf = np.empty((n, k), dtype=np.float32)
    out = np.empty((m, n), dtype=np.float32)
    lib().orc_w4a16_ct_forward(_p(x), _p(packed), _p(scale), m, n, k, group_size, _p(wbuf), _p(out))
    return out


def num_threads() -> int:
    return int(lib().orc_num_threads())


# ---- BASELINE-distribution problems ---------------------------------------------


@dataclass
class Problem:
    """One seeded W4A16 problem in every format the path consumes.

    x16 is the fp16 (or bf16) bit pattern of the activations; xf is the same
    values as fp32 (what the oracle multiplies).  u is the unsigned nibble
    matrix [N,K]; z the zero points [K/G,N] (8 everywhere when symmetric).
    Scales are rounded to fp16 first, so the oracle and the kernels see the
    same values.
    """

    m: int
    n: int
    k: int
    group_size: int
    x16: np.ndarray
    xf: np.ndarray
    u: np.ndarray
    z: np.ndarray
    scale_kn: np.ndarray  # fp32 [K/G, N], values exactly representable in fp16
    g_idx: np.ndarray | None
    symmetric: bool
    bf16: bool = False

    @property
    def scale_nk(self) -> np.ndarray:
        return np.ascontiguousarray(self.scale_kn.T)

    def ct_packed(self) -> np.ndarray:
        assert self.symmetric and self.g_idx is None
        return pack_ct((self.u.astype(np.int16) - 8).astype(np.int8))

    def qweight(self) -> np.ndarray:
        return pack_gptq(self.u)

    def qzeros(self) -> np.ndarray:
        return pack_gptq_zeros(self.z)

    def dequant(self) -> np.ndarray:
        return dequant_gptq(self.qweight(), self.scale_kn, None if self.symmetric else self.qzeros(),
                            self.g_idx, self.group_size)

    def reference(self) -> np.ndarray:
        return gemm_f32(self.xf, self.dequant())


def make_problem(m: int, n: int, k: int, group_size: int = 128, seed: int = 0, symmetric: bool = True,
                 act_order: bool = False, bf16: bool = False) -> Problem:
    """BASELINE distributions: x ~ N(0,1); u ~ U{0..15}; scales |N(0,0.02)|+1e-3
    rounded to fp16; asymmetric zeros ~ U{0..15}; act-order g_idx[p[i]] = i // G
    for a seeded permutation p."""
    kg = k // group_size
    xf = normal(seed, 1, (m, k))
    if bf16:
        x16 = f32_to_bf16_bits(xf)
        xf = bf16_bits_to_f32(x16)
    else:
        x16 = f32_to_f16_bits(xf)
        xf = f16_bits_to_f32(x16)
    u = uint4(seed, 2, (n, k))
    s = f16_bits_to_f32(f32_to_f16_bits(abs_normal(seed, 3, (kg, n))))
    if symmetric:
        z = np.full((kg, n), 8, dtype=np.uint8)
    else:
        z = uint4(seed, 4, (kg, n))
    g_idx = None
    if act_order:
        p = perm(seed, 5, k)
        g_idx = np.empty(k, dtype=np.int32)
        g_idx[p] = np.arange(k, dtype=np.int32) // group_size
    return Problem(m, n, k, group_size, x16, xf, u, z, s, g_idx, symmetric, bf16)

"""Shared test data + tolerance metrics for the GPU parity tests.

Tolerances (all computed against the fp32 CPU oracle, oracle/):
  * rel_max  = max|y - y_ref| / max|y_ref|  <= 5e-3 (fp16) / 2e-2 (bf16):
    the reference's own bar (pulsar/tests/test_w4a16_gemm.py:35-38).
  * rel_l2   = ||y - y_ref|| / ||y_ref||     <= 1e-3 (fp16): the north-star bar.
  * max_abs_excess = max(|y - y_ref| - ulp16(y_ref) / 2) <= 1e-2 (fp16): the
    north-star max-abs bound once the unavoidable rounding of the fp16 OUTPUT is
    taken out (half an fp16 ulp is 0.0156 for |y| >= 32, which alone exceeds
    1e-2 at the BASELINE magnitudes).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from oracle import oracle as O

TOL_REL_MAX = {torch.float16: 5e-3, torch.bfloat16: 2e-2}
TOL_REL_L2 = {torch.float16: 1e-3, torch.bfloat16: 8e-3}
TOL_ABS_EXCESS = {torch.float16: 1e-2, torch.bfloat16: None}


@dataclass
class Case:
    m: int
    n: int
    k: int
    g: int
    dtype: torch.dtype
    x: torch.Tensor            # [M, K] device, dtype
    vals: np.ndarray           # signed int4 [N, K] (symmetric) or None
    u: np.ndarray              # unsigned nibbles [N, K]
    z: np.ndarray              # zero points [K/G, N]
    scale_nk: np.ndarray       # fp32 [N, K/G]
    g_idx: np.ndarray | None
    y_ref: np.ndarray          # fp32 oracle [M, N]

    def ct_packed(self) -> torch.Tensor:
        return torch.from_numpy(O.pack_ct(self.vals)).cuda()

    def qweight(self) -> torch.Tensor:
        return torch.from_numpy(O.pack_gptq(self.u)).cuda()

    def qzeros(self) -> torch.Tensor:
        return torch.from_numpy(O.pack_gptq_zeros(self.z)).cuda()

    def scale(self, dtype=None, kn=False) -> torch.Tensor:
        s = np.ascontiguousarray(self.scale_nk.T) if kn else self.scale_nk
        t = torch.from_numpy(np.ascontiguousarray(s)).cuda()
        return t.to(dtype) if dtype is not None else t


def to_device_x(x16: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    t = torch.from_numpy(x16.view(np.int16).copy())
    return t.view(dtype).cuda()


def reference_case(m, n, k, g, dtype, seed=0) -> Case:
    """The reference test's distributions (test_w4a16_gemm.py:65-69): vals in
    [-8, 8), scale U(0.01, 0.05), x ~ 0.1 N(0,1); the oracle sees the unrounded
    fp32 x and scale, as in the reference (input rounding is inside the tolerance)."""
    rng = np.random.default_rng(seed)
    vals = rng.integers(-8, 8, size=(n, k)).astype(np.int8)
    scale = (rng.random((n, k // g)) * 0.04 + 0.01).astype(np.float32)
    xf = (rng.standard_normal((m, k)) * 0.1).astype(np.float32)
    x16 = O.f32_to_bf16_bits(xf) if dtype == torch.bfloat16 else O.f32_to_f16_bits(xf)
    y_ref = O.gemm_f32(xf, O.dequant_ct(O.pack_ct(vals), scale, g))
    u = (vals.astype(np.int16) + 8).astype(np.uint8)
    return Case(m, n, k, g, dtype, to_device_x(x16, dtype), vals, u, np.full((k // g, n), 8, np.uint8), scale,
                None, y_ref)


def baseline_case(m, n, k, g=128, dtype=torch.float16, seed=0, symmetric=True, act_order=False,
                  rows: np.ndarray | None = None) -> Case:
    """BASELINE.json distributions (x ~ N(0,1); u ~ U{0..15}; scales |N(0,.02)|+1e-3
    rounded to fp16; zeros ~ U{0..15} when asymmetric; act-order g_idx).  Inputs
    are rounded first, so the oracle sees exactly what the kernel sees.  `rows`
    restricts the oracle to a subset of output rows (rows of y are independent)."""
    p = O.make_problem(m, n, k, g, seed=seed, symmetric=symmetric, act_order=act_order,
                       bf16=dtype == torch.bfloat16)
    w = p.dequant()
    xf = p.xf if rows is None else np.ascontiguousarray(p.xf[rows])
    y_ref = O.gemm_f32(xf, w)
    vals = (p.u.astype(np.int16) - 8).astype(np.int8) if symmetric else None
    return Case(m, n, k, g, dtype, to_device_x(p.x16, dtype), vals, p.u, p.z, p.scale_nk, p.g_idx, y_ref)


def metrics(y: torch.Tensor, y_ref: np.ndarray) -> dict:
    yf = y.float().cpu().numpy().astype(np.float64)
    ref = y_ref.astype(np.float64)
    err = np.abs(yf - ref)
    denom = np.abs(ref).max()
    ref16 = np.abs(ref).astype(np.float16).astype(np.float64)
    half_ulp = np.spacing(np.maximum(ref16, 6.1e-5).astype(np.float16)).astype(np.float64) / 2
    return {
        "max_abs": float(err.max()) if err.size else 0.0,
        "rel_max": float(err.max() / denom) if denom > 0 else float(err.max() if err.size else 0.0),
        "rel_l2": float(np.linalg.norm(yf - ref) / max(np.linalg.norm(ref), 1e-30)),
        "max_abs_excess": float((err - half_ulp).max()) if err.size else 0.0,
        "finite": bool(np.isfinite(yf).all()),
    }


def check(y: torch.Tensor, y_ref: np.ndarray, dtype: torch.dtype, what: str, rel_l2: bool = True,
          abs_excess: bool = True) -> dict:
    r = metrics(y, y_ref)
    msg = f"{what}: " + " ".join(f"{k}={v:.3e}" if isinstance(v, float) else f"{k}={v}" for k, v in r.items())
    assert r["finite"], msg
    assert r["rel_max"] <= TOL_REL_MAX[dtype], msg
    if rel_l2:
        assert r["rel_l2"] <= TOL_REL_L2[dtype], msg
    if abs_excess and TOL_ABS_EXCESS[dtype] is not None:
        assert r["max_abs_excess"] <= TOL_ABS_EXCESS[dtype], msg
    return r

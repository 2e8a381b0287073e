"""Writes tests/golden/w4a16_golden.npz.

The reference stores no golden vectors for the W4A16 path (all of its test
data is generated from torch seeds), so these fixtures are written by this
build's CPU oracle after it passed the independent checks in
tests/test_oracle.py (reference MARLIN decoder, numpy rounding / matmul,
known answers).  They pin the oracle and the GPU kernels against silent
regressions; they are not an independent source of truth.

Contents (all small):
  rt_*   the reference round-trip case (N=128, K=256, G=64; test_w4a16_marlin.py:122)
  odd_*  a padded MARLIN shape (N=100, K=136)
  g_*    a small GEMM (M=3, N=64, K=256, G=64)
  ao_*   asymmetric act-order GPTQ (N=64, K=256, G=64)

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def main() -> None:
    out = {}
    # reference round trip shape, seed 2
    vals = (O.uint4(2, 1, (128, 256)).astype(np.int16) - 8).astype(np.int8)
    scale = O.abs_normal(2, 2, (128, 256 // 64))
    out["rt_packed"] = O.pack_ct(vals)
    out["rt_scale"] = scale
    out["rt_marlin"] = O.repack_marlin(out["rt_packed"])
    out["rt_scale_marlin"] = O.scale_transpose(scale)
    # padded shape
    vals = (O.uint4(3, 1, (100, 136)).astype(np.int16) - 8).astype(np.int8)
    out["odd_packed"] = O.pack_ct(vals)
    out["odd_marlin"] = O.repack_marlin(out["odd_packed"])
    # small GEMM
    p = O.make_problem(3, 64, 256, 64, seed=4)
    out["g_x"] = p.xf
    out["g_packed"] = p.ct_packed()
    out["g_scale"] = p.scale_nk
    out["g_group"] = np.int64(64)
    out["g_y"] = p.reference()
    # asymmetric act-order
    a = O.make_problem(2, 64, 256, 64, seed=5, symmetric=False, act_order=True)
    out["ao_gidx"] = a.g_idx
    out["ao_group"] = np.int64(64)
    out["ao_qweight"] = a.qweight()
    out["ao_qzeros"] = a.qzeros()
    out["ao_scales"] = a.scale_kn
    out["ao_perm"] = O.gidx_perm(a.g_idx, 64)
    out["ao_marlin"] = O.repack_gptq_marlin(out["ao_qweight"], out["ao_perm"])
    out["ao_w"] = a.dequant()
    np.savez_compressed(os.path.join(HERE, "w4a16_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "w4a16_golden.npz"))


if __name__ == "__main__":
    main()

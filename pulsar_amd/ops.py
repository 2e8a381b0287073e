"""Python wrappers and fake (meta) kernels for the W4A16 ops.

Same wrapper names, argument meaning and fake-kernel output shapes as the
reference pulsar/src/pulsar/core/ops.py:117-165,369-445, so code written
against `pulsar.core.ops` switches by importing `pulsar_amd.ops`.  The ops
themselves are registered by _pulsar_w4a16_torch.so (torch.ops.pulsar.*).
"""

from __future__ import annotations

import torch

# MARLIN tiling constants; must match the C ABI's size rule (pw4_marlin_words).
_MARLIN_BN = 64
_MARLIN_BK = 64


def _gemm_w4a16_fake(x, weight_packed, weight_scale, group_size):
    return x.new_empty((x.shape[0], weight_packed.shape[0]))


def _gemm_w4a16_split_fake(x, weight_packed, weight_scale, group_size, num_splits):
    return x.new_empty((x.shape[0], weight_packed.shape[0]))


def _repack_w4a16_fake(weight_packed, weight_scale, group_size):
    n = weight_packed.shape[0]
    k = weight_packed.shape[1] * 8
    npad = -(-n // _MARLIN_BN) * _MARLIN_BN
    kpad = -(-k // _MARLIN_BK) * _MARLIN_BK
    weight_marlin = weight_packed.new_empty((npad * kpad // 8,))
    scale_marlin = weight_scale.new_empty((k // group_size, n), dtype=torch.float32)
    return weight_marlin, scale_marlin


def _gemm_w4a16_marlin_fake(x, weight_marlin, scale_marlin, group_size):
    return x.new_empty((x.shape[0], scale_marlin.shape[1]))


def _gemm_w4a16_marlin_split_fake(x, weight_marlin, scale_marlin, group_size, num_splits):
    return x.new_empty((x.shape[0], scale_marlin.shape[1]))


def _repack_w4a16_gptq_fake(qweight, g_idx, group_size):
    k = qweight.shape[0] * 8
    n = qweight.shape[1]
    npad = -(-n // _MARLIN_BN) * _MARLIN_BN
    kpad = -(-k // _MARLIN_BK) * _MARLIN_BK
    weight_marlin = qweight.new_empty((npad * kpad // 8,))
    perm = qweight.new_empty((k if g_idx is not None else 0,))
    return weight_marlin, perm


def _gemm_w4a16_gptq_fake(x, weight_marlin, scales, qzeros, perm, group_size):
    return x.new_empty((x.shape[0], scales.shape[1]))


def _gemm_w4a16_silu_mul_fake(x, weight_marlin, scales, qzeros, perm, group_size):
    return x.new_empty((x.shape[0], scales.shape[1] // 2))


def _register_fakes() -> None:
    fakes = {
        "pulsar::gemm_w4a16": _gemm_w4a16_fake,
        "pulsar::gemm_w4a16_split": _gemm_w4a16_split_fake,
        "pulsar::repack_w4a16": _repack_w4a16_fake,
        "pulsar::gemm_w4a16_marlin": _gemm_w4a16_marlin_fake,
        "pulsar::gemm_w4a16_marlin_split": _gemm_w4a16_marlin_split_fake,
        "pulsar::repack_w4a16_gptq": _repack_w4a16_gptq_fake,
        "pulsar::gemm_w4a16_gptq": _gemm_w4a16_gptq_fake,
        "pulsar::gemm_w4a16_silu_mul": _gemm_w4a16_silu_mul_fake,
    }
    for name, func in fakes.items():
        torch.library.register_fake(name, func)


_register_fakes()


def gemm_w4a16(x: torch.Tensor, weight_packed: torch.Tensor, weight_scale: torch.Tensor,
               group_size: int) -> torch.Tensor:
    """Fused w4a16 dequant-GEMM computing y = x @ dequant(W)^T.

    y[m, n] = sum_k x[m, k] * int4(weight_packed[n, k]) * weight_scale[n, k // group_size].

    Args:
        x: [M, K] fp16 or bf16, contiguous.
        weight_packed: int32 [N, K/8]; column k in nibble k % 8 of word [n, k // 8],
            LSB-first, two's complement in [-8, 7].
        weight_scale: [N, K/group_size], any float dtype (upcast to fp32).
        group_size: quantization group along K (multiple of 16; K a multiple of it).

    Returns:
        y [M, N] in x's dtype.
    """
    return torch.ops.pulsar.gemm_w4a16(x, weight_packed, weight_scale, group_size)


def gemm_w4a16_split(x, weight_packed, weight_scale, group_size: int, num_splits: int) -> torch.Tensor:
    """gemm_w4a16 with the K-split count forced to num_splits (split + combine path)."""
    return torch.ops.pulsar.gemm_w4a16_split(x, weight_packed, weight_scale, group_size, num_splits)


def repack_w4a16(weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                 group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Repack the compressed-tensors packing into the MARLIN fragment layout.

    Returns (weight_marlin int32 [Npad*Kpad/8], scale_marlin fp32 [K/group_size, N]);
    Npad / Kpad are N / K rounded up to 64.  Bit-identical to the reference packer.
    """
    return torch.ops.pulsar.repack_w4a16(weight_packed, weight_scale, group_size)


def gemm_w4a16_marlin(x: torch.Tensor, weight_marlin: torch.Tensor, scale_marlin: torch.Tensor,
                      group_size: int) -> torch.Tensor:
    """y = x @ dequant(W)^T from (weight_marlin, scale_marlin) produced by repack_w4a16."""
    return torch.ops.pulsar.gemm_w4a16_marlin(x, weight_marlin, scale_marlin, group_size)


def gemm_w4a16_marlin_split(x, weight_marlin, scale_marlin, group_size: int, num_splits: int) -> torch.Tensor:
    """gemm_w4a16_marlin with the K-split count forced (test seam)."""
    return torch.ops.pulsar.gemm_w4a16_marlin_split(x, weight_marlin, scale_marlin, group_size, num_splits)


def repack_w4a16_gptq(qweight: torch.Tensor, g_idx: torch.Tensor | None,
                      group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """GPTQ qweight int32 [K/8, N] (+ optional act-order g_idx [K]) -> (weight_marlin, perm).

    perm is int32 [K] (empty without g_idx): repacked row j is original row perm[j].
    """
    return torch.ops.pulsar.repack_w4a16_gptq(qweight, g_idx, group_size)


def gemm_w4a16_gptq(x: torch.Tensor, weight_marlin: torch.Tensor, scales: torch.Tensor,
                    qzeros: torch.Tensor | None, perm: torch.Tensor | None, group_size: int) -> torch.Tensor:
    """y = x[:, perm] @ ((u - z) * s)^T with scales [K/G, N] (fp16/fp32) and optional GPTQ qzeros."""
    if perm is not None and perm.numel() == 0:
        perm = None
    return torch.ops.pulsar.gemm_w4a16_gptq(x, weight_marlin, scales, qzeros, perm, group_size)


def gemm_w4a16_silu_mul(x: torch.Tensor, weight_marlin: torch.Tensor, scales: torch.Tensor,
                        qzeros: torch.Tensor | None, perm: torch.Tensor | None, group_size: int) -> torch.Tensor:
    """silu(x @ Wg^T) * (x @ Wu^T), [M, N/2], from a gate|up weight interleaved by 8 columns
    (fused columns 16j..16j+7 gate 8j..8j+7, 16j+8..16j+15 up 8j..8j+7): the reference MLP's
    at::silu(gate) * up after two at::linear calls (qwen3.cpp:116-118) as one op."""
    if perm is not None and perm.numel() == 0:
        perm = None
    return torch.ops.pulsar.gemm_w4a16_silu_mul(x, weight_marlin, scales, qzeros, perm, group_size)

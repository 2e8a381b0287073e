// pulsar_w4a16_ops.hpp -- the at::Tensor operator API of the W4A16 path,
// same names, signatures and contracts as the reference pulsar-core C++ API
// (pulsar-core/inc/pulsar/ops.hpp:148-189), so C++ callers switch by linking
// pulsar_amd/_pulsar_w4a16_torch.so instead of pulsar_core.  Each function
// checks its arguments like the reference (TORCH_CHECK -> c10::Error),
// allocates its output (and any workspace) with the caching allocator on the
// input's device, and launches asynchronously on the current HIP stream
// through the C ABI in pulsar_w4a16.h.
#pragma once

#include <ATen/ATen.h>

#include <optional>
#include <tuple>

namespace pulsar {

// y = x @ dequant(W)^T from the compressed-tensors packing.
//   x [M, K] fp16/bf16 contiguous; weight_packed int32 [N, K/8]; weight_scale [N, K/G]
//   (any float dtype, upcast to fp32 like the reference).  Returns y [M, N] in x's dtype.
// Reference: ops.hpp:148-161, w4a16_gemm.cu:471-478.
at::Tensor gemm_w4a16_cuda(const at::Tensor& x, const at::Tensor& weight_packed, const at::Tensor& weight_scale,
                           int64_t group_size);

// Same result with the K-split count forced to num_splits >= 1 (split + combine path).
// Reference: ops.hpp:163-173, w4a16_gemm.cu:480-489.
at::Tensor gemm_w4a16_split_cuda(const at::Tensor& x, const at::Tensor& weight_packed,
                                 const at::Tensor& weight_scale, int64_t group_size, int64_t num_splits);

// One-time repack -> (weight_marlin int32 [Npad*Kpad/8], scale_marlin fp32 [K/G, N]).
// Reference: ops.hpp:175-182, w4a16_marlin.cu:354-406.
std::tuple<at::Tensor, at::Tensor> repack_w4a16_cuda(const at::Tensor& weight_packed,
                                                     const at::Tensor& weight_scale, int64_t group_size);

// y = x @ dequant(W)^T from the repacked layout.
// Reference: ops.hpp:184-189, w4a16_marlin.cu:408-551.
at::Tensor gemm_w4a16_marlin_cuda(const at::Tensor& x, const at::Tensor& weight_marlin,
                                  const at::Tensor& scale_marlin, int64_t group_size);

// ---- extensions with no counterpart in the reference -------------------------

// gemm_w4a16_marlin with a forced K-split count (test seam, like gemm_w4a16_split).
at::Tensor gemm_w4a16_marlin_split_cuda(const at::Tensor& x, const at::Tensor& weight_marlin,
                                        const at::Tensor& scale_marlin, int64_t group_size, int64_t num_splits);

// GPTQ checkpoint ingestion: qweight int32 [K/8, N] (unsigned nibbles along K),
// optional act-order g_idx [K].  Returns (weight_marlin, perm) where perm is
// int32 [K] (empty when g_idx is absent).  Raises if g_idx is not a grouping of
// exactly group_size rows per group.
std::tuple<at::Tensor, at::Tensor> repack_w4a16_gptq_cuda(const at::Tensor& qweight,
                                                          const std::optional<at::Tensor>& g_idx,
                                                          int64_t group_size);

// y = x[:, perm] @ ((u - z) * s)^T with scales [K/G, N] (fp16 or fp32), optional
// GPTQ qzeros int32 [K/G, N/8] (absent: symmetric zero 8) and optional perm.
at::Tensor gemm_w4a16_gptq_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scales,
                                const std::optional<at::Tensor>& qzeros, const std::optional<at::Tensor>& perm,
                                int64_t group_size);

// The MLP gate in one op: y [M, N/2] = silu(x @ Wg^T) * (x @ Wu^T) from a
// gate|up weight interleaved by 8 columns (fused columns 16j..16j+7 gate
// 8j..8j+7, 16j+8..16j+15 up 8j..8j+7; N % 16 == 0); scales, qzeros and perm as
// for gemm_w4a16_gptq_cuda in the same column order.  Replaces two at::linear
// calls and at::silu(gate) * up (pulsar-core/src/model/qwen3.cpp:116-118).
at::Tensor gemm_w4a16_silu_mul_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scales,
                                    const std::optional<at::Tensor>& qzeros, const std::optional<at::Tensor>& perm,
                                    int64_t group_size);

}  // namespace pulsar

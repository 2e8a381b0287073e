// pulsar_w4a16_model.hpp -- the W4A16 linears at the model's at::linear sites,
// in C++.  The reference decode step calls at::linear(h, W) on dense weights
// for q, k, v, o, gate, up and down (pulsar-core/src/model/qwen3.cpp:82-84,
// 114, 117-119), with W taken from the weights map by name (qwen3.cpp:48-70).
// A W4A16Linear holds one such weight in the MARLIN layout and computes
// y = x @ dequant(W)^T (+ bias) through the operator API of
// pulsar_w4a16_ops.hpp; Qwen3LayerW4A16 holds one layer's linears fused the way
// the kernels want them (q|k|v as one GEMM, gate|up as one SiLU-gated GEMM) and
// runs the linear part of Qwen3Model::block around the caller's norm weights
// and attention.  The same layer serves Qwen2Model::block
// (pulsar-core/src/model/qwen2.cpp:72-93), whose q, k and v projections carry
// a bias (at::linear(h, W, b), qwen2.cpp:78-80): the biases ride in the linears.
#pragma once

#include <ATen/ATen.h>
#include <ATen/core/Dict.h>

#include <functional>
#include <optional>
#include <string>
#include <tuple>
#include <vector>

namespace pulsar {

class W4A16Linear {
   public:
    W4A16Linear() = default;
    // weight_marlin int32 [roundup(N,64) * roundup(K,64) / 8]; scales fp16/fp32 [K/G, N];
    // qzeros int32 [K/G, N/8] (GPTQ zero points, absent: symmetric); perm int32 [K]
    // (act-order, absent: natural order).  silu_gate: the weight is gate|up interleaved
    // by 8 columns and forward() returns silu(gate) * up, [.., N/2].
    // bias: [N] in any float dtype, added to the GEMM output: one rounding to x's
    // dtype of the fp32 sum of the rounded GEMM output and the bias as stored.
    W4A16Linear(at::Tensor weight_marlin, at::Tensor scales, int64_t group_size, int64_t in_features,
                int64_t out_features, std::optional<at::Tensor> qzeros = std::nullopt,
                std::optional<at::Tensor> perm = std::nullopt, bool silu_gate = false,
                std::optional<at::Tensor> bias = std::nullopt);

    // The reference's quantized weight: weight_packed int32 [N, K/8] (two's complement
    // nibbles along K, ops.hpp:148-152) and weight_scale [N, K/G], repacked once with
    // repack_w4a16_cuda (fp32 scale_marlin [K/G, N]).
    static W4A16Linear from_packed(const at::Tensor& weight_packed, const at::Tensor& weight_scale,
                                   int64_t group_size);
    // A GPTQ checkpoint's tensors: qweight int32 [K/8, N], scales [K/G, N], qzeros int32
    // [K/G, N/8] holding z itself, g_idx [K] for act-order (k // G everywhere, the natural
    // order, needs no permutation and is dropped).
    static W4A16Linear from_gptq(const at::Tensor& qweight, const at::Tensor& scales, int64_t group_size,
                                 const std::optional<at::Tensor>& qzeros, const std::optional<at::Tensor>& g_idx);
    // N-concatenation of linears that share their input (q|k|v): the MARLIN words are
    // column-block major, so members whose N is a multiple of 64 concatenate as buffers.
    static W4A16Linear concat(const std::vector<W4A16Linear>& parts);
    // The same linear with a bias [N] (or none).
    W4A16Linear with_bias(std::optional<at::Tensor> bias) const;
    // Whether concat (or silu_gate, for two members) accepts these members: same K,
    // group size, scale dtype, zero-point presence, bias presence and act-order
    // permutation, and N % 64 == 0 for every member but the last (every member for a
    // SiLU gate, which takes no bias).
    static bool can_fuse(const std::vector<W4A16Linear>& parts, bool silu_gate = false);
    // The MLP gate silu(x Wg^T) * (x Wu^T) as one GEMM: gate and up interleaved by 8
    // columns, regrouped from the two repacked weights (no requantisation).
    static W4A16Linear silu_gate(const W4A16Linear& gate, const W4A16Linear& up);

    // x [..., K] fp16 or bf16 -> [..., N] (or [..., N/2] for a SiLU gate), x's dtype.
    at::Tensor forward(const at::Tensor& x) const;

    int64_t in_features() const { return in_; }
    int64_t out_features() const { return silu_ ? out_ / 2 : out_; }
    int64_t group_size() const { return group_size_; }
    bool is_silu_gate() const { return silu_; }
    const at::Tensor& weight_marlin() const { return weight_marlin_; }
    const at::Tensor& scales() const { return scales_; }
    const std::optional<at::Tensor>& qzeros() const { return qzeros_; }
    const std::optional<at::Tensor>& perm() const { return perm_; }
    const std::optional<at::Tensor>& bias() const { return bias_; }

   private:
    at::Tensor weight_marlin_, scales_;
    std::optional<at::Tensor> qzeros_, perm_, bias_;
    int64_t group_size_ = 0, in_ = 0, out_ = 0;
    bool silu_ = false;
};

// One Qwen3 / Llama layer's W4A16 linears, fused for the kernels where the
// members allow it: q|k|v as one GEMM and gate|up as one SiLU-gated GEMM.  An
// act-order checkpoint usually permutes q, k and v (and gate and up)
// differently; those stay separate linears.
struct Qwen3LayerW4A16 {
    std::vector<W4A16Linear> qkv;      // {q|k|v}, or {q, k, v}
    W4A16Linear o;                     // o_proj
    std::vector<W4A16Linear> gate_up;  // {SiLU-gated gate|up}, or {gate, up}
    W4A16Linear down;                  // down_proj
    int64_t q_dim = 0, kv_dim = 0;

    // The layer's quantized linears from a checkpoint's weights map, under the
    // engine's names (qwen3.cpp:55-69): <prefix>self_attn.{q,k,v,o}_proj.* and
    // <prefix>mlp.{gate,up,down}_proj.*, each either the reference's packed format
    // (weight_packed, weight_scale) or GPTQ (qweight, scales, qzeros, g_idx), plus
    // an optional <...>_proj.bias (Qwen2's q, k and v, qwen2.cpp:57-62).
    static Qwen3LayerW4A16 from_weights(const c10::Dict<std::string, at::Tensor>& weights, const std::string& prefix,
                                        int64_t group_size);

    // q, k, v = linear(h, q_proj / k_proj / v_proj)  (qwen3.cpp:82-84): one GEMM split
    // three ways when fused.
    std::tuple<at::Tensor, at::Tensor, at::Tensor> qkv_proj(const at::Tensor& h) const;
    // x + linear(o, o_proj)  (qwen3.cpp:114)
    at::Tensor o_proj_residual(const at::Tensor& x, const at::Tensor& attn) const;
    // x + linear(silu(linear(h2, gate)) * linear(h2, up), down)  (qwen3.cpp:116-119)
    at::Tensor mlp_residual(const at::Tensor& x, const at::Tensor& h2) const;
};

// y = x / sqrt(mean(x^2) + eps) * weight in fp32, cast to x's dtype: the arithmetic of
// the reference's rmsnorm_cuda (pulsar-core/src/kernels/rmsnorm.cu:10,47-49), here in
// ATen (the norm is outside the W4A16 path).
at::Tensor rmsnorm_ref(const at::Tensor& x, const at::Tensor& weight, double eps);

// The attention of Qwen3Model::block, from (q, k, v) to o [T, n_heads * head_dim].
using AttentionFn = std::function<at::Tensor(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v)>;

// Qwen3Model::block (qwen3.cpp:77-121) with W4A16 linears; RoPE, QK-norm, paged
// attention and the KV cache are the caller's, inside `attention`:
//   h = rmsnorm(x, ln1); q, k, v = qkv(h); o = attention(q, k, v)
//   x = x + o_proj(o); h2 = rmsnorm(x, ln2); x = x + down(silu(gate(h2)) * up(h2))
at::Tensor qwen3_block_w4a16(const Qwen3LayerW4A16& layer, const at::Tensor& x, const at::Tensor& ln1,
                             const at::Tensor& ln2, double eps, const AttentionFn& attention);

// Qwen2Model::block (qwen2.cpp:72-93) has the same linear structure; its q, k and v
// biases come with the layer (from_weights), and its RoPE (no QK-norm) is the
// caller's, inside `attention`.
inline at::Tensor qwen2_block_w4a16(const Qwen3LayerW4A16& layer, const at::Tensor& x, const at::Tensor& ln1,
                                    const at::Tensor& ln2, double eps, const AttentionFn& attention) {
    return qwen3_block_w4a16(layer, x, ln1, ln2, eps, attention);
}

}  // namespace pulsar

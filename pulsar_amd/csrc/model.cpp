// The W4A16 linears at the model's at::linear sites (include/pulsar_w4a16_model.hpp)
// and their registration as the torch class pulsar.Qwen3W4A16Layer.
#include "pulsar_w4a16_model.hpp"

#include <torch/custom_class.h>
#include <torch/library.h>

#include "pulsar_w4a16_ops.hpp"

namespace pulsar {

namespace {

constexpr int64_t kMarlinBN = 64, kMarlinBK = 64;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool has(const std::optional<at::Tensor>& t) { return t.has_value() && t->defined() && t->numel() > 0; }

// MARLIN words of an [n, k] weight as its 8-column groups [n/8, Kpad/64, 2, 32]: a
// 64-column block's half chunk holds 8 groups of 8 columns, 32 words each.
at::Tensor groups8(const at::Tensor& words, int64_t n, int64_t k) {
    const int64_t ncb = n / kMarlinBN, nch = ceil_div(k, kMarlinBK);
    return words.view({ncb, nch, 2, 8, 32}).permute({0, 3, 1, 2, 4}).reshape({ncb * 8, nch, 2, 32});
}

// [kg, n] and [kg, n] -> [kg, 2n] interleaved in runs of `width` columns
at::Tensor interleave(const at::Tensor& a, const at::Tensor& b, int64_t kg, int64_t width) {
    return at::stack({a.view({kg, -1, width}), b.view({kg, -1, width})}, 2).reshape({kg, -1}).contiguous();
}

at::Tensor need(const c10::Dict<std::string, at::Tensor>& w, const std::string& name) {
    TORCH_CHECK(w.contains(name), "Qwen3LayerW4A16: missing weight '", name, "'");
    return w.at(name);
}

std::optional<at::Tensor> maybe(const c10::Dict<std::string, at::Tensor>& w, const std::string& name) {
    if (!w.contains(name)) return std::nullopt;
    return w.at(name);
}

// One quantized linear under <p>: the reference's packed format or GPTQ, with
// its bias when the map holds one (Qwen2's q, k and v).
W4A16Linear load_linear(const c10::Dict<std::string, at::Tensor>& w, const std::string& p, int64_t group_size) {
    if (w.contains(p + "weight_packed")) {
        return W4A16Linear::from_packed(w.at(p + "weight_packed"), need(w, p + "weight_scale"), group_size)
            .with_bias(maybe(w, p + "bias"));
    }
    TORCH_CHECK(w.contains(p + "qweight"), "Qwen3LayerW4A16: no quantized weight under '", p,
                "' (expected weight_packed + weight_scale, or qweight + scales)");
    return W4A16Linear::from_gptq(w.at(p + "qweight"), need(w, p + "scales"), group_size, maybe(w, p + "qzeros"),
                                  maybe(w, p + "g_idx"))
        .with_bias(maybe(w, p + "bias"));
}

}  // namespace

W4A16Linear::W4A16Linear(at::Tensor weight_marlin, at::Tensor scales, int64_t group_size, int64_t in_features,
                         int64_t out_features, std::optional<at::Tensor> qzeros, std::optional<at::Tensor> perm,
                         bool silu_gate, std::optional<at::Tensor> bias)
    : weight_marlin_(std::move(weight_marlin)),
      scales_(std::move(scales)),
      qzeros_(has(qzeros) ? std::move(qzeros) : std::nullopt),
      perm_(has(perm) ? std::move(perm) : std::nullopt),
      bias_(has(bias) ? std::move(bias) : std::nullopt),
      group_size_(group_size),
      in_(in_features),
      out_(out_features),
      silu_(silu_gate) {
    const int64_t k = in_, n = out_, g = group_size_;
    TORCH_CHECK(g > 0 && k % g == 0 && k % 8 == 0, "W4A16Linear: in_features ", k,
                " must be a multiple of 8 and of group_size ", g);
    TORCH_CHECK(weight_marlin_.scalar_type() == at::kInt &&
                    weight_marlin_.numel() == ceil_div(n, kMarlinBN) * kMarlinBN * ceil_div(k, kMarlinBK) * kMarlinBK / 8,
                "W4A16Linear: weight_marlin must be int32 with roundup(N,64)*roundup(K,64)/8 words");
    TORCH_CHECK(scales_.dim() == 2 && scales_.size(0) == k / g && scales_.size(1) == n &&
                    (scales_.scalar_type() == at::kHalf || scales_.scalar_type() == at::kFloat),
                "W4A16Linear: scales must be fp16/fp32 [K/G, N]");
    if (qzeros_) {
        TORCH_CHECK(qzeros_->scalar_type() == at::kInt && qzeros_->dim() == 2 && qzeros_->size(0) == k / g &&
                        qzeros_->size(1) == n / 8,
                    "W4A16Linear: qzeros must be int32 [K/G, N/8]");
    }
    if (perm_) TORCH_CHECK(perm_->dim() == 1 && perm_->size(0) == k, "W4A16Linear: perm must be int32 [K]");
    if (silu_) TORCH_CHECK(n % 16 == 0, "W4A16Linear: a SiLU gate needs N (gate|up) % 16 == 0");
    if (bias_) {
        TORCH_CHECK(!silu_, "W4A16Linear: a SiLU gate takes no bias");
        TORCH_CHECK(bias_->dim() == 1 && bias_->size(0) == n && at::isFloatingType(bias_->scalar_type()),
                    "W4A16Linear: bias must be a floating-point [N] = [", n, "]");
        bias_ = bias_->contiguous();
    }
}

W4A16Linear W4A16Linear::with_bias(std::optional<at::Tensor> bias) const {
    return W4A16Linear(weight_marlin_, scales_, group_size_, in_, out_, qzeros_, perm_, silu_, std::move(bias));
}

W4A16Linear W4A16Linear::from_packed(const at::Tensor& weight_packed, const at::Tensor& weight_scale,
                                     int64_t group_size) {
    TORCH_CHECK(weight_packed.dim() == 2, "W4A16Linear: weight_packed must be [N, K/8]");
    const int64_t n = weight_packed.size(0), k = weight_packed.size(1) * 8;
    auto [wm, sm] = repack_w4a16_cuda(weight_packed.contiguous(), weight_scale.contiguous(), group_size);
    return W4A16Linear(wm, sm, group_size, k, n);
}

W4A16Linear W4A16Linear::from_gptq(const at::Tensor& qweight, const at::Tensor& scales, int64_t group_size,
                                   const std::optional<at::Tensor>& qzeros, const std::optional<at::Tensor>& g_idx) {
    TORCH_CHECK(qweight.dim() == 2, "W4A16Linear: qweight must be [K/8, N]");
    const int64_t k = qweight.size(0) * 8, n = qweight.size(1);
    std::optional<at::Tensor> gi;
    if (has(g_idx)) {
        auto g32 = g_idx->to(at::kInt);
        auto natural = at::arange(k, g32.options()).div(group_size, "floor");
        if (!at::equal(g32, natural)) gi = g32.contiguous();
    }
    auto [wm, perm] = repack_w4a16_gptq_cuda(qweight.contiguous(), gi, group_size);
    const auto sc = (scales.scalar_type() == at::kHalf || scales.scalar_type() == at::kFloat) ? scales
                                                                                              : scales.to(at::kFloat);
    return W4A16Linear(wm, sc.contiguous(), group_size, k, n,
                       has(qzeros) ? std::optional<at::Tensor>(qzeros->contiguous()) : std::nullopt,
                       gi ? std::optional<at::Tensor>(perm) : std::nullopt);
}

bool W4A16Linear::can_fuse(const std::vector<W4A16Linear>& parts, bool silu_gate) {
    if (parts.empty() || (silu_gate && parts.size() != 2)) return false;
    const W4A16Linear& p0 = parts[0];
    for (size_t i = 0; i < parts.size(); ++i) {
        const W4A16Linear& p = parts[i];
        if (p.silu_ || p.in_ != p0.in_ || p.group_size_ != p0.group_size_ ||
            p.scales_.scalar_type() != p0.scales_.scalar_type() || p.qzeros_.has_value() != p0.qzeros_.has_value() ||
            p.bias_.has_value() != p0.bias_.has_value() || (silu_gate && p.bias_) ||
            p.perm_.has_value() != p0.perm_.has_value() || (p.perm_ && !at::equal(*p.perm_, *p0.perm_))) {
            return false;
        }
        if ((silu_gate || i + 1 < parts.size()) && p.out_ % kMarlinBN != 0) return false;
        if (silu_gate && p.out_ != p0.out_) return false;
    }
    return true;
}

W4A16Linear W4A16Linear::concat(const std::vector<W4A16Linear>& parts) {
    TORCH_CHECK(!parts.empty(), "W4A16Linear::concat: no parts");
    if (parts.size() == 1) return parts[0];
    const W4A16Linear& p0 = parts[0];
    std::vector<at::Tensor> words, scales, zeros, biases;
    int64_t n = 0;
    for (size_t i = 0; i < parts.size(); ++i) {
        const W4A16Linear& p = parts[i];
        TORCH_CHECK(!p.silu_, "W4A16Linear::concat: a SiLU gate cannot be a member");
        TORCH_CHECK(p.in_ == p0.in_ && p.group_size_ == p0.group_size_ &&
                        p.scales_.scalar_type() == p0.scales_.scalar_type(),
                    "W4A16Linear::concat: members differ in K, group size or scale dtype");
        TORCH_CHECK(p.qzeros_.has_value() == p0.qzeros_.has_value(), "W4A16Linear::concat: members differ in zero points");
        TORCH_CHECK(p.bias_.has_value() == p0.bias_.has_value(), "W4A16Linear::concat: members differ in bias");
        TORCH_CHECK(p.perm_.has_value() == p0.perm_.has_value() && (!p.perm_ || at::equal(*p.perm_, *p0.perm_)),
                    "W4A16Linear::concat: members have different act-order permutations");
        TORCH_CHECK(i + 1 == parts.size() || p.out_ % kMarlinBN == 0,
                    "W4A16Linear::concat: every member but the last needs out_features % 64 == 0");
        words.push_back(p.weight_marlin_);
        scales.push_back(p.scales_);
        if (p.qzeros_) zeros.push_back(*p.qzeros_);
        if (p.bias_) biases.push_back(*p.bias_);
        n += p.out_;
    }
    return W4A16Linear(at::cat(words), at::cat(scales, 1), p0.group_size_, p0.in_, n,
                       zeros.empty() ? std::nullopt : std::optional<at::Tensor>(at::cat(zeros, 1)), p0.perm_,
                       /*silu_gate=*/false,
                       biases.empty() ? std::nullopt : std::optional<at::Tensor>(at::cat(biases)));
}

W4A16Linear W4A16Linear::silu_gate(const W4A16Linear& gate, const W4A16Linear& up) {
    const int64_t f = gate.out_, k = gate.in_, g = gate.group_size_;
    TORCH_CHECK(!gate.silu_ && !up.silu_, "W4A16Linear::silu_gate: members must be plain linears");
    TORCH_CHECK(up.out_ == f && up.in_ == k && up.group_size_ == g && up.scales_.scalar_type() == gate.scales_.scalar_type(),
                "W4A16Linear::silu_gate: gate and up differ in shape, group size or scale dtype");
    TORCH_CHECK(f % kMarlinBN == 0, "W4A16Linear::silu_gate: the intermediate size must be a multiple of 64");
    TORCH_CHECK(gate.qzeros_.has_value() == up.qzeros_.has_value(), "W4A16Linear::silu_gate: zero points must match");
    TORCH_CHECK(!gate.bias_ && !up.bias_, "W4A16Linear::silu_gate: gate and up take no bias");
    TORCH_CHECK(gate.perm_.has_value() == up.perm_.has_value() && (!gate.perm_ || at::equal(*gate.perm_, *up.perm_)),
                "W4A16Linear::silu_gate: gate and up have different act-order permutations");
    const int64_t nch = ceil_div(k, kMarlinBK), kg = k / g;
    auto grouped = at::stack({groups8(gate.weight_marlin_, f, k), groups8(up.weight_marlin_, f, k)}, 1);
    auto words = grouped.reshape({2 * f / kMarlinBN, 8, nch, 2, 32}).permute({0, 2, 3, 1, 4}).reshape({-1}).contiguous();
    std::optional<at::Tensor> zeros;
    if (gate.qzeros_) zeros = interleave(*gate.qzeros_, *up.qzeros_, kg, 1);
    return W4A16Linear(words, interleave(gate.scales_, up.scales_, kg, 8), g, k, 2 * f, zeros, gate.perm_, true);
}

at::Tensor W4A16Linear::forward(const at::Tensor& x) const {
    TORCH_CHECK(x.size(-1) == in_, "W4A16Linear: x has ", x.size(-1), " features, expected ", in_);
    auto lead = x.sizes().vec();
    lead.pop_back();
    auto x2 = x.reshape({-1, in_}).contiguous();
    at::Tensor y = silu_ ? gemm_w4a16_silu_mul_cuda(x2, weight_marlin_, scales_, qzeros_, perm_, group_size_)
                         : gemm_w4a16_gptq_cuda(x2, weight_marlin_, scales_, qzeros_, perm_, group_size_);
    // at::linear's bias (qwen2.cpp:78-80).  add_ sums the GEMM output, already
    // rounded to x's dtype, and the bias in fp32, and rounds the sum again: two
    // roundings where at::linear rounds x @ W^T + b once (at most one more
    // rounding of x's dtype per element)
    if (bias_) y.add_(*bias_);
    lead.push_back(out_features());
    return y.view(lead);
}

Qwen3LayerW4A16 Qwen3LayerW4A16::from_weights(const c10::Dict<std::string, at::Tensor>& weights,
                                              const std::string& prefix, int64_t group_size) {
    Qwen3LayerW4A16 l;
    const W4A16Linear q = load_linear(weights, prefix + "self_attn.q_proj.", group_size);
    const W4A16Linear k = load_linear(weights, prefix + "self_attn.k_proj.", group_size);
    const W4A16Linear v = load_linear(weights, prefix + "self_attn.v_proj.", group_size);
    TORCH_CHECK(k.out_features() == v.out_features(), "Qwen3LayerW4A16: k_proj and v_proj differ in size");
    l.q_dim = q.out_features();
    l.kv_dim = k.out_features();
    if (W4A16Linear::can_fuse({q, k, v})) {
        l.qkv = {W4A16Linear::concat({q, k, v})};
    } else {
        l.qkv = {q, k, v};
    }
    l.o = load_linear(weights, prefix + "self_attn.o_proj.", group_size);
    const W4A16Linear gate = load_linear(weights, prefix + "mlp.gate_proj.", group_size);
    const W4A16Linear up = load_linear(weights, prefix + "mlp.up_proj.", group_size);
    if (W4A16Linear::can_fuse({gate, up}, /*silu_gate=*/true)) {
        l.gate_up = {W4A16Linear::silu_gate(gate, up)};
    } else {
        l.gate_up = {gate, up};
    }
    l.down = load_linear(weights, prefix + "mlp.down_proj.", group_size);
    return l;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> Qwen3LayerW4A16::qkv_proj(const at::Tensor& h) const {
    if (qkv.size() == 3) return {qkv[0].forward(h), qkv[1].forward(h), qkv[2].forward(h)};
    const at::Tensor y = qkv.at(0).forward(h);
    auto parts = y.split_with_sizes({q_dim, kv_dim, kv_dim}, -1);
    return {parts[0].contiguous(), parts[1].contiguous(), parts[2].contiguous()};
}

at::Tensor Qwen3LayerW4A16::o_proj_residual(const at::Tensor& x, const at::Tensor& attn) const {
    return x + o.forward(attn);
}

at::Tensor Qwen3LayerW4A16::mlp_residual(const at::Tensor& x, const at::Tensor& h2) const {
    const at::Tensor a = gate_up.size() == 1 ? gate_up[0].forward(h2)
                                             : at::silu(gate_up.at(0).forward(h2)) * gate_up.at(1).forward(h2);
    return x + down.forward(a);
}

at::Tensor rmsnorm_ref(const at::Tensor& x, const at::Tensor& weight, double eps) {
    const at::Tensor xf = x.to(at::kFloat);
    const at::Tensor inv = at::rsqrt(xf.pow(2).mean({-1}, /*keepdim=*/true) + eps);
    return (xf * inv * weight.to(at::kFloat)).to(x.scalar_type());
}

at::Tensor qwen3_block_w4a16(const Qwen3LayerW4A16& layer, const at::Tensor& x, const at::Tensor& ln1,
                             const at::Tensor& ln2, double eps, const AttentionFn& attention) {
    auto [q, k, v] = layer.qkv_proj(rmsnorm_ref(x, ln1, eps));
    const at::Tensor x1 = layer.o_proj_residual(x, attention(q, k, v));
    return layer.mlp_residual(x1, rmsnorm_ref(x1, ln2, eps));
}

namespace {

// torch.classes.pulsar.Qwen3W4A16Layer: one layer built from a weights map, for
// callers (and tests) that reach the C++ layer from Python.
class Qwen3W4A16LayerModule : public torch::CustomClassHolder {
   public:
    Qwen3W4A16LayerModule(c10::Dict<std::string, at::Tensor> weights, std::string prefix, int64_t group_size,
                          int64_t n_heads, int64_t n_kv_heads, int64_t head_dim)
        : layer_(Qwen3LayerW4A16::from_weights(weights, prefix, group_size)),
          n_heads_(n_heads),
          n_kv_heads_(n_kv_heads),
          head_dim_(head_dim) {
        TORCH_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "Qwen3W4A16Layer: n_heads % n_kv_heads != 0");
        TORCH_CHECK(layer_.q_dim == n_heads * head_dim && layer_.kv_dim == n_kv_heads * head_dim,
                    "Qwen3W4A16Layer: q/k/v sizes do not match the head counts");
    }

    std::tuple<at::Tensor, at::Tensor, at::Tensor> qkv(const at::Tensor& h) { return layer_.qkv_proj(h); }
    // (linears the q/k/v projections run as, linears the gate/up projections run as): 1 when fused
    std::tuple<int64_t, int64_t> fusion() { return {(int64_t)layer_.qkv.size(), (int64_t)layer_.gate_up.size()}; }
    at::Tensor o_residual(const at::Tensor& x, const at::Tensor& attn) { return layer_.o_proj_residual(x, attn); }
    at::Tensor mlp_residual(const at::Tensor& x, const at::Tensor& h2) { return layer_.mlp_residual(x, h2); }

    // The whole block with attention over a one-token context: each token attends only
    // to itself, where softmax over a single key is 1, so o = v with each kv head
    // repeated for its n_heads / n_kv_heads query heads.
    at::Tensor block_self_attention(const at::Tensor& x, const at::Tensor& ln1, const at::Tensor& ln2, double eps) {
        const int64_t rep = n_heads_ / n_kv_heads_, hd = head_dim_, nkv = n_kv_heads_;
        return qwen3_block_w4a16(layer_, x, ln1, ln2, eps, [rep, hd, nkv](const at::Tensor&, const at::Tensor&,
                                                                          const at::Tensor& v) {
            const int64_t t = v.size(0);
            return v.view({t, nkv, 1, hd}).expand({t, nkv, rep, hd}).reshape({t, nkv * rep * hd});
        });
    }

   private:
    Qwen3LayerW4A16 layer_;
    int64_t n_heads_, n_kv_heads_, head_dim_;
};

}  // namespace

}  // namespace pulsar

TORCH_LIBRARY_FRAGMENT(pulsar, m) {
    m.class_<pulsar::Qwen3W4A16LayerModule>("Qwen3W4A16Layer")
        .def(torch::init<c10::Dict<std::string, at::Tensor>, std::string, int64_t, int64_t, int64_t, int64_t>())
        .def("qkv", &pulsar::Qwen3W4A16LayerModule::qkv)
        .def("fusion", &pulsar::Qwen3W4A16LayerModule::fusion)
        .def("o_residual", &pulsar::Qwen3W4A16LayerModule::o_residual)
        .def("mlp_residual", &pulsar::Qwen3W4A16LayerModule::mlp_residual)
        .def("block_self_attention", &pulsar::Qwen3W4A16LayerModule::block_self_attention);
}

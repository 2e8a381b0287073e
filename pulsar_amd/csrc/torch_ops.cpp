// at::Tensor shim over the C ABI (include/pulsar_w4a16.h) and the torch op
// registration.  The four reference schemas are kept verbatim
// (pulsar/ext/ops.cpp:39-52) under the `pulsar` namespace and implemented for
// the CUDA dispatch key, which is the HIP device key of ROCm PyTorch
// (pulsar/ext/ops.cpp:61,68-71).  The precondition messages follow the
// reference TORCH_CHECKs (w4a16_gemm.cu:324-348, w4a16_marlin.cu:356-371,414-442).
#include "pulsar_w4a16_ops.hpp"

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <map>
#include <mutex>
#include <vector>

#include "pulsar_w4a16.h"

namespace pulsar {
namespace {

constexpr int64_t kMarlinBN = 64, kMarlinBK = 64;

int64_t roundup(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// ROCm PyTorch keeps HIP devices under the CUDA device type ("masquerading"),
// so the guard and the current-stream query are the masquerading variants.
using DeviceGuard = c10::hip::HIPGuardMasqueradingAsCUDA;

pw4_stream_t current_stream() {
    return reinterpret_cast<pw4_stream_t>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
}

void check_status(int rc, const char* op) {
    if (rc == PW4_ERR_HIP) {
        TORCH_CHECK(false, op, ": ", pw4_status_string(rc), ": ", pw4_last_hip_error());
    }
    TORCH_CHECK(rc == PW4_OK, op, ": ", pw4_status_string(rc));
}

int x_dtype_code(const at::Tensor& x) { return x.scalar_type() == at::kBFloat16 ? PW4_DTYPE_BF16 : PW4_DTYPE_F16; }

// GEMM workspaces: one per (device, stream).  The C ABI needs the zero region
// at the start of a workspace to be zero on entry and leaves it zero, and
// calls on one stream are ordered, so the calls of a stream share one buffer.
// Under HIP graph capture three rules keep that true:
//  * a buffer is never freed.  When a call needs more, the smaller buffer is
//    retired but kept alive until the process exits, so a graph that captured
//    its address still replays into valid memory that nothing else uses;
//  * only the zero region (the first PW4_ZERO_REGION_BYTES) has to be zero;
//    the rest is scratch that every call writes before it reads it;
//  * a buffer allocated while the stream captures has its zero region
//    cleared by a fill node of the graph (zero_() records a kernel), so a
//    replay clears it before the GEMM.  The fill is recorded once per
//    capture: the calls after it in the graph find the region as the earlier
//    ones left it, zero.  Such a fill never ran eagerly, so the next eager
//    call on the stream clears the region first, and a later capture records
//    a fill of its own until then;
//  * graphs captured on one stream share that stream's buffer, so they are
//    replayed in order (on one stream, or synchronised), like the calls of a
//    stream.
struct StreamWorkspace {
    at::Tensor buf;
    bool zeroed_eagerly = true;  // false until a buffer allocated under capture is zeroed outside it
    unsigned long long fill_capture = 0;  // capture id whose graph already holds the fill (0: none)
};

at::Tensor workspace(size_t bytes, const at::Tensor& like) {
    if (bytes == 0) return at::Tensor();
    static std::mutex mu;
    static std::map<std::pair<int64_t, int64_t>, StreamWorkspace> cache;
    static std::vector<at::Tensor> retired;
    const auto stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA();
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    TORCH_CHECK(hipStreamGetCaptureInfo(stream.stream(), &cs, &cid) == hipSuccess,
                "W4A16 workspace: hipStreamGetCaptureInfo failed");
    const bool capturing = cs == hipStreamCaptureStatusActive;
    const std::pair<int64_t, int64_t> key{like.device().index(), (int64_t)stream.id()};
    std::lock_guard<std::mutex> lock(mu);
    StreamWorkspace& w = cache[key];
    auto clear_zero_region = [&]() {
        w.buf.narrow(0, 0, std::min<int64_t>(w.buf.numel(), (int64_t)PW4_ZERO_REGION_BYTES)).zero_();
        w.zeroed_eagerly = !capturing;
        w.fill_capture = capturing ? cid : 0;
    };
    if (!w.buf.defined() || (size_t)w.buf.numel() < bytes) {
        const size_t grow = w.buf.defined() ? std::max(bytes, (size_t)w.buf.numel() * 2) : bytes;
        if (w.buf.defined()) retired.push_back(std::move(w.buf));
        w.buf = at::empty({(int64_t)grow}, like.options().dtype(at::kByte));
        clear_zero_region();
    } else if (!w.zeroed_eagerly && !(capturing && w.fill_capture == cid)) {
        clear_zero_region();  // eagerly, or as a fill node of this capture
    }
    return w.buf;
}

void* ptr_or_null(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

at::Tensor gemm_w4a16_run(const at::Tensor& x, const at::Tensor& weight_packed, const at::Tensor& weight_scale,
                          int64_t group_size, int64_t forced_splits) {
    TORCH_CHECK(x.is_cuda() && weight_packed.is_cuda() && weight_scale.is_cuda(),
                "gemm_w4a16: all inputs must be CUDA tensors");
    TORCH_CHECK(x.scalar_type() == at::kHalf || x.scalar_type() == at::kBFloat16, "gemm_w4a16: x must be fp16 or bf16");
    TORCH_CHECK(weight_packed.scalar_type() == at::kInt, "gemm_w4a16: weight_packed must be int32");
    TORCH_CHECK(x.dim() == 2, "gemm_w4a16: x must be 2-D [M, K]");
    TORCH_CHECK(weight_packed.dim() == 2, "gemm_w4a16: weight_packed must be 2-D [N, K/8]");
    TORCH_CHECK(weight_scale.dim() == 2, "gemm_w4a16: weight_scale must be 2-D [N, K/group_size]");
    TORCH_CHECK(x.is_contiguous(), "gemm_w4a16: x must be contiguous");
    const int64_t M = x.size(0), K = x.size(1), N = weight_packed.size(0);
    TORCH_CHECK(group_size > 0 && group_size % 16 == 0, "gemm_w4a16: group_size must be a positive multiple of 16");
    TORCH_CHECK(K % 8 == 0 && weight_packed.size(1) == K / 8,
                "gemm_w4a16: weight_packed must be [N, K/8] with K a multiple of 8");
    TORCH_CHECK(K % group_size == 0, "gemm_w4a16: K must be a multiple of group_size");
    TORCH_CHECK(weight_scale.size(0) == N && weight_scale.size(1) == K / group_size,
                "gemm_w4a16: weight_scale must be [N, K/group_size]");

    DeviceGuard guard(x.device());
    auto wp = weight_packed.contiguous();
    auto ws = weight_scale.to(at::kFloat).contiguous();
    auto y = at::empty({M, N}, x.options());
    if (M == 0 || N == 0) return y;
    const size_t wsb = pw4_gemm_w4a16_workspace_size(M, N, K, group_size, forced_splits);
    at::Tensor wsp = workspace(wsb, x);
    const int rc = pw4_gemm_w4a16(x.data_ptr(), x_dtype_code(x), wp.data_ptr<int32_t>(), ws.data_ptr<float>(),
                                  y.data_ptr(), M, N, K, group_size, forced_splits, ptr_or_null(wsp), wsb,
                                  current_stream());
    check_status(rc, "gemm_w4a16");
    return y;
}

at::Tensor marlin_run(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scales,
                      const std::optional<at::Tensor>& qzeros, const std::optional<at::Tensor>& perm,
                      int64_t group_size, int64_t forced_splits, const char* op, bool fp32_scales_only,
                      bool silu = false) {
    TORCH_CHECK(x.is_cuda() && weight_marlin.is_cuda() && scales.is_cuda(), op, ": all inputs must be CUDA tensors");
    TORCH_CHECK(x.scalar_type() == at::kHalf || x.scalar_type() == at::kBFloat16, op, ": x must be fp16 or bf16");
    TORCH_CHECK(weight_marlin.scalar_type() == at::kInt, op, ": weight_marlin must be int32");
    if (fp32_scales_only) {
        TORCH_CHECK(scales.scalar_type() == at::kFloat, op, ": scale_marlin must be fp32");
    } else {
        TORCH_CHECK(scales.scalar_type() == at::kFloat || scales.scalar_type() == at::kHalf, op,
                    ": scales must be fp32 or fp16");
    }
    TORCH_CHECK(x.dim() == 2, op, ": x must be 2-D [M, K]");
    TORCH_CHECK(scales.dim() == 2, op, ": scale_marlin must be 2-D [K/G, N]");
    TORCH_CHECK(group_size > 0 && group_size % 16 == 0, op, ": group_size must be a positive multiple of 16");
    TORCH_CHECK(x.is_contiguous(), op, ": x must be contiguous");
    const int64_t M = x.size(0), K = x.size(1), N = scales.size(1), Kg = scales.size(0);
    TORCH_CHECK(Kg == K / group_size && K % group_size == 0, op, ": scale_marlin K/G must match x's K");
    TORCH_CHECK(K % 8 == 0, op, ": K must be a multiple of 8");
    const int64_t Kpad = roundup(K, kMarlinBK), Npad = roundup(N, kMarlinBN);
    TORCH_CHECK(weight_marlin.numel() == Npad * Kpad / 8, op, ": weight_marlin has wrong size for this shape");
    const int32_t* zp = nullptr;
    at::Tensor zc, pc;
    if (qzeros.has_value() && qzeros->defined()) {
        TORCH_CHECK(qzeros->is_cuda() && qzeros->scalar_type() == at::kInt, op, ": qzeros must be a CUDA int32 tensor");
        TORCH_CHECK(N % 8 == 0 && qzeros->dim() == 2 && qzeros->size(0) == Kg && qzeros->size(1) == N / 8, op,
                    ": qzeros must be [K/group_size, N/8]");
        zc = qzeros->contiguous();
        zp = zc.data_ptr<int32_t>();
    }
    const int32_t* pp = nullptr;
    if (perm.has_value() && perm->defined() && perm->numel() > 0) {
        TORCH_CHECK(perm->is_cuda() && perm->scalar_type() == at::kInt, op, ": perm must be a CUDA int32 tensor");
        TORCH_CHECK(perm->dim() == 1 && perm->size(0) == K, op, ": perm must be [K]");
        pc = perm->contiguous();
        pp = pc.data_ptr<int32_t>();
    }
    DeviceGuard guard(x.device());
    auto wm = weight_marlin.contiguous();
    auto sm = scales.contiguous();
    if (silu) {
        TORCH_CHECK(N % 16 == 0, op, ": N (gate|up interleaved by 8) must be a multiple of 16");
        auto y = at::empty({M, N / 2}, x.options());
        if (M == 0 || N == 0) return y;
        const size_t wsb = pw4_gemm_w4a16_silu_mul_workspace_size(M, N, K, group_size, pp != nullptr);
        at::Tensor wsp = workspace(wsb, x);
        const int rc = pw4_gemm_w4a16_silu_mul(x.data_ptr(), x_dtype_code(x), wm.data_ptr<int32_t>(), sm.data_ptr(),
                                               sm.scalar_type() == at::kFloat ? PW4_DTYPE_F32 : PW4_DTYPE_F16, zp, pp,
                                               y.data_ptr(), M, N, K, group_size, ptr_or_null(wsp), wsb,
                                               current_stream());
        check_status(rc, op);
        return y;
    }
    auto y = at::empty({M, N}, x.options());
    if (M == 0 || N == 0) return y;
    const size_t wsb = pw4_gemm_w4a16_marlin_workspace_size(M, N, K, group_size, pp != nullptr, forced_splits);
    at::Tensor wsp = workspace(wsb, x);
    const int rc = pw4_gemm_w4a16_marlin(x.data_ptr(), x_dtype_code(x), wm.data_ptr<int32_t>(), sm.data_ptr(),
                                         sm.scalar_type() == at::kFloat ? PW4_DTYPE_F32 : PW4_DTYPE_F16, zp, pp,
                                         y.data_ptr(), M, N, K, group_size, forced_splits, ptr_or_null(wsp), wsb,
                                         current_stream());
    check_status(rc, op);
    return y;
}

}  // namespace

at::Tensor gemm_w4a16_cuda(const at::Tensor& x, const at::Tensor& weight_packed, const at::Tensor& weight_scale,
                           int64_t group_size) {
    return gemm_w4a16_run(x, weight_packed, weight_scale, group_size, 0);
}

at::Tensor gemm_w4a16_split_cuda(const at::Tensor& x, const at::Tensor& weight_packed,
                                 const at::Tensor& weight_scale, int64_t group_size, int64_t num_splits) {
    TORCH_CHECK(num_splits >= 1, "gemm_w4a16_split: num_splits must be >= 1");
    return gemm_w4a16_run(x, weight_packed, weight_scale, group_size, num_splits);
}

std::tuple<at::Tensor, at::Tensor> repack_w4a16_cuda(const at::Tensor& weight_packed,
                                                     const at::Tensor& weight_scale, int64_t group_size) {
    TORCH_CHECK(weight_packed.is_cuda() && weight_scale.is_cuda(), "repack_w4a16: inputs must be CUDA tensors");
    TORCH_CHECK(weight_packed.scalar_type() == at::kInt, "repack_w4a16: weight_packed must be int32");
    TORCH_CHECK(weight_packed.dim() == 2 && weight_scale.dim() == 2,
                "repack_w4a16: weight_packed [N,K/8] and weight_scale [N,K/G]");
    TORCH_CHECK(group_size > 0 && group_size % 16 == 0, "repack_w4a16: group_size must be a positive multiple of 16");
    const int64_t N = weight_packed.size(0), K = weight_packed.size(1) * 8;
    TORCH_CHECK(K % group_size == 0, "repack_w4a16: K must be a multiple of group_size");
    const int64_t Kg = K / group_size;
    TORCH_CHECK(weight_scale.size(0) == N && weight_scale.size(1) == Kg,
                "repack_w4a16: weight_scale must be [N, K/group_size]");
    const auto st = weight_scale.scalar_type();
    TORCH_CHECK(st == at::kFloat || st == at::kHalf || st == at::kBFloat16,
                "repack_w4a16: weight_scale must be fp32, fp16 or bf16");
    DeviceGuard guard(weight_packed.device());
    auto wp = weight_packed.contiguous();
    auto ws = weight_scale.contiguous();
    auto weight_marlin = at::empty({pw4_marlin_words(N, K)}, wp.options());
    auto scale_marlin = at::empty({Kg, N}, ws.options().dtype(at::kFloat));
    const int sd = st == at::kFloat ? PW4_DTYPE_F32 : (st == at::kHalf ? PW4_DTYPE_F16 : PW4_DTYPE_BF16);
    const int rc = pw4_repack_w4a16(wp.data_ptr<int32_t>(), ws.data_ptr(), sd, N, K, group_size,
                                    weight_marlin.data_ptr<int32_t>(), scale_marlin.data_ptr<float>(),
                                    current_stream());
    check_status(rc, "repack_w4a16");
    return {weight_marlin, scale_marlin};
}

at::Tensor gemm_w4a16_marlin_cuda(const at::Tensor& x, const at::Tensor& weight_marlin,
                                  const at::Tensor& scale_marlin, int64_t group_size) {
    return marlin_run(x, weight_marlin, scale_marlin, std::nullopt, std::nullopt, group_size, 0,
                      "gemm_w4a16_marlin", true);
}

at::Tensor gemm_w4a16_marlin_split_cuda(const at::Tensor& x, const at::Tensor& weight_marlin,
                                        const at::Tensor& scale_marlin, int64_t group_size, int64_t num_splits) {
    TORCH_CHECK(num_splits >= 1, "gemm_w4a16_marlin_split: num_splits must be >= 1");
    return marlin_run(x, weight_marlin, scale_marlin, std::nullopt, std::nullopt, group_size, num_splits,
                      "gemm_w4a16_marlin_split", true);
}

std::tuple<at::Tensor, at::Tensor> repack_w4a16_gptq_cuda(const at::Tensor& qweight,
                                                          const std::optional<at::Tensor>& g_idx,
                                                          int64_t group_size) {
    TORCH_CHECK(qweight.is_cuda() && qweight.scalar_type() == at::kInt && qweight.dim() == 2,
                "repack_w4a16_gptq: qweight must be a CUDA int32 [K/8, N] tensor");
    TORCH_CHECK(group_size > 0 && group_size % 16 == 0,
                "repack_w4a16_gptq: group_size must be a positive multiple of 16");
    const int64_t K = qweight.size(0) * 8, N = qweight.size(1);
    TORCH_CHECK(K % group_size == 0, "repack_w4a16_gptq: K must be a multiple of group_size");
    DeviceGuard guard(qweight.device());
    auto qw = qweight.contiguous();
    auto weight_marlin = at::empty({pw4_marlin_words(N, K)}, qw.options());
    at::Tensor perm = at::empty({0}, qw.options());
    const int32_t* pp = nullptr;
    if (g_idx.has_value() && g_idx->defined()) {
        TORCH_CHECK(g_idx->is_cuda() && g_idx->dim() == 1 && g_idx->size(0) == K,
                    "repack_w4a16_gptq: g_idx must be a CUDA [K] tensor");
        auto gi = g_idx->to(at::kInt).contiguous();
        perm = at::empty({K}, qw.options());
        auto status = at::empty({1}, qw.options());
        int rc = pw4_gidx_to_perm(gi.data_ptr<int32_t>(), K, group_size, perm.data_ptr<int32_t>(),
                                  status.data_ptr<int32_t>(), current_stream());
        check_status(rc, "repack_w4a16_gptq");
        TORCH_CHECK(status.item<int32_t>() == 0, "repack_w4a16_gptq: ", pw4_status_string(PW4_ERR_GIDX));
        pp = perm.data_ptr<int32_t>();
    }
    const int rc = pw4_repack_gptq(qw.data_ptr<int32_t>(), pp, N, K, weight_marlin.data_ptr<int32_t>(),
                                   current_stream());
    check_status(rc, "repack_w4a16_gptq");
    return {weight_marlin, perm};
}

at::Tensor gemm_w4a16_gptq_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scales,
                                const std::optional<at::Tensor>& qzeros, const std::optional<at::Tensor>& perm,
                                int64_t group_size) {
    return marlin_run(x, weight_marlin, scales, qzeros, perm, group_size, 0, "gemm_w4a16_gptq", false);
}

// silu(x @ Wg^T) * (x @ Wu^T) from a gate|up weight interleaved by 8 columns:
// the MLP gate of qwen3.cpp:116-118 in one op.
at::Tensor gemm_w4a16_silu_mul_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scales,
                                    const std::optional<at::Tensor>& qzeros, const std::optional<at::Tensor>& perm,
                                    int64_t group_size) {
    return marlin_run(x, weight_marlin, scales, qzeros, perm, group_size, 0, "gemm_w4a16_silu_mul", false, true);
}

}  // namespace pulsar

// Schema strings: the first four are the reference ABI verbatim.
TORCH_LIBRARY_FRAGMENT(pulsar, m) {
    m.def("gemm_w4a16(Tensor x, Tensor weight_packed, Tensor weight_scale, int group_size) -> Tensor");
    m.def(
        "gemm_w4a16_split(Tensor x, Tensor weight_packed, Tensor weight_scale, "
        "int group_size, int num_splits) -> Tensor");
    m.def("repack_w4a16(Tensor weight_packed, Tensor weight_scale, int group_size) -> (Tensor, Tensor)");
    m.def("gemm_w4a16_marlin(Tensor x, Tensor weight_marlin, Tensor scale_marlin, int group_size) -> Tensor");
    m.def(
        "gemm_w4a16_marlin_split(Tensor x, Tensor weight_marlin, Tensor scale_marlin, int group_size, "
        "int num_splits) -> Tensor");
    m.def("repack_w4a16_gptq(Tensor qweight, Tensor? g_idx, int group_size) -> (Tensor, Tensor)");
    m.def(
        "gemm_w4a16_gptq(Tensor x, Tensor weight_marlin, Tensor scales, Tensor? qzeros, Tensor? perm, "
        "int group_size) -> Tensor");
    m.def(
        "gemm_w4a16_silu_mul(Tensor x, Tensor weight_marlin, Tensor scales, Tensor? qzeros, Tensor? perm, "
        "int group_size) -> Tensor");
}

TORCH_LIBRARY_IMPL(pulsar, CUDA, m) {
    m.impl("gemm_w4a16", TORCH_FN(pulsar::gemm_w4a16_cuda));
    m.impl("gemm_w4a16_split", TORCH_FN(pulsar::gemm_w4a16_split_cuda));
    m.impl("repack_w4a16", TORCH_FN(pulsar::repack_w4a16_cuda));
    m.impl("gemm_w4a16_marlin", TORCH_FN(pulsar::gemm_w4a16_marlin_cuda));
    m.impl("gemm_w4a16_marlin_split", TORCH_FN(pulsar::gemm_w4a16_marlin_split_cuda));
    m.impl("repack_w4a16_gptq", TORCH_FN(pulsar::repack_w4a16_gptq_cuda));
    m.impl("gemm_w4a16_gptq", TORCH_FN(pulsar::gemm_w4a16_gptq_cuda));
    m.impl("gemm_w4a16_silu_mul", TORCH_FN(pulsar::gemm_w4a16_silu_mul_cuda));
}

// pw4_selftest -- a torch-free C++ caller of the C ABI in include/pulsar_w4a16.h.
//
// Links libpulsar_w4a16.so and the HIP runtime only: device memory comes from
// hipMalloc, inputs are made on the host, and every result is checked against
// a CPU dequantise-then-GEMM in double precision.  It is what a non-ATen C++
// caller of the reference's operators (pulsar-core/inc/pulsar/ops.hpp:156-189)
// does after switching to this library, and it doubles as that caller's
// worked example:
//   1. pw4_repack_w4a16 once per weight (compressed-tensors int4 -> MARLIN),
//   2. one workspace sized by the *_workspace_size queries, cleared once,
//   3. GEMM calls on a stream, each returning a PW4_* status.
//
// Usage: pw4_selftest [-v]   (exit status 0 when every case passes)
//
// Tolerances are the parity bars of the library's GPU tests:
//   max|y - ref| / max|ref| <= 5e-3 (fp16 x) or 2e-2 (bf16 x),
//   ||y - ref|| / ||ref||   <= 1e-3 (fp16 x).

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "pulsar_w4a16.h"

namespace {

bool g_verbose = false;

#define HIP_OK(call)                                                                          \
  do {                                                                                        \
    hipError_t e_ = (call);                                                                   \
    if (e_ != hipSuccess) {                                                                   \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #call, hipGetErrorString(e_)); \
      std::exit(2);                                                                           \
    }                                                                                         \
  } while (0)

// splitmix64: a fixed, seedable stream of 64-bit values.
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double uniform() { return (next() >> 11) * (1.0 / 9007199254740992.0); }
  double normal() {  // Box-Muller
    double u1 = uniform(), u2 = uniform();
    if (u1 < 1e-300) u1 = 1e-300;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
  }
};

// IEEE binary16 and bfloat16 conversions, round to nearest even (finite inputs).
uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t exp = int32_t((x >> 23) & 0xffu) - 127 + 15;
  uint32_t mant = x & 0x7fffffu;
  if (exp >= 31) return uint16_t(sign | 0x7c00u);
  if (exp <= 0) {
    if (exp < -10) return uint16_t(sign);
    mant |= 0x800000u;
    const int shift = 14 - exp;
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return uint16_t(sign | h);
  }
  uint32_t h = (uint32_t(exp) << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry into the exponent is the right result
  return uint16_t(sign | h);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  float v;
  if (exp == 0) {
    v = std::ldexp(float(mant), -24);
  } else if (exp == 31) {
    v = mant ? NAN : INFINITY;
  } else {
    v = std::ldexp(float(mant | 0x400u), int(exp) - 25);
  }
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  bits |= sign;
  std::memcpy(&v, &bits, 4);
  return v;
}

uint16_t f32_to_bf16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  return uint16_t((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

float bf16_to_f32(uint16_t b) {
  const uint32_t x = uint32_t(b) << 16;
  float v;
  std::memcpy(&v, &x, 4);
  return v;
}

// One linear layer on the host: int4 values q[n][k] in [-8, 7] packed the
// compressed-tensors way (nibble k%8 of int32 word [n][k/8], two's complement),
// fp32 scales [N][K/G], activations [M][K] rounded to the activation dtype.
struct Layer {
  int64_t M, N, K, G;
  int x_dtype;
  std::vector<int32_t> packed;  // [N][K/8]
  std::vector<float> scale;     // [N][K/G]
  std::vector<uint16_t> x;      // [M][K] fp16 or bf16 bits
  std::vector<double> ref;      // [M][N]

  Layer(int64_t m, int64_t n, int64_t k, int64_t g, int dtype, uint64_t seed) : M(m), N(n), K(k), G(g), x_dtype(dtype) {
    Rng rng(seed);
    std::vector<int8_t> q(size_t(N * K));
    for (auto& v : q) v = int8_t(int(rng.next() >> 60) - 8);
    packed.assign(size_t(N * K / 8), 0);
    for (int64_t n_ = 0; n_ < N; ++n_)
      for (int64_t k_ = 0; k_ < K; ++k_)
        packed[size_t(n_ * (K / 8) + k_ / 8)] |= int32_t(uint32_t(q[size_t(n_ * K + k_)] & 0xf) << (4 * (k_ % 8)));
    scale.resize(size_t(N * (K / G)));
    for (auto& s : scale) s = float(1e-3 + 0.02 * std::fabs(rng.normal()));
    x.resize(size_t(M * K));
    std::vector<double> xf(size_t(M * K));
    for (size_t i = 0; i < x.size(); ++i) {
      const float v = float(rng.normal());
      x[i] = dtype == PW4_DTYPE_BF16 ? f32_to_bf16(v) : f32_to_f16(v);
      xf[i] = dtype == PW4_DTYPE_BF16 ? bf16_to_f32(x[i]) : f16_to_f32(x[i]);
    }
    // y = x @ (q * s)^T in double
    std::vector<double> w(static_cast<size_t>(K));
    ref.assign(size_t(M * N), 0.0);
    for (int64_t n_ = 0; n_ < N; ++n_) {
      for (int64_t k_ = 0; k_ < K; ++k_)
        w[size_t(k_)] = double(q[size_t(n_ * K + k_)]) * double(scale[size_t(n_ * (K / G) + k_ / G)]);
      for (int64_t m_ = 0; m_ < M; ++m_) {
        const double* xr = xf.data() + m_ * K;
        double acc = 0.0;
        for (int64_t k_ = 0; k_ < K; ++k_) acc += xr[k_] * w[size_t(k_)];
        ref[size_t(m_ * N + n_)] = acc;
      }
    }
  }

  // The parity bars of the GPU tests; prints the metrics of one result.
  bool check(const std::vector<uint16_t>& y, const char* what) const {
    double max_err = 0, max_ref = 0, se = 0, sr = 0;
    for (size_t i = 0; i < ref.size(); ++i) {
      const double v = x_dtype == PW4_DTYPE_BF16 ? bf16_to_f32(y[i]) : f16_to_f32(y[i]);
      const double e = std::fabs(v - ref[i]);
      if (!(e <= max_err)) max_err = e;  // a NaN sticks
      max_ref = std::fmax(max_ref, std::fabs(ref[i]));
      se += e * e;
      sr += ref[i] * ref[i];
    }
    const double rel_max = max_err / max_ref, rel_l2 = std::sqrt(se / sr);
    const bool bf16 = x_dtype == PW4_DTYPE_BF16;
    const bool ok = rel_max <= (bf16 ? 2e-2 : 5e-3) && (bf16 || rel_l2 <= 1e-3);
    std::printf("%-4s %-34s M=%-4lld N=%-5lld K=%-5lld %s  rel_max=%.2e rel_l2=%.2e\n", ok ? "ok" : "FAIL", what,
                (long long)M, (long long)N, (long long)K, bf16 ? "bf16" : "fp16", rel_max, rel_l2);
    return ok;
  }
};

template <typename T>
T* upload(const std::vector<T>& v) {
  T* d = nullptr;
  HIP_OK(hipMalloc(&d, v.size() * sizeof(T)));
  HIP_OK(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}

// A workspace shared by every GEMM call below, sized by the largest query and
// cleared once, as the workspace contract asks.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  void reserve(size_t b) {
    if (b <= bytes) return;
    if (ptr) HIP_OK(hipFree(ptr));
    HIP_OK(hipMalloc(&ptr, b));
    HIP_OK(hipMemset(ptr, 0, b));
    bytes = b;
  }
  bool zero_region_clear() const {
    if (!ptr) return true;
    const size_t n = bytes < PW4_ZERO_REGION_BYTES ? bytes : PW4_ZERO_REGION_BYTES;
    std::vector<uint8_t> h(n);
    HIP_OK(hipMemcpy(h.data(), ptr, n, hipMemcpyDeviceToHost));
    for (uint8_t b : h)
      if (b) return false;
    return true;
  }
};

bool status_ok(int rc, const char* what) {
  if (rc == PW4_OK) return true;
  std::printf("FAIL %s returned %d (%s; %s)\n", what, rc, pw4_status_string(rc), pw4_last_hip_error());
  return false;
}

// MARLIN path: repack once, then pw4_gemm_w4a16_marlin with fp32 scales.
bool marlin_case(const char* what, const Layer& L, int64_t num_splits, Workspace& ws, hipStream_t st, bool timed) {
  int32_t* packed = upload(L.packed);
  float* scale = upload(L.scale);
  uint16_t* x = upload(L.x);
  int32_t *wm = nullptr;
  float* sm = nullptr;
  uint16_t* y = nullptr;
  HIP_OK(hipMalloc(&wm, size_t(pw4_marlin_words(L.N, L.K)) * 4));
  HIP_OK(hipMalloc(&sm, size_t(L.N * (L.K / L.G)) * 4));
  HIP_OK(hipMalloc(&y, size_t(L.M * L.N) * 2));
  bool ok = status_ok(pw4_repack_w4a16(packed, scale, PW4_DTYPE_F32, L.N, L.K, L.G, wm, sm, st), "pw4_repack_w4a16");
  ws.reserve(pw4_gemm_w4a16_marlin_workspace_size(L.M, L.N, L.K, L.G, 0, num_splits));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (ok && timed) {
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    ok = status_ok(pw4_time_next_kernel(e0, e1), "pw4_time_next_kernel");
  }
  if (ok)
    ok = status_ok(pw4_gemm_w4a16_marlin(x, L.x_dtype, wm, sm, PW4_DTYPE_F32, nullptr, nullptr, y, L.M, L.N, L.K,
                                         L.G, num_splits, ws.ptr, ws.bytes, st),
                   "pw4_gemm_w4a16_marlin");
  HIP_OK(hipStreamSynchronize(st));
  if (ok) {
    std::vector<uint16_t> h(size_t(L.M * L.N));
    HIP_OK(hipMemcpy(h.data(), y, h.size() * 2, hipMemcpyDeviceToHost));
    ok = L.check(h, what);
    if (timed && g_verbose) {
      float ms = 0;
      HIP_OK(hipEventElapsedTime(&ms, e0, e1));
      std::printf("     kernel time of that call (pw4_time_next_kernel): %.2f us\n", ms * 1e3);
    }
  }
  if (e0) HIP_OK(hipEventDestroy(e0));
  if (e1) HIP_OK(hipEventDestroy(e1));
  for (void* p : {(void*)packed, (void*)scale, (void*)x, (void*)wm, (void*)sm, (void*)y}) HIP_OK(hipFree(p));
  return ok;
}

// Compressed-tensors path without a repack: pw4_gemm_w4a16.
bool ct_case(const char* what, const Layer& L, int64_t num_splits, Workspace& ws, hipStream_t st) {
  int32_t* packed = upload(L.packed);
  float* scale = upload(L.scale);
  uint16_t* x = upload(L.x);
  uint16_t* y = nullptr;
  HIP_OK(hipMalloc(&y, size_t(L.M * L.N) * 2));
  ws.reserve(pw4_gemm_w4a16_workspace_size(L.M, L.N, L.K, L.G, num_splits));
  bool ok = status_ok(
      pw4_gemm_w4a16(x, L.x_dtype, packed, scale, y, L.M, L.N, L.K, L.G, num_splits, ws.ptr, ws.bytes, st),
      "pw4_gemm_w4a16");
  HIP_OK(hipStreamSynchronize(st));
  if (ok) {
    std::vector<uint16_t> h(size_t(L.M * L.N));
    HIP_OK(hipMemcpy(h.data(), y, h.size() * 2, hipMemcpyDeviceToHost));
    ok = L.check(h, what);
  }
  for (void* p : {(void*)packed, (void*)scale, (void*)x, (void*)y}) HIP_OK(hipFree(p));
  return ok;
}

// The reference's precondition checks come back as status codes, before any launch.
bool error_cases(Workspace& ws, hipStream_t st) {
  bool ok = true;
  auto expect = [&](int rc, int want, const char* what) {
    const bool good = rc == want;
    std::printf("%-4s %-34s -> %d (%s)\n", good ? "ok" : "FAIL", what, rc, pw4_status_string(rc));
    ok = ok && good;
  };
  void* dummy = nullptr;
  HIP_OK(hipMalloc(&dummy, 1 << 20));
  const int64_t M = 4, N = 64, K = 256;
  // group_size % 16 != 0 (reference w4a16_marlin.cu:414-442)
  expect(pw4_gemm_w4a16_marlin(dummy, PW4_DTYPE_F16, (const int32_t*)dummy, dummy, PW4_DTYPE_F32, nullptr, nullptr,
                               dummy, M, N, K, 40, 0, ws.ptr, ws.bytes, st),
         PW4_ERR_SHAPE, "group_size 40");
  // K % group_size != 0
  expect(pw4_gemm_w4a16(dummy, PW4_DTYPE_F16, (const int32_t*)dummy, (const float*)dummy, dummy, M, N, 200, 128, 0,
                        ws.ptr, ws.bytes, st),
         PW4_ERR_SHAPE, "K % group_size");
  // unknown activation dtype
  expect(pw4_gemm_w4a16_marlin(dummy, 7, (const int32_t*)dummy, dummy, PW4_DTYPE_F32, nullptr, nullptr, dummy, M, N,
                               K, 128, 0, ws.ptr, ws.bytes, st),
         PW4_ERR_ARG, "x_dtype 7");
  // a forced K split with no workspace
  if (pw4_gemm_w4a16_marlin_workspace_size(M, N, K, 128, 0, 2) > 0)
    expect(pw4_gemm_w4a16_marlin(dummy, PW4_DTYPE_F16, (const int32_t*)dummy, dummy, PW4_DTYPE_F32, nullptr, nullptr,
                                 dummy, M, N, K, 128, 2, nullptr, 0, st),
           PW4_ERR_WORKSPACE, "split without workspace");
  HIP_OK(hipStreamSynchronize(st));
  HIP_OK(hipFree(dummy));
  return ok;
}

}  // namespace

int main(int argc, char** argv) {
  for (int i = 1; i < argc; ++i)
    if (!std::strcmp(argv[i], "-v")) g_verbose = true;
  if (pw4_abi_version() != PW4_ABI_VERSION) {
    std::printf("FAIL ABI version %d, header %d\n", pw4_abi_version(), PW4_ABI_VERSION);
    return 1;
  }
  int dev_count = 0;
  if (hipGetDeviceCount(&dev_count) != hipSuccess || dev_count < 1) {
    std::printf("FAIL no HIP device\n");
    return 2;
  }
  HIP_OK(hipSetDevice(0));
  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  Workspace ws;
  bool ok = true;
  // Each case takes a different plan of the library: the decode kernel's
  // direct store, its K slices summed by the exchange tree, its K windows (more
  // slices than the tree takes: one unit per workgroup, 1024-K windows staged
  // by copy waves), a forced K split through fp32 partials, a 256-wide prefill
  // tile, the same with a K-slice combine, and the compressed-tensors kernel
  // with no repack.
  ok &= marlin_case("marlin decode, direct", Layer(1, 4096, 4096, 128, PW4_DTYPE_F16, 1), 0, ws, st, true);
  ok &= marlin_case("marlin decode, K slices", Layer(8, 1024, 14336, 128, PW4_DTYPE_BF16, 2), 0, ws, st, true);
  ok &= marlin_case("marlin decode, K windows", Layer(24, 2112, 28672, 128, PW4_DTYPE_F16, 7), 0, ws, st, true);
  ok &= marlin_case("marlin decode, forced split 3", Layer(4, 512, 4096, 128, PW4_DTYPE_F16, 3), 3, ws, st, false);
  ok &= marlin_case("marlin prefill", Layer(300, 1024, 2048, 128, PW4_DTYPE_F16, 4), 0, ws, st, true);
  ok &= marlin_case("marlin prefill, forced split 4", Layer(260, 520, 2048, 64, PW4_DTYPE_BF16, 5), 4, ws, st, false);
  ok &= ct_case("compressed-tensors, no repack", Layer(64, 512, 1024, 32, PW4_DTYPE_F16, 6), 0, ws, st);
  ok &= error_cases(ws, st);
  const bool clear = ws.zero_region_clear();
  std::printf("%-4s workspace zero region left zero after every call\n", clear ? "ok" : "FAIL");
  ok &= clear;
  if (ws.ptr) HIP_OK(hipFree(ws.ptr));
  HIP_OK(hipStreamDestroy(st));
  std::printf("%s\n", ok ? "pw4_selftest: all cases passed" : "pw4_selftest: FAILED");
  return ok ? 0 : 1;
}

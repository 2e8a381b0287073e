// Memory-bound W4A16 GEMM for small M (decode): y[M,N] = x[M,K] @ dequant(W)^T.
//
// Work split.  grid.x walks 64-column blocks, grid.y walks K slices.  A
// workgroup is 4 waves; wave w owns 16 output columns and streams its K slice
// in 128-K steps.  Per step every lane issues ONE 16-byte global load: lane
// (c = l%16, h = l/16) fetches the four words of column c in 32-K tile h,
// which are 16 contiguous bytes in both layouts, so a wave instruction reads
// four fully used 256-byte segments (MARLIN) and U steps are kept in flight.
//
// Math.  The four words feed four v_mfma_f32_16x16x32 (word s of every lane in
// step s).  B is dequantized to exact integers (u - z in fp16, or 128 + u in
// bf16 with the bias removed in fp32), accumulated per quant group in fp32,
// then scaled per group and column in fp32: no rounding of q * scale.  The x
// slice is staged once into LDS in the K order the weight words use.
//
// Reference counterpart: w4a16_marlin_kernel / gemm_w4a16_kernel at BM = 16
// (pulsar-core/src/kernels/w4a16_marlin.cu:197-304, w4a16_gemm.cu:153-264);
// its split-K partials + fixed-order combine (w4a16_common.cuh:94-120) are
// restated by combine_kernel below.
#include "w4a16_common.h"
#include "w4a16_kernels.h"

namespace pw4 {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // 128-K steps whose loads are issued ahead

template <bool BF16, int LAYOUT, typename ST, int MT, int NGRP, bool ZP>
__global__ __launch_bounds__(kThreads) void decode_kernel(const DecodeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, h = lane >> 4;
    const int cb = blockIdx.x;
    const int split = blockIdx.y;
    const int kb = split * a.k_per_split;
    const int kend_layout = a.ktiles * 32;
    const int ke = min(kb + a.k_per_split, kend_layout);
    const int M = a.M, N = a.N, K = a.K;
    const int rs = a.rowstride;
    const int ntiles = (ke - kb) / 32;  // ke - kb is a multiple of 32

    // ---- stage x[0:M, kb:ke] into LDS, permuted to the weight K order ------
    for (int i = tid; i < M * ntiles; i += kThreads) {
        const int m = i / ntiles, t = i - m * ntiles;
        const int k = kb + t * 32;
        u32x4 in[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int kk = k + p * 8;
            if (a.perm) {
                uint16_t hv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    hv[e] = (kk + e < K) ? a.x[(int64_t)m * K + min(max(a.perm[kk + e], 0), K - 1)] : (uint16_t)0;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) in[p][e] = (uint32_t)hv[2 * e] | ((uint32_t)hv[2 * e + 1] << 16);
            } else if (kk < K) {  // K % 8 == 0: pieces are all-in or all-out
                in[p] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)m * K + kk);
            } else {
                in[p] = u32x4{0u, 0u, 0u, 0u};
            }
        }
        u32x4 out[4];
        permute_tile<LAYOUT>(in, out);
        u32x4* dst = reinterpret_cast<u32x4*>(smem + m * rs + t * 32);
#pragma unroll
        for (int p = 0; p < 4; ++p) dst[p] = out[p];
    }

    // bf16: per-row, per-group sums of x to remove the +128 bias.
    float* xsum = reinterpret_cast<float*>(smem + ((M * rs + 7) & ~7));
    const int g_first = kb / a.G;
    const int ngl = (ke - 1) / a.G - g_first + 1;
    __syncthreads();
    if constexpr (BF16) {
        for (int i = tid; i < M * ngl; i += kThreads) {
            const int m = i / ngl, gl = i - m * ngl;
            const int k0 = max((g_first + gl) * a.G, kb), k1 = min((g_first + gl + 1) * a.G, ke);
            float s = 0.f;
            for (int k = k0; k < k1; ++k) {
                s += __builtin_bit_cast(float, (uint32_t)smem[m * rs + (k - kb)] << 16);
            }
            xsum[i] = s;
        }
        __syncthreads();
    }

    const int ncol = cb * 64 + wave * 16 + c;  // this lane's B column == D column
    const bool col_ok = ncol < N;
    const int nsteps = (ke - kb + 127) / 128;
    const ST* scales = reinterpret_cast<const ST*>(a.scales);
    const uint32_t wdefault = LAYOUT == LAYOUT_MARLIN ? 0x88888888u : 0u;

    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    struct Step {
        u32x4 w;
        float s[NGRP];
        uint32_t z[NGRP];
    };

    auto load_step = [&](int st, Step& o) {
        const int k0 = kb + st * 128;
        const int t = k0 / 32 + h;
        o.w = u32x4{wdefault, wdefault, wdefault, wdefault};
        if (k0 + 32 * h < ke) {
            if constexpr (LAYOUT == LAYOUT_MARLIN) {
                const int64_t off = ((int64_t)cb * a.nchunks + (t >> 1)) * kChunkWords + (t & 1) * 256 +
                                    (wave * 16 + c) * 4;
                o.w = *reinterpret_cast<const u32x4*>(a.w + off);
            } else if (col_ok) {
                const int64_t off = (int64_t)ncol * (K / 8) + t * 4;
                if ((K & 31) == 0) {
                    o.w = *reinterpret_cast<const u32x4*>(a.w + off);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) o.w[j] = (t * 32 + j * 8 < K) ? a.w[off + j] : 0u;
                }
            }
        }
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            const int g = min(k0 / a.G + gi, a.Kg - 1);
            if constexpr (LAYOUT == LAYOUT_MARLIN) {
                o.s[gi] = col_ok ? load_scale(scales + (int64_t)g * N + ncol) : 0.f;
                if constexpr (ZP) o.z[gi] = col_ok ? a.qzeros[(int64_t)g * (N >> 3) + (ncol >> 3)] : 0u;
            } else {
                o.s[gi] = col_ok ? load_scale(scales + (int64_t)ncol * a.Kg + g) : 0.f;
            }
        }
    };

    auto compute_step = [&](int st, const Step& in) {
        const int k0 = kb + st * 128;
        const int kl = k0 - kb + 32 * h;  // local K of this lane's tile
        const bool tile_ok = k0 + 32 * h < ke;
        // zero point of the group this lane's tile belongs to
        uint32_t zl[NGRP];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            if constexpr (ZP) {
                zl[gi] = (in.z[gi] >> (4 * (ncol & 7))) & 0xfu;
            } else {
                zl[gi] = 8u;
            }
        }
        const int my_gi = NGRP == 1 ? 0 : (h * NGRP) / 4;
        uint32_t zsel = zl[0];
#pragma unroll
        for (int gi = 1; gi < NGRP; ++gi) zsel = my_gi == gi ? zl[gi] : zsel;
        const uint32_t z1024 = (0x6400u | zsel) * 0x10001u;
        const uint32_t z64 = (0x5400u | (zsel << 4)) * 0x10001u;

        f32x4 tmp[NGRP][MT];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) tmp[gi][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

        const uint32_t wq[4] = {in.w[0], in.w[1], in.w[2], in.w[3]};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint32_t q = wq[s];
            if constexpr (LAYOUT == LAYOUT_CT) q ^= 0x88888888u;  // two's complement -> u
            u32x4 b;
            if constexpr (BF16) {
                b = dq_bf16_biased(q);
            } else {
                b = dq_f16_exact(q, z1024, z64);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int row = mt * 16 + c;
                u32x4 av = u32x4{0u, 0u, 0u, 0u};
                if (row < M && tile_ok) {
                    av = *reinterpret_cast<const u32x4*>(smem + row * rs + kl + 8 * s);
                }
#pragma unroll
                for (int gi = 0; gi < NGRP; ++gi) {
                    u32x4 ag = av;
                    if constexpr (NGRP > 1) {
                        if (my_gi != gi) ag = u32x4{0u, 0u, 0u, 0u};
                    }
                    tmp[gi][mt] = mfma16x16x32<BF16>(ag, b, tmp[gi][mt]);
                }
            }
        }
        // per-group fp32 scaling (and bias removal for bf16)
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            const float sc = in.s[gi];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                if constexpr (BF16) {
                    const float zf = 128.f + (float)zl[gi];
                    const int gl = k0 / a.G + gi - g_first;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int row = mt * 16 + 4 * h + j;
                        const float xs = (row < M && gl < ngl) ? xsum[row * ngl + gl] : 0.f;
                        acc[mt][j] += sc * (tmp[gi][mt][j] - zf * xs);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[mt][j] += sc * tmp[gi][mt][j];
                }
            }
        }
    };

    Step cur[kUnroll], nxt[kUnroll];
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
        if (i < nsteps) load_step(i, cur[i]);
    }
    for (int st0 = 0; st0 < nsteps; st0 += kUnroll) {
#pragma unroll
        for (int i = 0; i < kUnroll; ++i) {
            if (st0 + kUnroll + i < nsteps) load_step(st0 + kUnroll + i, nxt[i]);
        }
#pragma unroll
        for (int i = 0; i < kUnroll; ++i) {
            if (st0 + i < nsteps) compute_step(st0 + i, cur[i]);
        }
#pragma unroll
        for (int i = 0; i < kUnroll; ++i) cur[i] = nxt[i];
    }

    // ---- epilogue: D lane holds column ncol, rows 16mt + 4h + j ------------
    if (col_ok) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = mt * 16 + 4 * h + j;
                if (row < M) {
                    if (a.partial == nullptr) {
                        a.y[(int64_t)row * N + ncol] = f32_to_out<BF16>(acc[mt][j]);
                    } else {
                        a.partial[((int64_t)split * M + row) * N + ncol] = acc[mt][j];
                    }
                }
            }
        }
    }
}

// Fixed-order sum of the K-slice partials (deterministic), then the cast to
// y's dtype: the restatement of w4a16_common.cuh:97-111.
template <bool BF16>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ partial, uint16_t* __restrict__ y,
                                                      int64_t mn, int splits) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    if (i + 4 <= mn && (mn & 3) == 0) {
        f32x4 s = *reinterpret_cast<const f32x4*>(partial + i);
        for (int k = 1; k < splits; ++k) s += *reinterpret_cast<const f32x4*>(partial + (int64_t)k * mn + i);
        u32x2 o;
        o[0] = (uint32_t)f32_to_out<BF16>(s[0]) | ((uint32_t)f32_to_out<BF16>(s[1]) << 16);
        o[1] = (uint32_t)f32_to_out<BF16>(s[2]) | ((uint32_t)f32_to_out<BF16>(s[3]) << 16);
        *reinterpret_cast<u32x2*>(y + i) = o;
    } else {
        for (int64_t e = i; e < min(i + 4, mn); ++e) {
            float s = 0.f;
            for (int k = 0; k < splits; ++k) s += partial[(int64_t)k * mn + e];
            y[e] = f32_to_out<BF16>(s);
        }
    }
}

template <bool BF16, int LAYOUT, typename ST, int MT, int NGRP, bool ZP>
hipError_t launch_one(const DecodeConfig& cfg, const DecodeArgs& a, int grid_x, hipStream_t stream) {
    auto kern = decode_kernel<BF16, LAYOUT, ST, MT, NGRP, ZP>;
    if (cfg.lds_bytes > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)cfg.lds_bytes);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3(grid_x, cfg.splits), dim3(kThreads), cfg.lds_bytes, stream, a);
    return hipGetLastError();
}

template <bool BF16, int LAYOUT, typename ST, bool ZP>
hipError_t launch_mt(const DecodeConfig& cfg, const DecodeArgs& a, int grid_x, hipStream_t stream) {
#define PW4_NGRP(MT_)                                                                   \
    if (cfg.ngrp == 1) return launch_one<BF16, LAYOUT, ST, MT_, 1, ZP>(cfg, a, grid_x, stream); \
    if (cfg.ngrp == 2) return launch_one<BF16, LAYOUT, ST, MT_, 2, ZP>(cfg, a, grid_x, stream); \
    return hipErrorInvalidValue;
    switch (cfg.mt) {
        case 1: { PW4_NGRP(1) }
        case 2: { PW4_NGRP(2) }
        case 4: { PW4_NGRP(4) }
        default: return hipErrorInvalidValue;
    }
#undef PW4_NGRP
}

}  // namespace

hipError_t launch_decode(int layout, int xtype, int stype, bool zp, const DecodeConfig& cfg, const DecodeArgs& a,
                         int grid_x, hipStream_t stream) {
    const bool bf = xtype == X_BF16;
    if (layout == LAYOUT_CT) {
        if (zp || stype != S_F32) return hipErrorInvalidValue;
        return bf ? launch_mt<true, LAYOUT_CT, float, false>(cfg, a, grid_x, stream)
                  : launch_mt<false, LAYOUT_CT, float, false>(cfg, a, grid_x, stream);
    }
    if (stype == S_F32) {
        if (zp) {
            return bf ? launch_mt<true, LAYOUT_MARLIN, float, true>(cfg, a, grid_x, stream)
                      : launch_mt<false, LAYOUT_MARLIN, float, true>(cfg, a, grid_x, stream);
        }
        return bf ? launch_mt<true, LAYOUT_MARLIN, float, false>(cfg, a, grid_x, stream)
                  : launch_mt<false, LAYOUT_MARLIN, float, false>(cfg, a, grid_x, stream);
    }
    if (zp) {
        return bf ? launch_mt<true, LAYOUT_MARLIN, _Float16, true>(cfg, a, grid_x, stream)
                  : launch_mt<false, LAYOUT_MARLIN, _Float16, true>(cfg, a, grid_x, stream);
    }
    return bf ? launch_mt<true, LAYOUT_MARLIN, _Float16, false>(cfg, a, grid_x, stream)
              : launch_mt<false, LAYOUT_MARLIN, _Float16, false>(cfg, a, grid_x, stream);
}

hipError_t launch_combine(const float* partial, uint16_t* y, int64_t mn, int splits, int xtype,
                          hipStream_t stream) {
    const int64_t blocks = ceil_div(ceil_div(mn, 4), 256);
    if (blocks == 0) return hipSuccess;
    if (xtype == X_BF16) {
        hipLaunchKernelGGL(combine_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, partial, y, mn, splits);
    } else {
        hipLaunchKernelGGL(combine_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, partial, y, mn, splits);
    }
    return hipGetLastError();
}

}  // namespace pw4

// Memory-bound W4A16 GEMM for small M (decode): y[M,N] = x[M,K] @ dequant(W)^T.
//
// Work split.  grid.x walks 64-column blocks, grid.y walks K slices.  A
// workgroup is 4 waves; wave w owns 16 output columns and streams its K slice
// in 128-K steps.  Per step every lane issues ONE 16-byte global load: lane
// (c = l%16, h = l/16) fetches the four words of column c in 32-K tile h,
// which are 16 contiguous bytes in both layouts, so a wave instruction reads
// four fully used 256-byte segments (MARLIN).  The loads of the next U steps
// sit in a register ring, and the first U are issued before the activations
// are staged, so HBM latency overlaps the prologue.
//
// Math.  The four words feed four v_mfma_f32_16x16x32.  B is the biased
// integer form of the nibbles (1024 + u or 1024 + 16u in fp16, 128 + u in
// bf16: two bitwise ops per pair, exact), and the activations of the 16u
// slots are staged pre-multiplied by 1/16.  The bias and the zero point are
// removed through the accumulator's initial value: every 128-K step starts
// from -(bias * sum(a) + z * sum(a * w)) for its rows, computed in fp32 while
// staging.  Each step's result is then scaled per column in fp32, so q * scale
// is never rounded to 16 bits.
//
// K slices.  With more than one slice, every workgroup writes its fp32
// partial tile, and the last workgroup to arrive for a column block (arrival
// counter) sums the partials in slice order -- the fixed-order combine of the
// reference (w4a16_common.cuh:94-120) without a second launch -- then resets
// the counter to zero for the next call.
//
// Reference counterpart: w4a16_marlin_kernel / gemm_w4a16_kernel at BM = 16
// (pulsar-core/src/kernels/w4a16_marlin.cu:197-304, w4a16_gemm.cu:153-264).
#include "w4a16_common.h"
#include "w4a16_kernels.h"

namespace pw4 {
namespace {

constexpr int kThreads = 256;

// (a & mask) | (b & ~mask) in one v_bfi_b32.  gfx950 VOP3 takes no literal
// operand, so the compiler would spend an AND and an OR on `(q & m) | c`;
// here the mask lives in an SGPR and the splice constant in a VGPR.
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
    return r;
}

// Biased B fragment of one weight word (see dq_f16_biased / dq_bf16_biased):
// fp16 pairs 1024 + u (pairs 0, 2) and 1024 + 16u (pairs 1, 3); bf16 pairs
// 128 + u.  `one` holds the splice constant (0x64006400 or 0x43004300).
template <bool BF16, int LAYOUT>
__device__ __forceinline__ u32x4 dq_biased(uint32_t q, uint32_t one) {
    if constexpr (LAYOUT == LAYOUT_CT) q ^= 0x88888888u;  // two's complement -> u
    u32x4 r;
    if constexpr (BF16) {
        r[0] = bfi(0x000f000fu, q, one);
        r[1] = bfi(0x000f000fu, q >> 4, one);
        r[2] = bfi(0x000f000fu, q >> 8, one);
        r[3] = bfi(0x000f000fu, q >> 12, one);
    } else {
        const uint32_t q8 = q >> 8;
        r[0] = bfi(0x000f000fu, q, one);
        r[1] = bfi(0x00f000f0u, q, one);
        r[2] = bfi(0x000f000fu, q8, one);
        r[3] = bfi(0x00f000f0u, q8, one);
    }
    return r;
}

template <bool BF16>
__device__ __forceinline__ float half_lo(uint32_t d) {
    if constexpr (BF16) {
        return __builtin_bit_cast(float, d << 16);
    } else {
        return (float)as_h2(d)[0];
    }
}
template <bool BF16>
__device__ __forceinline__ float half_hi(uint32_t d) {
    if constexpr (BF16) {
        return __builtin_bit_cast(float, d & 0xffff0000u);
    } else {
        return (float)as_h2(d)[1];
    }
}

// LDS layout: x rows [M][rowstride] halves, then CP and CQ, each
// [steps][NGRP][MT*16] fp32 (CQ only with zero points).
__host__ __device__ inline size_t x_bytes(int M, int rowstride) { return ((size_t)M * rowstride * 2 + 15) / 16 * 16; }
__host__ __device__ inline size_t corr_floats(int kps, int ngrp, int mt) { return (size_t)(kps / 128) * ngrp * mt * 16; }

template <bool BF16, int LAYOUT, typename ST, int MT, int NGRP, bool ZP, int U>
__global__ __launch_bounds__(kThreads) void decode_kernel(const DecodeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ int s_last;
    constexpr int MP = MT * 16;
    constexpr float kBias = BF16 ? 128.f : 1024.f;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int c = lane & 15, h = lane >> 4;
    const int cb = blockIdx.x;
    const int split = blockIdx.y;
    const int M = a.M, N = a.N, K = a.K;
    const int rs = a.rowstride;
    const int kb = split * a.k_per_split;
    const int klen = max(min(kb + a.k_per_split, a.ktiles * 32) - kb, 0);  // multiple of 32
    const int ntiles = klen / 32;
    const int nsteps = (ntiles + 3) / 4;

    float* CP = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + x_bytes(M, rs));
    float* CQ = CP + corr_floats(a.k_per_split, NGRP, MT);

    const int ncol = cb * 64 + wave * 16 + c;  // this lane's B column == D column
    const bool col_ok = ncol < N;
    const int ncol_c = min(ncol, N - 1);       // clamped: loads stay in bounds
    const ST* scales = reinterpret_cast<const ST*>(a.scales);

    // Raw loaded values only: converting here would make the prefetch wait
    // for its own loads.
    struct Step {
        u32x4 w;
        ST s[NGRP];
        uint32_t z[NGRP];
    };
    const int gshift = a.G_log2;  // G is a power of two on this path

    // Lane part of the MARLIN word offset inside one (column block, chunk
    // pair); the chunk part is uniform and goes through scalar registers.
    // A step that runs past the layout's last chunk (Kpad % 128 == 64) points
    // its upper two tiles back at the last chunk: they meet zero activations.
    const int loff = (h >> 1) * kChunkWords + (h & 1) * 256 + (wave * 16 + c) * 4;
    const int loff_tail = (h & 1) * 256 + (wave * 16 + c) * 4;

    // ---- weight / scale / zero loads of one 128-K step ----------------------
    // Steps past the slice are clamped to its last step (a harmless re-read);
    // tiles past the slice's end are multiplied by zero activations.
    auto load_step = [&](int st, Step& o) {
        st = min(st, max(nsteps - 1, 0));
        const int k0 = kb + st * 128;
        if constexpr (LAYOUT == LAYOUT_MARLIN) {
            const int kc = min(k0 >> 6, a.nchunks - 1);  // an empty slice reads the last chunk
            const uint32_t* seg = a.w + ((int64_t)cb * a.nchunks + kc) * kChunkWords;
            o.w = *reinterpret_cast<const u32x4*>(seg + (kc + 1 < a.nchunks ? loff : loff_tail));
        } else {
            const int t = min(k0 / 32 + h, a.ktiles - 1);
            const int64_t off = (int64_t)ncol_c * (K / 8) + t * 4;
            if ((K & 31) == 0) {
                o.w = *reinterpret_cast<const u32x4*>(a.w + off);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) o.w[j] = (t * 32 + j * 8 < K) ? a.w[off + j] : 0u;
            }
        }
        const int g0 = k0 >> gshift;
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            const int g = min(g0 + gi, a.Kg - 1);
            if constexpr (LAYOUT == LAYOUT_MARLIN) {
                o.s[gi] = (scales + (int64_t)g * N)[ncol_c];
                if constexpr (ZP) o.z[gi] = (a.qzeros + (int64_t)g * (N >> 3))[ncol_c >> 3];
            } else {
                o.s[gi] = scales[(int64_t)ncol_c * a.Kg + g];
            }
        }
    };

    Step ring[U];
#pragma unroll
    for (int i = 0; i < U; ++i) load_step(i, ring[i]);

    // ---- stage x[0:M, kb:kb+klen] into LDS, permuted to the weight K order ---
    // One item = one row x one 128-K step; it also produces the step's
    // correction sums for that row.
    for (int i = tid; i < M * nsteps; i += kThreads) {
        const int m = i / nsteps, st = i - m * nsteps;
        float P[NGRP], Q[NGRP];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) P[gi] = Q[gi] = 0.f;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const int tl = st * 4 + tt;
            if (tl >= ntiles) {  // zero activations for tiles past the slice
                u32x4* dst = reinterpret_cast<u32x4*>(smem + m * rs + tl * 32);
#pragma unroll
                for (int p = 0; p < 4; ++p) dst[p] = u32x4{0u, 0u, 0u, 0u};
            } else {
                const int k = kb + tl * 32;
                u32x4 in[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int kk = k + p * 8;
                    if (a.perm) {
                        uint16_t hv[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            hv[e] = (kk + e < K) ? a.x[(int64_t)m * K + min(max(a.perm[kk + e], 0), K - 1)]
                                                 : (uint16_t)0;
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
                float sp = 0.f, sq = 0.f;
#pragma unroll
                for (int p = 0; p < 4; ++p) {
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        if constexpr (!BF16) {
                            if (d & 1) out[p][d] = as_u32(as_h2(out[p][d]) * as_h2(0x2c002c00u));  // x / 16
                        }
                        const float v = half_lo<BF16>(out[p][d]) + half_hi<BF16>(out[p][d]);
                        sp += v;
                        sq += (!BF16 && (d & 1)) ? 16.f * v : v;
                    }
                }
                const int gi = NGRP == 1 ? 0 : tt / 2;
                P[gi] += sp;
                Q[gi] += sq;
                u32x4* dst = reinterpret_cast<u32x4*>(smem + m * rs + tl * 32);
#pragma unroll
                for (int p = 0; p < 4; ++p) dst[p] = out[p];
            }
        }
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            const int idx = (st * NGRP + gi) * MP + m;
            if constexpr (ZP) {
                CP[idx] = -kBias * P[gi];
                CQ[idx] = -Q[gi];
            } else {
                CP[idx] = -(kBias * P[gi] + 8.f * Q[gi]);
            }
        }
    }
    __syncthreads();

    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // A rows past M read row M-1 (their D rows are never stored); tiles past
    // the slice read the zeros staged above.
    const uint32_t one = BF16 ? 0x43004300u : 0x64006400u;
    int arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) arow[mt] = min(mt * 16 + c, M - 1) * rs + 32 * h;

    auto compute_step = [&](int st, const Step& in) {
        const int kl = st * 128;  // local K of the step
        const int my_gi = NGRP == 1 ? 0 : h / 2;
        f32x4 tmp[NGRP][MT];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            float zf = 8.f;
            if constexpr (ZP) zf = (float)((in.z[gi] >> (4 * (ncol_c & 7))) & 0xfu);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int idx = (st * NGRP + gi) * MP + mt * 16 + 4 * h;
                const f32x4 cp = *reinterpret_cast<const f32x4*>(CP + idx);
                if constexpr (ZP) {
                    const f32x4 cq = *reinterpret_cast<const f32x4*>(CQ + idx);
#pragma unroll
                    for (int j = 0; j < 4; ++j) tmp[gi][mt][j] = cp[j] + zf * cq[j];
                } else {
                    tmp[gi][mt] = cp;
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const u32x4 b = dq_biased<BF16, LAYOUT>(in.w[s], one);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const u32x4 av = *reinterpret_cast<const u32x4*>(smem + arow[mt] + kl + 8 * s);
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
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[mt][j] += load_scale(&in.s[gi]) * tmp[gi][mt][j];
    };

    // Full blocks of U steps: unconditional refills (clamped past the end) so
    // the ring registers are written by the loads themselves, never through a
    // branch join that would force a wait.  Then the tail, without refills.
    int st0 = 0;
    for (; st0 + U <= nsteps; st0 += U) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            compute_step(st0 + i, ring[i]);
            load_step(st0 + i + U, ring[i]);
            // keep the refill right behind its step: without the barrier the
            // scheduler batches all U computes first and drains the ring
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < U; ++i) {
        if (st0 + i < nsteps) compute_step(st0 + i, ring[i]);
    }

    // ---- epilogue: D lane holds column ncol, rows 16mt + 4h + j ------------
    if (a.partial == nullptr) {
        if (col_ok) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = mt * 16 + 4 * h + j;
                    if (row < M) a.y[(int64_t)row * N + ncol] = f32_to_out<BF16>(acc[mt][j]);
                }
        }
        return;
    }
    // Cross-workgroup hand-off without an L2 write-back.  The partials travel
    // as device-scope atomic stores and loads (sc1: written through to, and
    // read from, the device coherence point), and the arrival counter is a
    // device-scope atomic.  Every wave waits for its partial stores to be
    // acknowledged (vmcnt 0) before the barrier that precedes the counter
    // increment, so whoever sees the last arrival also sees every partial.
    // Agent-scope fences would be equivalent but write back the whole L2.
    float* part = a.partial + ((int64_t)cb * a.splits + split) * M * 64;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = mt * 16 + 4 * h + j;
            if (row < M)
                __hip_atomic_store(part + row * 64 + wave * 16 + c, acc[mt][j], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        s_last = __hip_atomic_fetch_add(a.counters + cb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 a.splits - 1;
    }
    __syncthreads();
    if (!s_last) return;
    const float* base = a.partial + (int64_t)cb * a.splits * M * 64;
    for (int i = tid; i < M * 64; i += kThreads) {
        float s = 0.f;
        for (int sp = 0; sp < a.splits; ++sp) {
            s += __hip_atomic_load(base + (int64_t)sp * M * 64 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const int row = i >> 6, col = cb * 64 + (i & 63);
        if (col < N) a.y[(int64_t)row * N + col] = f32_to_out<BF16>(s);
    }
    if (tid == 0) __hip_atomic_store(a.counters + cb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kRing = 8;

template <bool BF16, int LAYOUT, typename ST, int MT, int NGRP, bool ZP>
hipError_t launch_one(const DecodeConfig& cfg, const DecodeArgs& a, int grid_x, hipStream_t stream) {
    auto kern = decode_kernel<BF16, LAYOUT, ST, MT, NGRP, ZP, kRing>;
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
#define PW4_NGRP(MT_)                                                                               \
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

// Fixed-order sum of [splits, M, N] fp32 partials, then the cast to y's dtype
// (the prefill path's split-K combine; restates w4a16_common.cuh:97-111).
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

}  // namespace

size_t decode_lds_bytes(int M, int kps, int ngrp, bool zp) {
    const int mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    return x_bytes(M, kps + 8) + corr_floats(kps, ngrp, mt) * 4 * (zp ? 2 : 1);
}

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

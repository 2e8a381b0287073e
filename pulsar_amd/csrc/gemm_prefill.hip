// Compute-bound W4A16 GEMM for large M (prefill): y[M,N] = x[M,K] @ dequant(W)^T.
//
// Tiling.  A workgroup (4 waves, 2 x 2) owns a 128 x 128 output tile and walks
// K in 64-wide chunks (one MARLIN chunk: two 32-K tiles).  Each wave computes
// 64 x 64 with 2 x 2 v_mfma_f32_32x32x16 accumulators.  The x tile (permuted
// to the weight K order, rows padded to 144 B so the 16-byte LDS reads are
// conflict free) and the packed int4 weight tile are double buffered in LDS;
// the next chunk's global loads are in flight while the current chunk's
// MFMAs run.  Weights stay int4 in LDS and are dequantized into B registers
// right before the MFMA, with the group scale folded in (one fp16 rounding,
// as the reference does in w4a16_marlin.cu:103-126).
//
// Lane map for a 32-K tile: lane (c = l%32, h = l/32) in MFMA step s uses
// weight word tg = 2h + s of column c (an 8-byte LDS read covers both steps)
// and the matching 16 bytes of the permuted x row.
//
// Reference counterpart: gemm_w4a16_kernel / w4a16_marlin_kernel at BM = 64
// (w4a16_gemm.cu:153-264, w4a16_marlin.cu:197-304).
#include "w4a16_common.h"
#include "w4a16_kernels.h"

namespace pw4 {
namespace {

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 64;
constexpr int AROW = BK + 8;          // halves per staged x row (144 bytes)
constexpr int CT_BROW = 10;           // words per staged CT weight column (8 + 2 pad)
constexpr int B_WORDS_MARLIN = 2 * kChunkWords;
constexpr int B_WORDS_CT = BN * CT_BROW;

template <int LAYOUT>
constexpr int b_words() {
    return LAYOUT == LAYOUT_MARLIN ? B_WORDS_MARLIN : B_WORDS_CT;
}

template <bool BF16, int LAYOUT, typename ST, bool ZP>
__global__ __launch_bounds__(kThreads) void prefill_kernel(const PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * AROW];
    __shared__ __attribute__((aligned(16))) uint32_t sB[2][b_words<LAYOUT>()];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int c = lane & 31, h = lane >> 5;
    const int M = a.M, N = a.N, K = a.K;

    // ---- tile order: XCD-aware, then grouped along M for L2 reuse ----------
    const int num_m = (int)ceil_div(M, BM), num_n = (int)ceil_div(N, BN);
    const int nwg = num_m * num_n;
    int pid = blockIdx.x;
    if ((nwg & 7) == 0) pid = (pid & 7) * (nwg >> 3) + (pid >> 3);  // consecutive tiles share an XCD
    constexpr int GM = 8;
    const int group = pid / (GM * num_n);
    const int first_m = group * GM;
    const int gsz = min(num_m - first_m, GM);
    const int in_group = pid - group * GM * num_n;
    const int tile_m = first_m + in_group % gsz;
    const int tile_n = in_group / gsz;
    const int m0 = tile_m * BM, n0 = tile_n * BN;

    const int split = blockIdx.z;
    const int c_begin = split * a.chunks_per_split;
    const int c_end = min(c_begin + a.chunks_per_split, a.nchunks);

    const ST* scales = reinterpret_cast<const ST*>(a.scales);
    const uint32_t wdefault = LAYOUT == LAYOUT_MARLIN ? 0x88888888u : 0u;

    // ---- global -> register staging for one chunk --------------------------
    // x: thread (row = tid/2, t = tid%2) owns one 32-K tile row (64 bytes).
    const int a_row = tid >> 1, a_t = tid & 1;
    u32x4 ra[4];
    u32x4 rb;
    auto load_chunk = [&](int kc) {
        const int gm = m0 + a_row;
        const int k = kc * BK + a_t * 32;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int kk = k + p * 8;
            ra[p] = (gm < M && kk < K) ? *reinterpret_cast<const u32x4*>(a.x + (int64_t)gm * K + kk)
                                       : u32x4{0u, 0u, 0u, 0u};
        }
        rb = u32x4{wdefault, wdefault, wdefault, wdefault};
        if constexpr (LAYOUT == LAYOUT_MARLIN) {
            const int cbl = tid >> 7;
            const int cbg = n0 / kMarlinBN + cbl;
            if (cbg * kMarlinBN < round_up(N, kMarlinBN)) {
                const int64_t off = ((int64_t)cbg * a.nchunks + kc) * kChunkWords + (tid & 127) * 4;
                rb = *reinterpret_cast<const u32x4*>(a.w + off);
            }
        } else {
            const int col = tid >> 1, half = tid & 1;
            const int n = n0 + col;
            const int kt = kc * BK + half * 32;
            if (n < N && kt < K) {
                const int64_t off = (int64_t)n * (K / 8) + kt / 8;
                if ((K & 31) == 0) {
                    rb = *reinterpret_cast<const u32x4*>(a.w + off);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) rb[j] = (kt + j * 8 < K) ? a.w[off + j] : 0u;
                }
            }
        }
    };
    auto store_chunk = [&](int buf) {
        u32x4 out[4];
        permute_tile<LAYOUT>(ra, out);
        u32x4* dst = reinterpret_cast<u32x4*>(&sA[buf][a_row * AROW + a_t * 32]);
#pragma unroll
        for (int p = 0; p < 4; ++p) dst[p] = out[p];
        if constexpr (LAYOUT == LAYOUT_MARLIN) {
            *reinterpret_cast<u32x4*>(&sB[buf][tid * 4]) = rb;
        } else {
            const int col = tid >> 1, half = tid & 1;
            uint32_t* d = &sB[buf][col * CT_BROW + half * 4];
            *reinterpret_cast<u32x2*>(d) = u32x2{rb[0], rb[1]};
            *reinterpret_cast<u32x2*>(d + 2) = u32x2{rb[2], rb[3]};
        }
    };

    // ---- per-chunk scale / zero values for this lane's two columns ----------
    // [t][half][nt]: groups of K offsets 32t + 16*half of the chunk.
    float sv[2][2][2];
    uint32_t zv[2][2][2];
    auto load_scales = [&](int kc) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int n = n0 + wn * 64 + nt * 32 + c;
            const bool ok = n < N;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int g = min((kc * BK + t * 32 + hf * 16) / a.G, a.Kg - 1);
                    if constexpr (LAYOUT == LAYOUT_MARLIN) {
                        sv[t][hf][nt] = ok ? load_scale(scales + (int64_t)g * N + n) : 0.f;
                        if constexpr (ZP) {
                            const uint32_t zw = ok ? a.qzeros[(int64_t)g * (N >> 3) + (n >> 3)] : 0u;
                            zv[t][hf][nt] = (zw >> (4 * (n & 7))) & 0xfu;
                        } else {
                            zv[t][hf][nt] = 8u;
                        }
                    } else {
                        sv[t][hf][nt] = ok ? load_scale(scales + (int64_t)n * a.Kg + g) : 0.f;
                        zv[t][hf][nt] = 8u;
                    }
                }
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    auto compute_chunk = [&](int buf) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            u32x4 av[2][2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const int row = wm * 64 + mt * 32 + c;
                const u32x4* src = reinterpret_cast<const u32x4*>(&sA[buf][row * AROW + t * 32 + h * 16]);
                av[mt][0] = src[0];
                av[mt][1] = src[1];
            }
            u32x4 bv[2][2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int col = wn * 64 + nt * 32 + c;
                u32x2 q;
                if constexpr (LAYOUT == LAYOUT_MARLIN) {
                    const int cbl = col >> 6, c64 = col & 63;
                    q = *reinterpret_cast<const u32x2*>(&sB[buf][cbl * kChunkWords + t * 256 + c64 * 4 + 2 * h]);
                } else {
                    q = *reinterpret_cast<const u32x2*>(&sB[buf][col * CT_BROW + t * 4 + 2 * h]);
                    q[0] ^= 0x88888888u;
                    q[1] ^= 0x88888888u;
                }
                // scale / zero per 16-K half this lane's pairs fall in
                float s_lo, s_hi;
                uint32_t z_lo, z_hi;
                if constexpr (LAYOUT == LAYOUT_MARLIN) {
                    s_lo = sv[t][0][nt];
                    s_hi = sv[t][1][nt];
                    z_lo = zv[t][0][nt];
                    z_hi = zv[t][1][nt];
                } else {  // CT words 2h, 2h+1 lie entirely in half h
                    s_lo = s_hi = sv[t][h][nt];
                    z_lo = z_hi = 8u;
                }
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    if constexpr (BF16) {
                        // per-half zero handled through zf; halves share a zero unless G == 16
                        u32x4 lo = dq_bf16_scaled(q[s], 128.f + (float)z_lo, s_lo, s_lo);
                        if (z_lo != z_hi || s_lo != s_hi) {
                            const u32x4 hi = dq_bf16_scaled(q[s], 128.f + (float)z_hi, s_hi, s_hi);
                            lo[2] = hi[2];
                            lo[3] = hi[3];
                        }
                        bv[nt][s] = lo;
                    } else {
                        const f16x2 slo2 = f16x2{(_Float16)s_lo, (_Float16)s_lo};
                        const f16x2 shi2 = f16x2{(_Float16)s_hi, (_Float16)s_hi};
                        u32x4 r = dq_f16_scaled(q[s], (0x6400u | z_lo) * 0x10001u,
                                                (0x5400u | (z_lo << 4)) * 0x10001u, slo2, shi2);
                        if (ZP && z_lo != z_hi) {
                            const u32x4 r2 = dq_f16_scaled(q[s], (0x6400u | z_hi) * 0x10001u,
                                                           (0x5400u | (z_hi << 4)) * 0x10001u, slo2, shi2);
                            r[2] = r2[2];
                            r[3] = r2[3];
                        }
                        bv[nt][s] = r;
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mfma32x32x16<BF16>(av[mt][s], bv[nt][s], acc[mt][nt]);
        }
    };

    if (c_begin < c_end) {
        load_chunk(c_begin);
        load_scales(c_begin);
        store_chunk(0);
        __syncthreads();
        int buf = 0;
        for (int kc = c_begin; kc < c_end; ++kc) {
            const bool more = kc + 1 < c_end;
            if (more) load_chunk(kc + 1);
            compute_chunk(buf);
            if (more) {
                store_chunk(buf ^ 1);
                load_scales(kc + 1);
            }
            __syncthreads();
            buf ^= 1;
        }
    }

    // ---- epilogue: D lane holds column c, rows 8*(e/4) + 4h + e%4 -----------
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int n = n0 + wn * 64 + nt * 32 + c;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * 64 + mt * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                if (m < M) {
                    if (a.partial == nullptr) {
                        a.y[(int64_t)m * N + n] = f32_to_out<BF16>(acc[mt][nt][e]);
                        if (a.y32) a.y32[(int64_t)m * N + n] = acc[mt][nt][e];
                    } else {
                        a.partial[((int64_t)split * M + m) * N + n] = acc[mt][nt][e];
                    }
                }
            }
        }
}

// x_out[m, j..j+8) = x[m, perm[j..j+8)]: one 16-byte store per thread (K % 8
// == 0 on every path; the output is a 256-byte aligned workspace).  The 8
// element reads of a thread are independent, so they are in flight together.
__global__ __launch_bounds__(256) void gather_x_kernel(const uint16_t* __restrict__ x, const int32_t* __restrict__ perm,
                                                       uint16_t* __restrict__ out, int M, int K) {
    const int k8 = K >> 3;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)M * k8) return;
    const int64_t m = i / k8;
    const int j = (int)(i - m * k8) * 8;
    int idx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) idx[e] = perm[j + e];
    const uint16_t* row = x + m * K;
    uint32_t v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t lo = row[min(max(idx[2 * e], 0), K - 1)];  // clamped: a bad perm cannot fault
        const uint32_t hi = row[min(max(idx[2 * e + 1], 0), K - 1)];
        v[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(out + m * K + j) = make_uint4(v[0], v[1], v[2], v[3]);
}

// The same gather with the source row staged in LDS: workgroup (m, s) copies
// row m of x into LDS with 16-byte loads, then writes outputs
// [s * kseg, (s + 1) * kseg) of the row from LDS.  The direct gather above
// sends every element read to the address path as its own cache line (a
// random permutation scatters a wave's 64 reads over the whole row); staged,
// HBM sees the row once and the scattered reads are LDS reads.  Needs a
// 16-byte aligned x and K * 2 bytes of LDS (checked at launch).
constexpr int kGatherThreads = 256;
__global__ __launch_bounds__(kGatherThreads) void gather_x_lds_kernel(const uint16_t* __restrict__ x,
                                                                      const int32_t* __restrict__ perm,
                                                                      uint16_t* __restrict__ out, int K, int kseg) {
    extern __shared__ __attribute__((aligned(16))) uint16_t srow[];
    const int64_t m = blockIdx.x;
    const int k8 = K >> 3;
    const uint4* src = reinterpret_cast<const uint4*>(x + m * K);
    for (int i = threadIdx.x; i < k8; i += kGatherThreads) reinterpret_cast<uint4*>(srow)[i] = src[i];
    __syncthreads();
    const int j_end = min((int)(blockIdx.y + 1) * kseg, K);
    for (int j = (int)blockIdx.y * kseg + threadIdx.x * 8; j < j_end; j += kGatherThreads * 8) {
        const int4 p0 = *reinterpret_cast<const int4*>(perm + j);
        const int4 p1 = *reinterpret_cast<const int4*>(perm + j + 4);
        const int idx[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        uint32_t v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = srow[min(max(idx[2 * e], 0), K - 1)];  // clamped: a bad perm cannot fault
            const uint32_t hi = srow[min(max(idx[2 * e + 1], 0), K - 1)];
            v[e] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4*>(out + m * K + j) = make_uint4(v[0], v[1], v[2], v[3]);
    }
}

template <bool BF16, int LAYOUT, typename ST, bool ZP>
hipError_t launch_one(const PrefillArgs& a, hipStream_t stream, KernelEvents ev) {
    const int nwg = (int)(ceil_div(a.M, BM) * ceil_div(a.N, BN));
    launch_kernel(prefill_kernel<BF16, LAYOUT, ST, ZP>, dim3(nwg, 1, a.splits), dim3(kThreads), 0, stream, ev.start,
                  ev.stop, a);
    return hipGetLastError();
}

}  // namespace

int prefill_tile_m() { return BM; }
int prefill_tile_n() { return BN; }

hipError_t launch_prefill(int layout, int xtype, int stype, bool zp, const PrefillArgs& a, hipStream_t stream,
                          KernelEvents ev) {
    const bool bf = xtype == X_BF16;
    if (layout == LAYOUT_CT) {
        if (zp || stype != S_F32) return hipErrorInvalidValue;
        return bf ? launch_one<true, LAYOUT_CT, float, false>(a, stream, ev)
                  : launch_one<false, LAYOUT_CT, float, false>(a, stream, ev);
    }
    if (stype == S_F32) {
        if (zp) return bf ? launch_one<true, LAYOUT_MARLIN, float, true>(a, stream, ev)
                          : launch_one<false, LAYOUT_MARLIN, float, true>(a, stream, ev);
        return bf ? launch_one<true, LAYOUT_MARLIN, float, false>(a, stream, ev)
                  : launch_one<false, LAYOUT_MARLIN, float, false>(a, stream, ev);
    }
    if (zp) return bf ? launch_one<true, LAYOUT_MARLIN, _Float16, true>(a, stream, ev)
                      : launch_one<false, LAYOUT_MARLIN, _Float16, true>(a, stream, ev);
    return bf ? launch_one<true, LAYOUT_MARLIN, _Float16, false>(a, stream, ev)
              : launch_one<false, LAYOUT_MARLIN, _Float16, false>(a, stream, ev);
}

hipError_t launch_gather_x(const uint16_t* x, const int32_t* perm, uint16_t* out, int M, int K, hipStream_t stream,
                           int staged) {
    if (K % 8 != 0) return hipErrorInvalidValue;
    const int64_t n = (int64_t)M * (K / 8);
    if (n == 0) return hipSuccess;
    const bool fits = K * 2 <= 65536 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)perm & 15) == 0 &&
                      ((uintptr_t)out & 15) == 0 && M <= 65535;
    if (staged < 0) staged = M > kGatherStagedMinM;
    if (staged && fits) {
        // about 512 workgroups, each segment at least one pass of the block
        const int ksplit = (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div(512, M), K / (kGatherThreads * 8)));
        const int kseg = (int)ceil_div(ceil_div(K, ksplit), 8) * 8;
        hipLaunchKernelGGL(gather_x_lds_kernel, dim3((unsigned)M, (unsigned)ceil_div(K, kseg)), dim3(kGatherThreads),
                           (size_t)K * 2, stream, x, perm, out, K, kseg);
    } else {
        hipLaunchKernelGGL(gather_x_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, stream, x, perm, out, M,
                           K);
    }
    return hipGetLastError();
}

}  // namespace pw4

// Compute-bound W4A16 GEMM for large M on the MARLIN layout with fp16
// activations: y[M,N] = x[M,K] @ dequant(W)^T, 256 x 256 output tile per
// workgroup.
//
// Tiling.  Four waves; wave w owns MARLIN column block w of the tile (64
// columns) for all 256 rows: 8 x 2 tiles of v_mfma_f32_32x32x16_f16 with the
// fp32 accumulators in AGPRs.  Splitting the tile by columns means every
// weight nibble is dequantized exactly once per workgroup; the activation
// tile is read from LDS by all four waves instead.  K advances in 64-wide
// chunks (one MARLIN chunk per column block).
//
// Pipeline.  Three LDS stages of (activations 32 KB, packed weights 8 KB,
// scales, zero points), filled with global_load_lds (no VGPRs; each lane
// names its own global address, the 64 lanes of an instruction fill 64
// consecutive LDS elements).  The copies are issued from inline assembly so
// that the compiler does not serialise them: it would otherwise wait for
// every outstanding LDS copy before each LDS read.  The kernel counts them
// itself instead: every wave issues the same number of copies per chunk, so
// "chunk i has landed" is vmcnt <= (copies of chunk i+1), then a barrier.
// Activation rows are XOR-swizzled in 16-byte units (chunk ^ ((row >> 1) & 7)):
// rows r and r + 8 of one ds_read_b128 land on different banks.  gfx950 counts
// no LDS bank conflicts with this swizzle; with chunk ^ (row & 7) it counted
// 43% of LDS-active cycles as conflict stalls (SQ_LDS_BANK_CONFLICT, gate_up
// at M = 4096).
//
// Dequant.  Pair p of MARLIN word tg (nibbles p, p+4) holds natural K
// {8p + 2tg, 8p + 2tg + 1}, so pair p of a column's four words is the K run
// [8p, 8p + 8) -- exactly what one lane supplies to an MFMA.  fp16 x, per
// pair: shift, splice into 1024.0 (exact 1024 + u), subtract 1024 + z
// (exact), times the group scale (one fp16 rounding, as the reference's
// dequant_scale, w4a16_marlin.cu:103-113).  bf16 x (gfx950 has no packed bf16
// arithmetic): splice into 128.0 (exact 128 + u), then per value one fp32 fma
// (128 + u) * s - (128 + z) * s with s the scale rounded to bf16 -- both
// products are exact in fp32 -- and one v_cvt_pk_bf16_f32 per pair: the
// reference's bf16 fragment round(q * round(s)) bit for bit
// (w4a16_marlin.cu:115-126).
//
// Exact scaling (fp16 x, 128-row tiles).  Rounding (u - z) * s to fp16 costs
// up to 2^-11 of every weight; summed over K = 14336-28672 that is ~1e-2 of
// absolute error at the BASELINE magnitudes.  In this mode B = u - z (exact in
// fp16) and the group scale is applied in fp32 to the accumulators instead:
// with s_g the scale of group g for the lane's column, the running sum is
// rescaled by s_(g-1) / s_g when group g starts and multiplied by the last
// group's scale at the end, so acc = sum_g s_g * P_g with P_g the exact
// fp32 sum of group g.  One multiply per accumulator per group (the
// accumulators are VGPRs here), and no second accumulator set.
//
// Reference counterpart: w4a16_marlin_kernel at BM = 64
// (pulsar-core/src/kernels/w4a16_marlin.cu:197-304).
#include <algorithm>

#include "w4a16_common.h"
#include "w4a16_kernels.h"

namespace pw4 {
namespace {

constexpr int kT = 256;
constexpr int TM = 256, TN = 256, TK = 64;  // full tile; the tail variant has TM = 128
constexpr int kStages = 3;
constexpr int kBStage = TN * TK / 2;
constexpr int kSStage = 4 * 256;      // per wave 256 bytes of scales (64 fp32, or 64 fp16 + pad)
constexpr int kZStage = 4 * 256;      // per wave 256 bytes of zero-point words (8 used)

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)p;
}

// One LDS copy instruction: lane l copies 16 (or 4) bytes from g to
// LDS[lds + l * 16 (or 4)].  M0 (the LDS base) is saved and restored around
// it; the s_nop covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ void lds_copy16(const void* g, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(lds)
        : "memory");
}
__device__ __forceinline__ void lds_copy4(const void* g, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(lds)
        : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Scales below this magnitude (zero included) count as this value, with their
// sign, in exact mode: the group then contributes ~2^-64 of its sum instead of
// nothing, and the ratio of two scales stays finite.
constexpr float kMinScale = 0x1p-64f;

__device__ __forceinline__ float exact_scale(float s) {
    return __builtin_fabsf(s) < kMinScale ? __builtin_copysignf(kMinScale, s) : s;
}

// RT = 32-row MFMA tiles per wave: 8 (256-row tile) or 4 (128-row tile, for
// the N columns of the last wave, every tile of a 128-row plan, and exact
// scaling; see launch_prefill256).
// 128-row tiles (RT = 4) use 78 KB of LDS, so two workgroups fit on a CU if
// each wave keeps to 256 registers (two waves per SIMD).
template <bool BF16, typename ST, bool ZP, bool PARTIAL, int RT, bool EXACT = false>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(RT == 4 ? 2 : 1, RT == 4 ? 2 : 1)))
void prefill256_kernel(const PrefillArgs a, const NibbleMasks mk) {
    static_assert(!EXACT || (!BF16 && RT == 4), "exact scaling: fp16 activations, 128-row tiles");
    constexpr int TMR = 32 * RT;                 // rows of this tile
    constexpr int kAStage = TMR * TK * 2;        // bytes
    __shared__ __attribute__((aligned(16))) uint8_t sA[kStages][kAStage];
    __shared__ __attribute__((aligned(16))) uint8_t sB[kStages][kBStage];
    __shared__ __attribute__((aligned(16))) uint8_t sS[kStages][kSStage];
    __shared__ __attribute__((aligned(16))) uint8_t sZ[kStages][kZStage];
    // copies per wave per chunk: RT activation, 2 weight, 1 scale, 1 zero point
    constexpr int kCopies = RT + 2 + 1 + (ZP ? 1 : 0);

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int c = lane & 31, hb = lane >> 5;
    const int M = a.M, N = a.N, K = a.K;

    // ---- tile order: XCD-aware, then grouped along M for L2 reuse ----------
    // this launch covers columns [n_begin, n_end) of the output
    const int num_m = (M + TMR - 1) / TMR, num_n = (a.n_end - a.n_begin + TN - 1) / TN;
    const int nwg = num_m * num_n;
    int pid = blockIdx.x;
    if ((nwg & 7) == 0) pid = (pid & 7) * (nwg >> 3) + (pid >> 3);  // consecutive tiles share an XCD
    constexpr int GM = 4;
    const int group = pid / (GM * num_n);
    const int first_m = group * GM;
    const int gsz = min(num_m - first_m, GM);
    const int in_group = pid - group * GM * num_n;
    const int m0 = (first_m + in_group % gsz) * TMR;
    const int n0 = a.n_begin + (in_group / gsz) * TN;

    const int split = blockIdx.z;
    const int c_begin = split * a.chunks_per_split;
    const int c_end = min(c_begin + a.chunks_per_split, a.nchunks);
    const int nck = max(c_end - c_begin, 0);

    const int ncb = (N + 63) / 64;              // MARLIN column blocks present
    const int cbw = min(n0 / 64 + wave, ncb - 1);  // this wave's block (clamped: junk columns are never stored)
    const int ncol0 = n0 + wave * 64;           // first column of this wave
    const ST* scales = reinterpret_cast<const ST*>(a.scales);

    // ---- copies of one chunk into a stage (unconditional: constant count) ---
    // Rows past M, columns past N read clamped addresses; their results are
    // never stored.
    auto issue = [&](int kc, int st) {
        const uint32_t abase = lds_addr(&sA[st][0]) + wave * RT * 1024;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const int row = wave * (8 * RT) + i * 8 + (lane >> 3);
            const int kch = (lane & 7) ^ ((row >> 1) & 7);
            const int gm = min(m0 + row, M - 1);
            lds_copy16(a.x + (int64_t)gm * K + kc * TK + kch * 8, abase + i * 64 * 16);
        }
        const uint32_t* wsrc = a.w + ((int64_t)cbw * a.nchunks + kc) * kChunkWords;
        const uint32_t bbase = lds_addr(&sB[st][0]) + wave * 2048;
#pragma unroll
        for (int i = 0; i < 2; ++i) lds_copy16(wsrc + (i * 64 + lane) * 4, bbase + i * 1024);
        const int g = min(kc * TK / a.G, a.Kg - 1);
        const uint32_t sbase = lds_addr(&sS[st][0]) + wave * 256;
        if constexpr (sizeof(ST) == 4) {
            lds_copy4(scales + (int64_t)g * N + min(ncol0 + lane, N - 1), sbase);
        } else {
            lds_copy4(scales + (int64_t)g * N + min(ncol0 + 2 * lane, N - 2), sbase);  // N even
        }
        if constexpr (ZP) {
            const int nw = N / 8;
            lds_copy4(a.qzeros + (int64_t)g * nw + min(ncol0 / 8 + lane, nw - 1), lds_addr(&sZ[st][0]) + wave * 256);
        }
    };

    f32x16 acc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[rt][ct][e] = 0.f;

    // splice constant in a VGPR (the mask comes in an SGPR): one v_and_or_b32
    uint32_t one;
    asm volatile("v_mov_b32 %0, %1" : "=v"(one) : "s"(BF16 ? 0x43004300u : 0x64006400u));

    // exact mode: the effective scale of the group the accumulators are in,
    // per column tile (1 until the first chunk; an empty slice stores 0 * 1)
    float s_run[2] = {1.f, 1.f};

    // One chunk = four 16-K steps; step s is pair s % 2 of 32-K tile s / 2, and
    // this lane's K run in it is [16s + 8hb, +8): activation 16-byte unit
    // 2s + hb, weight nibble pair 2(s % 2) + hb.  Operands of step s + 1 (eight
    // A fragments, the dequantized B) are fetched while step s's 16 MFMAs run.
    // new_group (exact mode): this chunk starts a quant group after another one.
    auto compute = [&](int st, bool new_group) {
        const uint8_t* A = &sA[st][0];
        const uint8_t* B = &sB[st][0] + wave * 2048;
        u32x4 wq[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) wq[t][ct] = *reinterpret_cast<const u32x4*>(B + t * 1024 + (ct * 32 + c) * 16);
        f16x2 s2[2], z2[2];   // fp16: scale, 1024 + z
        float sb[2], cz[2];   // bf16: scale rounded to bf16, -(128 + z) * scale
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int cl = ct * 32 + c;  // column inside the wave's block
            float sf;
            if constexpr (sizeof(ST) == 4) {
                sf = *reinterpret_cast<const float*>(&sS[st][wave * 256 + cl * 4]);
            } else {
                sf = (float)*reinterpret_cast<const _Float16*>(&sS[st][wave * 256 + cl * 2]);
            }
            uint32_t z = 8u;
            if constexpr (ZP) z = (*reinterpret_cast<const uint32_t*>(&sZ[st][wave * 256 + (cl >> 3) * 4]) >> (4 * (cl & 7))) & 0xfu;
            if constexpr (BF16) {
                sb[ct] = (float)(__bf16)sf;
                cz[ct] = -(128.f + (float)z) * sb[ct];
            } else if constexpr (EXACT) {
                z2[ct] = as_h2((0x6400u | z) * 0x10001u);  // 1024 + z
                const float se = exact_scale(sf);
                if (new_group) {
                    const float r = s_run[ct] / se;
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                        for (int e = 0; e < 16; ++e) acc[rt][ct][e] *= r;
                }
                s_run[ct] = se;
            } else {
                const _Float16 sh = (_Float16)sf;
                s2[ct] = f16x2{sh, sh};
                z2[ct] = as_h2((0x6400u | z) * 0x10001u);  // 1024 + z
            }
        }
        auto load_a = [&](int s, u32x4 (&av)[RT]) {
            const int kch = 2 * s + hb;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int row = rt * 32 + c;
                av[rt] = *reinterpret_cast<const u32x4*>(A + row * (TK * 2) + ((kch ^ ((row >> 1) & 7)) * 16));
            }
        };
        auto dequant = [&](int s, u32x4 (&bv)[2]) {
            const int sh = 8 * (s & 1) + 4 * hb;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int tg = 0; tg < 4; ++tg) {
                    const uint32_t v = ((wq[s >> 1][ct][tg] >> sh) & mk.lo) | one;
                    if constexpr (BF16) {
                        bv[ct][tg] = pack_bf16x2_rne(__builtin_fmaf(__builtin_bit_cast(float, v << 16), sb[ct], cz[ct]),
                                                     __builtin_fmaf(__builtin_bit_cast(float, v & 0xffff0000u), sb[ct],
                                                                    cz[ct]));
                    } else if constexpr (EXACT) {
                        bv[ct][tg] = as_u32(as_h2(v) - z2[ct]);  // u - z, exact
                    } else {
                        bv[ct][tg] = as_u32((as_h2(v) - z2[ct]) * s2[ct]);
                    }
                }
        };
        u32x4 av[2][RT], bv[2][2];
        load_a(0, av[0]);
        dequant(0, bv[0]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int cur = s & 1;
            if (s < 3) {
                load_a(s + 1, av[cur ^ 1]);
                dequant(s + 1, bv[cur ^ 1]);
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) acc[rt][ct] = mfma32x32x16<BF16>(av[cur][rt], bv[cur][ct], acc[rt][ct]);
            // interleave (256-row tiles, one workgroup per CU): per A fragment of
            // the next step, two MFMAs and its dequant share.  128-row tiles run
            // two workgroups per CU, whose waves cover each other's latency; the
            // compiler's own schedule is faster there (measured 3-10%).
            if (RT == 8 && s < 3) {
#pragma unroll
                for (int i = 0; i < RT; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);         // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, (BF16 ? 56 : 32) / RT, 0);  // VALU
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if (nck > 0) issue(c_begin, 0);
    if (nck > 1) issue(c_begin + 1, 1);
    // position of the chunk in its quant group (G is a multiple of 64)
    const int cpg = a.G / TK;
    int gk = EXACT ? c_begin % cpg : 0;
    for (int i = 0; i < nck; ++i) {
        const int st = i % kStages;
        if (i + 1 < nck) {
            wait_vmcnt<kCopies>();  // this wave's copies of chunk i have landed
        } else {
            wait_vmcnt<0>();
        }
        __syncthreads();            // everyone's have; everyone is done with chunk i - 1
        if (i + 2 < nck) issue(c_begin + i + 2, (i + 2) % kStages);
        compute(st, i > 0 && gk == 0);
        if constexpr (EXACT) gk = gk + 1 == cpg ? 0 : gk + 1;
    }
    if constexpr (EXACT) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[rt][ct][e] *= s_run[ct];
    }

    // ---- epilogue: D lane holds column c, rows 8*(e/4) + 4*hb + e%4 ---------
    // Range-checked buffer stores: the resource covers rows [m0, M) of the
    // output (below 2 GiB), so rows past M are dropped by the hardware; lanes
    // whose column is past N start at 2 GiB, beyond the range.
    const int rows = min(M - m0, TMR);
    if constexpr (!PARTIAL) {
        if (a.silu) {
            // gate|up interleaved by 8: a gate lane (column c % 16 < 8) takes its
            // up value from lane ^ 8 (column c + 8, same rows) and stores
            // silu(gate) * up into y [M, N/2]; up lanes store nothing
            const int nh = N >> 1;
            const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(a.y + (int64_t)m0 * nh, (short)0,
                                                                                rows * nh * 2, 0x00020000);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const int n = ncol0 + ct * 32 + c;
                const int on = (n >> 4 << 3) | (n & 7);
                const uint32_t base = (n < N && (c & 8) == 0) ? (uint32_t)(4 * hb * nh + on) * 2u : 0x80000000u;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int r = rt * 32 + 8 * (e >> 2) + (e & 3);
                        const float g = acc[rt][ct][e];
                        const float u = __shfl_xor(g, 8);
                        const uint32_t off = base + (uint32_t)(r * nh * 2);
                        __builtin_amdgcn_raw_buffer_store_b16(f32_to_out<BF16>(silu_mul(g, u)), out, (int)off, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            return;
        }
        const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(a.y + (int64_t)m0 * N, (short)0,
                                                                            rows * N * 2, 0x00020000);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int n = ncol0 + ct * 32 + c;
            const uint32_t base = n < N ? (uint32_t)(4 * hb * N + n) * 2u : 0x80000000u;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int r = rt * 32 + 8 * (e >> 2) + (e & 3);  // row offset without 4 * hb
                    const uint32_t off = base + (uint32_t)(r * N * 2);
                    __builtin_amdgcn_raw_buffer_store_b16(f32_to_out<BF16>(acc[rt][ct][e]), out, (int)off, 0, 0);
                }
            // one fragment at a time keeps the converted values few
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
            a.partial + ((int64_t)split * M + m0) * N, (short)0, rows * N * 4, 0x00020000);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int n = ncol0 + ct * 32 + c;
            const uint32_t base = n < N ? (uint32_t)(4 * hb * N + n) * 4u : 0x80000000u;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int r = rt * 32 + 8 * (e >> 2) + (e & 3);
                    const uint32_t off = base + (uint32_t)(r * N * 4);
                    // copy out first: bit-casting the vector element itself
                    // reads element 0 (clang)
                    const float v = acc[rt][ct][e];
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), out, (int)off, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
}

}  // namespace

bool prefill256_ok(int layout, int xtype, int64_t N, int64_t K, int64_t G) {
    // 32-bit buffer offsets: a 256-row fp32 partial tile of the output must
    // stay below 2 GiB
    return layout == LAYOUT_MARLIN && (xtype == X_F16 || xtype == X_BF16) && K % TK == 0 && G % TK == 0 && N % 8 == 0 &&
           N <= (int64_t{1} << 20);
}

int prefill256_tile() { return TM; }

// Tail balancing of an unsplit launch of 256-row tiles: the number of
// trailing N-tile columns to run as 128-row tiles, and the cost in waves of
// full tiles (a half tile counts 0.55: its dequant is shared by half the
// MFMAs; a split must save 0.1 wave).
int64_t prefill256_tail_cols(int64_t M, int64_t N, int cus, double* waves) {
    const int64_t num_m = ceil_div(M, TM), num_n = ceil_div(N, TN);
    double best = cus > 0 ? (double)ceil_div(num_m * num_n, cus) : 1.0;
    int64_t nt = 0;
    if (cus > 0) {
        for (int64_t t = 1; t <= num_n; ++t) {
            const double cost = (double)ceil_div(num_m * (num_n - t), cus) +
                                0.55 * (double)ceil_div(ceil_div(M, TM / 2) * t, cus);
            if (cost < best - 0.1) {
                best = cost;
                nt = t;
            }
        }
    }
    if (waves) *waves = best;
    return nt;
}

// Tail balancing.  With the 256 x 256 tile, a tile count that is not a
// multiple of the CU count leaves a partial last wave (qkv at M = 4096: 384
// tiles on 256 CUs, 1.5 waves run as 2).  The last nt N-tile columns are then
// done by a second launch with 128-row tiles: twice the workgroups at half the
// work each, filling the last wave (qkv: 256 full tiles, then 256 half tiles).
// Same arithmetic per output element, so the result does not change.
template <bool BF16, typename ST, bool ZP>
void launch_variant(const PrefillArgs& a, hipStream_t stream, KernelEvents ev) {
    const NibbleMasks mk{};
    const int64_t num_m = ceil_div(a.M, TM), num_n = ceil_div(a.N, TN);
    const int64_t tiles128 = ceil_div(a.M, TM / 2) * num_n;  // 128-row tiles over every column
    PrefillArgs w = a;  // a launch over every column of the output
    w.n_begin = 0;
    w.n_end = a.N;
    if constexpr (!BF16) {
        if (a.exact) {  // exact scaling: 128-row tiles only (the plan asks for no others)
            const dim3 grid((unsigned)tiles128, 1, a.partial != nullptr ? a.splits : 1);
            if (a.partial != nullptr) {
                launch_kernel(prefill256_kernel<false, ST, ZP, true, 4, true>, grid, dim3(kT), 0, stream, ev.start,
                              ev.stop, w, mk);
            } else {
                launch_kernel(prefill256_kernel<false, ST, ZP, false, 4, true>, grid, dim3(kT), 0, stream, ev.start,
                              ev.stop, w, mk);
            }
            return;
        }
    }
    if (a.partial != nullptr) {  // K slices: fp32 partials of 256- or 128-row tiles
        if (a.tile_rows == TM / 2) {
            launch_kernel(prefill256_kernel<BF16, ST, ZP, true, 4>, dim3((unsigned)tiles128, 1, a.splits), dim3(kT), 0,
                          stream, ev.start, ev.stop, w, mk);
        } else {
            launch_kernel(prefill256_kernel<BF16, ST, ZP, true, 8>, dim3((unsigned)(num_m * num_n), 1, a.splits),
                          dim3(kT), 0, stream, ev.start, ev.stop, w, mk);
        }
        return;
    }
    if (a.tile_rows == TM / 2) {  // every tile 128 rows: twice the workgroups, two per CU
        launch_kernel(prefill256_kernel<BF16, ST, ZP, false, 4>, dim3((unsigned)tiles128), dim3(kT), 0, stream,
                      ev.start, ev.stop, w, mk);
        return;
    }
    const int64_t nt = prefill256_tail_cols(a.M, a.N, a.cus, nullptr);
    const int64_t nfull = num_n - nt;
    if (nfull > 0) {
        PrefillArgs f = a;
        f.n_begin = 0;
        f.n_end = (int)std::min<int64_t>(a.N, nfull * TN);
        launch_kernel(prefill256_kernel<BF16, ST, ZP, false, 8>, dim3((unsigned)(num_m * nfull)), dim3(kT), 0, stream,
                      ev.start, nt > 0 ? nullptr : ev.stop, f, mk);
    }
    if (nt > 0) {
        PrefillArgs h = a;
        h.n_begin = (int)(nfull * TN);
        h.n_end = a.N;
        launch_kernel(prefill256_kernel<BF16, ST, ZP, false, 4>, dim3((unsigned)(ceil_div(a.M, TM / 2) * nt)), dim3(kT),
                      0, stream, nfull > 0 ? nullptr : ev.start, ev.stop, h, mk);
    }
}

template <bool BF16>
void launch_dtype(int stype, bool zp, const PrefillArgs& a, hipStream_t stream, KernelEvents ev) {
    if (stype == S_F32) {
        zp ? launch_variant<BF16, float, true>(a, stream, ev) : launch_variant<BF16, float, false>(a, stream, ev);
    } else {
        zp ? launch_variant<BF16, _Float16, true>(a, stream, ev) : launch_variant<BF16, _Float16, false>(a, stream, ev);
    }
}

hipError_t launch_prefill256(int xtype, int stype, bool zp, const PrefillArgs& a, hipStream_t stream, KernelEvents ev) {
    xtype == X_BF16 ? launch_dtype<true>(stype, zp, a, stream, ev) : launch_dtype<false>(stype, zp, a, stream, ev);
    return hipGetLastError();
}

}  // namespace pw4

// Compute-bound W4A16 GEMM for large M on the MARLIN layout with fp16 or
// bf16 activations: y[M,N] = x[M,K] @ dequant(W)^T, one 256-column output
// tile of 256 or 128 rows per workgroup.
//
// Tiling.  256-row tiles: eight waves; waves 2b and 2b + 1 own the two
// 32-column halves of MARLIN column block b (64 columns) for all 256 rows,
// 8 tiles of v_mfma_f32_32x32x16 each.  128-row tiles: four waves; wave w owns
// column block w for all 128 rows, 4 x 2 tiles.  Either way a wave holds 128
// fp32 accumulators per lane in VGPRs, two waves share a SIMD, every weight
// nibble is dequantized exactly once per workgroup, and the activation tile
// is read from LDS by every wave.  K advances in 64-wide chunks (one MARLIN
// chunk per column block).
//
// Pipeline.  Three LDS stages of (activations 32 or 16 KB, packed weights
// 8 KB, scales, zero points), filled with global_load_lds (no VGPRs; each lane
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
// pair: splice into 1024.0 or 64.0 (exact 1024 + u or 64 + u, by the pair's
// bit position), subtract 1024 + z or 64 + z (exact), and -- unless scaling
// exactly -- times the group scale (one fp16 rounding, as the reference's
// dequant_scale, w4a16_marlin.cu:103-113).  bf16 x (gfx950 has no packed bf16
// arithmetic): splice into 128.0 (exact 128 + u), then per value one fp32 fma
// (128 + u) * s - (128 + z) * s with s the scale rounded to bf16 -- both
// products are exact in fp32 -- and one v_cvt_pk_bf16_f32 per pair: the
// reference's bf16 fragment round(q * round(s)) bit for bit
// (w4a16_marlin.cu:115-126).
//
// Exact scaling (fp16 x, the default).  Rounding (u - z) * s to fp16 costs up
// to 2^-11 of every weight; summed over K = 14336-28672 that is ~1e-2 of
// absolute error for x ~ N(0, 1) and scales ~ |N(0, 0.02)| (the benchmark's
// Llama-3 distributions).  In this mode B = u - z (exact in
// fp16) and the group scale is applied in fp32 to the accumulators instead:
// with s_g the scale of group g for the lane's column, the running sum is
// rescaled by s_(g-1) / s_g when group g starts and multiplied by the last
// group's scale at the end, so acc = sum_g s_g * P_g with P_g the exact
// fp32 sum of group g.  One multiply per accumulator per group, and no second
// accumulator set.
//
// Reference counterpart: w4a16_marlin_kernel at BM = 64
// (pulsar-core/src/kernels/w4a16_marlin.cu:197-304).
#include <algorithm>
#include <type_traits>

#include "w4a16_common.h"
#include "w4a16_kernels.h"

namespace pw4 {
namespace {

constexpr int TM = 256, TN = 256, TK = 64;  // full tile; the tail variant has TM = 128
constexpr int kStages = 3;
constexpr int kBStage = TN * TK / 2;
constexpr int kSlot = 256;  // per wave and stage: 256 bytes of scales (64 fp32, or 64 fp16 + pad), of zero-point words

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)p;
}

// One LDS copy instruction: lane l copies 16 (or 4) bytes from base + off
// (base wave-uniform in SGPRs, off a 32-bit per-lane byte offset) to
// LDS[lds + l * 16 (or 4)].  M0 (the LDS base) is saved and restored around
// it; the s_nop covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ void lds_copy16(const void* base, uint32_t off, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds)
        : "memory");
}
__device__ __forceinline__ void lds_copy4(const void* base, uint32_t off, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds)
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

// RT = 32-row MFMA tiles per wave, and the number of waves: 4 (128-row tile:
// wave w owns MARLIN column block w, two column tiles of 32) or 8 (256-row
// tile: waves 2b and 2b + 1 own the two 32-column halves of block b, so each
// wave dequantizes only its own columns).  Either way 128 fp32 accumulators
// per lane, kept in VGPRs, and two waves per SIMD (256 registers each):
// 128-row tiles (75-78 KB of LDS) run two workgroups per CU, 256-row tiles
// (123-132 KB) one.
//
// KS = 2 (128-row tiles only): eight waves in two K halves of four.  Half h
// runs the 128-row tile's pipeline over the second half of the workgroup's
// chunks (h = 1) or the first (h = 0) in LDS stages of its own, both halves
// meeting at the same barriers; at the end half 1 hands its accumulators to
// half 0 through LDS, which adds them (first half + second half, the sum of
// two K slices in slice order) and stores.  One such workgroup per CU (150-156
// KB of LDS) runs a tile at the rate of two 128-row workgroups per CU with no
// fp32 partials in memory.
template <bool BF16, typename ST, bool ZP, bool PARTIAL, int RT, bool EXACT, int KS>
__global__ __launch_bounds__(64 * RT * KS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill256_kernel(const PrefillArgs a, const NibbleMasks mk) {
    static_assert(RT == 4 || RT == 8, "128- or 256-row tiles");
    static_assert(KS == 1 || (KS == 2 && RT == 4), "K halves: 128-row tiles");
    static_assert(!EXACT || !BF16, "exact scaling: fp16 activations");
    constexpr int NW = RT;                       // waves of one K half
    constexpr int CT = 8 / RT;                   // 32-column MFMA tiles per wave
    constexpr int WPB = NW / 4;                  // waves per 64-column block
    constexpr int TMR = 32 * RT;                 // rows of this tile
    constexpr int kAStage = TMR * TK * 2;        // bytes
    constexpr int kARows = TMR / NW;             // activation rows each wave copies
    constexpr int kACopies = kARows / 8;         // one copy instruction moves 8 rows of 128 bytes
    constexpr int kBCopies = 2 / WPB;            // the block's two 1 KB weight tiles, shared by its waves
    constexpr int kZSlot = ZP ? NW * kSlot : 16;
    // per K half: [stages] activations, then weights, scales, zero points
    constexpr int kOffB = kStages * kAStage, kOffS = kOffB + kStages * kBStage, kOffZ = kOffS + kStages * NW * kSlot;
    constexpr int kHalfBytes = kOffZ + kStages * kZSlot;
    __shared__ __attribute__((aligned(16))) uint8_t smem[KS * kHalfBytes];
    static_assert(KS == 1 || NW * RT * CT * 16 * 64 * 4 <= KS * kHalfBytes, "the K-half sum fits the stages");
    // copies per wave per chunk: activations, weights, 1 scale, 1 zero point
    constexpr int kCopies = kACopies + kBCopies + 1 + (ZP ? 1 : 0);

    const int tid = threadIdx.x;
    const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = KS == 2 ? wave_all / NW : 0;  // K half
    const int wave = KS == 2 ? wave_all % NW : wave_all;
    uint8_t* const half = smem + ks * kHalfBytes;
    auto sA = [&](int st) { return half + st * kAStage; };
    auto sB = [&](int st) { return half + kOffB + st * kBStage; };
    auto sS = [&](int st) { return half + kOffS + st * NW * kSlot; };
    auto sZ = [&](int st) { return half + kOffZ + st * kZSlot; };
    const int lane = tid & 63;
    const int c = lane & 31, hb = lane >> 5;
    const int cbl = wave / WPB, cth = wave % WPB;  // column block of the tile, 32-column half (8 waves)
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
    const int c_first = split * a.chunks_per_split;
    const int nck_all = max(min(c_first + a.chunks_per_split, a.nchunks) - c_first, 0);
    // K halves: the first ceil(n / 2) chunks of the slice, then the rest;
    // every wave runs niter barriers
    const int niter = KS == 2 ? (nck_all + 1) / 2 : nck_all;
    const int c_begin = c_first + ks * niter;
    const int nck = ks ? nck_all - niter : niter;  // this wave's chunks

    const int ncb = (N + 63) / 64;              // MARLIN column blocks present
    const int cbw = min(n0 / 64 + cbl, ncb - 1);  // this wave's block (clamped: junk columns are never stored)
    const int ncol0 = n0 + cbl * 64;            // first column of this wave's block
    const ST* scales = reinterpret_cast<const ST*>(a.scales);

    // ---- copies of one chunk into a stage (unconditional: constant count) ---
    // Per-lane byte offsets are fixed for the whole K loop; the bases move.
    // Rows past M, columns past N read clamped addresses; their results are
    // never stored.  Offsets stay below 2^32: prefill256_ok bounds K.
    uint32_t a_off[kACopies];
#pragma unroll
    for (int i = 0; i < kACopies; ++i) {
        const int row = wave * kARows + i * 8 + (lane >> 3);
        const int kch = (lane & 7) ^ ((row >> 1) & 7);
        a_off[i] = (uint32_t)((min(m0 + row, M - 1) - m0) * K + kch * 8) * 2u;
    }
    const uint32_t s_off = sizeof(ST) == 4 ? (uint32_t)min(ncol0 + lane, N - 1) * 4u
                                           : (uint32_t)min(ncol0 + 2 * lane, N - 2) * 2u;  // N even
    const int nw = N / 8;
    const uint32_t z_off = (uint32_t)min(ncol0 / 8 + lane, nw - 1) * 4u;
    const uint16_t* x_tile = a.x + (int64_t)m0 * K;
    auto issue = [&](int kc, int st, int g) {
        const uint32_t abase = lds_addr(sA(st)) + wave * kARows * 128;
#pragma unroll
        for (int i = 0; i < kACopies; ++i) lds_copy16(x_tile + kc * TK, a_off[i], abase + i * 1024);
        const uint32_t* wsrc = a.w + ((int64_t)cbw * a.nchunks + kc) * kChunkWords;
        const uint32_t bbase = lds_addr(sB(st)) + cbl * 2048;
#pragma unroll
        for (int i = 0; i < kBCopies; ++i) {
            const int tt = cth * kBCopies + i;
            lds_copy16(wsrc, (uint32_t)(tt * 64 + lane) * 16u, bbase + tt * 1024);
        }
        lds_copy4(scales + (int64_t)g * N, s_off, lds_addr(sS(st)) + wave * kSlot);
        if constexpr (ZP) lds_copy4(a.qzeros + (int64_t)g * nw, z_off, lds_addr(sZ(st)) + wave * kSlot);
    };

    f32x16 acc[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[rt][ct][e] = 0.f;

    // Dequant constants.  fp16: the lane's nibble pair sits at bit 4 * hb of
    // each half-word on even steps (at 8 + 4 * hb on odd steps, shifted down by
    // 8 first).  At bit 0 it is spliced into 1024.0 (0x6400: exact 1024 + u),
    // at bit 4 into 64.0 (0x5400: mantissa 16u is exact 64 + u), so an even
    // step needs no shift.  bf16: spliced into 128.0 after a shift.  Masks and
    // splice constants live in VGPRs, which gives one v_and_or_b32 each.
    uint32_t one, msk;
    if constexpr (BF16) {
        asm volatile("v_mov_b32 %0, %1" : "=v"(one) : "s"(0x43004300u));
        msk = mk.lo;
    } else {
        one = hb ? 0x54005400u : 0x64006400u;
        msk = hb ? mk.hi : mk.lo;
        asm volatile("" : "+v"(one), "+v"(msk));  // opaque: keeps one v_and_or_b32 per word
    }
    const uint32_t zsplice = hb ? 0x5400u : 0x6400u, zsh = 4u * hb;

    // exact mode: the effective scale of the group the accumulators are in,
    // per column tile (1 until the first chunk; an empty slice stores 0 * 1)
    float s_run[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) s_run[ct] = 1.f;

    // One chunk = four 16-K steps; step s is pair s % 2 of 32-K tile s / 2, and
    // this lane's K run in it is [16s + 8hb, +8): activation 16-byte unit
    // 2s + hb, weight nibble pair 2(s % 2) + hb.  Operands of step s + 1 (the
    // A fragments, the dequantized B) are fetched while step s's MFMAs run.
    // new_group (exact mode): this chunk starts a quant group after another one.
    auto compute = [&](int st, bool new_group) {
        const uint8_t* A = sA(st);
        const uint8_t* B = sB(st) + cbl * 2048;
        u32x4 wq[2][CT];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
                wq[t][ct] = *reinterpret_cast<const u32x4*>(B + t * 1024 + ((cth * CT + ct) * 32 + c) * 16);
        f16x2 s2[CT];
        uint32_t z2[CT];     // fp16: the zero point spliced like the nibbles (1024 + z or 64 + z)
        float sb[CT], cz[CT];  // bf16: scale rounded to bf16, -(128 + z) * scale
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int cl = (cth * CT + ct) * 32 + c;  // column inside the block
            float sf;
            if constexpr (sizeof(ST) == 4) {
                sf = *reinterpret_cast<const float*>(sS(st) + wave * kSlot + cl * 4);
            } else {
                sf = (float)*reinterpret_cast<const _Float16*>(sS(st) + wave * kSlot + cl * 2);
            }
            uint32_t z = 8u;
            if constexpr (ZP) z = (*reinterpret_cast<const uint32_t*>(sZ(st) + wave * kSlot + (cl >> 3) * 4) >> (4 * (cl & 7))) & 0xfu;
            if constexpr (BF16) {
                sb[ct] = (float)(__bf16)sf;
                cz[ct] = -(128.f + (float)z) * sb[ct];
            } else {
                z2[ct] = (zsplice | (z << zsh)) * 0x10001u;
                if constexpr (EXACT) {
                    const float se = exact_scale(sf);
                    if (new_group) {
                        const float r = s_run[ct] * __builtin_amdgcn_rcpf(se);
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                            for (int e = 0; e < 16; ++e) acc[rt][ct][e] *= r;
                    }
                    s_run[ct] = se;
                } else {
                    const _Float16 sh = (_Float16)sf;
                    s2[ct] = f16x2{sh, sh};
                }
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
        auto dequant = [&](int s, u32x4 (&bv)[CT]) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                for (int tg = 0; tg < 4; ++tg) {
                    if constexpr (BF16) {
                        const uint32_t v = ((wq[s >> 1][ct][tg] >> (8 * (s & 1) + 4 * hb)) & msk) | one;
                        bv[ct][tg] = pack_bf16x2_rne(__builtin_fmaf(__builtin_bit_cast(float, v << 16), sb[ct], cz[ct]),
                                                     __builtin_fmaf(__builtin_bit_cast(float, v & 0xffff0000u), sb[ct],
                                                                    cz[ct]));
                    } else {
                        const uint32_t w = (s & 1) ? wq[s >> 1][ct][tg] >> 8 : wq[s >> 1][ct][tg];
                        const f16x2 u = as_h2((w & msk) | one) - as_h2(z2[ct]);  // u - z, exact
                        bv[ct][tg] = EXACT ? as_u32(u) : as_u32(u * s2[ct]);
                    }
                }
        };
        u32x4 av[2][RT], bv[2][CT];
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
                for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = mfma32x32x16<BF16>(av[cur][rt], bv[cur][ct], acc[rt][ct]);
            // (two waves per SIMD cover each other's latency; the compiler's own
            // schedule beat an explicit MFMA / DS read / VALU interleave by 3-10%)
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // quant group of the next chunk to issue, and the chunk's place in it (G is
    // a multiple of 64); issues run in chunk order
    const int cpg = a.G / TK;
    int ig = c_begin / cpg, igk = c_begin - ig * cpg;
    auto next_group = [&]() {
        const int g = min(ig, a.Kg - 1);
        if (++igk == cpg) {
            igk = 0;
            ++ig;
        }
        return g;
    };
    if (nck > 0) issue(c_begin, 0, next_group());
    if (nck > 1) issue(c_begin + 1, 1, next_group());
    int gk = EXACT ? c_begin % cpg : 0;  // place of the chunk being computed in its group
    int st = 0, st2 = 2;                 // stages of chunks i and i + 2
    for (int i = 0; i < niter; ++i) {
        if (i + 1 < nck) {
            wait_vmcnt<kCopies>();  // this wave's copies of chunk i have landed
        } else {
            wait_vmcnt<0>();
        }
        __syncthreads();            // everyone's have; everyone is done with chunk i - 1
        if (i + 2 < nck) issue(c_begin + i + 2, st2, next_group());
        // (KS = 2: the second half may have one chunk fewer; it still joins
        // the barrier of the last iteration)
        if (KS == 1 || i < nck) compute(st, i > 0 && gk == 0);
        if constexpr (EXACT) gk = gk + 1 == cpg ? 0 : gk + 1;
        st = st == kStages - 1 ? 0 : st + 1;
        st2 = st2 == kStages - 1 ? 0 : st2 + 1;
    }
    if constexpr (EXACT) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[rt][ct][e] *= s_run[ct];
    }
    if constexpr (KS == 2) {
        // the second half's accumulators to the first through LDS (the stages
        // are free once every wave is past its last chunk): 16-byte rows,
        // lane-consecutive, [wave][tile][e / 4][lane]
        f32x4* red = reinterpret_cast<f32x4*>(smem);
        __syncthreads();
        if (ks == 1) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                    for (int e4 = 0; e4 < 4; ++e4) {
                        const f32x4 v{acc[rt][ct][4 * e4], acc[rt][ct][4 * e4 + 1], acc[rt][ct][4 * e4 + 2],
                                      acc[rt][ct][4 * e4 + 3]};
                        red[(((wave * RT + rt) * CT + ct) * 4 + e4) * 64 + lane] = v;
                    }
        }
        __syncthreads();
        if (ks == 1) return;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                for (int e4 = 0; e4 < 4; ++e4) {
                    const f32x4 v = red[(((wave * RT + rt) * CT + ct) * 4 + e4) * 64 + lane];
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[rt][ct][4 * e4 + j] += v[j];
                }
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
            for (int ct = 0; ct < CT; ++ct) {
                const int n = ncol0 + (cth * CT + ct) * 32 + c;
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
        for (int ct = 0; ct < CT; ++ct) {
            const int n = ncol0 + (cth * CT + ct) * 32 + c;
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
        if (a.y32) {
            // the accumulators before rounding (pw4_observe_next_call)
            const __amdgpu_buffer_rsrc_t out32 = __builtin_amdgcn_make_buffer_rsrc(a.y32 + (int64_t)m0 * N, (short)0,
                                                                                  rows * N * 4, 0x00020000);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const int n = ncol0 + (cth * CT + ct) * 32 + c;
                const uint32_t base = n < N ? (uint32_t)(4 * hb * N + n) * 4u : 0x80000000u;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int r = rt * 32 + 8 * (e >> 2) + (e & 3);
                        // copy out first: bit-casting the vector element itself
                        // reads element 0 (clang)
                        const float v = acc[rt][ct][e];
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), out32,
                                                              (int)(base + (uint32_t)(r * N * 4)), 0, 0);
                    }
                }
            }
        }
    } else {
        const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
            a.partial + ((int64_t)split * M + m0) * N, (short)0, rows * N * 4, 0x00020000);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int n = ncol0 + (cth * CT + ct) * 32 + c;
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
    // 32-bit per-lane activation offsets inside a 256-row tile: 256 * K * 2 bytes
    return layout == LAYOUT_MARLIN && (xtype == X_F16 || xtype == X_BF16) && K % TK == 0 && G % TK == 0 && N % 8 == 0 &&
           N <= (int64_t{1} << 20) && K <= (int64_t{1} << 22);
}

int prefill256_tile() { return TM; }

// Tail balancing of an unsplit launch of 256-row tiles: the number of
// trailing N-tile columns to run as 128-row tiles, and the cost in waves of
// full tiles (a split must save 0.1 wave).  128-row tiles run two per CU: a
// round of up to 2 x CUs of them costs one wave, and a last round of at most
// one per CU 0.69 (a chunk per 1.1 us alone against 1.6 for a 256-row tile).
// Before, every CU-sized group of 128-row tiles counted 0.55 of a wave, which
// priced a lone tail round too low: bf16 qkv at M = 1024 ran all 24 column
// tiles as 192 lone 128-row workgroups in 73 us.
int64_t prefill256_tail_cols(int64_t M, int64_t N, int cus, double* waves) {
    constexpr double kSoloRound = 1.1 / 1.6;
    const int64_t num_m = ceil_div(M, TM), num_n = ceil_div(N, TN);
    double best = cus > 0 ? (double)ceil_div(num_m * num_n, cus) : 1.0;
    int64_t nt = 0;
    if (cus > 0) {
        for (int64_t t = 1; t <= num_n; ++t) {
            const int64_t half = ceil_div(M, TM / 2) * t;  // 128-row tiles of the tail
            const int64_t pairs = half / (2 * (int64_t)cus), rest = half - pairs * 2 * (int64_t)cus;
            const double cost = (double)ceil_div(num_m * (num_n - t), cus) + (double)pairs +
                                (rest == 0 ? 0.0 : rest <= cus ? kSoloRound : 1.0);
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
    const bool exact = !BF16 && a.exact;
    auto launch = [&](auto rt, auto ksc, dim3 grid, const PrefillArgs& args, hipEvent_t start, hipEvent_t stop,
                      auto partial) {
        constexpr int RT = decltype(rt)::value;
        constexpr int KSV = decltype(ksc)::value;
        constexpr bool P = decltype(partial)::value;
        const dim3 block(64 * RT * KSV);
        if constexpr (!BF16) {
            if (exact) {
                launch_kernel(prefill256_kernel<false, ST, ZP, P, RT, true, KSV>, grid, block, 0, stream, start, stop,
                              args, mk);
                return;
            }
        }
        launch_kernel(prefill256_kernel<BF16, ST, ZP, P, RT, false, KSV>, grid, block, 0, stream, start, stop, args, mk);
    };
    using One = std::integral_constant<int, 1>;
    using Two = std::integral_constant<int, 2>;
    auto full = [&](auto... v) { launch(std::integral_constant<int, 8>{}, One{}, v...); };
    auto half = [&](auto... v) { launch(std::integral_constant<int, 4>{}, One{}, v...); };
    // 128-row tiles whose workgroup runs the chunks as two K halves (8 waves)
    auto halves = [&](auto... v) { launch(std::integral_constant<int, 4>{}, Two{}, v...); };
    const bool k2 = a.tile_rows == TM / 2 && a.k_halves == 2;
    if (a.partial != nullptr) {  // K slices: fp32 partials of 256- or 128-row tiles
        if (k2) {
            halves(dim3((unsigned)tiles128, 1, a.splits), w, ev.start, ev.stop, std::true_type{});
        } else if (a.tile_rows == TM / 2) {
            half(dim3((unsigned)tiles128, 1, a.splits), w, ev.start, ev.stop, std::true_type{});
        } else {
            full(dim3((unsigned)(num_m * num_n), 1, a.splits), w, ev.start, ev.stop, std::true_type{});
        }
        return;
    }
    if (k2) {  // one 8-wave workgroup per CU
        halves(dim3((unsigned)tiles128), w, ev.start, ev.stop, std::false_type{});
        return;
    }
    if (a.tile_rows == TM / 2) {  // every tile 128 rows: twice the workgroups, two per CU
        half(dim3((unsigned)tiles128), w, ev.start, ev.stop, std::false_type{});
        return;
    }
    const int64_t nt = prefill256_tail_cols(a.M, a.N, a.cus, nullptr);
    const int64_t nfull = num_n - nt;
    if (nfull > 0) {
        PrefillArgs f = a;
        f.n_begin = 0;
        f.n_end = (int)std::min<int64_t>(a.N, nfull * TN);
        full(dim3((unsigned)(num_m * nfull)), f, ev.start, nt > 0 ? nullptr : ev.stop, std::false_type{});
    }
    if (nt > 0) {
        PrefillArgs h = a;
        h.n_begin = (int)(nfull * TN);
        h.n_end = a.N;
        half(dim3((unsigned)(ceil_div(a.M, TM / 2) * nt)), h, nfull > 0 ? nullptr : ev.start, ev.stop,
             std::false_type{});
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

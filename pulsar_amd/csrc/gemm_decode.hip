// Memory-bound W4A16 GEMM for small M (decode): y[M,N] = x[M,K] @ dequant(W)^T.
//
// Work split.  The weight matrix is cut into units of nb columns (16, 32 or
// 64) and, when the activations of the whole K range do not fit in LDS, into
// K slices.  Workgroups are persistent: gridDim.x = (workgroups per slice) x
// slices, sized to what the CUs hold at once, and a workgroup loops over the
// units of its slice (every wps-th unit).  A workgroup has 8 waves: nb/16
// column waves, each owning a 16-column strip of the unit, times 8/(nb/16) K
// waves that take interleaved 128-K steps of the slice and are summed through
// LDS at the end of each unit.
//
// Streaming.  Per 128-K step every lane issues ONE 16-byte global load: lane
// (c = l%16, h = l/16) fetches the four words of column c in 32-K tile h,
// which are 16 contiguous bytes in both layouts (MARLIN: a wave instruction
// reads four fully used 256-byte segments).  The loads of the wave's next U
// steps (4, or 8 for long units at M > 8) sit in a register ring that runs on
// across unit boundaries, so a unit change costs no HBM round trip.  The activation slice is copied into LDS
// once per workgroup with global_load_lds (no VGPRs), issued before the first
// weight loads.
//
// Math.  The four words feed four v_mfma_f32_16x16x32.  fp16: B = u - z
// exactly (exponent splice of the nibble into 1024.0, then one packed add or
// fma per pair), accumulated per 128-K step in fp32 and scaled per column in
// fp32, so q * scale is never rounded to 16 bits.  bf16 has no cheap packed
// subtract, so B = 128 + u (exact), and a second MFMA on the same activation
// fragment with B = -(128 + z) in every K position (exact in bf16) takes the
// bias back out of the fp32 accumulator.  The
// activations stay in natural K order: MARLIN word tg of a 32-K tile holds
// K {8p + 2tg, 8p + 2tg + 1} in its nibble pair p, so pair s of the tile's
// four words is the contiguous run [8s, 8s + 8) that MFMA s multiplies; a
// compressed-tensors word is such a run already (its pairs re-ordered with
// v_perm).  Either way the A operand is one 16-byte LDS read.
//
// K slices across workgroups, when the activation slice does not fit in LDS.
// Exchange tree (TREE instantiations; power-of-two slice counts up to 8): the
// slices of a unit pair up level by level, each side swapping its fp32 sum
// with its partner's through a 64-bit {value, flag} slot, so the sum is the
// fixed tree ((s0 + s1) + (s2 + s3)) + ... whatever the arrival order.
// Counter path (forced split counts, M > 32): every workgroup writes its fp32
// partial tile and the last to arrive for a unit (arrival counter) sums the
// partials in slice order -- the fixed-order combine of the reference
// (w4a16_common.cuh:94-120) without a second launch -- and resets the counter.
// Windowed plans (WIN instantiations), taken where the slices would exceed
// the tree's eight: no K slices; each workgroup takes one unit over the whole
// K, and copy waves beside the eight compute waves stage the activations in K
// windows through two LDS buffers, one barrier per window.
//
// Reference counterpart: w4a16_marlin_kernel / gemm_w4a16_kernel at BM = 16
// (pulsar-core/src/kernels/w4a16_marlin.cu:197-304, w4a16_gemm.cu:153-264).
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

#include "w4a16_common.h"
#include "w4a16_kernels.h"

namespace pw4 {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRing = 8;
// copy waves of a windowed plan (after the eight compute waves)
constexpr int kCopyWaves = 4;

// (a & mask) | b for a splice constant b with no bits under the mask.  The
// masks come from the kernel arguments (see NibbleMasks) and b from a VGPR,
// so the compiler cannot fold them into literals (gfx950 VOP3 takes none) and
// emits one v_and_or_b32.  Plain code, not inline assembly: the compiler sees
// the VGPR write and inserts the wait states an MFMA reading it needs.
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) { return (a & mask) | b; }

// One LDS-DMA copy: lane l copies 16 bytes from g to LDS[lds + 16 l].  Issued
// from inline assembly with M0 (the LDS base) saved and restored around it and
// an s_nop for the M0 -> LDS-DMA hazard: through the builtin the compiler would
// wait for every outstanding vector load (the weight ring included) before
// the next barrier or LDS read.  The kernel waits for these copies itself.
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

// s_waitcnt vmcnt(n) leaving lgkmcnt / expcnt alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// fp16 B fragment = u - z, exact, for one weight word.  `one` = 0x64006400.
//   MARLIN (unsigned nibbles): pairs (n_i, n_i+4), i = 0..3.
//   CT (two's complement): pairs (n_2i, n_2i+1), i.e. natural K order.
// MARLIN: pair (MFMA) s takes zero point zlo for s < 2 and zhi for s >= 2;
// they differ only when a quant group is 16 K wide, where MFMAs 0-1 and 2-3 of
// a lane fall in different groups.  CT: the whole word is one MFMA's K run,
// so all its pairs take zlo (the caller passes the word's zero point).
template <int LAYOUT>
__device__ __forceinline__ u32x4 dq_f16(uint32_t q, uint32_t one, uint32_t zlo, uint32_t zhi, const NibbleMasks& mk) {
    const f16x2 z1024_lo = as_h2((0x6400u | zlo) * 0x10001u);             // 1024 + z
    const f16x2 z64_lo = as_h2((0x5400u | (zlo << 4)) * 0x10001u);        // 64 + z
    const f16x2 z1024_hi = as_h2((0x6400u | zhi) * 0x10001u);
    const f16x2 z64_hi = as_h2((0x5400u | (zhi << 4)) * 0x10001u);
    const f16x2 sixteenth = as_h2(0x2c002c00u);
    u32x4 r;
    if constexpr (LAYOUT == LAYOUT_MARLIN) {
        const uint32_t q8 = q >> 8;
        r[0] = as_u32(as_h2(bfi(mk.lo, q, one)) - z1024_lo);
        r[1] = as_u32(as_h2(bfi(mk.hi, q, one)) * sixteenth - z64_lo);
        r[2] = as_u32(as_h2(bfi(mk.lo, q8, one)) - z1024_hi);
        r[3] = as_u32(as_h2(bfi(mk.hi, q8, one)) * sixteenth - z64_hi);
    } else {
        q ^= 0x88888888u;  // two's complement -> u
        const f16x2 mul = as_h2(0x2c003c00u);                                 // {1, 1/16}
        const f16x2 sub = f16x2{z1024_lo[0], z64_lo[0]};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // byte i (nibbles 2i, 2i+1) into bytes 0 and 2, then splice
            const uint32_t w = __builtin_amdgcn_perm(0u, q, 0x0c000c00u | (uint32_t)i | ((uint32_t)i << 16));
            r[i] = as_u32(as_h2(bfi(mk.ct, w, one)) * mul - sub);
        }
    }
    return r;
}

// Quant group (0 .. NGRP-1) of the K run that lane group h supplies to MFMA s
// of a 128-K step: MFMA s takes K 32h + 8s .. +8, and a group is 128 / NGRP wide.
template <int NGRP>
__host__ __device__ constexpr int step_group(int h, int s) {
    return ((4 * h + s) * NGRP) >> 4;
}
// Whether any lane group of MFMA s falls in group gi (a compile-time fact).
template <int NGRP>
__host__ __device__ constexpr bool group_in_mfma(int gi, int s) {
    return step_group<NGRP>(0, s) == gi || step_group<NGRP>(1, s) == gi || step_group<NGRP>(2, s) == gi ||
           step_group<NGRP>(3, s) == gi;
}

// bf16 B fragment = 128 + u (exact), same pair order as dq_f16.
template <int LAYOUT>
__device__ __forceinline__ u32x4 dq_bf16(uint32_t q, uint32_t one, const NibbleMasks& mk) {
    u32x4 r;
    if constexpr (LAYOUT == LAYOUT_MARLIN) {
        r[0] = bfi(mk.lo, q, one);
        r[1] = bfi(mk.lo, q >> 4, one);
        r[2] = bfi(mk.lo, q >> 8, one);
        r[3] = bfi(mk.lo, q >> 12, one);
    } else {
        q ^= 0x88888888u;
        const uint32_t q4 = q >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // byte 0 = byte i of q (low nibble n_2i), byte 2 = byte i of q >> 4
            // (low nibble n_2i+1), then splice both low nibbles
            const uint32_t w = __builtin_amdgcn_perm(q4, q, 0x0c000c00u | (uint32_t)i | ((uint32_t)(4 + i) << 16));
            r[i] = bfi(mk.lo, w, one);
        }
    }
    return r;
}

template <bool BF16>
__device__ __forceinline__ float half_to_f32(uint16_t v) {
    if constexpr (BF16) {
        return __builtin_bit_cast(float, (uint32_t)v << 16);
    } else {
        return (float)__builtin_bit_cast(_Float16, v);
    }
}

// LDS layout (bytes from the start):
//   X     [M][rowstride] halves, rowstride = kps + 8, padded to whole 1 KB
//         copy blocks: the workgroup's activation slice in natural K order
//   RED   [2][8 waves][MT*16][16] fp32: per-unit cross-wave sums, double buffered
//   XN    (act-order in LDS only) [M][K] halves: x as given, padded to 1 KB,
//         from which X is gathered
__host__ __device__ inline size_t x_slots(int M, int kps) { return ((size_t)M * (kps / 8 + 1) + 63) / 64 * 64; }
__host__ __device__ inline size_t red_floats(int mt) { return (size_t)2 * kWaves * mt * 16 * 16; }
__host__ __device__ inline size_t xn_slots(int M, int K) { return ((size_t)M * (K / 8) + 63) / 64 * 64; }
// act-order in LDS: 16-byte x columns (8 K positions) of the permutation each
// thread gathers, loaded ahead of the weight ring, K <= 8 * PXC * 512: 2 up to
// K = 8192 (16 VGPRs, two workgroups per CU still fit), 8 up to K = 32768
constexpr int kPermColsMax = 8;

// s_waitcnt lgkmcnt(0); s_barrier: a workgroup barrier over LDS traffic only.
// __syncthreads() is a workgroup release fence plus the barrier, and once
// global atomics are in flight that fence waits for every outstanding vector
// memory operation, the weight ring included.  The memory clobber keeps the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// PXC > 0: act-order in LDS (one slice, not windowed): the workgroup copies x
// as given into XN and gathers its slice X[m][j] = XN[m][perm[j]] itself, in
// place of a separate gather launch; each thread gathers PXC 16-byte columns.
template <bool BF16, int LAYOUT, typename ST, int MT, int NGRP, bool ZP, int U, bool TREE, bool WIN, bool SBK, int PXC>
__global__ __launch_bounds__(WIN ? kThreads + 64 * kCopyWaves : kThreads) void decode_kernel(const DecodeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ int s_last;
    constexpr int MP = MT * 16;
    static_assert(NGRP == 1 || NGRP == 2 || NGRP == 4 || NGRP == 8, "quant groups per 128-K step");
    constexpr bool PX = PXC > 0;
    static_assert(!PX || (!TREE && !WIN && LAYOUT == LAYOUT_MARLIN), "act-order in LDS: one slice, MARLIN");
    // Block scales (SBK; MARLIN, one quant group per step): the scale (and
    // zero point) of the four steps of a ring block come in one load per lane
    // at the block's first step -- lane group h fetches step h's -- and reach
    // the other lane groups through ds_bpermute, in place of one load per step.
    constexpr bool SB = SBK && LAYOUT == LAYOUT_MARLIN && NGRP == 1 && !WIN && U % 4 == 0;
    // vector memory instructions per ring step (weights, scales, zero points);
    // block scales: per four steps
    constexpr int kLoadsPerStep = 1 + NGRP + (ZP ? NGRP : 0);
    constexpr int kLoadsPerRing = SB ? U + (U / 4) * (ZP ? 2 : 1) : U * kLoadsPerStep;
    // vmcnt is six bits: waiting for "all but the ring" waits for at most 63
    // younger loads (with more, a few ring loads are waited for as well)
    constexpr int kRingLoads = kLoadsPerRing < 63 ? kLoadsPerRing : 63;

    const int tid = threadIdx.x;
    // wave-uniform by construction; readfirstlane tells the compiler, so that
    // everything derived from it (K wave, unit columns, step bookkeeping) is
    // scalar arithmetic and scalar branches
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int c = lane & 15, h = lane >> 4;
    const int M = a.M, N = a.N, K = a.K;
    const int nb = a.nb;
    // No integer divides before the first loads: nb / 16 and 8 / (nb / 16)
    // are powers of two, the slice is blockIdx.y, and the unit count follows
    // from ups = ceil(ncg / wps).
    const int cwn_log2 = __builtin_ctz((unsigned)nb >> 4);  // column waves: 1, 2 or 4
    const int cwn = 1 << cwn_log2;
    const int kwn_log2 = 3 - cwn_log2;                      // K waves per 16-column strip
    const int kwn = 1 << kwn_log2;
    const int cw = wave & (cwn - 1), kw = wave >> cwn_log2;
    const int split = blockIdx.y;
    const int wl = blockIdx.x;
    const int n_units = wl + (a.ups - 1) * a.wps < a.ncg ? a.ups : a.ups - 1;
    const int rs = a.rowstride;
    const int kb = split * a.k_per_split;
    const int klen = max(min(kb + a.k_per_split, a.ktiles * 32) - kb, 0);  // multiple of 32
    const int nsteps = (klen / 32 + 3) / 4;
    // Steps per unit, the same for every wave; at least one, so that an empty
    // K slice still finishes its units (zero partials) and counts its arrival.
    const int spu = max((nsteps + kwn - 1) >> kwn_log2, 1);
    const int spu_pad = (spu + U - 1) / U * U;  // positions per unit, a whole number of ring blocks

    // the staged x: one buffer of the slice, or (WIN) two buffers of a K window
    const int nslots = (int)x_slots(M, a.kwin);
    float* RED = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + (size_t)nslots * 16 * (WIN ? 2 : 1));
    const ST* scales = reinterpret_cast<const ST*>(a.scales);

    // ---- the activation slice into LDS --------------------------------------
    // 16-byte slots, row-major over [M][kwin/8 + 1] in natural K order (the
    // last slot of a row is padding); each wave instruction fills 64
    // consecutive slots (one global_load_lds_dwordx4) from per-lane global
    // addresses.  Lanes whose slot is past K, past the slice or in the pad are
    // masked off: the copy never writes those slots, and the ones a step
    // reads are zeroed below.
    const int spr = a.kwin / 8 + 1;
    const int kvalid = max(min(klen, K - kb), 0);  // halves of real activations in the slice
    const uint32_t smem_base = (uint32_t)(uintptr_t)smem;
    // window w of the slice (K kb + w * kwin ..) into buffer w & 1, wave
    // instructions b0, b0 + bstep, ...; kv: halves of the window to copy
    auto copy_window = [&](int w, int b0, int bstep, int kv) {
        const uint32_t base = smem_base + (uint32_t)((w & 1) * nslots * 16);
        const int64_t k0 = (int64_t)kb + (int64_t)w * a.kwin;
        for (int b = b0; b * 64 < nslots; b += bstep) {
            const int f = b * 64 + lane;
            const int row = (int)__umulhi((uint32_t)f, a.spr_recip);  // f / spr (exact; checked at launch)
            const int s8 = f - row * spr;
            if (row < M && s8 * 8 < kv) lds_copy16(a.x + (int64_t)row * K + k0 + s8 * 8, base + b * 1024);
        }
    };
    if constexpr (WIN) {
        // Windowed plans (one slice of whole windows, one unit per workgroup,
        // checked at launch): the eight compute waves copy window 0, and the
        // kCopyWaves copy waves copy window w + 1 into the other buffer while
        // they compute window w.  The copies count in the copying waves'
        // vmcnt only, so the compute waves' weight rings never wait for them;
        // the waves meet at one barrier per window (the compute waves'
        // barrier before each window's first step), after which the buffer of
        // window w - 1 is free.  The copy waves then take part in the unit
        // end's barriers (one, or two with a single reduction buffer), so
        // every barrier of the workgroup has all its waves.  One copy wave
        // was measured 2.2x slower than four (down M = 16 37.9 against 17.2
        // us): a wave's 1 KB copies in flight do not cover the L2 latency
        // under a full weight stream.
        if (wave >= kWaves) {
            const int cwave = wave - kWaves;
            const int nwin = (nsteps * 128) / a.kwin;
            if (nwin > 1) copy_window(1, cwave, kCopyWaves, a.kwin);
            __syncthreads();  // the compute waves' barrier after their window-0 copies
            for (int w = 1; w < nwin; ++w) {
                wait_vmcnt<0>();  // window w is in LDS
                lds_barrier();    // ... and every compute wave is done with window w - 1
                if (w + 1 < nwin) copy_window(w + 1, cwave, kCopyWaves, a.kwin);
            }
            for (int u = 0; u < n_units; ++u) {
                if (a.red_single) lds_barrier();
                lds_barrier();
            }
            return;
        }
    }
    // act-order in LDS: x as given into XN (M * K halves, contiguous in both),
    // then each thread's permutation columns, all ahead of the weight ring, so
    // the gather below overlaps the ring's first round trip
    const uint32_t xn_off = __builtin_amdgcn_readfirstlane(
        (uint32_t)(nslots * 16) + (uint32_t)(a.red_single ? red_floats(MT) * 2 : red_floats(MT) * 4));
    u32x4 pcol[PX ? PXC : 1][2];
    if constexpr (PX) {
        const int nxs = M * (K / 8);  // 16-byte slots of x
        for (int b = wave; b * 64 < nxs; b += kWaves) {
            const int f = b * 64 + lane;
            if (f < nxs) lds_copy16(a.x + (int64_t)f * 8, smem_base + xn_off + b * 1024);
        }
        // columns past K / 8 re-read the last one (unused): constant count, no branch
#pragma unroll
        for (int i = 0; i < PXC; ++i) {
            const int s8 = min(tid + i * kThreads, K / 8 - 1);
            pcol[i][0] = *reinterpret_cast<const u32x4*>(a.perm + s8 * 8);
            pcol[i][1] = *reinterpret_cast<const u32x4*>(a.perm + s8 * 8 + 4);
        }
    } else {
        copy_window(0, wave, kWaves, WIN ? min(kvalid, a.kwin) : kvalid);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- weight / scale / zero loads of the wave's t-th step ----------------
    // Raw values only: converting here would make the prefetch wait for its
    // own loads.  Positions past the wave's last step re-read it; steps past
    // the slice (uneven K-wave split) load the slice's last step unused.  The
    // weight words are read once per launch: non-temporal loads (measured on a
    // plain streaming read: 5.70 -> 5.90 TB/s over 60 MB, 6.48 -> 7.18 over
    // 1 GiB).
    struct Step {
        u32x4 w;
        ST s[NGRP];
        uint32_t z[NGRP];
    };
    const int gshift = a.G_log2;  // G is a power of two on this path
    const int lane_w = (h >> 1) * kChunkWords + (h & 1) * 256 + (cw * 16 + c) * 4;
    const int lane_w_tail = (h & 1) * 256 + (cw * 16 + c) * 4;
    // head: the first step of a ring block (a compile-time fact of the slot);
    // with block scales only those load scales, for steps j + h.
    auto load_step = [&](int u, int j, Step& o, bool head) {
        const int jh = min(j + h, spu - 1);  // block scales: lane group h's step
        if (u >= n_units) {
            u = max(n_units - 1, 0);
            j = spu - 1;
        }
        j = min(j, spu - 1);  // padding positions re-read the unit's last step
        const int st = min(kw + j * kwn, max(nsteps - 1, 0));
        const int k0 = kb + st * 128;
        const int col0 = (wl + u * a.wps) * nb;
        const int ncol_c = min(col0 + cw * 16 + c, N - 1);
        if constexpr (LAYOUT == LAYOUT_MARLIN) {
            const int kc = min(k0 >> 6, a.nchunks - 1);
            const uint32_t* seg = a.w + ((int64_t)(col0 >> 6) * a.nchunks + kc) * kChunkWords + (col0 & 63) * 4;
            o.w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(seg + (kc + 1 < a.nchunks ? lane_w : lane_w_tail)));
        } else {
            const int t = min(k0 / 32 + h, a.ktiles - 1);
            const int64_t off = (int64_t)ncol_c * (K / 8) + t * 4;
            if ((K & 31) == 0) {
                o.w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.w + off));
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) o.w[q] = (t * 32 + q * 8 < K) ? a.w[off + q] : 0u;
            }
        }
        if constexpr (SB) {
            if (head) {
                // past the workgroup's last unit (u clamped) the values are unused
                const int sth = min(kw + jh * kwn, max(nsteps - 1, 0));
                const int g = min((kb + sth * 128) >> gshift, a.Kg - 1);
                o.s[0] = (scales + (int64_t)g * N)[ncol_c];
                if constexpr (ZP) o.z[0] = (a.qzeros + (int64_t)g * (N >> 3))[ncol_c >> 3];
            }
            return;
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
    // Block scales at a block's first step: step t's scale and zero-point word
    // for this lane's column, from lane (c, t) of the head slot's loads.
    float sblk[4] = {1.f, 1.f, 1.f, 1.f};
    uint32_t zblk[4] = {0u, 0u, 0u, 0u};
    auto block_scales = [&](const Step& in) {
        if constexpr (SB) {
            const int sv = __builtin_bit_cast(int, load_scale(&in.s[0]));
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int src = (c + 16 * t) << 2;
                sblk[t] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, sv));
                if constexpr (ZP) zblk[t] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)in.z[0]);
            }
        }
    };

    // Issue the ring in the refills' order (weights, scale per step): the
    // loop body's vmcnt waits must hold for its first block too, and loads
    // grouped by kind here would make every block wait for half the ring.
    Step ring[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
        load_step(0, i, ring[i], i % 4 == 0);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- finish the slice: zero fill, (bf16) corrections ---------------------
    if constexpr (LAYOUT == LAYOUT_MARLIN) {
        wait_vmcnt<kRingLoads>();  // this wave's slice copies are done; its ring is still in flight
    } else {
        wait_vmcnt<0>();
    }
    if constexpr (PX) {
        // every wave's XN copies have landed (each waited for its own above);
        // slot (row, s8) of X gathers XN[row][perm[8 s8 .. 8 s8 + 7]]
        lds_barrier();
        const uint16_t* XN = smem + xn_off / 2;
#pragma unroll
        for (int i = 0; i < PXC; ++i) {
            const int s8 = tid + i * kThreads;
            if (s8 >= K / 8) continue;
            for (int row = 0; row < M; ++row) {
                const uint16_t* xr = XN + row * K;
                u32x4 v;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const int e = 2 * w;  // elements e, e + 1: perm entries e / 4 words in
                    const uint32_t lo = xr[pcol[i][e >> 2][e & 3]];
                    const uint32_t hi = xr[pcol[i][(e + 1) >> 2][(e + 1) & 3]];
                    v[w] = lo | (hi << 16);
                }
                *reinterpret_cast<u32x4*>(smem + (row * spr + s8) * 8) = v;
            }
        }
    }
    // zero the slots the steps read past the real activations (windowed plans
    // have none: their slice is whole windows of real activations)
    if constexpr (!WIN) {
        const int zfrom = kvalid / 8, zto = nsteps * 16;
        for (int i = tid; i < M * (zto - zfrom); i += kThreads) {
            const int row = i / (zto - zfrom), s8 = zfrom + (i - row * (zto - zfrom));
            *reinterpret_cast<u32x4*>(smem + (row * spr + s8) * 8) = u32x4{0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();
    // ---- main loop -----------------------------------------------------------
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // The splice constant in a VGPR (the masks come in SGPRs): one VOP3 may
    // read a single SGPR, so this is what lets `(q & m) | c` be one
    // v_and_or_b32.  The move is opaque so the constant is not re-folded.
    uint32_t one;
    asm volatile("v_mov_b32 %0, %1" : "=v"(one) : "s"(BF16 ? 0x43004300u : 0x64006400u));
    int arow[MT];  // A rows past M read row M-1: their D rows are never stored
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) arow[mt] = min(mt * 16 + c, M - 1) * rs + 32 * h;
    // this lane group's quant group in MFMAs 0-1 and in MFMAs 2-3 of a step
    const int g_lo = step_group<NGRP>(h, 0), g_hi = step_group<NGRP>(h, 2);

    // t: the step's place in its ring block (block scales: sblk[t], zblk[t])
    auto compute_step = [&](int u, int j, const Step& in, int t) {
        const int st = kw + j * kwn;
        if (j >= spu || st >= nsteps) return;  // padding, or an uneven K-wave split
        int kl = st * 128;
        if constexpr (WIN) {
            // step j of each K wave lies in window j / jw; the window's buffer
            const int win = j >> a.jw_log2;
            kl = (st - (win << (a.jw_log2 + kwn_log2))) * 128 + (win & 1) * nslots * 8;
        }
        const int col0 = (wl + u * a.wps) * nb;
        const int ncol_c = min(col0 + cw * 16 + c, N - 1);
        uint32_t zl[NGRP];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            const uint32_t zw = SB ? zblk[t] : in.z[gi];
            zl[gi] = ZP ? (zw >> (4 * (ncol_c & 7))) & 0xfu : 8u;
        }
        f32x4 tmp[NGRP][MT];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) tmp[gi][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        // bf16: B = 128 + u (exact), so each group's sum carries (128 + z) * sum(x)
        // too; a second MFMA on the same activations with B = -(128 + z) in every
        // K position (exact in bf16: 0xC300 | z) removes it in the accumulator.
        u32x4 zneg[NGRP];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            const uint32_t v = (0xC300u | zl[gi]) * 0x10001u;
            zneg[gi] = u32x4{v, v, v, v};
        }
        uint32_t zlo = zl[0], zhi = zl[0];
#pragma unroll
        for (int gi = 1; gi < NGRP; ++gi) {
            zlo = g_lo == gi ? zl[gi] : zlo;
            zhi = g_hi == gi ? zl[gi] : zhi;
        }
        // MARLIN: pair s of word tg holds natural K 8s + 2tg, 8s + 2tg + 1, so
        // pair s of the four words is the contiguous K run [8s, 8s + 8) of the
        // tile, which MFMA s multiplies with natural-order activations.  CT:
        // word s is that run already (dq_* emits its pairs in K order).
        u32x4 d[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if constexpr (BF16) {
                d[w] = dq_bf16<LAYOUT>(in.w[w], one, a.masks);
            } else {
                if constexpr (LAYOUT == LAYOUT_MARLIN) {
                    d[w] = dq_f16<LAYOUT>(in.w[w], one, zlo, zhi, a.masks);
                } else {
                    const uint32_t zw = w < 2 ? zlo : zhi;  // word w is MFMA w's K run
                    d[w] = dq_f16<LAYOUT>(in.w[w], one, zw, zw, a.masks);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            u32x4 b;
            if constexpr (LAYOUT == LAYOUT_MARLIN) {
                b = u32x4{d[0][s], d[1][s], d[2][s], d[3][s]};
            } else {
                b = d[s];
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const u32x4 av = *reinterpret_cast<const u32x4*>(smem + arow[mt] + kl + 8 * s);
                // one MFMA per quant group present in MFMA s, each on the lanes of
                // that group only (the others supply zero activations)
#pragma unroll
                for (int gi = 0; gi < NGRP; ++gi) {
                    if (!group_in_mfma<NGRP>(gi, s)) continue;
                    u32x4 ag = av;
                    if constexpr (NGRP > 1) {
                        if ((s < 2 ? g_lo : g_hi) != gi) ag = u32x4{0u, 0u, 0u, 0u};
                    }
                    tmp[gi][mt] = mfma16x16x32<BF16>(ag, b, tmp[gi][mt]);
                    if constexpr (BF16) tmp[gi][mt] = mfma16x16x32<BF16>(ag, zneg[gi], tmp[gi][mt]);
                }
            }
        }
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[mt][r] += (SB ? sblk[t] : load_scale(&in.s[gi])) * tmp[gi][mt][r];
    };

    // ---- K slices through a pairwise exchange tree ---------------------------
    // splits = 2^levels; output element i = tid + 512 e of the unit, e < 2
    // (M * nb <= 1024).  At level l the slices pair up as subtrees of 2^l:
    // each side swaps its sum for the 64-bit slot's previous content {value,
    // flag}; the side that finds its partner's value adds it (a + b == b + a
    // in fp32, so the sum does not depend on who came first), clears the
    // slot and goes up a level; after the top level it stores y.  Value and
    // flag travel in one atomic, so nothing else needs ordering.  A swap's
    // answer is read one unit later: by then only weight loads issued after
    // it are outstanding, and in-order vmcnt lets the wave wait for the swap
    // alone instead of draining the ring.
    constexpr int kMaxLevels = 3;
    constexpr int kMaxE = 2;
    const int levels = a.tree_levels;
    const int nout_all = M * nb;
    uint64_t t_old[kMaxLevels + 1][kMaxE];
    float t_v[kMaxLevels + 1][kMaxE];
    bool t_alive[kMaxLevels + 1][kMaxE];
    int t_cg[kMaxLevels + 1];  // unit of the stage (wave-uniform), -1 when empty
#pragma unroll
    for (int k = 0; k <= kMaxLevels; ++k) {
        t_cg[k] = -1;
#pragma unroll
        for (int e = 0; e < kMaxE; ++e) {
            t_old[k][e] = 0;
            t_v[k][e] = 0.f;
            t_alive[k][e] = false;
        }
    }
    auto slot = [&](int level, int cg, int i) {
        const int node = (a.splits - (a.splits >> level)) + (split >> (level + 1));
        return a.slots + (((int64_t)node * a.ncg + cg) * nout_all + i);
    };
    auto swap_in = [&](int level, int cg, int i, float v) -> uint64_t {
        const unsigned long long mine = (unsigned long long)__builtin_bit_cast(uint32_t, v) | (1ull << 32);
        return __hip_atomic_exchange(slot(level, cg, i), mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto tree_advance = [&]() {
#pragma unroll
        for (int k = kMaxLevels - 1; k >= 0; --k) {
            if (k >= levels || t_cg[k] < 0) continue;
            const int cg = t_cg[k];
            t_cg[k] = -1;
            if (k + 1 < levels) t_cg[k + 1] = cg;  // stage k + 1 was emptied earlier in this loop
#pragma unroll
            for (int e = 0; e < kMaxE; ++e) {
                const int i = tid + e * kThreads;
                bool go = false;
                float v = 0.f;
                if (t_alive[k][e]) {
                    if ((t_old[k][e] >> 32) != 0) {  // the partner was first: combine, clear the slot
                        v = __builtin_bit_cast(float, (uint32_t)t_old[k][e]) + t_v[k][e];
                        __hip_atomic_store(slot(k, cg, i), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        go = true;
                    }
                    t_alive[k][e] = false;
                }
                if (k + 1 < levels) {
                    t_alive[k + 1][e] = go;
                    t_v[k + 1][e] = v;
                    if (go) t_old[k + 1][e] = swap_in(k + 1, cg, i, v);
                } else if (go) {
                    const int row = i >> (4 + cwn_log2), n = cg * nb + (i & (nb - 1));
                    if (n < N) {
                        a.y[(int64_t)row * N + n] = f32_to_out<BF16>(v);
                        if (a.y32) a.y32[(int64_t)row * N + n] = v;
                    }
                }
            }
        }
    };

    // ---- end of a unit: sum the K waves in fixed order, store ----------------
    int rbuf = 0;
    auto finish_unit = [&](int u) {
        // one RED buffer (LDS-tight plans): wait until the previous unit's
        // reduction has read it; two: alternate
        if (a.red_single) lds_barrier();
        float* red = RED + rbuf * (red_floats(MT) / 2);
        if (!a.red_single) rbuf ^= 1;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(wave * MP + mt * 16 + 4 * h + r) * 16 + c] = acc[mt][r];
            acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        lds_barrier();
        const int cg = wl + u * a.wps;
        const int col0 = cg * nb;
        const int nout = M * nb;
        auto reduced = [&](int i) {
            const int row = i >> (4 + cwn_log2), col = i & (nb - 1);
            const int cwi = col >> 4, ci = col & 15;
            // all kwn reads issued before the first add, summed in K-wave order
            float t[kWaves];
#pragma unroll
            for (int k = 0; k < kWaves; ++k) t[k] = k < kwn ? red[((k * cwn + cwi) * MP + row) * 16 + ci] : 0.f;
            float v = 0.f;
#pragma unroll
            for (int k = 0; k < kWaves; ++k) v += t[k];
            return v;
        };
        if constexpr (TREE) {
            tree_advance();
            t_cg[0] = cg;
#pragma unroll
            for (int e = 0; e < kMaxE; ++e) {
                const int i = tid + e * kThreads;
                const bool mine = i < nout;
                const float v = mine ? reduced(i) : 0.f;
                t_v[0][e] = v;
                t_alive[0][e] = mine;
                if (mine) t_old[0][e] = swap_in(0, cg, i, v);
            }
            return;
        }
        if (a.partial == nullptr) {
            if (a.silu) {
                // gate|up pairs: column c and c + 8 of each 16-column strip,
                // elements i and i ^ 8, held by lanes tid and tid ^ 8 of one
                // wave (nout is a multiple of 16, so both run the same trips)
                const int nh = N >> 1;
                for (int i = tid; i < nout; i += kThreads) {
                    const int row = i >> (4 + cwn_log2), c = i & (nb - 1);
                    const float v = reduced(i);
                    const float up = __shfl_xor(v, 8);
                    const int n = ((col0 + c) >> 4 << 3) | (c & 7);  // output column: strip * 8 + c % 8
                    if ((c & 8) == 0 && col0 + c < N) a.y[(int64_t)row * nh + n] = f32_to_out<BF16>(silu_mul(v, up));
                }
                return;
            }
            for (int i = tid; i < nout; i += kThreads) {
                const int row = i >> (4 + cwn_log2), n = col0 + (i & (nb - 1));
                const float v = reduced(i);
                if (n < N) {
                    a.y[(int64_t)row * N + n] = f32_to_out<BF16>(v);
                    if (a.y32) a.y32[(int64_t)row * N + n] = v;
                }
            }
            return;
        }
        // K slices across workgroups: the partials travel as device-scope
        // atomic stores and loads (sc1: written through to, and read from, the
        // device coherence point), the arrival counter is a device-scope
        // atomic, and every wave waits for its partial stores to be
        // acknowledged (vmcnt 0) before the barrier that precedes the counter
        // increment, so whoever sees the last arrival also sees every partial.
        // Agent-scope fences would be equivalent but write back the whole L2.
        float* part = a.partial + ((int64_t)cg * a.splits + split) * nout;
        for (int i = tid; i < nout; i += kThreads) {
            __hip_atomic_store(part + i, reduced(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            s_last = __hip_atomic_fetch_add(a.counters + cg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     a.splits - 1;
        }
        __syncthreads();
        if (s_last) {
            const float* base = a.partial + (int64_t)cg * a.splits * nout;
            for (int i = tid; i < nout; i += kThreads) {
                float v = 0.f;
                for (int sp = 0; sp < a.splits; ++sp) {
                    v += __hip_atomic_load(base + (int64_t)sp * nout + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                const int row = i >> (4 + cwn_log2), n = col0 + (i & (nb - 1));
                if (n < N) {
                    a.y[(int64_t)row * N + n] = f32_to_out<BF16>(v);
                    if (a.y32) a.y32[(int64_t)row * N + n] = v;
                }
            }
            if (tid == 0) __hip_atomic_store(a.counters + cg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };

    // Unit-major loop.  A unit's steps are padded to a multiple of U, so unit
    // boundaries fall on ring-block boundaries: one copy of the unit epilogue,
    // and the ring slots stay compile-time.  Refills are unconditional
    // (clamped past the end) so the ring registers are written by the loads
    // themselves, never through a branch join that would force a wait.
    // Every block refills the ring (the unit's next block, or the next unit's
    // first) except the workgroup's very last block, which is peeled out of
    // the loop: a wave cannot retire before its loads return, and a refill
    // branch inside the loop would merge two ring states at its head, which
    // makes the compiler's vmcnt waits wait for half the ring.
    // WIN: the barrier before each window's first step (see the copy waves)
    auto win_sync = [&](int j) {
        if constexpr (WIN) {
            if (j > 0 && j < spu && (j & ((1 << a.jw_log2) - 1)) == 0) lds_barrier();
        }
    };
    const int nblk = spu_pad / U;
    for (int u = 0; u < n_units; ++u) {
        const int refill_blocks = u + 1 < n_units ? nblk : nblk - 1;
        for (int b = 0; b < refill_blocks; ++b) {
            const int jb = b * U;
            const bool same = b + 1 < nblk;
            const int tu = same ? u : u + 1, tj = same ? jb + U : 0;
#pragma unroll
            for (int i = 0; i < U; ++i) {
                win_sync(jb + i);
                if (i % 4 == 0) block_scales(ring[i]);  // before the refill overwrites the head slot
                compute_step(u, jb + i, ring[i], i % 4);
                load_step(tu, tj + i, ring[i], i % 4 == 0);
                // keep the refill right behind its step: without the barrier
                // the scheduler batches all U computes first and drains the ring
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (refill_blocks < nblk) {
#pragma unroll
            for (int i = 0; i < U; ++i) {
                win_sync((nblk - 1) * U + i);
                if (i % 4 == 0) block_scales(ring[i]);
                compute_step(u, (nblk - 1) * U + i, ring[i], i % 4);
            }
        }
        finish_unit(u);
    }
    if constexpr (TREE) {
        // the last units' exchanges: one level per round trip
#pragma unroll
        for (int r = 0; r < kMaxLevels; ++r) tree_advance();
    }
}

using DecodeFn = void (*)(const DecodeArgs);

// Instantiated for MT 1 and 2 (M <= 32; larger M runs the prefill kernels).
// The exchange tree is a separate instantiation: its atomics in the unit loop
// make the compiler's wait counts for the weight ring more conservative, which
// the plain variants should not pay for.  Quant groups narrower than 64 K
// (NGRP 4 and 8) exist for the 4-step ring without the tree only.  Windowed
// variants (WIN) exist for the MARLIN layout and NGRP 1 and 2, without the
// tree.
// Act-order in LDS (px: 0, or the columns per thread, 2 or 8) exists for the
// plans that take it: MARLIN, 16-row tiles, the 4-step ring, one slice, one
// quant group per step.
template <bool BF16, int LAYOUT, typename ST, bool ZP, int U, int MT, bool TREE, bool WIN>
DecodeFn pick_ngrp(int ngrp, bool sb, int px) {
    constexpr bool kPx = LAYOUT == LAYOUT_MARLIN && MT == 1 && U == 4 && !TREE && !WIN;
    switch (ngrp) {
        case 1:
            if constexpr (LAYOUT == LAYOUT_MARLIN && !WIN) {
                if constexpr (kPx) {
                    if (px == 2) {
                        return sb ? decode_kernel<BF16, LAYOUT, ST, MT, 1, ZP, U, TREE, WIN, true, 2>
                                  : decode_kernel<BF16, LAYOUT, ST, MT, 1, ZP, U, TREE, WIN, false, 2>;
                    }
                    if (px == kPermColsMax) {
                        return sb ? decode_kernel<BF16, LAYOUT, ST, MT, 1, ZP, U, TREE, WIN, true, kPermColsMax>
                                  : decode_kernel<BF16, LAYOUT, ST, MT, 1, ZP, U, TREE, WIN, false, kPermColsMax>;
                    }
                }
                if (px) return nullptr;
                if (sb) return decode_kernel<BF16, LAYOUT, ST, MT, 1, ZP, U, TREE, WIN, true, 0>;
            }
            if (px) return nullptr;
            return decode_kernel<BF16, LAYOUT, ST, MT, 1, ZP, U, TREE, WIN, false, 0>;
        case 2:
            if (px) return nullptr;
            return decode_kernel<BF16, LAYOUT, ST, MT, 2, ZP, U, TREE, WIN, false, 0>;
        case 4:
            if (px) return nullptr;
            if constexpr (!TREE && !WIN && U == 4) return decode_kernel<BF16, LAYOUT, ST, MT, 4, ZP, U, TREE, WIN, false, 0>;
            return nullptr;
        case 8:
            if (px) return nullptr;
            if constexpr (!TREE && !WIN && U == 4) return decode_kernel<BF16, LAYOUT, ST, MT, 8, ZP, U, TREE, WIN, false, 0>;
            return nullptr;
        default: return nullptr;
    }
}

template <bool BF16, int LAYOUT, typename ST, bool ZP, int U>
DecodeFn pick_mt_u(int mt, int ngrp, bool tree, bool win, bool sb, int px) {
    if (tree) {
        if (win) return nullptr;
        if (mt == 1) return pick_ngrp<BF16, LAYOUT, ST, ZP, U, 1, true, false>(ngrp, sb, px);
        if (mt == 2) return pick_ngrp<BF16, LAYOUT, ST, ZP, U, 2, true, false>(ngrp, sb, px);
        return nullptr;
    }
    if (win) {
        if constexpr (LAYOUT == LAYOUT_MARLIN) {
            if (mt == 1) return pick_ngrp<BF16, LAYOUT, ST, ZP, U, 1, false, true>(ngrp, sb, px);
            if (mt == 2) return pick_ngrp<BF16, LAYOUT, ST, ZP, U, 2, false, true>(ngrp, sb, px);
        }
        return nullptr;
    }
    if (mt == 1) return pick_ngrp<BF16, LAYOUT, ST, ZP, U, 1, false, false>(ngrp, sb, px);
    if (mt == 2) return pick_ngrp<BF16, LAYOUT, ST, ZP, U, 2, false, false>(ngrp, sb, px);
    return nullptr;
}

template <bool BF16, int LAYOUT, typename ST, bool ZP>
DecodeFn pick_mt(int mt, int ngrp, int ring, bool tree, bool win, bool sb, int px) {
    return ring == 4 ? pick_mt_u<BF16, LAYOUT, ST, ZP, 4>(mt, ngrp, tree, win, sb, px)
                     : pick_mt_u<BF16, LAYOUT, ST, ZP, kRing>(mt, ngrp, tree, win, sb, px);
}

template <bool BF16>
DecodeFn pick_layout(int layout, int stype, bool zp, int mt, int ngrp, int ring, bool tree, bool win, bool sb,
                     int px) {
    if (layout == LAYOUT_CT) {
        return (zp || stype != S_F32) ? nullptr
                                      : pick_mt<BF16, LAYOUT_CT, float, false>(mt, ngrp, ring, tree, win, sb, px);
    }
    if (stype == S_F32) {
        return zp ? pick_mt<BF16, LAYOUT_MARLIN, float, true>(mt, ngrp, ring, tree, win, sb, px)
                  : pick_mt<BF16, LAYOUT_MARLIN, float, false>(mt, ngrp, ring, tree, win, sb, px);
    }
    return zp ? pick_mt<BF16, LAYOUT_MARLIN, _Float16, true>(mt, ngrp, ring, tree, win, sb, px)
              : pick_mt<BF16, LAYOUT_MARLIN, _Float16, false>(mt, ngrp, ring, tree, win, sb, px);
}

DecodeFn pick_decode(int layout, int xtype, int stype, bool zp, int mt, int ngrp, int ring, bool tree, bool win,
                     bool sb, int px) {
    return xtype == X_BF16 ? pick_layout<true>(layout, stype, zp, mt, ngrp, ring, tree, win, sb, px)
                           : pick_layout<false>(layout, stype, zp, mt, ngrp, ring, tree, win, sb, px);
}

hipError_t prepare(DecodeFn fn, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

// Fixed-order sum of [splits, M, N] fp32 partials, then the cast to y's dtype
// (the prefill path's split-K combine; restates w4a16_common.cuh:97-111).
template <bool BF16>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ partial, uint16_t* __restrict__ y,
                                                      int64_t mn, int splits, float* __restrict__ y32) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    if (i + 4 <= mn && (mn & 3) == 0) {
        f32x4 s = *reinterpret_cast<const f32x4*>(partial + i);
        for (int k = 1; k < splits; ++k) s += *reinterpret_cast<const f32x4*>(partial + (int64_t)k * mn + i);
        u32x2 o;
        o[0] = (uint32_t)f32_to_out<BF16>(s[0]) | ((uint32_t)f32_to_out<BF16>(s[1]) << 16);
        o[1] = (uint32_t)f32_to_out<BF16>(s[2]) | ((uint32_t)f32_to_out<BF16>(s[3]) << 16);
        *reinterpret_cast<u32x2*>(y + i) = o;
        if (y32) *reinterpret_cast<f32x4*>(y32 + i) = s;
    } else {
        for (int64_t e = i; e < min(i + 4, mn); ++e) {
            float s = 0.f;
            for (int k = 0; k < splits; ++k) s += partial[(int64_t)k * mn + e];
            y[e] = f32_to_out<BF16>(s);
            if (y32) y32[e] = s;
        }
    }
}

// Output element o of y [M, N/2]: row o / (N/2); strip (o % (N/2)) / 8 holds
// the gate column strip * 16 + o % 8 and the up column 8 further.
__device__ __forceinline__ int64_t silu_gate_index(int64_t o, int64_t nh) {
    const int64_t row = o / nh, oc = o - row * nh;
    return row * (2 * nh) + ((oc >> 3) << 4) + (oc & 7);
}

// Fixed-order sum of gate|up interleaved [splits, M, N] fp32 partials, then
// silu(gate) * up in fp32 and the cast to y [M, N/2]: the split-K combine of a
// SiLU-gated GEMM.
template <bool BF16>
__global__ __launch_bounds__(256) void combine_silu_kernel(const float* __restrict__ partial, uint16_t* __restrict__ y,
                                                           int64_t mn, int64_t nh, int splits) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (o >= mn / 2) return;
    const int64_t gi = silu_gate_index(o, nh);
    float g = 0.f, u = 0.f;
    for (int k = 0; k < splits; ++k) {
        g += partial[(int64_t)k * mn + gi];
        u += partial[(int64_t)k * mn + gi + 8];
    }
    y[o] = f32_to_out<BF16>(silu_mul(g, u));
}

// y [M, N/2] = silu(gate) * up from a finished GEMM output h [M, N] (gate|up
// interleaved by 8), for plans whose GEMM cannot pair the columns itself.
template <bool BF16>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ h, uint16_t* __restrict__ y,
                                                       int64_t total, int64_t nh) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (o >= total) return;
    const int64_t gi = silu_gate_index(o, nh);
    y[o] = f32_to_out<BF16>(silu_mul(half_to_f32<BF16>(h[gi]), half_to_f32<BF16>(h[gi + 8])));
}

}  // namespace

size_t decode_lds_bytes(int M, int kps, int ngrp, bool zp, bool bf16, bool red_single, bool windowed, int k_perm) {
    const int mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    size_t b = x_slots(M, kps) * 16 * (windowed ? 2 : 1) + red_floats(mt) * 4 / (red_single ? 2 : 1);
    if (k_perm > 0) b += xn_slots(M, k_perm) * 16;
    return b;
}

int decode_perm_cols(int64_t K) {
    return K <= 8 * 2 * kThreads ? 2 : K <= 8 * kPermColsMax * kThreads ? kPermColsMax : 0;
}

int decode_threads() { return kThreads; }

int decode_blocks_per_cu(int layout, int xtype, int stype, bool zp, int mt, int ngrp, int ring, bool tree,
                         size_t lds, bool windowed, bool block_scales, int perm_cols) {
    const DecodeFn fn = pick_decode(layout, xtype, stype, zp, mt, ngrp, ring, tree, windowed, block_scales, perm_cols);
    if (fn == nullptr) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    static std::mutex mu;
    static std::map<std::tuple<int, const void*, size_t>, int> cache;
    const auto key = std::make_tuple(dev, (const void*)fn, lds);
    {
        std::lock_guard<std::mutex> lock(mu);
        auto it = cache.find(key);
        if (it != cache.end()) return it->second;
    }
    int n = 0;
    if (prepare(fn, lds) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void*)fn, kThreads + (windowed ? 64 * kCopyWaves : 0), lds) !=
            hipSuccess) {
        (void)hipGetLastError();  // do not leave the failure for the next launch check to report
        return 0;
    }
    std::lock_guard<std::mutex> lock(mu);
    cache[key] = n;
    return n;
}

hipError_t launch_decode(int layout, int xtype, int stype, bool zp, const DecodeConfig& cfg, const DecodeArgs& a,
                         hipStream_t stream, KernelEvents ev) {
    const bool win = cfg.kwin > 0;
    const DecodeFn fn =
        pick_decode(layout, xtype, stype, zp, cfg.mt, cfg.ngrp, cfg.ring, cfg.tree, win, cfg.block_scales, cfg.perm_cols);
    if (fn == nullptr) return hipErrorInvalidValue;
    // the kernel maps slots to rows with a multiply-high by spr_recip, exact
    // while slot * spr < 2^32
    const uint64_t spr = (uint64_t)a.kwin / 8 + 1;
    if (a.kwin <= 0 || a.kwin % 128 != 0 || x_slots(a.M, a.kwin) * spr >= (uint64_t{1} << 32)) {
        return hipErrorInvalidValue;
    }
    if (win) {
        // what the windowed kernel's barrier schedule rests on: one slice of
        // whole windows of real activations, every K wave the same number of
        // steps in every window, one unit per workgroup
        const int kwn = 8 / (a.nb / 16);
        const int64_t kext = (int64_t)a.ktiles * 32;
        const int64_t jw = (int64_t)a.kwin / 128 / kwn;
        if (a.splits != 1 || a.tree_levels != 0 || a.partial != nullptr || a.k_per_split != kext ||
            kext != a.K || kext % a.kwin != 0 || kext / a.kwin < 2 || jw < 1 || (int64_t{1} << a.jw_log2) != jw ||
            jw * 128 * kwn != a.kwin || a.ups != 1 || a.wps != a.ncg || a.M > 32) {
            return hipErrorInvalidValue;
        }
    } else if (a.kwin != a.k_per_split) {
        return hipErrorInvalidValue;
    }
    if (cfg.perm_cols) {
        // what the in-LDS gather rests on: one slice over all of K, x and the
        // permutation present, each thread's columns within the variant's, and
        // the LDS size holding XN behind the slice and the reduction buffers
        if (a.perm == nullptr || a.splits != 1 || a.k_per_split < a.K || a.K % 8 != 0 ||
            (int64_t)a.K > 8 * (int64_t)cfg.perm_cols * kThreads || a.M > 16 ||
            cfg.lds_bytes < decode_lds_bytes(a.M, a.kwin, cfg.ngrp, zp, xtype == X_BF16, cfg.red_single, false, a.K)) {
            return hipErrorInvalidValue;
        }
    } else if (a.perm != nullptr) {
        return hipErrorInvalidValue;
    }
    hipError_t e = prepare(fn, cfg.lds_bytes);
    if (e != hipSuccess) return e;
    launch_kernel(fn, dim3(a.wps, a.splits), dim3(kThreads + (win ? 64 * kCopyWaves : 0)), (uint32_t)cfg.lds_bytes, stream,
                  ev.start, ev.stop, a);
    return hipGetLastError();
}

hipError_t launch_combine_silu(const float* partial, uint16_t* y, int64_t M, int64_t N, int splits, int xtype,
                               hipStream_t stream) {
    if (N % 16 != 0) return hipErrorInvalidValue;
    const int64_t blocks = ceil_div(M * N / 2, 256);
    if (blocks == 0) return hipSuccess;
    if (xtype == X_BF16) {
        hipLaunchKernelGGL(combine_silu_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, partial, y, M * N,
                           N / 2, splits);
    } else {
        hipLaunchKernelGGL(combine_silu_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, partial, y, M * N,
                           N / 2, splits);
    }
    return hipGetLastError();
}

hipError_t launch_silu_mul(const uint16_t* h, uint16_t* y, int64_t M, int64_t N, int xtype, hipStream_t stream) {
    if (N % 16 != 0) return hipErrorInvalidValue;
    const int64_t blocks = ceil_div(M * N / 2, 256);
    if (blocks == 0) return hipSuccess;
    if (xtype == X_BF16) {
        hipLaunchKernelGGL(silu_mul_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, h, y, M * N / 2, N / 2);
    } else {
        hipLaunchKernelGGL(silu_mul_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, h, y, M * N / 2, N / 2);
    }
    return hipGetLastError();
}

hipError_t launch_combine(const float* partial, uint16_t* y, int64_t mn, int splits, int xtype,
                          hipStream_t stream, float* y32) {
    const int64_t blocks = ceil_div(ceil_div(mn, 4), 256);
    if (blocks == 0) return hipSuccess;
    if (xtype == X_BF16) {
        hipLaunchKernelGGL(combine_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, partial, y, mn, splits,
                           y32);
    } else {
        hipLaunchKernelGGL(combine_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, partial, y, mn, splits,
                           y32);
    }
    return hipGetLastError();
}

}  // namespace pw4

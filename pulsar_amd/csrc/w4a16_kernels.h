// Internal launch interface between the C-ABI layer (capi.hip) and the
// kernel translation units.  Not part of the public header.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pw4 {

// Events that take one GEMM call's kernel timestamps (pw4_time_next_kernel):
// `start` the start of the call's first GEMM dispatch, `stop` the end of its
// last (a split-K combine or SiLU pass after it is not included).  Null: none.
struct KernelEvents {
    hipEvent_t start = nullptr, stop = nullptr;
    // pw4_observe_next_call: [M, N] fp32 that receives the accumulators each
    // y element is rounded from, or null (a diagnostic for the parity tests)
    float* y32 = nullptr;
};

// The events (and observation buffer) armed on the calling thread, which are
// disarmed: every GEMM and repack entry point takes them first, so they never
// outlive the call they were armed for.
KernelEvents take_kernel_events();

// hipLaunchKernelGGL, or hipExtLaunchKernelGGL when an event is given (that
// launch path costs the runtime more, so untimed launches do not take it).
template <typename F, typename... Args>
void launch_kernel(F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t stream, hipEvent_t start,
                   hipEvent_t stop, Args... args) {
    if (start != nullptr || stop != nullptr) {
        hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, start, stop, 0, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
}

enum XType : int { X_F16 = 0, X_BF16 = 1 };
enum SType : int { S_F32 = 0, S_F16 = 1 };

// Decode GEMM (M <= 32).  The columns are cut into units of nb (16, 32 or
// 64) and K into `splits` slices; a grid of wps x splits persistent
// workgroups of 8 waves, workgroup (w, s) taking slice s and the units
// w, w + wps, w + 2 wps, ...  With more than one slice, each workgroup writes
// an fp32 partial tile per unit and the last one to finish a unit sums the
// partials in slice order and stores y.
// Nibble masks for the exponent-splice dequant, passed at run time so the
// compiler keeps them in SGPRs (see bfi in gemm_decode.hip).
struct NibbleMasks {
    uint32_t lo = 0x000f000fu;  // nibbles 0 and 4 of a word
    uint32_t hi = 0x00f000f0u;  // nibbles 1 and 5
    uint32_t ct = 0x00f0000fu;  // low nibble of byte 0, high nibble of byte 2
};

struct DecodeArgs {
    const uint16_t* x;       // [M, K] fp16 / bf16 bits (already act-order permuted, unless perm is given)
    const int32_t* perm;     // act-order in LDS (DecodeConfig::perm_cols): the K permutation, x as given; else null
    const uint32_t* w;       // MARLIN words, or CT [N, K/8]
    const void* scales;      // MARLIN: [Kg, N]; CT: [N, Kg] fp32
    const uint32_t* qzeros;  // [Kg, N/8] (MARLIN, asymmetric) or null
    uint16_t* y;             // [M, N] output
    float* partial;          // [ncg, splits, M, nb] fp32, or null for the direct store
    int32_t* counters;       // [ncg] arrival counters (zero on entry, left zero)
    unsigned long long* slots;  // exchange tree [splits - 1][ncg][M * nb] (zero on entry, left
                                // zero), or null; used instead of partial/counters
    int tree_levels;         // log2(splits) with the exchange tree
    int red_single;          // one cross-wave reduction buffer (see decode_lds_bytes)
    int nb;                  // columns per unit: 16, 32 or 64
    int ncg;                 // units (column groups) per slice
    int wps;                 // workgroups per slice
    int ups;                 // units of the busiest workgroup: ceil(ncg / wps)
    uint32_t spr_recip;      // ceil(2^32 / (k_per_split / 8 + 1)): slot -> row without a divide
    int M, N, K, G, Kg;
    int G_log2;              // log2(G); G is a power of two on this path
    int ktiles;              // 32-wide K tiles present in the weight layout
    int nchunks;             // MARLIN: Kpad / 64
    int k_per_split;         // multiple of 128
    int rowstride;           // LDS row stride of the staged x, in halves (kwin + 8)
    int kwin;                // K of the staged x window: k_per_split, or a K window (windowed plans)
    int jw_log2;             // windowed plans: log2(steps per K wave per window)
    int splits;
    // SiLU-gated output (direct store only): the columns are gate|up
    // interleaved by 8 (fused columns 16j..16j+7 gate, 16j+8..16j+15 up) and
    // y is [M, N/2] = silu(gate) * up
    int silu;
    NibbleMasks masks;
    // [M, N] fp32, or null: the accumulators each stored y element was rounded
    // from (pw4_observe_next_call; not for SiLU-gated output)
    float* y32;
};

struct DecodeConfig {
    int nb;      // columns per unit
    int wps;     // workgroups per K slice
    int mt;      // 16-row M tiles per wave (1 or 2)
    int ngrp;    // quant groups per 128-K step (1 when G % 128 == 0, 2 when G == 64)
    int splits;  // K slices
    int k_per_split;
    int ring;    // weight-load ring depth in steps: 4 or 8
    // one scale (and zero-point) load per four ring steps, handed between lane
    // groups with ds_bpermute (MARLIN, G >= 128, not windowed); else one per step
    bool block_scales = false;
    // act-order gathered in LDS by the decode kernel itself (see DecodeArgs::perm):
    // the permutation's 16-byte columns per thread (decode_perm_cols), 0 for none
    int perm_cols = 0;
    bool red_single;
    bool tree;   // K slices through the exchange tree (splits a power of two, M <= 32)
    // K window of a windowed plan, 0 for none: one slice, one unit per
    // workgroup, the activations staged window by window into two LDS buffers
    // by copy waves beside the eight compute waves (MARLIN layout, M <= 32,
    // NGRP <= 2)
    int kwin;
    size_t lds_bytes;
};

// LDS bytes of one decode workgroup for an M x kps activation slice, and its
// thread count.
// red_single: one cross-wave reduction buffer instead of two (one more
// barrier per unit), for plans whose activation slice leaves no room.
// windowed: kps is the K window, staged in two buffers.
// k_perm: K of x as given, staged whole for the in-LDS act-order gather, or 0.
size_t decode_lds_bytes(int M, int kps, int ngrp, bool zp, bool bf16, bool red_single, bool windowed = false,
                        int k_perm = 0);
// Permutation columns per thread of the in-LDS act-order gather for K (2 or
// 8), or 0 past what it takes.
int decode_perm_cols(int64_t K);
int decode_threads();
// Resident decode workgroups per CU for the kernel variant and LDS size
// (0 when the variant does not exist or the runtime cannot tell).
int decode_blocks_per_cu(int layout, int xtype, int stype, bool zp, int mt, int ngrp, int ring, bool tree,
                         size_t lds, bool windowed = false, bool block_scales = false, int perm_cols = 0);

hipError_t launch_decode(int layout, int xtype, int stype, bool zp, const DecodeConfig& cfg, const DecodeArgs& a,
                         hipStream_t stream, KernelEvents ev = {});
// y32: null, or an fp32 copy of each sum before it is rounded into y.
hipError_t launch_combine(const float* partial, uint16_t* y, int64_t mn, int splits, int xtype, hipStream_t stream,
                          float* y32 = nullptr);
// The same fixed-order sum over [splits, M, N] partials of gate|up interleaved
// columns (N % 16 == 0), writing y [M, N/2] = silu(gate) * up.
hipError_t launch_combine_silu(const float* partial, uint16_t* y, int64_t M, int64_t N, int splits, int xtype,
                               hipStream_t stream);
// y [M, N/2] = silu(gate) * up from a GEMM output h [M, N] in the same
// interleaved column order, h and y in x's dtype.
hipError_t launch_silu_mul(const uint16_t* h, uint16_t* y, int64_t M, int64_t N, int xtype, hipStream_t stream);

// Prefill GEMM (large M): 128 x 128 output tile per workgroup, BK = 64.
struct PrefillArgs {
    const uint16_t* x;       // [M, K] (already act-order permuted when needed)
    const uint32_t* w;
    const void* scales;
    const uint32_t* qzeros;
    uint16_t* y;
    float* partial;          // [splits, M, N] when splits > 1
    int M, N, K, G, Kg;
    int ktiles;
    int nchunks;
    int chunks_per_split;    // in 64-K chunks
    int splits;
    int n_begin, n_end;      // output columns a launch covers (set by the 256-tile launcher)
    int cus;                 // compute units of the device (tail balancing)
    int tile_rows;           // 256-wide kernel: 256-row tiles (tail balanced when unsplit) or 128-row tiles
    int k_halves;            // 256-wide kernel, 128-row tiles: 2 runs each K slice as two halves in one
                             // 8-wave workgroup summed through LDS, else 1
    int silu;                // 256-wide kernel, unsplit: y [M, N/2] = silu(gate) * up (see DecodeArgs)
    int exact;               // 256-wide kernel, fp16 x: B = u - z and the scale applied to the fp32
                             // accumulators per group
    float* y32;              // [M, N] fp32 copy of the unsplit output before rounding, or null
};

hipError_t launch_prefill(int layout, int xtype, int stype, bool zp, const PrefillArgs& a, hipStream_t stream,
                          KernelEvents ev = {});
int prefill_tile_m();
int prefill_tile_n();

// Prefill GEMM on a 256 x 256 output tile (MARLIN layout, fp16 or bf16 activations,
// K and the group size multiples of 64).  Same arguments as launch_prefill.
bool prefill256_ok(int layout, int xtype, int64_t N, int64_t K, int64_t G);
int prefill256_tile();
// Unsplit 256-row launches: N-tile columns run as 128-row tail tiles, and the
// launch's cost in waves of full tiles (into *waves when not null).
int64_t prefill256_tail_cols(int64_t M, int64_t N, int cus, double* waves);
hipError_t launch_prefill256(int xtype, int stype, bool zp, const PrefillArgs& a, hipStream_t stream,
                             KernelEvents ev = {});

// x_out[m, j] = x[m, perm[j]].  staged: 1 stages each source row in LDS (when
// K * 2 <= 64 KB and the pointers are 16-byte aligned), 0 reads it directly,
// -1 picks staged for M > kGatherStagedMinM.
constexpr int kGatherStagedMinM = 16;
hipError_t launch_gather_x(const uint16_t* x, const int32_t* perm, uint16_t* out, int M, int K, hipStream_t stream,
                           int staged = -1);

// Repack kernels.
// Compressed-tensors words [N, K/8] -> MARLIN words, and scales [N, K/G]
// (stype_in 0 fp32, 1 fp16, 2 bf16) -> fp32 [K/G, N], in one launch.
// `start` / `stop`: events the launch hands to hipExtLaunchKernel (the
// dispatch's start / end timestamps), or null.
hipError_t launch_repack_ct(const uint32_t* packed, const void* ws, int stype_in, uint32_t* wm, float* sm, int N,
                            int K, int G, hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// perm (act-order) takes an LDS-staged kernel sized by `cus`, the device's CU count.
// cols_override / grid_override (tuning sweeps and tests; 0 = heuristic): the
// act-order kernel's column block width (8, 16, 32 or 64) and its number of
// workgroups (each walks the blocks gridDim.x apart).
hipError_t launch_repack_gptq(const uint32_t* qweight, const int32_t* perm, uint32_t* wm, int N, int K,
                              hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr,
                              int cus = 256, int cols_override = 0, int grid_override = 0);
hipError_t launch_gidx_perm(const int32_t* g_idx, int32_t* perm, int32_t* status, int K, int G, hipStream_t stream);

}  // namespace pw4

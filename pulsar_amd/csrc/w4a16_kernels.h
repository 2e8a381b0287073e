// Internal launch interface between the C-ABI layer (capi.hip) and the
// kernel translation units.  Not part of the public header.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pw4 {

enum XType : int { X_F16 = 0, X_BF16 = 1 };
enum SType : int { S_F32 = 0, S_F16 = 1 };

// Decode GEMM (M <= 64): one workgroup = 4 waves = one 64-column block x one
// K slice; wave w owns columns 16w..16w+15 of the block.  With more than one
// K slice, each workgroup writes an fp32 partial tile and the last one to
// finish for a column block sums the partials in slice order and stores y.
struct DecodeArgs {
    const uint16_t* x;       // [M, K] fp16 / bf16 bits
    const uint32_t* w;       // MARLIN words, or CT [N, K/8]
    const void* scales;      // MARLIN: [Kg, N]; CT: [N, Kg] fp32
    const uint32_t* qzeros;  // [Kg, N/8] (MARLIN, asymmetric) or null
    const int32_t* perm;     // [K] act-order gather of x, or null
    uint16_t* y;             // [M, N] output
    float* partial;          // [cols, splits, M, 64] fp32, or null for the direct store
    int32_t* counters;       // [cols] arrival counters (zero on entry, left zero)
    int M, N, K, G, Kg;
    int G_log2;              // log2(G) when G is a power of two, else -1
    int ktiles;              // 32-wide K tiles present in the weight layout
    int nchunks;             // MARLIN: Kpad / 64
    int k_per_split;         // multiple of 128
    int rowstride;           // LDS row stride of the staged x, in halves
    int splits;
};

struct DecodeConfig {
    int mt;      // 16-row M tiles per wave (1, 2, 4)
    int ngrp;    // quant groups per 128-K step (1 when G % 128 == 0, 2 when G == 64)
    int splits;  // K slices (grid.y)
    int k_per_split;
    size_t lds_bytes;
};

// LDS bytes the decode kernel needs for an M x kps activation slice.
size_t decode_lds_bytes(int M, int kps, int ngrp, bool zp);

hipError_t launch_decode(int layout, int xtype, int stype, bool zp, const DecodeConfig& cfg, const DecodeArgs& a,
                         int grid_x, hipStream_t stream);
hipError_t launch_combine(const float* partial, uint16_t* y, int64_t mn, int splits, int xtype, hipStream_t stream);

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
};

hipError_t launch_prefill(int layout, int xtype, int stype, bool zp, const PrefillArgs& a, hipStream_t stream);
int prefill_tile_m();
int prefill_tile_n();

// x_out[m, j] = x[m, perm[j]]
hipError_t launch_gather_x(const uint16_t* x, const int32_t* perm, uint16_t* out, int M, int K, hipStream_t stream);

// Repack kernels.
hipError_t launch_repack_ct(const uint32_t* packed, uint32_t* wm, int N, int K, hipStream_t stream);
hipError_t launch_repack_gptq(const uint32_t* qweight, const int32_t* perm, uint32_t* wm, int N, int K,
                              hipStream_t stream);
hipError_t launch_scale_transpose(const void* ws, int stype_in, float* sm, int N, int Kg, hipStream_t stream);
hipError_t launch_gidx_perm(const int32_t* g_idx, int32_t* perm, int32_t* status, int K, int G, hipStream_t stream);

}  // namespace pw4

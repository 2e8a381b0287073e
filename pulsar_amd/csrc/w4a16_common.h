// Device-side building blocks shared by the W4A16 kernels (gfx950 / CDNA4).
//
// Weight layouts the kernels read:
//   * MARLIN -- the reference fragment layout produced by repack_w4a16
//     (reference pulsar-core/src/kernels/w4a16_marlin.cu:27-54).  Word order is
//     column block (64 cols) > K chunk (64) > K tile (2 x 32) > N subtile
//     (8 x 8 cols) > lane (32).  For column n and 32-wide K tile t the four
//     words tg = 0..3 are 16 contiguous bytes; word tg holds nibbles whose K
//     offsets, in the order the dequant below emits them, are
//       {2tg, 2tg+1, 8+2tg, 9+2tg, 16+2tg, 17+2tg, 24+2tg, 25+2tg}.
//     Stored nibbles are unsigned u (signed value + 8).
//   * CT -- the compressed-tensors packing [N, K/8] int32, nibble k%8 of word
//     [n, k/8], two's complement (reference w4a16_gemm.cu:20-26).  Word j of
//     a 32-K tile, after the dequant below, yields K offsets
//       8j + {0, 4, 1, 5, 2, 6, 3, 7}.
//
// MFMA K slots carry whatever K order the weight word yields; the activation
// tile is stored in LDS in the same order (a permutation inside each 32-K
// tile), so a lane's eight A halves are one 16-byte LDS read.  The dot product
// does not depend on the order of K, only on A and B agreeing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pw4 {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum Layout : int { LAYOUT_MARLIN = 0, LAYOUT_CT = 1 };

constexpr int kMarlinBN = 64;     // columns per Marlin column block
constexpr int kMarlinBK = 64;     // K per Marlin chunk
constexpr int kChunkWords = 512;  // int32 words per (column block, chunk)

__host__ __device__ inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
__host__ __device__ inline int64_t ceil_div(int64_t v, int64_t m) { return (v + m - 1) / m; }

template <typename T>
__device__ __forceinline__ T bitcast(const auto& v) {
    return __builtin_bit_cast(T, v);
}

__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// ---- MFMA wrappers ---------------------------------------------------------
// v_mfma_f32_16x16x32_{f16,bf16}: lane l supplies A row l%16 / B column l%16
// with K block l/16 (8 values); D lane l holds column l%16, rows 4*(l/16)+i.
template <bool BF16>
__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4& a, const u32x4& b, const f32x4& c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
    }
}

// v_mfma_f32_32x32x16_{f16,bf16}: lane l supplies A row l%32 / B column l%32
// with K block l/32; D lane l holds column l%32, rows 8*(i/4) + 4*(l/32) + i%4.
template <bool BF16>
__device__ __forceinline__ f32x16 mfma32x32x16(const u32x4& a, const u32x4& b, const f32x16& c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
    }
}

// ---- int4 -> 16-bit dequant ------------------------------------------------
// The exponent-splice trick (published with the FasterTransformer / AWQ
// kernels): OR-ing a nibble into the mantissa of 1024.0 (fp16 0x6400) gives
// the exact value 1024 + n; a nibble at bit 4 gives 1024 + 16n.  Each word
// yields the pairs (n0,n4) (n1,n5) (n2,n6) (n3,n7).

// fp16 with the group scale folded in (one rounding, like the reference's
// q*scale -> fp16 B fragment, w4a16_marlin.cu:103-113).  s_lo scales pairs 0,1
// and s_hi pairs 2,3 (the two 16-K halves of the tile for the MARLIN layout).
__device__ __forceinline__ u32x4 dq_f16_scaled(uint32_t q, uint32_t z1024, uint32_t z64, f16x2 s_lo, f16x2 s_hi) {
    const uint32_t q8 = q >> 8;
    const f16x2 sixteenth = as_h2(0x2c002c00u);
    u32x4 r;
    r[0] = as_u32((as_h2((q & 0x000f000fu) | 0x64006400u) - as_h2(z1024)) * s_lo);
    r[1] = as_u32((as_h2((q & 0x00f000f0u) | 0x64006400u) * sixteenth - as_h2(z64)) * s_lo);
    r[2] = as_u32((as_h2((q8 & 0x000f000fu) | 0x64006400u) - as_h2(z1024)) * s_hi);
    r[3] = as_u32((as_h2((q8 & 0x00f000f0u) | 0x64006400u) * sixteenth - as_h2(z64)) * s_hi);
    return r;
}

// bf16, biased: out = 128 + u (exact in bf16: 0x4300 is 128.0 and the nibble
// lands in the low mantissa bits).  The kernel removes (128 + z) * sum(x)
// per group in fp32.
__device__ __forceinline__ u32x4 dq_bf16_biased(uint32_t q) {
    u32x4 r;
    r[0] = (q & 0x000f000fu) | 0x43004300u;
    r[1] = ((q >> 4) & 0x000f000fu) | 0x43004300u;
    r[2] = ((q >> 8) & 0x000f000fu) | 0x43004300u;
    r[3] = ((q >> 12) & 0x000f000fu) | 0x43004300u;
    return r;
}

__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
    // v_cvt_pk_bf16_f32 rounds to nearest even.
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    bf16x2 v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// bf16 with the group scale folded in: ((128+u) - (128+z)) * s in fp32, then
// one rounding to bf16.  zf = 128 + z.
__device__ __forceinline__ u32x4 dq_bf16_scaled(uint32_t q, float zf, float s_lo, float s_hi) {
    const u32x4 b = dq_bf16_biased(q);
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float s = i < 2 ? s_lo : s_hi;
        const float lo = (__builtin_bit_cast(float, b[i] << 16) - zf) * s;
        const float hi = (__builtin_bit_cast(float, b[i] & 0xffff0000u) - zf) * s;
        r[i] = pack_bf16x2_rne(lo, hi);
    }
    return r;
}

// ---- activation permutation inside a 32-K tile -------------------------------
// Input: the tile's 16 dwords (pairs of consecutive halves) d[0..15].
// MARLIN: the lane that holds word tg reads pairs {tg, 4+tg, 8+tg, 12+tg}; store
//   pair q at position (q%4)*4 + q/4 so those four pairs are contiguous.
// CT: word j needs halves 8j + {0,4,1,5,2,6,3,7}; store each 8-half group in
//   that order.
template <int LAYOUT>
__device__ __forceinline__ void permute_tile(const u32x4 in[4], u32x4 out[4]) {
    if constexpr (LAYOUT == LAYOUT_MARLIN) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) out[j][i] = in[i][j];
    } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t d0 = in[g][0], d1 = in[g][1], d2 = in[g][2], d3 = in[g][3];
            out[g][0] = (d0 & 0xffffu) | (d2 << 16);
            out[g][1] = (d0 >> 16) | (d2 & 0xffff0000u);
            out[g][2] = (d1 & 0xffffu) | (d3 << 16);
            out[g][3] = (d1 >> 16) | (d3 & 0xffff0000u);
        }
    }
}

template <typename T>
__device__ __forceinline__ float load_scale(const T* p) {
    if constexpr (sizeof(T) == 4) {
        return *p;
    } else if constexpr (__is_same(T, _Float16)) {
        return (float)*p;
    } else {
        return __builtin_bit_cast(float, (uint32_t)(*reinterpret_cast<const uint16_t*>(p)) << 16);
    }
}

// silu(g) * u in fp32: g * u / (1 + e^-g), e^-g as 2^(-g log2 e) on the
// hardware exp2 and the quotient through the hardware reciprocal (1 ulp; the
// result is rounded to 16 bits).  For g below about -88 the exponential
// overflows to +inf and the product is -0 (the limit), for g above about 88 it
// is 0 and the result is g * u.
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
    return g * u * __builtin_amdgcn_rcpf(1.0f + e);
}

template <bool BF16>
__device__ __forceinline__ uint16_t f32_to_out(float v) {
    if constexpr (BF16) {
        return __builtin_bit_cast(uint16_t, (__bf16)v);
    } else {
        return __builtin_bit_cast(uint16_t, (_Float16)v);
    }
}

}  // namespace pw4

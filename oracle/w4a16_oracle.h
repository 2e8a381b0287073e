/*
 * CPU oracle for the W4A16 linear-layer path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, in plain C, the reference algorithm for every step of
 * the W4A16 path so the HIP kernels can be checked against it.  Only the test
 * suite, the smoke check and the benchmark's CPU-baseline leg may load it, and
 * only as the checker; the product library never links or calls it.
 *
 * Reference files followed (paths relative to the reference checkout):
 *   packing convention    pulsar-core/src/kernels/w4a16_gemm.cu:18-36,53-57
 *                         pulsar/tests/test_w4a16_gemm.py:41-53 (_pack_int4)
 *   dequant + fp32 GEMM   pulsar/tests/test_w4a16_gemm.py:56-62 (_oracle)
 *   Marlin repack         pulsar-core/src/kernels/w4a16_marlin.cu:27-54,128-185,373-375
 *   Marlin inverse map    pulsar/tests/test_w4a16_marlin.py:137-171
 *   split-K semantics     pulsar-core/src/kernels/w4a16_common.cuh:94-132
 *
 * Extensions with no counterpart in the reference (asymmetric zero points,
 * GPTQ qweight/qzeros packing, act-order g_idx) follow the public GPTQ
 * checkpoint convention and are pinned by invariants (see the header of each
 * function and tests/test_oracle.py).
 */
#ifndef PULSAR_W4A16_ORACLE_H
#define PULSAR_W4A16_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (IEEE round-to-nearest-even) ---------------------- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n);
void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n);
void orc_f32_to_bf16_n(const float* src, uint16_t* dst, int64_t n);
void orc_bf16_to_f32_n(const uint16_t* src, float* dst, int64_t n);

/* ---- seeded synthetic data (splitmix64 stream) ---------------------------- */
/* Fills `out` with n samples.  Every call with the same (seed, stream) pair
 * produces the same values on every host. */
void orc_fill_normal(uint64_t seed, uint64_t stream, float mean, float std, float* out, int64_t n);
void orc_fill_uint4(uint64_t seed, uint64_t stream, uint8_t* out, int64_t n); /* U{0..15} */
/* |N(0, std)| + offset : the BASELINE scale distribution */
void orc_fill_abs_normal(uint64_t seed, uint64_t stream, float std, float offset, float* out, int64_t n);
/* random permutation of 0..n-1 (Fisher-Yates driven by the same stream) */
void orc_fill_perm(uint64_t seed, uint64_t stream, int32_t* out, int64_t n);

/* ---- compressed-tensors packing: int32 [N, K/8], signed nibbles ----------- */
/* vals [N,K] in [-8,7]; nibble k%8 of word [n, k/8], LSB-first, two's complement */
int orc_pack_ct(const int8_t* vals, int64_t N, int64_t K, int32_t* packed);
int orc_unpack_ct(const int32_t* packed, int64_t N, int64_t K, int8_t* vals);

/* ---- GPTQ packing --------------------------------------------------------- */
/* u [N,K] in [0,15] -> qweight [K/8, N]: nibble k%8 of word [k/8, n] = u[n,k] */
int orc_pack_gptq(const uint8_t* u, int64_t N, int64_t K, int32_t* qweight);
int orc_unpack_gptq(const int32_t* qweight, int64_t N, int64_t K, uint8_t* u);
/* z [Kg,N] in [0,15] -> qzeros [Kg, N/8]: nibble n%8 of word [g, n/8] = z[g,n] */
int orc_pack_gptq_zeros(const uint8_t* z, int64_t Kg, int64_t N, int32_t* qzeros);
int orc_unpack_gptq_zeros(const int32_t* qzeros, int64_t Kg, int64_t N, uint8_t* z);
/* compressed-tensors [N,K/8] signed <-> GPTQ [K/8,N] unsigned (u = signed + 8) */
int orc_ct_to_gptq(const int32_t* packed, int64_t N, int64_t K, int32_t* qweight);

/* ---- Marlin fragment layout (reference repack) --------------------------- */
#define ORC_MARLIN_BN 64
#define ORC_MARLIN_BK 64
#define ORC_MARLIN_KTILE 32
#define ORC_MARLIN_NSUB 8
int64_t orc_marlin_words(int64_t N, int64_t K); /* roundup(N,64)*roundup(K,64)/8 */
/* Forward map from the compressed-tensors packing (reference repack_weight_kernel). */
int orc_repack_marlin(const int32_t* packed, int64_t N, int64_t K, int32_t* wm);
/* Forward map from per-element unsigned nibbles u[N,K] (u = stored Marlin nibble). */
int orc_marlin_from_u(const uint8_t* u, int64_t N, int64_t K, int32_t* wm);
/* Inverse map: Marlin words -> stored nibbles u[N,K] (padding discarded). */
int orc_marlin_to_u(const int32_t* wm, int64_t N, int64_t K, uint8_t* u);
/* scale_marlin[g, n] = weight_scale[n, g] */
int orc_scale_transpose(const float* ws, int64_t N, int64_t Kg, float* sm);

/* ---- act-order ------------------------------------------------------------ */
/* perm = stable argsort(g_idx).  Returns 0 on success, -2 if some group id is
 * out of [0, K/G) or some group does not hold exactly G rows. */
int orc_gidx_perm(const int32_t* g_idx, int64_t K, int64_t G, int32_t* perm);
/* GPTQ qweight [K/8,N] (+ optional perm [K]) -> Marlin words.  Row j of the
 * repacked matrix is original row perm[j] (identity when perm == NULL). */
int orc_repack_gptq_marlin(const int32_t* qweight, const int32_t* perm, int64_t N, int64_t K, int32_t* wm);

/* ---- dequantization ------------------------------------------------------- */
/* w[n,k] = int4(packed[n,k]) * scale[n, k/G]   (reference _oracle) */
int orc_dequant_ct(const int32_t* packed, const float* scale, int64_t N, int64_t K, int64_t G, float* w);
/* w[n,k] = (u[n,k] - z[g,n]) * s[g,n],  g = g_idx ? g_idx[k] : k/G.
 * scales [Kg,N] fp32; qzeros [Kg,N/8] or NULL for the implicit zero 8. */
int orc_dequant_gptq(
    const int32_t* qweight, const float* scales, const int32_t* qzeros, const int32_t* g_idx,
    int64_t N, int64_t K, int64_t G, float* w);

/* ---- fp32 GEMM: y[M,N] = x[M,K] @ w[N,K]^T (OpenMP, blocked) ------------- */
void orc_gemm_f32(const float* x, const float* w, int64_t M, int64_t N, int64_t K, float* y);
/* K-split restatement: sum over `splits` contiguous K-chunk runs of BK=64,
 * added in fixed split order (w4a16_common.cuh:94-132). */
void orc_gemm_f32_split(const float* x, const float* w, int64_t M, int64_t N, int64_t K, int splits, float* y);

/* Fused restatement used for the CPU baseline: dequantize the compressed-
 * tensors weights into `wbuf` [N,K] then run the fp32 GEMM. */
void orc_w4a16_ct_forward(
    const float* x, const int32_t* packed, const float* scale, int64_t M, int64_t N, int64_t K, int64_t G,
    float* wbuf, float* y);

int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif

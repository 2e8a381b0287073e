/*
 * CPU oracle for the W4A16 linear-layer path -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
 * this file, and only as the checker.  The product path never calls it.
 * Reference citations per function are in w4a16_oracle.h and below.
 */
#include "w4a16_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* IEEE-754 conversions, round to nearest even.                               */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
    }
    const int e = (int)exp - 127 + 15;
    if (e >= 31) {
        return (uint16_t)(sign | 0x7c00u);
    }
    if (e <= 0) { /* half subnormal or zero */
        if (e < -10) {
            return (uint16_t)sign;
        }
        man |= 0x800000u;
        const int shift = 14 - e;
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1u))) {
            ++h;
        }
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        ++h; /* a carry into the exponent is the correct rounding */
    }
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do {
                ++e;
                man <<= 1;
            } while ((man & 0x400u) == 0);
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 0x1fu) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu)) {
        return (uint16_t)((x >> 16) | 0x40u); /* quiet nan */
    }
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    const uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n) {
#pragma omp parallel for if (n > (1 << 16))
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}
void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n) {
#pragma omp parallel for if (n > (1 << 16))
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}
void orc_f32_to_bf16_n(const float* src, uint16_t* dst, int64_t n) {
#pragma omp parallel for if (n > (1 << 16))
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_bf16(src[i]);
}
void orc_bf16_to_f32_n(const uint16_t* src, float* dst, int64_t n) {
#pragma omp parallel for if (n > (1 << 16))
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_bf16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------- */
/* splitmix64 (Steele, Lea, Flood 2014; public-domain constants).             */

static uint64_t sm_next(uint64_t* s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static uint64_t sm_init(uint64_t seed, uint64_t stream) {
    uint64_t s = seed ^ (stream * 0xd1b54a32d192ed03ull);
    (void)sm_next(&s);
    return s;
}

/* uniform double in (0, 1] */
static double sm_unit(uint64_t* s) {
    return ((double)(sm_next(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void orc_fill_normal(uint64_t seed, uint64_t stream, float mean, float std, float* out, int64_t n) {
    uint64_t s = sm_init(seed, stream);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = sm_unit(&s), u2 = sm_unit(&s);
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + std * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + std * r * sin(two_pi * u2));
    }
}

void orc_fill_abs_normal(uint64_t seed, uint64_t stream, float std, float offset, float* out, int64_t n) {
    orc_fill_normal(seed, stream, 0.0f, std, out, n);
    for (int64_t i = 0; i < n; ++i) out[i] = fabsf(out[i]) + offset;
}

void orc_fill_uint4(uint64_t seed, uint64_t stream, uint8_t* out, int64_t n) {
    uint64_t s = sm_init(seed, stream);
    uint64_t bits = 0;
    int left = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (left == 0) {
            bits = sm_next(&s);
            left = 16;
        }
        out[i] = (uint8_t)(bits & 0xfu);
        bits >>= 4;
        --left;
    }
}

void orc_fill_perm(uint64_t seed, uint64_t stream, int32_t* out, int64_t n) {
    uint64_t s = sm_init(seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = (int32_t)i;
    for (int64_t i = n - 1; i > 0; --i) {
        const int64_t j = (int64_t)(sm_next(&s) % (uint64_t)(i + 1));
        const int32_t t = out[i];
        out[i] = out[j];
        out[j] = t;
    }
}

/* ------------------------------------------------------------------------- */
/* compressed-tensors packing (test_w4a16_gemm.py:41-53; w4a16_gemm.cu:20-26,53-57) */

int orc_pack_ct(const int8_t* vals, int64_t N, int64_t K, int32_t* packed) {
    if (K % 8) return -1;
    const int64_t W = K / 8;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t w = 0; w < W; ++w) {
            uint32_t word = 0;
            for (int j = 0; j < 8; ++j) {
                word |= ((uint32_t)vals[n * K + w * 8 + j] & 0xfu) << (4 * j);
            }
            packed[n * W + w] = (int32_t)word;
        }
    }
    return 0;
}

int orc_unpack_ct(const int32_t* packed, int64_t N, int64_t K, int8_t* vals) {
    if (K % 8) return -1;
    const int64_t W = K / 8;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            const int nib = (int)(((uint32_t)packed[n * W + k / 8] >> (4 * (k % 8))) & 0xfu);
            vals[n * K + k] = (int8_t)(nib >= 8 ? nib - 16 : nib);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* GPTQ packing: qweight [K/8, N] unsigned nibbles along K; qzeros [Kg, N/8]. */

int orc_pack_gptq(const uint8_t* u, int64_t N, int64_t K, int32_t* qweight) {
    if (K % 8) return -1;
    for (int64_t r = 0; r < K / 8; ++r) {
        for (int64_t n = 0; n < N; ++n) {
            uint32_t word = 0;
            for (int j = 0; j < 8; ++j) word |= ((uint32_t)u[n * K + r * 8 + j] & 0xfu) << (4 * j);
            qweight[r * N + n] = (int32_t)word;
        }
    }
    return 0;
}

int orc_unpack_gptq(const int32_t* qweight, int64_t N, int64_t K, uint8_t* u) {
    if (K % 8) return -1;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            u[n * K + k] = (uint8_t)(((uint32_t)qweight[(k / 8) * N + n] >> (4 * (k % 8))) & 0xfu);
        }
    }
    return 0;
}

int orc_pack_gptq_zeros(const uint8_t* z, int64_t Kg, int64_t N, int32_t* qzeros) {
    if (N % 8) return -1;
    for (int64_t g = 0; g < Kg; ++g) {
        for (int64_t c = 0; c < N / 8; ++c) {
            uint32_t word = 0;
            for (int j = 0; j < 8; ++j) word |= ((uint32_t)z[g * N + c * 8 + j] & 0xfu) << (4 * j);
            qzeros[g * (N / 8) + c] = (int32_t)word;
        }
    }
    return 0;
}

int orc_unpack_gptq_zeros(const int32_t* qzeros, int64_t Kg, int64_t N, uint8_t* z) {
    if (N % 8) return -1;
    for (int64_t g = 0; g < Kg; ++g) {
        for (int64_t n = 0; n < N; ++n) {
            z[g * N + n] = (uint8_t)(((uint32_t)qzeros[g * (N / 8) + n / 8] >> (4 * (n % 8))) & 0xfu);
        }
    }
    return 0;
}

int orc_ct_to_gptq(const int32_t* packed, int64_t N, int64_t K, int32_t* qweight) {
    if (K % 8) return -1;
    const int64_t W = K / 8;
    for (int64_t r = 0; r < W; ++r) {
        for (int64_t n = 0; n < N; ++n) {
            /* signed two's-complement nibble s -> u = s + 8 == nibble ^ 8 */
            qweight[r * N + n] = (int32_t)((uint32_t)packed[n * W + r] ^ 0x88888888u);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Marlin layout (w4a16_marlin.cu:27-54 layout, :128-174 forward map,
 * :373-375 padded sizes; inverse in test_w4a16_marlin.py:144-171).
 *
 * Word order: column block cb (64 cols) > K chunk kc (64) > K tile kt (2 x 32)
 * > N subtile ns (8 x 8 cols) > lane (32).  Lane L covers column
 * cb*64 + ns*8 + L/4 and, with t = L%4, nibble p holds the K offset
 * (p%4)*8 + 2t + p/4 inside its 32-wide K tile.  Stored nibble = unsigned u
 * (signed + 8); rows/columns beyond N/K store 8.                            */

static int64_t roundup64(int64_t v) { return (v + 63) / 64 * 64; }

int64_t orc_marlin_words(int64_t N, int64_t K) { return roundup64(N) * roundup64(K) / 8; }

static int marlin_koff(int p, int t) { return (p % 4) * 8 + 2 * t + p / 4; }

typedef int (*nib_fn)(const void* ctx, int64_t n, int64_t k);

static void marlin_forward(nib_fn get, const void* ctx, int64_t N, int64_t K, int32_t* wm) {
    const int64_t ncb = roundup64(N) / 64, nkc = roundup64(K) / 64;
#pragma omp parallel for collapse(2) if (ncb * nkc > 64)
    for (int64_t cb = 0; cb < ncb; ++cb) {
        for (int64_t kc = 0; kc < nkc; ++kc) {
            int32_t* out = wm + (cb * nkc + kc) * 512;
            for (int kt = 0; kt < 2; ++kt) {
                for (int ns = 0; ns < 8; ++ns) {
                    for (int lane = 0; lane < 32; ++lane) {
                        const int64_t n = cb * 64 + ns * 8 + lane / 4;
                        const int64_t kb = kc * 64 + kt * 32;
                        uint32_t word = 0;
                        for (int p = 0; p < 8; ++p) {
                            const int64_t k = kb + marlin_koff(p, lane % 4);
                            const int nib = (n < N && k < K) ? get(ctx, n, k) : 8;
                            word |= ((uint32_t)nib & 0xfu) << (4 * p);
                        }
                        out[(kt * 8 + ns) * 32 + lane] = (int32_t)word;
                    }
                }
            }
        }
    }
}

typedef struct {
    const int32_t* p;
    int64_t W;
} ct_ctx;
static int ct_nib(const void* c, int64_t n, int64_t k) {
    const ct_ctx* x = (const ct_ctx*)c;
    return (int)((((uint32_t)x->p[n * x->W + k / 8] >> (4 * (k % 8))) & 0xfu) ^ 8u);
}

typedef struct {
    const uint8_t* u;
    int64_t K;
} u_ctx;
static int u_nib(const void* c, int64_t n, int64_t k) {
    const u_ctx* x = (const u_ctx*)c;
    return x->u[n * x->K + k];
}

typedef struct {
    const int32_t* q;
    const int32_t* perm;
    int64_t N;
} gptq_ctx;
static int gptq_nib(const void* c, int64_t n, int64_t k) {
    const gptq_ctx* x = (const gptq_ctx*)c;
    const int64_t src = x->perm ? x->perm[k] : k;
    return (int)(((uint32_t)x->q[(src / 8) * x->N + n] >> (4 * (src % 8))) & 0xfu);
}

int orc_repack_marlin(const int32_t* packed, int64_t N, int64_t K, int32_t* wm) {
    if (K % 8) return -1;
    ct_ctx c = {packed, K / 8};
    marlin_forward(ct_nib, &c, N, K, wm);
    return 0;
}

int orc_marlin_from_u(const uint8_t* u, int64_t N, int64_t K, int32_t* wm) {
    u_ctx c = {u, K};
    marlin_forward(u_nib, &c, N, K, wm);
    return 0;
}

int orc_marlin_to_u(const int32_t* wm, int64_t N, int64_t K, uint8_t* u) {
    const int64_t nkc = roundup64(K) / 64, total = orc_marlin_words(N, K);
    for (int64_t w = 0; w < total; ++w) {
        const int lane = (int)(w % 32), ns = (int)((w / 32) % 8), kt = (int)((w / 256) % 2);
        const int64_t kc = (w / 512) % nkc, cb = w / 512 / nkc;
        const int64_t n = cb * 64 + ns * 8 + lane / 4;
        for (int p = 0; p < 8; ++p) {
            const int64_t k = kc * 64 + kt * 32 + marlin_koff(p, lane % 4);
            if (n < N && k < K) u[n * K + k] = (uint8_t)(((uint32_t)wm[w] >> (4 * p)) & 0xfu);
        }
    }
    return 0;
}

int orc_scale_transpose(const float* ws, int64_t N, int64_t Kg, float* sm) {
    for (int64_t n = 0; n < N; ++n)
        for (int64_t g = 0; g < Kg; ++g) sm[g * N + n] = ws[n * Kg + g];
    return 0;
}

/* ------------------------------------------------------------------------- */
/* act-order                                                                  */

int orc_gidx_perm(const int32_t* g_idx, int64_t K, int64_t G, int32_t* perm) {
    if (G <= 0 || K % G) return -1;
    const int64_t Kg = K / G;
    int64_t* fill = (int64_t*)calloc((size_t)Kg, sizeof(int64_t));
    if (!fill) return -3;
    int rc = 0;
    for (int64_t k = 0; k < K && rc == 0; ++k) {
        const int32_t g = g_idx[k];
        if (g < 0 || g >= Kg || fill[g] >= G) {
            rc = -2;
        } else {
            perm[(int64_t)g * G + fill[g]++] = (int32_t)k; /* stable: ascending k per group */
        }
    }
    free(fill);
    return rc;
}

int orc_repack_gptq_marlin(const int32_t* qweight, const int32_t* perm, int64_t N, int64_t K, int32_t* wm) {
    if (K % 8) return -1;
    gptq_ctx c = {qweight, perm, N};
    marlin_forward(gptq_nib, &c, N, K, wm);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* dequantization (test_w4a16_gemm.py:56-62)                                  */

int orc_dequant_ct(const int32_t* packed, const float* scale, int64_t N, int64_t K, int64_t G, float* w) {
    if (K % 8 || G <= 0 || K % G) return -1;
    const int64_t W = K / 8, Kg = K / G;
#pragma omp parallel for if (N * K > (1 << 18))
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            const int nib = (int)(((uint32_t)packed[n * W + k / 8] >> (4 * (k % 8))) & 0xfu);
            const int v = nib >= 8 ? nib - 16 : nib;
            w[n * K + k] = (float)v * scale[n * Kg + k / G];
        }
    }
    return 0;
}

int orc_dequant_gptq(
    const int32_t* qweight, const float* scales, const int32_t* qzeros, const int32_t* g_idx,
    int64_t N, int64_t K, int64_t G, float* w) {
    if (K % 8 || G <= 0 || K % G || (qzeros && N % 8)) return -1;
    const int64_t Kg = K / G;
#pragma omp parallel for if (N * K > (1 << 18))
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t k = 0; k < K; ++k) {
            const int u = (int)(((uint32_t)qweight[(k / 8) * N + n] >> (4 * (k % 8))) & 0xfu);
            const int64_t g = g_idx ? g_idx[k] : k / G;
            if (g < 0 || g >= Kg) {
                w[n * K + k] = NAN;
                continue;
            }
            const int z = qzeros ? (int)(((uint32_t)qzeros[g * (N / 8) + n / 8] >> (4 * (n % 8))) & 0xfu) : 8;
            w[n * K + k] = (float)(u - z) * scales[g * N + n];
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* fp32 GEMM: register-blocked 4 rows x 2 columns, 8-wide K partial sums.     */

static void gemm_block(const float* x, const float* w, int64_t M, int64_t N, int64_t K, int64_t k0, int64_t k1,
                       float* y, int accumulate) {
    const int64_t mb = (M + 3) / 4, nb = (N + 1) / 2;
#pragma omp parallel for collapse(2) schedule(static) if (M * N * (k1 - k0) > (1 << 20))
    for (int64_t bn = 0; bn < nb; ++bn) {
        for (int64_t bm = 0; bm < mb; ++bm) {
            const int64_t m0 = bm * 4, n0 = bn * 2;
            float acc[4][2][8];
            memset(acc, 0, sizeof(acc));
            const float* xr[4];
            const float* wr[2];
            for (int i = 0; i < 4; ++i) xr[i] = x + (m0 + i < M ? m0 + i : m0) * K;
            for (int j = 0; j < 2; ++j) wr[j] = w + (n0 + j < N ? n0 + j : n0) * K;
            int64_t k = k0;
            for (; k + 8 <= k1; k += 8) {
                for (int i = 0; i < 4; ++i)
                    for (int j = 0; j < 2; ++j)
                        for (int l = 0; l < 8; ++l) acc[i][j][l] += xr[i][k + l] * wr[j][k + l];
            }
            float tail[4][2];
            memset(tail, 0, sizeof(tail));
            for (; k < k1; ++k)
                for (int i = 0; i < 4; ++i)
                    for (int j = 0; j < 2; ++j) tail[i][j] += xr[i][k] * wr[j][k];
            for (int i = 0; i < 4; ++i) {
                if (m0 + i >= M) continue;
                for (int j = 0; j < 2; ++j) {
                    if (n0 + j >= N) continue;
                    float s = 0.0f;
                    for (int l = 0; l < 8; ++l) s += acc[i][j][l];
                    s += tail[i][j];
                    float* dst = &y[(m0 + i) * N + n0 + j];
                    *dst = accumulate ? *dst + s : s;
                }
            }
        }
    }
}

void orc_gemm_f32(const float* x, const float* w, int64_t M, int64_t N, int64_t K, float* y) {
    gemm_block(x, w, M, N, K, 0, K, y, 0);
}

void orc_gemm_f32_split(const float* x, const float* w, int64_t M, int64_t N, int64_t K, int splits, float* y) {
    const int64_t nchunks = (K + 63) / 64;
    const int64_t cps = (nchunks + splits - 1) / splits;
    for (int64_t i = 0; i < M * N; ++i) y[i] = 0.0f;
    for (int s = 0; s < splits; ++s) {
        const int64_t c0 = (int64_t)s * cps;
        int64_t c1 = c0 + cps;
        if (c1 > nchunks) c1 = nchunks;
        if (c0 >= c1) continue; /* empty split contributes 0 */
        const int64_t k0 = c0 * 64, k1 = c1 * 64 < K ? c1 * 64 : K;
        gemm_block(x, w, M, N, K, k0, k1, y, 1);
    }
}

void orc_w4a16_ct_forward(
    const float* x, const int32_t* packed, const float* scale, int64_t M, int64_t N, int64_t K, int64_t G,
    float* wbuf, float* y) {
    orc_dequant_ct(packed, scale, N, K, G, wbuf);
    orc_gemm_f32(x, wbuf, M, N, K, y);
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

// One-time weight re-layout kernels.
//
// Both repacks emit the reference MARLIN word layout (pulsar-core/src/kernels/
// w4a16_marlin.cu:27-54): for column n and 32-wide K tile t the four words
// tg = 0..3 are 16 contiguous bytes at
//     ((n/64 * nchunks + t/2) * 512 + (t%2) * 256 + (n%64) * 4) words,
// and nibble p of word tg holds K offset (p%4)*8 + 2tg + p/4 of the tile, stored
// unsigned (signed + 8), with 8 in padding.  A thread builds those 16 bytes
// for one (n, t): if b_j is byte tg of source word j (K 8j..8j+7 of the tile),
// word tg = sum_j (b_j & 0xf) << 4j | (b_j >> 4) << (16 + 4j).
//
// The reference builds each word with eight scattered nibble reads
// (w4a16_marlin.cu:139-174); here a thread turns one (n, t) tile's four source
// words into its 16 output bytes in registers.  A workgroup takes a 64-column
// block and 16 tiles (512 K): for the CT layout its lanes read each source row
// as 256-byte runs, the transformed tiles pass through LDS, and each tile of
// the block leaves as one contiguous 1 KB run; GPTQ rows are [K/8, N], so
// lanes over n read them coalesced as they are and no LDS is needed.
#include "w4a16_common.h"
#include "w4a16_kernels.h"

namespace pw4 {
namespace {

__device__ __forceinline__ u32x4 transpose_tile_bytes(const uint32_t src[4]) {
    u32x4 out;
#pragma unroll
    for (int tg = 0; tg < 4; ++tg) {
        uint32_t w = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t b = (src[j] >> (8 * tg)) & 0xffu;
            w |= (b & 0xfu) << (4 * j);
            w |= (b >> 4) << (16 + 4 * j);
        }
        out[tg] = w;
    }
    return out;
}

__device__ __forceinline__ int64_t marlin_offset(int n, int t, int nchunks) {
    return ((int64_t)(n >> 6) * nchunks + (t >> 1)) * kChunkWords + (t & 1) * 256 + (n & 63) * 4;
}

constexpr int kRepackThreads = 256;
constexpr int kRepackTiles = 16;  // 32-K tiles per workgroup (a multiple of 2: whole MARLIN chunks)

// compressed-tensors [N, K/8] (signed) -> MARLIN, and the scales [N, K/G] ->
// scale_marlin [K/G, N] fp32 (w4a16_marlin.cu:177-185) in the same launch.
// grid: (Npad/64, Kpad/512 rounded up).
// Words.  Read: item r = (row r / 16, tile r % 16) of the block, 16 lanes per 256-byte
// run of a row.  Write: item r = (tile r / 64, column r % 64), 64 lanes per 1 KB run.
// LDS rows are padded by 16 bytes so the column-wise reads of the write phase spread
// over the banks.  VEC: rows are 16-byte aligned (K % 32 == 0, aligned base), so a
// whole tile of a row is one 16-byte load; otherwise every tile is read word by word.
// Scales.  A workgroup writes the groups whose first K lies in its 512-K range, for
// its 64 columns: 64 consecutive columns per write (one group per workgroup at G = 128).
template <bool VEC, typename T>
__global__ __launch_bounds__(kRepackThreads) void repack_ct_kernel(const uint32_t* __restrict__ packed,
                                                                   uint32_t* __restrict__ wm,
                                                                   const T* __restrict__ ws, float* __restrict__ sm,
                                                                   int N, int K, int G, int nchunks) {
    constexpr int kRow = kRepackTiles + 1;  // u32x4 per LDS row
    __shared__ u32x4 tiles[64 * kRow];
    const int n0 = blockIdx.x * 64, t0 = blockIdx.y * kRepackTiles;
    const int ktiles = nchunks * 2;  // tiles in the padded layout
    const int64_t rw = K / 8;        // source words per row
#pragma unroll
    for (int q = 0; q < 64 * kRepackTiles / kRepackThreads; ++q) {
        const int r = q * kRepackThreads + threadIdx.x;
        const int row = r / kRepackTiles, tt = r % kRepackTiles;
        const int n = n0 + row, t = t0 + tt;
        uint32_t src[4];
        if (VEC && n < N && t * 32 + 32 <= K) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(packed + (int64_t)n * rw + t * 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) src[j] = v[j] ^ 0x88888888u;  // signed s -> u = s ^ 8
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = t * 32 + j * 8;  // K % 8 == 0: a source word is all-in or all-out
                src[j] = (n < N && k < K) ? (packed[(int64_t)n * rw + k / 8] ^ 0x88888888u) : 0x88888888u;
            }
        }
        tiles[row * kRow + tt] = transpose_tile_bytes(src);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 64 * kRepackTiles / kRepackThreads; ++q) {
        const int r = q * kRepackThreads + threadIdx.x;
        const int tt = r / 64, col = r % 64;
        const int t = t0 + tt;
        if (t < ktiles) *reinterpret_cast<u32x4*>(wm + marlin_offset(n0 + col, t, nchunks)) = tiles[col * kRow + tt];
    }
    const int Kg = K / G;
    const int k_lo = t0 * 32, k_hi = k_lo + kRepackTiles * 32;
    const int g_lo = (k_lo + G - 1) / G, g_hi = min((k_hi + G - 1) / G, Kg);
    for (int i = threadIdx.x; i < (g_hi - g_lo) * 64; i += kRepackThreads) {
        const int g = g_lo + (i >> 6), n = n0 + (i & 63);
        if (n < N) sm[(int64_t)g * N + n] = load_scale(ws + (int64_t)n * Kg + g);
    }
}

// GPTQ qweight [K/8, N] (unsigned) -> MARLIN, rows gathered through perm when
// given (repacked row j = original row perm[j]).  grid: (Npad/64, Kpad/512 rounded
// up); thread (column i % 64, tile i / 64 + 4q) for q < 4: for each source row the
// 64 lanes of a wave read 256 contiguous bytes and write one 1 KB output run.
__global__ __launch_bounds__(kRepackThreads) void repack_gptq_kernel(const uint32_t* __restrict__ qweight,
                                                                     const int32_t* __restrict__ perm,
                                                                     uint32_t* __restrict__ wm, int N, int K,
                                                                     int nchunks) {
    const int n = blockIdx.x * 64 + (threadIdx.x & 63);
    const int ktiles = nchunks * 2;
#pragma unroll
    for (int q = 0; q < kRepackTiles / 4; ++q) {
        const int t = blockIdx.y * kRepackTiles + q * 4 + (threadIdx.x >> 6);
        if (t >= ktiles) break;
        uint32_t src[4];
        if (perm == nullptr) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int k = t * 32 + j * 8;
                src[j] = (n < N && k < K) ? qweight[(int64_t)(k / 8) * N + n] : 0x88888888u;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t w = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int k = t * 32 + j * 8 + e;
                    uint32_t nib = 8u;
                    if (n < N && k < K) {
                        const int sk = min(max(perm[k], 0), K - 1);  // clamped: a bad perm cannot fault
                        nib = (qweight[(int64_t)(sk >> 3) * N + n] >> (4 * (sk & 7))) & 0xfu;
                    }
                    w |= nib << (4 * e);
                }
                src[j] = w;
            }
        }
        *reinterpret_cast<u32x4*>(wm + marlin_offset(n, t, nchunks)) = transpose_tile_bytes(src);
    }
}

// GPTQ qweight [K/8, N] -> MARLIN through the act-order permutation: a
// workgroup takes NB columns over the whole K.  It stages the columns' source
// words (all K/8 rows) and the permutation (clamped to [0, K), 16 bits) in LDS,
// then assembles the MARLIN words from nibbles gathered in LDS, so each source
// word is read from HBM once (gathering straight from qweight reads it once per
// nibble).  A thread takes 4 adjacent columns of one 32-K tile: each 8-entry run
// of the permutation is one 16-byte LDS read shared by the tile's threads, and
// each source row one 16-byte read for the 4 columns.  grid: Npad/NB.
// Staging reads 4 adjacent columns of a row per 16-byte load (VEC: N % 4 == 0
// and 16-byte aligned qweight; otherwise word by word), 8 loads in flight per
// thread, and the permutation 4 entries per 16-byte load (K % 4 == 0 always:
// K % 8 == 0 on this path).
constexpr int kPermThreads = 512;
template <int NB, bool VEC>
__global__ __launch_bounds__(kPermThreads) void repack_gptq_perm_kernel(const uint32_t* __restrict__ qweight,
                                                                        const int32_t* __restrict__ perm,
                                                                        uint32_t* __restrict__ wm, int N, int K,
                                                                        int nchunks) {
    static_assert(NB % 4 == 0, "4 columns per thread");
    extern __shared__ __attribute__((aligned(16))) uint32_t lds_words[];
    const int k8 = K >> 3;
    uint32_t* sq = lds_words;                                      // [K/8][NB]
    uint16_t* sp = reinterpret_cast<uint16_t*>(lds_words + k8 * NB);  // [Kpad]
    const int kpad = nchunks * 64;
    const int n0 = blockIdx.x * NB;
    // staging, kStage loads in flight per thread before their LDS stores (a
    // store right behind its load would make every step a memory round trip)
    constexpr int kStage = 8;
    constexpr int kQuadsPerRow = NB / 4;
    const u32x4 pad4 = u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};  // padding: nibble 8
    for (int i0 = threadIdx.x; i0 < k8 * kQuadsPerRow; i0 += kPermThreads * kStage) {
        u32x4 v[kStage];
#pragma unroll
        for (int q = 0; q < kStage; ++q) {
            const int i = i0 + q * kPermThreads;
            const int r = i / kQuadsPerRow, c = (i % kQuadsPerRow) * 4;
            const uint32_t* src = qweight + (int64_t)r * N + n0 + c;
            v[q] = pad4;
            if (i < k8 * kQuadsPerRow) {
                if (VEC && n0 + c + 3 < N) {
                    v[q] = *reinterpret_cast<const u32x4*>(src);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n0 + c + e < N) v[q][e] = src[e];
                }
            }
        }
#pragma unroll
        for (int q = 0; q < kStage; ++q) {
            const int i = i0 + q * kPermThreads;
            if (i < k8 * kQuadsPerRow) *reinterpret_cast<u32x4*>(sq + (int64_t)i * 4) = v[q];
        }
    }
    // padding rows (k >= K) point at row 0 and are masked below
    for (int k0 = threadIdx.x * 4; k0 < kpad; k0 += kPermThreads * 4 * kStage) {
        u32x4 v[kStage];
#pragma unroll
        for (int q = 0; q < kStage; ++q) {
            const int k = k0 + q * kPermThreads * 4;
            v[q] = u32x4{0u, 0u, 0u, 0u};
            if (k < K) {  // K % 4 == 0: whole vectors
                if constexpr (VEC) {
                    v[q] = *reinterpret_cast<const u32x4*>(perm + k);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[q][e] = (uint32_t)perm[k + e];
                }
            }
        }
#pragma unroll
        for (int q = 0; q < kStage; ++q) {
            const int k = k0 + q * kPermThreads * 4;
            if (k < kpad) {
                uint32_t p2[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    // clamped: a bad perm cannot fault
                    const uint32_t a = (uint32_t)min(max((int)v[q][2 * h], 0), K - 1);
                    const uint32_t b = (uint32_t)min(max((int)v[q][2 * h + 1], 0), K - 1);
                    p2[h] = a | (b << 16);
                }
                *reinterpret_cast<u32x2*>(sp + k) = u32x2{p2[0], p2[1]};
            }
        }
    }
    __syncthreads();
    constexpr int kQuads = NB / 4;  // threads per tile
    const int ktiles = nchunks * 2;
    // Each gathered nibble goes straight to its MARLIN place: K offset 8j + e of
    // the tile (run j, entry e) is nibble j + 4 (e % 2) of word e / 2 -- the
    // word transpose_tile_bytes would build from source run j's byte e / 2.
    for (int i = threadIdx.x; i < ktiles * kQuads; i += kPermThreads) {
        const int t = i / kQuads, c0 = (i % kQuads) * 4;
        uint32_t out[4][4] = {};  // [column q][MARLIN word tg]
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kb = t * 32 + j * 8;
            if (kb >= K) {  // padding rows (K % 8 == 0: whole runs): nibble 8
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int tg = 0; tg < 4; ++tg) out[q][tg] |= (8u << (4 * j)) | (8u << (4 * j + 16));
                continue;
            }
            const u32x4 pk = *reinterpret_cast<const u32x4*>(sp + kb);  // 8 permutation entries
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int sk = (pk[e >> 1] >> (16 * (e & 1))) & 0xffff;
                const u32x4 row = *reinterpret_cast<const u32x4*>(sq + (sk >> 3) * NB + c0);
                const int sh = 4 * (sk & 7);
#pragma unroll
                for (int q = 0; q < 4; ++q) out[q][e >> 1] |= ((row[q] >> sh) & 0xfu) << (4 * j + 16 * (e & 1));
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            *reinterpret_cast<u32x4*>(wm + marlin_offset(n0 + c0 + q, t, nchunks)) =
                u32x4{out[q][0], out[q][1], out[q][2], out[q][3]};
        }
    }
}

// perm = stable argsort(g_idx) for an act-order checkpoint: one workgroup per
// group collects, in ascending k, the rows that belong to it.  status bit 0:
// some group does not hold exactly G rows; bit 1: a group id out of range.
// The entries are ranked 256 at a time in k order (ballot and popcount within a
// wave, counts of the earlier waves through LDS); a thread loads its entries of
// kGidxBatch such steps at once, so a step costs one barrier rather than a
// memory round trip, and the wave counts are double buffered so that one
// barrier per step suffices.
constexpr int kGidxBatch = 16;
__global__ __launch_bounds__(256) void gidx_perm_kernel(const int32_t* __restrict__ g_idx, int32_t* __restrict__ perm,
                                                        int32_t* __restrict__ status, int K, int G) {
    __shared__ int wave_cnt[2][4];
    const int g = blockIdx.x;
    const int Kg = K / G;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int base_count = 0;
    int buf = 0;
    for (int kb = 0; kb < K; kb += 256 * kGidxBatch) {
        int gv[kGidxBatch];
#pragma unroll
        for (int b = 0; b < kGidxBatch; ++b) {
            const int k = kb + b * 256 + tid;
            gv[b] = k < K ? g_idx[k] : -1;
        }
#pragma unroll
        for (int b = 0; b < kGidxBatch; ++b) {
            const int k = kb + b * 256 + tid;
            if (kb + b * 256 >= K) break;  // uniform: every thread leaves at the same step
            if (g == 0 && k < K && (gv[b] < 0 || gv[b] >= Kg)) atomicOr(status, 2);
            const bool mine = k < K && gv[b] == g;
            const uint64_t mask = __ballot(mine);
            const int before_lane = __popcll(mask & ((1ull << lane) - 1ull));
            if (lane == 0) wave_cnt[buf][wave] = __popcll(mask);
            __syncthreads();
            int before_wave = 0, total = 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                before_wave += w < wave ? wave_cnt[buf][w] : 0;
                total += wave_cnt[buf][w];
            }
            const int pos = base_count + before_wave + before_lane;
            if (mine && pos < G) perm[(int64_t)g * G + pos] = k;
            base_count += total;
            buf ^= 1;  // the next step writes the other buffer: no barrier before it
        }
    }
    if (tid == 0 && base_count != G) atomicOr(status, 1);
}

__global__ __launch_bounds__(64) void clear_status_kernel(int32_t* __restrict__ status) {
    if (threadIdx.x == 0) *status = 0;
}

}  // namespace

template <typename T>
void launch_repack_ct_typed(const uint32_t* packed, const T* ws, uint32_t* wm, float* sm, int N, int K, int G,
                            hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const int npad = (int)round_up(N, kMarlinBN), kpad = (int)round_up(K, kMarlinBK);
    const dim3 grid(npad / 64, (unsigned)ceil_div(kpad / 32, kRepackTiles));
    // the 16-byte row reads need 16-byte aligned rows: K % 32 == 0 and an aligned base
    if ((K % 32) != 0 || (reinterpret_cast<uintptr_t>(packed) & 15) != 0) {
        launch_kernel(repack_ct_kernel<false, T>, grid, dim3(kRepackThreads), 0, stream, start, stop, packed, wm, ws,
                      sm, N, K, G, kpad / kMarlinBK);
    } else {
        launch_kernel(repack_ct_kernel<true, T>, grid, dim3(kRepackThreads), 0, stream, start, stop, packed, wm, ws,
                      sm, N, K, G, kpad / kMarlinBK);
    }
}

hipError_t launch_repack_ct(const uint32_t* packed, const void* ws, int stype_in, uint32_t* wm, float* sm, int N,
                            int K, int G, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    if (N == 0 || K == 0) return hipSuccess;
    if (G <= 0 || K % G != 0) return hipErrorInvalidValue;
    switch (stype_in) {
        case 0: launch_repack_ct_typed(packed, reinterpret_cast<const float*>(ws), wm, sm, N, K, G, stream, start, stop); break;
        case 1: launch_repack_ct_typed(packed, reinterpret_cast<const _Float16*>(ws), wm, sm, N, K, G, stream, start, stop); break;
        case 2: launch_repack_ct_typed(packed, reinterpret_cast<const __bf16*>(ws), wm, sm, N, K, G, stream, start, stop); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

namespace {
template <int NB>
hipError_t launch_repack_gptq_perm(const uint32_t* qweight, const int32_t* perm, uint32_t* wm, int N, int K,
                                   int npad, int kpad, size_t lds, hipStream_t stream, hipEvent_t start,
                                   hipEvent_t stop) {
    // 16-byte staging loads: 4-column quads of a row and 4-entry runs of perm aligned
    const bool vec = N % 4 == 0 && ((reinterpret_cast<uintptr_t>(qweight) | reinterpret_cast<uintptr_t>(perm)) & 15) == 0;
    const auto fn = vec ? repack_gptq_perm_kernel<NB, true> : repack_gptq_perm_kernel<NB, false>;
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    launch_kernel(fn, dim3(npad / NB), dim3(kPermThreads), (uint32_t)lds, stream, start, stop, qweight, perm, wm, N,
                  K, kpad / kMarlinBK);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_repack_gptq(const uint32_t* qweight, const int32_t* perm, uint32_t* wm, int N, int K,
                              hipStream_t stream, hipEvent_t start, hipEvent_t stop, int cus) {
    const int npad = (int)round_up(N, kMarlinBN), kpad = (int)round_up(K, kMarlinBK);
    if (npad == 0 || kpad == 0) return hipSuccess;
    if (perm != nullptr && K <= 65535) {
        // act-order through LDS: the widest column block whose source words and
        // permutation fit and that still gives every CU a workgroup, else the
        // narrowest that fits
        constexpr size_t kLdsCap = 152 * 1024;
        int nb = 0;
        for (int w : {64, 32, 16, 8, 4}) {
            const size_t lds = (size_t)(K / 8) * w * 4 + (size_t)kpad * 2;
            if (lds > kLdsCap) continue;
            nb = w;
            if (npad / w >= cus) break;
        }
        if (nb != 0) {
            const size_t lds = (size_t)(K / 8) * nb * 4 + (size_t)kpad * 2;
            switch (nb) {
                case 64: return launch_repack_gptq_perm<64>(qweight, perm, wm, N, K, npad, kpad, lds, stream, start, stop);
                case 32: return launch_repack_gptq_perm<32>(qweight, perm, wm, N, K, npad, kpad, lds, stream, start, stop);
                case 16: return launch_repack_gptq_perm<16>(qweight, perm, wm, N, K, npad, kpad, lds, stream, start, stop);
                case 8: return launch_repack_gptq_perm<8>(qweight, perm, wm, N, K, npad, kpad, lds, stream, start, stop);
                default: return launch_repack_gptq_perm<4>(qweight, perm, wm, N, K, npad, kpad, lds, stream, start, stop);
            }
        }
    }
    launch_kernel(repack_gptq_kernel, dim3(npad / 64, (unsigned)ceil_div(kpad / 32, kRepackTiles)),
                  dim3(kRepackThreads), 0, stream, start, stop, qweight, perm, wm, N, K, kpad / kMarlinBK);
    return hipGetLastError();
}


hipError_t launch_gidx_perm(const int32_t* g_idx, int32_t* perm, int32_t* status, int K, int G, hipStream_t stream) {
    // the status word is cleared by a kernel rather than a memset, so that a
    // caller capturing the stream into a graph records a kernel node
    hipLaunchKernelGGL(clear_status_kernel, dim3(1), dim3(64), 0, stream, status);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || K == 0) return e;
    hipLaunchKernelGGL(gidx_perm_kernel, dim3(K / G), dim3(256), 0, stream, g_idx, perm, status, K, G);
    return hipGetLastError();
}

}  // namespace pw4

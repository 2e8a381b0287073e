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

// 8 x 8 nibble transpose in registers: nibble j of a[i] moves to nibble i of
// a[j].  Three rounds of block swaps -- 4-nibble halves and bytes with
// v_perm_b32, single nibbles with masks -- 32 VALU instructions.
__device__ __forceinline__ void transpose_nibbles8(uint32_t (&a)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = __builtin_amdgcn_perm(a[i + 4], a[i], 0x05040100u);  // halves 0 of a[i], a[i+4]
        const uint32_t hi = __builtin_amdgcn_perm(a[i + 4], a[i], 0x07060302u);  // halves 1
        a[i] = lo;
        a[i + 4] = hi;
    }
    constexpr int kByteRows[4] = {0, 1, 4, 5};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = kByteRows[q];
        const uint32_t x = __builtin_amdgcn_perm(a[i + 2], a[i], 0x06020400u);  // bytes 0, 2 of a[i], a[i+2]
        const uint32_t y = __builtin_amdgcn_perm(a[i + 2], a[i], 0x07030501u);  // bytes 1, 3
        a[i] = x;
        a[i + 2] = y;
    }
    constexpr uint32_t m = 0x0f0f0f0fu;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const uint32_t x = (a[i] & m) | ((a[i + 1] << 4) & ~m);
        const uint32_t y = ((a[i] >> 4) & m) | (a[i + 1] & ~m);
        a[i] = x;
        a[i + 1] = y;
    }
}

// GPTQ qweight [K/8, N] -> MARLIN through the act-order permutation.  A
// column block of NB columns is repacked over the whole K at once, so every
// source word is read from HBM once whatever the permutation.  The block's
// columns are taken in NW = NB / 8 strided groups: group g holds columns
// g, g + NW, ..., g + 7 NW.
//   Staging.  A thread loads the 8 source words of one group in one source
//   row (4-byte loads; the NW threads of a row read NW * 4 contiguous bytes
//   per load), transposes the 8 x 8 nibbles so that each word holds the
//   group's 8 columns at one K, and stores the 8 words of K 8r..8r+7 to LDS:
//   S[g][k], nibble c = column g + NW c at K k; row K holds nibble 8 for the
//   padding.  The permutation is staged once, as 16-bit entries clamped to
//   [0, K) with padding entries pointing at row K (PG: too long for LDS beside
//   the words; the gather reads it from global memory).
//   Gather.  A thread takes one 32-K tile of one group: 32 LDS reads of
//   S[g][perm[k]] give the tile's 32 K positions for 8 columns, and four 8 x 8
//   transposes turn them into the 8 columns' MARLIN words (word tg takes K
//   offsets 8p + 2tg for p < 4 and 8(p-4) + 2tg + 1 above, as its nibble p).
//   Store c of the NW threads of a tile then writes columns NW c .. NW c +
//   NW - 1, NW * 16 contiguous bytes: with adjacent columns per group, each
//   store would put 16 bytes in each of 64 lines, which measured twice as slow
//   as the whole write at full lines.  At 16 columns the groups are adjacent
//   (for 16-byte loads), and the tile's two threads swap half their words
//   before storing, so that their stores pair up into 32-byte runs.
// Workgroups are persistent and walk column blocks gridDim.x apart; those of
// one XCD (dispatch assigns workgroup i to XCD i % 8) take adjacent blocks, so
// the parts of a source line are fetched into one L2.
// VEC: 16-byte aligned perm (and, for adjacent-column groups, rows).  IT:
// staging items a thread loads per batch, all in flight before the first is
// stored.
constexpr int kPermThreads = 512;
template <int NB, bool VEC, bool PG, int IT>
__global__ __launch_bounds__(kPermThreads) void repack_gptq_perm_kernel(const uint32_t* __restrict__ qweight,
                                                                        const int32_t* __restrict__ perm,
                                                                        uint32_t* __restrict__ wm, int N, int K,
                                                                        int nchunks, int nblocks) {
    static_assert(NB % 8 == 0, "8-column groups");
    constexpr int NW = NB / 8;
    // strided groups from 32 columns (NW * 4 contiguous bytes per load and
    // NW * 16 per store); below, groups of adjacent columns, loaded 16 bytes
    // at a time, read faster than 4- or 8-byte runs
    constexpr bool SG = NB >= 32;
    auto col = [&](int blk, int g, int c) { return blk * NB + (SG ? g + NW * c : 8 * g + c); };
    extern __shared__ __attribute__((aligned(16))) uint32_t lds_words[];
    const int rs = K + 4;  // words per column group: K rows, the padding row, 16-byte alignment
    uint16_t* sp = reinterpret_cast<uint16_t*>(lds_words + NW * rs);  // [kpad], unless PG
    const int kpad = nchunks * 64;
    const int ktiles = nchunks * 2;
    const int nitems = (K >> 3) * NW;  // staging items of a block
    const int grid = gridDim.x;
    const int first = (grid & 7) == 0 ? (int)(blockIdx.x & 7) * (grid >> 3) + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
    if (first >= nblocks) return;
    const int tid = threadIdx.x;

    // Block blk into LDS.  Every load is issued, from a clamped address where
    // the item or its column is out of range, and the padding selected when
    // the words are stored: a load inside a divergent branch is waited for
    // where the branch joins, one at a time.
    auto stage = [&](int blk) {
        if constexpr (!SG && VEC && NW == 2) {
            // 16 columns, one 64-byte run per row: lane l of a wave loads the
            // 16-byte quad 4 (l % 4) of rows r0 + l / 4 and r0 + l / 4 + 16
            // (four lanes per run).  Lanes 2j and 2j + 1 then swap one row's
            // quads through DPP, so that the first holds both quads of group
            // (l % 4) / 2 in the first row and the second in the other row: the
            // wave's 64 items (32 rows x 2 groups), as in the loop below.  The
            // loop runs by whole waves, since a lane's partner must be active.
            const int lane = tid & 63, p = lane & 3, g = p >> 1;
            const bool second = (p & 1) != 0;
            const int nrows = K >> 3;
            const int c0 = blk * NB + 4 * p;  // this lane's quad
            for (int base = tid & ~63; base < nitems; base += IT * kPermThreads) {
                u32x4 va[IT], vb[IT];
#pragma unroll
                for (int q = 0; q < IT; ++q) {
                    const int ra = ((base + q * kPermThreads) >> 1) + (lane >> 2), rb = ra + 16;
                    va[q] = *reinterpret_cast<const u32x4*>(ra < nrows && c0 + 3 < N ? qweight + (int64_t)ra * N + c0
                                                                                      : qweight);
                    vb[q] = *reinterpret_cast<const u32x4*>(rb < nrows && c0 + 3 < N ? qweight + (int64_t)rb * N + c0
                                                                                      : qweight);
                }
#pragma unroll
                for (int q = 0; q < IT; ++q) {
                    const int ra = ((base + q * kPermThreads) >> 1) + (lane >> 2);
                    const int r = second ? ra + 16 : ra;
                    uint32_t a[8];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t send = second ? va[q][e] : vb[q][e];
                        const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xB1, 0xF, 0xF, true);
                        a[e] = second ? recv : va[q][e];
                        a[e + 4] = second ? vb[q][e] : recv;
                    }
                    if (r < nrows) {
#pragma unroll
                        for (int c = 0; c < 8; ++c) {
                            // whole 4-column quads (N % 4 == 0)
                            if (col(blk, g, c & 4) + 3 >= N) a[c] = 0x88888888u;
                        }
                        transpose_nibbles8(a);
                        uint32_t* dst = lds_words + g * rs + r * 8;
                        *reinterpret_cast<u32x4*>(dst) = u32x4{a[0], a[1], a[2], a[3]};
                        *reinterpret_cast<u32x4*>(dst + 4) = u32x4{a[4], a[5], a[6], a[7]};
                    }
                }
            }
            return;
        }
        for (int i0 = tid; i0 < nitems; i0 += IT * kPermThreads) {
            uint32_t v[IT][8];
#pragma unroll
            for (int q = 0; q < IT; ++q) {
                const int i = i0 + q * kPermThreads;
                const bool ok = i < nitems;
                const uint32_t* row = qweight + (ok ? (int64_t)(i / NW) * N : 0);
                const int g = i % NW;
                if constexpr (!SG && VEC) {  // adjacent columns: two 16-byte loads
                    const int c0 = col(blk, g, 0);
                    const u32x4 a = *reinterpret_cast<const u32x4*>(ok && c0 + 3 < N ? row + c0 : qweight);
                    const u32x4 b = *reinterpret_cast<const u32x4*>(ok && c0 + 7 < N ? row + c0 + 4 : qweight);
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        v[q][c] = a[c];
                        v[q][c + 4] = b[c];
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const int n = col(blk, g, c);
                        v[q][c] = *(ok && n < N ? row + n : qweight);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < IT; ++q) {
                const int i = i0 + q * kPermThreads;
                if (i < nitems) {
                    const int g = i % NW;
                    uint32_t a[8];
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        // 16-byte loads take whole 4-column quads (N % 4 == 0)
                        const int n = !SG && VEC ? col(blk, g, c & 4) + 3 : col(blk, g, c);
                        a[c] = n < N ? v[q][c] : 0x88888888u;
                    }
                    transpose_nibbles8(a);
                    uint32_t* dst = lds_words + g * rs + (i / NW) * 8;
                    *reinterpret_cast<u32x4*>(dst) = u32x4{a[0], a[1], a[2], a[3]};
                    *reinterpret_cast<u32x4*>(dst + 4) = u32x4{a[4], a[5], a[6], a[7]};
                }
            }
        }
    };
    // Block blk from LDS to the MARLIN words.
    auto gather = [&](int blk) {
        for (int i = tid; i < ktiles * NW; i += kPermThreads) {
            const int t = i / NW, w = i % NW;
            const uint32_t* grp = lds_words + w * rs;
            uint32_t g[32];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int kb = t * 32 + h * 8;
                uint32_t sk[8];
                if constexpr (PG) {
                    u32x4 p[2];
                    const int kc = kb < K ? kb : 0;  // unconditional loads, as in the staging
                    if constexpr (VEC) {
                        p[0] = *reinterpret_cast<const u32x4*>(perm + kc);
                        p[1] = *reinterpret_cast<const u32x4*>(perm + kc + 4);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) p[e >> 2][e & 3] = (uint32_t)perm[kc + e];
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        sk[e] = kb < K ? (uint32_t)min(max((int)p[e >> 2][e & 3], 0), K - 1) : (uint32_t)K;
                } else {
                    const u32x4 pk = *reinterpret_cast<const u32x4*>(sp + kb);
#pragma unroll
                    for (int e = 0; e < 8; ++e) sk[e] = (pk[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) g[8 * h + e] = grp[sk[e]];
            }
            uint32_t out[4][8];
#pragma unroll
            for (int tg = 0; tg < 4; ++tg) {
#pragma unroll
                for (int p = 0; p < 8; ++p) out[tg][p] = g[8 * (p & 3) + 2 * tg + (p >> 2)];
                transpose_nibbles8(out[tg]);
            }
            if constexpr (!SG && NW == 2) {
                // 16 columns: lanes 2j and 2j + 1 hold columns 0-7 and 8-15 of
                // one tile.  They swap four words (the first lane's odd columns
                // for the second's even ones, DPP quad_perm [1, 0, 3, 2]), so that
                // store c of the pair writes columns 2c and 2c + 1: 32 contiguous
                // bytes instead of 16 bytes in each of two lines.
                uint32_t recv[4][4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int tg = 0; tg < 4; ++tg) {
                        const uint32_t send = w ? out[tg][2 * j] : out[tg][2 * j + 1];
                        recv[j][tg] = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xB1, 0xF, 0xF, true);
                    }
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    u32x4 v;
#pragma unroll
                    for (int tg = 0; tg < 4; ++tg) {
                        if (c < 4) {
                            v[tg] = w ? recv[c][tg] : out[tg][2 * c];
                        } else {
                            v[tg] = w ? out[tg][2 * c - 7] : recv[c - 4][tg];
                        }
                    }
                    *reinterpret_cast<u32x4*>(wm + marlin_offset(blk * NB + 2 * c + w, t, nchunks)) = v;
                }
            } else {
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    *reinterpret_cast<u32x4*>(wm + marlin_offset(col(blk, w, c), t, nchunks)) =
                        u32x4{out[0][c], out[1][c], out[2][c], out[3][c]};
            }
        }
    };

    // the permutation, once for all blocks
    if constexpr (!PG) {
        for (int k = tid * 4; k < kpad; k += kPermThreads * 4) {
            u32x4 p = u32x4{0u, 0u, 0u, 0u};
            const int kc = k < K ? k : 0;  // K % 8 == 0: whole vectors
            if constexpr (VEC) {
                p = *reinterpret_cast<const u32x4*>(perm + kc);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) p[e] = (uint32_t)perm[kc + e];
            }
            uint32_t e4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)  // clamped: a bad perm cannot fault
                e4[e] = k < K ? (uint32_t)min(max((int)p[e], 0), K - 1) : (uint32_t)K;
            *reinterpret_cast<u32x2*>(sp + k) = u32x2{e4[0] | (e4[1] << 16), e4[2] | (e4[3] << 16)};
        }
    }
    if (tid < NW) lds_words[tid * rs + K] = 0x88888888u;
    for (int blk = first; blk < nblocks; blk += grid) {
        stage(blk);
        __syncthreads();
        gather(blk);
        __syncthreads();
    }
}

// perm = stable argsort(g_idx) for an act-order checkpoint: one workgroup per
// group collects, in ascending k, the rows that belong to it.  status bit 0:
// some group does not hold exactly G rows; bit 1: a group id out of range.
// Wave w of the workgroup's kGidxWaves takes the w-th span of k (whole steps of
// 64 lanes x EPL entries; VEC: four consecutive entries per lane, one 16-byte
// load).  Pass 1: each wave counts its rows of the group with ballots, no
// barrier.  One barrier hands the counts over.  Pass 2: each wave walks its
// span again and writes row k at the group's count of earlier rows (earlier
// waves, earlier steps, lower lanes, the lane's earlier entries).  A lane
// loads its entries of kGidxBatch steps at once: the walks are bound by their
// memory round trips.
template <bool VEC, int kGidxWaves, int kGidxBatch>
__global__ __launch_bounds__(64 * kGidxWaves) void gidx_perm_kernel(const int32_t* __restrict__ g_idx,
                                                                    int32_t* __restrict__ perm,
                                                                    int32_t* __restrict__ status, int K, int G) {
    constexpr int EPL = VEC ? 4 : 1, kStep = 64 * EPL;
    __shared__ int wave_cnt[kGidxWaves];
    const int g = blockIdx.x;
    const int Kg = K / G;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int span = (K + kGidxWaves * kStep - 1) / (kGidxWaves * kStep) * kStep;
    const int k_begin = wave * span, k_end = min(k_begin + span, K);  // VEC: K % 4 == 0, whole 4-entry runs
    const uint64_t below = (1ull << lane) - 1ull;
    // one batch of kGidxBatch steps: the group's rows among entries k0 + kStep b + EPL lane + j
    auto batch = [&](int k0, bool (&mine)[kGidxBatch][EPL]) {
        int gv[kGidxBatch][EPL];
#pragma unroll
        for (int b = 0; b < kGidxBatch; ++b) {
            const int k = k0 + b * kStep + lane * EPL;
            if constexpr (VEC) {
                const int4 v = k < k_end ? *reinterpret_cast<const int4*>(g_idx + k) : make_int4(-1, -1, -1, -1);
                gv[b][0] = v.x;
                gv[b][1] = v.y;
                gv[b][2] = v.z;
                gv[b][3] = v.w;
            } else {
                gv[b][0] = k < k_end ? g_idx[k] : -1;
            }
        }
#pragma unroll
        for (int b = 0; b < kGidxBatch; ++b)
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const int k = k0 + b * kStep + lane * EPL + j;
                if (g == 0 && k < k_end && (gv[b][j] < 0 || gv[b][j] >= Kg)) atomicOr(status, 2);
                mine[b][j] = k < k_end && gv[b][j] == g;
            }
    };
    int count = 0;
    for (int k0 = k_begin; k0 < k_end; k0 += kStep * kGidxBatch) {
        bool mine[kGidxBatch][EPL];
        batch(k0, mine);
#pragma unroll
        for (int b = 0; b < kGidxBatch; ++b)
#pragma unroll
            for (int j = 0; j < EPL; ++j) count += __popcll(__ballot(mine[b][j]));
    }
    if (lane == 0) wave_cnt[wave] = count;
    __syncthreads();
    int pos = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kGidxWaves; ++w) {
        pos += w < wave ? wave_cnt[w] : 0;
        total += wave_cnt[w];
    }
    for (int k0 = k_begin; k0 < k_end; k0 += kStep * kGidxBatch) {
        bool mine[kGidxBatch][EPL];
        batch(k0, mine);
#pragma unroll
        for (int b = 0; b < kGidxBatch; ++b) {
            int lower = 0, step = 0;
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const uint64_t mask = __ballot(mine[b][j]);
                lower += __popcll(mask & below);
                step += __popcll(mask);
            }
            int at = pos + lower;
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                if (mine[b][j] && at < G) perm[(int64_t)g * G + at] = k0 + b * kStep + lane * EPL + j;
                at += mine[b][j] ? 1 : 0;
            }
            pos += step;
        }
    }
    if (tid == 0 && total != G) atomicOr(status, 1);
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
template <int NB, int IT>
hipError_t launch_repack_gptq_perm(const uint32_t* qweight, const int32_t* perm, uint32_t* wm, int N, int K,
                                   int npad, int kpad, size_t lds, bool pg, int grid, hipStream_t stream,
                                   hipEvent_t start, hipEvent_t stop) {
    // 16-byte loads: 4-entry runs of perm, and (adjacent-column groups) 4-column quads of a row
    const bool vec = (reinterpret_cast<uintptr_t>(perm) & 15) == 0 &&
                     (NB >= 32 || (N % 4 == 0 && (reinterpret_cast<uintptr_t>(qweight) & 15) == 0));
    auto pick = [&]() {
        if constexpr (NB == 8) {  // the permutation from global memory only at 8 columns
            if (pg) return vec ? repack_gptq_perm_kernel<NB, true, true, IT> : repack_gptq_perm_kernel<NB, false, true, IT>;
        }
        return vec ? repack_gptq_perm_kernel<NB, true, false, IT> : repack_gptq_perm_kernel<NB, false, false, IT>;
    };
    const auto fn = pick();
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    launch_kernel(fn, dim3(grid), dim3(kPermThreads), (uint32_t)lds, stream, start, stop, qweight, perm, wm, N, K,
                  kpad / kMarlinBK, npad / NB);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_repack_gptq(const uint32_t* qweight, const int32_t* perm, uint32_t* wm, int N, int K,
                              hipStream_t stream, hipEvent_t start, hipEvent_t stop, int cus, int cols_override,
                              int grid_override) {
    const int npad = (int)round_up(N, kMarlinBN), kpad = (int)round_up(K, kMarlinBK);
    if (npad == 0 || kpad == 0) return hipSuccess;
    if (perm != nullptr && K <= 65535) {
        // act-order through LDS: the widest block (64 or 32 columns in strided
        // groups, else 16 or 8 adjacent) whose words and permutation fit and
        // whose blocks cover at least 0.8 of the CUs, else the narrowest that
        // fits; past that, 8 columns with the permutation read from global
        // memory.  One workgroup per block up to two blocks per CU, else one
        // persistent workgroup per CU.  Measured on MI355X, kernel only, us:
        // Llama-3-8B gate 15.0 at 64 columns (224 blocks; 20.3-21.0 at 32), q
        // 7.06 at 16 (7.43 at 32 on half the CUs, 8.1 at 64), k 4.9 at 8 (6.3
        // at 32), down 20.4 at 16 (the widest that fits K = 14336); 70B o 21.9
        // at 32 (24.1 at 16), qkv 31.2 with 320 workgroups (37.9 with 256
        // walking 1.25 blocks each), gate_up 132 with 256 persistent
        // workgroups (138 with 512).
        constexpr size_t kLdsCap = 152 * 1024;
        auto words_bytes = [&](int w) { return (size_t)(w / 8) * (K + 4) * 4; };
        const size_t perm_bytes = (size_t)kpad * 2;
        auto fits = [&](int w) { return words_bytes(w) + perm_bytes <= kLdsCap; };
        int nb = 0;
        bool pg = false;
        if (cols_override != 0 && fits(cols_override)) {
            nb = cols_override;
        } else {
            for (int w : {64, 32, 16, 8}) {
                if (!fits(w)) continue;
                nb = w;
                if (5 * (npad / w) >= 4 * cus) break;
            }
        }
        if (nb == 0 && words_bytes(8) <= kLdsCap) {
            nb = 8;
            pg = true;
        }
        if (nb != 0) {
            const size_t lds = words_bytes(nb) + (pg ? 0 : perm_bytes);
            const int nblocks = npad / nb;
            const int grid = grid_override > 0 ? std::min(nblocks, grid_override)
                                               : (nblocks <= 2 * cus ? nblocks : cus);
            // four staging items per thread cover a block of K * NB <= 4 * 64 * 512 (K = 4096 at 32 columns)
            const bool it8 = (int64_t)(K / 8) * (nb / 8) > 4 * kPermThreads;
            switch (nb * (it8 ? -1 : 1)) {
                case 64: return launch_repack_gptq_perm<64, 4>(qweight, perm, wm, N, K, npad, kpad, lds, pg, grid, stream, start, stop);
                case -64: return launch_repack_gptq_perm<64, 8>(qweight, perm, wm, N, K, npad, kpad, lds, pg, grid, stream, start, stop);
                case 32: return launch_repack_gptq_perm<32, 4>(qweight, perm, wm, N, K, npad, kpad, lds, pg, grid, stream, start, stop);
                case -32: return launch_repack_gptq_perm<32, 8>(qweight, perm, wm, N, K, npad, kpad, lds, pg, grid, stream, start, stop);
                case 16: return launch_repack_gptq_perm<16, 4>(qweight, perm, wm, N, K, npad, kpad, lds, pg, grid, stream, start, stop);
                case -16: return launch_repack_gptq_perm<16, 8>(qweight, perm, wm, N, K, npad, kpad, lds, pg, grid, stream, start, stop);
                case 8: return launch_repack_gptq_perm<8, 4>(qweight, perm, wm, N, K, npad, kpad, lds, pg, grid, stream, start, stop);
                default: return launch_repack_gptq_perm<8, 8>(qweight, perm, wm, N, K, npad, kpad, lds, pg, grid, stream, start, stop);
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
    // Past K = 4096, eight waves with 16-byte loads where g_idx is 16-byte aligned
    // and K holds whole 4-entry runs (K = 14336: 17.4 -> 9.6 us, 28672: 29.2 ->
    // 18.1 us against four waves of single entries); up to K = 4096 four waves
    // of single entries are faster (5.2 against 7.8 us at 4096).
    if ((reinterpret_cast<uintptr_t>(g_idx) & 15) == 0 && K % 4 == 0 && K > 4096) {
        hipLaunchKernelGGL((gidx_perm_kernel<true, 8, 8>), dim3(K / G), dim3(512), 0, stream, g_idx, perm, status, K,
                           G);
    } else {
        hipLaunchKernelGGL((gidx_perm_kernel<false, 4, 16>), dim3(K / G), dim3(256), 0, stream, g_idx, perm, status,
                           K, G);
    }
    return hipGetLastError();
}

}  // namespace pw4

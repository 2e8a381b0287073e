/*
 * pulsar_w4a16.h -- C ABI of the MI355X (gfx950) W4A16 linear-layer library
 * (libpulsar_w4a16.so).
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer
 * (hipMalloc'd or torch-owned), every size is an element count, every call is
 * asynchronous on `stream` and returns 0 or a negative PW4_ERR_* status.  The
 * GEMMs read x and the weight words as 16-byte vectors: those two pointers
 * must be 16-byte aligned (any allocation is, and so is any row slice of x
 * since K % 8 == 0), else the call returns PW4_ERR_ARG.  No
 * entry point allocates device memory: scratch space is passed in through
 * (workspace, workspace_bytes) and sized with the matching *_workspace_size
 * query, so the GEMMs are safe under HIP graph capture.
 *
 * Workspace contract.  A non-empty workspace begins with a region of
 * PW4_ZERO_REGION_BYTES (K-split arrival counters and exchange slots) that
 * must be zero when the workspace is first used (clear it once after
 * allocating); every GEMM call leaves it zero when it completes, so the
 * workspace can be reused by later calls without clearing.  The bytes after
 * it are scratch.  Calls that share a workspace must be ordered (one stream,
 * or explicit synchronisation); concurrent calls need distinct workspaces.
 *
 * Each entry point replaces one operator of the reference pulsar-core C++ API
 * (pulsar-core/inc/pulsar/ops.hpp) and keeps its argument meaning and its
 * precondition checks; the at::Tensor wrappers that keep the reference C++
 * signatures verbatim live in pulsar_amd/csrc/torch_ops.cpp.
 */
#ifndef PULSAR_W4A16_H
#define PULSAR_W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* pw4_stream_t; /* == hipStream_t */

/* status codes */
#define PW4_OK 0
#define PW4_ERR_ARG (-1)       /* null or misaligned pointer, unknown dtype, negative size */
#define PW4_ERR_SHAPE (-2)     /* inconsistent sizes / group size (reference TORCH_CHECKs) */
#define PW4_ERR_WORKSPACE (-3) /* workspace missing or smaller than the *_workspace_size query */
#define PW4_ERR_HIP (-4)       /* a HIP runtime call or kernel launch failed */
#define PW4_ERR_GIDX (-5)      /* act-order g_idx is not a valid grouping */

/* bytes at the start of every non-empty GEMM workspace that hold the K-split
 * arrival counters and exchange slots (zero before first use, left zero by
 * every call) */
#define PW4_ZERO_REGION_BYTES (16u << 20)

/* element types */
#define PW4_DTYPE_F16 0
#define PW4_DTYPE_BF16 1
#define PW4_DTYPE_F32 2

/* Human-readable text for a status code (static storage). */
const char* pw4_status_string(int status);
/* Text of the last HIP error seen by this thread inside the library. */
const char* pw4_last_hip_error(void);
/* Kernel timing (no counterpart in the reference; a profiling facility).
 * Arms the calling thread for its next GEMM or repack call (pw4_gemm_w4a16,
 * pw4_gemm_w4a16_marlin, pw4_gemm_w4a16_silu_mul, pw4_repack_w4a16 or
 * pw4_repack_gptq): that call takes the two events (hipEvent_t, created with
 * timing enabled on the call's device) before it checks its arguments, so
 * they never outlive it, and launches its kernels through hipExtLaunchKernel
 * with them.  GEMM: `start` takes the start of the first GEMM dispatch,
 * `stop` the end of the last -- the interval a kernel trace reports, without
 * the queue latency in front of the kernel; a repack, gather, split-K combine
 * or SiLU pass of the call is not inside it.  Repack: `start` and `stop` take
 * the start and end of the repack kernel (pw4_repack_w4a16: words and scales
 * in one dispatch).  A call that fails or launches nothing leaves the events
 * unset.  Read them with hipEventElapsedTime after the stream syncs.
 * (NULL, NULL) disarms; exactly one NULL is PW4_ERR_ARG.  Not for use under
 * graph capture. */
int pw4_time_next_kernel(void* start_event, void* stop_event);

/* Diagnostic hook, no counterpart in the reference (it is for parity tests):
 * arms the calling thread's next GEMM or repack call to also write, into the
 * device buffer y32 (fp32 [M, N]), the fp32 value each element of y was
 * rounded from -- the accumulators before the cast to the output dtype -- on
 * every plan (decode direct store, exchange tree, K-slice counter path,
 * unsplit prefill kernels, split-K combine) except SiLU-gated calls, which
 * write no such value.  The call takes the buffer before it checks its
 * arguments, so it never outlives that call; NULL disarms. */
int pw4_observe_next_call(float* y32);

/* Diagnostic, no counterpart in the reference (it is for tests and tuning):
 * writes into buf (len bytes, NUL-terminated) the plan a GEMM call with these
 * arguments would run, e.g. "decode nb=16 wps=256 splits=1 tree=0 win=0 ring=4
 * mt=1 bs=1 px=0" (bs: one scale load per four steps; px: act-order gathered
 * in the kernel's LDS, its permutation columns per thread) or "prefill256
 * rows=128 splits=2 exact=1 khalves=2" (khalves: two K halves per 8-wave
 * workgroup, summed in LDS).  layout: PW4_LAYOUT_CT
 * (pw4_gemm_w4a16) or PW4_LAYOUT_MARLIN (pw4_gemm_w4a16_marlin; with silu
 * nonzero pw4_gemm_w4a16_silu_mul).  Launches nothing.  The plan depends on
 * the current device's compute-unit count (256 assumed when no device
 * answers).  PW4_ERR_ARG when buf is too small. */
#define PW4_LAYOUT_CT 0
#define PW4_LAYOUT_MARLIN 1
int pw4_plan_describe(int layout, int x_dtype, int scale_dtype, int has_zp, int has_perm, int silu, int64_t M,
                      int64_t N, int64_t K, int64_t group_size, int64_t num_splits, char* buf, size_t len);

/* ABI version of this header: bumped on any incompatible change. */
int pw4_abi_version(void);
#define PW4_ABI_VERSION 2

/* Number of int32 words of the MARLIN layout for an [N, K] weight:
 * roundup(N, 64) * roundup(K, 64) / 8.
 * Mirrors the size rule of repack_w4a16 (pulsar-core/src/kernels/w4a16_marlin.cu:373-375;
 * pulsar/src/pulsar/core/ops.py:139-155). */
int64_t pw4_marlin_words(int64_t N, int64_t K);

/* ---------------------------------------------------------------------------
 * repack_w4a16: compressed-tensors int4 weights -> MARLIN layout.
 * Replaces pulsar::repack_w4a16_cuda (pulsar-core/inc/pulsar/ops.hpp:181-182;
 * pulsar-core/src/kernels/w4a16_marlin.cu:354-406).
 *   weight_packed  int32 [N, K/8], nibble k%8 of word [n, k/8], two's complement
 *   weight_scale   [N, K/group_size] in scale_dtype (F32, F16 or BF16)
 *   weight_marlin  out, int32 [pw4_marlin_words(N, K)]  (bit-exact reference layout)
 *   scale_marlin   out, fp32 [K/group_size, N] = transpose of weight_scale
 * Preconditions (reference w4a16_marlin.cu:356-371): group_size > 0,
 * group_size % 16 == 0, K % 8 == 0, K % group_size == 0. */
int pw4_repack_w4a16(const int32_t* weight_packed, const void* weight_scale, int scale_dtype, int64_t N, int64_t K,
                     int64_t group_size, int32_t* weight_marlin, float* scale_marlin, pw4_stream_t stream);

/* ---------------------------------------------------------------------------
 * gemm_w4a16 / gemm_w4a16_split: y = x @ dequant(W)^T straight from the
 * compressed-tensors packing.
 * Replaces pulsar::gemm_w4a16_cuda and pulsar::gemm_w4a16_split_cuda
 * (pulsar-core/inc/pulsar/ops.hpp:156-173; pulsar-core/src/kernels/w4a16_gemm.cu:317-489).
 *   x              [M, K] fp16 or bf16 (x_dtype), row-major contiguous
 *   weight_packed  int32 [N, K/8] as above
 *   weight_scale   fp32 [N, K/group_size]   (the reference upcasts to fp32 too, w4a16_gemm.cu:352)
 *   y              out, [M, N] in x_dtype
 *   num_splits     0: the library picks the K split; >= 1: force exactly that many
 *                  K slices through the fp32-partials + fixed-order combine path
 *                  (slices beyond the K extent are empty and add 0), as the
 *                  reference's gemm_w4a16_split does.
 * Preconditions (reference w4a16_gemm.cu:324-348): K % 8 == 0, group_size > 0,
 * group_size % 16 == 0, K % group_size == 0.  M == 0 or N == 0 is a no-op. */
size_t pw4_gemm_w4a16_workspace_size(int64_t M, int64_t N, int64_t K, int64_t group_size, int64_t num_splits);
int pw4_gemm_w4a16(const void* x, int x_dtype, const int32_t* weight_packed, const float* weight_scale, void* y,
                   int64_t M, int64_t N, int64_t K, int64_t group_size, int64_t num_splits, void* workspace,
                   size_t workspace_bytes, pw4_stream_t stream);

/* ---------------------------------------------------------------------------
 * gemm_w4a16_marlin: y = x @ dequant(W)^T from the MARLIN layout.
 * Replaces pulsar::gemm_w4a16_marlin_cuda (pulsar-core/inc/pulsar/ops.hpp:184-189;
 * pulsar-core/src/kernels/w4a16_marlin.cu:408-551), extended with optional
 * asymmetric zero points and act-order (neither exists in the reference):
 *   x              [M, K] fp16 or bf16
 *   weight_marlin  int32 [pw4_marlin_words(N, K)] from pw4_repack_w4a16 / pw4_repack_gptq
 *   scales         [K/group_size, N] in scale_dtype (F32 as repack_w4a16 returns, or F16)
 *   qzeros         NULL (symmetric, zero point 8) or int32 [K/group_size, N/8] GPTQ
 *                  zero points: nibble n%8 of word [g, n/8], used as stored (w = (u - z) * s)
 *   perm           NULL or int32 [K]: the act-order permutation from pw4_gidx_to_perm;
 *                  the kernel computes y = x[:, perm] @ dequant(W_repacked)^T
 *   num_splits     as for pw4_gemm_w4a16
 * Preconditions (reference w4a16_marlin.cu:414-442): group_size > 0,
 * group_size % 16 == 0, K % group_size == 0, K % 8 == 0; N % 8 == 0 when qzeros. */
size_t pw4_gemm_w4a16_marlin_workspace_size(int64_t M, int64_t N, int64_t K, int64_t group_size, int has_perm,
                                            int64_t num_splits);
int pw4_gemm_w4a16_marlin(const void* x, int x_dtype, const int32_t* weight_marlin, const void* scales,
                          int scale_dtype, const int32_t* qzeros, const int32_t* perm, void* y, int64_t M, int64_t N,
                          int64_t K, int64_t group_size, int64_t num_splits, void* workspace,
                          size_t workspace_bytes, pw4_stream_t stream);

/* ---------------------------------------------------------------------------
 * gemm_w4a16_marlin_noalloc: pw4_gemm_w4a16_marlin without a workspace
 * argument.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, results and errors as
 * pw4_gemm_w4a16_marlin, whose kernels it runs; it allocates nothing.  Its
 * workspace is a fixed array of PW4_NOALLOC_SCRATCH_BYTES in the library's
 * device code (one per device, held until the process exits); a call whose
 * plan needs more returns PW4_ERR_WORKSPACE before launching anything (an
 * automatic prefill plan whose K-slice partials would not fit runs unsplit
 * instead).  The array used is the current device's: `stream` must belong to
 * the current device (PW4_ERR_ARG otherwise).  The first call on a device
 * clears the array's zero region with a fill kernel on `stream`, and every
 * call leaves it zero.  When that first call is made under stream capture,
 * the fill is recorded into the graph once (ahead of the graph's first
 * no-alloc call, so a replay clears the region before using it) and the next
 * call outside a capture clears it for good.  All calls on one device share
 * the array: calls that overlap in time on one device (different streams,
 * graphs replayed on different streams, or host threads without ordering)
 * race and give wrong results. */
#define PW4_NOALLOC_SCRATCH_BYTES (64u << 20)
int pw4_gemm_w4a16_marlin_noalloc(const void* x, int x_dtype, const int32_t* weight_marlin, const void* scales,
                                  int scale_dtype, const int32_t* qzeros, const int32_t* perm, void* y, int64_t M,
                                  int64_t N, int64_t K, int64_t group_size, int64_t num_splits, pw4_stream_t stream);

/* ---------------------------------------------------------------------------
 * gemm_w4a16_silu_mul: the SwiGLU gate of the MLP in one call,
 *   y [M, N/2] = silu(x @ Wg^T) * (x @ Wu^T),
 * replacing the reference's two at::linear calls on gate_proj and up_proj and
 * the at::silu(gate) * up that follows them (pulsar-core/src/model/qwen3.cpp:
 * 116-118).  No reference counterpart as one op.  The weight is gate|up
 * interleaved by 8 columns: fused columns 16j..16j+7 are gate columns
 * 8j..8j+7 and 16j+8..16j+15 are up columns 8j..8j+7 (N = 2 * intermediate,
 * N % 16 == 0), in the MARLIN layout; scales, qzeros and perm as for
 * pw4_gemm_w4a16_marlin, in the same fused column order.  silu and the
 * product are computed in fp32 on the fp32 GEMM results and rounded once to
 * x's dtype where the kernel pairs the columns itself (decode without K
 * slices, the 256-wide prefill kernel, the split-K combine); other plans
 * round the GEMM output to x's dtype first and gate it in a second pass. */
size_t pw4_gemm_w4a16_silu_mul_workspace_size(int64_t M, int64_t N, int64_t K, int64_t group_size, int has_perm);
int pw4_gemm_w4a16_silu_mul(const void* x, int x_dtype, const int32_t* weight_marlin, const void* scales,
                            int scale_dtype, const int32_t* qzeros, const int32_t* perm, void* y, int64_t M, int64_t N,
                            int64_t K, int64_t group_size, void* workspace, size_t workspace_bytes,
                            pw4_stream_t stream);

/* ---------------------------------------------------------------------------
 * GPTQ ingestion (no counterpart in the reference, which has no zero points
 * and no act-order; these follow the public GPTQ checkpoint convention).
 *
 * pw4_gidx_to_perm: perm = stable argsort(g_idx) for an act-order checkpoint.
 *   g_idx [K] int32 group id of each input row; every group must hold exactly
 *   group_size rows.  status_dev is an int32 device word the call zeroes and
 *   then sets nonzero if g_idx is not such a grouping (read it after the stream
 *   syncs: nonzero means PW4_ERR_GIDX).
 * pw4_repack_gptq: qweight int32 [K/8, N] (nibble k%8 of word [k/8, n], unsigned)
 *   -> MARLIN layout; repacked row j is original row perm[j] (perm may be NULL).
 *   GPTQ symmetric nibbles and the reference's MARLIN nibbles are the same bytes,
 *   so for perm == NULL the output equals pw4_repack_w4a16 of the matching
 *   compressed-tensors tensor. */
int pw4_gidx_to_perm(const int32_t* g_idx, int64_t K, int64_t group_size, int32_t* perm, int32_t* status_dev,
                     pw4_stream_t stream);
int pw4_repack_gptq(const int32_t* qweight, const int32_t* perm, int64_t N, int64_t K, int32_t* weight_marlin,
                    pw4_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* PULSAR_W4A16_H */

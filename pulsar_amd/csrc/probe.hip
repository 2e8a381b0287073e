// Measurement probe for bench.py (libpw4_probe.so, not part of the W4A16
// library or its C ABI): a plain streaming read of a device buffer, the
// read-only HBM rate a memory-bound kernel can expect on this device.
//
// Each thread reads 16-byte vectors in a grid-stride loop, four loads in
// flight per iteration, and folds them into an XOR; the fold is stored only if
// it equals a value the caller never passes (`sink` is written by no launch in
// practice), so the loads stay but nothing is written.  The loads are plain or
// non-temporal (`nt`), as the decode kernel's weight loads are.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ u32x4 load16(const u32x4* p) {
    if constexpr (NT) {
        return __builtin_nontemporal_load(p);
    } else {
        return *p;
    }
}

template <bool NT>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, int64_t n16,
                                                          uint32_t never, uint32_t* __restrict__ sink) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 a = load16<NT>(p + i), b = load16<NT>(p + i + stride), c = load16<NT>(p + i + 2 * stride),
                    d = load16<NT>(p + i + 3 * stride);
        acc ^= a ^ b ^ c ^ d;
    }
    for (; i < n16; i += stride) acc ^= load16<NT>(p + i);
    const uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (v == never) sink[blockIdx.x & 1023] = v;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) from the 16-byte aligned device buffer `p` with
// `blocks` workgroups of 256 threads on `stream`, with non-temporal loads when `nt`
// is non-zero.  `sink` is a device buffer of at least 1024 uint32 that the kernel
// writes only if the XOR of everything it read equals `never`.  Returns a hipError_t.
int pw4_probe_stream_read(const void* p, int64_t bytes, int blocks, int nt, uint32_t never, uint32_t* sink,
                          hipStream_t stream) {
    if (p == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 != 0 || blocks <= 0 ||
        (reinterpret_cast<uintptr_t>(p) & 15) != 0) {
        return (int)hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(nt ? stream_read_kernel<true> : stream_read_kernel<false>, dim3((unsigned)blocks), dim3(256), 0,
                       stream, reinterpret_cast<const u32x4*>(p), bytes / 16, never, sink);
    return (int)hipGetLastError();
}

// The same read, launched through hipExtLaunchKernel with two HIP events that
// take the dispatch's own start and end timestamps (the kernel's duration
// without the queue latency in front of it).
int pw4_probe_stream_read_timed(const void* p, int64_t bytes, int blocks, int nt, uint32_t never, uint32_t* sink,
                                hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    if (p == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 != 0 || blocks <= 0 ||
        (reinterpret_cast<uintptr_t>(p) & 15) != 0 || start == nullptr || stop == nullptr) {
        return (int)hipErrorInvalidValue;
    }
    hipExtLaunchKernelGGL(nt ? stream_read_kernel<true> : stream_read_kernel<false>, dim3((unsigned)blocks), dim3(256),
                          0, stream, start, stop, 0, reinterpret_cast<const u32x4*>(p), bytes / 16, never, sink);
    return (int)hipGetLastError();
}

}  // extern "C"

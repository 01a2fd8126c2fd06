// Bandwidth and launch-cost reference kernels for the benchmark.
//
// gdsllm_read_stream reads a buffer once with 16-byte non-temporal loads and
// keeps the data only in a running XOR (written out only when it equals an
// opaque key the caller passes, i.e. never), so its duration is what one
// launch of this size needs to move the bytes from HBM into the compute units
// and nothing else.  gdsllm_empty_launch is a kernel with no work: the fixed
// cost of one launch back to back with others.  Neither is on the matvec
// path; they give the measured ceilings the GEMV is compared against.

#include "common.h"

namespace gdsllm {
namespace {

constexpr int kStreamThreads = 256;

__global__ __launch_bounds__(kStreamThreads) void read_stream(const uint4* __restrict__ p, int64_t n16,
                                                             uint32_t key, uint32_t* __restrict__ sink) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kStreamThreads;
    int64_t i = static_cast<int64_t>(blockIdx.x) * kStreamThreads + threadIdx.x;
    uint32_t acc = 0;
    // four loads in flight per thread
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = load_nt16(p + i), b = load_nt16(p + i + stride);
        const uint4 c = load_nt16(p + i + 2 * stride), d = load_nt16(p + i + 3 * stride);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = load_nt16(p + i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == key) sink[blockIdx.x] = acc;
}

__global__ void empty_kernel() {}

}  // namespace
}  // namespace gdsllm

using namespace gdsllm;

extern "C" int gdsllm_read_stream(const void* src, int64_t bytes, int64_t workgroups, uint32_t key, void* sink,
                                  void* stream) {
    if (bytes < 0 || workgroups < 1 || workgroups > (1 << 20))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gdsllm_read_stream: bytes >= 0 and 1 <= workgroups <= 2^20");
    if (bytes == 0) return ok();
    if (!src || !sink) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gdsllm_read_stream: null pointer");
    if (bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(sink) % 4)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT,
                         "gdsllm_read_stream: src must be 16-byte aligned with bytes % 16 == 0, sink 4-byte aligned");
    read_stream<<<dim3(static_cast<unsigned>(workgroups)), dim3(kStreamThreads), 0, as_stream(stream)>>>(
        static_cast<const uint4*>(src), bytes / 16, key, static_cast<uint32_t*>(sink));
    return check_hip(hipGetLastError(), "gdsllm_read_stream launch");
}

extern "C" int gdsllm_empty_launch(int64_t workgroups, void* stream) {
    if (workgroups < 1 || workgroups > (1 << 20))
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gdsllm_empty_launch: 1 <= workgroups <= 2^20");
    empty_kernel<<<dim3(static_cast<unsigned>(workgroups)), dim3(64), 0, as_stream(stream)>>>();
    return check_hip(hipGetLastError(), "gdsllm_empty_launch launch");
}

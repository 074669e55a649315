// Measurement probe (not part of the attention C ABI): the rate a plain
// streaming copy sustains on this GPU (bytes read + bytes written), the
// practical ceiling of kernels that read and write HBM in equal parts such as
// the prefill QK norm / RoPE / KV write and the KV-cache suffix writer.
//
// Every workgroup copies one contiguous region; each thread has 4 independent
// 16-byte loads in flight per step, all loads and stores non-temporal (the
// fastest of 2-8 loads in flight, with or without the non-temporal hints, at
// 1-8 workgroups per CU).  bench.py copies buffers far larger than the 256 MB
// last-level cache.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t probe_u4 __attribute__((ext_vector_type(4)));
constexpr int kCopyInFlight = 4;

__global__ __launch_bounds__(256) void hbm_copy_kernel(const probe_u4* __restrict__ src,
                                                       probe_u4* __restrict__ dst, int64_t n16) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * per;
    const int64_t end = begin + per < n16 ? begin + per : n16;
    int64_t i = begin + threadIdx.x;
    for (; i + (kCopyInFlight - 1) * 256 < end; i += kCopyInFlight * 256) {
        probe_u4 v[kCopyInFlight];
#pragma unroll
        for (int u = 0; u < kCopyInFlight; ++u) v[u] = __builtin_nontemporal_load(src + i + u * 256);
#pragma unroll
        for (int u = 0; u < kCopyInFlight; ++u) __builtin_nontemporal_store(v[u], dst + i + u * 256);
    }
    for (; i < end; i += 256) dst[i] = src[i];
}

}  // namespace

// Copies `bytes` (a multiple of 16) from `src` to `dst` (not overlapping) with
// `blocks` workgroups of 256 threads.  Returns 0 or the hipError_t.
extern "C" int32_t grout_probe_hbm_copy(const void* src, void* dst, int64_t bytes, int32_t blocks,
                                        void* stream) {
    if (src == nullptr || dst == nullptr || bytes <= 0 || bytes % 16 != 0 || blocks <= 0) return -9;
    hipLaunchKernelGGL(hbm_copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), static_cast<const probe_u4*>(src),
                       static_cast<probe_u4*>(dst), bytes / 16);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int32_t>(e);
}

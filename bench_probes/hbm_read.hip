// Measurement probe (not part of the attention C ABI): the HBM read rate a
// plain streaming kernel sustains on this GPU, the practical ceiling of the
// HBM-bound kernels next to the 8 TB/s of the MI355X specification.
//
// Every thread reads 16-byte chunks with a grid stride (4 independent loads in
// flight per iteration) and folds them into one word, written once so the
// loads cannot be dropped.  bench.py reads a buffer far larger than the
// 256 MB last-level cache.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t probe_u4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void hbm_read_kernel(const probe_u4* __restrict__ src, int64_t n16,
                                                       uint32_t* __restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const probe_u4 a = __builtin_nontemporal_load(src + i);
        const probe_u4 b = __builtin_nontemporal_load(src + i + stride);
        const probe_u4 c = __builtin_nontemporal_load(src + i + 2 * stride);
        const probe_u4 d = __builtin_nontemporal_load(src + i + 3 * stride);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const probe_u4 a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = acc;
}

}  // namespace

// Reads `bytes` (a multiple of 16) from `src` with `blocks` workgroups of 256
// threads; `out` holds blocks * 256 words.  Returns 0 or the hipError_t.
extern "C" int32_t grout_probe_hbm_read(const void* src, int64_t bytes, uint32_t* out,
                                        int32_t blocks, void* stream) {
    if (src == nullptr || out == nullptr || bytes <= 0 || bytes % 16 != 0 || blocks <= 0) return -9;
    hipLaunchKernelGGL(hbm_read_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream),
                       static_cast<const probe_u4*>(src), bytes / 16, out);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int32_t>(e);
}

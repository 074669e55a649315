// Measurement probe (not part of the attention C ABI): the HBM read rate a
// plain streaming kernel sustains on this GPU, the practical ceiling of the
// HBM-bound kernels next to the 8 TB/s of the MI355X specification.
//
// Every workgroup streams one contiguous region of the buffer; each thread has
// 16 independent 16-byte non-temporal loads in flight per step (one 64 KB step
// per workgroup), folded into one word that is written once so the loads
// cannot be dropped.  With only 4 loads in flight per thread the probe itself
// was latency-bound (6.0-6.3 TB/s against 7.0-7.2 with 16).  bench.py reads a
// buffer far larger than the 256 MB last-level cache and keeps the best of a
// few workgroups-per-CU counts.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t probe_u4 __attribute__((ext_vector_type(4)));
constexpr int kInFlight = 16;

__global__ __launch_bounds__(256) void hbm_read_kernel(const probe_u4* __restrict__ src, int64_t n16,
                                                       uint32_t* __restrict__ out) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * per;
    const int64_t end = begin + per < n16 ? begin + per : n16;
    int64_t i = begin + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (kInFlight - 1) * 256 < end; i += kInFlight * 256) {
        probe_u4 v[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) v[u] = __builtin_nontemporal_load(src + i + u * 256);
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < end; i += 256) {
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

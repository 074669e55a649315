// Measurement probe (not part of the attention C ABI): sustained rate of
// v_mfma_f32_32x32x16_f16 on this GPU for operands that change every
// instruction and are distributed like the prefill kernel's.
//
// The dense fp16 figure of the MI355X specification (2516.6 TFLOP/s) is a
// clock-times-width number; what the matrix cores sustain depends on the
// operand data (measured here: all-zero operands run far faster than N(0,1)
// ones).  bench.py runs this probe next to the prefill kernel and reports the
// prefill rate against both figures.
//
// Each of the 8 wavefronts of a workgroup (two per SIMD) holds 8 A and 8 B
// operand sets and 4 independent accumulators, so the matrix core always has
// an independent MFMA to issue and no instruction other than the MFMAs and
// the loop counter runs in the timed loop.
//   mode 0: A and B ~ N(0,1)            (Q K^T of the prefill kernel)
//   mode 1: A ~ N(0,1), B = u1*u2 in [0,1) (P V: softmax weights times V)
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace {

typedef _Float16 probe_half8_t __attribute__((ext_vector_type(8)));
typedef float probe_float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float probe_u01(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return (static_cast<float>(x >> 8) + 0.5f) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ float probe_gauss(uint32_t x) {
    return sqrtf(-2.0f * logf(probe_u01(x))) * cosf(6.2831853f * probe_u01(x * 2654435761u + 12345u));
}

__global__ __launch_bounds__(512, 1) void mfma_probe_kernel(float* out, int iters, int mode, uint32_t seed) {
    probe_half8_t a[8], b[8];
    const uint32_t base = (blockIdx.x * 512u + threadIdx.x) * 977u + seed;
    for (int j = 0; j < 8; ++j)
        for (int i = 0; i < 8; ++i) {
            const uint32_t h = base + static_cast<uint32_t>(j * 64 + i);
            a[j][i] = static_cast<_Float16>(probe_gauss(h));
            const float bv = (mode == 1) ? probe_u01(h * 3u) * probe_u01(h * 5u) : probe_gauss(h * 7u);
            b[j][i] = static_cast<_Float16>(bv);
        }
    probe_float16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j], b[j], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j + 1], b[(j + 3) & 7], c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[(j + 5) & 7], b[j + 1], c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[(j + 2) & 7], b[(j + 6) & 7], c3, 0, 0, 0);
        }
    }
    float s = 0.0f;
    for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * 512 + threadIdx.x] = s;
}

}  // namespace

// Launches `blocks` workgroups of 512 threads, each running iters x 16 MFMAs
// per wavefront; returns 0 or the hipError_t of the launch.  FLOPs of one
// launch: blocks * 8 * iters * 16 * 32768.
extern "C" int32_t grout_probe_mfma_f16(float* out, int32_t blocks, int32_t iters, int32_t mode,
                                        uint32_t seed, void* stream) {
    if (out == nullptr || blocks <= 0 || iters <= 0 || mode < 0 || mode > 1) return -9;
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(static_cast<unsigned>(blocks)), dim3(512), 0,
                       reinterpret_cast<hipStream_t>(stream), out, iters, mode, seed);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int32_t>(e);
}

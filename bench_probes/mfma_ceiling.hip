// Measurement probe (not part of the attention C ABI): sustained rate of
// v_mfma_f32_32x32x16_f16 on this GPU for operand data distributed like the
// prefill kernel's.
//
// The dense fp16 figure of the MI355X specification (2516.6 TFLOP/s) is a
// clock-times-width number; what the matrix cores sustain depends on the
// operand data (all-zero operands run far faster than N(0,1) ones, since the
// chip's power limit lowers the clock with switching activity).  bench.py runs
// this probe next to the prefill kernel and reports the prefill rate against
// both figures.
//
// The operands come from two f16 buffers that the caller fills (bench.py:
// A ~ N(0,1); B ~ N(0,1) for the Q K^T kind, B = u1*u2 in [0,1) for the P V
// kind).  Each wavefront lane loads 8 A and 8 B 16-byte chunks once, then runs
// 16 MFMAs per loop trip on 4 independent accumulators, so the matrix core
// always has an independent MFMA to issue and nothing but the MFMAs and the
// loop counter runs in the timed loop.  The operands stay in registers (no
// spills: 32 operand + 64 accumulator VGPRs), so the rate is the matrix core's
// and not the memory system's.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 probe_half8_t __attribute__((ext_vector_type(8)));
typedef float probe_float16_t __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(512, 1) void mfma_probe_kernel(const probe_half8_t* __restrict__ a_src,
                                                            const probe_half8_t* __restrict__ b_src,
                                                            uint32_t chunk_mask, float* out, int iters) {
    const uint32_t g = blockIdx.x * 512u + threadIdx.x;
    probe_half8_t a[8], b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = a_src[(g * 8u + j) & chunk_mask];
        b[j] = b_src[(g * 8u + j) & chunk_mask];
    }
    probe_float16_t c[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) c[q] = probe_float16_t{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 16; ++j)
            c[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j & 7], b[(j * 3 + 1) & 7], c[j & 3], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < 16; ++i) s += c[q][i];
    out[g] = s;
}

}  // namespace

// Launches `blocks` workgroups of 512 threads, each wavefront running iters x 16
// MFMAs; a_src / b_src hold n_chunks 16-byte chunks of f16 each (n_chunks a
// power of two); out holds blocks * 512 floats.  Returns 0 or the hipError_t of
// the launch.  FLOPs of one launch: blocks * 8 * iters * 16 * 32768.
extern "C" int32_t grout_probe_mfma_f16(const void* a_src, const void* b_src, int64_t n_chunks,
                                        float* out, int32_t blocks, int32_t iters, void* stream) {
    if (a_src == nullptr || b_src == nullptr || out == nullptr || blocks <= 0 || iters <= 0 ||
        n_chunks <= 0 || n_chunks > (int64_t{1} << 31) || (n_chunks & (n_chunks - 1)) != 0)
        return -9;
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(static_cast<unsigned>(blocks)), dim3(512), 0,
                       reinterpret_cast<hipStream_t>(stream),
                       reinterpret_cast<const probe_half8_t*>(a_src),
                       reinterpret_cast<const probe_half8_t*>(b_src),
                       static_cast<uint32_t>(n_chunks - 1), out, iters);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int32_t>(e);
}

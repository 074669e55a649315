// Checkpoint tensors to f16 on the device: the element conversion of grout's
// weight loader (cast_to_f16, src/loader.rs:107-145), run as an HBM-bound
// kernel after a raw byte copy instead of a per-element host loop.
//   F16:  bit copy;
//   BF16: f16::from_f32(bf16::to_f32(x)) (bf16 -> f32 is exact, one RNE rounding);
//   F32:  f16::from_f32(x) (RNE, overflow to inf, f16 subnormals kept);
//   F64:  f16::from_f32(x as f32) (two RNE roundings, as the reference does).
// The destination may be a row range of a merged matrix, so q/k/v and
// gate/up land in qkv_proj / gate_up_proj without a separate concatenation
// (concat_weight_rows_2d, src/model.rs:6021-6070).
#include "abi_util.h"
#include "common.h"

namespace grout {

template <int kDtype>
__device__ __forceinline__ half_t cast_one(const unsigned char* src, int64_t i) {
    if constexpr (kDtype == GROUT_DTYPE_F16) {
        return __builtin_bit_cast(half_t, reinterpret_cast<const uint16_t*>(src)[i]);
    } else if constexpr (kDtype == GROUT_DTYPE_BF16) {
        const uint32_t bits = static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(src)[i]) << 16;
        return static_cast<half_t>(__builtin_bit_cast(float, bits));
    } else if constexpr (kDtype == GROUT_DTYPE_F32) {
        return static_cast<half_t>(reinterpret_cast<const float*>(src)[i]);
    } else {
        // Two roundings, f64 -> f32 -> f16.  The empty asm keeps the f32 value
        // opaque: otherwise the two truncations fold into one f64 -> f16
        // rounding, which differs on values just past an f16 tie.
        float f = static_cast<float>(reinterpret_cast<const double*>(src)[i]);
        asm volatile("" : "+v"(f));
        return static_cast<half_t>(f);
    }
}

// Thread t converts elements [8t, 8t + 8) with one 16-byte store; the loads
// are 16, 16, 32 or 64 contiguous bytes per thread.  A scalar tail handles
// n % 8 (only the last thread has one).
template <int kDtype>
__global__ __launch_bounds__(256) void cast_to_f16_kernel(const unsigned char* __restrict__ src,
                                                          uint16_t* __restrict__ dst, int64_t n) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t i0 = t * 8;
    if (i0 >= n) return;
    if (i0 + 8 <= n) {
        half8_t o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = cast_one<kDtype>(src, i0 + e);
        store_half8(dst + i0, o);
    } else {
        for (int64_t i = i0; i < n; ++i) dst[i] = __builtin_bit_cast(uint16_t, cast_one<kDtype>(src, i));
    }
}

}  // namespace grout

using namespace grout;

extern "C" int32_t grout_cast_to_f16(const void* src, int32_t src_dtype, uint16_t* dst,
                                     int64_t n, grout_stream_t stream) {
    GROUT_REQUIRE_PTR(src);
    GROUT_REQUIRE_PTR(dst);
    GROUT_REQUIRE(src_dtype >= GROUT_DTYPE_F16 && src_dtype <= GROUT_DTYPE_F64, GROUT_ERR_ARG);
    GROUT_REQUIRE(n >= 0, GROUT_ERR_ARG);
    if (n == 0) return GROUT_OK;
    const int64_t threads = (n + 7) / 8;
    const int64_t blocks = (threads + 255) / 256;
    GROUT_REQUIRE(blocks <= 0x7fffffff, GROUT_ERR_ARG);
    const unsigned char* s = static_cast<const unsigned char*>(src);
    const dim3 grid(static_cast<unsigned>(blocks));
    const hipStream_t hs = to_hip(stream);
    switch (src_dtype) {
        case GROUT_DTYPE_F16: hipLaunchKernelGGL(cast_to_f16_kernel<GROUT_DTYPE_F16>, grid, dim3(256), 0, hs, s, dst, n); break;
        case GROUT_DTYPE_BF16: hipLaunchKernelGGL(cast_to_f16_kernel<GROUT_DTYPE_BF16>, grid, dim3(256), 0, hs, s, dst, n); break;
        case GROUT_DTYPE_F32: hipLaunchKernelGGL(cast_to_f16_kernel<GROUT_DTYPE_F32>, grid, dim3(256), 0, hs, s, dst, n); break;
        default: hipLaunchKernelGGL(cast_to_f16_kernel<GROUT_DTYPE_F64>, grid, dim3(256), 0, hs, s, dst, n); break;
    }
    return launch_status();
}

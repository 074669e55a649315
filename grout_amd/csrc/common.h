// Shared device helpers for the gfx950 attention kernels: vector types, MFMA
// wrappers, 16-byte global/LDS moves and wave-level exchanges.
//
// Lane layouts (verified on gfx950):
//  * v_mfma_f32_32x32x16_f16: A lane l holds row l%32, k = 8*(l/32)+i;
//    B lane l holds column l%32, k = 8*(l/32)+i; C register r of lane l is
//    row 8*(r/4) + 4*(l/32) + r%4, column l%32.
//  * v_mfma_f32_16x16x32_f16: A lane l holds row l%16, k = 8*(l/16)+i;
//    B lane l holds column l%16, k = 8*(l/16)+i; C register r of lane l is
//    row 4*(l/16) + r, column l%16.
//  * ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
//    (i%4) of the 8-byte chunk addressed by lane 4*j + i/4, as element j.
//  * v_permlane32_swap(a, b): returns {a with lanes 32..63 replaced by b's
//    lanes 0..31, b with lanes 0..31 replaced by a's lanes 32..63}.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace grout {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;
constexpr int kWave = 64;

__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 16-byte global load / store of 8 halves.
__device__ __forceinline__ half8_t load_half8(const uint16_t* p) {
    return *reinterpret_cast<const half8_t*>(p);
}
__device__ __forceinline__ void store_half8(uint16_t* p, half8_t v) {
    *reinterpret_cast<half8_t*>(p) = v;
}
__device__ __forceinline__ uint4_t load_u128(const void* p) {
    return *reinterpret_cast<const uint4_t*>(p);
}
__device__ __forceinline__ void store_u128(void* p, uint4_t v) {
    *reinterpret_cast<uint4_t*>(p) = v;
}

typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// Transposing LDS read of 4 halves (see the layout note at the top).
__device__ __forceinline__ half4_t lds_read_tr16(const half_t* lds_ptr) {
    short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4_t*)(lds_ptr));
    return __builtin_bit_cast(half4_t, v);
}

// Value of lane l^32 for every lane l.
__device__ __forceinline__ float swap_halves(float x) {
    int xi = __builtin_bit_cast(int, x);
    auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
    int lane = __lane_id();
    return __builtin_bit_cast(float, lane < 32 ? (int)r[1] : (int)r[0]);
}

// Value of lane l ^ 16: v_permlane16_swap exchanges 16-lane rows 2i and 2i+1
// between its two operands; with both equal, an odd row's partner arrives in
// the first result, an even row's in the second.
__device__ __forceinline__ float swap_rows16(float x) {
    int xi = __builtin_bit_cast(int, x);
    auto r = __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
    int lane = __lane_id();
    return __builtin_bit_cast(float, (lane & 16) ? (int)r[0] : (int)r[1]);
}

// Orders LDS traffic of one wavefront (lanes exchange data through LDS
// without a workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ half8_t cat(half4_t a, half4_t b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

}  // namespace grout

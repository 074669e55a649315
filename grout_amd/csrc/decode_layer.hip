// Decode-layer ops either side of the attention step: the fused residual add +
// RMSNorm of one hidden row, the f16 GEMV of the QKV / output projections,
// and the two-stage greedy argmax that turns logits into the next token.
//
// Replaces add_rms_norm_decode_raw_f16 (src/kernels.rs:3076-3216), the cuBLAS
// GemvInPlace nodes of the decode graph (src/cublas.rs:572-607, recorded at
// src/model.rs:3166-3175 and :3505-3512) and argmax_blocks_f16 +
// argmax_reduce_blocks_to_u32 (src/kernels.rs:345-392, :458-505).
//
// All three are HBM- or latency-bound; the kernels are shaped for that:
//  * the norm is one workgroup of 1024 threads holding the row in registers
//    between the sum of squares and the normalisation (one read of each
//    input, one write of each output);
//  * the GEMV streams each weight row with all 256 threads of a workgroup
//    (16-byte non-temporal loads, up to 8 rows x 3 chunks in flight per
//    thread) and accumulates in f32 with v_dot2_f32_f16 (exact f16 products);
//  * the argmax reduces (value, index) pairs, the lowest index winning ties,
//    in 2048-element blocks and then over the blocks.
#include <math.h>

#include "abi_util.h"
#include "common.h"

namespace grout {

// ------------------------------------------------------------------ norm --

constexpr int kNormThreads = 1024;
constexpr int kNormChunks = 4;  // 16-byte chunks per thread: n <= 8 * 1024 * 4
constexpr int kNormMaxN = 8 * kNormThreads * kNormChunks;

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// kEmbed = false: the row is residual + x (add_rms_norm_decode_raw_f16).
// kEmbed = true: the row is embedding row *token of `residual` (the table,
// [vocab, n]) and x is absent: embedding_batch_f16 followed by rms_norm_f16
// (src/kernels.rs:693-711, :304-344), with residual_out receiving the row.
template <bool kEmbed>
__global__ __launch_bounds__(kNormThreads) void rms_norm_decode_kernel(
    const uint16_t* residual, const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, uint16_t* residual_out, float eps, int n,
    const uint32_t* __restrict__ token, uint32_t vocab) {
    // residual_out may be residual itself (the decode graph updates the
    // residual stream in place): each thread reads its chunks before the
    // barrier and writes the same chunks after it.
    if constexpr (kEmbed) {
        // A token id past the table (never produced by the argmax; only a bad
        // initial value) reads the last row instead of faulting.
        const uint32_t t = min(*token, vocab - 1u);
        residual += static_cast<int64_t>(t) * n;
    }
    __shared__ float red[kNormThreads / kWave];
    const int tid = threadIdx.x;
    float c[kNormChunks][8];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k) {
        const int i = (tid + k * kNormThreads) * 8;
        if (i < n) {
            const half8_t r8 = load_half8(residual + i);
            if constexpr (kEmbed) {
#pragma unroll
                for (int e = 0; e < 8; ++e) c[k][e] = static_cast<float>(r8[e]);
            } else {
                const half8_t x8 = load_half8(x + i);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    c[k][e] = static_cast<float>(r8[e]) + static_cast<float>(x8[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += c[k][e] * c[k][e];
        }
    }
    ss = wave_sum_f32(ss);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / kWave; ++i) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(n) + eps);
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k) {
        const int i = (tid + k * kNormThreads) * 8;
        if (i < n) {
#pragma clang fp contract(off)
            const half8_t w8 = load_half8(w + i);
            half8_t o, rs;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                o[e] = static_cast<half_t>((c[k][e] * inv) * static_cast<float>(w8[e]));
                rs[e] = static_cast<half_t>(c[k][e]);
            }
            store_half8(out + i, o);
            store_half8(residual_out + i, rs);
        }
    }
}

// -------------------------------------------------------------- SiLU * up --

constexpr int kPointwiseThreads = 256;

// silu_mul_2d_f16 (src/kernels.rs:271-301): out = f16(sigmoid(g) * g * u) in
// f32 with sigmoid(g) = 1 / (1 + exp(-g)), for f16 inputs g and u.
__device__ __forceinline__ half_t silu_mul1(half_t g16, half_t u16) {
#pragma clang fp contract(off)
    const float g = static_cast<float>(g16);
    const float sig = 1.0f / (1.0f + expf(-g));
    float p = (sig * g) * static_cast<float>(u16);
    // The product is rounded to f32, then to f16, as the reference computes
    // it: the empty asm keeps the backend from folding the multiply and the
    // conversion into one v_fma_mixlo_f16 (a single rounding, 1 ulp away in
    // rare cases).
    asm volatile("" : "+v"(p));
    return static_cast<half_t>(p);
}

// 8 elements per thread.
__global__ __launch_bounds__(kPointwiseThreads) void silu_mul_kernel(
    const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up, uint16_t* __restrict__ out,
    int n) {
    const int i = (static_cast<int>(blockIdx.x) * kPointwiseThreads + static_cast<int>(threadIdx.x)) * 8;
    if (i >= n) return;
    const half8_t g8 = load_half8(gate + i);
    const half8_t u8 = load_half8(up + i);
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = silu_mul1(g8[e], u8[e]);
    store_half8(out + i, o);
}

// ------------------------------------------------------------------ GEMV --

constexpr int kGemvThreads = 256;
// 16-byte chunks per thread per row in flight.  3 measured 1.6% faster than 2
// on the Qwen3-32B token step (11.72 -> 11.54 ms, with the residency cap
// re-tuned below); 4 no better than 3.
constexpr int kGemvUnroll = 3;
constexpr int kGemvMaxK = 32768;

__device__ __forceinline__ float dot8(half8_t a, half8_t b, float acc) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const half2_t a2 = {a[2 * p], a[2 * p + 1]};
        const half2_t b2 = {b[2 * p], b[2 * p + 1]};
        acc = __builtin_amdgcn_fdot2(a2, b2, acc, false);
    }
    return acc;
}

// Sums each of v[0..R) over the 64 lanes by recursive halving: at the step of
// offset 32 the lanes with bit 5 set keep rows [R/2, R) and the others rows
// [0, R/2), each adding its partner's half; after log2(R) such steps every
// lane holds one row, and the remaining xor steps complete the sum.  Row r
// ends in v[0] of lane r * (64 / R) (and the lanes above it up to the next
// row).  6 + R - 1 shuffles instead of 6 R.
template <int R>
__device__ __forceinline__ float wave_multi_sum(float (&v)[R], int lane) {
    int off = 32;
#pragma unroll
    for (int half = R / 2; half >= 1; half /= 2, off /= 2) {
        const bool up = (lane & off) != 0;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float keep = up ? v[i + half] : v[i];
            const float send = up ? v[i] : v[i + half];
            v[i] = keep + __shfl_xor(send, off);
        }
    }
#pragma unroll
    for (; off > 0; off >>= 1) v[0] += __shfl_xor(v[0], off);
    return v[0];
}

// Workgroup b computes out rows b*R + [0, R).  kSilu (the gate_up GEMV with
// SiLU * up in its epilogue): workgroup b computes gate rows b*R/2 + [0, R/2)
// and the matching up rows half_m + b*R/2 + [0, R/2) as its R rows, rounds
// each sum to f16 as the plain GEMV stores it, and writes f16(silu(g) * u)
// for its R/2 outputs: bit-identical to the GEMV followed by silu_mul_kernel,
// without the second launch and the intermediate's round trip.  Thread t of the workgroup
// reads the 16-byte chunks t, t + 256, ... of each of the R rows (4 KB of a
// row per workgroup load step, contiguous), so a row of k halves is streamed
// by all 256 threads at once and R * kGemvUnroll chunks per thread are in
// flight.  Weight chunks are loaded non-temporal: each is read once per token
// step, and streaming them past the caches measured 5-6% faster per GEMV and
// 7.7% on the Qwen3-32B token step (12.57 -> 11.60 ms).  x chunks come from
// global memory with the default policy (the same chunk for all R rows; every
// workgroup hits it in L2).  Products are exact in f32
// (v_dot2_f32_f16); the sum order is per thread, then across lanes, then
// across the four wavefronts.
template <int R, bool kSilu = false>
__global__ __launch_bounds__(kGemvThreads) void gemv_f16_kernel(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ x, uint16_t* __restrict__ out,
    int m, int k, int half_m = 0) {
    static_assert(!kSilu || R >= 2, "a SiLU workgroup pairs R/2 gate rows with R/2 up rows");
    __shared__ float red[kGemvThreads / kWave][R];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int nchunk = k / 8;
    constexpr int kOut = kSilu ? R / 2 : R;  // outputs per workgroup
    const int row0 = static_cast<int>(blockIdx.x) * kOut;
    const half8_t* xc = reinterpret_cast<const half8_t*>(x);
    const half8_t* wr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        // Outputs past m repeat the last row (not stored).
        const int o = min(row0 + r % kOut, m - 1);
        const int row = (kSilu && r >= kOut) ? half_m + o : o;
        wr[r] = reinterpret_cast<const half8_t*>(W + static_cast<int64_t>(row) * k);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    int c = tid;
    for (; c + kGemvThreads * (kGemvUnroll - 1) < nchunk; c += kGemvThreads * kGemvUnroll) {
        half8_t wv[kGemvUnroll][R];
        half8_t xv[kGemvUnroll];
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
#pragma unroll
            for (int r = 0; r < R; ++r) wv[u][r] = __builtin_nontemporal_load(&wr[r][c + kGemvThreads * u]);
            xv[u] = xc[c + kGemvThreads * u];
        }
        // Keep every load of the step ahead of the first dot product: left to
        // itself the scheduler interleaves them and waits for each in turn.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = dot8(wv[u][r], xv[u], acc[r]);
    }
    {
        // Fewer than kGemvUnroll chunks are left; for rows of k <= 4096 that
        // is the whole row, as the loop above never runs.  Their loads go out
        // together too, then the dot products run in chunk order (Qwen3-4B
        // token step 2.557 -> 2.527 ms against one chunk at a time).
        half8_t wv[kGemvUnroll - 1][R];
        half8_t xv[kGemvUnroll - 1];
#pragma unroll
        for (int u = 0; u < kGemvUnroll - 1; ++u) {
            if (c + kGemvThreads * u < nchunk) {
#pragma unroll
                for (int r = 0; r < R; ++r) wv[u][r] = __builtin_nontemporal_load(&wr[r][c + kGemvThreads * u]);
                xv[u] = xc[c + kGemvThreads * u];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kGemvUnroll - 1; ++u) {
            if (c + kGemvThreads * u < nchunk) {
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] = dot8(wv[u][r], xv[u], acc[r]);
            }
        }
    }
    const float v = wave_multi_sum<R>(acc, lane);
    constexpr int kStride = kWave / R;
    if (lane % kStride == 0) red[wave][lane / kStride] = v;
    __syncthreads();
    if constexpr (kSilu) {
        if (tid < kOut && row0 + tid < m) {
            float tg = red[0][tid], tu = red[0][tid + kOut];
#pragma unroll
            for (int w = 1; w < kGemvThreads / kWave; ++w) {
                tg += red[w][tid];
                tu += red[w][tid + kOut];
            }
            out[row0 + tid] = __builtin_bit_cast(
                uint16_t, silu_mul1(static_cast<half_t>(tg), static_cast<half_t>(tu)));
        }
    } else if (tid < R && row0 + tid < m) {
        float t = red[0][tid];
#pragma unroll
        for (int w = 1; w < kGemvThreads / kWave; ++w) t += red[w][tid];
        out[row0 + tid] = __builtin_bit_cast(uint16_t, static_cast<half_t>(t));
    }
}

// ---------------------------------------------------------------- argmax --

constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxBlock = kArgmaxThreads * 8;  // logits per first-stage block

// (v, i) beats (bv, bi) when larger, or equal with a lower index.
__device__ __forceinline__ void argmax_take(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__device__ __forceinline__ void argmax_block_reduce(float& bv, int& bi, float* sv, int* si) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        argmax_take(bv, bi, ov, oi);
    }
    const int tid = threadIdx.x;
    if ((tid & (kWave - 1)) == 0) {
        sv[tid / kWave] = bv;
        si[tid / kWave] = bi;
    }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
#pragma unroll
    for (int wv = 1; wv < kArgmaxThreads / kWave; ++wv) argmax_take(bv, bi, sv[wv], si[wv]);
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_blocks_kernel(
    const uint16_t* __restrict__ logits, int n, float* __restrict__ block_max,
    uint32_t* __restrict__ block_idx) {
    __shared__ float sv[kArgmaxThreads / kWave];
    __shared__ int si[kArgmaxThreads / kWave];
    const int base = static_cast<int>(blockIdx.x) * kArgmaxBlock + threadIdx.x * 8;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (base + 8 <= n) {
        const half8_t v = load_half8(logits + base);
#pragma unroll
        for (int e = 0; e < 8; ++e) argmax_take(bv, bi, static_cast<float>(v[e]), base + e);
    } else {
        for (int e = 0; base + e < n; ++e)
            argmax_take(bv, bi, static_cast<float>(__builtin_bit_cast(half_t, logits[base + e])), base + e);
    }
    argmax_block_reduce(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        block_max[blockIdx.x] = bv;
        block_idx[blockIdx.x] = static_cast<uint32_t>(bi);
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_reduce_kernel(
    const float* __restrict__ block_max, const uint32_t* __restrict__ block_idx, int nblocks,
    uint32_t* __restrict__ token) {
    __shared__ float sv[kArgmaxThreads / kWave];
    __shared__ int si[kArgmaxThreads / kWave];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int b = threadIdx.x; b < nblocks; b += kArgmaxThreads)
        argmax_take(bv, bi, block_max[b], static_cast<int>(block_idx[b]));
    argmax_block_reduce(bv, bi, sv, si);
    if (threadIdx.x == 0) token[0] = static_cast<uint32_t>(bi == 0x7fffffff ? 0 : bi);
}

}  // namespace grout

using namespace grout;

extern "C" int32_t grout_add_rms_norm_decode(const uint16_t* residual, const uint16_t* x,
                                             const uint16_t* weight, uint16_t* out,
                                             uint16_t* residual_out, float eps, int32_t n,
                                             grout_stream_t stream) {
    GROUT_REQUIRE_PTR(residual);
    GROUT_REQUIRE_PTR(x);
    GROUT_REQUIRE_PTR(weight);
    GROUT_REQUIRE_PTR(out);
    GROUT_REQUIRE_PTR(residual_out);
    GROUT_REQUIRE(n >= 8 && n % 8 == 0 && n <= kNormMaxN, GROUT_ERR_ARG);
    GROUT_REQUIRE(eps >= 0.0f && eps < 1.0e30f, GROUT_ERR_ARG);
    hipLaunchKernelGGL(rms_norm_decode_kernel<false>, dim3(1), dim3(kNormThreads), 0,
                       to_hip(stream), residual, x, weight, out, residual_out, eps, n, nullptr, 0u);
    return launch_status();
}

extern "C" int32_t grout_embed_rms_norm_decode(const uint32_t* token, const uint16_t* table,
                                               int32_t vocab, const uint16_t* weight,
                                               uint16_t* out, uint16_t* residual_out, float eps,
                                               int32_t n, grout_stream_t stream) {
    GROUT_REQUIRE(token != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(token) & 3u) == 0, GROUT_ERR_ALIGNMENT);
    GROUT_REQUIRE_PTR(table);
    GROUT_REQUIRE_PTR(weight);
    GROUT_REQUIRE_PTR(out);
    GROUT_REQUIRE_PTR(residual_out);
    GROUT_REQUIRE(n >= 8 && n % 8 == 0 && n <= kNormMaxN && vocab >= 1, GROUT_ERR_ARG);
    GROUT_REQUIRE(eps >= 0.0f && eps < 1.0e30f, GROUT_ERR_ARG);
    hipLaunchKernelGGL(rms_norm_decode_kernel<true>, dim3(1), dim3(kNormThreads), 0,
                       to_hip(stream), table, nullptr, weight, out, residual_out, eps, n, token,
                       static_cast<uint32_t>(vocab));
    return launch_status();
}

extern "C" int32_t grout_silu_mul_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out,
                                      int32_t n, grout_stream_t stream) {
    GROUT_REQUIRE_PTR(gate);
    GROUT_REQUIRE_PTR(up);
    GROUT_REQUIRE_PTR(out);
    GROUT_REQUIRE(n >= 8 && n % 8 == 0 && n <= (1 << 30), GROUT_ERR_ARG);
    const unsigned blocks = static_cast<unsigned>((n / 8 + kPointwiseThreads - 1) / kPointwiseThreads);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(kPointwiseThreads), 0, to_hip(stream),
                       gate, up, out, n);
    return launch_status();
}

// Residency of the largest plain GEMVs (>= 2^28 weight elements: lm_head,
// 8 rows per workgroup) with rows longer than 4096: their launches reserve
// unused LDS so that at most kGemvResident workgroups share a CU, fewer
// concurrent row streams per CU.  With 2 chunks in flight per row this was
// worth 0.6% of the Qwen3-32B token step; with 3 it is within 0.01 ms of 3, 4
// or uncapped.  Short rows (Qwen3-4B's lm_head, k = 2560) run uncapped: their
// workgroups are short-lived, and the cap cost 21 us of the 4B token step.
constexpr int kGemvResident = 2;
constexpr size_t gemv_reserve_lds(int resident) {
    return static_cast<size_t>(160 * 1024 / resident - 1024);  // static LDS stays below 1 KB
}

extern "C" int32_t grout_gemv_f16(const uint16_t* weight, const uint16_t* x, uint16_t* out,
                                  int32_t m, int32_t k, grout_stream_t stream) {
    GROUT_REQUIRE_PTR(weight);
    GROUT_REQUIRE_PTR(x);
    GROUT_REQUIRE(out != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(out) & 1u) == 0, GROUT_ERR_ALIGNMENT);
    GROUT_REQUIRE(m >= 1 && k >= 8 && k % 8 == 0 && k <= kGemvMaxK, GROUT_ERR_ARG);
    // Rows per workgroup, measured on the Qwen3-32B token step: 2 for the
    // projections (qkv 10240, o_proj and down 5120 rows: 11.41 against 11.51
    // ms/token with 8 and 4), 8 only for vocabulary-sized outputs (lm_head at
    // 2 rows cost 0.1 ms more), 1 below 2048 rows so short outputs still
    // spread over the CUs.
    const int rows = m >= 16 * 1024 ? 8 : m >= 2 * 1024 ? 2 : 1;
    const unsigned blocks = static_cast<unsigned>((m + rows - 1) / rows);
    const hipStream_t s = to_hip(stream);
    const dim3 block(kGemvThreads);
    const size_t lds = static_cast<int64_t>(m) * k >= (int64_t{1} << 28) && k > 4096
                           ? gemv_reserve_lds(kGemvResident)
                           : 0;
    switch (rows) {
        case 8: hipLaunchKernelGGL(gemv_f16_kernel<8>, dim3(blocks), block, lds, s, weight, x, out, m, k); break;
        case 2: hipLaunchKernelGGL(gemv_f16_kernel<2>, dim3(blocks), block, 0, s, weight, x, out, m, k); break;
        default: hipLaunchKernelGGL(gemv_f16_kernel<1>, dim3(blocks), block, 0, s, weight, x, out, m, k); break;
    }
    return launch_status();
}

extern "C" int32_t grout_gemv_silu_mul_f16(const uint16_t* gate_up, const uint16_t* x, uint16_t* out,
                                           int32_t n, int32_t k, grout_stream_t stream) {
    GROUT_REQUIRE_PTR(gate_up);
    GROUT_REQUIRE_PTR(x);
    GROUT_REQUIRE(out != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(out) & 1u) == 0, GROUT_ERR_ALIGNMENT);
    GROUT_REQUIRE(n >= 1 && n <= (1 << 29) && k >= 8 && k % 8 == 0 && k <= kGemvMaxK, GROUT_ERR_ARG);
    // One gate row and its up row per workgroup (n workgroups), at full
    // residency: on the Qwen3-32B token step 11.30 ms/token against 11.41
    // with 4 + 4 rows and 11.44 with 2 + 2; capping the 2-row workgroups'
    // residency at 2 or 4 per CU measured 13.71 and 11.81.
    hipLaunchKernelGGL((gemv_f16_kernel<2, true>), dim3(static_cast<unsigned>(n)), dim3(kGemvThreads),
                       0, to_hip(stream), gate_up, x, out, n, k, n);
    return launch_status();
}

// Logit counts up to 2^30 (block offsets stay inside int).
constexpr int32_t kArgmaxMaxN = 1 << 30;

extern "C" int32_t grout_argmax_blocks(int32_t n) {
    if (n < 1 || n > kArgmaxMaxN) return GROUT_ERR_ARG;
    return (n + kArgmaxBlock - 1) / kArgmaxBlock;
}

extern "C" int32_t grout_argmax_f16(const uint16_t* logits, float* block_max, uint32_t* block_idx,
                                    uint32_t* token, int32_t n, grout_stream_t stream) {
    GROUT_REQUIRE_PTR(logits);
    GROUT_REQUIRE(block_max != nullptr && block_idx != nullptr && token != nullptr,
                  GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE(((reinterpret_cast<uintptr_t>(block_max) | reinterpret_cast<uintptr_t>(block_idx) |
                    reinterpret_cast<uintptr_t>(token)) & 3u) == 0,
                  GROUT_ERR_ALIGNMENT);
    GROUT_REQUIRE(n >= 1 && n <= kArgmaxMaxN, GROUT_ERR_ARG);
    const int nblocks = (n + kArgmaxBlock - 1) / kArgmaxBlock;
    hipLaunchKernelGGL(argmax_blocks_kernel, dim3(nblocks), dim3(kArgmaxThreads), 0, to_hip(stream),
                       logits, n, block_max, block_idx);
    const int32_t st = launch_status();
    if (st != GROUT_OK) return st;
    hipLaunchKernelGGL(argmax_reduce_kernel, dim3(1), dim3(kArgmaxThreads), 0, to_hip(stream),
                       block_max, block_idx, nblocks, token);
    return launch_status();
}

// Fused per-head Q/K RMSNorm + RoPE + KV-cache write (prefill and decode).
//
// Replaces qk_norm_rope_kv_prefill_raw_f16 (src/kernels.rs:3415-3732) and
// qk_norm_rope_kv_decode_raw_f16 (src/kernels.rs:3750-4016).
//
// The op is HBM-bound (read q,k,v once, write q_out and two cache rows), so
// the kernel is organised for 16-byte accesses and for computing each RoPE
// angle once per token instead of once per head:
//  * A workgroup owns a few tokens and a range of heads.  It first evaluates
//    cos/sin(f32(pos) * inv_freq[j]) for its tokens into LDS (64 per token).
//  * Eight lanes own one 128-wide head row: lane t holds elements
//    [8t, 8t+8) of the low half and [64+8t, 64+8t+8) of the high half, so
//    each RoPE pair (j, j+64) sits in one lane and every access is 16 bytes.
//  * The row's sum of squares is reduced over the 8 lanes with xor shuffles.
// Arithmetic follows the reference order: ss = sum(lo*lo + hi*hi),
// inv = 1/sqrt(ss/128 + eps), n = x*inv*w, y_lo = n_lo*cos - n_hi*sin,
// y_hi = n_hi*cos + n_lo*sin, f16 round-to-nearest-even.  Contraction into
// FMA is disabled so each product rounds as written.
#include "abi_util.h"
#include "common.h"

namespace grout {

constexpr int kNormThreads = 256;
constexpr int kNormRowSlots = kNormThreads / 8;  // rows in flight per workgroup
constexpr int kNormMaxTokens = 8;                // tokens per workgroup (LDS sin/cos table)
// Prefill launches reserve dynamic LDS so that at most kNormResident
// workgroups (16 waves) share a CU instead of the 8 that registers and the
// static 4 KB table allow: fewer concurrent row streams per CU measured
// 1.5-3% faster at 8192-32768 tokens (c3: 33.2 -> 32.5 us with the buffers
// resident in the last-level cache, 42.3 -> 40.9 us with them in HBM) and no
// different on grids of at most 4 workgroups per CU.
//
// The outputs are stored with the default policy.  Non-temporal stores made
// this kernel 5% faster on its own with its data in HBM, but the prefill
// attention that reads q_out and the cache rows next then finds them outside
// the last-level cache: the norm + attention pair measured 0.3-0.7% slower
// (c3 537.7 against 536.3 us, 16384 tokens 2034 against 2020 us, 512 tokens
// 16.2 against 15.6 us).
constexpr int kNormResident = 4;
constexpr size_t kNormReserveLds =
    160 * 1024 / kNormResident - 2 * kNormMaxTokens * 64 * sizeof(float) - 1024;

template <bool kDevicePos>
__global__ __launch_bounds__(kNormThreads) void qk_norm_rope_kv_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ q_weight,
    const uint16_t* __restrict__ k_weight, const float* __restrict__ inv_freq,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, float eps, int position_start,
    const uint32_t* __restrict__ d_position, int seq_len, int num_q_heads, int num_kv_heads,
    int max_seq_len, int tokens_per_block, int heads_per_block) {
#pragma clang fp contract(off)
    __shared__ float s_cos[kNormMaxTokens][64];
    __shared__ float s_sin[kNormMaxTokens][64];

    const int tid = threadIdx.x;
    const int tok0 = blockIdx.x * tokens_per_block;
    const int ntok = min(tokens_per_block, seq_len - tok0);
    const int heads = num_q_heads + num_kv_heads;
    const int head0 = blockIdx.y * heads_per_block;
    const int nhead = min(heads_per_block, heads - head0);
    // Decode reads the slot from device memory (u32 bitcast to i32,
    // src/kernels.rs:3934-3937) so the launch can be replayed in a graph.
    const int pos0 = (kDevicePos ? static_cast<int>(*d_position) : position_start) + tok0;

    // theta is the reference's f32 product; its sine/cosine are evaluated in
    // f64 and rounded once to f32 (correctly rounded), so the angle table does
    // not depend on the f32 sin/cos implementation.  One evaluation per
    // (token, frequency) serves every head of the token.
    for (int i = tid; i < ntok * 64; i += kNormThreads) {
        const int t = i >> 6, j = i & 63;
        const float theta = static_cast<float>(pos0 + t) * inv_freq[j];
        double sv, cv;
        sincos(static_cast<double>(theta), &sv, &cv);
        s_cos[t][j] = static_cast<float>(cv);
        s_sin[t][j] = static_cast<float>(sv);
    }
    __syncthreads();

    const int lane8 = tid & 7;
    const int rows = ntok * nhead;
    for (int r = tid >> 3; r < rows; r += kNormRowSlots) {
        const int t = r / nhead;
        const int h = head0 + (r - t * nhead);
        const int s = tok0 + t;
        const int pos = pos0 + t;
        const bool is_q = h < num_q_heads;
        const int kvh = h - num_q_heads;
        const uint16_t* src = is_q ? q + (static_cast<int64_t>(s) * num_q_heads + h) * kHeadDim
                                   : k + (static_cast<int64_t>(s) * num_kv_heads + kvh) * kHeadDim;
        const uint16_t* w = is_q ? q_weight : k_weight;
        const half8_t xlo = load_half8(src + 8 * lane8);
        const half8_t xhi = load_half8(src + 64 + 8 * lane8);
        const half8_t wlo = load_half8(w + 8 * lane8);
        const half8_t whi = load_half8(w + 64 + 8 * lane8);

        // Sum of squares: lane t adds pairs 8t..8t+7 in order, then the 8
        // partials combine pairwise ((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7)).
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float a = static_cast<float>(xlo[i]);
            const float b = static_cast<float>(xhi[i]);
            ss += a * a + b * b;
        }
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        const float inv_rms = 1.0f / sqrtf(ss / 128.0f + eps);

        half8_t ylo, yhi;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float n_lo = static_cast<float>(xlo[i]) * inv_rms * static_cast<float>(wlo[i]);
            const float n_hi = static_cast<float>(xhi[i]) * inv_rms * static_cast<float>(whi[i]);
            const float c = s_cos[t][8 * lane8 + i];
            const float sn = s_sin[t][8 * lane8 + i];
            ylo[i] = static_cast<half_t>(n_lo * c - n_hi * sn);
            yhi[i] = static_cast<half_t>(n_hi * c + n_lo * sn);
        }

        if (is_q) {
            uint16_t* dst = q_out + (static_cast<int64_t>(s) * num_q_heads + h) * kHeadDim;
            store_half8(dst + 8 * lane8, ylo);
            store_half8(dst + 64 + 8 * lane8, yhi);
        } else if (static_cast<unsigned>(pos) < static_cast<unsigned>(max_seq_len)) {
            const int64_t slot = (static_cast<int64_t>(kvh) * max_seq_len + pos) * kHeadDim;
            store_half8(k_cache + slot + 8 * lane8, ylo);
            store_half8(k_cache + slot + 64 + 8 * lane8, yhi);
            const uint16_t* vsrc = v + (static_cast<int64_t>(s) * num_kv_heads + kvh) * kHeadDim;
            store_u128(v_cache + slot + 8 * lane8, load_u128(vsrc + 8 * lane8));
            store_u128(v_cache + slot + 64 + 8 * lane8, load_u128(vsrc + 64 + 8 * lane8));
        }
    }
}

// Work split: long prompts give each workgroup several tokens and all heads
// (one LDS angle table serves every head); short ones spread heads over
// workgroups so a decode step uses a few CUs instead of one.
static void norm_launch_shape(int seq_len, int heads, int* tpb, int* hpb) {
    if (seq_len >= 4096) {
        *tpb = 4;
    } else if (seq_len >= 1024) {
        *tpb = 2;
    } else {
        *tpb = 1;
    }
    *hpb = (static_cast<int64_t>(seq_len) * heads >= 4096) ? heads : kNormRowSlots;
}

}  // namespace grout

using namespace grout;

extern "C" int32_t grout_qk_norm_rope_kv_prefill(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_weight,
    const uint16_t* k_weight, const float* inv_freq, uint16_t* q_out, uint16_t* k_cache,
    uint16_t* v_cache, float eps, int32_t position_start, int32_t seq_len, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len, grout_stream_t stream) {
    // Mirrors the ensure!s of execute_qk_norm_rope_kv_prefill_op_ctx
    // (src/model.rs:4480-4560), expressed on sizes instead of tensor shapes.
    GROUT_REQUIRE_PTR(q);
    GROUT_REQUIRE_PTR(k);
    GROUT_REQUIRE_PTR(v);
    GROUT_REQUIRE_PTR(q_weight);
    GROUT_REQUIRE_PTR(k_weight);
    GROUT_REQUIRE_PTR(inv_freq);
    GROUT_REQUIRE_PTR(q_out);
    GROUT_REQUIRE_PTR(k_cache);
    GROUT_REQUIRE_PTR(v_cache);
    GROUT_REQUIRE(head_dim == kHeadDim, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
                  GROUT_ERR_HEADS);
    GROUT_REQUIRE(seq_len >= 0 && position_start >= 0 && max_seq_len > 0, GROUT_ERR_SEQ_RANGE);
    GROUT_REQUIRE(static_cast<int64_t>(position_start) + seq_len <= max_seq_len,
                  GROUT_ERR_SEQ_RANGE);
    GROUT_REQUIRE(eps >= 0.0f && eps < 1.0e30f, GROUT_ERR_ARG);
    if (seq_len == 0) return GROUT_OK;

    int tpb, hpb;
    const int heads = num_q_heads + num_kv_heads;
    norm_launch_shape(seq_len, heads, &tpb, &hpb);
    dim3 grid((seq_len + tpb - 1) / tpb, (heads + hpb - 1) / hpb);
    hipLaunchKernelGGL(qk_norm_rope_kv_kernel<false>, grid, dim3(kNormThreads), kNormReserveLds,
                       to_hip(stream),
                       q, k, v, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache, eps,
                       position_start, static_cast<const uint32_t*>(nullptr), seq_len,
                       num_q_heads, num_kv_heads, max_seq_len, tpb, hpb);
    return launch_status();
}

extern "C" int32_t grout_qk_norm_rope_kv_decode(
    const uint16_t* qkv, const uint16_t* q_weight, const uint16_t* k_weight,
    const float* inv_freq, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
    const uint32_t* d_position, float eps, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t max_seq_len, grout_stream_t stream) {
    GROUT_REQUIRE_PTR(qkv);
    GROUT_REQUIRE_PTR(q_weight);
    GROUT_REQUIRE_PTR(k_weight);
    GROUT_REQUIRE_PTR(inv_freq);
    GROUT_REQUIRE_PTR(q_out);
    GROUT_REQUIRE_PTR(k_cache);
    GROUT_REQUIRE_PTR(v_cache);
    GROUT_REQUIRE(d_position != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(d_position) & 3u) == 0, GROUT_ERR_ALIGNMENT);
    GROUT_REQUIRE(head_dim == kHeadDim, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
                  GROUT_ERR_HEADS);
    GROUT_REQUIRE(max_seq_len > 0, GROUT_ERR_SEQ_RANGE);
    GROUT_REQUIRE(eps >= 0.0f && eps < 1.0e30f, GROUT_ERR_ARG);

    // The QKV vector is [Q | K | V]; with seq_len = 1 those are exactly the
    // prefill kernel's q [1,Hq,D], k [1,Hkv,D] and v [1,Hkv,D].
    const uint16_t* q = qkv;
    const uint16_t* k = qkv + static_cast<int64_t>(num_q_heads) * kHeadDim;
    const uint16_t* v = qkv + static_cast<int64_t>(num_q_heads + num_kv_heads) * kHeadDim;
    int tpb, hpb;
    const int heads = num_q_heads + num_kv_heads;
    norm_launch_shape(1, heads, &tpb, &hpb);
    dim3 grid(1, (heads + hpb - 1) / hpb);
    hipLaunchKernelGGL(qk_norm_rope_kv_kernel<true>, grid, dim3(kNormThreads), 0, to_hip(stream),
                       q, k, v, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache, eps, 0,
                       d_position, 1, num_q_heads, num_kv_heads, max_seq_len, tpb, hpb);
    return launch_status();
}

// Split-K GQA decode attention and its log-sum-exp merge.
//
// Replaces fmha_decode_gqa_split (src/kernels.rs:2586-2749) and
// splitk_reduce_merge (src/kernels.rs:2771-2868).  The scratch layout, the
// split boundaries and the per-split numerics are the reference's:
//   s_kv = pos + 1; tiles = ceil(s_kv/BN); per = ceil(tiles/NKS);
//   split s covers tokens [s*per*BN, min((s*per+per)*BN, s_kv));
//   O_s = f16(acc/max(l,1e-8)), LSE_s = m + log2(max(l,1e-8)) in log2 units,
//   att_partial [Hkv, NKS*G, D] split-major, lse_partial [Hkv, NKS*G].
//
// Decode is HBM-bound (4-8 FLOP per byte), so the kernel is shaped for bytes
// in flight, not for arithmetic:
//  * Workgroup = (split, kv_head), 4 wavefronts.  Each wavefront walks
//    32-token sub-tiles of the split (wave w takes sub-tiles w, w+4, ...),
//    prefetching the next sub-tile's K and V (16 KB) into registers while the
//    current one is computed.
//  * All G query heads of the KV head share every K/V byte: S^T = K Q^T and
//    O^T += V^T P^T run on v_mfma_f32_16x16x32_f16 with the G heads (padded
//    to 16) as the N dimension.  K rows feed the A operand straight from
//    16-byte global loads; Q^T is held in registers for the whole split.
//  * The S^T accumulator layout is reused as the P^T operand of the PV
//    product (no data movement): the reduction slots of lane group q are the
//    tokens {4q..4q+3, 16+4q..16+4q+3} of the sub-tile.  V^T is produced in
//    the same slot order by parking the V sub-tile in a per-wave LDS buffer
//    and reading it back with ds_read_b64_tr_b16 (gfx950 transposing read).
//  * The four wavefronts' (m, l, acc) are combined through LDS at the end.
#include <math.h>

#include "abi_util.h"
#include "common.h"

namespace grout {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = kDecWaves * kWave;
constexpr int kDecSub = 32;                 // tokens per wavefront iteration
constexpr int kDecVStride = kHeadDim + 16;  // halves per LDS V row (288 B: spreads banks)
constexpr int kDecVWaveBytes = kDecSub * kDecVStride * 2;
constexpr int kDecRedBytes = kDecWaves * (16 * kHeadDim + 32) * 4;
constexpr int kDecLdsBytes =
    (kDecWaves * kDecVWaveBytes > kDecRedBytes) ? kDecWaves * kDecVWaveBytes : kDecRedBytes;
constexpr float kNegBig = -1.0e30f;

struct DecodeSplitArgs {
    const uint16_t* q;
    const uint16_t* k_cache;
    const uint16_t* v_cache;
    uint16_t* att_partial;
    float* lse_partial;
    const uint32_t* d_position;
    float scale_log2;
    int group;
    int max_seq_len;
    int block_n;
    int num_splits;
};

__device__ __forceinline__ half8_t zero_half8() { return half8_t{}; }

__global__ __launch_bounds__(kDecThreads) void attn_decode_split_kernel(DecodeSplitArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[kDecLdsBytes];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int n = lane & 15;     // head column of the MFMA tiles
    const int qgrp = lane >> 4;  // lane group: k-slice / token quartet

    // Position from device memory; clamped so no read leaves the cache.
    uint32_t pos = *a.d_position;
    if (pos >= static_cast<uint32_t>(a.max_seq_len)) pos = a.max_seq_len - 1;
    const int s_kv = static_cast<int>(pos) + 1;
    const int tiles = (s_kv + a.block_n - 1) / a.block_n;
    const int per = (tiles + a.num_splits - 1) / a.num_splits;
    const int tb = split * per;
    const int te = min(tb + per, tiles);
    const int tok_begin = tb * a.block_n;
    const int tok_end = (tb < te) ? min(te * a.block_n, s_kv) : tok_begin;

    // Q^T as the B operand: lane holds head n, dims 32c + 8*qgrp + [0,8).
    half8_t qop[4];
    {
        const uint16_t* qh = a.q + (static_cast<int64_t>(kvh) * a.group + n) * kHeadDim;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            qop[c] = (n < a.group) ? load_half8(qh + 32 * c + 8 * qgrp) : zero_half8();
    }

    const uint16_t* kh = a.k_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;
    const uint16_t* vh = a.v_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;
    half_t* vl = reinterpret_cast<half_t*>(lds + wave * kDecVWaveBytes);

    float m = kNegBig;
    float l = 0.0f;
    float4_t acc[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[db] = float4_t{0.f, 0.f, 0.f, 0.f};

    // Register prefetch of one sub-tile: K as A operands, V as 8 rows-quartets.
    half8_t kop[2][4], vreg[8];
    auto fetch = [&](int t) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const int tok = t + 16 * mb + n;
            const bool ok = tok < tok_end;
            const uint16_t* kr = kh + static_cast<int64_t>(ok ? tok : tok_begin) * kHeadDim;
#pragma unroll
            for (int c = 0; c < 4; ++c) kop[mb][c] = ok ? load_half8(kr + 32 * c + 8 * qgrp) : zero_half8();
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int tok = t + 4 * i + qgrp;
            const bool ok = tok < tok_end;
            vreg[i] = ok ? load_half8(vh + static_cast<int64_t>(tok) * kHeadDim + 8 * n) : zero_half8();
        }
    };

    int t = tok_begin + kDecSub * wave;
    if (t < tok_end) fetch(t);
    for (; t < tok_end; t += kDecSub * kDecWaves) {
        half8_t kcur[2][4], vcur[8];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int c = 0; c < 4; ++c) kcur[mb][c] = kop[mb][c];
#pragma unroll
        for (int i = 0; i < 8; ++i) vcur[i] = vreg[i];
        const int tn = t + kDecSub * kDecWaves;
        if (tn < tok_end) fetch(tn);

        // S^T[token, head] for 32 tokens: lane holds head n, tokens
        // t + 16*mb + 4*qgrp + r.
        float4_t s[2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            s[mb] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; ++c) s[mb] = mfma16x16x32(kcur[mb][c], qop[c], s[mb]);
        }
        float mx = kNegBig;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = t + 16 * mb + 4 * qgrp + r;
                const float x = (tok < tok_end) ? s[mb][r] * a.scale_log2 : kNegBig;
                s[mb][r] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, swap_halves(mx));
        const float m_new = fmaxf(m, mx);
        const float alpha = exp2f(m - m_new);
        float psum = 0.0f;
        half8_t pop;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = exp2f(s[mb][r] - m_new);
                psum += p;
                pop[4 * mb + r] = static_cast<half_t>(p);
            }
        l = l * alpha + psum;
        m = m_new;
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[db] *= alpha;

        // Park V rows t+4i+qgrp (dims 8n..8n+7) in LDS, read back transposed.
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<half8_t*>(vl + (4 * i + qgrp) * kDecVStride + 8 * n) = vcur[i];
        wave_lds_sync();
        const half_t* vr0 = vl + (4 * qgrp + (n >> 2)) * kDecVStride + 4 * (n & 3);
        const half_t* vr1 = vr0 + 16 * kDecVStride;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const half8_t vop = cat(lds_read_tr16(vr0 + 16 * db), lds_read_tr16(vr1 + 16 * db));
            acc[db] = mfma16x16x32(vop, pop, acc[db]);
        }
        wave_lds_sync();
    }

    // Combine the wavefronts: per head M = max m_w, L = sum l_w 2^(m_w-M),
    // O = sum acc_w 2^(m_w-M) / max(L, 1e-8).
    l += __shfl_xor(l, 16);
    l += swap_halves(l);
    __syncthreads();  // V buffers are reused for the reduction
    float* red = reinterpret_cast<float*>(lds) + wave * (16 * kHeadDim + 32);
    if (qgrp == 0) {
        red[16 * kHeadDim + n] = m;
        red[16 * kHeadDim + 16 + n] = l;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[n * kHeadDim + 16 * db + 4 * qgrp + r] = acc[db][r];
    __syncthreads();

    const int g = threadIdx.x >> 4;        // head handled by this thread
    const int d0 = (threadIdx.x & 15) * 8;  // 8 output dims
    if (g < a.group) {
        const float* base = reinterpret_cast<const float*>(lds);
        const int wstride = 16 * kHeadDim + 32;
        float M = kNegBig;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, base[w * wstride + 16 * kHeadDim + g]);
        float L = 0.0f, f[kDecWaves];
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) {
            f[w] = exp2f(base[w * wstride + 16 * kHeadDim + g] - M);
            L += base[w * wstride + 16 * kHeadDim + 16 + g] * f[w];
        }
        const float l_safe = fmaxf(L, 1.0e-8f);
        half8_t o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float x = 0.0f;
#pragma unroll
            for (int w = 0; w < kDecWaves; ++w) x += base[w * wstride + g * kHeadDim + d0 + e] * f[w];
            o[e] = static_cast<half_t>(x / l_safe);
        }
        const int64_t row = (static_cast<int64_t>(kvh) * a.num_splits + split) * a.group + g;
        store_half8(a.att_partial + row * kHeadDim + d0, o);
        if (d0 == 0) a.lse_partial[row] = M + log2f(l_safe);
    }
}

// One wavefront per (head, kv_head): weights from the split LSEs, then each
// lane accumulates two output dims over the splits.
__global__ __launch_bounds__(kWave) void attn_decode_merge_kernel(
    const uint16_t* __restrict__ att, const float* __restrict__ lse, uint16_t* __restrict__ out,
    int group, int num_splits) {
    const int g = blockIdx.x;
    const int kvh = blockIdx.y;
    const int lane = threadIdx.x;
    const float* L = lse + static_cast<int64_t>(kvh) * num_splits * group;

    float mx = -INFINITY;
    for (int s = lane; s < num_splits; s += kWave) mx = fmaxf(mx, L[s * group + g]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.0f;
    for (int s = lane; s < num_splits; s += kWave) sum += exp2f(L[s * group + g] - mx);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    const float safe = fmaxf(sum, 1.0e-8f);

    float acc0 = 0.0f, acc1 = 0.0f;
    const uint16_t* base = att + (static_cast<int64_t>(kvh) * num_splits * group + g) * kHeadDim + 2 * lane;
    for (int s = 0; s < num_splits; ++s) {
        const float w = exp2f(L[s * group + g] - mx) / safe;
        const uint32_t pair = *reinterpret_cast<const uint32_t*>(base + static_cast<int64_t>(s) * group * kHeadDim);
        const half_t h0 = __builtin_bit_cast(half_t, static_cast<uint16_t>(pair & 0xffffu));
        const half_t h1 = __builtin_bit_cast(half_t, static_cast<uint16_t>(pair >> 16));
        acc0 += static_cast<float>(h0) * w;
        acc1 += static_cast<float>(h1) * w;
    }
    const uint16_t o0 = __builtin_bit_cast(uint16_t, static_cast<half_t>(acc0));
    const uint16_t o1 = __builtin_bit_cast(uint16_t, static_cast<half_t>(acc1));
    *reinterpret_cast<uint32_t*>(out + (static_cast<int64_t>(kvh) * group + g) * kHeadDim + 2 * lane) =
        static_cast<uint32_t>(o0) | (static_cast<uint32_t>(o1) << 16);
}

static float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    uint32_t x;
    if (e == 0x1fu) {
        x = sign | 0x7f800000u | (mant << 13);
    } else if (e != 0) {
        x = sign | ((e + 112u) << 23) | (mant << 13);
    } else if (mant == 0) {
        x = sign;
    } else {
        float f = static_cast<float>(mant) * (1.0f / 16777216.0f);
        __builtin_memcpy(&x, &f, 4);
        x |= sign;
    }
    float f;
    __builtin_memcpy(&f, &x, 4);
    return f;
}

}  // namespace grout

using namespace grout;

extern "C" int32_t grout_attn_decode_split(const uint16_t* q, const uint16_t* k_cache,
                                           const uint16_t* v_cache, uint16_t* att_partial,
                                           float* lse_partial, uint16_t qk_scale_f16,
                                           const uint32_t* d_position, int32_t num_kv_heads,
                                           int32_t group, int32_t head_dim, int32_t max_seq_len,
                                           int32_t block_n, int32_t num_splits,
                                           grout_stream_t stream) {
    GROUT_REQUIRE_PTR(q);
    GROUT_REQUIRE_PTR(k_cache);
    GROUT_REQUIRE_PTR(v_cache);
    GROUT_REQUIRE_PTR(att_partial);
    GROUT_REQUIRE_PTR(lse_partial);
    GROUT_REQUIRE(d_position != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(d_position) & 3u) == 0, GROUT_ERR_ALIGNMENT);
    GROUT_REQUIRE(head_dim == kHeadDim, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(num_kv_heads > 0 && num_kv_heads <= 65535, GROUT_ERR_HEADS);
    GROUT_REQUIRE(group >= 1 && group <= GROUT_MAX_DECODE_GROUP, GROUT_ERR_GROUP);
    GROUT_REQUIRE(max_seq_len > 0, GROUT_ERR_SEQ_RANGE);
    GROUT_REQUIRE(block_n >= 1 && block_n <= 4096, GROUT_ERR_SPLITS);
    GROUT_REQUIRE(num_splits >= 1 && num_splits <= GROUT_MAX_DECODE_SPLITS, GROUT_ERR_SPLITS);
    const float scale = f16_bits_to_f32(qk_scale_f16);
    GROUT_REQUIRE(scale > 0.0f && scale < 65536.0f, GROUT_ERR_ARG);

    DecodeSplitArgs a;
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.att_partial = att_partial;
    a.lse_partial = lse_partial;
    a.d_position = d_position;
    // src/kernels.rs:2618-2622: qk_scale_f32 / ln(2), both f32.
    a.scale_log2 = scale / logf(2.0f);
    a.group = group;
    a.max_seq_len = max_seq_len;
    a.block_n = block_n;
    a.num_splits = num_splits;
    hipLaunchKernelGGL(attn_decode_split_kernel, dim3(num_splits, num_kv_heads), dim3(kDecThreads),
                       0, to_hip(stream), a);
    return launch_status();
}

extern "C" int32_t grout_attn_decode_merge(const uint16_t* att_partial, const float* lse_partial,
                                           uint16_t* out, int32_t num_kv_heads, int32_t group,
                                           int32_t head_dim, int32_t num_splits,
                                           grout_stream_t stream) {
    GROUT_REQUIRE_PTR(att_partial);
    GROUT_REQUIRE_PTR(lse_partial);
    GROUT_REQUIRE_PTR(out);
    GROUT_REQUIRE(head_dim == kHeadDim, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(num_kv_heads > 0 && num_kv_heads <= 65535, GROUT_ERR_HEADS);
    GROUT_REQUIRE(group >= 1 && group <= GROUT_MAX_DECODE_GROUP, GROUT_ERR_GROUP);
    GROUT_REQUIRE(num_splits >= 1 && num_splits <= GROUT_MAX_DECODE_SPLITS, GROUT_ERR_SPLITS);
    hipLaunchKernelGGL(attn_decode_merge_kernel, dim3(group, num_kv_heads), dim3(kWave), 0,
                       to_hip(stream), att_partial, lse_partial, out, group, num_splits);
    return launch_status();
}

extern "C" int64_t grout_attn_decode_partial_bytes(int32_t num_kv_heads, int32_t group,
                                                   int32_t head_dim, int32_t num_splits) {
    if (num_kv_heads <= 0 || group <= 0 || head_dim <= 0 || num_splits <= 0) return GROUT_ERR_ARG;
    return static_cast<int64_t>(num_kv_heads) * num_splits * group * head_dim * 2;
}

extern "C" int64_t grout_attn_decode_lse_bytes(int32_t num_kv_heads, int32_t group,
                                               int32_t num_splits) {
    if (num_kv_heads <= 0 || group <= 0 || num_splits <= 0) return GROUT_ERR_ARG;
    return static_cast<int64_t>(num_kv_heads) * num_splits * group * 4;
}

extern "C" int32_t grout_attn_decode_pick_splits(int32_t cu_count, int32_t num_kv_heads,
                                                 int32_t max_context, int32_t block_n) {
    if (cu_count <= 0) cu_count = 256;
    if (num_kv_heads <= 0 || block_n <= 0 || max_context <= 0) return 1;
    // Two resident workgroups per CU keep ~64 KB of K/V loads in flight per CU;
    // a split shorter than 8 tiles spends more on its prologue and the merge
    // than it saves.
    const int64_t tiles = (static_cast<int64_t>(max_context) + block_n - 1) / block_n;
    int64_t want = (2 * static_cast<int64_t>(cu_count) + num_kv_heads - 1) / num_kv_heads;
    const int64_t cap = (tiles + 7) / 8;
    if (want > cap) want = cap;
    if (want < 1) want = 1;
    if (want > GROUT_MAX_DECODE_SPLITS) want = GROUT_MAX_DECODE_SPLITS;
    return static_cast<int32_t>(want);
}

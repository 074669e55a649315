// Causal GQA flash-attention prefill on CDNA4 MFMA.
//
// Replaces fmha_prefill_causal (src/kernels.rs:1146-1295, grout's default
// prefill), fmha_prefill_gqa (:1322-1495), fmha_prefill_gqa_lpt (:1513-1862)
// and flash_attn_causal_seq_f16 (:1037-1127).  Semantics: query row m at
// position query_start+m attends keys n < min(kv_len, query_start+m+1) of the
// cache head q_head/G; base-2 online softmax with c = qk_scale/ln2:
//   m' = max(m, c*rowmax(s)); p = 2^(c*s - m'); alpha = 2^(m - m');
//   l = l*alpha + sum(p); acc = acc*alpha + f16(p) V; out = f16(acc/max(l,1e-8)).
//
// Shape of the kernel (MI355X-first):
//  * Workgroup = 4 wavefronts, one per SIMD.  A wavefront owns 64 query rows
//    of one query head; the 4 wavefronts of a workgroup are query heads of
//    the same KV head (GQA packing: a K/V tile is fetched once from HBM for
//    G heads), e.g. G=4: 4 heads x the same 64 positions.
//  * K/V tiles of 64 keys are staged in LDS, double buffered: the next
//    tile's global loads are issued before the current tile is computed and
//    land in the other buffer after it; one workgroup barrier per tile.
//  * S^T = K Q^T on v_mfma_f32_32x32x16_f16 (K rows = A operand, 16-byte LDS
//    reads; Q^T = B operand held in registers for the whole loop), so each
//    lane owns one query row and the row softmax needs a single cross-lane
//    step (v_permlane32_swap).
//  * O^T += V^T P^T: P^T comes straight from the S^T accumulators (the
//    reduction slots are ordered to match), V^T from ds_read_b64_tr_b16.
//  * Causal tile skipping per wavefront; masking only on diagonal tiles.
//  * Heavy (late-position) workgroups launch first (longest-processing-time
//    order) and all workgroups of one KV head go to one XCD so its K/V stay
//    in that XCD's L2.
#include <math.h>

#include "abi_util.h"
#include "common.h"

namespace grout {

constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfRows = 64;              // query rows per wavefront
constexpr int kPfBN = 64;                // keys per tile
constexpr int kPfKStride = kHeadDim + 8;   // halves per LDS K row (272 B)
constexpr int kPfVStride = kHeadDim + 16;  // halves per LDS V row (288 B)
constexpr int kPfKTile = kPfBN * kPfKStride;
constexpr int kPfVTile = kPfBN * kPfVStride;
constexpr int kPfStage = kPfKTile + kPfVTile;  // halves per buffer stage
constexpr float kPfNegBig = -1.0e30f;

struct PrefillArgs {
    const uint16_t* q;
    const uint16_t* k_cache;
    const uint16_t* v_cache;
    uint16_t* out;
    float scale_log2;
    int num_q_heads;
    int group;
    int q_len;
    int kv_len;
    int query_start;
    int max_seq_len;
    int n_pos_tiles;       // ceil(q_len / 64)
    int tasks_per_head;    // n_pos_tiles * group wavefront tasks per KV head
    int blocks_per_head;   // ceil(tasks_per_head / 4)
};

__global__ __launch_bounds__(kPfThreads, 1) void attn_prefill_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) half_t pf_lds[2 * kPfStage];

    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int l32 = lane & 31;
    const int hl = lane >> 5;  // which half of the wavefront

    // XCD-aware, longest-first task order.
    const int nb = gridDim.x;
    const int b = blockIdx.x;
    const int T = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    const int kvh = T / a.blocks_per_head;
    const int rblk = T % a.blocks_per_head;
    const int u = rblk * kPfWaves + wave;
    const bool task_ok = u < a.tasks_per_head;
    const int pt = a.n_pos_tiles - 1 - u / a.group;
    const int g = u % a.group;
    const int qh = kvh * a.group + g;
    const int row0 = pt * kPfRows;
    const int pos0 = a.query_start + row0;

    const int pt_max = a.n_pos_tiles - 1 - (rblk * kPfWaves) / a.group;
    const int blk_kv_end = min(a.kv_len, a.query_start + pt_max * kPfRows + kPfRows);
    const int ntiles = (blk_kv_end + kPfBN - 1) / kPfBN;
    const int wave_kv_end = task_ok ? min(a.kv_len, pos0 + kPfRows) : 0;
    const int wave_tiles = (wave_kv_end + kPfBN - 1) / kPfBN;

    // Q^T (B operand): qop[nb][kk] = Q[row0 + 32nb + l32][16kk + 8hl + 0..7].
    half8_t qop[2][8];
#pragma unroll
    for (int nbk = 0; nbk < 2; ++nbk) {
        const int row = row0 + 32 * nbk + l32;
        const bool ok = task_ok && row < a.q_len;
        const uint16_t* qr = a.q + (static_cast<int64_t>(ok ? row : 0) * a.num_q_heads + qh) * kHeadDim;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            qop[nbk][kk] = ok ? load_half8(qr + 16 * kk + 8 * hl) : half8_t{};
    }

    const uint16_t* kh = a.k_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;
    const uint16_t* vh = a.v_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;

    // Cooperative tile load: 1024 16-byte chunks of K and of V per tile;
    // thread tid moves chunks tid + 256*i (row = chunk/16, col8 = chunk%16).
    uint4_t kst[4], vst[4];
    auto gload = [&](int tile) {
        const int n0 = tile * kPfBN;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + kPfThreads * i;
            const int row = c >> 4, col = (c & 15) * 8;
            const int n = n0 + row;
            const bool ok = n < blk_kv_end;
            kst[i] = ok ? load_u128(kh + static_cast<int64_t>(n) * kHeadDim + col) : uint4_t{0, 0, 0, 0};
            vst[i] = ok ? load_u128(vh + static_cast<int64_t>(n) * kHeadDim + col) : uint4_t{0, 0, 0, 0};
        }
    };
    auto lstore = [&](int buf) {
        half_t* ks = pf_lds + buf * kPfStage;
        half_t* vs = ks + kPfKTile;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + kPfThreads * i;
            const int row = c >> 4, col = (c & 15) * 8;
            store_u128(ks + row * kPfKStride + col, kst[i]);
            store_u128(vs + row * kPfVStride + col, vst[i]);
        }
    };

    float16_t o[4][2];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int nbk = 0; nbk < 2; ++nbk)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][nbk][r] = 0.0f;
    float m_run[2] = {kPfNegBig, kPfNegBig};
    float l_run[2] = {0.0f, 0.0f};
    const float c = a.scale_log2;

    if (ntiles > 0) {
        gload(0);
        lstore(0);
    }
    __syncthreads();

    for (int j = 0; j < ntiles; ++j) {
        const int buf = j & 1;
        if (j + 1 < ntiles) gload(j + 1);

        if (j < wave_tiles) {
            const half_t* ks = pf_lds + buf * kPfStage;
            const half_t* vs = ks + kPfKTile;
            const int n0 = j * kPfBN;

            // S^T[mb][nb]: rows = keys n0 + 32mb + 8(r/4) + 4hl + r%4, col = query row.
            float16_t s[2][2];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int nbk = 0; nbk < 2; ++nbk)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[mb][nbk][r] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    const half8_t ka = *reinterpret_cast<const half8_t*>(
                        ks + (32 * mb + l32) * kPfKStride + 16 * kk + 8 * hl);
#pragma unroll
                    for (int nbk = 0; nbk < 2; ++nbk) s[mb][nbk] = mfma32x32x16(ka, qop[nbk][kk], s[mb][nbk]);
                }
            }

            const bool need_mask = (n0 + kPfBN - 1 > pos0) || (n0 + kPfBN > a.kv_len);
            half8_t pop[4][2];
#pragma unroll
            for (int nbk = 0; nbk < 2; ++nbk) {
                const int qpos = pos0 + 32 * nbk + l32;
                float mx = kPfNegBig;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float x = s[mb][nbk][r];
                        if (need_mask) {
                            const int n = n0 + 32 * mb + 8 * (r >> 2) + 4 * hl + (r & 3);
                            if (n > qpos || n >= a.kv_len) x = kPfNegBig;
                            s[mb][nbk][r] = x;
                        }
                        mx = fmaxf(mx, x);
                    }
                mx = fmaxf(mx, swap_halves(mx));
                const float m_new = fmaxf(m_run[nbk], mx * c);
                const float alpha = exp2f(m_run[nbk] - m_new);
                float psum = 0.0f;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float p = exp2f(fmaf(s[mb][nbk][r], c, -m_new));
                        psum += p;
                        pop[2 * mb + (r >> 3)][nbk][r & 7] = static_cast<half_t>(p);
                    }
                l_run[nbk] = l_run[nbk] * alpha + psum;
                m_run[nbk] = m_new;
#pragma unroll
                for (int db = 0; db < 4; ++db) o[db][nbk] *= alpha;
            }

            // O^T[db][nb] += V^T[32 dims, 16 keys] P^T[16 keys, 32 rows] for 4 key steps.
            // 16-lane group gi: dims 32db + 16(gi&1) + i, key half hl = gi>>1.
            const int gi = lane >> 4, ii = lane & 15;
            const half_t* vb = vs + (4 * (gi >> 1) + (ii >> 2)) * kPfVStride + 16 * (gi & 1) + 4 * (ii & 3);
#pragma unroll
            for (int ks2 = 0; ks2 < 4; ++ks2) {
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const half_t* p0 = vb + (16 * ks2) * kPfVStride + 32 * db;
                    const half8_t va = cat(lds_read_tr16(p0), lds_read_tr16(p0 + 8 * kPfVStride));
#pragma unroll
                    for (int nbk = 0; nbk < 2; ++nbk) o[db][nbk] = mfma32x32x16(va, pop[ks2][nbk], o[db][nbk]);
                }
            }
        }

        if (j + 1 < ntiles) lstore(buf ^ 1);
        __syncthreads();
    }

    if (!task_ok) return;
    // out[row][d] with d = 32db + 8(r/4) + 4hl + r%4.
#pragma unroll
    for (int nbk = 0; nbk < 2; ++nbk) {
        const int row = row0 + 32 * nbk + l32;
        const float lt = l_run[nbk] + swap_halves(l_run[nbk]);
        const float l_safe = fmaxf(lt, 1.0e-8f);
        if (row < a.q_len) {
            uint16_t* orow = a.out + (static_cast<int64_t>(row) * a.num_q_heads + qh) * kHeadDim;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    half4_t h;
#pragma unroll
                    for (int e = 0; e < 4; ++e) h[e] = static_cast<half_t>(o[db][nbk][4 * i + e] / l_safe);
                    *reinterpret_cast<half4_t*>(orow + 32 * db + 8 * i + 4 * hl) = h;
                }
        }
    }
}

}  // namespace grout

using namespace grout;

extern "C" int32_t grout_attn_prefill(const uint16_t* q, const uint16_t* k_cache,
                                      const uint16_t* v_cache, uint16_t* out, float qk_scale,
                                      int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                      int32_t q_len, int32_t kv_len, int32_t query_start,
                                      int32_t max_seq_len, grout_stream_t stream) {
    // Mirrors the ensure!s of attend_seq_arc_into_ctx_with_position
    // (src/model.rs:5564-5637) on sizes.
    GROUT_REQUIRE_PTR(q);
    GROUT_REQUIRE_PTR(k_cache);
    GROUT_REQUIRE_PTR(v_cache);
    GROUT_REQUIRE_PTR(out);
    GROUT_REQUIRE(head_dim == kHeadDim, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
                  GROUT_ERR_HEADS);
    GROUT_REQUIRE(max_seq_len > 0, GROUT_ERR_SEQ_RANGE);
    GROUT_REQUIRE(q_len >= 0 && query_start >= 0, GROUT_ERR_KV_LEN);
    GROUT_REQUIRE(kv_len >= 1 && kv_len <= max_seq_len, GROUT_ERR_KV_LEN);
    GROUT_REQUIRE(qk_scale > 0.0f && qk_scale < 1.0e30f, GROUT_ERR_ARG);
    if (q_len == 0) return GROUT_OK;

    PrefillArgs a;
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.out = out;
    // src/kernels.rs:1170-1174: qk_scale / ln(2) in f32.
    a.scale_log2 = qk_scale / logf(2.0f);
    a.num_q_heads = num_q_heads;
    a.group = num_q_heads / num_kv_heads;
    a.q_len = q_len;
    a.kv_len = kv_len;
    a.query_start = query_start;
    a.max_seq_len = max_seq_len;
    a.n_pos_tiles = (q_len + kPfRows - 1) / kPfRows;
    a.tasks_per_head = a.n_pos_tiles * a.group;
    a.blocks_per_head = (a.tasks_per_head + kPfWaves - 1) / kPfWaves;
    const int64_t blocks = static_cast<int64_t>(a.blocks_per_head) * num_kv_heads;
    GROUT_REQUIRE(blocks <= 0x7fffffff, GROUT_ERR_KV_LEN);
    hipLaunchKernelGGL(attn_prefill_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kPfThreads),
                       0, to_hip(stream), a);
    return launch_status();
}

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
//  * Workgroup = 8 wavefronts, two per SIMD.  A wavefront owns 32 query rows
//    of one query head; the 8 wavefront tasks of a workgroup belong to the
//    same KV head (GQA packing: a K/V tile is fetched once from HBM for all
//    of them), e.g. G=4: 4 heads x the same 64 positions.
//  * K/V tiles of 64 keys go straight from HBM into LDS (direct-to-LDS DMA,
//    no register staging) through a 3-stage ring: tile j+2 is issued right
//    after the barrier that opens tile j; one workgroup barrier per tile.
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

constexpr int kPfBN = 64;     // keys per tile
// LDS tile layout: key row n of a tile sits in 1 KB block n%16 at row n/16
// (256 B rows inside a block); blocks are 1040 B (K) / 1056 B (V) apart.
// One direct-to-LDS copy fills one block (rows b, b+16, b+32, b+48), the
// MFMA operand reads (8 or 16 consecutive keys, or 4 keys x 32 B for the
// transposing V reads) hit distinct banks, and every read address is a
// per-lane base plus an immediate offset.
constexpr int kPfKBlock = 1040;
constexpr int kPfVBlock = 1056;
constexpr int kPfKBytes = 16 * kPfKBlock;
constexpr int kPfVBytes = 16 * kPfVBlock;
constexpr int kPfStageBytes = kPfKBytes + kPfVBytes;
constexpr int kPfStages = 3;
constexpr float kPfNegBig = -1.0e30f;
// Lazy rescale: the running max used for p = 2^(c*s - m) is only raised when
// a row's max grows by more than this (log2 units), so p <= 2^8 and O is
// rescaled on few tiles.  The normalised result is the same function.
constexpr float kPfRescaleSlack = 8.0f;

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
    int n_pos_tiles;       // ceil(q_len / rows per wavefront)
    int tasks_per_head;    // n_pos_tiles * group wavefront tasks per KV head
    int blocks_per_head;   // ceil(tasks_per_head / waves per workgroup)
};

// Asynchronous 16-byte HBM -> LDS copy (global_load_lds_dwordx4, scalar base
// + 32-bit per-lane byte offset): lane l's 16 bytes land at LDS byte
// lds_base + 16*l (lds_base wave-uniform).  Issued through inline asm so the
// compiler does not serialise consecutive copies behind vmcnt(0) waits; the
// kernel waits for them itself with s_waitcnt vmcnt before its workgroup
// barrier.  M0 carries the LDS base (this kernel keeps nothing else in M0);
// one wait state separates the M0 write from the copy.
__device__ __forceinline__ void lds_dma16(const void* gbase, uint32_t voff, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff), "s"(gbase), "s"(lds_base)
        : "memory");
}

// s_waitcnt immediate for "at most n vector-memory ops outstanding" (gfx9
// encoding: vmcnt bits [3:0]+[15:14]; expcnt [6:4] and lgkmcnt [11:8] at their
// maximum, i.e. not waited on).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

// NBK: 32-row query blocks per wavefront (rows = 32*NBK); WAVES: wavefronts
// per workgroup (all on query heads of one KV head).
template <int NBK, int WAVES>
__global__ __launch_bounds__(WAVES * kWave, 1) void attn_prefill_kernel(PrefillArgs a) {
    constexpr int kRows = 32 * NBK;
    constexpr int kDmaPerWave = 16 / WAVES;  // K blocks (and V blocks) per wavefront
    __shared__ __attribute__((aligned(1024))) unsigned char pf_lds[kPfStages * kPfStageBytes];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int l32 = lane & 31;
    const int hl = lane >> 5;  // which half of the wavefront

    // XCD-aware, longest-first task order: consecutive workgroup ids go to
    // different XCDs, so T groups all workgroups of a KV head on one XCD, and
    // within a head the latest (heaviest) position tiles come first.
    const int nb = gridDim.x;
    const int b = blockIdx.x;
    const int T = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    const int kvh = T / a.blocks_per_head;
    const int rblk = T % a.blocks_per_head;
    const int u = rblk * WAVES + wave;
    const bool task_ok = u < a.tasks_per_head;
    const int pt = a.n_pos_tiles - 1 - u / a.group;
    const int g = u % a.group;
    const int qh = kvh * a.group + g;
    const int row0 = pt * kRows;
    const int pos0 = a.query_start + row0;

    const int pt_max = a.n_pos_tiles - 1 - (rblk * WAVES) / a.group;
    const int blk_kv_end = min(a.kv_len, a.query_start + pt_max * kRows + kRows);
    const int ntiles = (blk_kv_end + kPfBN - 1) / kPfBN;
    const int wave_kv_end = task_ok ? min(a.kv_len, pos0 + kRows) : 0;
    const int wave_tiles = (wave_kv_end + kPfBN - 1) / kPfBN;

    const uint16_t* kh = a.k_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;
    const uint16_t* vh = a.v_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;

    // HBM -> LDS copy of tile `tile` into stage `st`: this wavefront fills K
    // and V blocks wave*kDmaPerWave + r; lane l moves row b + 16*(l/16), 16-byte
    // column l%16.  On the block's last tile rows at or past blk_kv_end are
    // clamped to the last valid row (they are masked in the softmax).
    const uint32_t lds0 = static_cast<uint32_t>(
        (uintptr_t)((__attribute__((address_space(3))) unsigned char*)(pf_lds)));
    const uint32_t lane_off = 4096u * static_cast<uint32_t>(lane >> 4) + 16u * (lane & 15);
    auto issue_tile = [&](int tile, int st) {
        const uint32_t kb = lds0 + st * kPfStageBytes;
        const uint32_t vb = kb + kPfKBytes;
        const int n0 = tile * kPfBN;
        const bool clamp = n0 + kPfBN > blk_kv_end;
#pragma unroll
        for (int r = 0; r < kDmaPerWave; ++r) {
            const int blk = wave * kDmaPerWave + r;
            int64_t row_base = static_cast<int64_t>(n0 + blk) * kHeadDim;
            uint32_t off = lane_off;
            if (clamp) {
                // Address from the tile start: n0 <= blk_kv_end - 1, so every
                // clamped row is >= n0 and the unsigned offset stays in range.
                const int row = min(n0 + blk + 16 * (lane >> 4), blk_kv_end - 1);
                row_base = static_cast<int64_t>(n0) * kHeadDim;
                off = static_cast<uint32_t>(row - n0) * 256u + 16u * (lane & 15);
            }
            lds_dma16(kh + row_base, off, kb + kPfKBlock * blk);
            lds_dma16(vh + row_base, off, vb + kPfVBlock * blk);
        }
    };

    if (ntiles > 0) issue_tile(0, 0);
    if (ntiles > 1) issue_tile(1, 1);

    // Q^T (B operand): qop[nb][kk] = Q[row0 + 32nb + l32][16kk + 8hl + 0..7].
    half8_t qop[NBK][8];
#pragma unroll
    for (int nbk = 0; nbk < NBK; ++nbk) {
        const int row = row0 + 32 * nbk + l32;
        const bool ok = task_ok && row < a.q_len;
        const uint16_t* qr = a.q + (static_cast<int64_t>(ok ? row : 0) * a.num_q_heads + qh) * kHeadDim;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) qop[nbk][kk] = load_half8(qr + 16 * kk + 8 * hl);
        if (!ok) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) qop[nbk][kk] = half8_t{};
        }
    }

    float16_t o[4][NBK];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int nbk = 0; nbk < NBK; ++nbk)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][nbk][r] = 0.0f;
    float m_run[NBK], l_run[NBK];
#pragma unroll
    for (int nbk = 0; nbk < NBK; ++nbk) {
        m_run[nbk] = kPfNegBig;
        l_run[nbk] = 0.0f;
    }
    const float c = a.scale_log2;

    // Per-lane LDS read offsets.  K (A operand of S^T = K Q^T): key 32mb + l32,
    // dims 16kk + 8hl.  V^T (A operand of O^T += V^T P^T) via the transposing
    // read: 16-lane group gi = lane/16 covers dims 32db + 16(gi&1) + [0,16) and
    // keys 16ks + 4(gi>>1) + [0,4) (+8 for reduction slots 4..7).
    const int gi = lane >> 4, ii = lane & 15;
    const uint32_t k_lane = (l32 & 15) * kPfKBlock + (l32 >> 4) * 256 + 16 * hl;
    const uint32_t v_lane = (4 * (gi >> 1) + (ii >> 2)) * kPfVBlock + 32 * (gi & 1) + 8 * (ii & 3);

    for (int j = 0; j < ntiles; ++j) {
        const int st = j % kPfStages;
        // Tile j is in LDS for this wavefront once at most the copies of tile
        // j+1 (issued last iteration; vector-memory loads retire in order) are
        // outstanding.
        if (j + 1 < ntiles) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kDmaPerWave));
        } else {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        }
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // Every wavefront is past tile j-1, so its stage can be refilled.
        if (j + 2 < ntiles) issue_tile(j + 2, (j + 2) % kPfStages);

        if (j < wave_tiles) {
            const unsigned char* kb = pf_lds + st * kPfStageBytes;
            const unsigned char* vb = kb + kPfKBytes;
            const int n0 = j * kPfBN;

            // S^T[mb][nb]: rows = keys n0 + 32mb + 8(r/4) + 4hl + r%4, col = query row.
            float16_t s[2][NBK];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int nbk = 0; nbk < NBK; ++nbk)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[mb][nbk][r] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    const half8_t ka = *reinterpret_cast<const half8_t*>(kb + k_lane + 512 * mb + 32 * kk);
#pragma unroll
                    for (int nbk = 0; nbk < NBK; ++nbk) s[mb][nbk] = mfma32x32x16(ka, qop[nbk][kk], s[mb][nbk]);
                }
            }

            const bool need_mask = (n0 + kPfBN - 1 > pos0) || (n0 + kPfBN > a.kv_len);
            half8_t pop[4][NBK];
#pragma unroll
            for (int nbk = 0; nbk < NBK; ++nbk) {
                if (need_mask) {
                    const int qpos = pos0 + 32 * nbk + l32;
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int n = n0 + 32 * mb + 8 * (r >> 2) + 4 * hl + (r & 3);
                            if (n > qpos || n >= a.kv_len) s[mb][nbk][r] = kPfNegBig;
                        }
                }
                float mx = kPfNegBig;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[mb][nbk][r]);
                mx = fmaxf(mx, swap_halves(mx));
                const float m_cand = mx * c;
                if (__any(m_cand > m_run[nbk] + kPfRescaleSlack)) {
                    const float m_new = fmaxf(m_run[nbk], m_cand);
                    const float alpha = __builtin_amdgcn_exp2f(m_run[nbk] - m_new);
                    l_run[nbk] *= alpha;
#pragma unroll
                    for (int db = 0; db < 4; ++db) o[db][nbk] *= alpha;
                    m_run[nbk] = m_new;
                }
                const float m_use = m_run[nbk];
                float psum = 0.0f;
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float p = __builtin_amdgcn_exp2f(fmaf(s[mb][nbk][r], c, -m_use));
                        psum += p;
                        pop[2 * mb + (r >> 3)][nbk][r & 7] = static_cast<half_t>(p);
                    }
                l_run[nbk] += psum;
            }

            // O^T[db][nb] += V^T[32 dims, 16 keys] P^T[16 keys, 32 rows], 4 key steps.
#pragma unroll
            for (int ks2 = 0; ks2 < 4; ++ks2) {
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const unsigned char* p0 = vb + v_lane + 256 * ks2 + 64 * db;
                    const half8_t va = cat(lds_read_tr16(reinterpret_cast<const half_t*>(p0)),
                                           lds_read_tr16(reinterpret_cast<const half_t*>(p0 + 8 * kPfVBlock)));
#pragma unroll
                    for (int nbk = 0; nbk < NBK; ++nbk) o[db][nbk] = mfma32x32x16(va, pop[ks2][nbk], o[db][nbk]);
                }
            }
        }
    }

    if (!task_ok) return;
    // out[row][d] with d = 32db + 8(r/4) + 4hl + r%4.
#pragma unroll
    for (int nbk = 0; nbk < NBK; ++nbk) {
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

template <int NBK, int WAVES>
static int32_t launch_prefill(PrefillArgs a, int num_kv_heads, hipStream_t stream) {
    constexpr int kRows = 32 * NBK;
    a.n_pos_tiles = (a.q_len + kRows - 1) / kRows;
    a.tasks_per_head = a.n_pos_tiles * a.group;
    a.blocks_per_head = (a.tasks_per_head + WAVES - 1) / WAVES;
    const int64_t blocks = static_cast<int64_t>(a.blocks_per_head) * num_kv_heads;
    if (blocks > 0x7fffffff) return GROUT_ERR_KV_LEN;
    hipLaunchKernelGGL((attn_prefill_kernel<NBK, WAVES>), dim3(static_cast<unsigned>(blocks)),
                       dim3(WAVES * kWave), 0, stream, a);
    return launch_status();
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
    // 8 wavefronts x 32 query rows: two wavefronts per SIMD, so one's softmax
    // (VALU, v_exp_f32) overlaps the other's MFMAs; LDS reads stay below the
    // measured ~125-160 B/clk/CU.
    return launch_prefill<1, 8>(a, num_kv_heads, to_hip(stream));
}

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
//  * Ping-pong: waves 0-3 and 4-7 run the same per-tile program one phase
//    apart.  A tile is a GEMM phase (PV of the previous tile + S of this
//    tile, 32 MFMAs) and a softmax phase (VALU, v_exp_f32); each tile starts
//    with the two groups in opposite phases, so one wave of a SIMD feeds the
//    matrix core (at raised issue priority) while the other does its softmax.
//    One workgroup barrier per tile guards the stage ring.
//  * K/V tiles of 64 keys go straight from HBM into LDS (direct-to-LDS DMA,
//    no register staging) through a 4-stage ring; tile t+2 is issued in
//    tile step t, at the start of each wavefront's softmax phase.
//  * S^T = K Q^T on v_mfma_f32_32x32x16_f16 (K rows = A operand, 16-byte LDS
//    reads; Q^T = B operand held in registers for the whole loop), so each
//    lane owns one query row and the row softmax needs a single cross-lane
//    step (v_permlane32_swap).
//  * O^T += V^T P^T: P^T comes straight from the S^T accumulators (the
//    reduction slots are ordered to match), V^T from ds_read_b64_tr_b16.
//    LDS operands are read a few MFMAs ahead into a register ring.
//  * The running max is raised only when P would leave f16 range, so most
//    tiles need no row max and no rescale.
//  * Causal tile skipping per wavefront; masking only on diagonal tiles.
//  * Heavy (late-position) workgroups launch first (longest-processing-time
//    order) and all workgroups of one KV head go to one XCD so its K/V stay
//    in that XCD's L2.
//  * Small launches (row blocks of at most 8 key tiles, one workgroup per
//    query head and row block within the CU count) take a short form: the 8
//    wavefronts of a workgroup take one key tile each and merge in LDS.
#include <math.h>

#include <type_traits>

#include "abi_util.h"
#include "common.h"

namespace grout {

constexpr int kPfBN = 64;     // keys per tile
// LDS tile layout: key row n of a tile sits in 1 KB block n%16 at row n/16
// (256 B rows inside a block); blocks are 1040 B (K) / 1088 B (V) apart.
// One direct-to-LDS copy fills one block (rows b, b+16, b+32, b+48), the
// MFMA operand reads (8 or 16 consecutive keys, or 4 keys x 32 B for the
// transposing V reads) hit distinct banks, and every read address is a
// per-lane base plus an immediate offset.
constexpr int kPfKBlock = 1040;
constexpr int kPfVBlock = 1088;
constexpr int kPfKBytes = 16 * kPfKBlock;
constexpr int kPfVBytes = 16 * kPfVBlock;
constexpr int kPfStageBytes = kPfKBytes + kPfVBytes;
constexpr int kPfStages = 4;
constexpr int kPfOutBytes = 32 * 256;  // one wavefront's f16 output tile
static_assert(4 * kPfOutBytes <= kPfStageBytes, "a stage holds the output tiles of 4 wavefronts");
constexpr float kPfNegBig = -1.0e30f;
// Lazy rescale: the running max used for p = 2^(c*s - m) is only raised when
// some p of a tile would reach this bound (f16 holds up to 65504), so O is
// rescaled on few tiles and no per-tile row max is needed otherwise.
constexpr float kPfPsumLimit = 32768.0f;
// LDS operand read-ahead of the GEMM phase, in MFMAs.
constexpr int kPfAhead = 4;

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
    int n_pos_tiles;       // ceil(q_len / rows per wavefront) (split: padded to whole q blocks)
    int tasks_per_head;    // n_pos_tiles * group wavefront tasks per KV head
    int blocks_per_head;   // ceil(tasks_per_head / waves per workgroup)
    // Split-K form only (fmha_prefill_gqa_lpt_split's generics and scratch).
    uint16_t* att_partial;  // [tiles, num_splits*block_m*split_group, 128]
    float* lse_partial;     // [tiles, num_splits*block_m*split_group]
    int block_m;            // BM: query rows per q block (a multiple of 32)
    int block_n;            // BN: keys per split-range tile
    int split_group;        // GROUP: q heads per logical tile
    int num_splits;
    // Dynamic schedule only (kDyn): claim counters (kPfQueues XCD queues, the
    // shared pool, the exit counter; kPfSchedStride u32 apart, zero on entry
    // and exit), the number of persistent workgroups, the KV-head count and
    // the first block (per head) that goes to the shared pool.
    uint32_t* sched;
    int n_wg;
    int num_kv_heads;
    int pool_block0;
};

// Dynamic schedule.  A task is a workgroup-sized unit (one block of the static
// grid).  The KV heads h = q (mod kPfQueues) belong to XCD q: their blocks
// [0, pool_block0) form its heavy queue and the lighter blocks
// [pool_block0, blocks_per_head) its light queue, each heaviest first with the
// heads interleaved.  A persistent workgroup claims from the heavy queue of
// the XCD it runs on (a head's K/V stay in that XCD's L2), then from the
// fullest other heavy queue, then from its own light queue while that holds
// at least half as many tasks as the fullest light queue, else from the
// fullest: XCDs that run faster take over the slower ones' heavy blocks, the
// last tasks anywhere are light ones, and most light tasks still run where
// their head's K/V are cached.
constexpr int kPfQueues = 8;
constexpr int kPfLight = kPfQueues;             // counter index of light queue q: kPfLight + q
constexpr int kPfExit = 2 * kPfQueues;          // counter index of the exit counter
constexpr int kPfSchedCounters = 2 * kPfQueues + 1;
constexpr int kPfSchedStride = 64;  // u32: one 256-byte line per counter
constexpr int kPfClaimAttempts = 64;

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

// f16(f32(o / l)) for f32 o and l > 0, with rl = 1/l rounded to f64: the f64
// product o*rl is within 2^-52 (relative) of o/l, while a quotient of two f32
// values in the f32 normal range is never an f32 rounding midpoint and lies
// more than 2^-49 (relative) from every one; so the product rounds to the same
// f32 as the correctly rounded division.  Quotients below 2^-126 give +-0 in
// f16 either way.  About 4 instructions against the ~10 of an f32 division.
__device__ __forceinline__ half_t div_to_half(float o, double rl) {
    float f = static_cast<float>(static_cast<double>(o) * rl);
    // Keeps the two roundings: the code generator otherwise folds
    // f64 -> f32 -> f16 into a single f64 -> f16 rounding, another function.
    asm("" : "+v"(f));
    return static_cast<half_t>(f);
}

// s_waitcnt immediate for "at most n vector-memory ops outstanding" (gfx9
// encoding: vmcnt bits [3:0]+[15:14]; expcnt [6:4] and lgkmcnt [11:8] at their
// maximum, i.e. not waited on).
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

// Workgroup barrier that also orders LDS: this wavefront's LDS reads have
// completed (a stage may be refilled right after the barrier) and the
// compiler moves no memory access across it.
__device__ __forceinline__ void pf_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Workgroup: 8 wavefronts x 32 query rows, all on query heads of one KV head.
// Waves 0-3 (group A, one per SIMD) and 4-7 (group B) run the same per-tile
// program one phase apart ("ping-pong"): a tile is two phases, GEMM (PV of the
// previous tile + S of this tile, 32 MFMAs) and softmax (VALU + v_exp_f32).
// After each tile's barrier group A starts with its GEMM phase and group B
// with its softmax, so each SIMD has one wavefront feeding the matrix core
// while the other does its softmax.  Between the phases there is no barrier:
// a second one per tile, to hold the groups in step, measured 0.5% slower.
constexpr int kPfWaves = 8;
constexpr int kPfRows = 32;

// kSplit: the split-K form (fmha_prefill_gqa_lpt_split, src/kernels.rs:1872-2142).
// Workgroup (task, blockIdx.y = split); every wavefront restricts its keys to
// its split's range, computed from the reference's q block of its rows
// (block_m is a multiple of 32, so a wavefront's rows lie in one block), and
// stores a normalised partial and its log2 LSE instead of the output.
// kDyn: persistent workgroups that claim tasks from the per-XCD queues above
// instead of taking one task from blockIdx; each task runs exactly as in the
// static grid, so the output is bit-identical.
// kWaves = 4: group A alone (one wavefront per SIMD, no ping-pong partner), for
// grids too small to fill the GPU: a tile step then takes one GEMM phase and
// one softmax phase of one wavefront instead of two of each, which shortens
// the latency of the heaviest workgroup.  Every wavefront computes exactly what
// it computes in the 8-wavefront workgroup, so the output is bit-identical.
template <bool kSplit, bool kDyn, int kWaves = kPfWaves>
__global__ __launch_bounds__(kWaves * kWave, 1) void attn_prefill_kernel(PrefillArgs a) {
    static_assert(!(kSplit && kDyn), "the split-K form keeps the static grid");
    static_assert(kWaves == kPfWaves || (kWaves == 4 && !kSplit && !kDyn),
                  "the 4-wavefront form is the plain static grid only");
    constexpr int kDmaPerWave = 16 / kWaves;  // K blocks (and V blocks) per wavefront
    __shared__ __attribute__((aligned(1024))) unsigned char pf_lds[kPfStages * kPfStageBytes];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int grp = wave >> 2;  // 0: group A, 1: group B (one phase behind)
    const int lane = tid % kWave;
    const int l32 = lane & 31;
    const int hl = lane >> 5;  // which half of the wavefront

    // XCD-aware, longest-first task order: consecutive workgroup ids go to
    // different XCDs, so T groups all workgroups of a KV head on one XCD, and
    // within a head the latest (heaviest) position tiles come first.  With
    // fewer than 8 KV heads a head spans hx = 8/Hkv XCDs, which take its blocks
    // in turn (block i*hx + j on the head's j-th XCD): each XCD then gets the
    // same mix of heavy and light blocks, not a contiguous (heavy or light) run.
    const int nb = gridDim.x;
    const int b = blockIdx.x;
    int T = b;
    if (nb % 8 == 0) {
        const int hkv = nb / a.blocks_per_head;
        const int x = b % 8, i = b / 8;
        if (hkv < 8 && 8 % hkv == 0) {
            const int hx = 8 / hkv;
            T = (x / hx) * a.blocks_per_head + i * hx + x % hx;
        } else {
            T = x * (nb / 8) + i;
        }
    }

    // Dynamic schedule state (wave 0 claims; the task goes to all waves
    // through LDS).  The claim on the own queue is issued one task ahead, after
    // the previous task's loop, so its round trip overlaps that epilogue.
    __shared__ int s_task;
    int my_q = 0, nhq_own = 0, nq_own = 0;
    bool own_live = false;
    uint32_t pre_j = 0xffffffffu;  // prefetched own-queue ticket (wave 0, lane 0)
    int pre_ticket = -1;           // the same, read back (wave 0, uniform); -1: none
    if constexpr (kDyn) {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        my_q = static_cast<int>(xcc % kPfQueues);
        nhq_own = a.num_kv_heads > my_q ? (a.num_kv_heads - my_q + kPfQueues - 1) / kPfQueues : 0;
        nq_own = nhq_own * a.pool_block0;
        own_live = nq_own > 0;
        if (wave == 0 && lane == 0 && own_live)
            pre_j = __hip_atomic_fetch_add(a.sched + my_q * kPfSchedStride, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
        if (wave == 0 && own_live) pre_ticket = static_cast<int>(__shfl(pre_j, 0));
    }
    // Task j of heavy queue q: KV head q + kPfQueues*(j % nhq), block j / nhq;
    // of light queue q: the same head, block pool_block0 + j / nhq.
    auto queue_task = [&](int q, int nhq, int j) {
        return (q + kPfQueues * (j % nhq)) * a.blocks_per_head + j / nhq;
    };
    const int light_blocks = a.blocks_per_head - a.pool_block0;

    for (;;) {
    if constexpr (kDyn) {
        if (wave == 0) {
            int task = -1;
            const int j0 = pre_ticket;
            if (own_live && j0 >= 0 && j0 < nq_own) {
                // nhq_own passes through an empty asm so that the division's
                // constants are derived here, not held across the task loop.
                int nhq = nhq_own;
                asm volatile("" : "+s"(nhq));
                task = queue_task(my_q, nhq, j0);
            } else {
                own_live = false;
            }
            // Own heavy queue empty: claim from the fullest other heavy queue,
            // else from the own light queue if it holds at least half as many
            // tasks as the fullest light queue, else from the fullest; leave
            // once all are empty.  Lane i < 2*kPfQueues reads counter i.
            for (int attempt = 0; attempt < kPfClaimAttempts && task < 0; ++attempt) {
                int rem = 0;
                if (lane < 2 * kPfQueues) {
                    const int q = lane % kPfQueues;
                    const int nhq = a.num_kv_heads > q ? (a.num_kv_heads - q + kPfQueues - 1) / kPfQueues : 0;
                    const uint32_t nq = static_cast<uint32_t>(nhq * (lane < kPfQueues ? a.pool_block0 : light_blocks));
                    const uint32_t c = __hip_atomic_load(a.sched + lane * kPfSchedStride, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                    rem = static_cast<int>(nq - min(c, nq));
                }
                int best = -1, best_rem = 0;
#pragma unroll
                for (int q = 0; q < kPfQueues; ++q) {
                    const int r = __shfl(rem, q);
                    if (r > best_rem) {
                        best_rem = r;
                        best = q;
                    }
                }
                if (best < 0) {
#pragma unroll
                    for (int q = 0; q < kPfQueues; ++q) {
                        const int r = __shfl(rem, kPfLight + q);
                        if (r > best_rem) {
                            best_rem = r;
                            best = kPfLight + q;
                        }
                    }
                    const int own_rem = __shfl(rem, kPfLight + my_q);
                    if (own_rem > 0 && (own_rem << 1) >= best_rem) best = kPfLight + my_q;
                }
                if (best < 0) break;
                uint32_t j = 0;
                if (lane == 0)
                    j = __hip_atomic_fetch_add(a.sched + best * kPfSchedStride, 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                j = __shfl(j, 0);
                const int q = best % kPfQueues;
                const int nhq = (a.num_kv_heads - q + kPfQueues - 1) / kPfQueues;
                if (best < kPfQueues) {
                    if (j < static_cast<uint32_t>(nhq * a.pool_block0)) task = queue_task(q, nhq, static_cast<int>(j));
                } else if (j < static_cast<uint32_t>(nhq * light_blocks)) {
                    task = queue_task(q, nhq, static_cast<int>(j)) + a.pool_block0;
                }
            }
            if (lane == 0) s_task = task;
        }
        pf_barrier();  // also: every wavefront is past the previous task's LDS reads
        T = s_task;
        if (T < 0) break;
    }
    const int kvh = T / a.blocks_per_head;
    const int rblk = T % a.blocks_per_head;
    const int u = rblk * kWaves + wave;
    const bool task_ok = u < a.tasks_per_head;
    const int pt = a.n_pos_tiles - 1 - u / a.group;
    const int g = u % a.group;
    const int qh = kvh * a.group + g;
    const int row0 = pt * kPfRows;
    const int pos0 = a.query_start + row0;

    const int pt_max = a.n_pos_tiles - 1 - (rblk * kWaves) / a.group;
    const int blk_kv_end = min(a.kv_len, a.query_start + pt_max * kPfRows + kPfRows);
    int wave_kv_end = task_ok ? min(a.kv_len, pos0 + kPfRows) : 0;
    // Key range [lo, hi) of this wavefront (all keys unless split) and the
    // workgroup's range of 64-key tiles [tile0, tile0 + ntiles).
    int key_lo = 0, key_hi = a.kv_len, tile0 = 0, blk_end = blk_kv_end;
    if constexpr (kSplit) {
        // src/kernels.rs:2036-2043 for q block bq: tc = ceil(min(m_end, kv_len)/BN),
        // tps = ceil(tc/NKS), split s covers tiles [s*tps, min(s*tps+tps, tc)).
        auto split_range = [&](int bq, int& lo, int& hi) {
            const int m_end = a.query_start + (bq + 1) * a.block_m;
            const int tc = (min(m_end, a.kv_len) + a.block_n - 1) / a.block_n;
            const int tps = (tc + a.num_splits - 1) / a.num_splits;
            const int st = static_cast<int>(blockIdx.y) * tps;
            const int et = min(st + tps, tc);
            lo = st * a.block_n;
            hi = max(lo, min(et * a.block_n, a.kv_len));
        };
        split_range(row0 / a.block_m, key_lo, key_hi);
        wave_kv_end = min(wave_kv_end, key_hi);
        if (wave_kv_end <= key_lo) wave_kv_end = 0;  // empty range: no tile
        // The ranges grow with the q block, so the workgroup's union runs from
        // its lowest block's start to its highest block's end.
        const int pt_min = max(0, a.n_pos_tiles - 1 - (rblk * kWaves + kWaves - 1) / a.group);
        int lo_min, hi_min, lo_max, hi_max;
        split_range(pt_min * kPfRows / a.block_m, lo_min, hi_min);
        split_range(pt_max * kPfRows / a.block_m, lo_max, hi_max);
        blk_end = min(blk_kv_end, hi_max);
        tile0 = lo_min / kPfBN;
        if (blk_end <= lo_min) blk_end = tile0 * kPfBN;  // no key in any range
    }
    const int ntiles = max(0, (blk_end + kPfBN - 1) / kPfBN - tile0);
    // This wavefront's active tiles [wave_t0, wave_tiles), relative to tile0.
    const int wave_t0 = (wave_kv_end > 0) ? key_lo / kPfBN - tile0 : 0;
    const int wave_tiles = (wave_kv_end > 0) ? (wave_kv_end + kPfBN - 1) / kPfBN - tile0 : 0;

    const uint16_t* kh = a.k_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;
    const uint16_t* vh = a.v_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;

    // HBM -> LDS copy of tile `tile` into stage `st`: this wavefront fills K
    // and V blocks wave*kDmaPerWave + r; lane l moves row b + 16*(l/16), 16-byte
    // column l%16.  On the block's last tile rows at or past blk_kv_end are
    // clamped to the last valid row (they are masked in the softmax).
    const uint32_t lds0 = static_cast<uint32_t>(
        (uintptr_t)((__attribute__((address_space(3))) unsigned char*)(pf_lds)));
    // kFresh: the lane terms are derived again from the lane id at this call,
    // so the compiler cannot hoist them out of the persistent task loop and
    // keep (or spill) them across it; used for the prologue's two tiles.
    auto issue_tile = [&](int tile, int st, auto fresh) {
        int ln = lane;
        if constexpr (decltype(fresh)::value) asm volatile("" : "+v"(ln));
        const uint32_t lane_off = 4096u * static_cast<uint32_t>(ln >> 4) + 16u * (ln & 15);
        const uint32_t kb = lds0 + st * kPfStageBytes;
        const uint32_t vb = kb + kPfKBytes;
        const int n0 = (tile0 + tile) * kPfBN;
        const bool clamp = n0 + kPfBN > blk_kv_end;
#pragma unroll
        for (int r = 0; r < kDmaPerWave; ++r) {
            const int blk = wave * kDmaPerWave + r;
            int64_t row_base = static_cast<int64_t>(n0 + blk) * kHeadDim;
            uint32_t off = lane_off;
            if (clamp) {
                // Address from the tile start: n0 <= blk_kv_end - 1, so every
                // clamped row is >= n0 and the unsigned offset stays in range.
                const int row = min(n0 + blk + 16 * (ln >> 4), blk_kv_end - 1);
                row_base = static_cast<int64_t>(n0) * kHeadDim;
                off = static_cast<uint32_t>(row - n0) * 256u + 16u * (ln & 15);
            }
            lds_dma16(kh + row_base, off, kb + kPfKBlock * blk);
            lds_dma16(vh + row_base, off, vb + kPfVBlock * blk);
        }
    };

    // Tiles 0 and 1 are copied ahead; tile t+2 is issued in tile step t
    // (after the barrier that opens it), into the stage of tile t-2, whose
    // last reader (group B's PV of tile t-2, in its GEMM(t-1)) ended before
    // that barrier.
    if (ntiles > 0) issue_tile(0, 0, std::integral_constant<bool, kDyn>{});
    if (ntiles > 1) issue_tile(1, 1, std::integral_constant<bool, kDyn>{});

    // Q^T (B operand): qop[kk] = Q[row0 + l32][16kk + 8hl + 0..7].
    half8_t qop[8];
    {
        const int row = row0 + l32;
        const bool ok = task_ok && row < a.q_len;
        const uint16_t* qr = a.q + (static_cast<int64_t>(ok ? row : 0) * a.num_q_heads + qh) * kHeadDim;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) qop[kk] = load_half8(qr + 16 * kk + 8 * hl);
        if (!ok) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) qop[kk] = half8_t{};
        }
    }
    // Settle the Q loads here.  The compiler's wait insertion does not see the
    // asm DMAs, so a Q load still pending at the loop would make it wait
    // for Q inside the loop with a vmcnt that, counted by the hardware, also
    // covers the next tile's copies: one stall per tile.  The asm "use" makes
    // it wait once, before the loop.
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) asm volatile("" : "+v"(qop[kk]));

    float16_t o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    float m_run = kPfNegBig, l_run = 0.0f;
    const float c = a.scale_log2;
    float16_t s[2];  // S^T of the tile in flight
    half8_t pop[4];  // P^T of the last softmaxed tile
#pragma unroll
    for (int k = 0; k < 4; ++k) pop[k] = half8_t{};
    // The V half of the last stage is what GEMM(0) multiplies with P = 0:
    // zero it (finite), before the first barrier.  Tile 3 refills it only
    // after both groups are past GEMM(0).
    {
        uint4_t* vz = reinterpret_cast<uint4_t*>(pf_lds + (kPfStages - 1) * kPfStageBytes + kPfKBytes);
        for (int i = tid; i < kPfVBytes / 16; i += kWaves * kWave) vz[i] = uint4_t{0u, 0u, 0u, 0u};
    }

    // Per-lane LDS read offsets.  K (A operand of S^T = K Q^T): key 32mb + l32,
    // dims 16kk + 8hl.  V^T (A operand of O^T += V^T P^T) via the transposing
    // read: 16-lane group gi = lane/16 covers dims 32db + 16(gi&1) + [0,16) and
    // keys 16ks + 4(gi>>1) + [0,4) (+8 for reduction slots 4..7).
    const int gi = lane >> 4, ii = lane & 15;
    const uint32_t k_lane = (l32 & 15) * kPfKBlock + (l32 >> 4) * 256 + 16 * hl;
    const uint32_t v_lane = (4 * (gi >> 1) + (ii >> 2)) * kPfVBlock + 32 * (gi & 1) + 8 * (ii & 3);

    // GEMM phase of tile j: O^T += V^T P^T of tile j-1 (MFMA slots 0-15:
    // key step i/4, dim block i%4), then S^T = K Q^T of tile j (slots 16-31:
    // dim step (i-16)/2, key block i%2).  One software pipeline over the 32
    // slots: each slot's LDS operand is read kPfAhead slots before its MFMA
    // into a ring of registers, so LDS latency hides behind ~kPfAhead MFMAs;
    // a scheduling fence per slot keeps that order.
    //
    // Every GEMM phase runs all 32 slots (one code path keeps register
    // allocation tight): at j = 0 the PV half multiplies P = 0 with the V
    // stage zeroed below (adds exactly +0 to O); at j = wave_tiles the S half
    // reads a stage inside LDS and its result is never used.
    // A split wavefront whose range starts after the workgroup's first tile
    // runs the GEMM phases before it too: its P is still zero there (PV adds
    // exactly +0; the V tile is finite cache data) and those S tiles are
    // never softmaxed.  One skip condition keeps the accumulators in place.
    auto gemm_phase = [&](int j) {
        if (j > wave_tiles) return;
        constexpr int kRing = kPfAhead + 1;
        const unsigned char* vb = pf_lds + ((j + kPfStages - 1) % kPfStages) * kPfStageBytes + kPfKBytes + v_lane;
        const unsigned char* kb = pf_lds + (j % kPfStages) * kPfStageBytes + k_lane;
        auto read_op = [&](int i) {
            if (i < 16) {
                // V^T[32 dims of block i%4, 16 keys of step i/4].
                const unsigned char* p0 = vb + 256 * (i >> 2) + 64 * (i & 3);
                return cat(lds_read_tr16(reinterpret_cast<const half_t*>(p0)),
                           lds_read_tr16(reinterpret_cast<const half_t*>(p0 + 8 * kPfVBlock)));
            }
            // K[32 keys of block i%2, 16 dims of step (i-16)/2].
            return *reinterpret_cast<const half8_t*>(kb + 512 * (i & 1) + 32 * ((i - 16) >> 1));
        };
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[mb][r] = 0.0f;
        half8_t ring[kRing];
        // Issue priority above the softmax-phase wave on the same SIMD while
        // feeding the matrix core (measured: ~1% faster; raising the softmax
        // phase instead does nothing).
        __builtin_amdgcn_s_setprio(2);
#pragma unroll
        for (int i = 0; i < kPfAhead; ++i) ring[i % kRing] = read_op(i);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            if (i + kPfAhead < 32) ring[(i + kPfAhead) % kRing] = read_op(i + kPfAhead);
            if (i < 16) {
                o[i & 3] = mfma32x32x16(ring[i % kRing], pop[i >> 2], o[i & 3]);
            } else {
                s[i & 1] = mfma32x32x16(ring[i % kRing], qop[(i - 16) >> 1], s[i & 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
    };

    // Softmax phase of tile j: mask, running max (lazy), P = 2^(c*s - m), row sum.
    // Masked scores: -1e30 as the reference adds (src/kernels.rs:1242-1257).
    // The split form may have rows with every key of a range masked (the
    // range starts past the row's position); -inf gives them p = 0 and so
    // O = 0, LSE = -1e30, weight 0 in the merge (the reference's -1e30 gives
    // such rows p = 1 and an LSE near -1.3e29: also weight 0).
    constexpr float kMasked = kSplit ? -__builtin_inff() : kPfNegBig;
    auto softmax_phase = [&](int j) {
        if (j < wave_t0 || j >= wave_tiles) return;
        const int n0 = (tile0 + j) * kPfBN;
        bool need_mask = (n0 + kPfBN - 1 > pos0) || (n0 + kPfBN > a.kv_len);
        if constexpr (kSplit) need_mask = need_mask || n0 < key_lo || n0 + kPfBN > key_hi;
        if (need_mask) {
            // Keys n in [key_lo, n_end) stay, n_end = min(position + 1, key_hi,
            // kv_len) clamped to >= key_lo: one unsigned compare per score.
            const int n_end = max(key_lo, min(min(pos0 + l32 + 1, key_hi), a.kv_len));
            const uint32_t span = static_cast<uint32_t>(n_end - key_lo);
            const int rel0 = n0 - key_lo + 4 * hl;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int rel = rel0 + 32 * mb + 8 * (r >> 2) + (r & 3);
                    if (static_cast<uint32_t>(rel) >= span) s[mb][r] = kMasked;
                }
        }
        // P = 2^(c*s - m) with the running max m as it stands; the row sum
        // runs in four independent f32 chains.
        auto exp_tile = [&](float m_use) {
            // Each chain starts from its first pair rather than from 0.0f: the
            // compiler keeps a float 0 + x (it is not x for x = -0), and those
            // four adds measured ~1% of the kernel's time.  p >= 0, so the
            // sums are the same values.
            float ps[4];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const float p0 = __builtin_amdgcn_exp2f(fmaf(s[mb][r], c, -m_use));
                    const float p1 = __builtin_amdgcn_exp2f(fmaf(s[mb][r + 1], c, -m_use));
                    const int k = (r >> 1) & 3;
                    ps[k] = (mb == 0 && r < 8) ? (p0 + p1) : ps[k] + (p0 + p1);
                    pop[2 * mb + (r >> 3)][r & 7] = static_cast<half_t>(p0);
                    pop[2 * mb + (r >> 3)][(r & 7) + 1] = static_cast<half_t>(p1);
                }
            return (ps[0] + ps[1]) + (ps[2] + ps[3]);
        };
        float psum = exp_tile(m_run);
        // The max is only raised when P would leave f16 range: a lane's partial
        // row sum below 2^15 bounds each of its p below 2^15 (the test also
        // catches inf).  Then the tile's row max becomes the running max, O and
        // l are rescaled and P is recomputed.  Until then p <= 2^15 keeps full
        // f16 relative precision, so the normalised result is the same function.
        if (__any(!(psum < kPfPsumLimit))) {
            float mx = kPfNegBig;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[mb][r]);
            mx = fmaxf(mx, swap_halves(mx));
            const float m_new = fmaxf(m_run, mx * c);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] *= alpha;
            m_run = m_new;
            psum = exp_tile(m_run);
        }
        l_run += psum;
    };

    // Tile step t: group A runs GEMM(t) then softmax(t), group B softmax(t-1)
    // then GEMM(t).  GEMM(ntiles) is the last PV; softmax of a tile outside
    // the wavefront's range is a no-op.  Each group has its own straight-line
    // loop (B's is A's rotated by one phase); both pass the same ntiles+1
    // barriers, one at the start of each step.  Tile t+2 is issued after the
    // barrier of step t into the stage of tile t-2, whose last reader (group
    // B's GEMM(t-1), the PV of tile t-2) ended before that barrier.
    static_assert(kPfStages == 4, "the wait below assumes one tile in flight behind tile t");
    auto open_tile_step = [&](int t) {
        if (t < ntiles) {
            // Tile t is in LDS once at most the copies of tile t+1 are
            // outstanding (vector-memory loads retire in order).
            if (t + 1 < ntiles) {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kDmaPerWave));
            } else {
                __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
            }
        }
        pf_barrier();
    };
    // The copies of tile t+2 go out at the start of each wavefront's softmax
    // phase of step t: group A's after its GEMM phase, group B's at the
    // start of the step.  Issued by all eight wavefronts right after the
    // barrier, the copies queue behind each other and hold up the GEMM phase
    // of group A (measured ~1% slower, bit-identical output).
    if (kWaves == 4 || grp == 0) {
        for (int t = 0; t <= ntiles; ++t) {
            open_tile_step(t);
            gemm_phase(t);
            if (t + 2 < ntiles) issue_tile(t + 2, (t + 2) % kPfStages, std::false_type{});
            softmax_phase(t);
        }
    } else {
        for (int t = 0; t <= ntiles; ++t) {
            open_tile_step(t);
            if (t + 2 < ntiles) issue_tile(t + 2, (t + 2) % kPfStages, std::false_type{});
            softmax_phase(t - 1);
            gemm_phase(t);
        }
    }

    if constexpr (kDyn) {
        if (wave == 0 && lane == 0 && own_live)
            pre_j = __hip_atomic_fetch_add(a.sched + my_q * kPfSchedStride, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (task_ok) {
    // Row row0 + l32 of O^T holds dims d = 32db + 8(r/4) + 4hl + r%4.
    const float lt = l_run + swap_halves(l_run);
    const float l_safe = fmaxf(lt, 1.0e-8f);
    // O / l_safe is the reference's true division (src/kernels.rs:1289-1291),
    // rounded to f32 and then to f16: div_to_half gives that same f16 from one
    // f64 reciprocal per row.  (An f32 reciprocal and multiplies is not the
    // same operation: up to 1 f16 ulp away.)
    const double rl = 1.0 / static_cast<double>(l_safe);
    if constexpr (kSplit) {
        // Logical tile (q block, head group) = bq * (Hq/GROUP) + qh/GROUP; its
        // row r = (row % BM) * GROUP + qh % GROUP in split-major scratch
        // (src/kernels.rs:2105-2141).  Rows past q_len (zero Q) are written
        // too, as the reference's padded tile rows are.
        const int row = row0 + l32;
        const int m_eff = a.block_m * a.split_group;
        const int64_t tile = static_cast<int64_t>(row / a.block_m) * (a.num_q_heads / a.split_group) +
                             qh / a.split_group;
        const int64_t prow = (tile * a.num_splits + blockIdx.y) * m_eff +
                             (row % a.block_m) * a.split_group + qh % a.split_group;
        uint16_t* prow_p = a.att_partial + prow * kHeadDim;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                half4_t h;
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = div_to_half(o[db][4 * i + e], rl);
                *reinterpret_cast<half4_t*>(prow_p + 32 * db + 8 * i + 4 * hl) = h;
            }
        if (hl == 0) a.lse_partial[prow] = m_run + log2f(l_safe);
    } else {
        half4_t hv[16];
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) hv[4 * db + i][e] = div_to_half(o[db][4 * i + e], rl);
        if constexpr (kDyn) {
            // The ticket claimed after the loop is read back before the
            // stores go out: vmcnt also counts stores, so reading it after
            // them would wait for the stores as well.
            if (wave == 0) pre_ticket = own_live ? static_cast<int>(__shfl(pre_j, 0)) : -1;
            asm volatile("" ::: "memory");
        }
        // The 32 x 128 tile goes out in whole rows: written to LDS in the
        // accumulator layout, read back 16 bytes a lane, so one store covers 4
        // rows x 256 bytes.  (Stored from the accumulator layout, every store
        // touches 32 rows, 16 bytes each: 8x the write requests, ~2 us a task.)
        // Group A uses stage (ntiles+1) % 4, group B stage (ntiles+2) % 4: no
        // tile is copied into either after tile ntiles-1 and their last
        // readers ended before the last barrier.  16-byte chunk c of row r
        // sits at chunk c ^ (r % 16), so the row reads are free of bank
        // conflicts.
        // Lane terms derived here from the lane id (the empty asm stops the
        // compiler from hoisting them out of the persistent task loop and
        // spilling them across it).
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int lr = ln & 31, lb = ln >> 4, cc = ln & 15;
        const int sw_w = 16 * (lr & 15);
        const int sw_r = 16 * (cc ^ lb);  // read row r = lb + 4k: r % 16 = lb | 4(k % 4)
        unsigned char* ot = pf_lds + ((ntiles + 1 + grp) % kPfStages) * kPfStageBytes + (wave & 3) * kPfOutBytes;
        unsigned char* wrow = ot + lr * 256 + 8 * (ln >> 5);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<half4_t*>(wrow + ((16 * (4 * db + i)) ^ sw_w)) = hv[4 * db + i];
        // A wavefront's LDS accesses complete in order; the fence keeps the
        // compiler from moving the reads above the writes.
        asm volatile("" ::: "memory");
        const unsigned char* rrow = ot + lb * 256;
        uint16_t* orow = a.out + (static_cast<int64_t>(row0 + lb) * a.num_q_heads + qh) * kHeadDim + 8 * cc;
        const int64_t ostep = static_cast<int64_t>(4) * a.num_q_heads * kHeadDim;  // 4 rows
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint4_t v = *reinterpret_cast<const uint4_t*>(rrow + 1024 * k + (sw_r ^ (64 * (k & 3))));
            if (row0 + lb + 4 * k < a.q_len) *reinterpret_cast<uint4_t*>(orow + ostep * k) = v;
        }
    }
    } else if constexpr (kDyn) {
        if (wave == 0) pre_ticket = own_live ? static_cast<int>(__shfl(pre_j, 0)) : -1;
    }  // task_ok
    if constexpr (!kDyn) break;
    }  // task loop

    if constexpr (kDyn) {
        // The last workgroup to leave clears the counters for the next launch:
        // every other one has stopped claiming before its exit increment.
        if (tid == 0) {
            const uint32_t done = __hip_atomic_fetch_add(a.sched + kPfExit * kPfSchedStride, 1u,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (done + 1 == static_cast<uint32_t>(a.n_wg)) {
                for (int q = 0; q < kPfSchedCounters; ++q)
                    __hip_atomic_store(a.sched + q * kPfSchedStride, 0u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// Short prefill: for a launch whose row blocks need at most kSpWaves key tiles
// and whose (query head, 32-row block) pairs fit one workgroup per CU.  The
// grid above would walk up to 8 tiles in sequence in its heaviest workgroup;
// here one workgroup takes one (query head, row block), its 8 wavefronts take
// one 64-key tile each, and the 8 online-softmax partials (m, l, O) meet in
// LDS: the critical path is one tile and a merge.  Each wavefront computes
// S^T = K Q^T with K straight from global memory (an A operand is 16
// contiguous bytes of one key row) and O^T += V^T P^T with V copied into its
// own LDS region (the transposing reads need it there), in the LDS layout and
// lane mapping of the main kernel.  The merge follows the split-K reduction:
// M = max_w m_w, out = f16(sum_w 2^(m_w-M) O_w / max(sum_w 2^(m_w-M) l_w, 1e-8)).
// Keys outside a row's causal range are -inf (a wavefront whose tile holds no
// key of a row keeps m = -1e30, l = 0, O = 0 for it: weight 0); tile 0 holds
// key 0, which every row sees, so M is always a real score.
constexpr int kSpWaves = 8;
constexpr int kSpORow = 132;  // f32 per LDS row of a merge partial (16-lane groups hit distinct banks)
constexpr int kSpOBytes = 32 * kSpORow * 4;
static_assert(kSpOBytes + 256 <= kPfVBytes, "a wavefront's merge partial fits its V region");

__global__ __launch_bounds__(kSpWaves * kWave, 1) void attn_prefill_short_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(1024))) unsigned char sp_lds[kSpWaves * kPfVBytes];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int l32 = lane & 31;
    const int hl = lane >> 5;

    // Heaviest row blocks first; the query heads of a row block are consecutive.
    const int qh = static_cast<int>(blockIdx.x % a.num_q_heads);
    const int pt = a.n_pos_tiles - 1 - static_cast<int>(blockIdx.x / a.num_q_heads);
    const int kvh = qh / a.group;
    const int row0 = pt * kPfRows;
    const int pos0 = a.query_start + row0;
    const int blk_kv_end = min(a.kv_len, pos0 + kPfRows);
    const int ntiles = (blk_kv_end + kPfBN - 1) / kPfBN;  // <= kSpWaves (host check)

    unsigned char* vw = sp_lds + wave * kPfVBytes;
    float16_t o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    float m_w = kPfNegBig, l_w = 0.0f;

    if (wave < ntiles) {
        const int n0 = wave * kPfBN;
        const uint16_t* kh = a.k_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;
        const uint16_t* vh = a.v_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;
        // K operands: kop[mb][kk] = K[n0 + 32mb + l32][16kk + 8hl .. +8]; rows
        // at or past blk_kv_end read the last valid row (masked below).
        half8_t kop[2][8];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const int key = min(n0 + 32 * mb + l32, blk_kv_end - 1);
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
                kop[mb][kk] = load_half8(kh + static_cast<int64_t>(key) * kHeadDim + 16 * kk + 8 * hl);
        }
        // V tile into this wavefront's region: copy r fills block r with rows
        // n0 + r + 16j, j = lane/16, clamped like the K rows.  K, V and Q are
        // in flight together (vector-memory ops retire in order, so the first
        // MFMA's wait covers all three): one memory round trip for the tile.
        const uint32_t vw0 = static_cast<uint32_t>(
            (uintptr_t)((__attribute__((address_space(3))) unsigned char*)(vw)));
        const bool clamp = n0 + kPfBN > blk_kv_end;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            int64_t row_base = static_cast<int64_t>(n0 + r) * kHeadDim;
            uint32_t off = 4096u * static_cast<uint32_t>(lane >> 4) + 16u * (lane & 15);
            if (clamp) {
                const int row = min(n0 + r + 16 * (lane >> 4), blk_kv_end - 1);
                row_base = static_cast<int64_t>(n0) * kHeadDim;
                off = static_cast<uint32_t>(row - n0) * 256u + 16u * (lane & 15);
            }
            lds_dma16(vh + row_base, off, vw0 + kPfVBlock * r);
        }
        half8_t qop[8];
        {
            const int row = row0 + l32;
            const bool ok = row < a.q_len;
            const uint16_t* qr = a.q + (static_cast<int64_t>(ok ? row : 0) * a.num_q_heads + qh) * kHeadDim;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) qop[kk] = ok ? load_half8(qr + 16 * kk + 8 * hl) : half8_t{};
        }
        float16_t s[2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[mb][r] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) s[mb] = mfma32x32x16(kop[mb][kk], qop[kk], s[mb]);
        if (n0 + kPfBN - 1 > pos0 || n0 + kPfBN > a.kv_len) {
            const int n_end = min(pos0 + l32 + 1, a.kv_len);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = n0 + 32 * mb + 8 * (r >> 2) + 4 * hl + (r & 3);
                    if (key >= n_end) s[mb][r] = -__builtin_inff();
                }
        }
        const float c = a.scale_log2;
        float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = (mb == 0 ? 2 : 0); r < 16; r += 2) mx = fmaxf(mx, fmaxf(s[mb][r], s[mb][r + 1]));
        mx = fmaxf(mx, swap_halves(mx));
        m_w = fmaxf(kPfNegBig, mx * c);
        half8_t pop[4];
        float ps[4];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const float p0 = __builtin_amdgcn_exp2f(fmaf(s[mb][r], c, -m_w));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(s[mb][r + 1], c, -m_w));
                const int k = (r >> 1) & 3;
                ps[k] = (mb == 0 && r < 8) ? (p0 + p1) : ps[k] + (p0 + p1);
                pop[2 * mb + (r >> 3)][r & 7] = static_cast<half_t>(p0);
                pop[2 * mb + (r >> 3)][(r & 7) + 1] = static_cast<half_t>(p1);
            }
        l_w = (ps[0] + ps[1]) + (ps[2] + ps[3]);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // this wavefront's V copies landed
        asm volatile("" ::: "memory");
        const int gi = lane >> 4, ii = lane & 15;
        const unsigned char* vb = vw + (4 * (gi >> 1) + (ii >> 2)) * kPfVBlock + 32 * (gi & 1) + 8 * (ii & 3);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const unsigned char* p0 = vb + 256 * (i >> 2) + 64 * (i & 3);
            const half8_t va = cat(lds_read_tr16(reinterpret_cast<const half_t*>(p0)),
                                   lds_read_tr16(reinterpret_cast<const half_t*>(p0 + 8 * kPfVBlock)));
            o[i & 3] = mfma32x32x16(va, pop[i >> 2], o[i & 3]);
        }
    }

    // Every wavefront's partial into its own region (its V reads are done
    // after the barrier), rows of kSpORow f32, then m and the row sum l.
    pf_barrier();
    {
        float* orow = reinterpret_cast<float*>(vw) + l32 * kSpORow;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4_t v = {o[db][4 * j], o[db][4 * j + 1], o[db][4 * j + 2], o[db][4 * j + 3]};
                *reinterpret_cast<float4_t*>(orow + 32 * db + 8 * j + 4 * hl) = v;
            }
        const float lt = l_w + swap_halves(l_w);
        float* ml = reinterpret_cast<float*>(vw + kSpOBytes);
        if (hl == 0) {
            ml[l32] = m_w;
            ml[32 + l32] = lt;
        }
    }
    pf_barrier();
    // Thread (row, 8 dims): the 8 partials of its row.
    const int row = tid >> 4, d8 = tid & 15;
    float mw[kSpWaves];
    float M = kPfNegBig;
#pragma unroll
    for (int w = 0; w < kSpWaves; ++w) {
        mw[w] = reinterpret_cast<const float*>(sp_lds + w * kPfVBytes + kSpOBytes)[row];
        M = fmaxf(M, mw[w]);
    }
    float L = 0.0f;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < kSpWaves; ++w) {
        const float wt = __builtin_amdgcn_exp2f(mw[w] - M);
        const float* base = reinterpret_cast<const float*>(sp_lds + w * kPfVBytes);
        L += wt * base[kSpOBytes / 4 + 32 + row];
        const float4_t x0 = *reinterpret_cast<const float4_t*>(base + row * kSpORow + 8 * d8);
        const float4_t x1 = *reinterpret_cast<const float4_t*>(base + row * kSpORow + 8 * d8 + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc[e] += wt * x0[e];
            acc[4 + e] += wt * x1[e];
        }
    }
    const double rl = 1.0 / static_cast<double>(fmaxf(L, 1.0e-8f));
    half8_t h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = div_to_half(acc[e], rl);
    if (row0 + row < a.q_len)
        store_half8(a.out + (static_cast<int64_t>(row0 + row) * a.num_q_heads + qh) * kHeadDim + 8 * d8, h);
}

// The short form applies when every row block needs at most kSpWaves key
// tiles and the (query head, row block) pairs number at most one per CU.
// (The last row block's key range ends at min(kv_len, query_start + 32 *
// row blocks), as the kernel computes it.)
static bool prefill_short_fits(const PrefillArgs& a, int cus) {
    const int64_t n_blocks = (static_cast<int64_t>(a.q_len) + kPfRows - 1) / kPfRows;
    const int64_t last_end = min(static_cast<int64_t>(a.kv_len),
                                 static_cast<int64_t>(a.query_start) + kPfRows * n_blocks);
    return last_end <= static_cast<int64_t>(kSpWaves) * kPfBN && n_blocks * a.num_q_heads <= cus;
}

static int32_t launch_prefill(PrefillArgs a, int num_kv_heads, hipStream_t stream) {
    a.n_pos_tiles = (a.q_len + kPfRows - 1) / kPfRows;
    a.tasks_per_head = a.n_pos_tiles * a.group;
    a.blocks_per_head = (a.tasks_per_head + kPfWaves - 1) / kPfWaves;
    const int64_t blocks = static_cast<int64_t>(a.blocks_per_head) * num_kv_heads;
    if (blocks > 0x7fffffff) return GROUT_ERR_KV_LEN;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return static_cast<int32_t>(e);
    if (prefill_short_fits(a, cus)) {
        const int64_t sblocks = static_cast<int64_t>(a.n_pos_tiles) * a.num_q_heads;
        hipLaunchKernelGGL(attn_prefill_short_kernel, dim3(static_cast<unsigned>(sblocks)),
                           dim3(kSpWaves * kWave), 0, stream, a);
        return launch_status();
    }
    if (2 * blocks <= static_cast<int64_t>(cus)) {
        // At most half the CUs busy: 4-wavefront workgroups, twice as many.
        a.blocks_per_head = (a.tasks_per_head + 3) / 4;
        const int64_t blocks4 = static_cast<int64_t>(a.blocks_per_head) * num_kv_heads;
        hipLaunchKernelGGL((attn_prefill_kernel<false, false, 4>), dim3(static_cast<unsigned>(blocks4)),
                           dim3(4 * kWave), 0, stream, a);
        return launch_status();
    }
    hipLaunchKernelGGL((attn_prefill_kernel<false, false>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kPfWaves * kWave), 0, stream, a);
    return launch_status();
}

// Dynamic schedule: one persistent workgroup per CU (the kernel's LDS allows
// one) when the static grid would run more than two rounds of workgroups;
// smaller grids keep the static launch, which then leaves the counters alone.
static int32_t launch_prefill_sched(PrefillArgs a, int num_kv_heads, uint32_t* sched,
                                    hipStream_t stream) {
    a.n_pos_tiles = (a.q_len + kPfRows - 1) / kPfRows;
    a.tasks_per_head = a.n_pos_tiles * a.group;
    a.blocks_per_head = (a.tasks_per_head + kPfWaves - 1) / kPfWaves;
    const int64_t blocks = static_cast<int64_t>(a.blocks_per_head) * num_kv_heads;
    if (blocks > 0x7fffffff) return GROUT_ERR_KV_LEN;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return static_cast<int32_t>(e);
    if (cus <= 0 || blocks <= 2 * static_cast<int64_t>(cus)) return launch_prefill(a, num_kv_heads, stream);
    a.sched = sched;
    a.n_wg = cus;
    a.num_kv_heads = num_kv_heads;
    // The lightest quarter of each head's blocks goes to the XCD light queues.
    a.pool_block0 = a.blocks_per_head - a.blocks_per_head / 4;
    hipLaunchKernelGGL((attn_prefill_kernel<false, true>), dim3(static_cast<unsigned>(cus)),
                       dim3(kPfWaves * kWave), 0, stream, a);
    return launch_status();
}

// Merge of the split-K partials (prefill_splitk_reduce_merge,
// src/kernels.rs:2151-2323): thread = (row < q_len, q head, 8 dims); weights
// w_s = 2^(lse_s - max) / max(sum, 1e-8), out = f16(sum_s w_s * att_s).
__global__ __launch_bounds__(256) void attn_prefill_split_merge_kernel(
    const uint16_t* __restrict__ att, const float* __restrict__ lse, uint16_t* __restrict__ out,
    int num_q_heads, int q_len, int block_m, int group, int num_splits) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t total = static_cast<int64_t>(q_len) * num_q_heads * (kHeadDim / 8);
    if (idx >= total) return;
    const int d0 = static_cast<int>(idx % (kHeadDim / 8)) * 8;
    const int64_t rh = idx / (kHeadDim / 8);
    const int head = static_cast<int>(rh % num_q_heads);
    const int row = static_cast<int>(rh / num_q_heads);
    const int m_eff = block_m * group;
    const int64_t tile = static_cast<int64_t>(row / block_m) * (num_q_heads / group) + head / group;
    const int r = (row % block_m) * group + head % group;
    const float* l = lse + tile * num_splits * m_eff + r;
    float mx = l[0];
    for (int s = 1; s < num_splits; ++s) mx = fmaxf(mx, l[static_cast<int64_t>(s) * m_eff]);
    float sum = 0.0f;
    for (int s = 0; s < num_splits; ++s) sum += __builtin_amdgcn_exp2f(l[static_cast<int64_t>(s) * m_eff] - mx);
    const float inv = 1.0f / fmaxf(sum, 1.0e-8f);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint16_t* p = att + (tile * num_splits * m_eff + r) * kHeadDim + d0;
    for (int s = 0; s < num_splits; ++s) {
        const float w = __builtin_amdgcn_exp2f(l[static_cast<int64_t>(s) * m_eff] - mx) * inv;
        const half8_t x = load_half8(p + static_cast<int64_t>(s) * m_eff * kHeadDim);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += static_cast<float>(x[e]) * w;
    }
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<half_t>(acc[e]);
    store_half8(out + (static_cast<int64_t>(row) * num_q_heads + head) * kHeadDim + d0, o);
}

static int32_t launch_prefill_split(PrefillArgs a, int num_kv_heads, hipStream_t stream) {
    const int64_t q_blocks = (static_cast<int64_t>(a.q_len) + a.block_m - 1) / a.block_m;
    const int64_t pos_tiles = q_blocks * (a.block_m / kPfRows);
    const int64_t tasks = pos_tiles * a.group;
    const int64_t bph = (tasks + kPfWaves - 1) / kPfWaves;
    const int64_t blocks = bph * num_kv_heads;
    if (pos_tiles > 0x3fffffff || blocks > 0x7fffffff) return GROUT_ERR_KV_LEN;
    a.n_pos_tiles = static_cast<int>(pos_tiles);
    a.tasks_per_head = static_cast<int>(tasks);
    a.blocks_per_head = static_cast<int>(bph);
    hipLaunchKernelGGL((attn_prefill_kernel<true, false>), dim3(static_cast<unsigned>(blocks), a.num_splits),
                       dim3(kPfWaves * kWave), 0, stream, a);
    return launch_status();
}

// Scratch geometry of the split-K form: tiles = ceil(q_len/BM) * (Hq/GROUP),
// rows per tile num_splits * BM * GROUP (src/kernels.rs:1922-1944).
static int64_t prefill_split_rows(int32_t num_q_heads, int32_t q_len, int32_t block_m,
                                  int32_t group, int32_t num_splits) {
    if (num_q_heads <= 0 || q_len < 0 || block_m <= 0 || group <= 0 || num_splits <= 0 ||
        num_q_heads % group != 0)
        return GROUT_ERR_ARG;
    const int64_t tiles = (static_cast<int64_t>(q_len) + block_m - 1) / block_m * (num_q_heads / group);
    return tiles * num_splits * block_m * group;
}

}  // namespace grout

using namespace grout;

// Shared by both prefill entry points: the ensure!s of
// attend_seq_arc_into_ctx_with_position (src/model.rs:5564-5637) on sizes, then
// the static grid (sched == nullptr) or the dynamic schedule.
static int32_t prefill_entry(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                             uint16_t* out, float qk_scale, int32_t num_q_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t q_len, int32_t kv_len,
                             int32_t query_start, int32_t max_seq_len, uint32_t* sched,
                             grout_stream_t stream) {
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

    PrefillArgs a = {};
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
    if (sched == nullptr) return launch_prefill(a, num_kv_heads, to_hip(stream));
    return launch_prefill_sched(a, num_kv_heads, sched, to_hip(stream));
}

extern "C" int32_t grout_attn_prefill(const uint16_t* q, const uint16_t* k_cache,
                                      const uint16_t* v_cache, uint16_t* out, float qk_scale,
                                      int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                      int32_t q_len, int32_t kv_len, int32_t query_start,
                                      int32_t max_seq_len, grout_stream_t stream) {
    return prefill_entry(q, k_cache, v_cache, out, qk_scale, num_q_heads, num_kv_heads, head_dim,
                         q_len, kv_len, query_start, max_seq_len, nullptr, stream);
}

extern "C" int32_t grout_attn_prefill_sched(const uint16_t* q, const uint16_t* k_cache,
                                            const uint16_t* v_cache, uint16_t* out,
                                            float qk_scale, int32_t num_q_heads,
                                            int32_t num_kv_heads, int32_t head_dim, int32_t q_len,
                                            int32_t kv_len, int32_t query_start,
                                            int32_t max_seq_len, uint32_t* sched_counters,
                                            grout_stream_t stream) {
    GROUT_REQUIRE(sched_counters != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(sched_counters) & 3u) == 0, GROUT_ERR_ALIGNMENT);
    return prefill_entry(q, k_cache, v_cache, out, qk_scale, num_q_heads, num_kv_heads, head_dim,
                         q_len, kv_len, query_start, max_seq_len, sched_counters, stream);
}

extern "C" int64_t grout_attn_prefill_sched_counter_bytes(void) {
    return static_cast<int64_t>(kPfSchedCounters) * kPfSchedStride * 4;
}

extern "C" int32_t grout_attn_prefill_split(const uint16_t* q, const uint16_t* k_cache,
                                            const uint16_t* v_cache, uint16_t* att_partial,
                                            float* lse_partial, float qk_scale, int32_t num_q_heads,
                                            int32_t num_kv_heads, int32_t head_dim, int32_t q_len,
                                            int32_t kv_len, int32_t query_start,
                                            int32_t max_seq_len, int32_t block_m, int32_t block_n,
                                            int32_t group, int32_t num_splits,
                                            grout_stream_t stream) {
    // The prefill checks, plus the microbench's group check
    // (benchmarks/src/bin/attention_microbench.rs:411-421) and this
    // kernel's tile limits.
    GROUT_REQUIRE_PTR(q);
    GROUT_REQUIRE_PTR(k_cache);
    GROUT_REQUIRE_PTR(v_cache);
    GROUT_REQUIRE_PTR(att_partial);
    GROUT_REQUIRE_PTR(lse_partial);
    GROUT_REQUIRE(head_dim == kHeadDim, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
                  GROUT_ERR_HEADS);
    GROUT_REQUIRE(max_seq_len > 0, GROUT_ERR_SEQ_RANGE);
    GROUT_REQUIRE(q_len >= 0 && query_start >= 0, GROUT_ERR_KV_LEN);
    GROUT_REQUIRE(kv_len >= 1 && kv_len <= max_seq_len, GROUT_ERR_KV_LEN);
    GROUT_REQUIRE(qk_scale > 0.0f && qk_scale < 1.0e30f, GROUT_ERR_ARG);
    GROUT_REQUIRE(group >= 1 && (num_q_heads / num_kv_heads) % group == 0, GROUT_ERR_GROUP);
    GROUT_REQUIRE(block_m >= kPfRows && block_m % kPfRows == 0 && block_m <= 65536, GROUT_ERR_ARG);
    GROUT_REQUIRE(block_n >= 1 && block_n <= 65536, GROUT_ERR_SPLITS);
    GROUT_REQUIRE(num_splits >= 1 && num_splits <= GROUT_MAX_PREFILL_SPLITS, GROUT_ERR_SPLITS);
    if (q_len == 0) return GROUT_OK;

    PrefillArgs a = {};
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.out = nullptr;
    a.scale_log2 = qk_scale / logf(2.0f);
    a.num_q_heads = num_q_heads;
    a.group = num_q_heads / num_kv_heads;
    a.q_len = q_len;
    a.kv_len = kv_len;
    a.query_start = query_start;
    a.max_seq_len = max_seq_len;
    a.att_partial = att_partial;
    a.lse_partial = lse_partial;
    a.block_m = block_m;
    a.block_n = block_n;
    a.split_group = group;
    a.num_splits = num_splits;
    return launch_prefill_split(a, num_kv_heads, to_hip(stream));
}

extern "C" int32_t grout_attn_prefill_split_merge(const uint16_t* att_partial,
                                                  const float* lse_partial, uint16_t* out,
                                                  int32_t num_q_heads, int32_t head_dim,
                                                  int32_t q_len, int32_t block_m, int32_t group,
                                                  int32_t num_splits, grout_stream_t stream) {
    GROUT_REQUIRE_PTR(att_partial);
    GROUT_REQUIRE_PTR(lse_partial);
    GROUT_REQUIRE_PTR(out);
    GROUT_REQUIRE(head_dim == kHeadDim, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(num_q_heads > 0, GROUT_ERR_HEADS);
    GROUT_REQUIRE(q_len >= 0, GROUT_ERR_KV_LEN);
    GROUT_REQUIRE(group >= 1 && num_q_heads % group == 0, GROUT_ERR_GROUP);
    GROUT_REQUIRE(block_m >= 1 && block_m <= 65536, GROUT_ERR_ARG);
    GROUT_REQUIRE(num_splits >= 1 && num_splits <= GROUT_MAX_PREFILL_SPLITS, GROUT_ERR_SPLITS);
    if (q_len == 0) return GROUT_OK;
    const int64_t threads = static_cast<int64_t>(q_len) * num_q_heads * (kHeadDim / 8);
    const int64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffff) return GROUT_ERR_KV_LEN;
    hipLaunchKernelGGL(attn_prefill_split_merge_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       to_hip(stream), att_partial, lse_partial, out, num_q_heads, q_len, block_m,
                       group, num_splits);
    return launch_status();
}

extern "C" int64_t grout_attn_prefill_split_partial_bytes(int32_t num_q_heads, int32_t head_dim,
                                                          int32_t q_len, int32_t block_m,
                                                          int32_t group, int32_t num_splits) {
    if (head_dim <= 0) return GROUT_ERR_ARG;
    const int64_t rows = prefill_split_rows(num_q_heads, q_len, block_m, group, num_splits);
    return rows < 0 ? rows : rows * head_dim * 2;
}

extern "C" int64_t grout_attn_prefill_split_lse_bytes(int32_t num_q_heads, int32_t q_len,
                                                      int32_t block_m, int32_t group,
                                                      int32_t num_splits) {
    const int64_t rows = prefill_split_rows(num_q_heads, q_len, block_m, group, num_splits);
    return rows < 0 ? rows : rows * 4;
}

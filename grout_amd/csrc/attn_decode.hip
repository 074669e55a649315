// Split-K GQA decode attention, its log-sum-exp merge, and the fused decode
// step (QK norm/RoPE/KV write + split + merge in one launch).
//
// Replaces fmha_decode_gqa_split (src/kernels.rs:2586-2749),
// splitk_reduce_merge (src/kernels.rs:2771-2868) and, in the fused form, the
// qk_norm_rope_kv_decode_raw_f16 -> fmha_decode_gqa_split -> splitk_reduce_merge
// sequence grout records per layer (src/model.rs:3194-3221, 3428-3473).
// The scratch layout, the split boundaries and the per-split numerics are the
// reference's:
//   s_kv = pos + 1; tiles = ceil(s_kv/BN); per = ceil(tiles/NKS);
//   split s covers tokens [s*per*BN, min((s*per+per)*BN, s_kv));
//   O_s = f16(acc/max(l,1e-8)), LSE_s = m + log2(max(l,1e-8)) in log2 units,
//   att_partial [Hkv, NKS*G, D] split-major, lse_partial [Hkv, NKS*G].
//
// Decode is HBM-bound (4-8 FLOP per byte); the kernel is shaped for bytes in
// flight:
//  * Workgroup = (split, kv_head), 4 wavefronts, one per CU.
//    Each wavefront streams its own 16-token sub-chunks of the split (K 4 KB +
//    V 4 KB each) through a private 2-stage LDS ring with direct HBM->LDS
//    copies; it waits only for its own copies, so the stream has no
//    workgroup barrier, and the next copy goes out as soon as the operands
//    of the current sub-chunk have been read.
//  * All G query heads of the KV head share every K/V byte: S^T = K Q^T runs
//    on v_mfma_f32_16x16x32_f16 and O^T += V^T P^T on v_mfma_f32_16x16x16_f16
//    with the G heads (padded to 16) as N.  The S^T accumulator layout is
//    exactly the P^T operand (reduction slot j of lane group q is token
//    4q+j); V^T is read in the same order with one ds_read_b64_tr_b16 per 16
//    dims.
//  * Token rows sit unpadded in LDS with their 16-byte chunks XOR-swizzled
//    by the copy itself (each lane fetches the chunk that belongs at its
//    destination), so the K and V^T operand reads are bank-conflict free.
//  * The four wavefronts' (m, l, acc) are combined through LDS at the end.
//  * Fused form: every workgroup recomputes its G query rows (RMSNorm +
//    RoPE, as the prefill/decode norm kernel); the split holding the new
//    position also writes its K/V row to the cache and patches it into the
//    sub-chunk whose copy read the cache before that store.  The
//    last workgroup of a KV head merges the splits, found with a counter;
//    the partials travel through agent-coherent (sc1) stores and loads so no
//    L2-wide writeback/invalidate is needed.  When asked to, the merger of
//    the last KV head to complete advances the device position.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "abi_util.h"
#include "common.h"

namespace grout {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = kDecWaves * kWave;
// Each wavefront streams its own 16-token sub-chunks (sub-chunks w, w+4, ...
// of the split) through a private ring of kDecWaveStages stages; a stage is
// the sub-chunk's K rows (4 KB) then its V rows (4 KB).  No workgroup barrier
// is needed inside the stream.
//
// Two stages keep at most 64 KB of copies in flight per CU, 16 MB over the
// chip, about what HBM's bandwidth times its loaded latency needs.  Measured
// (fused step, caches cycled): 4 stages, twice that in flight, ran 3-11%
// slower at every shape (Qwen3-32B 32K 26.8 vs 25.9 us, 8K 13.05 vs 11.65 us;
// Qwen3-4B 4K 9.44 vs 8.95 us), 3 stages in between; 1 stage is too little
// (26.97 us at 32K).  The surplus only queues in the memory system, where
// some workgroups' requests wait longer than others' and the slowest
// workgroup sets the end of the step.
constexpr int kDecSubTok = 16;
constexpr int kDecSubBytes = kDecSubTok * 256;
constexpr int kDecWaveStages = 2;
constexpr int kDecWaveBytes = kDecWaveStages * 2 * kDecSubBytes;
// The stages (64 KB) and, after the stream, the wave combine and (fused form)
// the merge's batch of partial rows (128 KB) share one LDS buffer.  The
// larger fused buffer does not limit the stream: the fused grid is one
// workgroup per CU, and padding the kernel past half of a CU's LDS measured
// the same.  The split-only form keeps the stage size, so two of its
// workgroups still share a CU when its grid is larger than the CU count.
constexpr int kDecStageLdsBytes = kDecWaves * kDecWaveBytes;
constexpr int kDecMergeLdsBytes = 128 * 1024;
// Partial rows (256 B each) of one merge batch: the 32 splits of 16 query
// heads, or the 64 splits of 8 that 4 KV heads take on 256 CUs.
constexpr int kDecMergeRows = kDecMergeLdsBytes / 256;
constexpr int kDecFusedLdsBytes = kDecStageLdsBytes > kDecMergeLdsBytes ? kDecStageLdsBytes
                                                                        : kDecMergeLdsBytes;
constexpr int kDecMinSplitTokens = 64;
// Chunk swizzle of a 256-byte token row in a stage: LDS chunk c of row tr
// holds global chunk c ^ dec_swz(tr).  Distinct over the 16 rows (K reads:
// one row per lane) and, for the transposing V reads, spreading each 32-lane
// half over all 64 banks.
__device__ __forceinline__ int dec_swz(int tr) { return 2 * (tr & 7) + (tr >> 3); }
// Final combine of the wavefronts: per wave 16 head rows of kHeadDim + 4
// floats (the pad puts the 16 rows a lane group writes in distinct banks),
// then m and l of the 16 heads.
constexpr int kDecRedRow = kHeadDim + 4;
constexpr int kDecRedStride = 16 * kDecRedRow + 32;   // floats per wave
constexpr float kNegBig = -1.0e30f;
// Lazy rescale slack of the decode softmax (log2 units): p <= 2^8.
constexpr float kDecRescaleSlack = 8.0f;
// Merge counters sit in separate 256-byte lines so the heads' atomics do not
// serialise on one line.
constexpr int kDecCounterStride = 64;  // u32 elements

static_assert(kDecWaves * kDecRedStride * 4 <= kDecStageLdsBytes,
              "wave combine reuses the stage buffers");

struct DecodeArgs {
    // Attention (all forms).
    const uint16_t* q;          // [Hkv, G, D] rotated queries (split-only form)
    const uint16_t* k_cache;
    const uint16_t* v_cache;
    uint16_t* att_partial;
    float* lse_partial;
    float scale_log2;
    int group;
    int num_kv_heads;
    int max_seq_len;
    int block_n;
    int num_splits;
    // Fused form only.
    const uint16_t* qkv;        // [Q(Hq*D) | K(Hkv*D) | V(Hkv*D)]
    const uint16_t* q_weight;
    const uint16_t* k_weight;
    const float* inv_freq;
    uint16_t* q_out;            // rows [0, Hq) written
    uint16_t* k_cache_w;        // = k_cache, writable
    uint16_t* v_cache_w;        // = v_cache, writable
    uint16_t* out;              // [Hkv, G, D]
    uint32_t* counters;         // Hkv + 1 counters kDecCounterStride apart, zero on entry and exit
    uint32_t* position_w;       // = the position argument, advanced when advance_position
    float eps;
    int num_q_heads;
    int advance_position;
};

// Asynchronous 16-byte HBM -> LDS copy (global_load_lds_dwordx4, scalar base
// + 32-bit per-lane byte offset); lane l's 16 bytes land at LDS byte
// lds_base + 16*l.  Inline asm keeps the compiler from serialising the copies
// behind vmcnt(0) waits; the kernel waits for them with s_waitcnt vmcnt before
// its workgroup barrier.  M0 carries the LDS base; one wait state separates
// the M0 write from the copy.  The K/V stream is read once per step, so the
// copies carry the non-temporal hint.
__device__ __forceinline__ void dec_lds_dma16(const void* gbase, uint32_t voff, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, %1 nt"
        :
        : "v"(voff), "s"(gbase), "s"(lds_base)
        : "memory");
}

// Same copy with a full 64-bit per-lane source address.
__device__ __forceinline__ void dec_lds_dma16_ptr(const void* gptr, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, off"
        :
        : "v"(gptr), "s"(lds_base)
        : "memory");
}

// Same copy, device-coherent (sc1): reads data that workgroups on other
// XCDs wrote with sc1 stores, past any stale line in this XCD's L2.
__device__ __forceinline__ void dec_lds_dma16_ptr_sc1(const void* gptr, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %0, off sc1"
        :
        : "v"(gptr), "s"(lds_base)
        : "memory");
}

constexpr int dec_waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

// s_waitcnt vmcnt(min(n, N)) for a wave-uniform n >= 0: the count must be an
// immediate, so each value has its own instruction (a chain of scalar
// compares); a count above N waits for more than asked, never for less.
template <int N>
__device__ __forceinline__ void dec_wait_vm_atmost(int n) {
    if constexpr (N == 0) {
        __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(0));
    } else {
        if (n >= N) {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(N));
        } else {
            dec_wait_vm_atmost<N - 1>(n);
        }
    }
}

// Per-workgroup inputs staged into LDS ahead of the K/V stream, 256 B rows:
// split-only form: rows [0,G) = the G rotated query rows; fused form: rows
// [0,G) = raw query rows of the QKV vector, then K row, V row, q_weight,
// k_weight and inv_freq (64 f32 = 256 B).
constexpr int kDecProRows = GROUT_MAX_DECODE_GROUP + 5;
constexpr int kDecProDmas = (kDecProRows + 3) / 4;

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

// Max / sum over each 32-lane half of the wavefront, every lane of the half
// ending with the same value: DPP quad swaps (lane ^ 1, ^ 2), the 8-lane and
// 16-lane mirrors, then v_permlane16_swap (lane ^ 16).  Each step pairs
// lanes that already hold equal values, so the sum is the same float in
// every lane of the half.
template <typename Op>
__device__ __forceinline__ float half32_reduce(float x, Op op) {
    auto dpp = [](float v, auto ctrl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                     decltype(ctrl)::value, 0xf, 0xf, false));
    };
    x = op(x, dpp(x, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
    x = op(x, dpp(x, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
    x = op(x, dpp(x, std::integral_constant<int, 0x141>{}));  // row_half_mirror
    x = op(x, dpp(x, std::integral_constant<int, 0x140>{}));  // row_mirror
    return op(x, swap_rows16(x));
}

// RMSNorm + RoPE of one 128-wide row held by 8 lanes (lane t: elements
// [8t,8t+8) and [64+8t, 64+8t+8)), same operation order as
// qk_norm_rope_kv_kernel.
__device__ __forceinline__ void norm_rope_row8(half8_t xlo, half8_t xhi, half8_t wlo, half8_t whi,
                                               const float* s_cos, const float* s_sin, float eps,
                                               int lane8, half8_t& ylo, half8_t& yhi) {
#pragma clang fp contract(off)
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
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float n_lo = static_cast<float>(xlo[i]) * inv_rms * static_cast<float>(wlo[i]);
        const float n_hi = static_cast<float>(xhi[i]) * inv_rms * static_cast<float>(whi[i]);
        const float cv = s_cos[8 * lane8 + i];
        const float sv = s_sin[8 * lane8 + i];
        ylo[i] = static_cast<half_t>(n_lo * cv - n_hi * sv);
        yhi[i] = static_cast<half_t>(n_hi * cv + n_lo * sv);
    }
}

// Workgroup barrier that waits only for this wave's LDS traffic: copies into
// LDS stay in flight across it.  The asm memory clobber keeps the compiler
// from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Agent-coherent 16-byte store: one global_store_dwordx4 with the sc1 cache
// policy, the form a relaxed agent-scope atomic store takes on this target,
// so a workgroup on another XCD sees it without an L2-wide writeback or
// invalidate.  The kernel orders it with s_waitcnt vmcnt(0) before the
// counter increment that publishes it.
__device__ __forceinline__ void store16_agent(uint16_t* p, half8_t v) {
    const uint4_t u = __builtin_bit_cast(uint4_t, v);
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(u) : "memory");
}

__device__ __forceinline__ float4_t mfma16x16x16(half4_t a, half4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// The position pointer is the first kernel argument, outside DecodeArgs:
// this file is compiled with -amdgpu-kernarg-preload-count=2, so the pointer
// arrives in SGPRs at dispatch and the position load is the kernel's first
// memory access instead of waiting on a kernel-argument load (c4 25.43 ->
// 25.21 us, Qwen3-4B 4K 8.65 -> 8.55 us, bit-identical).
template <bool kFused>
__global__ __launch_bounds__(kDecThreads, 1) void attn_decode_kernel(const uint32_t* __restrict__ d_position,
                                                                     DecodeArgs a) {
    __shared__ __attribute__((aligned(1024))) unsigned char lds[kFused ? kDecFusedLdsBytes : kDecStageLdsBytes];
    __shared__ __attribute__((aligned(1024))) unsigned char pro[kDecProDmas * 1024];
    __shared__ __attribute__((aligned(16))) half_t q_lds[GROUT_MAX_DECODE_GROUP * kHeadDim];
    __shared__ float s_cos[64], s_sin[64];
    __shared__ uint32_t s_flag;
    __shared__ float s_wsum[GROUT_MAX_DECODE_GROUP];  // merge: sum of the split weights per query row

    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int n = lane & 15;     // head column of the MFMA tiles
    const int qgrp = lane >> 4;  // lane group: k-slice / token quartet
    const int G = a.group;

    // Position from device memory; reads are clamped to the cache.
    const uint32_t pos_raw = *d_position;
    // Prologue inputs into `pro` (wave 0).  None depends on the position, so
    // the copies go out while the position load is in flight; the K/V
    // sub-chunk copies follow once the split range is known.
    const uint32_t pro0 = static_cast<uint32_t>(
        (uintptr_t)((__attribute__((address_space(3))) unsigned char*)(pro)));
    const int n_pro = kFused ? G + 5 : G;
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < kDecProDmas; ++i) {
            if (4 * i < n_pro) {
                int r = 4 * i + (lane >> 4);
                if (r >= n_pro) r = 0;  // pad lanes repeat row 0
                const unsigned char* src;
                if constexpr (kFused) {
                    const int64_t hq = a.num_q_heads, hkv = a.num_kv_heads;
                    if (r < G) {
                        src = reinterpret_cast<const unsigned char*>(a.qkv + (static_cast<int64_t>(kvh) * G + r) * kHeadDim);
                    } else if (r == G) {
                        src = reinterpret_cast<const unsigned char*>(a.qkv + (hq + kvh) * kHeadDim);
                    } else if (r == G + 1) {
                        src = reinterpret_cast<const unsigned char*>(a.qkv + (hq + hkv + kvh) * kHeadDim);
                    } else if (r == G + 2) {
                        src = reinterpret_cast<const unsigned char*>(a.q_weight);
                    } else if (r == G + 3) {
                        src = reinterpret_cast<const unsigned char*>(a.k_weight);
                    } else {
                        src = reinterpret_cast<const unsigned char*>(a.inv_freq);
                    }
                } else {
                    src = reinterpret_cast<const unsigned char*>(a.q + (static_cast<int64_t>(kvh) * G + r) * kHeadDim);
                }
                dec_lds_dma16_ptr(src + 16 * (lane & 15), pro0 + 1024u * i);
            }
        }
    }
    const uint32_t pos = pos_raw < static_cast<uint32_t>(a.max_seq_len) ? pos_raw
                                                                         : a.max_seq_len - 1;
    const int s_kv = static_cast<int>(pos) + 1;
    int tok_begin, tok_end;
    if constexpr (kFused) {
        // The fused form's partials never leave the launch, so its splits
        // are balanced in 16-token sub-chunks: split s takes sub-chunks
        // [s*n/NKS, (s+1)*n/NKS) of n = ceil(s_kv/16).  The reference's
        // ceil(tiles/NKS) tiles per split leaves the last splits short or
        // empty (s_kv 4097, BN 32, 32 splits: 25 splits of 160 tokens, one of
        // 97 and six empty; here 128-129 tokens each).
        const int64_t nsub_all = (s_kv + kDecSubTok - 1) / kDecSubTok;
        const int sb = static_cast<int>(split * nsub_all / a.num_splits);
        const int se = static_cast<int>((split + 1) * nsub_all / a.num_splits);
        tok_begin = sb * kDecSubTok;
        tok_end = (sb < se) ? min(se * kDecSubTok, s_kv) : tok_begin;
    } else {
        const int tiles = (s_kv + a.block_n - 1) / a.block_n;
        const int per = (tiles + a.num_splits - 1) / a.num_splits;
        const int tb = split * per;
        const int te = min(tb + per, tiles);
        tok_begin = tb * a.block_n;
        tok_end = (tb < te) ? min(te * a.block_n, s_kv) : tok_begin;
    }
    const int nsub = (tok_end - tok_begin + kDecSubTok - 1) / kDecSubTok;
    // Wavefront w owns sub-chunks w, w+4, w+8, ... of the split (its k-th is
    // w + 4k): a fixed assignment, so every launch accumulates the same
    // tokens in the same order and the output is bit-reproducible.
    const int nk = nsub > wave ? (nsub - wave + kDecWaves - 1) / kDecWaves : 0;
    const int n_first = min(kDecWaveStages, nk);

    const uint16_t* kh = a.k_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;
    const uint16_t* vh = a.v_cache + static_cast<int64_t>(kvh) * a.max_seq_len * kHeadDim;

    // Sub-chunk copy: sub-chunk `sub` of the split (tokens t0 + [0,16),
    // t0 = tok_begin + 16*sub), this wavefront's k-th, lands in its stage
    // k % kDecWaveStages.  Copy i moves
    // token rows 4i..4i+3: 1 KB contiguous in the cache, 1 KB contiguous in
    // LDS.  Lane l takes row tr = 4i + l/16 and source chunk (l%16) ^ swz(tr),
    // so LDS chunk c of row tr holds global chunk c ^ swz(tr): the MFMA operand
    // reads below are bank-conflict free without padding.  Rows at or past
    // tok_end repeat row tok_end-1 (their scores are masked).
    const uint32_t lds0 = static_cast<uint32_t>(
        (uintptr_t)((__attribute__((address_space(3))) unsigned char*)(lds)));
    const uint32_t wave_lds = lds0 + static_cast<uint32_t>(wave) * kDecWaveBytes;
    auto issue_sub = [&](int k, int sub) {
        const int t0 = tok_begin + kDecSubTok * sub;
        const uint32_t kb = wave_lds + (k % kDecWaveStages) * 2 * kDecSubBytes;
        const uint32_t vb = kb + kDecSubBytes;
        const uint16_t* kbase = kh + static_cast<int64_t>(t0) * kHeadDim;
        const uint16_t* vbase = vh + static_cast<int64_t>(t0) * kHeadDim;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tr = 4 * i + (lane >> 4);
            const int tok = min(t0 + tr, tok_end - 1);  // t0 < tok_end: offset stays >= 0
            const uint32_t off = static_cast<uint32_t>(tok - t0) * 256u + 16u * ((lane & 15) ^ dec_swz(tr));
            dec_lds_dma16(kbase, off, kb + 1024u * i);
            dec_lds_dma16(vbase, off, vb + 1024u * i);
        }
    };

#pragma unroll
    for (int k = 0; k < kDecWaveStages; ++k)
        if (k < n_first) issue_sub(k, wave + kDecWaves * k);
    // Wave 0's prologue copies are older than its sub-chunk copies (8 each).
    if (wave == 0) {
        const int later = n_first;
        if (later >= 4) {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(32));
        } else if (later == 3) {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(24));
        } else if (later == 2) {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(16));
        } else if (later == 1) {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(8));
        } else {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(0));
        }
    }

    // The split holding the new position (fused form) leaves the rotated K
    // row in `pro` row G (over the raw one) next to the V row (row G+1); the
    // wavefront whose sub-chunk holds the position patches both into its
    // stage once the copy of that sub-chunk has landed.
    const bool owns_new_row = kFused && (tok_end == s_kv) && (tok_begin < tok_end) &&
                              pos_raw < static_cast<uint32_t>(a.max_seq_len);
    if constexpr (kFused) {
        if (tid < 64) {
            // f32 angle as the reference computes it; sin/cos correctly
            // rounded to f32 via f64 (as qk_norm_rope_kv_kernel).
            const float inv_f = *reinterpret_cast<const float*>(pro + (G + 4) * 256 + 4 * tid);
            const float theta = static_cast<float>(static_cast<int>(pos_raw)) * inv_f;
            double sv, cv;
            sincos(static_cast<double>(theta), &sv, &cv);
            s_cos[tid] = static_cast<float>(cv);
            s_sin[tid] = static_cast<float>(sv);
        }
        lds_barrier();  // also publishes `pro`
        const int row = tid >> 3, lane8 = tid & 7;
        const bool do_q = row < G;
        const bool do_k = row == G && owns_new_row;
        if (do_q || do_k) {
            const unsigned char* x = pro + row * 256;
            const unsigned char* w = pro + (do_q ? G + 2 : G + 3) * 256;
            half8_t ylo, yhi;
            norm_rope_row8(*reinterpret_cast<const half8_t*>(x + 16 * lane8),
                           *reinterpret_cast<const half8_t*>(x + 128 + 16 * lane8),
                           *reinterpret_cast<const half8_t*>(w + 16 * lane8),
                           *reinterpret_cast<const half8_t*>(w + 128 + 16 * lane8), s_cos, s_sin,
                           a.eps, lane8, ylo, yhi);
            if (do_q) {
                *reinterpret_cast<half8_t*>(q_lds + row * kHeadDim + 8 * lane8) = ylo;
                *reinterpret_cast<half8_t*>(q_lds + row * kHeadDim + 64 + 8 * lane8) = yhi;
                if (split == 0) {
                    uint16_t* qo = a.q_out + static_cast<int64_t>(kvh * G + row) * kHeadDim;
                    store_half8(qo + 8 * lane8, ylo);
                    store_half8(qo + 64 + 8 * lane8, yhi);
                }
            } else {
                const unsigned char* vsrc = pro + (G + 1) * 256;
                const half8_t vlo = *reinterpret_cast<const half8_t*>(vsrc + 16 * lane8);
                const half8_t vhi = *reinterpret_cast<const half8_t*>(vsrc + 128 + 16 * lane8);
                // Each of these 8 lanes overwrites exactly the 32 B it read.
                *reinterpret_cast<half8_t*>(pro + G * 256 + 16 * lane8) = ylo;
                *reinterpret_cast<half8_t*>(pro + G * 256 + 128 + 16 * lane8) = yhi;
                const int64_t slot = (static_cast<int64_t>(kvh) * a.max_seq_len + pos) * kHeadDim;
                store_half8(a.k_cache_w + slot + 8 * lane8, ylo);
                store_half8(a.k_cache_w + slot + 64 + 8 * lane8, yhi);
                store_half8(a.v_cache_w + slot + 8 * lane8, vlo);
                store_half8(a.v_cache_w + slot + 64 + 8 * lane8, vhi);
            }
        }
        lds_barrier();
    } else {
        lds_barrier();  // publishes `pro`
    }

    // Q^T as the B operand: lane holds head n, dims 32c + 8*qgrp + [0,8).
    half8_t qop[4];
    {
        const half_t* qsrc = kFused ? q_lds : reinterpret_cast<const half_t*>(pro);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            qop[c] = (n < G) ? *reinterpret_cast<const half8_t*>(qsrc + n * kHeadDim + 32 * c + 8 * qgrp)
                             : half8_t{};
    }
    // Sub-chunk and row of the new position (owner split only).
    const int pos_local = static_cast<int>(pos) - tok_begin;
    const int sub_pos = owns_new_row ? pos_local / kDecSubTok : -1;
    const int tr_pos = pos_local % kDecSubTok;

    float m = kNegBig;
    float l = 0.0f;
    float4_t acc[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[db] = float4_t{0.f, 0.f, 0.f, 0.f};

    // Per-lane LDS read offsets within a stage (swizzled rows).  K (A operand
    // of S^T = K Q^T): token row n, global chunk 4cc + qgrp.  V^T (A operand
    // of O^T += V^T P^T, transposing read; 16-lane group qgrp, lane n): token
    // row 4qgrp + n/4, dims 16db + 4(n%4), i.e. 16-byte chunk 2db + (n%4)/2,
    // half 8*(n%2).
    uint32_t k_off[4], v_off[8];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) k_off[cc] = n * 256 + 16 * ((4 * cc + qgrp) ^ dec_swz(n));
    {
        const int tr = 4 * qgrp + (n >> 2);
#pragma unroll
        for (int db = 0; db < 8; ++db)
            v_off[db] = kDecSubBytes + tr * 256 + 16 * ((2 * db + ((n & 3) >> 1)) ^ dec_swz(tr)) + 8 * (n & 1);
    }

    for (int k = 0; k < nk; ++k) {
        // Sub-chunk k has landed once only the copies of this wavefront's later
        // sub-chunks (8 each, up to kDecWaveStages - 1 of them) are outstanding.
        const int younger = min(kDecWaveStages - 1, nk - 1 - k);
        if (younger >= 3) {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(24));
        } else if (younger == 2) {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(16));
        } else if (younger == 1) {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(8));
        } else {
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(0));
        }
        const int cur = wave + kDecWaves * k;
        unsigned char* kb = lds + wave * kDecWaveBytes + (k % kDecWaveStages) * 2 * kDecSubBytes;
        if (cur == sub_pos) {
            // The copy read the cache before the new row was stored: lanes
            // 0-15 put the rotated K row, lanes 16-31 the V row into row
            // tr_pos (swizzled).  A wavefront's LDS accesses complete in order.
            if (lane < 32) {
                const int j = lane & 15;
                const half8_t x = *reinterpret_cast<const half8_t*>(pro + (G + (lane >> 4)) * 256 + 16 * j);
                *reinterpret_cast<half8_t*>(kb + (lane >> 4) * kDecSubBytes + tr_pos * 256 +
                                            16 * (j ^ dec_swz(tr_pos))) = x;
            }
        }

        // All LDS operands of the sub-chunk first: once they have arrived the
        // stage takes the wavefront's sub-chunk k + kDecWaveStages, so the copy
        // goes out before the MFMA and softmax chain instead of after it.
        half8_t ka[4];
        half4_t va[8];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) ka[cc] = *reinterpret_cast<const half8_t*>(kb + k_off[cc]);
#pragma unroll
        for (int db = 0; db < 8; ++db) va[db] = lds_read_tr16(reinterpret_cast<const half_t*>(kb + v_off[db]));
        if (k + kDecWaveStages < nk) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue_sub(k + kDecWaveStages, cur + kDecWaves * kDecWaveStages);
        }

        const int t = tok_begin + kDecSubTok * cur;  // first token
        // S^T[token, head]: lane holds head n, tokens t + 4qgrp + r.
        float4_t s = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) s = mfma16x16x32(ka[cc], qop[cc], s);
        float mx = kNegBig;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = t + 4 * qgrp + r;
            const float x = (tok < tok_end) ? s[r] * a.scale_log2 : kNegBig;
            s[r] = x;
            mx = fmaxf(mx, x);
        }
        mx = fmaxf(mx, swap_rows16(mx));
        mx = fmaxf(mx, swap_halves(mx));
        // Lazy rescale: the running max m moves only when a score exceeds it
        // by more than kDecRescaleSlack, so p = 2^(s - m) <= 2^8 stays well
        // inside f16; the (rare) rescale is the only VALU work on acc.
        if (__any(mx > m + kDecRescaleSlack)) {
            const float m_new = fmaxf(m, mx);
            const float alpha = __builtin_amdgcn_exp2f(m - m_new);
            l *= alpha;
#pragma unroll
            for (int db = 0; db < 8; ++db) acc[db] *= alpha;
            m = m_new;
        }
        float psum = 0.0f;
        half4_t pop;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float p = __builtin_amdgcn_exp2f(s[r] - m);
            psum += p;
            pop[r] = static_cast<half_t>(p);
        }
        l += psum;
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[db] = mfma16x16x16(va[db], pop, acc[db]);
    }

    // Combine the wavefronts: per head M = max m_w, L = sum l_w 2^(m_w-M),
    // O = sum acc_w 2^(m_w-M) / max(L, 1e-8).
    l += swap_rows16(l);
    l += swap_halves(l);
    lds_barrier();  // stage buffers are reused for the combine
    float* red = reinterpret_cast<float*>(lds) + wave * kDecRedStride;
    if (qgrp == 0) {
        red[16 * kDecRedRow + n] = m;
        red[16 * kDecRedRow + 16 + n] = l;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db)
        *reinterpret_cast<float4_t*>(red + n * kDecRedRow + 16 * db + 4 * qgrp) = acc[db];
    lds_barrier();

    {
        const int g = tid >> 4;        // head handled by this thread
        const int d0 = (tid & 15) * 8; // 8 output dims
        if (g < G) {
            const float* base = reinterpret_cast<const float*>(lds);
            float M = kNegBig;
#pragma unroll
            for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, base[w * kDecRedStride + 16 * kDecRedRow + g]);
            float L = 0.0f, f[kDecWaves];
#pragma unroll
            for (int w = 0; w < kDecWaves; ++w) {
                f[w] = __builtin_amdgcn_exp2f(base[w * kDecRedStride + 16 * kDecRedRow + g] - M);
                L += base[w * kDecRedStride + 16 * kDecRedRow + 16 + g] * f[w];
            }
            const float l_safe = fmaxf(L, 1.0e-8f);
            const float inv_l = 1.0f / l_safe;
            half8_t o;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float x = 0.0f;
#pragma unroll
                for (int w = 0; w < kDecWaves; ++w) x += base[w * kDecRedStride + g * kDecRedRow + d0 + e] * f[w];
                o[e] = static_cast<half_t>(x * inv_l);
            }
            const int64_t prow = (static_cast<int64_t>(kvh) * a.num_splits + split) * G + g;
            const float lse_v = M + log2f(l_safe);
            if constexpr (kFused) {
                store16_agent(a.att_partial + prow * kHeadDim + d0, o);
                if (d0 == 0)
                    __hip_atomic_store(a.lse_partial + prow, lse_v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                store_half8(a.att_partial + prow * kHeadDim + d0, o);
                if (d0 == 0) a.lse_partial[prow] = lse_v;
            }
        }
    }

    if constexpr (kFused) {
        // Last workgroup of this KV head merges its splits.  Every partial is
        // complete at the coherence point (sc1 stores, vmcnt(0)) before this
        // workgroup's counter increment; the merging workgroup reads them with
        // sc1 loads after its own increment returned the final count.
        __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(0));
        lds_barrier();
        uint32_t head_ticket = 0xffffffffu;
        if (tid == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(&a.counters[kvh * kDecCounterStride], 1u, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT);
            uint32_t flag = 0;
            if (prev + 1 == static_cast<uint32_t>(a.num_splits)) {
                flag = 1;
                // This head is complete: reset its counter for the next launch.
                __hip_atomic_store(&a.counters[kvh * kDecCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                // Position advance: every workgroup of every head read the
                // position before its head increment, so the merger of the
                // last head to complete may store position+1.  The head count
                // is only read after the merge; its latency overlaps the
                // merge's own round trip.
                if (a.advance_position)
                    head_ticket = __hip_atomic_fetch_add(&a.counters[a.num_kv_heads * kDecCounterStride], 1u,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            s_flag = flag;
        }
        lds_barrier();
        if (s_flag == 0) return;

        // Merge of this KV head: O[g] = sum_s w_s O_s[g] / sum_s w_s with
        // w_s = 2^(lse_s - M), the combination of attn_decode_merge_kernel.
        // The head's partial rows are contiguous (row s*G + g); batches of up
        // to kMergeRows rows go straight into the free stage buffers with
        // device-coherent (sc1) copies, and their LSEs arrive with sc1 dword
        // loads into a transposed [g][split] table (padded with -1e30), one
        // memory round trip per batch.  Thread t owns row g = it/32 and dims
        // 4(it%32)..+3 for it = t, t+256 (G <= 16); per 32 splits it reads
        // its LSEs as 16-byte vectors, then accumulates with independent
        // LDS reads, keeping an online (max, sum, acc) across chunks.
        constexpr int kMergeRows = kDecMergeRows;
        static_assert(kMergeRows * 256 <= kDecFusedLdsBytes, "merge batch must fit the LDS buffer");
        static_assert(GROUT_MAX_DECODE_GROUP * 32 <= 2 * kDecThreads, "two merge items per thread");
        // LSE table: G rows of SBp <= kMergeRows / G + 31 entries (16-byte
        // aligned rows: the sums read them as float4).
        __shared__ __attribute__((aligned(16))) float lse_tab[kMergeRows + 31 * GROUT_MAX_DECODE_GROUP];
        const int NS = a.num_splits;
        const int SB = kMergeRows / G;        // splits per batch
        const int SBp = (SB + 31) & ~31;      // row length of the LSE table
        const uint16_t* part_h = a.att_partial + static_cast<int64_t>(kvh) * NS * G * kHeadDim;
        const float* lse_h = a.lse_partial + static_cast<int64_t>(kvh) * NS * G;
        const unsigned char* rows_l = lds;
        float* lse_t = lse_tab;
        // One batch of up to kMergeRows partial rows: rows into the stages,
        // LSEs into the [g][split] table (padded with -1e30 to SBp).
        auto load_batch = [&](int s0, int ns_b) {
            const int rows = ns_b * G;
            const uint16_t* src = part_h + static_cast<int64_t>(s0) * G * kHeadDim;
            // Copy i moves rows 4i..4i+3 (lane l: row 4i + l/16, 16-byte chunk
            // l%16) to LDS byte 1024i + 16l; pad lanes re-read the last row.
            const int ncopies = (rows + 3) / 4;
            for (int i = wave; i < ncopies; i += kDecWaves) {
                const int r = min(4 * i + (lane >> 4), rows - 1);
                dec_lds_dma16_ptr_sc1(src + static_cast<int64_t>(r) * kHeadDim + 8 * (lane & 15), lds0 + 1024u * i);
            }
            for (int i = tid; i < G * SBp; i += kDecThreads) {
                const int g = i / SBp, sp = i - g * SBp;
                float v = kNegBig;
                if (sp < ns_b)
                    v = __hip_atomic_load(lse_h + static_cast<int64_t>(s0 + sp) * G + g, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
                lse_t[i] = v;
            }
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(0));
            lds_barrier();
        };
        if (NS <= SB && NS <= 64) {
            // All splits in one batch: the weights w_s = 2^(lse_s - M) of a
            // query row are computed once, by one 32-lane half per row (split
            // s at lane s%32, s/32 its slot), into the [g][split] table;
            // then each thread sums its 4 dims over the splits.
            //
            // When the head's NS*G LSEs fill whole 16-byte chunks at a
            // 16-byte aligned address, wave 0 first copies them as stored
            // ([split][g], sc1) into `pro`, free since the stream ended, and
            // only then do the waves copy the partial rows.  Wave 0 waits for
            // the LSE copies alone, so the weights are computed while the rows
            // are still landing.
            const int rows = NS * G;
            const bool lse_first = (rows & 3) == 0 && (reinterpret_cast<uintptr_t>(lse_h) & 15) == 0;
            static_assert(kMergeRows * 4 <= kDecProDmas * 1024, "LSE block (rows <= kMergeRows) must fit `pro`");
            const float* lse_raw = reinterpret_cast<const float*>(pro);
            if (lse_first) {
                if (wave == 0) {
                    // Copy i moves LSEs 256i + [0, 256); lanes past the end
                    // re-read the last chunk into slots past the table.
                    for (int i = 0; i < (rows + 255) / 256; ++i)
                        dec_lds_dma16_ptr_sc1(lse_h + min(256 * i + 4 * lane, rows - 4), pro0 + 1024u * i);
                }
                const int ncopies = rows / 4;
                for (int i = wave; i < ncopies; i += kDecWaves)
                    dec_lds_dma16_ptr_sc1(part_h + static_cast<int64_t>(4 * i + (lane >> 4)) * kHeadDim + 8 * (lane & 15),
                                          lds0 + 1024u * i);
                // Wave 0's row copies (at most kMergeRows / 16 = 32) are younger
                // than its LSE copies.
                static_assert(kMergeRows / 16 <= 32, "row copies per wave within the wait");
                if (wave == 0) dec_wait_vm_atmost<32>((ncopies + kDecWaves - 1) / kDecWaves);
                lds_barrier();
            } else {
                load_batch(0, NS);
            }
            for (int gi = tid >> 5; gi < G; gi += kDecThreads / 32) {
                const int l = tid & 31;
                float* lrow = lse_t + gi * SBp;
                float v0, v1;
                if (lse_first) {
                    v0 = l < NS ? lse_raw[l * G + gi] : kNegBig;
                    v1 = l + 32 < NS ? lse_raw[(l + 32) * G + gi] : kNegBig;
                } else {
                    v0 = lrow[l];
                    v1 = NS > 32 ? lrow[32 + l] : kNegBig;
                }
                const float mx = half32_reduce(fmaxf(v0, v1), [](float x, float y) { return fmaxf(x, y); });
                const float w0 = __builtin_amdgcn_exp2f(v0 - mx);
                const float w1 = NS > 32 ? __builtin_amdgcn_exp2f(v1 - mx) : 0.0f;
                const float sw = half32_reduce(w0 + w1, [](float x, float y) { return x + y; });
                lrow[l] = w0;
                if (NS > 32) lrow[32 + l] = w1;
                if (l == 0) s_wsum[gi] = sw;
            }
            __builtin_amdgcn_s_waitcnt(dec_waitcnt_vm(0));
            lds_barrier();
            if (G * 64 <= kDecThreads) {
                // G <= 4: thread t sums row g = t/64, dims 2(t%64)..+1, so all
                // 256 threads share the rows (items of 4 dims would leave half
                // of them idle).  Same per-element sums as below.
                if (tid < G * 64) {
                    const int g = tid >> 6, c = tid & 63;
                    const float* wrow = lse_t + g * SBp;
                    const unsigned char* rbase = rows_l + g * 256 + 4 * c;
                    const int xstride = G * 256;
                    float acc2[2] = {0.f, 0.f};
                    for (int sc = 0; sc < NS; sc += 32) {
                        if (NS - sc >= 32) {
                            const unsigned char* xb = rbase + sc * xstride;
                            half2_t xs[32];
#pragma unroll
                            for (int u = 0; u < 32; ++u)
                                xs[u] = *reinterpret_cast<const half2_t*>(xb + u * xstride);
                            float wv[32];
#pragma unroll
                            for (int u = 0; u < 8; ++u) {
                                const float4_t w4 = *reinterpret_cast<const float4_t*>(wrow + sc + 4 * u);
#pragma unroll
                                for (int e = 0; e < 4; ++e) wv[4 * u + e] = w4[e];
                            }
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int u = 0; u < 32; ++u)
#pragma unroll
                                for (int e = 0; e < 2; ++e) acc2[e] += wv[u] * static_cast<float>(xs[u][e]);
                        } else {
                            for (int u = sc; u < NS; ++u) {
                                const float w = wrow[u];
                                const half2_t x = *reinterpret_cast<const half2_t*>(rbase + u * xstride);
#pragma unroll
                                for (int e = 0; e < 2; ++e) acc2[e] += w * static_cast<float>(x[e]);
                            }
                        }
                    }
                    const float inv = 1.0f / fmaxf(s_wsum[g], 1.0e-8f);
                    half2_t h;
#pragma unroll
                    for (int e = 0; e < 2; ++e) h[e] = static_cast<half_t>(acc2[e] * inv);
                    *reinterpret_cast<half2_t*>(a.out + (static_cast<int64_t>(kvh) * G + g) * kHeadDim + 2 * c) = h;
                }
            } else {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int it = tid + kDecThreads * k;
                if (it < G * 32) {
                    const int g = it >> 5, c = it & 31;
                    const float* wrow = lse_t + g * SBp;
                    const unsigned char* rbase = rows_l + g * 256 + 8 * c;
                    float acc4[4] = {0.f, 0.f, 0.f, 0.f};
                    for (int sc = 0; sc < NS; sc += 32) {
                        if (NS - sc >= 32) {
                            const unsigned char* xb = rbase + sc * G * 256;
                            const int xstride = G * 256;
                            half4_t xs[32];
#pragma unroll
                            for (int u = 0; u < 32; ++u)
                                xs[u] = *reinterpret_cast<const half4_t*>(xb + u * xstride);
                            float wv[32];
#pragma unroll
                            for (int u = 0; u < 8; ++u) {
                                const float4_t w4 = *reinterpret_cast<const float4_t*>(wrow + sc + 4 * u);
#pragma unroll
                                for (int e = 0; e < 4; ++e) wv[4 * u + e] = w4[e];
                            }
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int u = 0; u < 32; ++u)
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc4[e] += wv[u] * static_cast<float>(xs[u][e]);
                        } else {
                            for (int u = sc; u < NS; ++u) {
                                const float w = wrow[u];
                                const half4_t x = *reinterpret_cast<const half4_t*>(rbase + u * G * 256);
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc4[e] += w * static_cast<float>(x[e]);
                            }
                        }
                    }
                    const float inv = 1.0f / fmaxf(s_wsum[g], 1.0e-8f);
                    half4_t h;
#pragma unroll
                    for (int e = 0; e < 4; ++e) h[e] = static_cast<half_t>(acc4[e] * inv);
                    *reinterpret_cast<half4_t*>(a.out + (static_cast<int64_t>(kvh) * G + g) * kHeadDim + 4 * c) = h;
                }
            }
            }  // G > 4
        } else {
        float m_i[2] = {-INFINITY, -INFINITY}, s_i[2] = {0.0f, 0.0f};
        float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        for (int s0 = 0; s0 < NS; s0 += SB) {
            const int ns_b = min(SB, NS - s0);
            load_batch(s0, ns_b);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int it = tid + kDecThreads * k;
                if (it < G * 32) {
                    const int g = it >> 5, c = it & 31;
                    const float* lrow = lse_t + g * SBp;
                    const unsigned char* rbase = rows_l + g * 256 + 8 * c;
                    for (int sc = 0; sc < ns_b; sc += 32) {
                        float lv[32];
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            const float4_t v4 = *reinterpret_cast<const float4_t*>(lrow + sc + 4 * u);
#pragma unroll
                            for (int e = 0; e < 4; ++e) lv[4 * u + e] = v4[e];
                        }
                        float mb = m_i[k];
#pragma unroll
                        for (int u = 0; u < 32; ++u) mb = fmaxf(mb, lv[u]);
                        const float r = (m_i[k] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_i[k] - mb);
                        s_i[k] *= r;
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[k][e] *= r;
                        m_i[k] = mb;
                        const int nu = min(32, ns_b - sc);
                        if (nu == 32) {
                            // All 32 row reads are issued before the arithmetic
                            // (the fence keeps them together), so the chunk
                            // pays one LDS latency instead of one per split.
                            const unsigned char* xb = rbase + sc * G * 256;
                            const int xstride = G * 256;
                            half4_t xs[32];
#pragma unroll
                            for (int u = 0; u < 32; ++u)
                                xs[u] = *reinterpret_cast<const half4_t*>(xb + u * xstride);
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int u = 0; u < 32; ++u) {
                                const float w = __builtin_amdgcn_exp2f(lv[u] - mb);
                                s_i[k] += w;
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[k][e] += w * static_cast<float>(xs[u][e]);
                            }
                        } else {
                            for (int u = 0; u < nu; ++u) {
                                const float w = __builtin_amdgcn_exp2f(lv[u] - mb);
                                s_i[k] += w;
                                const half4_t x = *reinterpret_cast<const half4_t*>(rbase + (sc + u) * G * 256);
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[k][e] += w * static_cast<float>(x[e]);
                            }
                        }
                    }
                }
            }
            lds_barrier();  // the next batch overwrites the rows
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int it = tid + kDecThreads * k;
            if (it < G * 32) {
                const int g = it >> 5, c = it & 31;
                const float inv = 1.0f / fmaxf(s_i[k], 1.0e-8f);
                half4_t h;
#pragma unroll
                for (int e = 0; e < 4; ++e) h[e] = static_cast<half_t>(acc[k][e] * inv);
                *reinterpret_cast<half4_t*>(a.out + (static_cast<int64_t>(kvh) * G + g) * kHeadDim + 4 * c) = h;
            }
        }
        }  // batched merge
        if (tid == 0 && head_ticket == static_cast<uint32_t>(a.num_kv_heads) - 1u) {
            __hip_atomic_store(&a.counters[a.num_kv_heads * kDecCounterStride], 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            // The position saturates at max_seq_len: a step at or past the end
            // of the cache wrote no row and does not move it further.
            if (pos_raw < static_cast<uint32_t>(a.max_seq_len))
                __hip_atomic_store(a.position_w, pos_raw + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Standalone merge: one workgroup of 64 lanes per (head, kv_head); split
// weights are staged in LDS, then each lane accumulates two output dims.
__global__ __launch_bounds__(kWave) void attn_decode_merge_kernel(
    const uint16_t* __restrict__ att, const float* __restrict__ lse, uint16_t* __restrict__ out,
    int group, int num_splits) {
    __shared__ float w_lds[GROUT_MAX_DECODE_SPLITS];
    const int g = blockIdx.x;
    const int kvh = blockIdx.y;
    const int lane = threadIdx.x;
    const float* L = lse + static_cast<int64_t>(kvh) * num_splits * group;

    float mx = -INFINITY;
    for (int s = lane; s < num_splits; s += kWave) mx = fmaxf(mx, L[s * group + g]);
    mx = wave_max(mx);
    float sum = 0.0f;
    for (int s = lane; s < num_splits; s += kWave) {
        const float e = exp2f(L[s * group + g] - mx);
        w_lds[s] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    const float safe = fmaxf(sum, 1.0e-8f);
    __syncthreads();

    float acc0 = 0.0f, acc1 = 0.0f;
    const uint16_t* base = att + (static_cast<int64_t>(kvh) * num_splits * group + g) * kHeadDim + 2 * lane;
#pragma unroll 8
    for (int s = 0; s < num_splits; ++s) {
        const float w = w_lds[s] / safe;
        const uint32_t pair = *reinterpret_cast<const uint32_t*>(base + static_cast<int64_t>(s) * group * kHeadDim);
        acc0 += static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(pair & 0xffffu))) * w;
        acc1 += static_cast<float>(__builtin_bit_cast(half_t, static_cast<uint16_t>(pair >> 16))) * w;
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

static int32_t check_attention_args(const uint16_t* k_cache, const uint16_t* v_cache,
                                    const uint16_t* att_partial, const float* lse_partial,
                                    const uint32_t* d_position, int32_t num_kv_heads,
                                    int32_t group, int32_t head_dim, int32_t max_seq_len,
                                    int32_t block_n, int32_t num_splits, uint16_t qk_scale_f16) {
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
    return GROUT_OK;
}

extern "C" int32_t grout_attn_decode_split(const uint16_t* q, const uint16_t* k_cache,
                                           const uint16_t* v_cache, uint16_t* att_partial,
                                           float* lse_partial, uint16_t qk_scale_f16,
                                           const uint32_t* d_position, int32_t num_kv_heads,
                                           int32_t group, int32_t head_dim, int32_t max_seq_len,
                                           int32_t block_n, int32_t num_splits,
                                           grout_stream_t stream) {
    GROUT_REQUIRE_PTR(q);
    const int32_t st = check_attention_args(k_cache, v_cache, att_partial, lse_partial, d_position,
                                            num_kv_heads, group, head_dim, max_seq_len, block_n,
                                            num_splits, qk_scale_f16);
    if (st != GROUT_OK) return st;
    DecodeArgs a = {};
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.att_partial = att_partial;
    a.lse_partial = lse_partial;
    // src/kernels.rs:2618-2622: qk_scale_f32 / ln(2), both f32.
    a.scale_log2 = f16_bits_to_f32(qk_scale_f16) / logf(2.0f);
    a.group = group;
    a.num_kv_heads = num_kv_heads;
    a.max_seq_len = max_seq_len;
    a.block_n = block_n;
    a.num_splits = num_splits;
    hipLaunchKernelGGL(attn_decode_kernel<false>, dim3(num_splits, num_kv_heads), dim3(kDecThreads),
                       0, to_hip(stream), d_position, a);
    return launch_status();
}

static int32_t fused_decode(
    const uint16_t* qkv, const uint16_t* q_weight, const uint16_t* k_weight,
    const float* inv_freq, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
    uint16_t* att_partial, float* lse_partial, uint16_t* out, uint32_t* counters,
    uint32_t* d_position, float eps, uint16_t qk_scale_f16, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len, int32_t block_n,
    int32_t num_splits, int32_t advance_position, grout_stream_t stream) {
    GROUT_REQUIRE_PTR(qkv);
    GROUT_REQUIRE_PTR(q_weight);
    GROUT_REQUIRE_PTR(k_weight);
    GROUT_REQUIRE_PTR(inv_freq);
    GROUT_REQUIRE_PTR(q_out);
    GROUT_REQUIRE_PTR(out);
    GROUT_REQUIRE(counters != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(counters) & 3u) == 0, GROUT_ERR_ALIGNMENT);
    GROUT_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
                  GROUT_ERR_HEADS);
    GROUT_REQUIRE(eps >= 0.0f && eps < 1.0e30f, GROUT_ERR_ARG);
    const int32_t group = num_q_heads / num_kv_heads;
    const int32_t st = check_attention_args(k_cache, v_cache, att_partial, lse_partial, d_position,
                                            num_kv_heads, group, head_dim, max_seq_len, block_n,
                                            num_splits, qk_scale_f16);
    if (st != GROUT_OK) return st;
    DecodeArgs a = {};
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.att_partial = att_partial;
    a.lse_partial = lse_partial;
    a.scale_log2 = f16_bits_to_f32(qk_scale_f16) / logf(2.0f);
    a.group = group;
    a.num_kv_heads = num_kv_heads;
    a.max_seq_len = max_seq_len;
    a.block_n = block_n;
    a.num_splits = num_splits;
    a.qkv = qkv;
    a.q_weight = q_weight;
    a.k_weight = k_weight;
    a.inv_freq = inv_freq;
    a.q_out = q_out;
    a.k_cache_w = k_cache;
    a.v_cache_w = v_cache;
    a.out = out;
    a.counters = counters;
    a.position_w = d_position;
    a.eps = eps;
    a.num_q_heads = num_q_heads;
    a.advance_position = advance_position != 0;
    hipLaunchKernelGGL(attn_decode_kernel<true>, dim3(num_splits, num_kv_heads), dim3(kDecThreads),
                       0, to_hip(stream), d_position, a);
    return launch_status();
}

extern "C" int32_t grout_attn_decode_fused(
    const uint16_t* qkv, const uint16_t* q_weight, const uint16_t* k_weight,
    const float* inv_freq, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
    uint16_t* att_partial, float* lse_partial, uint16_t* out, uint32_t* counters,
    uint32_t* d_position, float eps, uint16_t qk_scale_f16, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len, int32_t block_n,
    int32_t num_splits, int32_t advance_position, grout_stream_t stream) {
    return fused_decode(qkv, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache, att_partial,
                        lse_partial, out, counters, d_position, eps, qk_scale_f16, num_q_heads,
                        num_kv_heads, head_dim, max_seq_len, block_n, num_splits,
                        advance_position, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free fused decode: the same kernel with its split partials, LSEs
// and merge counters in a static device array instead of caller buffers.
//
// Layout of `scratch`: [0, 64 KiB) merge counters (kDecCounterStride apart, one
// 256-byte line per KV head plus the head counter), then the LSEs (f32, one
// per (kv_head, split, g) row), then the partial rows (f16, 256 B each) from
// the next 256-byte boundary.
constexpr size_t kNoAllocBytes = static_cast<size_t>(GROUT_NOALLOC_SCRATCH_BYTES);
constexpr size_t kNoAllocCounterBytes = 64 * 1024;
static_assert(kNoAllocCounterBytes ==
                  static_cast<size_t>(GROUT_NOALLOC_MAX_KV_HEADS + 1) * kDecCounterStride * 4,
              "one counter line per KV head plus the head counter");
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {

// Per-device address of `scratch` (the name is only a host-side stand-in):
// looked up with that device current, then used for every kernel argument.
// A device counts as set up only once the lookup has succeeded, so a failed
// set-up is tried again by the next call.  Nothing is written to the array
// at set-up: static device storage is zero when the code object is loaded,
// and every launch leaves the merge counters zero again.
struct NoAllocDevice {
    std::mutex mu;
    unsigned char* ptr = nullptr;  // non-null once set up
};
constexpr int kNoAllocMaxDevices = 64;
NoAllocDevice g_noalloc[kNoAllocMaxDevices];

}  // namespace

extern "C" int32_t grout_attn_decode_fused_noalloc(
    const uint16_t* qkv, const uint16_t* q_weight, const uint16_t* k_weight,
    const float* inv_freq, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, uint16_t* out,
    uint32_t* d_position, float eps, uint16_t qk_scale_f16, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len, int32_t block_n,
    int32_t num_splits, int32_t advance_position, grout_stream_t stream) {
    GROUT_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
                  GROUT_ERR_HEADS);
    GROUT_REQUIRE(num_splits >= 1 && num_splits <= GROUT_MAX_DECODE_SPLITS, GROUT_ERR_SPLITS);
    GROUT_REQUIRE(num_kv_heads <= GROUT_NOALLOC_MAX_KV_HEADS, GROUT_ERR_SCRATCH);
    const int64_t rows = static_cast<int64_t>(num_q_heads) * num_splits;  // Hkv * NS * G
    const int64_t lse_bytes = (rows * 4 + 255) & ~static_cast<int64_t>(255);
    const int64_t need = static_cast<int64_t>(kNoAllocCounterBytes) + lse_bytes + rows * kHeadDim * 2;
    GROUT_REQUIRE(need <= static_cast<int64_t>(kNoAllocBytes), GROUT_ERR_SCRATCH);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int32_t>(e);
    GROUT_REQUIRE(dev >= 0 && dev < kNoAllocMaxDevices, GROUT_ERR_SCRATCH);
    NoAllocDevice& d = g_noalloc[dev];
    unsigned char* base = nullptr;
    {
        std::lock_guard<std::mutex> lock(d.mu);
        if (d.ptr == nullptr) {
            // The first call on a device must not run under stream capture:
            // the symbol lookup is not a stream operation and has no place
            // in a graph.  The caller makes one call before capturing.
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            e = hipStreamIsCapturing(to_hip(stream), &cs);
            if (e != hipSuccess) return static_cast<int32_t>(e);
            if (cs != hipStreamCaptureStatusNone) return GROUT_ERR_GRAPH;
            void* p = nullptr;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return static_cast<int32_t>(e);
            d.ptr = static_cast<unsigned char*>(p);
        }
        base = d.ptr;
    }
    uint32_t* counters = reinterpret_cast<uint32_t*>(base);
    float* lse = reinterpret_cast<float*>(base + kNoAllocCounterBytes);
    uint16_t* att = reinterpret_cast<uint16_t*>(base + kNoAllocCounterBytes + lse_bytes);
    return fused_decode(qkv, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache, att, lse, out,
                        counters, d_position, eps, qk_scale_f16, num_q_heads, num_kv_heads,
                        head_dim, max_seq_len, block_n, num_splits, advance_position, stream);
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

extern "C" int64_t grout_attn_decode_counter_bytes(int32_t num_kv_heads) {
    if (num_kv_heads <= 0) return GROUT_ERR_ARG;
    return static_cast<int64_t>(num_kv_heads + 1) * kDecCounterStride * 4;
}

extern "C" int32_t grout_attn_decode_pick_splits_grouped(int32_t cu_count, int32_t num_kv_heads,
                                                         int32_t group, int32_t max_context,
                                                         int32_t block_n) {
    if (cu_count <= 0) cu_count = 256;
    if (num_kv_heads <= 0 || block_n <= 0 || max_context <= 0) return 1;
    if (group <= 0) group = 1;
    // One workgroup per CU streaming at the longest context; a split shorter
    // than kDecMinSplitTokens spends more on its prologue and the merge than
    // it saves.
    const int64_t tiles = (static_cast<int64_t>(max_context) + block_n - 1) / block_n;
    const int64_t min_tiles = (kDecMinSplitTokens + block_n - 1) / block_n;
    int64_t want = (static_cast<int64_t>(cu_count) + num_kv_heads - 1) / num_kv_heads;
    // The fused merge loads NS * G partial rows through one CU per KV head:
    // keep them to one batch where that still keeps half the CUs streaming
    // (64 Q / 4 KV heads at 32K: 64 splits 21.9 us, 32 splits 20.3 us).
    const int64_t one_batch = kDecMergeRows / group;
    const int64_t half_cus = (static_cast<int64_t>(cu_count) / 2 + num_kv_heads - 1) / num_kv_heads;
    if (want > one_batch) want = one_batch > half_cus ? one_batch : half_cus;
    const int64_t cap = (tiles + min_tiles - 1) / min_tiles;
    if (want > cap) want = cap;
    if (want < 1) want = 1;
    if (want > GROUT_MAX_DECODE_SPLITS) want = GROUT_MAX_DECODE_SPLITS;
    return static_cast<int32_t>(want);
}

extern "C" int32_t grout_attn_decode_pick_splits(int32_t cu_count, int32_t num_kv_heads,
                                                 int32_t max_context, int32_t block_n) {
    return grout_attn_decode_pick_splits_grouped(cu_count, num_kv_heads, 1, max_context, block_n);
}

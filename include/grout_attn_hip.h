/*
 * grout_attn_hip.h — C ABI of the MI355X (gfx950) Qwen3 attention hot path.
 *
 * Drop-in for the attention ops of NikVisel/grout's Qwen3Engine: the fused
 * per-head Q/K RMSNorm + RoPE + KV-cache write, causal flash-attention
 * prefill, split-K GQA decode and its merge, and the hipGraph replay of the
 * decode step.  Every kernel is hand-written HIP for CDNA4; nothing here is
 * generated from the reference's cuTile code.
 *
 * Calling rules (all entry points):
 *  - Return int32_t: 0 = GROUT_OK, < 0 = argument validation failed (one
 *    code per reference `ensure!`, see grout_status_string), > 0 = the
 *    hipError_t of a failed launch.
 *  - Tensor pointers are borrowed device memory; f16 tensors are IEEE
 *    binary16 (passed as uint16_t*).  Every pointer must be 16-byte aligned.
 *  - Nothing is allocated or freed and nothing synchronises the host: every
 *    launch is asynchronous on `stream` (NULL = the default stream), so the
 *    decode entry points can be recorded into a hipGraph and replayed.
 *  - Functions are reentrant; kernels are compiled into this library.
 *  - Layouts are grout's: KV cache [num_kv_heads, max_seq_len, head_dim] f16
 *    row-major (src/model.rs:1450-1455); prefill Q/O [seq, num_q_heads,
 *    head_dim]; decode Q = the first num_q_heads*head_dim elements of q_out,
 *    viewed [num_kv_heads, group, head_dim]; decode out [num_kv_heads, group,
 *    head_dim] (== [1, num_q_heads, head_dim]).  head_dim must be 128, as
 *    grout's engine requires (src/model.rs:1327).
 *
 * Citations are to files of the upstream NikVisel/grout tree.
 */
#ifndef GROUT_ATTN_HIP_H
#define GROUT_ATTN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as hipStream_t (struct ihipStream_t*), declared without HIP headers. */
typedef struct ihipStream_t* grout_stream_t;

/* ----------------------------------------------------------- status codes */
enum {
    GROUT_OK = 0,
    GROUT_ERR_NULL_POINTER = -1,  /* a required pointer is NULL */
    GROUT_ERR_ALIGNMENT = -2,     /* a tensor pointer is not 16-byte aligned */
    GROUT_ERR_HEAD_DIM = -3,      /* head_dim != 128 (src/model.rs:1327, :4520-4524) */
    GROUT_ERR_HEADS = -4,         /* heads <= 0 or num_q_heads % num_kv_heads != 0 */
    GROUT_ERR_SEQ_RANGE = -5,     /* position_start + seq_len > max_seq_len (src/model.rs:4525-4531) */
    GROUT_ERR_KV_LEN = -6,        /* kv_len / query_start / q_len out of range */
    GROUT_ERR_GROUP = -7,         /* decode group outside [1, 16] */
    GROUT_ERR_SPLITS = -8,        /* num_splits or block_n out of range */
    GROUT_ERR_ARG = -9,           /* any other invalid scalar argument */
    GROUT_ERR_GRAPH = -10,        /* graph handle misuse */
    GROUT_ERR_SCRATCH = -11       /* the static scratch of a *_noalloc entry point is too small */
};

/* Human-readable text for a status code (static storage). */
const char* grout_status_string(int32_t status);

/* Limits of the decode kernels. */
#define GROUT_HEAD_DIM 128
#define GROUT_MAX_DECODE_GROUP 16
#define GROUT_MAX_DECODE_SPLITS 1024
#define GROUT_MAX_PREFILL_SPLITS 1024

/* -------------------------------------------------------------- RoPE table */
/* Replaces build_inv_freq (src/model.rs:5992-6003): host-side, f32,
 * out[j] = 1 / theta^((2j)/head_dim) for j < head_dim/2.  No device work. */
int32_t grout_build_inv_freq(float theta, int32_t head_dim, float* out_host);

/* --------------------------------------------- fused QK norm + RoPE + KV */
/* Replaces qk_norm_rope_kv_prefill_raw_f16 (src/kernels.rs:3415-3732) as
 * launched by execute_qk_norm_rope_kv_prefill_op_ctx (src/model.rs:4463-4598).
 *   q [seq_len, num_q_heads, 128], k/v [seq_len, num_kv_heads, 128] f16;
 *   q_weight/k_weight [128] f16; inv_freq [64] f32;
 *   q_out [seq_len, num_q_heads, 128] f16 (may not alias q);
 *   k_cache/v_cache [num_kv_heads, max_seq_len, 128] f16, rows
 *   [position_start, position_start+seq_len) written.
 * Per row: n = x * rsqrt(sum(x^2)/128 + eps) * w (f32); RoPE on halves
 * (j, j+64) at theta = f32(position_start+s) * inv_freq[j]; f16 RNE store.
 * V is copied bit-exactly. */
int32_t grout_qk_norm_rope_kv_prefill(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                      const uint16_t* q_weight, const uint16_t* k_weight,
                                      const float* inv_freq, uint16_t* q_out,
                                      uint16_t* k_cache, uint16_t* v_cache, float eps,
                                      int32_t position_start, int32_t seq_len,
                                      int32_t num_q_heads, int32_t num_kv_heads,
                                      int32_t head_dim, int32_t max_seq_len,
                                      grout_stream_t stream);

/* --------------------------------------------- fused decode variant */
/* Replaces qk_norm_rope_kv_decode_raw_f16 (src/kernels.rs:3750-4016) as
 * recorded in the decode graph (src/model.rs:3194-3221).
 *   qkv = the QKV GEMV output [Q(num_q_heads*128) | K(num_kv_heads*128) |
 *   V(num_kv_heads*128)] f16; q_out rows [0, num_q_heads) of a
 *   [num_q_heads+num_kv_heads, 128] buffer are written;
 *   *d_position (device u32) is the cache slot and the RoPE position.
 * A device position >= max_seq_len writes no cache slot (bounds guard). */
int32_t grout_qk_norm_rope_kv_decode(const uint16_t* qkv, const uint16_t* q_weight,
                                     const uint16_t* k_weight, const float* inv_freq,
                                     uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                                     const uint32_t* d_position, float eps,
                                     int32_t num_q_heads, int32_t num_kv_heads,
                                     int32_t head_dim, int32_t max_seq_len,
                                     grout_stream_t stream);

/* ------------------------------------------------- KV-cache suffix writer */
/* Replaces kv_cache_update_seq_f16 (src/kernels.rs:759-800) as launched by
 * kv_cache_update_seq_arc_ctx_with_position (src/model.rs:5464-5480): the
 * unfused KV write of chunked prefill and MTP suffixes.
 *   new_k/new_v [seq_len, num_kv_heads, head_dim] f16; cache rows
 *   [position_start, position_start+seq_len) of k_cache/v_cache
 *   [num_kv_heads, max_seq_len, head_dim] take them bit-exactly; every other
 *   row is untouched.  head_dim is any multiple of 4 (grout uses 128);
 *   pointers 16-byte aligned (8-byte when head_dim % 8 != 0). */
int32_t grout_kv_cache_update_seq(const uint16_t* new_k, const uint16_t* new_v,
                                  uint16_t* k_cache, uint16_t* v_cache, int32_t position_start,
                                  int32_t seq_len, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t max_seq_len, grout_stream_t stream);
/* Replaces kv_cache_update_seq_dynpos_f16 (src/kernels.rs:807-846), the
 * graph-captured form (src/model.rs:5483-5502): the start slot is the device
 * u32 *d_position.  A row whose slot falls at or past max_seq_len is not
 * written (bounds guard). */
int32_t grout_kv_cache_update_seq_dynpos(const uint16_t* new_k, const uint16_t* new_v,
                                         uint16_t* k_cache, uint16_t* v_cache,
                                         const uint32_t* d_position, int32_t seq_len,
                                         int32_t num_kv_heads, int32_t head_dim,
                                         int32_t max_seq_len, grout_stream_t stream);

/* -------------------------------------------------- causal prefill attention */
/* Replaces fmha_prefill_causal / fmha_prefill_gqa / fmha_prefill_gqa_lpt /
 * flash_attn_causal_seq_f16 (src/kernels.rs:1037-1862) as dispatched by
 * attend_seq_arc_into_ctx_with_position (src/model.rs:5638-5834).
 *   q [q_len, num_q_heads, 128] f16; K/V read from the caches
 *   [num_kv_heads, max_seq_len, 128] rows [0, kv_len) with row stride 128 and
 *   head stride max_seq_len*128 (the explicit cache stride avoids the
 *   kv_len*D head-stride assumption of src/kernels.rs:1559-1568);
 *   out [q_len, num_q_heads, 128] f16.
 * Query row m sits at position query_start+m and attends keys
 * n < min(kv_len, query_start+m+1); kv_head = q_head / (num_q_heads/num_kv_heads).
 * Softmax in base 2 with qk_scale/ln2 folded in, f32 accumulation, P rounded
 * to f16 for the PV product, out = f16(acc / max(l, 1e-8)).
 * Small launches (every 32-row block needs at most 512 keys, and query heads x
 * row blocks is at most the CU count) split each row block's keys across the
 * wavefronts of one workgroup and merge the partials on chip: the same math,
 * rounded in another order (within the attention tolerance, not bit-identical
 * to the grid form). */
int32_t grout_attn_prefill(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           uint16_t* out, float qk_scale, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t q_len,
                           int32_t kv_len, int32_t query_start, int32_t max_seq_len,
                           grout_stream_t stream);

/* Same computation, scheduled dynamically: one persistent workgroup per CU
 * claims workgroup-sized tasks.  XCD q owns the KV heads h = q (mod 8): the
 * heavier three quarters of their blocks form its heavy queue, the lighter
 * quarter its light queue, each heaviest first.  A workgroup claims from its
 * XCD's heavy queue, then from the fullest other heavy queue, then from its
 * own light queue while that holds at least half as many tasks as the fullest
 * light queue, else from the fullest: XCDs that run faster take over the
 * slower ones' heavy blocks, the last tasks are light ones, and most tasks run
 * where their head's K/V are cached (the reference's LPT order,
 * fmha_prefill_gqa_lpt src/kernels.rs:1513-1862, made dynamic).  Output
 * bit-identical to grout_attn_prefill.  Grids of at most two rounds of
 * workgroups use the static launch and leave the counters alone.
 *   sched_counters: grout_attn_prefill_sched_counter_bytes() bytes, 4-byte
 *   aligned, zero before the first call; every call leaves them zero.
 * Calls that overlap on one set of counters race. */
int32_t grout_attn_prefill_sched(const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, uint16_t* out, float qk_scale,
                                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t q_len, int32_t kv_len, int32_t query_start,
                                 int32_t max_seq_len, uint32_t* sched_counters,
                                 grout_stream_t stream);
int64_t grout_attn_prefill_sched_counter_bytes(void);

/* -------------------------------------------------------- split-K prefill */
/* Replaces fmha_prefill_gqa_lpt_split (src/kernels.rs:1872-2142), launched by
 * the attention microbench (benchmarks/src/bin/attention_microbench.rs:418-469)
 * with generics BM = block_m, BN = block_n, GROUP = group, NUM_KV_SPLITS =
 * num_splits.  Same Q/cache layouts and masking as grout_attn_prefill (cache
 * head stride max_seq_len).  Logical tile (q block b, head group hg) has index
 * b * (num_q_heads/group) + hg and rows r = bm*group + g = query row
 * b*block_m + bm of q head hg*group + g (zero Q past q_len).  Split s of q
 * block b covers keys of the tiles [s*tps, min(s*tps+tps, tc)) of block_n
 * keys, tc = ceil(min(query_start+(b+1)*block_m, kv_len)/block_n),
 * tps = ceil(tc/num_splits).
 *   att_partial [tiles, num_splits*block_m*group, 128] f16, row
 *   s*block_m*group + r: f16(acc/max(l,1e-8)) over the split's keys;
 *   lse_partial [tiles, num_splits*block_m*group] f32, m + log2(max(l,1e-8)).
 * A row with no key in a split's range stores O = 0, LSE = -1e30 (weight 0 in
 * the merge; the reference stores another weight-0 value there).
 * block_m must be a multiple of 32; group must divide num_q_heads/num_kv_heads.
 * Sizes: grout_attn_prefill_split_partial_bytes / _lse_bytes. */
int32_t grout_attn_prefill_split(const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, uint16_t* att_partial,
                                 float* lse_partial, float qk_scale, int32_t num_q_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t q_len,
                                 int32_t kv_len, int32_t query_start, int32_t max_seq_len,
                                 int32_t block_m, int32_t block_n, int32_t group,
                                 int32_t num_splits, grout_stream_t stream);

/* Replaces prefill_splitk_reduce_merge (src/kernels.rs:2151-2323): for rows
 * below q_len, out[row, head, :] = f16(sum_s w_s * att_s) with
 * w_s = 2^(lse_s - max) / max(sum, 1e-8); out [q_len, num_q_heads, 128]. */
int32_t grout_attn_prefill_split_merge(const uint16_t* att_partial, const float* lse_partial,
                                       uint16_t* out, int32_t num_q_heads, int32_t head_dim,
                                       int32_t q_len, int32_t block_m, int32_t group,
                                       int32_t num_splits, grout_stream_t stream);

/* Scratch bytes of grout_attn_prefill_split (< 0: invalid arguments). */
int64_t grout_attn_prefill_split_partial_bytes(int32_t num_q_heads, int32_t head_dim,
                                               int32_t q_len, int32_t block_m, int32_t group,
                                               int32_t num_splits);
int64_t grout_attn_prefill_split_lse_bytes(int32_t num_q_heads, int32_t q_len, int32_t block_m,
                                           int32_t group, int32_t num_splits);

/* ------------------------------------------ decode-layer ops around attention */
/* Replaces add_rms_norm_decode_raw_f16 (src/kernels.rs:3076-3216) as recorded
 * in the decode graph (src/model.rs:3151-3163, 3513-3526): for one row of n,
 * combined = f32(residual) + f32(x); inv = 1/sqrt(sum(combined^2)/n + eps);
 * out = f16(combined*inv*weight); residual_out = f16(combined).
 * n a multiple of 8, at most 32768; buffers 16-byte aligned; residual_out
 * may be residual itself, out may alias no input. */
int32_t grout_add_rms_norm_decode(const uint16_t* residual, const uint16_t* x,
                                  const uint16_t* weight, uint16_t* out, uint16_t* residual_out,
                                  float eps, int32_t n, grout_stream_t stream);

/* Replaces embedding_batch_f16 + rms_norm_f16 at the head of the decode graph
 * (src/kernels.rs:693-711, 304-344; src/model.rs:3120-3149) in one launch:
 * row = table[*token] ([vocab, n] f16), residual_out = row,
 * out = f16(row * 1/sqrt(sum(row^2)/n + eps) * weight).  *token is read on
 * the device (the previous step's argmax); an id >= vocab reads row vocab-1. */
int32_t grout_embed_rms_norm_decode(const uint32_t* token, const uint16_t* table, int32_t vocab,
                                    const uint16_t* weight, uint16_t* out, uint16_t* residual_out,
                                    float eps, int32_t n, grout_stream_t stream);

/* Replaces silu_mul_2d_f16 (src/kernels.rs:271-301; src/model.rs:3556-3565):
 * out[i] = f16(sigmoid(g) * g * u), g = f32(gate[i]), u = f32(up[i]),
 * sigmoid(g) = 1 / (1 + exp(-g)).  n a multiple of 8, at most 2^30; 16-byte
 * aligned. */
int32_t grout_silu_mul_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out, int32_t n,
                           grout_stream_t stream);

/* Replaces the cuBLAS GemvInPlace nodes of the decode graph (src/cublas.rs:572-607:
 * cublasGemmEx(OP_T, OP_N, m, 1, k) on a row-major [m, k] f16 weight):
 * out[i] = f16(sum_j weight[i][j] * x[j]) with f32 accumulation.
 * k a multiple of 8, at most 32768; weight and x 16-byte aligned. */
int32_t grout_gemv_f16(const uint16_t* weight, const uint16_t* x, uint16_t* out, int32_t m,
                       int32_t k, grout_stream_t stream);

/* The decode graph's gate_up GemvInPlace node followed by silu_mul_2d_f16
 * (src/model.rs:3529-3535, 3556-3565) in one launch; the reference records two
 * ops.  gate_up is the merged [2n, k] weight (gate rows [0, n), up rows
 * [n, 2n)); out[i] = grout_silu_mul_f16 of the f16 rows i and n + i of
 * grout_gemv_f16(gate_up, x), bit for bit, without the [2n] intermediate.
 * n at most 2^29; k and alignment as grout_gemv_f16. */
int32_t grout_gemv_silu_mul_f16(const uint16_t* gate_up, const uint16_t* x, uint16_t* out,
                                int32_t n, int32_t k, grout_stream_t stream);

/* Replaces argmax_blocks_f16 + argmax_reduce_blocks_to_u32 (src/kernels.rs:345-392,
 * 458-505), the in-graph greedy token pick: *token = the lowest index of the
 * largest f32(logits[i]) over [0, n) (NaN logits are never picked).
 * block_max / block_idx: grout_argmax_blocks(n) entries of scratch each.
 * 1 <= n <= 2^30. */
int32_t grout_argmax_blocks(int32_t n);
int32_t grout_argmax_f16(const uint16_t* logits, float* block_max, uint32_t* block_idx,
                         uint32_t* token, int32_t n, grout_stream_t stream);

/* ----------------------------------------------------- split-K GQA decode */
/* Replaces fmha_decode_gqa_split (src/kernels.rs:2586-2749) as recorded at
 * src/model.rs:3428-3452.
 *   q [num_kv_heads, group, 128] f16 (first num_q_heads*128 of q_out);
 *   s_kv = *d_position + 1 keys are read from the caches;
 *   att_partial [num_kv_heads, num_splits*group, 128] f16, split-major
 *   (row split*group + g); lse_partial [num_kv_heads, num_splits*group] f32,
 *   log2 units.  Split s covers KV tiles of block_n tokens
 *   [s*per, min(s*per+per, tiles)), tiles = ceil(s_kv/block_n),
 *   per = ceil(tiles/num_splits) (src/kernels.rs:2624-2629); an empty split
 *   writes O = 0, LSE = -1e30.
 *   qk_scale_f16 is the binary16 bit pattern of the scale: grout rounds
 *   1/sqrt(128) to f16 before the launch (src/model.rs:3427).
 * A device position >= max_seq_len is clamped to max_seq_len-1 (no reads
 * outside the cache). */
int32_t grout_attn_decode_split(const uint16_t* q, const uint16_t* k_cache,
                                const uint16_t* v_cache, uint16_t* att_partial,
                                float* lse_partial, uint16_t qk_scale_f16,
                                const uint32_t* d_position, int32_t num_kv_heads,
                                int32_t group, int32_t head_dim, int32_t max_seq_len,
                                int32_t block_n, int32_t num_splits, grout_stream_t stream);

/* ------------------------------------------------------------ split-K merge */
/* Replaces splitk_reduce_merge (src/kernels.rs:2771-2868) as recorded at
 * src/model.rs:3453-3473:  w_s = 2^(lse_s - max) / max(sum 2^(lse_s - max), 1e-8),
 * out[kvh, g, :] = f16(sum_s w_s * att_partial[kvh, s*group+g, :]). */
int32_t grout_attn_decode_merge(const uint16_t* att_partial, const float* lse_partial,
                                uint16_t* out, int32_t num_kv_heads, int32_t group,
                                int32_t head_dim, int32_t num_splits, grout_stream_t stream);

/* --------------------------------------------------- fused decode step */
/* One launch doing what grout's decode graph records as three ops per layer
 * (src/model.rs:3194-3221, 3428-3473): RMSNorm + RoPE of the G query rows of
 * each KV head (q_out rows [0, num_q_heads) are written, as A3 does), the
 * K/V-cache write at *d_position, split-K GQA attention over s_kv =
 * *d_position + 1 keys into att_partial/lse_partial (same layout as
 * grout_attn_decode_split; the partials are scratch of this launch, so its
 * splits are balanced instead: split s covers the 16-token sub-chunks
 * [s*n/num_splits, (s+1)*n/num_splits) of n = ceil(s_kv/16), and block_n is
 * only validated) and the LSE merge into out
 * [num_kv_heads, group, 128].  The last workgroup of each KV head merges: it
 * is found by an agent-scope counter in `counters`, and the partials reach it
 * through device-coherent stores completed before that counter moves.  Every
 * sum runs in a fixed order, so identical inputs give a bit-identical out.
 * A workgroup takes 143 KB of LDS (the merge's batch buffer), one per CU:
 * num_splits * num_kv_heads beyond the CU count runs in rounds, so take the
 * count from grout_attn_decode_pick_splits_grouped.
 *   counters: grout_attn_decode_counter_bytes(num_kv_heads) bytes, zero
 *   before the first call; every call leaves them zero again.
 *   advance_position != 0: the launch ends by storing *d_position + 1, so a
 *   graph replayed once per token needs no position write in between; a
 *   position at or past max_seq_len (no cache row written) is left as it is.
 * Calls that overlap on one set of counters race. */
int32_t grout_attn_decode_fused(const uint16_t* qkv, const uint16_t* q_weight,
                                const uint16_t* k_weight, const float* inv_freq,
                                uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                                uint16_t* att_partial, float* lse_partial, uint16_t* out,
                                uint32_t* counters, uint32_t* d_position, float eps,
                                uint16_t qk_scale_f16, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len,
                                int32_t block_n, int32_t num_splits, int32_t advance_position,
                                grout_stream_t stream);
int64_t grout_attn_decode_counter_bytes(int32_t num_kv_heads);

/* The fused decode step without caller scratch.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as grout_attn_decode_fused minus
 * att_partial, lse_partial and counters, which live in one static device
 * array of GROUT_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends):
 * 64 KiB of merge counters, then num_q_heads * num_splits LSEs (f32) and
 * partial rows (256 B).  Calls needing more, or num_kv_heads above
 * GROUT_NOALLOC_MAX_KV_HEADS, return GROUT_ERR_SCRATCH.  Nothing is
 * allocated.  The first successful call on a device looks up the array's
 * address (no stream work: the array is zero when the library is loaded,
 * and every launch leaves its counters zero); that first call must not be
 * made on a stream under capture, and returns GROUT_ERR_GRAPH if it is, so a
 * caller makes one call before capturing.  A failed look-up is retried by
 * the next call.  All calls on one GPU share the array: calls that overlap
 * on one GPU (two streams, two threads) race. */
#define GROUT_NOALLOC_SCRATCH_BYTES 4194304 /* 4 MiB */
#define GROUT_NOALLOC_MAX_KV_HEADS 255
int32_t grout_attn_decode_fused_noalloc(const uint16_t* qkv, const uint16_t* q_weight,
                                        const uint16_t* k_weight, const float* inv_freq,
                                        uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                                        uint16_t* out, uint32_t* d_position, float eps,
                                        uint16_t qk_scale_f16, int32_t num_q_heads,
                                        int32_t num_kv_heads, int32_t head_dim,
                                        int32_t max_seq_len, int32_t block_n, int32_t num_splits,
                                        int32_t advance_position, grout_stream_t stream);

/* Bytes of att_partial (f16) and lse_partial (f32) for a split count, as
 * allocated at src/model.rs:2508-2525.  Returns < 0 on invalid arguments. */
int64_t grout_attn_decode_partial_bytes(int32_t num_kv_heads, int32_t group, int32_t head_dim,
                                        int32_t num_splits);
int64_t grout_attn_decode_lse_bytes(int32_t num_kv_heads, int32_t group, int32_t num_splits);

/* Split count for a decode graph: enough (kv_head, split) workgroups to keep
 * every CU streaming at the longest context the graph will see, without
 * splits shorter than a few tiles.  Replaces the fixed NUM_KV_SPLITS default
 * (src/model.rs:128-135).  Returns >= 1. */
int32_t grout_attn_decode_pick_splits(int32_t cu_count, int32_t num_kv_heads,
                                      int32_t max_context, int32_t block_n);

/* The same count given the query heads per KV head (group): where the splits
 * of a KV head times group exceed the 512 partial rows grout_attn_decode_fused
 * merges in one batch, it takes fewer splits, as long as at least half the
 * CUs keep streaming (64 Q / 4 KV heads on 256 CUs: 32 splits rather than
 * 64).  group = 1 gives grout_attn_decode_pick_splits.  Returns >= 1. */
int32_t grout_attn_decode_pick_splits_grouped(int32_t cu_count, int32_t num_kv_heads,
                                              int32_t group, int32_t max_context,
                                              int32_t block_n);

/* Number of compute units of a device (hipDeviceAttributeMultiprocessorCount). */
int32_t grout_device_cu_count(int32_t device, int32_t* cu_count);

/* --------------------------------------------------------- hipGraph helpers */
/* Replace cuda-async's CudaGraph::scope / launch (src/model.rs:3118-3648,
 * :388-391).  begin/end wrap hipStreamBeginCapture / EndCapture +
 * hipGraphInstantiate on `stream` (thread-local capture mode). */
typedef struct grout_graph grout_graph;
int32_t grout_graph_begin(grout_stream_t stream);
int32_t grout_graph_end(grout_stream_t stream, grout_graph** graph);
int32_t grout_graph_launch(grout_graph* graph, grout_stream_t stream);
int32_t grout_graph_destroy(grout_graph* graph);

/* Stream-ordered write of a device u32 (the decode position), replacing the
 * 4-byte memcpy_htod_async of DecodeCudaGraphRunner::launch_step
 * (src/model.rs:363-376).  The value travels as a kernel argument, so no host
 * buffer has to outlive the call. */
int32_t grout_set_position_async(uint32_t* d_position, uint32_t position,
                                 grout_stream_t stream);

/* ------------------------------------------------- decode graph runner */
/* The attention slice of DecodeCudaGraphRunner (src/model.rs:318-493): one
 * hipGraph holding the fused decode step (grout_attn_decode_fused: QK
 * norm/RoPE/KV write, split-K decode, merge) for one layer's buffers,
 * replayed per token on the runner's stream.  Every step writes the position
 * (stream-ordered) before its replay; the graph also advances it, which
 * grout_decode_runner_run relies on between its replays.  Replays are
 * asynchronous: synchronise the runner's stream (or wait on an event recorded
 * on it) before reading attn_out, q_out or the caches.  All pointers are
 * borrowed and must outlive the runner, which owns *d_position and the
 * counters while it lives. */
typedef struct grout_decode_layer {
    const uint16_t* qkv;       /* [(Hq + 2*Hkv) * 128] f16 QKV GEMV output */
    const uint16_t* q_weight;  /* [128] f16 */
    const uint16_t* k_weight;  /* [128] f16 */
    const float* inv_freq;     /* [64] f32 */
    uint16_t* q_out;           /* [(Hq + Hkv) * 128] f16 (rows [0,Hq) used) */
    uint16_t* k_cache;         /* [Hkv, max_seq_len, 128] f16 */
    uint16_t* v_cache;         /* [Hkv, max_seq_len, 128] f16 */
    uint16_t* att_partial;     /* grout_attn_decode_partial_bytes */
    float* lse_partial;        /* grout_attn_decode_lse_bytes */
    uint16_t* attn_out;        /* [Hkv, G, 128] f16 */
    uint32_t* d_position;      /* device u32 */
    uint32_t* counters;        /* grout_attn_decode_counter_bytes, zeroed */
    float eps;
    uint16_t qk_scale_f16;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t max_seq_len;
    int32_t block_n;
    int32_t num_splits;
} grout_decode_layer;

typedef struct grout_decode_runner grout_decode_runner;
/* Validates, runs the step once eagerly (the prime pass of
 * src/model.rs:2561-3115) at `prime_position`, then captures it. */
int32_t grout_decode_runner_create(const grout_decode_layer* layer, uint32_t prime_position,
                                   grout_stream_t stream, grout_decode_runner** runner);
/* launch_step (src/model.rs:363-403): stream-ordered write of the device
 * position, then a replay of the graph.  No host sync. */
int32_t grout_decode_runner_step(grout_decode_runner* runner, uint32_t position);
/* `count` consecutive steps at positions first_position .. first_position+count-1
 * without returning to the caller in between: launch_step (src/model.rs:363-403)
 * repeated, for a decode loop whose per-token state stays on the device (the
 * reference's graph writes the sampled token in place).  Only the first step
 * may write the position; the graph advances it for the others.  No host sync. */
int32_t grout_decode_runner_run(grout_decode_runner* runner, uint32_t first_position,
                                int32_t count);
/* zero_kv_caches (src/model.rs:433-462): clear both caches in place; pointers
 * stay valid for the captured graph.  Synchronises the runner's stream. */
int32_t grout_decode_runner_zero_kv(grout_decode_runner* runner);
/* Waits for the runner's stream (queued replays use the borrowed buffers),
 * then frees the graph. */
int32_t grout_decode_runner_destroy(grout_decode_runner* runner);

/* ------------------------------------------- checkpoint formats */
/* Source element types of grout_cast_to_f16 (safetensors dtypes the
 * reference's loader accepts, src/loader.rs:109-145). */
#define GROUT_DTYPE_F16 0
#define GROUT_DTYPE_BF16 1
#define GROUT_DTYPE_F32 2
#define GROUT_DTYPE_F64 3

/* Replaces cast_to_f16 (src/loader.rs:107-145) on the device: dst[i] =
 * f16(src[i]) for n elements, round to nearest even (F64 via f32, as the
 * reference).  src and dst 16-byte aligned (dst may be a row range of a
 * merged matrix: concat_weight_rows_2d, src/model.rs:6021-6070). */
int32_t grout_cast_to_f16(const void* src, int32_t src_dtype, uint16_t* dst, int64_t n,
                          grout_stream_t stream);

/* ----------------------------------------- Qwen3 decode token step */
/* The whole decode graph of DecodeCudaGraphRunner (src/model.rs:3118-3648)
 * on this library's kernels: embedding + input RMSNorm of *token, then per
 * layer [add + input RMSNorm] -> qkv GEMV -> fused QK norm/RoPE/KV write +
 * split-K decode + merge -> o_proj GEMV -> add + post-attention RMSNorm ->
 * gate_up GEMV -> SiLU * up -> down GEMV; then the final add + RMSNorm, the
 * lm_head GEMV into `logits` and the greedy argmax into *token, which the
 * next step's embedding reads.  The last layer's attention advances
 * *d_position.  Weights, caches and buffers are borrowed. */
typedef struct grout_qwen3_layer {
    const uint16_t* input_norm;      /* [hidden] input_layernorm */
    const uint16_t* qkv_proj;        /* [(Hq + 2*Hkv)*128, hidden], rows Q | K | V
                                        (src/model.rs:1390-1401) */
    const uint16_t* q_norm;          /* [128] */
    const uint16_t* k_norm;          /* [128] */
    const uint16_t* o_proj;          /* [hidden, Hq*128] */
    const uint16_t* post_attn_norm;  /* [hidden] post_attention_layernorm */
    const uint16_t* gate_up_proj;    /* [2*intermediate, hidden], rows gate | up */
    const uint16_t* down_proj;       /* [hidden, intermediate] */
    uint16_t* k_cache;               /* [Hkv, max_seq_len, 128] */
    uint16_t* v_cache;               /* [Hkv, max_seq_len, 128] */
} grout_qwen3_layer;

typedef struct grout_qwen3_model {
    int32_t num_layers;
    int32_t hidden;          /* multiple of 8, <= 32768 */
    int32_t intermediate;    /* multiple of 8, <= 32768 */
    int32_t vocab;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;        /* 128 */
    int32_t max_seq_len;
    int32_t block_n;         /* decode KV tile (32) */
    int32_t num_splits;      /* grout_attn_decode_pick_splits */
    float eps;
    uint16_t qk_scale_f16;
    const grout_qwen3_layer* layers;  /* num_layers entries (copied by the runner) */
    const uint16_t* embed_tokens;     /* [vocab, hidden] */
    const uint16_t* final_norm;       /* [hidden] */
    const uint16_t* lm_head;          /* [vocab, hidden] (embed_tokens when tied) */
    const float* inv_freq;            /* [64] grout_build_inv_freq */
    uint32_t* token;                  /* device u32: this step's input, next step's token */
    uint32_t* d_position;             /* device u32 */
    uint16_t* logits;                 /* [vocab] f16 */
    void* workspace;                  /* grout_qwen3_workspace_bytes, 256-byte aligned */
} grout_qwen3_model;

/* Bytes of activations + scratch the step needs (< 0: invalid model). */
int64_t grout_qwen3_workspace_bytes(const grout_qwen3_model* model);
/* One eager step in stream order at *d_position (the sequence the graph
 * holds).  The workspace's attention counters must be zero before the first
 * step on it (grout_qwen3_runner_create clears them). */
int32_t grout_qwen3_decode_step(const grout_qwen3_model* model, grout_stream_t stream);

typedef struct grout_qwen3_runner grout_qwen3_runner;
/* Clears the counters, runs one eager prime step at prime_position (it writes
 * the caches there, replaces *token and advances the position, as any step),
 * then captures the step into a hipGraph. */
int32_t grout_qwen3_runner_create(const grout_qwen3_model* model, uint32_t prime_position,
                                  grout_stream_t stream, grout_qwen3_runner** runner);
/* seed_token (src/model.rs:343-356): stream-ordered write of *token. */
int32_t grout_qwen3_runner_seed_token(grout_qwen3_runner* runner, uint32_t token);
/* launch_step (src/model.rs:363-403): stream-ordered position write, graph
 * replay; when token_out is not NULL, the new token is copied back and the
 * stream synchronised. */
int32_t grout_qwen3_runner_step(grout_qwen3_runner* runner, uint32_t position,
                                uint32_t* token_out);
/* `count` consecutive steps from first_position without host round trips
 * (each step embeds the token the previous one picked).  No host sync:
 * synchronise the runner's stream before reading logits, *token or caches. */
int32_t grout_qwen3_runner_run(grout_qwen3_runner* runner, uint32_t first_position,
                               int32_t count);
/* Waits for the runner's stream (queued replays use the borrowed buffers),
 * then frees the graph. */
int32_t grout_qwen3_runner_destroy(grout_qwen3_runner* runner);
/* A runner is used from one host thread at a time; two runners sharing a
 * workspace, token or position buffer race on the device. */

#ifdef __cplusplus
}
#endif
#endif /* GROUT_ATTN_HIP_H */

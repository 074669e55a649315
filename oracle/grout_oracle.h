/*
 * grout_oracle.h — CPU restatement of grout's Qwen3 attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (grout_amd/, include/)
 * links or calls this code.  It is loaded by tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py, always as the checker or the timed
 * CPU baseline, never as the thing measured on the GPU.
 *
 * Every function restates one reference function (file:line under the
 * upstream NikVisel/grout tree) in plain C99 with f32 arithmetic and f16
 * storage (IEEE binary16 bit patterns in uint16_t, round-to-nearest-even).
 * Built with -ffp-contract=off so every a*b+c rounds twice, as written.
 */
#ifndef GROUT_ORACLE_H
#define GROUT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* f32 <-> binary16, round-to-nearest-even, subnormals and inf/nan kept. */
uint16_t go_f32_to_f16(float f);
float go_f16_to_f32(uint16_t h);
void go_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);
void go_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);

/* src/model.rs:5992-6003 build_inv_freq: inv[j] = 1 / theta^((2j)/D), f32. */
void go_build_inv_freq(float theta, int32_t head_dim, float* out);

/* src/kernels.rs:3415-3732 qk_norm_rope_kv_prefill_raw_f16.
 * q [S,Hq,D], k/v [S,Hkv,D]; q_out [S,Hq,D]; caches [Hkv,max_seq,D]. */
void go_qk_norm_rope_kv_prefill(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const uint16_t* q_weight, const uint16_t* k_weight,
                                const float* inv_freq, uint16_t* q_out, uint16_t* k_cache,
                                uint16_t* v_cache, float eps, int32_t position_start,
                                int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t max_seq_len);

/* src/kernels.rs:3750-4016 qk_norm_rope_kv_decode_raw_f16.
 * qkv = [Q(Hq*D) | K(Hkv*D) | V(Hkv*D)]; q_out rows [0,Hq) written. */
void go_qk_norm_rope_kv_decode(const uint16_t* qkv, const uint16_t* q_weight,
                               const uint16_t* k_weight, const float* inv_freq,
                               uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                               uint32_t position, float eps, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len);

/* benchmarks/src/bin/attention_microbench.rs:665-702 cpu_reference, generalised
 * to GQA on the [Hkv,max_seq,D] cache, query_start>0 and kv_len: row m (query
 * position query_start+m) attends keys n < min(kv_len, query_start+m+1).
 * f32 throughout, two-pass softmax with expf, out f32 [q_len,Hq,D].
 * Rows m = row_begin, row_begin+row_step, ... are computed (row_step=1: all);
 * other rows of out are left untouched.  nthreads<=0: OpenMP default. */
void go_attn_prefill_f32(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         float* out, float qk_scale, int32_t num_q_heads, int32_t num_kv_heads,
                         int32_t head_dim, int32_t q_len, int32_t kv_len, int32_t query_start,
                         int32_t max_seq_len, int32_t row_begin, int32_t row_step,
                         int32_t nthreads);

/* src/kernels.rs:2586-2749 fmha_decode_gqa_split.  q [Hkv,G,D] (first Hq*D of
 * q_out); att_partial [Hkv, NKS*G, D] f16 split-major (split*G+g);
 * lse_partial [Hkv, NKS*G] f32 in log2 units.  qk_scale_f16 is the f16 bit
 * pattern of the scale (src/model.rs:3427 rounds 1/sqrt(D) to f16).
 * fused_ranges = 0: the reference's split boundaries (go_decode_split_range);
 * 1: the boundaries of this repository's fused decode step (no counterpart in
 * the reference; go_decode_split_range_fused), same per-split arithmetic. */
void go_attn_decode_split(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                          uint16_t* att_partial, float* lse_partial, uint16_t qk_scale_f16,
                          uint32_t position, int32_t num_kv_heads, int32_t group,
                          int32_t head_dim, int32_t max_seq_len, int32_t block_n,
                          int32_t num_splits, int32_t nthreads, int32_t fused_ranges);

/* Token range [begin, end) of split `split` in the fused decode step: n =
 * ceil(s_kv/16) sub-chunks of 16 tokens, split s takes [s*n/NKS, (s+1)*n/NKS). */
void go_decode_split_range_fused(int32_t s_kv, int32_t num_splits, int32_t split,
                                 int32_t* tok_begin, int32_t* tok_end);

/* src/kernels.rs:2771-2868 splitk_reduce_merge.  out [Hkv, G, D] f16. */
void go_attn_decode_merge(const uint16_t* att_partial, const float* lse_partial, uint16_t* out,
                          int32_t num_kv_heads, int32_t group, int32_t head_dim,
                          int32_t num_splits);

/* Tile range of one split, src/kernels.rs:2624-2629:
 * tiles = ceil(s_kv/BN); per = ceil(tiles/NKS); [split*per, min(split*per+per, tiles)). */
void go_decode_split_range(int32_t s_kv, int32_t block_n, int32_t num_splits, int32_t split,
                           int32_t* tile_begin, int32_t* tile_end);

/* src/kernels.rs:759-800 kv_cache_update_seq_f16: cache slot
 * [h, position_start + r, :] = new[r, h, :] for r < seq_len (every other slot
 * untouched); new [seq_len, Hkv, D], caches [Hkv, max_seq, D]. */
void go_kv_cache_update_seq(const uint16_t* new_k, const uint16_t* new_v, uint16_t* k_cache,
                            uint16_t* v_cache, int32_t position_start, int32_t seq_len,
                            int32_t num_kv_heads, int32_t head_dim, int32_t max_seq);

/* src/kernels.rs:1872-2142 fmha_prefill_gqa_lpt_split (cache head stride
 * max_seq_len): att_partial [tiles, NKS*BM*GROUP, D] f16, lse_partial
 * [tiles, NKS*BM*GROUP] f32, tiles = ceil(q_len/BM) * (Hq/GROUP). */
void go_attn_prefill_split(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           uint16_t* att_partial, float* lse_partial, float qk_scale,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t q_len, int32_t kv_len, int32_t query_start,
                           int32_t max_seq_len, int32_t block_m, int32_t block_n,
                           int32_t group, int32_t num_splits, int32_t nthreads);

/* src/kernels.rs:2151-2323 prefill_splitk_reduce_merge -> out [q_len, Hq, D]. */
void go_attn_prefill_split_merge(const uint16_t* att_partial, const float* lse_partial,
                                 uint16_t* out, int32_t num_q_heads, int32_t head_dim,
                                 int32_t q_len, int32_t block_m, int32_t group,
                                 int32_t num_splits);

/* src/kernels.rs:3076-3216 add_rms_norm_decode_raw_f16 (one row of n). */
void go_add_rms_norm(const uint16_t* residual, const uint16_t* x, const uint16_t* w,
                     uint16_t* out, uint16_t* residual_out, float eps, int32_t n);

/* src/cublas.rs:572-607 GemvInPlace: out[m] = f16(W[m,k] x[k]), f32 accumulation. */
void go_gemv_f16(const uint16_t* w, const uint16_t* x, uint16_t* out, int32_t m, int32_t k,
                 int32_t nthreads);

/* src/kernels.rs:345-505 two-stage greedy argmax: lowest index of the largest logit. */
uint32_t go_argmax_f16(const uint16_t* logits, int32_t n);

/* src/kernels.rs:271-301 silu_mul_2d_f16. */
void go_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, int32_t n);

/* src/loader.rs:107-145 cast_to_f16; dtype 0 F16, 1 BF16, 2 F32, 3 F64. */
int32_t go_cast_to_f16(const void* src, int32_t dtype, uint16_t* out, int64_t n);

#ifdef __cplusplus
}
#endif
#endif

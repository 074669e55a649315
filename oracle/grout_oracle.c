/*
 * grout_oracle.c — CPU restatement of grout's Qwen3 attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke()
 * and the CPU baseline of bench.py.  Never linked into the product.
 *
 * Each function cites the reference function it restates (paths relative to
 * the upstream NikVisel/grout tree).  Arithmetic is f32 in the order the
 * reference writes it; f16 values are IEEE binary16 bit patterns rounded to
 * nearest-even.  Compile with -ffp-contract=off (oracle/Makefile does).
 *
 * Parity pins (tests/test_oracle.py): every function here is checked against
 * the reference's KV-slot known-answer test, closed forms, invariants and an
 * independent float64 brute force; none is "parity unpinned".
 */
#include "grout_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ f16 -- */

uint16_t go_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14 */
        if (ax < 0x33000000u) return (uint16_t)sign;          /* <= 2^-25 ties to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value / 2^-24 = m * 2^(e-126) */
        uint32_t qv = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (qv & 1u))) qv++;
        return (uint16_t)(sign | qv);
    }
    uint32_t r = ax - 0x38000000u; /* rebias 127 -> 15 */
    uint32_t h = (r + 0x0fffu + ((r >> 13) & 1u)) >> 13;
    return (uint16_t)(sign | h);
}

float go_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0x1fu) {
        x = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else { /* subnormal: m * 2^-24 */
        float v = (float)m * (1.0f / 16777216.0f);
        memcpy(&x, &v, 4);
        x |= sign;
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void go_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = go_f32_to_f16(in[i]);
}

void go_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = go_f16_to_f32(in[i]);
}

static inline float h2f(uint16_t h) { return go_f16_to_f32(h); }

/* ------------------------------------------------------------- inv_freq -- */

/* src/model.rs:5992-6003: for i in (0..D).step_by(2) { p = i as f32 / D as f32;
 * inv.push(1.0 / theta.powf(p)) }  (Rust f32::powf is libm powf on linux-gnu). */
void go_build_inv_freq(float theta, int32_t head_dim, float* out) {
    for (int32_t i = 0; i < head_dim; i += 2) {
        float p = (float)i / (float)head_dim;
        out[i / 2] = 1.0f / powf(theta, p);
    }
}

/* --------------------------------------------------- fused norm + RoPE -- */

/* One head row: RMSNorm with f16 weight, then GPT-NeoX half rotation.
 * src/kernels.rs:3577-3586 (ss = reduce_sum(lo*lo + hi*hi); inv = rsqrt(ss/D + eps)),
 * :3629-3630 (n = x * inv * w), :3640-3648 (theta = f32(pos) * inv_freq[j];
 * y_lo = n_lo*cos - n_hi*sin; y_hi = n_hi*cos + n_lo*sin), f16 RNE store.
 *
 * Two choices the reference leaves open are fixed here:
 *  - reduce_sum's order: the H pair terms form 8 sequential partial sums of
 *    H/8 terms each, combined pairwise ((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7));
 *  - sin/cos of the f32 angle: correctly rounded to f32 (evaluated in f64).
 * With these, the result is a deterministic function of the f16 inputs;
 * tests/test_oracle.py pins it to an independent float64 formulation. */
static void norm_rope_row(const uint16_t* x, const uint16_t* w, const float* inv_freq,
                          int32_t pos, float eps, int32_t D, uint16_t* y) {
    const int32_t H = D / 2;
    const int32_t chunk = H / 8;
    float part[8];
    for (int32_t t = 0; t < 8; ++t) {
        float acc = 0.0f;
        for (int32_t i = 0; i < chunk; ++i) {
            int32_t j = t * chunk + i;
            float lo = h2f(x[j]), hi = h2f(x[j + H]);
            acc += lo * lo + hi * hi;
        }
        part[t] = acc;
    }
    float ss = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
    float inv_rms = 1.0f / sqrtf(ss / (float)D + eps);
    float posf = (float)pos;
    for (int32_t j = 0; j < H; ++j) {
        float lo = h2f(x[j]), hi = h2f(x[j + H]);
        float n_lo = lo * inv_rms * h2f(w[j]);
        float n_hi = hi * inv_rms * h2f(w[j + H]);
        float theta = posf * inv_freq[j];
        float c = (float)cos((double)theta), s = (float)sin((double)theta);
        float y_lo = n_lo * c - n_hi * s;
        float y_hi = n_hi * c + n_lo * s;
        y[j] = go_f32_to_f16(y_lo);
        y[j + H] = go_f32_to_f16(y_hi);
    }
}

/* src/kernels.rs:3415-3732 qk_norm_rope_kv_prefill_raw_f16; grid (S, Hq+Hkv)
 * at src/model.rs:4567-4595.  Row (s, h<Hq): q_out[s,h] = rope(norm(q[s,h], q_w));
 * row (s, Hq+h): k_cache[h, ps+s] = rope(norm(k[s,h], k_w)), v_cache[h, ps+s] = v[s,h]. */
void go_qk_norm_rope_kv_prefill(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const uint16_t* q_weight, const uint16_t* k_weight,
                                const float* inv_freq, uint16_t* q_out, uint16_t* k_cache,
                                uint16_t* v_cache, float eps, int32_t position_start,
                                int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t max_seq_len) {
    const int64_t D = head_dim;
    for (int32_t s = 0; s < seq_len; ++s) {
        int32_t pos = position_start + s;
        for (int32_t h = 0; h < num_q_heads; ++h) {
            int64_t off = ((int64_t)s * num_q_heads + h) * D;
            norm_rope_row(q + off, q_weight, inv_freq, pos, eps, head_dim, q_out + off);
        }
        for (int32_t h = 0; h < num_kv_heads; ++h) {
            int64_t in_off = ((int64_t)s * num_kv_heads + h) * D;
            int64_t slot = ((int64_t)h * max_seq_len + pos) * D;
            norm_rope_row(k + in_off, k_weight, inv_freq, pos, eps, head_dim, k_cache + slot);
            memcpy(v_cache + slot, v + in_off, (size_t)D * sizeof(uint16_t));
        }
    }
}

/* src/kernels.rs:3750-4016 qk_norm_rope_kv_decode_raw_f16; grid (Hq+Hkv, 2).
 * The QKV GEMV output is read in 64-element blocks q:2h, k:2Hq+2h,
 * v:2Hq+2Hkv+2h (:3853-3855), i.e. rows of D at h, Hq+h, Hq+Hkv+h. */
void go_qk_norm_rope_kv_decode(const uint16_t* qkv, const uint16_t* q_weight,
                               const uint16_t* k_weight, const float* inv_freq,
                               uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                               uint32_t position, float eps, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len) {
    const int64_t D = head_dim;
    int32_t pos = (int32_t)position; /* bitcast u32 -> i32, :3934-3937 */
    for (int32_t h = 0; h < num_q_heads; ++h)
        norm_rope_row(qkv + h * D, q_weight, inv_freq, pos, eps, head_dim, q_out + h * D);
    for (int32_t h = 0; h < num_kv_heads; ++h) {
        int64_t slot = ((int64_t)h * max_seq_len + pos) * D;
        norm_rope_row(qkv + (num_q_heads + h) * D, k_weight, inv_freq, pos, eps, head_dim,
                      k_cache + slot);
        memcpy(v_cache + slot, qkv + (num_q_heads + num_kv_heads + h) * D,
               (size_t)D * sizeof(uint16_t));
    }
}

/* ------------------------------------------------ fp32 attention oracle -- */

/* Widen rows [0, rows) of each head of a [heads, max_seq, D] f16 cache. */
static float* widen_cache(const uint16_t* cache, int32_t heads, int32_t rows, int32_t D,
                          int32_t max_seq_len) {
    float* out = (float*)malloc((size_t)heads * rows * D * sizeof(float));
    if (!out) return NULL;
    for (int32_t h = 0; h < heads; ++h)
        go_f16_to_f32_array(cache + (int64_t)h * max_seq_len * D, out + (int64_t)h * rows * D,
                            (int64_t)rows * D);
    return out;
}

/* benchmarks/src/bin/attention_microbench.rs:665-702 cpu_reference:
 *   dot += q*k (f32, d order); score = dot*scale; two-pass softmax with exp;
 *   acc += scores[n] / denom * v.
 * Generalised: K/V come from the cache, kvh = qh / (Hq/Hkv), keys n < min(kv_len,
 * query_start+m+1) (causal rule of src/kernels.rs:1242-1257). */
void go_attn_prefill_f32(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         float* out, float qk_scale, int32_t num_q_heads, int32_t num_kv_heads,
                         int32_t head_dim, int32_t q_len, int32_t kv_len, int32_t query_start,
                         int32_t max_seq_len, int32_t row_begin, int32_t row_step,
                         int32_t nthreads) {
    const int32_t D = head_dim;
    const int32_t qgs = num_q_heads / num_kv_heads;
    if (row_step < 1) row_step = 1;
    int32_t kv_rows = kv_len < max_seq_len ? kv_len : max_seq_len;
    if (kv_rows < 0) kv_rows = 0;
    float* kf = widen_cache(k_cache, num_kv_heads, kv_rows, D, max_seq_len);
    float* vf = widen_cache(v_cache, num_kv_heads, kv_rows, D, max_seq_len);
    if ((kv_rows > 0) && (!kf || !vf)) {
        free(kf);
        free(vf);
        return;
    }
    int32_t nrows = row_begin < q_len ? (q_len - row_begin + row_step - 1) / row_step : 0;
    int64_t tasks = (int64_t)nrows * num_q_heads;
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float* scores = (float*)malloc((size_t)(kv_rows > 0 ? kv_rows : 1) * sizeof(float));
        float qrow[512];
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (int64_t t = 0; t < tasks; ++t) {
            int32_t m = row_begin + (int32_t)(t / num_q_heads) * row_step;
            int32_t qh = (int32_t)(t % num_q_heads);
            int32_t kvh = qh / qgs;
            int64_t q_off = ((int64_t)m * num_q_heads + qh) * D;
            float* o = out + q_off;
            int32_t mpos = query_start + m;
            int32_t nmax = mpos + 1 < kv_rows ? mpos + 1 : kv_rows;
            if (nmax <= 0) {
                for (int32_t d = 0; d < D; ++d) o[d] = 0.0f;
                continue;
            }
            for (int32_t d = 0; d < D; ++d) qrow[d] = h2f(q[q_off + d]);
            const float* kh = kf + (int64_t)kvh * kv_rows * D;
            const float* vh = vf + (int64_t)kvh * kv_rows * D;
            float max_score = -INFINITY;
            for (int32_t n = 0; n < nmax; ++n) {
                const float* kr = kh + (int64_t)n * D;
                float dot = 0.0f;
                for (int32_t d = 0; d < D; ++d) dot += qrow[d] * kr[d];
                float score = dot * qk_scale;
                scores[n] = score;
                max_score = fmaxf(max_score, score);
            }
            float denom = 0.0f;
            for (int32_t n = 0; n < nmax; ++n) {
                scores[n] = expf(scores[n] - max_score);
                denom += scores[n];
            }
            for (int32_t d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (int32_t n = 0; n < nmax; ++n) acc += scores[n] / denom * vh[(int64_t)n * D + d];
                o[d] = acc;
            }
        }
        free(scores);
    }
    free(kf);
    free(vf);
}

/* ------------------------------------------------ split-K decode oracle -- */

void go_decode_split_range(int32_t s_kv, int32_t block_n, int32_t num_splits, int32_t split,
                           int32_t* tile_begin, int32_t* tile_end) {
    int32_t tiles = (s_kv + block_n - 1) / block_n;
    int32_t per = (tiles + num_splits - 1) / num_splits;
    int32_t b = split * per;
    int32_t e = b + per;
    if (e > tiles) e = tiles;
    *tile_begin = b;
    *tile_end = e;
}

void go_decode_split_range_fused(int32_t s_kv, int32_t num_splits, int32_t split,
                                 int32_t* tok_begin, int32_t* tok_end) {
    int64_t n = ((int64_t)s_kv + 15) / 16;
    int32_t b = (int32_t)(split * n / num_splits);
    int32_t e = (int32_t)((split + 1) * n / num_splits);
    *tok_begin = 16 * b;
    *tok_end = b < e ? (16 * e < s_kv ? 16 * e : s_kv) : 16 * b;
}

/* src/kernels.rs:2586-2749 fmha_decode_gqa_split, one (kv_head, split) per task.
 *   scale_log2 = f32(qk_scale_f16) / ln(2)                       (:2618-2622)
 *   m = -1e30, l[BN][G] = 1, acc[G][D] = 0                        (:2635-2639)
 *   per tile j: qk[n][g] = k[n].q[g] (f32 acc); last global tile adds -1e30 to
 *   slots n >= s_kv (:2676-2683); qk *= scale_log2; m_ij = max(m, max_n qk);
 *   p = exp2(qk - m_ij); alpha = exp2(m - m_ij); l = l*alpha + p;
 *   acc = acc*alpha + sum_n f16(p)*v                               (:2687-2722)
 *   O = f16(acc / max(sum_n l, 1e-8)); LSE = m + log2(max(sum_n l, 1e-8)) (:2729-2748)
 * Cache slots at or beyond max_seq_len read as 0 (tile loads past the view are
 * zero-filled).  The split's tokens [b, e) run in BN-token tiles from b, and
 * slots at or past e get the -1e30; with the reference's boundaries that is
 * exactly its rule (only the last global tile has slots past s_kv). */
void go_attn_decode_split(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                          uint16_t* att_partial, float* lse_partial, uint16_t qk_scale_f16,
                          uint32_t position, int32_t num_kv_heads, int32_t group,
                          int32_t head_dim, int32_t max_seq_len, int32_t block_n,
                          int32_t num_splits, int32_t nthreads, int32_t fused_ranges) {
    const int32_t D = head_dim, G = group, BN = block_n;
    const int32_t s_kv = (int32_t)position + 1;
    const float ln2 = logf(2.0f);
    const float scale_log2 = h2f(qk_scale_f16) / ln2;
    int64_t tasks = (int64_t)num_kv_heads * num_splits;
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float* qf = (float*)malloc((size_t)G * D * sizeof(float));
        float* acc = (float*)malloc((size_t)G * D * sizeof(float));
        float* l = (float*)malloc((size_t)BN * G * sizeof(float));
        float* qk = (float*)malloc((size_t)BN * G * sizeof(float));
        float* kt = (float*)malloc((size_t)BN * D * sizeof(float));
        float* vt = (float*)malloc((size_t)BN * D * sizeof(float));
        float* m = (float*)malloc((size_t)G * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t t = 0; t < tasks; ++t) {
            int32_t kvh = (int32_t)(t / num_splits);
            int32_t split = (int32_t)(t % num_splits);
            int32_t b, e;
            if (fused_ranges) {
                go_decode_split_range_fused(s_kv, num_splits, split, &b, &e);
            } else {
                int32_t tb, te;
                go_decode_split_range(s_kv, BN, num_splits, split, &tb, &te);
                b = tb * BN;
                e = tb < te ? (te * BN < s_kv ? te * BN : s_kv) : b;
            }
            for (int32_t i = 0; i < G * D; ++i) {
                qf[i] = h2f(q[(int64_t)kvh * G * D + i]);
                acc[i] = 0.0f;
            }
            for (int32_t g = 0; g < G; ++g) m[g] = 0.0f - 1.0e30f;
            for (int32_t i = 0; i < BN * G; ++i) l[i] = 1.0f;
            const uint16_t* kh = k_cache + (int64_t)kvh * max_seq_len * D;
            const uint16_t* vh = v_cache + (int64_t)kvh * max_seq_len * D;
            for (int32_t t0 = b; t0 < e; t0 += BN) {
                for (int32_t n = 0; n < BN; ++n) {
                    int32_t tok = t0 + n;
                    for (int32_t d = 0; d < D; ++d) {
                        kt[n * D + d] = tok < max_seq_len ? h2f(kh[(int64_t)tok * D + d]) : 0.0f;
                        vt[n * D + d] = tok < max_seq_len ? h2f(vh[(int64_t)tok * D + d]) : 0.0f;
                    }
                }
                for (int32_t n = 0; n < BN; ++n)
                    for (int32_t g = 0; g < G; ++g) {
                        float dot = 0.0f;
                        for (int32_t d = 0; d < D; ++d) dot += kt[n * D + d] * qf[g * D + d];
                        qk[n * G + g] = dot;
                    }
                if (t0 + BN > e) {
                    for (int32_t n = 0; n < BN; ++n) {
                        float add = (t0 + n < e) ? 0.0f : (0.0f - 1.0e30f);
                        for (int32_t g = 0; g < G; ++g) qk[n * G + g] = qk[n * G + g] + add;
                    }
                }
                for (int32_t i = 0; i < BN * G; ++i) qk[i] = qk[i] * scale_log2;
                for (int32_t g = 0; g < G; ++g) {
                    float mx = qk[g];
                    for (int32_t n = 1; n < BN; ++n) mx = fmaxf(mx, qk[n * G + g]);
                    float m_ij = fmaxf(m[g], mx);
                    float alpha = exp2f(m[g] - m_ij);
                    for (int32_t n = 0; n < BN; ++n) {
                        float p = exp2f(qk[n * G + g] - m_ij);
                        l[n * G + g] = l[n * G + g] * alpha + p;
                        qk[n * G + g] = h2f(go_f32_to_f16(p)); /* f16(p) feeds the PV mma */
                    }
                    for (int32_t d = 0; d < D; ++d) {
                        float a = acc[g * D + d] * alpha;
                        for (int32_t n = 0; n < BN; ++n) a += vt[n * D + d] * qk[n * G + g];
                        acc[g * D + d] = a;
                    }
                    m[g] = m_ij;
                }
            }
            for (int32_t g = 0; g < G; ++g) {
                float ls = 0.0f;
                for (int32_t n = 0; n < BN; ++n) ls += l[n * G + g];
                float l_safe = fmaxf(ls, 1.0e-8f);
                int64_t row = (int64_t)kvh * num_splits * G + (int64_t)split * G + g;
                for (int32_t d = 0; d < D; ++d)
                    att_partial[row * D + d] = go_f32_to_f16(acc[g * D + d] / l_safe);
                lse_partial[row] = m[g] + log2f(l_safe);
            }
        }
        free(qf);
        free(acc);
        free(l);
        free(qk);
        free(kt);
        free(vt);
        free(m);
    }
}

/* src/kernels.rs:2771-2868 splitk_reduce_merge:
 *   lse_max = max_s lse_s; w_s = 2^(lse_s - lse_max) / max(sum_s 2^(lse_s - lse_max), 1e-8);
 *   out[g][d] = f16(sum_s w_s * O_s[g][d]), O_s read from the split-major scratch. */
void go_attn_decode_merge(const uint16_t* att_partial, const float* lse_partial, uint16_t* out,
                          int32_t num_kv_heads, int32_t group, int32_t head_dim,
                          int32_t num_splits) {
    const int32_t D = head_dim, G = group, NS = num_splits;
    float* w = (float*)malloc((size_t)NS * sizeof(float));
    for (int32_t kvh = 0; kvh < num_kv_heads; ++kvh) {
        for (int32_t g = 0; g < G; ++g) {
            const float* lse = lse_partial + (int64_t)kvh * NS * G;
            float mx = lse[g];
            for (int32_t s = 1; s < NS; ++s) mx = fmaxf(mx, lse[s * G + g]);
            float sum = 0.0f;
            for (int32_t s = 0; s < NS; ++s) {
                w[s] = exp2f(lse[s * G + g] - mx);
                sum += w[s];
            }
            float safe = fmaxf(sum, 1.0e-8f);
            for (int32_t s = 0; s < NS; ++s) w[s] = w[s] / safe;
            for (int32_t d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (int32_t s = 0; s < NS; ++s) {
                    int64_t row = (int64_t)kvh * NS * G + (int64_t)s * G + g;
                    acc += h2f(att_partial[row * D + d]) * w[s];
                }
                out[((int64_t)kvh * G + g) * D + d] = go_f32_to_f16(acc);
            }
        }
    }
    free(w);
}

/* src/kernels.rs:759-800 kv_cache_update_seq_f16: each cache tile owns absolute
 * slots s_global and takes input row s_global - position_start when
 * position_start <= s_global < position_start + seq_len (:783-797). */
void go_kv_cache_update_seq(const uint16_t* new_k, const uint16_t* new_v, uint16_t* k_cache,
                            uint16_t* v_cache, int32_t position_start, int32_t seq_len,
                            int32_t num_kv_heads, int32_t head_dim, int32_t max_seq) {
    for (int32_t h = 0; h < num_kv_heads; ++h) {
        for (int32_t s_global = 0; s_global < max_seq; ++s_global) {
            if (s_global < position_start || s_global >= position_start + seq_len) continue;
            const int64_t row = s_global - position_start;
            const int64_t src = (row * num_kv_heads + h) * head_dim;
            const int64_t dst = ((int64_t)h * max_seq + s_global) * head_dim;
            for (int32_t d = 0; d < head_dim; ++d) {
                k_cache[dst + d] = new_k[src + d];
                v_cache[dst + d] = new_v[src + d];
            }
        }
    }
}

/* src/kernels.rs:1872-2142 fmha_prefill_gqa_lpt_split (generics BM, BN, GROUP,
 * NUM_KV_SPLITS; M_EFF = BM*GROUP), with the K/V head stride taken from the
 * cache (max_seq_len), not kv_len (src/kernels.rs:1922-1928 assumes
 * kv_len == max_seq_len).  Logical tile = (q block b, head group hg), index
 * b*num_head_groups + hg (:1998); tile row r = bm*GROUP + g is query row
 * b*BM + bm of q head hg*GROUP + g (:2017-2024), zero Q beyond q_len (the
 * tensor view's out-of-bounds fill); KV head hg*GROUP / (Hq/Hkv) (:1999).
 * Split s covers KV tiles [s*tps, min(s*tps+tps, tc)) with
 * tc = ceil(min(m_end, kv_len)/BN), tps = ceil(tc/NKS) (:2036-2043); tiles
 * at or past mask_start = min((query_start+b*BM)/BN, kv_len/BN) get the
 * additive -1e30 mask for n >= kv_len or n > query position (:2063-2075);
 * rows beyond kv_len read as zero.  Per tile: m_ij = max(m_i, rowmax(qk)*c),
 * p = 2^(qk*c - m_ij), l = l*alpha + sum(p), acc = acc*alpha + f16(p) V
 * (:2077-2102); c = qk_scale / ln 2.  Stores att = f16(acc / max(l, 1e-8))
 * at [tile, s*M_EFF + r, :] and lse = m + log2(max(l, 1e-8)) at
 * [tile, s*M_EFF + r] (:2105-2141). */
void go_attn_prefill_split(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           uint16_t* att_partial, float* lse_partial, float qk_scale,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t q_len, int32_t kv_len, int32_t query_start,
                           int32_t max_seq_len, int32_t block_m, int32_t block_n,
                           int32_t group, int32_t num_splits, int32_t nthreads) {
    const int32_t D = head_dim, BM = block_m, BN = block_n, GR = group, NKS = num_splits;
    const int32_t qgs = num_q_heads / num_kv_heads;
    const int32_t num_q_blocks = (q_len + BM - 1) / BM;
    const int32_t num_head_groups = num_q_heads / GR;
    const int32_t m_eff = BM * GR;
    const float c = qk_scale / logf(2.0f);
    const int64_t tasks = (int64_t)num_q_blocks * num_head_groups * NKS;
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float* qf = (float*)malloc((size_t)m_eff * D * sizeof(float));
        float* acc = (float*)malloc((size_t)m_eff * D * sizeof(float));
        float* qk = (float*)malloc((size_t)m_eff * BN * sizeof(float));
        float* kt = (float*)malloc((size_t)BN * D * sizeof(float));
        float* vt = (float*)malloc((size_t)BN * D * sizeof(float));
        uint16_t* ph = (uint16_t*)malloc((size_t)m_eff * BN * sizeof(uint16_t));
        float* mi = (float*)malloc((size_t)m_eff * sizeof(float));
        float* li = (float*)malloc((size_t)m_eff * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t t = 0; t < tasks; ++t) {
            const int32_t split = (int32_t)(t % NKS);
            const int64_t tile = t / NKS;
            const int32_t b = (int32_t)(tile / num_head_groups);
            const int32_t hg = (int32_t)(tile % num_head_groups);
            const int32_t kvh = hg * GR / qgs;
            for (int32_t r = 0; r < m_eff; ++r) {
                const int32_t row = b * BM + r / GR, head = hg * GR + r % GR;
                for (int32_t d = 0; d < D; ++d) {
                    qf[(int64_t)r * D + d] =
                        row < q_len ? h2f(q[((int64_t)row * num_q_heads + head) * D + d]) : 0.0f;
                    acc[(int64_t)r * D + d] = 0.0f;
                }
                mi[r] = 0.0f - 1.0e30f;
                li[r] = 0.0f;
            }
            const int32_t m_end = query_start + (b + 1) * BM;
            const int32_t k_seqlen_tiles = kv_len / BN;
            int32_t mask_start = (query_start + b * BM) / BN;
            if (mask_start > k_seqlen_tiles) mask_start = k_seqlen_tiles;
            const int32_t lim = m_end < kv_len ? m_end : kv_len;
            const int32_t tc = (lim + BN - 1) / BN;
            const int32_t tps = (tc + NKS - 1) / NKS;
            const int32_t st = split * tps;
            const int32_t et = st + tps < tc ? st + tps : tc;
            const uint16_t* kh = k_cache + (int64_t)kvh * max_seq_len * D;
            const uint16_t* vh = v_cache + (int64_t)kvh * max_seq_len * D;
            for (int32_t j = st; j < et; ++j) {
                for (int32_t n = 0; n < BN; ++n) {
                    const int32_t tok = j * BN + n;
                    const int ok = tok < kv_len && tok < max_seq_len;
                    for (int32_t d = 0; d < D; ++d) {
                        kt[n * D + d] = ok ? h2f(kh[(int64_t)tok * D + d]) : 0.0f;
                        vt[n * D + d] = ok ? h2f(vh[(int64_t)tok * D + d]) : 0.0f;
                    }
                }
                for (int32_t r = 0; r < m_eff; ++r) {
                    const int32_t mpos = query_start + b * BM + r / GR;
                    float rmax = 0.0f - 1.0e30f;
                    for (int32_t n = 0; n < BN; ++n) {
                        float dot = 0.0f;
                        for (int32_t d = 0; d < D; ++d) dot += qf[(int64_t)r * D + d] * kt[n * D + d];
                        if (j >= mask_start) {
                            const int32_t na = j * BN + n;
                            const int keep = na < kv_len && mpos >= na;
                            dot = dot + (keep ? 0.0f : 0.0f - 1.0e30f);
                        }
                        qk[(int64_t)r * BN + n] = dot;
                        rmax = n == 0 ? dot : fmaxf(rmax, dot);
                    }
                    const float m_ij = fmaxf(mi[r], rmax * c);
                    float l_ij = 0.0f;
                    for (int32_t n = 0; n < BN; ++n) {
                        const float p = exp2f(qk[(int64_t)r * BN + n] * c - m_ij);
                        l_ij += p;
                        ph[(int64_t)r * BN + n] = go_f32_to_f16(p);
                    }
                    const float alpha = exp2f(mi[r] - m_ij);
                    li[r] = li[r] * alpha + l_ij;
                    for (int32_t d = 0; d < D; ++d) {
                        float a = acc[(int64_t)r * D + d] * alpha;
                        float pv = 0.0f;
                        for (int32_t n = 0; n < BN; ++n) pv += h2f(ph[(int64_t)r * BN + n]) * vt[n * D + d];
                        acc[(int64_t)r * D + d] = a + pv;
                    }
                    mi[r] = m_ij;
                }
            }
            const int64_t base = tile * (int64_t)NKS * m_eff + (int64_t)split * m_eff;
            for (int32_t r = 0; r < m_eff; ++r) {
                const float l_safe = fmaxf(li[r], 1.0e-8f);
                for (int32_t d = 0; d < D; ++d)
                    att_partial[(base + r) * D + d] = go_f32_to_f16(acc[(int64_t)r * D + d] / l_safe);
                lse_partial[base + r] = mi[r] + log2f(l_safe);
            }
        }
        free(qf); free(acc); free(qk); free(kt); free(vt); free(ph); free(mi); free(li);
    }
}

/* src/kernels.rs:2151-2323 prefill_splitk_reduce_merge: per tile row r,
 * w_s = 2^(lse_s - max_s lse) / max(sum, 1e-8) (:2273-2289) and
 * out[row, head, :] = f16(sum_s w_s * f32(att_s)) (:2291-2320), written for
 * rows below q_len only. */
void go_attn_prefill_split_merge(const uint16_t* att_partial, const float* lse_partial,
                                 uint16_t* out, int32_t num_q_heads, int32_t head_dim,
                                 int32_t q_len, int32_t block_m, int32_t group,
                                 int32_t num_splits) {
    const int32_t D = head_dim, BM = block_m, GR = group, NKS = num_splits;
    const int32_t num_q_blocks = (q_len + BM - 1) / BM;
    const int32_t num_head_groups = num_q_heads / GR;
    const int32_t m_eff = BM * GR;
    float* w = (float*)malloc((size_t)NKS * sizeof(float));
    for (int64_t tile = 0; tile < (int64_t)num_q_blocks * num_head_groups; ++tile) {
        const int32_t b = (int32_t)(tile / num_head_groups);
        const int32_t hg = (int32_t)(tile % num_head_groups);
        for (int32_t r = 0; r < m_eff; ++r) {
            const int32_t row = b * BM + r / GR, head = hg * GR + r % GR;
            if (row >= q_len) continue;
            const float* lse = lse_partial + tile * (int64_t)NKS * m_eff;
            float mx = lse[r];
            for (int32_t s = 1; s < NKS; ++s) mx = fmaxf(mx, lse[(int64_t)s * m_eff + r]);
            float sum = 0.0f;
            for (int32_t s = 0; s < NKS; ++s) {
                w[s] = exp2f(lse[(int64_t)s * m_eff + r] - mx);
                sum += w[s];
            }
            const float safe = fmaxf(sum, 1.0e-8f);
            for (int32_t s = 0; s < NKS; ++s) w[s] = w[s] / safe;
            for (int32_t d = 0; d < D; ++d) {
                float a = 0.0f;
                for (int32_t s = 0; s < NKS; ++s) {
                    const int64_t prow = tile * (int64_t)NKS * m_eff + (int64_t)s * m_eff + r;
                    a += h2f(att_partial[prow * D + d]) * w[s];
                }
                out[((int64_t)row * num_q_heads + head) * D + d] = go_f32_to_f16(a);
            }
        }
    }
    free(w);
}

/* ------------------------------------------------------ decode-layer ops -- */

/* src/kernels.rs:3076-3216 add_rms_norm_decode_raw_f16 (one row of n):
 * combined = f32(residual) + f32(x) (:3143-3146), ss = sum combined^2 (f32,
 * sequential here; the reference's order is a per-lane sum then a tree),
 * inv = 1 / sqrt(ss/n + eps) (:3149-3153), out = f16(combined*inv*w),
 * residual_out = f16(combined) (:3183-3188). */
void go_add_rms_norm(const uint16_t* residual, const uint16_t* x, const uint16_t* w,
                     uint16_t* out, uint16_t* residual_out, float eps, int32_t n) {
    float ss = 0.0f;
    for (int32_t i = 0; i < n; ++i) {
        float c = h2f(residual[i]) + h2f(x[i]);
        ss += c * c;
    }
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int32_t i = 0; i < n; ++i) {
        float c = h2f(residual[i]) + h2f(x[i]);
        out[i] = go_f32_to_f16((c * inv) * h2f(w[i]));
        residual_out[i] = go_f32_to_f16(c);
    }
}

/* src/cublas.rs:260-345, 572-607 GemvInPlace: cublasGemmEx(OP_T, OP_N, m, 1,
 * k) over a row-major [m, k] f16 matrix: out[i] = f16(sum_j W[i][j] x[j]),
 * f32 accumulation (CUBLAS_COMPUTE_32F_FAST_16F, the default at :74). */
void go_gemv_f16(const uint16_t* w, const uint16_t* x, uint16_t* out, int32_t m, int32_t k,
                 int32_t nthreads) {
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for num_threads(nt) schedule(static)
#endif
    for (int32_t i = 0; i < m; ++i) {
        const uint16_t* row = w + (int64_t)i * k;
        float acc = 0.0f;
        for (int32_t j = 0; j < k; ++j) acc += h2f(row[j]) * h2f(x[j]);
        out[i] = go_f32_to_f16(acc);
    }
    (void)nthreads;
}

/* src/kernels.rs:345-392 argmax_blocks_f16 + :458-505
 * argmax_reduce_blocks_to_u32: the largest f32(logit) over [0, n), the lowest
 * index among equal maxima (reduce_max, then reduce_min over the indices
 * equal to it).  NaN logits are never chosen; 0 if every logit is NaN. */
uint32_t go_argmax_f16(const uint16_t* logits, int32_t n) {
    int64_t best = -1;
    float bv = 0.0f;
    for (int32_t i = 0; i < n; ++i) {
        float v = h2f(logits[i]);
        if (v != v) continue;
        if (best < 0 || v > bv) {
            bv = v;
            best = i;
        }
    }
    return best < 0 ? 0u : (uint32_t)best;
}

/* src/kernels.rs:271-301 silu_mul_2d_f16: y = f16((sigmoid(g) * g) * u) in
 * f32, sigmoid(g) = 1 / (1 + exp(-g)) (:288-293). */
void go_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, int32_t n) {
    for (int32_t i = 0; i < n; ++i) {
        const float g = h2f(gate[i]);
        const float sig = 1.0f / (1.0f + expf(-g));
        out[i] = go_f32_to_f16((sig * g) * h2f(up[i]));
    }
}

/* src/loader.rs:107-145 cast_to_f16: F16 bit copy; BF16 -> f32 (exact) ->
 * f16::from_f32; F32 -> f16::from_f32; F64 -> `x as f32` -> f16::from_f32.
 * dtype codes: 0 F16, 1 BF16, 2 F32, 3 F64.  Returns -1 on an unknown dtype. */
int32_t go_cast_to_f16(const void* src, int32_t dtype, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        switch (dtype) {
            case 0: out[i] = ((const uint16_t*)src)[i]; break;
            case 1: {
                uint32_t bits = (uint32_t)((const uint16_t*)src)[i] << 16;
                float f;
                memcpy(&f, &bits, 4);
                out[i] = go_f32_to_f16(f);
                break;
            }
            case 2: out[i] = go_f32_to_f16(((const float*)src)[i]); break;
            case 3: out[i] = go_f32_to_f16((float)((const double*)src)[i]); break;
            default: return -1;
        }
    }
    return 0;
}

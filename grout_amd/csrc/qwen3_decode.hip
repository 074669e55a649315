// The whole Qwen3 decode token step as one hipGraph: grout's
// DecodeCudaGraphRunner (src/model.rs:318-493, graph recorded at
// :3118-3648) with every node a kernel of this library.
//
// Per replay: embedding + input RMSNorm of the token the previous replay
// picked; for each layer [add + input RMSNorm] -> qkv GEMV -> fused QK
// norm/RoPE/KV write + split-K decode + merge -> o_proj GEMV -> add +
// post-attention RMSNorm -> gate_up GEMV with SiLU * up -> down GEMV; then the
// final add + RMSNorm, the lm_head GEMV and the greedy argmax, which writes
// the next token where the embedding reads it.  The last layer's attention
// advances the device position, so consecutive replays need no host writes.
//
// The residual stream follows the reference's buffers: the residual add of
// each sub-layer is deferred into the next norm (hidden -> hidden_after_attn
// -> hidden), src/model.rs:3133-3164, :3513-3526, :3568-3585.
#include <new>
#include <vector>

#include "abi_util.h"
#include "common.h"

using namespace grout;

namespace {

// Device workspace carved into the step's activations and scratch; every
// buffer starts on a 256-byte boundary.
struct Qwen3Workspace {
    int64_t hidden, hidden_after_attn, normed, qkv, q_out, attn_out, attn_proj, ff, ff_down, att_partial, lse_partial, counters, block_max, block_idx, total;
};

int64_t align256(int64_t v) { return (v + 255) & ~int64_t{255}; }

int32_t check_model(const grout_qwen3_model& M) {
    GROUT_REQUIRE(M.layers != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE(M.num_layers >= 1, GROUT_ERR_ARG);
    GROUT_REQUIRE(M.num_q_heads > 0 && M.num_kv_heads > 0 && M.num_q_heads % M.num_kv_heads == 0,
                  GROUT_ERR_HEADS);
    GROUT_REQUIRE(M.head_dim == GROUT_HEAD_DIM, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(M.hidden >= 8 && M.hidden % 8 == 0 && M.intermediate >= 8 &&
                      M.intermediate % 8 == 0 && M.vocab >= 1,
                  GROUT_ERR_ARG);
    GROUT_REQUIRE(M.max_seq_len >= 1, GROUT_ERR_SEQ_RANGE);
    return GROUT_OK;
}

int32_t layout(const grout_qwen3_model& M, Qwen3Workspace* w) {
    const int32_t st = check_model(M);
    if (st != GROUT_OK) return st;
    const int32_t group = M.num_q_heads / M.num_kv_heads;
    const int64_t partial = grout_attn_decode_partial_bytes(M.num_kv_heads, group, M.head_dim,
                                                            M.num_splits);
    const int64_t lse = grout_attn_decode_lse_bytes(M.num_kv_heads, group, M.num_splits);
    const int64_t nblk = grout_argmax_blocks(M.vocab);
    if (partial < 0 || lse < 0) return GROUT_ERR_SPLITS;
    if (nblk < 0) return GROUT_ERR_ARG;
    const int64_t h2 = int64_t{2} * M.hidden;
    const int64_t d = M.head_dim;
    int64_t at = 0;
    auto take = [&at](int64_t bytes) {
        const int64_t off = at;
        at = align256(at + bytes);
        return off;
    };
    w->hidden = take(h2);
    w->hidden_after_attn = take(h2);
    w->normed = take(h2);
    w->qkv = take(2 * d * (M.num_q_heads + 2 * M.num_kv_heads));
    w->q_out = take(2 * d * (M.num_q_heads + M.num_kv_heads));
    w->attn_out = take(2 * d * M.num_q_heads);
    w->attn_proj = take(h2);
    w->ff = take(int64_t{2} * M.intermediate);
    w->ff_down = take(h2);
    w->att_partial = take(partial);
    w->lse_partial = take(lse);
    w->counters = take(grout_attn_decode_counter_bytes(M.num_kv_heads));
    w->block_max = take(4 * nblk);
    w->block_idx = take(4 * nblk);
    w->total = at;
    return GROUT_OK;
}

template <typename T>
T* at(void* base, int64_t off) {
    return reinterpret_cast<T*>(static_cast<unsigned char*>(base) + off);
}

}  // namespace

struct grout_qwen3_runner {
    grout_qwen3_model model;
    std::vector<grout_qwen3_layer> layers;
    hipStream_t stream = nullptr;
    grout_graph* graph = nullptr;
};

extern "C" int64_t grout_qwen3_workspace_bytes(const grout_qwen3_model* model) {
    if (model == nullptr) return GROUT_ERR_NULL_POINTER;
    Qwen3Workspace w;
    const int32_t st = layout(*model, &w);
    return st == GROUT_OK ? w.total : st;
}

// Records (or runs) one token step in stream order.  Every op validates its
// own arguments; the first failure is returned.
extern "C" int32_t grout_qwen3_decode_step(const grout_qwen3_model* model,
                                           grout_stream_t stream) {
    GROUT_REQUIRE(model != nullptr, GROUT_ERR_NULL_POINTER);
    const grout_qwen3_model& M = *model;
    Qwen3Workspace w;
    int32_t st = layout(M, &w);
    if (st != GROUT_OK) return st;
    GROUT_REQUIRE(M.workspace != nullptr && M.token != nullptr && M.d_position != nullptr,
                  GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(M.workspace) & 255u) == 0, GROUT_ERR_ALIGNMENT);
    void* ws = M.workspace;
    uint16_t* hidden = at<uint16_t>(ws, w.hidden);
    uint16_t* hidden_after_attn = at<uint16_t>(ws, w.hidden_after_attn);
    uint16_t* normed = at<uint16_t>(ws, w.normed);
    uint16_t* qkv = at<uint16_t>(ws, w.qkv);
    uint16_t* q_out = at<uint16_t>(ws, w.q_out);
    uint16_t* attn_out = at<uint16_t>(ws, w.attn_out);
    uint16_t* attn_proj = at<uint16_t>(ws, w.attn_proj);
    uint16_t* ff = at<uint16_t>(ws, w.ff);
    uint16_t* ff_down = at<uint16_t>(ws, w.ff_down);
    uint16_t* att_partial = at<uint16_t>(ws, w.att_partial);
    float* lse_partial = at<float>(ws, w.lse_partial);
    uint32_t* counters = at<uint32_t>(ws, w.counters);
    float* block_max = at<float>(ws, w.block_max);
    uint32_t* block_idx = at<uint32_t>(ws, w.block_idx);
    const int32_t qkv_rows = M.head_dim * (M.num_q_heads + 2 * M.num_kv_heads);
    const int32_t attn_width = M.head_dim * M.num_q_heads;

    // src/model.rs:3120-3149: embedding, then the plain RMSNorm of layer 0.
    st = grout_embed_rms_norm_decode(M.token, M.embed_tokens, M.vocab, M.layers[0].input_norm,
                                     normed, hidden, M.eps, M.hidden, stream);
    for (int32_t l = 0; st == GROUT_OK && l < M.num_layers; ++l) {
        const grout_qwen3_layer& L = M.layers[l];
        if (l > 0) {  // :3151-3163 fold the previous layer's MLP residual in
            st = grout_add_rms_norm_decode(hidden_after_attn, ff_down, L.input_norm, normed,
                                           hidden, M.eps, M.hidden, stream);
            if (st != GROUT_OK) break;
        }
        st = grout_gemv_f16(L.qkv_proj, normed, qkv, qkv_rows, M.hidden, stream);  // :3170-3176
        if (st != GROUT_OK) break;
        st = grout_attn_decode_fused(qkv, L.q_norm, L.k_norm, M.inv_freq, q_out, L.k_cache,
                                     L.v_cache, att_partial, lse_partial, attn_out, counters,
                                     M.d_position, M.eps, M.qk_scale_f16, M.num_q_heads,
                                     M.num_kv_heads, M.head_dim, M.max_seq_len, M.block_n,
                                     M.num_splits, l == M.num_layers - 1 ? 1 : 0, stream);
        if (st != GROUT_OK) break;
        st = grout_gemv_f16(L.o_proj, attn_out, attn_proj, M.hidden, attn_width, stream);
        if (st != GROUT_OK) break;  // :3505-3511
        st = grout_add_rms_norm_decode(hidden, attn_proj, L.post_attn_norm, normed,
                                       hidden_after_attn, M.eps, M.hidden, stream);
        if (st != GROUT_OK) break;  // :3513-3526
        // :3529-3535 gate_up GEMV and :3556-3565 SiLU * up, in one launch.
        st = grout_gemv_silu_mul_f16(L.gate_up_proj, normed, ff, M.intermediate, M.hidden, stream);
        if (st != GROUT_OK) break;
        st = grout_gemv_f16(L.down_proj, ff, ff_down, M.hidden, M.intermediate, stream);
    }                               // :3568-3574
    if (st != GROUT_OK) return st;
    // :3580-3594 final add + RMSNorm; :3612-3640 lm_head GEMV and argmax.
    st = grout_add_rms_norm_decode(hidden_after_attn, ff_down, M.final_norm, normed, hidden, M.eps,
                                   M.hidden, stream);
    if (st != GROUT_OK) return st;
    st = grout_gemv_f16(M.lm_head, normed, M.logits, M.vocab, M.hidden, stream);
    if (st != GROUT_OK) return st;
    return grout_argmax_f16(M.logits, block_max, block_idx, M.token, M.vocab, stream);
}

extern "C" int32_t grout_qwen3_runner_create(const grout_qwen3_model* model,
                                             uint32_t prime_position, grout_stream_t stream,
                                             grout_qwen3_runner** runner) {
    GROUT_REQUIRE(model != nullptr && runner != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE(stream != nullptr, GROUT_ERR_GRAPH);
    *runner = nullptr;
    Qwen3Workspace w;
    int32_t st = layout(*model, &w);
    if (st != GROUT_OK) return st;
    GROUT_REQUIRE(prime_position < static_cast<uint32_t>(model->max_seq_len), GROUT_ERR_SEQ_RANGE);
    GROUT_REQUIRE(model->workspace != nullptr, GROUT_ERR_NULL_POINTER);
    grout_qwen3_runner* r = new (std::nothrow) grout_qwen3_runner;
    if (r == nullptr) return GROUT_ERR_GRAPH;
    r->layers.assign(model->layers, model->layers + model->num_layers);
    r->model = *model;
    r->model.layers = r->layers.data();  // the caller's array need not outlive the runner
    r->stream = to_hip(stream);
    // The attention counters must start at zero; the fused kernel leaves them so.
    hipError_t e = hipMemsetAsync(at<unsigned char>(model->workspace, w.counters), 0,
                                  static_cast<size_t>(w.block_max - w.counters), r->stream);
    // Prime pass (src/model.rs:2561-3115): every op once, eagerly, so argument
    // errors surface outside capture.  It writes the caches at prime_position,
    // replaces *token and advances the position, as a step does.
    if (e == hipSuccess) {
        st = grout_set_position_async(model->d_position, prime_position, stream);
        if (st == GROUT_OK) st = grout_qwen3_decode_step(&r->model, stream);
        if (st == GROUT_OK) {
            e = hipStreamSynchronize(r->stream);
            if (e != hipSuccess) st = static_cast<int32_t>(e);
        }
    } else {
        st = static_cast<int32_t>(e);
    }
    if (st == GROUT_OK) st = grout_graph_begin(stream);
    if (st != GROUT_OK) {
        delete r;
        return st;
    }
    const int32_t rec = grout_qwen3_decode_step(&r->model, stream);
    grout_graph* g = nullptr;
    st = grout_graph_end(stream, &g);
    if (rec != GROUT_OK || st != GROUT_OK) {
        grout_graph_destroy(g);
        delete r;
        return rec != GROUT_OK ? rec : st;
    }
    r->graph = g;
    *runner = r;
    return GROUT_OK;
}

extern "C" int32_t grout_qwen3_runner_seed_token(grout_qwen3_runner* runner, uint32_t token) {
    GROUT_REQUIRE(runner != nullptr && runner->graph != nullptr, GROUT_ERR_GRAPH);
    GROUT_REQUIRE(token < static_cast<uint32_t>(runner->model.vocab), GROUT_ERR_ARG);
    return grout_set_position_async(runner->model.token, token,
                                    reinterpret_cast<grout_stream_t>(runner->stream));
}

extern "C" int32_t grout_qwen3_runner_step(grout_qwen3_runner* runner, uint32_t position,
                                           uint32_t* token_out) {
    GROUT_REQUIRE(runner != nullptr && runner->graph != nullptr, GROUT_ERR_GRAPH);
    GROUT_REQUIRE(position < static_cast<uint32_t>(runner->model.max_seq_len),
                  GROUT_ERR_SEQ_RANGE);
    // launch_step writes the position on every step (src/model.rs:363-403):
    // the device copy may have been moved outside the runner (an eager step,
    // the caller).
    grout_stream_t gs = reinterpret_cast<grout_stream_t>(runner->stream);
    int32_t st = grout_set_position_async(runner->model.d_position, position, gs);
    if (st == GROUT_OK) st = grout_graph_launch(runner->graph, gs);
    if (st != GROUT_OK) return st;
    if (token_out == nullptr) return GROUT_OK;
    // launch_step (src/model.rs:363-403): 4-byte read-back of the new token.
    hipError_t e = hipMemcpyAsync(token_out, runner->model.token, 4, hipMemcpyDeviceToHost,
                                  runner->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(runner->stream);
    return e == hipSuccess ? GROUT_OK : static_cast<int32_t>(e);
}

extern "C" int32_t grout_qwen3_runner_run(grout_qwen3_runner* runner, uint32_t first_position,
                                          int32_t count) {
    GROUT_REQUIRE(runner != nullptr && runner->graph != nullptr, GROUT_ERR_GRAPH);
    GROUT_REQUIRE(count >= 0, GROUT_ERR_ARG);
    if (count == 0) return GROUT_OK;
    GROUT_REQUIRE(static_cast<uint64_t>(first_position) + static_cast<uint64_t>(count) <=
                      static_cast<uint64_t>(runner->model.max_seq_len),
                  GROUT_ERR_SEQ_RANGE);
    // The first step writes the position; each replay advances it in the
    // graph and nothing else runs on the runner's stream in between.
    int32_t st = grout_qwen3_runner_step(runner, first_position, nullptr);
    grout_stream_t gs = reinterpret_cast<grout_stream_t>(runner->stream);
    for (int32_t i = 1; st == GROUT_OK && i < count; ++i) st = grout_graph_launch(runner->graph, gs);
    return st;
}

extern "C" int32_t grout_qwen3_runner_destroy(grout_qwen3_runner* runner) {
    if (runner == nullptr) return GROUT_OK;
    // Replays still queued on the runner's stream use the graph and the
    // caller's buffers: let them finish first.
    const hipError_t e = hipStreamSynchronize(runner->stream);
    const int32_t st = grout_graph_destroy(runner->graph);
    delete runner;
    if (e != hipSuccess) return static_cast<int32_t>(e);
    return st;
}

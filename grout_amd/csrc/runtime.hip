// Host runtime around the kernels: status strings, the RoPE table, device
// queries, hipGraph capture helpers and the decode graph runner.
//
// Replaces, for the attention slice, cuda-async's CudaGraph::scope/launch and
// grout's DecodeCudaGraphRunner (src/model.rs:318-493, capture at
// :3118-3648): the runner records {fused QK norm/RoPE/KV write, split-K
// decode, merge} once after a prime pass and replays them per token with only
// the device position rewritten.
#include <math.h>

#include <new>

#include "abi_util.h"
#include "common.h"

namespace grout {

__global__ void set_u32_kernel(uint32_t* p, uint32_t value) { *p = value; }

}  // namespace grout

using namespace grout;

struct grout_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

struct grout_decode_runner {
    grout_decode_layer layer;
    hipStream_t stream = nullptr;
    grout_graph* graph = nullptr;
};

extern "C" const char* grout_status_string(int32_t status) {
    switch (status) {
        case GROUT_OK: return "ok";
        case GROUT_ERR_NULL_POINTER: return "a required pointer is NULL";
        case GROUT_ERR_ALIGNMENT: return "a tensor pointer is not 16-byte aligned";
        case GROUT_ERR_HEAD_DIM: return "head_dim must be 128";
        case GROUT_ERR_HEADS: return "invalid head counts (num_q_heads % num_kv_heads != 0)";
        case GROUT_ERR_SEQ_RANGE: return "position range exceeds max_seq_len";
        case GROUT_ERR_KV_LEN: return "kv_len / query_start / q_len out of range";
        case GROUT_ERR_GROUP: return "decode query group outside [1, 16]";
        case GROUT_ERR_SPLITS: return "num_splits or block_n out of range";
        case GROUT_ERR_ARG: return "invalid scalar argument";
        case GROUT_ERR_GRAPH: return "invalid graph handle or capture state";
        case GROUT_ERR_SCRATCH:
            return "the call needs more than the library's static scratch (GROUT_NOALLOC_SCRATCH_BYTES)";
        default: break;
    }
    if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
    return "unknown status";
}

extern "C" int32_t grout_build_inv_freq(float theta, int32_t head_dim, float* out_host) {
    GROUT_REQUIRE(out_host != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE(head_dim > 0 && head_dim % 2 == 0, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(theta > 0.0f, GROUT_ERR_ARG);
    // src/model.rs:5994-5997: p = i as f32 / D as f32; 1.0 / theta.powf(p).
    for (int32_t i = 0; i < head_dim; i += 2) {
        const float p = static_cast<float>(i) / static_cast<float>(head_dim);
        out_host[i / 2] = 1.0f / powf(theta, p);
    }
    return GROUT_OK;
}

extern "C" int32_t grout_device_cu_count(int32_t device, int32_t* cu_count) {
    GROUT_REQUIRE(cu_count != nullptr, GROUT_ERR_NULL_POINTER);
    int v = 0;
    hipError_t e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return static_cast<int32_t>(e);
    *cu_count = v;
    return GROUT_OK;
}

extern "C" int32_t grout_set_position_async(uint32_t* d_position, uint32_t position,
                                            grout_stream_t stream) {
    GROUT_REQUIRE(d_position != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(d_position) & 3u) == 0, GROUT_ERR_ALIGNMENT);
    hipLaunchKernelGGL(set_u32_kernel, dim3(1), dim3(1), 0, to_hip(stream), d_position, position);
    return launch_status();
}

extern "C" int32_t grout_graph_begin(grout_stream_t stream) {
    GROUT_REQUIRE(stream != nullptr, GROUT_ERR_GRAPH);  // the legacy stream cannot capture
    hipError_t e = hipStreamBeginCapture(to_hip(stream), hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? GROUT_OK : static_cast<int32_t>(e);
}

extern "C" int32_t grout_graph_end(grout_stream_t stream, grout_graph** graph) {
    GROUT_REQUIRE(stream != nullptr && graph != nullptr, GROUT_ERR_GRAPH);
    *graph = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(to_hip(stream), &g);
    if (e != hipSuccess) return static_cast<int32_t>(e);
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return static_cast<int32_t>(e);
    }
    grout_graph* out = new (std::nothrow) grout_graph;
    if (out == nullptr) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(g);
        return GROUT_ERR_GRAPH;
    }
    out->graph = g;
    out->exec = exec;
    *graph = out;
    return GROUT_OK;
}

extern "C" int32_t grout_graph_launch(grout_graph* graph, grout_stream_t stream) {
    GROUT_REQUIRE(graph != nullptr && graph->exec != nullptr, GROUT_ERR_GRAPH);
    hipError_t e = hipGraphLaunch(graph->exec, to_hip(stream));
    return e == hipSuccess ? GROUT_OK : static_cast<int32_t>(e);
}

extern "C" int32_t grout_graph_destroy(grout_graph* graph) {
    if (graph == nullptr) return GROUT_OK;
    hipError_t e1 = graph->exec ? hipGraphExecDestroy(graph->exec) : hipSuccess;
    hipError_t e2 = graph->graph ? hipGraphDestroy(graph->graph) : hipSuccess;
    delete graph;
    if (e1 != hipSuccess) return static_cast<int32_t>(e1);
    return e2 == hipSuccess ? GROUT_OK : static_cast<int32_t>(e2);
}

// The decode step of one layer: the fused norm/RoPE/KV write + split + merge
// (src/model.rs:3194-3221, :3428-3473 in one launch), advancing the position.
static int32_t record_decode_step(const grout_decode_layer& L, hipStream_t s) {
    return grout_attn_decode_fused(L.qkv, L.q_weight, L.k_weight, L.inv_freq, L.q_out, L.k_cache,
                                   L.v_cache, L.att_partial, L.lse_partial, L.attn_out, L.counters,
                                   L.d_position, L.eps, L.qk_scale_f16, L.num_q_heads,
                                   L.num_kv_heads, L.head_dim, L.max_seq_len, L.block_n,
                                   L.num_splits, 1, reinterpret_cast<grout_stream_t>(s));
}

extern "C" int32_t grout_decode_runner_create(const grout_decode_layer* layer,
                                              uint32_t prime_position, grout_stream_t stream,
                                              grout_decode_runner** runner) {
    GROUT_REQUIRE(layer != nullptr && runner != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE(stream != nullptr, GROUT_ERR_GRAPH);
    *runner = nullptr;
    const grout_decode_layer& L = *layer;
    GROUT_REQUIRE_PTR(L.attn_out);
    GROUT_REQUIRE(L.counters != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE(L.num_q_heads > 0 && L.num_kv_heads > 0 && L.num_q_heads % L.num_kv_heads == 0,
                  GROUT_ERR_HEADS);
    GROUT_REQUIRE(prime_position < static_cast<uint32_t>(L.max_seq_len > 0 ? L.max_seq_len : 0),
                  GROUT_ERR_SEQ_RANGE);
    hipStream_t s = to_hip(stream);
    // Prime pass: run every op once eagerly so argument errors surface
    // outside capture (src/model.rs:2561-3115).
    int32_t st = grout_set_position_async(L.d_position, prime_position, stream);
    if (st != GROUT_OK) return st;
    st = record_decode_step(L, s);
    if (st != GROUT_OK) return st;
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return static_cast<int32_t>(e);

    st = grout_graph_begin(stream);
    if (st != GROUT_OK) return st;
    int32_t rec = record_decode_step(L, s);
    grout_graph* g = nullptr;
    st = grout_graph_end(stream, &g);
    if (rec != GROUT_OK) {
        grout_graph_destroy(g);
        return rec;
    }
    if (st != GROUT_OK) return st;
    grout_decode_runner* r = new (std::nothrow) grout_decode_runner;
    if (r == nullptr) {
        grout_graph_destroy(g);
        return GROUT_ERR_GRAPH;
    }
    r->layer = L;
    r->stream = s;
    r->graph = g;
    *runner = r;
    return GROUT_OK;
}

extern "C" int32_t grout_decode_runner_step(grout_decode_runner* runner, uint32_t position) {
    GROUT_REQUIRE(runner != nullptr && runner->graph != nullptr, GROUT_ERR_GRAPH);
    // src/model.rs:363-376 ensures the position fits; the cache bound is the
    // engine's max_seq_len.
    GROUT_REQUIRE(position < static_cast<uint32_t>(runner->layer.max_seq_len), GROUT_ERR_SEQ_RANGE);
    // The position is written on every step, as launch_step does
    // (src/model.rs:363-403): the device copy may have been moved by anything
    // outside the runner (an eager step, the caller).
    grout_stream_t gs = reinterpret_cast<grout_stream_t>(runner->stream);
    const int32_t st = grout_set_position_async(runner->layer.d_position, position, gs);
    if (st != GROUT_OK) return st;
    return grout_graph_launch(runner->graph, gs);
}

extern "C" int32_t grout_decode_runner_run(grout_decode_runner* runner, uint32_t first_position,
                                           int32_t count) {
    GROUT_REQUIRE(runner != nullptr && runner->graph != nullptr, GROUT_ERR_GRAPH);
    GROUT_REQUIRE(count >= 0, GROUT_ERR_ARG);
    if (count == 0) return GROUT_OK;
    GROUT_REQUIRE(static_cast<uint64_t>(first_position) + static_cast<uint64_t>(count) <=
                      static_cast<uint64_t>(runner->layer.max_seq_len),
                  GROUT_ERR_SEQ_RANGE);
    // The first step writes the position; every replay advances the device
    // position itself, and nothing else runs on the runner's stream in
    // between, so the following replays need no host write.
    int32_t st = grout_decode_runner_step(runner, first_position);
    grout_stream_t gs = reinterpret_cast<grout_stream_t>(runner->stream);
    for (int32_t i = 1; st == GROUT_OK && i < count; ++i) st = grout_graph_launch(runner->graph, gs);
    return st;
}

extern "C" int32_t grout_decode_runner_zero_kv(grout_decode_runner* runner) {
    GROUT_REQUIRE(runner != nullptr, GROUT_ERR_GRAPH);
    const grout_decode_layer& L = runner->layer;
    const size_t bytes = static_cast<size_t>(L.num_kv_heads) * L.max_seq_len * L.head_dim * 2;
    hipError_t e = hipMemsetAsync(L.k_cache, 0, bytes, runner->stream);
    if (e == hipSuccess) e = hipMemsetAsync(L.v_cache, 0, bytes, runner->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(runner->stream);
    return e == hipSuccess ? GROUT_OK : static_cast<int32_t>(e);
}

extern "C" int32_t grout_decode_runner_destroy(grout_decode_runner* runner) {
    if (runner == nullptr) return GROUT_OK;
    // Replays still queued on the runner's stream use the graph and the
    // caller's buffers: let them finish first.
    const hipError_t e = hipStreamSynchronize(runner->stream);
    int32_t st = grout_graph_destroy(runner->graph);
    delete runner;
    if (e != hipSuccess) return static_cast<int32_t>(e);
    return st;
}

// Unfused KV-cache suffix writer: rows [position_start, position_start+seq_len)
// of every KV head's cache take new_k/new_v, bit for bit.
//
// Replaces kv_cache_update_seq_f16 (src/kernels.rs:759-800, host position,
// launched at src/model.rs:5464-5480 for chunked prefill and MTP suffixes) and
// kv_cache_update_seq_dynpos_f16 (src/kernels.rs:807-846, device position,
// the graph-captured decode path at src/model.rs:5483-5502).
//   new_k/new_v [seq_len, num_kv_heads, head_dim] f16, contiguous;
//   k_cache/v_cache [num_kv_heads, max_seq_len, head_dim] f16.
// HBM-bound copy: every thread moves one 16-byte (or, for head_dim % 8 != 0,
// 8-byte) unit of K and the same unit of V; consecutive threads cover one
// head's rows of a 16-token tile, so the cache side is written in long
// contiguous runs.
#include "abi_util.h"
#include "common.h"

namespace grout {

// Tokens per tile.  Lane i enumerates [token tile][head][token in tile][unit],
// so the 256 lanes of a workgroup (head_dim 128: 16 tokens x 16 units) write
// one head's 16 consecutive cache rows, 4 KB contiguous, and read 256-byte
// rows 2 KB apart that the neighbouring workgroups (the other heads of the
// tile) read beside them.  Row-major lanes (512-byte pieces of eight heads
// per workgroup) measured 2% slower with the data in HBM and 6% with it in
// the last-level cache (c3 shapes).
constexpr int kKvTileTokens = 16;

template <typename Unit, bool kDevicePos>
__global__ __launch_bounds__(256) void kv_cache_update_kernel(
    const Unit* __restrict__ new_k, const Unit* __restrict__ new_v, Unit* __restrict__ k_cache,
    Unit* __restrict__ v_cache, int position_start, const uint32_t* __restrict__ d_position,
    int64_t total_units, int units_per_row, int num_kv_heads, int max_seq_len, int seq_len) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= total_units) return;
    const int u = static_cast<int>(i % units_per_row);
    const int64_t r = i / units_per_row;
    const int t_in = static_cast<int>(r % kKvTileTokens);
    const int64_t ht = r / kKvTileTokens;  // = tile * num_kv_heads + h
    const int h = static_cast<int>(ht % num_kv_heads);
    const int64_t s = (ht / num_kv_heads) * kKvTileTokens + t_in;
    if (s >= seq_len) return;  // the last tile is ragged
    int64_t pos;
    if constexpr (kDevicePos) {
        pos = static_cast<int64_t>(*d_position) + s;
        if (pos >= max_seq_len) return;  // bounds guard: a slot past the cache is not written
    } else {
        pos = position_start + s;
    }
    const int64_t src = (s * num_kv_heads + h) * units_per_row + u;
    const int64_t dst = (static_cast<int64_t>(h) * max_seq_len + pos) * units_per_row + u;
    // Non-temporal stores: the rows are not read again by this kernel, and
    // streaming them past the caches measured 5% faster with the data in HBM
    // (c3: 14.4 -> 13.6 us) and 7% with it in the last-level cache.
    // (Non-temporal loads lose whenever the new rows are still cached from
    // their producer.)
    __builtin_nontemporal_store(new_k[src], k_cache + dst);
    __builtin_nontemporal_store(new_v[src], v_cache + dst);
}

template <bool kDevicePos>
static int32_t launch_kv_update(const uint16_t* new_k, const uint16_t* new_v, uint16_t* k_cache,
                                uint16_t* v_cache, int32_t position_start,
                                const uint32_t* d_position, int32_t seq_len,
                                int32_t num_kv_heads, int32_t head_dim, int32_t max_seq_len,
                                hipStream_t stream) {
    const bool wide = head_dim % 8 == 0;
    const int units_per_row = wide ? head_dim / 8 : head_dim / 4;
    const int64_t tiles = (static_cast<int64_t>(seq_len) + kKvTileTokens - 1) / kKvTileTokens;
    const int64_t total = tiles * kKvTileTokens * num_kv_heads * units_per_row;
    if (total == 0) return GROUT_OK;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) return GROUT_ERR_SEQ_RANGE;
    if (wide) {
        hipLaunchKernelGGL((kv_cache_update_kernel<uint4_t, kDevicePos>), dim3(static_cast<unsigned>(blocks)),
                           dim3(256), 0, stream, reinterpret_cast<const uint4_t*>(new_k),
                           reinterpret_cast<const uint4_t*>(new_v), reinterpret_cast<uint4_t*>(k_cache),
                           reinterpret_cast<uint4_t*>(v_cache), position_start, d_position, total,
                           units_per_row, num_kv_heads, max_seq_len, seq_len);
    } else {
        typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));
        hipLaunchKernelGGL((kv_cache_update_kernel<uint2_t, kDevicePos>), dim3(static_cast<unsigned>(blocks)),
                           dim3(256), 0, stream, reinterpret_cast<const uint2_t*>(new_k),
                           reinterpret_cast<const uint2_t*>(new_v), reinterpret_cast<uint2_t*>(k_cache),
                           reinterpret_cast<uint2_t*>(v_cache), position_start, d_position, total,
                           units_per_row, num_kv_heads, max_seq_len, seq_len);
    }
    return launch_status();
}

// Shared checks of both entry points (the shape ensure!s of
// kv_cache_update_seq_arc_ctx_with_position, src/model.rs:5396-5423, on sizes).
static int32_t check_kv_update(const uint16_t* new_k, const uint16_t* new_v, uint16_t* k_cache,
                               uint16_t* v_cache, int32_t seq_len, int32_t num_kv_heads,
                               int32_t head_dim, int32_t max_seq_len) {
    GROUT_REQUIRE(new_k != nullptr && new_v != nullptr && k_cache != nullptr && v_cache != nullptr,
                  GROUT_ERR_NULL_POINTER);
    // head_dim is free here (grout's engine uses 128); rows move in 8- or
    // 16-byte units, so it must be a multiple of 4.
    GROUT_REQUIRE(head_dim > 0 && head_dim % 4 == 0, GROUT_ERR_HEAD_DIM);
    GROUT_REQUIRE(num_kv_heads > 0, GROUT_ERR_HEADS);
    GROUT_REQUIRE(max_seq_len > 0 && seq_len >= 0, GROUT_ERR_SEQ_RANGE);
    const uintptr_t align = head_dim % 8 == 0 ? 15u : 7u;
    GROUT_REQUIRE(((reinterpret_cast<uintptr_t>(new_k) | reinterpret_cast<uintptr_t>(new_v) |
                    reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) &
                   align) == 0,
                  GROUT_ERR_ALIGNMENT);
    return GROUT_OK;
}

}  // namespace grout

using namespace grout;

extern "C" int32_t grout_kv_cache_update_seq(const uint16_t* new_k, const uint16_t* new_v,
                                             uint16_t* k_cache, uint16_t* v_cache,
                                             int32_t position_start, int32_t seq_len,
                                             int32_t num_kv_heads, int32_t head_dim,
                                             int32_t max_seq_len, grout_stream_t stream) {
    const int32_t st = check_kv_update(new_k, new_v, k_cache, v_cache, seq_len, num_kv_heads,
                                       head_dim, max_seq_len);
    if (st != GROUT_OK) return st;
    // src/model.rs:5425-5431: position_start + seq_len <= max_seq_len.
    GROUT_REQUIRE(position_start >= 0 &&
                      static_cast<int64_t>(position_start) + seq_len <= max_seq_len,
                  GROUT_ERR_SEQ_RANGE);
    return launch_kv_update<false>(new_k, new_v, k_cache, v_cache, position_start, nullptr,
                                   seq_len, num_kv_heads, head_dim, max_seq_len, to_hip(stream));
}

extern "C" int32_t grout_kv_cache_update_seq_dynpos(const uint16_t* new_k, const uint16_t* new_v,
                                                    uint16_t* k_cache, uint16_t* v_cache,
                                                    const uint32_t* d_position, int32_t seq_len,
                                                    int32_t num_kv_heads, int32_t head_dim,
                                                    int32_t max_seq_len, grout_stream_t stream) {
    GROUT_REQUIRE(d_position != nullptr, GROUT_ERR_NULL_POINTER);
    GROUT_REQUIRE((reinterpret_cast<uintptr_t>(d_position) & 3u) == 0, GROUT_ERR_ALIGNMENT);
    const int32_t st = check_kv_update(new_k, new_v, k_cache, v_cache, seq_len, num_kv_heads,
                                       head_dim, max_seq_len);
    if (st != GROUT_OK) return st;
    return launch_kv_update<true>(new_k, new_v, k_cache, v_cache, 0, d_position, seq_len,
                                  num_kv_heads, head_dim, max_seq_len, to_hip(stream));
}

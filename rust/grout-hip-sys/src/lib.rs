//! Rust binding of the MI355X (gfx950) Qwen3 attention hot path,
//! `libgrout_attn_hip.so` (C ABI: `include/grout_attn_hip.h`).
//!
//! This crate is what grout's `Qwen3Engine` links in place of its cuTile
//! attention kernels (`src/kernels.rs` attention ops, `src/flash_decode.rs`)
//! and of the CUDA-graph decode capture:
//!
//! | grout call site | entry point here |
//! |---|---|
//! | `src/model.rs:4567-4595` prefill QK norm + RoPE + KV write | [`grout_qk_norm_rope_kv_prefill`] |
//! | `src/model.rs:5638-5834` prefill attention (every variant) | [`grout_attn_prefill`] |
//! | `src/model.rs:3194-3221` decode QK norm + RoPE + KV write | [`grout_qk_norm_rope_kv_decode`] |
//! | `src/model.rs:3428-3452` split-K GQA decode | [`grout_attn_decode_split`] |
//! | `src/model.rs:3453-3473` split-K merge | [`grout_attn_decode_merge`] |
//! | the three decode ops in one launch | [`grout_attn_decode_fused`] |
//! | `src/model.rs:318-493` `DecodeCudaGraphRunner` | [`Graph`], [`DecodeRunner`], [`Qwen3Runner`] |
//!
//! Calling rules (from the header): every function returns a status
//! (0 = ok, < 0 = argument validation, > 0 = `hipError_t`); pointers are
//! borrowed device memory.  The kernel entry points (`grout_qk_norm_rope_*`,
//! `grout_attn_*`, `grout_kv_cache_*`, the decode-layer ops) allocate nothing
//! and never synchronise the host, so the decode ones can be captured into a
//! hipGraph.  The runners are set-up objects and do block: `*_create`
//! allocates, captures and synchronises, `*_destroy` synchronises its
//! stream, and a step that returns a token (`token_out`) waits for it.
//! [`check`] turns a status into a `Result` whose error converts into
//! `anyhow::Error` at grout's `?` sites.
//!
//! Not compiled in this repository (its build image has no Rust toolchain);
//! `tests/test_rust_binding.py` checks the declarations below against the C
//! header, function by function and field by field.
#![allow(non_camel_case_types)]

use std::ffi::{c_void, CStr};
use std::os::raw::c_char;

/// `hipStream_t` (the header's `grout_stream_t`); null is the default stream.
pub type HipStream = *mut c_void;

pub const GROUT_HEAD_DIM: i32 = 128;
pub const GROUT_MAX_DECODE_GROUP: i32 = 16;
pub const GROUT_MAX_DECODE_SPLITS: i32 = 1024;
pub const GROUT_MAX_PREFILL_SPLITS: i32 = 1024;

pub const GROUT_OK: i32 = 0;
pub const GROUT_ERR_NULL_POINTER: i32 = -1;
pub const GROUT_ERR_ALIGNMENT: i32 = -2;
pub const GROUT_ERR_HEAD_DIM: i32 = -3;
pub const GROUT_ERR_HEADS: i32 = -4;
pub const GROUT_ERR_SEQ_RANGE: i32 = -5;
pub const GROUT_ERR_KV_LEN: i32 = -6;
pub const GROUT_ERR_GROUP: i32 = -7;
pub const GROUT_ERR_SPLITS: i32 = -8;
pub const GROUT_ERR_ARG: i32 = -9;
pub const GROUT_ERR_GRAPH: i32 = -10;
pub const GROUT_ERR_SCRATCH: i32 = -11;

/// Static scratch of [`grout_attn_decode_fused_noalloc`] (per GPU) and the
/// largest KV-head count it takes.
pub const GROUT_NOALLOC_SCRATCH_BYTES: i32 = 4194304;
pub const GROUT_NOALLOC_MAX_KV_HEADS: i32 = 255;

/// Source element types of [`grout_cast_to_f16`] (`src/loader.rs:109-145`).
pub const GROUT_DTYPE_F16: i32 = 0;
pub const GROUT_DTYPE_BF16: i32 = 1;
pub const GROUT_DTYPE_F32: i32 = 2;
pub const GROUT_DTYPE_F64: i32 = 3;

/// Opaque handles.
#[repr(C)]
pub struct GroutGraph {
    _opaque: [u8; 0],
}
#[repr(C)]
pub struct GroutDecodeRunner {
    _opaque: [u8; 0],
}
#[repr(C)]
pub struct GroutQwen3Runner {
    _opaque: [u8; 0],
}

/// `grout_decode_layer`: one layer's buffers for the decode graph runner.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct GroutDecodeLayer {
    pub qkv: *const u16,
    pub q_weight: *const u16,
    pub k_weight: *const u16,
    pub inv_freq: *const f32,
    pub q_out: *mut u16,
    pub k_cache: *mut u16,
    pub v_cache: *mut u16,
    pub att_partial: *mut u16,
    pub lse_partial: *mut f32,
    pub attn_out: *mut u16,
    pub d_position: *mut u32,
    pub counters: *mut u32,
    pub eps: f32,
    pub qk_scale_f16: u16,
    pub num_q_heads: i32,
    pub num_kv_heads: i32,
    pub head_dim: i32,
    pub max_seq_len: i32,
    pub block_n: i32,
    pub num_splits: i32,
}

/// `grout_qwen3_layer`: one transformer layer's weights and caches.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct GroutQwen3Layer {
    pub input_norm: *const u16,
    pub qkv_proj: *const u16,
    pub q_norm: *const u16,
    pub k_norm: *const u16,
    pub o_proj: *const u16,
    pub post_attn_norm: *const u16,
    pub gate_up_proj: *const u16,
    pub down_proj: *const u16,
    pub k_cache: *mut u16,
    pub v_cache: *mut u16,
}

/// `grout_qwen3_model`: the whole decode token step.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct GroutQwen3Model {
    pub num_layers: i32,
    pub hidden: i32,
    pub intermediate: i32,
    pub vocab: i32,
    pub num_q_heads: i32,
    pub num_kv_heads: i32,
    pub head_dim: i32,
    pub max_seq_len: i32,
    pub block_n: i32,
    pub num_splits: i32,
    pub eps: f32,
    pub qk_scale_f16: u16,
    pub layers: *const GroutQwen3Layer,
    pub embed_tokens: *const u16,
    pub final_norm: *const u16,
    pub lm_head: *const u16,
    pub inv_freq: *const f32,
    pub token: *mut u32,
    pub d_position: *mut u32,
    pub logits: *mut u16,
    pub workspace: *mut c_void,
}

extern "C" {
    pub fn grout_status_string(status: i32) -> *const c_char;
    pub fn grout_build_inv_freq(theta: f32, head_dim: i32, out_host: *mut f32) -> i32;

    pub fn grout_qk_norm_rope_kv_prefill(
        q: *const u16, k: *const u16, v: *const u16, q_weight: *const u16, k_weight: *const u16,
        inv_freq: *const f32, q_out: *mut u16, k_cache: *mut u16, v_cache: *mut u16, eps: f32,
        position_start: i32, seq_len: i32, num_q_heads: i32, num_kv_heads: i32, head_dim: i32,
        max_seq_len: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_qk_norm_rope_kv_decode(
        qkv: *const u16, q_weight: *const u16, k_weight: *const u16, inv_freq: *const f32,
        q_out: *mut u16, k_cache: *mut u16, v_cache: *mut u16, d_position: *const u32, eps: f32,
        num_q_heads: i32, num_kv_heads: i32, head_dim: i32, max_seq_len: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_kv_cache_update_seq(
        new_k: *const u16, new_v: *const u16, k_cache: *mut u16, v_cache: *mut u16,
        position_start: i32, seq_len: i32, num_kv_heads: i32, head_dim: i32, max_seq_len: i32,
        stream: HipStream,
    ) -> i32;
    pub fn grout_kv_cache_update_seq_dynpos(
        new_k: *const u16, new_v: *const u16, k_cache: *mut u16, v_cache: *mut u16,
        d_position: *const u32, seq_len: i32, num_kv_heads: i32, head_dim: i32, max_seq_len: i32,
        stream: HipStream,
    ) -> i32;

    pub fn grout_attn_prefill(
        q: *const u16, k_cache: *const u16, v_cache: *const u16, out: *mut u16, qk_scale: f32,
        num_q_heads: i32, num_kv_heads: i32, head_dim: i32, q_len: i32, kv_len: i32,
        query_start: i32, max_seq_len: i32, stream: HipStream,
    ) -> i32;
    /// The same prefill with a dynamic per-XCD schedule; `sched_counters` is
    /// [`grout_attn_prefill_sched_counter_bytes`] zeroed bytes kept by the engine.
    pub fn grout_attn_prefill_sched(
        q: *const u16, k_cache: *const u16, v_cache: *const u16, out: *mut u16, qk_scale: f32,
        num_q_heads: i32, num_kv_heads: i32, head_dim: i32, q_len: i32, kv_len: i32,
        query_start: i32, max_seq_len: i32, sched_counters: *mut u32, stream: HipStream,
    ) -> i32;
    pub fn grout_attn_prefill_sched_counter_bytes() -> i64;
    pub fn grout_attn_prefill_split(
        q: *const u16, k_cache: *const u16, v_cache: *const u16, att_partial: *mut u16,
        lse_partial: *mut f32, qk_scale: f32, num_q_heads: i32, num_kv_heads: i32, head_dim: i32,
        q_len: i32, kv_len: i32, query_start: i32, max_seq_len: i32, block_m: i32, block_n: i32,
        group: i32, num_splits: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_attn_prefill_split_merge(
        att_partial: *const u16, lse_partial: *const f32, out: *mut u16, num_q_heads: i32,
        head_dim: i32, q_len: i32, block_m: i32, group: i32, num_splits: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_attn_prefill_split_partial_bytes(
        num_q_heads: i32, head_dim: i32, q_len: i32, block_m: i32, group: i32, num_splits: i32,
    ) -> i64;
    pub fn grout_attn_prefill_split_lse_bytes(
        num_q_heads: i32, q_len: i32, block_m: i32, group: i32, num_splits: i32,
    ) -> i64;

    pub fn grout_add_rms_norm_decode(
        residual: *const u16, x: *const u16, weight: *const u16, out: *mut u16,
        residual_out: *mut u16, eps: f32, n: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_embed_rms_norm_decode(
        token: *const u32, table: *const u16, vocab: i32, weight: *const u16, out: *mut u16,
        residual_out: *mut u16, eps: f32, n: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_silu_mul_f16(
        gate: *const u16, up: *const u16, out: *mut u16, n: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_gemv_f16(
        weight: *const u16, x: *const u16, out: *mut u16, m: i32, k: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_gemv_silu_mul_f16(
        gate_up: *const u16, x: *const u16, out: *mut u16, n: i32, k: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_argmax_blocks(n: i32) -> i32;
    pub fn grout_argmax_f16(
        logits: *const u16, block_max: *mut f32, block_idx: *mut u32, token: *mut u32, n: i32,
        stream: HipStream,
    ) -> i32;

    pub fn grout_attn_decode_split(
        q: *const u16, k_cache: *const u16, v_cache: *const u16, att_partial: *mut u16,
        lse_partial: *mut f32, qk_scale_f16: u16, d_position: *const u32, num_kv_heads: i32,
        group: i32, head_dim: i32, max_seq_len: i32, block_n: i32, num_splits: i32,
        stream: HipStream,
    ) -> i32;
    pub fn grout_attn_decode_merge(
        att_partial: *const u16, lse_partial: *const f32, out: *mut u16, num_kv_heads: i32,
        group: i32, head_dim: i32, num_splits: i32, stream: HipStream,
    ) -> i32;
    pub fn grout_attn_decode_fused(
        qkv: *const u16, q_weight: *const u16, k_weight: *const u16, inv_freq: *const f32,
        q_out: *mut u16, k_cache: *mut u16, v_cache: *mut u16, att_partial: *mut u16,
        lse_partial: *mut f32, out: *mut u16, counters: *mut u32, d_position: *mut u32, eps: f32,
        qk_scale_f16: u16, num_q_heads: i32, num_kv_heads: i32, head_dim: i32, max_seq_len: i32,
        block_n: i32, num_splits: i32, advance_position: i32, stream: HipStream,
    ) -> i32;
    /// The fused step with its scratch in the library's static device
    /// array; no counterpart in grout, for callers that cannot allocate.
    pub fn grout_attn_decode_fused_noalloc(
        qkv: *const u16, q_weight: *const u16, k_weight: *const u16, inv_freq: *const f32,
        q_out: *mut u16, k_cache: *mut u16, v_cache: *mut u16, out: *mut u16,
        d_position: *mut u32, eps: f32, qk_scale_f16: u16, num_q_heads: i32, num_kv_heads: i32,
        head_dim: i32, max_seq_len: i32, block_n: i32, num_splits: i32, advance_position: i32,
        stream: HipStream,
    ) -> i32;
    pub fn grout_attn_decode_counter_bytes(num_kv_heads: i32) -> i64;
    pub fn grout_attn_decode_partial_bytes(
        num_kv_heads: i32, group: i32, head_dim: i32, num_splits: i32,
    ) -> i64;
    pub fn grout_attn_decode_lse_bytes(num_kv_heads: i32, group: i32, num_splits: i32) -> i64;
    pub fn grout_attn_decode_pick_splits(
        cu_count: i32, num_kv_heads: i32, max_context: i32, block_n: i32,
    ) -> i32;
    pub fn grout_attn_decode_pick_splits_grouped(
        cu_count: i32, num_kv_heads: i32, group: i32, max_context: i32, block_n: i32,
    ) -> i32;
    pub fn grout_device_cu_count(device: i32, cu_count: *mut i32) -> i32;

    pub fn grout_graph_begin(stream: HipStream) -> i32;
    pub fn grout_graph_end(stream: HipStream, graph: *mut *mut GroutGraph) -> i32;
    pub fn grout_graph_launch(graph: *mut GroutGraph, stream: HipStream) -> i32;
    pub fn grout_graph_destroy(graph: *mut GroutGraph) -> i32;
    pub fn grout_set_position_async(d_position: *mut u32, position: u32, stream: HipStream)
        -> i32;

    pub fn grout_decode_runner_create(
        layer: *const GroutDecodeLayer, prime_position: u32, stream: HipStream,
        runner: *mut *mut GroutDecodeRunner,
    ) -> i32;
    pub fn grout_decode_runner_step(runner: *mut GroutDecodeRunner, position: u32) -> i32;
    pub fn grout_decode_runner_run(
        runner: *mut GroutDecodeRunner, first_position: u32, count: i32,
    ) -> i32;
    pub fn grout_decode_runner_zero_kv(runner: *mut GroutDecodeRunner) -> i32;
    pub fn grout_decode_runner_destroy(runner: *mut GroutDecodeRunner) -> i32;

    pub fn grout_cast_to_f16(
        src: *const c_void, src_dtype: i32, dst: *mut u16, n: i64, stream: HipStream,
    ) -> i32;

    pub fn grout_qwen3_workspace_bytes(model: *const GroutQwen3Model) -> i64;
    pub fn grout_qwen3_decode_step(model: *const GroutQwen3Model, stream: HipStream) -> i32;
    pub fn grout_qwen3_runner_create(
        model: *const GroutQwen3Model, prime_position: u32, stream: HipStream,
        runner: *mut *mut GroutQwen3Runner,
    ) -> i32;
    pub fn grout_qwen3_runner_seed_token(runner: *mut GroutQwen3Runner, token: u32) -> i32;
    pub fn grout_qwen3_runner_step(
        runner: *mut GroutQwen3Runner, position: u32, token_out: *mut u32,
    ) -> i32;
    pub fn grout_qwen3_runner_run(
        runner: *mut GroutQwen3Runner, first_position: u32, count: i32,
    ) -> i32;
    pub fn grout_qwen3_runner_destroy(runner: *mut GroutQwen3Runner) -> i32;
}

/// A failed entry point: the status code and the library's text for it.
#[derive(Debug, Clone)]
pub struct GroutError {
    pub status: i32,
    pub message: String,
}

impl std::fmt::Display for GroutError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "grout_attn_hip: {} ({})", self.message, self.status)
    }
}

impl std::error::Error for GroutError {}

/// Status -> `Result`, so grout's call sites keep their `?` flow
/// (`GroutError` converts into `anyhow::Error`).
pub fn check(status: i32) -> Result<(), GroutError> {
    if status == GROUT_OK {
        return Ok(());
    }
    // SAFETY: grout_status_string returns a pointer to static storage.
    let message = unsafe { CStr::from_ptr(grout_status_string(status)) }
        .to_string_lossy()
        .into_owned();
    Err(GroutError { status, message })
}

/// Result of a size query (`*_bytes`): negative values are status codes.
pub fn check_bytes(v: i64) -> Result<usize, GroutError> {
    if v < 0 {
        check(v as i32)?;
    }
    Ok(v as usize)
}

/// An instantiated hipGraph captured from a stream (replaces cuda-async's
/// `CudaGraph::scope` in the decode capture, `src/model.rs:3118-3648`).
pub struct Graph {
    raw: *mut GroutGraph,
}

impl Graph {
    /// Captures everything `record` enqueues on `stream` into a graph.  The
    /// capture is ended even when `record` fails, and its error wins.
    pub fn capture<F>(stream: HipStream, record: F) -> Result<Graph, GroutError>
    where
        F: FnOnce(HipStream) -> Result<(), GroutError>,
    {
        // SAFETY: begin/end pair on the same stream; `raw` is written by end.
        check(unsafe { grout_graph_begin(stream) })?;
        let rec = record(stream);
        let mut raw = std::ptr::null_mut();
        let end = check(unsafe { grout_graph_end(stream, &mut raw) });
        let graph = Graph { raw };
        rec?;
        end?;
        Ok(graph)
    }

    /// One replay on `stream` (no host sync).
    pub fn launch(&self, stream: HipStream) -> Result<(), GroutError> {
        // SAFETY: `raw` came from grout_graph_end and is live until drop.
        check(unsafe { grout_graph_launch(self.raw, stream) })
    }
}

impl Drop for Graph {
    fn drop(&mut self) {
        // SAFETY: destroy accepts null and frees what end created.
        unsafe {
            grout_graph_destroy(self.raw);
        }
    }
}

/// The attention slice of `DecodeCudaGraphRunner` (`src/model.rs:318-493`)
/// for one layer: the fused decode step captured once, replayed per token.
/// The buffers in `layer` are borrowed for the runner's lifetime.
pub struct DecodeRunner {
    raw: *mut GroutDecodeRunner,
}

impl DecodeRunner {
    /// # Safety
    /// Every pointer in `layer` must stay valid until the runner is dropped.
    pub unsafe fn new(
        layer: &GroutDecodeLayer, prime_position: u32, stream: HipStream,
    ) -> Result<DecodeRunner, GroutError> {
        let mut raw = std::ptr::null_mut();
        check(grout_decode_runner_create(layer, prime_position, stream, &mut raw))?;
        Ok(DecodeRunner { raw })
    }

    /// `launch_step`: position write + replay (`src/model.rs:363-403`).
    pub fn step(&mut self, position: u32) -> Result<(), GroutError> {
        check(unsafe { grout_decode_runner_step(self.raw, position) })
    }

    /// `count` consecutive steps issued without returning in between.
    pub fn run(&mut self, first_position: u32, count: i32) -> Result<(), GroutError> {
        check(unsafe { grout_decode_runner_run(self.raw, first_position, count) })
    }

    /// `zero_kv_caches` (`src/model.rs:433-462`); synchronises the stream.
    pub fn zero_kv(&mut self) -> Result<(), GroutError> {
        check(unsafe { grout_decode_runner_zero_kv(self.raw) })
    }
}

impl Drop for DecodeRunner {
    fn drop(&mut self) {
        // SAFETY: destroy waits for queued replays, then frees the graph.
        unsafe {
            grout_decode_runner_destroy(self.raw);
        }
    }
}

/// The whole decode token step as one hipGraph (`DecodeCudaGraphRunner`
/// with the graph of `src/model.rs:3118-3648`).
pub struct Qwen3Runner {
    raw: *mut GroutQwen3Runner,
}

impl Qwen3Runner {
    /// # Safety
    /// Every pointer reachable from `model` (weights, caches, token,
    /// position, logits, workspace) must stay valid until the runner is
    /// dropped; the layer array is copied.
    pub unsafe fn new(
        model: &GroutQwen3Model, prime_position: u32, stream: HipStream,
    ) -> Result<Qwen3Runner, GroutError> {
        let mut raw = std::ptr::null_mut();
        check(grout_qwen3_runner_create(model, prime_position, stream, &mut raw))?;
        Ok(Qwen3Runner { raw })
    }

    /// `seed_token` (`src/model.rs:343-356`).
    pub fn seed_token(&mut self, token: u32) -> Result<(), GroutError> {
        check(unsafe { grout_qwen3_runner_seed_token(self.raw, token) })
    }

    /// `launch_step` (`src/model.rs:363-403`): returns the sampled token.
    pub fn step(&mut self, position: u32) -> Result<u32, GroutError> {
        let mut token = 0u32;
        check(unsafe { grout_qwen3_runner_step(self.raw, position, &mut token) })?;
        Ok(token)
    }

    /// `count` consecutive steps with the token chain kept on the device.
    pub fn run(&mut self, first_position: u32, count: i32) -> Result<(), GroutError> {
        check(unsafe { grout_qwen3_runner_run(self.raw, first_position, count) })
    }
}

impl Drop for Qwen3Runner {
    fn drop(&mut self) {
        // SAFETY: destroy waits for queued replays, then frees the graph.
        unsafe {
            grout_qwen3_runner_destroy(self.raw);
        }
    }
}

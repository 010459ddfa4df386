//! `extern "C"` block for the gfx950 tensor-op library (`librustllm_hip.so`):
//! one declaration per function of `include/rustllm_hip.h`, same names, same
//! argument order and meaning.  It replaces the `metal` crate dependency of
//! `src/metal/*`; `src/hip/mod.rs` builds the `MetalContext` /
//! `MetalBuffer` / `MetalExecution` types of `src/metal/mod.rs` on top of it.
//!
//! Conventions (as the header states them): every fallible call returns an
//! `rl_status` (0 = `RL_OK`), one code per `TinyError` variant the op layer
//! raises (`src/error.rs:4-43`; `RL_ERR_DEVICE` stands for
//! `TinyError::Metal`); ops enqueue on the context's stream and return
//! (the `*_encode` twins); `rl_execution_finish` is the commit + wait.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_void};

pub type rl_status = i32;
pub const RL_OK: rl_status = 0;
pub const RL_ERR_INVALID_ARGUMENT: rl_status = 1; // TinyError::InvalidArgument
pub const RL_ERR_INVALID_SHAPE: rl_status = 2; // TinyError::InvalidShape
pub const RL_ERR_SHAPE_MISMATCH: rl_status = 3; // TinyError::ShapeMismatch { left, right }
pub const RL_ERR_INVALID_DIMENSION: rl_status = 4; // TinyError::InvalidDimension
pub const RL_ERR_UNSUPPORTED_DTYPE: rl_status = 5; // TinyError::UnsupportedDType
pub const RL_ERR_NON_CONTIGUOUS: rl_status = 6; // TinyError::NonContiguousTensor
pub const RL_ERR_POSITION_OUT_OF_RANGE: rl_status = 7; // TinyError::PositionOutOfRange { .. }
pub const RL_ERR_MODEL_FORMAT: rl_status = 8; // TinyError::ModelFormat
pub const RL_ERR_DEVICE: rl_status = 9; // TinyError::Metal
pub const RL_ERR_INVALID_TOKEN_ID: rl_status = 10; // TinyError::InvalidTokenId { .. }

#[repr(C)]
pub struct rl_context {
    _private: [u8; 0],
}
#[repr(C)]
pub struct rl_graph {
    _private: [u8; 0],
}
#[repr(C)]
pub struct rl_event {
    _private: [u8; 0],
}

/// MetalBuffer's three fields (src/metal/buffer.rs:8-12): device pointer,
/// element count, byte length.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct rl_buffer {
    pub data: *mut c_void,
    pub len: u64,
    pub byte_len: u64,
}

/// MetalDecodeProfile's counters (src/profile.rs:7-16).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct rl_profile {
    pub command_buffers: u64,
    pub compute_encoders: u64,
    pub kernel_dispatches: u64,
    pub commits: u64,
    pub waits: u64,
    pub buffer_allocations: u64,
    pub allocated_bytes: u64,
}

pub const RL_ERROR_MAX_RANK: usize = 16;

/// The data of the TinyError variants that carry fields (src/error.rs:7-24)
/// for the thread's last failure; `code` selects which fields are set.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct rl_error_payload {
    pub code: rl_status,
    pub left_rank: u32,
    pub right_rank: u32,
    pub token_id: u32,
    pub left: [u64; RL_ERROR_MAX_RANK],
    pub right: [u64; RL_ERROR_MAX_RANK],
    pub start_pos: u64,
    pub seq_len: u64,
    pub max_seq_len: u64,
    pub vocab_size: u64,
}

#[link(name = "rustllm_hip")]
extern "C" {
    // errors and version
    pub fn rl_last_error_message() -> *const c_char;
    pub fn rl_last_error_payload(out: *mut rl_error_payload) -> rl_status;
    pub fn rl_version() -> *const c_char;
    // context (src/metal/context.rs:10-44)
    pub fn rl_context_create(device: i32, out: *mut *mut rl_context) -> rl_status;
    pub fn rl_context_create_on_stream(
        device: i32,
        stream: *mut c_void,
        out: *mut *mut rl_context,
    ) -> rl_status;
    pub fn rl_context_destroy(ctx: *mut rl_context);
    pub fn rl_context_stream(ctx: *const rl_context) -> *mut c_void;
    pub fn rl_device_count() -> i32;
    pub fn rl_context_trim(ctx: *mut rl_context) -> rl_status;
    // buffers (src/metal/buffer.rs:8-169)
    pub fn rl_buffer_empty(
        ctx: *mut rl_context,
        len: u64,
        element_size: u64,
        out: *mut rl_buffer,
    ) -> rl_status;
    pub fn rl_buffer_from_host(
        ctx: *mut rl_context,
        host: *const c_void,
        len: u64,
        element_size: u64,
        out: *mut rl_buffer,
    ) -> rl_status;
    pub fn rl_buffer_to_host(
        ctx: *mut rl_context,
        buffer: *const rl_buffer,
        host: *mut c_void,
        byte_len: u64,
    ) -> rl_status;
    pub fn rl_buffer_copy(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dst: *const rl_buffer,
        byte_len: u64,
    ) -> rl_status;
    pub fn rl_buffer_release(ctx: *mut rl_context, buffer: *mut rl_buffer);
    // execution (src/metal/execution.rs:11-36), graphs and events
    pub fn rl_execution_begin(ctx: *mut rl_context) -> rl_status;
    pub fn rl_execution_finish(ctx: *mut rl_context) -> rl_status;
    pub fn rl_graph_capture_begin(ctx: *mut rl_context) -> rl_status;
    pub fn rl_context_set_fusion(ctx: *mut rl_context, enabled: i32) -> rl_status;
    pub fn rl_graph_capture_end(ctx: *mut rl_context, out: *mut *mut rl_graph) -> rl_status;
    pub fn rl_graph_launch(ctx: *mut rl_context, graph: *mut rl_graph) -> rl_status;
    pub fn rl_graph_destroy(graph: *mut rl_graph);
    pub fn rl_event_create(ctx: *mut rl_context, out: *mut *mut rl_event) -> rl_status;
    pub fn rl_event_record(ctx: *mut rl_context, event: *mut rl_event) -> rl_status;
    pub fn rl_event_wait(ctx: *mut rl_context, event: *mut rl_event) -> rl_status;
    pub fn rl_event_elapsed_ms(start: *mut rl_event, end: *mut rl_event, ms: *mut f32) -> rl_status;
    pub fn rl_event_destroy(event: *mut rl_event);
    pub fn rl_event_time_next_kernel(
        ctx: *mut rl_context,
        start: *mut rl_event,
        stop: *mut rl_event,
    ) -> rl_status;
    // submission counters (src/metal/context.rs:48-54, src/profile.rs:7-16)
    pub fn rl_profile_begin(ctx: *mut rl_context);
    pub fn rl_profile_take(ctx: *mut rl_context, out: *mut rl_profile) -> i32;
    pub fn rl_profile_dispatches(ctx: *const rl_context, kernel_name: *const c_char) -> u64;
    // element-wise (src/ops/{add,mul,silu,swiglu,cast}.rs)
    pub fn rl_add_f32(
        ctx: *mut rl_context,
        a: *const rl_buffer,
        b: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_add_f16(
        ctx: *mut rl_context,
        a: *const rl_buffer,
        b: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_mul_f32(
        ctx: *mut rl_context,
        a: *const rl_buffer,
        b: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_mul_f16(
        ctx: *mut rl_context,
        a: *const rl_buffer,
        b: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_silu_f32(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_silu_f16(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_swiglu_f16(
        ctx: *mut rl_context,
        gate: *const rl_buffer,
        up: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_swiglu_f32(
        ctx: *mut rl_context,
        gate: *const rl_buffer,
        up: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_cast_f32_to_f16(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_cast_f16_to_f32(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_add_broadcast_f32(
        ctx: *mut rl_context,
        x: *const rl_buffer,
        bias: *const rl_buffer,
        rows: u64,
        cols: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_add_broadcast_f16(
        ctx: *mut rl_context,
        x: *const rl_buffer,
        bias: *const rl_buffer,
        rows: u64,
        cols: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    // data movement (src/ops/contiguous.rs, src/tensor/repeat_kv.rs)
    pub fn rl_contiguous_f32(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dims: *const u64,
        strides: *const u64,
        rank: u32,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_contiguous_f16(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dims: *const u64,
        strides: *const u64,
        rank: u32,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_repeat_kv_f32(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        batch: u64,
        kv_heads: u64,
        seq_len: u64,
        head_dim: u64,
        repeats: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_repeat_kv_f16(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        batch: u64,
        kv_heads: u64,
        seq_len: u64,
        head_dim: u64,
        repeats: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    // reductions (src/ops/{rmsnorm,softmax,attention_scale_mask}.rs)
    pub fn rl_rmsnorm_f32(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        weight: *const rl_buffer,
        rows: u64,
        hidden: u64,
        eps: f32,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_rmsnorm_f16(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        weight: *const rl_buffer,
        rows: u64,
        hidden: u64,
        eps: f32,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_add_rmsnorm_f32(
        ctx: *mut rl_context,
        x: *const rl_buffer,
        residual: *const rl_buffer,
        weight: *const rl_buffer,
        rows: u64,
        hidden: u64,
        eps: f32,
        sum_out: *const rl_buffer,
        norm_out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_add_rmsnorm_f16(
        ctx: *mut rl_context,
        x: *const rl_buffer,
        residual: *const rl_buffer,
        weight: *const rl_buffer,
        rows: u64,
        hidden: u64,
        eps: f32,
        sum_out: *const rl_buffer,
        norm_out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_softmax_f32(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        rows: u64,
        width: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_softmax_f16(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        rows: u64,
        width: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_attention_scale_mask_f32(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        scale: f32,
        query_len: u64,
        key_len: u64,
        query_start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_attention_scale_mask_f16(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        scale: f32,
        query_len: u64,
        key_len: u64,
        query_start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_attention_softmax_f32(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        scale: f32,
        query_len: u64,
        key_len: u64,
        query_start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_attention_softmax_f16(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        scale: f32,
        query_len: u64,
        key_len: u64,
        query_start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    // RoPE (src/ops/rope.rs)
    pub fn rl_rope_f32(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        seq_len: u64,
        head_dim: u64,
        start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_rope_f16(
        ctx: *mut rl_context,
        input: *const rl_buffer,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        seq_len: u64,
        head_dim: u64,
        start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_rope_strided_f32(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dims: *const u64,
        strides: *const u64,
        rank: u32,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        table_rows: u64,
        start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_rope_strided_f16(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dims: *const u64,
        strides: *const u64,
        rank: u32,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        table_rows: u64,
        start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    // KV cache (src/ops/kv_cache_write.rs, src/model/kv_cache.rs)
    pub fn rl_kv_cache_write_f32(
        ctx: *mut rl_context,
        cache: *const rl_buffer,
        kv_heads: u64,
        max_seq: u64,
        head_dim: u64,
        source: *const rl_buffer,
        seq_len: u64,
        start: u64,
    ) -> rl_status;
    pub fn rl_kv_cache_write_f16(
        ctx: *mut rl_context,
        cache: *const rl_buffer,
        kv_heads: u64,
        max_seq: u64,
        head_dim: u64,
        source: *const rl_buffer,
        seq_len: u64,
        start: u64,
    ) -> rl_status;
    pub fn rl_kv_cache_write_strided_f32(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dims: *const u64,
        strides: *const u64,
        rank: u32,
        cache: *const rl_buffer,
        max_seq: u64,
        start: u64,
    ) -> rl_status;
    pub fn rl_kv_cache_write_strided_f16(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dims: *const u64,
        strides: *const u64,
        rank: u32,
        cache: *const rl_buffer,
        max_seq: u64,
        start: u64,
    ) -> rl_status;
    pub fn rl_rope_kv_cache_write_f32(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dims: *const u64,
        strides: *const u64,
        rank: u32,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        table_rows: u64,
        start_pos: u64,
        cache: *const rl_buffer,
        max_seq: u64,
    ) -> rl_status;
    pub fn rl_rope_kv_cache_write_f16(
        ctx: *mut rl_context,
        src: *const rl_buffer,
        dims: *const u64,
        strides: *const u64,
        rank: u32,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        table_rows: u64,
        start_pos: u64,
        cache: *const rl_buffer,
        max_seq: u64,
    ) -> rl_status;
    pub fn rl_qkv_rope_kv_append_f32(
        ctx: *mut rl_context,
        q_src: *const rl_buffer,
        q_dims: *const u64,
        q_strides: *const u64,
        k_src: *const rl_buffer,
        k_dims: *const u64,
        k_strides: *const u64,
        v_src: *const rl_buffer,
        v_dims: *const u64,
        v_strides: *const u64,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        table_rows: u64,
        start_pos: u64,
        q_out: *const rl_buffer,
        k_cache: *const rl_buffer,
        v_cache: *const rl_buffer,
        max_seq: u64,
    ) -> rl_status;
    pub fn rl_qkv_rope_kv_append_f16(
        ctx: *mut rl_context,
        q_src: *const rl_buffer,
        q_dims: *const u64,
        q_strides: *const u64,
        k_src: *const rl_buffer,
        k_dims: *const u64,
        k_strides: *const u64,
        v_src: *const rl_buffer,
        v_dims: *const u64,
        v_strides: *const u64,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        table_rows: u64,
        start_pos: u64,
        q_out: *const rl_buffer,
        k_cache: *const rl_buffer,
        v_cache: *const rl_buffer,
        max_seq: u64,
    ) -> rl_status;
    // the same plus repeat_kv of the cache prefixes (src/tensor/repeat_kv.rs)
    pub fn rl_qkv_rope_kv_append_repeat_f32(
        ctx: *mut rl_context,
        q_src: *const rl_buffer,
        q_dims: *const u64,
        q_strides: *const u64,
        k_src: *const rl_buffer,
        k_dims: *const u64,
        k_strides: *const u64,
        v_src: *const rl_buffer,
        v_dims: *const u64,
        v_strides: *const u64,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        table_rows: u64,
        start_pos: u64,
        q_out: *const rl_buffer,
        k_cache: *const rl_buffer,
        v_cache: *const rl_buffer,
        max_seq: u64,
        n_rep: u64,
        k_rep: *const rl_buffer,
        v_rep: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_qkv_rope_kv_append_repeat_f16(
        ctx: *mut rl_context,
        q_src: *const rl_buffer,
        q_dims: *const u64,
        q_strides: *const u64,
        k_src: *const rl_buffer,
        k_dims: *const u64,
        k_strides: *const u64,
        v_src: *const rl_buffer,
        v_dims: *const u64,
        v_strides: *const u64,
        cos_table: *const rl_buffer,
        sin_table: *const rl_buffer,
        table_rows: u64,
        start_pos: u64,
        q_out: *const rl_buffer,
        k_cache: *const rl_buffer,
        v_cache: *const rl_buffer,
        max_seq: u64,
        n_rep: u64,
        k_rep: *const rl_buffer,
        v_rep: *const rl_buffer,
    ) -> rl_status;
    // embedding (src/ops/embedding.rs)
    pub fn rl_embedding_f32(
        ctx: *mut rl_context,
        weight: *const rl_buffer,
        vocab_size: u64,
        hidden_size: u64,
        token_ids: *const u32,
        n_tokens: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_embedding_f16(
        ctx: *mut rl_context,
        weight: *const rl_buffer,
        vocab_size: u64,
        hidden_size: u64,
        token_ids: *const u32,
        n_tokens: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    // attention core (src/nn/attention.rs:216-247, src/tensor/gqa_matmul.rs)
    pub fn rl_attention_f32(
        ctx: *mut rl_context,
        q: *const rl_buffer,
        k: *const rl_buffer,
        v: *const rl_buffer,
        batch: u64,
        q_heads: u64,
        kv_heads: u64,
        q_len: u64,
        kv_len: u64,
        head_dim: u64,
        kv_capacity: u64,
        scale: f32,
        query_start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_attention_f16(
        ctx: *mut rl_context,
        q: *const rl_buffer,
        k: *const rl_buffer,
        v: *const rl_buffer,
        batch: u64,
        q_heads: u64,
        kv_heads: u64,
        q_len: u64,
        kv_len: u64,
        head_dim: u64,
        kv_capacity: u64,
        scale: f32,
        query_start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_attention_f16_noalloc(
        ctx: *mut rl_context,
        q: *const rl_buffer,
        k: *const rl_buffer,
        v: *const rl_buffer,
        batch: u64,
        q_heads: u64,
        kv_heads: u64,
        q_len: u64,
        kv_len: u64,
        head_dim: u64,
        kv_capacity: u64,
        scale: f32,
        query_start_pos: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_gqa_qk_matmul_f32(
        ctx: *mut rl_context,
        q: *const rl_buffer,
        k: *const rl_buffer,
        batch: u64,
        q_heads: u64,
        kv_heads: u64,
        q_len: u64,
        kv_len: u64,
        head_dim: u64,
        kv_capacity: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_gqa_qk_matmul_f16(
        ctx: *mut rl_context,
        q: *const rl_buffer,
        k: *const rl_buffer,
        batch: u64,
        q_heads: u64,
        kv_heads: u64,
        q_len: u64,
        kv_len: u64,
        head_dim: u64,
        kv_capacity: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_gqa_pv_matmul_f32(
        ctx: *mut rl_context,
        probs: *const rl_buffer,
        v: *const rl_buffer,
        batch: u64,
        q_heads: u64,
        kv_heads: u64,
        q_len: u64,
        kv_len: u64,
        head_dim: u64,
        kv_capacity: u64,
        out: *const rl_buffer,
    ) -> rl_status;
    pub fn rl_gqa_pv_matmul_f16(
        ctx: *mut rl_context,
        probs: *const rl_buffer,
        v: *const rl_buffer,
        batch: u64,
        q_heads: u64,
        kv_heads: u64,
        q_len: u64,
        kv_len: u64,
        head_dim: u64,
        kv_capacity: u64,
        out: *const rl_buffer,
    ) -> rl_status;
}

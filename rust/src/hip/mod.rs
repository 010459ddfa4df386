//! The HIP replacement of `src/metal/{context,buffer,execution}.rs`: the same
//! public types (`MetalContext`, `MetalBuffer`, `MetalExecution`), so
//! `src/ops/*`, `src/tensor/*`, `src/nn/*` and `src/model/*` keep their
//! signatures, built on the C ABI of `librustllm_hip.so` (`ffi.rs`).
//!
//! `src/metal/mod.rs` becomes `pub use crate::hip::{MetalBuffer, MetalContext,
//! MetalExecution, CommandBufferRef};` and each op body swaps its pipeline /
//! encoder lines for one `ffi::rl_<op>` call (see `ops_glue` below).
//! No `metal` crate, no runtime shader compilation: the kernels are built
//! ahead of time for gfx950.
//!
//! Threading is the reference's: a context is used from one thread
//! (`MetalContext` is `!Sync`, src/metal/context.rs:14-17); all work of a
//! context runs in order on its one HIP stream.

pub mod ffi;

use std::cell::{Cell, RefCell};
use std::collections::BTreeMap;
use std::ffi::{CStr, CString};
use std::marker::PhantomData;
use std::os::raw::c_void;

use crate::error::{Result, TinyError};
use crate::profile::MetalDecodeProfile;
use ffi::*;

/// Converts a library status into the TinyError variant it names
/// (src/error.rs:4-43), with the variant's data for ShapeMismatch,
/// PositionOutOfRange and InvalidTokenId read back through
/// `rl_last_error_payload`.
pub(crate) fn check(status: rl_status) -> Result<()> {
    if status == RL_OK {
        return Ok(());
    }
    let message = unsafe { CStr::from_ptr(rl_last_error_message()) }
        .to_string_lossy()
        .into_owned();
    let mut payload = std::mem::MaybeUninit::<rl_error_payload>::zeroed();
    let payload_code = unsafe { rl_last_error_payload(payload.as_mut_ptr()) };
    let payload = unsafe { payload.assume_init() };
    let dims = |values: &[u64; RL_ERROR_MAX_RANK], rank: u32| -> Vec<usize> {
        values[..(rank as usize).min(RL_ERROR_MAX_RANK)]
            .iter()
            .map(|&d| d as usize)
            .collect()
    };
    let has_payload = payload_code == status;
    Err(match status {
        RL_ERR_INVALID_ARGUMENT => TinyError::InvalidArgument(message),
        RL_ERR_INVALID_SHAPE => TinyError::InvalidShape(message),
        RL_ERR_SHAPE_MISMATCH if has_payload => TinyError::ShapeMismatch {
            left: dims(&payload.left, payload.left_rank),
            right: dims(&payload.right, payload.right_rank),
        },
        RL_ERR_INVALID_DIMENSION => TinyError::InvalidDimension(message),
        RL_ERR_UNSUPPORTED_DTYPE => TinyError::UnsupportedDType(message),
        RL_ERR_NON_CONTIGUOUS => TinyError::NonContiguousTensor(message),
        RL_ERR_POSITION_OUT_OF_RANGE if has_payload => TinyError::PositionOutOfRange {
            start_pos: payload.start_pos as usize,
            seq_len: payload.seq_len as usize,
            max_seq_len: payload.max_seq_len as usize,
        },
        RL_ERR_MODEL_FORMAT => TinyError::ModelFormat(message),
        RL_ERR_INVALID_TOKEN_ID if has_payload => TinyError::InvalidTokenId {
            token_id: payload.token_id,
            vocab_size: payload.vocab_size as usize,
        },
        // RL_ERR_DEVICE, and a data-carrying code whose payload was
        // overwritten (never the case for the call just made): the message.
        _ => TinyError::Metal(message),
    })
}

// ------------------------------------------------------------------ context

/// src/metal/context.rs:10-18.  Owns one `rl_context` (device 0, one
/// in-order stream at the default priority, the stream-ordered buffer pool).
pub struct MetalContext {
    raw: *mut rl_context,
    profiling: Cell<bool>,
    _not_sync: PhantomData<Cell<()>>,
}

/// The library's dispatch names (the `kernel_dispatches_by_name` keys).
const KERNEL_NAMES: &[&str] = &[
    "add_f32", "add_f16", "mul_f32", "mul_f16", "silu_f32", "silu_f16", "swiglu_f32",
    "swiglu_f16", "cast_f32_to_f16", "cast_f16_to_f32", "add_broadcast_f32",
    "add_broadcast_f16", "contiguous_f32", "contiguous_f16", "repeat_kv_f32", "repeat_kv_f16",
    "rmsnorm_f32", "rmsnorm_f16", "add_rmsnorm_f32", "add_rmsnorm_f16", "softmax_f32",
    "softmax_f16", "attention_scale_mask_f32", "attention_scale_mask_f16",
    "attention_softmax_f32", "attention_softmax_f16", "rope_f32", "rope_f16",
    "rope_strided_f32", "rope_strided_f16", "kv_cache_write_f32", "kv_cache_write_f16",
    "rope_kv_cache_write_f32", "rope_kv_cache_write_f16", "qkv_rope_kv_append_f32",
    "qkv_rope_kv_append_f16", "qkv_rope_kv_append_repeat_f32", "qkv_rope_kv_append_repeat_f16",
    "embedding_f32", "embedding_f16", "attention_f32",
    "attention_f16", "gqa_qk_f32", "gqa_qk_f16", "gqa_pv_f32", "gqa_pv_f16",
];

impl MetalContext {
    /// MetalContext::new (src/metal/context.rs:27-44).
    pub fn new() -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        check(unsafe { rl_context_create(0, &mut raw) })?;
        Ok(Self { raw, profiling: Cell::new(false), _not_sync: PhantomData })
    }

    /// src/metal/context.rs:48-50.
    pub fn begin_decode_submission_profile(&self) {
        unsafe { rl_profile_begin(self.raw) };
        self.profiling.set(true);
    }

    /// src/metal/context.rs:52-54.
    pub fn take_decode_submission_profile(&self) -> Option<MetalDecodeProfile> {
        if !self.profiling.replace(false) {
            return None;
        }
        let mut by_name = BTreeMap::new();
        for name in KERNEL_NAMES {
            let key = CString::new(*name).expect("kernel name");
            let n = unsafe { rl_profile_dispatches(self.raw, key.as_ptr()) };
            if n > 0 {
                by_name.insert((*name).to_owned(), n as usize);
            }
        }
        let mut p = rl_profile::default();
        if unsafe { rl_profile_take(self.raw, &mut p) } == 0 {
            return None;
        }
        Some(MetalDecodeProfile {
            command_buffers: p.command_buffers as usize,
            compute_encoders: p.compute_encoders as usize,
            kernel_dispatches: p.kernel_dispatches as usize,
            commits: p.commits as usize,
            waits: p.waits as usize,
            buffer_allocations: p.buffer_allocations as usize,
            allocated_bytes: p.allocated_bytes as usize,
            kernel_dispatches_by_name: by_name,
        })
    }

    pub(crate) fn raw(&self) -> *mut rl_context {
        self.raw
    }
}

impl Drop for MetalContext {
    fn drop(&mut self) {
        unsafe { rl_context_destroy(self.raw) }
    }
}

// ------------------------------------------------------------------- buffer

/// src/metal/buffer.rs:8-12: a pooled device allocation with its element
/// count and byte length.  HBM is not host-mapped, so `as_slice` /
/// `as_f16_slice` read through a host mirror downloaded on first use after
/// the producing execution finished; an op that writes the buffer in place
/// (the KV-cache write) calls `invalidate_host_mirror` first, and the next
/// read downloads again.  Earlier mirrors stay alive with the buffer, so a
/// slice handed out before stays valid (it shows the contents of its time).
pub struct MetalBuffer {
    ctx: *mut rl_context,
    raw: rl_buffer,
    mirrors: RefCell<Vec<Box<[u8]>>>,
    mirror_fresh: Cell<bool>,
}

impl MetalBuffer {
    fn upload(context: &MetalContext, data: *const c_void, len: usize, es: usize) -> Self {
        // buffer.rs:16-19 etc.: empty data is a programming error.
        assert!(len > 0, "cannot create a MetalBuffer from empty data");
        let mut raw = rl_buffer { data: std::ptr::null_mut(), len: 0, byte_len: 0 };
        check(unsafe { rl_buffer_from_host(context.raw(), data, len as u64, es as u64, &mut raw) })
            .expect("device upload");
        Self::wrap(context, raw)
    }

    fn wrap(context: &MetalContext, raw: rl_buffer) -> Self {
        Self {
            ctx: context.raw(),
            raw,
            mirrors: RefCell::new(Vec::new()),
            mirror_fresh: Cell::new(false),
        }
    }

    /// buffer.rs:15-34
    pub fn from_slice(context: &MetalContext, data: &[f32]) -> Self {
        Self::upload(context, data.as_ptr().cast(), data.len(), 4)
    }
    /// buffer.rs:36-55
    pub fn from_u32_slice(context: &MetalContext, data: &[u32]) -> Self {
        Self::upload(context, data.as_ptr().cast(), data.len(), 4)
    }
    /// buffer.rs:57-73
    pub fn from_f16_slice(context: &MetalContext, data: &[half::f16]) -> Self {
        Self::upload(context, data.as_ptr().cast(), data.len(), 2)
    }
    /// buffer.rs:75-91
    pub fn from_i8_slice(context: &MetalContext, data: &[i8]) -> Self {
        Self::upload(context, data.as_ptr().cast(), data.len(), 1)
    }
    /// buffer.rs:93-109
    pub fn from_u8_slice(context: &MetalContext, data: &[u8]) -> Self {
        Self::upload(context, data.as_ptr().cast(), data.len(), 1)
    }

    /// buffer.rs:111-126 (f32 elements).
    pub fn empty(context: &MetalContext, len: usize) -> Self {
        Self::empty_with_element_size(context, len, std::mem::size_of::<f32>())
    }

    /// buffer.rs:128-142.  Counted as an allocation by an active profile.
    pub fn empty_with_element_size(context: &MetalContext, len: usize, element_size: usize) -> Self {
        assert!(len > 0 && element_size > 0, "invalid MetalBuffer size");
        len.checked_mul(element_size).expect("MetalBuffer byte size overflow");
        let mut raw = rl_buffer { data: std::ptr::null_mut(), len: 0, byte_len: 0 };
        check(unsafe { rl_buffer_empty(context.raw(), len as u64, element_size as u64, &mut raw) })
            .expect("device allocation");
        Self::wrap(context, raw)
    }

    pub fn len(&self) -> usize {
        self.raw.len as usize
    }
    pub fn byte_len(&self) -> usize {
        self.raw.byte_len as usize
    }
    pub fn is_empty(&self) -> bool {
        self.raw.len == 0
    }
    /// The C handle (buffer.rs:156-158 returned the Metal buffer).
    pub fn raw(&self) -> &rl_buffer {
        &self.raw
    }

    /// Marks the host mirror stale after an in-place device write.
    pub(crate) fn invalidate_host_mirror(&self) {
        self.mirror_fresh.set(false);
    }

    fn host_bytes(&self) -> &[u8] {
        if !self.mirror_fresh.get() {
            let mut bytes = vec![0u8; self.byte_len()].into_boxed_slice();
            check(unsafe {
                rl_buffer_to_host(self.ctx, &self.raw, bytes.as_mut_ptr().cast(), bytes.len() as u64)
            })
            .expect("device download");
            self.mirrors.borrow_mut().push(bytes);
            self.mirror_fresh.set(true);
        }
        let mirrors = self.mirrors.borrow();
        let last = mirrors.last().expect("mirror");
        // The boxed bytes never move or drop while `self` lives.
        unsafe { std::slice::from_raw_parts(last.as_ptr(), last.len()) }
    }

    /// buffer.rs:160-164
    pub fn as_slice(&self) -> &[f32] {
        let bytes = self.host_bytes();
        unsafe { std::slice::from_raw_parts(bytes.as_ptr().cast(), self.len()) }
    }
    /// buffer.rs:166-169
    pub fn as_f16_slice(&self) -> &[half::f16] {
        let bytes = self.host_bytes();
        unsafe { std::slice::from_raw_parts(bytes.as_ptr().cast(), self.len()) }
    }
}

impl Drop for MetalBuffer {
    fn drop(&mut self) {
        // Back to the pool; reuse is stream-ordered, so kernels still reading
        // the block finish first.
        unsafe { rl_buffer_release(self.ctx, &mut self.raw) }
    }
}

// ---------------------------------------------------------------- execution

/// Stands in for `metal::CommandBufferRef` in the crate-private `*_encode`
/// signatures: ops encoded "into the command buffer" are enqueued on the
/// context's stream, in order.
pub struct CommandBufferRef {
    ctx: *mut rl_context,
}

impl CommandBufferRef {
    pub(crate) fn raw(&self) -> *mut rl_context {
        self.ctx
    }
}

/// src/metal/execution.rs:5-37.
pub struct MetalExecution<'a> {
    context: &'a MetalContext,
    command_buffer: CommandBufferRef,
}

impl<'a> MetalExecution<'a> {
    /// execution.rs:11-21: opens a batch (counted as one command buffer).
    pub fn new(context: &'a MetalContext) -> Self {
        check(unsafe { rl_execution_begin(context.raw()) }).expect("execution begin");
        Self { context, command_buffer: CommandBufferRef { ctx: context.raw() } }
    }
    pub fn context(&self) -> &'a MetalContext {
        self.context
    }
    pub fn command_buffer(&self) -> &CommandBufferRef {
        &self.command_buffer
    }
    /// execution.rs:30-36: commit + wait.  Device errors, which the
    /// reference never checks, surface here as a panic carrying
    /// `TinyError::Metal`'s message.
    pub fn finish(self) {
        check(unsafe { rl_execution_finish(self.context.raw()) }).expect("device execution");
    }
}

// --------------------------------------------------------- op glue (example)

/// How an op body reads after the change: validation is the library's (same
/// order and messages as the reference), the output is allocated where the
/// reference allocates it, and the dispatch is one call.
pub(crate) mod ops_glue {
    use super::*;

    /// ops::add_f32_encode (src/ops/add.rs:18-49).
    pub(crate) fn add_f32_encode(
        context: &MetalContext,
        command_buffer: &CommandBufferRef,
        a: &MetalBuffer,
        b: &MetalBuffer,
    ) -> Result<MetalBuffer> {
        if a.len() != b.len() {
            return Err(TinyError::InvalidShape(format!(
                "add requires equal buffer lengths, got {} and {}",
                a.len(),
                b.len(),
            )));
        }
        let output = MetalBuffer::empty(context, a.len());
        check(unsafe { rl_add_f32(command_buffer.raw(), a.raw(), b.raw(), output.raw()) })?;
        Ok(output)
    }

    /// ops::kv_cache_write_f16_encode (src/ops/kv_cache_write.rs:54-69): the
    /// cache is written in place, so its host mirror goes stale.
    pub(crate) fn kv_cache_write_f16_encode(
        command_buffer: &CommandBufferRef,
        cache: &MetalBuffer,
        kv_heads: usize,
        max_seq: usize,
        head_dim: usize,
        source: &MetalBuffer,
        seq_len: usize,
        start: usize,
    ) -> Result<()> {
        check(unsafe {
            rl_kv_cache_write_f16(
                command_buffer.raw(),
                cache.raw(),
                kv_heads as u64,
                max_seq as u64,
                head_dim as u64,
                source.raw(),
                seq_len as u64,
                start as u64,
            )
        })?;
        cache.invalidate_host_mirror();
        Ok(())
    }
}

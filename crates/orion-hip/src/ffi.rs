//! Raw bindings to include/orion_hip.h.
//!
//! Every call returns 0 on success, 1 (`ORION_HIP_ERR_INTERNAL`) for an
//! invariant or index violation and 2 (`ORION_HIP_ERR_BACKEND`) for a device
//! or runtime failure; the message and stage of the last failure on the
//! calling thread come from `orion_hip_last_error` / `_stage`.  The struct
//! layouts below are the ones tests/abi/abi_check.cpp static_asserts.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_float, c_int, c_void};

pub const ORION_HIP_OK: c_int = 0;
pub const ORION_HIP_ERR_INTERNAL: c_int = 1;
pub const ORION_HIP_ERR_BACKEND: c_int = 2;

pub const ORION_DTYPE_F32: i32 = 0;
pub const ORION_DTYPE_F16: i32 = 1;
pub const ORION_DTYPE_BF16: i32 = 2;
pub const ORION_DTYPE_I8: i32 = 3;
pub const ORION_DTYPE_I4: i32 = 4;

#[repr(C)]
pub struct orion_hip_device {
    _p: [u8; 0],
}
#[repr(C)]
pub struct orion_hip_model {
    _p: [u8; 0],
}
#[repr(C)]
pub struct orion_hip_checkpoint {
    _p: [u8; 0],
}

/// ModelMetadata (traits.rs:95-123) plus the paged-cache geometry of
/// TransformerModel::new (transformer.rs:148-177).  60 bytes.
#[repr(C)]
#[derive(Debug, Clone, Copy, Default)]
pub struct orion_hip_model_desc {
    pub num_layers: i32,
    pub hidden_size: i32,
    pub num_attention_heads: i32,
    pub num_kv_heads: i32,
    pub head_dim: i32,
    pub intermediate_size: i32,
    pub vocab_size: i32,
    pub max_position_embeddings: i32,
    pub rms_norm_eps: c_float,
    pub rope_theta: c_float,
    pub has_qkv_bias: i32,
    pub tied_lm_head: i32,
    pub num_blocks: i32,
    pub block_size: i32,
    pub kv_dtype: i32,
}

/// ForwardBatch (traits.rs:193-228) with the block tables in CSR form.
/// 72 bytes.
#[repr(C)]
#[derive(Debug)]
pub struct orion_hip_batch {
    pub num_tokens: i64,
    pub num_seqs: i64,
    pub tokens: *const u32,
    pub positions: *const u32,
    pub slot_token_counts: *const i64,
    pub context_lens: *const i64,
    /// [num_seqs + 1]
    pub block_table_offsets: *const i64,
    pub block_table_ids: *const u32,
    pub has_prefill: i32,
}

/// The fields of orion_core::SamplingParams the device sampler reads.
/// 16 bytes.
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct orion_hip_sampling_params {
    pub temperature: c_float,
    pub top_k: i32,
    pub top_p: c_float,
    pub repetition_penalty: c_float,
}

extern "C" {
    pub fn orion_hip_last_error() -> *const c_char;
    pub fn orion_hip_last_error_stage() -> *const c_char;

    pub fn orion_hip_device_count(count: *mut c_int) -> c_int;
    pub fn orion_hip_device_open(ordinal: c_int, out: *mut *mut orion_hip_device) -> c_int;
    pub fn orion_hip_device_close(dev: *mut orion_hip_device);
    pub fn orion_hip_device_name(dev: *mut orion_hip_device, buf: *mut c_char, len: usize)
        -> c_int;
    pub fn orion_hip_mem_info(dev: *mut orion_hip_device, total: *mut u64, free: *mut u64)
        -> c_int;
    pub fn orion_hip_synchronize(dev: *mut orion_hip_device) -> c_int;
    pub fn orion_hip_supports_dtype(dev: *mut orion_hip_device, dtype: c_int) -> c_int;

    pub fn orion_hip_model_create(
        dev: *mut orion_hip_device,
        desc: *const orion_hip_model_desc,
        out: *mut *mut orion_hip_model,
    ) -> c_int;
    pub fn orion_hip_model_destroy(model: *mut orion_hip_model);
    pub fn orion_hip_model_upload_weight(
        model: *mut orion_hip_model,
        which: c_int,
        layer: c_int,
        host: *const c_void,
        dtype: c_int,
        count: usize,
    ) -> c_int;
    pub fn orion_hip_model_forward(
        model: *mut orion_hip_model,
        batch: *const orion_hip_batch,
        logits: *mut f32,
        argmax_out: *mut i64,
    ) -> c_int;

    pub fn orion_hip_checkpoint_open(dir: *const c_char, out: *mut *mut orion_hip_checkpoint)
        -> c_int;
    pub fn orion_hip_checkpoint_close(ck: *mut orion_hip_checkpoint);
    pub fn orion_hip_model_load_checkpoint(
        model: *mut orion_hip_model,
        ck: *const orion_hip_checkpoint,
    ) -> c_int;

    pub fn orion_hip_model_sample(
        model: *mut orion_hip_model,
        params: *const orion_hip_sampling_params,
        prev_offsets: *const i64,
        prev_tokens: *const u32,
        h_uniform: *const f32,
        h_tokens: *mut i32,
    ) -> c_int;
}

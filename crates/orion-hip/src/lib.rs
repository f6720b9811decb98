//! HIP backend for OrionServe-RS on AMD MI355X (gfx950).
//!
//! [`HipBackend`] implements [`orion_core::Backend`] (traits.rs:159-183) over a
//! device handle; [`HipTransformerModel`] implements
//! [`orion_core::LanguageModel`] (traits.rs:297-309) over a model handle that
//! owns the device weights and the paged KV arena, so `Engine::step`
//! (orion-runtime/src/engine.rs:310) drives it exactly as it drives the CPU
//! `TransformerModel`.  All arithmetic runs in liborion_hip.so; this crate
//! only marshals `ForwardBatch` into the C-ABI batch and maps status codes to
//! `EngineError`.
//!
//! NOT VERIFIED: written without a Rust toolchain; see Cargo.toml.
#![warn(missing_debug_implementations)]

pub mod ffi;

use std::collections::HashMap;
use std::ffi::{CStr, CString};
use std::path::Path;
use std::sync::Mutex;

use orion_core::{
    Backend, DType, Device, EngineError, ForwardBatch, ForwardOutput, LanguageModel, ModelError,
    ModelMetadata,
};
use orion_models::{Architecture, HfConfig};

const BACKEND: &str = "hip";

fn last_error() -> (String, String) {
    // SAFETY: the library returns NUL-terminated thread-local strings that
    // stay valid until the next failing call on this thread.
    unsafe {
        (
            CStr::from_ptr(ffi::orion_hip_last_error()).to_string_lossy().into_owned(),
            CStr::from_ptr(ffi::orion_hip_last_error_stage()).to_string_lossy().into_owned(),
        )
    }
}

/// `EngineError::Backend::stage` is `&'static str`; the library's stage names
/// are a small fixed set, so each distinct one is leaked once.
fn intern(stage: String) -> &'static str {
    static STAGES: Mutex<Option<HashMap<String, &'static str>>> = Mutex::new(None);
    let mut g = STAGES.lock().unwrap_or_else(|p| p.into_inner());
    let map = g.get_or_insert_with(HashMap::new);
    if let Some(s) = map.get(&stage) {
        return s;
    }
    let leaked: &'static str = Box::leak(stage.clone().into_boxed_str());
    map.insert(stage, leaked);
    leaked
}

/// Status code -> `EngineError` (error.rs:118-130): 1 is an invariant or index
/// violation (`Internal`), anything else a device failure (`Backend`).
fn check(rc: i32) -> Result<(), EngineError> {
    if rc == ffi::ORION_HIP_OK {
        return Ok(());
    }
    let (msg, stage) = last_error();
    if rc == ffi::ORION_HIP_ERR_INTERNAL {
        return Err(EngineError::Internal(msg));
    }
    Err(EngineError::Backend { backend: BACKEND, stage: intern(stage), reason: msg })
}

/// Load-time failures map back to the `ModelError` kind the library's message
/// starts with (the checkpoint loader uses the reference's wording).
fn check_load(rc: i32, dir: &Path) -> Result<(), ModelError> {
    if rc == ffi::ORION_HIP_OK {
        return Ok(());
    }
    let (msg, _) = last_error();
    Err(if msg.starts_with("tensor not found") {
        ModelError::TensorNotFound(msg)
    } else if msg.starts_with("unsupported dtype") {
        ModelError::UnsupportedDtype(msg)
    } else if msg.starts_with("missing file") {
        ModelError::MissingFile(dir.to_path_buf())
    } else if msg.starts_with("path not found") {
        ModelError::PathNotFound(dir.to_path_buf())
    } else {
        ModelError::Malformed { file: dir.display().to_string(), reason: msg }
    })
}

/// One MI355X.  Construction fails instead of returning a dead handle, as the
/// CUDA backend's constructor does (orion-cuda/src/lib.rs:110-132).
#[derive(Debug)]
pub struct HipBackend {
    dev: *mut ffi::orion_hip_device,
    ordinal: usize,
}

// SAFETY: the library serialises each device's work on one stream and keeps
// its error state thread-local; the engine calls from one thread (ADR 006).
unsafe impl Send for HipBackend {}
unsafe impl Sync for HipBackend {}

impl HipBackend {
    pub fn new(ordinal: usize) -> Result<Self, EngineError> {
        let mut dev = std::ptr::null_mut();
        // SAFETY: out-pointer to a local.
        check(unsafe { ffi::orion_hip_device_open(ordinal as i32, &mut dev) })?;
        Ok(Self { dev, ordinal })
    }

    /// Number of visible GPUs (0 when none).
    pub fn device_count() -> usize {
        let mut n = 0;
        // SAFETY: out-pointer to a local.
        if unsafe { ffi::orion_hip_device_count(&mut n) } != 0 {
            return 0;
        }
        n.max(0) as usize
    }

    /// Marketing name of the GPU.
    pub fn device_name(&self) -> String {
        let mut buf = [0 as std::os::raw::c_char; 256];
        // SAFETY: buffer and its length.
        unsafe { ffi::orion_hip_device_name(self.dev, buf.as_mut_ptr(), buf.len()) };
        // SAFETY: the library NUL-terminates within `len`.
        unsafe { CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned()
    }

    fn mem(&self) -> Option<(u64, u64)> {
        let (mut total, mut free) = (0u64, 0u64);
        // SAFETY: out-pointers to locals.
        (unsafe { ffi::orion_hip_mem_info(self.dev, &mut total, &mut free) } == 0)
            .then_some((total, free))
    }
}

impl Drop for HipBackend {
    fn drop(&mut self) {
        // SAFETY: the handle came from orion_hip_device_open and is closed once.
        unsafe { ffi::orion_hip_device_close(self.dev) }
    }
}

impl Backend for HipBackend {
    fn name(&self) -> &'static str {
        BACKEND
    }

    /// `Device` has only `Cpu` and `Cuda(usize)` (traits.rs:61-65); the GPU
    /// ordinal is reported through `Cuda` so orion-core needs no change.
    fn device(&self) -> Device {
        Device::Cuda(self.ordinal)
    }

    fn total_memory(&self) -> Option<u64> {
        self.mem().map(|(t, _)| t)
    }

    fn available_memory(&self) -> Option<u64> {
        self.mem().map(|(_, f)| f)
    }

    fn synchronize(&self) -> Result<(), EngineError> {
        // SAFETY: valid handle.
        check(unsafe { ffi::orion_hip_synchronize(self.dev) })
    }

    fn supports_dtype(&self, dtype: DType) -> bool {
        let code = match dtype {
            DType::F32 => ffi::ORION_DTYPE_F32,
            DType::F16 => ffi::ORION_DTYPE_F16,
            DType::BF16 => ffi::ORION_DTYPE_BF16,
            DType::I8 => ffi::ORION_DTYPE_I8,
            DType::I4 => ffi::ORION_DTYPE_I4,
        };
        // SAFETY: valid handle.
        unsafe { ffi::orion_hip_supports_dtype(self.dev, code) == 1 }
    }
}

/// A Llama/Qwen2 decoder whose weights and paged KV arena live on the GPU
/// (TransformerModel, transformer.rs:137-443, on the device).
#[derive(Debug)]
pub struct HipTransformerModel {
    meta: ModelMetadata,
    // Declared before `backend`: the model handle is destroyed first.
    model: ModelHandle,
    backend: HipBackend,
    /// Only for `Sync` (the reference keeps its KvStore behind a Mutex for the
    /// same reason); the engine calls `forward` from one thread.
    lock: Mutex<()>,
}

#[derive(Debug)]
struct ModelHandle(*mut ffi::orion_hip_model);

impl Drop for ModelHandle {
    fn drop(&mut self) {
        // SAFETY: the handle came from orion_hip_model_create and is destroyed once.
        unsafe { ffi::orion_hip_model_destroy(self.0) }
    }
}

// SAFETY: see HipBackend; all access to the handle goes through `lock`.
unsafe impl Send for HipTransformerModel {}
unsafe impl Sync for HipTransformerModel {}

impl HipTransformerModel {
    /// An empty model of this shape (weights zero until uploaded or loaded).
    /// `kv_dtype` is the arena's element type: `DType::BF16` for serving,
    /// `DType::F32` for the reference's own dtype.
    pub fn new(
        meta: ModelMetadata,
        intermediate_size: usize,
        has_qkv_bias: bool,
        tied_lm_head: bool,
        num_blocks: usize,
        block_size: usize,
        kv_dtype: DType,
        backend: HipBackend,
    ) -> Result<Self, EngineError> {
        let desc = ffi::orion_hip_model_desc {
            num_layers: meta.num_layers as i32,
            hidden_size: meta.hidden_size as i32,
            num_attention_heads: meta.num_attention_heads as i32,
            num_kv_heads: meta.num_kv_heads as i32,
            head_dim: meta.head_dim as i32,
            intermediate_size: intermediate_size as i32,
            vocab_size: meta.vocab_size as i32,
            max_position_embeddings: meta.max_position_embeddings as i32,
            rms_norm_eps: meta.rms_norm_eps,
            rope_theta: meta.rope_theta,
            has_qkv_bias: has_qkv_bias as i32,
            tied_lm_head: tied_lm_head as i32,
            num_blocks: num_blocks as i32,
            block_size: block_size as i32,
            kv_dtype: match kv_dtype {
                DType::F32 => ffi::ORION_DTYPE_F32,
                _ => ffi::ORION_DTYPE_BF16,
            },
        };
        let mut model = std::ptr::null_mut();
        // SAFETY: valid device handle, desc and out-pointer.
        check(unsafe { ffi::orion_hip_model_create(backend.dev, &desc, &mut model) })?;
        Ok(Self { meta, model: ModelHandle(model), backend, lock: Mutex::new(()) })
    }

    /// TransformerModel::from_directory (transformer.rs:180-205) on the GPU:
    /// the reference's own config parsing, then every safetensors tensor copied
    /// from the file mapping to the device in its stored dtype.
    pub fn from_directory(
        dir: &Path,
        num_blocks: usize,
        block_size: usize,
        backend: HipBackend,
    ) -> Result<Self, ModelError> {
        let config = HfConfig::load(dir)?;
        let arch = Architecture::detect(&config)?;
        let name = dir
            .file_name()
            .map(|s| s.to_string_lossy().into_owned())
            .unwrap_or_else(|| "model".into());
        let meta = config.to_metadata(name)?;
        let model = Self::new(
            meta,
            config.ffn_dim(),
            arch.has_qkv_bias(),
            config.ties_embeddings(),
            num_blocks,
            block_size,
            DType::BF16,
            backend,
        )
        .map_err(|e| ModelError::Malformed { file: dir.display().to_string(), reason: e.to_string() })?;
        let cdir = CString::new(dir.as_os_str().to_string_lossy().as_bytes())
            .map_err(|_| ModelError::PathNotFound(dir.to_path_buf()))?;
        let mut ck = std::ptr::null_mut();
        // SAFETY: NUL-terminated path, out-pointer to a local.
        check_load(unsafe { ffi::orion_hip_checkpoint_open(cdir.as_ptr(), &mut ck) }, dir)?;
        // SAFETY: valid model and checkpoint handles; the checkpoint is closed once.
        let rc = unsafe { ffi::orion_hip_model_load_checkpoint(model.model.0, ck) };
        unsafe { ffi::orion_hip_checkpoint_close(ck) };
        check_load(rc, dir)?;
        tracing::info!(
            architecture = %model.meta.architecture,
            layers = model.meta.num_layers,
            device = %model.backend.device_name(),
            "loaded model onto the GPU"
        );
        Ok(model)
    }

    /// The batch in C-ABI form: CSR block tables, counts widened to i64.
    fn run(&self, batch: &ForwardBatch, logits: *mut f32, argmax: *mut i64) -> Result<(), EngineError> {
        let s = batch.num_sequences();
        let mut offs = Vec::with_capacity(s + 1);
        let mut ids = Vec::with_capacity(batch.block_tables.iter().map(Vec::len).sum());
        offs.push(0i64);
        for t in &batch.block_tables {
            ids.extend_from_slice(t);
            offs.push(ids.len() as i64);
        }
        let counts: Vec<i64> = batch.slot_token_counts.iter().map(|&c| c as i64).collect();
        let ctx: Vec<i64> = batch.context_lens.iter().map(|&c| c as i64).collect();
        let raw = ffi::orion_hip_batch {
            num_tokens: batch.num_tokens() as i64,
            num_seqs: s as i64,
            tokens: batch.tokens.as_ptr(),
            positions: batch.positions.as_ptr(),
            slot_token_counts: counts.as_ptr(),
            context_lens: ctx.as_ptr(),
            block_table_offsets: offs.as_ptr(),
            block_table_ids: ids.as_ptr(),
            has_prefill: batch.has_prefill as i32,
        };
        let _g = self.lock.lock().unwrap_or_else(|p| p.into_inner());
        // SAFETY: every pointer in `raw` borrows a vector alive for the call;
        // `logits` / `argmax` are null or sized [num_sequences * vocab] / [num_sequences].
        check(unsafe { ffi::orion_hip_model_forward(self.model.0, &raw, logits, argmax) })
    }

    /// Forward that returns only each sequence's greedy token (the reference's
    /// argmax, runtime/src/sampling.rs:196-207): the logits stay on the device.
    pub fn forward_greedy(&self, batch: &ForwardBatch) -> Result<Vec<i64>, EngineError> {
        batch.validate()?;
        let mut am = vec![0i64; batch.num_sequences()];
        self.run(batch, std::ptr::null_mut(), am.as_mut_ptr())?;
        Ok(am)
    }
}

impl LanguageModel for HipTransformerModel {
    fn metadata(&self) -> &ModelMetadata {
        &self.meta
    }

    fn forward(&self, batch: &ForwardBatch) -> Result<ForwardOutput, EngineError> {
        batch.validate()?; // traits.rs:232-261
        let mut logits = vec![0f32; batch.num_sequences() * self.meta.vocab_size];
        self.run(batch, logits.as_mut_ptr(), std::ptr::null_mut())?;
        Ok(ForwardOutput {
            logits,
            vocab_size: self.meta.vocab_size,
            sequence_ids: batch.sequence_ids.clone(),
        })
    }

    fn backend(&self) -> &dyn Backend {
        &self.backend
    }
}

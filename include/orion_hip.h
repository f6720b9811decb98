/*
 * orion_hip.h — C ABI of the MI355X (gfx950) backend for OrionServe-RS's hot path.
 *
 * The hot path is the reference's TransformerModel::forward
 * (crates/orion-models/src/transformer.rs:359-442): RMSNorm, Q/K/V projections,
 * RoPE, the paged KV-cache write, paged grouped-query attention over block
 * tables, the output projection, the SwiGLU MLP and the LM head.  This library
 * runs all of it on one AMD Instinct MI355X with hand-written HIP kernels.
 *
 * The reference binds a device through two Rust traits
 * (crates/orion-core/src/traits.rs):
 *   - `Backend` (traits.rs:159-183): name/device/memory/synchronize/dtype.
 *     -> orion_hip_device_* below.
 *   - `LanguageModel` (traits.rs:297-309): `forward(&ForwardBatch) ->
 *     ForwardOutput`.  -> orion_hip_model_* below.
 * A Rust crate wraps these entry points as `HipBackend: Backend` and
 * `HipTransformerModel: LanguageModel` so the scheduler and engine drive it
 * unchanged.
 *
 * Conventions
 *   - Every call returns an int status: 0 = ok, ORION_HIP_ERR_INTERNAL for an
 *     invariant/index violation (the reference's EngineError::Internal,
 *     crates/orion-core/src/error.rs:125-130), ORION_HIP_ERR_BACKEND for a
 *     device failure (EngineError::Backend, error.rs:118-124).  The message is
 *     in orion_hip_last_error() and the failing stage in
 *     orion_hip_last_error_stage(); both are thread-local.
 *   - Handles are opaque.  A device owns one HIP stream; every operation on
 *     the device (and on models created on it) is enqueued on that stream in
 *     call order.  Calls on one handle must not overlap (the reference engine
 *     is single-threaded, docs/adr/006-single-threaded-engine-loop.md); handles
 *     may be moved between threads.
 *   - Pointers named `d_*` are device pointers (from orion_hip_alloc); all
 *     others are host pointers.
 */
#ifndef ORION_HIP_H
#define ORION_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORION_HIP_OK 0
#define ORION_HIP_ERR_INTERNAL 1
#define ORION_HIP_ERR_BACKEND 2

/* DType, same order as the reference enum (traits.rs:21-29). */
#define ORION_DTYPE_F32 0
#define ORION_DTYPE_F16 1
#define ORION_DTYPE_BF16 2
#define ORION_DTYPE_I8 3
#define ORION_DTYPE_I4 4

typedef struct orion_hip_device orion_hip_device;
typedef struct orion_hip_model orion_hip_model;

/* Last error on this thread. */
const char* orion_hip_last_error(void);
const char* orion_hip_last_error_stage(void);

/* ---------------------------------------------------------------------------
 * Backend (traits.rs:159-183)
 * ------------------------------------------------------------------------- */

/* Number of visible GPUs; 0 when none (reference: orion-cuda device_count,
 * crates/orion-cuda/src/lib.rs:82-90). */
int orion_hip_device_count(int* count);

/* Opens a device.  Fails instead of returning a dead handle
 * (CudaBackend::new, crates/orion-cuda/src/lib.rs:110-132). */
int orion_hip_device_open(int ordinal, orion_hip_device** out);
void orion_hip_device_close(orion_hip_device* dev);

/* Backend::name is "hip"; this gives the marketing name of the GPU. */
int orion_hip_device_name(orion_hip_device* dev, char* buf, size_t len);

/* Backend::total_memory / available_memory (traits.rs:167-173). */
int orion_hip_mem_info(orion_hip_device* dev, uint64_t* total, uint64_t* free_bytes);

/* Backend::synchronize (traits.rs:175-179): waits for the device stream. */
int orion_hip_synchronize(orion_hip_device* dev);

/* Backend::supports_dtype (traits.rs:182): F32, F16 and BF16 -> 1, else 0. */
int orion_hip_supports_dtype(orion_hip_device* dev, int dtype);

/* Device buffers and copies (used by the op-level entry points below). */
int orion_hip_alloc(orion_hip_device* dev, size_t bytes, void** d_ptr);
int orion_hip_free(orion_hip_device* dev, void* d_ptr);
int orion_hip_memcpy_h2d(orion_hip_device* dev, void* d_dst, const void* src, size_t bytes);
int orion_hip_memcpy_d2h(orion_hip_device* dev, void* dst, const void* d_src, size_t bytes);
int orion_hip_memcpy_d2d(orion_hip_device* dev, void* d_dst, const void* d_src, size_t bytes);
int orion_hip_memset(orion_hip_device* dev, void* d_dst, int value, size_t bytes);

/* Stream-ordered timer: start records an event on the device stream; stop
 * records a second one, waits for it and returns the elapsed milliseconds. */
int orion_hip_timer_start(orion_hip_device* dev);
int orion_hip_timer_stop(orion_hip_device* dev, float* ms);

/* Per-kernel timing of the attention and GEMM ops (no counterpart in the
 * reference: a measurement aid for roofline figures).  While enabled, every
 * orion_hip_paged_attention_decode / _prefill call records HIP events on the
 * device stream around its main kernel and around the split-K merge kernel
 * (decode only), and every orion_hip_gemm call around its launches (the GEMM
 * and, when it splits K, its reduce); nothing synchronises until _read, which
 * waits for the recorded events and returns the summed milliseconds and the
 * call count since the last enable.  Kernel indices: 0 = decode split-K
 * kernel, 1 = decode merge kernel, 2 = prefill kernel, 3 = orion_hip_gemm. */
int orion_hip_kernel_timing(orion_hip_device* dev, int enable);
int orion_hip_kernel_timing_read(orion_hip_device* dev, int kernel, double* total_ms,
                                 int64_t* calls);
/* The same events one launch at a time: up to `capacity` per-launch durations
 * (ms, in launch order) into ms_out, and the number of recorded launches in
 * *calls (for medians). */
int orion_hip_kernel_timing_samples(orion_hip_device* dev, int kernel, float* ms_out,
                                    int64_t capacity, int64_t* calls);

/* ---------------------------------------------------------------------------
 * LanguageModel (traits.rs:297-309) over TransformerModel
 * (transformer.rs:137-443)
 * ------------------------------------------------------------------------- */

/* Shape of a Llama/Qwen2 decoder (ModelMetadata, traits.rs:95-123, plus the
 * paged-cache geometry passed to TransformerModel::new, transformer.rs:148-177). */
typedef struct orion_hip_model_desc {
  int32_t num_layers;
  int32_t hidden_size;
  int32_t num_attention_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t intermediate_size; /* ffn_dim, config.rs:238-240 */
  int32_t vocab_size;
  int32_t max_position_embeddings;
  float rms_norm_eps;
  float rope_theta;
  int32_t has_qkv_bias; /* Architecture::has_qkv_bias, config.rs:134-139 */
  int32_t tied_lm_head; /* lm_head absent -> embed_tokens, transformer.rs:108-112 */
  int32_t num_blocks;   /* KV arena capacity in blocks */
  int32_t block_size;   /* tokens per block, power of two in [4, 256] */
  int32_t kv_dtype;     /* ORION_DTYPE_F32 or ORION_DTYPE_BF16 */
} orion_hip_model_desc;

/* Weight identifiers (HF names, transformer.rs:6-19).  Ids >= ORION_W_INPUT_NORM
 * are per layer. */
#define ORION_W_EMBED 0      /* model.embed_tokens.weight     [vocab, hidden]    */
#define ORION_W_FINAL_NORM 1 /* model.norm.weight             [hidden]           */
#define ORION_W_LM_HEAD 2    /* lm_head.weight                [vocab, hidden]    */
#define ORION_W_INPUT_NORM 3 /* input_layernorm.weight        [hidden]           */
#define ORION_W_Q 4          /* self_attn.q_proj.weight       [Hq*d, hidden]     */
#define ORION_W_K 5          /* self_attn.k_proj.weight       [Hkv*d, hidden]    */
#define ORION_W_V 6          /* self_attn.v_proj.weight       [Hkv*d, hidden]    */
#define ORION_W_O 7          /* self_attn.o_proj.weight       [hidden, Hq*d]     */
#define ORION_W_Q_BIAS 8     /* self_attn.q_proj.bias         [Hq*d]   (Qwen2)   */
#define ORION_W_K_BIAS 9     /* self_attn.k_proj.bias         [Hkv*d]  (Qwen2)   */
#define ORION_W_V_BIAS 10    /* self_attn.v_proj.bias         [Hkv*d]  (Qwen2)   */
#define ORION_W_POST_NORM 11 /* post_attention_layernorm.weight [hidden]         */
#define ORION_W_GATE 12      /* mlp.gate_proj.weight          [ffn, hidden]      */
#define ORION_W_UP 13        /* mlp.up_proj.weight            [ffn, hidden]      */
#define ORION_W_DOWN 14      /* mlp.down_proj.weight          [hidden, ffn]      */

/* Creates a model with zeroed weights and a zeroed KV arena
 * (TransformerModel::new, transformer.rs:148-177; KvStore::new, attention.rs:45-62).
 * The RoPE table is built on the host with the reference formula
 * (tensor.rs:228-253) and kept on the device. */
int orion_hip_model_create(orion_hip_device* dev, const orion_hip_model_desc* desc,
                           orion_hip_model** out);
void orion_hip_model_destroy(orion_hip_model* model);

/* Uploads one weight (ModelWeights::load, transformer.rs:62-120).  `dtype` is
 * the host data's type (F32, F16 or BF16); `count` elements.  Matrices are
 * stored as bf16 on the device (f32 input is rounded to nearest even), norm
 * gains and biases as f32. */
int orion_hip_model_upload_weight(orion_hip_model* model, int which, int layer,
                                  const void* host, int dtype, size_t count);

/* Fills every weight with a seeded synthetic initialisation (no checkpoint):
 * matrices ~ N(0, std) (integer Irwin-Hall sum of four 16-bit uniforms, then
 * rounded to bf16), norm gains 1, biases ~ N(0, std).  Bit-reproducible on any
 * host with orion_hip_synthetic_value(). */
int orion_hip_model_init_synthetic(orion_hip_model* model, uint64_t seed, float std);

/* The value orion_hip_model_init_synthetic() gives element `index` of weight
 * (`which`, `layer`), as f32 (for matrices: already rounded to bf16). */
float orion_hip_synthetic_value(uint64_t seed, int which, int layer, uint64_t index, float std);

/* ---- Safetensors checkpoints (crates/orion-models/src/loader.rs) ----------
 * A host-side handle over every `*.safetensors` file of a directory, memory-
 * mapped; names resolve to the first file (sorted paths) holding them
 * (CheckpointLoader::open, loader.rs:113-164).  Errors name the reference's
 * ModelError kind in the message: "path not found", "missing file",
 * "malformed", "tensor not found", "shape mismatch", "unsupported dtype". */
typedef struct orion_hip_checkpoint orion_hip_checkpoint;
int orion_hip_checkpoint_open(const char* dir, orion_hip_checkpoint** out);
void orion_hip_checkpoint_close(orion_hip_checkpoint* ck);
/* Distinct tensor names (CheckpointLoader::len, loader.rs:166-169). */
int orion_hip_checkpoint_num_tensors(const orion_hip_checkpoint* ck, int64_t* count);
/* Tensor `index` in sorted-name order (CheckpointLoader::names, :180-185):
 * its name (NUL-terminated, truncated to name_len), dtype (ORION_DTYPE_F32,
 * F16, BF16, or -1 for any other safetensors dtype), rank and shape
 * (up to 8 dimensions). */
int orion_hip_checkpoint_tensor_info(const orion_hip_checkpoint* ck, int64_t index, char* name,
                                     size_t name_len, int32_t* dtype, int32_t* ndim,
                                     int64_t* shape8);
/* Copies tensor `name` widened to f32 (CheckpointLoader::tensor, :188-202),
 * `count` must equal its element count.  Test hook. */
int orion_hip_checkpoint_read_f32(const orion_hip_checkpoint* ck, const char* name, float* out,
                                  size_t count);
/* Uploads every weight the model needs, by the Llama/Qwen2 names
 * (ModelWeights::load, transformer.rs:62-120), straight from the mapping in
 * the file's dtype: shapes are checked against the model description, Q/K/V
 * biases are read when the model has them (absent ones stay zero, as the
 * reference's optional_vector), and an untied model whose checkpoint has no
 * `lm_head.weight` gets the embedding as its head (transformer.rs:108-112). */
int orion_hip_model_load_checkpoint(orion_hip_model* model, const orion_hip_checkpoint* ck);

/* ---- Sampling on the device (runtime/src/sampling.rs DefaultSampler) -------
 * Per-row parameters, as SamplingParams (orion-core/src/sampling.rs:22-70)
 * holds them; each is validated as SamplingParams::validate does (:84-106) and
 * a violation is an ORION_HIP_ERR_INTERNAL naming the field. */
typedef struct orion_hip_sampling_params {
  float temperature;        /* 0 = greedy */
  int32_t top_k;            /* 0 = off */
  float top_p;              /* (0, 1]; 1 = off */
  float repetition_penalty; /* > 0; 1 = off */
} orion_hip_sampling_params;

/* Sampler::sample for every row of d_logits [rows, vocab] (device memory,
 * filtered in place as the reference's &mut logits): repetition penalty over
 * the row's previous tokens (host CSR: prev_offsets[rows + 1], prev_tokens),
 * then argmax for greedy rows, else temperature, top-k, top-p, softmax and the
 * draw with the row's uniform r in [0, 1) (host, h_uniform[rows]; the
 * reference draws it from the request's ChaCha8Rng).  Writes one token per
 * row to host memory.  vocab <= 262144. */
int orion_hip_sample(orion_hip_device* dev, float* d_logits, int64_t rows, int64_t vocab,
                     const orion_hip_sampling_params* params, const int64_t* prev_offsets,
                     const uint32_t* prev_tokens, const float* h_uniform, int32_t* h_tokens);

/* The same over the logits of the model's last forward (one row per sequence),
 * which then never leave the device. */
int orion_hip_model_sample(orion_hip_model* model, const orion_hip_sampling_params* params,
                           const int64_t* prev_offsets, const uint32_t* prev_tokens,
                           const float* h_uniform, int32_t* h_tokens);

/* Reads one weight back as f32 (count elements).  Test hook. */
int orion_hip_model_download_weight(orion_hip_model* model, int which, int layer, float* host,
                                    size_t count);

/* ForwardBatch (traits.rs:193-210) in CSR form.  Block table of sequence s is
 * block_table_ids[block_table_offsets[s] .. block_table_offsets[s+1]]. */
typedef struct orion_hip_batch {
  int64_t num_tokens;
  int64_t num_seqs;
  const uint32_t* tokens;              /* [num_tokens] */
  const uint32_t* positions;           /* [num_tokens] */
  const int64_t* slot_token_counts;    /* [num_seqs], sums to num_tokens */
  const int64_t* context_lens;         /* [num_seqs] (carried, not used; as the reference) */
  const int64_t* block_table_offsets;  /* [num_seqs + 1] */
  const uint32_t* block_table_ids;
  int32_t has_prefill;
} orion_hip_batch;

/* LanguageModel::forward (transformer.rs:359-442): validates the batch
 * (traits.rs:232-261), writes this batch's K/V into the paged arena, runs all
 * layers and returns last-row logits [num_seqs, vocab] f32 into host memory.
 * `logits` may be NULL when only `argmax_out` is wanted.  `argmax_out`
 * (optional, [num_seqs]) receives the greedy token of each row with the
 * reference's tie rule (runtime/src/sampling.rs:196-207); -1 where no logit
 * exceeds -inf.  A refused batch (ORION_HIP_ERR_INTERNAL) leaves the arena and
 * the weights untouched: its block ids are checked before any K/V is written
 * (the other checks before anything is launched). */
int orion_hip_model_forward(orion_hip_model* model, const orion_hip_batch* batch, float* logits,
                            int64_t* argmax_out);

/* KvStore::read / write (attention.rs:107-134) for one (layer, block, slot,
 * head) vector of head_dim f32 values; bounds errors as the reference. */
int orion_hip_model_kv_read(orion_hip_model* model, int64_t layer, uint32_t block, int64_t slot,
                            int64_t head, int is_value, float* out);
int orion_hip_model_kv_write(orion_hip_model* model, int64_t layer, uint32_t block, int64_t slot,
                             int64_t head, int is_value, const float* vec, int64_t len);

/* Device address and byte size of the model's KV arena; its geometry and
 * block-internal layout come from orion_hip_model_kv_layout. */
int orion_hip_model_kv_arena(orion_hip_model* model, void** d_arena, size_t* bytes);

/* ---------------------------------------------------------------------------
 * Op-level entry points (device pointers, enqueued on the device stream).
 * These are the per-kernel validation gate of docs/cuda.md:80-116.
 * ------------------------------------------------------------------------- */

/* Geometry of a paged KV arena (KvStore, attention.rs:34-62).  head_major = 0
 * is the reference layout [layer][block][k|v][slot][kv_head][dim]
 * (attention.rs:11-22); head_major = 1 stores each block as
 * [kv_head][k|v][slot][dim], so one head's K (or V) of a block is one
 * contiguous block_size x dim run.  Block ids index either the same way. */
typedef struct orion_hip_kv_layout {
  int64_t num_layers;
  int64_t num_blocks;
  int64_t block_size;
  int64_t num_kv_heads;
  int64_t head_dim;
  int32_t dtype; /* ORION_DTYPE_F32 or ORION_DTYPE_BF16 */
  int32_t head_major;
} orion_hip_kv_layout;

/* Geometry and layout of a model's KV arena (KvStore::new, attention.rs:45-62),
 * for use with the op-level entry points on orion_hip_model_kv_arena. */
int orion_hip_model_kv_layout(orion_hip_model* model, orion_hip_kv_layout* out);

/* Work plan for paged decode attention over one batch of query rows.  Built
 * on the host from host copies of the rows' positions, their sequence index
 * and the CSR block tables: each row's context is cut into chunks and the
 * (row, kv head, chunk) items are ordered longest first, which keeps the chip
 * evenly loaded on ragged batches; each item carries its table offset and first
 * block id.  A plan depends only on the batch, so one plan serves every layer
 * of a forward pass.  The plan also owns the split-K workspace.  Rows whose
 * position has no block in their table are rejected (EngineError::Internal).
 * Rows whose tables start with the same block ids (a shared prefix, as
 * prefix caching leaves them) attend that prefix together on bf16 arenas at
 * head_dim 64/128: the query heads of up to 16 / (query heads per KV head)
 * such rows share one work item per prefix piece ("packed" items), so each
 * prefix block is read once per pack rather than once per row. */
typedef struct orion_hip_decode_plan orion_hip_decode_plan;
int orion_hip_decode_plan_create(orion_hip_device* dev, const uint32_t* positions,
                                 const int32_t* row_seq, const int64_t* block_table_offsets,
                                 const uint32_t* block_table_ids, int64_t num_rows,
                                 int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                 int64_t block_size, orion_hip_decode_plan** out);
void orion_hip_decode_plan_destroy(orion_hip_decode_plan* plan);
/* Chunk length in tokens, number of work items, chunks of the longest row. */
int orion_hip_decode_plan_info(const orion_hip_decode_plan* plan, int64_t* chunk,
                               int64_t* num_work, int64_t* max_splits);
/* Packed prefix items among num_work (as planned for a bf16 arena) and the
 * rows each packs (0 when nothing is packed).  No counterpart in the
 * reference: a planning statistic for tests and measurement. */
int orion_hip_decode_plan_packed(const orion_hip_decode_plan* plan, int64_t* packed_items,
                                 int64_t* rows_per_pack);

/* paged_attention (attention.rs:219-295) for `num_rows` independent query
 * rows: row r attends positions 0..=d_positions[r] of the sequence
 * d_row_seq[r] through that sequence's block table (CSR d_bt_offsets /
 * d_bt_ids).  d_q and d_out are [num_rows, num_q_heads, head_dim] f32.
 * `plan` must come from the same positions (host copy) and geometry.  Block
 * ids and table lengths are not re-checked on the device: the caller
 * guarantees every (position / block_size) < table length and every id
 * < num_blocks (orion_hip_model_forward checks this on the host). */
int orion_hip_paged_attention_decode(orion_hip_device* dev, const orion_hip_kv_layout* kv,
                                     const void* d_arena, int64_t layer, const float* d_q,
                                     int64_t num_rows, int64_t num_q_heads,
                                     const uint32_t* d_positions, const int32_t* d_row_seq,
                                     const int64_t* d_bt_offsets, const uint32_t* d_bt_ids,
                                     const orion_hip_decode_plan* plan, float* d_out);

/* paged_attention (attention.rs:219-295) for prefill chunks, as a dense
 * causal MFMA contraction: sequence s contributes query rows
 * d_q[d_row_start[s] .. d_row_start[s] + d_row_count[s]) whose positions are
 * consecutive from d_first_pos[s]; row i attends 0..=d_first_pos[s] + i.  Same
 * result per row as orion_hip_paged_attention_decode.  `max_rows` bounds every
 * d_row_count (it sizes the grid), `max_position` every position.  bf16 KV
 * only (an f32 arena returns a Backend error).  Operand precision `hilo`:
 * 0 rounds Q and the softmax weights P to bf16 (the MFMA-rate path for bf16
 * inputs); 1 carries each as a hi + lo bf16 pair (~16-bit products, twice the
 * MFMA work); 2 carries Q as a pair and rounds P; 3 rounds Q and carries P as
 * a pair.  Adding 16 to the mode writes each output row in the split operand
 * layout the prefill GEMMs read (per 8 values: 8 hi bf16, the value's top 16
 * bits, then 8 lo bf16, the top 16 bits of the remainder; the same bytes as
 * f32), which needs every sequence whole (a batch the kernel would cut into
 * key parts is a Backend error).  Other values are an Internal error.
 * Table lengths and block ids are the caller's guarantee, as for decode. */
int orion_hip_paged_attention_prefill(orion_hip_device* dev, const orion_hip_kv_layout* kv,
                                      const void* d_arena, int64_t layer, const float* d_q,
                                      int64_t num_q_heads, int64_t num_seqs,
                                      const int32_t* d_row_start, const int32_t* d_row_count,
                                      const uint32_t* d_first_pos, const int64_t* d_bt_offsets,
                                      const uint32_t* d_bt_ids, int64_t max_rows,
                                      int64_t max_position, int32_t hilo, float* d_out);

/* Slot mapping + KV write (transformer.rs:371-387 and :283-297) fused with
 * RoPE (tensor.rs:283-298): for each row, rotates its Q heads from d_q_in
 * (row stride q_stride elements) into d_q_out [rows, Hq*d] (must not alias
 * d_q_in), rotates its K heads from d_k, and writes K and V (d_v) into the
 * arena at (table[pos / bs], pos % bs).  Row strides are in elements, so the
 * three parts of one fused QKV buffer can be passed directly.  d_cos / d_sin
 * are the RoPE table [max_positions, head_dim/2] (tensor.rs:228-253).  As for
 * attention, table lengths and block ids are the caller's guarantee. */
int orion_hip_rope_and_cache(orion_hip_device* dev, const orion_hip_kv_layout* kv, void* d_arena,
                             int64_t layer, int64_t num_rows, int64_t num_q_heads,
                             const float* d_q_in, int64_t q_stride, float* d_q_out,
                             const float* d_k, int64_t k_stride, const float* d_v,
                             int64_t v_stride, const uint32_t* d_positions,
                             const int32_t* d_row_seq, const int64_t* d_bt_offsets,
                             const uint32_t* d_bt_ids, const float* d_cos, const float* d_sin);

/* rms_norm (tensor.rs:143-163): d_out[r] = d_x[r] * (1/sqrt(mean(x^2)+eps)) * w.
 * d_out may equal d_x. */
int orion_hip_rmsnorm(orion_hip_device* dev, const float* d_x, const float* d_weight,
                      int64_t rows, int64_t cols, float eps, float* d_out);

/* linear (tensor.rs:96-130): d_out[M,N] = d_x[M,K] * W[N,K]^T (+ bias[N]),
 * W bf16 row-major, x/out f32, f32 accumulation on bf16 MFMA (x is split
 * into two bf16 terms so its f32 value is kept to ~16 mantissa bits).
 * epilogue: ORION_GEMM_STORE writes (+ bias); ORION_GEMM_ACCUMULATE adds into
 * d_out (residual connection, transformer.rs:328-332); ORION_GEMM_SWIGLU
 * treats W's rows as gate/up interleaved in groups of 8 ([gate 0..7, up 0..7,
 * gate 8..15, ...], N a multiple of 16) and writes swiglu(gate, up)
 * (tensor.rs:175-189) into d_out[M, N/2]. */
#define ORION_GEMM_STORE 0
#define ORION_GEMM_ACCUMULATE 1
#define ORION_GEMM_SWIGLU 2
int orion_hip_gemm(orion_hip_device* dev, const float* d_x, const uint16_t* d_w,
                   const float* d_bias, int64_t M, int64_t N, int64_t K, int epilogue,
                   float* d_out);

/* orion_hip_gemm that allocates nothing (no counterpart in the reference: it
 * is for callers that cannot allocate device memory, such as code under HIP
 * graph capture or a serving loop that forbids hipMalloc).  Same arguments,
 * kernels and results as orion_hip_gemm; the split-K partial tiles of
 * decode-shaped calls (M <= 64) and the K-split sums of larger calls with
 * few output tiles go to a fixed 64 MiB device array that each GPU holds
 * for the life of the process, instead of the device's grown scratch.  A
 * shape whose required scratch exceeds 64 MiB is refused with
 * ORION_HIP_ERR_BACKEND.  The optional extra K splits of long-K calls (K >=
 * 8192 with fewer than 768 output tiles) are dropped when they do not fit,
 * so such a call can differ from orion_hip_gemm in f32 summation order.  Every call on one GPU shares that GPU's array;
 * the library orders the calls made through it on one GPU (any device
 * handle, any thread): each call's stream waits for an event recorded after
 * the previous call's launches.  Work that bypasses that order races on the
 * array: a captured graph of such a call replayed while another call runs. */
int orion_hip_gemm_noalloc(orion_hip_device* dev, const float* d_x, const uint16_t* d_w,
                           const float* d_bias, int64_t M, int64_t N, int64_t K, int epilogue,
                           float* d_out);

/* swiglu (tensor.rs:175-189): d_gate = silu(d_gate) * d_up, elementwise. */
int orion_hip_silu_mul(orion_hip_device* dev, float* d_gate, const float* d_up, int64_t count);

/* Greedy argmax per row (runtime/src/sampling.rs:196-207). */
int orion_hip_argmax(orion_hip_device* dev, const float* d_logits, int64_t rows, int64_t cols,
                     int64_t* d_out);

#ifdef __cplusplus
}
#endif

#endif /* ORION_HIP_H */

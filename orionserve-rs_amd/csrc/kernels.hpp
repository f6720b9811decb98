// Host-side launch wrappers for the gfx950 kernels (internal interface of
// liborion_hip.so; the public C ABI lives in include/orion_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <vector>

namespace orion {

// Geometry of a paged KV arena [layer][block][k|v][slot][kv_head][head_dim].
struct KvGeom {
  int64_t num_layers, num_blocks, block_size, num_kv_heads, head_dim;
  bool dtype_bf16;
  bool head_major = false;  // block-internal order [kv_head][k|v][slot] instead of [k|v][slot][kv_head]
};

// Element strides of the arena (one layer = num_blocks blocks).  Reference
// layout (attention.rs:11-22): [block][k|v][slot][kv_head][dim].  Head-major
// layout: [block][kv_head][k|v][slot][dim], so one head's K (or V) of a block
// is one contiguous block_size x dim run.
struct ArenaStrides {
  int64_t blk, v_off, slot, head, layer;
};
inline ArenaStrides arena_strides(const KvGeom& kv) {
  ArenaStrides a;
  const int64_t bs = kv.block_size, hkv = kv.num_kv_heads, D = kv.head_dim;
  a.blk = 2 * bs * hkv * D;
  if (kv.head_major) {
    a.head = 2 * bs * D;
    a.v_off = bs * D;
    a.slot = D;
  } else {
    a.head = D;
    a.v_off = bs * hkv * D;
    a.slot = hkv * D;
  }
  a.layer = kv.num_blocks * a.blk;
  return a;
}

// ---- attention --------------------------------------------------------------
// One decode work item: KV head `item % Hkv` of query row `item / Hkv` over
// context tokens [start, end), the row's piece `split` of `nsplit`.  The block
// table slice of the piece starts at block_table_ids[tbl_off]; blk0 is its
// first entry, so the first step's loads can be issued before the slice
// arrives.
struct DecodeWork {
  // shared: 1 when the item reads a block that another planned row also
  // reads, 2 for a packed prefix item (DecodePlanHost::num_packed)
  int32_t item, start, end, nsplit, tbl_off, blk0, shared, split;
};
// Decode work plan: packed prefix items first, then the others longest first;
// built on the host from the
// query positions and block tables, shared by every layer of a forward.
struct DecodePlanHost {
  int chunk = 0;       // longest piece, in tokens
  int max_splits = 0;  // most pieces of any row
  bool balanced = false;  // per-row piece lengths (else fixed chunks)
  std::vector<DecodeWork> work;
  std::vector<int32_t> row_nsplit;  // pieces per row (0: row not planned)
  std::vector<int32_t> rows;  // rows covered when a skip mask was given (else all)
  // No block is attended by two planned rows: K/V are then read once and
  // streamed past the caches; shared (prefix) blocks keep cached loads.
  bool stream_kv = true;
  // Some blocks are shared but some work items read none of them: those
  // items stream, the others keep cached loads (DecodeWork::shared).
  bool mixed_kv = false;
  // Packed items (DecodeWork::shared == 2, num_packed of them): a piece of a
  // prefix that up to pack_r rows share (identical leading block ids),
  // attended for all of them at once -- their query heads fill the query
  // columns of one MFMA wave, so the prefix is read once per pack instead of
  // once per row.  Entry item = pack * hkv + kv_head; the pack's rows are
  // pack_rows[pack * pack_r .. + pack_r) (-1: unused).  Their prefix pieces
  // are splits 0 .. np-1 of each of those rows; the rows' remaining context
  // follows as ordinary items with splits np ...
  int num_packed = 0;
  int pack_r = 0;
  std::vector<int32_t> pack_rows;
};
struct DecodePlanDev {
  const DecodeWork* work = nullptr;
  const int32_t* row_nsplit = nullptr;  // DecodePlanHost::row_nsplit on the device
  int num_work = 0;
  int chunk = 0;
  int max_splits = 0;
  float* ws = nullptr;  // split-K partials, decode_workspace_bytes()
  size_t ws_bytes = 0;
  const int32_t* rows = nullptr;  // rows to merge (nullptr: every row)
  int num_rows = 0;
  bool stream_kv = true;  // DecodePlanHost::stream_kv
  bool mixed_kv = false;  // DecodePlanHost::mixed_kv
  // packed prefix items (DecodePlanHost::num_packed, counted in num_work),
  // DecodePlanHost::pack_rows on the device, and rows per pack
  int num_packed = 0;
  const int32_t* pack_rows = nullptr;
  int pack_r = 0;
};
// pack_r: rows per packed prefix item; 0 packs nothing.  The decode kernels
// take packed items only on bf16 arenas at head_dim 64/128 with
// pack_r = 16 / (query heads per KV head) >= 2 (decode_pack_rows).
void build_decode_plan(const uint32_t* positions, const int32_t* row_seq,
                       const int64_t* bt_offsets, const uint32_t* bt_ids, int64_t rows,
                       int64_t hkv, int64_t block_size, int64_t wave_slots,
                       const uint8_t* skip_rows, DecodePlanHost* plan, int pack_r = 0);
size_t decode_workspace_bytes(int64_t rows, int64_t hq, int64_t D, int64_t max_splits);
// Rows per packed prefix item for this arena and grouping (0: no packing).
int decode_pack_rows(const KvGeom& kv, int64_t hq);
// Which launches of a decode pass to issue (the merge only runs when the
// plan splits some row).
enum class DecodePhase { kBoth, kSplit, kMerge };
// Merges split partials held in plan.ws (the decode split layout over `rows`
// batch rows, plan.max_splits slots per (row, head)) of the rows plan.rows
// lists, plan.row_nsplit[row] parts each, into out (the chunked-prefill key
// parts use it too).
hipError_t launch_split_merge(hipStream_t st, int64_t D, int64_t rows, int64_t hq,
                              const DecodePlanDev& plan, float* out);
hipError_t launch_paged_decode(hipStream_t st, const KvGeom& kv, const void* arena, int64_t layer,
                               const float* q, int64_t rows, int64_t hq,
                               const uint32_t* positions, const int32_t* row_seq,
                               const int64_t* bt_off, const uint32_t* bt_ids,
                               const DecodePlanDev& plan, float* out,
                               DecodePhase phase = DecodePhase::kBoth);

// Prefill work list: one entry per (sequence, tile of packed rows, part of
// its keys), longest first (by the key tiles it reads), so the longest
// workgroups are dispatched first.  A sequence whose tiles would read far
// more keys than an even share of the CUs is cut into nparts key ranges; each
// part writes unnormalised partial results (the decode split layout) that a
// merge combines.  Built on the host from the chunk lengths and first
// positions; the device copy is what launch_paged_prefill takes.
struct PrefillTile {
  int32_t seq, tile;
  int32_t kt0, kt1;      // key tiles [kt0, kt1) (64 keys each) this workgroup reads
  int32_t part, nparts;  // nparts > 1: partial results of part `part`
};
struct PrefillPlan {
  std::vector<PrefillTile> order;
  int max_parts = 1;
  // batch rows whose results come in parts, and parts per batch row (0 for
  // rows of unsplit sequences; sized to the batch's rows)
  std::vector<int32_t> split_rows, row_parts;
};
int prefill_waves();      // waves per prefill workgroup (8, or 4 with ORION_PREFILL_WAVES=4)
// 16-row MFMA tiles of packed rows per prefill wave: two, one at head_dim 256
// (its query operands and output accumulators take twice the registers).
constexpr int prefill_wave_row_tiles(int64_t head_dim) { return head_dim > 128 ? 1 : 2; }
int prefill_tile_rows(int64_t head_dim);  // packed rows per prefill workgroup
// Largest head_dim the attention and RoPE kernels take (any even value up to
// it; the reference accepts any even head_dim).
constexpr int kMaxHeadDim = 2048;
// Prefill operand precision bits (launch_paged_prefill `operands`): each set
// bit carries that operand as a hi + lo bf16 pair, each clear one rounds it
// to bf16.
constexpr int kPrefillQHiLo = 1, kPrefillPHiLo = 2;
// cus: compute units (one prefill workgroup each); hkv: KV heads (workgroups
// per work-list entry); cus = 0 never splits.
void build_prefill_order(const int32_t* row_start, const int32_t* row_count,
                         const uint32_t* first_pos, int64_t num_seqs, int64_t group, int64_t hkv,
                         int64_t cus, PrefillPlan* plan, int64_t head_dim = 128);
// Where split parts go: the decode split workspace layout over the batch's
// rows (slot = (row * hq + head) * max_parts + part).
struct PrefillSplitOut {
  float* ws_o = nullptr;
  float* ws_ml = nullptr;
  int max_parts = 1;
  // finished rows are written in the split operand layout of GemmFuse::x_hilo
  // (only when no row comes in parts)
  int out_hilo = 0;
};
hipError_t launch_paged_prefill(hipStream_t st, const KvGeom& kv, const void* arena,
                                int64_t layer, const float* q, int64_t hq,
                                const PrefillTile* order, int64_t num_tiles,
                                const int32_t* row_start, const int32_t* row_count,
                                const uint32_t* first_pos, const int64_t* bt_off,
                                const uint32_t* bt_ids, int operands, float* out,
                                const PrefillSplitOut& split = PrefillSplitOut{});
// Packed (row, query head) rows per prefill workgroup tile.

// ---- GEMM -------------------------------------------------------------------
enum class Epilogue : int {
  kStore = 0,       // out = x W^T (+ bias)
  kAccumulate = 1,  // out += x W^T
  kSwiGLU = 2,      // W rows interleaved in groups of 8 gate / 8 up rows;
                    // out[:, N/2] = silu(gate) * up
};
// K-slice partial tiles a split-K decode GEMM left unreduced for its consumer
// to sum (ws == nullptr: the GEMM wrote its output).  Element (row, col) =
// bias[col] (if any) + sum over slices ks, in slice order, of
// ws[((ks * n_tiles + col / bn) * tile_rows + row) * bn + col % bn].
struct GemmPartials {
  const float* ws = nullptr;
  int kslices = 0, n_tiles = 0, bn = 0, tile_rows = 0;
  const float* bias = nullptr;
};
#ifdef __HIPCC__
__device__ inline float partial_sum(const GemmPartials& p, int64_t row, int64_t col) {
  const int64_t tile = col / p.bn, c = col - tile * p.bn;
  const float* e = p.ws + (tile * p.tile_rows + row) * p.bn + c;
  const int64_t stride = (int64_t)p.n_tiles * p.tile_rows * p.bn;
  // Slices are loaded 8 at a time with every load of a group in flight, then
  // added in slice order (a slice past the end adds +0, which leaves the sum
  // unchanged).
  const float bias = p.bias ? p.bias[col] : 0.f;
  float v = 0.f;
  for (int ks0 = 0; ks0 < p.kslices; ks0 += 8) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = ks0 + j < p.kslices ? e[(ks0 + j) * stride] : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) v += t[j];
  }
  return p.bias ? v + bias : v;
}
#endif

// Scratch for split-K decode GEMMs: the K-slice partial tiles.
struct GemmScratch {
  float* ws = nullptr;
  size_t ws_bytes = 0;
};
// Fusions a decode-shaped split-K GEMM (gemm_splitk_fusable) performs with
// its neighbours, so the RMSNorm and residual-add launches between the layer's
// GEMMs disappear:
//  - norm_*: x is the residual stream, and the GEMM multiplies
//    rms_norm(x[row]) * norm_weight, with the row's scale taken from the
//    per-row f64 sum-of-squares slots [row][norm_slots] a previous GEMM wrote
//    (summed in slot order) -- the same per-element roundings as rmsnorm;
//  - sumsq_out (kAccumulate): after out += x W^T, the GEMM writes the f64 sum
//    of squares of each updated row in gemm_sumsq_slots(N) slots per row
//    (slot j covers columns 64j .. 64j+63);
//  - defer (kStore): the K-slice partials are left unreduced for the consumer
//    (launch_rope_and_cache) instead of a reduce launch.
struct GemmFuse {
  const double* norm_sumsq = nullptr;
  int norm_slots = 0;
  const float* norm_weight = nullptr;
  float norm_eps = 0.f;
  double* sumsq_out = nullptr;
  GemmPartials* defer = nullptr;
  // The same weights in the decode kernel's packed order (launch_gemv_pack with
  // this shape and w_packed_deferred); read instead of w by the decode-shaped
  // split-K kernel and the LDS-tiled kernel (which then also takes M in
  // (64, 256)).  w may be null when w_packed is given.
  const uint16_t* w_packed = nullptr;
  bool w_packed_deferred = false;
  // The LDS-tiled kernel only (M > 64): x arrives already split into its
  // bf16 hi/lo pair (the layout launch_rmsnorm and the SwiGLU epilogue write
  // with `hilo`: per row, K/8 groups of [8 hi bf16 | 8 lo bf16], the same
  // bytes as f32), and a SwiGLU output is written that way.
  bool x_hilo = false;
  bool out_hilo = false;
};
// Bytes of W [N, K] in the decode kernel's packed order (0: K not a multiple
// of 32), and the kernel that writes it from row-major W.  `deferred` must be
// what the consuming launch_gemm calls will have (GemmFuse::defer set, store
// epilogue, no sums of squares).
size_t gemv_packed_bytes(int64_t N, int64_t K, bool deferred);
hipError_t launch_gemv_pack(hipStream_t st, const uint16_t* w, int64_t N, int64_t K,
                            bool deferred, uint16_t* out);
// The inverse: row-major W [N, K] from its packed copy.
hipError_t launch_gemv_unpack(hipStream_t st, const uint16_t* packed, int64_t N, int64_t K,
                              bool deferred, uint16_t* w);
bool gemm_splitk_fusable(int64_t M, int64_t N, int64_t K);
int gemm_sumsq_slots(int64_t N);

// Scratch a launch_gemm of this shape needs (0 / 0: none).
// Scratch a launch_gemm call of this shape uses: the decode GEMMs' K-slice
// partials, or the LDS-tiled GEMM's K-split sums (launch_gemm leaves a tiled
// GEMM unsplit when the scratch it is given is smaller).
// preferred: include the optional long-K splits (callers that can grow
// their scratch); false: only what the call requires.
void gemm_scratch_need(int64_t M, int64_t N, int64_t K, size_t* ws_bytes, bool preferred = true);
hipError_t launch_gemm(hipStream_t st, const float* x, const uint16_t* w, const float* bias,
                       int64_t M, int64_t N, int64_t K, Epilogue ep, float* out,
                       const GemmScratch* scratch = nullptr, const GemmFuse* fuse = nullptr);

// ---- sampling (runtime/src/sampling.rs DefaultSampler) ----------------------
// Per-row SamplingParams fields the sampler reads (orion-core/src/sampling.rs).
struct SampleParams {
  float temperature;
  int32_t top_k;
  float top_p;
  float repetition_penalty;
};
constexpr int64_t kSampleMaxVocab = 262144;
// logits [rows, vocab] are filtered in place; probs_ws holds rows * vocab
// floats; out gets one token per row.
hipError_t launch_sample(hipStream_t st, float* logits, int64_t rows, int64_t vocab,
                         const SampleParams* params, const int64_t* prev_off,
                         const uint32_t* prev_tok, const float* uniform, float* probs_ws,
                         int32_t* out);

// ---- elementwise / normalisation -------------------------------------------
// sumsq: when set, also the row sums of squares in the residual GEMMs' slot
// layout (gemm_sumsq_slots(hidden) f64 per row).
hipError_t launch_embed(hipStream_t st, const uint32_t* tokens, int64_t n, const uint16_t* table,
                        int64_t hidden, float* out, double* sumsq = nullptr);
// rows selected by `row_index` (nullptr = identity)
// hilo: out holds each row as cols/8 groups of [8 hi bf16 | 8 lo bf16] (hi =
// the f32 value truncated to bf16, lo = the remainder truncated), the input
// layout of GemmFuse::x_hilo; needs cols % 8 == 0.
hipError_t launch_rmsnorm(hipStream_t st, const float* x, const int32_t* row_index,
                          const float* weight, int64_t rows, int64_t cols, float eps, float* out,
                          bool hilo = false);
// hidden[r] += (deferred GEMM output)[r], then out = rms_norm(hidden[r]) (the
// residual add of transformer.rs:328-345 fused with the next norm).  With
// row_index, only the gathered rows are computed and hidden is not written.
hipError_t launch_rope_and_cache(hipStream_t st, const KvGeom& kv, void* arena, int64_t layer,
                                 int64_t rows, int64_t hq, const float* q_in, int64_t q_stride,
                                 float* q_out, const float* k, int64_t k_stride, const float* v,
                                 int64_t v_stride, const uint32_t* positions,
                                 const int32_t* row_seq, const int64_t* bt_off,
                                 const uint32_t* bt_ids, const float* cos_t, const float* sin_t,
                                 const GemmPartials* qkv_partials = nullptr);
hipError_t launch_silu_mul(hipStream_t st, float* gate, const float* up, int64_t count);
hipError_t launch_argmax(hipStream_t st, const float* logits, int64_t rows, int64_t cols,
                         int64_t* out);
hipError_t launch_f32_to_bf16(hipStream_t st, const float* in, uint16_t* out, int64_t count);
hipError_t launch_synthetic_bf16(hipStream_t st, uint16_t* out, int64_t count, uint64_t key,
                                 float mul);
hipError_t launch_synthetic_f32(hipStream_t st, float* out, int64_t count, uint64_t key,
                                float mul);
hipError_t launch_fill_f32(hipStream_t st, float* out, int64_t count, float value);

// Synthetic-weight generator shared by host and device: splitmix64 of a
// per-tensor key plus the element index; the sum of the hash's four 16-bit
// fields (Irwin-Hall, mean 131070, sd 65536/sqrt(3)) centred and scaled.
__host__ __device__ inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
__host__ __device__ inline float synthetic_normal(uint64_t key, uint64_t index, float mul) {
  const uint64_t h = splitmix64(key + index);
  const int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
                    (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48);
  return (float)(s - 131070) * mul;
}
inline uint64_t synthetic_key(uint64_t seed, int which, int layer) {
  return splitmix64(seed ^ ((uint64_t)(which + 1) << 48) ^ ((uint64_t)(layer + 1) << 24));
}
constexpr float kIrwinHallSd = 37837.2265625f;  // 65536 / sqrt(3), rounded to f32

}  // namespace orion

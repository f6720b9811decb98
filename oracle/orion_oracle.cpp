// CPU oracle for the OrionServe-RS hot path.  TEST INFRASTRUCTURE ONLY.
//
// This file is the checker that the HIP backend is compared against.  It is a
// line-by-line C++ restatement of the reference CPU backend (which is Rust and
// cannot be compiled in this environment).  Only tests/, the smoke check and
// the bench's cpu_baseline leg may load it; the product library never does.
//
// Build: oracle/Makefile  (-O2 -ffp-contract=off, no fast-math, OpenMP).
// -ffp-contract=off matters: Rust never fuses a*b+c into an FMA, so neither
// may this restatement.  OpenMP is used only over *independent outputs*
// (rows x out-features in linear, (row, q-head) in attention), so every output
// element goes through exactly the same arithmetic sequence as in the
// single-threaded reference and the result is bit-identical at any thread count.
//
// Every function names the reference file:line it restates (paths relative to
// the reference repository root).
//
// Pinning (what checks this restatement beyond retyping it):
//   - locate / KvStore offsets: reference KATs (attention.rs:358-372) and brute
//     force enumeration (tests/test_oracle.py).
//   - linear / rms_norm / silu / swiglu / softmax / rope: reference KATs
//     (tensor.rs:315-536), closed forms, numpy/torch float64 cross-checks.
//   - paged_attention: reference KATs (attention.rs:378-658) and torch SDPA on
//     the de-paged dense K/V.
//   - model forward: reference fixture model (transformer.rs:459-523) and its
//     invariants (transformer.rs:601-746), plus a float64 numpy restatement.
//   - bit-level agreement with the compiled Rust binary for transcendental
//     results (expf/powf/cosf/sinf) is unpinned: the oracle calls glibc, which
//     is what Rust's f32 methods lower to on linux-gnu.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#include <limits>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_API extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_last_error;

int fail(const std::string& msg) {
  g_last_error = msg;
  return 1;  // EngineError::Internal
}

}  // namespace

ORACLE_API const char* oracle_last_error() { return g_last_error.c_str(); }

ORACLE_API int oracle_num_threads() {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

ORACLE_API void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

// ---------------------------------------------------------------------------
// tensor.rs
// ---------------------------------------------------------------------------

// tensor.rs:96-130 `linear`: out[i][j] = (sum_k x[i][k]*W[j][k]) + (b[j] or 0.0),
// sequential f32 accumulation starting from 0.0, W is [out_features, in_features].
// Rows are computed in blocks of 16, each block against 2 weight rows at a
// time, with the 16 row accumulators held in 4-wide vector registers: this is
// only data parallelism across independent outputs.  Each accumulator still
// sees the reference's exact operation sequence (acc = acc + x*w, rounded
// after the multiply and after the add, k ascending, starting from 0.0).
typedef float orc_v4 __attribute__((vector_size(16)));

ORACLE_API int oracle_linear(const float* x, int64_t n, int64_t k, const float* w,
                             int64_t out_features, int64_t in_features,
                             const float* bias, int64_t bias_len, float* out) {
  if (k != in_features)
    return fail("linear shape mismatch: input has " + std::to_string(k) +
                " features, weight expects " + std::to_string(in_features));
  if (bias && bias_len != out_features)
    return fail("bias has " + std::to_string(bias_len) + " elements, expected " +
                std::to_string(out_features));
  constexpr int64_t R = 16;
  const int64_t nb = (n + R - 1) / R;
  // x transposed per 16-row block, [block][t][16], zero rows past n
  std::vector<orc_v4> xt((size_t)nb * k * (R / 4));
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nb; ++b) {
    float* dst = reinterpret_cast<float*>(xt.data() + (size_t)b * k * (R / 4));
    for (int64_t r = 0; r < R; ++r) {
      const int64_t i = b * R + r;
      for (int64_t t = 0; t < k; ++t) dst[t * R + r] = i < n ? x[i * k + t] : 0.0f;
    }
  }
  const int64_t jb = (out_features + 1) / 2;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < nb; ++b) {
    for (int64_t jj = 0; jj < jb; ++jj) {
      const int64_t j0 = jj * 2;
      const bool two = j0 + 1 < out_features;
      const float* w0 = w + j0 * in_features;
      const float* w1 = two ? w0 + in_features : w0;
      const orc_v4* xb = xt.data() + (size_t)b * k * (R / 4);
      orc_v4 a0 = {0, 0, 0, 0}, a1 = a0, a2 = a0, a3 = a0;
      orc_v4 c0 = a0, c1 = a0, c2 = a0, c3 = a0;
      for (int64_t t = 0; t < k; ++t) {
        const orc_v4* xv = xb + t * 4;
        const float s0 = w0[t], s1 = w1[t];
        const orc_v4 v0 = {s0, s0, s0, s0}, v1 = {s1, s1, s1, s1};
        a0 = a0 + xv[0] * v0;
        a1 = a1 + xv[1] * v0;
        a2 = a2 + xv[2] * v0;
        a3 = a3 + xv[3] * v0;
        c0 = c0 + xv[0] * v1;
        c1 = c1 + xv[1] * v1;
        c2 = c2 + xv[2] * v1;
        c3 = c3 + xv[3] * v1;
      }
      float ra[R], rc[R];
      __builtin_memcpy(ra, &a0, 16); __builtin_memcpy(ra + 4, &a1, 16);
      __builtin_memcpy(ra + 8, &a2, 16); __builtin_memcpy(ra + 12, &a3, 16);
      __builtin_memcpy(rc, &c0, 16); __builtin_memcpy(rc + 4, &c1, 16);
      __builtin_memcpy(rc + 8, &c2, 16); __builtin_memcpy(rc + 12, &c3, 16);
      for (int64_t r = 0; r < R; ++r) {
        const int64_t i = b * R + r;
        if (i >= n) break;
        out[i * out_features + j0] = ra[r] + (bias ? bias[j0] : 0.0f);
        if (two) out[i * out_features + j0 + 1] = rc[r] + (bias ? bias[j0 + 1] : 0.0f);
      }
    }
  }
  return 0;
}

// tensor.rs:143-163 `rms_norm` (in place): sum of squares in f64 (sequential),
// rms = sqrt(sum/cols + eps) in f64, scale = (1/rms) as f32, v = v*scale*w in f32.
ORACLE_API int oracle_rms_norm(float* x, int64_t rows, int64_t cols, const float* weight,
                               int64_t weight_len, float eps) {
  if (weight_len != cols)
    return fail("rms_norm weight has " + std::to_string(weight_len) + " elements, expected " +
                std::to_string(cols));
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float* row = x + r * cols;
    double sum_sq = 0.0;
    for (int64_t c = 0; c < cols; ++c) sum_sq += (double)row[c] * (double)row[c];
    const double rms = std::sqrt((sum_sq / (double)cols) + (double)eps);
    const float scale = (float)(1.0 / rms);
    for (int64_t c = 0; c < cols; ++c) row[c] = row[c] * scale * weight[c];
  }
  return 0;
}

// tensor.rs:167-169 `silu`: x / (1 + exp(-x)).
ORACLE_API float oracle_silu(float x) { return x / (1.0f + std::exp(-x)); }

// tensor.rs:175-189 `swiglu`: gate = silu(gate) * up, elementwise, in place.
ORACLE_API int oracle_swiglu(float* gate, int64_t gate_rows, int64_t gate_cols, const float* up,
                             int64_t up_rows, int64_t up_cols) {
  if (gate_rows != up_rows || gate_cols != up_cols)
    return fail("swiglu shape mismatch");
  const int64_t len = gate_rows * gate_cols;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < len; ++i) gate[i] = oracle_silu(gate[i]) * up[i];
  return 0;
}

// tensor.rs:192-209 `softmax_inplace`: max via fold(-inf, f32::max); a
// non-finite max gives the uniform distribution; otherwise exp(x-max) with a
// sequential f32 sum, then divide when the sum is positive.
static inline float rust_f32_max(float a, float b) {
  // f32::max ignores a NaN operand.
  if (std::isnan(a)) return b;
  if (std::isnan(b)) return a;
  return a > b ? a : b;
}

ORACLE_API void oracle_softmax_inplace(float* x, int64_t len) {
  float mx = -std::numeric_limits<float>::infinity();
  for (int64_t i = 0; i < len; ++i) mx = rust_f32_max(mx, x[i]);
  if (!std::isfinite(mx)) {
    const float uniform = 1.0f / (float)len;
    for (int64_t i = 0; i < len; ++i) x[i] = uniform;
    return;
  }
  float sum = 0.0f;
  for (int64_t i = 0; i < len; ++i) {
    x[i] = std::exp(x[i] - mx);
    sum += x[i];
  }
  if (sum > 0.0f)
    for (int64_t i = 0; i < len; ++i) x[i] /= sum;
}

// tensor.rs:228-253 `RopeTable::new`: inv_freq = 1 / theta^(2i/d) (f32 powf),
// angle = pos * inv_freq, cos/sin in f32; tables are [max_positions, head_dim/2].
ORACLE_API int oracle_rope_table(int64_t head_dim, int64_t max_positions, float theta,
                                 float* cos_out, float* sin_out) {
  if (head_dim % 2 != 0)
    return fail("RoPE requires an even head_dim, got " + std::to_string(head_dim));
  const int64_t half = head_dim / 2;
  for (int64_t pos = 0; pos < max_positions; ++pos) {
    for (int64_t i = 0; i < half; ++i) {
      const float inv_freq = 1.0f / std::pow(theta, 2.0f * (float)i / (float)head_dim);
      const float angle = (float)pos * inv_freq;
      cos_out[pos * half + i] = std::cos(angle);
      sin_out[pos * half + i] = std::sin(angle);
    }
  }
  return 0;
}

// tensor.rs:283-298 `apply_rope`: rotate-half pairing (i, i + d/2).
ORACLE_API int oracle_apply_rope(float* vec, int64_t len, const float* cos, const float* sin,
                                 int64_t table_width) {
  const int64_t half = len / 2;
  if (table_width != half)
    return fail("RoPE table width " + std::to_string(table_width) +
                " does not match half of head_dim " + std::to_string(half));
  for (int64_t i = 0; i < half; ++i) {
    const float x0 = vec[i];
    const float x1 = vec[i + half];
    vec[i] = x0 * cos[i] - x1 * sin[i];
    vec[i + half] = x0 * sin[i] + x1 * cos[i];
  }
  return 0;
}

// ---------------------------------------------------------------------------
// attention.rs
// ---------------------------------------------------------------------------

// attention.rs:182-186 `locate`: (table[pos / bs], pos % bs), or None past the table.
ORACLE_API int oracle_locate(const uint32_t* table, int64_t table_len, int64_t position,
                             int64_t block_size, uint32_t* block, int64_t* slot) {
  const int64_t logical = position / block_size;
  if (logical >= table_len) return 0;
  *block = table[logical];
  *slot = position % block_size;
  return 1;
}

// attention.rs:34-176 `KvStore`: the arena layout [layer][block][k|v][slot][head][dim].
struct KvDims {
  int64_t num_layers, num_blocks, block_size, num_kv_heads, head_dim;
};

// attention.rs:82-104 `block_stride` / `region_offset` / `slot_offset`.
static inline int64_t kv_slot_offset(const KvDims& d, int64_t layer, uint32_t block,
                                     int is_value, int64_t slot, int64_t head) {
  const int64_t stride = d.block_size * d.num_kv_heads * d.head_dim;
  const int64_t per_block = 2 * stride;
  const int64_t per_layer = d.num_blocks * per_block;
  return layer * per_layer + (int64_t)block * per_block + (is_value ? stride : 0) +
         (slot * d.num_kv_heads + head) * d.head_dim;
}

// attention.rs:136-175 `check_bounds`.
static int kv_check_bounds(const KvDims& d, int64_t layer, uint32_t block, int64_t slot,
                           int64_t head, int64_t vec_len) {
  if (layer >= d.num_layers || layer < 0)
    return fail("layer " + std::to_string(layer) + " out of range (have " +
                std::to_string(d.num_layers) + ")");
  if ((int64_t)block >= d.num_blocks)
    return fail("block " + std::to_string(block) + " out of range (have " +
                std::to_string(d.num_blocks) + ")");
  if (slot >= d.block_size || slot < 0)
    return fail("slot " + std::to_string(slot) + " out of range (block holds " +
                std::to_string(d.block_size) + ")");
  if (head >= d.num_kv_heads || head < 0)
    return fail("kv head " + std::to_string(head) + " out of range (have " +
                std::to_string(d.num_kv_heads) + ")");
  if (vec_len != d.head_dim)
    return fail("vector length " + std::to_string(vec_len) + " does not match head_dim " +
                std::to_string(d.head_dim));
  return 0;
}

ORACLE_API int64_t oracle_kv_len(int64_t L, int64_t nb, int64_t bs, int64_t hkv, int64_t d) {
  return L * nb * 2 * bs * hkv * d;
}

ORACLE_API int64_t oracle_kv_offset(int64_t L, int64_t nb, int64_t bs, int64_t hkv, int64_t d,
                                    int64_t layer, uint32_t block, int is_value, int64_t slot,
                                    int64_t head) {
  KvDims dims{L, nb, bs, hkv, d};
  return kv_slot_offset(dims, layer, block, is_value, slot, head);
}

// attention.rs:107-119 `KvStore::write`.
ORACLE_API int oracle_kv_write(float* arena, int64_t L, int64_t nb, int64_t bs, int64_t hkv,
                               int64_t d, int64_t layer, uint32_t block, int64_t slot,
                               int64_t head, int is_value, const float* vec, int64_t vec_len) {
  KvDims dims{L, nb, bs, hkv, d};
  if (kv_check_bounds(dims, layer, block, slot, head, vec_len)) return 1;
  std::memcpy(arena + kv_slot_offset(dims, layer, block, is_value, slot, head), vec,
              sizeof(float) * d);
  return 0;
}

// attention.rs:122-134 `KvStore::read`.
ORACLE_API int oracle_kv_read(const float* arena, int64_t L, int64_t nb, int64_t bs, int64_t hkv,
                              int64_t d, int64_t layer, uint32_t block, int64_t slot,
                              int64_t head, int is_value, float* out) {
  KvDims dims{L, nb, bs, hkv, d};
  if (kv_check_bounds(dims, layer, block, slot, head, d)) return 1;
  std::memcpy(out, arena + kv_slot_offset(dims, layer, block, is_value, slot, head),
              sizeof(float) * d);
  return 0;
}

// attention.rs:219-295 `paged_attention`, for one query head (the reference's
// per-head loop body, :255-292).  Returns nonzero on a table/bounds error.
static int attention_one_head(const float* arena, const KvDims& dims, const float* q,
                              const uint32_t* table, int64_t table_len, int64_t query_position,
                              int64_t layer, int64_t kv_head, float scale, float* scores,
                              float* o) {
  const int64_t d = dims.head_dim;
  const int64_t attend_len = query_position + 1;
  for (int64_t pos = 0; pos < attend_len; ++pos) {
    uint32_t block;
    int64_t slot;
    if (!oracle_locate(table, table_len, pos, dims.block_size, &block, &slot))
      return fail("position " + std::to_string(pos) + " is outside the block table of " +
                  std::to_string(table_len) + " blocks");
    if (kv_check_bounds(dims, layer, block, slot, kv_head, d)) return 1;
    const float* k = arena + kv_slot_offset(dims, layer, block, 0, slot, kv_head);
    float dot = 0.0f;
    for (int64_t t = 0; t < d; ++t) dot += q[t] * k[t];
    scores[pos] = dot * scale;
  }
  oracle_softmax_inplace(scores, attend_len);
  for (int64_t t = 0; t < d; ++t) o[t] = 0.0f;
  for (int64_t pos = 0; pos < attend_len; ++pos) {
    const float w = scores[pos];
    if (w == 0.0f) continue;
    uint32_t block;
    int64_t slot;
    if (!oracle_locate(table, table_len, pos, dims.block_size, &block, &slot))
      return fail("position " + std::to_string(pos) + " unmapped");
    const float* v = arena + kv_slot_offset(dims, layer, block, 1, slot, kv_head);
    for (int64_t t = 0; t < d; ++t) o[t] += w * v[t];
  }
  return 0;
}

// attention.rs:219-295 `paged_attention` for one query row, all heads.
// `context_len` is accepted and ignored, as in the reference (attention.rs:227-236):
// the attended length is query_position + 1.
ORACLE_API int oracle_paged_attention(const float* arena, int64_t L, int64_t nb, int64_t bs,
                                      int64_t hkv_store, int64_t d_store, const float* query,
                                      int64_t query_len, const uint32_t* table, int64_t table_len,
                                      int64_t context_len, int64_t query_position, int64_t layer,
                                      int64_t num_query_heads, int64_t num_kv_heads,
                                      int64_t head_dim, int64_t block_size, float* out,
                                      int64_t out_len) {
  (void)context_len;
  (void)bs;
  KvDims dims{L, nb, block_size, hkv_store, d_store};
  if (query_len != num_query_heads * head_dim || out_len != query_len)
    return fail("attention expected " + std::to_string(num_query_heads * head_dim) +
                " query elements, got " + std::to_string(query_len) + " (out " +
                std::to_string(out_len) + ")");
  if (num_kv_heads == 0 || num_query_heads % num_kv_heads != 0)
    return fail(std::to_string(num_query_heads) + " query heads cannot be grouped over " +
                std::to_string(num_kv_heads) + " kv heads");
  const int64_t group = num_query_heads / num_kv_heads;
  const float scale = 1.0f / std::sqrt((float)head_dim);
  std::vector<float> scores(query_position + 1);
  for (int64_t qh = 0; qh < num_query_heads; ++qh) {
    if (attention_one_head(arena, dims, query + qh * head_dim, table, table_len, query_position,
                           layer, qh / group, scale, scores.data(), out + qh * head_dim))
      return 1;
  }
  return 0;
}

// Batched decode attention over many independent query rows (the reference's
// per-row loop at transformer.rs:300-326 with all rows' KV already written).
// Each (row, head) output is computed exactly as paged_attention does it;
// OpenMP runs independent (row, head) pairs in parallel.
//   q: [rows, Hq*d]; row_seq[row] selects the CSR table; positions[row] is the
//   query position.
ORACLE_API int oracle_paged_attention_rows(const float* arena, int64_t L, int64_t nb, int64_t bs,
                                           int64_t hkv, int64_t d, int64_t layer, int64_t hq,
                                           int64_t rows, const float* q, const uint32_t* positions,
                                           const int32_t* row_seq, const int64_t* bt_offsets,
                                           const uint32_t* bt_ids, float* out) {
  KvDims dims{L, nb, bs, hkv, d};
  if (hkv == 0 || hq % hkv != 0) return fail("bad head grouping");
  const int64_t group = hq / hkv;
  const float scale = 1.0f / std::sqrt((float)d);
  int err = 0;
  std::string err_msg;
#pragma omp parallel
  {
    std::vector<float> scores;
#pragma omp for collapse(2) schedule(dynamic, 4)
    for (int64_t r = 0; r < rows; ++r) {
      for (int64_t h = 0; h < hq; ++h) {
        const int64_t seq = row_seq[r];
        const int64_t pos = positions[r];
        scores.resize(pos + 1);
        const uint32_t* table = bt_ids + bt_offsets[seq];
        const int64_t table_len = bt_offsets[seq + 1] - bt_offsets[seq];
        if (attention_one_head(arena, dims, q + (r * hq + h) * d, table, table_len, pos, layer,
                               h / group, scale, scores.data(), out + (r * hq + h) * d)) {
#pragma omp critical
          {
            err = 1;
            err_msg = g_last_error;
          }
        }
      }
    }
  }
  if (err) return fail(err_msg);
  return 0;
}

// runtime/src/sampling.rs:196-207 `argmax`: strict '>' scan from -inf, lowest
// index wins ties; -1 when nothing exceeds -inf (the reference's None).
ORACLE_API int64_t oracle_argmax(const float* logits, int64_t len) {
  int64_t best = -1;
  float best_val = -std::numeric_limits<float>::infinity();
  for (int64_t i = 0; i < len; ++i) {
    if (logits[i] > best_val) {
      best_val = logits[i];
      best = i;
    }
  }
  return best;
}

// ---- DefaultSampler (runtime/src/sampling.rs) -----------------------------
// The filters in the reference's order (sampling.rs:9-23): repetition
// penalty, then (unless greedy) temperature, top-k, top-p, softmax and the
// draw.  The draw takes the uniform r the reference's ChaCha8Rng would give
// (`rng.random::<f32>()`, sampling.rs:209-210) as an input: the RNG stream is
// the caller's.  Also reports how close r lies to the nearest cumulative
// boundary, so a caller can tell draws that any f32 rounding difference of
// the probabilities could move.
static const float kMasked = -1.0e30f;  // sampling.rs:36

// sampling.rs:46-60: sign-aware, once per distinct token, out-of-range ignored.
static void oracle_repetition_penalty(float* logits, int64_t len, const uint32_t* prev,
                                      int64_t nprev, float penalty) {
  if (penalty == 1.0f) return;
  std::vector<uint32_t> seen(prev, prev + nprev);
  std::sort(seen.begin(), seen.end());
  seen.erase(std::unique(seen.begin(), seen.end()), seen.end());
  for (uint32_t t : seen) {
    if ((int64_t)t >= len) continue;
    const float l = logits[t];
    logits[t] = l > 0.0f ? l / penalty : l * penalty;
  }
}

// sampling.rs:67-75
static void oracle_temperature(float* logits, int64_t len, float temperature) {
  if (temperature == 1.0f) return;
  const float inv = 1.0f / temperature;
  for (int64_t i = 0; i < len; ++i) logits[i] *= inv;
}

// sampling.rs:82-99: the k-th largest value is the threshold; strictly
// smaller logits are masked (ties with the threshold survive).
static void oracle_top_k(float* logits, int64_t len, int64_t k) {
  if (k == 0 || k >= len) return;
  std::vector<float> sorted(logits, logits + len);
  std::nth_element(sorted.begin(), sorted.begin() + (k - 1), sorted.end(),
                   [](float a, float b) { return a > b; });
  const float threshold = sorted[k - 1];
  for (int64_t i = 0; i < len; ++i)
    if (logits[i] < threshold) logits[i] = kMasked;
}

// sampling.rs:160-190: max over all, exp of the unmasked, sequential sum,
// per-element division; uniform when everything is masked or the sum is 0.
static void oracle_sampling_softmax(const float* logits, int64_t len, float* out) {
  float mx = -std::numeric_limits<float>::infinity();
  for (int64_t i = 0; i < len; ++i)
    if (logits[i] > mx) mx = logits[i];
  if (!std::isfinite(mx) || mx <= kMasked) {
    for (int64_t i = 0; i < len; ++i) out[i] = 1.0f / (float)len;
    return;
  }
  float sum = 0.0f;
  for (int64_t i = 0; i < len; ++i) {
    out[i] = 0.0f;
    if (logits[i] <= kMasked) continue;
    const float e = expf(logits[i] - mx);
    out[i] = e;
    sum += e;
  }
  if (sum > 0.0f) {
    for (int64_t i = 0; i < len; ++i) out[i] /= sum;
  } else {
    for (int64_t i = 0; i < len; ++i) out[i] = 1.0f / (float)len;
  }
}

// sampling.rs:108-144.  The reference's sort is unstable; equal
// probabilities are ordered here by index (the device does the same).
static void oracle_top_p(float* logits, int64_t len, float p) {
  if (p >= 1.0f) return;
  std::vector<float> probs(len);
  oracle_sampling_softmax(logits, len, probs.data());
  std::vector<std::pair<int64_t, float>> cand;
  for (int64_t i = 0; i < len; ++i)
    if (probs[i] > 0.0f && logits[i] > kMasked) cand.push_back({i, probs[i]});
  if (cand.empty()) return;
  std::stable_sort(cand.begin(), cand.end(),
                   [](const std::pair<int64_t, float>& a, const std::pair<int64_t, float>& b) {
                     return a.second > b.second;
                   });
  float cumulative = 0.0f;
  size_t cutoff = cand.size();
  for (size_t r = 0; r < cand.size(); ++r) {
    cumulative += cand[r].second;
    if (cumulative >= p) {
      cutoff = r + 1;
      break;
    }
  }
  for (size_t r = cutoff; r < cand.size(); ++r) logits[cand[r].first] = kMasked;
}

// Sampler::sample for DefaultSampler (sampling.rs:266-293) with the draw's
// uniform given.  `logits` is modified in place, as the reference's &mut row.
// Returns the token (-1 for an empty row); *margin = the distance from r to
// the nearest cumulative boundary of the final distribution (0 for greedy).
ORACLE_API int64_t oracle_sample(float* logits, int64_t len, const uint32_t* prev, int64_t nprev,
                                 float temperature, int64_t top_k, float top_p, float penalty,
                                 float r, float* margin) {
  if (margin) *margin = 0.0f;
  if (len <= 0) return -1;
  oracle_repetition_penalty(logits, len, prev, nprev, penalty);
  if (temperature == 0.0f) return oracle_argmax(logits, len);
  oracle_temperature(logits, len, temperature);
  oracle_top_k(logits, len, top_k);
  oracle_top_p(logits, len, top_p);
  std::vector<float> probs(len);
  oracle_sampling_softmax(logits, len, probs.data());
  // sample_from (sampling.rs:208-223)
  float cumulative = 0.0f, lo = 0.0f;
  for (int64_t i = 0; i < len; ++i) {
    lo = cumulative;
    cumulative += probs[i];
    if (r < cumulative) {
      if (margin) *margin = std::min(r - lo, cumulative - r);
      return i;
    }
  }
  int64_t last = -1;
  for (int64_t i = len - 1; i >= 0; --i)
    if (probs[i] > 0.0f) {
      last = i;
      break;
    }
  if (margin) *margin = r - cumulative;
  return last >= 0 ? last : len - 1;
}

// orion-cuda/src/lib.rs:206-224 `Tolerance::matches` and :269-317 `validate`:
// abs OR rel agreement; non-finite values match only the identical bit pattern.
ORACLE_API int64_t oracle_validate(const float* expected, const float* actual, int64_t n,
                                   float tol_abs, float tol_rel, float* max_abs, float* max_rel,
                                   int64_t* worst_index) {
  int64_t mismatches = 0;
  float mabs = 0.0f, mrel = 0.0f, worst = 0.0f;
  int64_t widx = -1;
  for (int64_t i = 0; i < n; ++i) {
    const float e = expected[i], a = actual[i];
    bool ok;
    if (!std::isfinite(e) || !std::isfinite(a)) {
      uint32_t be, ba;
      std::memcpy(&be, &e, 4);
      std::memcpy(&ba, &a, 4);
      ok = be == ba;
    } else {
      const float diff = std::fabs(e - a);
      ok = diff <= tol_abs || diff <= tol_rel * std::fabs(e);
    }
    if (!ok) ++mismatches;
    if (std::isfinite(e) && std::isfinite(a)) {
      const float ab = std::fabs(e - a);
      const float rel = std::fabs(e) > std::numeric_limits<float>::epsilon() ? ab / std::fabs(e) : 0.0f;
      mabs = mabs > ab ? mabs : ab;
      mrel = mrel > rel ? mrel : rel;
      if (ab > worst) {
        worst = ab;
        widx = i;
      }
    }
  }
  *max_abs = mabs;
  *max_rel = mrel;
  *worst_index = widx;
  return mismatches;
}

// ---------------------------------------------------------------------------
// transformer.rs: the model
// ---------------------------------------------------------------------------

struct OracleModelDesc {
  int32_t num_layers, hidden, num_q_heads, num_kv_heads, head_dim, ffn, vocab, max_positions;
  float rms_norm_eps, rope_theta;
  int32_t has_qkv_bias, tied_lm_head, num_blocks, block_size;
};

// Weight identifiers; the per-layer ones take a layer index.
enum OracleWeight {
  W_EMBED = 0,
  W_FINAL_NORM = 1,
  W_LM_HEAD = 2,
  W_INPUT_NORM = 3,
  W_Q = 4,
  W_K = 5,
  W_V = 6,
  W_O = 7,
  W_Q_BIAS = 8,
  W_K_BIAS = 9,
  W_V_BIAS = 10,
  W_POST_NORM = 11,
  W_GATE = 12,
  W_UP = 13,
  W_DOWN = 14,
};

struct OracleLayer {
  std::vector<float> input_norm, q, k, v, o, q_bias, k_bias, v_bias, post_norm, gate, up, down;
};

// transformer.rs:137-144 `TransformerModel` (weights + RoPE table + KV arena).
struct OracleModel {
  OracleModelDesc desc;
  std::vector<float> embed, final_norm, lm_head;
  std::vector<OracleLayer> layers;
  std::vector<float> rope_cos, rope_sin;
  std::vector<float> kv;
  KvDims dims;
  // Store K/V rounded to bf16 (nearest even), the KV dtype of the benchmark's
  // bf16 configurations; the reference's own KvStore is f32 (false).
  bool kv_bf16 = false;
};

ORACLE_API void* oracle_model_create(const OracleModelDesc* d) {
  if (d->num_kv_heads <= 0 || d->num_q_heads % d->num_kv_heads != 0) {
    fail("query heads cannot be grouped over kv heads");
    return nullptr;
  }
  auto* m = new OracleModel();
  m->desc = *d;
  m->layers.resize(d->num_layers);
  const int64_t half = d->head_dim / 2;
  m->rope_cos.resize((int64_t)d->max_positions * half);
  m->rope_sin.resize((int64_t)d->max_positions * half);
  // transformer.rs:148-177 `new`: RoPE table built once at load.
  if (oracle_rope_table(d->head_dim, d->max_positions, d->rope_theta, m->rope_cos.data(),
                        m->rope_sin.data())) {
    delete m;
    return nullptr;
  }
  m->dims = KvDims{d->num_layers, d->num_blocks, d->block_size, d->num_kv_heads, d->head_dim};
  m->kv.assign(oracle_kv_len(d->num_layers, d->num_blocks, d->block_size, d->num_kv_heads,
                             d->head_dim),
               0.0f);
  return m;
}

ORACLE_API void oracle_model_destroy(void* p) { delete static_cast<OracleModel*>(p); }

static float bf16_round_f32(float f);

// The arena's element type: 0 = f32 (KvStore, attention.rs:34-62), 1 = bf16
// values (each K/V element rounded to bf16, nearest even, when written).
ORACLE_API void oracle_model_set_kv_bf16(void* p, int on) {
  static_cast<OracleModel*>(p)->kv_bf16 = on != 0;
}

ORACLE_API float* oracle_model_kv(void* p, int64_t* len) {
  auto* m = static_cast<OracleModel*>(p);
  *len = (int64_t)m->kv.size();
  return m->kv.data();
}

static std::vector<float>* oracle_weight_slot(OracleModel* m, int which, int layer,
                                              int64_t* expect) {
  const auto& d = m->desc;
  const int64_t H = d.hidden, qd = (int64_t)d.num_q_heads * d.head_dim,
                kvd = (int64_t)d.num_kv_heads * d.head_dim, F = d.ffn, V = d.vocab;
  if (which >= W_INPUT_NORM && (layer < 0 || layer >= d.num_layers)) return nullptr;
  OracleLayer* l = which >= W_INPUT_NORM ? &m->layers[layer] : nullptr;
  switch (which) {
    case W_EMBED: *expect = V * H; return &m->embed;
    case W_FINAL_NORM: *expect = H; return &m->final_norm;
    case W_LM_HEAD: *expect = V * H; return &m->lm_head;
    case W_INPUT_NORM: *expect = H; return &l->input_norm;
    case W_Q: *expect = qd * H; return &l->q;
    case W_K: *expect = kvd * H; return &l->k;
    case W_V: *expect = kvd * H; return &l->v;
    case W_O: *expect = H * qd; return &l->o;
    case W_Q_BIAS: *expect = qd; return &l->q_bias;
    case W_K_BIAS: *expect = kvd; return &l->k_bias;
    case W_V_BIAS: *expect = kvd; return &l->v_bias;
    case W_POST_NORM: *expect = H; return &l->post_norm;
    case W_GATE: *expect = F * H; return &l->gate;
    case W_UP: *expect = F * H; return &l->up;
    case W_DOWN: *expect = H * F; return &l->down;
    default: return nullptr;
  }
}

ORACLE_API int oracle_model_set_weight(void* p, int which, int layer, const float* data,
                                       int64_t n) {
  auto* m = static_cast<OracleModel*>(p);
  int64_t expect = 0;
  auto* slot = oracle_weight_slot(m, which, layer, &expect);
  if (!slot) return fail("unknown weight id/layer");
  if (n != expect)
    return fail("weight has " + std::to_string(n) + " elements, expected " +
                std::to_string(expect));
  slot->assign(data, data + n);
  return 0;
}

// transformer.rs:230-347 `layer_forward`.
static int oracle_layer_forward(OracleModel* m, int64_t layer, std::vector<float>& hidden,
                                int64_t n, const uint32_t* positions,
                                const std::vector<std::pair<uint32_t, int64_t>>& slots,
                                const std::vector<int32_t>& seq_of_row, const int64_t* bt_offsets,
                                const uint32_t* bt_ids) {
  const auto& d = m->desc;
  const OracleLayer& w = m->layers[layer];
  const int64_t H = d.hidden, hd = d.head_dim, hq = d.num_q_heads, hkv = d.num_kv_heads;
  const int64_t qd = hq * hd, kvd = hkv * hd, F = d.ffn;
  const bool bias = d.has_qkv_bias && !w.q_bias.empty();

  // :245-246 pre-norm
  std::vector<float> normed = hidden;
  if (oracle_rms_norm(normed.data(), n, H, w.input_norm.data(), H, d.rms_norm_eps)) return 1;
  // :248-250 Q/K/V projections (+ optional Qwen2 bias, transformer.rs:76-84)
  std::vector<float> q(n * qd), k(n * kvd), v(n * kvd);
  if (oracle_linear(normed.data(), n, H, w.q.data(), qd, H, bias ? w.q_bias.data() : nullptr, qd,
                    q.data()))
    return 1;
  if (oracle_linear(normed.data(), n, H, w.k.data(), kvd, H,
                    (bias && !w.k_bias.empty()) ? w.k_bias.data() : nullptr, kvd, k.data()))
    return 1;
  if (oracle_linear(normed.data(), n, H, w.v.data(), kvd, H,
                    (bias && !w.v_bias.empty()) ? w.v_bias.data() : nullptr, kvd, v.data()))
    return 1;
  // :255-279 RoPE on every Q and K head
  const int64_t half = hd / 2;
  for (int64_t row = 0; row < n; ++row) {
    const int64_t pos = positions[row];
    if (pos >= d.max_positions)
      return fail("position " + std::to_string(pos) + " exceeds the RoPE table (" +
                  std::to_string(d.max_positions) + " entries)");
    const float* c = m->rope_cos.data() + pos * half;
    const float* s = m->rope_sin.data() + pos * half;
    for (int64_t h = 0; h < hq; ++h)
      if (oracle_apply_rope(q.data() + row * qd + h * hd, hd, c, s, half)) return 1;
    for (int64_t h = 0; h < hkv; ++h)
      if (oracle_apply_rope(k.data() + row * kvd + h * hd, hd, c, s, half)) return 1;
  }
  // :283-297 write every row's K and V before any attention
  if (m->kv_bf16) {
    for (float& x : k) x = bf16_round_f32(x);
    for (float& x : v) x = bf16_round_f32(x);
  }
  for (int64_t row = 0; row < n; ++row) {
    for (int64_t h = 0; h < hkv; ++h) {
      if (oracle_kv_write(m->kv.data(), d.num_layers, d.num_blocks, d.block_size, hkv, hd, layer,
                          slots[row].first, slots[row].second, h, 0,
                          k.data() + row * kvd + h * hd, hd))
        return 1;
      if (oracle_kv_write(m->kv.data(), d.num_layers, d.num_blocks, d.block_size, hkv, hd, layer,
                          slots[row].first, slots[row].second, h, 1,
                          v.data() + row * kvd + h * hd, hd))
        return 1;
    }
  }
  // :300-326 attention, one row at a time
  std::vector<float> attn(n * qd);
  if (oracle_paged_attention_rows(m->kv.data(), d.num_layers, d.num_blocks, d.block_size, hkv, hd,
                                  layer, hq, n, q.data(), positions, seq_of_row.data(),
                                  bt_offsets, bt_ids, attn.data()))
    return 1;
  // :328-332 output projection + residual
  std::vector<float> proj(n * H);
  if (oracle_linear(attn.data(), n, qd, w.o.data(), H, qd, nullptr, 0, proj.data())) return 1;
  for (int64_t i = 0; i < n * H; ++i) hidden[i] += proj[i];
  // :335-345 MLP
  normed = hidden;
  if (oracle_rms_norm(normed.data(), n, H, w.post_norm.data(), H, d.rms_norm_eps)) return 1;
  std::vector<float> gate(n * F), up(n * F);
  if (oracle_linear(normed.data(), n, H, w.gate.data(), F, H, nullptr, 0, gate.data())) return 1;
  if (oracle_linear(normed.data(), n, H, w.up.data(), F, H, nullptr, 0, up.data())) return 1;
  if (oracle_swiglu(gate.data(), n, F, up.data(), n, F)) return 1;
  std::vector<float> mlp(n * H);
  if (oracle_linear(gate.data(), n, F, w.down.data(), H, F, nullptr, 0, mlp.data())) return 1;
  for (int64_t i = 0; i < n * H; ++i) hidden[i] += mlp[i];
  return 0;
}

// transformer.rs:359-442 `forward` together with traits.rs:232-261 `validate`.
// Batch in CSR form: tokens/positions [n], slot_token_counts/context_lens [S],
// block tables bt_ids[bt_offsets[s] .. bt_offsets[s+1]].  logits: [S, vocab].
// `layers_to_run` < 0 runs all layers (a smaller value is a test hook).
ORACLE_API int oracle_model_forward(void* p, int64_t n, int64_t S, const uint32_t* tokens,
                                    const uint32_t* positions, const int64_t* slot_token_counts,
                                    const int64_t* context_lens, const int64_t* bt_offsets,
                                    const uint32_t* bt_ids, float* logits) {
  (void)context_lens;
  auto* m = static_cast<OracleModel*>(p);
  const auto& d = m->desc;
  int64_t summed = 0;
  for (int64_t s = 0; s < S; ++s) summed += slot_token_counts[s];
  if (summed != n)
    return fail("ForwardBatch slot token counts sum to " + std::to_string(summed) +
                " but there are " + std::to_string(n) + " tokens");
  if (n == 0) return 0;
  // :371-387 seq_of_row and slot mapping
  std::vector<int32_t> seq_of_row;
  seq_of_row.reserve(n);
  for (int64_t s = 0; s < S; ++s)
    for (int64_t c = 0; c < slot_token_counts[s]; ++c) seq_of_row.push_back((int32_t)s);
  std::vector<std::pair<uint32_t, int64_t>> slots(n);
  for (int64_t row = 0; row < n; ++row) {
    const int64_t seq = seq_of_row[row];
    uint32_t block;
    int64_t slot;
    if (!oracle_locate(bt_ids + bt_offsets[seq], bt_offsets[seq + 1] - bt_offsets[seq],
                       positions[row], d.block_size, &block, &slot))
      return fail("position " + std::to_string(positions[row]) +
                  " has no block in the table for sequence " + std::to_string(seq));
    slots[row] = {block, slot};
  }
  // :208-223 embed
  const int64_t H = d.hidden;
  std::vector<float> hidden(n * H);
  for (int64_t i = 0; i < n; ++i) {
    if ((int64_t)tokens[i] >= d.vocab)
      return fail("token id " + std::to_string(tokens[i]) + " is outside the vocabulary of " +
                  std::to_string(d.vocab));
    std::memcpy(hidden.data() + i * H, m->embed.data() + (int64_t)tokens[i] * H, 4 * H);
  }
  for (int64_t l = 0; l < d.num_layers; ++l)
    if (oracle_layer_forward(m, l, hidden, n, positions, slots, seq_of_row, bt_offsets, bt_ids))
      return 1;
  // :401-405 final norm
  if (oracle_rms_norm(hidden.data(), n, H, m->final_norm.data(), H, d.rms_norm_eps)) return 1;
  // :410-428 last row of each sequence
  std::vector<float> tail(S * H);
  int64_t cursor = 0;
  for (int64_t s = 0; s < S; ++s) {
    if (slot_token_counts[s] == 0) return fail("a scheduled sequence contributed zero tokens");
    cursor += slot_token_counts[s];
    std::memcpy(tail.data() + s * H, hidden.data() + (cursor - 1) * H, 4 * H);
  }
  // :430-441 LM head (tied to the embedding when absent)
  const std::vector<float>& head =
      (d.tied_lm_head || m->lm_head.empty()) ? m->embed : m->lm_head;
  return oracle_linear(tail.data(), S, H, head.data(), d.vocab, H, nullptr, 0, logits);
}

// ---------------------------------------------------------------------------
// Synthetic weights (test input generator, not a reference function)
// ---------------------------------------------------------------------------

// The HIP library's counter-based synthetic weights (orion_hip_synthetic_value
// / orion_hip_model_init_synthetic), restated so the oracle can hold the same
// model the bench runs without a GPU: splitmix64 of a per-tensor key plus the
// element index, the sum of the hash's four 16-bit fields (Irwin-Hall, mean
// 131070, sd 65536/sqrt(3)) centred and scaled by std / sd in f32, rounded to
// bf16 (nearest even) and widened back.  Norm weights are ones.  Checked
// element-wise against the library's host entry point and a numpy restatement
// (tests/test_cfg4_golden.py).
namespace {
uint64_t syn_mix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
}  // namespace

// f32 -> bf16 (nearest even; NaN stays NaN) -> f32.
static float bf16_round_f32(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    u = ((u >> 16) | 0x40u) << 16;
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
  }
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

ORACLE_API void oracle_synthetic_fill(uint64_t seed, int which, int layer, float std_,
                                      int64_t count, float* out) {
  const bool is_norm = which == 1 || which == 3 || which == 11;  // final, input, post norm
  if (is_norm) {
    for (int64_t i = 0; i < count; ++i) out[i] = 1.0f;
    return;
  }
  const int lay = which >= 3 ? layer : -1;
  const uint64_t key =
      syn_mix(seed ^ ((uint64_t)(which + 1) << 48) ^ ((uint64_t)(lay + 1) << 24));
  const float mul = std_ / 37837.2265625f;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    const uint64_t h = syn_mix(key + (uint64_t)i);
    const int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
                      (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48);
    out[i] = bf16_round_f32((float)(s - 131070) * mul);
  }
}

// Exercises the C-ABI the way a foreign caller (the Rust orion-hip crate's
// #[repr(C)] structs and extern "C" block) binds it: only include/orion_hip.h,
// plain pointers and sizes, the library linked as a shared object.
//
//   abi_check layout            prints sizes and field offsets of the ABI
//                               structs as JSON (no GPU call)
//   abi_check forward OUT.bin   opens device 0, builds a small model with
//                               synthetic weights, runs a prefill forward and
//                               a decode forward and writes their logits and
//                               greedy tokens to OUT.bin; also checks the
//                               Internal error path of an out-of-vocabulary
//                               token
//
// The static_asserts pin the layouts the Rust bindings declare (C rules on
// x86-64 Linux: 8-byte pointers and int64_t, 4-byte int32_t and float), so a
// change to a struct in the header breaks this build instead of the FFI.
#include <cmath>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/orion_hip.h"

static_assert(sizeof(orion_hip_model_desc) == 60, "orion_hip_model_desc size");
static_assert(offsetof(orion_hip_model_desc, num_layers) == 0, "");
static_assert(offsetof(orion_hip_model_desc, max_position_embeddings) == 28, "");
static_assert(offsetof(orion_hip_model_desc, rms_norm_eps) == 32, "");
static_assert(offsetof(orion_hip_model_desc, rope_theta) == 36, "");
static_assert(offsetof(orion_hip_model_desc, has_qkv_bias) == 40, "");
static_assert(offsetof(orion_hip_model_desc, kv_dtype) == 56, "");
static_assert(sizeof(orion_hip_batch) == 72, "orion_hip_batch size");
static_assert(offsetof(orion_hip_batch, num_seqs) == 8, "");
static_assert(offsetof(orion_hip_batch, tokens) == 16, "");
static_assert(offsetof(orion_hip_batch, positions) == 24, "");
static_assert(offsetof(orion_hip_batch, slot_token_counts) == 32, "");
static_assert(offsetof(orion_hip_batch, context_lens) == 40, "");
static_assert(offsetof(orion_hip_batch, block_table_offsets) == 48, "");
static_assert(offsetof(orion_hip_batch, block_table_ids) == 56, "");
static_assert(offsetof(orion_hip_batch, has_prefill) == 64, "");
static_assert(sizeof(orion_hip_sampling_params) == 16, "orion_hip_sampling_params size");
static_assert(offsetof(orion_hip_sampling_params, top_k) == 4, "");
static_assert(offsetof(orion_hip_sampling_params, top_p) == 8, "");
static_assert(offsetof(orion_hip_sampling_params, repetition_penalty) == 12, "");
static_assert(sizeof(orion_hip_kv_layout) == 48, "orion_hip_kv_layout size");
static_assert(offsetof(orion_hip_kv_layout, dtype) == 40, "");
static_assert(offsetof(orion_hip_kv_layout, head_major) == 44, "");


static void print_layout() {
  std::printf("{\"orion_hip_model_desc\": {\"size\": %zu, \"offsets\": {", sizeof(orion_hip_model_desc));
  const char* sep = "";
#define P(T, f) std::printf("%s\"%s\": %zu", sep, #f, offsetof(T, f)), sep = ", "
  P(orion_hip_model_desc, num_layers); P(orion_hip_model_desc, hidden_size);
  P(orion_hip_model_desc, num_attention_heads); P(orion_hip_model_desc, num_kv_heads);
  P(orion_hip_model_desc, head_dim); P(orion_hip_model_desc, intermediate_size);
  P(orion_hip_model_desc, vocab_size); P(orion_hip_model_desc, max_position_embeddings);
  P(orion_hip_model_desc, rms_norm_eps); P(orion_hip_model_desc, rope_theta);
  P(orion_hip_model_desc, has_qkv_bias); P(orion_hip_model_desc, tied_lm_head);
  P(orion_hip_model_desc, num_blocks); P(orion_hip_model_desc, block_size);
  P(orion_hip_model_desc, kv_dtype);
  std::printf("}}, \"orion_hip_batch\": {\"size\": %zu, \"offsets\": {", sizeof(orion_hip_batch));
  sep = "";
  P(orion_hip_batch, num_tokens); P(orion_hip_batch, num_seqs); P(orion_hip_batch, tokens);
  P(orion_hip_batch, positions); P(orion_hip_batch, slot_token_counts);
  P(orion_hip_batch, context_lens); P(orion_hip_batch, block_table_offsets);
  P(orion_hip_batch, block_table_ids); P(orion_hip_batch, has_prefill);
  std::printf("}}, \"orion_hip_sampling_params\": {\"size\": %zu, \"offsets\": {",
              sizeof(orion_hip_sampling_params));
  sep = "";
  P(orion_hip_sampling_params, temperature); P(orion_hip_sampling_params, top_k);
  P(orion_hip_sampling_params, top_p); P(orion_hip_sampling_params, repetition_penalty);
  std::printf("}}, \"orion_hip_kv_layout\": {\"size\": %zu, \"offsets\": {",
              sizeof(orion_hip_kv_layout));
  sep = "";
  P(orion_hip_kv_layout, num_layers); P(orion_hip_kv_layout, num_blocks);
  P(orion_hip_kv_layout, block_size); P(orion_hip_kv_layout, num_kv_heads);
  P(orion_hip_kv_layout, head_dim); P(orion_hip_kv_layout, dtype);
  P(orion_hip_kv_layout, head_major);
#undef P
  std::printf("}}}\n");
}

static int check(int rc, const char* what) {
  if (rc != ORION_HIP_OK)
    std::fprintf(stderr, "%s failed (%d): %s [%s]\n", what, rc, orion_hip_last_error(),
                 orion_hip_last_error_stage());
  return rc;
}

// The reference's greedy rule (runtime/src/sampling.rs:196-207).
static int64_t argmax_ref(const float* v, int64_t n) {
  int64_t best = -1;
  float bv = -INFINITY;
  for (int64_t i = 0; i < n; ++i)
    if (v[i] > bv) bv = v[i], best = i;
  return best;
}

static int run_forward(const char* out_path) {
  int count = 0;
  if (check(orion_hip_device_count(&count), "device_count") || count < 1) return 2;
  orion_hip_device* dev = nullptr;
  if (check(orion_hip_device_open(0, &dev), "device_open")) return 2;
  orion_hip_model_desc desc{};
  desc.num_layers = 2;
  desc.hidden_size = 256;
  desc.num_attention_heads = 4;
  desc.num_kv_heads = 2;
  desc.head_dim = 64;
  desc.intermediate_size = 512;
  desc.vocab_size = 1000;
  desc.max_position_embeddings = 512;
  desc.rms_norm_eps = 1e-5f;
  desc.rope_theta = 10000.0f;
  desc.has_qkv_bias = 1;
  desc.tied_lm_head = 0;
  desc.num_blocks = 32;
  desc.block_size = 16;
  desc.kv_dtype = ORION_DTYPE_F32;
  orion_hip_model* model = nullptr;
  if (check(orion_hip_model_create(dev, &desc, &model), "model_create")) return 2;
  if (check(orion_hip_model_init_synthetic(model, 77, 0.05f), "init_synthetic")) return 2;

  // prefill: two sequences of 5 and 9 tokens, tables [3, 4] and [10, 11]
  const int64_t V = desc.vocab_size;
  std::vector<uint32_t> tokens = {1, 17, 300, 5, 999, 42, 42, 7, 8, 650, 11, 12, 13, 14};
  std::vector<uint32_t> positions = {0, 1, 2, 3, 4, 0, 1, 2, 3, 4, 5, 6, 7, 8};
  std::vector<int64_t> counts = {5, 9}, ctx = {5, 9}, bt_off = {0, 2, 4};
  std::vector<uint32_t> bt_ids = {3, 4, 10, 11};
  orion_hip_batch b{};
  b.num_tokens = (int64_t)tokens.size();
  b.num_seqs = 2;
  b.tokens = tokens.data();
  b.positions = positions.data();
  b.slot_token_counts = counts.data();
  b.context_lens = ctx.data();
  b.block_table_offsets = bt_off.data();
  b.block_table_ids = bt_ids.data();
  b.has_prefill = 1;
  std::vector<float> logits(2 * V), logits2(2 * V);
  std::vector<int64_t> am(2), am2(2);
  if (check(orion_hip_model_forward(model, &b, logits.data(), am.data()), "forward prefill"))
    return 2;
  // decode: the greedy tokens at positions 5 and 9
  std::vector<uint32_t> t2 = {(uint32_t)am[0], (uint32_t)am[1]}, p2 = {5, 9};
  std::vector<int64_t> c2 = {1, 1}, x2 = {6, 10};
  orion_hip_batch d = b;
  d.num_tokens = 2;
  d.tokens = t2.data();
  d.positions = p2.data();
  d.slot_token_counts = c2.data();
  d.context_lens = x2.data();
  d.has_prefill = 0;
  if (check(orion_hip_model_forward(model, &d, logits2.data(), am2.data()), "forward decode"))
    return 2;
  int bad = 0;
  for (int s = 0; s < 2; ++s) {
    if (am[s] != argmax_ref(&logits[s * V], V) || am2[s] != argmax_ref(&logits2[s * V], V)) {
      std::fprintf(stderr, "device argmax differs from the reference rule on row %d\n", s);
      bad = 1;
    }
    for (int64_t i = 0; i < V; ++i)
      if (!std::isfinite(logits[s * V + i]) || !std::isfinite(logits2[s * V + i])) bad = 1;
  }
  // error path: an out-of-vocabulary token is EngineError::Internal (status 1)
  std::vector<uint32_t> t3 = {(uint32_t)V, 1};
  orion_hip_batch e = d;
  e.tokens = t3.data();
  const int rc = orion_hip_model_forward(model, &e, nullptr, nullptr);
  if (rc != ORION_HIP_ERR_INTERNAL || std::strlen(orion_hip_last_error()) == 0) {
    std::fprintf(stderr, "OOV token returned %d (%s)\n", rc, orion_hip_last_error());
    bad = 1;
  }
  FILE* f = std::fopen(out_path, "wb");
  if (!f) return 2;
  std::fwrite(logits.data(), 4, logits.size(), f);
  std::fwrite(logits2.data(), 4, logits2.size(), f);
  std::fwrite(am.data(), 8, 2, f);
  std::fwrite(am2.data(), 8, 2, f);
  std::fclose(f);
  orion_hip_model_destroy(model);
  orion_hip_device_close(dev);
  std::printf("abi_check forward: %s\n", bad ? "FAILED" : "ok");
  return bad;
}

int main(int argc, char** argv) {
  if (argc >= 2 && std::strcmp(argv[1], "layout") == 0) {
    print_layout();
    return 0;
  }
  if (argc >= 3 && std::strcmp(argv[1], "forward") == 0) return run_forward(argv[2]);
  std::fprintf(stderr, "usage: abi_check layout | abi_check forward OUT.bin\n");
  return 2;
}

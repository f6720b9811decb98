// Device-side DefaultSampler (crates/orion-runtime/src/sampling.rs:266-293):
// repetition penalty, then greedy argmax or temperature -> top-k -> top-p ->
// softmax -> draw, over rows of logits already in HBM, so only one token per
// row crosses to the host instead of the [rows, vocab] f32 logits.
//
// One 1024-thread workgroup per row.  The row is walked in tiles of
// 1024 x 8 elements: thread t holds elements [8t, 8t + 8) of each tile (two
// 16-byte loads, so a wave reads 2 KiB contiguously).  Order-sensitive
// quantities (the draw's cumulative sum, the tie ranks of top-p) are formed in
// index order inside a thread's 8 elements and by a fixed-tree prefix across
// threads and tiles: deterministic, and equal to the reference's sequential
// f32 sums up to rounding.
//
// The uniform `r` of each draw comes from the caller (the reference draws it
// from a per-request ChaCha8Rng, sampling.rs:209-210); everything after it is
// computed here.
#include "common.hpp"
#include "kernels.hpp"


namespace orion {

namespace {

constexpr int kT = 1024;  // threads per row
constexpr int kWavesPerRow = kT / 64;
constexpr float kMasked = -1.0e30f;  // sampling.rs:36

// Order-preserving uint key of a float (larger float -> larger key); NaN maps
// below every number, so it never wins a selection.
__device__ inline uint32_t fkey(float f) {
  if (f != f) return 0u;
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ inline float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

struct Scratch {
  float f[kWavesPerRow];
  uint32_t u[kWavesPerRow];
  int64_t i[kWavesPerRow];
};

// Block reductions in a fixed order (lanes by butterfly, then waves 0..15).
__device__ float block_sum(float v, Scratch& s) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < kWavesPerRow; ++w) t += s.f[w];
  return t;
}
__device__ float block_max(float v, Scratch& s) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.f[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = s.f[0];
  for (int w = 1; w < kWavesPerRow; ++w) t = fmaxf(t, s.f[w]);
  return t;
}
__device__ uint32_t block_count(uint32_t v, Scratch& s) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.u[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t t = 0;
  for (int w = 0; w < kWavesPerRow; ++w) t += s.u[w];
  return t;
}
__device__ int64_t block_min_i64(int64_t v, Scratch& s) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, (int64_t)__shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.i[threadIdx.x >> 6] = v;
  __syncthreads();
  int64_t t = s.i[0];
  for (int w = 1; w < kWavesPerRow; ++w) t = min(t, s.i[w]);
  return t;
}
__device__ int64_t block_max_i64(int64_t v, Scratch& s) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, (int64_t)__shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s.i[threadIdx.x >> 6] = v;
  __syncthreads();
  int64_t t = s.i[0];
  for (int w = 1; w < kWavesPerRow; ++w) t = max(t, s.i[w]);
  return t;
}

// Exclusive prefix of per-thread values in thread order, by a fixed tree
// (inclusive lane scan by shuffles, then the wave totals in wave order):
// deterministic.  `wave_tot` is a 16-entry shared array of the value type.
template <typename V>
__device__ V block_exclusive_prefix(V v, V* wave_tot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  V inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    const V n = __shfl_up(inc, o);
    if (lane >= o) inc += n;
  }
  __syncthreads();
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  V base = V(0);
  for (int w = 0; w < wave; ++w) base += wave_tot[w];
  return base + inc - v;
}

constexpr int kE = 8;            // contiguous elements per thread per tile
constexpr int kTile = kT * kE;   // elements per tile
constexpr int kLdsRow = 32768;  // rows up to this many entries are held in LDS

}  // namespace

// LDS_ROW: the row is copied into LDS (vocab <= kLdsRow) and every
// probability is recomputed from it when needed; otherwise it stays in memory
// (logits filtered in place, probabilities in probs_ws).
template <bool LDS_ROW>
__global__ void __launch_bounds__(kT)
    sample_kernel(float* __restrict__ logits, int64_t vocab,
                  const SampleParams* __restrict__ params, const int64_t* __restrict__ prev_off,
                  const uint32_t* __restrict__ prev_tok, const float* __restrict__ uniform,
                  float* __restrict__ probs_ws, int32_t* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ Scratch s;
  __shared__ float lds_x[LDS_ROW ? kLdsRow : 1];
  __shared__ uint32_t seen_mem[LDS_ROW ? 1 : kSampleMaxVocab / 32];
  // the penalty's bitmap shares the row's LDS (the row is loaded after it)
  uint32_t* seen = LDS_ROW ? reinterpret_cast<uint32_t*>(lds_x) : seen_mem;
  const int64_t row = blockIdx.x;
  float* gx = logits + row * vocab;
  float* gp = probs_ws + row * vocab;
  const SampleParams sp = params[row];
  const int tid = threadIdx.x;
  const int ntiles = (int)((vocab + kTile - 1) / kTile);
  float dummy = 0.f;
  auto idx = [&](int t, int e) { return (int64_t)t * kTile + (int64_t)tid * kE + e; };
  auto valid = [&](int t, int e) { return idx(t, e) < vocab; };
  auto X = [&](int t, int e) -> float& {
    if (!valid(t, e)) return dummy;
    if constexpr (LDS_ROW) return lds_x[idx(t, e)];
    else return gx[idx(t, e)];
  };

  // ---- repetition penalty (sampling.rs:46-60): once per distinct token ----
  if (sp.repetition_penalty != 1.0f) {
    for (int64_t w = tid; w < (vocab + 31) / 32; w += kT) seen[w] = 0u;
    __syncthreads();
    for (int64_t j = prev_off[row] + tid; j < prev_off[row + 1]; j += kT) {
      const uint32_t t = prev_tok[j];
      if ((int64_t)t >= vocab) continue;
      const uint32_t bit = 1u << (t & 31);
      if (!(atomicOr(&seen[t >> 5], bit) & bit)) {
        const float l = gx[t];
        gx[t] = l > 0.0f ? l / sp.repetition_penalty : l * sp.repetition_penalty;
      }
    }
    __syncthreads();
  }
  if constexpr (LDS_ROW) {
    __syncthreads();  // the bitmap is done with
    for (int64_t i = tid; i < vocab; i += kT) lds_x[i] = gx[i];
    __syncthreads();
  }
  // f(t, e) over every element, in index order per thread
  auto each = [&](auto f) {
    for (int t = 0; t < ntiles; ++t)
#pragma unroll
      for (int e = 0; e < kE; ++e)
        if (valid(t, e)) f(t, e);
  };

  // ---- greedy (SamplingParams::mode, temperature 0): argmax, strict '>' in
  // index order, lowest index on ties, NaN never wins (sampling.rs:196-207) ----
  if (sp.temperature == 0.0f) {
    float best = -INFINITY;
    int64_t bi = INT64_MAX;
    each([&](int t, int e) {
      if (X(t, e) > best) {
        best = X(t, e);
        bi = idx(t, e);
      }
    });
    const float bmax = block_max(best, s);
    const int64_t win = block_min_i64((best == bmax && bi != INT64_MAX) ? bi : INT64_MAX, s);
    if (tid == 0) out[row] = win == INT64_MAX ? -1 : (int32_t)win;
    return;
  }

  // ---- temperature (sampling.rs:67-75) ----
  if (sp.temperature != 1.0f) {
    const float inv = 1.0f / sp.temperature;
    each([&](int t, int e) { X(t, e) = X(t, e) * inv; });
  }
  __syncthreads();

  // ---- top-k (sampling.rs:82-99): the k-th largest value by a 4-pass radix
  // select on order-preserving keys; strictly smaller logits are masked ----
  if (sp.top_k > 0 && (int64_t)sp.top_k < vocab) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sel_prefix, sel_rank;
    if (tid == 0) {
      sel_prefix = 0u;
      sel_rank = (uint32_t)sp.top_k;  // rank among the remaining, 1-based
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) hist[tid] = 0u;
      __syncthreads();
      const uint32_t pre = sel_prefix;
      const uint32_t hi_mask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
      each([&](int t, int e) {
        const uint32_t k = fkey(X(t, e));
        if ((k & hi_mask) == pre) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      });
      __syncthreads();
      // bucket b holds the rank-th largest when the buckets above it hold
      // fewer than `rank` keys and b completes them (bucket 0 takes the rest)
      if (tid < 256) {
        const uint32_t rank = sel_rank;
        uint32_t higher = 0;
        for (int b2 = 255; b2 > tid; --b2) higher += hist[b2];
        if (higher < rank && (higher + hist[tid] >= rank || tid == 0)) {
          sel_prefix = pre | ((uint32_t)tid << shift);
          sel_rank = rank - higher;
        }
      }
      __syncthreads();
    }
    const float thr = key_float(sel_prefix);
    each([&](int t, int e) {
      if (X(t, e) < thr) X(t, e) = kMasked;
    });
    __syncthreads();
  }

  // softmax (sampling.rs:160-190) of the current row: its max and sum, and
  // each probability e / sum (recomputed from the row when it lives in
  // registers, stored in probs_ws otherwise)
  float sm_max = 0.f, sm_sum = 1.f;
  bool sm_uniform = true;
  const float sm_u = 1.0f / (float)vocab;
  auto P = [&](int t, int e) -> float {
    if constexpr (LDS_ROW) {
      const float v = X(t, e);
      return sm_uniform ? sm_u : (v <= kMasked ? 0.0f : expf(v - sm_max)) / sm_sum;
    } else {
      return valid(t, e) ? gp[idx(t, e)] : 0.0f;
    }
  };
  auto softmax_row = [&]() {
    float mloc = -INFINITY;
    each([&](int t, int e) { mloc = X(t, e) > mloc ? X(t, e) : mloc; });
    sm_max = block_max(mloc, s);
    sm_uniform = !(sm_max == sm_max) || isinf(sm_max) || sm_max <= kMasked;
    float part = 0.f;
    if (!sm_uniform) {
      each([&](int t, int e) {
        const float v = X(t, e);
        const float ev = v <= kMasked ? 0.0f : expf(v - sm_max);
        if constexpr (!LDS_ROW) gp[idx(t, e)] = ev;
        part += ev;
      });
    }
    sm_sum = block_sum(part, s);
    if (!sm_uniform && !(sm_sum > 0.0f)) sm_uniform = true;
    if constexpr (!LDS_ROW)
      each([&](int t, int e) { gp[idx(t, e)] = sm_uniform ? sm_u : gp[idx(t, e)] / sm_sum; });
    __syncthreads();
  };

  // ---- top-p (sampling.rs:108-144): keep the most probable candidates until
  // their mass reaches p, the crossing one included.  The crossing
  // probability K is found by a 4-pass radix select on probability keys
  // (descending), the bucket masses summed exactly in 2^-40 fixed point with
  // integer atomics (order-independent, so deterministic); then tokens above
  // K are kept, plus the first tied ones (index order) the cumulative sum
  // needs. ----
  if (sp.top_p < 1.0f) {
    softmax_row();
    constexpr double kFix = 1099511627776.0;  // 2^40
    // (at least one unit: the first candidate always reaches a positive p)
    const unsigned long long p_fix =
        max((unsigned long long)((double)sp.top_p * kFix), 1ull);
    __shared__ unsigned long long bmass[256];
    __shared__ unsigned long long sel_above;
    __shared__ uint32_t sel_key;
    __shared__ int sel_found;
    if (tid == 0) {
      sel_above = 0ull;
      sel_key = 0u;
      sel_found = 1;
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) bmass[tid] = 0ull;
      __syncthreads();
      const uint32_t pre = sel_key;
      const uint32_t hi_mask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
      each([&](int t, int e) {
        const float pv = P(t, e);
        const uint32_t k = __float_as_uint(pv);
        if (pv > 0.0f && X(t, e) > kMasked && (k & hi_mask) == pre)
          atomicAdd(&bmass[(k >> shift) & 255u], (unsigned long long)((double)pv * kFix));
      });
      __syncthreads();
      // bucket b holds the crossing when the mass above it stays below p and
      // b's mass reaches it; if no bucket does, the whole candidate mass is
      // below p and every candidate stays (cutoff = len)
      if (tid < 256) {
        const unsigned long long above0 = sel_above;
        unsigned long long higher = 0;
        for (int b2 = 255; b2 > tid; --b2) higher += bmass[b2];
        const unsigned long long above = above0 + higher;
        if (above < p_fix && above + bmass[tid] >= p_fix) {
          sel_key = pre | ((uint32_t)tid << shift);
          sel_above = above;
        } else if (tid == 0 && above + bmass[0] < p_fix) {
          if (shift == 24) sel_found = 0;
          sel_key = pre;  // the crossing is in no deeper bucket either
          sel_above = above;
        }
      }
      __syncthreads();
      if (!sel_found) break;
    }
    if (sel_found) {
      const float K = __uint_as_float(sel_key);
      const float above = (float)((double)sel_above / kFix);
      uint32_t ties_loc = 0;
      each([&](int t, int e) {
        const float pv = P(t, e);
        ties_loc += (pv > 0.0f && X(t, e) > kMasked && pv == K) ? 1u : 0u;
      });
      const uint32_t ties = block_count(ties_loc, s);
      // tied tokens the cumulative sum takes before reaching p (at least one)
      uint32_t need = 0;
      float cum = above;
      while (need < ties && cum < sp.top_p) {
        cum += K;
        ++need;
      }
      // tie ranks in index order: a prefix over threads per tile, carried
      // across tiles
      uint32_t carry = 0;
      for (int t = 0; t < ntiles; ++t) {
        uint32_t mine = 0;
        float pv[kE];
#pragma unroll
        for (int e = 0; e < kE; ++e) {
          pv[e] = valid(t, e) && X(t, e) > kMasked ? P(t, e) : 0.0f;
          mine += (pv[e] > 0.0f && pv[e] == K) ? 1u : 0u;
        }
        uint32_t rank = carry + block_exclusive_prefix(mine, s.u);
        carry += block_count(mine, s);
#pragma unroll
        for (int e = 0; e < kE; ++e) {
          if (!(pv[e] > 0.0f)) continue;
          bool keep = pv[e] > K;
          if (pv[e] == K) keep = rank++ < need;
          if (!keep) X(t, e) = kMasked;
        }
      }
      __syncthreads();
    }
  }

  // The filtered row goes back in place (the reference's &mut logits).
  if constexpr (LDS_ROW) each([&](int t, int e) { gx[idx(t, e)] = X(t, e); });

  // ---- final softmax and the draw (sample_from, sampling.rs:208-223): the
  // first index whose cumulative probability exceeds r; past the end, the
  // last index with a non-zero probability ----
  softmax_row();
  const float r = uniform[row];
  int64_t first = INT64_MAX, last_nz = -1;
  float carry = 0.f;  // cumulative probability before the tile
  for (int t = 0; t < ntiles; ++t) {
    if (first != INT64_MAX) break;  // uniform over the workgroup
    float mine = 0.f;
    float pv[kE];
#pragma unroll
    for (int e = 0; e < kE; ++e) {
      pv[e] = valid(t, e) ? P(t, e) : 0.0f;
      mine += pv[e];
    }
    float cum = carry + block_exclusive_prefix(mine, s.f);
    int64_t hit = INT64_MAX;
#pragma unroll
    for (int e = 0; e < kE; ++e) {
      if (!valid(t, e)) continue;
      cum += pv[e];
      if (hit == INT64_MAX && r < cum) hit = idx(t, e);
      if (pv[e] > 0.0f) last_nz = idx(t, e);
    }
    first = block_min_i64(hit, s);  // cumulative sums only grow: the first tile with a hit
    carry += block_sum(mine, s);
  }
  if (first == INT64_MAX) {
    const int64_t last = block_max_i64(last_nz, s);
    if (tid == 0) out[row] = (int32_t)(last >= 0 ? last : vocab - 1);
  } else if (tid == 0) {
    out[row] = (int32_t)first;
  }
}

hipError_t launch_sample(hipStream_t st, float* logits, int64_t rows, int64_t vocab,
                         const SampleParams* params, const int64_t* prev_off,
                         const uint32_t* prev_tok, const float* uniform, float* probs_ws,
                         int32_t* out) {
  if (rows == 0) return hipSuccess;
  if (vocab <= 0 || vocab > kSampleMaxVocab || rows > INT32_MAX) return hipErrorInvalidValue;
  if (vocab <= kLdsRow)
    hipLaunchKernelGGL(sample_kernel<true>, dim3((unsigned)rows), dim3(kT), 0, st, logits, vocab,
                       params, prev_off, prev_tok, uniform, probs_ws, out);
  else
    hipLaunchKernelGGL(sample_kernel<false>, dim3((unsigned)rows), dim3(kT), 0, st, logits,
                       vocab, params, prev_off, prev_tok, uniform, probs_ws, out);
  return hipGetLastError();
}

}  // namespace orion

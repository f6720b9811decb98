// Paged grouped-query decode attention for gfx950.
//
// Computes the reference's `paged_attention` (crates/orion-models/src/
// attention.rs:219-295) for many independent query rows at once: row r, query
// head h attends positions 0..=pos[r] of its sequence through the block table,
// kv_head = h / (Hq / Hkv), scores (q . k) * (1/sqrt(d)), softmax, sum w * v.
//
// Design (bandwidth-bound; the KV cache is read exactly once):
//   * One wave per (row, kv head, context split).  The wave owns all G = Hq/Hkv
//     query heads of the GQA group, so each K/V row is read from HBM once for
//     the whole group.
//   * Split-K over the context in partitions of `partition` tokens; each split
//     keeps an online-softmax state (max, sum, unnormalised output) and a small
//     combine kernel merges the splits.  Rows that fit in one split are
//     finished in place.
//   * KV layout is the reference arena [layer][block][k|v][slot][head][dim]
//     (attention.rs:11-22).  A token's head vector is D contiguous elements, so
//     CH = D*sizeof(T)/16 lanes cover it with one 16-byte load each and a wave
//     load covers TPW = 64/CH tokens: fully coalesced 1 KiB per instruction.
//   * The block table slice of a split (<= 64 entries) is held one entry per
//     lane and fetched with a lane shuffle, so no dependent global load sits
//     between a token index and its KV address.
//   * Each group of CH lanes (one token per load) keeps its own running max,
//     so the online softmax needs no cross-lane traffic inside the loop; the
//     TPW partial states are merged once at the end of the split.
#include "common.hpp"
#include "kernels.hpp"

namespace orion {

template <typename T>
struct KvVec;

template <>
struct KvVec<float> {
  static constexpr int EPL = 4;
  __device__ static inline void load(const float* p, bool valid, float (&out)[4]) {
    float4 v = valid ? *reinterpret_cast<const float4*>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  }
};

template <>
struct KvVec<uint16_t> {
  static constexpr int EPL = 8;
  __device__ static inline void load(const uint16_t* p, bool valid, float (&out)[8]) {
    uint4 v = valid ? *reinterpret_cast<const uint4*>(p) : make_uint4(0u, 0u, 0u, 0u);
    out[0] = bf16lo(v.x);
    out[1] = bf16hi(v.x);
    out[2] = bf16lo(v.y);
    out[3] = bf16hi(v.y);
    out[4] = bf16lo(v.z);
    out[5] = bf16hi(v.z);
    out[6] = bf16lo(v.w);
    out[7] = bf16hi(v.w);
  }
};

template <typename T, int D, int G>
__global__ void __launch_bounds__(256)
    paged_decode_kernel(const T* __restrict__ kv_layer, int64_t blk_stride, int64_t v_off,
                        int64_t slot_stride, int bs_log2, int num_kv_heads, int num_q_heads,
                        int num_items, const float* __restrict__ q,
                        const uint32_t* __restrict__ positions, const int32_t* __restrict__ row_seq,
                        const int64_t* __restrict__ bt_off, const uint32_t* __restrict__ bt_ids,
                        int partition, int max_splits, float scale, float* __restrict__ out,
                        float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  constexpr int EPL = KvVec<T>::EPL;
  constexpr int CH = D / EPL;   // lanes per token vector
  constexpr int TPW = 64 / CH;  // tokens per wave load
  constexpr int R = 16 / TPW;   // loads per lane per 16-token step
  static_assert(TPW >= 1 && TPW <= 16 && R * TPW == 16, "unsupported head_dim/dtype");

  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= num_items) return;
  const int row = item / num_kv_heads;
  const int kvh = item - row * num_kv_heads;
  const int split = blockIdx.y;
  const int len = (int)positions[row] + 1;
  const int start = split * partition;
  if (start >= len) return;
  const int end = min(len, start + partition);
  const int nsplit = (len + partition - 1) / partition;

  const int t = lane / CH;  // token slot within a wave load
  const int c = lane % CH;  // chunk of the head vector
  const int bs_mask = (1 << bs_log2) - 1;

  // Query chunk for all G heads of the group.
  float qr[G][EPL];
  {
    const float* qp = q + ((int64_t)row * num_q_heads + (int64_t)kvh * G) * D + c * EPL;
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EPL; e += 4) {
        float4 v = *reinterpret_cast<const float4*>(qp + g * D + e);
        qr[g][e] = v.x;
        qr[g][e + 1] = v.y;
        qr[g][e + 2] = v.z;
        qr[g][e + 3] = v.w;
      }
    }
  }

  // Block-table slice of this split, one entry per lane.
  const int seq = row_seq[row];
  const uint32_t* tbl = bt_ids + bt_off[seq];
  const int first_blk = start >> bs_log2;
  const int nblk = ((end - 1) >> bs_log2) - first_blk + 1;
  const int my_blk = lane < nblk ? (int)tbl[first_blk + lane] : 0;

  const T* kbase = kv_layer + (int64_t)kvh * D + c * EPL;

  float m[G], l[G], o[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[g][e] = 0.f;
  }

  for (int base = start; base < end; base += 16) {
    float kf[R][EPL], vf[R][EPL];
    bool valid[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = base + r * TPW + t;
      valid[r] = j < end;
      const int bi = valid[r] ? (j >> bs_log2) - first_blk : 0;
      const int blk = __shfl(my_blk, bi);
      const int64_t off = (int64_t)blk * blk_stride + (int64_t)(j & bs_mask) * slot_stride;
      KvVec<T>::load(kbase + off, valid[r], kf[r]);
      KvVec<T>::load(kbase + off + v_off, valid[r], vf[r]);
    }
    // Partial dot products over this lane's chunk, then sum over the CH lanes.
    float s[R][G];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc += qr[g][e] * kf[r][e];
        s[r][g] = group_sum<CH>(acc);
      }
    }
    // Online softmax per head over this token group's R tokens.
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        s[r][g] = valid[r] ? s[r][g] * scale : -INFINITY;
        mx = fmaxf(mx, s[r][g]);
      }
      const float m_new = fmaxf(m[g], mx);
      if (m_new == -INFINITY) continue;  // no token yet in this group
      const float alpha = __expf(m[g] - m_new);
      m[g] = m_new;
      float p[R];
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        p[r] = __expf(s[r][g] - m_new);
        psum += p[r];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        float acc = o[g][e] * alpha;
#pragma unroll
        for (int r = 0; r < R; ++r) acc += p[r] * vf[r][e];
        o[g][e] = acc;
      }
    }
  }

  // Merge the TPW token groups (lanes c, c+CH, c+2CH, ...).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mg = m[g];
#pragma unroll
    for (int off = CH; off < 64; off <<= 1) mg = fmaxf(mg, __shfl_xor(mg, off));
    const float f = (m[g] == -INFINITY) ? 0.f : __expf(m[g] - mg);
    float lg = l[g] * f;
#pragma unroll
    for (int off = CH; off < 64; off <<= 1) lg += __shfl_xor(lg, off);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float v = o[g][e] * f;
#pragma unroll
      for (int off = CH; off < 64; off <<= 1) v += __shfl_xor(v, off);
      o[g][e] = v;
    }
    m[g] = mg;
    l[g] = lg;
  }

  if (t != 0) return;
  const int64_t head0 = (int64_t)row * num_q_heads + (int64_t)kvh * G;
  if (nsplit == 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float inv = 1.f / l[g];
      float* op = out + (head0 + g) * D + c * EPL;
#pragma unroll
      for (int e = 0; e < EPL; e += 4)
        *reinterpret_cast<float4*>(op + e) =
            make_float4(o[g][e] * inv, o[g][e + 1] * inv, o[g][e + 2] * inv, o[g][e + 3] * inv);
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t slot = (head0 + g) * max_splits + split;
      float* op = ws_o + slot * D + c * EPL;
#pragma unroll
      for (int e = 0; e < EPL; e += 4)
        *reinterpret_cast<float4*>(op + e) =
            make_float4(o[g][e], o[g][e + 1], o[g][e + 2], o[g][e + 3]);
      if (c == 0) *reinterpret_cast<float2*>(ws_ml + slot * 2) = make_float2(m[g], l[g]);
    }
  }
}

// Merges the per-split states of rows whose context spans several splits.
// One wave per (row, query head).
template <int D>
__global__ void __launch_bounds__(256)
    paged_decode_combine_kernel(int num_rows, int num_q_heads, const uint32_t* __restrict__ positions,
                                int partition, int max_splits, const float* __restrict__ ws_o,
                                const float* __restrict__ ws_ml, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)num_rows * num_q_heads) return;
  const int row = (int)(item / num_q_heads);
  const int len = (int)positions[row] + 1;
  const int nsplit = (len + partition - 1) / partition;
  if (nsplit <= 1) return;
  const float* ml = ws_ml + item * max_splits * 2;
  float mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, ml[2 * s]);
  float lsum = 0.f;
  constexpr int PER = D / 64;
  float acc[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) acc[i] = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float w = __expf(ml[2 * s] - mx);
    lsum += w * ml[2 * s + 1];
    const float* op = ws_o + (item * max_splits + s) * D;
#pragma unroll
    for (int i = 0; i < PER; ++i) acc[i] += w * op[lane + 64 * i];
  }
  const float inv = 1.f / lsum;
#pragma unroll
  for (int i = 0; i < PER; ++i) out[item * D + lane + 64 * i] = acc[i] * inv;
}

template <typename T, int D>
static hipError_t launch_decode_g(int G, dim3 grid, hipStream_t st, const T* kv, int64_t bstr,
                                  int64_t voff, int64_t sstr, int bsl, int hkv, int hq, int items,
                                  const float* q, const uint32_t* pos, const int32_t* rs,
                                  const int64_t* bo, const uint32_t* bi, int P, int ms, float scale,
                                  float* out, float* wo, float* wml) {
#define ORION_DECODE_CASE(GG)                                                                   \
  case GG:                                                                                      \
    hipLaunchKernelGGL((paged_decode_kernel<T, D, GG>), grid, dim3(256), 0, st, kv, bstr, voff, \
                       sstr, bsl, hkv, hq, items, q, pos, rs, bo, bi, P, ms, scale, out, wo,    \
                       wml);                                                                    \
    break;
  switch (G) {
    ORION_DECODE_CASE(1)
    ORION_DECODE_CASE(2)
    ORION_DECODE_CASE(3)
    ORION_DECODE_CASE(4)
    ORION_DECODE_CASE(5)
    ORION_DECODE_CASE(6)
    ORION_DECODE_CASE(7)
    ORION_DECODE_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef ORION_DECODE_CASE
  return hipGetLastError();
}

int decode_partition_for(int64_t num_items, int64_t max_len, int64_t block_size) {
  // Enough (item, split) waves to cover the chip several times over, with
  // partitions no shorter than 64 tokens.  A partition is a multiple of 16
  // tokens and of the block size, and spans at most 64 blocks.
  int P = 512;
  while (P > 64 && num_items * ((max_len + P - 1) / P) < 4096) P >>= 1;
  if (P < block_size) P = (int)block_size;
  if (P / block_size > 64) P = (int)(64 * block_size);
  return P;
}

hipError_t launch_paged_decode(hipStream_t st, const KvGeom& kv, const void* arena, int64_t layer,
                               const float* q, int64_t rows, int64_t hq,
                               const uint32_t* positions, const int32_t* row_seq,
                               const int64_t* bt_off, const uint32_t* bt_ids, int64_t max_position,
                               float* out, float* ws, size_t ws_bytes) {
  if (rows == 0) return hipSuccess;
  const int64_t hkv = kv.num_kv_heads, D = kv.head_dim;
  const int G = (int)(hq / hkv);
  const int64_t items = rows * hkv;
  const int P = decode_partition_for(items, max_position + 1, kv.block_size);
  const int max_splits = (int)((max_position + 1 + P - 1) / P);
  const size_t need = decode_workspace_bytes(rows, hq, D, max_splits);
  if (max_splits > 1 && need > ws_bytes) return hipErrorOutOfMemory;
  float* ws_o = ws;
  float* ws_ml = ws ? ws + rows * hq * max_splits * D : nullptr;
  int bs_log2 = 0;
  while ((1 << bs_log2) < kv.block_size) ++bs_log2;
  const int64_t slot_stride = hkv * D;
  const int64_t v_off = kv.block_size * slot_stride;
  const int64_t blk_stride = 2 * v_off;
  const int64_t layer_elems = kv.num_blocks * blk_stride;
  const float scale = 1.0f / sqrtf((float)D);
  dim3 grid((unsigned)((items + 3) / 4), (unsigned)max_splits);
  hipError_t e;
  if (kv.dtype_bf16) {
    const uint16_t* base = static_cast<const uint16_t*>(arena) + layer * layer_elems;
    if (D == 128)
      e = launch_decode_g<uint16_t, 128>(G, grid, st, base, blk_stride, v_off, slot_stride,
                                         bs_log2, (int)hkv, (int)hq, (int)items, q, positions,
                                         row_seq, bt_off, bt_ids, P, max_splits, scale, out, ws_o,
                                         ws_ml);
    else if (D == 64)
      e = launch_decode_g<uint16_t, 64>(G, grid, st, base, blk_stride, v_off, slot_stride,
                                        bs_log2, (int)hkv, (int)hq, (int)items, q, positions,
                                        row_seq, bt_off, bt_ids, P, max_splits, scale, out, ws_o,
                                        ws_ml);
    else
      return hipErrorInvalidValue;
  } else {
    const float* base = static_cast<const float*>(arena) + layer * layer_elems;
    if (D == 128)
      e = launch_decode_g<float, 128>(G, grid, st, base, blk_stride, v_off, slot_stride, bs_log2,
                                      (int)hkv, (int)hq, (int)items, q, positions, row_seq,
                                      bt_off, bt_ids, P, max_splits, scale, out, ws_o, ws_ml);
    else if (D == 64)
      e = launch_decode_g<float, 64>(G, grid, st, base, blk_stride, v_off, slot_stride, bs_log2,
                                     (int)hkv, (int)hq, (int)items, q, positions, row_seq, bt_off,
                                     bt_ids, P, max_splits, scale, out, ws_o, ws_ml);
    else
      return hipErrorInvalidValue;
  }
  if (e != hipSuccess || max_splits == 1) return e;
  dim3 cgrid((unsigned)((rows * hq + 3) / 4));
  if (D == 128)
    hipLaunchKernelGGL(paged_decode_combine_kernel<128>, cgrid, dim3(256), 0, st, (int)rows,
                       (int)hq, positions, P, max_splits, ws_o, ws_ml, out);
  else
    hipLaunchKernelGGL(paged_decode_combine_kernel<64>, cgrid, dim3(256), 0, st, (int)rows,
                       (int)hq, positions, P, max_splits, ws_o, ws_ml, out);
  return hipGetLastError();
}

size_t decode_workspace_bytes(int64_t rows, int64_t hq, int64_t D, int64_t max_splits) {
  if (max_splits <= 1) return 0;
  return (size_t)(rows * hq * max_splits) * (size_t)(D + 2) * sizeof(float);
}

int64_t decode_max_splits(int64_t rows, int64_t hkv, int64_t max_position, int64_t block_size) {
  const int P = decode_partition_for(rows * hkv, max_position + 1, block_size);
  return (max_position + 1 + P - 1) / P;
}

}  // namespace orion

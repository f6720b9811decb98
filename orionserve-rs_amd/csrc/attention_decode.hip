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

#include <algorithm>
#include <type_traits>
#include <vector>

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
__device__ __forceinline__ void decode_wave_valu(
    const T* __restrict__ kv_layer, int64_t blk_stride, int64_t v_off, int64_t slot_stride,
    int64_t head_stride, int bs_log2, int num_q_heads, const float* __restrict__ q,
    const uint32_t* __restrict__ tbl,
    int max_splits, float scale, float* __restrict__ out, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, int row, int kvh, int start, int end, int split, int nsplit) {
  constexpr int EPL = KvVec<T>::EPL;
  constexpr int CH = D / EPL;   // lanes per token vector
  constexpr int TPW = 64 / CH;  // tokens per wave load
  constexpr int R = 16 / TPW;   // loads per lane per 16-token step
  static_assert(TPW >= 1 && TPW <= 16 && R * TPW == 16, "unsupported head_dim/dtype");

  const int lane = threadIdx.x & 63;

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

  // Block-table slice of this chunk (tbl points at its first entry), one
  // entry per lane.
  const int first_blk = start >> bs_log2;
  const int nblk = ((end - 1) >> bs_log2) - first_blk + 1;
  const int my_blk = lane < nblk ? (int)tbl[lane] : 0;

  const T* kbase = kv_layer + (int64_t)kvh * head_stride + c * EPL;

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

// One wave per work item (row, KV head, context chunk), four items per
// workgroup; the work list is ordered longest chunk first.
template <typename T, int D, int G>
__global__ void __launch_bounds__(256)
    paged_decode_kernel(const T* __restrict__ kv_layer, int64_t blk_stride, int64_t v_off,
                        int64_t slot_stride, int64_t head_stride, int bs_log2, int num_kv_heads,
                        int num_q_heads,
                        const DecodeWork* __restrict__ work, int num_work, const float* __restrict__ q,
                        const uint32_t* __restrict__ positions, const int32_t* __restrict__ row_seq,
                        const int64_t* __restrict__ bt_off, const uint32_t* __restrict__ bt_ids,
                        int max_splits, float scale, float* __restrict__ out,
                        float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= num_work) return;
  const DecodeWork wk = work[w];
  const int row = wk.item / num_kv_heads, kvh = wk.item - row * num_kv_heads;
  decode_wave_valu<T, D, G>(kv_layer, blk_stride, v_off, slot_stride, head_stride, bs_log2,
                            num_q_heads, q,
                            bt_ids + wk.tbl_off, max_splits, scale, out, ws_o, ws_ml, row, kvh,
                            wk.start, wk.end, wk.split, wk.nsplit);
}

// Second-generation bf16 decode wave: both contractions on MFMA.
//
//   S = K . Q^T   (v_mfma_f32_16x16x32_bf16, A = K tile straight from HBM,
//                  B = query group hi/lo; out lane l: token 4*(l/16)+i, head l%16)
//   O^T = V^T . P^T (v_mfma_f32_16x16x16bf16_1k, K = the step's 16 tokens)
//
// The score layout of the first product is exactly the B-operand layout of
// the second (lane l: head l%16, tokens 4*(l/16)..+4), so the softmax weights
// never leave registers; they are split into hi + lo bf16 terms.  V arrives
// row-major ([token][dim], one coalesced 16-byte load per lane), is written to
// a padded per-wave LDS tile, and read back column-wise with ds_read_tr16_b64,
// which hands lane i of each 16-lane group element (i%4) of the 8-byte chunk
// addressed by lane 4r + i/4 as its r-th value.  Every per-head quantity (max,
// rescale, sum, output) lives in the lanes l with l%16 = head.
// K/V loads.  STREAM: every block is read once, and nontemporal (streaming)
// loads keep it from displacing the tables, queries and partial outputs in the
// caches (measured: 5.17 -> 5.62 TB/s on config 2).  Blocks shared by several
// rows (a common prefix) keep ordinary loads so the repeats can hit in L2/MALL.
template <bool STREAM>
__device__ __forceinline__ uint4 kv_load16(const uint16_t* p) {
  if constexpr (STREAM) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return uint4{v.x, v.y, v.z, v.w};
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}

// PR > 1: a packed item -- the query columns hold the G heads of each of up
// to PR rows (prow[0 .. PR), -1 unused) that share this piece's blocks;
// column c is head c % G of row prow[c / G].
template <int D, int G, bool STREAM, bool BIG_BLOCKS, int PR = 1>
__device__ __forceinline__ void decode_wave_mfma2(
    const uint16_t* __restrict__ kv_layer, uint32_t blk_stride, uint32_t v_off,
    uint32_t slot_stride, uint32_t head_stride, int bs_log2, int num_q_heads, const float* __restrict__ q,
    const uint32_t* __restrict__ tbl, int blk0, int max_splits, float scale,
    float* __restrict__ out, float* __restrict__ ws_o, float* __restrict__ ws_ml, uint16_t* VL,
    uint16_t* QL, uint16_t* KL, int row, int kvh,
    int start, int end, int split, int nsplit, const int32_t* __restrict__ prow = nullptr) {
  constexpr int QC = G * PR;      // query columns in use
  constexpr int KCH = D / 32;     // K . Q^T MFMA k-steps
  constexpr int DT = D / 16;      // output dim tiles of the P.V MFMA
  constexpr int CH = D / 8;       // lanes per V row (16 bytes each)
  constexpr int TPW = 64 / CH;    // V rows per wave load
  constexpr int RV = 16 / TPW;    // V loads per lane per step
  constexpr int VROW = D + 8;     // padded LDS row, in bf16 elements
  static_assert(QC <= 16 && TPW <= 16 && (16 % TPW) == 0, "unsupported shape");

  const int lane = threadIdx.x & 63;
  const int bs_mask = (1 << bs_log2) - 1;
  const int l16 = lane & 15;  // token (K load) / head (scores, output)
  const int grp = lane >> 4;  // 16-lane group

  // The query loads go out first (they are the first data the item needs),
  // then the table slice; the first K/V step is issued before either is
  // waited on (its block id travels in the work record).
  constexpr int KCH_ = D / 32;
  const int kd_ = grp * 8;
  float4 qr[2 * KCH_];
  // this lane's query column: head qhead of row qrow (columns past QC repeat
  // column QC - 1; their scores are never used)
  int qrow = row, qhead = min(l16, G - 1);
  if constexpr (PR > 1) {
    const int col = min(l16, QC - 1);
    const int pr = prow[col / G];
    qrow = pr >= 0 ? pr : prow[0];
    qhead = col % G;
  }
  {
    const float* qp = q + ((int64_t)qrow * num_q_heads + (int64_t)kvh * G + qhead) * D + kd_;
#pragma unroll
    for (int j = 0; j < KCH_; ++j) {
      qr[2 * j] = *reinterpret_cast<const float4*>(qp + 32 * j);
      qr[2 * j + 1] = *reinterpret_cast<const float4*>(qp + 32 * j + 4);
    }
  }
  const int first_blk = start >> bs_log2;
  const int nblk = ((end - 1) >> bs_log2) - first_blk + 1;
  const int my_blk = lane < nblk ? (int)tbl[lane] : 0;

  const uint16_t* base_k = kv_layer + (uint32_t)kvh * head_stride;
  const int kd = grp * 8;          // K dims chunk
  const int vt = lane / CH;        // V row within a wave load
  const int vc = lane % CH;        // V 16-byte chunk

  // blk_hint >= 0 supplies the step's block id directly (the first step uses
  // the plan's copy, so its loads need not wait for the table slice).
  auto issue = [&](uint4 (&ks)[RV], uint4 (&vs)[RV], int b, int blk_hint) {
    if constexpr (BIG_BLOCKS) {
      const int blk = blk_hint >= 0
                          ? blk_hint
                          : __builtin_amdgcn_readlane(my_blk, (b >> bs_log2) - first_blk);
      // 64-bit block offset (a layer may exceed 2^32 elements); uniform
      const uint16_t* bb = base_k + (size_t)(uint32_t)blk * blk_stride;
#pragma unroll
      for (int r = 0; r < RV; ++r) {
        const int jv = min(b + r * TPW + vt, end - 1);
        const uint16_t* rp = bb + (uint32_t)(jv & bs_mask) * slot_stride + vc * 8;
        ks[r] = kv_load16<STREAM>(rp);
        vs[r] = kv_load16<STREAM>(rp + v_off);
      }
    } else {
#pragma unroll
      for (int r = 0; r < RV; ++r) {
        const int jv = min(b + r * TPW + vt, end - 1);
        const int bv = __shfl(my_blk, (jv >> bs_log2) - first_blk);
        const uint16_t* rp = base_k + (size_t)(uint32_t)bv * blk_stride +
                             (uint32_t)(jv & bs_mask) * slot_stride + vc * 8;
        ks[r] = kv_load16<STREAM>(rp);
        vs[r] = kv_load16<STREAM>(rp + v_off);
      }
    }
  };

  // Register sets of the K/V pipeline; the first step is issued now.
  uint4 ka[RV], va_[RV], kb[RV], vb[RV];
  const int nsteps = (end - start + 15) >> 4;
  auto step_base = [&](int i) { return min(start + 16 * i, end - 1) & ~15; };
  issue(ka, va_, step_base(0), BIG_BLOCKS ? blk0 : -1);

  // ---- query group as the B operand of S = K . Q^T (hi/lo bf16) ----
  // Kept in a small per-wave LDS tile [hi|lo][G][D + 8] rather than in 32
  // VGPRs.  B-operand column l16 >= G reads head l16 % G: those columns of S
  // are never used, and duplicating a real head keeps them finite.
  constexpr int QROW = D + 8;
  const int qh = l16 % QC;
  {
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      uint4 hv, lv;
      split2_trunc(qr[2 * j].x, qr[2 * j].y, hv.x, lv.x);
      split2_trunc(qr[2 * j].z, qr[2 * j].w, hv.y, lv.y);
      split2_trunc(qr[2 * j + 1].x, qr[2 * j + 1].y, hv.z, lv.z);
      split2_trunc(qr[2 * j + 1].z, qr[2 * j + 1].w, hv.w, lv.w);
      if (l16 < QC) {
        *reinterpret_cast<uint4*>(&QL[l16 * QROW + 32 * j + kd]) = hv;
        *reinterpret_cast<uint4*>(&QL[(QC + l16) * QROW + 32 * j + kd]) = lv;
      }
    }
  }
  wave_lds_sync();
  auto qb = [&](int j, int lo) -> bf16x8 {
    uint4 v;
    __builtin_memcpy(&v, (const void*)&QL[(lo * QC + qh) * QROW + 32 * j + kd], 16);
    return __builtin_bit_cast(bf16x8, v);
  };

  float m = -INFINITY, lsum = 0.f;  // for head l16 (replicated over the groups)
  f32x4 o[DT];                      // O^T tile dt: dims 16dt + 4*grp + i, head l16
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // LDS addresses: V row-major write (row vt + TPW*r, chunk vc) and the
  // transposed read (lane 4r + q of a group addresses row 4*grp + r, dims
  // 4q .. 4q+3 of the tile).
  const uint32_t vl_base = (uint32_t)(uintptr_t)VL;
  // K tile [16 tokens][CH units of 16 bytes]; unit u of token t sits at
  // t*CH + (u ^ kswz(t)), which keeps both the row writes (a wave writes TPW
  // whole rows) and the fragment reads (16 tokens x one unit per group) free
  // of LDS bank conflicts.
  const uint32_t kl_base = (uint32_t)(uintptr_t)KL;
  auto kswz = [](int t) { return D == 128 ? (t & 15) : ((t >> 1) & (CH - 1)); };
  const uint32_t w_off = (uint32_t)(vt * VROW + vc * 8) * 2;
  const uint32_t r_off = (uint32_t)((4 * grp + (l16 >> 2)) * VROW + 4 * (l16 & 3)) * 2;
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;

  // Softmax reference: m is a per-head value shared by the four lane groups.
  // Weights are exp(s - m); m is raised (with an exact cross-group max and a
  // rescale) only when some score exceeds it by more than kLazy, so weights
  // stay <= e^kLazy and the cross-lane exchange is rare after the first step.
  constexpr float kLazy = 8.0f;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) u32x4 lds_u4;
  auto compute = [&](const uint4 (&ks)[RV], const uint4 (&vs)[RV], int b, int buf) {
    // Stage V (row-major, padded rows) and K (swizzled 16-byte units) into
    // LDS.  One buffer per wave: its LDS operations execute in order, and the
    // fence at the end of the step keeps the compiler from moving these
    // writes above the previous reads.
    (void)buf;
    const uint32_t wb = vl_base + w_off;
#pragma unroll
    for (int r = 0; r < RV; ++r) {
      *(lds_u4*)(uintptr_t)(wb + r * TPW * VROW * 2) = __builtin_bit_cast(u32x4, vs[r]);
      const int tt = r * TPW + vt;
      *(lds_u4*)(uintptr_t)(kl_base + (uint32_t)(tt * CH + (vc ^ kswz(tt))) * 16) =
          __builtin_bit_cast(u32x4, ks[r]);
    }
    wave_lds_sync();
    // S = K . Q^T, the A fragments (token l16, dims 32c + 8grp .. +8) read
    // back from the K tile
    f32x4 sh = {0.f, 0.f, 0.f, 0.f}, sl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const bf16x8 ka = __builtin_bit_cast(
          bf16x8, *(const lds_u4*)(uintptr_t)(kl_base +
                                              (uint32_t)(l16 * CH + ((4 * c + grp) ^ kswz(l16))) * 16));
      sh = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb(c, 0), sh, 0, 0, 0);
      sl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb(c, 1), sl, 0, 0, 0);
    }
    float s[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = (b + 4 * grp + i < end) ? (sh[i] + sl[i]) * scale : -INFINITY;
      mx = fmaxf(mx, s[i]);
    }
    if (__builtin_amdgcn_ballot_w64(mx > m + kLazy) != 0) {
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m, mx);
      const float alpha = __expf(m - m_new);
      m = m_new;
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t) o[t] *= alpha;
    }
    float pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pv[i] = __expf(s[i] - m);
    lsum += (pv[0] + pv[1]) + (pv[2] + pv[3]);
    uint2 hi2, lo2;
    split2_trunc(pv[0], pv[1], hi2.x, lo2.x);
    split2_trunc(pv[2], pv[3], hi2.y, lo2.y);
    const v4s pb_hi = __builtin_bit_cast(v4s, hi2);
    const v4s pb_lo = __builtin_bit_cast(v4s, lo2);
    // O^T += V^T . P^T
    const uint32_t rb = vl_base + r_off;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const v4s va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(rb + t * 32));
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb_hi, o[t], 0, 0, 0);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb_lo, o[t], 0, 0, 0);
    }
    wave_lds_sync();
  };

  // Two register sets in ping-pong: step i computes on one set while the
  // next step's loads land in the other.  Loads are unconditional (token
  // indices clamped into the chunk), so the compiler's wait counts are exact,
  // and a full pair of steps is one basic block, so one step's softmax and
  // P.V overlap the next step's Q.K^T.  LDS buffer parity = step parity.
  int i = 0;
  for (; i + 2 <= nsteps; i += 2) {
    issue(kb, vb, step_base(i + 1), -1);
    compute(ka, va_, start + 16 * i, 0);
    issue(ka, va_, step_base(i + 2), -1);
    compute(kb, vb, start + 16 * (i + 1), 1);
  }
  if (i < nsteps) compute(ka, va_, start + 16 * i, 0);

  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  if (l16 >= QC) return;
  int orow = row, ohead = l16;
  if constexpr (PR > 1) {
    orow = prow[l16 / G];
    ohead = l16 % G;
    if (orow < 0) return;
  }
  const int64_t hidx = (int64_t)orow * num_q_heads + (int64_t)kvh * G + ohead;
  if (nsplit == 1) {
    const float inv = 1.f / lsum;
    float* op = out + hidx * D + 4 * grp;
#pragma unroll
    for (int t = 0; t < DT; ++t)
      *reinterpret_cast<float4*>(op + 16 * t) =
          make_float4(o[t][0] * inv, o[t][1] * inv, o[t][2] * inv, o[t][3] * inv);
  } else {
    const int64_t slot = hidx * max_splits + split;
    float* op = ws_o + slot * D + 4 * grp;
#pragma unroll
    for (int t = 0; t < DT; ++t)
      *reinterpret_cast<float4*>(op + 16 * t) = make_float4(o[t][0], o[t][1], o[t][2], o[t][3]);
    if (grp == 0) *reinterpret_cast<float2*>(ws_ml + slot * 2) = make_float2(m, lsum);
  }
}

// KV: 0 cached K/V loads, 1 streaming, 2 per item (streaming unless the item
// reads a shared block, DecodeWork::shared).  Three waves per SIMD (three
// workgroups per CU); groups above 8 at head_dim 128 hold too much query
// tile in LDS for three, and take two.
// PR > 1: the plan holds packed prefix items (DecodeWork::shared == 2), PR
// rows each, whose rows are pack_rows[pack * PR ..]; they take cached loads.
template <int D, int G, int KV, bool BIG_BLOCKS, int PR = 1>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu((D == 128 && G * PR > 8) ? 2 : 3)))
    paged_decode_mfma2_kernel(const uint16_t* __restrict__ kv_layer, uint32_t blk_stride,
                              uint32_t v_off, uint32_t slot_stride,
                              uint32_t head_stride, int bs_log2, int num_kv_heads,
                              int num_q_heads, const DecodeWork* __restrict__ work, int num_work,
                              const float* __restrict__ q, const uint32_t* __restrict__ positions,
                              const int32_t* __restrict__ row_seq,
                              const int64_t* __restrict__ bt_off,
                              const uint32_t* __restrict__ bt_ids, int max_splits,
                              float scale, float* __restrict__ out, float* __restrict__ ws_o,
                              float* __restrict__ ws_ml, const int32_t* __restrict__ pack_rows) {
  __shared__ __attribute__((aligned(16))) uint16_t lds_v[4][16 * (D + 8)];
  __shared__ __attribute__((aligned(16))) uint16_t lds_q[4][2 * G * PR * (D + 8)];
  __shared__ __attribute__((aligned(16))) uint16_t lds_k[4][16 * D];
  const int wv = threadIdx.x >> 6;
  const int w = blockIdx.x * 4 + wv;
  if (w >= num_work) return;
  const DecodeWork wk = work[w];
  const int row = wk.item / num_kv_heads, kvh = wk.item - row * num_kv_heads;
  if constexpr (PR > 1) {
    if (__builtin_amdgcn_readfirstlane(wk.shared) == 2) {  // row = the pack index
      decode_wave_mfma2<D, G, false, BIG_BLOCKS, PR>(
          kv_layer, blk_stride, v_off, slot_stride, head_stride, bs_log2, num_q_heads, q,
          bt_ids + wk.tbl_off, wk.blk0, max_splits, scale, out, ws_o, ws_ml, lds_v[wv],
          lds_q[wv], lds_k[wv], -1, kvh, wk.start, wk.end, wk.split, wk.nsplit,
          pack_rows + (int64_t)row * PR);
      return;
    }
  }
  auto run = [&](auto stream_tag) {
    decode_wave_mfma2<D, G, decltype(stream_tag)::value, BIG_BLOCKS>(
        kv_layer, blk_stride, v_off, slot_stride, head_stride, bs_log2, num_q_heads, q,
        bt_ids + wk.tbl_off, wk.blk0, max_splits, scale, out, ws_o, ws_ml, lds_v[wv], lds_q[wv],
        lds_k[wv], row, kvh, wk.start, wk.end, wk.split, wk.nsplit);
  };
  if constexpr (KV == 2) {
    if (__builtin_amdgcn_readfirstlane(wk.shared) == 1)
      run(std::false_type{});
    else
      run(std::true_type{});
  } else {
    run(std::integral_constant<bool, KV == 1>{});
  }
}

// Merges the per-split states of rows whose context spans several splits.
// One wave per (row, query head).  Fast path (<= 64 splits): lane s holds
// split s's (max, sum), and the first MAXS splits' partial outputs are loaded
// before any reduction, so the merge costs one memory round trip.
template <int D>
__global__ void __launch_bounds__(256)
    paged_decode_combine_kernel(int num_rows, int num_q_heads,
                                const int32_t* __restrict__ row_nsplit,
                                const int32_t* __restrict__ row_list,
                                int max_splits, const float* __restrict__ ws_o,
                                const float* __restrict__ ws_ml, float* __restrict__ out) {
  constexpr int PER = D / 64;
  constexpr int MAXS = 16;
  const int lane = threadIdx.x & 63;
  const int64_t slot = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (slot >= (int64_t)num_rows * num_q_heads) return;
  // num_rows counts row_list entries when a list is given.
  const int li = (int)(slot / num_q_heads);
  const int row = row_list ? row_list[li] : li;
  const int64_t item = (int64_t)row * num_q_heads + (slot - (int64_t)li * num_q_heads);
  const int nsplit = row_nsplit[row];
  if (nsplit <= 1) return;
  const float* ml = ws_ml + item * max_splits * 2;
  const float* ob = ws_o + item * max_splits * D;
  float acc[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) acc[i] = 0.f;
  float lsum;
  if (nsplit <= 64) {
    const float2 e = lane < nsplit ? *reinterpret_cast<const float2*>(ml + 2 * lane)
                                   : make_float2(-INFINITY, 0.f);
    // Partial outputs in rounds of MAXS splits, every load of a round issued
    // before its first use (split indices clamped; the weight of a split past
    // the end is 0).
    float ov[MAXS][PER];
#pragma unroll
    for (int j = 0; j < MAXS; ++j)
#pragma unroll
      for (int i = 0; i < PER; ++i)
        ov[j][i] = ob[(int64_t)min(j, nsplit - 1) * D + lane + 64 * i];
    const float mx = wave_max(e.x);
    const float w = lane < nsplit ? __expf(e.x - mx) : 0.f;
    lsum = wave_sum(w * e.y);
    for (int base = 0; base < nsplit; base += MAXS) {
      if (base > 0) {
#pragma unroll
        for (int j = 0; j < MAXS; ++j)
#pragma unroll
          for (int i = 0; i < PER; ++i)
            ov[j][i] = ob[(int64_t)min(base + j, nsplit - 1) * D + lane + 64 * i];
      }
#pragma unroll
      for (int j = 0; j < MAXS; ++j) {
        const float wj = __shfl(w, min(base + j, 63));
        const float wk = base + j < nsplit ? wj : 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i) acc[i] += wk * ov[j][i];
      }
    }
  } else {
    float mx = -INFINITY;
    for (int s = lane; s < nsplit; s += 64) mx = fmaxf(mx, ml[2 * s]);
    mx = wave_max(mx);
    float ls = 0.f;
    for (int s = lane; s < nsplit; s += 64) ls += __expf(ml[2 * s] - mx) * ml[2 * s + 1];
    lsum = wave_sum(ls);
    for (int s = 0; s < nsplit; ++s) {
      const float wj = __expf(ml[2 * s] - mx);
#pragma unroll
      for (int i = 0; i < PER; ++i) acc[i] += wj * ob[(int64_t)s * D + lane + 64 * i];
    }
  }
  const float inv = 1.f / lsum;
#pragma unroll
  for (int i = 0; i < PER; ++i) out[item * D + lane + 64 * i] = acc[i] * inv;
}

// ---------------------------------------------------------------------------
// Any head_dim and GQA group (the shapes the kernels above do not cover)
// ---------------------------------------------------------------------------

// paged_attention (attention.rs:219-295) accepts any even head_dim and any
// grouping of query heads over KV heads.  This wave covers what the MFMA and
// per-dtype VALU waves do not: any even head_dim up to kMaxHeadDim, any group
// size.  One wave per work item (row, KV head, chunk).  Lane l holds
// dimensions {128c + 2l, 128c + 2l + 1} of every vector, for c < NC (NC
// 128-dimension chunks, the smallest template width covering D); a 16-token
// step loads the 16 keys, reduces each score over the wave, and updates the
// online softmax (max, sum, output) of one query head.  The G query heads of
// the item run one after another over the same chunk, so heads after the
// first re-read its K/V from the caches.  Partial results use the same split
// layout as the other waves.
template <typename T>
__device__ inline float2 load_pair(const T* p, bool valid);
template <>
__device__ inline float2 load_pair<float>(const float* p, bool valid) {
  return valid ? *reinterpret_cast<const float2*>(p) : make_float2(0.f, 0.f);
}
template <>
__device__ inline float2 load_pair<uint16_t>(const uint16_t* p, bool valid) {
  const uint32_t v = valid ? *reinterpret_cast<const uint32_t*>(p) : 0u;
  return make_float2(bf16lo(v), bf16hi(v));
}

template <typename T, int NC>
__global__ void __launch_bounds__(256)
    paged_decode_any_kernel(const T* __restrict__ kv_layer, int64_t blk_stride, int64_t v_off,
                            int64_t slot_stride, int64_t head_stride, int bs_log2,
                            int num_kv_heads, int num_q_heads, int D,
                            const DecodeWork* __restrict__ work, int num_work,
                            const float* __restrict__ q, const uint32_t* __restrict__ bt_ids,
                            int max_splits, float scale, float* __restrict__ out,
                            float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= num_work) return;
  const DecodeWork wk = work[w];
  const int row = wk.item / num_kv_heads, kvh = wk.item - row * num_kv_heads;
  const int G = num_q_heads / num_kv_heads;
  const int lane = threadIdx.x & 63;
  bool has[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) has[c] = 128 * c + 2 * lane < D;
  const int start = wk.start, end = wk.end;
  const int split = wk.split;
  const int bs_mask = (1 << bs_log2) - 1;
  const int first_blk = start >> bs_log2;
  const int nblk = ((end - 1) >> bs_log2) - first_blk + 1;
  const uint32_t* tbl = bt_ids + wk.tbl_off;
  const int my_blk = lane < nblk ? (int)tbl[lane] : 0;
  const T* kbase = kv_layer + (int64_t)kvh * head_stride + 2 * lane;
  for (int g = 0; g < G; ++g) {
    const int64_t head = (int64_t)row * num_q_heads + (int64_t)kvh * G + g;
    const float* qp = q + head * D + 2 * lane;
    float2 qv[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c)
      qv[c] = has[c] ? *reinterpret_cast<const float2*>(qp + 128 * c) : make_float2(0.f, 0.f);
    float m = -INFINITY, l = 0.f;
    float o[2 * NC];
#pragma unroll
    for (int e = 0; e < 2 * NC; ++e) o[e] = 0.f;
    for (int base = start; base < end; base += 16) {
      float s[16];
      int64_t off[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = base + r;
        const bool valid = j < end;
        const int blk = __shfl(my_blk, valid ? (j >> bs_log2) - first_blk : 0);
        off[r] = (int64_t)blk * blk_stride + (int64_t)(j & bs_mask) * slot_stride;
        float part = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const float2 kk = load_pair<T>(kbase + off[r] + 128 * c, valid && has[c]);
          part += qv[c].x * kk.x + qv[c].y * kk.y;
        }
        const float dot = wave_sum(part);
        s[r] = valid ? dot * scale : -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
      const float m_new = fmaxf(m, mx);
      const float alpha = __expf(m - m_new);
      float psum = 0.f;
#pragma unroll
      for (int e = 0; e < 2 * NC; ++e) o[e] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool valid = base + r < end;
        const float p = valid ? __expf(s[r] - m_new) : 0.f;
        psum += p;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const float2 vv = load_pair<T>(kbase + off[r] + v_off + 128 * c, valid && has[c]);
          o[2 * c] += p * vv.x;
          o[2 * c + 1] += p * vv.y;
        }
      }
      l = l * alpha + psum;
      m = m_new;
    }
    if (wk.nsplit == 1) {
      const float inv = 1.f / l;
      float* op = out + head * D + 2 * lane;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (has[c])
          *reinterpret_cast<float2*>(op + 128 * c) = make_float2(o[2 * c] * inv, o[2 * c + 1] * inv);
    } else {
      const int64_t slot = head * max_splits + split;
      float* op = ws_o + slot * D + 2 * lane;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (has[c]) *reinterpret_cast<float2*>(op + 128 * c) = make_float2(o[2 * c], o[2 * c + 1]);
      if (lane == 0) *reinterpret_cast<float2*>(ws_ml + slot * 2) = make_float2(m, l);
    }
  }
}

// Merges the split partials for any even head_dim up to kMaxHeadDim: one wave
// per (row, query head), splits in order, lane l holding dimensions l + 64 i
// for i < NI.
template <int NI>
__global__ void __launch_bounds__(256)
    paged_decode_combine_any_kernel(int num_rows, int num_q_heads, int D,
                                    const int32_t* __restrict__ row_nsplit,
                                    const int32_t* __restrict__ row_list,
                                    int max_splits, const float* __restrict__ ws_o,
                                    const float* __restrict__ ws_ml, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t slot = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (slot >= (int64_t)num_rows * num_q_heads) return;
  const int li = (int)(slot / num_q_heads);
  const int row = row_list ? row_list[li] : li;
  const int64_t item = (int64_t)row * num_q_heads + (slot - (int64_t)li * num_q_heads);
  const int nsplit = row_nsplit[row];
  if (nsplit <= 1) return;
  const float* ml = ws_ml + item * max_splits * 2;
  const float* ob = ws_o + item * max_splits * D;
  float mx = -INFINITY;
  for (int s = lane; s < nsplit; s += 64) mx = fmaxf(mx, ml[2 * s]);
  mx = wave_max(mx);
  float ls = 0.f;
  for (int s = lane; s < nsplit; s += 64) ls += __expf(ml[2 * s] - mx) * ml[2 * s + 1];
  const float inv = 1.f / wave_sum(ls);
  float acc[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) acc[i] = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float wj = __expf(ml[2 * s] - mx);
#pragma unroll
    for (int i = 0; i < NI; ++i)
      if (lane + 64 * i < D) acc[i] += wj * ob[(int64_t)s * D + lane + 64 * i];
  }
#pragma unroll
  for (int i = 0; i < NI; ++i)
    if (lane + 64 * i < D) out[item * D + lane + 64 * i] = acc[i] * inv;
}

// ---------------------------------------------------------------------------
// Host side: launch (the work list comes from decode_plan.cpp)
// ---------------------------------------------------------------------------

template <typename T, int D>
static hipError_t launch_valu(int G, dim3 grid, hipStream_t st, const T* kv, const ArenaStrides& a,
                              int bsl, int hkv, int hq, const DecodeWork* work, int nwork,
                              const float* q, const uint32_t* pos, const int32_t* rs,
                              const int64_t* bo, const uint32_t* bi, int ms, float scale,
                              float* out, float* wo, float* wml) {
#define ORION_VALU_CASE(GG)                                                                   \
  case GG:                                                                                    \
    hipLaunchKernelGGL((paged_decode_kernel<T, D, GG>), grid, dim3(256), 0, st, kv, a.blk,    \
                       a.v_off, a.slot, a.head, bsl, hkv, hq, work, nwork, q, pos, rs, bo, bi, \
                       ms, scale, out, wo, wml);                                              \
    break;
  switch (G) {
    ORION_VALU_CASE(1)
    ORION_VALU_CASE(2)
    ORION_VALU_CASE(3)
    ORION_VALU_CASE(4)
    ORION_VALU_CASE(5)
    ORION_VALU_CASE(6)
    ORION_VALU_CASE(7)
    ORION_VALU_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef ORION_VALU_CASE
  return hipGetLastError();
}

template <int D, int KV, bool BIG>
static hipError_t launch_mfma2(int G, dim3 grid, hipStream_t st, const uint16_t* kv,
                               const ArenaStrides& a, int bsl, int hkv, int hq,
                               const DecodeWork* work, int nwork, const float* q,
                               const uint32_t* pos, const int32_t* rs, const int64_t* bo,
                               const uint32_t* bi, int ms, float scale, float* out,
                               float* wo, float* wml, const int32_t* pack_rows) {
#define ORION_MFMA2_CASE(GG)                                                                   \
  case GG:                                                                                     \
    if (pack_rows && 16 / GG >= 2)                                                             \
      hipLaunchKernelGGL((paged_decode_mfma2_kernel<D, GG, KV, BIG, (16 / GG >= 2 ? 16 / GG : 1)>), \
                         grid, dim3(256), 0, st, kv, (uint32_t)a.blk, (uint32_t)a.v_off,       \
                         (uint32_t)a.slot, (uint32_t)a.head, bsl, hkv, hq, work, nwork, q, pos, \
                         rs, bo, bi, ms, scale, out, wo, wml, pack_rows);                     \
    else                                                                                       \
      hipLaunchKernelGGL((paged_decode_mfma2_kernel<D, GG, KV, BIG>), grid, dim3(256), 0, st,   \
                         kv, (uint32_t)a.blk, (uint32_t)a.v_off, (uint32_t)a.slot,             \
                         (uint32_t)a.head, bsl, hkv, hq, work, nwork, q, pos, rs, bo, bi, ms,  \
                         scale, out, wo, wml, nullptr);                                        \
    break;
  switch (G) {
    ORION_MFMA2_CASE(1)
    ORION_MFMA2_CASE(2)
    ORION_MFMA2_CASE(3)
    ORION_MFMA2_CASE(4)
    ORION_MFMA2_CASE(5)
    ORION_MFMA2_CASE(6)
    ORION_MFMA2_CASE(7)
    ORION_MFMA2_CASE(8)
    ORION_MFMA2_CASE(9)
    ORION_MFMA2_CASE(10)
    ORION_MFMA2_CASE(11)
    ORION_MFMA2_CASE(12)
    ORION_MFMA2_CASE(13)
    ORION_MFMA2_CASE(14)
    ORION_MFMA2_CASE(15)
    ORION_MFMA2_CASE(16)
    default:
      return hipErrorInvalidValue;
  }
#undef ORION_MFMA2_CASE
  return hipGetLastError();
}

// Merges the split-K partials of every row (or of plan.rows) into out.
static hipError_t launch_combine(hipStream_t st, int64_t D, int64_t rows, int64_t hq,
                                 const DecodePlanDev& plan, int ms, const float* ws_o,
                                 const float* ws_ml, float* out) {
  const int64_t nr = plan.rows ? plan.num_rows : rows;
  if (nr == 0) return hipSuccess;
  dim3 cgrid((unsigned)((nr * hq + 3) / 4));
  if (D != 64 && D != 128) {
    if (D > kMaxHeadDim) return hipErrorInvalidValue;
#define ORION_COMBINE_ANY(NI)                                                                  \
  hipLaunchKernelGGL(paged_decode_combine_any_kernel<NI>, cgrid, dim3(256), 0, st, (int)nr,  \
                     (int)hq, (int)D, plan.row_nsplit, plan.rows, ms, ws_o, ws_ml, out)
    if (D <= 256)
      ORION_COMBINE_ANY(4);
    else if (D <= 512)
      ORION_COMBINE_ANY(8);
    else if (D <= 1024)
      ORION_COMBINE_ANY(16);
    else
      ORION_COMBINE_ANY(32);
#undef ORION_COMBINE_ANY
  } else if (D == 128)
    hipLaunchKernelGGL(paged_decode_combine_kernel<128>, cgrid, dim3(256), 0, st, (int)nr,
                       (int)hq, plan.row_nsplit, plan.rows, ms, ws_o, ws_ml, out);
  else
    hipLaunchKernelGGL(paged_decode_combine_kernel<64>, cgrid, dim3(256), 0, st, (int)nr,
                       (int)hq, plan.row_nsplit, plan.rows, ms, ws_o, ws_ml, out);
  return hipGetLastError();
}

hipError_t launch_split_merge(hipStream_t st, int64_t D, int64_t rows, int64_t hq,
                              const DecodePlanDev& plan, float* out) {
  const int ms = plan.max_splits;
  if (rows == 0 || ms <= 1 || (plan.rows && plan.num_rows == 0)) return hipSuccess;
  if (!plan.ws || plan.ws_bytes < decode_workspace_bytes(rows, hq, D, ms) || !plan.row_nsplit)
    return hipErrorInvalidValue;
  const float* ws_o = plan.ws;
  const float* ws_ml = ws_o + rows * hq * ms * D;
  return launch_combine(st, D, rows, hq, plan, ms, ws_o, ws_ml, out);
}

hipError_t launch_paged_decode(hipStream_t st, const KvGeom& kv, const void* arena, int64_t layer,
                               const float* q, int64_t rows, int64_t hq,
                               const uint32_t* positions, const int32_t* row_seq,
                               const int64_t* bt_off, const uint32_t* bt_ids,
                               const DecodePlanDev& plan, float* out, DecodePhase phase) {
  if (rows == 0 || plan.num_work == 0) return hipSuccess;
  const int64_t hkv = kv.num_kv_heads, D = kv.head_dim;
  if (hkv <= 0 || hq % hkv != 0) return hipErrorInvalidValue;
  const int G = (int)(hq / hkv);
  const int ms = plan.max_splits;
  if (ms > 1 && plan.ws_bytes < decode_workspace_bytes(rows, hq, D, ms))
    return hipErrorInvalidValue;
  float* ws_o = plan.ws;
  float* ws_ml = ws_o ? ws_o + rows * hq * ms * D : nullptr;
  if (phase == DecodePhase::kMerge) {
    if (ms <= 1) return hipSuccess;
    return launch_combine(st, D, rows, hq, plan, ms, ws_o, ws_ml, out);
  }
  int bs_log2 = 0;
  while ((1 << bs_log2) < kv.block_size) ++bs_log2;
  const ArenaStrides a = arena_strides(kv);
  const float scale = 1.0f / sqrtf((float)D);
  const dim3 grid((unsigned)((plan.num_work + 3) / 4));
  hipError_t e;
  // bf16 arenas at head_dim 64/128 with up to 16 query heads per KV head (the
  // MFMA B operand's 16 columns) take the MFMA wave; f32 arenas take the VALU
  // wave up to 8; everything else the general wave.
  // packed prefix items exist only for the MFMA wave, pack_r = 16 / G rows
  const bool mfma = kv.dtype_bf16 && (D == 64 || D == 128) && G <= 16;
  if (plan.num_packed && (!mfma || G > 8 || plan.pack_r != 16 / G || !plan.pack_rows))
    return hipErrorInvalidValue;
  if ((D != 64 && D != 128) || G > (kv.dtype_bf16 ? 16 : 8)) {
    if (D > kMaxHeadDim || (D & 1)) return hipErrorInvalidValue;
#define ORION_ANY(TT, NC)                                                                      \
  hipLaunchKernelGGL((paged_decode_any_kernel<TT, NC>), grid, dim3(256), 0, st,                \
                     static_cast<const TT*>(arena) + layer * a.layer, a.blk, a.v_off, a.slot,  \
                     a.head, bs_log2, (int)hkv, (int)hq, (int)D, plan.work, plan.num_work, q,  \
                     bt_ids, ms, scale, out, ws_o, ws_ml)
#define ORION_ANY_D(TT)            \
  do {                             \
    if (D <= 256)                  \
      ORION_ANY(TT, 2);            \
    else if (D <= 512)             \
      ORION_ANY(TT, 4);            \
    else if (D <= 1024)            \
      ORION_ANY(TT, 8);            \
    else                           \
      ORION_ANY(TT, 16);           \
  } while (0)
    if (kv.dtype_bf16)
      ORION_ANY_D(uint16_t);
    else
      ORION_ANY_D(float);
#undef ORION_ANY_D
#undef ORION_ANY
    e = hipGetLastError();
  } else if (kv.dtype_bf16) {
    // in-block strides travel as 32-bit values; block offsets are 64-bit
    if (a.blk > (int64_t)UINT32_MAX) return hipErrorInvalidValue;
    const uint16_t* base = static_cast<const uint16_t*>(arena) + layer * a.layer;
    const bool big = kv.block_size >= 16;
#define ORION_MFMA2(DD, SS, BB)                                                                      \
  launch_mfma2<DD, SS, BB>(G, grid, st, base, a, bs_log2, (int)hkv, (int)hq, plan.work,          \
                       plan.num_work, q, positions, row_seq, bt_off, bt_ids, ms, scale, out,    \
                       ws_o, ws_ml, plan.num_packed ? plan.pack_rows : nullptr)
    // per-item load flavour only with whole-block steps (blocks of >= 16 slots)
    const int kvm = plan.stream_kv ? 1 : (plan.mixed_kv && big) ? 2 : 0;
    if (D == 128)
      e = big ? (kvm == 1 ? ORION_MFMA2(128, 1, true)
                 : kvm == 2 ? ORION_MFMA2(128, 2, true) : ORION_MFMA2(128, 0, true))
              : (kvm == 1 ? ORION_MFMA2(128, 1, false) : ORION_MFMA2(128, 0, false));
    else if (D == 64)
      e = big ? (kvm == 1 ? ORION_MFMA2(64, 1, true)
                 : kvm == 2 ? ORION_MFMA2(64, 2, true) : ORION_MFMA2(64, 0, true))
              : (kvm == 1 ? ORION_MFMA2(64, 1, false) : ORION_MFMA2(64, 0, false));
    else
      return hipErrorInvalidValue;
#undef ORION_MFMA2
  } else {
    const float* base = static_cast<const float*>(arena) + layer * a.layer;
    if (D == 128)
      e = launch_valu<float, 128>(G, grid, st, base, a, bs_log2, (int)hkv, (int)hq, plan.work,
                                  plan.num_work, q, positions, row_seq, bt_off, bt_ids, ms,
                                  scale, out, ws_o, ws_ml);
    else if (D == 64)
      e = launch_valu<float, 64>(G, grid, st, base, a, bs_log2, (int)hkv, (int)hq, plan.work,
                                 plan.num_work, q, positions, row_seq, bt_off, bt_ids, ms,
                                 scale, out, ws_o, ws_ml);
    else
      return hipErrorInvalidValue;
  }
  if (e != hipSuccess || ms == 1 || phase == DecodePhase::kSplit) return e;
  return launch_combine(st, D, rows, hq, plan, ms, ws_o, ws_ml, out);
}

}  // namespace orion

// Chunked-prefill causal attention over the paged KV cache, on bf16 MFMA.
//
// Same result per query row as the reference's paged_attention
// (crates/orion-models/src/attention.rs:219-295): query head h reads kv head
// h / (Hq/Hkv), attends positions 0..=its own position (context_len is not
// consulted), scores are (q.k) / sqrt(d), softmax, weighted sum of V.  The
// rows of one prefill chunk hold consecutive positions, so a chunk is one
// dense causal contraction against its sequence's cached prefix plus itself.
//
// Work unit (one 256-thread workgroup): one (sequence, kv head) and a tile of
// 128 "packed rows", packed row p = (chunk row p / G, query head p % G) with
// G = Hq/Hkv.  Packing the G query heads that share a kv head into the M
// dimension means every K/V tile staged in LDS is used by all of them: K and
// V are read from HBM once per 128 packed rows instead of once per head.
// Each of the 4 waves owns 32 packed rows (two 16-row MFMA tiles).
//
// Per 64-key tile:
//   S^T = K . Q^T   (v_mfma_f32_16x16x32_bf16; A = K rows from LDS, B = the
//                    wave's queries held in registers as bf16 fragments)
//   online softmax per query (a query is one lane column of S^T, so its
//   running max / sum are per-lane scalars; the max is only exchanged across
//   the four lane groups when a score exceeds it by more than 8)
//   O^T += V^T . P^T (A = V^T via ds_read_tr16_b64 from the row-major LDS V
//                    tile, B = P^T, which is the S^T accumulator layout
//                    converted in place)
// K/V tiles are double-buffered in LDS; the global loads of tile t+1 and the
// block-table lookups of tile t+2 are in flight while tile t computes.
//
// Operand precision, per operand (OPS = kPrefillQHiLo | kPrefillPHiLo bits):
// an operand without its bit is rounded to bf16 (RNE, the MFMA-rate path for
// bf16 inputs); with it, it is carried as a hi + lo bf16 pair (two MFMAs), so
// its products keep ~16 mantissa bits, matching the decode kernels'
// precision.  Q's rounding moves every score (the softmax amplifies it); P's
// only the weights' last bits.
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <type_traits>
#include <utility>
#include <vector>

namespace orion {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kBN = 64;                     // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;               // log2 units: weights stay <= 2^8

// RNE pack of two f32 into bf16x2 bits (v_cvt_pk_bf16_f32).
__device__ inline uint32_t pack_bf16_rne(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ inline bf16x8 u4_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// s_waitcnt vmcnt(N) with the other counters untouched (gfx9 encoding:
// vmcnt bits [3:0] and [15:14]).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}


}  // namespace

// LDS K/V tiles are unpadded rows of D bf16 (kBN rows), written by
// global_load_lds (each wave instruction fills 1 KiB: 64 lanes x 16 bytes in
// lane order).  The 16-byte chunks of row r are stored XOR-permuted,
// chunk' = chunk ^ swz(r), chosen per tile by measurement on gfx950 so that
// the K fragment read (ds_read_b128: 16 consecutive rows x 2 chunk groups
// per 32-lane pass) and the transposed V read (ds_read_b64_tr_b16: 16 rows x
// 2 adjacent chunks) run at the bank-conflict-free rate.
template <int D>
__device__ inline int swz_k(int r) {
  return D == 128 ? (r & 15) : (r & 7);
}
template <int D>
__device__ inline int swz_v(int r) {
  if constexpr (D == 128) return ((r & 7) << 1) | ((r >> 3) & 1);
  else return r & 7;
}

// WAVES waves per workgroup (16 * kNR packed rows each); STAGES K/V tiles
// resident in LDS, STAGES - 1 of them in flight.
template <int D, int OPS, bool BIG, int WAVES, int STAGES>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2)))
    paged_prefill_kernel(const uint16_t* __restrict__ kv_layer, uint32_t blk_stride,
                         uint32_t v_off, uint32_t slot_stride, uint32_t head_stride,
                         int bs_log2, int num_kv_heads,
                         int num_q_heads, const float* __restrict__ q,
                         const PrefillTile* __restrict__ order,
                         const int32_t* __restrict__ row_start,
                         const int32_t* __restrict__ row_count,
                         const uint32_t* __restrict__ first_pos,
                         const int64_t* __restrict__ bt_offsets,
                         const uint32_t* __restrict__ bt_ids, float scale_log2,
                         float* __restrict__ out, PrefillSplitOut split) {
  constexpr int kWaves = WAVES;
  constexpr int kNR = prefill_wave_row_tiles(D);  // 16-row MFMA tiles per wave
  constexpr int kBM = kWaves * 16 * kNR;          // packed rows per workgroup
  constexpr bool QHL = (OPS & kPrefillQHiLo) != 0, PHL = (OPS & kPrefillPHiLo) != 0;
  constexpr int kStages = STAGES;
  static_assert(kStages >= 2 && kStages <= 3, "LDS stages");
  constexpr int KCH = D / 32;           // S^T k-steps
  constexpr int DT = D / 16;            // O^T dim tiles
  constexpr int CPR = D / 8;            // 16-byte chunks per key row
  constexpr int RPI = 64 / CPR;         // key rows per wave load instruction
  constexpr int LPW = kBN / kWaves / RPI;  // load instructions per wave (K and V each)
  constexpr int TILE = kBN * D;         // one K or V tile, elements
  static_assert(LPW >= 1 && RPI * LPW * kWaves == kBN, "tile shape");

  // [k|v][buf]: every K or V read is a per-lane base (K or V region) plus an
  // immediate offset below 64 KiB.
  __shared__ __attribute__((aligned(1024))) uint16_t lds[2][kStages][TILE];

  const int item = blockIdx.x / num_kv_heads;  // the kv heads of one tile are adjacent
  const int kvh = blockIdx.x - item * num_kv_heads;
  const PrefillTile pt = order[item];
  const int seq = pt.seq, tile = pt.tile;
  const int G = num_q_heads / num_kv_heads;
  const int cnt = row_count[seq];
  const int P = cnt * G;
  if (tile * kBM >= P) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int grp = lane >> 4;
  const int bs_mask = (1 << bs_log2) - 1;

  const int pos0 = (int)first_pos[seq];
  const int64_t rs = row_start[seq];
  const uint32_t* tbl = bt_ids + bt_offsets[seq];
  const int p_lo = tile * kBM;
  const int p_hi = min(P, p_lo + kBM) - 1;
  const int kv_len = pos0 + p_hi / G + 1;          // keys this workgroup reads
  const int min_pos = pos0 + p_lo / G;             // no masking below this key
  const int ntiles = (kv_len + kBN - 1) / kBN;
  // this entry's key tiles [t0, t_end)
  const int t0 = pt.kt0, t_end = min(pt.kt1, ntiles), nloc = t_end - t0;

  // ---- this lane's queries (packed rows of its two row tiles) ----
  int qpos[kNR];
  bf16x8 qhi[kNR][KCH], qlo[kNR][KCH];
#pragma unroll
  for (int rt = 0; rt < kNR; ++rt) {
    const int p = min(p_lo + wave * 16 * kNR + rt * 16 + l16, P - 1);
    const int r = p / G;
    qpos[rt] = pos0 + r;
    const float* qp = q + ((rs + r) * num_q_heads + (int64_t)kvh * G + (p - r * G)) * D + grp * 8;
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const float4 x0 = *reinterpret_cast<const float4*>(qp + 32 * c);
      const float4 x1 = *reinterpret_cast<const float4*>(qp + 32 * c + 4);
      uint4 h, l;
      if constexpr (QHL) {
        split2_trunc(x0.x, x0.y, h.x, l.x);
        split2_trunc(x0.z, x0.w, h.y, l.y);
        split2_trunc(x1.x, x1.y, h.z, l.z);
        split2_trunc(x1.z, x1.w, h.w, l.w);
        qlo[rt][c] = u4_bf16x8(l);
      } else {
        h.x = pack_bf16_rne(x0.x, x0.y);
        h.y = pack_bf16_rne(x0.z, x0.w);
        h.z = pack_bf16_rne(x1.x, x1.y);
        h.w = pack_bf16_rne(x1.z, x1.w);
        (void)l;
      }
      qhi[rt][c] = u4_bf16x8(h);
    }
  }

  // ---- K/V tile loader: wave instruction j fills rows wave*RPI*LPW + j*RPI
  // + lane / CPR; the lane stores LDS chunk lane % CPR of its row, which
  // holds global chunk (lane % CPR) ^ swz(row).  With blocks of >= 16 slots
  // a wave's 16 rows of a tile lie in one block: one (uniform) table read. ----
  constexpr int NID = BIG ? 1 : LPW;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int ld_row0 = wave * RPI * LPW + lane / CPR;
  const uint16_t* head_base = kv_layer + (uint32_t)kvh * head_stride;
  uint32_t ld_off_k[LPW], ld_off_v[LPW];  // element offsets of the fetched chunks
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    ld_off_k[j] = (uint32_t)(((lane % CPR) ^ swz_k<D>(ld_row0 + j * RPI)) * 8);
    ld_off_v[j] = (uint32_t)(((lane % CPR) ^ swz_v<D>(ld_row0 + j * RPI)) * 8) + v_off;
  }
  uint32_t ids_next[NID];       // block ids of the tile after the one in flight
  auto key_of = [&](int t, int j) { return min(t * kBN + ld_row0 + j * RPI, kv_len - 1); };
  auto load_ids = [&](int t, uint32_t (&ids)[NID]) {
    const int tt = min(t, ntiles - 1);
    if constexpr (BIG) {
      // uniform index: a scalar load, counted apart from the tile loads
      ids[0] = tbl[__builtin_amdgcn_readfirstlane(
          min(tt * kBN + wave_u * RPI * LPW, kv_len - 1) >> bs_log2)];
    } else {
#pragma unroll
      for (int j = 0; j < LPW; ++j) ids[j] = tbl[key_of(tt, j) >> bs_log2];
    }
  };
  const uint32_t lds_base = (uint32_t)(uintptr_t)&lds[0][0][0];
  auto load_tile = [&](int t, int buf, const uint32_t (&ids)[NID]) {
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      // block offset in 64 bits (a layer may exceed 2^32 elements), the
      // in-block offset in 32
      const size_t off = (size_t)ids[BIG ? 0 : j] * blk_stride +
                         __umul24((uint32_t)(key_of(t, j) & bs_mask), slot_stride);
      const uint32_t dk =
          lds_base + (uint32_t)((buf * TILE + (wave_u * LPW + j) * RPI * D) * 2);
      lds_load16(head_base + off + ld_off_k[j], __builtin_amdgcn_readfirstlane(dk));
      lds_load16(head_base + off + ld_off_v[j],
                 __builtin_amdgcn_readfirstlane(dk + kStages * TILE * 2));
    }
  };

  // Tile-load accounting: a wave's tile loads are 2*LPW global_load_lds
  // (counted by vmcnt, completing in issue order); with small blocks the
  // per-row block ids are LPW vector loads issued after them.
  constexpr int kTileOps = 2 * LPW;
  constexpr int kIdOps = BIG ? 0 : LPW;

  constexpr int kAhead = kStages - 1;  // tiles in flight while one computes
  constexpr int kBehind = (kAhead - 1) * (kTileOps + kIdOps);  // loads after the next tile's

  // ---- prologue: tiles 0 .. kAhead-1 into LDS buffers 0 .. kAhead-1, ids of
  // tile kAhead ----
  {
    uint32_t ids0[NID];
#pragma unroll
    for (int i = 0; i < kAhead; ++i) {
      if (i < nloc) {
        load_ids(t0 + i, ids0);
        load_tile(t0 + i, i, ids0);
      }
    }
    load_ids(t0 + kAhead, ids_next);
  }
  if (nloc >= kAhead)
    wait_vmcnt<kBehind>();  // tile 0 has landed (the later ones and the ids may not)
  else
    wait_vmcnt<0>();
  __syncthreads();

  float m[kNR];                 // running max of raw scores (q.k), per query
  f32x4 o[kNR][DT];             // O^T: dims 16d + 4*grp + i, query l16
  f32x4 lsum[kNR];              // row sums of the weights, from a ones-row MFMA
#pragma unroll
  for (int rt = 0; rt < kNR; ++rt) {
    m[rt] = -INFINITY;
    lsum[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < DT; ++t) o[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const bf16x8 ones = __builtin_bit_cast(bf16x8, uint4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u,
                                                       0x3F803F80u});

  // Loop-invariant LDS byte addresses (buffer 0).  K fragment: row
  // kt*16 + l16, chunk 4c + grp (kt only adds a constant: the swizzles depend
  // on the low 4 row bits only).  Transposed V read, lane 4rr + cc of a group: row
  // 4*grp + rr (+16, +32: constants), dims 16d + 4cc .. +3.
  const int vr = 4 * grp + (l16 >> 2);
  const int vcc = l16 & 3;
  uint32_t k_addr[KCH], v_addr[DT];
#pragma unroll
  for (int c = 0; c < KCH; ++c)
    k_addr[c] = lds_base + (uint32_t)(l16 * D + (((4 * c + grp) ^ swz_k<D>(l16)) * 8)) * 2;
#pragma unroll
  for (int d = 0; d < DT; ++d)
    v_addr[d] = lds_base + (uint32_t)(kStages * TILE + vr * D +
                                      ((2 * d + (vcc >> 1)) ^ swz_v<D>(vr)) * 8 + (vcc & 1) * 4) * 2;
  const float lazy_raw = kLazy / scale_log2;

  // One key tile; BUF (the LDS buffer holding it) is a compile-time constant
  // so every LDS read is a loop-invariant address plus an immediate offset.
  auto step = [&](int t, auto buf_tag) {
    constexpr int BUF = decltype(buf_tag)::value;
    constexpr uint32_t kBufOff = BUF * TILE * 2;
    // Tile t + kAhead goes into the buffer tile t - 1 used (every wave passed
    // the barrier that ended step t - 1, so its reads are done).
    if (t + kAhead < t_end) {
      load_tile(t + kAhead, (BUF + kAhead) % kStages, ids_next);
      load_ids(t + kAhead + 1, ids_next);
    }

    // S^T[rt][kt]: raw scores of keys t*64 + kt*16 + 4*grp + i, query l16.
    // (the first k-step starts from a zero C operand: no zeroing moves)
    f32x4 s[kNR][4];
    // K fragments one k-step ahead of the MFMAs that consume them.
    u32x4 kf[2][4];
    auto read_k = [&](int c, u32x4 (&dst)[4]) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        dst[kt] = *(const lds_u32x4*)(uintptr_t)(k_addr[c] + kBufOff + kt * 16 * D * 2);
    };
    read_k(0, kf[0]);
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      if (c + 1 < KCH) read_k(c + 1, kf[(c + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the MFMAs
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const bf16x8 ka = __builtin_bit_cast(bf16x8, kf[c & 1][kt]);
#pragma unroll
        for (int rt = 0; rt < kNR; ++rt) {
          s[rt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              ka, qhi[rt][c], c == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[rt][kt], 0, 0, 0);
          if constexpr (QHL)
            s[rt][kt] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qlo[rt][c], s[rt][kt], 0, 0, 0);
        }
      }
    }

    // Online softmax: weights exp2((s - m) * scale_log2); m only rises (with
    // an exact cross-group max and a rescale) when a score exceeds it by
    // more than kLazy in log2 units.
    const bool masked = t * kBN + kBN - 1 > min_pos;
    bf16x8 phi[kNR][2], plo[kNR][2];
#pragma unroll
    for (int rt = 0; rt < kNR; ++rt) {
      if (masked) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (t * kBN + kt * 16 + 4 * grp + i > qpos[rt]) s[rt][kt][i] = -INFINITY;
      }
      // three-input maxes (v_max3_f32): 8 per 16 scores
      float mx = fmaxf(fmaxf(s[rt][0][0], s[rt][0][1]), s[rt][0][2]);
      mx = fmaxf(fmaxf(mx, s[rt][0][3]), s[rt][1][0]);
#pragma unroll
      for (int e = 5; e < 16; e += 2)
        mx = fmaxf(fmaxf(mx, s[rt][e >> 2][e & 3]), s[rt][(e + 1) >> 2][(e + 1) & 3]);
      if (__builtin_amdgcn_ballot_w64(mx > m[rt] + lazy_raw) != 0) {
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m[rt], mx);
        // A query with no key yet in this part (every score so far masked)
        // keeps m = -inf while other lanes of the wave raise theirs: its
        // alpha must be 1 (o and lsum are still 0), not exp2(-inf + inf) = NaN.
        const float alpha =
            m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f((m[rt] - m_new) * scale_log2);
        m[rt] = m_new;
        lsum[rt] *= alpha;
#pragma unroll
        for (int d = 0; d < DT; ++d) o[rt][d] *= alpha;
      }
      // (a part that starts past some rows' positions sees no key of theirs:
      // m stays -inf and every weight must come out 0, not NaN)
      const float nm = m[rt] == -INFINITY ? 0.f : -m[rt] * scale_log2;
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        float pv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][2 * kp][i], scale_log2, nm));
          pv[4 + i] =
              __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][2 * kp + 1][i], scale_log2, nm));
        }
        uint4 h, l;
        if constexpr (PHL) {
          split2_trunc(pv[0], pv[1], h.x, l.x);
          split2_trunc(pv[2], pv[3], h.y, l.y);
          split2_trunc(pv[4], pv[5], h.z, l.z);
          split2_trunc(pv[6], pv[7], h.w, l.w);
          plo[rt][kp] = u4_bf16x8(l);
        } else {
          h.x = pack_bf16_rne(pv[0], pv[1]);
          h.y = pack_bf16_rne(pv[2], pv[3]);
          h.z = pack_bf16_rne(pv[4], pv[5]);
          h.w = pack_bf16_rne(pv[6], pv[7]);
          (void)l;
        }
        phi[rt][kp] = u4_bf16x8(h);
      }
    }

    // O^T[rt][d] += V^T . P^T; k-slots 0..3 = keys kp*32 + 4*grp + rr,
    // slots 4..7 = the same + 16 (the layout of S^T tiles 2kp and 2kp + 1).
    // The row sums come from the same P^T against a row of ones.
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) {
#pragma unroll
      for (int rt = 0; rt < kNR; ++rt) {
        lsum[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, phi[rt][kp], lsum[rt], 0, 0, 0);
        if constexpr (PHL)
          lsum[rt] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, plo[rt][kp], lsum[rt], 0, 0, 0);
      }
    }
    // V^T fragments (two transposed reads per 32 keys) one dim tile ahead.
    typedef short v8s __attribute__((ext_vector_type(8)));
    v8s vf[2][2];
    auto read_v = [&](int d, v8s (&dst)[2]) {
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        const uint32_t a0 = v_addr[d] + kBufOff + kp * 32 * D * 2;
        const v4s v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)a0);
        const v4s v1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(a0 + 16 * D * 2));
        dst[kp] = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    };
    read_v(0, vf[0]);
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      if (d + 1 < DT) read_v(d + 1, vf[(d + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        const bf16x8 va = __builtin_bit_cast(bf16x8, vf[d & 1][kp]);
#pragma unroll
        for (int rt = 0; rt < kNR; ++rt) {
          o[rt][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, phi[rt][kp], o[rt][d], 0, 0, 0);
          if constexpr (PHL)
            o[rt][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, plo[rt][kp], o[rt][d], 0, 0, 0);
        }
      }
    }

    // Tile t + 1 must have landed; the tiles after it (and their ids) may
    // still be in flight.
    if (t + kAhead < t_end)
      wait_vmcnt<kBehind>();
    else
      wait_vmcnt<0>();
    __syncthreads();
  };

  for (int u = 0; u < nloc; u += kStages) {
    step(t0 + u, std::integral_constant<int, 0>{});
    if (u + 1 < nloc) step(t0 + u + 1, std::integral_constant<int, 1>{});
    if constexpr (kStages > 2)
      if (u + 2 < nloc) step(t0 + u + 2, std::integral_constant<int, 2>{});
  }

  // ---- normalise and store: lane holds dims 16d + 4*grp .. +3 of query l16 ----
#pragma unroll
  for (int rt = 0; rt < kNR; ++rt) {
    const int p = p_lo + wave * 16 * kNR + rt * 16 + l16;
    if (pt.nparts > 1 && p < P) {  // unnormalised part, merged afterwards
      const int r = p / G;
      const int64_t slot =
          ((rs + r) * num_q_heads + (int64_t)kvh * G + (p - r * G)) * split.max_parts + pt.part;
      float* op = split.ws_o + slot * D + 4 * grp;
#pragma unroll
      for (int d = 0; d < DT; ++d)
        *reinterpret_cast<float4*>(op + 16 * d) =
            make_float4(o[rt][d][0], o[rt][d][1], o[rt][d][2], o[rt][d][3]);
      // max in scaled-score units (natural exp), as the decode waves write it
      if (grp == 0)
        *reinterpret_cast<float2*>(split.ws_ml + slot * 2) =
            make_float2(m[rt] * (scale_log2 / kLog2e), lsum[rt][0]);
    } else if (p < P) {
      const int r = p / G;
      const float inv = 1.0f / lsum[rt][0];
      const int64_t head = (rs + r) * num_q_heads + (int64_t)kvh * G + (p - r * G);
      if (split.out_hilo) {
        // the O GEMM's split operand layout: per 8 dims [8 hi bf16 | 8 lo bf16];
        // this lane's 4 dims are half grp & 1 of group 2d + grp / 2
        uint2* hb = reinterpret_cast<uint2*>(out + head * D) + (grp >> 1) * 4 + (grp & 1);
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          uint16_t h[4], l[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) split1_trunc(o[rt][d][i] * inv, h[i], l[i]);
          hb[8 * d] = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
          hb[8 * d + 2] =
              make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
        }
      } else {
        float* op = out + head * D + 4 * grp;
#pragma unroll
        for (int d = 0; d < DT; ++d)
          *reinterpret_cast<float4*>(op + 16 * d) =
              make_float4(o[rt][d][0] * inv, o[rt][d][1] * inv, o[rt][d][2] * inv,
                          o[rt][d][3] * inv);
      }
    }
  }
}

hipError_t launch_paged_prefill(hipStream_t st, const KvGeom& kv, const void* arena,
                                int64_t layer, const float* q, int64_t hq,
                                const PrefillTile* order, int64_t num_tiles,
                                const int32_t* row_start, const int32_t* row_count,
                                const uint32_t* first_pos, const int64_t* bt_offsets,
                                const uint32_t* bt_ids, int operands, float* out,
                                const PrefillSplitOut& split) {
  if (num_tiles == 0) return hipSuccess;
  if (!kv.dtype_bf16) return hipErrorNotSupported;
  const int64_t hkv = kv.num_kv_heads, D = kv.head_dim;
  if (hkv <= 0 || hq % hkv != 0 || (D != 64 && D != 128 && D != 256)) return hipErrorInvalidValue;
  int bs_log2 = 0;
  while ((1 << bs_log2) < kv.block_size) ++bs_log2;
  const ArenaStrides a = arena_strides(kv);
  const int64_t layer_elems = a.layer;
  // in-block strides travel as 32-bit values (the slot product as a 24-bit
  // multiply); block offsets are 64-bit
  if (a.blk > (int64_t)UINT32_MAX || a.slot >= (1 << 24) || kv.block_size >= (1 << 24))
    return hipErrorInvalidValue;
  const uint16_t* base = static_cast<const uint16_t*>(arena) + layer * layer_elems;
  if (num_tiles * hkv > INT32_MAX) return hipErrorInvalidValue;
  const float scale_log2 = kLog2e / sqrtf((float)D);
  const dim3 grid((unsigned)(num_tiles * hkv));
  const int waves = prefill_waves();
#define ORION_PREFILL_W(DD, HH, BB, WW, SS)                                                      \
  hipLaunchKernelGGL((paged_prefill_kernel<DD, HH, BB, WW, SS>), grid, dim3(WW * 64), 0, st, base, \
                     (uint32_t)a.blk, (uint32_t)a.v_off, (uint32_t)a.slot, (uint32_t)a.head,   \
                     bs_log2,                                                                  \
                     (int)hkv, (int)hq, q, order, row_start, row_count, first_pos, bt_offsets, \
                     bt_ids, scale_log2, out, split)
// (head_dim 256: 8 waves with 2 stages, 128 KiB of LDS, whatever the knob)
#define ORION_PREFILL_B(DD, HH, BB)                       \
  do {                                                    \
    if (waves == 4 && DD <= 128)                          \
      ORION_PREFILL_W(DD, HH, BB, (DD > 128 ? 8 : 4), 2); \
    else                                                  \
      ORION_PREFILL_W(DD, HH, BB, 8, (DD > 128 ? 2 : 3)); \
  } while (0)
#define ORION_PREFILL(DD, HH)        \
  do {                               \
    if (big)                         \
      ORION_PREFILL_B(DD, HH, true); \
    else                             \
      ORION_PREFILL_B(DD, HH, false);\
  } while (0)
  const bool big = kv.block_size >= 16;
  const int ops = operands & (kPrefillQHiLo | kPrefillPHiLo);
#define ORION_PREFILL_D(DD)                                          \
  do {                                                               \
    if (ops == (kPrefillQHiLo | kPrefillPHiLo)) ORION_PREFILL(DD, 3); \
    else if (ops == kPrefillQHiLo) ORION_PREFILL(DD, 1);              \
    else if (ops == kPrefillPHiLo) ORION_PREFILL(DD, 2);              \
    else ORION_PREFILL(DD, 0);                                        \
  } while (0)
  if (D == 256)
    ORION_PREFILL_D(256);
  else if (D == 128)
    ORION_PREFILL_D(128);
  else
    ORION_PREFILL_D(64);
#undef ORION_PREFILL_D
#undef ORION_PREFILL
#undef ORION_PREFILL_B
#undef ORION_PREFILL_W
  return hipGetLastError();
}

}  // namespace orion

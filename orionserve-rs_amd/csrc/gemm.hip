// Projection GEMMs on bf16 MFMA for gfx950: out[M,N] = x[M,K] . W[N,K]^T.
//
// Restates the reference's `linear` (crates/orion-models/src/tensor.rs:96-130):
// W keeps the HF layout [out_features, in_features] (row-major, K contiguous),
// which is exactly the MFMA B-operand layout: a lane loads 8 consecutive k of
// one output column with one 16-byte load, straight from HBM into registers.
//
// Activations arrive in f32.  Each 8-element A fragment is split on the fly
// into hi = the top 16 bits of x and lo = the top 16 bits of (x - hi) and both
// are multiplied against the bf16 weight (two MFMAs, f32 accumulation), so the
// product carries ~16 mantissa bits of x instead of 8.  Weights are exact
// (bf16 checkpoints widen exactly in the reference loader), so the only
// departure from the reference's f32 arithmetic is summation order plus a
// ~2^-16 relative term per product.
//
// The epilogue fuses the bias add, the residual accumulate
// (transformer.rs:328-332, :345) or SwiGLU (tensor.rs:175-189) on gate/up rows
// interleaved in groups of 8.
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <array>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>

namespace orion {

__device__ inline bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// x -> (hi, lo) bf16 fragments by truncation (x = hi + lo to ~2^-16 relative).
__device__ inline void split8(const float (&a)[8], bf16x8& hi, bf16x8& lo) {
  uint4 hv, lv;
  split2_trunc(a[0], a[1], hv.x, lv.x);
  split2_trunc(a[2], a[3], hv.y, lv.y);
  split2_trunc(a[4], a[5], hv.z, lv.z);
  split2_trunc(a[6], a[7], hv.w, lv.w);
  hi = as_bf16x8(hv);
  lo = as_bf16x8(lv);
}

// Decode-shaped (small M) weight-streaming GEMM.  Workgroup = KW waves on one
// 16*NT-column tile of up to 16*MT rows; the waves split K into KW contiguous
// ranges and each walks its range UNR k-steps (32 k each) at a time, so UNR
// weight loads per column tile are in flight before the MFMAs consume them.
// Each x fragment (loaded from L2) feeds NT column tiles.  The KW partial
// tiles are summed through LDS in wave order (deterministic) and the epilogue
// is applied once.  Weights are read from HBM exactly once per 16*MT rows.
template <int MT, int NT, int KW, int UNR>
__global__ void __launch_bounds__(64 * KW)
    gemm_skinny_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                       const float* __restrict__ bias, int M, int N, int K, int ep,
                       float* __restrict__ out) {
  constexpr int BN = 16 * NT;
  constexpr int BM = 16 * MT;
  __shared__ float red[KW][BM][BN + 1];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int mt_count = min(MT, (M - m0 + 15) >> 4);
  const int ksteps = K >> 5;
  const int ks0 = wave * ksteps / KW;
  const int ks1 = (wave + 1) * ksteps / KW;
  const int lr = lane & 15;
  const int lk = (lane >> 4) * 8;

  const uint16_t* wrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = min(n0 + nt * 16 + lr, N - 1);
    wrow[nt] = w + (int64_t)n * K + lk;
  }
  const float* xrow[MT];
  bool xvalid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + mt * 16 + lr;
    xvalid[mt] = m < M;
    xrow[mt] = x + (int64_t)min(m, M - 1) * K + lk;
  }

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int ks = ks0; ks < ks1; ks += UNR) {
    // Fragments for UNR k-steps (indices clamped into the range; the
    // products of a clamped step are skipped below).
    bf16x8 b[UNR][NT];
    float4 a0[UNR][MT], a1[UNR][MT];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int k = min(ks + u, ks1 - 1) << 5;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        b[u][nt] = as_bf16x8(*reinterpret_cast<const uint4*>(wrow[nt] + k));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (mt < mt_count && xvalid[mt]) {
          a0[u][mt] = *reinterpret_cast<const float4*>(xrow[mt] + k);
          a1[u][mt] = *reinterpret_cast<const float4*>(xrow[mt] + k + 4);
        } else {
          a0[u][mt] = make_float4(0.f, 0.f, 0.f, 0.f);
          a1[u][mt] = a0[u][mt];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      if (ks + u < ks1) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (mt < mt_count) {
            const float a[8] = {a0[u][mt].x, a0[u][mt].y, a0[u][mt].z, a0[u][mt].w,
                                a1[u][mt].x, a1[u][mt].y, a1[u][mt].z, a1[u][mt].w};
            bf16x8 ahi, alo;
            split8(a, ahi, alo);
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
              acc[mt][nt] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, b[u][nt], acc[mt][nt], 0, 0, 0);
              acc[mt][nt] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, b[u][nt], acc[mt][nt], 0, 0, 0);
            }
          }
        }
      }
    }
  }

  // C fragment layout: lane holds rows 4*(lane/16) + i, column lane % 16.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (mt < mt_count) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          red[wave][mt * 16 + (lane >> 4) * 4 + i][nt * 16 + lr] = acc[mt][nt][i];
    }
  }
  __syncthreads();

  const int rows = min(BM, M - m0);
  if (ep == (int)Epilogue::kSwiGLU) {
    // Tile columns nt*16 + [0,8) are gate rows, nt*16 + [8,16) the matching up rows.
    const int half_n = N >> 1;
    for (int idx = threadIdx.x; idx < rows * NT * 8; idx += 64 * KW) {
      const int r = idx / (NT * 8);
      const int cc = idx - r * (NT * 8);
      const int nt = cc >> 3, j = cc & 7;
      const int gcol = n0 + nt * 16 + j;
      if (gcol >= N) continue;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int wv = 0; wv < KW; ++wv) {
        g += red[wv][r][nt * 16 + j];
        u += red[wv][r][nt * 16 + 8 + j];
      }
      const float act = g / (1.0f + __expf(-g)) * u;
      out[(int64_t)(m0 + r) * half_n + (n0 >> 1) + nt * 8 + j] = act;
    }
  } else {
    for (int idx = threadIdx.x; idx < rows * BN; idx += 64 * KW) {
      const int r = idx / BN;
      const int cc = idx - r * BN;
      const int col = n0 + cc;
      if (col >= N) continue;
      float v = 0.f;
#pragma unroll
      for (int wv = 0; wv < KW; ++wv) v += red[wv][r][cc];
      float* op = out + (int64_t)(m0 + r) * N + col;
      if (ep == (int)Epilogue::kAccumulate)
        *op += v;
      else
        *op = bias ? v + bias[col] : v;
    }
  }
}

// Prefill-shaped (large M) GEMM: 128 x 128 output tile per 256-thread
// workgroup (2 x 2 waves of 64 x 64), k-steps of 32.  The f32 activation tile
// (128 x 32) and the bf16 weight tile (128 x 32) are copied HBM -> LDS with
// global_load_lds (no staging registers), double-buffered so the next
// k-step's copy is in flight while this one computes.  Each wave splits its A
// fragments into hi/lo bf16 on the fly (as the skinny kernel does) and issues
// 4 x 4 x 2 MFMAs per k-step; B fragments are reused by the 4 row tiles and A
// fragments by the 4 column tiles.  LDS rows are XOR-swizzled in 16-byte
// chunks (conflict-free 16-byte fragment reads; the DMA writes stay linear).
namespace {
constexpr int kTM = 128, kTN = 128, kTK = 32;
// A tile row r: 8 chunks of 4 floats; chunk c stored at c ^ swz_a(r).
__device__ inline int swz_a(int r) {
  return ((r >> 2) & 1) | (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2);
}
// B tile row n: 4 chunks of 8 bf16; chunk c stored at c ^ swz_b(n).
__device__ inline int swz_b(int n) { return (n >> 2) & 3; }
}  // namespace

// W is either row-major [N, K] (pk.nt == 0) or in the decode GEMM's packed
// order (launch_gemv_pack with geometry pk): there a 16-column x 32-k MFMA B
// fragment is one contiguous KiB, lane l's 16 bytes at l * 16, so each of the
// tile's 8 fragments per k-step is copied to LDS verbatim and read back with
// one conflict-free ds_read_b128 per lane.
struct PackedGeom {
  int nt = 0, ks = 0, n_tiles = 0;  // columns per decode workgroup / 64, k-steps per slice
};

// HILO: x carried as a truncated hi + lo bf16 pair (two MFMAs, ~16 bits of
// x per product); otherwise rounded to bf16 (nearest even, one MFMA).
// XS (with HILO): x is already in that split layout (GemmFuse::x_hilo), so a
// fragment's two 16-byte LDS chunks are its hi and lo bf16x8 as they are.
// NTW: 16-column tiles per wave (4: 128-column workgroup tiles; 8: 256).
// out_hilo: the SwiGLU epilogue writes its output in the split layout.
template <bool HILO, int NTW, bool XS = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NTW == 8 ? 2 : 1)))
    gemm_tiled_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                      const float* __restrict__ bias, int M, int N, int K, int ep,
                      float* __restrict__ out, PackedGeom pk, int gm, int kspan,
                      float* __restrict__ partial, bool out_hilo) {
  static_assert(HILO || !XS, "a pre-split x needs the hi/lo MFMAs");
  constexpr int TN = 32 * NTW;   // workgroup columns
  constexpr int BJ = NTW / 2;    // B copies (1 KiB each) per wave per k-step
  __shared__ __attribute__((aligned(1024))) float As[2][kTM * kTK];
  __shared__ __attribute__((aligned(1024))) uint16_t Bs[2][TN * kTK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, grp = lane >> 4;
  // Tile order.  gm == 0: the 2D grid is (n tile, m tile).  gm > 0: a 1D grid
  // of 8 * ceil(tiles / 8) workgroups in XCD-aware grouped order: workgroup b
  // runs on XCD b % 8 (round-robin dispatch), each XCD takes a contiguous
  // eighth of the tiles and walks it in groups of gm m tiles, n outer, so the
  // tiles in flight on one XCD share A and B slabs in its L2.
  int mt_i = blockIdx.y, nt_i = blockIdx.x;
  if (gm > 0) {
    const int gx = (N + TN - 1) / TN, gy = (M + kTM - 1) / kTM, total = gx * gy;
    const int b = blockIdx.x;
    const int per = (total + 7) / 8;
    const int t = (b & 7) * per + (b >> 3);
    if (t >= total) return;  // padding workgroups (before any barrier)
    const int g = t / (gm * gx), within = t - g * gm * gx;
    const int gm_eff = min(gm, gy - g * gm);
    mt_i = g * gm + within % gm_eff;
    nt_i = within / gm_eff;
  }
  const int m0 = mt_i * kTM, n0 = nt_i * TN;

  // ---- DMA addressing: A = 4 wave instructions (8 rows x 128 B each),
  // B = 2 wave instructions (16 rows x 64 B each). ----
  const float* a_src[4];
  const uint16_t* b_src[BJ];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = (wave * 4 + j) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ swz_a(r);
    a_src[j] = x + (int64_t)min(m0 + r, M - 1) * K + c * 4;
  }
  // Packed W: fragment f = wave * 2 + j holds columns n0 + 16 f .. + 16.  Its
  // chunk (decode workgroup share) within a K slice, and the last fragment
  // column group the packed copy holds (columns past it are past N anyway).
  const bool packed = pk.nt > 0;
  int64_t b_chunk[BJ] = {};
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    if (packed) {
      const int c16 = min(n0 / 16 + wave * BJ + j, pk.n_tiles * 4 * pk.nt - 1);
      const int tile = c16 / (4 * pk.nt), rem = c16 - tile * 4 * pk.nt;
      b_chunk[j] = ((int64_t)tile * 4 + rem / pk.nt) * pk.nt + rem % pk.nt;
      b_src[j] = w + (int64_t)lane * 8;
    } else {
      const int r = (wave * BJ + j) * 16 + (lane >> 2);
      const int c = (lane & 3) ^ swz_b(r);
      b_src[j] = w + (int64_t)min(n0 + r, N - 1) * K + c * 8;
    }
  }
  const int64_t slice_elems = (int64_t)pk.n_tiles * 4 * pk.nt * pk.ks * 512;  // one K slice
  const uint32_t as_base = (uint32_t)(uintptr_t)&As[0][0];
  const uint32_t bs_base = (uint32_t)(uintptr_t)&Bs[0][0];
  auto load_tile = [&](int ks, int buf) {
    const int k0 = ks * kTK;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      lds_load16(a_src[j] + k0, as_base + (uint32_t)(buf * kTM * kTK * 4 + (wave * 4 + j) * 1024));
    if (packed) {
      const int slice = ks / pk.ks, step = ks - slice * pk.ks;
#pragma unroll
      for (int j = 0; j < BJ; ++j)
        lds_load16(b_src[j] + slice * slice_elems + (b_chunk[j] * pk.ks + step) * 512,
                   bs_base + (uint32_t)(buf * TN * kTK * 2 + (wave * BJ + j) * 1024));
    } else {
#pragma unroll
      for (int j = 0; j < BJ; ++j)
        lds_load16(b_src[j] + k0, bs_base + (uint32_t)(buf * TN * kTK * 2 + (wave * BJ + j) * 1024));
    }
  };

  // ---- fragment read addresses (bytes, buffer 0) ----
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  uint32_t a_rd0[4], a_rd1[4], b_rd[NTW];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int r = wm * 64 + mt * 16 + l16;
    a_rd0[mt] = as_base + (uint32_t)(r * kTK + (((2 * grp) ^ swz_a(r)) * 4)) * 4;
    a_rd1[mt] = as_base + (uint32_t)(r * kTK + (((2 * grp + 1) ^ swz_a(r)) * 4)) * 4;
  }
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    const int n = wn * 16 * NTW + nt * 16 + l16;
    b_rd[nt] = packed ? bs_base + (uint32_t)((wn * NTW + nt) * 1024 + lane * 16)
                      : bs_base + (uint32_t)(n * kTK + ((grp ^ swz_b(n)) * 8)) * 2;
  }

  f32x4 acc[4][NTW];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // K split z = blockIdx.z covers k-steps [z * kspan, min(ksteps, (z + 1) * kspan))
  const int ks_begin = blockIdx.z * kspan;
  const int ksteps = min(K / kTK, ks_begin + kspan);
  load_tile(ks_begin, 0);
  wait_vmem_all();
  __syncthreads();
  for (int ks = ks_begin; ks < ksteps; ++ks) {
    const int buf = (ks - ks_begin) & 1;
    if (ks + 1 < ksteps) load_tile(ks + 1, buf ^ 1);
    const uint32_t aoff = (uint32_t)(buf * kTM * kTK * 4);
    const uint32_t boff = (uint32_t)(buf * TN * kTK * 2);
    bf16x8 bw[NTW];
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt)
      bw[nt] = __builtin_bit_cast(bf16x8, *(const lds_u32x4*)(uintptr_t)(b_rd[nt] + boff));
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const u32x4 lo4 = *(const lds_u32x4*)(uintptr_t)(a_rd0[mt] + aoff);
      const u32x4 hi4 = *(const lds_u32x4*)(uintptr_t)(a_rd1[mt] + aoff);
      const float a[8] = {__uint_as_float(lo4.x), __uint_as_float(lo4.y),
                          __uint_as_float(lo4.z), __uint_as_float(lo4.w),
                          __uint_as_float(hi4.x), __uint_as_float(hi4.y),
                          __uint_as_float(hi4.z), __uint_as_float(hi4.w)};
      bf16x8 ahi, alo;
      if constexpr (XS) {
        ahi = __builtin_bit_cast(bf16x8, lo4);
        alo = __builtin_bit_cast(bf16x8, hi4);
        (void)a;
      } else if constexpr (HILO) {
        split8(a, ahi, alo);
      } else {
        typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
        typedef float f32x8 __attribute__((ext_vector_type(8)));
        const f32x8 av = {a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7]};
        ahi = __builtin_bit_cast(bf16x8, __builtin_convertvector(av, bf16x8v));
        (void)alo;
      }
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, bw[nt], acc[mt][nt], 0, 0, 0);
        if constexpr (HILO)
          acc[mt][nt] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bw[nt], acc[mt][nt], 0, 0, 0);
      }
    }
    wait_vmem_all();
    __syncthreads();
  }

  // ---- epilogue: acc[mt][nt][i] = C[m0 + wm*64 + mt*16 + 4*grp + i][n0 + wn*64 + nt*16 + l16] ----
  if (partial) {  // one K split: raw sums, reduced by gemm_tiled_reduce_kernel
    float* pz = partial + (int64_t)blockIdx.z * M * N;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        const int col = n0 + wn * 16 * NTW + nt * 16 + l16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = m0 + wm * 64 + mt * 16 + 4 * grp + i;
          if (row < M && col < N) pz[(int64_t)row * N + col] = acc[mt][nt][i];
        }
      }
    return;
  }
  if (ep == (int)Epilogue::kAccumulate) {
    // Residual add, one 16-row tile at a time: all of its residual values are
    // loaded before any sum is stored.  Written as `out[i] += v` per element,
    // every load would wait for the stores before it (loads and stores to one
    // array keep their order), one memory round trip per element: at config
    // 4's prefill O and down shapes that epilogue cost 76 and 84 us per
    // launch.  (Loading the whole tile at once, or before the k-loop, takes
    // the kernel past the registers of three workgroups per CU.)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      float res[NTW][4];
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        const int col = n0 + wn * 16 * NTW + nt * 16 + l16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = m0 + wm * 64 + mt * 16 + 4 * grp + i;
          res[nt][i] = (row < M && col < N) ? out[(int64_t)row * N + col] : 0.f;
        }
      }
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        const int col = n0 + wn * 16 * NTW + nt * 16 + l16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = m0 + wm * 64 + mt * 16 + 4 * grp + i;
          if (row < M && col < N) out[(int64_t)row * N + col] = res[nt][i] + acc[mt][nt][i];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) {
      const int col = n0 + wn * 16 * NTW + nt * 16 + l16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + wm * 64 + mt * 16 + 4 * grp + i;
        const float v = acc[mt][nt][i];
        if (ep == (int)Epilogue::kSwiGLU) {
          // Tile columns [0, 8) are gate rows of W, [8, 16) the matching up rows.
          const float u = __shfl_xor(v, 8);
          if (l16 < 8 && row < M && col < N) {
            const float act = v / (1.0f + __expf(-v)) * u;
            const int c8 = (n0 + wn * 16 * NTW + nt * 16) >> 1;  // a multiple of 8
            if (out_hilo) {
              uint16_t h, lo;
              split1_trunc(act, h, lo);
              uint16_t* o16 = reinterpret_cast<uint16_t*>(out) + (int64_t)row * N + c8 * 2;
              o16[l16] = h;
              o16[8 + l16] = lo;
            } else {
              out[(int64_t)row * (N >> 1) + c8 + l16] = act;
            }
          }
        } else if (row < M && col < N) {
          out[(int64_t)row * N + col] = bias ? v + bias[col] : v;
        }
      }
    }
  }
}

// Sums the K splits of gemm_tiled_kernel in split order, then the store (+
// bias) or accumulate epilogue.
__global__ void __launch_bounds__(256)
    gemm_tiled_reduce_kernel(const float* __restrict__ partial, int splits, int64_t M, int64_t N,
                             const float* __restrict__ bias, int ep, float* __restrict__ out) {
  const int64_t total = M * N;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    float v = 0.f;
    for (int z = 0; z < splits; ++z) v += partial[z * total + i];
    if (ep == (int)Epilogue::kAccumulate)
      out[i] += v;
    else
      out[i] = bias ? v + bias[i % N] : v;
  }
}

// Decode-shaped (M <= 64) weight-streaming GEMM, split over K across
// workgroups.  Workgroup (256 threads) = 4 waves x NT column tiles of 16 =
// 64*NT output columns, over one K slice of KSTEPS k-steps (32 k each).
//   1. Every wave issues all of its slice's weight loads at once
//      (KSTEPS x NT 16-byte loads per lane straight into MFMA B fragments),
//      so a wave keeps KSTEPS*NT KiB in flight.
//   2. Meanwhile the workgroup stages the activation slice x[0:M, slice] in
//      LDS once, already split into hi/lo bf16 A fragments (lane-major), so
//      the 4 waves share one read of x instead of one read per 16 columns.
//   3. MFMAs; with one K slice the epilogue is applied directly.  With
//      several, each workgroup writes its partial tile to the scratch and a
//      second kernel sums the slices in slice order (deterministic) and
//      applies the epilogue.
template <int MT, int NT, int KSTEPS>
__global__ void __launch_bounds__(256)
    gemm_gemv_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                     const float* __restrict__ bias, int M, int N, int K, int ep,
                     float* __restrict__ out, float* __restrict__ partial,
                     const double* __restrict__ nsq, int nslots, const float* __restrict__ nw,
                     float neps, int wpacked) {
  constexpr int BN = 64 * NT;
  __shared__ __attribute__((aligned(16))) uint4 xs[2][MT * KSTEPS * 64];  // [hi|lo][frag][lane]
  __shared__ float nscale[MT * 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, grp = lane >> 4;
  const int n0 = blockIdx.x * BN;
  const int kslices = gridDim.y;
  const int k0 = blockIdx.y * KSTEPS * 32;
  const int nsteps = min(KSTEPS, (K - k0) >> 5);

  // Load order: the activation slice (and norm inputs) first, the weights
  // last, so staging the activations and the first MFMAs wait only for the
  // L2-resident inputs while the weight stream is still arriving (a wave's
  // loads complete in issue order).
  // 1. activation slice fragments: fragment f = (mt, step), lane l holds row
  //    mt*16 + l%16, k = step*32 + (l/16)*8 .. +8.
  constexpr int FR = MT * KSTEPS * 64 / 256;  // fragments per thread
  static_assert(MT * KSTEPS * 64 % 256 == 0, "fragments must split evenly over the workgroup");
  // Every load below is unconditional (clamped address, value selected
  // afterwards), so the waits can count them in issue order.
  // Fragment j of a thread is f = wave + 4j, so fragments j and j + KSTEPS/4
  // cover the same k (next row tile): the norm weight is loaded for the first
  // KSTEPS/4 only.
  static_assert(KSTEPS % 4 == 0, "fragments of one k repeat every KSTEPS/4");
  constexpr int FW = KSTEPS / 4;
  float4 xa[FR][2], wa[FW][2];
  const float* nwp = nsq ? nw : x;
#pragma unroll
  for (int j = 0; j < FR; ++j) {
    const int idx = tid + j * 256;
    const int fl = idx & 63, f = idx >> 6;
    const int mt = f / KSTEPS, s2 = f - mt * KSTEPS;
    const int row = mt * 16 + (fl & 15);
    const int kk = k0 + min(s2, nsteps - 1) * 32 + (fl >> 4) * 8;
    const float* xp = x + (int64_t)min(row, M - 1) * K + kk;
    xa[j][0] = *reinterpret_cast<const float4*>(xp);
    xa[j][1] = *reinterpret_cast<const float4*>(xp + 4);
    if (j < FW) {
      const float* wp = nwp + (nsq ? kk : 0);
      wa[j][0] = *reinterpret_cast<const float4*>(wp);
      wa[j][1] = *reinterpret_cast<const float4*>(wp + 4);
    }
  }
  // Fused RMSNorm: the row's f64 sum-of-squares slots, TPR threads per row,
  // each summing up to kSlotsPerThread consecutive slots (larger rows take
  // the loop below, after the weights).
  constexpr int TPR = MT == 1 ? 16 : MT == 2 ? 8 : 4, kSlotsPerThread = 8;
  const bool early_norm = nsq && nslots <= TPR * kSlotsPerThread;
  const int spt = (nslots + TPR - 1) / TPR;
  double sq[kSlotsPerThread];
  {
    const int row = tid / TPR, j = tid % TPR;
    // (x stands in as a readable address when there is nothing to load)
    const double* sp = early_norm ? nsq + (int64_t)min(row, M - 1) * nslots
                                  : reinterpret_cast<const double*>(x);
    const int last = early_norm ? nslots - 1 : 0;
#pragma unroll
    for (int i = 0; i < kSlotsPerThread; ++i) {
      const int slot = j * spt + i;
      const bool use = early_norm && row < M && i < spt && slot < nslots;
      const double v = sp[min(slot, last)];
      sq[i] = use ? v : 0.0;
    }
  }

  // 2. weight loads (clamped column and k-step: unconditional loads)
  //    in k-step order, so the MFMAs of step s wait only for its loads
  //    Row-major W: lane (l16, grp) reads W[col][k .. k+8) of its column.
  //    Packed W (wpacked, launch_gemv_pack): the workgroup's whole share is
  //    one contiguous chunk, in dispatch order, and a wave load one
  //    contiguous KiB.
  bf16x8 bw[KSTEPS][NT];
  const uint16_t* wrow[NT];
  int wstep;
  if (wpacked) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      wrow[nt] = w + (((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * (4 * NT) + wave * NT + nt) *
                         (KSTEPS * 512) + lane * 8;
    wstep = 512;
  } else {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      wrow[nt] = w + (int64_t)min(n0 + (wave * NT + nt) * 16 + l16, N - 1) * K + k0 + grp * 8;
    wstep = 32;
  }
#pragma unroll
  for (int s2 = 0; s2 < KSTEPS; ++s2)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      bw[s2][nt] = __builtin_bit_cast(
          bf16x8, *reinterpret_cast<const uint4*>(wrow[nt] + min(s2, nsteps - 1) * wstep));
  // nothing that waits for a load may be scheduled above this point
  __builtin_amdgcn_sched_barrier(0);

  // 3. row scales: scale = 1 / sqrt(mean(x^2) + eps), as rmsnorm_kernel
  //    computes it from the f64 sum; x * scale * weight below keeps rmsnorm's
  //    order of the two products.
  {
    // (computed unconditionally so the slot loads stay ahead of the weights)
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < kSlotsPerThread; ++i) t += sq[i];
    // TPR consecutive lanes hold one row: fixed-order butterfly
#pragma unroll
    for (int o = TPR / 2; o > 0; o >>= 1) t += __shfl_xor(t, o);
    const int row = tid / TPR;
    if (early_norm && tid % TPR == 0 && row < MT * 16)
      nscale[row] = row < M ? (float)(1.0 / sqrt(t / (double)K + (double)neps)) : 0.f;
  }
  if (nsq) {
    if (!early_norm && tid < MT * 16) {
      float sc = 0.f;
      if (tid < M) {
        double t = 0.0;
        for (int j = 0; j < nslots; ++j) t += nsq[(int64_t)tid * nslots + j];
        sc = (float)(1.0 / sqrt(t / (double)K + (double)neps));
      }
      nscale[tid] = sc;
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < FR; ++j) {
    const int idx = tid + j * 256;
    const int fl = idx & 63, f = idx >> 6;
    const int row = (f / KSTEPS) * 16 + (fl & 15);
    const bool live = row < M && (f % KSTEPS) < nsteps;
    float a[8] = {xa[j][0].x, xa[j][0].y, xa[j][0].z, xa[j][0].w,
                  xa[j][1].x, xa[j][1].y, xa[j][1].z, xa[j][1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = live ? a[e] : 0.f;
    if (nsq) {
      const float sc = row < M ? nscale[row] : 0.f;
      const float4* wj = wa[j % FW];
      const float wv[8] = {wj[0].x, wj[0].y, wj[0].z, wj[0].w,
                           wj[1].x, wj[1].y, wj[1].z, wj[1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = a[e] * sc * wv[e];
    }
    uint4 hv, lv;
    split2_trunc(a[0], a[1], hv.x, lv.x);
    split2_trunc(a[2], a[3], hv.y, lv.y);
    split2_trunc(a[4], a[5], hv.z, lv.z);
    split2_trunc(a[6], a[7], hv.w, lv.w);
    xs[0][idx] = hv;
    xs[1][idx] = lv;
  }
  __syncthreads();

  // 3. MFMAs
  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < KSTEPS; ++s2) {
    if (s2 < nsteps) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bf16x8 ahi = __builtin_bit_cast(bf16x8, xs[0][(mt * KSTEPS + s2) * 64 + lane]);
        const bf16x8 alo = __builtin_bit_cast(bf16x8, xs[1][(mt * KSTEPS + s2) * 64 + lane]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, bw[s2][nt], acc[mt][nt], 0, 0, 0);
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bw[s2][nt], acc[mt][nt], 0, 0, 0);
        }
      }
    }
  }

  // C fragment: acc[mt][nt][i] = C[mt*16 + 4*grp + i][n0 + (wave*NT + nt)*16 + l16]
  auto epilogue = [&](int row, int tile_col0, float v) {
    const int col = tile_col0 + l16;
    if (ep == (int)Epilogue::kSwiGLU) {
      const float u = __shfl_xor(v, 8);
      if (l16 < 8 && row < M && col < N)
        out[(int64_t)row * (N >> 1) + (tile_col0 >> 1) + l16] = v / (1.0f + __expf(-v)) * u;
    } else if (row < M && col < N) {
      float* op = out + (int64_t)row * N + col;
      if (ep == (int)Epilogue::kAccumulate)
        *op += v;
      else
        *op = bias ? v + bias[col] : v;
    }
  };
  if (kslices == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          epilogue(mt * 16 + 4 * grp + i, n0 + (wave * NT + nt) * 16, acc[mt][nt][i]);
    return;
  }
  // Partial tile of this K slice: partial[slice][tile][row][BN], rows < 16*MT.
  // gemm_gemv_reduce_kernel (or the consumer of deferred partials) sums the
  // slices in order; the kernel boundary orders the two.
  const int64_t tile_elems = (int64_t)MT * 16 * BN;
  float* mine = partial + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * tile_elems;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        mine[(mt * 16 + 4 * grp + i) * BN + (wave * NT + nt) * 16 + l16] = acc[mt][nt][i];
}

// Sums the K-slice partials of gemm_gemv_kernel in slice order and applies
// the epilogue.  One thread per (row, 16-column tile lane); SwiGLU pairs lanes
// 8 apart within a 16-column tile.
template <int MT, int NT>
__global__ void __launch_bounds__(256)
    gemm_gemv_reduce_kernel(const float* __restrict__ partial, int kslices, int n_tiles,
                            const float* __restrict__ bias, int M, int N, int ep,
                            float* __restrict__ out, double* __restrict__ sumsq) {
  constexpr int BN = 64 * NT;
  const int64_t tile_elems = (int64_t)MT * 16 * BN;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over n_tiles * M * BN
  const int64_t per_tile = (int64_t)M * BN;
  if (idx >= (int64_t)n_tiles * per_tile) return;  // whole 16-lane groups exit together
  const int tile = (int)(idx / per_tile);
  const int rem = (int)(idx - tile * per_tile);
  const int row = rem / BN, c = rem - row * BN;
  const int col = tile * BN + c;
  // The residual (accumulate) or bias (store) first, then the slices 8 (or
  // 24) at a time with every load of a group in flight, added in slice order (a slice
  // past the end adds +0, which leaves the sum unchanged).
  float pre = 0.f;
  if (col < N && ep == (int)Epilogue::kAccumulate)
    pre = out[(int64_t)row * N + col];
  else if (col < N && bias && ep == (int)Epilogue::kStore)
    pre = bias[col];
  const float* pp = partial + (int64_t)tile * tile_elems + row * BN + c;
  const int64_t slice_stride = (int64_t)n_tiles * tile_elems;
  float v = 0.f;
  auto sum_slices = [&](auto group) {
    constexpr int NG = decltype(group)::value;
    for (int ks0 = 0; ks0 < kslices; ks0 += NG) {
      float t[NG];
#pragma unroll
      for (int j = 0; j < NG; ++j)
        t[j] = ks0 + j < kslices ? pp[(ks0 + j) * slice_stride] : 0.f;
#pragma unroll
      for (int j = 0; j < NG; ++j) v += t[j];
    }
  };
  // up to 24 slices (config 4's down projection has 22) in one round of loads
  if (kslices > 8)
    sum_slices(std::integral_constant<int, 24>{});
  else
    sum_slices(std::integral_constant<int, 8>{});
  if (ep == (int)Epilogue::kSwiGLU) {
    const float u = __shfl_xor(v, 8);
    if ((c & 15) < 8 && col < N)
      out[(int64_t)row * (N >> 1) + ((col & ~15) >> 1) + (c & 7)] = v / (1.0f + __expf(-v)) * u;
  } else {
    float nv = 0.f;
    if (col < N) {
      if (ep == (int)Epilogue::kAccumulate)
        nv = pre + v;
      else
        nv = bias ? v + pre : v;
      out[(int64_t)row * N + col] = nv;
    }
    // Sum of squares of the updated row, one f64 slot per (row, 64 columns):
    // a wave covers 64 consecutive columns of one row.
    if (sumsq) {
      const double q = wave_sum_f64((double)nv * (double)nv);
      const int slot = col >> 6, nslots = (N + 63) >> 6;
      if ((threadIdx.x & 63) == 0 && slot < nslots) sumsq[(int64_t)row * nslots + slot] = q;
    }
  }
}

template <int MT, int NT, int UNR>
static void launch_skinny(int KW, dim3 grid, hipStream_t st, const float* x, const uint16_t* w,
                          const float* bias, int M, int N, int K, int ep, float* out) {
  switch (KW) {
    case 16:
      hipLaunchKernelGGL((gemm_skinny_kernel<MT, NT, 16, UNR>), grid, dim3(1024), 0, st, x, w,
                         bias, M, N, K, ep, out);
      break;
    case 8:
      hipLaunchKernelGGL((gemm_skinny_kernel<MT, NT, 8, UNR>), grid, dim3(512), 0, st, x, w,
                         bias, M, N, K, ep, out);
      break;
    case 4:
      hipLaunchKernelGGL((gemm_skinny_kernel<MT, NT, 4, UNR>), grid, dim3(256), 0, st, x, w,
                         bias, M, N, K, ep, out);
      break;
    default:
      hipLaunchKernelGGL((gemm_skinny_kernel<MT, NT, 1, UNR>), grid, dim3(64), 0, st, x, w,
                         bias, M, N, K, ep, out);
      break;
  }
}

namespace {
// Split-K decode GEMM geometry: NT x 64 columns per workgroup (BN) and KS
// k-steps of 32 per K slice; the slices are summed by gemm_gemv_reduce_kernel
// (or by the consumer of deferred partials).  Chosen per shape from M = 32
// measurements on the config-4 projections:
//   N <= 4096, K <= 4096 (QKV, O)  NT 1, KS 8 (O: 32 x 8 workgroups)
//     partials left to the consumer (QKV into RoPE): NT 2, KS 8; narrower
//     tiles only repeat the norm and activation staging (7.1 -> 9.9 us in the
//     decode step)
//   N > 4096 (gate/up, LM head)    NT 2, KS 8
//   K > 4096 (down)                NT 1, KS 8 (704 workgroups at 3 per CU;
//     NT 2, KS 16 had 176 at one per CU: decode step 1.690 -> 1.676 ms)
// Few column tiles want narrow tiles (more workgroups).  ORION_GEMV_NT /
// ORION_GEMV_KS override every shape (measurement knobs; NT in {1, 2, 4}, KS
// in {4, 8, 16}).
int gemv_knob(const char* name, int a, int b, int c) {
  const char* e = getenv(name);
  const int v = e ? atoi(e) : 0;
  return (v == a || v == b || v == c) ? v : 0;
}
struct GemvShape {
  int mt, nt, ks, n_tiles, kslices;
  size_t ws_bytes;
};
GemvShape gemv_shape(int64_t M, int64_t N, int64_t K, bool deferred = false) {
  static const int knob_nt = gemv_knob("ORION_GEMV_NT", 1, 2, 4);
  static const int knob_ks = gemv_knob("ORION_GEMV_KS", 4, 8, 16);
  GemvShape g;
  g.mt = (int)((M + 15) / 16);
  if (K > 4096) {
    g.nt = 1, g.ks = 8;
  } else if (N > 4096) {
    g.nt = 2, g.ks = 8;
  } else if (deferred) {
    g.nt = 2, g.ks = 8;
  } else {
    g.nt = 1, g.ks = 8;
  }
  if (knob_nt) g.nt = knob_nt;
  if (knob_ks) g.ks = knob_ks;
  // ORION_GEMV_GEOM="defer:NT:KS,longk:NT:KS,wide:NT:KS,other:NT:KS,head:NT:KS"
  // (any subset): per-group override (measurement knob; NT in {1, 2, 4}, KS
  // in {4, 8, 16}); "head" (N > 16384, an LM head) refines "wide".
  static const std::array<std::pair<int, int>, 5> geom = [] {
    std::array<std::pair<int, int>, 5> r{};
    const char* e = getenv("ORION_GEMV_GEOM");
    if (!e) return r;
    const char* names[5] = {"defer", "longk", "wide", "other", "head"};
    for (int i = 0; i < 5; ++i) {
      const char* p = strstr(e, names[i]);
      int nt = 0, ks = 0;
      if (p && sscanf(p + strlen(names[i]), ":%d:%d", &nt, &ks) == 2 &&
          (nt == 1 || nt == 2 || nt == 4) && (ks == 4 || ks == 8 || ks == 16))
        r[i] = {nt, ks};
    }
    return r;
  }();
  {
    int grp = deferred ? 0 : K > 4096 ? 1 : N > 4096 ? 2 : 3;
    if (grp == 2 && N > 16384 && geom[4].first) grp = 4;
    if (geom[grp].first) g.nt = geom[grp].first, g.ks = geom[grp].second;
  }
  g.n_tiles = (int)((N + 64 * g.nt - 1) / (64 * g.nt));
  g.kslices = (int)((K + g.ks * 32 - 1) / (g.ks * 32));
  g.ws_bytes = g.kslices > 1 ? (size_t)g.kslices * g.n_tiles * g.mt * 16 * 64 * g.nt * 4 : 0;
  return g;
}
template <int MT, int NT, int KS>
void launch_gemv_t(const GemvShape& g, hipStream_t st, const float* x, const uint16_t* w,
                   const float* bias, int M, int N, int K, int ep, float* out,
                   const GemmScratch* sc, const GemmFuse& f, bool reduce) {
  hipLaunchKernelGGL((gemm_gemv_kernel<MT, NT, KS>),
                     dim3((unsigned)g.n_tiles, (unsigned)g.kslices), dim3(256), 0, st, x,
                     f.w_packed ? f.w_packed : w, bias,
                     M, N, K, ep, out, sc ? sc->ws : nullptr, f.norm_sumsq, f.norm_slots,
                     f.norm_weight, f.norm_eps, f.w_packed ? 1 : 0);
  if (g.kslices > 1 && reduce) {
    const int64_t threads = (int64_t)g.n_tiles * M * 64 * NT;
    hipLaunchKernelGGL((gemm_gemv_reduce_kernel<MT, NT>),
                       dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, sc->ws,
                       g.kslices, g.n_tiles, bias, M, N, ep, out, f.sumsq_out);
  }
}
template <int MT, int NT>
void launch_gemv_nt(const GemvShape& g, hipStream_t st, const float* x, const uint16_t* w,
                    const float* bias, int M, int N, int K, int ep, float* out,
                    const GemmScratch* sc, const GemmFuse& f, bool reduce) {
  if (g.ks == 4)
    launch_gemv_t<MT, NT, 4>(g, st, x, w, bias, M, N, K, ep, out, sc, f, reduce);
  else if (g.ks == 16)
    launch_gemv_t<MT, NT, 16>(g, st, x, w, bias, M, N, K, ep, out, sc, f, reduce);
  else
    launch_gemv_t<MT, NT, 8>(g, st, x, w, bias, M, N, K, ep, out, sc, f, reduce);
}
template <int MT>
void launch_gemv(const GemvShape& g, hipStream_t st, const float* x, const uint16_t* w,
                 const float* bias, int M, int N, int K, int ep, float* out,
                 const GemmScratch* sc, const GemmFuse& f, bool reduce) {
  if (g.nt == 1)
    launch_gemv_nt<MT, 1>(g, st, x, w, bias, M, N, K, ep, out, sc, f, reduce);
  else if (g.nt == 4)
    launch_gemv_nt<MT, 4>(g, st, x, w, bias, M, N, K, ep, out, sc, f, reduce);
  else
    launch_gemv_nt<MT, 2>(g, st, x, w, bias, M, N, K, ep, out, sc, f, reduce);
}
}  // namespace

// One thread per 16-byte unit of the packed layout: unit u = (chunk, step,
// lane) with chunk = ((slice * n_tiles + tile) * 4 + wave) * NT + nt, i.e.
// the order in which gemm_gemv_kernel's workgroups (x = column tile, y = K
// slice), waves, column tiles, k-steps and lanes read it.  Columns past N and
// k past K are zero.
__global__ void __launch_bounds__(256)
    gemv_pack_kernel(const uint16_t* __restrict__ w, int N, int K, int nt, int ks, int n_tiles,
                     int64_t units, uint4* __restrict__ out) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const int lane = (int)(u & 63);
  const int64_t q = u >> 6;
  const int s = (int)(q % ks);
  const int64_t chunk = q / ks;
  const int nti = (int)(chunk % nt);
  const int wave = (int)((chunk / nt) & 3);
  const int64_t wg = chunk / (4 * nt);
  const int bx = (int)(wg % n_tiles), by = (int)(wg / n_tiles);
  const int col = bx * 64 * nt + (wave * nt + nti) * 16 + (lane & 15);
  const int k = by * ks * 32 + s * 32 + (lane >> 4) * 8;
  uint4 v = uint4{0u, 0u, 0u, 0u};
  if (col < N && k < K) v = *reinterpret_cast<const uint4*>(w + (int64_t)col * K + k);
  out[u] = v;
}

// The inverse of gemv_pack_kernel: unit u goes back to W[col][k .. k+8).
__global__ void __launch_bounds__(256)
    gemv_unpack_kernel(const uint4* __restrict__ in, int N, int K, int nt, int ks, int n_tiles,
                       int64_t units, uint16_t* __restrict__ w) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const int lane = (int)(u & 63);
  const int64_t q = u >> 6;
  const int s = (int)(q % ks);
  const int64_t chunk = q / ks;
  const int nti = (int)(chunk % nt);
  const int wave = (int)((chunk / nt) & 3);
  const int64_t wg = chunk / (4 * nt);
  const int bx = (int)(wg % n_tiles), by = (int)(wg / n_tiles);
  const int col = bx * 64 * nt + (wave * nt + nti) * 16 + (lane & 15);
  const int k = by * ks * 32 + s * 32 + (lane >> 4) * 8;
  if (col < N && k < K) *reinterpret_cast<uint4*>(w + (int64_t)col * K + k) = in[u];
}

size_t gemv_packed_bytes(int64_t N, int64_t K, bool deferred) {
  if (K % 32 != 0 || K <= 0 || N <= 0) return 0;
  const GemvShape g = gemv_shape(1, N, K, deferred);
  return (size_t)g.n_tiles * g.kslices * 4 * g.nt * g.ks * 1024;
}

hipError_t launch_gemv_pack(hipStream_t st, const uint16_t* w, int64_t N, int64_t K,
                            bool deferred, uint16_t* out) {
  if (K % 32 != 0 || K <= 0 || N <= 0 || N > INT32_MAX || K > INT32_MAX)
    return hipErrorInvalidValue;
  const GemvShape g = gemv_shape(1, N, K, deferred);
  const int64_t units = (int64_t)gemv_packed_bytes(N, K, deferred) / 16;
  hipLaunchKernelGGL(gemv_pack_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, st, w,
                     (int)N, (int)K, g.nt, g.ks, g.n_tiles, units, reinterpret_cast<uint4*>(out));
  return hipGetLastError();
}

hipError_t launch_gemv_unpack(hipStream_t st, const uint16_t* packed, int64_t N, int64_t K,
                              bool deferred, uint16_t* w) {
  if (K % 32 != 0 || K <= 0 || N <= 0 || N > INT32_MAX || K > INT32_MAX)
    return hipErrorInvalidValue;
  const GemvShape g = gemv_shape(1, N, K, deferred);
  const int64_t units = (int64_t)gemv_packed_bytes(N, K, deferred) / 16;
  hipLaunchKernelGGL(gemv_unpack_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<const uint4*>(packed), (int)N, (int)K, g.nt, g.ks,
                     g.n_tiles, units, w);
  return hipGetLastError();
}

bool gemm_splitk_fusable(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 64 || K % 32 != 0 || K > INT32_MAX || N < 1 || N > INT32_MAX) return false;
  const GemvShape g = gemv_shape(M, N, K);
  return g.kslices > 1 && g.kslices <= 65535;
}

int gemm_sumsq_slots(int64_t N) {
  return (int)((N + 63) / 64);
}

// K splits of the LDS-tiled GEMM.  A call with fewer output tiles than CUs
// leaves CUs idle, so its K is split until the tiles x splits reach
// kTiledFill workgroups, up to 8 splits of at least 16 k-steps each; the
// splits' raw sums go to the scratch and gemm_tiled_reduce_kernel adds them.
// (Measured on config 5: the 16-tile LM head went 108 -> 28 us with 4
// splits; splitting the 504-tile O and down projections saved about what
// their 31 us reduce launches cost, so they stay whole.)  Not for the SwiGLU
// epilogue (its column pairs sit in one tile).  ORION_GEMM_TILED_SPLIT=n
// forces n (measurement knob, read per call).
// A long K (>= 256 k-steps) with fewer tiles than the resident slots (3
// workgroups x 256 CUs) is also split, into up to 2 x slots workgroups of at
// least 64 k-steps: config 5's down projection (K 18944, 504 tiles) went
// 664-697 -> 585 us + a 37 us reduce with 3 splits, while shorter-K calls
// with the same tile count (QKV, O) gained nothing.  These long-K splits are
// preferred, not required: a caller whose scratch cannot hold them (the
// no-allocation entry point) runs the required count.
namespace {
constexpr int64_t kTiledFill = 256;
constexpr int64_t kTiledSlots = 768;
int tiled_ksplits(int64_t M, int64_t N, int64_t K, bool preferred = true) {
  const int64_t tiles = ((N + kTN - 1) / kTN) * ((M + kTM - 1) / kTM);
  const int64_t ksteps = K / kTK;
  if (const char* e = getenv("ORION_GEMM_TILED_SPLIT")) {
    const int64_t f = atoll(e);
    return (int)std::max<int64_t>(1, std::min<int64_t>(f, std::max<int64_t>(1, ksteps / 4)));
  }
  int s = 1;
  while (s < 8 && tiles * s < kTiledFill && ksteps / (2 * s) >= 16) s *= 2;
  if (preferred && tiles < kTiledSlots && ksteps >= 256) {
    int64_t p = std::min<int64_t>(8, 2 * kTiledSlots / tiles);
    while (p > 1 && ksteps / p < 64) --p;
    s = std::max<int>(s, (int)p);
  }
  return s;
}
}  // namespace

void gemm_scratch_need(int64_t M, int64_t N, int64_t K, size_t* ws_bytes, bool preferred) {
  *ws_bytes = 0;
  if (M < 1 || K % 32 != 0) return;
  if (M > 64) {
    const int s = tiled_ksplits(M, N, K, preferred);
    if (s > 1) *ws_bytes = (size_t)s * (size_t)M * (size_t)N * sizeof(float);
    return;
  }
  const GemvShape g = gemv_shape(M, N, K), gd = gemv_shape(M, N, K, true);
  *ws_bytes = std::max(g.ws_bytes, gd.ws_bytes);
}

hipError_t launch_gemm(hipStream_t st, const float* x, const uint16_t* w, const float* bias,
                       int64_t M, int64_t N, int64_t K, Epilogue ep, float* out,
                       const GemmScratch* scratch, const GemmFuse* fuse) {
  const GemmFuse f = fuse ? *fuse : GemmFuse{};
  if (f.defer) *f.defer = GemmPartials{};
  const bool needs_splitk = f.norm_sumsq || f.sumsq_out;
  if (needs_splitk && (!gemm_splitk_fusable(M, N, K) || (f.sumsq_out && ep != Epilogue::kAccumulate) ||
                       (f.norm_sumsq && (!f.norm_weight || f.norm_slots < 1))))
    return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  if (K % 32 != 0 || K == 0) return hipErrorInvalidValue;
  if (ep == Epilogue::kSwiGLU && N % 16 != 0) return hipErrorInvalidValue;
  // ORION_GEMM_TILED_MIN_M: smallest M that takes the LDS-tiled kernel.
  static const int64_t tiled_min_m = [] {
    const char* e = getenv("ORION_GEMM_TILED_MIN_M");
    return e ? (int64_t)atoll(e) : (int64_t)256;
  }();
  // split-layout activations exist only for the LDS-tiled kernel
  if ((f.x_hilo || f.out_hilo) && (M <= 64 || (M < tiled_min_m && !f.w_packed)))
    return hipErrorInvalidValue;
  // Decode-shaped M: split-K weight streaming (needs the scratch when K spans
  // several slices).
  if (M <= 64 && N <= INT32_MAX && K <= INT32_MAX) {
    // A consumer that takes the unreduced partials gets them (no reduce
    // launch); only for the store epilogue.
    const bool wants_defer = f.defer && ep == Epilogue::kStore && !f.sumsq_out;
    const GemvShape g = gemv_shape(M, N, K, wants_defer);
    const bool fits = g.kslices == 1 || (scratch && scratch->ws_bytes >= g.ws_bytes);
    if (needs_splitk && !fits) return hipErrorInvalidValue;
    if (fits && g.kslices <= 65535) {
      const int m = (int)M, n = (int)N, k = (int)K, e = (int)ep;
      const bool deferred = wants_defer && g.kslices > 1;
      if (deferred) {
        f.defer->ws = scratch->ws;
        f.defer->kslices = g.kslices;
        f.defer->n_tiles = g.n_tiles;
        f.defer->bn = 64 * g.nt;
        f.defer->tile_rows = g.mt * 16;
        f.defer->bias = bias;
      }
      switch (g.mt) {
        case 1: launch_gemv<1>(g, st, x, w, bias, m, n, k, e, out, scratch, f, !deferred); break;
        case 2: launch_gemv<2>(g, st, x, w, bias, m, n, k, e, out, scratch, f, !deferred); break;
        case 3: launch_gemv<3>(g, st, x, w, bias, m, n, k, e, out, scratch, f, !deferred); break;
        default: launch_gemv<4>(g, st, x, w, bias, m, n, k, e, out, scratch, f, !deferred); break;
      }
      return hipGetLastError();
    }
  }
  // The LDS-tiled kernel takes every larger M, and every M > 64 when only the
  // packed copy exists (the skinny kernel reads row-major W).
  if (M >= tiled_min_m || f.w_packed) {
    if (M > (int64_t)65535 * kTM || N > INT32_MAX || K > INT32_MAX) return hipErrorInvalidValue;
    PackedGeom pk;
    if (f.w_packed) {
      const GemvShape gp = gemv_shape(1, N, K, f.w_packed_deferred);
      pk.nt = gp.nt;
      pk.ks = gp.ks;
      pk.n_tiles = gp.n_tiles;
    }
    // 128 x 256 workgroup tiles (64 x 128 per wave, 2 workgroups per CU) for
    // wide outputs: per MFMA a third less LDS traffic (copies + fragment
    // reads) than 128 x 128 tiles at 3 per CU.  Measured at config 4's prefill
    // shapes: gate/up (N 11264) 649-673 -> 692-700 TFLOP/s; QKV (2560) even,
    // down (2048) -3 %, O (2048) -13 % (too few tiles for 2 per CU).
    // ORION_GEMM_WIDE=0/1 forces the choice (measurement knob, read per call).
    const char* wide_env = getenv("ORION_GEMM_WIDE");
    const bool wide = wide_env ? wide_env[0] == '1' : N >= 8192;
    const int tn = wide ? 2 * kTN : kTN;
    dim3 grid((unsigned)((N + tn - 1) / tn), (unsigned)((M + kTM - 1) / kTM));
    // XCD-aware grouped tile order with groups of 4 m tiles (measured at the
    // config-4 prefill shapes against the row-major grid: QKV 529 -> 563, O
    // 405 -> 443, down 513 -> 536 TFLOP/s, gate/up unchanged; groups of 8 and
    // 16 gained less).  ORION_GEMM_GM=g overrides the group (0: the 2D
    // row-major grid; measurement knob, read per call).
    int gm = 4;
    if (const char* e = getenv("ORION_GEMM_GM")) gm = std::max(0, atoi(e));
    if (gm > 0) {
      const int64_t total = (int64_t)grid.x * grid.y;
      grid = dim3((unsigned)(((total + 7) / 8) * 8), 1);
    }
    // K splits (tiled_ksplits), when the scratch holds their sums
    const size_t avail = scratch ? scratch->ws_bytes : 0;
    auto fits = [&](int s) { return (size_t)s * (size_t)M * (size_t)N * sizeof(float) <= avail; };
    int splits = ep == Epilogue::kSwiGLU ? 1 : tiled_ksplits(M, N, K);
    if (splits > 1 && !fits(splits)) splits = tiled_ksplits(M, N, K, false);
    if (splits > 1 && !fits(splits)) splits = 1;
    const int ksteps = (int)(K / kTK), kspan = (ksteps + splits - 1) / splits;
    // every split must start below K: with kspan rounded up, ceil(ksteps /
    // kspan) splits cover K (a forced count such as 16 splits of 66 k-steps
    // would otherwise leave splits 14 and 15 starting past the last row)
    splits = (ksteps + kspan - 1) / kspan;
    grid.z = (unsigned)splits;
    float* partial = splits > 1 ? scratch->ws : nullptr;
    // ORION_GEMM_ACT=bf16 rounds the activations to bf16 (one MFMA per
    // fragment) instead of the hi/lo pair (measurement knob, read per call).
    const char* act = getenv("ORION_GEMM_ACT");
    const bool hilo = !(act && act[0] == 'b');
    if (f.x_hilo && !hilo) return hipErrorInvalidValue;
    auto kern = f.x_hilo ? (wide ? gemm_tiled_kernel<true, 8, true> : gemm_tiled_kernel<true, 4, true>)
                : wide   ? (hilo ? gemm_tiled_kernel<true, 8> : gemm_tiled_kernel<false, 8>)
                         : (hilo ? gemm_tiled_kernel<true, 4> : gemm_tiled_kernel<false, 4>);
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, x, f.w_packed ? f.w_packed : w, bias,
                       (int)M, (int)N, (int)K, (int)ep, out, pk, gm, kspan, partial,
                       f.out_hilo && ep == Epilogue::kSwiGLU);
    if (splits > 1) {
      const int64_t total = M * N;
      const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
      hipLaunchKernelGGL(gemm_tiled_reduce_kernel, dim3(blocks), dim3(256), 0, st, partial,
                         splits, M, N, bias, (int)ep, out);
    }
    return hipGetLastError();
  }
  // Rows per tile (MT x 16) and columns per tile (NT x 16): wide column tiles
  // only when there are many of them.  Waves per tile (KW, splitting K): as
  // many as it takes for each wave's whole k-range (<= UNR steps of 32) to be
  // in flight in one round, up to 16; the LDS reduction buffer
  // KW x 16MT x (16NT+1) floats stays <= 64 KiB.
  const int MT = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  const int NT = (MT <= 2 && N >= 8192) ? 4 : (N > 4096 ? 2 : 1);
  constexpr int UNR = 4;
  const int64_t ksteps = K / 32;
  const int kw_cap = (MT * NT <= 4) ? 16 : 8;
  int KW = 1;
  while (KW < kw_cap && (ksteps + KW - 1) / KW > UNR) KW <<= 1;
  if (KW == 2) KW = 4;
  const int BN = 16 * NT, BM = 16 * MT;
  dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  const int m = (int)M, n = (int)N, k = (int)K, e = (int)ep;
  if (MT == 1) {
    if (NT == 4) launch_skinny<1, 4, UNR>(KW, grid, st, x, w, bias, m, n, k, e, out);
    else if (NT == 2) launch_skinny<1, 2, UNR>(KW, grid, st, x, w, bias, m, n, k, e, out);
    else launch_skinny<1, 1, UNR>(KW, grid, st, x, w, bias, m, n, k, e, out);
  } else if (MT == 2) {
    if (NT == 4) launch_skinny<2, 4, UNR>(KW, grid, st, x, w, bias, m, n, k, e, out);
    else if (NT == 2) launch_skinny<2, 2, UNR>(KW, grid, st, x, w, bias, m, n, k, e, out);
    else launch_skinny<2, 1, UNR>(KW, grid, st, x, w, bias, m, n, k, e, out);
  } else {
    if (NT == 2) launch_skinny<4, 2, UNR>(KW, grid, st, x, w, bias, m, n, k, e, out);
    else launch_skinny<4, 1, UNR>(KW, grid, st, x, w, bias, m, n, k, e, out);
  }
  return hipGetLastError();
}

}  // namespace orion

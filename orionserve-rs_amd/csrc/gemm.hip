// Projection GEMMs on bf16 MFMA for gfx950: out[M,N] = x[M,K] . W[N,K]^T.
//
// Restates the reference's `linear` (crates/orion-models/src/tensor.rs:96-130):
// W keeps the HF layout [out_features, in_features] (row-major, K contiguous),
// which is exactly the MFMA B-operand layout: a lane loads 8 consecutive k of
// one output column with one 16-byte load, straight from HBM into registers.
//
// Activations arrive in f32.  Each 8-element A fragment is split on the fly
// into hi = bf16(x) and lo = bf16(x - hi) and both are multiplied against the
// bf16 weight (two MFMAs, f32 accumulation), so the product carries ~16
// mantissa bits of x instead of 8.  Weights are exact (bf16 checkpoints widen
// exactly in the reference loader), so the only departure from the reference's
// f32 arithmetic is summation order plus a ~2^-17 relative term per product.
//
// Shape of the launch (decode-oriented, weight-streaming):
//   workgroup = 4 waves, tile = 64 rows x (16*NT) columns, the four waves
//   split K into contiguous quarters and reduce through LDS.  Every weight
//   element is read from HBM once per 64-row block of x.  The epilogue fuses
//   the bias add, the residual accumulate (transformer.rs:328-332, :345) or
//   SwiGLU (tensor.rs:175-189) on gate/up rows interleaved in groups of 8.
#include "common.hpp"
#include "kernels.hpp"

namespace orion {

__device__ inline bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ inline void split8(const float (&a)[8], bf16x8& hi, bf16x8& lo) {
  uint16_t h[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) split_bf16(a[i], h[i], l[i]);
  uint4 hv, lv;
  hv.x = h[0] | ((uint32_t)h[1] << 16);
  hv.y = h[2] | ((uint32_t)h[3] << 16);
  hv.z = h[4] | ((uint32_t)h[5] << 16);
  hv.w = h[6] | ((uint32_t)h[7] << 16);
  lv.x = l[0] | ((uint32_t)l[1] << 16);
  lv.y = l[2] | ((uint32_t)l[3] << 16);
  lv.z = l[4] | ((uint32_t)l[5] << 16);
  lv.w = l[6] | ((uint32_t)l[7] << 16);
  hi = as_bf16x8(hv);
  lo = as_bf16x8(lv);
}

template <int NT>
__global__ void __launch_bounds__(256)
    gemm_skinny_kernel(const float* __restrict__ x, const uint16_t* __restrict__ w,
                       const float* __restrict__ bias, int M, int N, int K, int ep,
                       float* __restrict__ out) {
  constexpr int BN = 16 * NT;
  __shared__ float red[4][64][BN + 1];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 64;
  const int n0 = blockIdx.x * BN;
  const int mt_count = min(4, (M - m0 + 15) >> 4);
  const int ksteps = K >> 5;
  const int ks0 = wave * ksteps / 4;
  const int ks1 = (wave + 1) * ksteps / 4;
  const int lr = lane & 15;
  const int lk = (lane >> 4) * 8;

  const uint16_t* wrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = min(n0 + nt * 16 + lr, N - 1);
    wrow[nt] = w + (int64_t)n * K + lk;
  }
  const float* xrow[4];
  bool xvalid[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int m = m0 + mt * 16 + lr;
    xvalid[mt] = m < M;
    xrow[mt] = x + (int64_t)min(m, M - 1) * K + lk;
  }

  f32x4 acc[4][NT];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int ks = ks0; ks < ks1; ++ks) {
    const int k = ks << 5;
    bf16x8 b[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) b[nt] = as_bf16x8(*reinterpret_cast<const uint4*>(wrow[nt] + k));
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (mt < mt_count) {
        float a[8];
        if (xvalid[mt]) {
          const float4 a0 = *reinterpret_cast<const float4*>(xrow[mt] + k);
          const float4 a1 = *reinterpret_cast<const float4*>(xrow[mt] + k + 4);
          a[0] = a0.x; a[1] = a0.y; a[2] = a0.z; a[3] = a0.w;
          a[4] = a1.x; a[5] = a1.y; a[6] = a1.z; a[7] = a1.w;
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) a[i] = 0.f;
        }
        bf16x8 ahi, alo;
        split8(a, ahi, alo);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, b[nt], acc[mt][nt], 0, 0, 0);
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, b[nt], acc[mt][nt], 0, 0, 0);
        }
      }
    }
  }

  // C fragment layout: lane holds rows 4*(lane/16) + i, column lane % 16.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    if (mt < mt_count) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][mt * 16 + (lane >> 4) * 4 + i][nt * 16 + lr] = acc[mt][nt][i];
    }
  }
  __syncthreads();

  const int rows = min(64, M - m0);
  if (ep == (int)Epilogue::kSwiGLU) {
    // Tile columns nt*16 + [0,8) are gate rows, nt*16 + [8,16) the matching up rows.
    const int half_n = N >> 1;
    for (int idx = threadIdx.x; idx < rows * NT * 8; idx += 256) {
      const int r = idx / (NT * 8);
      const int cc = idx - r * (NT * 8);
      const int nt = cc >> 3, j = cc & 7;
      const int gcol = n0 + nt * 16 + j;
      if (gcol >= N) continue;
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) {
        g += red[wv][r][nt * 16 + j];
        u += red[wv][r][nt * 16 + 8 + j];
      }
      const float act = g / (1.0f + __expf(-g)) * u;
      out[(int64_t)(m0 + r) * half_n + (n0 >> 1) + nt * 8 + j] = act;
    }
  } else {
    for (int idx = threadIdx.x; idx < rows * BN; idx += 256) {
      const int r = idx / BN;
      const int cc = idx - r * BN;
      const int col = n0 + cc;
      if (col >= N) continue;
      float v = red[0][r][cc] + red[1][r][cc] + red[2][r][cc] + red[3][r][cc];
      float* op = out + (int64_t)(m0 + r) * N + col;
      if (ep == (int)Epilogue::kAccumulate)
        *op += v;
      else
        *op = bias ? v + bias[col] : v;
    }
  }
}

hipError_t launch_gemm(hipStream_t st, const float* x, const uint16_t* w, const float* bias,
                       int64_t M, int64_t N, int64_t K, Epilogue ep, float* out) {
  if (M == 0 || N == 0) return hipSuccess;
  if (K % 32 != 0 || K == 0) return hipErrorInvalidValue;
  if (ep == Epilogue::kSwiGLU && N % 16 != 0) return hipErrorInvalidValue;
  int NT = 1;
  if (N / 64 >= 512) NT = 4;
  else if (N / 32 >= 512) NT = 2;
  const int BN = 16 * NT;
  dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + 63) / 64));
  switch (NT) {
    case 1:
      hipLaunchKernelGGL(gemm_skinny_kernel<1>, grid, dim3(256), 0, st, x, w, bias, (int)M, (int)N,
                         (int)K, (int)ep, out);
      break;
    case 2:
      hipLaunchKernelGGL(gemm_skinny_kernel<2>, grid, dim3(256), 0, st, x, w, bias, (int)M, (int)N,
                         (int)K, (int)ep, out);
      break;
    default:
      hipLaunchKernelGGL(gemm_skinny_kernel<4>, grid, dim3(256), 0, st, x, w, bias, (int)M, (int)N,
                         (int)K, (int)ep, out);
      break;
  }
  return hipGetLastError();
}

}  // namespace orion

// Row-wise and elementwise kernels around the attention/GEMM hot path:
// embedding gather, RMSNorm, RoPE fused with the paged KV write (slot mapping),
// SwiGLU, greedy argmax, weight conversion and synthetic initialisation.
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace orion {

// TransformerModel::embed (transformer.rs:208-223): row gather, bf16 -> f32.
// Token ids are range-checked on the host before launch.  With `sumsq`, also
// the row's f64 sums of squares, one slot per 64 consecutive columns (the
// slots the residual GEMMs leave for the fused RMSNorm of the next GEMM), so
// layer 0's QKV GEMM applies its norm the same way.  Workgroup (row, y) takes
// 64-column chunks 4y .. 4y + 3, one per wave (one load and at most one
// reduction per wave).
__global__ void __launch_bounds__(256)
    embed_kernel(const uint32_t* __restrict__ tokens, const uint16_t* __restrict__ table,
                 int64_t hidden, float* __restrict__ out, double* __restrict__ sumsq) {
  const int64_t row = blockIdx.x;
  const uint16_t* src = table + (int64_t)tokens[row] * hidden;
  float* dst = out + row * hidden;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nslots = (hidden + 63) >> 6;
  for (int64_t c = (int64_t)blockIdx.y * 4 + wave; c < nslots; c += (int64_t)gridDim.y * 4) {
    const int64_t i = c * 64 + lane;
    const float v = i < hidden ? bf16_to_f32(src[i]) : 0.f;
    if (i < hidden) dst[i] = v;
    if (sumsq) {
      const double q = wave_sum_f64((double)v * (double)v);
      if (lane == 0) sumsq[row * nslots + c] = q;
    }
  }
}

hipError_t launch_embed(hipStream_t st, const uint32_t* tokens, int64_t n, const uint16_t* table,
                        int64_t hidden, float* out, double* sumsq) {
  if (n == 0) return hipSuccess;
  const int64_t nslots = (hidden + 63) >> 6;
  const unsigned gy = (unsigned)std::min<int64_t>((nslots + 3) / 4, 64);
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)n, gy), dim3(256), 0, st, tokens, table, hidden,
                     out, sumsq);
  return hipGetLastError();
}

// rms_norm (tensor.rs:143-163): sum of squares in f64 as the reference does,
// scale = (f32)(1 / sqrt(sum/cols + eps)), v * scale * w in f32.
// One workgroup per output row; `row_index` optionally gathers input rows
// (the last row of each sequence before the LM head, transformer.rs:410-428).
__global__ void __launch_bounds__(256)
    rmsnorm_kernel(const float* __restrict__ x, const int32_t* __restrict__ row_index,
                   const float* __restrict__ weight, int64_t cols, float eps,
                   float* __restrict__ out, bool hilo) {
#pragma clang fp contract(off)
  __shared__ double part[4];
  const int64_t orow = blockIdx.x;
  const int64_t irow = row_index ? row_index[orow] : orow;
  const float* xr = x + irow * cols;
  float* orow_p = out + orow * cols;
  // Fast path: the row in registers (float4 loads, up to 8 per thread), read
  // once; the output is the same f32 expression as the general path.
  constexpr int kMaxV = 8;
  if ((cols & 3) == 0 && cols <= 1024 * kMaxV &&
      ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(orow_p) |
        reinterpret_cast<uintptr_t>(weight)) & 15) == 0) {
    const int n4 = (int)(cols >> 2);
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    float4 v[kMaxV];
#pragma unroll
    for (int j = 0; j < kMaxV; ++j) {
      const int i = (int)threadIdx.x + 256 * j;
      v[j] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kMaxV; ++j)
      s += (double)v[j].x * (double)v[j].x + (double)v[j].y * (double)v[j].y +
           (double)v[j].z * (double)v[j].z + (double)v[j].w * (double)v[j].w;
    s = wave_sum_f64(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const double total = part[0] + part[1] + part[2] + part[3];
    const float scale = (float)(1.0 / sqrt(total / (double)cols + (double)eps));
    const float4* w4 = reinterpret_cast<const float4*>(weight);
    float4* o4 = reinterpret_cast<float4*>(orow_p);
#pragma unroll
    for (int j = 0; j < kMaxV; ++j) {
      const int i = (int)threadIdx.x + 256 * j;
      if (i < n4) {
        const float4 w = w4[i];
        const float4 y = make_float4(v[j].x * scale * w.x, v[j].y * scale * w.y,
                                     v[j].z * scale * w.z, v[j].w * scale * w.w);
        if (hilo) {
          // float4 i is half i & 1 of group i >> 1: its 4 hi and 4 lo values
          uint16_t h[4], l[4];
          split1_trunc(y.x, h[0], l[0]);
          split1_trunc(y.y, h[1], l[1]);
          split1_trunc(y.z, h[2], l[2]);
          split1_trunc(y.w, h[3], l[3]);
          uint2* g = reinterpret_cast<uint2*>(orow_p) + (i >> 1) * 4 + (i & 1);
          g[0] = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
          g[2] = make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
        } else {
          o4[i] = y;
        }
      }
    }
    return;
  }
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < cols; i += 256) {
    const double v = (double)xr[i];
    s += v * v;
  }
  s = wave_sum_f64(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const double total = part[0] + part[1] + part[2] + part[3];
  const float scale = (float)(1.0 / sqrt(total / (double)cols + (double)eps));
  if (hilo) {
    uint16_t* o16 = reinterpret_cast<uint16_t*>(orow_p);
    for (int64_t i = threadIdx.x; i < cols; i += 256) {
      uint16_t h, l;
      split1_trunc(xr[i] * scale * weight[i], h, l);
      o16[(i >> 3) * 16 + (i & 7)] = h;
      o16[(i >> 3) * 16 + 8 + (i & 7)] = l;
    }
    return;
  }
  for (int64_t i = threadIdx.x; i < cols; i += 256) orow_p[i] = xr[i] * scale * weight[i];
}

hipError_t launch_rmsnorm(hipStream_t st, const float* x, const int32_t* row_index,
                          const float* weight, int64_t rows, int64_t cols, float eps, float* out,
                          bool hilo) {
  if (rows == 0) return hipSuccess;
  if (hilo && cols % 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, st, x, row_index, weight,
                     cols, eps, out, hilo);
  return hipGetLastError();
}

// RoPE (apply_rope, tensor.rs:283-298: rotate-half, i paired with i + d/2) on
// every Q head and K head of a row (transformer.rs:255-279), then the KV write
// for that row (transformer.rs:283-297) at its slot: block = table[pos / bs],
// slot = pos % bs (`locate`, attention.rs:182-186; the slot mapping of
// transformer.rs:371-387).  Positions and table lengths are checked on the host.
template <typename T>
__device__ inline void store_kv(T* p, float v);
template <>
__device__ inline void store_kv<float>(float* p, float v) { *p = v; }
template <>
__device__ inline void store_kv<uint16_t>(uint16_t* p, float v) { *p = f32_to_bf16(v); }

// One workgroup per (row, head): heads [0, hq) are Q, [hq, hq + hkv) K and
// the rest V, which are also the column ranges of the fused QKV output, so
// head u covers columns [u * D, (u + 1) * D).  Thread i holds elements i,
// i + blockDim, ... and takes each one's rotate-half partner (e +- D/2) from
// LDS (D floats of dynamic shared memory).
template <typename T>
__global__ void __launch_bounds__(256)
    rope_cache_kernel(T* __restrict__ kv_layer, int64_t blk_stride, int64_t v_off,
                      int64_t slot_stride, int64_t head_stride, int bs_log2, int hq, int hkv,
                      int D,
                      const float* __restrict__ q_in, int64_t q_stride, float* __restrict__ q_out,
                      const float* __restrict__ k, int64_t k_stride, const float* __restrict__ v,
                      int64_t v_stride, const uint32_t* __restrict__ positions,
                      const int32_t* __restrict__ row_seq, const int64_t* __restrict__ bt_off,
                      const uint32_t* __restrict__ bt_ids, const float* __restrict__ cos_t,
                      const float* __restrict__ sin_t, GemmPartials qkv) {
#pragma clang fp contract(off)
  extern __shared__ float xs[];
  const int64_t row = blockIdx.x;
  const int unit = blockIdx.y;
  const bool is_q = unit < hq, is_k = !is_q && unit < hq + hkv;
  const int h = is_q ? unit : is_k ? unit - hq : unit - hq - hkv;
  const uint32_t pos = positions[row];
  const int seq = row_seq[row];
  const uint32_t blk = bt_ids[bt_off[seq] + (pos >> bs_log2)];
  const int64_t slot = pos & ((1u << bs_log2) - 1);
  T* kdst = kv_layer + (int64_t)blk * blk_stride + slot * slot_stride + h * head_stride;

  // Inputs come from the q/k/v buffers, or straight from the QKV GEMM's
  // unreduced partials.
  auto input = [&](int e) {
    if (qkv.ws) return partial_sum(qkv, row, (int64_t)unit * D + e);
    return is_q ? q_in[row * q_stride + h * D + e]
         : is_k ? k[row * k_stride + h * D + e]
                : v[row * v_stride + h * D + e];
  };
  if (!is_q && !is_k) {  // uniform over the workgroup
    for (int e = threadIdx.x; e < D; e += blockDim.x) store_kv<T>(kdst + v_off + e, input(e));
    return;
  }
  for (int e = threadIdx.x; e < D; e += blockDim.x) xs[e] = input(e);
  __syncthreads();
  const int half = D >> 1;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const float x = xs[i];
    const int j = i < half ? i : i - half;
    const float c = cos_t[(int64_t)pos * half + j], sn = sin_t[(int64_t)pos * half + j];
    // out[j] = x0 cos - x1 sin, out[j + half] = x0 sin + x1 cos (x0 = x[j], x1 = x[j + half])
    const float y = i < half ? x * c - xs[i + half] * sn : xs[j] * sn + x * c;
    if (is_q)
      q_out[row * (int64_t)hq * D + h * D + i] = y;
    else
      store_kv<T>(kdst + i, y);
  }
}

// The same RoPE + KV write for inputs in the q/k/v buffers (the prefill
// route), vectorised: thread t of a (row, head) takes dims 4t .. 4t+3 and
// their rotate-half partners 4t + D/2 .. (no LDS, no barrier; the same f32
// expressions per element as rope_cache_kernel).  One thread per 8 elements,
// a flat grid over (row, head, t); needs D % 8 == 0 and 16-byte aligned rows.
template <typename T>
__device__ inline void store_kv4(T* p, float4 v);
template <>
__device__ inline void store_kv4<float>(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
template <>
__device__ inline void store_kv4<uint16_t>(uint16_t* p, float4 v) {
  *reinterpret_cast<uint2*>(p) = make_uint2(
      (uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16),
      (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16));
}

template <typename T>
__global__ void __launch_bounds__(256)
    rope_cache_vec_kernel(T* __restrict__ kv_layer, int64_t blk_stride, int64_t v_off,
                          int64_t slot_stride, int64_t head_stride, int bs_log2, int hq, int hkv,
                          int D, int64_t rows, const float* __restrict__ q_in, int64_t q_stride,
                          float* __restrict__ q_out, const float* __restrict__ k,
                          int64_t k_stride, const float* __restrict__ v, int64_t v_stride,
                          const uint32_t* __restrict__ positions,
                          const int32_t* __restrict__ row_seq,
                          const int64_t* __restrict__ bt_off, const uint32_t* __restrict__ bt_ids,
                          const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
#pragma clang fp contract(off)
  const int half = D >> 1, tpu = D >> 3;  // threads per (row, head)
  const int units = hq + 2 * hkv;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * units * tpu) return;
  const int64_t row = idx / ((int64_t)units * tpu);
  const int rem = (int)(idx - row * units * tpu);
  const int unit = rem / tpu, t = rem - unit * tpu;
  const bool is_q = unit < hq, is_k = !is_q && unit < hq + hkv;
  const int h = is_q ? unit : is_k ? unit - hq : unit - hq - hkv;
  const float* src = is_q ? q_in + row * q_stride + h * D
                     : is_k ? k + row * k_stride + h * D
                            : v + row * v_stride + h * D;
  const float4 x0 = *reinterpret_cast<const float4*>(src + 4 * t);
  const float4 x1 = *reinterpret_cast<const float4*>(src + half + 4 * t);
  const uint32_t pos = positions[row];
  if (is_q || is_k) {
    const float4 c = *reinterpret_cast<const float4*>(cos_t + (int64_t)pos * half + 4 * t);
    const float4 sn = *reinterpret_cast<const float4*>(sin_t + (int64_t)pos * half + 4 * t);
    const float4 y0 = make_float4(x0.x * c.x - x1.x * sn.x, x0.y * c.y - x1.y * sn.y,
                                  x0.z * c.z - x1.z * sn.z, x0.w * c.w - x1.w * sn.w);
    const float4 y1 = make_float4(x0.x * sn.x + x1.x * c.x, x0.y * sn.y + x1.y * c.y,
                                  x0.z * sn.z + x1.z * c.z, x0.w * sn.w + x1.w * c.w);
    if (is_q) {
      float* dst = q_out + row * (int64_t)hq * D + h * D;
      *reinterpret_cast<float4*>(dst + 4 * t) = y0;
      *reinterpret_cast<float4*>(dst + half + 4 * t) = y1;
      return;
    }
    const int seq = row_seq[row];
    const uint32_t blk = bt_ids[bt_off[seq] + (pos >> bs_log2)];
    T* kdst = kv_layer + (int64_t)blk * blk_stride +
              (int64_t)(pos & ((1u << bs_log2) - 1)) * slot_stride + h * head_stride;
    store_kv4<T>(kdst + 4 * t, y0);
    store_kv4<T>(kdst + half + 4 * t, y1);
    return;
  }
  const int seq = row_seq[row];
  const uint32_t blk = bt_ids[bt_off[seq] + (pos >> bs_log2)];
  T* vdst = kv_layer + (int64_t)blk * blk_stride +
            (int64_t)(pos & ((1u << bs_log2) - 1)) * slot_stride + h * head_stride + v_off;
  store_kv4<T>(vdst + 4 * t, x0);
  store_kv4<T>(vdst + half + 4 * t, x1);
}

hipError_t launch_rope_and_cache(hipStream_t st, const KvGeom& kv, void* arena, int64_t layer,
                                 int64_t rows, int64_t hq, const float* q_in, int64_t q_stride,
                                 float* q_out, const float* k, int64_t k_stride, const float* v,
                                 int64_t v_stride, const uint32_t* positions,
                                 const int32_t* row_seq, const int64_t* bt_off,
                                 const uint32_t* bt_ids, const float* cos_t, const float* sin_t,
                                 const GemmPartials* qkv_partials) {
  if (rows == 0) return hipSuccess;
  const GemmPartials qp = qkv_partials ? *qkv_partials : GemmPartials{};
  int bs_log2 = 0;
  while ((1 << bs_log2) < kv.block_size) ++bs_log2;
  const ArenaStrides a = arena_strides(kv);
  if (kv.head_dim > kMaxHeadDim || kv.head_dim % 2 || hq + 2 * kv.num_kv_heads > 65535 ||
      rows > INT32_MAX)
    return hipErrorInvalidValue;
  // Inputs in the q/k/v buffers with 16-byte aligned rows: the vectorised
  // kernel (one thread per 8 elements instead of one per element).
  const int64_t D = kv.head_dim, units = hq + 2 * kv.num_kv_heads;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!qp.ws && D % 8 == 0 && q_stride % 4 == 0 && k_stride % 4 == 0 && v_stride % 4 == 0 &&
      al16(q_in) && al16(k) && al16(v) && al16(q_out) && al16(cos_t) && al16(sin_t) &&
      al16(arena)) {
    const int64_t threads = rows * units * (D / 8);
    if ((threads + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
    const dim3 vgrid((unsigned)((threads + 255) / 256));
    if (kv.dtype_bf16)
      hipLaunchKernelGGL(rope_cache_vec_kernel<uint16_t>, vgrid, dim3(256), 0, st,
                         static_cast<uint16_t*>(arena) + layer * a.layer, a.blk, a.v_off, a.slot,
                         a.head, bs_log2, (int)hq, (int)kv.num_kv_heads, (int)D, rows, q_in,
                         q_stride, q_out, k, k_stride, v, v_stride, positions, row_seq, bt_off,
                         bt_ids, cos_t, sin_t);
    else
      hipLaunchKernelGGL(rope_cache_vec_kernel<float>, vgrid, dim3(256), 0, st,
                         static_cast<float*>(arena) + layer * a.layer, a.blk, a.v_off, a.slot,
                         a.head, bs_log2, (int)hq, (int)kv.num_kv_heads, (int)D, rows, q_in,
                         q_stride, q_out, k, k_stride, v, v_stride, positions, row_seq, bt_off,
                         bt_ids, cos_t, sin_t);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)rows, (unsigned)(hq + 2 * kv.num_kv_heads));
  const dim3 block((unsigned)std::min<int64_t>((kv.head_dim + 63) & ~63, 256));
  const size_t lds = (size_t)kv.head_dim * sizeof(float);
  if (kv.dtype_bf16) {
    uint16_t* base = static_cast<uint16_t*>(arena) + layer * a.layer;
    hipLaunchKernelGGL(rope_cache_kernel<uint16_t>, grid, block, lds, st, base,
                       a.blk, a.v_off, a.slot, a.head, bs_log2, (int)hq, (int)kv.num_kv_heads,
                       (int)kv.head_dim, q_in, q_stride, q_out, k, k_stride, v, v_stride,
                       positions, row_seq, bt_off, bt_ids, cos_t, sin_t, qp);
  } else {
    float* base = static_cast<float*>(arena) + layer * a.layer;
    hipLaunchKernelGGL(rope_cache_kernel<float>, grid, block, lds, st, base,
                       a.blk, a.v_off, a.slot, a.head, bs_log2, (int)hq, (int)kv.num_kv_heads,
                       (int)kv.head_dim, q_in, q_stride, q_out, k, k_stride, v, v_stride,
                       positions, row_seq, bt_off, bt_ids, cos_t, sin_t, qp);
  }
  return hipGetLastError();
}

// swiglu (tensor.rs:175-189): gate = gate / (1 + exp(-gate)) * up.
__global__ void silu_mul_kernel(float* __restrict__ gate, const float* __restrict__ up, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float g = gate[i];
    gate[i] = g / (1.0f + __expf(-g)) * up[i];
  }
}

hipError_t launch_silu_mul(hipStream_t st, float* gate, const float* up, int64_t count) {
  if (count == 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 4096);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, st, gate, up, count);
  return hipGetLastError();
}

// argmax (runtime/src/sampling.rs:196-207): strict '>' from -inf, so NaN and
// -inf never win and the lowest index wins a tie; -1 if nothing qualifies.
// One 1024-thread workgroup per row; each thread scans its float4s in
// increasing index order, four loads in flight.
__global__ void __launch_bounds__(1024)
    argmax_kernel(const float* __restrict__ logits, int64_t cols, int64_t* __restrict__ out) {
  constexpr int T = 1024;
  __shared__ float bv[T / 64];
  __shared__ int64_t bi[T / 64];
  const float* row = logits + (int64_t)blockIdx.x * cols;
  float best = -INFINITY;
  int64_t idx = -1;
  auto take = [&](float v, int64_t i) {
    if (v > best) {  // indices arrive in increasing order: '>' keeps the lowest
      best = v;
      idx = i;
    }
  };
  auto take4 = [&](const float4& v, int64_t i4) {
    take(v.x, 4 * i4);
    take(v.y, 4 * i4 + 1);
    take(v.z, 4 * i4 + 2);
    take(v.w, 4 * i4 + 3);
  };
  if ((cols & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    const int64_t n4 = cols >> 2;
    int64_t i = threadIdx.x;
    for (; i + 3 * T < n4; i += 4 * T) {
      const float4 a = r4[i], b = r4[i + T], c = r4[i + 2 * T], d = r4[i + 3 * T];
      take4(a, i);
      take4(b, i + T);
      take4(c, i + 2 * T);
      take4(d, i + 3 * T);
    }
    for (; i < n4; i += T) take4(r4[i], i);
  } else {
    for (int64_t i = threadIdx.x; i < cols; i += T) take(row[i], i);
  }
  auto merge = [&](float ov, int64_t oi) {
    if (oi >= 0 && (idx < 0 || ov > best || (ov == best && oi < idx))) {
      best = ov;
      idx = oi;
    }
  };
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int64_t oi = __shfl_xor(idx, off);
    merge(ov, oi);
  }
  if ((threadIdx.x & 63) == 0) {
    bv[threadIdx.x >> 6] = best;
    bi[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int wv = 1; wv < T / 64; ++wv) merge(bv[wv], bi[wv]);
    out[blockIdx.x] = idx;
  }
}

hipError_t launch_argmax(hipStream_t st, const float* logits, int64_t rows, int64_t cols,
                         int64_t* out) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(1024), 0, st, logits, cols, out);
  return hipGetLastError();
}

__global__ void f32_to_bf16_kernel(const float* __restrict__ in, uint16_t* __restrict__ out,
                                   int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = f32_to_bf16(in[i]);
}

hipError_t launch_f32_to_bf16(hipStream_t st, const float* in, uint16_t* out, int64_t count) {
  if (count == 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 8192);
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, st, in, out, count);
  return hipGetLastError();
}

__global__ void synthetic_bf16_kernel(uint16_t* __restrict__ out, int64_t n, uint64_t key,
                                      float mul) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = f32_to_bf16(synthetic_normal(key, (uint64_t)i, mul));
}

hipError_t launch_synthetic_bf16(hipStream_t st, uint16_t* out, int64_t count, uint64_t key,
                                 float mul) {
  if (count == 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 16384);
  hipLaunchKernelGGL(synthetic_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, st, out, count,
                     key, mul);
  return hipGetLastError();
}

__global__ void synthetic_f32_kernel(float* __restrict__ out, int64_t n, uint64_t key, float mul) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = bf16_to_f32(f32_to_bf16(synthetic_normal(key, (uint64_t)i, mul)));
}

hipError_t launch_synthetic_f32(hipStream_t st, float* out, int64_t count, uint64_t key,
                                float mul) {
  if (count == 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 16384);
  hipLaunchKernelGGL(synthetic_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, out, count,
                     key, mul);
  return hipGetLastError();
}

__global__ void fill_f32_kernel(float* __restrict__ out, int64_t n, float value) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = value;
}

hipError_t launch_fill_f32(hipStream_t st, float* out, int64_t count, float value) {
  if (count == 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 8192);
  hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, out, count, value);
  return hipGetLastError();
}

}  // namespace orion

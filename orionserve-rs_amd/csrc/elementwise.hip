// Row-wise and elementwise kernels around the attention/GEMM hot path:
// embedding gather, RMSNorm, RoPE fused with the paged KV write (slot mapping),
// SwiGLU, greedy argmax, weight conversion and synthetic initialisation.
#include "common.hpp"
#include "kernels.hpp"

namespace orion {

// TransformerModel::embed (transformer.rs:208-223): row gather, bf16 -> f32.
// Token ids are range-checked on the host before launch.
__global__ void embed_kernel(const uint32_t* __restrict__ tokens, const uint16_t* __restrict__ table,
                             int64_t hidden, float* __restrict__ out) {
  const int64_t row = blockIdx.x;
  const uint16_t* src = table + (int64_t)tokens[row] * hidden;
  float* dst = out + row * hidden;
  for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = bf16_to_f32(src[i]);
}

hipError_t launch_embed(hipStream_t st, const uint32_t* tokens, int64_t n, const uint16_t* table,
                        int64_t hidden, float* out) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)n), dim3(256), 0, st, tokens, table, hidden, out);
  return hipGetLastError();
}

// rms_norm (tensor.rs:143-163): sum of squares in f64 as the reference does,
// scale = (f32)(1 / sqrt(sum/cols + eps)), v * scale * w in f32.
// One workgroup per output row; `row_index` optionally gathers input rows
// (the last row of each sequence before the LM head, transformer.rs:410-428).
__global__ void __launch_bounds__(256)
    rmsnorm_kernel(const float* __restrict__ x, const int32_t* __restrict__ row_index,
                   const float* __restrict__ weight, int64_t cols, float eps,
                   float* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ double part[4];
  const int64_t orow = blockIdx.x;
  const int64_t irow = row_index ? row_index[orow] : orow;
  const float* xr = x + irow * cols;
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
  float* orow_p = out + orow * cols;
  for (int64_t i = threadIdx.x; i < cols; i += 256) orow_p[i] = xr[i] * scale * weight[i];
}

hipError_t launch_rmsnorm(hipStream_t st, const float* x, const int32_t* row_index,
                          const float* weight, int64_t rows, int64_t cols, float eps, float* out) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, st, x, row_index, weight,
                     cols, eps, out);
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
                      const float* __restrict__ sin_t) {
#pragma clang fp contract(off)
  const int64_t row = blockIdx.x;
  const int half = D >> 1;
  const uint32_t pos = positions[row];
  const float* cs = cos_t + (int64_t)pos * half;
  const float* sn = sin_t + (int64_t)pos * half;
  const int seq = row_seq[row];
  const uint32_t blk = bt_ids[bt_off[seq] + (pos >> bs_log2)];
  const int64_t slot = pos & ((1u << bs_log2) - 1);
  T* kdst = kv_layer + (int64_t)blk * blk_stride + slot * slot_stride;
  T* vdst = kdst + v_off;

  const int pairs_q = hq * half;
  const int pairs_k = hkv * half;
  for (int idx = threadIdx.x; idx < pairs_q + pairs_k; idx += blockDim.x) {
    if (idx < pairs_q) {
      const int h = idx / half, i = idx - h * half;
      const float* src = q_in + row * q_stride + h * D;
      const float x0 = src[i], x1 = src[i + half];
      float* dst = q_out + row * (int64_t)hq * D + h * D;
      dst[i] = x0 * cs[i] - x1 * sn[i];
      dst[i + half] = x0 * sn[i] + x1 * cs[i];
    } else {
      const int kk = idx - pairs_q;
      const int h = kk / half, i = kk - h * half;
      const float* src = k + row * k_stride + h * D;
      const float x0 = src[i], x1 = src[i + half];
      store_kv<T>(kdst + h * head_stride + i, x0 * cs[i] - x1 * sn[i]);
      store_kv<T>(kdst + h * head_stride + i + half, x0 * sn[i] + x1 * cs[i]);
    }
  }
  for (int idx = threadIdx.x; idx < hkv * D; idx += blockDim.x) {
    const int h = idx / D;
    store_kv<T>(vdst + h * head_stride + (idx - h * D), v[row * v_stride + idx]);
  }
}

hipError_t launch_rope_and_cache(hipStream_t st, const KvGeom& kv, void* arena, int64_t layer,
                                 int64_t rows, int64_t hq, const float* q_in, int64_t q_stride,
                                 float* q_out, const float* k, int64_t k_stride, const float* v,
                                 int64_t v_stride, const uint32_t* positions,
                                 const int32_t* row_seq, const int64_t* bt_off,
                                 const uint32_t* bt_ids, const float* cos_t, const float* sin_t) {
  if (rows == 0) return hipSuccess;
  int bs_log2 = 0;
  while ((1 << bs_log2) < kv.block_size) ++bs_log2;
  const ArenaStrides a = arena_strides(kv);
  if (kv.dtype_bf16) {
    uint16_t* base = static_cast<uint16_t*>(arena) + layer * a.layer;
    hipLaunchKernelGGL(rope_cache_kernel<uint16_t>, dim3((unsigned)rows), dim3(256), 0, st, base,
                       a.blk, a.v_off, a.slot, a.head, bs_log2, (int)hq, (int)kv.num_kv_heads,
                       (int)kv.head_dim, q_in, q_stride, q_out, k, k_stride, v, v_stride,
                       positions, row_seq, bt_off, bt_ids, cos_t, sin_t);
  } else {
    float* base = static_cast<float*>(arena) + layer * a.layer;
    hipLaunchKernelGGL(rope_cache_kernel<float>, dim3((unsigned)rows), dim3(256), 0, st, base,
                       a.blk, a.v_off, a.slot, a.head, bs_log2, (int)hq, (int)kv.num_kv_heads,
                       (int)kv.head_dim, q_in, q_stride, q_out, k, k_stride, v, v_stride,
                       positions, row_seq, bt_off, bt_ids, cos_t, sin_t);
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
__global__ void __launch_bounds__(256)
    argmax_kernel(const float* __restrict__ logits, int64_t cols, int64_t* __restrict__ out) {
  __shared__ float bv[4];
  __shared__ int64_t bi[4];
  const float* row = logits + (int64_t)blockIdx.x * cols;
  float best = -INFINITY;
  int64_t idx = -1;
  for (int64_t i = threadIdx.x; i < cols; i += 256) {
    const float v = row[i];
    if (v > best) {  // strided scan visits increasing i, so '>' keeps the lowest index
      best = v;
      idx = i;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int64_t oi = __shfl_xor(idx, off);
    if (oi >= 0 && (idx < 0 || ov > best || (ov == best && oi < idx))) {
      best = ov;
      idx = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    bv[threadIdx.x >> 6] = best;
    bi[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int wv = 1; wv < 4; ++wv) {
      if (bi[wv] >= 0 && (idx < 0 || bv[wv] > best || (bv[wv] == best && bi[wv] < idx))) {
        best = bv[wv];
        idx = bi[wv];
      }
    }
    out[blockIdx.x] = idx;
  }
}

hipError_t launch_argmax(hipStream_t st, const float* logits, int64_t rows, int64_t cols,
                         int64_t* out) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)rows), dim3(256), 0, st, logits, cols, out);
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

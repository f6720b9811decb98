// Host runtime behind the C ABI (include/orion_hip.h): device handles,
// model weights and KV arena in HBM, batch validation/upload and the forward
// pass orchestration.  Mirrors the reference's CpuBackend/TransformerModel
// (crates/orion-models/src/backend.rs, transformer.rs) with every tensor
// operation running as a gfx950 kernel on the device's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/orion_hip.h"
#include "checkpoint.hpp"
#include "kernels.hpp"

#define ORION_EXPORT extern "C" __attribute__((visibility("default")))

using namespace orion;

namespace {

thread_local std::string g_err;
thread_local std::string g_stage;

int set_err(int code, const char* stage, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  g_stage = stage;
  return code;
}

int internal(const char* stage, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  g_stage = stage;
  return ORION_HIP_ERR_INTERNAL;
}

#define HIP_TRY(stage, expr)                                                               \
  do {                                                                                     \
    hipError_t _e = (expr);                                                                \
    if (_e != hipSuccess)                                                                  \
      return set_err(ORION_HIP_ERR_BACKEND, stage, "%s: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

// A device allocation that grows on demand (never shrinks).
struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  hipError_t reserve(size_t want) {
    if (want <= bytes) return hipSuccess;
    if (ptr) {
      // The old buffer may still be in use by queued work.
      hipError_t e = hipDeviceSynchronize();
      if (e != hipSuccess) return e;
      e = hipFree(ptr);
      if (e != hipSuccess) return e;
      ptr = nullptr;
      bytes = 0;
    }
    size_t rounded = std::max<size_t>(want, 256);
    rounded = (rounded + (1 << 20) - 1) & ~((size_t)(1 << 20) - 1);
    hipError_t e = hipMalloc(&ptr, rounded);
    if (e != hipSuccess) {
      ptr = nullptr;
      return e;
    }
    bytes = rounded;
    return hipSuccess;
  }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

uint16_t host_f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float host_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

float host_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t mant = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {  // subnormal: renormalise
      exp = 127 - 15 + 1;
      while (!(mant & 0x400)) {
        mant <<= 1;
        --exp;
      }
      mant &= 0x3ff;
      bits = sign | (exp << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

}  // namespace

struct orion_hip_device {
  int ordinal = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev_start = nullptr, ev_stop = nullptr;
  std::string name;
  int64_t wave_slots = 2048;  // resident decode waves: CUs x 4 SIMDs x 2
  // Split-K GEMM scratch (partial tiles), shared by every call on this
  // device's stream.
  DevBuf gemm_ws;
  DevBuf prefill_order;  // op-level prefill work list (+ key-part merge lists)
  DevBuf prefill_ws;     // op-level prefill key-part partials
  DevBuf sample_io, sample_ws;  // sampler inputs/outputs and probabilities
  // This device's address of the file-scope `scratch` array
  // (orion_hip_gemm_noalloc); never freed.
  void* noalloc_scratch = nullptr;
  // Per-kernel timing (orion_hip_kernel_timing): event pairs per kernel
  // index, resolved when read.
  bool ktiming = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> kevents[4];
  std::vector<hipEvent_t> event_pool;
  hipEvent_t take_event() {
    if (!event_pool.empty()) {
      hipEvent_t e = event_pool.back();
      event_pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
  void recycle_events() {
    for (auto& v : kevents) {
      for (auto& p : v) {
        event_pool.push_back(p.first);
        event_pool.push_back(p.second);
      }
      v.clear();
    }
  }
};

struct orion_hip_decode_plan {
  orion_hip_device* dev = nullptr;
  int64_t rows = 0, hq = 0, hkv = 0, head_dim = 0, block_size = 0;
  // host: the plan as built for a bf16 arena (shared prefixes packed where
  // the MFMA wave takes them); plain: the same rows without packing, built
  // only when host packs something (an f32 arena takes it).  Each device
  // buffer holds the work items, the pieces per row, then the pack rows.
  DecodePlanHost host, plain;
  DevBuf work, work_plain, ws;
  ~orion_hip_decode_plan() {
    work.release();
    work_plain.release();
    ws.release();
  }
  static DecodePlanDev view_of(const DecodePlanHost& h, const DevBuf& b) {
    DecodePlanDev d;
    d.work = b.as<const DecodeWork>();
    const char* base = b.as<const char>();
    d.row_nsplit = reinterpret_cast<const int32_t*>(base + h.work.size() * sizeof(DecodeWork));
    d.num_work = (int)h.work.size();
    d.chunk = h.chunk;
    d.max_splits = h.max_splits;
    d.stream_kv = h.stream_kv;
    d.mixed_kv = h.mixed_kv;
    d.num_packed = h.num_packed;
    d.pack_rows = reinterpret_cast<const int32_t*>(base + h.work.size() * sizeof(DecodeWork) +
                                                   h.row_nsplit.size() * sizeof(int32_t));
    d.pack_r = h.pack_r;
    return d;
  }
  DecodePlanDev view(bool bf16) const {
    DecodePlanDev d = (!bf16 && host.num_packed) ? view_of(plain, work_plain) : view_of(host, work);
    d.ws = ws.as<float>();
    d.ws_bytes = ws.bytes;
    return d;
  }
};

struct LayerDev {
  float* input_norm = nullptr;
  float* post_norm = nullptr;
  uint16_t* w_qkv = nullptr;  // [Hq*d + 2*Hkv*d, hidden]
  float* b_qkv = nullptr;     // [Hq*d + 2*Hkv*d] or null
  uint16_t* w_o = nullptr;    // [hidden, Hq*d]
  uint16_t* w_gu = nullptr;   // [2*ffn, hidden], gate/up rows interleaved by 8
  uint16_t* w_down = nullptr; // [hidden, ffn]
  // The same four matrices in the decode GEMM's packed order (launch_gemv_pack),
  // which every GEMM of a forward reads.  The row-major ones above exist only
  // while weights are written or read back (ensure_rowmajor / release_rowmajor).
  uint16_t* p_qkv = nullptr;
  uint16_t* p_o = nullptr;
  uint16_t* p_gu = nullptr;
  uint16_t* p_down = nullptr;
};

struct orion_hip_model {
  orion_hip_device* dev = nullptr;
  orion_hip_model_desc desc{};
  int64_t qd = 0, kvd = 0, qkvd = 0;
  KvGeom kv{};
  std::vector<void*> allocations;
  std::vector<size_t> alloc_bytes;
  uint16_t* w_embed = nullptr;
  uint16_t* w_lm = nullptr;  // null when tied
  float* final_norm = nullptr;
  uint16_t* p_head = nullptr;  // LM head (or tied embedding) in packed order
  bool packs_valid = false;    // packed copies match the row-major weights
  bool rowmajor_live = true;   // row-major layer matrices / LM head allocated
  std::vector<LayerDev> layers;
  float* rope_cos = nullptr;
  float* rope_sin = nullptr;
  void* arena = nullptr;
  size_t arena_bytes = 0;
  int64_t last_rows = 0;  // rows of `logits` the last forward produced

  // activations / batch buffers (grown on demand)
  DevBuf hidden, xn, qkv, qrot, attn, act, logits, argmax, ws, sumsq;
  DevBuf b_batch, b_plan;  // the batch and the attention plans (one copy each)
  void* pinned[2] = {nullptr, nullptr};  // their pinned staging areas
  size_t pinned_bytes[2] = {0, 0};

  ~orion_hip_model() {
    for (void* p : allocations) (void)hipFree(p);
    for (DevBuf* b : {&hidden, &xn, &qkv, &qrot, &attn, &act, &logits, &argmax, &ws, &sumsq,
                      &b_batch, &b_plan})
      b->release();
    for (void* p : pinned)
      if (p) (void)hipHostFree(p);
  }

  // Frees one allocation made by alloc (the device is synchronised first).
  template <typename T>
  hipError_t release(T** p) {
    if (!*p) return hipSuccess;
    for (size_t i = 0; i < allocations.size(); ++i) {
      if (allocations[i] == static_cast<void*>(*p)) {
        hipError_t e = hipStreamSynchronize(dev->stream);
        if (e == hipSuccess) e = hipFree(allocations[i]);
        allocations.erase(allocations.begin() + i);
        alloc_bytes.erase(alloc_bytes.begin() + i);
        *p = nullptr;
        return e;
      }
    }
    return hipErrorInvalidValue;
  }

  template <typename T>
  hipError_t alloc(T** out, size_t count) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(count * sizeof(T), 256);
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return e;
    allocations.push_back(p);
    alloc_bytes.push_back(bytes);
    *out = static_cast<T*>(p);
    return hipSuccess;
  }
};

// ---------------------------------------------------------------------------
// Errors
// ---------------------------------------------------------------------------

ORION_EXPORT const char* orion_hip_last_error(void) { return g_err.c_str(); }
ORION_EXPORT const char* orion_hip_last_error_stage(void) { return g_stage.c_str(); }

// ---------------------------------------------------------------------------
// Backend
// ---------------------------------------------------------------------------

ORION_EXPORT int orion_hip_device_count(int* count) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) n = 0;  // no driver / no GPU: zero devices, not an error
  *count = n;
  return ORION_HIP_OK;
}

// ---------------------------------------------------------------------------
// Scratch of the no-allocation GEMM entry point (orion_hip_gemm_noalloc)
// ---------------------------------------------------------------------------

// Split-K partial tiles of orion_hip_gemm_noalloc.  Every GPU the library runs
// on holds its own copy for the life of the process.  Host code never uses
// the array's name as an address (on the host it is only a stand-in): the
// device address is resolved once per device, with that device current, at
// orion_hip_device_open, and kept in g_noalloc_scratch.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

static std::mutex g_noalloc_mu;
static void* g_noalloc_scratch[256] = {};
// Per GPU: an event recorded after the last orion_hip_gemm_noalloc launch on
// that GPU (from any device handle, each with its own stream).  The next call
// makes its stream wait for it, so calls through different handles of one GPU
// run one after another on the shared array instead of racing on it.
static hipEvent_t g_noalloc_done[256] = {};
static bool g_noalloc_recorded[256] = {};

// Resolves this device's address of `scratch` (the device must be current).
static hipError_t resolve_noalloc_scratch(int ordinal, void** out) {
  if (ordinal < 0 || ordinal >= 256) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_scratch[ordinal]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_noalloc_scratch[ordinal] = p;
    e = hipEventCreateWithFlags(&g_noalloc_done[ordinal], hipEventDisableTiming);
    if (e != hipSuccess) return e;
  }
  *out = g_noalloc_scratch[ordinal];
  return hipSuccess;
}

ORION_EXPORT int orion_hip_device_open(int ordinal, orion_hip_device** out) {
  *out = nullptr;
  int n = 0;
  orion_hip_device_count(&n);
  if (n == 0) return set_err(ORION_HIP_ERR_BACKEND, "device_open", "no HIP devices are visible");
  if (ordinal < 0 || ordinal >= n)
    return set_err(ORION_HIP_ERR_BACKEND, "device_open", "device %d requested, %d available",
                   ordinal, n);
  HIP_TRY("device_open", hipSetDevice(ordinal));
  hipDeviceProp_t prop;
  HIP_TRY("device_open", hipGetDeviceProperties(&prop, ordinal));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_err(ORION_HIP_ERR_BACKEND, "device_open",
                   "device %d is %s; this library is built for gfx950 (MI355X) only", ordinal,
                   prop.gcnArchName);
  auto dev = std::make_unique<orion_hip_device>();
  dev->ordinal = ordinal;
  dev->name = prop.name;
  dev->wave_slots = (int64_t)prop.multiProcessorCount * 8;
  HIP_TRY("device_open", hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking));
  HIP_TRY("device_open", hipEventCreate(&dev->ev_start));
  HIP_TRY("device_open", hipEventCreate(&dev->ev_stop));
  HIP_TRY("device_open", resolve_noalloc_scratch(ordinal, &dev->noalloc_scratch));
  *out = dev.release();
  return ORION_HIP_OK;
}

ORION_EXPORT void orion_hip_device_close(orion_hip_device* dev) {
  if (!dev) return;
  (void)hipSetDevice(dev->ordinal);
  (void)hipStreamSynchronize(dev->stream);
  (void)hipEventDestroy(dev->ev_start);
  (void)hipEventDestroy(dev->ev_stop);
  dev->recycle_events();
  for (hipEvent_t e : dev->event_pool) (void)hipEventDestroy(e);
  dev->gemm_ws.release();
  dev->prefill_order.release();
  dev->prefill_ws.release();
  dev->sample_io.release();
  dev->sample_ws.release();
  (void)hipStreamDestroy(dev->stream);
  delete dev;
}

ORION_EXPORT int orion_hip_device_name(orion_hip_device* dev, char* buf, size_t len) {
  if (!buf || len == 0) return internal("device_name", "empty buffer");
  std::snprintf(buf, len, "%s", dev->name.c_str());
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_mem_info(orion_hip_device* dev, uint64_t* total, uint64_t* free_bytes) {
  HIP_TRY("mem_info", hipSetDevice(dev->ordinal));
  size_t f = 0, t = 0;
  HIP_TRY("mem_info", hipMemGetInfo(&f, &t));
  *total = t;
  *free_bytes = f;
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_synchronize(orion_hip_device* dev) {
  HIP_TRY("synchronize", hipStreamSynchronize(dev->stream));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_supports_dtype(orion_hip_device* dev, int dtype) {
  (void)dev;
  return dtype == ORION_DTYPE_F32 || dtype == ORION_DTYPE_F16 || dtype == ORION_DTYPE_BF16;
}

ORION_EXPORT int orion_hip_alloc(orion_hip_device* dev, size_t bytes, void** d_ptr) {
  HIP_TRY("alloc", hipSetDevice(dev->ordinal));
  HIP_TRY("alloc", hipMalloc(d_ptr, std::max<size_t>(bytes, 256)));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_free(orion_hip_device* dev, void* d_ptr) {
  HIP_TRY("free", hipStreamSynchronize(dev->stream));
  HIP_TRY("free", hipFree(d_ptr));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_memcpy_h2d(orion_hip_device* dev, void* d_dst, const void* src,
                                      size_t bytes) {
  HIP_TRY("memcpy_h2d", hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, dev->stream));
  HIP_TRY("memcpy_h2d", hipStreamSynchronize(dev->stream));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_memcpy_d2h(orion_hip_device* dev, void* dst, const void* d_src,
                                      size_t bytes) {
  HIP_TRY("memcpy_d2h", hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, dev->stream));
  HIP_TRY("memcpy_d2h", hipStreamSynchronize(dev->stream));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_memcpy_d2d(orion_hip_device* dev, void* d_dst, const void* d_src,
                                      size_t bytes) {
  HIP_TRY("memcpy_d2d", hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, dev->stream));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_memset(orion_hip_device* dev, void* d_dst, int value, size_t bytes) {
  HIP_TRY("memset", hipMemsetAsync(d_dst, value, bytes, dev->stream));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_timer_start(orion_hip_device* dev) {
  HIP_TRY("timer", hipEventRecord(dev->ev_start, dev->stream));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_timer_stop(orion_hip_device* dev, float* ms) {
  HIP_TRY("timer", hipEventRecord(dev->ev_stop, dev->stream));
  HIP_TRY("timer", hipEventSynchronize(dev->ev_stop));
  HIP_TRY("timer", hipEventElapsedTime(ms, dev->ev_start, dev->ev_stop));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_kernel_timing(orion_hip_device* dev, int enable) {
  HIP_TRY("kernel_timing", hipSetDevice(dev->ordinal));
  HIP_TRY("kernel_timing", hipStreamSynchronize(dev->stream));
  dev->recycle_events();
  dev->ktiming = enable != 0;
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_kernel_timing_read(orion_hip_device* dev, int kernel, double* total_ms,
                                              int64_t* calls) {
  const char* st = "kernel_timing";
  if (kernel < 0 || kernel > 3) return internal(st, "kernel index %d is not 0 .. 3", kernel);
  double sum = 0.0;
  for (auto& p : dev->kevents[kernel]) {
    HIP_TRY(st, hipEventSynchronize(p.second));
    float ms = 0.f;
    HIP_TRY(st, hipEventElapsedTime(&ms, p.first, p.second));
    sum += ms;
  }
  *total_ms = sum;
  *calls = (int64_t)dev->kevents[kernel].size();
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_kernel_timing_samples(orion_hip_device* dev, int kernel, float* ms_out,
                                                 int64_t capacity, int64_t* calls) {
  const char* st = "kernel_timing";
  if (kernel < 0 || kernel > 3) return internal(st, "kernel index %d is not 0 .. 3", kernel);
  int64_t i = 0;
  for (auto& p : dev->kevents[kernel]) {
    if (i >= capacity) break;
    HIP_TRY(st, hipEventSynchronize(p.second));
    HIP_TRY(st, hipEventElapsedTime(&ms_out[i], p.first, p.second));
    ++i;
  }
  *calls = (int64_t)dev->kevents[kernel].size();
  return ORION_HIP_OK;
}

// Records a (start, stop) event pair for kernel index k around `launch` when
// per-kernel timing is on.
template <typename F>
static hipError_t timed_launch(orion_hip_device* dev, int k, F&& launch) {
  if (!dev->ktiming) return launch();
  hipEvent_t a = dev->take_event(), b = dev->take_event();
  if (!a || !b) return hipErrorOutOfMemory;
  hipError_t e = hipEventRecord(a, dev->stream);
  if (e == hipSuccess) e = launch();
  if (e == hipSuccess) e = hipEventRecord(b, dev->stream);
  if (e != hipSuccess) {
    dev->event_pool.push_back(a);
    dev->event_pool.push_back(b);
    return e;
  }
  dev->kevents[k].push_back({a, b});
  return hipSuccess;
}

// The split-K GEMM scratch for a call of this shape, grown on demand.
static hipError_t gemm_scratch(orion_hip_device* dev, int64_t M, int64_t N, int64_t K,
                               GemmScratch* sc) {
  size_t ws = 0;
  gemm_scratch_need(M, N, K, &ws);
  if (ws > dev->gemm_ws.bytes) {
    hipError_t e = dev->gemm_ws.reserve(ws);
    if (e != hipSuccess) return e;
  }
  sc->ws = dev->gemm_ws.as<float>();
  sc->ws_bytes = dev->gemm_ws.bytes;
  return hipSuccess;
}

static hipError_t gemm_on(orion_hip_device* dev, const float* x, const uint16_t* w,
                          const float* bias, int64_t M, int64_t N, int64_t K, Epilogue ep,
                          float* out, const GemmFuse* fuse = nullptr) {
  GemmScratch sc;
  hipError_t e = gemm_scratch(dev, M, N, K, &sc);
  if (e != hipSuccess) return e;
  return launch_gemm(dev->stream, x, w, bias, M, N, K, ep, out, &sc, fuse);
}

// ---------------------------------------------------------------------------
// Model
// ---------------------------------------------------------------------------

static int check_desc(const orion_hip_model_desc* d) {
  const char* st = "model_create";
  if (d->num_layers <= 0 || d->hidden_size <= 0 || d->num_attention_heads <= 0 ||
      d->num_kv_heads <= 0 || d->head_dim <= 0 || d->intermediate_size <= 0 ||
      d->vocab_size <= 0 || d->max_position_embeddings <= 0 || d->num_blocks <= 0)
    return internal(st, "model dimensions must be positive");
  if (d->num_attention_heads % d->num_kv_heads != 0)
    return internal(st, "%d query heads cannot be grouped over %d kv heads",
                    d->num_attention_heads, d->num_kv_heads);
  if (d->block_size < 4 || d->block_size > 256 || (d->block_size & (d->block_size - 1)))
    return internal(st, "block_size must be a power of two in [4, 256], got %d", d->block_size);
  // RoPE rotates halves (tensor.rs:283-298), so head_dim is even; the
  // attention kernels cover every even head_dim up to kMaxHeadDim and any
  // grouping (MFMA for 64 and 128 with groups up to 16 on bf16 arenas, a general wave
  // otherwise).
  if (d->head_dim % 2 || d->head_dim > kMaxHeadDim)
    return set_err(ORION_HIP_ERR_BACKEND, st, "head_dim %d unsupported (even, at most %d)",
                   d->head_dim, kMaxHeadDim);
  if (d->hidden_size % 32 || d->intermediate_size % 32 ||
      (d->num_attention_heads * d->head_dim) % 32)
    return set_err(ORION_HIP_ERR_BACKEND, st,
                   "hidden, intermediate and Hq*head_dim must be multiples of 32");
  if (d->kv_dtype != ORION_DTYPE_F32 && d->kv_dtype != ORION_DTYPE_BF16)
    return set_err(ORION_HIP_ERR_BACKEND, st, "kv_dtype must be F32 or BF16");
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_model_create(orion_hip_device* dev, const orion_hip_model_desc* desc,
                                        orion_hip_model** out) {
  *out = nullptr;
  if (int rc = check_desc(desc)) return rc;
  HIP_TRY("model_create", hipSetDevice(dev->ordinal));
  auto m = std::make_unique<orion_hip_model>();
  m->dev = dev;
  m->desc = *desc;
  const auto& d = *desc;
  m->qd = (int64_t)d.num_attention_heads * d.head_dim;
  m->kvd = (int64_t)d.num_kv_heads * d.head_dim;
  m->qkvd = m->qd + 2 * m->kvd;
  // Block-internal KV layout of the arena: the reference order unless
  // ORION_KV_LAYOUT=head-major (read at model creation; both measure the same
  // on the decode and prefill kernels).
  const char* lay = getenv("ORION_KV_LAYOUT");
  const bool head_major = lay && std::strcmp(lay, "head-major") == 0;
  m->kv = KvGeom{d.num_layers, d.num_blocks, d.block_size, d.num_kv_heads, d.head_dim,
                 d.kv_dtype == ORION_DTYPE_BF16, head_major};
  const int64_t H = d.hidden_size, F = d.intermediate_size, V = d.vocab_size;
  const char* st = "model_create";
  HIP_TRY(st, m->alloc(&m->w_embed, (size_t)(V * H)));
  if (!d.tied_lm_head) HIP_TRY(st, m->alloc(&m->w_lm, (size_t)(V * H)));
  HIP_TRY(st, m->alloc(&m->final_norm, (size_t)H));
  m->layers.resize(d.num_layers);
  for (auto& L : m->layers) {
    HIP_TRY(st, m->alloc(&L.input_norm, (size_t)H));
    HIP_TRY(st, m->alloc(&L.post_norm, (size_t)H));
    HIP_TRY(st, m->alloc(&L.w_qkv, (size_t)(m->qkvd * H)));
    if (d.has_qkv_bias) HIP_TRY(st, m->alloc(&L.b_qkv, (size_t)m->qkvd));
    HIP_TRY(st, m->alloc(&L.w_o, (size_t)(H * m->qd)));
    HIP_TRY(st, m->alloc(&L.w_gu, (size_t)(2 * F * H)));
    HIP_TRY(st, m->alloc(&L.w_down, (size_t)(H * F)));
  }
  // Zero every weight so an un-uploaded tensor is deterministic.
  for (size_t i = 0; i < m->allocations.size(); ++i)
    HIP_TRY(st, hipMemsetAsync(m->allocations[i], 0, m->alloc_bytes[i], dev->stream));
  const int64_t half = d.head_dim / 2;
  const int64_t tab = (int64_t)d.max_position_embeddings * half;
  HIP_TRY(st, m->alloc(&m->rope_cos, (size_t)tab));
  HIP_TRY(st, m->alloc(&m->rope_sin, (size_t)tab));
  {
    // RopeTable::new (tensor.rs:228-253), computed on the host with the same
    // f32 libm calls as the reference and uploaded once.
    std::vector<float> c(tab), s(tab);
    for (int64_t pos = 0; pos < d.max_position_embeddings; ++pos)
      for (int64_t i = 0; i < half; ++i) {
        const float inv_freq =
            1.0f / std::pow(d.rope_theta, 2.0f * (float)i / (float)d.head_dim);
        const float angle = (float)pos * inv_freq;
        c[pos * half + i] = std::cos(angle);
        s[pos * half + i] = std::sin(angle);
      }
    HIP_TRY(st, hipMemcpy(m->rope_cos, c.data(), tab * 4, hipMemcpyHostToDevice));
    HIP_TRY(st, hipMemcpy(m->rope_sin, s.data(), tab * 4, hipMemcpyHostToDevice));
  }
  // KvStore::new (attention.rs:45-62): zero-filled arena.
  const size_t esz = m->kv.dtype_bf16 ? 2 : 4;
  m->arena_bytes = (size_t)d.num_layers * d.num_blocks * 2 * d.block_size * d.num_kv_heads *
                   d.head_dim * esz;
  HIP_TRY(st, hipMalloc(&m->arena, m->arena_bytes));
  m->allocations.push_back(m->arena);
  m->alloc_bytes.push_back(m->arena_bytes);
  HIP_TRY(st, hipMemsetAsync(m->arena, 0, m->arena_bytes, dev->stream));
  HIP_TRY(st, hipStreamSynchronize(dev->stream));
  *out = m.release();
  return ORION_HIP_OK;
}

ORION_EXPORT void orion_hip_model_destroy(orion_hip_model* model) {
  if (!model) return;
  (void)hipSetDevice(model->dev->ordinal);
  (void)hipStreamSynchronize(model->dev->stream);
  delete model;
}

// Where a weight lives on the device: base pointer, element type, and the
// row mapping used by the fused layouts.
struct WeightSlot {
  void* base = nullptr;
  bool bf16 = true;
  int64_t rows = 0, cols = 0;
  // destination row of source row r: (r / group) * stride + offset + r % group
  int64_t group = 0, stride = 0, offset = 0;
};

static hipError_t ensure_rowmajor(orion_hip_model* m);

static int weight_slot(orion_hip_model* m, int which, int layer, WeightSlot* s) {
  const auto& d = m->desc;
  const bool matrix = which == ORION_W_LM_HEAD || which == ORION_W_Q || which == ORION_W_K ||
                      which == ORION_W_V || which == ORION_W_O || which == ORION_W_GATE ||
                      which == ORION_W_UP || which == ORION_W_DOWN;
  if (matrix && (which != ORION_W_LM_HEAD || !d.tied_lm_head))
    HIP_TRY("weight", ensure_rowmajor(m));
  const int64_t H = d.hidden_size, F = d.intermediate_size, V = d.vocab_size;
  if (which >= ORION_W_INPUT_NORM && (layer < 0 || layer >= d.num_layers))
    return internal("upload_weight", "layer %d out of range (have %d)", layer, d.num_layers);
  LayerDev* L = which >= ORION_W_INPUT_NORM ? &m->layers[layer] : nullptr;
  *s = WeightSlot{};
  switch (which) {
    case ORION_W_EMBED: *s = {m->w_embed, true, V, H}; break;
    case ORION_W_LM_HEAD:
      if (!m->w_lm) return internal("upload_weight", "model has a tied LM head");
      *s = {m->w_lm, true, V, H};
      break;
    case ORION_W_FINAL_NORM: *s = {m->final_norm, false, 1, H}; break;
    case ORION_W_INPUT_NORM: *s = {L->input_norm, false, 1, H}; break;
    case ORION_W_POST_NORM: *s = {L->post_norm, false, 1, H}; break;
    case ORION_W_Q: *s = {L->w_qkv, true, m->qd, H}; break;
    case ORION_W_K: *s = {L->w_qkv + m->qd * H, true, m->kvd, H}; break;
    case ORION_W_V: *s = {L->w_qkv + (m->qd + m->kvd) * H, true, m->kvd, H}; break;
    case ORION_W_O: *s = {L->w_o, true, H, m->qd}; break;
    case ORION_W_Q_BIAS:
    case ORION_W_K_BIAS:
    case ORION_W_V_BIAS: {
      if (!L->b_qkv) return internal("upload_weight", "model has no QKV bias");
      const int64_t off = which == ORION_W_Q_BIAS ? 0 : which == ORION_W_K_BIAS ? m->qd : m->qd + m->kvd;
      *s = {L->b_qkv + off, false, 1, which == ORION_W_Q_BIAS ? m->qd : m->kvd};
      break;
    }
    case ORION_W_GATE: *s = {L->w_gu, true, F, H, 8, 16, 0}; break;
    case ORION_W_UP: *s = {L->w_gu, true, F, H, 8, 16, 8}; break;
    case ORION_W_DOWN: *s = {L->w_down, true, H, F}; break;
    default: return internal("upload_weight", "unknown weight id %d", which);
  }
  return ORION_HIP_OK;
}

static int upload_rows(orion_hip_model* m, const WeightSlot& s, const void* host_conv,
                       size_t esz, const char* st) {
  hipStream_t stream = m->dev->stream;
  if (s.group == 0) {
    HIP_TRY(st, hipMemcpyAsync(s.base, host_conv, (size_t)(s.rows * s.cols) * esz,
                               hipMemcpyHostToDevice, stream));
  } else {
    // rows come in groups of `group`; group g lands at row g*stride + offset.
    const size_t row_bytes = (size_t)s.cols * esz;
    HIP_TRY(st, hipMemcpy2DAsync(static_cast<char*>(s.base) + s.offset * row_bytes,
                                 s.stride * row_bytes, host_conv, s.group * row_bytes,
                                 s.group * row_bytes, (size_t)(s.rows / s.group),
                                 hipMemcpyHostToDevice, stream));
  }
  HIP_TRY(st, hipStreamSynchronize(stream));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_model_upload_weight(orion_hip_model* model, int which, int layer,
                                               const void* host, int dtype, size_t count) {
  const char* st = "upload_weight";
  WeightSlot s;
  if (int rc = weight_slot(model, which, layer, &s)) return rc;
  model->packs_valid = false;
  if ((int64_t)count != s.rows * s.cols)
    return internal(st, "weight %d has %zu elements, expected %lld", which, count,
                    (long long)(s.rows * s.cols));
  if (dtype != ORION_DTYPE_F32 && dtype != ORION_DTYPE_F16 && dtype != ORION_DTYPE_BF16)
    return set_err(ORION_HIP_ERR_BACKEND, st, "unsupported host dtype %d", dtype);
  HIP_TRY(st, hipSetDevice(model->dev->ordinal));
  // Convert on the host (loader.rs:74-98 widens to f32; device matrices are bf16).
  if (s.bf16) {
    if (dtype == ORION_DTYPE_BF16) return upload_rows(model, s, host, 2, st);
    std::vector<uint16_t> conv(count);
    if (dtype == ORION_DTYPE_F32) {
      const float* f = static_cast<const float*>(host);
      for (size_t i = 0; i < count; ++i) conv[i] = host_f32_to_bf16(f[i]);
    } else {
      const uint16_t* h = static_cast<const uint16_t*>(host);
      for (size_t i = 0; i < count; ++i) conv[i] = host_f32_to_bf16(host_f16_to_f32(h[i]));
    }
    return upload_rows(model, s, conv.data(), 2, st);
  }
  std::vector<float> conv(count);
  if (dtype == ORION_DTYPE_F32) {
    std::memcpy(conv.data(), host, count * 4);
  } else if (dtype == ORION_DTYPE_BF16) {
    const uint16_t* h = static_cast<const uint16_t*>(host);
    for (size_t i = 0; i < count; ++i) conv[i] = host_bf16_to_f32(h[i]);
  } else {
    const uint16_t* h = static_cast<const uint16_t*>(host);
    for (size_t i = 0; i < count; ++i) conv[i] = host_f16_to_f32(h[i]);
  }
  return upload_rows(model, s, conv.data(), 4, st);
}

// ---------------------------------------------------------------------------
// Safetensors checkpoints
// ---------------------------------------------------------------------------

struct orion_hip_checkpoint {
  std::unique_ptr<Checkpoint> ck;
};

ORION_EXPORT int orion_hip_checkpoint_open(const char* dir, orion_hip_checkpoint** out) {
  const char* st = "checkpoint_open";
  if (!dir || !out) return internal(st, "null argument");
  *out = nullptr;
  Checkpoint::Error kind;
  std::string err;
  std::unique_ptr<Checkpoint> ck = Checkpoint::open(dir, &kind, &err);
  if (!ck) return internal(st, "%s", err.c_str());
  *out = new orion_hip_checkpoint{std::move(ck)};
  return ORION_HIP_OK;
}

ORION_EXPORT void orion_hip_checkpoint_close(orion_hip_checkpoint* ck) { delete ck; }

ORION_EXPORT int orion_hip_checkpoint_num_tensors(const orion_hip_checkpoint* ck,
                                                  int64_t* count) {
  if (!ck || !count) return internal("checkpoint_num_tensors", "null argument");
  *count = (int64_t)ck->ck->names().size();
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_checkpoint_tensor_info(const orion_hip_checkpoint* ck, int64_t index,
                                                  char* name, size_t name_len, int32_t* dtype,
                                                  int32_t* ndim, int64_t* shape8) {
  const char* st = "checkpoint_tensor_info";
  if (!ck) return internal(st, "null checkpoint");
  const auto& names = ck->ck->names();
  if (index < 0 || index >= (int64_t)names.size())
    return internal(st, "tensor index %lld out of range (have %zu)", (long long)index,
                    names.size());
  const CheckpointTensor* t = ck->ck->find(names[index]);
  if (t->shape.size() > 8) return internal(st, "tensor `%s` has rank > 8", t->name.c_str());
  if (name && name_len) {
    const size_t n = std::min(name_len - 1, t->name.size());
    std::memcpy(name, t->name.data(), n);
    name[n] = '\0';
  }
  if (dtype) *dtype = t->dtype;
  if (ndim) *ndim = (int32_t)t->shape.size();
  if (shape8)
    for (size_t i = 0; i < t->shape.size(); ++i) shape8[i] = t->shape[i];
  return ORION_HIP_OK;
}

namespace {

int64_t numel(const CheckpointTensor& t) {
  int64_t n = 1;
  for (int64_t d : t.shape) n *= d;
  return n;
}

std::string shape_str(const std::vector<int64_t>& v) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + std::to_string(v[i]);
  return s + "]";
}

// Looks a tensor up with the reference's checks (loader.rs:188-235): present,
// the expected shape, a dtype the device path reads.
int checked_tensor(const Checkpoint& ck, const std::string& name,
                   const std::vector<int64_t>& shape, const char* st,
                   const CheckpointTensor** out) {
  const CheckpointTensor* t = ck.find(name);
  if (!t) return internal(st, "tensor not found: %s", name.c_str());
  if (t->shape != shape)
    return internal(st, "shape mismatch for `%s`: expected %s, got %s", name.c_str(),
                    shape_str(shape).c_str(), shape_str(t->shape).c_str());
  if (t->dtype < 0)
    return internal(st, "unsupported dtype %s (tensor `%s`)", t->dtype_name.c_str(),
                    name.c_str());
  *out = t;
  return ORION_HIP_OK;
}

}  // namespace

ORION_EXPORT int orion_hip_checkpoint_read_f32(const orion_hip_checkpoint* ck, const char* name,
                                               float* out, size_t count) {
  const char* st = "checkpoint_read_f32";
  if (!ck || !name || !out) return internal(st, "null argument");
  const CheckpointTensor* t = ck->ck->find(name);
  if (!t) return internal(st, "tensor not found: %s", name);
  if (t->dtype < 0)
    return internal(st, "unsupported dtype %s (tensor `%s`)", t->dtype_name.c_str(), name);
  if ((int64_t)count != numel(*t))
    return internal(st, "tensor `%s` has %lld elements, asked for %zu", name,
                    (long long)numel(*t), count);
  for (size_t i = 0; i < count; ++i) {
    if (t->dtype == ORION_DTYPE_F32) {
      std::memcpy(&out[i], static_cast<const char*>(t->data) + 4 * i, 4);
    } else {
      uint16_t h;
      std::memcpy(&h, static_cast<const char*>(t->data) + 2 * i, 2);
      out[i] = t->dtype == ORION_DTYPE_BF16 ? host_bf16_to_f32(h) : host_f16_to_f32(h);
    }
  }
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_model_load_checkpoint(orion_hip_model* model,
                                                 const orion_hip_checkpoint* ck) {
  const char* st = "load_checkpoint";
  if (!model || !ck) return internal(st, "null argument");
  const auto& d = model->desc;
  const int64_t H = d.hidden_size, F = d.intermediate_size, V = d.vocab_size;
  const int64_t qd = (int64_t)d.num_attention_heads * d.head_dim;
  const int64_t kvd = (int64_t)d.num_kv_heads * d.head_dim;
  const Checkpoint& c = *ck->ck;
  auto put = [&](int which, int layer, const std::string& name,
                 const std::vector<int64_t>& shape) -> int {
    const CheckpointTensor* t = nullptr;
    if (int rc = checked_tensor(c, name, shape, st, &t)) return rc;
    return orion_hip_model_upload_weight(model, which, layer, t->data, t->dtype,
                                         (size_t)numel(*t));
  };
  if (int rc = put(ORION_W_EMBED, -1, "model.embed_tokens.weight", {V, H})) return rc;
  for (int l = 0; l < d.num_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l);
    struct Item {
      int which;
      const char* suffix;
      std::vector<int64_t> shape;
    };
    const Item items[] = {
        {ORION_W_INPUT_NORM, ".input_layernorm.weight", {H}},
        {ORION_W_Q, ".self_attn.q_proj.weight", {qd, H}},
        {ORION_W_K, ".self_attn.k_proj.weight", {kvd, H}},
        {ORION_W_V, ".self_attn.v_proj.weight", {kvd, H}},
        {ORION_W_O, ".self_attn.o_proj.weight", {H, qd}},
        {ORION_W_POST_NORM, ".post_attention_layernorm.weight", {H}},
        {ORION_W_GATE, ".mlp.gate_proj.weight", {F, H}},
        {ORION_W_UP, ".mlp.up_proj.weight", {F, H}},
        {ORION_W_DOWN, ".mlp.down_proj.weight", {H, F}},
    };
    for (const Item& it : items)
      if (int rc = put(it.which, l, p + it.suffix, it.shape)) return rc;
    if (d.has_qkv_bias) {
      // Optional (loader.rs:226-235): absent biases stay zero; a present one
      // of the wrong shape is an error.
      const Item biases[] = {{ORION_W_Q_BIAS, ".self_attn.q_proj.bias", {qd}},
                             {ORION_W_K_BIAS, ".self_attn.k_proj.bias", {kvd}},
                             {ORION_W_V_BIAS, ".self_attn.v_proj.bias", {kvd}}};
      for (const Item& it : biases)
        if (c.find(p + it.suffix))
          if (int rc = put(it.which, l, p + it.suffix, it.shape)) return rc;
    }
  }
  if (int rc = put(ORION_W_FINAL_NORM, -1, "model.norm.weight", {H})) return rc;
  if (!d.tied_lm_head) {
    const char* head = c.find("lm_head.weight") ? "lm_head.weight" : "model.embed_tokens.weight";
    if (int rc = put(ORION_W_LM_HEAD, -1, head, {V, H})) return rc;
  }
  HIP_TRY(st, hipStreamSynchronize(model->dev->stream));
  return ORION_HIP_OK;
}

// ---------------------------------------------------------------------------
// Sampling
// ---------------------------------------------------------------------------

namespace {

// SamplingParams::validate (orion-core/src/sampling.rs:84-106), the fields the
// sampler reads.
int check_sampling(const orion_hip_sampling_params& p, int64_t row, const char* st) {
  if (!std::isfinite(p.temperature) || p.temperature < 0.0f)
    return internal(st, "row %lld: temperature must be a finite value >= 0.0, got %g",
                    (long long)row, (double)p.temperature);
  if (!std::isfinite(p.top_p) || p.top_p <= 0.0f || p.top_p > 1.0f)
    return internal(st, "row %lld: top_p must be in (0.0, 1.0], got %g", (long long)row,
                    (double)p.top_p);
  if (!std::isfinite(p.repetition_penalty) || p.repetition_penalty <= 0.0f)
    return internal(st, "row %lld: repetition_penalty must be a finite value > 0.0, got %g",
                    (long long)row, (double)p.repetition_penalty);
  if (p.top_k < 0) return internal(st, "row %lld: top_k must be >= 0", (long long)row);
  return ORION_HIP_OK;
}

int sample_on(orion_hip_device* dev, float* d_logits, int64_t rows, int64_t vocab,
              const orion_hip_sampling_params* params, const int64_t* prev_off,
              const uint32_t* prev_tok, const float* uniform, int32_t* tokens, const char* st) {
  if (rows < 0) return internal(st, "rows must be >= 0");
  if (rows == 0) return ORION_HIP_OK;
  if (!d_logits || !params || !prev_off || !uniform || !tokens)
    return internal(st, "null argument");
  if (vocab <= 0) return internal(st, "sampler received an empty logits row");
  if (vocab > kSampleMaxVocab)
    return set_err(ORION_HIP_ERR_BACKEND, st, "vocab %lld exceeds the device sampler's %lld",
                   (long long)vocab, (long long)kSampleMaxVocab);
  for (int64_t r = 0; r < rows; ++r) {
    if (int rc = check_sampling(params[r], r, st)) return rc;
    if (!(uniform[r] >= 0.0f && uniform[r] < 1.0f))
      return internal(st, "row %lld: the uniform draw must be in [0, 1)", (long long)r);
    if (prev_off[r + 1] < prev_off[r]) return internal(st, "prev_offsets must not decrease");
  }
  if (prev_off[0] != 0) return internal(st, "prev_offsets[0] must be 0");
  const int64_t nprev = prev_off[rows];
  if (nprev > 0 && !prev_tok) return internal(st, "null prev_tokens");
  // One staging copy: params | offsets | tokens | uniforms | outputs.
  const size_t o_par = 0;
  const size_t o_off = (o_par + rows * sizeof(SampleParams) + 7) & ~(size_t)7;
  const size_t o_tok = o_off + (rows + 1) * 8;
  const size_t o_uni = (o_tok + nprev * 4 + 3) & ~(size_t)3;
  const size_t o_out = o_uni + rows * 4;
  const size_t total = o_out + rows * 4;
  std::vector<char> host(total);
  for (int64_t r = 0; r < rows; ++r) {
    const SampleParams sp{params[r].temperature, params[r].top_k, params[r].top_p,
                          params[r].repetition_penalty};
    std::memcpy(host.data() + o_par + r * sizeof(SampleParams), &sp, sizeof(sp));
  }
  std::memcpy(host.data() + o_off, prev_off, (rows + 1) * 8);
  if (nprev) std::memcpy(host.data() + o_tok, prev_tok, nprev * 4);
  std::memcpy(host.data() + o_uni, uniform, rows * 4);
  HIP_TRY(st, hipSetDevice(dev->ordinal));
  HIP_TRY(st, dev->sample_io.reserve(total));
  HIP_TRY(st, dev->sample_ws.reserve((size_t)rows * vocab * 4));
  hipStream_t stream = dev->stream;
  char* d = static_cast<char*>(dev->sample_io.ptr);
  HIP_TRY(st, hipMemcpyAsync(d, host.data(), o_out, hipMemcpyHostToDevice, stream));
  HIP_TRY(st, launch_sample(stream, d_logits, rows, vocab,
                            reinterpret_cast<const SampleParams*>(d + o_par),
                            reinterpret_cast<const int64_t*>(d + o_off),
                            reinterpret_cast<const uint32_t*>(d + o_tok),
                            reinterpret_cast<const float*>(d + o_uni),
                            dev->sample_ws.as<float>(), reinterpret_cast<int32_t*>(d + o_out)));
  HIP_TRY(st, hipMemcpyAsync(tokens, d + o_out, rows * 4, hipMemcpyDeviceToHost, stream));
  HIP_TRY(st, hipStreamSynchronize(stream));
  for (int64_t r = 0; r < rows; ++r)  // a greedy row with no number above -inf
    if (tokens[r] < 0) return internal(st, "row %lld: argmax over empty logits", (long long)r);
  return ORION_HIP_OK;
}

}  // namespace

ORION_EXPORT int orion_hip_sample(orion_hip_device* dev, float* d_logits, int64_t rows,
                                  int64_t vocab, const orion_hip_sampling_params* params,
                                  const int64_t* prev_offsets, const uint32_t* prev_tokens,
                                  const float* h_uniform, int32_t* h_tokens) {
  if (!dev) return internal("sample", "null device");
  return sample_on(dev, d_logits, rows, vocab, params, prev_offsets, prev_tokens, h_uniform,
                   h_tokens, "sample");
}

ORION_EXPORT int orion_hip_model_sample(orion_hip_model* model,
                                        const orion_hip_sampling_params* params,
                                        const int64_t* prev_offsets, const uint32_t* prev_tokens,
                                        const float* h_uniform, int32_t* h_tokens) {
  const char* st = "model_sample";
  if (!model) return internal(st, "null model");
  if (model->last_rows <= 0) return internal(st, "no forward has produced logits yet");
  return sample_on(model->dev, model->logits.as<float>(), model->last_rows,
                   model->desc.vocab_size, params, prev_offsets, prev_tokens, h_uniform,
                   h_tokens, st);
}

ORION_EXPORT int orion_hip_model_download_weight(orion_hip_model* model, int which, int layer,
                                                 float* host, size_t count) {
  const char* st = "download_weight";
  WeightSlot s;
  if (int rc = weight_slot(model, which, layer, &s)) return rc;
  if ((int64_t)count != s.rows * s.cols)
    return internal(st, "weight %d has %lld elements, asked for %zu", which,
                    (long long)(s.rows * s.cols), count);
  HIP_TRY(st, hipSetDevice(model->dev->ordinal));
  hipStream_t stream = model->dev->stream;
  const size_t esz = s.bf16 ? 2 : 4;
  std::vector<char> raw(count * esz);
  if (s.group == 0) {
    HIP_TRY(st, hipMemcpyAsync(raw.data(), s.base, count * esz, hipMemcpyDeviceToHost, stream));
  } else {
    const size_t row_bytes = (size_t)s.cols * esz;
    HIP_TRY(st, hipMemcpy2DAsync(raw.data(), s.group * row_bytes,
                                 static_cast<char*>(s.base) + s.offset * row_bytes,
                                 s.stride * row_bytes, s.group * row_bytes,
                                 (size_t)(s.rows / s.group), hipMemcpyDeviceToHost, stream));
  }
  HIP_TRY(st, hipStreamSynchronize(stream));
  if (s.bf16) {
    const uint16_t* b = reinterpret_cast<const uint16_t*>(raw.data());
    for (size_t i = 0; i < count; ++i) host[i] = host_bf16_to_f32(b[i]);
  } else {
    std::memcpy(host, raw.data(), count * 4);
  }
  return ORION_HIP_OK;
}

ORION_EXPORT float orion_hip_synthetic_value(uint64_t seed, int which, int layer, uint64_t index,
                                             float std_) {
  const bool is_norm =
      which == ORION_W_FINAL_NORM || which == ORION_W_INPUT_NORM || which == ORION_W_POST_NORM;
  if (is_norm) return 1.0f;
  const float mul = std_ / kIrwinHallSd;
  const uint64_t key = synthetic_key(seed, which, which >= ORION_W_INPUT_NORM ? layer : -1);
  return host_bf16_to_f32(host_f32_to_bf16(synthetic_normal(key, index, mul)));
}

static int init_one(orion_hip_model* m, int which, int layer, uint64_t seed, float std_) {
  const char* st = "init_synthetic";
  WeightSlot s;
  if (int rc = weight_slot(m, which, layer, &s)) return rc;
  m->packs_valid = false;
  hipStream_t stream = m->dev->stream;
  const float mul = std_ / kIrwinHallSd;
  const uint64_t key = synthetic_key(seed, which, which >= ORION_W_INPUT_NORM ? layer : -1);
  const int64_t count = s.rows * s.cols;
  const bool is_norm =
      which == ORION_W_FINAL_NORM || which == ORION_W_INPUT_NORM || which == ORION_W_POST_NORM;
  if (is_norm) {
    HIP_TRY(st, launch_fill_f32(stream, static_cast<float*>(s.base), count, 1.0f));
    return ORION_HIP_OK;
  }
  if (!s.bf16) {
    HIP_TRY(st, launch_synthetic_f32(stream, static_cast<float*>(s.base), count, key, mul));
    return ORION_HIP_OK;
  }
  if (s.group == 0) {
    HIP_TRY(st, launch_synthetic_bf16(stream, static_cast<uint16_t*>(s.base), count, key, mul));
    return ORION_HIP_OK;
  }
  // Interleaved gate/up: generate in logical order into a scratch buffer,
  // then scatter the row groups.
  DevBuf tmp;
  HIP_TRY(st, tmp.reserve((size_t)count * 2));
  HIP_TRY(st, launch_synthetic_bf16(stream, tmp.as<uint16_t>(), count, key, mul));
  const size_t row_bytes = (size_t)s.cols * 2;
  HIP_TRY(st, hipMemcpy2DAsync(static_cast<char*>(s.base) + s.offset * row_bytes,
                               s.stride * row_bytes, tmp.ptr, s.group * row_bytes,
                               s.group * row_bytes, (size_t)(s.rows / s.group),
                               hipMemcpyDeviceToDevice, stream));
  HIP_TRY(st, hipStreamSynchronize(stream));
  tmp.release();
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_model_init_synthetic(orion_hip_model* model, uint64_t seed, float std_) {
  HIP_TRY("init_synthetic", hipSetDevice(model->dev->ordinal));
  const auto& d = model->desc;
  if (int rc = init_one(model, ORION_W_EMBED, -1, seed, std_)) return rc;
  if (!d.tied_lm_head)
    if (int rc = init_one(model, ORION_W_LM_HEAD, -1, seed, std_)) return rc;
  if (int rc = init_one(model, ORION_W_FINAL_NORM, -1, seed, std_)) return rc;
  for (int l = 0; l < d.num_layers; ++l) {
    for (int w = ORION_W_INPUT_NORM; w <= ORION_W_DOWN; ++w) {
      if ((w == ORION_W_Q_BIAS || w == ORION_W_K_BIAS || w == ORION_W_V_BIAS) && !d.has_qkv_bias)
        continue;
      if (int rc = init_one(model, w, l, seed, std_)) return rc;
    }
  }
  HIP_TRY("init_synthetic", hipStreamSynchronize(model->dev->stream));
  return ORION_HIP_OK;
}

// ---------------------------------------------------------------------------
// KV arena access (KvStore::read/write, attention.rs:107-175)
// ---------------------------------------------------------------------------

static int kv_bounds(orion_hip_model* m, int64_t layer, uint32_t block, int64_t slot,
                     int64_t head, int64_t vec_len, const char* st) {
  const auto& d = m->desc;
  if (layer < 0 || layer >= d.num_layers)
    return internal(st, "layer %lld out of range (have %d)", (long long)layer, d.num_layers);
  if ((int64_t)block >= d.num_blocks)
    return internal(st, "block %u out of range (have %d)", block, d.num_blocks);
  if (slot < 0 || slot >= d.block_size)
    return internal(st, "slot %lld out of range (block holds %d)", (long long)slot, d.block_size);
  if (head < 0 || head >= d.num_kv_heads)
    return internal(st, "kv head %lld out of range (have %d)", (long long)head, d.num_kv_heads);
  if (vec_len != d.head_dim)
    return internal(st, "vector length %lld does not match head_dim %d", (long long)vec_len,
                    d.head_dim);
  return ORION_HIP_OK;
}

static size_t kv_offset_elems(orion_hip_model* m, int64_t layer, uint32_t block, int is_value,
                              int64_t slot, int64_t head) {
  const ArenaStrides a = arena_strides(m->kv);
  return (size_t)(layer * a.layer + (int64_t)block * a.blk + (is_value ? a.v_off : 0) +
                  slot * a.slot + head * a.head);
}

ORION_EXPORT int orion_hip_model_kv_read(orion_hip_model* model, int64_t layer, uint32_t block,
                                         int64_t slot, int64_t head, int is_value, float* out) {
  const char* st = "kv_read";
  if (int rc = kv_bounds(model, layer, block, slot, head, model->desc.head_dim, st)) return rc;
  const size_t off = kv_offset_elems(model, layer, block, is_value, slot, head);
  const int64_t d = model->desc.head_dim;
  hipStream_t stream = model->dev->stream;
  if (model->kv.dtype_bf16) {
    std::vector<uint16_t> tmp(d);
    HIP_TRY(st, hipMemcpyAsync(tmp.data(), static_cast<uint16_t*>(model->arena) + off, d * 2,
                               hipMemcpyDeviceToHost, stream));
    HIP_TRY(st, hipStreamSynchronize(stream));
    for (int64_t i = 0; i < d; ++i) out[i] = host_bf16_to_f32(tmp[i]);
  } else {
    HIP_TRY(st, hipMemcpyAsync(out, static_cast<float*>(model->arena) + off, d * 4,
                               hipMemcpyDeviceToHost, stream));
    HIP_TRY(st, hipStreamSynchronize(stream));
  }
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_model_kv_write(orion_hip_model* model, int64_t layer, uint32_t block,
                                          int64_t slot, int64_t head, int is_value,
                                          const float* vec, int64_t len) {
  const char* st = "kv_write";
  if (int rc = kv_bounds(model, layer, block, slot, head, len, st)) return rc;
  const size_t off = kv_offset_elems(model, layer, block, is_value, slot, head);
  hipStream_t stream = model->dev->stream;
  if (model->kv.dtype_bf16) {
    std::vector<uint16_t> tmp(len);
    for (int64_t i = 0; i < len; ++i) tmp[i] = host_f32_to_bf16(vec[i]);
    HIP_TRY(st, hipMemcpyAsync(static_cast<uint16_t*>(model->arena) + off, tmp.data(), len * 2,
                               hipMemcpyHostToDevice, stream));
    HIP_TRY(st, hipStreamSynchronize(stream));
  } else {
    HIP_TRY(st, hipMemcpyAsync(static_cast<float*>(model->arena) + off, vec, len * 4,
                               hipMemcpyHostToDevice, stream));
    HIP_TRY(st, hipStreamSynchronize(stream));
  }
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_model_kv_arena(orion_hip_model* model, void** d_arena, size_t* bytes) {
  *d_arena = model->arena;
  *bytes = model->arena_bytes;
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_model_kv_layout(orion_hip_model* model, orion_hip_kv_layout* out) {
  const KvGeom& g = model->kv;
  out->num_layers = g.num_layers;
  out->num_blocks = g.num_blocks;
  out->block_size = g.block_size;
  out->num_kv_heads = g.num_kv_heads;
  out->head_dim = g.head_dim;
  out->dtype = g.dtype_bf16 ? ORION_DTYPE_BF16 : ORION_DTYPE_F32;
  out->head_major = g.head_major ? 1 : 0;
  return ORION_HIP_OK;
}

// ---------------------------------------------------------------------------
// Forward (transformer.rs:359-442)
// ---------------------------------------------------------------------------

namespace {

struct HostBatch {
  std::vector<int32_t> row_seq;
  std::vector<int32_t> last_rows;
  std::vector<int64_t> seq_max_pos;  // largest position of each sequence's rows
  int64_t max_position = 0;
};

// ForwardBatch::validate (traits.rs:232-261) plus every check the reference
// performs while computing (transformer.rs:212-217, :257-262, :376-385,
// attention.rs:136-175, :411-419), done once on the host before launch; the
// block ids themselves are checked by validate_tables, before the first
// launch that reads or writes the KV arena.
int validate_batch(orion_hip_model* m, const orion_hip_batch* b, HostBatch* hb) {
  const char* st = "forward";
  const auto& d = m->desc;
  const int64_t n = b->num_tokens, S = b->num_seqs;
  if (n < 0 || S < 0) return internal(st, "negative batch sizes");
  int64_t summed = 0;
  for (int64_t s = 0; s < S; ++s) {
    if (b->slot_token_counts[s] < 0) return internal(st, "negative slot token count");
    summed += b->slot_token_counts[s];
  }
  if (summed != n)
    return internal(st, "ForwardBatch slot token counts sum to %lld but there are %lld tokens",
                    (long long)summed, (long long)n);
  if (n == 0) return ORION_HIP_OK;
  if (b->block_table_offsets[0] != 0) return internal(st, "block table offsets must start at 0");
  for (int64_t s = 0; s < S; ++s) {
    if (b->block_table_offsets[s + 1] < b->block_table_offsets[s])
      return internal(st, "block table offsets must be non-decreasing");
    if (b->slot_token_counts[s] == 0)
      return internal(st, "a scheduled sequence contributed zero tokens");
  }
  hb->row_seq.resize(n);
  hb->last_rows.resize(S);
  std::vector<int64_t>& seq_max_pos = hb->seq_max_pos;
  seq_max_pos.assign(S, -1);
  int64_t row = 0;
  for (int64_t s = 0; s < S; ++s) {
    for (int64_t c = 0; c < b->slot_token_counts[s]; ++c, ++row) {
      hb->row_seq[row] = (int32_t)s;
      const uint32_t tok = b->tokens[row];
      const int64_t pos = b->positions[row];
      if ((int64_t)tok >= d.vocab_size)
        return internal(st, "token id %u is outside the vocabulary of %d", tok, d.vocab_size);
      const int64_t tlen = b->block_table_offsets[s + 1] - b->block_table_offsets[s];
      if (pos / d.block_size >= tlen)
        return internal(st, "position %lld has no block in the table for sequence %lld",
                        (long long)pos, (long long)s);
      if (pos >= d.max_position_embeddings)
        return internal(st, "position %lld exceeds the RoPE table (%d entries)", (long long)pos,
                        d.max_position_embeddings);
      seq_max_pos[s] = std::max(seq_max_pos[s], pos);
      hb->max_position = std::max(hb->max_position, pos);
    }
    hb->last_rows[s] = (int32_t)(row - 1);
  }
  return ORION_HIP_OK;
}

// Every block a row can attend to (positions 0..=pos) must exist in the arena
// (attention.rs:136-175: the reference's KvStore bounds check).
int validate_tables(orion_hip_model* m, const orion_hip_batch* b, const HostBatch& hb) {
  const char* st = "forward";
  const auto& d = m->desc;
  for (int64_t s = 0; s < b->num_seqs; ++s) {
    const int64_t used = hb.seq_max_pos[s] / d.block_size + 1;
    const uint32_t* tbl = b->block_table_ids + b->block_table_offsets[s];
    for (int64_t i = 0; i < used; ++i)
      if ((int64_t)tbl[i] >= d.num_blocks)
        return internal(st, "block %u out of range (have %d)", tbl[i], d.num_blocks);
  }
  return ORION_HIP_OK;
}

}  // namespace

// The layer matrices and the (untied) LM head, with their packed copies and
// geometry.  A tied head's packed copy comes from the embedding, which stays
// row-major (the embedding gather reads it).
struct MatrixRef {
  uint16_t** rowmajor;
  uint16_t** packed;
  int64_t N, K;
  bool deferred;  // QKV: its partials go to RoPE unreduced
};
static std::vector<MatrixRef> matrices(orion_hip_model* m) {
  const auto& d = m->desc;
  const int64_t H = d.hidden_size, F = d.intermediate_size, V = d.vocab_size;
  std::vector<MatrixRef> v;
  for (LayerDev& L : m->layers) {
    v.push_back({&L.w_qkv, &L.p_qkv, m->qkvd, H, true});
    v.push_back({&L.w_o, &L.p_o, H, m->qd, false});
    v.push_back({&L.w_gu, &L.p_gu, 2 * F, H, false});
    v.push_back({&L.w_down, &L.p_down, H, F, false});
  }
  if (!d.tied_lm_head) v.push_back({&m->w_lm, &m->p_head, V, H, false});
  return v;
}

// Writes the packed copy of every layer matrix and the LM head (allocated on
// first use) from the row-major weights, in the geometry each forward GEMM
// call uses.
static hipError_t make_packs(orion_hip_model* m) {
  const auto& d = m->desc;
  hipStream_t stream = m->dev->stream;
  auto one = [&](uint16_t** dst, const uint16_t* w, int64_t N, int64_t K,
                 bool deferred) -> hipError_t {
    const size_t bytes = gemv_packed_bytes(N, K, deferred);
    if (!bytes) return hipErrorInvalidValue;
    if (!*dst) {
      hipError_t e = m->alloc(dst, bytes / 2);
      if (e != hipSuccess) return e;
    }
    return launch_gemv_pack(stream, w, N, K, deferred, *dst);
  };
  if (!m->rowmajor_live) return hipErrorInvalidValue;
  for (const MatrixRef& r : matrices(m)) {
    hipError_t e = one(r.packed, *r.rowmajor, r.N, r.K, r.deferred);
    if (e != hipSuccess) return e;
  }
  if (d.tied_lm_head) {
    hipError_t e = one(&m->p_head, m->w_embed, d.vocab_size, d.hidden_size, false);
    if (e != hipSuccess) return e;
  }
  m->packs_valid = true;
  return hipSuccess;
}

// Frees the row-major layer matrices and LM head once the packed copies hold
// the weights (one copy of every weight in HBM).
static hipError_t release_rowmajor(orion_hip_model* m) {
  if (!m->rowmajor_live || !m->packs_valid) return hipSuccess;
  for (const MatrixRef& r : matrices(m)) {
    hipError_t e = m->release(r.rowmajor);
    if (e != hipSuccess) return e;
  }
  m->rowmajor_live = false;
  return hipSuccess;
}

// Brings the row-major matrices back (unpacked from the packed copies) before
// a weight is written or read back.
static hipError_t ensure_rowmajor(orion_hip_model* m) {
  if (m->rowmajor_live) return hipSuccess;
  for (const MatrixRef& r : matrices(m)) {
    hipError_t e = m->alloc(r.rowmajor, (size_t)(r.N * r.K));
    if (e == hipSuccess)
      e = launch_gemv_unpack(m->dev->stream, *r.packed, r.N, r.K, r.deferred, *r.rowmajor);
    if (e != hipSuccess) return e;
  }
  m->rowmajor_live = true;
  return hipSuccess;
}

ORION_EXPORT int orion_hip_model_forward(orion_hip_model* m, const orion_hip_batch* b,
                                         float* logits_out, int64_t* argmax_out) {
  const char* st = "forward";
  HostBatch hb;
  if (int rc = validate_batch(m, b, &hb)) return rc;
  const int64_t n = b->num_tokens, S = b->num_seqs;
  if (n == 0) return ORION_HIP_OK;
  const auto& d = m->desc;
  const int64_t H = d.hidden_size, F = d.intermediate_size, V = d.vocab_size;
  const int64_t Hq = d.num_attention_heads;
  hipStream_t stream = m->dev->stream;
  HIP_TRY(st, hipSetDevice(m->dev->ordinal));

  // ---- capacity ----
  const int64_t nbt = b->block_table_offsets[S];
  HIP_TRY(st, m->hidden.reserve(n * H * 4));
  HIP_TRY(st, m->xn.reserve(n * H * 4));
  HIP_TRY(st, m->qkv.reserve(n * m->qkvd * 4));
  HIP_TRY(st, m->qrot.reserve(n * m->qd * 4));
  HIP_TRY(st, m->attn.reserve(n * m->qd * 4));
  HIP_TRY(st, m->act.reserve(n * F * 4));
  HIP_TRY(st, m->logits.reserve(S * V * 4));
  HIP_TRY(st, m->argmax.reserve(S * 8));
  // Decode-shaped batches run the layer with the split-K GEMM fusions: each
  // residual-add GEMM also writes the per-row sums of squares, the next GEMM
  // applies the RMSNorm to its input, and the QKV partials go straight into
  // RoPE + cache write.  ORION_GEMM_FUSE=0 runs the separate launches (read
  // per call, so a test can run one batch both ways in one process).
  const char* fuse_env = getenv("ORION_GEMM_FUSE");
  const bool allow_fuse = !(fuse_env && fuse_env[0] == '0');
  const bool fused = allow_fuse && gemm_splitk_fusable(n, m->qkvd, H) &&
                     gemm_splitk_fusable(n, H, m->qd) && gemm_splitk_fusable(n, 2 * F, H) &&
                     gemm_splitk_fusable(n, H, F);
  const int nslots = gemm_sumsq_slots(H);
  if (fused) HIP_TRY(st, m->sumsq.reserve(n * nslots * 8));
  // Every GEMM reads the packed weight copies (the decode kernel's order),
  // made on the first forward after a weight write, after which the row-major
  // matrices are freed: one copy of each weight stays in HBM.
  // ORION_GEMV_PACK=0 keeps the row-major matrices and reads them instead
  // (A/B knob, read once).
  static const bool allow_pack = [] {
    const char* v = getenv("ORION_GEMV_PACK");
    return !(v && v[0] == '0');
  }();
  const bool pack_layers = allow_pack, pack_head = allow_pack;
  if (allow_pack) {
    if (!m->packs_valid) HIP_TRY(st, make_packs(m));
    HIP_TRY(st, release_rowmajor(m));
  } else {
    HIP_TRY(st, ensure_rowmajor(m));
  }
  // Attention routing, shared by every layer.  A sequence whose rows are a
  // chunk of consecutive positions with at least half a prefill tile of
  // (row, query head) pairs goes to the MFMA prefill kernel (bf16 arena);
  // every other row goes to the split-K decode kernel.
  const int64_t G = Hq / d.num_kv_heads;
  std::vector<uint8_t> skip(n, 0);
  std::vector<int32_t> pf_start, pf_count;
  std::vector<uint32_t> pf_pos;
  std::vector<int64_t> pf_btoff;
  // Prefill attention operands: Q and P as hi + lo bf16 pairs (default);
  // ORION_PREFILL_OPERANDS=bf16 rounds both to bf16, =q keeps only Q as a
  // pair, =p only P (measurement knob, read per call).
  const char* pf_env = getenv("ORION_PREFILL_OPERANDS");
  int pf_ops = kPrefillQHiLo | kPrefillPHiLo;
  if (pf_env && std::strcmp(pf_env, "bf16") == 0) pf_ops = 0;
  if (pf_env && std::strcmp(pf_env, "q") == 0) pf_ops = kPrefillQHiLo;
  if (pf_env && std::strcmp(pf_env, "p") == 0) pf_ops = kPrefillPHiLo;
  // ORION_PREFILL_ROUTE=0 sends every row to the decode kernel (read per
  // call; lets tests compare the two routes on one batch).
  const char* route = getenv("ORION_PREFILL_ROUTE");
  const bool route_pf = !(route && route[0] == '0');
  if (route_pf && m->kv.dtype_bf16 &&
      (d.head_dim == 64 || d.head_dim == 128 || d.head_dim == 256)) {
    int64_t r0 = 0;
    for (int64_t s = 0; s < S; ++s) {
      const int64_t c = b->slot_token_counts[s];
      bool chunk = c * G >= 64;  // enough (row, head) pairs to fill MFMA row tiles
      for (int64_t i = 1; chunk && i < c; ++i)
        chunk = b->positions[r0 + i] == b->positions[r0] + (uint32_t)i;
      if (chunk) {
        pf_start.push_back((int32_t)r0);
        pf_count.push_back((int32_t)c);
        pf_pos.push_back(b->positions[r0]);
        pf_btoff.push_back(b->block_table_offsets[s]);
        std::fill(skip.begin() + r0, skip.begin() + r0 + c, (uint8_t)1);
      }
      r0 += c;
    }
  }
  const int64_t npf = (int64_t)pf_start.size();

  // Pinned staging area i (0: the batch, 1: the attention plans), grown on
  // demand.  Each forward ends with a stream sync, so the previous forward's
  // copies out of both are complete.
  auto staging = [&](int i, size_t bytes) -> hipError_t {
    if (bytes <= m->pinned_bytes[i]) return hipSuccess;
    if (m->pinned[i]) {
      hipError_t e = hipStreamSynchronize(stream);
      if (e == hipSuccess) e = hipHostFree(m->pinned[i]);
      if (e != hipSuccess) return e;
      m->pinned[i] = nullptr;
      m->pinned_bytes[i] = 0;
    }
    const size_t cap = std::max<size_t>(bytes * 2, 1 << 16);
    hipError_t e = hipHostMalloc(&m->pinned[i], cap, hipHostMallocDefault);
    if (e != hipSuccess) {
      m->pinned[i] = nullptr;
      return e;
    }
    m->pinned_bytes[i] = cap;
    return hipSuccess;
  };

  // ---- upload the batch: tokens, positions, row sequences, last rows and
  // block tables, one pinned staging area, one copy ----
  const size_t o_tok = 0;
  const size_t o_pos = o_tok + n * 4;
  const size_t o_rs = o_pos + n * 4;
  const size_t o_last = o_rs + n * 4;
  const size_t o_btoff = (o_last + S * 4 + 7) & ~(size_t)7;
  const size_t o_btids = o_btoff + (S + 1) * 8;
  const size_t total = o_btids + nbt * 4;
  HIP_TRY(st, staging(0, total));
  HIP_TRY(st, m->b_batch.reserve(total));
  {
    char* hp = static_cast<char*>(m->pinned[0]);
    std::memcpy(hp + o_tok, b->tokens, n * 4);
    std::memcpy(hp + o_pos, b->positions, n * 4);
    std::memcpy(hp + o_rs, hb.row_seq.data(), n * 4);
    std::memcpy(hp + o_last, hb.last_rows.data(), S * 4);
    std::memcpy(hp + o_btoff, b->block_table_offsets, (S + 1) * 8);
    std::memcpy(hp + o_btids, b->block_table_ids, nbt * 4);
    HIP_TRY(st, hipMemcpyAsync(m->b_batch.ptr, hp, total, hipMemcpyHostToDevice, stream));
  }
  const char* dp = m->b_batch.as<char>();
  const uint32_t* d_tok = reinterpret_cast<const uint32_t*>(dp + o_tok);
  const uint32_t* d_pos = reinterpret_cast<const uint32_t*>(dp + o_pos);
  const int32_t* d_rs = reinterpret_cast<const int32_t*>(dp + o_rs);
  const int32_t* d_last = reinterpret_cast<const int32_t*>(dp + o_last);
  const int64_t* d_btoff = reinterpret_cast<const int64_t*>(dp + o_btoff);
  const uint32_t* d_btids = reinterpret_cast<const uint32_t*>(dp + o_btids);

  // ---- block ids and attention plans.  Nothing before layer 0's RoPE / KV
  // write reads the arena or the plans, so the block ids are checked and the
  // plans built on the host (and copied up) while the GPU runs the embedding
  // and layer 0's QKV GEMM. ----
  PrefillPlan pfp;
  DecodePlanHost plan;
  DecodePlanDev dplan, pf_merge;
  PrefillSplitOut pf_out;
  const PrefillTile* d_pforder = nullptr;
  const int64_t* d_pfoff = nullptr;
  const int32_t *d_pfstart = nullptr, *d_pfcount = nullptr;
  const uint32_t* d_pfpos = nullptr;
  bool pf_split = false, o_presplit = false;
  // (set below, before the plans are built: whether layers run on pre-split
  // activations decides whether the O GEMM can take them too)
  bool presplit = false;
  auto plan_attention = [&]() -> int {
    if (int rc = validate_tables(m, b, hb)) return rc;
    if (npf)
      build_prefill_order(pf_start.data(), pf_count.data(), pf_pos.data(), npf, G,
                          d.num_kv_heads, m->dev->wave_slots / 8, &pfp, d.head_dim);
    pf_split = pfp.max_parts > 1;
    // Decode plan (longest-first chunk list) over the remaining rows.
    build_decode_plan(b->positions, hb.row_seq.data(), b->block_table_offsets,
                      b->block_table_ids, n, d.num_kv_heads, d.block_size, m->dev->wave_slots,
                      npf ? skip.data() : nullptr, &plan, decode_pack_rows(m->kv, Hq));
    // One workspace for the decode splits and the prefill key parts (their
    // launches are ordered on the stream: the decode merge has read the
    // splits before the prefill kernel writes its parts).
    HIP_TRY(st, m->ws.reserve(std::max(decode_workspace_bytes(n, Hq, d.head_dim, plan.max_splits),
                                       decode_workspace_bytes(n, Hq, d.head_dim, pfp.max_parts))));
    const std::vector<PrefillTile>& pf_order = pfp.order;
    const size_t o_work = 0;
    const size_t o_nsplit = o_work + plan.work.size() * sizeof(DecodeWork);
    const size_t o_pfoff = (o_nsplit + plan.row_nsplit.size() * 4 + 7) & ~(size_t)7;
    const size_t o_pfstart = o_pfoff + npf * 8;
    const size_t o_pfcount = o_pfstart + npf * 4;
    const size_t o_pfpos = o_pfcount + npf * 4;
    const size_t o_drows = o_pfpos + npf * 4;
    const size_t o_pforder = (o_drows + plan.rows.size() * 4 + 7) & ~(size_t)7;
    const size_t o_pfsplit = o_pforder + pf_order.size() * sizeof(PrefillTile);
    const size_t o_pfparts = o_pfsplit + (pf_split ? pfp.split_rows.size() * 4 : 0);
    const size_t o_packrows = o_pfparts + (pf_split ? pfp.row_parts.size() * 4 : 0);
    const size_t ptotal = std::max<size_t>(o_packrows + plan.pack_rows.size() * 4, 8);
    HIP_TRY(st, staging(1, ptotal));
    HIP_TRY(st, m->b_plan.reserve(ptotal));
    char* hp = static_cast<char*>(m->pinned[1]);
    std::memcpy(hp + o_work, plan.work.data(), plan.work.size() * sizeof(DecodeWork));
    std::memcpy(hp + o_nsplit, plan.row_nsplit.data(), plan.row_nsplit.size() * 4);
    std::memcpy(hp + o_pfoff, pf_btoff.data(), npf * 8);
    std::memcpy(hp + o_pfstart, pf_start.data(), npf * 4);
    std::memcpy(hp + o_pfcount, pf_count.data(), npf * 4);
    std::memcpy(hp + o_pfpos, pf_pos.data(), npf * 4);
    std::memcpy(hp + o_drows, plan.rows.data(), plan.rows.size() * 4);
    std::memcpy(hp + o_pforder, pf_order.data(), pf_order.size() * sizeof(PrefillTile));
    if (pf_split) {
      std::memcpy(hp + o_pfsplit, pfp.split_rows.data(), pfp.split_rows.size() * 4);
      std::memcpy(hp + o_pfparts, pfp.row_parts.data(), pfp.row_parts.size() * 4);
    }
    std::memcpy(hp + o_packrows, plan.pack_rows.data(), plan.pack_rows.size() * 4);
    char* pp = m->b_plan.as<char>();
    HIP_TRY(st, hipMemcpyAsync(pp, hp, ptotal, hipMemcpyHostToDevice, stream));
    dplan.work = reinterpret_cast<const DecodeWork*>(pp + o_work);
    dplan.row_nsplit = reinterpret_cast<const int32_t*>(pp + o_nsplit);
    dplan.num_work = (int)plan.work.size();
    dplan.chunk = plan.chunk;
    dplan.max_splits = plan.max_splits;
    dplan.ws = m->ws.as<float>();
    dplan.ws_bytes = m->ws.bytes;
    dplan.stream_kv = plan.stream_kv;
    dplan.mixed_kv = plan.mixed_kv;
    dplan.num_packed = plan.num_packed;
    dplan.pack_rows = reinterpret_cast<const int32_t*>(pp + o_packrows);
    dplan.pack_r = plan.pack_r;
    if (npf) {
      dplan.rows = reinterpret_cast<const int32_t*>(pp + o_drows);
      dplan.num_rows = (int)plan.rows.size();
    }
    d_pfoff = reinterpret_cast<const int64_t*>(pp + o_pfoff);
    d_pfstart = reinterpret_cast<const int32_t*>(pp + o_pfstart);
    d_pfcount = reinterpret_cast<const int32_t*>(pp + o_pfcount);
    d_pfpos = reinterpret_cast<const uint32_t*>(pp + o_pfpos);
    d_pforder = reinterpret_cast<const PrefillTile*>(pp + o_pforder);
    // the prefill key parts' merge (split rows, parts per row, the workspace)
    if (pf_split) {
      pf_merge.rows = reinterpret_cast<const int32_t*>(pp + o_pfsplit);
      pf_merge.num_rows = (int)pfp.split_rows.size();
      pf_merge.row_nsplit = reinterpret_cast<const int32_t*>(pp + o_pfparts);
      pf_merge.max_splits = pfp.max_parts;
      pf_merge.ws = m->ws.as<float>();
      pf_merge.ws_bytes = m->ws.bytes;
      pf_out.ws_o = pf_merge.ws;
      pf_out.ws_ml = pf_merge.ws + n * Hq * pfp.max_parts * d.head_dim;
      pf_out.max_parts = pfp.max_parts;
    }
    // The O GEMM's input is pre-split too when the prefill kernel writes
    // every attention row itself (no decode rows, no key parts).
    const char* presplit_env = getenv("ORION_GEMM_PRESPLIT");
    o_presplit = presplit && plan.work.empty() && npf > 0 && !pf_split &&
                 !(presplit_env && presplit_env[0] == '2');
    pf_out.out_hilo = o_presplit ? 1 : 0;
    return ORION_HIP_OK;
  };

  float* hidden = m->hidden.as<float>();
  float* xn = m->xn.as<float>();
  float* qkv = m->qkv.as<float>();
  float* qrot = m->qrot.as<float>();
  float* attn = m->attn.as<float>();
  float* act = m->act.as<float>();

  double* sumsq = fused ? m->sumsq.as<double>() : nullptr;
  // The norm a GEMM applies to its input (fused) / nothing (separate norm).
  auto norm_in = [&](const float* weight) {
    GemmFuse f;
    if (fused) {
      f.norm_sumsq = sumsq;
      f.norm_slots = nslots;
      f.norm_weight = weight;
      f.norm_eps = d.rms_norm_eps;
    }
    return f;
  };
  GemmFuse accumulate;  // residual-add GEMMs: out += x W^T (+ row sums of squares)
  accumulate.sumsq_out = sumsq;
  GemmPartials part{};
  // Prefill-shaped batches (every layer GEMM on the LDS-tiled kernel): the
  // two RMSNorms and the SwiGLU epilogue write their outputs already split
  // into the GEMM's bf16 hi/lo operands, so the QKV, gate/up and down GEMMs
  // load their activation fragments as they are.  The same truncated split,
  // so the results are bit-identical; ORION_GEMM_PRESPLIT=0 keeps f32
  // activations (measurement knob, read per call).
  const char* presplit_env = getenv("ORION_GEMM_PRESPLIT");
  const char* act_env = getenv("ORION_GEMM_ACT");
  presplit = !fused && n > 64 && pack_layers && H % 8 == 0 && F % 8 == 0 &&
             !(presplit_env && presplit_env[0] == '0') && !(act_env && act_env[0] == 'b');
  // (the fused route's embed also leaves the row sums of squares, so layer
  // 0's QKV GEMM applies its RMSNorm like every later layer's)
  HIP_TRY(st, launch_embed(stream, d_tok, n, m->w_embed, H, hidden, sumsq));
  for (int64_t l = 0; l < d.num_layers; ++l) {
    const LayerDev& L = m->layers[l];
    // QKV input: rms_norm(hidden) * input_norm -- inside the QKV GEMM when
    // the embed or the previous layer's down GEMM left the sums of squares,
    // else a kernel of its own.
    GemmFuse qkv_f = norm_in(L.input_norm);
    const float* qkv_x = hidden;
    if (!qkv_f.norm_sumsq) {
      HIP_TRY(st, launch_rmsnorm(stream, hidden, nullptr, L.input_norm, n, H, d.rms_norm_eps, xn,
                                 presplit));
      qkv_x = xn;
      qkv_f.x_hilo = presplit;
    }
    qkv_f.defer = &part;
    if (pack_layers) qkv_f.w_packed = L.p_qkv, qkv_f.w_packed_deferred = true;
    HIP_TRY(st, gemm_on(m->dev, qkv_x, L.w_qkv, L.b_qkv, n, m->qkvd, H, Epilogue::kStore, qkv,
                        &qkv_f));
    if (l == 0)
      if (int rc = plan_attention()) return rc;
    HIP_TRY(st, launch_rope_and_cache(stream, m->kv, m->arena, l, n, Hq, qkv, m->qkvd, qrot,
                                      qkv + m->qd, m->qkvd, qkv + m->qd + m->kvd, m->qkvd, d_pos,
                                      d_rs, d_btoff, d_btids, m->rope_cos, m->rope_sin, &part));
    HIP_TRY(st, launch_paged_decode(stream, m->kv, m->arena, l, qrot, n, Hq, d_pos, d_rs, d_btoff,
                                    d_btids, dplan, attn));
    if (npf) {
      HIP_TRY(st, launch_paged_prefill(stream, m->kv, m->arena, l, qrot, Hq, d_pforder,
                                       (int64_t)pfp.order.size(), d_pfstart, d_pfcount, d_pfpos,
                                       d_pfoff, d_btids, pf_ops, attn, pf_out));
      if (pf_split)
        HIP_TRY(st, launch_split_merge(stream, d.head_dim, n, Hq, pf_merge, attn));
    }
    GemmFuse o_f = accumulate;
    o_f.x_hilo = o_presplit;
    if (pack_layers) o_f.w_packed = L.p_o;
    HIP_TRY(st, gemm_on(m->dev, attn, L.w_o, nullptr, n, H, m->qd, Epilogue::kAccumulate,
                        hidden, &o_f));
    GemmFuse gu_f = norm_in(L.post_norm);
    if (pack_layers) gu_f.w_packed = L.p_gu;
    if (!fused)
      HIP_TRY(st, launch_rmsnorm(stream, hidden, nullptr, L.post_norm, n, H, d.rms_norm_eps, xn,
                                 presplit));
    gu_f.x_hilo = gu_f.out_hilo = presplit;
    HIP_TRY(st, gemm_on(m->dev, fused ? hidden : xn, L.w_gu, nullptr, n, 2 * F, H,
                        Epilogue::kSwiGLU, act, &gu_f));
    GemmFuse down_f = accumulate;
    down_f.x_hilo = presplit;
    if (pack_layers) down_f.w_packed = L.p_down;
    HIP_TRY(st, gemm_on(m->dev, act, L.w_down, nullptr, n, H, F, Epilogue::kAccumulate, hidden,
                        &down_f));
  }
  // Final norm on the last row of each sequence only (norm is row-wise, so
  // this equals norming all rows and then gathering), then the LM head.
  // When every row is its sequence's last row (a decode batch) and the layer
  // GEMMs left the row sums of squares, the LM head applies the norm while
  // staging its input, as the layer GEMMs do.
  bool head_norm = fused && S == n && gemm_splitk_fusable(S, V, H);
  for (int64_t i = 0; head_norm && i < S; ++i) head_norm = hb.last_rows[i] == (int32_t)i;
  GemmFuse head_f = head_norm ? norm_in(m->final_norm) : GemmFuse{};
  if (!head_norm)
    HIP_TRY(st, launch_rmsnorm(stream, hidden, d_last, m->final_norm, S, H, d.rms_norm_eps, xn));
  const uint16_t* head = m->w_lm ? m->w_lm : m->w_embed;
  float* logits = m->logits.as<float>();
  if (pack_head) head_f.w_packed = m->p_head;
  HIP_TRY(st, gemm_on(m->dev, head_norm ? hidden : xn, head, nullptr, S, V, H, Epilogue::kStore,
                      logits, &head_f));
  m->last_rows = S;
  if (argmax_out) {
    HIP_TRY(st, launch_argmax(stream, logits, S, V, m->argmax.as<int64_t>()));
    HIP_TRY(st, hipMemcpyAsync(argmax_out, m->argmax.ptr, S * 8, hipMemcpyDeviceToHost, stream));
  }
  if (logits_out)
    HIP_TRY(st, hipMemcpyAsync(logits_out, logits, S * V * 4, hipMemcpyDeviceToHost, stream));
  HIP_TRY(st, hipStreamSynchronize(stream));
  return ORION_HIP_OK;
}

// ---------------------------------------------------------------------------
// Op-level entry points
// ---------------------------------------------------------------------------

static int kv_geom_from(const orion_hip_kv_layout* kv, KvGeom* g, const char* st) {
  if (kv->dtype != ORION_DTYPE_F32 && kv->dtype != ORION_DTYPE_BF16)
    return set_err(ORION_HIP_ERR_BACKEND, st, "kv dtype must be F32 or BF16");
  if (kv->block_size < 1 || (kv->block_size & (kv->block_size - 1)) || kv->block_size > 256)
    return internal(st, "block_size must be a power of two <= 256");
  if (kv->head_dim <= 0 || kv->head_dim % 2 || kv->head_dim > kMaxHeadDim)
    return set_err(ORION_HIP_ERR_BACKEND, st, "head_dim %lld unsupported (even, at most %d)",
                   (long long)kv->head_dim, kMaxHeadDim);
  *g = KvGeom{kv->num_layers, kv->num_blocks, kv->block_size, kv->num_kv_heads, kv->head_dim,
              kv->dtype == ORION_DTYPE_BF16, kv->head_major != 0};
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_decode_plan_create(orion_hip_device* dev, const uint32_t* positions,
                                             const int32_t* row_seq,
                                             const int64_t* block_table_offsets,
                                             const uint32_t* block_table_ids, int64_t num_rows,
                                             int64_t num_q_heads, int64_t num_kv_heads,
                                             int64_t head_dim, int64_t block_size,
                                             orion_hip_decode_plan** out) {
  const char* st = "decode_plan";
  *out = nullptr;
  if (num_rows < 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads || head_dim <= 0 ||
      block_size < 1 || (block_size & (block_size - 1)) || block_size > 256)
    return internal(st, "invalid plan geometry");
  HIP_TRY(st, hipSetDevice(dev->ordinal));
  auto p = std::make_unique<orion_hip_decode_plan>();
  p->dev = dev;
  p->rows = num_rows;
  p->hq = num_q_heads;
  p->hkv = num_kv_heads;
  p->head_dim = head_dim;
  p->block_size = block_size;
  for (int64_t i = 0; i < num_rows; ++i) {
    const int64_t s = row_seq[i];
    const int64_t tl = block_table_offsets[s + 1] - block_table_offsets[s];
    if (s < 0 || (int64_t)positions[i] / block_size >= tl)
      return internal(st, "row %lld: position %u has no block in its table", (long long)i,
                      positions[i]);
  }
  // packing applies to bf16 arenas at head_dim 64/128 (the plan does not know
  // the arena's dtype yet: an f32 arena takes the unpacked copy)
  const KvGeom bf16_geom{1, 1, block_size, num_kv_heads, head_dim, true};
  const int pack_r = decode_pack_rows(bf16_geom, num_q_heads);
  build_decode_plan(positions, row_seq, block_table_offsets, block_table_ids, num_rows,
                    num_kv_heads, block_size, dev->wave_slots, nullptr, &p->host, pack_r);
  if (p->host.num_packed)
    build_decode_plan(positions, row_seq, block_table_offsets, block_table_ids, num_rows,
                      num_kv_heads, block_size, dev->wave_slots, nullptr, &p->plain, 0);
  // work items, then the pieces per row, then the pack rows, in one buffer
  auto upload = [&](const DecodePlanHost& h, DevBuf& buf) -> hipError_t {
    const size_t wbytes = h.work.size() * sizeof(DecodeWork);
    const size_t nbytes = h.row_nsplit.size() * sizeof(int32_t);
    const size_t pbytes = h.pack_rows.size() * sizeof(int32_t);
    hipError_t e = buf.reserve(wbytes + nbytes + pbytes);
    if (e != hipSuccess) return e;
    std::vector<char> staged(wbytes + nbytes + pbytes);
    std::memcpy(staged.data(), h.work.data(), wbytes);
    std::memcpy(staged.data() + wbytes, h.row_nsplit.data(), nbytes);
    std::memcpy(staged.data() + wbytes + nbytes, h.pack_rows.data(), pbytes);
    if (staged.empty()) return hipSuccess;
    e = hipMemcpyAsync(buf.ptr, staged.data(), staged.size(), hipMemcpyHostToDevice, dev->stream);
    if (e != hipSuccess) return e;
    return hipStreamSynchronize(dev->stream);  // staged is freed on return
  };
  HIP_TRY(st, upload(p->host, p->work));
  if (p->host.num_packed) HIP_TRY(st, upload(p->plain, p->work_plain));
  HIP_TRY(st, p->ws.reserve(decode_workspace_bytes(
                  num_rows, num_q_heads, head_dim,
                  std::max(p->host.max_splits, p->plain.max_splits))));
  HIP_TRY(st, hipStreamSynchronize(dev->stream));
  *out = p.release();
  return ORION_HIP_OK;
}

ORION_EXPORT void orion_hip_decode_plan_destroy(orion_hip_decode_plan* plan) {
  if (!plan) return;
  (void)hipSetDevice(plan->dev->ordinal);
  (void)hipStreamSynchronize(plan->dev->stream);
  delete plan;
}

ORION_EXPORT int orion_hip_decode_plan_packed(const orion_hip_decode_plan* plan,
                                              int64_t* packed_items, int64_t* rows_per_pack) {
  *packed_items = plan->host.num_packed;
  *rows_per_pack = plan->host.num_packed ? plan->host.pack_r : 0;
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_decode_plan_info(const orion_hip_decode_plan* plan, int64_t* chunk,
                                            int64_t* num_work, int64_t* max_splits) {
  *chunk = plan->host.chunk;
  *num_work = (int64_t)plan->host.work.size();
  *max_splits = plan->host.max_splits;
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_paged_attention_decode(
    orion_hip_device* dev, const orion_hip_kv_layout* kv, const void* d_arena, int64_t layer,
    const float* d_q, int64_t num_rows, int64_t num_q_heads, const uint32_t* d_positions,
    const int32_t* d_row_seq, const int64_t* d_bt_offsets, const uint32_t* d_bt_ids,
    const orion_hip_decode_plan* plan, float* d_out) {
  const char* st = "paged_attention_decode";
  KvGeom g;
  if (int rc = kv_geom_from(kv, &g, st)) return rc;
  if (g.num_kv_heads <= 0 || num_q_heads % g.num_kv_heads)
    return internal(st, "%lld query heads cannot be grouped over %lld kv heads",
                    (long long)num_q_heads, (long long)g.num_kv_heads);
  if (layer < 0 || layer >= g.num_layers)
    return internal(st, "layer %lld out of range (have %lld)", (long long)layer,
                    (long long)g.num_layers);
  if (!plan || plan->rows != num_rows || plan->hq != num_q_heads ||
      plan->hkv != g.num_kv_heads || plan->head_dim != g.head_dim ||
      plan->block_size != g.block_size)
    return internal(st, "decode plan does not match this call's geometry");
  HIP_TRY(st, hipSetDevice(dev->ordinal));
  if (!dev->ktiming) {
    HIP_TRY(st, launch_paged_decode(dev->stream, g, d_arena, layer, d_q, num_rows, num_q_heads,
                                    d_positions, d_row_seq, d_bt_offsets, d_bt_ids, plan->view(g.dtype_bf16),
                                    d_out));
    return ORION_HIP_OK;
  }
  // Timed: the split-K kernel and the merge kernel as separate launches.
  DecodePlanDev pv = plan->view(g.dtype_bf16);
  HIP_TRY(st, timed_launch(dev, 0, [&] {
            return launch_paged_decode(dev->stream, g, d_arena, layer, d_q, num_rows, num_q_heads,
                                       d_positions, d_row_seq, d_bt_offsets, d_bt_ids, pv, d_out,
                                       DecodePhase::kSplit);
          }));
  HIP_TRY(st, timed_launch(dev, 1, [&] {
            return launch_paged_decode(dev->stream, g, d_arena, layer, d_q, num_rows, num_q_heads,
                                       d_positions, d_row_seq, d_bt_offsets, d_bt_ids, pv, d_out,
                                       DecodePhase::kMerge);
          }));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_paged_attention_prefill(
    orion_hip_device* dev, const orion_hip_kv_layout* kv, const void* d_arena, int64_t layer,
    const float* d_q, int64_t num_q_heads, int64_t num_seqs, const int32_t* d_row_start,
    const int32_t* d_row_count, const uint32_t* d_first_pos, const int64_t* d_bt_offsets,
    const uint32_t* d_bt_ids, int64_t max_rows, int64_t max_position, int32_t hilo,
    float* d_out) {
  const char* st = "paged_attention_prefill";
  // value 16 added: write the output rows in the split operand layout of
  // the O GEMM (GemmFuse::x_hilo) instead of f32
  const bool out_split = (hilo & 16) != 0;
  hilo &= ~16;
  if (hilo < 0 || hilo > 3) return internal(st, "operand mode %d is not 0..3", (int)hilo);
  // 0: bf16 Q and P; 1: hi/lo both; 2: hi/lo Q, bf16 P; 3: bf16 Q, hi/lo P
  static const int kOps[4] = {0, kPrefillQHiLo | kPrefillPHiLo, kPrefillQHiLo, kPrefillPHiLo};
  KvGeom g;
  if (int rc = kv_geom_from(kv, &g, st)) return rc;
  if (g.num_kv_heads <= 0 || num_q_heads % g.num_kv_heads)
    return internal(st, "query heads cannot be grouped over kv heads");
  if (g.head_dim != 64 && g.head_dim != 128 && g.head_dim != 256)
    return set_err(ORION_HIP_ERR_BACKEND, st,
                   "prefill attention covers head_dim 64, 128 and 256 (got %lld); other shapes take "
                   "the decode entry point row by row", (long long)g.head_dim);
  HIP_TRY(st, hipSetDevice(dev->ordinal));
  (void)max_rows;
  (void)max_position;
  // The work list is built on the host: fetch the chunk lengths and first
  // positions (a synchronous copy; this entry point is for tests and timing,
  // the model forward builds the list from host data).
  std::vector<int32_t> h_count(num_seqs > 0 ? num_seqs : 0), h_start(h_count.size());
  std::vector<uint32_t> h_first(h_count.size());
  if (num_seqs > 0) {
    HIP_TRY(st, hipMemcpyAsync(h_count.data(), d_row_count, num_seqs * 4, hipMemcpyDeviceToHost,
                               dev->stream));
    HIP_TRY(st, hipMemcpyAsync(h_start.data(), d_row_start, num_seqs * 4, hipMemcpyDeviceToHost,
                               dev->stream));
    HIP_TRY(st, hipMemcpyAsync(h_first.data(), d_first_pos, num_seqs * 4, hipMemcpyDeviceToHost,
                               dev->stream));
    HIP_TRY(st, hipStreamSynchronize(dev->stream));
  }
  PrefillPlan pfp;
  build_prefill_order(h_start.data(), h_count.data(), h_first.data(), num_seqs,
                      num_q_heads / g.num_kv_heads, g.num_kv_heads, dev->wave_slots / 8, &pfp,
                      g.head_dim);
  const std::vector<PrefillTile>& order = pfp.order;
  // work list, then (when sequences are split into key parts) the merge's
  // row list and parts per row, in one device buffer
  const size_t ob = order.size() * sizeof(PrefillTile);
  const bool split = pfp.max_parts > 1;
  const size_t sb = split ? pfp.split_rows.size() * 4 : 0, pb = split ? pfp.row_parts.size() * 4 : 0;
  std::vector<char> staged(ob + sb + pb);
  if (ob) std::memcpy(staged.data(), order.data(), ob);
  if (sb) std::memcpy(staged.data() + ob, pfp.split_rows.data(), sb);
  if (pb) std::memcpy(staged.data() + ob + sb, pfp.row_parts.data(), pb);
  HIP_TRY(st, dev->prefill_order.reserve(std::max<size_t>(staged.size(), 1)));
  if (!staged.empty())
    HIP_TRY(st, hipMemcpy(dev->prefill_order.ptr, staged.data(), staged.size(),
                          hipMemcpyHostToDevice));
  const int64_t rows = (int64_t)pfp.row_parts.size();
  DecodePlanDev merge;
  PrefillSplitOut out_parts;
  if (split) {
    HIP_TRY(st, dev->prefill_ws.reserve(
                    decode_workspace_bytes(rows, num_q_heads, g.head_dim, pfp.max_parts)));
    const char* base = dev->prefill_order.as<const char>();
    merge.rows = reinterpret_cast<const int32_t*>(base + ob);
    merge.num_rows = (int)pfp.split_rows.size();
    merge.row_nsplit = reinterpret_cast<const int32_t*>(base + ob + sb);
    merge.max_splits = pfp.max_parts;
    merge.ws = dev->prefill_ws.as<float>();
    merge.ws_bytes = dev->prefill_ws.bytes;
    out_parts.ws_o = merge.ws;
    out_parts.ws_ml = merge.ws + rows * num_q_heads * pfp.max_parts * g.head_dim;
    out_parts.max_parts = pfp.max_parts;
  }
  if (out_split && split)
    return set_err(ORION_HIP_ERR_BACKEND, st,
                   "the split output layout needs every sequence whole (no key parts)");
  out_parts.out_hilo = out_split ? 1 : 0;
  // (timed together: the kernel and, for split sequences, the merge of parts)
  HIP_TRY(st, timed_launch(dev, 2, [&] {
            hipError_t e = launch_paged_prefill(dev->stream, g, d_arena, layer, d_q, num_q_heads,
                                                dev->prefill_order.as<const PrefillTile>(),
                                                (int64_t)order.size(), d_row_start, d_row_count,
                                                d_first_pos, d_bt_offsets, d_bt_ids, kOps[hilo],
                                                d_out, out_parts);
            if (e == hipSuccess && split)
              e = launch_split_merge(dev->stream, g.head_dim, rows, num_q_heads, merge, d_out);
            return e;
          }));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_rope_and_cache(orion_hip_device* dev, const orion_hip_kv_layout* kv,
                                          void* d_arena, int64_t layer, int64_t num_rows,
                                          int64_t num_q_heads, const float* d_q_in,
                                          int64_t q_stride, float* d_q_out, const float* d_k,
                                          int64_t k_stride, const float* d_v, int64_t v_stride,
                                          const uint32_t* d_positions, const int32_t* d_row_seq,
                                          const int64_t* d_bt_offsets, const uint32_t* d_bt_ids,
                                          const float* d_cos, const float* d_sin) {
  const char* st = "rope_and_cache";
  KvGeom g;
  if (int rc = kv_geom_from(kv, &g, st)) return rc;
  if (layer < 0 || layer >= g.num_layers) return internal(st, "layer out of range");
  HIP_TRY(st, hipSetDevice(dev->ordinal));
  HIP_TRY(st, launch_rope_and_cache(dev->stream, g, d_arena, layer, num_rows, num_q_heads, d_q_in,
                                    q_stride, d_q_out, d_k, k_stride, d_v, v_stride, d_positions,
                                    d_row_seq, d_bt_offsets, d_bt_ids, d_cos, d_sin));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_rmsnorm(orion_hip_device* dev, const float* d_x, const float* d_weight,
                                   int64_t rows, int64_t cols, float eps, float* d_out) {
  HIP_TRY("rmsnorm", hipSetDevice(dev->ordinal));
  HIP_TRY("rmsnorm", launch_rmsnorm(dev->stream, d_x, nullptr, d_weight, rows, cols, eps, d_out));
  return ORION_HIP_OK;
}

// Argument checks shared by orion_hip_gemm and orion_hip_gemm_noalloc.
static int gemm_args(const char* st, const float* d_bias, int64_t N, int64_t K, int epilogue,
                     Epilogue* ep) {
  if (K % 32 != 0 || K <= 0)
    return set_err(ORION_HIP_ERR_BACKEND, st, "K must be a positive multiple of 32, got %lld",
                   (long long)K);
  if (epilogue < ORION_GEMM_STORE || epilogue > ORION_GEMM_SWIGLU)
    return internal(st, "unknown epilogue %d", epilogue);
  if (epilogue != ORION_GEMM_STORE && d_bias)
    return internal(st, "bias is only supported with the store epilogue");
  if (epilogue == ORION_GEMM_SWIGLU && N % 16 != 0)
    return internal(st, "SwiGLU needs N (gate/up rows) to be a multiple of 16, got %lld",
                    (long long)N);
  *ep = epilogue == ORION_GEMM_ACCUMULATE ? Epilogue::kAccumulate
        : epilogue == ORION_GEMM_SWIGLU   ? Epilogue::kSwiGLU
                                          : Epilogue::kStore;
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_gemm(orion_hip_device* dev, const float* d_x, const uint16_t* d_w,
                                const float* d_bias, int64_t M, int64_t N, int64_t K,
                                int epilogue, float* d_out) {
  const char* st = "gemm";
  Epilogue ep;
  if (int rc = gemm_args(st, d_bias, N, K, epilogue, &ep)) return rc;
  HIP_TRY(st, hipSetDevice(dev->ordinal));
  HIP_TRY(st, timed_launch(dev, 3, [&] { return gemm_on(dev, d_x, d_w, d_bias, M, N, K, ep, d_out); }));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_gemm_noalloc(orion_hip_device* dev, const float* d_x,
                                        const uint16_t* d_w, const float* d_bias, int64_t M,
                                        int64_t N, int64_t K, int epilogue, float* d_out) {
  const char* st = "gemm_noalloc";
  Epilogue ep;
  if (int rc = gemm_args(st, d_bias, N, K, epilogue, &ep)) return rc;
  size_t need = 0;
  gemm_scratch_need(M, N, K, &need, false);
  if (need > kNoAllocScratchBytes)
    return set_err(ORION_HIP_ERR_BACKEND, st,
                   "M=%lld N=%lld K=%lld needs %zu bytes of split-K scratch; the "
                   "no-allocation entry point holds %zu",
                   (long long)M, (long long)N, (long long)K, need, kNoAllocScratchBytes);
  if (!dev->noalloc_scratch)
    return set_err(ORION_HIP_ERR_BACKEND, st, "device scratch address was not resolved");
  HIP_TRY(st, hipSetDevice(dev->ordinal));
  // The same kernels as orion_hip_gemm; every partial tile a call reads was
  // written earlier in the same call, so nothing needs clearing.
  GemmScratch sc;
  sc.ws = static_cast<float*>(dev->noalloc_scratch);
  sc.ws_bytes = kNoAllocScratchBytes;
  // Order against the previous call on this GPU (any handle, any host
  // thread): wait for its event, launch, record ours, all under the lock.
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  const int o = dev->ordinal;
  if (g_noalloc_recorded[o]) HIP_TRY(st, hipStreamWaitEvent(dev->stream, g_noalloc_done[o], 0));
  HIP_TRY(st, launch_gemm(dev->stream, d_x, d_w, d_bias, M, N, K, ep, d_out, &sc, nullptr));
  HIP_TRY(st, hipEventRecord(g_noalloc_done[o], dev->stream));
  g_noalloc_recorded[o] = true;
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_silu_mul(orion_hip_device* dev, float* d_gate, const float* d_up,
                                    int64_t count) {
  HIP_TRY("silu_mul", hipSetDevice(dev->ordinal));
  HIP_TRY("silu_mul", launch_silu_mul(dev->stream, d_gate, d_up, count));
  return ORION_HIP_OK;
}

ORION_EXPORT int orion_hip_argmax(orion_hip_device* dev, const float* d_logits, int64_t rows,
                                  int64_t cols, int64_t* d_out) {
  HIP_TRY("argmax", hipSetDevice(dev->ordinal));
  HIP_TRY("argmax", launch_argmax(dev->stream, d_logits, rows, cols, d_out));
  return ORION_HIP_OK;
}

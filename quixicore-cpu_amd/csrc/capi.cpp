// extern "C" boundary (include/quixicore_hip.h): host-visible validation in
// the reference's order, then the HIP launches.  No compute happens on the
// host and there is no CPU fallback: every result comes from a gfx950 kernel.
#include "quixicore_hip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <limits>
#include <mutex>
#include <string>
#include <vector>

#include "qc_internal.h"

namespace {

thread_local std::string g_last_error;

// Process-wide routing knobs (the qc_hip_set_* calls).  Each is an atomic and
// every call reads them once, into a snapshot, so a setter that races with
// calls on other threads is well defined: each call sees the old value or
// the new one.  The qgemm plan (waves, stages) is one word, so a call never
// sees half of a plan.
struct Knobs {
  std::atomic<int> rows_per_wave{0};
  std::atomic<int> qgemm_plan{0};   // waves | stages << 8
  std::atomic<int> qgemm_panel{0};
  std::atomic<int> qgemm_rows{0};
  std::atomic<int> qgemm_fold{0};
  std::atomic<int> cint8_dot{0};
  std::atomic<int> int8_route{qc::kInt8Auto};
  std::atomic<bool> norm_sequential{false};
};
Knobs g_knobs;

qc::GemvTuning tuning() {
  constexpr auto r = std::memory_order_relaxed;
  qc::GemvTuning t;
  t.rows_per_wave = g_knobs.rows_per_wave.load(r);
  const int plan = g_knobs.qgemm_plan.load(r);
  t.qgemm_waves = plan & 0xFF;
  t.qgemm_stages = plan >> 8;
  t.qgemm_panel = g_knobs.qgemm_panel.load(r);
  t.qgemm_rows = g_knobs.qgemm_rows.load(r);
  t.qgemm_fold = g_knobs.qgemm_fold.load(r);
  t.cint8_dot = g_knobs.cint8_dot.load(r);
  return t;
}

int int8_route() { return g_knobs.int8_route.load(std::memory_order_relaxed); }

int device_error(hipError_t e) {
  g_last_error = hipGetErrorString(e);
  return QC_DEVICE_ERROR;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// kernels/common/validation.h:8-18 (valid_product).
bool valid_product(std::initializer_list<long long> dims) {
  long long product = 1;
  for (long long d : dims) {
    if (d <= 0 || product > LLONG_MAX / d) return false;
    product *= d;
  }
  return true;
}

int block_bytes(int format) {
  return format == QC_Q8_0 ? 34 : (format == QC_Q4_0 ? 18 : 0);
}

// src/dispatch/qgemv.cpp:125-141 (validate): format, then n, k > 0 and
// k % 32 == 0, then the signed-offset overflow guard.  The int32 limit on n
// and k is this library's (grid and index width).
int validate(int format, long long n, long long k) {
  if (block_bytes(format) == 0) return QC_UNSUPPORTED_FORMAT;
  if (n <= 0 || k <= 0 || k % 32 != 0) return QC_INVALID_SHAPE;
  if (n > LLONG_MAX / k || n > LLONG_MAX / (k / 32)) return QC_INVALID_SHAPE;
  if (n > INT_MAX || k > INT_MAX) return QC_INVALID_SHAPE;
  return QC_OK;
}

// src/dispatch/qgemv.cpp:151-164 (packed_size).
int packed_bytes(int format, long long n, long long k, size_t* size) {
  const size_t blocks_per_row = static_cast<size_t>(k / 32);
  const size_t bb = static_cast<size_t>(block_bytes(format));
  if (static_cast<size_t>(n) > std::numeric_limits<size_t>::max() / blocks_per_row)
    return QC_INVALID_SHAPE;
  const size_t blocks = static_cast<size_t>(n) * blocks_per_row;
  if (blocks > std::numeric_limits<size_t>::max() / bb) return QC_INVALID_SHAPE;
  *size = blocks * bb;
  return QC_OK;
}

// Device ints for the synchronous (dev_status == NULL) paths: a per-device
// pool, one int per call in flight, so that synchronous calls from several
// host threads (on different streams) never share a flag.
struct FlagPool {
  std::mutex mu;
  std::vector<std::vector<int*>> free;   // [device] -> idle flags
};
FlagPool& flag_pool() {
  static FlagPool p;
  return p;
}

int* acquire_flag(int* dev, hipError_t* err) {
  *err = hipGetDevice(dev);
  if (*err != hipSuccess) return nullptr;
  FlagPool& p = flag_pool();
  {
    std::lock_guard<std::mutex> lock(p.mu);
    if (static_cast<int>(p.free.size()) <= *dev) p.free.resize(*dev + 1);
    std::vector<int*>& idle = p.free[*dev];
    if (!idle.empty()) {
      int* f = idle.back();
      idle.pop_back();
      return f;
    }
  }
  int* f = nullptr;
  *err = hipMalloc(&f, sizeof(int));
  return *err == hipSuccess ? f : nullptr;
}

void release_flag(int dev, int* f) {
  FlagPool& p = flag_pool();
  std::lock_guard<std::mutex> lock(p.mu);
  p.free[dev].push_back(f);
}

// Runs `launch(flag)` with a zeroed device flag and returns its value.
template <class F>
int with_flag(hipStream_t s, int* value, F&& launch) {
  hipError_t e = hipSuccess;
  int dev = 0;
  int* flag = acquire_flag(&dev, &e);
  if (flag == nullptr) return device_error(e);
  if ((e = hipMemsetAsync(flag, 0, sizeof(int), s)) == hipSuccess &&
      (e = launch(flag)) == hipSuccess &&
      (e = hipMemcpyAsync(value, flag, sizeof(int), hipMemcpyDeviceToHost, s)) == hipSuccess)
    e = hipStreamSynchronize(s);
  if (e == hipSuccess) {
    release_flag(dev, flag);
    return QC_OK;
  }
  // After a failure the flag may still be in use by queued work: keep it out
  // of the pool.
  return device_error(e);
}

// Synchronous all_finite over a device array.
int all_finite(const float* x, long long count, hipStream_t s, bool* finite) {
  int bad = 0;
  const int st = with_flag(s, &bad, [&](int* flag) {
    return qc::launch_nonfinite_scan(x, count, flag, s);
  });
  *finite = bad == 0;
  return st;
}

int finish(hipError_t e) { return e == hipSuccess ? QC_OK : device_error(e); }

}  // namespace

extern "C" {

const char* qc_hip_version(void) { return "quixicore-hip 0.1 (gfx950)"; }

const char* qc_hip_last_error(void) { return g_last_error.c_str(); }

int qc_hip_qgemv_packed_size(int format, long long n, long long k, size_t* size) {
  const int st = validate(format, n, k);
  if (st != QC_OK) return st;
  if (size == nullptr) return QC_INVALID_ARGUMENT;
  return packed_bytes(format, n, k, size);
}

int qc_hip_qgemv_pack(int format, const float* w, long long n, long long k, void* packed,
                      int* dev_status, void* stream) {
  int st = validate(format, n, k);
  if (st != QC_OK) return st;
  size_t ignored = 0;
  if (packed_bytes(format, n, k, &ignored) != QC_OK) return QC_INVALID_SHAPE;
  if (w == nullptr || packed == nullptr) return QC_INVALID_ARGUMENT;
  const hipStream_t s = as_stream(stream);
  if (dev_status != nullptr) return finish(qc::launch_pack(format, w, packed, n, k, dev_status, s));
  int bad = 0;
  st = with_flag(s, &bad, [&](int* flag) { return qc::launch_pack(format, w, packed, n, k, flag, s); });
  if (st != QC_OK) return st;
  return bad ? QC_INVALID_ARGUMENT : QC_OK;
}

int qc_hip_qgemv_unpack(int format, const void* packed, long long n, long long k, float* w,
                        void* stream) {
  const int st = validate(format, n, k);
  if (st != QC_OK) return st;
  size_t ignored = 0;
  if (packed_bytes(format, n, k, &ignored) != QC_OK) return QC_INVALID_SHAPE;
  if (packed == nullptr || w == nullptr) return QC_INVALID_ARGUMENT;
  return finish(qc::launch_unpack(format, packed, w, n, k, as_stream(stream)));
}

int qc_hip_qgemv(int format, const void* packed, const float* x, float* y, long long n,
                 long long k, void* stream) {
  const int st = validate(format, n, k);
  if (st != QC_OK) return st;
  size_t ignored = 0;
  if (packed_bytes(format, n, k, &ignored) != QC_OK) return QC_INVALID_SHAPE;
  if (packed == nullptr || x == nullptr || y == nullptr) return QC_INVALID_ARGUMENT;
  return finish(qc::launch_qgemm(format, packed, x, y, 1, n, k, as_stream(stream), tuning()));
}

// kernels/quantization/qgemm_ref.cpp:141-164: shape products first, then the
// null checks, then qgemv_packed_size (format and k validation).
int qc_hip_qgemm(int format, const void* packed, const float* x, float* y, long long m,
                 long long n, long long k, void* stream) {
  if (!valid_product({m, k}) || !valid_product({m, n})) return QC_INVALID_SHAPE;
  if (m > INT_MAX) return QC_INVALID_SHAPE;   // this library's dimension limit (as for n, k)
  if (packed == nullptr || x == nullptr || y == nullptr) return QC_INVALID_ARGUMENT;
  size_t size = 0;
  const int st = qc_hip_qgemv_packed_size(format, n, k, &size);
  if (st != QC_OK) return st;
  return finish(qc::launch_qgemm(format, packed, x, y, m, n, k, as_stream(stream), tuning()));
}

// qc_hip_qgemm without allocating: the same validation and kernels, with the
// scratch in a fixed per-GPU device array (see launch_qgemm_mfma_noalloc).
int qc_hip_qgemm_noalloc(int format, const void* packed, const float* x, float* y, long long m,
                         long long n, long long k, void* stream) {
  if (!valid_product({m, k}) || !valid_product({m, n})) return QC_INVALID_SHAPE;
  if (m > INT_MAX) return QC_INVALID_SHAPE;
  if (m > QC_QGEMM_NOALLOC_MAX_M || k > QC_QGEMM_NOALLOC_MAX_K) {
    g_last_error = "qgemm_noalloc: m <= " + std::to_string(QC_QGEMM_NOALLOC_MAX_M) +
                   " and k <= " + std::to_string(QC_QGEMM_NOALLOC_MAX_K) +
                   " (fixed scratch of " + std::to_string(qc::kQgemmNoAllocScratchBytes) +
                   " bytes)";
    return QC_INVALID_SHAPE;
  }
  if (packed == nullptr || x == nullptr || y == nullptr) return QC_INVALID_ARGUMENT;
  size_t size = 0;
  const int st = qc_hip_qgemv_packed_size(format, n, k, &size);
  if (st != QC_OK) return st;
  const hipError_t e = qc::launch_qgemm(format, packed, x, y, m, n, k, as_stream(stream),
                                        tuning(), /*noalloc=*/true);
  if (e == hipErrorOutOfMemory) {
    g_last_error = "qgemm_noalloc: this shape needs more than the fixed scratch of " +
                   std::to_string(qc::kQgemmNoAllocScratchBytes) + " bytes";
    return QC_INVALID_SHAPE;
  }
  return finish(e);
}

// kernels/quantization/quantization_ref.cpp:17-21 (quant_shape), 143-147.
int qc_hip_quantize_int8(const float* x, int8_t* codes, float* scales, long long rows,
                         long long dim, long long group_size, int* dev_status, void* stream) {
  if (!valid_product({rows, dim})) return QC_INVALID_SHAPE;
  if (group_size == 0) group_size = dim;
  if (group_size <= 0 || dim % group_size != 0) return QC_INVALID_SHAPE;
  if (x == nullptr || codes == nullptr || scales == nullptr) return QC_INVALID_ARGUMENT;
  const hipStream_t s = as_stream(stream);
  if (dev_status != nullptr)
    return finish(qc::launch_quantize_int8(x, codes, scales, rows, dim, group_size, dev_status, s));
  bool finite = false;
  int st = all_finite(x, rows * dim, s, &finite);
  if (st != QC_OK) return st;
  if (!finite) return QC_INVALID_ARGUMENT;
  hipError_t e = qc::launch_quantize_int8(x, codes, scales, rows, dim, group_size, nullptr, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return finish(e);
}

// src/dispatch/int8_gemm.cpp:67-94: shape, nulls, finite scales.
int qc_hip_int8_gemm(const int8_t* w, const int8_t* x, const float* ws, const float* as,
                     const int32_t* row_sum, const int* zp, float* y, long long m, long long n,
                     long long k, int asymmetric, int* dev_status, void* stream) {
  if (!valid_product({m, n, k})) return QC_INVALID_SHAPE;
  if (w == nullptr || x == nullptr || ws == nullptr || as == nullptr || y == nullptr ||
      (asymmetric && (row_sum == nullptr || zp == nullptr)))
    return QC_INVALID_ARGUMENT;
  const hipStream_t s = as_stream(stream);
  if (dev_status != nullptr)
    return finish(qc::launch_int8_gemm(w, x, ws, as, row_sum, zp, y, nullptr, m, n, k,
                                       asymmetric != 0, dev_status, s, int8_route()));
  bool finite = false;
  int st = all_finite(ws, n, s, &finite);
  if (st != QC_OK) return st;
  if (!finite) return QC_INVALID_ARGUMENT;
  st = all_finite(as, m, s, &finite);
  if (st != QC_OK) return st;
  if (!finite) return QC_INVALID_ARGUMENT;
  hipError_t e = qc::launch_int8_gemm(w, x, ws, as, row_sum, zp, y, nullptr, m, n, k,
                                      asymmetric != 0, nullptr, s, int8_route());
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return finish(e);
}

int qc_hip_qgemm_w8a8(const int8_t* w, const int8_t* x, const float* ws, const float* as,
                      float* y, long long m, long long n, long long k, int* dev_status,
                      void* stream) {
  return qc_hip_int8_gemm(w, x, ws, as, nullptr, nullptr, y, m, n, k, 0, dev_status, stream);
}

int qc_hip_int8_gemm_i32(const int8_t* w, const int8_t* x, int32_t* acc, long long m,
                         long long n, long long k, void* stream) {
  if (!valid_product({m, n, k})) return QC_INVALID_SHAPE;
  if (k > 131071) return QC_INVALID_SHAPE;
  if (w == nullptr || x == nullptr || acc == nullptr) return QC_INVALID_ARGUMENT;
  return finish(qc::launch_int8_gemm(w, x, nullptr, nullptr, nullptr, nullptr, nullptr, acc, m,
                                     n, k, false, nullptr, as_stream(stream), int8_route()));
}

int qc_hip_stream_read(const void* p, long long bytes, uint32_t* out, int grid, void* stream) {
  if (bytes <= 0 || bytes % 16 != 0 || grid <= 0) return QC_INVALID_SHAPE;
  if (p == nullptr || out == nullptr) return QC_INVALID_ARGUMENT;
  return finish(qc::launch_stream_read(p, bytes, out, grid, as_stream(stream)));
}

int qc_hip_nonfinite_scan(const float* x, long long count, int* dev_flag, void* stream) {
  if (count <= 0) return QC_INVALID_SHAPE;
  if (x == nullptr || dev_flag == nullptr) return QC_INVALID_ARGUMENT;
  return finish(qc::launch_nonfinite_scan(x, count, dev_flag, as_stream(stream)));
}

const char* qc_hip_qgemv_variant(int format) {
  if (block_bytes(format) == 0) return "unsupported";
  return format == QC_Q8_0 ? "hip_gfx950_q8_0" : "hip_gfx950_q4_0";
}

const char* qc_hip_int8_gemm_variant(void) { return "hip_gfx950_mfma_i8"; }

int qc_hip_set_gemv_rows_per_wave(int rows) {
  if (rows != 0 && rows != 1 && rows != 2 && rows != 4 && rows != 7 && rows != 8 && rows != 14)
    return QC_INVALID_ARGUMENT;
  g_knobs.rows_per_wave.store(rows, std::memory_order_relaxed);
  return QC_OK;
}

// Fused GEMVs over one x.  One launch when every matrix takes the M = 1
// kernel (K/32 even, 4-byte aligned W, 32-bit row counts); otherwise one
// qgemv per matrix, and for the activation form an elementwise pass over a
// temporary up vector.
namespace {

int fused_gemv(int format, int nseg, const void* const* w, float* const* y,
               const long long* rows, int act, const float* x, long long k, hipStream_t s) {
  bool fast = (k >> 5) % 2 == 0 && k < (1LL << 31) && reinterpret_cast<uintptr_t>(x) % 16 == 0;
  long long total = 0;
  for (int i = 0; i < nseg; ++i) {
    fast = fast && reinterpret_cast<uintptr_t>(w[i]) % 4 == 0;
    total += rows[i];
  }
  fast = fast && total < (1LL << 30);
  if (fast) {
    int r[3] = {0, 0, 0};
    for (int i = 0; i < nseg; ++i) r[i] = static_cast<int>(rows[i]);
    return finish(qc::launch_qgemv_multi(format, nseg, w, y, r, act, x, static_cast<int>(k), s));
  }
  const qc::GemvTuning t = tuning();
  if (act < 0) {
    for (int i = 0; i < nseg; ++i) {
      const hipError_t e = qc::launch_qgemm(format, w[i], x, y[i], 1, rows[i], k, s, t);
      if (e != hipSuccess) return device_error(e);
    }
    return QC_OK;
  }
  float* up = nullptr;
  hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&up), sizeof(float) * rows[0], s);
  if (e != hipSuccess) return device_error(e);
  e = qc::launch_qgemm(format, w[0], x, up, 1, rows[0], k, s, t);
  if (e == hipSuccess) e = qc::launch_qgemm(format, w[1], x, y[0], 1, rows[0], k, s, t);
  if (e == hipSuccess) {
    e = qc::launch_fused_activation(y[0], up, rows[0], act, s);
  }
  const hipError_t f = hipFreeAsync(up, s);
  return finish(e != hipSuccess ? e : f);
}

}  // namespace

// kernels/quantization/qgemv_fused_ref.cpp:194-229 (qgemv_up_gate): shape
// product, nulls, then the packed layout (format, K).
int qc_hip_qgemv_up_gate(int format, const void* packed_up, const void* packed_gate,
                         const float* x, float* up, float* gate, long long n, long long k,
                         void* stream) {
  if (!valid_product({n, k})) return QC_INVALID_SHAPE;
  if (!packed_up || !packed_gate || !x || !up || !gate) return QC_INVALID_ARGUMENT;
  size_t bytes = 0;
  const int st = qc_hip_qgemv_packed_size(format, n, k, &bytes);
  if (st != QC_OK) return st;
  const void* w[2] = {packed_up, packed_gate};
  float* y[2] = {up, gate};
  const long long rows[2] = {n, n};
  return fused_gemv(format, 2, w, y, rows, -1, x, k, as_stream(stream));
}

// kernels/quantization/qgemv_fused_ref.cpp:184-192,231-273
// (qgemv_up_gate_activation): out = activation(gate) * up, GELU-tanh or SiLU.
int qc_hip_qgemv_up_gate_activation(int format, const void* packed_up, const void* packed_gate,
                                    const float* x, float* out, long long n, long long k,
                                    int gelu_tanh, void* stream) {
  if (!valid_product({n, k})) return QC_INVALID_SHAPE;
  if (!packed_up || !packed_gate || !x || !out) return QC_INVALID_ARGUMENT;
  size_t bytes = 0;
  const int st = qc_hip_qgemv_packed_size(format, n, k, &bytes);
  if (st != QC_OK) return st;
  const void* w[2] = {packed_up, packed_gate};
  float* y[1] = {out};
  const long long rows[2] = {n, n};
  return fused_gemv(format, 2, w, y, rows, gelu_tanh ? 1 : 0, x, k, as_stream(stream));
}

// kernels/quantization/qgemv_fused_ref.cpp:275-327 (qgemv_qkv): products and
// the 2 * kv_dim overflow check, nulls, the Q layout (format, K), then the KV
// layout (shape).
int qc_hip_qgemv_qkv(int format, const void* packed_q, const void* packed_k,
                     const void* packed_v, const float* x, float* q, float* k_out,
                     float* v_out, long long query_dim, long long kv_dim, long long input_dim,
                     void* stream) {
  if (!valid_product({query_dim, kv_dim, input_dim})) return QC_INVALID_SHAPE;
  if (kv_dim > (LLONG_MAX - query_dim) / 2) return QC_INVALID_SHAPE;
  if (!packed_q || !packed_k || !packed_v || !x || !q || !k_out || !v_out)
    return QC_INVALID_ARGUMENT;
  size_t bytes = 0;
  const int st = qc_hip_qgemv_packed_size(format, query_dim, input_dim, &bytes);
  if (st != QC_OK) return st;
  if (qc_hip_qgemv_packed_size(format, kv_dim, input_dim, &bytes) != QC_OK)
    return QC_INVALID_SHAPE;
  const void* w[3] = {packed_q, packed_k, packed_v};
  float* y[3] = {q, k_out, v_out};
  const long long rows[3] = {query_dim, kv_dim, kv_dim};
  return fused_gemv(format, 3, w, y, rows, -1, x, input_dim, as_stream(stream));
}

// kernels/quantization/qgemv_fused_ref.cpp:342-443 (qgemv_qkv_rope_kv):
// products, even head_dim, position and slot ranges; nulls; the Q layout
// (format, K) and the KV layout (shape); then the item-count overflow check.
int qc_hip_qgemv_qkv_rope_kv(int format, const void* packed_q, const void* packed_k,
                             const void* packed_v, const float* x, const float* cosine,
                             const float* sine, float* q, float* key_cache, float* value_cache,
                             long long query_heads, long long kv_heads, long long head_dim,
                             long long input_dim, long long slots, long long max_position,
                             int position, int slot, void* stream) {
  if (!valid_product({query_heads, head_dim, input_dim}) ||
      !valid_product({slots, kv_heads, head_dim}) || head_dim % 2 != 0 || position < 0 ||
      position >= max_position || slot < -1 || slot >= slots)
    return QC_INVALID_SHAPE;
  if (!packed_q || !packed_k || !packed_v || !x || !cosine || !sine || !q || !key_cache ||
      !value_cache)
    return QC_INVALID_ARGUMENT;
  const long long query_dim = query_heads * head_dim;
  const long long kv_dim = kv_heads * head_dim;
  size_t bytes = 0;
  const int st = qc_hip_qgemv_packed_size(format, query_dim, input_dim, &bytes);
  if (st != QC_OK) return st;
  if (qc_hip_qgemv_packed_size(format, kv_dim, input_dim, &bytes) != QC_OK)
    return QC_INVALID_SHAPE;
  const long long half = head_dim / 2;
  const long long query_pairs = query_heads * half;
  const long long key_pairs = slot >= 0 ? kv_heads * half : 0;
  const long long value_rows = slot >= 0 ? kv_dim : 0;
  if (query_pairs > LLONG_MAX - key_pairs || query_pairs + key_pairs > LLONG_MAX - value_rows)
    return QC_INVALID_SHAPE;
  const float* rc = cosine + static_cast<long long>(position) * half;
  const float* rs = sine + static_cast<long long>(position) * half;
  float* kc = key_cache + (slot >= 0 ? slot * kv_dim : 0);
  float* vc = value_cache + (slot >= 0 ? slot * kv_dim : 0);
  const long long kv_rows = slot >= 0 ? kv_dim : 0;
  const hipStream_t s = as_stream(stream);
  const bool fast = (input_dim >> 5) % 2 == 0 && input_dim < (1LL << 31) &&
                    reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(packed_q) % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(packed_k) % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(packed_v) % 4 == 0 &&
                    query_dim + 2 * kv_rows < (1LL << 30);
  if (fast)
    return finish(qc::launch_qgemv_qkv_rope(format, packed_q, packed_k, packed_v, q, kc, vc,
                                            static_cast<int>(query_dim),
                                            static_cast<int>(kv_rows), static_cast<int>(half),
                                            rc, rs, x, static_cast<int>(input_dim), s));
  if (half > INT_MAX) return QC_INVALID_SHAPE;   // this library's dimension limit
  const qc::GemvTuning t = tuning();
  hipError_t e = qc::launch_qgemm(format, packed_q, x, q, 1, query_dim, input_dim, s, t);
  if (e == hipSuccess)
    e = qc::launch_rope_pairs(q, query_heads, static_cast<int>(half), rc, rs, s);
  if (e == hipSuccess && slot >= 0) {
    e = qc::launch_qgemm(format, packed_k, x, kc, 1, kv_dim, input_dim, s, t);
    if (e == hipSuccess)
      e = qc::launch_rope_pairs(kc, kv_heads, static_cast<int>(half), rc, rs, s);
    if (e == hipSuccess)
      e = qc::launch_qgemm(format, packed_v, x, vc, 1, kv_dim, input_dim, s, t);
  }
  return finish(e);
}

// Canonical int8 projections: shapes (rows, cols, groups; shared cols and
// groups; the mode's pairing), storage types, then pointers.
int qc_hip_cint8_project(int mode, const qc_cint8_weights* w, int nw, const void* x, int x_type,
                         long long m, void* const* y, const int* y_type, const float* bias,
                         int activation, const float* rope_cos, const float* rope_sin,
                         long long head_dim, void* stream) {
  if (mode < 0 || mode > 2 || activation < 0 || activation > 4 || w == nullptr || y == nullptr ||
      y_type == nullptr)
    return QC_INVALID_ARGUMENT;
  if (nw < 1 || nw > 3 || (mode == 1 && nw != 2) || (mode == 2 && nw == 2) || m < 1 ||
      m > INT_MAX)
    return QC_INVALID_SHAPE;
  long long total = 0;
  for (int i = 0; i < nw; ++i) {
    const qc_cint8_weights& a = w[i];
    if (!valid_product({a.rows, a.cols}) || a.groups < 1 || a.cols % a.groups != 0 ||
        a.cols != w[0].cols || a.groups != w[0].groups || a.cols > INT_MAX)
      return QC_INVALID_SHAPE;
    if (mode == 2 && (head_dim <= 0 || head_dim % 2 != 0 || a.rows % head_dim != 0))
      return QC_INVALID_SHAPE;
    total += a.rows;
  }
  if (mode == 1 && w[1].rows != w[0].rows) return QC_INVALID_SHAPE;
  if (mode == 1) total = 2 * w[0].rows;
  if (mode == 2 && m != 1) return QC_INVALID_SHAPE;
  if (total >= (1LL << 30) || !valid_product({m, total})) return QC_INVALID_SHAPE;
  const int nout = mode == 1 ? 1 : nw;
  auto known = [](int t) { return t == QC_STORAGE_F32 || t == QC_STORAGE_F16 || t == QC_STORAGE_BF16; };
  if (!known(x_type)) return QC_UNSUPPORTED_FORMAT;
  for (int i = 0; i < nout; ++i)
    if (!known(y_type[i])) return QC_UNSUPPORTED_FORMAT;
  if (x == nullptr || (mode == 2 && (rope_cos == nullptr || rope_sin == nullptr)))
    return QC_INVALID_ARGUMENT;
  for (int i = 0; i < nw; ++i)
    if (w[i].codes == nullptr || w[i].scales == nullptr ||
        (w[i].zero_points == nullptr) != (w[0].zero_points == nullptr))
      return QC_INVALID_ARGUMENT;
  for (int i = 0; i < nout; ++i)
    if (y[i] == nullptr) return QC_INVALID_ARGUMENT;
  qc::CInt8Launch L;
  L.mode = mode;
  L.nw = nw;
  for (int i = 0; i < nw; ++i) L.w[i] = w[i];
  L.x = x;
  L.xtype = x_type;
  L.ldx = w[0].cols;
  L.m = m;
  for (int i = 0; i < nout; ++i) {
    L.y[i] = y[i];
    L.ytype[i] = y_type[i];
  }
  L.bias = mode == 0 && nw == 1 ? bias : nullptr;
  L.act = mode == 0 && nw == 1 ? activation : 0;
  if (mode == 2) {
    L.half = static_cast<int>(head_dim / 2);
    L.nrope = nw == 1 ? 1 : 2;
    L.rope_cos = rope_cos;
    L.rope_sin = rope_sin;
  }
  const qc::GemvTuning t = tuning();
  const int rw = t.rows_per_wave;
  L.rows_per_wave = rw == 2 || rw == 4 || rw == 8 ? rw : 0;
  L.dot = t.cint8_dot;
  return finish(qc::launch_cint8(L, as_stream(stream)));
}

// The int8 branch of dequantize_canonical
// (kernels/quantization/quant_import_ref.cpp:753-770).  The caller (the
// drop-in) has run the reference's tensor validation; this checks what the
// kernel relies on.
int qc_hip_cint8_dequantize(const qc_cint8_weights* w, const int* group_index, float* out,
                            void* stream) {
  if (w == nullptr) return QC_INVALID_ARGUMENT;
  if (!valid_product({w->rows, w->cols}) || w->groups < 1 ||
      (group_index == nullptr && w->cols % w->groups != 0))
    return QC_INVALID_SHAPE;
  if (w->codes == nullptr || w->scales == nullptr || out == nullptr) return QC_INVALID_ARGUMENT;
  return finish(qc::launch_cint8_dequant(w->codes, w->scales, w->zero_points, group_index,
                                         w->rows, w->cols, w->groups, w->cols / w->groups, out,
                                         as_stream(stream)));
}

int qc_hip_cint8_quantized_gemm(const qc_cint8_weights* w, const qc_cint8_weights* a,
                                const int* a_int_zero_points, float* y, void* stream) {
  if (w == nullptr || a == nullptr) return QC_INVALID_ARGUMENT;
  if (!valid_product({w->rows, w->cols}) || !valid_product({a->rows, a->cols}) ||
      !valid_product({a->rows, w->rows}) || a->cols != w->cols || w->groups < 1 ||
      a->groups < 1 || w->cols % w->groups != 0 || a->cols % a->groups != 0)
    return QC_INVALID_SHAPE;
  if (w->codes == nullptr || w->scales == nullptr || a->codes == nullptr ||
      a->scales == nullptr || y == nullptr)
    return QC_INVALID_ARGUMENT;
  return finish(qc::launch_cint8_dual(*w, *a, a_int_zero_points, y, int8_route(),
                                      as_stream(stream)));
}

int qc_hip_storage_to_f32(const void* x, int type, long long count, float* out, void* stream) {
  if (count <= 0) return QC_INVALID_SHAPE;
  if (type != QC_STORAGE_F32 && type != QC_STORAGE_F16 && type != QC_STORAGE_BF16)
    return QC_UNSUPPORTED_FORMAT;
  if (x == nullptr || out == nullptr) return QC_INVALID_ARGUMENT;
  return finish(qc::launch_storage_to_f32(x, type, count, out, as_stream(stream)));
}

// src/dispatch/qgemv_w8a8.cpp:108-125 (qgemv_w8a8_packed_size).
int qc_hip_qgemv_w8a8_packed_size(int format, long long n, long long k, long long* bytes) {
  size_t size = 0;
  const int st = qc_hip_qgemv_packed_size(format, n, k, &size);
  if (st != QC_OK) return st;
  if (bytes == nullptr) return QC_INVALID_ARGUMENT;
  if (size > static_cast<size_t>(LLONG_MAX)) return QC_INVALID_SHAPE;
  *bytes = static_cast<long long>(size);
  return QC_OK;
}

// src/dispatch/qgemv_w8a8.cpp:130-153: format and shape (99-105), nulls, then a
// non-finite x, all before any work.
int qc_hip_qgemv_w8a8(int format, const void* packed, const float* x, float* y, long long n,
                      long long k, int* dev_status, void* stream) {
  const int st = validate(format, n, k);
  if (st != QC_OK) return st;
  size_t ignored = 0;
  if (packed_bytes(format, n, k, &ignored) != QC_OK) return QC_INVALID_SHAPE;
  if (packed == nullptr || x == nullptr || y == nullptr) return QC_INVALID_ARGUMENT;
  const hipStream_t s = as_stream(stream);
  if (dev_status != nullptr)
    return finish(qc::launch_qgemv_w8a8(format, packed, x, y, n, k, tuning().rows_per_wave,
                                        dev_status, s));
  bool finite = false;
  const int fst = all_finite(x, k, s, &finite);
  if (fst != QC_OK) return fst;
  if (!finite) return QC_INVALID_ARGUMENT;
  hipError_t e = qc::launch_qgemv_w8a8(format, packed, x, y, n, k, tuning().rows_per_wave,
                                       nullptr, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return finish(e);
}

const char* qc_hip_qgemv_w8a8_variant(int format) {
  if (block_bytes(format) == 0) return "unsupported";
  return format == QC_Q8_0 ? "hip_gfx950_w8a8_q8_0" : "hip_gfx950_w8a8_q4_0";
}

int qc_hip_set_qgemm_plan(int waves, int stages) {
  if (waves != 0 && waves != 4 && waves != 8) return QC_INVALID_ARGUMENT;
  if (stages != 0 && stages != 1 && stages != 2 && stages != 4 && stages != 8 && stages != 16)
    return QC_INVALID_ARGUMENT;
  g_knobs.qgemm_plan.store(waves | stages << 8, std::memory_order_relaxed);
  return QC_OK;
}

// kernels/norms/norm_quant_ref.cpp:106-114,117-130 (shape: rows x hidden
// product, finite eps >= 0, group 0 -> hidden dividing hidden; then nulls).
// Data-dependent failure (a group whose normalized values are not finite)
// is reported after the work, as the reference does: that group's scale and
// codes are left unwritten, everything else is written.
int qc_hip_rms_norm_add_quant_int8(const float* x, const float* residual, const float* weight,
                                   int8_t* codes, float* residual_out, float* scales,
                                   long long rows, long long hidden, float eps,
                                   long long group_size, int* dev_status, void* stream) {
  if (!valid_product({rows, hidden}) || !std::isfinite(eps) || eps < 0.0f)
    return QC_INVALID_SHAPE;
  if (group_size == 0) group_size = hidden;
  if (group_size <= 0 || hidden % group_size != 0) return QC_INVALID_SHAPE;
  if (!x || !residual || !weight || !codes || !residual_out || !scales)
    return QC_INVALID_ARGUMENT;
  const hipStream_t s = as_stream(stream);
  const bool seq = g_knobs.norm_sequential.load(std::memory_order_relaxed);
  if (dev_status != nullptr)
    return finish(qc::launch_rms_norm_add_quant_int8(x, residual, weight, codes, residual_out,
                                                     scales, rows, hidden, eps, group_size,
                                                     seq, dev_status, s));
  int bad = 0;
  const int st = with_flag(s, &bad, [&](int* flag) {
    return qc::launch_rms_norm_add_quant_int8(x, residual, weight, codes, residual_out, scales,
                                              rows, hidden, eps, group_size, seq, flag, s);
  });
  if (st != QC_OK) return st;
  return bad ? QC_INVALID_ARGUMENT : QC_OK;
}

// kernels/quantization/quantization_ref.cpp:190-197: shape, nulls, finite x.
int qc_hip_quantize_int8_asymmetric(const float* x, int8_t* codes, float* scales,
                                    int* zero_points, long long rows, long long dim,
                                    int* dev_status, void* stream) {
  if (!valid_product({rows, dim})) return QC_INVALID_SHAPE;
  if (!x || !codes || !scales || !zero_points) return QC_INVALID_ARGUMENT;
  const hipStream_t s = as_stream(stream);
  if (dev_status != nullptr)
    return finish(qc::launch_quantize_int8_asymmetric(x, codes, scales, zero_points, rows, dim,
                                                      dev_status, s));
  bool finite = false;
  const int st = all_finite(x, rows * dim, s, &finite);
  if (st != QC_OK) return st;
  if (!finite) return QC_INVALID_ARGUMENT;
  hipError_t e = qc::launch_quantize_int8_asymmetric(x, codes, scales, zero_points, rows, dim,
                                                     nullptr, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return finish(e);
}

// kernels/quantization/quantization_ref.cpp:228-244.
int qc_hip_dequantize_int8_asymmetric(const int8_t* codes, const float* scales,
                                      const int* zero_points, float* out, long long rows,
                                      long long dim, void* stream) {
  if (!valid_product({rows, dim})) return QC_INVALID_SHAPE;
  if (!codes || !scales || !zero_points || !out) return QC_INVALID_ARGUMENT;
  return finish(qc::launch_dequantize_int8_asymmetric(codes, scales, zero_points, out, rows,
                                                      dim, as_stream(stream)));
}

int qc_hip_set_qgemm_panel(int mode) {
  if (mode < -1 || mode > 2) return QC_INVALID_ARGUMENT;
  g_knobs.qgemm_panel.store(mode, std::memory_order_relaxed);
  return QC_OK;
}

int qc_hip_set_qgemm_rows(int mode) {
  if (mode < -1 || mode > 1) return QC_INVALID_ARGUMENT;
  g_knobs.qgemm_rows.store(mode, std::memory_order_relaxed);
  return QC_OK;
}

int qc_hip_set_cint8_dot(int mode) {
  if (mode < -1 || mode > 1) return QC_INVALID_ARGUMENT;
  g_knobs.cint8_dot.store(mode, std::memory_order_relaxed);
  return QC_OK;
}

int qc_hip_set_qgemm_fold(int mode) {
  if (mode < -1 || mode > 0) return QC_INVALID_ARGUMENT;
  g_knobs.qgemm_fold.store(mode, std::memory_order_relaxed);
  return QC_OK;
}

int qc_hip_set_norm_sequential_sum(int on) {
  g_knobs.norm_sequential.store(on != 0, std::memory_order_relaxed);
  return QC_OK;
}

int qc_hip_set_int8_gemm_route(int route) {
  if (route < qc::kInt8Auto || route > qc::kInt8Simple) return QC_INVALID_ARGUMENT;
  g_knobs.int8_route.store(route, std::memory_order_relaxed);
  return QC_OK;
}

}  // extern "C"

// C++ drop-in API (include/quixicore_cpu/*.h) over the C ABI.
//
// The reference ops are synchronous and take untyped host pointers.  Here a
// pointer the GPU can address (hipMalloc or managed memory) is used in
// place; any other buffer is staged: copied to a device buffer before the
// launch and, for outputs, copied back after it.  Every call waits for its
// kernels, so outputs are ready on return exactly as in the reference.
// Validation happens in the C ABI first, so an invalid call touches nothing.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstring>
#include <mutex>
#include <vector>

#include "quixicore_cpu/qgemm.h"
#include "quixicore_cpu/qgemv.h"
#include "quixicore_cpu/qgemv_w8a8.h"
#include "quixicore_cpu/quantization.h"
#include "quixicore_hip.h"
#include "qc_dropin.h"

namespace quixicore_cpu {
namespace detail {

hipStream_t library_stream() {
  static std::mutex mu;
  static std::vector<hipStream_t> streams;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (static_cast<int>(streams.size()) <= dev) streams.resize(dev + 1, nullptr);
  if (streams[dev] == nullptr) {
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    streams[dev] = s;
  }
  return streams[dev];
}

bool device_accessible(const void* p) {
  if (p == nullptr) return false;
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

Status from_hip(hipError_t e) {
  if (e == hipSuccess) return Status::kOk;
  return e == hipErrorOutOfMemory ? Status::kOutOfMemory : Status::kDeviceError;
}

Staging::~Staging() {
  for (void* p : owned_) (void)hipFree(p);
}

void* Staging::device(std::size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (workspace_ != nullptr) {
    void* p = workspace_->allocate(bytes);
    if (p == nullptr) status_ = Status::kOutOfMemory;
    return p;
  }
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    status_ = from_hip(e);
    return nullptr;
  }
  owned_.push_back(p);
  return p;
}

const void* Staging::in(const void* host_or_device, std::size_t bytes) {
  if (host_or_device == nullptr || device_accessible(host_or_device)) return host_or_device;
  void* d = device(bytes);
  if (d == nullptr) return nullptr;
  const hipError_t e = hipMemcpyAsync(d, host_or_device, bytes, hipMemcpyHostToDevice, stream_);
  if (e != hipSuccess) status_ = from_hip(e);
  return d;
}

void* Staging::out(void* host_or_device, std::size_t bytes) {
  if (host_or_device == nullptr || device_accessible(host_or_device)) return host_or_device;
  void* d = device(bytes);
  if (d == nullptr) return nullptr;
  back_.push_back({host_or_device, d, bytes});
  return d;
}

void* Staging::inout(void* host_or_device, std::size_t bytes) {
  if (host_or_device == nullptr || device_accessible(host_or_device)) return host_or_device;
  void* d = device(bytes);
  if (d == nullptr) return nullptr;
  const hipError_t e = hipMemcpyAsync(d, host_or_device, bytes, hipMemcpyHostToDevice, stream_);
  if (e != hipSuccess) status_ = from_hip(e);
  back_.push_back({host_or_device, d, bytes});
  return d;
}

Status Staging::finish(int capi_status) {
  if (capi_status != QC_OK) {
    (void)hipStreamSynchronize(stream_);
    return static_cast<Status>(capi_status);
  }
  for (const Back& b : back_) {
    const hipError_t e = hipMemcpyAsync(b.host, b.dev, b.bytes, hipMemcpyDeviceToHost, stream_);
    if (e != hipSuccess) return from_hip(e);
  }
  return from_hip(hipStreamSynchronize(stream_));
}

Status Staging::finish_written(int capi_status) {
  if (capi_status != QC_INVALID_ARGUMENT) return finish(capi_status);
  const Status copied = finish(QC_OK);
  return copied == Status::kOk ? Status::kInvalidArgument : copied;
}

}  // namespace detail

namespace {

using detail::Staging;

int fmt_id(QuantFormat f) { return static_cast<int>(f); }

size_t packed_or_zero(QuantFormat f, long long n, long long k) {
  size_t size = 0;
  return qc_hip_qgemv_packed_size(fmt_id(f), n, k, &size) == QC_OK ? size : 0;
}

}  // namespace

Status qgemv_packed_size(QuantFormat format, long long n, long long k, size_t* size) {
  return static_cast<Status>(qc_hip_qgemv_packed_size(fmt_id(format), n, k, size));
}

Status qgemv_pack(QuantFormat format, const float* weights, long long n, long long k,
                  void* packed) {
  size_t bytes = 0;
  const int st = qc_hip_qgemv_packed_size(fmt_id(format), n, k, &bytes);
  if (st != QC_OK) return static_cast<Status>(st);
  if (weights == nullptr || packed == nullptr) return Status::kInvalidArgument;
  Staging g(nullptr);
  const float* w = static_cast<const float*>(g.in(weights, sizeof(float) * n * k));
  void* p = g.out(packed, bytes);
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemv_pack(fmt_id(format), w, n, k, p, nullptr, g.stream()));
}

Status qgemv_unpack(QuantFormat format, const void* packed, long long n, long long k,
                    float* weights) {
  size_t bytes = 0;
  const int st = qc_hip_qgemv_packed_size(fmt_id(format), n, k, &bytes);
  if (st != QC_OK) return static_cast<Status>(st);
  if (packed == nullptr || weights == nullptr) return Status::kInvalidArgument;
  Staging g(nullptr);
  const void* p = g.in(packed, bytes);
  float* w = static_cast<float*>(g.out(weights, sizeof(float) * n * k));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemv_unpack(fmt_id(format), p, n, k, w, g.stream()));
}

Status qgemv(QuantFormat format, const void* packed, const float* x, float* y, long long n,
             long long k) {
  const size_t bytes = packed_or_zero(format, n, k);
  if (bytes == 0 || packed == nullptr || x == nullptr || y == nullptr)
    return static_cast<Status>(qc_hip_qgemv(fmt_id(format), packed, x, y, n, k, nullptr));
  Staging g(nullptr);
  const void* p = g.in(packed, bytes);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * k));
  float* yd = static_cast<float*>(g.out(y, sizeof(float) * n));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemv(fmt_id(format), p, xd, yd, n, k, g.stream()));
}

const char* qgemv_variant(QuantFormat format) { return qc_hip_qgemv_variant(fmt_id(format)); }

Status qgemv_up_gate(QuantFormat format, const void* packed_up, const void* packed_gate,
                     const float* x, float* up, float* gate, long long n, long long k) {
  const int pre = qc_hip_qgemv_up_gate(fmt_id(format), nullptr, nullptr, nullptr, nullptr,
                                       nullptr, n, k, nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (!packed_up || !packed_gate || !x || !up || !gate) return Status::kInvalidArgument;
  const size_t bytes = packed_or_zero(format, n, k);
  if (bytes == 0)
    return static_cast<Status>(
        qc_hip_qgemv_up_gate(fmt_id(format), packed_up, packed_gate, x, up, gate, n, k, nullptr));
  Staging g(nullptr);
  const void* pu = g.in(packed_up, bytes);
  const void* pg = g.in(packed_gate, bytes);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * k));
  float* ud = static_cast<float*>(g.out(up, sizeof(float) * n));
  float* gd = static_cast<float*>(g.out(gate, sizeof(float) * n));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemv_up_gate(fmt_id(format), pu, pg, xd, ud, gd, n, k, g.stream()));
}

Status qgemv_up_gate_activation(QuantFormat format, const void* packed_up,
                                const void* packed_gate, const float* x, float* out,
                                long long n, long long k, bool gelu_tanh) {
  const int pre = qc_hip_qgemv_up_gate_activation(fmt_id(format), nullptr, nullptr, nullptr,
                                                  nullptr, n, k, gelu_tanh, nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (!packed_up || !packed_gate || !x || !out) return Status::kInvalidArgument;
  const size_t bytes = packed_or_zero(format, n, k);
  if (bytes == 0)
    return static_cast<Status>(qc_hip_qgemv_up_gate_activation(
        fmt_id(format), packed_up, packed_gate, x, out, n, k, gelu_tanh, nullptr));
  Staging g(nullptr);
  const void* pu = g.in(packed_up, bytes);
  const void* pg = g.in(packed_gate, bytes);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * k));
  float* od = static_cast<float*>(g.out(out, sizeof(float) * n));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemv_up_gate_activation(fmt_id(format), pu, pg, xd, od, n, k,
                                                  gelu_tanh, g.stream()));
}

Status qgemv_qkv(QuantFormat format, const void* packed_q, const void* packed_k,
                 const void* packed_v, const float* x, float* q, float* k_out, float* v_out,
                 long long query_dim, long long kv_dim, long long input_dim) {
  const int pre = qc_hip_qgemv_qkv(fmt_id(format), nullptr, nullptr, nullptr, nullptr, nullptr,
                                   nullptr, nullptr, query_dim, kv_dim, input_dim, nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (!packed_q || !packed_k || !packed_v || !x || !q || !k_out || !v_out)
    return Status::kInvalidArgument;
  const size_t qb = packed_or_zero(format, query_dim, input_dim);
  const size_t kb = packed_or_zero(format, kv_dim, input_dim);
  if (qb == 0 || kb == 0)
    return static_cast<Status>(qc_hip_qgemv_qkv(fmt_id(format), packed_q, packed_k, packed_v, x,
                                                q, k_out, v_out, query_dim, kv_dim, input_dim,
                                                nullptr));
  Staging g(nullptr);
  const void* pq = g.in(packed_q, qb);
  const void* pk = g.in(packed_k, kb);
  const void* pv = g.in(packed_v, kb);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * input_dim));
  float* qd = static_cast<float*>(g.out(q, sizeof(float) * query_dim));
  float* kd = static_cast<float*>(g.out(k_out, sizeof(float) * kv_dim));
  float* vd = static_cast<float*>(g.out(v_out, sizeof(float) * kv_dim));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemv_qkv(fmt_id(format), pq, pk, pv, xd, qd, kd, vd, query_dim, kv_dim,
                                   input_dim, g.stream()));
}

// Only the position's cos / sin rows and the slot's cache rows are staged;
// the C ABI then sees one position and one slot.
Status qgemv_qkv_rope_kv(QuantFormat format, const void* packed_q, const void* packed_k,
                         const void* packed_v, const float* x, const float* cosine,
                         const float* sine, float* q, float* key_cache, float* value_cache,
                         long long query_heads, long long kv_heads, long long head_dim,
                         long long input_dim, long long slots, long long max_position,
                         int position, int slot) {
  const int pre = qc_hip_qgemv_qkv_rope_kv(fmt_id(format), nullptr, nullptr, nullptr, nullptr,
                                           nullptr, nullptr, nullptr, nullptr, nullptr,
                                           query_heads, kv_heads, head_dim, input_dim, slots,
                                           max_position, position, slot, nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (!packed_q || !packed_k || !packed_v || !x || !cosine || !sine || !q || !key_cache ||
      !value_cache)
    return Status::kInvalidArgument;
  const long long query_dim = query_heads * head_dim;
  const long long kv_dim = kv_heads * head_dim;
  const long long half = head_dim / 2;
  const size_t qb = packed_or_zero(format, query_dim, input_dim);
  const size_t kb = packed_or_zero(format, kv_dim, input_dim);
  if (qb == 0 || kb == 0)
    return static_cast<Status>(qc_hip_qgemv_qkv_rope_kv(
        fmt_id(format), packed_q, packed_k, packed_v, x, cosine, sine, q, key_cache,
        value_cache, query_heads, kv_heads, head_dim, input_dim, slots, max_position, position,
        slot, nullptr));
  Staging g(nullptr);
  const void* pq = g.in(packed_q, qb);
  const void* pk = slot >= 0 ? g.in(packed_k, kb) : packed_k;
  const void* pv = slot >= 0 ? g.in(packed_v, kb) : packed_v;
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * input_dim));
  const float* cd = static_cast<const float*>(g.in(cosine + position * half, sizeof(float) * half));
  const float* sd = static_cast<const float*>(g.in(sine + position * half, sizeof(float) * half));
  float* qd = static_cast<float*>(g.out(q, sizeof(float) * query_dim));
  float* kd = key_cache;
  float* vd = value_cache;
  if (slot >= 0) {
    kd = static_cast<float*>(g.out(key_cache + slot * kv_dim, sizeof(float) * kv_dim));
    vd = static_cast<float*>(g.out(value_cache + slot * kv_dim, sizeof(float) * kv_dim));
  }
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemv_qkv_rope_kv(fmt_id(format), pq, pk, pv, xd, cd, sd, qd, kd, vd,
                                           query_heads, kv_heads, head_dim, input_dim, 1, 1, 0,
                                           slot >= 0 ? 0 : -1, g.stream()));
}

Status qgemv_w8a8(QuantFormat format, const void* packed_weights, const float* x, float* y,
                  long long n, long long k) {
  const size_t bytes = packed_or_zero(format, n, k);
  if (bytes == 0 || packed_weights == nullptr || x == nullptr || y == nullptr)
    return static_cast<Status>(
        qc_hip_qgemv_w8a8(fmt_id(format), packed_weights, x, y, n, k, nullptr, nullptr));
  Staging g(nullptr);
  const void* p = g.in(packed_weights, bytes);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * k));
  float* yd = static_cast<float*>(g.out(y, sizeof(float) * n));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemv_w8a8(fmt_id(format), p, xd, yd, n, k, nullptr, g.stream()));
}

Status qgemv_w8a8_packed_size(QuantFormat format, long long n, long long k, long long* bytes) {
  return static_cast<Status>(qc_hip_qgemv_w8a8_packed_size(fmt_id(format), n, k, bytes));
}

Status qgemv_w8a8_pack(QuantFormat format, const float* weights, long long n, long long k,
                       void* packed) {
  return qgemv_pack(format, weights, n, k, packed);
}

const char* qgemv_w8a8_variant(QuantFormat format) {
  return qc_hip_qgemv_w8a8_variant(fmt_id(format));
}

Status qgemm(QuantFormat format, const void* packed_weights, const float* x, float* y,
             long long m, long long n, long long k) {
  const size_t bytes = packed_or_zero(format, n, k);
  if (bytes == 0 || m <= 0 || m > INT_MAX || packed_weights == nullptr || x == nullptr ||
      y == nullptr)
    return static_cast<Status>(
        qc_hip_qgemm(fmt_id(format), packed_weights, x, y, m, n, k, nullptr));
  Staging g(nullptr);
  const void* p = g.in(packed_weights, bytes);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * m * k));
  float* yd = static_cast<float*>(g.out(y, sizeof(float) * m * n));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_qgemm(fmt_id(format), p, xd, yd, m, n, k, g.stream()));
}

Status quantize_int8(const float* x, std::int8_t* codes, float* scales, long long rows,
                     long long dim, long long group_size) {
  // Shape and null validation first, without touching memory.
  const int pre = qc_hip_quantize_int8(nullptr, nullptr, nullptr, rows, dim, group_size,
                                       nullptr, nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (x == nullptr || codes == nullptr || scales == nullptr) return Status::kInvalidArgument;
  const long long groups = dim / (group_size == 0 ? dim : group_size);
  Staging g(nullptr);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * rows * dim));
  auto* cd = static_cast<std::int8_t*>(g.out(codes, static_cast<size_t>(rows * dim)));
  float* sd = static_cast<float*>(g.out(scales, sizeof(float) * rows * groups));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(
      qc_hip_quantize_int8(xd, cd, sd, rows, dim, group_size, nullptr, g.stream()));
}

Status rms_norm_add_quant_int8(const float* x, const float* residual, const float* weight,
                               std::int8_t* codes, float* residual_out, float* scales,
                               long long rows, long long hidden, float eps,
                               long long group_size) {
  // Shape and null validation first, without touching memory.
  const int pre = qc_hip_rms_norm_add_quant_int8(nullptr, nullptr, nullptr, nullptr, nullptr,
                                                 nullptr, rows, hidden, eps, group_size, nullptr,
                                                 nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (!x || !residual || !weight || !codes || !residual_out || !scales)
    return Status::kInvalidArgument;
  const long long groups = hidden / (group_size == 0 ? hidden : group_size);
  Staging g(nullptr);
  const size_t row_bytes = sizeof(float) * rows * hidden;
  // residual_out may be x or residual itself: stage such a buffer once
  float* rod = static_cast<float*>(g.inout(residual_out, row_bytes));
  const float* xd = x == residual_out ? rod : static_cast<const float*>(g.in(x, row_bytes));
  const float* rd =
      residual == residual_out ? rod : static_cast<const float*>(g.in(residual, row_bytes));
  const float* wd = static_cast<const float*>(g.in(weight, sizeof(float) * hidden));
  // an invalid group keeps the caller's codes and scale, as in the reference
  auto* cd = static_cast<std::int8_t*>(g.inout(codes, static_cast<size_t>(rows * hidden)));
  float* sd = static_cast<float*>(g.inout(scales, sizeof(float) * rows * groups));
  if (g.status() != Status::kOk) return g.status();
  return g.finish_written(qc_hip_rms_norm_add_quant_int8(xd, rd, wd, cd, rod, sd, rows, hidden,
                                                         eps, group_size, nullptr, g.stream()));
}

Status quantize_int8_asymmetric(const float* x, std::int8_t* codes, float* scales,
                                int* zero_points, long long rows, long long dim) {
  const int pre = qc_hip_quantize_int8_asymmetric(nullptr, nullptr, nullptr, nullptr, rows, dim,
                                                  nullptr, nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (!x || !codes || !scales || !zero_points) return Status::kInvalidArgument;
  Staging g(nullptr);
  const float* xd = static_cast<const float*>(g.in(x, sizeof(float) * rows * dim));
  auto* cd = static_cast<std::int8_t*>(g.out(codes, static_cast<size_t>(rows * dim)));
  float* sd = static_cast<float*>(g.out(scales, sizeof(float) * rows));
  int* zd = static_cast<int*>(g.out(zero_points, sizeof(int) * rows));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(
      qc_hip_quantize_int8_asymmetric(xd, cd, sd, zd, rows, dim, nullptr, g.stream()));
}

Status dequantize_int8_asymmetric(const std::int8_t* codes, const float* scales,
                                  const int* zero_points, float* out, long long rows,
                                  long long dim) {
  const int pre = qc_hip_dequantize_int8_asymmetric(nullptr, nullptr, nullptr, nullptr, rows,
                                                    dim, nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (!codes || !scales || !zero_points || !out) return Status::kInvalidArgument;
  Staging g(nullptr);
  const auto* cd = static_cast<const std::int8_t*>(g.in(codes, static_cast<size_t>(rows * dim)));
  const float* sd = static_cast<const float*>(g.in(scales, sizeof(float) * rows));
  const int* zd = static_cast<const int*>(g.in(zero_points, sizeof(int) * rows));
  float* od = static_cast<float*>(g.out(out, sizeof(float) * rows * dim));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_dequantize_int8_asymmetric(cd, sd, zd, od, rows, dim, g.stream()));
}

Status int8_gemm(const std::int8_t* weights, const std::int8_t* x, const float* weight_scale,
                 const float* activation_scale, const std::int32_t* weight_row_sum,
                 const int* activation_zero_point, float* y, long long m, long long n,
                 long long k, bool asymmetric) {
  const int pre = qc_hip_int8_gemm(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                   nullptr, m, n, k, 0, nullptr, nullptr);
  if (pre == QC_INVALID_SHAPE) return Status::kInvalidShape;
  if (weights == nullptr || x == nullptr || weight_scale == nullptr ||
      activation_scale == nullptr || y == nullptr ||
      (asymmetric && (weight_row_sum == nullptr || activation_zero_point == nullptr)))
    return Status::kInvalidArgument;
  Staging g(nullptr);
  const auto* wd = static_cast<const std::int8_t*>(g.in(weights, static_cast<size_t>(n * k)));
  const auto* xd = static_cast<const std::int8_t*>(g.in(x, static_cast<size_t>(m * k)));
  const auto* wsd = static_cast<const float*>(g.in(weight_scale, sizeof(float) * n));
  const auto* asd = static_cast<const float*>(g.in(activation_scale, sizeof(float) * m));
  const std::int32_t* rsd = nullptr;
  const int* zpd = nullptr;
  if (asymmetric) {
    rsd = static_cast<const std::int32_t*>(g.in(weight_row_sum, sizeof(std::int32_t) * n));
    zpd = static_cast<const int*>(g.in(activation_zero_point, sizeof(int) * m));
  }
  float* yd = static_cast<float*>(g.out(y, sizeof(float) * m * n));
  if (g.status() != Status::kOk) return g.status();
  return g.finish(qc_hip_int8_gemm(wd, xd, wsd, asd, rsd, zpd, yd, m, n, k, asymmetric ? 1 : 0,
                                   nullptr, g.stream()));
}

const char* int8_gemm_variant() { return qc_hip_int8_gemm_variant(); }

Status qgemm_w8a8(const std::int8_t* weights, const std::int8_t* x, const float* weight_scale,
                  const float* activation_scale, float* y, long long m, long long n,
                  long long k) {
  return int8_gemm(weights, x, weight_scale, activation_scale, nullptr, nullptr, y, m, n, k,
                   false);
}

Status qgemm_w8a8_azp(const std::int8_t* weights, const std::int8_t* x,
                      const float* weight_scale, const float* activation_scale,
                      const std::int32_t* weight_row_sum, const int* activation_zero_point,
                      float* y, long long m, long long n, long long k) {
  return int8_gemm(weights, x, weight_scale, activation_scale, weight_row_sum,
                   activation_zero_point, y, m, n, k, true);
}

}  // namespace quixicore_cpu

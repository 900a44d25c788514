// Reference-side binding of the gfx950 C ABI (include/quixicore_hip.h) into
// QuixiCore-CPU's own dispatch: the code a maintainer adds to the reference,
// e.g. as src/dispatch/hip_gfx950.h, called from qgemv(), qgemm(),
// quantize_int8() and int8_gemm() after their own validation.  It is compiled
// here by tests/cpp/reference_binding_check.cpp and driven with host buffers
// by tests/test_gpu_reference_binding.py.
//
// The reference's public ops take host pointers and return with their outputs
// ready (src/dispatch/qgemv.cpp:337-365, src/dispatch/int8_gemm.cpp:67-94).
// The C ABI takes device pointers and runs on a stream.  Each function below
// therefore stages its host operands into one device allocation, calls the
// C ABI with dev_status = NULL (the C ABI then validates in the reference's
// order, scans data-dependent conditions first and blocks), copies the
// outputs back only on success, so that outputs stay untouched on error as
// in the reference, and returns the C ABI status unchanged: 0..4 are the
// reference's Status values, 5 a device error (no Status counterpart; it
// reaches the caller as static_cast<Status>(5), which is not kOk).
#pragma once

#include <hip/hip_runtime_api.h>

#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <vector>

#include "quixicore_hip.h"

namespace quixicore_cpu::hip_gfx950 {

// True when device 0 is a gfx950 GPU (the variant's `supported` predicate).
inline bool available() {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count < 1) return false;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return false;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}

// The variant is chosen unless the reference's override names another one
// (QUIXICORE_CPU_QGEMV_VARIANT / QUIXICORE_CPU_INT8_GEMM_VARIANT = "ref" forces the
// CPU route for A/B runs, as the reference's tests do).
inline bool selected(const char* env_name) {
  const char* forced = std::getenv(env_name);
  return (forced == nullptr || std::strcmp(forced, "hip_gfx950") == 0) && available();
}

namespace detail {

// One device allocation holding every operand, each part 256-byte aligned.
class Staging {
 public:
  Staging() = default;
  Staging(const Staging&) = delete;
  Staging& operator=(const Staging&) = delete;
  ~Staging() {
    if (base_ != nullptr) (void)hipFree(base_);
  }

  // Reserves `bytes` for host buffer `host` (copied in by upload when `in`).
  std::size_t add(const void* host, std::size_t bytes, bool in) {
    const std::size_t off = total_;
    parts_.push_back({host, bytes, off, in});
    total_ += (bytes + 255) / 256 * 256;
    return parts_.size() - 1;
  }
  int upload() {
    if (hipMalloc(&base_, total_ == 0 ? 256 : total_) != hipSuccess) {
      base_ = nullptr;
      return QC_OUT_OF_MEMORY;
    }
    for (const Part& p : parts_)
      if (p.in && p.bytes != 0 &&
          hipMemcpy(static_cast<char*>(base_) + p.off, p.host, p.bytes, hipMemcpyHostToDevice) !=
              hipSuccess)
        return QC_DEVICE_ERROR;
    return QC_OK;
  }
  template <class T>
  T* device(std::size_t id) const {
    return parts_[id].bytes == 0 ? nullptr
                                 : reinterpret_cast<T*>(static_cast<char*>(base_) + parts_[id].off);
  }
  int download(std::size_t id, void* host) const {
    const Part& p = parts_[id];
    if (p.bytes == 0) return QC_OK;
    return hipMemcpy(host, static_cast<char*>(base_) + p.off, p.bytes, hipMemcpyDeviceToHost) ==
                   hipSuccess
               ? QC_OK
               : QC_DEVICE_ERROR;
  }

 private:
  struct Part {
    const void* host;
    std::size_t bytes;
    std::size_t off;
    bool in;
  };
  std::vector<Part> parts_;
  std::size_t total_ = 0;
  void* base_ = nullptr;
};

inline bool valid_product(std::initializer_list<long long> dims) {
  long long product = 1;
  for (long long d : dims) {
    if (d <= 0 || product > LLONG_MAX / d) return false;
    product *= d;
  }
  return true;
}

}  // namespace detail

// qgemv (include/quixicore_cpu/qgemv.h:108) for q8_0 / q4_0 with host buffers.
inline int qgemv(int format, const void* packed, const float* x, float* y, long long n,
                 long long k) {
  std::size_t bytes = 0;
  int st = qc_hip_qgemv_packed_size(format, n, k, &bytes);   // format, then shape
  if (st != QC_OK) return st;
  if (packed == nullptr || x == nullptr || y == nullptr) return QC_INVALID_ARGUMENT;
  detail::Staging s;
  const std::size_t w = s.add(packed, bytes, true);
  const std::size_t xi = s.add(x, sizeof(float) * k, true);
  const std::size_t yo = s.add(y, sizeof(float) * n, false);
  if ((st = s.upload()) != QC_OK) return st;
  st = qc_hip_qgemv(format, s.device<void>(w), s.device<float>(xi), s.device<float>(yo), n, k,
                    nullptr);
  if (st == QC_OK) st = s.download(yo, y);   // hipMemcpy waits for the null stream
  return st;
}

// qgemm (include/quixicore_cpu/qgemm.h:19): m activation rows, host buffers.
// The reference's order (kernels/quantization/qgemm_ref.cpp:143-154): shape,
// nulls, then format.
inline int qgemm(int format, const void* packed, const float* x, float* y, long long m,
                 long long n, long long k) {
  if (!detail::valid_product({m, k}) || !detail::valid_product({m, n})) return QC_INVALID_SHAPE;
  if (packed == nullptr || x == nullptr || y == nullptr) return QC_INVALID_ARGUMENT;
  std::size_t bytes = 0;
  int st = qc_hip_qgemv_packed_size(format, n, k, &bytes);
  if (st != QC_OK) return st;
  detail::Staging s;
  const std::size_t w = s.add(packed, bytes, true);
  const std::size_t xi = s.add(x, sizeof(float) * m * k, true);
  const std::size_t yo = s.add(y, sizeof(float) * m * n, false);
  if ((st = s.upload()) != QC_OK) return st;
  st = qc_hip_qgemm(format, s.device<void>(w), s.device<float>(xi), s.device<float>(yo), m, n, k,
                    nullptr);
  if (st == QC_OK) st = s.download(yo, y);
  return st;
}

// quantize_int8 (include/quixicore_cpu/quantization.h:42), host buffers.  The
// C ABI rejects a non-finite x with 3 before writing anything.
inline int quantize_int8(const float* x, std::int8_t* codes, float* scales, long long rows,
                         long long dim, long long group_size) {
  const long long g = group_size == 0 ? dim : group_size;
  if (!detail::valid_product({rows, dim}) || g <= 0 || dim % g != 0) return QC_INVALID_SHAPE;
  if (x == nullptr || codes == nullptr || scales == nullptr) return QC_INVALID_ARGUMENT;
  detail::Staging s;
  const std::size_t xi = s.add(x, sizeof(float) * rows * dim, true);
  const std::size_t co = s.add(codes, static_cast<std::size_t>(rows * dim), false);
  const std::size_t so = s.add(scales, sizeof(float) * rows * (dim / g), false);
  int st = s.upload();
  if (st != QC_OK) return st;
  st = qc_hip_quantize_int8(s.device<float>(xi), s.device<std::int8_t>(co), s.device<float>(so),
                            rows, dim, group_size, nullptr, nullptr);
  if (st == QC_OK) st = s.download(co, codes);
  if (st == QC_OK) st = s.download(so, scales);
  return st;
}

// int8_gemm (include/quixicore_cpu/qgemm.h:235), host buffers; row_sum and zp
// only when asymmetric.  The C ABI rejects non-finite scales with 3 before
// writing y.
inline int int8_gemm(const std::int8_t* w, const std::int8_t* x, const float* ws,
                     const float* as, const std::int32_t* row_sum, const int* zp, float* y,
                     long long m, long long n, long long k, bool asymmetric) {
  if (!detail::valid_product({m, n, k})) return QC_INVALID_SHAPE;
  if (w == nullptr || x == nullptr || ws == nullptr || as == nullptr || y == nullptr ||
      (asymmetric && (row_sum == nullptr || zp == nullptr)))
    return QC_INVALID_ARGUMENT;
  detail::Staging s;
  const std::size_t wi = s.add(w, static_cast<std::size_t>(n * k), true);
  const std::size_t xi = s.add(x, static_cast<std::size_t>(m * k), true);
  const std::size_t wsi = s.add(ws, sizeof(float) * n, true);
  const std::size_t asi = s.add(as, sizeof(float) * m, true);
  const std::size_t rsi = s.add(row_sum, asymmetric ? sizeof(std::int32_t) * n : 0, true);
  const std::size_t zpi = s.add(zp, asymmetric ? sizeof(int) * m : 0, true);
  const std::size_t yo = s.add(y, sizeof(float) * m * n, false);
  int st = s.upload();
  if (st != QC_OK) return st;
  st = qc_hip_int8_gemm(s.device<std::int8_t>(wi), s.device<std::int8_t>(xi),
                        s.device<float>(wsi), s.device<float>(asi),
                        s.device<std::int32_t>(rsi), s.device<int>(zpi), s.device<float>(yo),
                        m, n, k, asymmetric ? 1 : 0, nullptr, nullptr);
  if (st == QC_OK) st = s.download(yo, y);
  return st;
}

}  // namespace quixicore_cpu::hip_gfx950

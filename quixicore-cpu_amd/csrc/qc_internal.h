// Launchers shared between the kernel translation units and the C-ABI layer.
// Host-side only; every pointer here is a device pointer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "quixicore_hip.h"

namespace qc {

// Compute units of the current device (the grid planners size by it).
int device_cu_count();

// Scratch of the allocating entry points: one cache entry per (device,
// stream).  A call takes its stream's entry, holds the entry's `call` lock
// from its first use of the buffers to its last launch (host threads sharing
// a stream then enqueue whole calls, and stream order keeps one call's
// kernels from reading another's scratch), and asks for buffer `tag` of at
// least `bytes`.  A buffer only grows.  The one it replaces is freed after
// the stream drains, unless it was handed out while the stream was being
// captured into a graph (the graph has its address baked in): such a buffer
// is retired and kept until the process ends.  Calls on different streams
// never share a buffer; graphs captured on one stream share its buffers and
// must not be replayed concurrently.  An entry point that holds `call` must
// not call another that takes it.
constexpr int kStreamBuffers = 2;
struct StreamWorkspace {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex call;
  void* ptr[kStreamBuffers] = {nullptr, nullptr};
  size_t bytes[kStreamBuffers] = {0, 0};
  bool captured[kStreamBuffers] = {false, false};
};
hipError_t stream_workspace(hipStream_t s, StreamWorkspace** out);
hipError_t stream_buffer(StreamWorkspace* w, hipStream_t s, size_t bytes, int tag, void** out);

struct GemvTuning {
  int rows_per_wave = 0;  // GEMV rows per wavefront (1, 2, 4, 7, 8, 14; 0 = from the shape)
  int qgemm_waves = 0;    // small-batch GEMM waves per workgroup (4, 8; 0 = from the shape)
  int qgemm_stages = 0;   // small-batch GEMM K stages per workgroup (1..16; 0 = from the shape)
  int qgemm_panel = 0;    // 2-D GEMM route: 0 = for m >= 64, -1 = never, 1 / 2 = always (K ranges)
  int qgemm_rows = 0;     // exact-digit rows route for 2 <= m <= 8: 0 = by shape, -1 = never, 1 = always
  int qgemm_fold = 0;     // digit-layout GEMM builds its own digits: 0 = where it can, -1 = never
  int cint8_dot = 0;      // canonical int8, M = 1: digit-dot kernel 0 = where it applies, -1 = never
};

// y[m][n] = dequant(W)[n][:] . x[m][:]  (W canonical q8_0/q4_0 blocks).
// noalloc: never allocate (the MFMA route takes launch_qgemm_mfma_noalloc).
hipError_t launch_qgemm(int fmt, const void* W, const float* x, float* y, long long m,
                        long long n, long long k, hipStream_t s, const GemvTuning& t,
                        bool noalloc = false);

// M = 1 GEMV with exact int8 digit dots (K % 64 == 0, W 4-byte aligned).
hipError_t launch_qgemv_dot(int fmt, const void* W, const float* x, float* y, int n, int k,
                            int rows_per_wave, hipStream_t s);

// y[m][n] for m rows of x (K % 64 == 0, W 4-byte aligned, x rows of k
// floats): passes of up to 8 activation rows over W, each output
// bit-identical to launch_qgemv_dot of its row.  rows_per_wave: 0, 1, 2 or 4.
hipError_t launch_qgemm_rows(int fmt, const void* W, const float* x, float* y, int n, int k,
                             int m, int rows_per_wave, hipStream_t s);

// Fused GEMVs over one x in a single launch (K % 64 == 0, every W 4-byte
// aligned, x 16-byte aligned): nseg matrices W[i] of rows[i] rows into y[i] (act = -1), or up
// (W[0]) and gate (W[1]) of rows[0] rows into y[0] = activation(gate) * up
// (act 0: SiLU, 1: GELU-tanh).  Same numerics as launch_qgemm with m = 1.
hipError_t launch_qgemv_multi(int fmt, int nseg, const void* const* W, float* const* y,
                              const int* rows, int act, const float* x, int k, hipStream_t s);

// Single-token Q/K/V projections with split-half RoPE on Q and K, one launch
// (same layout conditions as launch_qgemv_multi): q_rows = query_heads *
// 2 * half rows of Wq into q; kv_rows (0: Q only) rows of Wk / Wv into kc /
// vc.  rc / rs: the position's cos / sin rows (half values).
hipError_t launch_qgemv_qkv_rope(int fmt, const void* Wq, const void* Wk, const void* Wv,
                                 float* q, float* kc, float* vc, int q_rows, int kv_rows,
                                 int half, const float* rc, const float* rs, const float* x,
                                 int k, hipStream_t s);

// Rotates the (d, d + half) pairs of `heads` heads of 2 * half values in place.
hipError_t launch_rope_pairs(float* out, long long heads, int half, const float* rc,
                             const float* rs, hipStream_t s);

// out[i] = activation(out[i]) * up[i] over n elements (act 0: SiLU, 1: GELU-tanh).
hipError_t launch_fused_activation(float* out, const float* up, long long n, int act,
                                   hipStream_t s);

// qgemv_w8a8: x quantized per 32-element block to int8, exact integer block
// dots, y bit-identical to the reference.  status (optional): set to 3 when x
// holds a non-finite value (the affected outputs are NaN).
hipError_t launch_qgemv_w8a8(int fmt, const void* W, const float* x, float* y, long long n,
                             long long k, int rows_per_wave, int* status, hipStream_t s);

// GEMM on MFMA (m >= 2, K % 64 == 0, W 4-byte aligned): int8 digit planes
// for up to 8 rows per pass, bf16 hi/lo above; for m >= 64 one 2-D tiled
// kernel (the panel route) instead of passes of 32 rows.  waves / stages:
// small-batch plan override (0 = from the shape); panel: 0 = from m, -1 =
// never, 1 / 2 = always (one / two K ranges).  fold: 0 = the digit-layout
// GEMM builds its own digits where it can (no prep launch), -1 = never.
hipError_t launch_qgemm_mfma(int fmt, const void* W, const float* x, float* y, int m, int n,
                             int k, hipStream_t s, int waves = 0, int stages = 0,
                             int panel = 0, int fold = 0);

// launch_qgemm_mfma without allocating: the scratch is a fixed device
// array of kQgemmNoAllocScratchBytes per GPU, shared by every such call on
// that GPU (calls must not overlap).  Passes of at most 32 rows, the fewest
// K splits.  hipErrorOutOfMemory, before anything is launched, when the
// call's scratch exceeds the array.
constexpr size_t kQgemmNoAllocScratchBytes = QC_QGEMM_NOALLOC_SCRATCH_BYTES;
hipError_t launch_qgemm_mfma_noalloc(int fmt, const void* W, const float* x, float* y, int m,
                                     int n, int k, hipStream_t s);

// Projections over canonical int8 weights (see qc_hip_cint8_project), all
// checks done by the caller.  half / nrope: mode 2's RoPE half head size and
// the number of leading matrices rotated (1: Q, 2: Q and K).
struct CInt8Launch {
  int mode = 0;
  int nw = 1;
  qc_cint8_weights w[3] = {};
  const void* x = nullptr;
  int xtype = QC_STORAGE_F32;
  long long ldx = 0;            // elements between activation rows
  long long m = 1;
  void* y[3] = {nullptr, nullptr, nullptr};
  int ytype[3] = {0, 0, 0};
  const float* bias = nullptr;
  int act = 0;
  int half = 0;
  int nrope = 0;
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  int rows_per_wave = 0;        // 2, 4 or (M = 1 digit kernel) 8; 0: from the shape
  int dot = 0;                  // 0: row-plane route (M >= 2) / digit-dot kernels where they
                                // apply; 1: digit-dot kernels only; -1: the f32 kernel
};
hipError_t launch_cint8(const CInt8Launch& launch, hipStream_t s);

// out[r][c] = scales[si] * (float(codes[r][c]) - zeros[si]) (zeros may be
// NULL), si = r * groups + (group_index ? group_index[c] : c / group_size).
hipError_t launch_cint8_dequant(const int8_t* codes, const float* scales, const float* zeros,
                                const int* group_index, long long rows, long long cols,
                                long long groups, long long group_size, float* out,
                                hipStream_t s);

// y[m][n] = sum_c w(n, c) * a(m, c) over canonical int8 weights w and
// activations a (a.rows = m), both decoded as scale * (code - zero).  Symmetric
// row-scaled weights against row-scaled activations whose zero points are
// integers (given as a_int_zero_points, or none) run as the int8 MFMA GEMM
// (exact int32 dot, dot - z * row_sum in int64, then (float * ws[n]) * as[m]);
// anything else as f32 decode and FMA accumulation, one wave per output.
hipError_t launch_cint8_dual(const qc_cint8_weights& w, const qc_cint8_weights& a,
                             const int* a_int_zero_points, float* y, int int8_route,
                             hipStream_t s);

// out[i] = x[i] decoded from QC_STORAGE_F32 / F16 / BF16, exactly.
hipError_t launch_storage_to_f32(const void* x, int type, long long count, float* out,
                                 hipStream_t s);

// Per-group symmetric int8 quantization.  status == nullptr: caller has
// already verified that x is finite.  Otherwise non-finite groups are left
// unwritten and *status is set to 3 (kInvalidArgument).
hipError_t launch_quantize_int8(const float* x, int8_t* codes, float* scales, long long rows,
                                long long dim, long long group, int* status, hipStream_t s);

// Residual add + RMSNorm + per-group int8 quantization (group divides
// hidden).  Groups whose normalized values are not finite are left
// unwritten and set *status = 3 (status must not be null).
// force_sequential replays the element-order sum of squares for every row
// (it is otherwise replayed only for rows on a float rounding boundary).
hipError_t launch_rms_norm_add_quant_int8(const float* x, const float* residual,
                                          const float* weight, int8_t* codes,
                                          float* residual_out, float* scales, long long rows,
                                          long long hidden, float eps, long long group,
                                          bool force_sequential, int* status, hipStream_t s);

// Per-row asymmetric int8.  status == nullptr: caller has verified that x is
// finite; otherwise non-finite rows are left unwritten and set *status = 3.
hipError_t launch_quantize_int8_asymmetric(const float* x, int8_t* codes, float* scales,
                                           int* zero_points, long long rows, long long dim,
                                           int* status, hipStream_t s);
hipError_t launch_dequantize_int8_asymmetric(const int8_t* codes, const float* scales,
                                             const int* zero_points, float* out, long long rows,
                                             long long dim, hipStream_t s);

// Streaming read of `bytes` (multiple of 16) by `grid` workgroups of 256
// threads; out receives grid * 256 words (measurement seam).
hipError_t launch_stream_read(const void* p, long long bytes, uint32_t* out, int grid,
                              hipStream_t s);

// *flag = 1 if any of x[0..count) is NaN or +-inf (flag must start at 0).
hipError_t launch_nonfinite_scan(const float* x, long long count, int* flag, hipStream_t s);

// y[m][n] = (float(sum_k W[n][k] X[m][k] - zp[m]*row_sum[n]) * ws[n]) * as[m].
// acc_out (optional, test seam) receives the exact accumulators as int32
// instead of y when non-null.  status (optional): set to 3 when a scale is
// non-finite.
// route: 0 = from the shape; 1 = full-line ring (K % 32 == 0), 2 = 64-byte
// step direct-to-LDS (K % 64 == 0), 3 = register-staged (K % 16 == 0),
// 4 = one thread per output.  Routes 1-3 also need 16-byte aligned W and X;
// a route that cannot take the shape falls back to the default.
enum Int8Route { kInt8Auto = 0, kInt8Ring = 1, kInt8Dma = 2, kInt8Staged = 3, kInt8Simple = 4 };
hipError_t launch_int8_gemm(const int8_t* W, const int8_t* X, const float* ws, const float* as,
                            const int32_t* row_sum, const int* zp, float* y, int32_t* acc_out,
                            long long m, long long n, long long k, bool asymmetric,
                            int* status, hipStream_t s, int route = kInt8Auto);

// Weight packing / unpacking on the device (bit-exact with the reference
// packers).  status: set to 3 on a non-finite weight (block left unwritten).
hipError_t launch_pack(int fmt, const float* w, void* packed, long long n, long long k,
                       int* status, hipStream_t s);
hipError_t launch_unpack(int fmt, const void* packed, float* w, long long n, long long k,
                         hipStream_t s);

}  // namespace qc

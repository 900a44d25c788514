/*
 * quixicore_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul path.
 *
 * Drop-in for the reference QuixiAI/QuixiCore-CPU ops listed beside each
 * entry point (paths relative to the reference root).  Plain C: pointers,
 * sizes and an opaque stream; no C++ or torch types.
 *
 * Conventions
 *   - Return value: the reference Status integers
 *     (include/quixicore_cpu/status.h:5-11) -- 0 kOk, 1 kInvalidShape,
 *     2 kUnsupportedFormat, 3 kInvalidArgument, 4 kOutOfMemory -- plus
 *     5 (QC_DEVICE_ERROR) when the HIP runtime rejects a launch or copy; that
 *     value has no counterpart in the reference.  Host-visible validation
 *     runs first, in the reference's order, and nothing is launched on error.
 *   - Tensor pointers are device pointers (hipMalloc, or managed memory)
 *     unless stated otherwise.  `stream` is a hipStream_t or NULL for the null
 *     stream.  Calls are asynchronous on `stream` unless stated otherwise.
 *   - Data-dependent checks (non-finite values) cannot return synchronously
 *     from an asynchronous call.  Entry points that have them take
 *     `int* dev_status`: a device int the caller zeroes beforehand, which
 *     the kernels set to 3 (kInvalidArgument) on a non-finite input.  Passing
 *     dev_status == NULL selects the reference's synchronous semantics
 *     instead: the inputs are scanned first, the call blocks, returns 3 and
 *     writes no output if any value is non-finite.
 *   - Results are deterministic: rerunning a call gives bit-identical output.
 *   - Scratch: entry points whose kernels need device scratch (qc_hip_qgemm
 *     from M = 2, the canonical int8 projections from M = 2, the affine
 *     canonical W8A8 route) take it from a per-(device, stream) cache that
 *     only grows; the first call on a stream, or one needing more, allocates
 *     (hipMalloc), later calls do not.  Calls on one stream share its buffers
 *     in stream order; graphs captured on a stream keep that stream's buffers
 *     and must not be replayed concurrently with each other.
 */
#ifndef QUIXICORE_HIP_H
#define QUIXICORE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QC_OK 0
#define QC_INVALID_SHAPE 1
#define QC_UNSUPPORTED_FORMAT 2
#define QC_INVALID_ARGUMENT 3
#define QC_OUT_OF_MEMORY 4
#define QC_DEVICE_ERROR 5

/* QuantFormat numbering (include/quixicore_cpu/qgemv.h:10-13). Other
 * reference formats return QC_UNSUPPORTED_FORMAT. */
#define QC_Q8_0 0
#define QC_Q4_0 1

/* Library version string, and the text of the last HIP error seen by this
 * thread ("" if none). */
const char* qc_hip_version(void);
const char* qc_hip_last_error(void);

/* Packed byte count of an n x k matrix: n * (k/32) * {34, 18}.  Host only.
 * Replaces qgemv_packed_size (include/quixicore_cpu/qgemv.h:70;
 * src/dispatch/qgemv.cpp:199-209). */
int qc_hip_qgemv_packed_size(int format, long long n, long long k, size_t* size);

/* Quantize row-major f32 weights w[n][k] (device) into canonical GGUF blocks
 * (device), bit-identical to the reference packers.  Replaces qgemv_pack
 * (include/quixicore_cpu/qgemv.h:77; src/dispatch/qgemv.cpp:210-275;
 * kernels/quantization/qgemv_ref.cpp:14-41, qgemv_w8a8_ref.cpp:45-77).  As in
 * the reference, blocks may be partially written when 3 is reported. */
int qc_hip_qgemv_pack(int format, const float* w, long long n, long long k, void* packed,
                      int* dev_status, void* stream);

/* Dequantize blocks to f32 w[n][k].  Replaces qgemv_unpack
 * (include/quixicore_cpu/qgemv.h:89; src/dispatch/qgemv.cpp:277-297). */
int qc_hip_qgemv_unpack(int format, const void* packed, long long n, long long k, float* w,
                        void* stream);

/* y[n] = dequant(W) . x, f32 activations and accumulation.  Replaces qgemv
 * (include/quixicore_cpu/qgemv.h:108; src/dispatch/qgemv.cpp:337-365). */
int qc_hip_qgemv(int format, const void* packed, const float* x, float* y, long long n,
                 long long k, void* stream);

/* Y[m][n] = X[m][:] . dequant(W)[n][:].  Replaces qgemm
 * (include/quixicore_cpu/qgemm.h:19; kernels/quantization/qgemm_ref.cpp:141-164);
 * every row equals qc_hip_qgemv of that row within the contract tolerance. */
int qc_hip_qgemm(int format, const void* packed, const float* x, float* y, long long m,
                 long long n, long long k, void* stream);

/* qc_hip_qgemm for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops): no counterpart in the reference.
 * Same validation, kernels and numerics; the small-batch kernels' scratch
 * (activation fragments, partial sums, row exponents) lives in a fixed
 * device array of QC_QGEMM_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends, instead of memory the library allocates.  Every call on a
 * GPU shares that GPU's array.  A per-GPU host lock is held from a call's
 * first launch to its last, so calls from several host threads on ONE stream
 * are safe (their launch sequences queue one after the other); calls on
 * different streams of one GPU can overlap on the device and race: serialize
 * those.  M >= 2 runs passes of at
 * most 32 rows (never the 2-D M >= 64 route, whose scratch grows with m) with
 * the fewest K splits.  Limits: m <= QC_QGEMM_NOALLOC_MAX_M and
 * k <= QC_QGEMM_NOALLOC_MAX_K, else 1 (QC_INVALID_SHAPE) with a message in
 * qc_hip_last_error().  Within k <= 8192 every such call fits; above it, a
 * call whose K-split partial sums (ceil(k/4096) * min(m, 32) * n * 4 bytes)
 * do not fit beside the fragments is also rejected with 1, before anything
 * is launched. */
#define QC_QGEMM_NOALLOC_SCRATCH_BYTES (16ull << 20)
#define QC_QGEMM_NOALLOC_MAX_M 1048576LL
#define QC_QGEMM_NOALLOC_MAX_K 16384LL
int qc_hip_qgemm_noalloc(int format, const void* packed, const float* x, float* y, long long m,
                         long long n, long long k, void* stream);

/* Fused decode projections over one x, one launch where the shapes allow:
 * up = W_up . x and gate = W_gate . x ([n][k] each).  Same numerics as
 * qc_hip_qgemv per matrix.  Replaces qgemv_up_gate
 * (include/quixicore_cpu/qgemv.h:144; kernels/quantization/
 * qgemv_fused_ref.cpp:194-229).  Formats other than q8_0 / q4_0 return 2. */
int qc_hip_qgemv_up_gate(int format, const void* packed_up, const void* packed_gate,
                         const float* x, float* up, float* gate, long long n, long long k,
                         void* stream);

/* out = activation(W_gate . x) * (W_up . x), activation GELU-tanh
 * (gelu_tanh != 0) or SiLU; the two projections are never stored.  Replaces
 * qgemv_up_gate_activation (include/quixicore_cpu/qgemv.h:147;
 * kernels/quantization/qgemv_fused_ref.cpp:184-192,231-273). */
int qc_hip_qgemv_up_gate_activation(int format, const void* packed_up, const void* packed_gate,
                                    const float* x, float* out, long long n, long long k,
                                    int gelu_tanh, void* stream);

/* q = W_q . x ([query_dim][input_dim]), k_out = W_k . x and v_out = W_v . x
 * ([kv_dim][input_dim] each) in one launch.  Replaces qgemv_qkv
 * (include/quixicore_cpu/qgemv.h:151; kernels/quantization/
 * qgemv_fused_ref.cpp:275-327). */
int qc_hip_qgemv_qkv(int format, const void* packed_q, const void* packed_k,
                     const void* packed_v, const float* x, float* q, float* k_out,
                     float* v_out, long long query_dim, long long kv_dim, long long input_dim,
                     void* stream);

/* One decode token's Q/K/V projections with split-half (GPT-NeoX) RoPE and
 * direct KV-cache insertion, one launch where the shapes allow.  Q is
 * [query_heads * head_dim][input_dim], K and V [kv_heads * head_dim]
 * [input_dim].  For each head and d < head_dim / 2, with a = row d and
 * b = row d + head_dim / 2 of that head's projection, c = cosine[position *
 * head_dim / 2 + d] and s = sine[...]: out[d] = a * c - b * s and
 * out[d + head_dim / 2] = b * c + a * s.  q receives rotated Q; the rotated K
 * and plain V go to key_cache / value_cache rows [slot * kv_heads *
 * head_dim, (slot + 1) * kv_heads * head_dim) (caches are [slots][kv_heads]
 * [head_dim]); slot == -1 skips K and V.  Projections have qc_hip_qgemv's
 * numerics.  Replaces qgemv_qkv_rope_kv (include/quixicore_cpu/qgemv.h:
 * 157-163; kernels/quantization/qgemv_fused_ref.cpp:342-443). */
int qc_hip_qgemv_qkv_rope_kv(int format, const void* packed_q, const void* packed_k,
                             const void* packed_v, const float* x, const float* cosine,
                             const float* sine, float* q, float* key_cache, float* value_cache,
                             long long query_heads, long long kv_heads, long long head_dim,
                             long long input_dim, long long slots, long long max_position,
                             int position, int slot, void* stream);

/* ---- Canonical int8 projections (the prepared storage seams) ----------
 * Weights in the reference's canonical kInt8Symmetric / kInt8Affine layout
 * (include/quixicore_cpu/quant_contract.h): int8 codes [rows][cols]
 * row-major, f32 scales [rows][groups] (groups = 1: one per row), and for
 * kInt8Affine f32 zero points of the same shape.  Element (n, c) is
 * scale * (code - zero) of group c / (cols / groups)
 * (kernels/quantization/qgemm_canonical.cpp:125-176). */
typedef struct qc_cint8_weights {
  const int8_t* codes;
  const float* scales;
  const float* zero_points;   /* NULL: symmetric */
  long long rows;
  long long cols;
  long long groups;
} qc_cint8_weights;

/* Float storage of activations and outputs (FloatStorageType order of
 * include/quixicore_cpu/float_storage.h:18): raw IEEE binary32 / binary16 /
 * bfloat16; 16-bit values are decoded exactly, accumulation is f32 and each
 * output is rounded once (bf16: nearest even, NaN kept). */
#define QC_STORAGE_F32 0
#define QC_STORAGE_F16 1
#define QC_STORAGE_BF16 2

/* y = x . dequant(W)^T for m activation rows x [m][cols] (x_type) over up to
 * three matrices sharing x, with the reference's prepared-projection
 * epilogues fused:
 *   mode 0: nw = 1..3 projections, y[i] = [m][w[i].rows] of y_type[i]; with
 *           nw = 1, bias (f32 [rows] or NULL) is added and `activation`
 *           applied (LinearActivation order: 0 none, 1 GELU-erf, 2 GELU-tanh,
 *           3 SiLU, 4 ReLU^2; qgemm_canonical.cpp:361-379,2570-2581).
 *   mode 1: nw = 2 (gate, up, same shape): y[0] = SiLU(gate) * up
 *           (qgemm_canonical.cpp:2550-2560); neither projection is stored.
 *   mode 2: m = 1, nw = 1 (Q) or 3 (Q, K, V), rows multiples of head_dim
 *           (even): the (d, d + head_dim/2) pairs of every Q (and K) head are
 *           stored rotated, out[d] = a*c - b*s, out[d + half] = b*c + a*s with
 *           c = rope_cos[d], s = rope_sin[d] (the position's row); y[0] = Q,
 *           y[1] / y[2] = the cache slot's K / V rows (qgemm_canonical.cpp:
 *           5032-5225).
 * The matrices must share cols and groups, and all or none have zero
 * points.  Status: 1 shapes, 2 unknown storage type, 3 NULL pointers or a
 * bad mode / activation. */
int qc_hip_cint8_project(int mode, const qc_cint8_weights* w, int nw, const void* x, int x_type,
                         long long m, void* const* y, const int* y_type, const float* bias,
                         int activation, const float* rope_cos, const float* rope_sin,
                         long long head_dim, void* stream);

/* y[m][n] = sum_c w(n, c) * a(m, c) for canonical int8 weights w ([n][cols])
 * and canonical int8 activations a (a->rows = m, a->cols = w->cols), both
 * decoded as scale * (code - zero): the int8 x int8 case of
 * qgemm_prepacked_quantized / qgemv_prepacked_quantized
 * (include/quixicore_cpu/qgemm.h:118-127; kernels/quantization/
 * qgemm_canonical.cpp:5415-5507).  Symmetric weights with one scale per row,
 * against activations with one scale per row and either no zero points or
 * integer ones also passed as a_int_zero_points (int [m]), run as the int8
 * MFMA GEMM: exact int32 dot, minus z * sum_c code_w(n, c) in int64, then
 * (float * scale_w[n]) * scale_a[m].  Any other combination (group scales,
 * affine weights, fractional activation zero points) is decoded in f32 and
 * accumulated by FMA, one wave per output.  Status: 1 shapes (non-positive
 * dims, groups not dividing cols, a->cols != w->cols), 3 NULL pointers. */
int qc_hip_cint8_quantized_gemm(const qc_cint8_weights* w, const qc_cint8_weights* a,
                                const int* a_int_zero_points, float* y, void* stream);

/* Decode of canonical int8 weights to f32 [rows][cols]:
 * out[r][c] = scale(r, g) * (float(code[r][c]) - zero(r, g)), each step
 * rounded in f32 (zero = 0 when w->zero_points is NULL), with
 * g = group_index[c] when group_index is not NULL (a column -> group table of
 * w->groups groups per row), else c / (cols / groups).  The int8 branch of
 * dequantize_canonical (include/quixicore_cpu/quant_import.h:53-54;
 * kernels/quantization/quant_import_ref.cpp:753-770).  Status: 1 when rows,
 * cols or groups is not positive or, without a group index, groups does not
 * divide cols; 3 for NULL codes, scales or out. */
int qc_hip_cint8_dequantize(const qc_cint8_weights* w, const int* group_index, float* out,
                            void* stream);

/* out[i] = x[i] for i < count, decoded exactly from QC_STORAGE_F32 / F16 /
 * BF16 (float_storage_to_f32, kernels/utils/float_storage_ref.cpp): the
 * staging step of quantize_canonical's FloatStorageInput
 * (kernels/quantization/quant_import_ref.cpp:154-172).  Status: 1 for
 * count <= 0, 2 for an unknown type, 3 for NULL pointers. */
int qc_hip_storage_to_f32(const void* x, int type, long long count, float* out, void* stream);

/* Activation-quantizing GEMV: x is quantized per 32-element block to int8
 * (scale = max|x_b| / 127, round half to even, clamp +-127), each block dot is
 * an exact integer sum, and y[r] = sum_b (float(dot) * d_w) * d_x in block
 * order -- bit-identical to the reference.  Replaces qgemv_w8a8
 * (include/quixicore_cpu/qgemv_w8a8.h:16; src/dispatch/qgemv_w8a8.cpp:130-153;
 * kernels/quantization/qgemv_w8a8_ref.cpp:18-41,120-177).  dev_status NULL:
 * a non-finite x returns 3 before any work (the call blocks).  Otherwise the
 * call is asynchronous, *dev_status is set to 3 and the affected outputs are
 * NaN. */
int qc_hip_qgemv_w8a8(int format, const void* packed, const float* x, float* y, long long n,
                      long long k, int* dev_status, void* stream);

/* Packed weight bytes for qgemv_w8a8 (the qgemv q8_0 / q4_0 layouts).
 * Replaces qgemv_w8a8_packed_size (include/quixicore_cpu/qgemv_w8a8.h:23;
 * src/dispatch/qgemv_w8a8.cpp:108-125). */
int qc_hip_qgemv_w8a8_packed_size(int format, long long n, long long k, long long* bytes);

/* Name of the route qgemv_w8a8 takes for a format.  Replaces
 * qgemv_w8a8_variant (include/quixicore_cpu/qgemv_w8a8.h:29). */
const char* qc_hip_qgemv_w8a8_variant(int format);

/* Per-group symmetric int8 quantization; group_size 0 means one group per
 * row.  Bit-identical codes and scales.  Replaces quantize_int8
 * (include/quixicore_cpu/quantization.h:42;
 * kernels/quantization/quantization_ref.cpp:143-168).  With dev_status set,
 * groups holding a non-finite value are left unwritten. */
int qc_hip_quantize_int8(const float* x, int8_t* codes, float* scales, long long rows,
                         long long dim, long long group_size, int* dev_status, void* stream);

/* residual_out = x + residual; codes / scales = per-group int8 quantization of
 * RMSNorm(residual_out) * weight (group_size 0: one group per row; scales is
 * [rows][hidden / group_size]).  Bit-identical to the reference.  Replaces
 * rms_norm_add_quant_int8 (include/quixicore_cpu/quantization.h:112-116;
 * kernels/norms/norm_quant_ref.cpp:1060-1068).  A group whose normalized
 * values are not finite keeps its scale and codes unwritten: with dev_status
 * NULL the call blocks and returns 3, with a device int it stays asynchronous
 * and sets it to 3.  residual_out may be the same array as x or residual. */
int qc_hip_rms_norm_add_quant_int8(const float* x, const float* residual, const float* weight,
                                   int8_t* codes, float* residual_out, float* scales,
                                   long long rows, long long hidden, float eps,
                                   long long group_size, int* dev_status, void* stream);

/* Per-row asymmetric int8: scale = (max - min) / 255 (or max(|min| / 127,
 * 1e-7) for a constant row), zero = rint(-128 - min / scale), code =
 * clamp(rint(x / scale) + zero, -128, 127), all in double as the reference.
 * Bit-identical.  Replaces quantize_int8_asymmetric
 * (include/quixicore_cpu/quantization.h:49-51;
 * kernels/quantization/quantization_ref.cpp:190-226).  dev_status as for
 * qc_hip_quantize_int8 (non-finite rows left unwritten). */
int qc_hip_quantize_int8_asymmetric(const float* x, int8_t* codes, float* scales,
                                    int* zero_points, long long rows, long long dim,
                                    int* dev_status, void* stream);

/* out = scale[row] * float(code - zero_point[row]).  Replaces
 * dequantize_int8_asymmetric (include/quixicore_cpu/quantization.h:52-54;
 * kernels/quantization/quantization_ref.cpp:228-244). */
int qc_hip_dequantize_int8_asymmetric(const int8_t* codes, const float* scales,
                                      const int* zero_points, float* out, long long rows,
                                      long long dim, void* stream);

/* y[m][n] = (float(sum_k W[n][k]*X[m][k] - zp[m]*row_sum[n]) * ws[n]) * as[m]
 * (the zp term only when asymmetric != 0).  Exact integer accumulation.
 * Replaces int8_gemm (include/quixicore_cpu/qgemm.h:235;
 * src/dispatch/int8_gemm.cpp:67-94).  With dev_status set, outputs are
 * written and 3 is reported when any scale is non-finite. */
int qc_hip_int8_gemm(const int8_t* w, const int8_t* x, const float* ws, const float* as,
                     const int32_t* row_sum, const int* zp, float* y, long long m, long long n,
                     long long k, int asymmetric, int* dev_status, void* stream);

/* Symmetric alias.  Replaces qgemm_w8a8 (include/quixicore_cpu/qgemm.h:250;
 * kernels/quantization/qgemm_extended_ref.cpp:142-147). */
int qc_hip_qgemm_w8a8(const int8_t* w, const int8_t* x, const float* ws, const float* as,
                      float* y, long long m, long long n, long long k, int* dev_status,
                      void* stream);

/* Measurement seam with no reference counterpart: reads `bytes` (a multiple
 * of 16) of device memory with 16-byte loads as fast as the chip allows and
 * stores one XOR word per thread into out (grid * 256 words).  bench.py times
 * it at the GEMV's footprint to give the streaming ceiling that the GEMV's
 * HBM efficiency is judged against. */
int qc_hip_stream_read(const void* p, long long bytes, uint32_t* out, int grid, void* stream);

/* Test seam: the exact int32 accumulators sum_k W[n][k]*X[m][k] into
 * acc[m][n] (k <= 131071).  No reference counterpart (the reference's
 * accumulators are internal to kernels/quantization/int8_gemm_*.cpp). */
int qc_hip_int8_gemm_i32(const int8_t* w, const int8_t* x, int32_t* acc, long long m,
                         long long n, long long k, void* stream);

/* Sets *dev_flag = 1 (device int, zeroed by the caller) if any of x[0..count)
 * is NaN or infinite.  The device form of all_finite
 * (kernels/quantization/quantization_ref.cpp:70-75). */
int qc_hip_nonfinite_scan(const float* x, long long count, int* dev_flag, void* stream);

/* Names of the routes the dispatch resolves to, like qgemv_variant
 * (include/quixicore_cpu/qgemv.h:166) and int8_gemm_variant
 * (include/quixicore_cpu/qgemm.h:240). */
const char* qc_hip_qgemv_variant(int format);
const char* qc_hip_int8_gemm_variant(void);

/* Rows each GEMV wavefront keeps in flight: 1, 2, 4, 7, 8 or 14 (capped by
 * the register budget for K), or 0 (default) to choose from the shape.
 * Tuning knob with no reference counterpart. */
int qc_hip_set_gemv_rows_per_wave(int rows);

/* Kernel route of the int8 GEMM entry points (process-wide): 0 (default)
 * chooses from the shape; 1 = full-line LDS ring (K % 32 == 0),
 * 2 = 64-byte-step direct-to-LDS pipeline (K % 64 == 0), 3 = register-staged
 * double buffer, 4 = one thread per output.  A route that cannot take a
 * shape or alignment falls back to the default.  Every route returns the
 * same bits.  Tuning and test knob with no reference counterpart. */
int qc_hip_set_int8_gemm_route(int route);

/* Work split of the small-batch GEMM (qc_hip_qgemm with M >= 2, K % 64 == 0;
 * process-wide): waves per workgroup (4 or 8) and 256-element K stages per
 * workgroup (1, 2, 4, 8 or 16; K is split into ceil(K / 256 / stages)
 * ranges); 0 leaves a field to the shape-based planner.  Results stay within
 * the contract tolerance for every split, and reruns with one split are
 * bit-identical.  Tuning and test knob with no reference counterpart. */
int qc_hip_set_qgemm_plan(int waves, int stages);

/* Route of qc_hip_qgemm for M >= 2 (K % 64 == 0): 0 (the default) runs the
 * 2-D tiled GEMM for M >= 64 and passes of at most 32 rows below; -1 always
 * uses the passes; 1 / 2 always use the 2-D GEMM with one / two K ranges.
 * Results stay within the contract tolerance on every route.  Tuning and
 * test knob with no reference counterpart. */
int qc_hip_set_qgemm_panel(int mode);

/* qgemm route for 2 <= m <= 8: 0 (default) = by shape (the exact-digit rows
 * kernel -- one pass over W for all rows, every row bit-identical to
 * qc_hip_qgemv of that row -- for m = 2 and K <= 4096, and for m <= 4 with
 * also N <= 8192; the MFMA small-batch kernels otherwise), -1 = never,
 * 1 = always.  Tuning and test knob with no reference counterpart. */
int qc_hip_set_qgemm_rows(int mode);

/* Canonical int8 projections (qc_hip_cint8_project): 0 (default) = two or
 * more activation rows with one scale per weight row, or three or more with
 * scale groups of 64 or a multiple of 128 columns (five or more with groups
 * of 32; K % 128 == 0 with groups), run on the row-plane route
 * (three int8 digit planes of each activation row under one row exponent,
 * the int8 MFMA GEMM, an exact combination per row or per group; K % 32 == 0,
 * K <= 16384, codes 16-byte aligned, not the RoPE mode), everything else on
 * the kernels with exact int8 digit dots per 32-element block (the GEMV's
 * encoding of x) where they apply (K % 64 == 0, codes 16-byte aligned, row
 * scales or groups of >= 32 columns); 1 = never the row-plane route; -1 =
 * always the f32 multiply-add kernel.  All stay within the contract
 * tolerance.  Tuning and test knob with no reference counterpart. */
int qc_hip_set_cint8_dot(int mode);

/* Small-batch MFMA kernels with int8 digit activations (2 <= m <= 8 per
 * pass): 0 (default) = the GEMM kernel builds each stage's digits from x
 * itself where it can (K % 256 == 0, x 16-byte aligned, K not split in two),
 * saving the separate digit-prep launch; -1 = always run the prep launch.
 * Both give the same bits.  Tuning and test knob with no reference
 * counterpart. */
int qc_hip_set_qgemm_fold(int mode);

/* on != 0: qc_hip_rms_norm_add_quant_int8 replays the element-order sum of
 * squares for every row instead of only for rows whose float norm the
 * parallel sum cannot settle (process-wide; results are identical either
 * way).  Test knob with no reference counterpart. */
int qc_hip_set_norm_sequential_sum(int on);

#ifdef __cplusplus
}
#endif

#endif /* QUIXICORE_HIP_H */

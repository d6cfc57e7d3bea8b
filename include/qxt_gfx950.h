/*
 * qxt_gfx950.h -- C ABI of the MI355X (gfx950) quantized-linear library.
 *
 * Every entry point takes device pointers, byte row strides, sizes and a HIP
 * stream (passed as `void *`; NULL is the default stream).  Work is enqueued
 * in stream order; no entry point synchronises unless its name says so.
 * Arguments are validated before anything is enqueued, so on any non-OK
 * status no output byte has been written.  Functions return `int` holding a
 * `qxt_status`.
 *
 * Reference interfaces each entry point replaces are cited as
 * `path:line` in the yiannisha/qpu-xla-triton source tree.
 */
#ifndef QXT_GFX950_H
#define QXT_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QXT_ABI_VERSION 2

/* Status values equal qpu_llama_status
 * (integrations/llama_cpp/include/qpu_llama_runtime.h:16-27). */
typedef enum qxt_status {
    QXT_OK = 0,
    QXT_INVALID_ARGUMENT = 1,
    QXT_DEVICE_UNAVAILABLE = 2,
    QXT_CAPABILITY_MISSING = 3,
    QXT_ALLOCATION_FAILED = 4,
    QXT_IO_FAILED = 5,
    QXT_SUBMISSION_FAILED = 6,
    QXT_TIMEOUT = 7,
    QXT_HASH_MISMATCH = 8,
    QXT_INTERNAL_ERROR = 9,
} qxt_status;

/* Failure-injection points, bit values as qpu_llama_failure_point
 * (qpu_llama_runtime.h:29-36).  A set bit makes the next matching step fail
 * before it touches the GPU: SUBMISSION -> QXT_SUBMISSION_FAILED from every
 * launching entry point, WAIT -> QXT_TIMEOUT from qxt_stream_wait,
 * ALLOCATION -> QXT_ALLOCATION_FAILED from allocating entry points. */
typedef enum qxt_failure_point {
    QXT_FAIL_NONE = 0,
    QXT_FAIL_DEVICE_OPEN = 1u << 0,
    QXT_FAIL_ALLOCATION = 1u << 1,
    QXT_FAIL_SUBMISSION = 1u << 2,
    QXT_FAIL_WAIT = 1u << 3,
} qxt_failure_point;

/* Flags of qxt_quantize_rows_int8 / qxt_w8a8_linear. */
#define QXT_QUANT_NO_SCALE_FLOOR 1u /* drop the 1/127 scale floor: NOT the reference contract */

/* Right-operand layouts of the W8A8 GEMM entry points. */
#define QXT_W8A8_WEIGHT_NK 0u  /* int8 [N, K] row-major (QuantizedMatrixInt8.values layout) */
#define QXT_W8A8_WEIGHT_K4N 1u /* uint32 [K/4, N]: pack_int8_quads(W).T (gemm_int8.py:32-40) */

typedef struct qxt_device_info {
    char arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t compute_units;  /* multiProcessorCount */
    int32_t clock_khz;      /* peak engine clock */
    int32_t memory_clock_khz;
    int32_t memory_bus_width;
    int64_t total_memory;   /* bytes of HBM */
    int32_t l2_bytes;
    int32_t lds_bytes_per_cu;
} qxt_device_info;

/* ---------------------------------------------------------------- runtime */

/* Library ABI version (QXT_ABI_VERSION). No reference counterpart. */
int qxt_abi_version(void);

/* Text of a status; replaces qpu_llama_status_string (qpu_llama_runtime.h:133). */
const char *qxt_status_string(int status);

/* Last error text of the calling thread; replaces qpu_llama_context_last_error
 * (qpu_llama_runtime.h:89). */
const char *qxt_last_error(void);

/* Process-wide failure-injection mask; replaces
 * qpu_llama_context_set_failure_mask (qpu_llama_runtime.h:93). */
void qxt_set_failure_mask(uint32_t mask);
uint32_t qxt_get_failure_mask(void);

/* Number of device and pinned-host allocations the library has made in this
 * process (hipMalloc / hipHostMalloc through its own code, successful calls
 * only).  No counterpart in the reference: it lets a caller check that an
 * entry point allocates nothing (qxt_w8a8_linear_noalloc). */
uint64_t qxt_allocation_count(void);

/* Properties of the current HIP device; replaces qpu_llama_context_capabilities
 * (qpu_llama_runtime.h:90-92). */
int qxt_device_query(qxt_device_info *out);

/* Wait for all work on `stream`; replaces qpu_llama_submission_wait
 * (qpu_llama_runtime.h:130) / qpu_llama_q4_0_submission_wait
 * (qpu_llama_q4_0.h:76-78).  Returns QXT_TIMEOUT under QXT_FAIL_WAIT. */
int qxt_stream_wait(void *stream);

/* One timed kernel launch (see qxt_timing_begin). */
typedef struct qxt_launch_record {
    char kernel[48]; /* kernel name, e.g. "q4_0_linear_kernel" */
    float ms;        /* device time between the kernel's start and end */
} qxt_launch_record;

/* Per-launch device timing for profiling: after qxt_timing_begin, every kernel
 * this thread launches records start/stop events (hipExtLaunchKernel); not for
 * use under graph capture.  qxt_timing_end waits for those events, writes up to
 * `capacity` records in launch order, stores the total count and stops timing.
 * Replaces the qpu_llama_q4_0_timing struct (qpu_llama_q4_0.h:50-61) filled by
 * qpu_llama_q4_0_submission_wait (qpu_llama_q4_0.c:812-824). */
int qxt_timing_begin(void);
int qxt_timing_end(qxt_launch_record *records, uint32_t capacity, uint32_t *count);

/* Measurement utility with no reference counterpart, for benchmarks: reads
 * `bytes` (a positive multiple of 16) at `src` (16-byte aligned) once, with
 * the fastest plain streaming pattern this library found for the device (a
 * grid of 2048 workgroups of 256 threads, 16-byte non-temporal loads
 * grid-stride), and stores in partials[w] the xor of the 32-bit words that
 * workgroup w read; the xor of all 2048 partials is the xor of every word of
 * the buffer.  Its device time over a buffer far larger than the caches is
 * the device's achievable HBM read rate. */
int qxt_hbm_read_probe(const void *src, size_t bytes, uint32_t *partials, void *stream);

/* ------------------------------------------------------------- quantisers */

/* fp32 rows x[rows, columns] -> native Q8_0 blocks u8 [rows, columns/32, 34].
 * d = fl32(absmax/127), inv = 1/d (0 if d == 0), q = clip(rint(x*inv), +-127),
 * d stored fp16 RNE.  columns % 32 == 0.  Replaces the host quantiser
 * quantize_q8_0_split (examples/benchmark_llama_cpp_qpu_persistent_q4.py:42-53)
 * and the ggml call at integrations/llama_cpp/backend/ggml-qpu.cpp:552-558. */
int qxt_quantize_q8_0(const float *x, size_t x_row_stride, void *blocks, size_t blocks_row_stride,
                      uint32_t rows, uint32_t columns, void *stream);

/* Self-check with no reference counterpart, for test suites: compares the
 * Q8_0 block scale d and inverse inv that the Q8_0 quantisers compute without
 * division sequences against fl32(absmax/127) and fl32(1/d) from IEEE
 * division, for every non-negative fp32 absmax (all 2^31 bit patterns), and
 * adds the number of patterns that differ to *mismatches, a device uint64
 * the caller zeroes. */
int qxt_q8_0_scale_check(uint64_t *mismatches, void *stream);

/* fp32 rows x[rows, columns] -> int8 q[rows, padded_columns] plus fp32 scales[rows].
 * scale = max(fl32(absmax/127), fl32(1/127)), q = clip(rint(x/scale), +-127);
 * columns [columns, padded_columns) are written as 0.  Replaces the host
 * quantiser PreparedW8A8Linear._prepare_values
 * (src/qpu_xla/models/tinyllama/quantization.py:156-171); the same rule
 * quantises weights per output channel (quantization.py:1085-1092). */
int qxt_quantize_rows_int8(const float *x, size_t x_row_stride, int8_t *q, size_t q_row_stride,
                           float *scales, uint32_t rows, uint32_t columns, uint32_t padded_columns,
                           uint32_t flags, void *stream);

/* fp32 weights w[rows, columns] -> native Q4_0 blocks u8 [rows, columns/32, 18],
 * ggml reference rule (d = first-max/-8, q = min(15, trunc(x/d + 8.5))).
 * Replaces upstream quantize_row_q4_0 as called at
 * integrations/llama_cpp/tests/qpu_ggml_backend_smoke.cpp:119. */
int qxt_quantize_q4_0(const float *w, size_t w_row_stride, void *blocks, size_t blocks_row_stride,
                      uint32_t rows, uint32_t columns, void *stream);

/* ------------------------------------------------------ GEGLU -> Q8_0 producer */

/* Host-only: fill table[65536] with GGML's exact-GELU fp16 lookup table, entry
 * i = fp16(fl32(0.5 x (1 + erf(x / sqrt 2)))) for x = the fp16 value with bits
 * i, the GELU evaluated in double.  Replaces ggml_gelu_fp16_table
 * (src/qpu_xla/kernels/ggml_geglu_q8.py:26-34).  No device work. */
int qxt_ggml_gelu_fp16_table(uint16_t *table);

/* fp32 gate, up [rows, columns] -> native Q8_0 blocks u8 [rows, columns/32, 34] of
 * v = fl32(table[fp16(gate)] * up) (fp16 RNE of the gate indexes the device copy of
 * qxt_ggml_gelu_fp16_table), quantised as qxt_quantize_q8_0.  columns % 32 == 0.
 * Replaces GGML_GEGLU_Q8_0_KERNEL (src/qpu_xla/kernels/ggml_geglu_q8.py:262-308),
 * bit-identical to ggml_geglu_q8_0_reference (ggml_geglu_q8.py:37-59). */
int qxt_ggml_geglu_q8_0(const float *gate, size_t gate_row_stride, const float *up, size_t up_row_stride,
                        const uint16_t *gelu_table, void *blocks, size_t blocks_row_stride, uint32_t rows,
                        uint32_t columns, void *stream);

/* As qxt_ggml_geglu_q8_0, written as split planes for the tiled linear: int8
 * values[rows, columns] and fp16 scale bits scales[rows, columns/32] held in
 * scale_bytes = 2 (u16) or 4 (u32, zero-extended, the reference's layout) bytes.
 * Replaces GGML_GEGLU_Q8_0_SPLIT_KERNEL (ggml_geglu_q8.py:311-385). */
int qxt_ggml_geglu_q8_0_split(const float *gate, size_t gate_row_stride, const float *up, size_t up_row_stride,
                              const uint16_t *gelu_table, void *scales, size_t scales_row_stride,
                              uint32_t scale_bytes, int8_t *values, size_t values_row_stride, uint32_t rows,
                              uint32_t columns, void *stream);

/* -------------------------------------------------------- Q4_0 x Q8_0 linear */

/* destination[r, output_column_start + j] =
 *   sum_b fl32(fl32(float(dot_b) * dw[wc, b]) * da[r, b]), summed in block order,
 * wc = weight_column_start + j, for r < rows, j < column_count.
 * activation: Q8_0 u8 [rows, blocks, 34]; weight: Q4_0 u8 [>= wc+1, blocks, 18].
 * Writes only destination[:, output_column_start : +column_count].  rows >= 16 run on the
 * int8 matrix cores (one MFMA per 32 x 32 outputs and block); 4 to 15 rows with blocks / 8
 * dividing 16 (K <= 4096) on v_mfma_i32_4x4x4_16b_i8; other shapes on v_dot4.
 * Replaces GGML_Q4_0_Q8_0_LINEAR_KERNEL (src/qpu_xla/kernels/ggml_q4_0.py:783-841)
 * and the device work of qpu_llama_q4_0_linear_submit (qpu_llama_q4_0.h:72-75). */
int qxt_ggml_q4_0_q8_0_linear(const void *activation, size_t activation_row_stride,
                              const void *weight, size_t weight_row_stride,
                              float *destination, size_t destination_row_stride,
                              uint32_t rows, uint32_t blocks,
                              uint32_t weight_column_start, uint32_t output_column_start,
                              uint32_t column_count, void *stream);

/* Q4_0 weight layouts of the decode path (qxt_q4_0_task.weight_layout). */
#define QXT_Q4_0_LAYOUT_NATIVE 0u /* ggml rows: [columns, blocks, 18] */
#define QXT_Q4_0_LAYOUT_LANES 1u  /* qxt_q4_0_pack_lanes output */

/* Bytes of the lane layout of a [columns, blocks, 18] Q4_0 matrix (0 when
 * blocks % 8 != 0).  No reference counterpart. */
size_t qxt_q4_0_lanes_bytes(uint32_t columns, uint32_t blocks);

/* Repack native Q4_0 rows into the lane layout read by the decode kernels:
 * the matrix is cut into units of 8 consecutive blocks of one column (144
 * bytes, native order: unit u = column * blocks/8 + block/8), units into
 * groups of 64, and chunk v (bytes 16v .. 16v+15) of unit l of group q is
 * stored at q * 9216 + (v * 64 + l) * 16; units past the matrix are zero.
 * Same bytes, no scale or code changes: the weight-preparation step of the
 * reference's prepared linear (qpu_llama_q4_0.c:343-395, which also re-lays
 * weights out for its kernel).  blocks % 8 == 0; weight and packed 16-byte
 * aligned, weight_row_stride % 16 == 0; packed_bytes >= qxt_q4_0_lanes_bytes. */
int qxt_q4_0_pack_lanes(const void *weight, size_t weight_row_stride, void *packed, size_t packed_bytes,
                        uint32_t columns, uint32_t blocks, void *stream);

/* qxt_ggml_q4_0_q8_0_linear over a lane-layout weight of `weight_columns`
 * columns (weight_column_start + column_count <= weight_columns); same
 * result bit for bit.  Four or more rows with blocks / 8 dividing 16 (K <= 4096)
 * run on v_mfma_i32_4x4x4_16b_i8 (four rows x four columns per 4-lane block);
 * other shapes on v_dot4. */
int qxt_ggml_q4_0_q8_0_linear_lanes(const void *activation, size_t activation_row_stride,
                                    const void *packed_weight, uint32_t weight_columns,
                                    float *destination, size_t destination_row_stride,
                                    uint32_t rows, uint32_t blocks,
                                    uint32_t weight_column_start, uint32_t output_column_start,
                                    uint32_t column_count, void *stream);

/* Prefill Q4_0 x Q8_0 linear over the reference's split / tiled operand layout:
 *   activation_q      int8 [rows, blocks*32] (the Q8_0 values, row stride in bytes, % 4 == 0),
 *   activation_scales fp16 bits [rows, blocks], elements of activation_scale_bytes = 2 (uint16)
 *                     or 4 (uint32 words holding the fp16 bits),
 *   weight_q          uint32 [blocks*8, columns]: word (8b + g, n) = signed int8 values
 *                     k = 4g .. 4g+3 of block b of column n (pack_ggml_q4_0_tiled_weights),
 *   weight_scales     fp16 bits [blocks, columns] (uint16),
 *   destination       fp32 [rows, columns].
 * Result as qxt_ggml_q4_0_q8_0_linear (per-block exact int32 dots on the matrix cores, scaled
 * by dw then da and summed in block order: bit-identical to ggml_q4_0_q8_0_reference).  Any
 * rows / columns (the reference needs multiples of 16).  Replaces
 * GGML_Q4_0_Q8_0_TILED_LINEAR_KERNEL (src/qpu_xla/kernels/ggml_q4_0.py:886-967) and its
 * persistent variant (src/qpu_xla/kernels/ggml_q4_0_persistent.py:11), whose results are
 * identical to the conventional launch. */
int qxt_ggml_q4_0_q8_0_tiled_linear(const void *activation_q, size_t activation_q_row_stride,
                                    const void *activation_scales, size_t activation_scales_row_stride,
                                    uint32_t activation_scale_bytes, const void *weight_q,
                                    size_t weight_q_row_stride, const void *weight_scales,
                                    size_t weight_scales_row_stride, float *destination,
                                    size_t destination_row_stride, uint32_t rows, uint32_t blocks,
                                    uint32_t columns, void *stream);

/* Debug twin of the linear above: dots[r, j, b] = exact int32 block dot of
 * row r with weight column weight_column_start + j (dots row stride
 * column_count * blocks * 4 bytes).  Exposes the int32 terms of
 * ggml_q4_0_q8_0_reference (src/qpu_xla/kernels/ggml_q4_0.py:96). */
int qxt_ggml_q4_0_q8_0_block_dots(const void *activation, size_t activation_row_stride,
                                  const void *weight, size_t weight_row_stride,
                                  int32_t *dots, uint32_t rows, uint32_t blocks,
                                  uint32_t weight_column_start, uint32_t column_count,
                                  void *stream);

/* ------------------------------------------------------- Q8_0 x Q8_0 linear */

/* destination[r, output_column_start + j] =
 *   sum_b fl32(fl32(float(dot_b) * da[r, b]) * dw[wc, b]) in block order (activation scale
 * first, as ggml_q8_0_q8_0_reference, src/qpu_xla/kernels/ggml_q8_0.py:26-51),
 * wc = weight_column_start + j.  activation and weight: native Q8_0 u8 [*, blocks, 34].
 * Any rows (the reference kernel takes exactly 4) and any column range.  Replaces
 * GGML_Q8_0_Q8_0_LINEAR_M4_KERNEL (ggml_q8_0.py:233-291). */
int qxt_ggml_q8_0_q8_0_linear(const void *activation, size_t activation_row_stride,
                              const void *weight, size_t weight_row_stride,
                              float *destination, size_t destination_row_stride,
                              uint32_t rows, uint32_t blocks,
                              uint32_t weight_column_start, uint32_t output_column_start,
                              uint32_t column_count, void *stream);

/* One linear of a Q4_0 batch.  Exactly one of `x` (fp32 rows [rows, blocks*32]
 * with 16-byte aligned rows, quantised to Q8_0 by the rule of qxt_quantize_q8_0:
 * in a pre-pass launch of the batch when the batch has more than 1024 work
 * items, else by every workgroup that reads them) and `activation` (native
 * Q8_0 blocks) is non-NULL; the
 * other fields mean what they mean for qxt_ggml_q4_0_q8_0_linear.  Batched
 * tasks need rows <= 4, blocks % 8 == 0 and 16-byte aligned weight rows.
 * weight_layout QXT_Q4_0_LAYOUT_LANES: `weight` is the base of a
 * qxt_q4_0_pack_lanes matrix and weight_row_stride is ignored. */
typedef struct qxt_q4_0_task {
    const float *x;
    size_t x_row_stride;
    const void *activation;
    size_t activation_row_stride;
    const void *weight;
    size_t weight_row_stride;
    float *destination;
    size_t destination_row_stride;
    uint32_t rows;
    uint32_t blocks;
    uint32_t weight_column_start;
    uint32_t output_column_start;
    uint32_t column_count;
    uint32_t weight_layout; /* QXT_Q4_0_LAYOUT_* */
} qxt_q4_0_task;

typedef struct qxt_q4_0_batch qxt_q4_0_batch;

/* Prepare a batch of independent Q4_0 x Q8_0 linears that one kernel launch
 * computes (e.g. every projection of a decode step); uploads a small task
 * table and allocates the Q8_0 buffer of the tasks' fp32 activations with
 * hipMalloc/hipMemcpy (synchronous).  The tensors the tasks point
 * at must outlive the batch.  Replaces the prepared-linear handle
 * qpu_llama_q4_0_linear_prepare (integrations/llama_cpp/include/qpu_llama_q4_0.h:63-66). */
int qxt_q4_0_batch_prepare(const qxt_q4_0_task *tasks, uint32_t count, qxt_q4_0_batch **batch);

/* Enqueue the whole batch on `stream`: the Q8_0 pre-pass (when a task has fp32
 * rows and the batch has more than 1024 work items) and the batch grid;
 * graph-capturable.
 * Replaces qpu_llama_q4_0_linear_submit (qpu_llama_q4_0.h:72-75). */
int qxt_q4_0_batch_launch(const qxt_q4_0_batch *batch, void *stream);

/* Number of workgroups one launch of the batch runs. No reference counterpart. */
uint32_t qxt_q4_0_batch_work_items(const qxt_q4_0_batch *batch);

/* Free the task table; replaces qpu_llama_q4_0_linear_destroy (qpu_llama_q4_0.h:67). */
void qxt_q4_0_batch_destroy(qxt_q4_0_batch *batch);

/* ------------------------------------------------------------------- W8A8 */

/* acc[m, n] = sum_k a[m, k] * w(n, k), exact int32.  a: int8 [m, k] (row stride
 * lda bytes, == the packed-K4 left operand of gemm_int8.py:23-40); w per
 * weight_layout.  k % 16 == 0, k*127*127 <= INT32_MAX.
 * Replaces TILED_W8A8_GEMM_KERNEL (src/qpu_xla/kernels/gemm_int8.py:285-320)
 * and W8A8_GEMV_KERNEL (src/qpu_xla/kernels/gemv_int8.py:129-153). */
int qxt_w8a8_gemm_i32(const int8_t *a, size_t lda, const void *w, size_t ldw, int32_t *acc,
                      size_t ldacc, uint32_t m, uint32_t n, uint32_t k, uint32_t weight_layout,
                      void *stream);

/* y[m, n] = fl32(fl32(float(acc) * row_scales[m]) * column_scales[n]) (+ bias[n] as a
 * separate add when bias != NULL), acc as in qxt_w8a8_gemm_i32 but never stored.
 * Replaces TILED_W8A8_GEMM_DEQUANTIZE_KERNEL (gemm_int8.py:323-370) plus the
 * affine_fp32 bias pass (src/qpu_xla/ops/affine.py:18-54). */
int qxt_w8a8_gemm_dequantize(const int8_t *a, size_t lda, const void *w, size_t ldw,
                             const float *row_scales, const float *column_scales,
                             const float *bias, float *y, size_t ldy, uint32_t m, uint32_t n,
                             uint32_t k, uint32_t weight_layout, void *stream);

/* Standalone epilogue over stored int32 accumulators, same arithmetic as above.
 * Replaces W8A8_DEQUANTIZE_KERNEL (src/qpu_xla/kernels/w8a8_epilogue.py:143-174). */
int qxt_w8a8_dequantize(const int32_t *acc, size_t ldacc, const float *row_scales,
                        const float *column_scales, const float *bias, float *y, size_t ldy,
                        uint32_t m, uint32_t n, void *stream);

/* Whole dynamic-W8A8 linear: per-row quantise x (into the caller's workspaces
 * qa [m, k] int8 with row stride ldqa, sa [m] fp32), int8 GEMM, fused dequant
 * + bias.  flags: QXT_QUANT_NO_SCALE_FLOOR.  Replaces PreparedW8A8Linear.execute
 * (quantization.py:279-330) with the fused epilogue of
 * _StagedW8A8Linear (src/qpu_xla/models/smolvla/accelerated.py:248-262). */
int qxt_w8a8_linear(const float *x, size_t ldx, int8_t *qa, size_t ldqa, float *sa,
                    const void *w, size_t ldw, const float *column_scales, const float *bias,
                    float *y, size_t ldy, uint32_t m, uint32_t n, uint32_t k,
                    uint32_t weight_layout, uint32_t flags, void *stream);

/* qxt_w8a8_linear without workspace arguments and without any allocation:
 * the quantised activation rows and row scales live in a static device array
 * of the library (64 MiB of int8 rows + 256 KiB of scales per GPU, held from
 * the library's first use on that GPU until the process ends).  Limits: m <=
 * 65,536 and m * k <= 64 MiB (2^26), else QXT_INVALID_ARGUMENT before anything
 * is enqueued.  Same result as qxt_w8a8_linear bit for bit.  Every call on one
 * GPU shares that GPU's array, so calls that overlap on one GPU (other streams,
 * other threads) race; order them on one stream.  No counterpart in the
 * reference: for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). */
int qxt_w8a8_linear_noalloc(const float *x, size_t ldx, const void *w, size_t ldw, const float *column_scales,
                            const float *bias, float *y, size_t ldy, uint32_t m, uint32_t n, uint32_t k,
                            uint32_t weight_layout, uint32_t flags, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* QXT_GFX950_H */

/*
 * qxt_llama_q4_0.h -- llama.cpp-facing prepared Q4_0 x Q8_0 linear on gfx950.
 *
 * Twin of the reference's native bridge
 * (integrations/llama_cpp/include/qpu_llama_q4_0.h:13-82 and the context part
 * of qpu_llama_runtime.h:16-133): same handles, descriptor fields, status
 * values, failure points and host-buffer semantics, so a ggml backend or the
 * CPU_REPACK M=1 hook swaps `qpu_llama_` for `qxt_llama_` and keeps its code.
 *
 * Semantics kept from the reference:
 *  - weights, activation and destination are HOST buffers; prepare uploads the
 *    resident column range once, submit copies the Q8_0 rows in, wait copies
 *    the selected output columns out;
 *  - validation happens before any work: a non-OK status writes no output
 *    byte, and a failed or timed-out wait leaves the destination untouched;
 *  - one in-flight submission per linear (busy -> QXT_INTERNAL_ERROR) and one
 *    per context; a wait failure or timeout poisons the context (later
 *    submissions return QXT_IO_FAILED), as the reference runtime does;
 *  - rows = 0 in an execution means the prepared row capacity.
 *
 * Differences (by design):
 *  - every row count up to the prepared capacity runs as is (M=1 is not
 *    replicated to 4 rows); rows >= 16 run on the int8 matrix-core kernel;
 *  - the CPU_REPACK weight layout (block_q4_0x4, nibbles XOR 0x88) is accepted
 *    directly (weight_format) and unpacked on the GPU, instead of by the
 *    caller (integrations/llama_cpp/backend/ggml-qpu.cpp:250-284);
 *  - qxt_llama_q4_0_submission_cpu_fallback exists (so a caller written for
 *    the reference links and keeps its control flow) but computes nothing:
 *    the library has no CPU compute path, so it returns
 *    QXT_CAPABILITY_MISSING and leaves the destination untouched;
 *  - the approximate COLUMN_W8 / ROWCOL_W8A8 modes (rows > 4, as in the
 *    reference) re-quantise the weights on the GPU at prepare time and run on
 *    the int8 matrix cores: COLUMN_W8 on the split-plane Q4_0 prefill kernel
 *    with one fp32 scale per column, ROWCOL_W8A8 on the W8A8 GEMM after a
 *    per-row int8 re-quantisation of each submitted activation; they need
 *    rows * K and resident columns * K below 2^31 (else QXT_CAPABILITY_MISSING).
 */
#ifndef QXT_LLAMA_Q4_0_H
#define QXT_LLAMA_Q4_0_H

#include <stddef.h>
#include <stdint.h>

#include "qxt_gfx950.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qxt_llama_context qxt_llama_context;
typedef struct qxt_llama_q4_0_linear qxt_llama_q4_0_linear;
typedef struct qxt_llama_q4_0_submission qxt_llama_q4_0_submission;

/* Extra failure point of the bridge (qpu_llama_runtime.h:35): the prepare
 * step reports a source-hash mismatch. */
#define QXT_FAIL_SOURCE_HASH (1u << 4)

/* Replaces qpu_llama_context_config (qpu_llama_runtime.h:44-48); the render
 * node becomes a HIP device ordinal. */
typedef struct qxt_llama_context_config {
    int32_t device;        /* HIP device ordinal */
    uint64_t timeout_ns;   /* wait timeout; 0 = 10 s (the reference default) */
    uint32_t failure_mask; /* qxt_failure_point bits | QXT_FAIL_SOURCE_HASH */
} qxt_llama_context_config;

/* Replaces qpu_llama_q4_0_weight_mode (qpu_llama_q4_0.h:16-20). */
typedef enum qxt_llama_q4_0_weight_mode {
    QXT_LLAMA_Q4_0_WEIGHT_EXACT = 0,
    /* int8 weights, one fp32 scale per column (qpu_llama_q4_0.c:332-386):
     * y = fl32(sum_b fl32(float(dot_b) * da_b) * cs[n]), block order. */
    QXT_LLAMA_Q4_0_WEIGHT_COLUMN_W8 = 1,
    /* int8 weights and int8 activation rows, one fp32 scale each
     * (qpu_llama_q4_0.c:526-571, 899-906): y = fl32(fl32(float(dot) * rs[m]) * cs[n]). */
    QXT_LLAMA_Q4_0_WEIGHT_ROWCOL_W8A8 = 2
} qxt_llama_q4_0_weight_mode;

/* Host layout of desc.weights. */
typedef enum qxt_llama_q4_0_weight_format {
    QXT_LLAMA_Q4_0_FORMAT_NATIVE = 0,    /* ggml Q4_0 rows: [output_columns][K/32] x 18 B */
    QXT_LLAMA_Q4_0_FORMAT_REPACK_4X4 = 1 /* ggml CPU_REPACK block_q4_0x4 groups of 4 columns (72 B) */
} qxt_llama_q4_0_weight_format;

/* Replaces qpu_llama_q4_0_linear_desc (qpu_llama_q4_0.h:22-33); the fields up
 * to expected_source_hash are the reference's, weight_format is new. */
typedef struct qxt_llama_q4_0_linear_desc {
    const void *weights;           /* host, format per weight_format */
    size_t weight_size;            /* bytes available at weights */
    uint32_t input_columns;        /* K, multiple of 32 */
    uint32_t output_columns;       /* N */
    uint32_t rows;                 /* row capacity of submissions, 1 .. 262140 */
    uint32_t resident_column_start; /* multiple of 16 */
    uint32_t resident_column_count; /* multiple of 16, non-zero */
    qxt_llama_q4_0_weight_mode weight_mode;
    uint32_t workgroups_per_supergroup; /* accepted and ignored (a VideoCore dispatch knob) */
    const char *expected_source_hash;   /* qxt_llama_q4_0_source_hash() */
    qxt_llama_q4_0_weight_format weight_format;
} qxt_llama_q4_0_linear_desc;

/* Same fields as qpu_llama_q4_0_execution (qpu_llama_q4_0.h:35-48). */
typedef struct qxt_llama_q4_0_execution {
    const void *activation;   /* host Q8_0 rows (34-byte blocks), or Q8_0x4 groups */
    size_t activation_size;
    size_t activation_offset;
    void *destination;        /* host fp32 [rows][output_columns] */
    size_t destination_size;
    size_t destination_offset;
    uint32_t column_start;    /* multiple of 16, inside the resident range */
    uint32_t column_count;    /* multiple of 16, non-zero */
    uint32_t rows;            /* 0 = the prepared capacity */
    uint32_t activation_interleave; /* 0 native rows; 4 or 8: CPU_REPACK block_q8_0x4 */
} qxt_llama_q4_0_execution;

/* Same fields as qpu_llama_q4_0_timing (qpu_llama_q4_0.h:50-61). */
typedef struct qxt_llama_q4_0_timing {
    uint64_t input_access_ns;
    uint64_t input_pack_ns;
    uint64_t input_sync_ns;
    uint64_t input_copy_ns;
    uint64_t submit_ns;
    uint64_t wait_ns;
    uint64_t submit_wait_ns;
    uint64_t output_sync_ns;
    uint64_t output_copy_ns;
    uint64_t complete_ns;
} qxt_llama_q4_0_timing;

/* Replaces qpu_llama_context_create / _destroy / _last_error /
 * _set_failure_mask (qpu_llama_runtime.h:85-94).  config may be NULL
 * (device 0, 10 s timeout, no injected failures). */
int qxt_llama_context_create(const qxt_llama_context_config *config, qxt_llama_context **result);
void qxt_llama_context_destroy(qxt_llama_context *context);
const char *qxt_llama_context_last_error(const qxt_llama_context *context);
void qxt_llama_context_set_failure_mask(qxt_llama_context *context, uint32_t failure_mask);

/* Text of a status ("ok", "invalid argument", ...); replaces
 * qpu_llama_status_string (qpu_llama_runtime.h:133).  Same strings as
 * qxt_status_string. */
const char *qxt_llama_status_string(int status);

/* Hash of the kernel sources this library was built from: the value
 * desc.expected_source_hash must carry (the reference's generated
 * *_source_hash strings, ggml-qpu.cpp:349). */
const char *qxt_llama_q4_0_source_hash(void);

/* Replaces qpu_llama_q4_0_linear_prepare / _destroy / _resident_bytes
 * (qpu_llama_q4_0.h:63-67,81; qpu_llama_q4_0.c:205-459). */
int qxt_llama_q4_0_linear_prepare(qxt_llama_context *context, const qxt_llama_q4_0_linear_desc *desc,
                                  qxt_llama_q4_0_linear **result);
void qxt_llama_q4_0_linear_destroy(qxt_llama_q4_0_linear *linear);
size_t qxt_llama_q4_0_linear_resident_bytes(const qxt_llama_q4_0_linear *linear);

/* Replaces qpu_llama_q4_0_linear_submit / _submission_wait /
 * _submission_destroy / _linear_execute (qpu_llama_q4_0.h:68-80;
 * qpu_llama_q4_0.c:461-946).  timing may be NULL. */
int qxt_llama_q4_0_linear_submit(qxt_llama_q4_0_linear *linear, const qxt_llama_q4_0_execution *execution,
                                 qxt_llama_q4_0_submission **result);
int qxt_llama_q4_0_submission_wait(qxt_llama_q4_0_submission *submission, qxt_llama_q4_0_timing *timing);
void qxt_llama_q4_0_submission_destroy(qxt_llama_q4_0_submission *submission);
int qxt_llama_q4_0_linear_execute(qxt_llama_q4_0_linear *linear, const qxt_llama_q4_0_execution *execution,
                                  qxt_llama_q4_0_timing *timing);

/* Replaces qpu_llama_q4_0_submission_cpu_fallback (qpu_llama_q4_0.h:79-80),
 * which the reference's M=1 hook calls after a failed wait
 * (backend/ggml-qpu-up-inline.cpp:379-388).  This library has no CPU compute
 * path: NULL -> QXT_INVALID_ARGUMENT; otherwise QXT_CAPABILITY_MISSING with
 * the context's last error set and no byte of the destination written, so the
 * caller's own CPU path computes the columns. */
int qxt_llama_q4_0_submission_cpu_fallback(qxt_llama_q4_0_submission *submission);

#ifdef __cplusplus
}
#endif

#endif

/*
 * qxt_ggml_hooks.h -- the ggml CPU_REPACK M=1 Q4_0 hooks, served by gfx950.
 *
 * llama.cpp's CPU_REPACK backend, patched by the reference
 * (integrations/llama_cpp/patches/0002-ggml-cpu-inline-m1-q4-hook.patch:9-29),
 * declares these four symbols weak and calls them when a shared object that
 * defines them is loaded into the process:
 *
 *   - ggml_backend_cpu_repack_buffer_set_tensor passes every 2-D Q4_0 weight,
 *     by tensor name, to ggml_qpu_m1_register_q4_0 (native ggml Q4_0 rows,
 *     before CPU_REPACK repacks them);
 *   - forward_mul_mat, for a one-row product with a registered weight, calls
 *     ggml_qpu_m1_execute with the row's Q8_0 activation and the destination
 *     row, then asks ggml_qpu_m1_cpu_columns_for how many leading output
 *     columns the CPU must still compute (0 = none, the GPU wrote them all).
 *
 * These definitions keep the semantics of the reference's implementation
 * (integrations/llama_cpp/backend/ggml-qpu-up-inline.cpp:261-440) on top of
 * the prepared linear of qxt_llama_q4_0.h:
 *
 *   - the same opt-in environment: GGML_QPU_M1_INLINE = 1/true/on enables
 *     registration and execution, GGML_QPU_M1_TENSORS is a comma-separated
 *     list of substrings of the tensor names to move (empty = none);
 *     GGML_QPU_TELEMETRY=0 silences the one-line JSON records on stderr;
 *   - one process-wide registry: a lazily created context (created at most
 *     once; a failed creation is not retried), one prepared linear per tensor
 *     name (rows = 1, every output column resident, exact weights), guarded by
 *     a mutex;
 *   - return values: 1 = registered / executed, 0 = declined or failed (the
 *     CPU then computes the product itself); a failed execution leaves the
 *     destination untouched and reports every column as a CPU column.
 *
 * The device work runs on the HIP device of the hook context (ordinal 0).
 * Registered linears live until ggml_qpu_m1_release (or process exit).
 */
#ifndef QXT_GGML_HOOKS_H
#define QXT_GGML_HOOKS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Prepare the Q4_0 weight `name` ([output_columns][input_columns/32] native
 * ggml blocks, weight_size bytes) for one-row products.  input_columns % 32
 * == 0, output_columns % 16 == 0.  Returns 1 when the weight is (already)
 * registered, 0 when the hook is disabled, the tensor is not selected, the
 * shape is unsupported or the preparation fails (message on stderr).
 * Replaces ggml_qpu_m1_register_q4_0 (ggml-qpu-up-inline.cpp:261-320). */
int ggml_qpu_m1_register_q4_0(const char *name, const void *weights, size_t weight_size, uint64_t input_columns,
                              uint64_t output_columns);

/* 1 when `name` is registered.  Replaces ggml_qpu_m1_weight_registered
 * (ggml-qpu-up-inline.cpp:322-331). */
int ggml_qpu_m1_weight_registered(const char *name);

/* destination[0 .. output_columns) = the Q4_0 x Q8_0 product of the
 * registered weight `name` with one Q8_0 row (activation_size bytes; native
 * 34-byte blocks, or the CPU_REPACK block_q8_0x4 form when activation_interleave
 * is 4 or 8 -- a single row is stored natively in both).  rows must be 1.
 * Returns 1 on success, 0 otherwise (destination untouched).  Replaces
 * ggml_qpu_m1_execute (ggml-qpu-up-inline.cpp:333-420). */
int ggml_qpu_m1_execute(const char *name, const void *activation_q8_0, size_t activation_size, float *destination,
                        uint64_t rows, uint64_t input_columns, uint64_t output_columns,
                        uint64_t activation_interleave);

/* Leading output columns of the last executed tensor the CPU must compute:
 * 0 after a successful execution, output_columns after a declined or failed
 * one, 0 for any other name.  Replaces ggml_qpu_m1_cpu_columns_for
 * (ggml-qpu-up-inline.cpp:422-431). */
uint64_t ggml_qpu_m1_cpu_columns_for(const char *name);

/* Number of successful executions.  Replaces ggml_qpu_m1_dispatch_count
 * (ggml-qpu-up-inline.cpp:433-436). */
uint64_t ggml_qpu_m1_dispatch_count(void);

/* Destroy every registered linear and the hook context (the next
 * registration creates a new context).  No reference counterpart: the
 * reference frees them in a static destructor at exit; this library frees
 * HIP resources only on request, never during process teardown. */
void ggml_qpu_m1_release(void);

#ifdef __cplusplus
}
#endif

#endif

// Shared host/device helpers of the gfx950 quantized-linear library.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qxt_gfx950.h"

namespace qxt {

// ---------------------------------------------------------------- host side

// Record `message` as the calling thread's last error and return `status`.
int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// OK when no failure is injected for `point`, else the mapped status (with a message).
int injected(uint32_t point);

// Map the result of a kernel launch (hipGetLastError) to a status.
int launch_status(const char *kernel_name);

inline hipStream_t as_stream(void *stream) { return reinterpret_cast<hipStream_t>(stream); }

inline bool aligned(const void *p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// Number of compute units of the current device (cached per device).
int compute_units();

// Every device and pinned-host allocation of the library goes through these;
// they count successful calls (qxt_allocation_count).
hipError_t counted_malloc(void **ptr, size_t bytes);
hipError_t counted_host_malloc(void **ptr, size_t bytes);
template <typename T>
hipError_t device_malloc(T **ptr, size_t bytes) {
    return counted_malloc(reinterpret_cast<void **>(ptr), bytes);
}
template <typename T>
hipError_t pinned_host_malloc(T **ptr, size_t bytes) {
    return counted_host_malloc(reinterpret_cast<void **>(ptr), bytes);
}

// Per-launch timing (qxt_timing_begin/end): when enabled on the calling
// thread, launches record device-side start/stop events.
bool timing_enabled();
void timing_events(hipEvent_t *start, hipEvent_t *stop);
void timing_record(const char *kernel_name, hipEvent_t start, hipEvent_t stop);

// Launch `kernel` on `stream`; every kernel of the library goes through here.
template <typename... KArgs, typename... Args>
int launch(const char *name, void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t stream,
           Args... args) {
    if (timing_enabled()) {
        hipEvent_t start = nullptr, stop = nullptr;
        timing_events(&start, &stop);
        hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), stream, start, stop, 0u,
                              static_cast<KArgs>(args)...);
        timing_record(name, start, stop);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), stream, static_cast<KArgs>(args)...);
    }
    return launch_status(name);
}

// Native-layout Q4_0 x Q8_0 linear for rows >= 16 on the int8 matrix cores
// (qxt_q4_0_tiled.hip); same contract and result as the small-M kernel.
bool q4_0_tiled_native_supported(size_t act_stride, size_t w_stride, uint32_t rows, uint32_t blocks,
                                 uint32_t weight_column_start, uint32_t column_count);
int q4_0_tiled_native(const void *activation, size_t activation_row_stride, const void *weight,
                      size_t weight_row_stride, float *destination, size_t destination_row_stride, uint32_t rows,
                      uint32_t blocks, uint32_t weight_column_start, uint32_t output_column_start,
                      uint32_t column_count, hipStream_t stream);

// Native-layout Q4_0 x Q8_0 linear for 1..15 rows and K <= 24576 with blocks
// spread one per lane (qxt_q4_0_stream.hip); same contract and result as the
// small-M kernel.  QXT_CAPABILITY_MISSING (no message, nothing launched) for
// shapes it does not take.
int q4_0_stream_native(const void *activation, size_t activation_row_stride, const void *weight,
                       size_t weight_row_stride, float *destination, size_t destination_row_stride, uint32_t rows,
                       uint32_t blocks, uint32_t weight_column_start, uint32_t output_column_start,
                       uint32_t column_count, hipStream_t stream);

// QXT_OK when a Q4_0 linear of `rows` rows and `blocks` blocks fits the LDS of
// one workgroup on the v_dot4 path, else QXT_CAPABILITY_MISSING with a
// message (qxt_q4_0.hip).
int q4_0_linear_capability(uint32_t rows, uint32_t blocks);

// Operands of the llama.cpp bridge's approximate weight modes
// (qxt_llama_approx.hip).  Weight codes are uint32 words of four consecutive
// k: word (i, n) at weight_q + i * weight_q_row_stride bytes + 4 n, i < blocks * 8;
// activation codes int8 [rows, blocks * 32] contiguous.
int q4_0_columns_w8(const void *weight, size_t weight_row_stride, uint32_t columns, uint32_t blocks,
                    uint32_t *weight_q, size_t weight_q_row_stride, float *column_scales, hipStream_t stream);
int q8_0_rows_w8(const void *activation, size_t activation_row_stride, uint32_t rows, uint32_t blocks,
                 int8_t *activation_q, float *row_scales, hipStream_t stream);
int q8_0_split_planes(const void *activation, size_t activation_row_stride, uint32_t rows, uint32_t blocks,
                      int8_t *activation_q, uint16_t *activation_scales, hipStream_t stream);
// COLUMN_W8 linear on the int8 matrix cores (qxt_q4_0_tiled.hip): split
// activation planes, weight codes as above, fp32 column scales.
int q4_0_tiled_column_w8(const int8_t *activation_q, const uint16_t *activation_scales, const uint32_t *weight_q,
                         size_t weight_q_row_stride, const float *column_scales, float *destination,
                         size_t destination_row_stride, uint32_t rows, uint32_t blocks, uint32_t columns,
                         hipStream_t stream);

// -------------------------------------------------------------- device side

constexpr int QK = 32;            // elements per GGML block
constexpr int Q4_0_BYTES = 18;    // fp16 d + 16 nibble bytes
constexpr int Q8_0_BYTES = 34;    // fp16 d + 32 int8

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    __half_raw raw;
    raw.x = static_cast<unsigned short>(bits16 & 0xFFFFu);
    return __half2float(__half(raw));
}

__device__ __forceinline__ uint32_t float_to_half_bits(float value) {
    // Round-to-nearest-even conversion (v_cvt_f16_f32 under the default mode).
    __half h = __float2half_rn(value);
    __half_raw raw = static_cast<__half_raw>(h);
    return raw.x;
}

// Per-row int8 quantisation rule (PreparedW8A8Linear._prepare_values,
// src/qpu_xla/models/tinyllama/quantization.py:156-171): scale =
// max(fl32(absmax / 127), fl32(1/127)) (the floor is optional), q =
// clip(rint(x / scale), +-127) with true division.  Shared by the
// standalone quantiser and the GEMV kernels that quantise in place.
__device__ __forceinline__ int clamp127(float r) {
    int q = static_cast<int>(r);
    return q < -127 ? -127 : (q > 127 ? 127 : q);
}

__device__ __forceinline__ float row_scale(float amax, bool floor) {
    float s = amax / 127.0f;
    // fl32(1/127) rounded from the double quotient, as np.float32(1.0 / 127.0).
    if (floor) s = fmaxf(s, static_cast<float>(1.0 / 127.0));
    return s;
}

__device__ __forceinline__ int quant_div(float v, float s) {
    // True IEEE division (no reciprocal shortcut): x / scale, then rint.
    return s > 0.0f ? clamp127(rintf(v / s)) : 0;
}

// quant_div for a whole row from its scale's reciprocal r = fl(1 / s) (IEEE
// division, once per row): q0 = fl(v r) is within an ulp of v / s, the
// residual fma(-q0, s, v) is exact, and fma(residual, r, q0) is the IEEE
// quotient fl(v / s) (Markstein's theorem: a correctly rounded reciprocal and
// one fused correction step give the correctly rounded quotient when nothing
// underflows).  kRecipScaleMin keeps every nonzero residual that can move a
// quotient of magnitude >= 1/4 in the normal range (smaller quotients round
// to 0 either way); below it, and for s = 0, use quant_div.
constexpr float kRecipScaleMin = 0x1p-70f;
__device__ __forceinline__ int quant_recip(float v, float s, float r) {
    const float q0 = v * r;
    const float e = fmaf(-q0, s, v);
    return clamp127(rintf(fmaf(e, r, q0)));
}

// The Q8_0 block scale d = fl(amax / 127) and inv = fl(1 / d) (0 when d is
// 0) -- the two IEEE divisions of the rule -- without the division
// sequences.  d: q0 = fl(amax r) with r = fl(1/127) is within an ulp of the
// quotient, the residual fma(-q0, 127, amax) is exact and fma(residual, r,
// q0) is the correctly rounded quotient (Markstein's theorem).  inv: the
// hardware reciprocal y0 of d, then one fused Newton step fma(fma(-d, y0, 1),
// y0, y0).  amax outside [2^-96, 2^120] (zero, tiny, huge, inf or NaN)
// divides.  Both results equal the IEEE divisions for every non-negative
// fp32 amax: qxt_q8_0_scale_check compares them over all 2^31 bit patterns
// on the device.
constexpr float kQ8FastScaleMin = 0x1p-96f, kQ8FastScaleMax = 0x1p120f;
__device__ __forceinline__ bool q8_0_fast_scale_range(float amax) {
    return amax >= kQ8FastScaleMin && amax <= kQ8FastScaleMax;  // false for NaN
}
// The division-free sequence alone: correct only where q8_0_fast_scale_range.
__device__ __forceinline__ void q8_0_scale_fast(float amax, float &d, float &inv) {
    const float r = static_cast<float>(1.0 / 127.0);
    const float q0 = amax * r;
    d = fmaf(fmaf(-q0, 127.0f, amax), r, q0);
    const float y0 = __builtin_amdgcn_rcpf(d);
    inv = fmaf(fmaf(-d, y0, 1.0f), y0, y0);
}
__device__ __forceinline__ void q8_0_scale(float amax, float &d, float &inv) {
    if (q8_0_fast_scale_range(amax)) {
        q8_0_scale_fast(amax, d, inv);
    } else {
        d = amax / 127.0f;
        inv = d != 0.0f ? 1.0f / d : 0.0f;
    }
}

__device__ __forceinline__ uint32_t pack_bytes(int q0, int q1, int q2, int q3) {
    return (static_cast<uint32_t>(q0) & 0xFFu) | ((static_cast<uint32_t>(q1) & 0xFFu) << 8) |
           ((static_cast<uint32_t>(q2) & 0xFFu) << 16) | ((static_cast<uint32_t>(q3) & 0xFFu) << 24);
}

// Signed 4 x int8 dot product accumulated into int32 (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

}  // namespace qxt

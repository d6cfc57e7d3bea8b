// Wavefront-reduction quantisers for gfx950.
//
//  * Q8_0 activations (one 32-element block per 8 lanes, float4 per lane),
//    arithmetic of quantize_q8_0_split
//    (examples/benchmark_llama_cpp_qpu_persistent_q4.py:42-53).
//  * Per-row int8 activations (one 256-thread workgroup per row, row held in
//    registers), arithmetic of PreparedW8A8Linear._prepare_values
//    (src/qpu_xla/models/tinyllama/quantization.py:156-171).
//  * Q4_0 weights (one block per 8 lanes), ggml's reference rule as used by
//    integrations/llama_cpp/tests/qpu_ggml_backend_smoke.cpp:119.
//
// All three are HBM-streaming kernels: each input byte is read once with
// 16-byte loads; absmax reductions use cross-lane shuffles inside the wave.
// Build with -ffp-contract=off: every multiply and add rounds on its own,
// as NumPy float32 arithmetic does.
#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float group8_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 1, 8));
    v = fmaxf(v, __shfl_xor(v, 2, 8));
    v = fmaxf(v, __shfl_xor(v, 4, 8));
    return v;
}

// Store a 32-bit word at a 2-byte-aligned address as two halves.
__device__ __forceinline__ void store_u32_at_even(uint8_t *p, uint32_t word) {
    uint16_t *h = reinterpret_cast<uint16_t *>(p);
    h[0] = static_cast<uint16_t>(word & 0xFFFFu);
    h[1] = static_cast<uint16_t>(word >> 16);
}

// Inputs are read once, lane-contiguously: 16-byte non-temporal loads on the
// vector path (the streaming read rate is ~10 % higher than with ordinary
// loads on MI355X).
template <bool VEC>
__device__ __forceinline__ float4 load4(const float *p) {
    if constexpr (VEC) {
        typedef float v4f __attribute__((ext_vector_type(4)));
        const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p));
        return make_float4(v[0], v[1], v[2], v[3]);
    } else {
        return make_float4(p[0], p[1], p[2], p[3]);
    }
}

// ------------------------------------------------------------------ Q8_0

template <bool VEC>
__global__ __launch_bounds__(kThreads) void q8_0_kernel(const float *__restrict__ x, size_t x_stride,
                                                        uint8_t *__restrict__ out, size_t out_stride,
                                                        uint32_t rows, uint32_t blocks) {
    const uint64_t gb = (static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 3;
    const int l8 = threadIdx.x & 7;
    if (gb >= static_cast<uint64_t>(rows) * blocks) return;  // whole 8-lane groups exit together
    const uint32_t row = static_cast<uint32_t>(gb / blocks);
    const uint32_t b = static_cast<uint32_t>(gb % blocks);
    const float *src = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(x) + row * x_stride) +
                       b * QK + l8 * 4;
    const float4 v = load4<VEC>(src);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = group8_max(amax);
    const float d = amax / 127.0f;
    const float inv = (d != 0.0f) ? 1.0f / d : 0.0f;
    const int q0 = clamp127(rintf(v.x * inv));
    const int q1 = clamp127(rintf(v.y * inv));
    const int q2 = clamp127(rintf(v.z * inv));
    const int q3 = clamp127(rintf(v.w * inv));
    uint8_t *dst = out + row * out_stride + static_cast<size_t>(b) * Q8_0_BYTES;
    if (l8 == 0) *reinterpret_cast<uint16_t *>(dst) = static_cast<uint16_t>(float_to_half_bits(d));
    store_u32_at_even(dst + 2 + 4 * l8, pack_bytes(q0, q1, q2, q3));
}

// ------------------------------------------------------------- per-row int8

__device__ __forceinline__ float block_max(float v, float *scratch) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    __syncthreads();
    v = scratch[0];
    for (int w = 1; w < kThreads / 64; ++w) v = fmaxf(v, scratch[w]);
    return v;
}

// NV > 0: the row (columns % 4 == 0, <= 1024 * NV columns) is held in registers.
template <int NV, bool VEC>
__global__ __launch_bounds__(kThreads) void rows_int8_kernel(const float *__restrict__ x, size_t x_stride,
                                                             int8_t *__restrict__ q, size_t q_stride,
                                                             float *__restrict__ scales, uint32_t columns,
                                                             uint32_t padded, bool floor) {
    __shared__ float scratch[kThreads / 64];
    const uint32_t row = blockIdx.x;
    const float *src = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(x) + row * x_stride);
    int8_t *dst = q + row * q_stride;
    const uint32_t chunks = columns >> 2;
    float4 v[NV];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t c = threadIdx.x + i * kThreads;
        if (c < chunks) {
            v[i] = load4<VEC>(src + 4 * c);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        }
    }
    const float s = row_scale(block_max(amax, scratch), floor);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t c = threadIdx.x + i * kThreads;
        if (c < chunks) {
            const uint32_t word = pack_bytes(quant_div(v[i].x, s), quant_div(v[i].y, s), quant_div(v[i].z, s),
                                             quant_div(v[i].w, s));
            if constexpr (VEC) {
                *reinterpret_cast<uint32_t *>(dst + 4 * c) = word;
            } else {
                for (int j = 0; j < 4; ++j) dst[4 * c + j] = static_cast<int8_t>((word >> (8 * j)) & 0xFF);
            }
        }
    }
    for (uint32_t c = columns + threadIdx.x; c < padded; c += kThreads) dst[c] = 0;
    if (threadIdx.x == 0) scales[row] = s;
}

// Any column count: two passes over the row (the second from cache).
__global__ __launch_bounds__(kThreads) void rows_int8_generic_kernel(const float *__restrict__ x, size_t x_stride,
                                                                     int8_t *__restrict__ q, size_t q_stride,
                                                                     float *__restrict__ scales, uint32_t columns,
                                                                     uint32_t padded, bool floor) {
    __shared__ float scratch[kThreads / 64];
    const uint32_t row = blockIdx.x;
    const float *src = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(x) + row * x_stride);
    int8_t *dst = q + row * q_stride;
    float amax = 0.0f;
    for (uint32_t c = threadIdx.x; c < columns; c += kThreads) amax = fmaxf(amax, fabsf(src[c]));
    const float s = row_scale(block_max(amax, scratch), floor);
    for (uint32_t c = threadIdx.x; c < columns; c += kThreads) dst[c] = static_cast<int8_t>(quant_div(src[c], s));
    for (uint32_t c = columns + threadIdx.x; c < padded; c += kThreads) dst[c] = 0;
    if (threadIdx.x == 0) scales[row] = s;
}

// ------------------------------------------------------------------ Q4_0

template <bool VEC>
__global__ __launch_bounds__(kThreads) void q4_0_kernel(const float *__restrict__ w, size_t w_stride,
                                                        uint8_t *__restrict__ out, size_t out_stride,
                                                        uint32_t rows, uint32_t blocks) {
    const uint64_t gb = (static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 3;
    const int l8 = threadIdx.x & 7;
    if (gb >= static_cast<uint64_t>(rows) * blocks) return;
    const uint32_t row = static_cast<uint32_t>(gb / blocks);
    const uint32_t b = static_cast<uint32_t>(gb % blocks);
    const float *src = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(w) + row * w_stride) +
                       b * QK + l8 * 4;
    const float4 v = load4<VEC>(src);
    const float e[4] = {v.x, v.y, v.z, v.w};
    // First element of largest magnitude (strict '>' keeps the earliest).
    float amax = 0.0f, vmax = 0.0f;
    int idx = l8 * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (fabsf(e[i]) > amax) {
            amax = fabsf(e[i]);
            vmax = e[i];
            idx = l8 * 4 + i;
        }
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        const float oa = __shfl_xor(amax, off, 8);
        const float ov = __shfl_xor(vmax, off, 8);
        const int oi = __shfl_xor(idx, off, 8);
        if (oa > amax || (oa == amax && oi < idx)) {
            amax = oa;
            vmax = ov;
            idx = oi;
        }
    }
    const float signed_max = amax > 0.0f ? vmax : 0.0f;
    const float d = signed_max / -8.0f;
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    int qv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float t = e[i] * id;
        const int c = static_cast<int>(truncf(t + 8.5f));
        qv[i] = c > 15 ? 15 : c;
    }
    // Lanes 0..3 hold elements 0..15 (low nibbles); lanes 4..7 elements 16..31 (high).
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) mine |= (static_cast<uint32_t>(qv[i]) & 0xFu) << (8 * i);
    const uint32_t high = __shfl_xor(mine, 4, 8);
    uint8_t *dst = out + row * out_stride + static_cast<size_t>(b) * Q4_0_BYTES;
    if (l8 == 0) *reinterpret_cast<uint16_t *>(dst) = static_cast<uint16_t>(float_to_half_bits(d));
    if (l8 < 4) store_u32_at_even(dst + 2 + 4 * l8, mine | (high << 4));
}

inline unsigned grid_for_blocks(uint64_t total_blocks) {
    return static_cast<unsigned>((total_blocks * 8 + kThreads - 1) / kThreads);
}

}  // namespace
}  // namespace qxt

using namespace qxt;

extern "C" {

int qxt_quantize_q8_0(const float *x, size_t x_row_stride, void *blocks, size_t blocks_row_stride,
                      uint32_t rows, uint32_t columns, void *stream) {
    if (x == nullptr || blocks == nullptr) return fail(QXT_INVALID_ARGUMENT, "q8_0: null pointer");
    if (rows == 0 || columns == 0 || columns % QK)
        return fail(QXT_INVALID_ARGUMENT, "q8_0: rows > 0 and columns a positive multiple of 32 required");
    const uint32_t nb = columns / QK;
    if (x_row_stride < columns * sizeof(float) || x_row_stride % sizeof(float) ||
        blocks_row_stride < static_cast<size_t>(nb) * Q8_0_BYTES || blocks_row_stride % 2 || !aligned(x, 4) ||
        !aligned(blocks, 2))
        return fail(QXT_INVALID_ARGUMENT, "q8_0: bad strides or alignment");
    int rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    const bool vec = aligned(x, 16) && x_row_stride % 16 == 0;
    const unsigned grid = grid_for_blocks(static_cast<uint64_t>(rows) * nb);
    auto *out = static_cast<uint8_t *>(blocks);
    return launch("q8_0_kernel", vec ? q8_0_kernel<true> : q8_0_kernel<false>, dim3(grid), dim3(kThreads), 0,
                  as_stream(stream), x, x_row_stride, out, blocks_row_stride, rows, nb);
}

int qxt_quantize_rows_int8(const float *x, size_t x_row_stride, int8_t *q, size_t q_row_stride, float *scales,
                           uint32_t rows, uint32_t columns, uint32_t padded_columns, uint32_t flags,
                           void *stream) {
    if (x == nullptr || q == nullptr || scales == nullptr)
        return fail(QXT_INVALID_ARGUMENT, "rows_int8: null pointer");
    if (rows == 0 || columns == 0 || padded_columns < columns)
        return fail(QXT_INVALID_ARGUMENT, "rows_int8: rows, columns > 0 and padded_columns >= columns required");
    if (x_row_stride < columns * sizeof(float) || x_row_stride % sizeof(float) || q_row_stride < padded_columns ||
        !aligned(x, 4) || !aligned(scales, 4))
        return fail(QXT_INVALID_ARGUMENT, "rows_int8: bad strides or alignment");
    if (flags & ~QXT_QUANT_NO_SCALE_FLOOR) return fail(QXT_INVALID_ARGUMENT, "rows_int8: unknown flags");
    int rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    const bool floor = (flags & QXT_QUANT_NO_SCALE_FLOOR) == 0;
    const bool vec = columns % 4 == 0 && aligned(x, 16) && x_row_stride % 16 == 0 && aligned(q, 4) &&
                     q_row_stride % 4 == 0;
    const uint32_t per_thread = (columns / 4 + kThreads - 1) / kThreads;
    auto kernel = rows_int8_generic_kernel;
    if (vec && per_thread <= 1) kernel = rows_int8_kernel<1, true>;
    else if (vec && per_thread <= 2) kernel = rows_int8_kernel<2, true>;
    else if (vec && per_thread <= 4) kernel = rows_int8_kernel<4, true>;
    else if (vec && per_thread <= 8) kernel = rows_int8_kernel<8, true>;
    else if (vec && per_thread <= 16) kernel = rows_int8_kernel<16, true>;
    return launch("rows_int8_kernel", kernel, dim3(rows), dim3(kThreads), 0, as_stream(stream), x, x_row_stride, q,
                  q_row_stride, scales, columns, padded_columns, floor);
}

int qxt_quantize_q4_0(const float *w, size_t w_row_stride, void *blocks, size_t blocks_row_stride, uint32_t rows,
                      uint32_t columns, void *stream) {
    if (w == nullptr || blocks == nullptr) return fail(QXT_INVALID_ARGUMENT, "q4_0: null pointer");
    if (rows == 0 || columns == 0 || columns % QK)
        return fail(QXT_INVALID_ARGUMENT, "q4_0: rows > 0 and columns a positive multiple of 32 required");
    const uint32_t nb = columns / QK;
    if (w_row_stride < columns * sizeof(float) || w_row_stride % sizeof(float) ||
        blocks_row_stride < static_cast<size_t>(nb) * Q4_0_BYTES || blocks_row_stride % 2 || !aligned(w, 4) ||
        !aligned(blocks, 2))
        return fail(QXT_INVALID_ARGUMENT, "q4_0: bad strides or alignment");
    int rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    const bool vec = aligned(w, 16) && w_row_stride % 16 == 0;
    const unsigned grid = grid_for_blocks(static_cast<uint64_t>(rows) * nb);
    auto *out = static_cast<uint8_t *>(blocks);
    return launch("q4_0_kernel", vec ? q4_0_kernel<true> : q4_0_kernel<false>, dim3(grid), dim3(kThreads), 0,
                  as_stream(stream), w, w_row_stride, out, blocks_row_stride, rows, nb);
}

}  // extern "C"

// Operand preparation for the llama.cpp bridge's approximate Q4_0 weight
// modes (COLUMN_W8, ROWCOL_W8A8; integrations/llama_cpp/src/qpu_llama_q4_0.c).
//
//  * q4_0_columns_w8_kernel: a Q4_0 weight column -> int8 codes with one fp32
//    column scale (prepare time, qpu_llama_q4_0.c:332-386).
//  * q8_0_rows_w8_kernel: a Q8_0 activation row -> int8 codes with one fp32
//    row scale (ROWCOL_W8A8 submissions, qpu_llama_q4_0.c:526-571).
//  * q8_0_split_kernel: Q8_0 rows -> int8 values [M, K] + fp16 scale bits
//    [M, K/32], the split planes the column-scale tiled kernel reads
//    (COLUMN_W8 submissions, qpu_llama_q4_0.c:572-607).
//
// One workgroup per column or row: a pass for the absolute maximum (of exact
// products: a 4- or 8-bit integer times an fp16 scale fits fp32's mantissa),
// then a pass that re-quantises.  Rounding rule of both re-quantisers:
// s = fl32(v / scale), q = trunc(fl32(s +- 0.5)) clamped to [-127, 127]
// (the fp32 addition included: s = 0.49999997 gives 1).  Built with
// -ffp-contract=off and correctly rounded fp32 division.
#include <cmath>

#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ int round_half_away_w8(float s) {
    const float shifted = s >= 0.0f ? s + 0.5f : s - 0.5f;
    return static_cast<int>(fminf(fmaxf(truncf(shifted), -127.0f), 127.0f));
}

// Maximum of v over the workgroup (every thread receives it).
__device__ __forceinline__ float workgroup_max(float v, float *lds) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    v = lds[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) v = fmaxf(v, lds[w]);
    return v;
}

// Four consecutive bytes at a 2-byte-aligned address.
__device__ __forceinline__ uint32_t load_u32_at_even(const uint8_t *p) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    return static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
}

// Word i of a Q4_0 row (elements 4i .. 4i + 3): fl32((code - 8) * d).
__device__ __forceinline__ void q4_0_word(const uint8_t *row, uint32_t i, float (&v)[4]) {
    const uint8_t *block = row + static_cast<size_t>(i >> 3) * Q4_0_BYTES;
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t *>(block));
    const uint32_t j = i & 7;
    // Elements 0..15 of a block are the low nibbles of its 16 code bytes,
    // elements 16..31 the high nibbles.
    const uint32_t bytes = load_u32_at_even(block + 2 + 4 * (j & 3));
    const uint32_t shift = j < 4 ? 0 : 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int code = static_cast<int>((bytes >> (8 * e + shift)) & 0xFu);
        v[e] = static_cast<float>(code - 8) * d;
    }
}

// Word i of a Q8_0 row: fl32(q * d).
__device__ __forceinline__ void q8_0_word(const uint8_t *row, uint32_t i, float (&v)[4]) {
    const uint8_t *block = row + static_cast<size_t>(i >> 3) * Q8_0_BYTES;
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t *>(block));
    const uint32_t bytes = load_u32_at_even(block + 2 + 4 * (i & 7));
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = static_cast<float>(static_cast<int8_t>(bytes >> (8 * e))) * d;
}

template <bool WEIGHT>
__device__ __forceinline__ void word_values(const uint8_t *row, uint32_t i, float (&v)[4]) {
    if constexpr (WEIGHT) q4_0_word(row, i, v);
    else q8_0_word(row, i, v);
}

// One workgroup per row of the source (a weight column or an activation
// row): codes go to out[i * out_words_stride] word by word (weights: the
// [K/4, N] word layout; activations: contiguous).
template <bool WEIGHT>
__global__ __launch_bounds__(kThreads) void requantize_w8_kernel(const uint8_t *__restrict__ src, size_t src_stride,
                                                                 uint32_t blocks, uint32_t *__restrict__ out,
                                                                 size_t out_row_words, size_t out_word_stride,
                                                                 float *__restrict__ scales) {
    __shared__ float lds[kThreads / 64];
    const uint8_t *row = src + static_cast<size_t>(blockIdx.x) * src_stride;
    const uint32_t words = blocks * 8;
    float maximum = 0.0f;
    for (uint32_t i = threadIdx.x; i < words; i += kThreads) {
        float v[4];
        word_values<WEIGHT>(row, i, v);
#pragma unroll
        for (int e = 0; e < 4; ++e) maximum = fmaxf(maximum, fabsf(v[e]));
    }
    maximum = workgroup_max(maximum, lds);
    const float scale = maximum > 0.0f ? maximum / 127.0f : 0.0f;
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
    uint32_t *dst = out + static_cast<size_t>(blockIdx.x) * out_row_words;
    for (uint32_t i = threadIdx.x; i < words; i += kThreads) {
        float v[4];
        word_values<WEIGHT>(row, i, v);
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int q = scale > 0.0f ? round_half_away_w8(v[e] / scale) : 0;
            word |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * e);
        }
        dst[i * out_word_stride] = word;
    }
}

// One thread per (row, word): int8 values and, for the block's first word,
// its fp16 scale bits.
__global__ __launch_bounds__(kThreads) void q8_0_split_kernel(const uint8_t *__restrict__ src, size_t src_stride,
                                                              uint32_t rows, uint32_t blocks, uint32_t *__restrict__ aq,
                                                              uint16_t *__restrict__ as) {
    const size_t words = static_cast<size_t>(blocks) * 8;
    const size_t idx = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= static_cast<size_t>(rows) * words) return;
    const size_t r = idx / words, i = idx - r * words;
    const uint8_t *block = src + r * src_stride + (i >> 3) * Q8_0_BYTES;
    aq[idx] = load_u32_at_even(block + 2 + 4 * (i & 7));
    if ((i & 7) == 0) as[r * blocks + (i >> 3)] = *reinterpret_cast<const uint16_t *>(block);
}

}  // namespace

int q4_0_columns_w8(const void *weight, size_t weight_row_stride, uint32_t columns, uint32_t blocks,
                    uint32_t *weight_q, size_t weight_q_row_stride, float *column_scales, hipStream_t stream) {
    if (weight_q_row_stride % 4 || weight_q_row_stride < static_cast<size_t>(columns) * 4)
        return fail(QXT_INVALID_ARGUMENT, "column-w8 weights: bad code row stride");
    return launch("q4_0_columns_w8_kernel", requantize_w8_kernel<true>, dim3(columns), dim3(kThreads), 0, stream,
                  static_cast<const uint8_t *>(weight), weight_row_stride, blocks, weight_q, size_t{1},
                  weight_q_row_stride / 4, column_scales);
}

int q8_0_rows_w8(const void *activation, size_t activation_row_stride, uint32_t rows, uint32_t blocks,
                 int8_t *activation_q, float *row_scales, hipStream_t stream) {
    return launch("q8_0_rows_w8_kernel", requantize_w8_kernel<false>, dim3(rows), dim3(kThreads), 0, stream,
                  static_cast<const uint8_t *>(activation), activation_row_stride, blocks,
                  reinterpret_cast<uint32_t *>(activation_q), static_cast<size_t>(blocks) * 8, size_t{1}, row_scales);
}

int q8_0_split_planes(const void *activation, size_t activation_row_stride, uint32_t rows, uint32_t blocks,
                      int8_t *activation_q, uint16_t *activation_scales, hipStream_t stream) {
    const size_t items = static_cast<size_t>(rows) * blocks * 8;
    const size_t grid = (items + kThreads - 1) / kThreads;
    if (grid > 0x7FFFFFFFu) return fail(QXT_INVALID_ARGUMENT, "q8_0 split: too many rows");
    return launch("q8_0_split_kernel", q8_0_split_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0, stream,
                  static_cast<const uint8_t *>(activation), activation_row_stride, rows, blocks,
                  reinterpret_cast<uint32_t *>(activation_q), activation_scales);
}

}  // namespace qxt

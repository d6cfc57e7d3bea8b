// Q4_0 x Q8_0 block-dot linear for gfx950 (M = 1 decode and small M).
//
// Arithmetic (reference src/qpu_xla/kernels/ggml_q4_0.py:81-100 and the QPU
// loop at :688-692): per 32-element block an exact int32 dot, then
// c_b = fl32(fl32(float(dot_b) * dw_b) * da_b), summed in block order
// ((0 + c_0) + c_1) + ...  This kernel reproduces that result bit for bit:
//
//   phase 1  the workgroup stages the Q8_0 activation rows in LDS as int8
//            words plus (fp32 scale, int32 element sum) per block;
//   phase 2  every thread streams one "unit" of weights -- 8 consecutive
//            blocks of one column, 144 bytes = 9 x 16-byte loads on the fast
//            path -- computes the 8 block terms c_b with v_dot4_i32_i8 and
//            writes them to LDS;
//   phase 3  one thread per (row, column) adds that column's c_b in block
//            order and stores the fp32 result.
//
// Nibble codes enter the dot as unsigned 0..15; the "- 8" of every element
// is applied once per block as -8 * sum(activation), which is exact in int32.
// The fast path needs blocks % 8 == 0 and 16-byte aligned weight rows (true
// for every K that is a multiple of 256); otherwise each thread takes one
// block with 2-byte loads.
#include <type_traits>

#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;
constexpr size_t kMaxLds = 64 * 1024;

struct Q4Args {
    const uint8_t *act;
    size_t act_stride;
    const uint8_t *w;
    size_t w_stride;
    float *dst;
    size_t dst_stride;
    int32_t *dots;  // non-null: debug mode, write int32 block dots instead of the sum
    int rows, blocks, wcol0, ocol0, ncols;
    int cpw;  // columns per workgroup
};

// LDS geometry (in 32-bit words) for a row group of MR rows.
struct Q4Lds {
    int aq_row;  // activation int8 words per row: 8 per block + 4 pad per 8 blocks
    int ad_row;  // (scale, sum) pairs per row: one per block + 1 pad per 8 blocks, x2 words
    int cbs;     // c_b stride per column
    __host__ __device__ Q4Lds(int blocks, bool fast) {
        aq_row = blocks * 8 + ((blocks + 7) / 8) * 4;
        ad_row = (2 * (blocks + (blocks + 7) / 8) + 3) & ~3;  // keeps the c_b region 16-byte aligned
        cbs = fast ? blocks + 4 : blocks + 1;
    }
    __host__ __device__ size_t words(int mr, int cpw) const {
        return static_cast<size_t>(mr) * (aq_row + ad_row) + static_cast<size_t>(mr) * cpw * cbs;
    }
};

// Word index of activation word j (0..7) of block b inside one LDS row.  The
// extra 4 words every 8 blocks keep lanes that read different 8-block units
// on distinct banks.
__device__ __forceinline__ int aq_index(int b, int j) { return b * 8 + (b >> 3) * 4 + j; }
__device__ __forceinline__ int ad_index(int b) { return 2 * (b + (b >> 3)); }

// Block i (0..7) of a 144-byte unit held as 36 little-endian words: returns
// the fp16 scale bits and the 4 words of packed nibbles.
template <int I>
__device__ __forceinline__ void unit_block(const uint32_t (&d)[36], uint32_t &sbits, uint32_t (&qs)[4]) {
    if constexpr ((I & 1) == 0) {
        constexpr int k = 9 * I / 2;  // block starts word-aligned: d then nibbles at +2 bytes
        sbits = d[k] & 0xFFFFu;
#pragma unroll
        for (int t = 0; t < 4; ++t) qs[t] = __builtin_amdgcn_alignbyte(d[k + t + 1], d[k + t], 2);
    } else {
        constexpr int k = (9 * I - 1) / 2;  // block starts at a half word: nibbles word-aligned
        sbits = d[k] >> 16;
#pragma unroll
        for (int t = 0; t < 4; ++t) qs[t] = d[k + 1 + t];
    }
}

// Exact int32 dot of one Q4_0 block (packed nibbles qs) with one Q8_0 block.
__device__ __forceinline__ int block_dot(const uint32_t (&qs)[4], const int *aq, int asum) {
    const int4 a0 = *reinterpret_cast<const int4 *>(aq);
    const int4 a1 = *reinterpret_cast<const int4 *>(aq + 4);
    int s = 0;
    s = dot4(static_cast<int>(qs[0] & 0x0F0F0F0Fu), a0.x, s);
    s = dot4(static_cast<int>(qs[1] & 0x0F0F0F0Fu), a0.y, s);
    s = dot4(static_cast<int>(qs[2] & 0x0F0F0F0Fu), a0.z, s);
    s = dot4(static_cast<int>(qs[3] & 0x0F0F0F0Fu), a0.w, s);
    s = dot4(static_cast<int>((qs[0] >> 4) & 0x0F0F0F0Fu), a1.x, s);
    s = dot4(static_cast<int>((qs[1] >> 4) & 0x0F0F0F0Fu), a1.y, s);
    s = dot4(static_cast<int>((qs[2] >> 4) & 0x0F0F0F0Fu), a1.z, s);
    s = dot4(static_cast<int>((qs[3] >> 4) & 0x0F0F0F0Fu), a1.w, s);
    return s - 8 * asum;
}

template <int MR, bool FAST, bool DOTS>
__global__ __launch_bounds__(kThreads) void q4_0_linear_kernel(Q4Args args) {
    extern __shared__ int lds[];
    const int B = args.blocks;
    const Q4Lds geo(B, FAST);
    int *aq = lds;                                  // [MR][aq_row]
    int *ad = aq + MR * geo.aq_row;                 // [MR][ad_row]  (scale bits as float, sum)
    float *cb = reinterpret_cast<float *>(ad + MR * geo.ad_row);  // [MR][cpw][cbs]

    const int r0 = blockIdx.y * MR;
    const int col_base = blockIdx.x * args.cpw;
    const int tile_cols = min(args.cpw, args.ncols - col_base);

    // ---- phase 1: stage the activation rows of this row group.
    for (int idx = threadIdx.x; idx < MR * B; idx += kThreads) {
        const int r = idx / B;
        const int b = idx - r * B;
        int words[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float d = 0.0f;
        int sum = 0;
        if (r0 + r < args.rows) {
            const uint16_t *p = reinterpret_cast<const uint16_t *>(args.act + (r0 + r) * args.act_stride +
                                                                   static_cast<size_t>(b) * Q8_0_BYTES);
            d = half_bits_to_float(p[0]);
#pragma unroll
            for (int h = 0; h < 16; ++h) {
                const uint32_t two = p[1 + h];
                words[h >> 1] |= static_cast<int>(two << (16 * (h & 1)));
                sum += static_cast<int8_t>(two & 0xFF) + static_cast<int8_t>(two >> 8);
            }
        }
        int *dstq = aq + r * geo.aq_row + aq_index(b, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) dstq[j] = words[j];
        ad[r * geo.ad_row + ad_index(b)] = __float_as_int(d);
        ad[r * geo.ad_row + ad_index(b) + 1] = sum;
    }
    __syncthreads();

    // ---- phase 2: block terms.
    if constexpr (FAST) {
        const int G = B >> 3;
        const int units = tile_cols * G;
        for (int u = threadIdx.x; u < units; u += kThreads) {
            const int col = u / G;
            const int g = u - col * G;
            const int n = args.wcol0 + col_base + col;
            const uint4 *src = reinterpret_cast<const uint4 *>(args.w + static_cast<size_t>(n) * args.w_stride +
                                                               static_cast<size_t>(g) * 144);
            uint32_t d[36];
#pragma unroll
            for (int v = 0; v < 9; ++v) {
                const uint4 x = src[v];
                d[4 * v + 0] = x.x;
                d[4 * v + 1] = x.y;
                d[4 * v + 2] = x.z;
                d[4 * v + 3] = x.w;
            }
            float terms[MR][8];
            int idots[MR][8];
            auto do_block = [&](auto ic) {
                constexpr int I = decltype(ic)::value;
                uint32_t sbits, qs[4];
                unit_block<I>(d, sbits, qs);
                const float dw = half_bits_to_float(sbits);
                const int b = g * 8 + I;
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    const int *arow = aq + r * geo.aq_row + aq_index(b, 0);
                    const int2 ds = *reinterpret_cast<const int2 *>(ad + r * geo.ad_row + ad_index(b));
                    const int dot = block_dot(qs, arow, ds.y);
                    idots[r][I] = dot;
                    float t = static_cast<float>(dot) * dw;
                    t = t * __int_as_float(ds.x);
                    terms[r][I] = t;
                }
            };
            do_block(std::integral_constant<int, 0>{});
            do_block(std::integral_constant<int, 1>{});
            do_block(std::integral_constant<int, 2>{});
            do_block(std::integral_constant<int, 3>{});
            do_block(std::integral_constant<int, 4>{});
            do_block(std::integral_constant<int, 5>{});
            do_block(std::integral_constant<int, 6>{});
            do_block(std::integral_constant<int, 7>{});
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                if constexpr (DOTS) {
                    if (r0 + r < args.rows) {
                        int32_t *out = args.dots + (static_cast<size_t>(r0 + r) * args.ncols + col_base + col) * B +
                                       g * 8;
#pragma unroll
                        for (int i = 0; i < 8; ++i) out[i] = idots[r][i];
                    }
                } else {
                    float4 *c4 = reinterpret_cast<float4 *>(cb + (r * args.cpw + col) * geo.cbs + g * 8);
                    c4[0] = make_float4(terms[r][0], terms[r][1], terms[r][2], terms[r][3]);
                    c4[1] = make_float4(terms[r][4], terms[r][5], terms[r][6], terms[r][7]);
                }
            }
        }
    } else {
        const int units = tile_cols * B;
        for (int u = threadIdx.x; u < units; u += kThreads) {
            const int col = u / B;
            const int b = u - col * B;
            const int n = args.wcol0 + col_base + col;
            const uint16_t *p = reinterpret_cast<const uint16_t *>(args.w + static_cast<size_t>(n) * args.w_stride +
                                                                   static_cast<size_t>(b) * Q4_0_BYTES);
            const float dw = half_bits_to_float(p[0]);
            uint32_t qs[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) qs[t] = static_cast<uint32_t>(p[1 + 2 * t]) | (static_cast<uint32_t>(p[2 + 2 * t]) << 16);
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                const int *arow = aq + r * geo.aq_row + aq_index(b, 0);
                const int2 ds = *reinterpret_cast<const int2 *>(ad + r * geo.ad_row + ad_index(b));
                const int dot = block_dot(qs, arow, ds.y);
                if constexpr (DOTS) {
                    if (r0 + r < args.rows)
                        args.dots[(static_cast<size_t>(r0 + r) * args.ncols + col_base + col) * B + b] = dot;
                } else {
                    float t = static_cast<float>(dot) * dw;
                    t = t * __int_as_float(ds.x);
                    cb[(r * args.cpw + col) * geo.cbs + b] = t;
                }
            }
        }
    }
    if constexpr (DOTS) return;
    __syncthreads();

    // ---- phase 3: in-order fp32 sum per (row, column).
    for (int t = threadIdx.x; t < MR * tile_cols; t += kThreads) {
        const int r = t / tile_cols;
        const int col = t - r * tile_cols;
        if (r0 + r >= args.rows) continue;
        const float *c = cb + (r * args.cpw + col) * geo.cbs;
        float acc = 0.0f;
        if constexpr (FAST) {
            for (int b = 0; b < B; b += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(c + b);
                acc += v.x;
                acc += v.y;
                acc += v.z;
                acc += v.w;
            }
        } else {
            for (int b = 0; b < B; ++b) acc += c[b];
        }
        float *out = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(args.dst) + (r0 + r) * args.dst_stride);
        out[args.ocol0 + col_base + col] = acc;
    }
}

template <int MR, bool DOTS>
int launch_q4(Q4Args args, bool fast, hipStream_t stream) {
    const Q4Lds geo(args.blocks, fast);
    const int units_per_col = fast ? args.blocks / 8 : args.blocks;
    int cpw = units_per_col >= kThreads ? 1 : kThreads / units_per_col;
    while (cpw > 1 && geo.words(MR, DOTS ? 0 : cpw) * 4 > kMaxLds) --cpw;
    const size_t lds = geo.words(MR, DOTS ? 0 : cpw) * 4;
    if (lds > kMaxLds)
        return fail(QXT_CAPABILITY_MISSING, "q4_0 linear: K=%d needs %zu bytes of LDS (> %zu)", args.blocks * 32,
                    lds, kMaxLds);
    args.cpw = cpw;
    dim3 grid((args.ncols + cpw - 1) / cpw, (args.rows + MR - 1) / MR, 1);
    return launch(DOTS ? "q4_0_block_dots_kernel" : "q4_0_linear_kernel",
                  fast ? q4_0_linear_kernel<MR, true, DOTS> : q4_0_linear_kernel<MR, false, DOTS>, grid,
                  dim3(kThreads), lds, stream, args);
}

template <bool DOTS>
int dispatch_q4(const Q4Args &args, hipStream_t stream) {
    const bool fast = args.blocks % 8 == 0 && aligned(args.w, 16) && args.w_stride % 16 == 0;
    switch (args.rows >= 4 ? 4 : args.rows) {
        case 1: return launch_q4<1, DOTS>(args, fast, stream);
        case 2: return launch_q4<2, DOTS>(args, fast, stream);
        case 3: return launch_q4<3, DOTS>(args, fast, stream);
        default: return launch_q4<4, DOTS>(args, fast, stream);
    }
}

int validate_q4(const void *activation, size_t activation_row_stride, const void *weight, size_t weight_row_stride,
                uint32_t rows, uint32_t blocks, uint32_t column_count) {
    if (activation == nullptr || weight == nullptr) return fail(QXT_INVALID_ARGUMENT, "q4_0 linear: null pointer");
    if (rows == 0 || blocks == 0 || column_count == 0)
        return fail(QXT_INVALID_ARGUMENT, "q4_0 linear: rows, blocks and column_count must be positive");
    if (rows > 65535u * 4u || blocks > (1u << 20) || column_count > (1u << 30))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 linear: problem too large");
    if (activation_row_stride < static_cast<size_t>(blocks) * Q8_0_BYTES || activation_row_stride % 2 ||
        weight_row_stride < static_cast<size_t>(blocks) * Q4_0_BYTES || weight_row_stride % 2 ||
        !aligned(activation, 2) || !aligned(weight, 2))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 linear: bad strides or alignment");
    return QXT_OK;
}

}  // namespace
}  // namespace qxt

using namespace qxt;

extern "C" {

int qxt_ggml_q4_0_q8_0_linear(const void *activation, size_t activation_row_stride, const void *weight,
                              size_t weight_row_stride, float *destination, size_t destination_row_stride,
                              uint32_t rows, uint32_t blocks, uint32_t weight_column_start,
                              uint32_t output_column_start, uint32_t column_count, void *stream) {
    int rc = validate_q4(activation, activation_row_stride, weight, weight_row_stride, rows, blocks, column_count);
    if (rc != QXT_OK) return rc;
    if (destination == nullptr || !aligned(destination, 4) || destination_row_stride % 4 ||
        destination_row_stride < (static_cast<size_t>(output_column_start) + column_count) * sizeof(float))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 linear: bad destination");
    if (static_cast<uint64_t>(weight_column_start) + column_count > (1ull << 31) ||
        static_cast<uint64_t>(output_column_start) + column_count > (1ull << 31))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 linear: column range overflows");
    rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    Q4Args args{static_cast<const uint8_t *>(activation),
                activation_row_stride,
                static_cast<const uint8_t *>(weight),
                weight_row_stride,
                destination,
                destination_row_stride,
                nullptr,
                static_cast<int>(rows),
                static_cast<int>(blocks),
                static_cast<int>(weight_column_start),
                static_cast<int>(output_column_start),
                static_cast<int>(column_count),
                0};
    return dispatch_q4<false>(args, as_stream(stream));
}

int qxt_ggml_q4_0_q8_0_block_dots(const void *activation, size_t activation_row_stride, const void *weight,
                                  size_t weight_row_stride, int32_t *dots, uint32_t rows, uint32_t blocks,
                                  uint32_t weight_column_start, uint32_t column_count, void *stream) {
    int rc = validate_q4(activation, activation_row_stride, weight, weight_row_stride, rows, blocks, column_count);
    if (rc != QXT_OK) return rc;
    if (dots == nullptr || !aligned(dots, 4)) return fail(QXT_INVALID_ARGUMENT, "q4_0 block dots: bad output");
    if (static_cast<uint64_t>(weight_column_start) + column_count > (1ull << 31))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 block dots: column range overflows");
    rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    Q4Args args{static_cast<const uint8_t *>(activation),
                activation_row_stride,
                static_cast<const uint8_t *>(weight),
                weight_row_stride,
                nullptr,
                0,
                dots,
                static_cast<int>(rows),
                static_cast<int>(blocks),
                static_cast<int>(weight_column_start),
                0,
                static_cast<int>(column_count),
                0};
    return dispatch_q4<true>(args, as_stream(stream));
}

}  // extern "C"

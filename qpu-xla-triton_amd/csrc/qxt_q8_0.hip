// Q8_0 x Q8_0 block-dot linear for gfx950 (small M).
//
// Arithmetic (reference src/qpu_xla/kernels/ggml_q8_0.py:26-51): per
// 32-element block an exact int32 dot of two signed int8 blocks, then
// c_b = fl32(fl32(float(dot_b) * da_b) * dw_b) -- the activation scale first,
// unlike the Q4_0 path -- summed in block order.  The kernel reproduces that
// result bit for bit.
//
// Two forms; in both a workgroup owns a tile of output columns, block terms
// go to LDS and one thread per (row, column) adds them in block order.  Up to
// 512 blocks (K <= 16384) the block-per-lane form (q8_0_stream_kernel, below)
// spreads each column's blocks over the lanes and keeps the activation in
// registers.  Beyond it, the unit form: on its fast path (blocks % 8 == 0,
// 16-byte aligned rows) a thread takes "units" of 8 consecutive blocks of one
// column (272 bytes = 17 x 16-byte loads, issued before the activation is
// staged in LDS); otherwise a thread takes one block with 2-byte loads.
#include <algorithm>
#include <type_traits>

#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;
constexpr size_t kMaxLds = 64 * 1024;
constexpr int kUnitWords = 68;  // 8 blocks x 34 bytes

struct Q8Task {
    const uint8_t *act;  // Q8_0 [rows, blocks, 34]
    const uint8_t *w;    // Q8_0 [N, blocks, 34]
    float *y;
    size_t act_stride, w_stride, y_stride;
    int rows, blocks, wcol0, ocol0, ncols, cpw;
};

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

struct Q8Lds {
    int aq_row;  // int8 words per activation row: 8 per block + 4 pad per 8 blocks
    int da_row;  // fp32 scales per activation row (multiple of 4)
    int cbs;     // block-term stride per column
    __host__ __device__ Q8Lds(int blocks, bool fast) {
        aq_row = blocks * 8 + ((blocks + 7) / 8) * 4;
        da_row = (blocks + 3) & ~3;
        cbs = fast ? blocks + 4 : blocks + 1;
    }
    __host__ __device__ size_t words(int mr, int cpw) const {
        return static_cast<size_t>(mr) * (aq_row + da_row) + static_cast<size_t>(mr) * cpw * cbs;
    }
};

__device__ __forceinline__ int aq_index(int b, int j) { return b * 8 + (b >> 3) * 4 + j; }

// Block i (0..7) of a 272-byte unit held as 68 little-endian words: the fp16
// scale bits and the 8 words of int8 values.
template <int I>
__device__ __forceinline__ void unit_block(const uint32_t (&d)[kUnitWords], uint32_t &sbits, uint32_t (&qs)[8]) {
    if constexpr ((I & 1) == 0) {
        constexpr int k = 17 * I / 2;  // word-aligned block: scale, then values at +2 bytes
        sbits = d[k] & 0xFFFFu;
#pragma unroll
        for (int t = 0; t < 8; ++t) qs[t] = __builtin_amdgcn_alignbyte(d[k + t + 1], d[k + t], 2);
    } else {
        constexpr int k = (17 * I - 1) / 2;  // block at a half word: values word-aligned
        sbits = d[k] >> 16;
#pragma unroll
        for (int t = 0; t < 8; ++t) qs[t] = d[k + 1 + t];
    }
}

__device__ __forceinline__ int block_dot8(const uint32_t (&qs)[8], const int *aq) {
    const int4 a0 = *reinterpret_cast<const int4 *>(aq);
    const int4 a1 = *reinterpret_cast<const int4 *>(aq + 4);
    int s = 0;
    s = dot4(static_cast<int>(qs[0]), a0.x, s);
    s = dot4(static_cast<int>(qs[1]), a0.y, s);
    s = dot4(static_cast<int>(qs[2]), a0.z, s);
    s = dot4(static_cast<int>(qs[3]), a0.w, s);
    s = dot4(static_cast<int>(qs[4]), a1.x, s);
    s = dot4(static_cast<int>(qs[5]), a1.y, s);
    s = dot4(static_cast<int>(qs[6]), a1.z, s);
    s = dot4(static_cast<int>(qs[7]), a1.w, s);
    return s;
}

// c_b in the reference's order: activation scale, then weight scale.
__device__ __forceinline__ float block_term(int dot, float da, float dw) {
    float v = static_cast<float>(dot) * da;
    return v * dw;
}

template <int MR, bool FAST>
__global__ __launch_bounds__(kThreads) void q8_0_linear_kernel(Q8Task t) {
    extern __shared__ int lds[];
    const int col_base = blockIdx.x * t.cpw;
    const int r0 = blockIdx.y * MR;
    const int B = t.blocks;
    const Q8Lds geo(B, FAST);
    int *aq = lds;
    float *da = reinterpret_cast<float *>(aq + MR * geo.aq_row);
    float *cb = da + MR * geo.da_row;
    const int tile_cols = min(t.cpw, t.ncols - col_base);
    const int G = FAST ? (B >> 3) : B;
    const int units = tile_cols * G;

    uint32_t wr[FAST ? kUnitWords : 1];
    auto load_unit = [&](int u) {
        const int col = u / G;
        const int g = u - col * G;
        const v4u *src = reinterpret_cast<const v4u *>(
            t.w + static_cast<size_t>(t.wcol0 + col_base + col) * t.w_stride + static_cast<size_t>(g) * 272);
#pragma unroll
        for (int v = 0; v < 17; ++v) {
            const v4u x = src[v];
            wr[4 * v + 0] = x[0];
            wr[4 * v + 1] = x[1];
            wr[4 * v + 2] = x[2];
            wr[4 * v + 3] = x[3];
        }
    };
    if constexpr (FAST) {
        if (static_cast<int>(threadIdx.x) < units) load_unit(threadIdx.x);
    }

    // Stage the activation rows (rows past t.rows become zero blocks).
    for (int idx = threadIdx.x; idx < MR * B; idx += kThreads) {
        const int r = idx / B;
        const int b = idx - r * B;
        int words[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float d = 0.0f;
        if (r0 + r < t.rows) {
            const uint16_t *p = reinterpret_cast<const uint16_t *>(t.act + (r0 + r) * t.act_stride +
                                                                   static_cast<size_t>(b) * Q8_0_BYTES);
            d = half_bits_to_float(p[0]);
#pragma unroll
            for (int h = 0; h < 16; ++h) words[h >> 1] |= static_cast<int>(static_cast<uint32_t>(p[1 + h]) << (16 * (h & 1)));
        }
        int *dst = aq + r * geo.aq_row + aq_index(b, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[j] = words[j];
        da[r * geo.da_row + b] = d;
    }
    __syncthreads();

    if constexpr (FAST) {
        for (int first = 0; first < units; first += kThreads) {
            const int u = first + threadIdx.x;
            if (first > 0 && u < units) load_unit(u);
            if (u >= units) continue;
            const int col = u / G;
            const int g = u - col * G;
            float terms[MR][8];
            auto do_block = [&](auto ic) {
                constexpr int I = decltype(ic)::value;
                uint32_t sbits, qs[8];
                unit_block<I>(wr, sbits, qs);
                const float dw = half_bits_to_float(sbits);
                const int b = g * 8 + I;
#pragma unroll
                for (int r = 0; r < MR; ++r)
                    terms[r][I] = block_term(block_dot8(qs, aq + r * geo.aq_row + aq_index(b, 0)), da[r * geo.da_row + b], dw);
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
                float4 *c4 = reinterpret_cast<float4 *>(cb + (r * t.cpw + col) * geo.cbs + g * 8);
                c4[0] = make_float4(terms[r][0], terms[r][1], terms[r][2], terms[r][3]);
                c4[1] = make_float4(terms[r][4], terms[r][5], terms[r][6], terms[r][7]);
            }
        }
    } else {
        for (int u = threadIdx.x; u < units; u += kThreads) {
            const int col = u / B;
            const int b = u - col * B;
            const uint16_t *p = reinterpret_cast<const uint16_t *>(
                t.w + static_cast<size_t>(t.wcol0 + col_base + col) * t.w_stride + static_cast<size_t>(b) * Q8_0_BYTES);
            const float dw = half_bits_to_float(p[0]);
            uint32_t qs[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) qs[q] = static_cast<uint32_t>(p[1 + 2 * q]) | (static_cast<uint32_t>(p[2 + 2 * q]) << 16);
#pragma unroll
            for (int r = 0; r < MR; ++r)
                cb[(r * t.cpw + col) * geo.cbs + b] =
                    block_term(block_dot8(qs, aq + r * geo.aq_row + aq_index(b, 0)), da[r * geo.da_row + b], dw);
        }
    }
    __syncthreads();

    for (int k = threadIdx.x; k < MR * tile_cols; k += kThreads) {
        const int r = k / tile_cols;
        const int col = k - r * tile_cols;
        if (r0 + r >= t.rows) continue;
        const float *c = cb + (r * t.cpw + col) * geo.cbs;
        float acc = 0.0f;
        for (int b = 0; b < B; ++b) acc += c[b];
        float *out = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(t.y) + (r0 + r) * t.y_stride);
        out[t.ocol0 + col_base + col] = acc;
    }
}

// ------------------------------------------------ block-per-lane form
//
// Lane l of a wave takes block kw * 64 + l of its columns (kw: the wave's
// place along K; past 256 blocks also block kw * 64 + l + 256), so one load
// instruction of a wave reads 64 consecutive 34-byte blocks of one weight
// row (2,176 contiguous bytes) instead of 64 scattered 16-byte pieces of
// 272-byte units.  Each lane keeps its blocks of the MR activation rows in
// registers for the whole launch, the wave walks
// its columns with the next columns' loads in flight, and the block terms go
// to LDS for the same ordered sums as the unit form.  Blocks sit at 2-byte
// offsets: each is read as the aligned dwords around its 32 values (2 x 16
// bytes + the 2 bytes after them) and its scale, through buffer descriptors
// whose range turns blocks past K (or a missing row) into zeros.

constexpr uint32_t kOutOfRange = 0x80000000u;  // descriptor ranges are below 2 GiB
#ifndef QXT_Q8_AHEAD
#define QXT_Q8_AHEAD 2
#endif
#ifndef QXT_Q8_WGS
#define QXT_Q8_WGS 2
#endif
constexpr int kStreamAhead = QXT_Q8_AHEAD;  // columns of loads in flight per wave

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

struct Q8StreamTask {
    const uint8_t *act, *w;
    float *y;
    uint32_t act_stride, w_stride, act_extent, w_extent;
    size_t y_stride;
    int rows, blocks, wcol0, ocol0, ncols, cpw, wk;  // wk: waves along K (blocks <= 64 * wk)
};

// One block's raw words: 8 aligned dwords around the values, the 2 bytes
// after them, the scale bits and the byte shift (0 or 2) that realigns them.
struct RawBlock {
    uint32_t w[8];
    uint32_t tail, sbits, shift;
};

__device__ __forceinline__ void load_block(__amdgpu_buffer_rsrc_t r, uint32_t o, RawBlock &b) {
    const uint32_t v = (o + 2) & ~3u;  // the 32 values start 2 bytes into the block
    const v4u x0 = __builtin_amdgcn_raw_buffer_load_b128(r, v, 0, 0);
    const v4u x1 = __builtin_amdgcn_raw_buffer_load_b128(r, v + 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        b.w[i] = x0[i];
        b.w[4 + i] = x1[i];
    }
    // 16-bit loads for the 2 bytes past the values and for the scale: a
    // 32-bit load ending past the last block of a tensor would read as zero.
    b.tail = __builtin_amdgcn_raw_buffer_load_b16(r, v + 32, 0, 0);
    b.sbits = __builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0);
    b.shift = (o + 2) & 3u;
}

__device__ __forceinline__ void block_values(const RawBlock &b, uint32_t (&qs)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) qs[i] = __builtin_amdgcn_alignbyte(i < 7 ? b.w[i + 1] : b.tail, b.w[i], b.shift);
}

template <int MR, int C>
__global__ __launch_bounds__(kThreads) void q8_0_stream_kernel(Q8StreamTask t) {
    extern __shared__ int lds[];
    float *cb = reinterpret_cast<float *>(lds);  // [MR][cpw][cbs] block terms
    const int cbs = ((t.blocks + 3) & ~3) + 4;  // float4-aligned rows, padded
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kw = wave % t.wk, cg = wave / t.wk, groups = (kThreads / 64) / t.wk;
    // Blocks b[c] = kw * 64 + lane + c * 64 * wk: C blocks of each column per lane.
    int b[C];
    bool in_k[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        b[c] = kw * 64 + lane + c * 64 * t.wk;
        in_k[c] = b[c] < t.blocks;
    }
    const int col_base = blockIdx.x * t.cpw;
    const int r0 = blockIdx.y * MR;
    const int tile_cols = min(t.cpw, t.ncols - col_base);
    const __amdgpu_buffer_rsrc_t ra = rsrc(t.act, t.act_extent);
    const __amdgpu_buffer_rsrc_t rw = rsrc(t.w, t.w_extent);

    auto w_offset = [&](int col, int c) -> uint32_t {
        return in_k[c] && col < tile_cols
                   ? static_cast<uint32_t>(t.wcol0 + col_base + col) * t.w_stride + static_cast<uint32_t>(b[c]) * 34u
                   : kOutOfRange;
    };
    // The first columns' weights are requested before the activation.
    RawBlock ring[kStreamAhead][C];
#pragma unroll
    for (int j = 0; j < kStreamAhead; ++j)
#pragma unroll
        for (int c = 0; c < C; ++c) load_block(rw, w_offset(cg + j * groups, c), ring[j][c]);

    uint32_t a[C][MR][8];
    float da[C][MR];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            RawBlock ab;
            load_block(ra, in_k[c] && r0 + r < t.rows
                               ? static_cast<uint32_t>(r0 + r) * t.act_stride + static_cast<uint32_t>(b[c]) * 34u
                               : kOutOfRange,
                       ab);
            block_values(ab, a[c][r]);
            da[c][r] = half_bits_to_float(ab.sbits);
        }

    // Columns cg, cg + groups, ... of the tile; slot j of the ring holds the
    // column of step s with s % kStreamAhead == j.
    const int steps = (tile_cols - cg + groups - 1) / groups;
    for (int s0 = 0; s0 < steps; s0 += kStreamAhead) {
#pragma unroll
        for (int j = 0; j < kStreamAhead; ++j) {
            const int s = s0 + j;
            if (s >= steps) break;
            const int col = cg + s * groups;
#pragma unroll
            for (int c = 0; c < C; ++c) {
                uint32_t qs[8];
                block_values(ring[j][c], qs);
                const float dw = half_bits_to_float(ring[j][c].sbits);
                load_block(rw, w_offset(col + kStreamAhead * groups, c), ring[j][c]);
                if (in_k[c]) {
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        int dot = 0;
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            dot = dot4(static_cast<int>(qs[i]), static_cast<int>(a[c][r][i]), dot);
                        cb[(r * t.cpw + col) * cbs + b[c]] = block_term(dot, da[c][r], dw);
                    }
                }
            }
        }
    }
    __syncthreads();

    // One thread per (row, column): the column's block terms in block order.
    for (int k = threadIdx.x; k < MR * tile_cols; k += kThreads) {
        const int r = k / tile_cols;
        const int col = k - r * tile_cols;
        if (r0 + r >= t.rows) continue;
        const float *c = cb + (r * t.cpw + col) * cbs;
        float acc = 0.0f;
        int i = 0;
        for (; i + 4 <= t.blocks; i += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(c + i);
            acc += v.x;
            acc += v.y;
            acc += v.z;
            acc += v.w;
        }
        for (; i < t.blocks; ++i) acc += c[i];
        float *out = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(t.y) + (r0 + r) * t.y_stride);
        out[t.ocol0 + col_base + col] = acc;
    }
}

template <int MR>
int launch_q8(Q8Task t, hipStream_t stream) {
    const bool fast = t.blocks % 8 == 0 && aligned(t.w, 16) && t.w_stride % 16 == 0;
    const Q8Lds geo(t.blocks, fast);
    const int row_groups = (t.rows + MR - 1) / MR;
    // Enough workgroups for two per CU, each at most one round of units.
    const long want = 2L * compute_units();
    const int max_cpw = static_cast<int>(std::max<long>(1, (static_cast<long>(t.ncols) * row_groups + want - 1) / want));
    const int per_col = fast ? t.blocks / 8 : t.blocks;
    int cpw = fast ? std::max(1, kThreads / std::max(1, per_col)) : std::max(1, kThreads / per_col);
    cpw = std::max(1, std::min({cpw, t.ncols, max_cpw}));
    while (cpw > 1 && geo.words(MR, cpw) * 4 > kMaxLds) --cpw;
    const size_t lds = geo.words(MR, cpw) * 4;
    if (lds > kMaxLds)
        return fail(QXT_CAPABILITY_MISSING, "q8_0 linear: K=%d needs %zu bytes of LDS (> %zu)", t.blocks * 32, lds,
                    kMaxLds);
    t.cpw = cpw;
    dim3 grid((t.ncols + cpw - 1) / cpw, row_groups, 1);
    if (fast) return launch("q8_0_linear_kernel", q8_0_linear_kernel<MR, true>, grid, dim3(kThreads), lds, stream, t);
    return launch("q8_0_linear_kernel", q8_0_linear_kernel<MR, false>, grid, dim3(kThreads), lds, stream, t);
}

// The block-per-lane form for K <= 512 blocks (16384 values; beyond 256
// blocks each lane takes two) with operands below 2 GiB;
// QXT_CAPABILITY_MISSING otherwise (the caller then takes the unit form).
template <int MR>
int launch_q8_stream(const Q8Task &u, hipStream_t stream) {
    if (u.blocks > 512) return QXT_CAPABILITY_MISSING;
    const uint64_t a_extent = static_cast<uint64_t>(u.rows - 1) * u.act_stride + static_cast<uint64_t>(u.blocks) * 34;
    const uint64_t w_extent =
        static_cast<uint64_t>(u.wcol0 + u.ncols - 1) * u.w_stride + static_cast<uint64_t>(u.blocks) * 34;
    if (a_extent >= (1ull << 31) || w_extent >= (1ull << 31)) return QXT_CAPABILITY_MISSING;
    Q8StreamTask t{};
    t.act = u.act;
    t.w = u.w;
    t.y = u.y;
    t.act_stride = static_cast<uint32_t>(u.act_stride);
    t.w_stride = static_cast<uint32_t>(u.w_stride);
    t.act_extent = static_cast<uint32_t>(a_extent);
    t.w_extent = static_cast<uint32_t>(w_extent);
    t.y_stride = u.y_stride;
    t.rows = u.rows;
    t.blocks = u.blocks;
    t.wcol0 = u.wcol0;
    t.ocol0 = u.ocol0;
    t.ncols = u.ncols;
    t.wk = u.blocks <= 64 ? 1 : u.blocks <= 128 ? 2 : 4;  // beyond 256 blocks: 2 per lane
    const int groups = (kThreads / 64) / t.wk;
    const int row_groups = (u.rows + MR - 1) / MR;
    // Two workgroups per CU, whole column groups per workgroup.
    const long want = static_cast<long>(QXT_Q8_WGS) * compute_units();
    int cpw = static_cast<int>((static_cast<long>(u.ncols) * row_groups + want - 1) / want);
    cpw = std::min(64, std::max(groups, (cpw + groups - 1) / groups * groups));
    const int cbs = ((u.blocks + 3) & ~3) + 4;
    // At most kMaxLds of block terms (whole column groups).
    const int lds_cols = static_cast<int>(kMaxLds / (static_cast<size_t>(MR) * cbs * 4)) / groups * groups;
    if (lds_cols < groups) return QXT_CAPABILITY_MISSING;
    cpw = std::min(cpw, lds_cols);
    const size_t lds = static_cast<size_t>(MR) * cpw * cbs * 4;
    t.cpw = cpw;
    const dim3 grid((u.ncols + cpw - 1) / cpw, row_groups, 1);
    if (u.blocks > 256)
        return launch("q8_0_linear_kernel", q8_0_stream_kernel<MR, 2>, grid, dim3(kThreads), lds, stream, t);
    return launch("q8_0_linear_kernel", q8_0_stream_kernel<MR, 1>, grid, dim3(kThreads), lds, stream, t);
}

template <int MR>
int dispatch_q8(const Q8Task &t, hipStream_t stream) {
#ifndef QXT_Q8_STREAM
#define QXT_Q8_STREAM 1
#endif
    if (QXT_Q8_STREAM) {
        const int rc = launch_q8_stream<MR>(t, stream);
        if (rc != QXT_CAPABILITY_MISSING) return rc;
    }
    return launch_q8<MR>(t, stream);
}

}  // namespace
}  // namespace qxt

using namespace qxt;

extern "C" int qxt_ggml_q8_0_q8_0_linear(const void *activation, size_t activation_row_stride, const void *weight,
                                         size_t weight_row_stride, float *destination, size_t destination_row_stride,
                                         uint32_t rows, uint32_t blocks, uint32_t weight_column_start,
                                         uint32_t output_column_start, uint32_t column_count, void *stream) {
    if (activation == nullptr || weight == nullptr || destination == nullptr)
        return fail(QXT_INVALID_ARGUMENT, "q8_0 linear: null pointer");
    if (rows == 0 || blocks == 0 || column_count == 0)
        return fail(QXT_INVALID_ARGUMENT, "q8_0 linear: rows, blocks and column_count must be positive");
    if (rows > 65535u * 4u || blocks > (1u << 20) || column_count > (1u << 30))
        return fail(QXT_INVALID_ARGUMENT, "q8_0 linear: problem too large");
    if (activation_row_stride < static_cast<size_t>(blocks) * Q8_0_BYTES || activation_row_stride % 2 ||
        weight_row_stride < static_cast<size_t>(blocks) * Q8_0_BYTES || weight_row_stride % 2 ||
        !aligned(activation, 2) || !aligned(weight, 2))
        return fail(QXT_INVALID_ARGUMENT, "q8_0 linear: bad strides or alignment");
    if (!aligned(destination, 4) || destination_row_stride % 4 ||
        destination_row_stride < (static_cast<size_t>(output_column_start) + column_count) * sizeof(float))
        return fail(QXT_INVALID_ARGUMENT, "q8_0 linear: bad destination");
    if (static_cast<uint64_t>(weight_column_start) + column_count > (1ull << 31) ||
        static_cast<uint64_t>(output_column_start) + column_count > (1ull << 31))
        return fail(QXT_INVALID_ARGUMENT, "q8_0 linear: column range overflows");
    int rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    Q8Task t{};
    t.act = static_cast<const uint8_t *>(activation);
    t.act_stride = activation_row_stride;
    t.w = static_cast<const uint8_t *>(weight);
    t.w_stride = weight_row_stride;
    t.y = destination;
    t.y_stride = destination_row_stride;
    t.rows = static_cast<int>(rows);
    t.blocks = static_cast<int>(blocks);
    t.wcol0 = static_cast<int>(weight_column_start);
    t.ocol0 = static_cast<int>(output_column_start);
    t.ncols = static_cast<int>(column_count);
    const hipStream_t s = as_stream(stream);
    switch (rows >= 4 ? 4 : rows) {
        case 1: return dispatch_q8<1>(t, s);
        case 2: return dispatch_q8<2>(t, s);
        case 3: return dispatch_q8<3>(t, s);
        default: return dispatch_q8<4>(t, s);
    }
}

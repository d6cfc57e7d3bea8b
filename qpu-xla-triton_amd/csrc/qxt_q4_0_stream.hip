// Q4_0 x Q8_0 linear over native ggml weight rows, one or more blocks per
// lane (small M, long K).
//
// Arithmetic (reference src/qpu_xla/kernels/ggml_q4_0.py:81-100): per
// 32-element block an exact int32 dot of the signed codes (nibble - 8) with
// the int8 activation, then c_b = fl32(fl32(float(dot_b) * dw_b) * da_b),
// summed in block order -- the oracle's result bit for bit.
//
// Lane l of a wave takes blocks kw * 64 + l + c * 64 * wk (c < C; kw: the
// wave's place along K, wk: waves along K) of its columns, so one load
// instruction of a wave reads 64 consecutive 18-byte blocks of one weight row
// (1,152 contiguous bytes).  The lane keeps its blocks of the MR activation
// rows in registers for the whole launch, together with -8 * sum(a) of each,
// the start of its dot: the nibbles then enter v_dot4 as unsigned codes
// 0..15 and the chain ends at the exact signed dot.  The wave walks its
// columns with the next columns' loads in flight; block terms go to LDS and
// one thread per (row, column) adds them in block order.  Blocks sit at
// 2-byte offsets: each is read as the aligned dwords around its bytes through
// buffer descriptors whose range turns blocks past K (or a missing row) into
// zeros.
#include <algorithm>

#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;
constexpr size_t kMaxLds = 64 * 1024;
constexpr uint32_t kOutOfRange = 0x80000000u;  // descriptor ranges are below 2 GiB
// Columns of loads in flight per wave (measured on MI355X: three against two
// M=2 K=4096 N=11008 9.7 -> 9.0 us, M=4 9.7 -> 9.6 us, equal within 0.2 us
// at the longer rows; four no better).
constexpr int kAhead = 3;

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

struct Q4StreamTask {
    const uint8_t *act, *w;
    float *y;
    uint32_t act_stride, w_stride, act_extent, w_extent;
    size_t y_stride;
    int rows, blocks, wcol0, ocol0, ncols, cpw, wk;  // wk: waves along K
};

// A Q4_0 block's raw words: the 4 aligned dwords around its 16 nibble bytes,
// the 2 bytes after them, the scale bits and the byte shift (0 or 2).
struct RawQ4 {
    uint32_t w[4];
    uint32_t tail, sbits, shift;
};

__device__ __forceinline__ void load_q4(__amdgpu_buffer_rsrc_t r, uint32_t o, RawQ4 &b) {
    const uint32_t v = (o + 2) & ~3u;  // the nibbles start 2 bytes into the block
    const v4u x = __builtin_amdgcn_raw_buffer_load_b128(r, v, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) b.w[i] = x[i];
    // 16-bit loads for the 2 bytes past the 16 and for the scale: a 32-bit
    // load ending past the last block of a tensor would read as zero.
    b.tail = __builtin_amdgcn_raw_buffer_load_b16(r, v + 16, 0, 0);
    b.sbits = __builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0);
    b.shift = (o + 2) & 3u;
}

// A Q8_0 activation block: its 8 value words in k order and its scale.
__device__ __forceinline__ void load_q8(__amdgpu_buffer_rsrc_t r, uint32_t o, uint32_t (&qs)[8], float &d) {
    const uint32_t v = (o + 2) & ~3u;
    const v4u x0 = __builtin_amdgcn_raw_buffer_load_b128(r, v, 0, 0);
    const v4u x1 = __builtin_amdgcn_raw_buffer_load_b128(r, v + 16, 0, 0);
    const uint32_t tail = __builtin_amdgcn_raw_buffer_load_b16(r, v + 32, 0, 0);
    const uint32_t sbits = __builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0);
    const uint32_t shift = (o + 2) & 3u;
    const uint32_t w[9] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3], tail};
#pragma unroll
    for (int i = 0; i < 8; ++i) qs[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], shift);
    d = half_bits_to_float(sbits);
}

template <int MR, int C>
__global__ __launch_bounds__(kThreads) void q4_0_stream_kernel(Q4StreamTask t) {
    extern __shared__ int lds[];
    float *cb = reinterpret_cast<float *>(lds);  // [MR][cpw][cbs] block terms
    const int cbs = ((t.blocks + 3) & ~3) + 4;   // float4-aligned rows, padded
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kw = wave % t.wk, cg = wave / t.wk, groups = (kThreads / 64) / t.wk;
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
                   ? static_cast<uint32_t>(t.wcol0 + col_base + col) * t.w_stride + static_cast<uint32_t>(b[c]) * 18u
                   : kOutOfRange;
    };
    // The first columns' weights are requested before the activation.
    RawQ4 ring[kAhead][C];
#pragma unroll
    for (int j = 0; j < kAhead; ++j)
#pragma unroll
        for (int c = 0; c < C; ++c) load_q4(rw, w_offset(cg + j * groups, c), ring[j][c]);

    uint32_t a[C][MR][8];
    float da[C][MR];
    int dot0[C][MR];  // -8 * sum of the block's activation values
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            load_q8(ra,
                    in_k[c] && r0 + r < t.rows
                        ? static_cast<uint32_t>(r0 + r) * t.act_stride + static_cast<uint32_t>(b[c]) * 34u
                        : kOutOfRange,
                    a[c][r], da[c][r]);
            int sum = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) sum = dot4(static_cast<int>(a[c][r][i]), 0x01010101, sum);
            dot0[c][r] = -8 * sum;
        }

    // Columns cg, cg + groups, ... of the tile; slot j of the ring holds the
    // column of step s with s % kAhead == j.
    const int steps = (tile_cols - cg + groups - 1) / groups;
    for (int s0 = 0; s0 < steps; s0 += kAhead) {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
            const int s = s0 + j;
            if (s >= steps) break;
            const int col = cg + s * groups;
#pragma unroll
            for (int c = 0; c < C; ++c) {
                // Byte i of the nibbles holds element i (low) and i + 16 (high).
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t nib = __builtin_amdgcn_alignbyte(i < 3 ? ring[j][c].w[i + 1] : ring[j][c].tail,
                                                                    ring[j][c].w[i], ring[j][c].shift);
                    lo[i] = nib & 0x0F0F0F0Fu;
                    hi[i] = (nib >> 4) & 0x0F0F0F0Fu;
                }
                const float dw = half_bits_to_float(ring[j][c].sbits);
                load_q4(rw, w_offset(col + kAhead * groups, c), ring[j][c]);
                if (in_k[c]) {
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        int dot = dot0[c][r];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            dot = dot4(static_cast<int>(lo[i]), static_cast<int>(a[c][r][i]), dot);
                            dot = dot4(static_cast<int>(hi[i]), static_cast<int>(a[c][r][4 + i]), dot);
                        }
                        float v = static_cast<float>(dot) * dw;
                        v = v * da[c][r];
                        cb[(r * t.cpw + col) * cbs + b[c]] = v;
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
        const float *cc = cb + (r * t.cpw + col) * cbs;
        float acc = 0.0f;
        int i = 0;
        for (; i + 4 <= t.blocks; i += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(cc + i);
            acc += v.x;
            acc += v.y;
            acc += v.z;
            acc += v.w;
        }
        for (; i < t.blocks; ++i) acc += cc[i];
        float *out = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(t.y) + (r0 + r) * t.y_stride);
        out[t.ocol0 + col_base + col] = acc;
    }
}

template <int MR>
int launch_stream(Q4StreamTask t, hipStream_t stream) {
    t.wk = t.blocks <= 64 ? 1 : t.blocks <= 128 ? 2 : 4;
    const int groups = (kThreads / 64) / t.wk;
    const int row_groups = (t.rows + MR - 1) / MR;
    // Two workgroups per CU, whole column groups per workgroup, at most
    // kMaxLds of block terms.
    const long want = 2L * compute_units();
    int cpw = static_cast<int>((static_cast<long>(t.ncols) * row_groups + want - 1) / want);
    cpw = std::min(64, std::max(groups, (cpw + groups - 1) / groups * groups));
    const int cbs = ((t.blocks + 3) & ~3) + 4;
    const int lds_cols = static_cast<int>(kMaxLds / (static_cast<size_t>(MR) * cbs * 4)) / groups * groups;
    if (lds_cols < groups) return QXT_CAPABILITY_MISSING;
    cpw = std::min(cpw, lds_cols);
    const size_t lds = static_cast<size_t>(MR) * cpw * cbs * 4;
    t.cpw = cpw;
    const dim3 grid((t.ncols + cpw - 1) / cpw, row_groups, 1);
    const int chunks = (t.blocks + 255) / 256;
    switch (chunks) {
        case 1: return launch("q4_0_linear_kernel", q4_0_stream_kernel<MR, 1>, grid, dim3(kThreads), lds, stream, t);
        case 2: return launch("q4_0_linear_kernel", q4_0_stream_kernel<MR, 2>, grid, dim3(kThreads), lds, stream, t);
        default: return launch("q4_0_linear_kernel", q4_0_stream_kernel<MR, 3>, grid, dim3(kThreads), lds, stream, t);
    }
}

}  // namespace

int q4_0_stream_native(const void *activation, size_t activation_row_stride, const void *weight,
                       size_t weight_row_stride, float *destination, size_t destination_row_stride, uint32_t rows,
                       uint32_t blocks, uint32_t weight_column_start, uint32_t output_column_start,
                       uint32_t column_count, hipStream_t stream) {
    if (rows == 0 || rows > 15 || blocks == 0 || blocks > 768 || column_count == 0) return QXT_CAPABILITY_MISSING;
    const uint64_t a_extent = static_cast<uint64_t>(rows - 1) * activation_row_stride + static_cast<uint64_t>(blocks) * 34;
    const uint64_t w_extent = static_cast<uint64_t>(weight_column_start + column_count - 1) * weight_row_stride +
                              static_cast<uint64_t>(blocks) * 18;
    if (a_extent >= (1ull << 31) || w_extent >= (1ull << 31) || activation_row_stride % 2 || weight_row_stride % 2 ||
        !aligned(activation, 2) || !aligned(weight, 2))
        return QXT_CAPABILITY_MISSING;
    Q4StreamTask t{};
    t.act = static_cast<const uint8_t *>(activation);
    t.w = static_cast<const uint8_t *>(weight);
    t.y = destination;
    t.act_stride = static_cast<uint32_t>(activation_row_stride);
    t.w_stride = static_cast<uint32_t>(weight_row_stride);
    t.act_extent = static_cast<uint32_t>(a_extent);
    t.w_extent = static_cast<uint32_t>(w_extent);
    t.y_stride = destination_row_stride;
    t.rows = static_cast<int>(rows);
    t.blocks = static_cast<int>(blocks);
    t.wcol0 = static_cast<int>(weight_column_start);
    t.ocol0 = static_cast<int>(output_column_start);
    t.ncols = static_cast<int>(column_count);
    switch (rows >= 4 ? 4 : rows) {
        case 1: return launch_stream<1>(t, stream);
        case 2: return launch_stream<2>(t, stream);
        case 3: return launch_stream<3>(t, stream);
        default: return launch_stream<4>(t, stream);
    }
}

}  // namespace qxt

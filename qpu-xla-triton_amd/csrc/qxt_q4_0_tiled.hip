// Q4_0 x Q8_0 prefill linear (M >= 16) on the int8 matrix cores of gfx950.
//
// Arithmetic is that of the reference oracle ggml_q4_0_q8_0_reference
// (src/qpu_xla/kernels/ggml_q4_0.py:81-100): per 32-element block an exact
// int32 dot, then c_b = fl32(fl32(float(dot_b) * dw_b) * da_b), summed in
// block order.  One v_mfma_i32_32x32x32_i8 computes the exact block dots of
// a 32 x 32 output tile for one block (K = 32 = one GGML block), and the
// lane that receives each dot applies that block's two scales and adds the
// term to its fp32 accumulator before the next block's dots arrive, so the
// result is bit-identical to the oracle.  (The reference's own tiled QPU
// program, ggml_q4_0.py:309-547, multiplies by the activation scale first
// and is checked against the oracle within rtol 2e-6; this kernel matches
// the oracle exactly.)
//
// The VALU operations per output and block (convert, two multiplies, add)
// are the kernels' floor, not the matrix core: one 32 x 32 x 32 MFMA per wave
// per block feeds the scaling of 16 outputs per lane.  Where registers allow
// (the split planes, and the staged kernel's small grids), the MFMA's
// accumulator input is a bias that makes the convert and the first multiply
// one fma (see kDotBiasBits): three instructions per output and block.  A 256-thread workgroup owns a
// 64 x 64 output tile (four waves of 32 x 32), and the dots of the next block
// are computed before the current block's are scaled.  Two operand layouts,
// two ways of feeding the matrix core:
//   * split planes (the reference's GGML_Q4_0_Q8_0_TILED_LINEAR_KERNEL
//     contract, ggml_q4_0.py:844-967): activation int8 [M, K] + fp16 scales
//     [M, B] (2-byte halves or 4-byte words), weight uint32 [B * 8, N] of
//     signed int8 quads (pack_ggml_q4_0_tiled_weights) + fp16 scales [B, N].
//     Aligned fragments are loaded by each lane directly, four blocks ahead;
//     scales are staged in LDS 32 blocks at a time (double-buffered).
//   * native 34-byte Q8_0 / 18-byte Q4_0 blocks (the linear's own layout):
//     the workgroup stages 8 blocks of its rows and columns at a time in LDS,
//     realigned and with the weight nibbles already converted to int8.
#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 64;   // output rows and columns per workgroup
constexpr int kChunk = 32;  // blocks of scales staged per LDS round

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr uint32_t kOutOfRange = 0x80000000u;  // operands are < 2 GiB: always out of range

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

struct TiledArgs {
    // split layout
    const uint8_t *aq;   // int8 [M, K]
    const uint8_t *as;   // fp16 scales [M, B] as 2- or 4-byte elements
    const uint8_t *wq;   // uint32 [B * 8, N]
    const uint8_t *ws;   // fp16 scales [B, N]
    const float *cs;     // fp32 column scales [N] (column-scale variant, ws unused)
    // native layout
    const uint8_t *act;  // Q8_0 [M, B, 34]
    const uint8_t *w;    // Q4_0 [>= wcol0 + N, B, 18]
    float *y;
    uint32_t aq_stride, as_stride, as_bytes, wq_stride, ws_stride, act_stride, w_stride;
    size_t y_stride;
    uint32_t a_extent, w_extent, as_extent, ws_extent;  // buffer-descriptor ranges
    int m, n, blocks, wcol0, ocol0;
};

// ------------------------------------------------- split planes, direct
//
// The split layout's fragments are 16-byte aligned: each lane loads its own
// straight into registers.  A = 16 activation bytes of row `am` (k half h);
// W = the 4 packed words of column `bn` for k half h (4 word rows, each
// contiguous over the columns of a wave).

struct RawFrags {
    v4u a, w;
};

// Per-lane byte offsets of this lane's fragments at block 0.  Lanes outside
// the matrix start at the end of the descriptor's range, so all their loads
// return zeros.
struct FragBase {
    uint32_t a, w;
};

__device__ __forceinline__ FragBase frag_base(const TiledArgs &t, int am, int bn, bool a_ok, bool b_ok, int h) {
    FragBase f;
    f.a = a_ok ? static_cast<uint32_t>(am) * t.aq_stride + 16 * h : t.a_extent;
    f.w = b_ok ? static_cast<uint32_t>(4 * h) * t.wq_stride + bn * 4 : t.w_extent;
    return f;
}

__device__ __forceinline__ void issue_frags(const TiledArgs &t, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rw,
                                            const FragBase &base, int b, RawFrags &f) {
    // Blocks past K add 2 GiB to every offset (the block index is uniform, so
    // this is one scalar select): out of range, zeros, no memory traffic, and
    // no wrap past 2^32 since every base is below 2 GiB.
    const bool in_k = b < t.blocks;
    f.a = __builtin_amdgcn_raw_buffer_load_b128(ra, base.a + (in_k ? static_cast<uint32_t>(b) * 32u : kOutOfRange), 0,
                                                0);
    const uint32_t wrow = in_k ? static_cast<uint32_t>(b) * 8u * t.wq_stride : kOutOfRange;
#pragma unroll
    for (int i = 0; i < 4; ++i) f.w[i] = __builtin_amdgcn_raw_buffer_load_b32(rw, base.w + wrow + i * t.wq_stride, 0, 0);
}

__device__ __forceinline__ void frags_of(const RawFrags &f, v4i &a, v4i &w) {
    a = v4i{static_cast<int>(f.a[0]), static_cast<int>(f.a[1]), static_cast<int>(f.a[2]), static_cast<int>(f.a[3])};
    w = v4i{static_cast<int>(f.w[0]), static_cast<int>(f.w[1]), static_cast<int>(f.w[2]), static_cast<int>(f.w[3])};
}

constexpr int kAhead = 4;  // blocks of fragments in flight ahead of the one being reduced
static_assert(kAhead % 2 == 0 && kChunk % kAhead == 0, "block parity must be static in the unrolled loop");

// Biased block dots.  The MFMA's accumulator input is the bit pattern of
// 1.5 * 2^23 in every output, so an output's bits are those of the float
// f = 1.5 * 2^23 + dot (|dot| <= 32 * 128 * 128 = 2^19 < 2^22 keeps it among
// that binade's integers).  Then fl32(float(dot) * dw) = fma(f, dw, c) with
// c = -1.5 * 2^23 * dw, exactly: c is exact (dw is an fp16 value, 11
// significant bits) and the fma rounds f * dw + c = dot * dw once.  For
// dot * dw = 0 the fma gives +0 where the product may be -0; the accumulator
// starts at +0 and so never holds -0, and adding either zero leaves it
// unchanged.  An infinite or NaN dw makes c non-finite, so the kernels note
// every non-finite weight scale they stage, and a workgroup that staged one
// computes its tile again with exact_terms_split / exact_terms_native.
constexpr int kDotBiasBits = 0x4B400000;
constexpr float kDotBias = 12582912.0f;

__device__ __forceinline__ v16i dot_bias() {
    v16i v;
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = kDotBiasBits;
    return v;
}

__device__ __forceinline__ bool half_bits_finite(uint32_t bits16) { return (bits16 & 0x7C00u) != 0x7C00u; }

// Row of output r (0..15) of a lane: the 32 x 32 MFMA's output layout.
__device__ __forceinline__ int out_row(int mbase, int r) { return mbase + 8 * (r >> 2) + (r & 3); }

// The exact per-block form, c_b = fl32(fl32(float(dot) * dw) * da) summed in
// block order, for one lane's 16 outputs (rows out_row(mbase, r), column bn),
// straight from the split planes in global memory (v_dot4 per 4 k), one
// output at a time so that it needs few registers.  Only for workgroups
// whose weight scales are not all finite.
__device__ __forceinline__ void exact_terms_split(const TiledArgs &t, int mbase, int bn, float (&acc)[16]) {
    const __amdgpu_buffer_rsrc_t ra = rsrc(t.aq, t.a_extent);
    const __amdgpu_buffer_rsrc_t rw = rsrc(t.wq, t.w_extent);
    const __amdgpu_buffer_rsrc_t ras = rsrc(t.as, t.as_extent);
    const __amdgpu_buffer_rsrc_t rws = rsrc(t.ws, t.ws_extent);
    const bool n_ok = bn < t.n;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = out_row(mbase, r);
        const bool m_ok = m < t.m;
        float sum = 0.0f;
#pragma unroll 1
        for (int b = 0; b < t.blocks; ++b) {
            const uint32_t ao = m_ok ? static_cast<uint32_t>(m) * t.aq_stride + b * 32 : kOutOfRange;
            const uint32_t wo = n_ok ? static_cast<uint32_t>(b * 8) * t.wq_stride + bn * 4 : kOutOfRange;
            int dot = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                dot = dot4(static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(ra, ao + 4 * j, 0, 0)),
                           static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(rw, wo + j * t.wq_stride, 0, 0)), dot);
            const float dw = half_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(
                rws, n_ok ? static_cast<uint32_t>(b) * t.ws_stride + bn * 2 : kOutOfRange, 0, 0));
            const float da = half_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(
                ras, m_ok ? static_cast<uint32_t>(m) * t.as_stride + b * t.as_bytes : kOutOfRange, 0, 0));
            sum = sum + (static_cast<float>(dot) * dw) * da;
        }
        acc[r] = sum;
    }
}

// The same from native 34-byte Q8_0 / 18-byte Q4_0 blocks (2-byte aligned:
// 16-bit loads).  Byte j of a Q4_0 block's nibbles holds element j (low) and
// j + 16 (high), each minus 8.
__device__ __forceinline__ void exact_terms_native(const TiledArgs &t, int mbase, int bn, float (&acc)[16]) {
    const __amdgpu_buffer_rsrc_t ra = rsrc(t.act, t.a_extent);
    const __amdgpu_buffer_rsrc_t rw = rsrc(t.w, t.w_extent);
    const bool n_ok = bn < t.n;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = out_row(mbase, r);
        const bool m_ok = m < t.m;
        float sum = 0.0f;
#pragma unroll 1
        for (int b = 0; b < t.blocks; ++b) {
            const uint32_t wo = n_ok ? static_cast<uint32_t>(t.wcol0 + bn) * t.w_stride + b * 18u : kOutOfRange;
            const uint32_t ao = m_ok ? static_cast<uint32_t>(m) * t.act_stride + b * 34u : kOutOfRange;
            int dot = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t nib = __builtin_amdgcn_raw_buffer_load_b16(rw, wo + 2 + 2 * j, 0, 0);
                const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(ra, ao + 2 + 2 * j, 0, 0);   // k = 2j, 2j+1
                const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(ra, ao + 18 + 2 * j, 0, 0);  // k = 2j+16, 2j+17
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t byte = (nib >> (8 * e)) & 0xFFu;
                    dot += static_cast<int8_t>(lo >> (8 * e)) * (static_cast<int>(byte & 0xFu) - 8);
                    dot += static_cast<int8_t>(hi >> (8 * e)) * (static_cast<int>(byte >> 4) - 8);
                }
            }
            const float dw = half_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(rw, wo, 0, 0));
            const float da = half_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(ra, ao, 0, 0));
            sum = sum + (static_cast<float>(dot) * dw) * da;
        }
        acc[r] = sum;
    }
}

// COLUMN: the column-scale variant (the llama.cpp bridge's COLUMN_W8 weight
// mode): int8 weights with one fp32 scale per column instead of fp16 block
// scales; each block adds fl32(float(dot) * da) and the column scale
// multiplies the finished sum once (ggml_q4_0.py:497-525).
// The block-scale form needs more than 168 registers either way, so it is
// compiled for at most two waves per SIMD: left to itself the scheduler kept
// one 16-register dot buffer and scaled each block right after its MFMA,
// waiting on the matrix core (M = 512 down projection 45.9 us against 42.8 us
// with the dots of the next block in flight).
template <bool COLUMN>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, COLUMN ? 8 : 2))) void q4_0_tiled_kernel(
    TiledArgs t) {
    // Scales of two chunks: the one being reduced and the next, written
    // while the current one is reduced (one barrier per chunk).
    __shared__ __attribute__((aligned(16))) float s_da[2][kChunk][kTile];
    __shared__ __attribute__((aligned(16))) float s_dw[2][kChunk][kTile];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
    const int h = lane >> 5, l32 = lane & 31;
    const int am = m0 + wm * 32 + l32;  // row of this lane's A fragment
    const int bn = n0 + wn * 32 + l32;  // column of this lane's B fragment (and of its outputs)
    const bool a_ok = am < t.m, b_ok = bn < t.n;

    const __amdgpu_buffer_rsrc_t ra = rsrc(t.aq, t.a_extent);
    const __amdgpu_buffer_rsrc_t rw = rsrc(t.wq, t.w_extent);
    const __amdgpu_buffer_rsrc_t ras = rsrc(t.as, t.as_extent);
    const __amdgpu_buffer_rsrc_t rws = rsrc(t.ws, t.ws_extent);
    const FragBase base = frag_base(t, am, bn, a_ok, b_ok, h);

    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    // Biased dots for the block-scale form; the column-scale form has no dw
    // and converts plain dots.
    const v16i cin = COLUMN ? v16i{} : dot_bias();
    bool finite = true;  // every weight scale this thread staged

    // Ring of fragment registers: slot j holds block b with b % kAhead == j.
    // The dots of block b + 1 are computed (`next`) before block b's dots are
    // scaled, so the matrix core's latency overlaps the scaling of the
    // previous block.
    RawFrags ring[kAhead];
#pragma unroll
    for (int j = 0; j < kAhead; ++j) issue_frags(t, ra, rw, base, j, ring[j]);
    // dots[b & 1] holds the dots of block b (kAhead and kChunk are even, so
    // the parity is known at compile time inside the unrolled groups).
    v16i dots[2];
    {
        v4i af, wf;
        frags_of(ring[0], af, wf);
        dots[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, wf, cin, 0, 0, 0);
        issue_frags(t, ra, rw, base, kAhead, ring[0]);
    }

    // Scales of blocks c0 .. c0 + kChunk - 1 for the tile's rows and columns
    // (zeros past M, N or K through out-of-range offsets): loaded into
    // registers a chunk ahead, written to LDS after the current chunk.
    constexpr int kPer = kChunk * kTile / kThreads;
    uint32_t da_bits[kPer], dw_bits[kPer];
    auto load_scales = [&](int c0) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = threadIdx.x + u * kThreads;
            const int cb = i / kTile, r = i - cb * kTile, b = c0 + cb;
            const int m = m0 + r, n = n0 + r;
            const bool in_k = b < t.blocks;
            const uint32_t ao = in_k && m < t.m ? static_cast<uint32_t>(m) * t.as_stride + b * t.as_bytes : kOutOfRange;
            const uint32_t wo = in_k && n < t.n ? static_cast<uint32_t>(b) * t.ws_stride + n * 2 : kOutOfRange;
            da_bits[u] = __builtin_amdgcn_raw_buffer_load_b16(ras, ao, 0, 0);
            if constexpr (!COLUMN) dw_bits[u] = __builtin_amdgcn_raw_buffer_load_b16(rws, wo, 0, 0);
        }
    };
    auto store_scales = [&](int buf) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = threadIdx.x + u * kThreads;
            const int cb = i / kTile, r = i - cb * kTile;
            s_da[buf][cb][r] = half_bits_to_float(da_bits[u]);
            if constexpr (!COLUMN) {
                s_dw[buf][cb][r] = half_bits_to_float(dw_bits[u]);
                finite = finite && half_bits_finite(dw_bits[u]);
            }
        }
    };
    load_scales(0);
    store_scales(0);
    load_scales(kChunk);
    __syncthreads();

    for (int c0 = 0, buf = 0; c0 < t.blocks; c0 += kChunk, buf ^= 1) {
        // Groups of kAhead blocks, the tail padded with blocks past K whose
        // fragments and scales are zero: their terms are exactly +0, and the
        // accumulator, which starts at +0, never holds -0, so adding them
        // changes nothing.
        const int nb = min(kChunk, t.blocks - c0);
        for (int cb0 = 0; cb0 < nb; cb0 += kAhead) {
            // The group's scales, read from LDS before any of its blocks is
            // reduced: one LDS round trip per group rather than per block
            // (measured on MI355X: the M = 512 down projection 60 -> 45 us).
            float gdw[kAhead];
            float4 gda[kAhead][4];
#pragma unroll
            for (int j = 0; j < kAhead; ++j) {
                if constexpr (!COLUMN) gdw[j] = s_dw[buf][cb0 + j][wn * 32 + l32];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    gda[j][q] = *reinterpret_cast<const float4 *>(&s_da[buf][cb0 + j][wm * 32 + 8 * q + 4 * h]);
            }
#pragma unroll
            for (int j = 0; j < kAhead; ++j) {
                const int cb = cb0 + j;
                {
                    // Dots of the next block (slot j + 1), then refill that
                    // slot with the block kAhead further on.
                    const int jn = (j + 1) % kAhead;
                    v4i af, wf;
                    frags_of(ring[jn], af, wf);
                    dots[(j + 1) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, wf, cin, 0, 0, 0);
                    issue_frags(t, ra, rw, base, c0 + cb + 1 + kAhead, ring[jn]);
                }
                const v16i &d = dots[j & 1];
                const float dw = COLUMN ? 1.0f : gdw[j];
                const float c = dw * -kDotBias;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float das[4] = {gda[j][q].x, gda[j][q].y, gda[j][q].z, gda[j][q].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float v;
                        if constexpr (COLUMN)
                            v = static_cast<float>(d[4 * q + e]);
                        else
                            v = fmaf(__int_as_float(d[4 * q + e]), dw, c);
                        v = v * das[e];
                        acc[4 * q + e] = acc[4 * q + e] + v;
                    }
                }
            }
        }
        // The other buffer was last read two chunks ago (before the previous
        // barrier): fill it with the next chunk and prefetch the one after.
        store_scales(buf ^ 1);
        load_scales(c0 + 2 * kChunk);
        __syncthreads();
    }
    if constexpr (!COLUMN) {
        if (__syncthreads_or(!finite)) exact_terms_split(t, m0 + wm * 32 + 4 * h, bn, acc);
    }
    if (!b_ok) return;
    const float cs = COLUMN ? t.cs[bn] : 1.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = m0 + wm * 32 + 8 * q + 4 * h + e;
            if (m < t.m)
                reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(t.y) + static_cast<size_t>(m) * t.y_stride)[t.ocol0 + bn] =
                    COLUMN ? acc[4 * q + e] * cs : acc[4 * q + e];
        }
}

// -------------------------------------------------- native blocks, staged
//
// Native fragments sit at 2-byte offsets, one scattered row per lane, so a
// workgroup stages kGroup blocks at a time of its 64 activation rows and 64
// weight columns in LDS instead: kGroup consecutive threads read the
// consecutive blocks of one row (contiguous bytes), realign them and convert
// the weight nibbles to int8 once per workgroup, and write per row (column)
// kGroup runs of 32 signed bytes in k order, rows padded to kPitch bytes,
// plus fp32 scales.  Global loads are issued a group ahead into registers and
// written to the other of two LDS buffers at the end of the current group
// (one barrier per group); the waves read 16-byte aligned fragments.
constexpr int kGroup = 4;                          // blocks per staged group (8: 10 % slower at M = 512)
constexpr int kPitch = kGroup * 32 + 16;           // bytes per staged row (padding spreads banks)
constexpr int kPairs = kTile * kGroup / kThreads;  // (row, block) pairs per thread per operand
static_assert(kPairs >= 1 && kGroup % 4 == 0, "a group is staged by whole pairs and scaled 4 blocks at a time");

struct StageBuf {
    uint8_t a[kTile * kPitch];
    uint8_t w[kTile * kPitch];
    float da[kGroup][kTile];
    float dw[kGroup][kTile];
};

// One group's raw loads for this thread: the aligned dwords around each
// block's 32 activation bytes (8, then the 2 bytes that follow) and 16 nibble
// bytes (4, then 2 bytes), the byte shift (0 or 2) that realigns them, and
// the fp16 scale bits.
struct StageRegs {
    uint32_t a[kPairs][9];
    uint32_t w[kPairs][5];
    uint32_t a_shift[kPairs], w_shift[kPairs];
    uint32_t da[kPairs], dw[kPairs];
};

// Signed int8 code - 8 of four packed nibbles: (v | 0x80) - 8 never borrows
// across bytes, and ^ 0x80 maps 0x78..0x87 to -8..7.
__device__ __forceinline__ uint32_t nibble_bytes_to_int8(uint32_t v) {
    return ((v | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

// Pair q of this thread: row (or column) and block within the group.
__device__ __forceinline__ void stage_pair(int q, int &row, int &jb) {
    const int p = threadIdx.x + q * kThreads;
    row = p / kGroup;
    jb = p % kGroup;
}

// Rows past M, columns past N and blocks past K load zeros (out-of-range
// offsets), so their values and scales stage as zeros.  SELECT computes every
// lane's offset and then selects it (no control flow in the loop); otherwise
// the offset is computed only under the condition, which the compiler turns
// into a branch around the weight offset.  The branch splits the loop body:
// the group's four MFMAs are then issued before any of its scaling, and all
// four blocks' dots and scales stay live (178 VGPRs: two workgroups per CU).
// The select form keeps the dots of one block ahead (155 VGPRs: three
// workgroups per CU).  Measured on MI355X at M = 512: K=2048 N=5632 (704
// workgroups) 43.0 -> 38.5 us with SELECT; K=5632 N=2048 (256 workgroups, one
// wave per SIMD) 48.7 us without, 56 us with.
template <bool SELECT>
__device__ __forceinline__ void stage_load(const TiledArgs &t, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rw,
                                           int m0, int n0, int g0, StageRegs &r) {
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
        int row, jb;
        stage_pair(q, row, jb);
        const int b = g0 + jb, m = m0 + row;
        uint32_t o;
        if constexpr (SELECT) {
            const uint32_t raw = static_cast<uint32_t>(m) * t.act_stride + static_cast<uint32_t>(b) * 34u;
            o = ((b < t.blocks) & (m < t.m)) ? raw : kOutOfRange;
        } else {
            o = b < t.blocks && m < t.m ? static_cast<uint32_t>(m) * t.act_stride + static_cast<uint32_t>(b) * 34u
                                        : kOutOfRange;
        }
        const uint32_t v = (o + 2) & ~3u;  // the 32 values start 2 bytes in
        const v4u x0 = __builtin_amdgcn_raw_buffer_load_b128(ra, v, 0, 0);
        const v4u x1 = __builtin_amdgcn_raw_buffer_load_b128(ra, v + 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.a[q][i] = x0[i];
            r.a[q][4 + i] = x1[i];
        }
        // Only 2 bytes of the ninth dword are ever needed (shift 2): a 16-bit
        // load, so the last block of a tensor ending 2 bytes into that dword
        // is not read as zero by a partly out-of-range 32-bit load.
        r.a[q][8] = __builtin_amdgcn_raw_buffer_load_b16(ra, v + 32, 0, 0);
        r.a_shift[q] = (o + 2) & 3u;
        r.da[q] = __builtin_amdgcn_raw_buffer_load_b16(ra, o, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
        int col, jb;
        stage_pair(q, col, jb);
        const int b = g0 + jb, n = n0 + col;
        uint32_t o;
        if constexpr (SELECT) {
            const uint32_t raw = static_cast<uint32_t>(t.wcol0 + n) * t.w_stride + static_cast<uint32_t>(b) * 18u;
            o = ((b < t.blocks) & (n < t.n)) ? raw : kOutOfRange;
        } else {
            o = b < t.blocks && n < t.n
                    ? static_cast<uint32_t>(t.wcol0 + n) * t.w_stride + static_cast<uint32_t>(b) * 18u
                    : kOutOfRange;
        }
        const uint32_t v = (o + 2) & ~3u;  // the 16 nibble bytes start 2 bytes in
        const v4u x0 = __builtin_amdgcn_raw_buffer_load_b128(rw, v, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.w[q][i] = x0[i];
        r.w[q][4] = __builtin_amdgcn_raw_buffer_load_b16(rw, v + 16, 0, 0);  // as for the activation
        r.w_shift[q] = (o + 2) & 3u;
        r.dw[q] = __builtin_amdgcn_raw_buffer_load_b16(rw, o, 0, 0);
    }
}

// Returns whether every weight scale this thread staged is finite.
__device__ __forceinline__ bool stage_store(const StageRegs &r, StageBuf &s) {
    bool finite = true;
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
        int row, jb;
        stage_pair(q, row, jb);
        uint32_t v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __builtin_amdgcn_alignbyte(r.a[q][i + 1], r.a[q][i], r.a_shift[q]);
        v4u *dst = reinterpret_cast<v4u *>(s.a + row * kPitch + jb * 32);
        dst[0] = v4u{v[0], v[1], v[2], v[3]};
        dst[1] = v4u{v[4], v[5], v[6], v[7]};
        s.da[jb][row] = half_bits_to_float(r.da[q]);
    }
#pragma unroll
    for (int q = 0; q < kPairs; ++q) {
        int col, jb;
        stage_pair(q, col, jb);
        // Byte j of the nibbles holds element j (low) and j + 16 (high).
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t nib = __builtin_amdgcn_alignbyte(r.w[q][i + 1], r.w[q][i], r.w_shift[q]);
            lo[i] = nibble_bytes_to_int8(nib & 0x0F0F0F0Fu);
            hi[i] = nibble_bytes_to_int8((nib >> 4) & 0x0F0F0F0Fu);
        }
        v4u *dst = reinterpret_cast<v4u *>(s.w + col * kPitch + jb * 32);
        dst[0] = v4u{lo[0], lo[1], lo[2], lo[3]};
        dst[1] = v4u{hi[0], hi[1], hi[2], hi[3]};
        s.dw[jb][col] = half_bits_to_float(r.dw[q]);
        finite = finite && half_bits_finite(r.dw[q]);
    }
    return finite;
}

template <bool SELECT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, SELECT ? 8 : 2))) void q4_0_staged_kernel(
    TiledArgs t) {
    __shared__ __attribute__((aligned(16))) StageBuf stage[2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
    const int h = lane >> 5, l32 = lane & 31;
    const int arow = wm * 32 + l32;  // staged row of this lane's A fragment
    const int wcol = wn * 32 + l32;  // staged column of this lane's B fragment (and of its outputs)
    const int bn = n0 + wcol;

    const __amdgpu_buffer_rsrc_t ra = rsrc(t.act, t.a_extent);
    const __amdgpu_buffer_rsrc_t rw = rsrc(t.w, t.w_extent);

    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    // Grids of two or more workgroups per CU need this kernel at three
    // workgroups per CU (at most 168 registers): there (SELECT) the dots stay
    // plain int32 and are converted.  The bias costs 16 registers (measured
    // at M = 512 gate_up: 169 VGPRs, two workgroups per CU, 44.0 us; made to
    // fit 168 by reading the activation scales two blocks at a time, 39.3 us;
    // plain dots 38.3 us).  Smaller grids run one or two workgroups per CU and
    // take it (down at M = 512 48.4 -> 46.4 us).
    constexpr bool BIASED = !SELECT;
    const v16i cin = BIASED ? dot_bias() : v16i{};

    StageRegs regs;
    stage_load<SELECT>(t, ra, rw, m0, n0, 0, regs);
    bool finite = stage_store(regs, stage[0]);
    stage_load<SELECT>(t, ra, rw, m0, n0, kGroup, regs);
    __syncthreads();

    auto frag = [&](const StageBuf &s, int j, v4i &a, v4i &w) {
        a = *reinterpret_cast<const v4i *>(s.a + arow * kPitch + j * 32 + 16 * h);
        w = *reinterpret_cast<const v4i *>(s.w + wcol * kPitch + j * 32 + 16 * h);
    };
    // Blocks past K are staged as zero values with zero scales: their terms
    // are exactly +0, and the accumulator, which starts at +0, never holds
    // -0, so adding them changes nothing.
    for (int g0 = 0, buf = 0; g0 < t.blocks; g0 += kGroup, buf ^= 1) {
        const StageBuf &s = stage[buf];
        // dots[j & 1] holds block j's dots; block j + 1's are computed before
        // block j's are scaled.
        v16i dots[2];
        {
            v4i a, w;
            frag(s, 0, a, w);
            dots[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, w, cin, 0, 0, 0);
        }
#pragma unroll
        for (int half = 0; half < kGroup; half += 4) {
            float gdw[4];
            float4 gda[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                gdw[j] = s.dw[half + j][wcol];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    gda[j][q] = *reinterpret_cast<const float4 *>(&s.da[half + j][wm * 32 + 8 * q + 4 * h]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int jb = half + j;
                if (jb + 1 < kGroup) {
                    v4i a, w;
                    frag(s, jb + 1, a, w);
                    dots[(jb + 1) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, w, cin, 0, 0, 0);
                }
                const v16i &d = dots[jb & 1];
                const float c = gdw[j] * -kDotBias;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float das[4] = {gda[j][q].x, gda[j][q].y, gda[j][q].z, gda[j][q].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float v = BIASED ? fmaf(__int_as_float(d[4 * q + e]), gdw[j], c)
                                         : static_cast<float>(d[4 * q + e]) * gdw[j];
                        v = v * das[e];
                        acc[4 * q + e] = acc[4 * q + e] + v;
                    }
                }
            }
            if constexpr (!SELECT) {
                // One wave per SIMD: issue each block's MFMA ahead of the
                // previous block's scaling (measured on MI355X at M = 512,
                // K = 5632, N = 2048: 46.7 -> 44.8 us; the large-grid form,
                // whose other workgroups cover the latency, got slower).
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (half + j + 1 < kGroup) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 48, 0);  // VALU: one block's scaling
                }
            }
        }
        // The other buffer was last read a group ago (before the previous
        // barrier): fill it with the next group and load the one after.
        finite = stage_store(regs, stage[buf ^ 1]) && finite;
        stage_load<SELECT>(t, ra, rw, m0, n0, g0 + 2 * kGroup, regs);
        __syncthreads();
    }
    if constexpr (BIASED) {
        if (__syncthreads_or(!finite)) exact_terms_native(t, m0 + wm * 32 + 4 * h, bn, acc);
    }
    if (bn >= t.n) return;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = m0 + wm * 32 + 8 * q + 4 * h + e;
            if (m < t.m)
                reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(t.y) + static_cast<size_t>(m) * t.y_stride)[t.ocol0 + bn] =
                    acc[4 * q + e];
        }
}

int launch_tiled(const TiledArgs &t, bool native, hipStream_t stream) {
    const dim3 grid((t.n + kTile - 1) / kTile, (t.m + kTile - 1) / kTile, 1);
    if (grid.y > 65535u) return fail(QXT_INVALID_ARGUMENT, "q4_0 tiled linear: too many rows");
    // Native 18/34-byte blocks are staged through LDS by the workgroup (their
    // fragments sit at 2-byte offsets, one scattered row per lane); the split
    // planes are read as fragments directly (measured on MI355X at M = 512:
    // native gate_up 103 -> 42 us staged; split 44 us direct, 64 us staged).
    if (native) {
        const long workgroups = static_cast<long>(grid.x) * grid.y;
        if (workgroups >= 2L * compute_units())
            return launch("q4_0_tiled_kernel", q4_0_staged_kernel<true>, grid, dim3(kThreads), 0, stream, t);
        return launch("q4_0_tiled_kernel", q4_0_staged_kernel<false>, grid, dim3(kThreads), 0, stream, t);
    }
    if (t.cs != nullptr) return launch("q4_0_tiled_kernel", q4_0_tiled_kernel<true>, grid, dim3(kThreads), 0, stream, t);
    return launch("q4_0_tiled_kernel", q4_0_tiled_kernel<false>, grid, dim3(kThreads), 0, stream, t);
}

bool below_2gib(uint64_t bytes) { return bytes < (1ull << 31); }

}  // namespace

bool q4_0_tiled_native_supported(size_t act_stride, size_t w_stride, uint32_t rows, uint32_t blocks,
                                 uint32_t weight_column_start, uint32_t column_count) {
    const uint64_t a_extent = static_cast<uint64_t>(rows - 1) * act_stride + static_cast<uint64_t>(blocks) * 34;
    const uint64_t w_extent =
        static_cast<uint64_t>(weight_column_start + column_count - 1) * w_stride + static_cast<uint64_t>(blocks) * 18;
    return rows >= 16 && below_2gib(a_extent) && below_2gib(w_extent);
}

int q4_0_tiled_native(const void *activation, size_t activation_row_stride, const void *weight,
                      size_t weight_row_stride, float *destination, size_t destination_row_stride, uint32_t rows,
                      uint32_t blocks, uint32_t weight_column_start, uint32_t output_column_start,
                      uint32_t column_count, hipStream_t stream) {
    TiledArgs t{};
    t.act = static_cast<const uint8_t *>(activation);
    t.w = static_cast<const uint8_t *>(weight);
    t.y = destination;
    t.act_stride = static_cast<uint32_t>(activation_row_stride);
    t.w_stride = static_cast<uint32_t>(weight_row_stride);
    t.y_stride = destination_row_stride;
    t.a_extent = static_cast<uint32_t>(static_cast<uint64_t>(rows - 1) * activation_row_stride + blocks * 34ull);
    t.w_extent = static_cast<uint32_t>(static_cast<uint64_t>(weight_column_start + column_count - 1) * weight_row_stride +
                                       blocks * 18ull);
    t.m = static_cast<int>(rows);
    t.n = static_cast<int>(column_count);
    t.blocks = static_cast<int>(blocks);
    t.wcol0 = static_cast<int>(weight_column_start);
    t.ocol0 = static_cast<int>(output_column_start);
    return launch_tiled(t, true, stream);
}

int q4_0_tiled_column_w8(const int8_t *activation_q, const uint16_t *activation_scales, const uint32_t *weight_q,
                         size_t weight_q_row_stride, const float *column_scales, float *destination,
                         size_t destination_row_stride, uint32_t rows, uint32_t blocks, uint32_t columns,
                         hipStream_t stream) {
    const uint64_t k = static_cast<uint64_t>(blocks) * 32;
    const uint64_t a_extent = static_cast<uint64_t>(rows) * k;
    const uint64_t as_extent = static_cast<uint64_t>(rows) * blocks * 2;
    const uint64_t w_extent = static_cast<uint64_t>(blocks * 8ull - 1) * weight_q_row_stride + columns * 4ull;
    if (!below_2gib(a_extent) || !below_2gib(as_extent) || !below_2gib(w_extent))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 column-w8 linear: operands must be smaller than 2 GiB");
    TiledArgs t{};
    t.aq = reinterpret_cast<const uint8_t *>(activation_q);
    t.as = reinterpret_cast<const uint8_t *>(activation_scales);
    t.wq = reinterpret_cast<const uint8_t *>(weight_q);
    t.cs = column_scales;
    t.y = destination;
    t.aq_stride = static_cast<uint32_t>(k);
    t.as_stride = blocks * 2;
    t.as_bytes = 2;
    t.wq_stride = static_cast<uint32_t>(weight_q_row_stride);
    t.y_stride = destination_row_stride;
    t.a_extent = static_cast<uint32_t>(a_extent);
    t.as_extent = static_cast<uint32_t>(as_extent);
    t.w_extent = static_cast<uint32_t>(w_extent);
    t.m = static_cast<int>(rows);
    t.n = static_cast<int>(columns);
    t.blocks = static_cast<int>(blocks);
    return launch_tiled(t, false, stream);
}

}  // namespace qxt

using namespace qxt;

extern "C" int qxt_ggml_q4_0_q8_0_tiled_linear(const void *activation_q, size_t activation_q_row_stride,
                                               const void *activation_scales, size_t activation_scales_row_stride,
                                               uint32_t activation_scale_bytes, const void *weight_q,
                                               size_t weight_q_row_stride, const void *weight_scales,
                                               size_t weight_scales_row_stride, float *destination,
                                               size_t destination_row_stride, uint32_t rows, uint32_t blocks,
                                               uint32_t columns, void *stream) {
    if (activation_q == nullptr || activation_scales == nullptr || weight_q == nullptr || weight_scales == nullptr ||
        destination == nullptr)
        return fail(QXT_INVALID_ARGUMENT, "q4_0 tiled linear: null pointer");
    if (rows == 0 || blocks == 0 || columns == 0)
        return fail(QXT_INVALID_ARGUMENT, "q4_0 tiled linear: rows, blocks and columns must be positive");
    if (activation_scale_bytes != 2 && activation_scale_bytes != 4)
        return fail(QXT_INVALID_ARGUMENT, "q4_0 tiled linear: activation scales are 2- or 4-byte elements");
    const uint64_t k = static_cast<uint64_t>(blocks) * 32;
    if (activation_q_row_stride < k || activation_q_row_stride % 4 || !aligned(activation_q, 4) ||
        activation_scales_row_stride < static_cast<uint64_t>(blocks) * activation_scale_bytes ||
        activation_scales_row_stride % activation_scale_bytes || !aligned(activation_scales, activation_scale_bytes) ||
        weight_q_row_stride < static_cast<uint64_t>(columns) * 4 || weight_q_row_stride % 4 || !aligned(weight_q, 4) ||
        weight_scales_row_stride < static_cast<uint64_t>(columns) * 2 || weight_scales_row_stride % 2 ||
        !aligned(weight_scales, 2))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 tiled linear: bad operand strides or alignment");
    if (!aligned(destination, 4) || destination_row_stride % 4 ||
        destination_row_stride < static_cast<uint64_t>(columns) * 4)
        return fail(QXT_INVALID_ARGUMENT, "q4_0 tiled linear: bad destination");
    const uint64_t a_extent = static_cast<uint64_t>(rows - 1) * activation_q_row_stride + k;
    const uint64_t as_extent =
        static_cast<uint64_t>(rows - 1) * activation_scales_row_stride + static_cast<uint64_t>(blocks) * activation_scale_bytes;
    const uint64_t w_extent = static_cast<uint64_t>(blocks * 8ull - 1) * weight_q_row_stride + columns * 4ull;
    const uint64_t ws_extent = static_cast<uint64_t>(blocks - 1) * weight_scales_row_stride + columns * 2ull;
    if (!below_2gib(a_extent) || !below_2gib(as_extent) || !below_2gib(w_extent) || !below_2gib(ws_extent))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 tiled linear: operands must be smaller than 2 GiB");
    int rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    TiledArgs t{};
    t.aq = static_cast<const uint8_t *>(activation_q);
    t.as = static_cast<const uint8_t *>(activation_scales);
    t.wq = static_cast<const uint8_t *>(weight_q);
    t.ws = static_cast<const uint8_t *>(weight_scales);
    t.y = destination;
    t.aq_stride = static_cast<uint32_t>(activation_q_row_stride);
    t.as_stride = static_cast<uint32_t>(activation_scales_row_stride);
    t.as_bytes = activation_scale_bytes;
    t.wq_stride = static_cast<uint32_t>(weight_q_row_stride);
    t.ws_stride = static_cast<uint32_t>(weight_scales_row_stride);
    t.y_stride = destination_row_stride;
    t.a_extent = static_cast<uint32_t>(a_extent);
    t.as_extent = static_cast<uint32_t>(as_extent);
    t.w_extent = static_cast<uint32_t>(w_extent);
    t.ws_extent = static_cast<uint32_t>(ws_extent);
    t.m = static_cast<int>(rows);
    t.n = static_cast<int>(columns);
    t.blocks = static_cast<int>(blocks);
    return launch_tiled(t, false, as_stream(stream));
}

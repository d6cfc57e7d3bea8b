// Q4_0 x Q8_0 block-dot linear for gfx950 (M = 1 decode and small M).
//
// Arithmetic (reference src/qpu_xla/kernels/ggml_q4_0.py:81-100 and the QPU
// loop at :688-692): per 32-element block an exact int32 dot, then
// c_b = fl32(fl32(float(dot_b) * dw_b) * da_b), summed in block order
// ((0 + c_0) + c_1) + ...  The kernel reproduces that result bit for bit.
//
// One workgroup (256 threads) owns a tile of `cpw` output columns of one
// linear ("work item").  Because the weight rows of consecutive columns are
// adjacent, the tile is one contiguous byte range of the [N, B, 18] weight
// tensor, cut into "units" of 8 consecutive blocks of one column (144 bytes,
// 9 x 16-byte loads on the fast path):
//
//   phase 0  each thread issues the loads of its U units into registers;
//   phase 1  while those loads are in flight the workgroup stages the Q8_0
//            activation rows in LDS (int8 words + fp32 scale + int32 element
//            sum per block) from native 34-byte blocks;
//   phase 2  each unit yields 8 block terms c_b (v_dot4_i32_i8) into LDS;
//   phase 3  one thread per (row, column) adds the column's c_b in block
//            order and stores the fp32 result.
//
// Nibble codes enter the dot as unsigned 0..15; the "- 8" of every element is
// applied once per block as -8 * sum(activation), exact in int32.  The fast
// path needs blocks % 8 == 0 and 16-byte aligned weight rows (every K that is
// a multiple of 256); otherwise each thread takes one block with 2-byte loads.
//
// Weight layouts.  Native: the [N, B, 18] ggml rows, a thread's unit at a
// 144-byte stride from its neighbour's, so one 16-byte load instruction of a
// wave touches 64 scattered pieces.  Lanes (qxt_q4_0_pack_lanes): the same
// 144-byte units in native order, cut into groups of 64; chunk v (16 bytes)
// of unit l of a group sits at group * 9216 + (v * 64 + l) * 16.  Consecutive
// lanes own consecutive units, so each load instruction of a wave reads 1 KB
// contiguous (two runs when the wave straddles a group edge), and those loads
// are issued non-temporal: measured on MI355X for the decode access pattern
// (7436 workgroups x 73,728 bytes, loads only): 5.0 TB/s native, 6.2 TB/s
// lanes, 7.0 TB/s lanes non-temporal (non-temporal native: 2.0 TB/s).
//
// Entry points: a single linear (stateless, native Q8_0 activation), its
// int32 block-dot debug twin, and a prepared batch of independent linears
// launched as one grid (the decode step of a model whose projections read
// separate activations).  A batch task may give fp32 activation rows: one
// pre-pass launch quantises all of them to Q8_0 (the rule of
// quantize_q8_0_split, examples/benchmark_llama_cpp_qpu_persistent_q4.py:42-53)
// into a buffer the batch owns, before the batch grid reads them as native
// blocks.  (Quantising inside every workgroup instead -- each workgroup of a
// linear re-quantising the whole row -- measured 86-97 us per cfg3 step
// against 79-81 us with the pre-pass.)
#include <algorithm>
#include <limits>
#include <new>
#include <type_traits>
#include <utility>
#include <vector>

#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;
constexpr size_t kMaxLds = 64 * 1024;       // LDS a workgroup may use to stage its activation rows
constexpr size_t kMaxLdsWide = 160 * 1024;  // gfx950 LDS per workgroup: wide single-linear tiles

struct Q4Task {
    const float *x;        // fp32 rows quantised to Q8_0 in the workgroup, or nullptr
    size_t x_stride;
    const uint8_t *act;    // native Q8_0 blocks [rows, blocks, 34] (when x is nullptr)
    const uint8_t *w;      // Q4_0 blocks [N, blocks, 18]
    float *y;              // fp32 output
    int32_t *dots;         // debug: int32 block dots [rows, ncols, blocks]
    size_t act_stride, w_stride, y_stride;  // row strides in bytes
    int rows, blocks, wcol0, ocol0, ncols, cpw;
    int lanes;             // weight in the lane-interleaved layout (w = packed matrix base)
};

constexpr int kLaneGroup = 64;                      // units per lane group
constexpr int kUnitBytes = 144;                     // 8 Q4_0 blocks of one column
constexpr int kGroupBytes = kLaneGroup * kUnitBytes;  // 9216

struct Q4Item {
    int task;
    int col_base;
    int ncols;  // columns of this work item (<= the task's cpw)
};

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Batch kernels read their tensor pointers from a device table, so the
// compiler cannot tell they address global memory and would emit FLAT
// loads.  A FLAT load also counts against the LDS counter, which turns every
// later wait for an LDS access into a wait for all outstanding weight loads
// (activation staging then starts only after the weights have landed).
// Every tensor access goes through a global-address-space pointer instead.
#define QXT_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const QXT_GLOBAL T *global_in(const void *p) {
    return (const QXT_GLOBAL T *)p;
}
template <typename T>
__device__ __forceinline__ QXT_GLOBAL T *global_out(void *p) {
    return (QXT_GLOBAL T *)p;
}
__device__ __forceinline__ float4 load_float4(const void *p) {
    const v4u raw = *global_in<v4u>(p);
    return make_float4(__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                       __uint_as_float(raw[3]));
}

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

// Exact int32 dot of one Q4_0 block (packed nibbles qs) with one Q8_0 block
// (activation words a0, a1 and their element sum asum).
__device__ __forceinline__ int block_dot(const uint32_t (&qs)[4], const int4 &a0, const int4 &a1, int asum) {
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

__device__ __forceinline__ int block_dot(const uint32_t (&qs)[4], const int *aq, int asum) {
    return block_dot(qs, *reinterpret_cast<const int4 *>(aq), *reinterpret_cast<const int4 *>(aq + 4), asum);
}

// The (scale, sum) record of block b of LDS row r.  Row-major by default:
// the pair (d, sum(a)) at ad[r * ad_row + ad_index(b)].  SCALES4 (the
// four-row matrix-core tiles) keeps the four rows of a block together
// instead: -8 * sum(a) of rows 0..3 at ad[aq_index(b, 0 .. 3)], d of rows
// 0..3 at ad[aq_index(b, 4 .. 7)], so one lane reads a block's records for
// all four rows with two 16-byte loads.
template <bool SCALES4>
__device__ __forceinline__ void store_scale_sum(int *ad, const Q4Lds &geo, int r, int b, float d, int sum) {
    if constexpr (SCALES4) {
        ad[aq_index(b, r)] = -8 * sum;
        ad[aq_index(b, 4 + r)] = __float_as_int(d);
    } else {
        ad[r * geo.ad_row + ad_index(b)] = __float_as_int(d);
        ad[r * geo.ad_row + ad_index(b) + 1] = sum;
    }
}

// Quantise element chunk e (float4 v: elements 4 (e % 8) .. of block e / 8 of
// row r) by the rule of q8_0_prepass_kernel -- 8 lanes per block, the dots use
// the fp16-rounded d -- into the LDS activation of row r; nothing is stored
// when `store` is false.  The 8 lanes of a block must be active together.
// FAST uses the division-free scale without its range check (no branch, so
// the chunks of one thread interleave) and returns whether the block's
// absmax was inside the range where that is exact; the caller quantises the
// chunk again without FAST when it was not.
template <bool SCALES4 = false, bool FAST = false>
__device__ __forceinline__ bool quantise_chunk(const float4 &v, int r, int rem, int *aq, int *ad, const Q4Lds &geo,
                                               bool store = true) {
    const int b = rem >> 3, l8 = rem & 7;
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    float d, inv;
    if constexpr (FAST) q8_0_scale_fast(amax, d, inv);
    else q8_0_scale(amax, d, inv);
    const int q0 = clamp127(rintf(v.x * inv)), q1 = clamp127(rintf(v.y * inv));
    const int q2 = clamp127(rintf(v.z * inv)), q3 = clamp127(rintf(v.w * inv));
    int sum = q0 + q1 + q2 + q3;
    sum += __shfl_xor(sum, 1, 8);
    sum += __shfl_xor(sum, 2, 8);
    sum += __shfl_xor(sum, 4, 8);
    if (store) {
        aq[r * geo.aq_row + aq_index(b, l8)] = static_cast<int>(pack_bytes(q0, q1, q2, q3));
        if (l8 == 0) store_scale_sum<SCALES4>(ad, geo, r, b, half_bits_to_float(float_to_half_bits(d)), sum);
    }
    return !FAST || q8_0_fast_scale_range(amax);
}

// A one-row fp32 activation of K <= kMaxPrefetchChunks * 4 * kThreads
// (6144) is requested before the weights, PC 16-byte chunks per thread, so
// that its quantisation waits only for its own loads: a wave's loads
// complete in order, and a row requested after the weights would arrive
// only after all of them.
constexpr int kMaxPrefetchChunks = 6;

// The prefetch value of one-row batches whose every activation is a native
// Q8_0 row of at most kThreads blocks (K <= 8192, e.g. the Q8_0 written by a
// pre-pass): each thread requests its block's 34 bytes before the weights
// and the workgroup stages the row from registers, so the staging waits only
// for the row.  (Requested after the weights, the staging of each workgroup
// waited for all of its weight loads first, then fetched the row block by
// block.)  Measured on MI355X, the cfg3 step's 7436-item batch: kernel
// 81.5-82.6 -> 80.3-80.9 us, wall per step with the pre-pass 0.091 ->
// 0.0865 ms (same box, alternating runs).
constexpr int kQ8RowPrefetch = -1;

// Chunks per thread that hold a one-row fp32 activation of `t` (2, 4 or 6),
// or 0 when the task does not qualify.
__host__ __device__ inline int prefetch_chunks(const Q4Task &t) {
    if (t.x == nullptr || t.rows != 1) return 0;
    const int chunks = (t.blocks * 8 + kThreads - 1) / kThreads;
    return chunks <= 2 ? 2 : chunks <= 4 ? 4 : chunks <= kMaxPrefetchChunks ? kMaxPrefetchChunks : 0;
}

template <int PC, int NT = kThreads>
__device__ __forceinline__ void prefetch_row(const Q4Task &t, float4 (&xv)[PC]) {
    const int total = t.blocks * 8;
#pragma unroll
    for (int u = 0; u < PC; ++u) {
        // Unconditional loads (lanes past the row re-read its last chunk, unused).
        const int e = min(u * NT + static_cast<int>(threadIdx.x), total - 1);
        xv[u] = load_float4(reinterpret_cast<const uint8_t *>(t.x) + e * 16);
    }
}

template <int PC, int NT = kThreads>
__device__ __forceinline__ void quantise_row(const Q4Task &t, const float4 (&xv)[PC], int *aq, int *ad,
                                             const Q4Lds &geo) {
    const int total = t.blocks * 8;  // a multiple of 8: whole 8-lane groups
    // Every lane quantises (lanes past the row work on a re-read chunk and
    // store nothing), so no load is sunk into a branch behind the weights.
    // The chunks use the division-free scale without a branch each; a thread
    // holding a block outside its range quantises its chunks again with the
    // checked rule (the 8 lanes of a block agree, their chunks sharing blocks).
    // Measured on MI355X, the staged decode of cfg3: per-chunk branches cost
    // more than the divisions they skip (0.414 -> 0.419 ms per step).
    bool exact = true;
#pragma unroll
    for (int u = 0; u < PC; ++u) {
        const int e = u * NT + threadIdx.x;
        exact &= quantise_chunk<false, true>(xv[u], 0, min(e, total - 1), aq, ad, geo, e < total);
    }
    if (!exact) {
#pragma unroll
        for (int u = 0; u < PC; ++u) {
            const int e = u * NT + threadIdx.x;
            quantise_chunk(xv[u], 0, min(e, total - 1), aq, ad, geo, e < total);
        }
    }
}

// Stage the activation rows r0 .. r0+MR-1 of `t` into LDS (rows >= t.rows
// become zeros), the (scale, sum) records in the layout of store_scale_sum.
template <int MR, bool SCALES4 = false>
__device__ __forceinline__ void stage_activation(const Q4Task &t, int r0, int *aq, int *ad, const Q4Lds &geo) {
    const int B = t.blocks;
    if (t.x != nullptr) {
        // fp32 rows (a small batch, no pre-pass): quantised to Q8_0 by the
        // rule of q8_0_prepass_kernel, 8 lanes per block and float4 per lane,
        // four loads in flight per thread; the dots use the fp16-rounded d.
        // `total` and every chunk start are multiples of 8, so the 8 lanes of
        // a block are active together.
        const int total = MR * B * 8;
        for (int base = 0; base < total; base += 4 * kThreads) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = base + u * kThreads + threadIdx.x;
                v[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                const int r = e / (B * 8);
                if (e < total && r0 + r < t.rows)
                    v[u] = load_float4(reinterpret_cast<const uint8_t *>(t.x) + (r0 + r) * t.x_stride +
                                       (e - r * B * 8) * 16);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = base + u * kThreads + threadIdx.x;
                if (e >= total) break;
                const int r = e / (B * 8);
                quantise_chunk<SCALES4>(v[u], r, e - r * B * 8, aq, ad, geo);
            }
        }
        return;
    }
    for (int idx = threadIdx.x; idx < MR * B; idx += kThreads) {
        const int r = idx / B;
        const int b = idx - r * B;
        int words[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float d = 0.0f;
        int sum = 0;
        if (r0 + r < t.rows) {
            const QXT_GLOBAL uint16_t *p =
                global_in<uint16_t>(t.act + (r0 + r) * t.act_stride + static_cast<size_t>(b) * Q8_0_BYTES);
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
        store_scale_sum<SCALES4>(ad, geo, r, b, d, sum);
    }
}

// Native Q8_0 activation rows of a four-row group for the matrix-core
// tiles, requested into registers before any weight load: 512 / NT (row,
// block) items per thread of an NT-thread workgroup (4 * blocks <= 512), 17
// half-words each.  The loads are unconditional (indexes clamped into the
// activation), so the compiler counts the weight loads issued after them
// exactly and the staging waits only for these.
template <int NT, int ITEMS = (512 + NT - 1) / NT>
struct Q8RowRegs {
    static constexpr int kItems = ITEMS;
    uint32_t h[kItems][17];
};

// Keeps the compiler from moving memory accesses across this point.  Placed
// after an activation row requested into registers ahead of the weights: the
// row's later use sits behind a per-thread branch (threads past the row's
// blocks have none), and without the barrier the compiler sinks the row's
// loads into that branch, after the weight loads, so that the row's first
// wait waits for every weight load.
__device__ __forceinline__ void pin_memory_order() { asm volatile("" ::: "memory"); }

template <int NT>
__device__ __forceinline__ void fetch_q8_rows(const Q4Task &t, int r0, Q8RowRegs<NT> &a) {
    const int B = t.blocks;
#pragma unroll
    for (int i = 0; i < Q8RowRegs<NT>::kItems; ++i) {
        const int idx = min(static_cast<int>(threadIdx.x) + i * NT, 4 * B - 1);
        const int r = idx / B;
        const int b = idx - r * B;
        const int row = min(r0 + r, t.rows - 1);
        const QXT_GLOBAL uint16_t *p =
            global_in<uint16_t>(t.act + row * t.act_stride + static_cast<size_t>(b) * Q8_0_BYTES);
#pragma unroll
        for (int k = 0; k < 17; ++k) a.h[i][k] = p[k];
    }
}

// The LDS image of fetch_q8_rows' items, the records in the SCALES4 layout.
// A row past t.rows holds a copy of the last row: a matrix-core output row
// depends on its own activation row only, and those rows are never stored.
template <int NT>
__device__ __forceinline__ void stage_q8_rows(const Q4Task &t, const Q8RowRegs<NT> &a, int *aq, int *ad,
                                              const Q4Lds &geo) {
    const int B = t.blocks;
#pragma unroll
    for (int i = 0; i < Q8RowRegs<NT>::kItems; ++i) {
        const int idx = static_cast<int>(threadIdx.x) + i * NT;
        if (idx >= 4 * B) break;
        const int r = idx / B;
        const int b = idx - r * B;
        int words[8];
        int sum = 0;
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            words[h] = static_cast<int>(a.h[i][1 + 2 * h] | (a.h[i][2 + 2 * h] << 16));
            sum = dot4(words[h], 0x01010101, sum);  // sum of the four signed bytes
        }
        int *dstq = aq + r * geo.aq_row + aq_index(b, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) dstq[j] = words[j];
        store_scale_sum<true>(ad, geo, r, b, half_bits_to_float(a.h[i][0]), sum);
    }
}

// One native Q8_0 activation row (blocks <= 512) into registers, 512 / NT
// blocks per thread, with unconditional loads (indexes clamped into the row)
// like fetch_q8_rows; stage_q8_row writes its LDS image with the row-major
// records.
template <int NT, int ITEMS>
__device__ __forceinline__ void fetch_q8_row(const Q4Task &t, Q8RowRegs<NT, ITEMS> &a) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
        const int b = min(static_cast<int>(threadIdx.x) + i * NT, t.blocks - 1);
        const QXT_GLOBAL uint16_t *p = global_in<uint16_t>(t.act + static_cast<size_t>(b) * Q8_0_BYTES);
#pragma unroll
        for (int k = 0; k < 17; ++k) a.h[i][k] = p[k];
    }
}

template <int NT, int ITEMS>
__device__ __forceinline__ void stage_q8_row(const Q4Task &t, const Q8RowRegs<NT, ITEMS> &a, int *aq, int *ad,
                                             const Q4Lds &geo) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
        const int b = static_cast<int>(threadIdx.x) + i * NT;
        if (b >= t.blocks) break;
        int words[8];
        int sum = 0;
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            words[h] = static_cast<int>(a.h[i][1 + 2 * h] | (a.h[i][2 + 2 * h] << 16));
            sum = dot4(words[h], 0x01010101, sum);  // sum of the four signed bytes
        }
        int *dstq = aq + aq_index(b, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) dstq[j] = words[j];
        store_scale_sum<false>(ad, geo, 0, b, half_bits_to_float(a.h[i][0]), sum);
    }
}

// Weight layout of a kernel instantiation: native rows, lane layout, or
// either (read from the task).  Separate instantiations keep the lane
// layout's non-temporal loads from being merged with the native rows'
// ordinary loads of the other branch.
enum WeightLayout { kNativeRows = 0, kLaneLayout = 1, kEitherLayout = 2 };

// CLAMP: every lane issues its loads, a lane past the tile re-reading the
// tile's last unit (its registers are never used).  The loads are then
// straight-line code, so the compiler counts them exactly and a later wait
// for an earlier load (a prefetched activation) does not wait for these.
// Without CLAMP, lanes past the tile skip their loads (cheaper for small
// tiles when nothing loaded earlier is waited for).
// Units of the four-row matrix-core path: in a wave of 64 consecutive units
// starting at a column boundary, lane 4 b + p takes column 4 (b / G) + p,
// block range b % G (G divides 16), so that every
// 4-lane block of v_mfma_i32_4x4x4_16b_i8 holds four columns of one block
// range.  The 64 units of a wave are the same, only permuted across lanes:
// each load instruction still reads one contiguous kilobyte of the lane
// layout.
// load_units of the matrix-core tiles: units in mfma4_unit order, every
// lane loading (CLAMP), G = 1 << lg.  Lane layout: one contiguous kilobyte
// per wave instruction, non-temporal; native rows: each lane's 144 bytes.
template <int U, int LAYOUT, int NT>
__device__ __forceinline__ void load_units_m4(const Q4Task &t, int col_base, int lg, int units, int first,
                                              uint32_t (&d)[U][36]) {
    const int lane = threadIdx.x & 63;
    const int b = lane >> 2, p = lane & 3;
    const int perm = ((((b >> lg) << 2) + p) << lg) + (b & ((1 << lg) - 1));
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int u = min(first + j * NT + (static_cast<int>(threadIdx.x) & ~63) + perm, units - 1);
        const int col = u >> lg, g = u & ((1 << lg) - 1);
        if constexpr (LAYOUT == kLaneLayout) {
            const size_t unit = (static_cast<size_t>(t.wcol0 + col_base + col) << lg) + g;
            const QXT_GLOBAL v4u *src =
                global_in<v4u>(t.w + (unit / kLaneGroup) * kGroupBytes + (unit % kLaneGroup) * 16);
#pragma unroll
            for (int v = 0; v < 9; ++v) {
                const v4u x = __builtin_nontemporal_load(src + v * kLaneGroup);
                d[j][4 * v + 0] = x[0];
                d[j][4 * v + 1] = x[1];
                d[j][4 * v + 2] = x[2];
                d[j][4 * v + 3] = x[3];
            }
        } else {
            const QXT_GLOBAL v4u *src = global_in<v4u>(
                t.w + static_cast<size_t>(t.wcol0 + col_base + col) * t.w_stride + static_cast<size_t>(g) * 144);
#pragma unroll
            for (int v = 0; v < 9; ++v) {
                const v4u x = src[v];
                d[j][4 * v + 0] = x[0];
                d[j][4 * v + 1] = x[1];
                d[j][4 * v + 2] = x[2];
                d[j][4 * v + 3] = x[3];
            }
        }
    }
}

template <int U, int LAYOUT = kEitherLayout, bool CLAMP = false>
__device__ __forceinline__ void load_units(const Q4Task &t, int col_base, int G, int units, int first,
                                           uint32_t (&d)[U][36]) {
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int lane_unit = first + j * kThreads + static_cast<int>(threadIdx.x);
        const int u = CLAMP ? min(lane_unit, units - 1) : lane_unit;
        if (CLAMP || u < units) {
            const int col = u / G;
            const int g = u - col * G;
            if (LAYOUT == kLaneLayout || (LAYOUT == kEitherLayout && t.lanes)) {
                const size_t unit = static_cast<size_t>(t.wcol0 + col_base + col) * G + g;
                const QXT_GLOBAL v4u *src =
                    global_in<v4u>(t.w + (unit / kLaneGroup) * kGroupBytes + (unit % kLaneGroup) * 16);
#pragma unroll
                for (int v = 0; v < 9; ++v) {
                    const v4u x = __builtin_nontemporal_load(src + v * kLaneGroup);
                    d[j][4 * v + 0] = x[0];
                    d[j][4 * v + 1] = x[1];
                    d[j][4 * v + 2] = x[2];
                    d[j][4 * v + 3] = x[3];
                }
            } else {
                const QXT_GLOBAL v4u *src = global_in<v4u>(
                    t.w + static_cast<size_t>(t.wcol0 + col_base + col) * t.w_stride + static_cast<size_t>(g) * 144);
#pragma unroll
                for (int v = 0; v < 9; ++v) {
                    const v4u x = src[v];
                    d[j][4 * v + 0] = x[0];
                    d[j][4 * v + 1] = x[1];
                    d[j][4 * v + 2] = x[2];
                    d[j][4 * v + 3] = x[3];
                }
            }
        }
    }
}

// Native [columns, blocks, 18] rows -> lane layout, one thread per 16-byte
// chunk of the packed matrix (units past the matrix are zero padding).
__global__ __launch_bounds__(kThreads) void pack_lanes_kernel(const uint8_t *__restrict__ w, size_t w_stride,
                                                              uint8_t *__restrict__ packed, size_t units,
                                                              size_t chunks, int G) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= chunks) return;
    const size_t group = idx / (9 * kLaneGroup);
    const int r = static_cast<int>(idx - group * 9 * kLaneGroup);
    const int v = r / kLaneGroup, l = r % kLaneGroup;
    const size_t unit = group * kLaneGroup + l;
    v4u x = {0u, 0u, 0u, 0u};
    if (unit < units) {
        const size_t col = unit / G, g = unit - col * G;
        x = *reinterpret_cast<const v4u *>(w + col * w_stride + g * kUnitBytes + v * 16);
    }
    *reinterpret_cast<v4u *>(packed + idx * 16) = x;
}

// One fp32 activation of a batch to quantise: rows x blocks Q8_0 blocks.
// Batches of at most this many work items quantise their fp32 activations
// inside each workgroup instead of in a pre-pass launch (a decode step's
// dependency stages: 128-704 items; the whole cfg3 step: 7436).
constexpr size_t kFusedQuantItems = 1024;

// Workgroups per CU below which a batch narrows its column tiles (measured
// on MI355X, the 88-launch staged decode step of cfg3: no narrowing 0.67 ms,
// one workgroup per CU 0.43 ms, two 0.49 ms, four and more slower still).
#ifndef QXT_BATCH_ITEMS_PER_CU
#define QXT_BATCH_ITEMS_PER_CU 1
#endif
constexpr int kBatchItemsPerCu = QXT_BATCH_ITEMS_PER_CU;

struct Q8Job {
    const float *x;
    size_t x_stride;
    uint8_t *out;     // Q8_0 [rows, blocks, 34], row stride blocks * 34
    int rows, blocks;
};

// Workgroup c quantises blocks [first, first + 32) of job `job` (8 lanes per
// block, one float4 each), the arithmetic of q8_0_kernel: d = absmax / 127,
// inv = 1 / d (0 for a zero block), q = clamp(rint(x * inv), +-127), d stored
// as fp16 (round to nearest even).
struct Q8Chunk {
    int job;
    int first;
};

__global__ __launch_bounds__(kThreads) void q8_0_prepass_kernel(const Q8Job *__restrict__ jobs,
                                                                const Q8Chunk *__restrict__ chunks) {
    const Q8Chunk c = chunks[blockIdx.x];
    const Q8Job j = jobs[c.job];
    const int gb = c.first + static_cast<int>(threadIdx.x >> 3);
    const int l8 = threadIdx.x & 7;
    if (gb >= j.rows * j.blocks) return;  // whole 8-lane groups exit together
    const int row = gb / j.blocks;
    const int b = gb - row * j.blocks;
    const float *src = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(j.x) + row * j.x_stride) +
                       b * QK + l8 * 4;
    const v4u raw = __builtin_nontemporal_load(global_in<v4u>(src));
    const float xs[4] = {__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                         __uint_as_float(raw[3])};
    float amax = fmaxf(fmaxf(fabsf(xs[0]), fabsf(xs[1])), fmaxf(fabsf(xs[2]), fabsf(xs[3])));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    float d, inv;
    q8_0_scale(amax, d, inv);
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = clamp127(rintf(xs[i] * inv));
    uint8_t *dst = j.out + (static_cast<size_t>(row) * j.blocks + b) * Q8_0_BYTES;
    const uint32_t word = pack_bytes(q[0], q[1], q[2], q[3]);
    // Block bytes 2 + 4 * l8 .. are 2-byte aligned: two half-word stores.
    QXT_GLOBAL uint16_t *h = global_out<uint16_t>(dst + 2 + 4 * l8);
    h[0] = static_cast<uint16_t>(word & 0xFFFFu);
    h[1] = static_cast<uint16_t>(word >> 16);
    if (l8 == 0) *global_out<uint16_t>(dst) = static_cast<uint16_t>(float_to_half_bits(d));
}

// Phase 2 of the fast path for one round of U units per thread (units
// first + j * kThreads + tid): the 8 block terms of every unit go to cb, or
// (DOTS) the exact int32 block dots go to t.dots.
template <int MR, int U, bool DOTS>
__device__ __forceinline__ void compute_fast(const Q4Task &t, int col_base, int r0, int G, int units, int first,
                                             const uint32_t (&wr)[U][36], const int *aq, const int *ad, float *cb,
                                             const Q4Lds &geo) {
    const int B = t.blocks;
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int u = first + j * kThreads + threadIdx.x;
        if (u >= units) continue;
        const int col = u / G;
        const int g = u - col * G;
        float terms[MR][8];
        int idots[MR][8];
        // One row: the unit's eight activation blocks are read from LDS up
        // front (24 reads in flight, 80 registers) instead of one block at a
        // time, which kept one or two reads in flight per unit.
        int4 pre_lo[MR == 1 ? 8 : 1], pre_hi[MR == 1 ? 8 : 1];
        int2 pre_ds[MR == 1 ? 8 : 1];
        if constexpr (MR == 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int b = g * 8 + i;
                pre_lo[i] = *reinterpret_cast<const int4 *>(aq + aq_index(b, 0));
                pre_hi[i] = *reinterpret_cast<const int4 *>(aq + aq_index(b, 4));
                pre_ds[i] = *reinterpret_cast<const int2 *>(ad + ad_index(b));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        auto do_block = [&](auto ic) {
            constexpr int I = decltype(ic)::value;
            uint32_t sbits, qs[4];
            unit_block<I>(wr[j], sbits, qs);
            const float dw = half_bits_to_float(sbits);
            const int b = g * 8 + I;
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                const int2 ds = MR == 1 ? pre_ds[I % (MR == 1 ? 8 : 1)]
                                        : *reinterpret_cast<const int2 *>(ad + r * geo.ad_row + ad_index(b));
                const int dot = MR == 1 ? block_dot(qs, pre_lo[I % (MR == 1 ? 8 : 1)], pre_hi[I % (MR == 1 ? 8 : 1)], ds.y)
                                        : block_dot(qs, aq + r * geo.aq_row + aq_index(b, 0), ds.y);
                idots[r][I] = dot;
                float v = static_cast<float>(dot) * dw;
                v = v * __int_as_float(ds.x);
                terms[r][I] = v;
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
                if (r0 + r < t.rows) {
                    QXT_GLOBAL int32_t *out =
                        global_out<int32_t>(t.dots + (static_cast<size_t>(r0 + r) * t.ncols + col_base + col) * B + g * 8);
#pragma unroll
                    for (int i = 0; i < 8; ++i) out[i] = idots[r][i];
                }
            } else {
                float4 *c4 = reinterpret_cast<float4 *>(cb + (r * t.cpw + col) * geo.cbs + g * 8);
                c4[0] = make_float4(terms[r][0], terms[r][1], terms[r][2], terms[r][3]);
                c4[1] = make_float4(terms[r][4], terms[r][5], terms[r][6], terms[r][7]);
            }
        }
    }
}

// Phase 2 of the four-row lane-layout path on the matrix cores: the units of
// one round in mfma4_unit order.  Per Q4_0 block, eight
// v_mfma_i32_4x4x4_16b_i8 (K = 4 each) give every lane the exact dots of its
// column with the four activation rows: operand A is activation row p of the
// lane's block range (lane 4 b + p), operand B the lane's own nibbles as
// unsigned codes, the accumulator starting from -8 * sum(a) of each row (the
// SCALES4 records), so every lane ends with the same exact signed dots as the
// v_dot4 path and the block terms are the same bits.
template <int U, int NT>
__device__ __forceinline__ void compute_mfma4(const Q4Task &t, int lg, int units, int first,
                                              const uint32_t (&wr)[U][36], const int *aq, const int *ad, float *cb,
                                              const Q4Lds &geo) {
    typedef int v4i_t __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const int b = lane >> 2, p = lane & 3;
    const int g = b & ((1 << lg) - 1);
    const int *arow = aq + p * geo.aq_row;
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int u = first + j * NT + (static_cast<int>(threadIdx.x) & ~63) + ((((b >> lg) << 2) + p) << lg) + g;
        const int col = u >> lg;
        float terms[4][8];
        auto do_block = [&](auto ic) {
            constexpr int I = decltype(ic)::value;
            uint32_t sbits, qs[4];
            unit_block<I>(wr[j], sbits, qs);
            const int bg = g * 8 + I;
            const int4 lo = *reinterpret_cast<const int4 *>(arow + aq_index(bg, 0));
            const int4 hi = *reinterpret_cast<const int4 *>(arow + aq_index(bg, 4));
            const int4 s8 = *reinterpret_cast<const int4 *>(ad + aq_index(bg, 0));
            const float4 da = *reinterpret_cast<const float4 *>(ad + aq_index(bg, 4));
            v4i_t acc = {s8.x, s8.y, s8.z, s8.w};
            acc = __builtin_amdgcn_mfma_i32_4x4x4i8(lo.x, static_cast<int>(qs[0] & 0x0F0F0F0Fu), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_4x4x4i8(lo.y, static_cast<int>(qs[1] & 0x0F0F0F0Fu), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_4x4x4i8(lo.z, static_cast<int>(qs[2] & 0x0F0F0F0Fu), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_4x4x4i8(lo.w, static_cast<int>(qs[3] & 0x0F0F0F0Fu), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_4x4x4i8(hi.x, static_cast<int>((qs[0] >> 4) & 0x0F0F0F0Fu), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_4x4x4i8(hi.y, static_cast<int>((qs[1] >> 4) & 0x0F0F0F0Fu), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_4x4x4i8(hi.z, static_cast<int>((qs[2] >> 4) & 0x0F0F0F0Fu), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_4x4x4i8(hi.w, static_cast<int>((qs[3] >> 4) & 0x0F0F0F0Fu), acc, 0, 0, 0);
            const float dw = half_bits_to_float(sbits);
            const float das[4] = {da.x, da.y, da.z, da.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = static_cast<float>(acc[r]) * dw;
                v = v * das[r];
                terms[r][I] = v;
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
        if (u < units) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float4 *c4 = reinterpret_cast<float4 *>(cb + (r * t.cpw + col) * geo.cbs + g * 8);
                c4[0] = make_float4(terms[r][0], terms[r][1], terms[r][2], terms[r][3]);
                c4[1] = make_float4(terms[r][4], terms[r][5], terms[r][6], terms[r][7]);
            }
        }
    }
}

// Phase 3: one thread per (row, column) adds the column's block terms in
// block order and stores the fp32 result.
template <int MR, bool FAST, int NT = kThreads>
__device__ __forceinline__ void sum_store(const Q4Task &t, int col_base, int r0, int tile_cols, const float *cb,
                                          const Q4Lds &geo) {
    const int B = t.blocks;
    for (int k = threadIdx.x; k < MR * tile_cols; k += NT) {
        const int r = k / tile_cols;
        const int col = k - r * tile_cols;
        if (r0 + r >= t.rows) continue;
        const float *c = cb + (r * t.cpw + col) * geo.cbs;
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
        QXT_GLOBAL float *out = global_out<float>(reinterpret_cast<uint8_t *>(t.y) + (r0 + r) * t.y_stride);
        out[t.ocol0 + col_base + col] = acc;
    }
}

// One linear: workgroup (x, y) owns columns [x * cpw, +cpw) and rows [y * MR, +MR).
template <int MR, int U, bool FAST, bool DOTS, int LAYOUT = kNativeRows>
__global__ __launch_bounds__(kThreads) void q4_0_linear_kernel(Q4Task t) {
    extern __shared__ int lds[];
    const int col_base = blockIdx.x * t.cpw;
    const int r0 = blockIdx.y * MR;
    const int B = t.blocks;
    const Q4Lds geo(B, FAST);
    int *aq = lds;                                                 // [MR][aq_row]
    int *ad = aq + MR * geo.aq_row;                                // [MR][ad_row] (fp32 scale bits, sum)
    float *cb = reinterpret_cast<float *>(ad + MR * geo.ad_row);  // [MR][cpw][cbs]
    const int tile_cols = min(t.cpw, t.ncols - col_base);

    const int G = FAST ? (B >> 3) : B;
    const int units = tile_cols * G;
    uint32_t wr[FAST ? U : 1][36];

    if constexpr (FAST) load_units<U, LAYOUT>(t, col_base, G, units, 0, wr);

    stage_activation<MR>(t, r0, aq, ad, geo);
    __syncthreads();

    if constexpr (FAST && MR == 4 && !DOTS) {
        // Wide tiles (several rounds of units): the next round's weights are
        // requested before the current round is computed.
        for (int first = 0; first < units; first += U * kThreads) {
            uint32_t wn[U][36];
            const bool more = first + U * kThreads < units;
            if (more) load_units<U, LAYOUT>(t, col_base, G, units, first + U * kThreads, wn);
            compute_fast<MR, U, DOTS>(t, col_base, r0, G, units, first, wr, aq, ad, cb, geo);
            if (more) {
#pragma unroll
                for (int j = 0; j < U; ++j)
#pragma unroll
                    for (int w = 0; w < 36; ++w) wr[j][w] = wn[j][w];
            }
        }
    } else if constexpr (FAST) {
        for (int first = 0; first < units; first += U * kThreads) {
            if (first > 0) load_units<U, LAYOUT>(t, col_base, G, units, first, wr);
            compute_fast<MR, U, DOTS>(t, col_base, r0, G, units, first, wr, aq, ad, cb, geo);
        }
    } else {
        for (int u = threadIdx.x; u < units; u += kThreads) {
            const int col = u / B;
            const int b = u - col * B;
            const QXT_GLOBAL uint16_t *p = global_in<uint16_t>(t.w + static_cast<size_t>(t.wcol0 + col_base + col) *
                                                                             t.w_stride +
                                                                   static_cast<size_t>(b) * Q4_0_BYTES);
            const float dw = half_bits_to_float(p[0]);
            uint32_t qs[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                qs[q] = static_cast<uint32_t>(p[1 + 2 * q]) | (static_cast<uint32_t>(p[2 + 2 * q]) << 16);
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                const int2 ds = *reinterpret_cast<const int2 *>(ad + r * geo.ad_row + ad_index(b));
                const int dot = block_dot(qs, aq + r * geo.aq_row + aq_index(b, 0), ds.y);
                if constexpr (DOTS) {
                    if (r0 + r < t.rows) t.dots[(static_cast<size_t>(r0 + r) * t.ncols + col_base + col) * B + b] = dot;
                } else {
                    float v = static_cast<float>(dot) * dw;
                    v = v * __int_as_float(ds.x);
                    cb[(r * t.cpw + col) * geo.cbs + b] = v;
                }
            }
        }
    }
    if constexpr (DOTS) return;
    __syncthreads();
    sum_store<MR, FAST>(t, col_base, r0, tile_cols, cb, geo);
}

// A batch of linears (fast path, rows <= MR): one workgroup per work item
// (a column tile of one task, at most U * kThreads units), items in task
// order.  The hardware dispatcher starts the next item's workgroup the
// moment a slot frees.  (Measured on MI355X at the 154-linear decode step:
// 101 us per launch this way, 138 us with a persistent grid walking the
// item queue round-robin with one item of weight prefetch, and 5-15 %
// slower when the last 2-8 x CUs items are cut into halves or quarters to
// shorten the drain.)
// PC > 0 (one-row batches whose every task gives an fp32 activation of
// K <= 256 * 4 * PC): the activation row is requested before the weights.  A
// compile-time choice: under a run-time branch the compiler cannot count
// the weight loads issued after it and waits for all of them.
//
// S > 1 (one-row tiles of at most 64 * (NT / 64) / S units, NT = 256 or 512
// threads: the items of prefetching batches, whose fp32 row is quantised in
// the workgroup, and single linears over a native Q8_0 row): each unit is
// split over S waves.  Wave w
// takes part w % S -- blocks [8/S * part, +8/S) -- of units 64 * (w / S) +
// lane, loading only the 16-byte chunks that hold them, so each wave's share
// of the block dots is 1/S of a unit instead of a whole unit on fewer lanes.

// Part P (of S) of a unit: blocks [8/S * P, +8/S), which lie in 16-byte
// chunks [2P, 2P + 2] (S = 4) or [4P, 4P + 4] (S = 2) -- block i of a
// 144-byte unit spans bytes 18 i .. 18 i + 17.
template <int S>
struct UnitParts {
    static constexpr int kBlocks = 8 / S;
    static constexpr int kChunks = S == 4 ? 3 : 5;
    static constexpr int kChunkStep = S == 4 ? 2 : 4;  // first chunk of part P = kChunkStep * P
    static_assert((18 * kBlocks * (S - 1) + 18 * kBlocks - 1) / 16 == kChunkStep * (S - 1) + kChunks - 1,
                  "the last part's chunks end with the unit");
};

// The chunks of this wave's part (first chunk c0, the same for the whole
// wave) of unit u: one code path for every part, so every wave issues the
// same loads and the waits that follow count them exactly.
template <int S, int LAYOUT>
__device__ __forceinline__ void load_part(const Q4Task &t, int col_base, int G, int units, int u, int c0,
                                          uint32_t (&d)[4 * UnitParts<S>::kChunks]) {
    const int uc = min(u, units - 1);  // unconditional: lanes past the tile re-read its last unit
    const int col = uc / G;
    const int g = uc - col * G;
    if (LAYOUT == kLaneLayout || (LAYOUT == kEitherLayout && t.lanes)) {
        const size_t unit = static_cast<size_t>(t.wcol0 + col_base + col) * G + g;
        const QXT_GLOBAL v4u *src = global_in<v4u>(t.w + (unit / kLaneGroup) * kGroupBytes + (unit % kLaneGroup) * 16) +
                                    c0 * kLaneGroup;
#pragma unroll
        for (int v = 0; v < UnitParts<S>::kChunks; ++v) {
            const v4u x = __builtin_nontemporal_load(src + v * kLaneGroup);
            d[4 * v + 0] = x[0];
            d[4 * v + 1] = x[1];
            d[4 * v + 2] = x[2];
            d[4 * v + 3] = x[3];
        }
    } else {
        const QXT_GLOBAL v4u *src = global_in<v4u>(t.w + static_cast<size_t>(t.wcol0 + col_base + col) * t.w_stride +
                                                   static_cast<size_t>(g) * 144) +
                                    c0;
#pragma unroll
        for (int v = 0; v < UnitParts<S>::kChunks; ++v) {
            const v4u x = src[v];
            d[4 * v + 0] = x[0];
            d[4 * v + 1] = x[1];
            d[4 * v + 2] = x[2];
            d[4 * v + 3] = x[3];
        }
    }
}

// Block terms of part P of unit u (one row) into cb; `pr` holds the part's
// chunks as load_part left them.
template <int S, int P>
__device__ __forceinline__ void compute_part(int G, int units, int u, const uint32_t (&pr)[4 * UnitParts<S>::kChunks],
                                             const int *aq, const int *ad, float *cb, const Q4Lds &geo) {
    using Parts = UnitParts<S>;
    constexpr int NB = Parts::kBlocks, I0 = NB * P, W0 = 4 * Parts::kChunkStep * P;
    if (u >= units) return;
    // The unit's words at their places in a whole unit (register renaming only).
    uint32_t d[36];
#pragma unroll
    for (int k = 0; k < 4 * Parts::kChunks; ++k) d[W0 + k] = pr[k];
    const int col = u / G;
    const int g = u - col * G;
    int4 lo[NB], hi[NB];
    int2 ds[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int b = g * 8 + I0 + i;
        lo[i] = *reinterpret_cast<const int4 *>(aq + aq_index(b, 0));
        hi[i] = *reinterpret_cast<const int4 *>(aq + aq_index(b, 4));
        ds[i] = *reinterpret_cast<const int2 *>(ad + ad_index(b));
    }
    float terms[NB];
    auto do_block = [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        uint32_t sbits, qs[4];
        unit_block<I0 + i>(d, sbits, qs);
        const float v = static_cast<float>(block_dot(qs, lo[i], hi[i], ds[i].y)) * half_bits_to_float(sbits);
        terms[i] = v * __int_as_float(ds[i].x);
    };
    do_block(std::integral_constant<int, 0>{});
    do_block(std::integral_constant<int, 1>{});
    if constexpr (NB == 4) {
        do_block(std::integral_constant<int, 2>{});
        do_block(std::integral_constant<int, 3>{});
    }
    float *dst = cb + col * geo.cbs + g * 8 + I0;
    if constexpr (NB == 4) *reinterpret_cast<float4 *>(dst) = make_float4(terms[0], terms[1], terms[2], terms[3]);
    else *reinterpret_cast<float2 *>(dst) = make_float2(terms[0], terms[1]);
}

template <int LAYOUT, int PC, int S, int NT = kThreads>
__device__ __forceinline__ void batch_item_split(const Q4Task &t, int col_base, int ncols) {
    static_assert(S == 2 || S == 4, "a unit splits into 2 or 4 parts");
    extern __shared__ int lds[];
    const int B = t.blocks;
    const int G = B >> 3;
    const int units = ncols * G;
    // The activation is requested before the weights: an fp32 row (PC > 0,
    // quantised here) or a native Q8_0 row (PC == 0, blocks <= 512).
    float4 xv[PC > 0 ? PC : 1];
    Q8RowRegs<NT> a8;
    // (Native rows are not pinned ahead of the weights here: pinned, cfg0's
    // single linear measured 4.16 -> 4.55 us back to back on MI355X.)
    if constexpr (PC > 0) prefetch_row<PC, NT>(t, xv);
    else fetch_q8_row(t, a8);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int part = wave % S;
    const int u = (wave / S) * 64 + static_cast<int>(threadIdx.x & 63);
    uint32_t pr[4 * UnitParts<S>::kChunks];
    load_part<S, LAYOUT>(t, col_base, G, units, u, UnitParts<S>::kChunkStep * part, pr);
    const Q4Lds geo(B, true);
    int *aq = lds;
    int *ad = aq + geo.aq_row;
    float *cb = reinterpret_cast<float *>(ad + geo.ad_row);
    if constexpr (PC > 0) quantise_row<PC, NT>(t, xv, aq, ad, geo);
    else stage_q8_row(t, a8, aq, ad, geo);
    __syncthreads();
    if constexpr (S == 2) {
        if (part == 0) compute_part<2, 0>(G, units, u, pr, aq, ad, cb, geo);
        else compute_part<2, 1>(G, units, u, pr, aq, ad, cb, geo);
    } else {
        switch (part) {
            case 0: compute_part<4, 0>(G, units, u, pr, aq, ad, cb, geo); break;
            case 1: compute_part<4, 1>(G, units, u, pr, aq, ad, cb, geo); break;
            case 2: compute_part<4, 2>(G, units, u, pr, aq, ad, cb, geo); break;
            default: compute_part<4, 3>(G, units, u, pr, aq, ad, cb, geo); break;
        }
    }
    __syncthreads();
    sum_store<1, true, NT>(t, col_base, 0, ncols, cb, geo);
}

template <int MR, int U, int LAYOUT, int PC>
__device__ __forceinline__ void batch_item(const Q4Task &t, int col_base, int ncols) {
    extern __shared__ int lds[];
    const int B = t.blocks;
    const int G = B >> 3;
    const int units = ncols * G;
    static_assert(PC == 0 || MR == 1, "the activation prefetch serves one-row batches");
    float4 xv[PC > 0 ? PC : 1];
    Q8RowRegs<kThreads, 1> a8;
    if constexpr (PC > 0) prefetch_row<PC>(t, xv);
    if constexpr (PC == kQ8RowPrefetch) {
        fetch_q8_row(t, a8);
        pin_memory_order();
    }
    uint32_t wr[U][36];
    load_units<U, LAYOUT, (PC != 0)>(t, col_base, G, units, 0, wr);
    const Q4Lds geo(B, true);
    int *aq = lds;
    int *ad = aq + MR * geo.aq_row;
    float *cb = reinterpret_cast<float *>(ad + MR * geo.ad_row);
    if constexpr (PC > 0) quantise_row<PC>(t, xv, aq, ad, geo);
    else if constexpr (PC == kQ8RowPrefetch) stage_q8_row(t, a8, aq, ad, geo);
    else stage_activation<MR>(t, 0, aq, ad, geo);
    __syncthreads();
    compute_fast<MR, U, false>(t, col_base, 0, G, units, 0, wr, aq, ad, cb, geo);
    __syncthreads();
    sum_store<MR, true>(t, col_base, 0, ncols, cb, geo);
}

template <int MR, int U, int LAYOUT, int PC, int S = 1, int NT = kThreads>
__device__ __forceinline__ void batch_item_any(const Q4Task &t, int col_base, int ncols) {
    if constexpr (S > 1) batch_item_split<LAYOUT, PC, S, NT>(t, col_base, ncols);
    else batch_item<MR, U, LAYOUT, PC>(t, col_base, ncols);
}

template <int MR, int U, int LAYOUT, int PC, int S = 1, int NT = kThreads>
__global__ __launch_bounds__(NT) void q4_0_batch_kernel(const Q4Task *__restrict__ tasks,
                                                        const Q4Item *__restrict__ items) {
    const Q4Item item = items[blockIdx.x];
    batch_item_any<MR, U, LAYOUT, PC, S, NT>(tasks[item.task], item.col_base, item.ncols);
}

// A batch of at most kArgTasks tasks travels in the kernel arguments: each
// workgroup finds its task and column tile from its index, without the two
// dependent reads of a device table (item, then task) before its first
// weight or activation request.  Task j's items start at first_item[j]
// (INT_MAX past the last task) and are its column tiles of cpw columns in
// order.
constexpr int kArgTasks = 4;
struct Q4ArgBatch {
    int first_item[kArgTasks];
    Q4Task task[kArgTasks];
};

template <int MR, int U, int LAYOUT, int PC, int S = 1, int NT = kThreads>
__global__ __launch_bounds__(NT) void q4_0_arg_batch_kernel(Q4ArgBatch a) {
    const int i = static_cast<int>(blockIdx.x);
    int ti = 0;
#pragma unroll
    for (int j = 1; j < kArgTasks; ++j) ti += i >= a.first_item[j] ? 1 : 0;
    const Q4Task t = a.task[ti];
    const int col_base = (i - a.first_item[ti]) * t.cpw;
    batch_item_any<MR, U, LAYOUT, PC, S, NT>(t, col_base, min(t.cpw, t.ncols - col_base));
}

// The four-row matrix-core tiles (compute_mfma4): workgroup (x, y) of NT
// threads owns columns [x * cpw, +cpw) and rows [4 y, +4), one unit per
// thread and round.
template <int LAYOUT, int NT>
__global__ __launch_bounds__(NT) void q4_0_mfma4_kernel(Q4Task t) {
    constexpr int MR = 4, U = 1;
    extern __shared__ int lds[];
    const int col_base = blockIdx.x * t.cpw;
    const int r0 = blockIdx.y * MR;
    const int B = t.blocks;
    const Q4Lds geo(B, true);
    int *aq = lds;                                                 // [MR][aq_row]
    int *ad = aq + MR * geo.aq_row;                                // SCALES4 records
    float *cb = reinterpret_cast<float *>(ad + MR * geo.ad_row);  // [MR][cpw][cbs]
    const int tile_cols = min(t.cpw, t.ncols - col_base);
    const int G = B >> 3;
    const int units = tile_cols * G;
    uint32_t wr[U][36];
    // The activation first, then two rounds of weights, so that the
    // staging waits only for the activation and the weight stream runs
    // through it.  The loads of every round are unconditional (lanes
    // past the tile re-read its last unit), so the compiler counts them
    // exactly in every wait.
    Q8RowRegs<NT> a;
    fetch_q8_rows(t, r0, a);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first
    uint32_t wn[U][36];
    const int lg = __builtin_ctz(G);
    load_units_m4<U, LAYOUT, NT>(t, col_base, lg, units, 0, wr);
    load_units_m4<U, LAYOUT, NT>(t, col_base, lg, units, U * NT, wn);
    __builtin_amdgcn_sched_barrier(0);
    stage_q8_rows(t, a, aq, ad, geo);
    __syncthreads();
    // Two register sets in turn (no copies between them): each is
    // refilled with the round after next as soon as it is computed.
    constexpr int R = U * NT;
    for (int first = 0;;) {
        compute_mfma4<U, NT>(t, lg, units, first, wr, aq, ad, cb, geo);
        load_units_m4<U, LAYOUT, NT>(t, col_base, lg, units, first + 2 * R, wr);
        if ((first += R) >= units) break;
        compute_mfma4<U, NT>(t, lg, units, first, wn, aq, ad, cb, geo);
        load_units_m4<U, LAYOUT, NT>(t, col_base, lg, units, first + 2 * R, wn);
        if ((first += R) >= units) break;
    }
    __syncthreads();
    sum_store<MR, true, NT>(t, col_base, r0, tile_cols, cb, geo);
}

// The four-row matrix-core tiles with each unit split over two waves of a
// 512-thread workgroup: wave w computes blocks [4 (w & 1), +4) of the units
// of wave w >> 1 of q4_0_mfma4_kernel<LAYOUT, 256>, loading only the five
// 16-byte chunks [4 (w & 1), +5) that hold them (one code path for both
// halves, the chunk offset being the same for the whole wave).
template <int S>
__device__ __forceinline__ int mfma4_split_unit(int lg, int first) {
    const int lane = threadIdx.x & 63;
    const int b = lane >> 2, p = lane & 3;
    const int perm = ((((b >> lg) << 2) + p) << lg) + (b & ((1 << lg) - 1));
    return first + (((static_cast<int>(threadIdx.x) >> 6) / S) << 6) + perm;
}

template <int LAYOUT, int S>
__device__ __forceinline__ void load_mfma4_half(const Q4Task &t, int col_base, int lg, int units, int first, int c0,
                                                uint32_t (&d)[4 * UnitParts<S>::kChunks]) {
    const int u = min(mfma4_split_unit<S>(lg, first), units - 1);
    const int col = u >> lg, g = u & ((1 << lg) - 1);
    const QXT_GLOBAL v4u *src;
    if constexpr (LAYOUT == kLaneLayout) {
        const size_t unit = (static_cast<size_t>(t.wcol0 + col_base + col) << lg) + g;
        src = global_in<v4u>(t.w + (unit / kLaneGroup) * kGroupBytes + (unit % kLaneGroup) * 16) + c0 * kLaneGroup;
    } else {
        src = global_in<v4u>(t.w + static_cast<size_t>(t.wcol0 + col_base + col) * t.w_stride +
                             static_cast<size_t>(g) * 144) +
              c0;
    }
#pragma unroll
    for (int v = 0; v < UnitParts<S>::kChunks; ++v) {
        const v4u x = LAYOUT == kLaneLayout ? __builtin_nontemporal_load(src + v * kLaneGroup) : src[v];
        d[4 * v + 0] = x[0];
        d[4 * v + 1] = x[1];
        d[4 * v + 2] = x[2];
        d[4 * v + 3] = x[3];
    }
}

template <int S, int H>
__device__ __forceinline__ void compute_mfma4_half(int lg, int units, int first,
                                                   const uint32_t (&pr)[4 * UnitParts<S>::kChunks], const int *aq,
                                                   const int *ad, float *cb, const Q4Lds &geo, int cpw) {
    typedef int v4i_t __attribute__((ext_vector_type(4)));
    using Parts = UnitParts<S>;
    constexpr int NB = Parts::kBlocks;
    const int lane = threadIdx.x & 63;
    const int b = lane >> 2, p = lane & 3;
    const int g = b & ((1 << lg) - 1);
    const int *arow = aq + p * geo.aq_row;
    const int u = mfma4_split_unit<S>(lg, first);
    const int col = u >> lg;
    uint32_t d[36];  // the unit's words at their places (register renaming only)
#pragma unroll
    for (int k = 0; k < 4 * Parts::kChunks; ++k) d[4 * Parts::kChunkStep * H + k] = pr[k];
    float terms[4][NB];
    auto do_block = [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr int I = NB * H + i;
        uint32_t sbits, qs[4];
        unit_block<I>(d, sbits, qs);
        const int bg = g * 8 + I;
        const int4 lo = *reinterpret_cast<const int4 *>(arow + aq_index(bg, 0));
        const int4 hi = *reinterpret_cast<const int4 *>(arow + aq_index(bg, 4));
        const int4 s8 = *reinterpret_cast<const int4 *>(ad + aq_index(bg, 0));
        const float4 da = *reinterpret_cast<const float4 *>(ad + aq_index(bg, 4));
        v4i_t acc = {s8.x, s8.y, s8.z, s8.w};
        acc = __builtin_amdgcn_mfma_i32_4x4x4i8(lo.x, static_cast<int>(qs[0] & 0x0F0F0F0Fu), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_4x4x4i8(lo.y, static_cast<int>(qs[1] & 0x0F0F0F0Fu), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_4x4x4i8(lo.z, static_cast<int>(qs[2] & 0x0F0F0F0Fu), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_4x4x4i8(lo.w, static_cast<int>(qs[3] & 0x0F0F0F0Fu), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_4x4x4i8(hi.x, static_cast<int>((qs[0] >> 4) & 0x0F0F0F0Fu), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_4x4x4i8(hi.y, static_cast<int>((qs[1] >> 4) & 0x0F0F0F0Fu), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_4x4x4i8(hi.z, static_cast<int>((qs[2] >> 4) & 0x0F0F0F0Fu), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_4x4x4i8(hi.w, static_cast<int>((qs[3] >> 4) & 0x0F0F0F0Fu), acc, 0, 0, 0);
        const float dw = half_bits_to_float(sbits);
        const float das[4] = {da.x, da.y, da.z, da.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float v = static_cast<float>(acc[r]) * dw;
            v = v * das[r];
            terms[r][i] = v;
        }
    };
    do_block(std::integral_constant<int, 0>{});
    do_block(std::integral_constant<int, 1>{});
    if constexpr (NB == 4) {
        do_block(std::integral_constant<int, 2>{});
        do_block(std::integral_constant<int, 3>{});
    }
    if (u < units) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float *dst = cb + (r * cpw + col) * geo.cbs + g * 8 + NB * H;
            if constexpr (NB == 4) *reinterpret_cast<float4 *>(dst) = make_float4(terms[r][0], terms[r][1], terms[r][2], terms[r][3]);
            else *reinterpret_cast<float2 *>(dst) = make_float2(terms[r][0], terms[r][1]);
        }
    }
}

template <int LAYOUT, int S>
__global__ __launch_bounds__(S * kThreads) void q4_0_mfma4_split_kernel(Q4Task t) {
    constexpr int MR = 4, NT = S * kThreads;
    extern __shared__ int lds[];
    const int col_base = blockIdx.x * t.cpw;
    const int r0 = blockIdx.y * MR;
    const int B = t.blocks;
    const Q4Lds geo(B, true);
    int *aq = lds;
    int *ad = aq + MR * geo.aq_row;
    float *cb = reinterpret_cast<float *>(ad + MR * geo.ad_row);
    const int tile_cols = min(t.cpw, t.ncols - col_base);
    const int G = B >> 3;
    const int units = tile_cols * G;
    const int part = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)) % S;
    const int c0 = UnitParts<S>::kChunkStep * part;
    Q8RowRegs<NT> a;
    fetch_q8_rows(t, r0, a);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first
    const int lg = __builtin_ctz(G);
    constexpr int R = NT / S;  // units per round: S waves per unit
    constexpr int W = 4 * UnitParts<S>::kChunks;
    uint32_t wr[W], wn[W];
    load_mfma4_half<LAYOUT, S>(t, col_base, lg, units, 0, c0, wr);
    load_mfma4_half<LAYOUT, S>(t, col_base, lg, units, R, c0, wn);
    __builtin_amdgcn_sched_barrier(0);
    stage_q8_rows(t, a, aq, ad, geo);
    __syncthreads();
    auto compute = [&](int first, const uint32_t (&pr)[W]) {
        if constexpr (S == 2) {
            if (part == 0) compute_mfma4_half<2, 0>(lg, units, first, pr, aq, ad, cb, geo, t.cpw);
            else compute_mfma4_half<2, 1>(lg, units, first, pr, aq, ad, cb, geo, t.cpw);
        } else {
            switch (part) {
                case 0: compute_mfma4_half<4, 0>(lg, units, first, pr, aq, ad, cb, geo, t.cpw); break;
                case 1: compute_mfma4_half<4, 1>(lg, units, first, pr, aq, ad, cb, geo, t.cpw); break;
                case 2: compute_mfma4_half<4, 2>(lg, units, first, pr, aq, ad, cb, geo, t.cpw); break;
                default: compute_mfma4_half<4, 3>(lg, units, first, pr, aq, ad, cb, geo, t.cpw); break;
            }
        }
    };
    for (int first = 0;;) {
        compute(first, wr);
        load_mfma4_half<LAYOUT, S>(t, col_base, lg, units, first + 2 * R, c0, wr);
        if ((first += R) >= units) break;
        compute(first, wn);
        load_mfma4_half<LAYOUT, S>(t, col_base, lg, units, first + 2 * R, c0, wn);
        if ((first += R) >= units) break;
    }
    __syncthreads();
    sum_store<MR, true, NT>(t, col_base, r0, tile_cols, cb, geo);
}

// A one-row single linear over native Q8_0 activations whose tiles hold at
// most 256 units: the stage kernels' split units (batch_item_split), one
// workgroup per column tile.
template <int LAYOUT, int S, int NT>
__global__ __launch_bounds__(NT) void q4_0_split_kernel(Q4Task t) {
    const int col_base = static_cast<int>(blockIdx.x) * t.cpw;
    batch_item_split<LAYOUT, 0, S, NT>(t, col_base, min(t.cpw, t.ncols - col_base));
}

// Threads per matrix-core tile workgroup (measured on MI355X, cfg2 back to
// back: 512 threads, two waves per SIMD, 11.2 / 6.8 us against 9.7 / 5.5 us
// with 256 at N = 11008 / 4096).
constexpr int kMfma4Threads = kThreads;

// Units each thread owns per round on the fast path.
constexpr int units_per_thread(int mr) { return mr == 1 ? 2 : 1; }

// Units per thread of the activation-prefetch batch kernels (one-row tasks;
// one unit: narrower tiles, fewer idle lanes re-reading a unit -- staged
// decode 0.47 -> 0.43 ms against two).
#ifndef QXT_PREFETCH_UNITS
#define QXT_PREFETCH_UNITS 1
#endif
constexpr int kPrefetchUnits = QXT_PREFETCH_UNITS;

#ifndef QXT_BALANCE_PREFETCH
#define QXT_BALANCE_PREFETCH 1
#endif
constexpr bool kBalancePrefetchTiles = QXT_BALANCE_PREFETCH != 0;
#ifndef QXT_BALANCE_MAXK
#define QXT_BALANCE_MAXK 4
#endif
constexpr uint64_t kMaxBalancedPerCu = QXT_BALANCE_MAXK;

// Whether one-row fp32 batches too large for the fused path (a whole decode
// step) still quantise inside each workgroup, with the activation prefetch,
// instead of running a pre-pass launch.
#ifndef QXT_PREFETCH_LARGE
#define QXT_PREFETCH_LARGE 0
#endif
constexpr bool kPrefetchLargeBatches = QXT_PREFETCH_LARGE != 0;

#ifndef QXT_SPLIT_UNITS
#define QXT_SPLIT_UNITS 1
#endif
constexpr bool kSplitUnits = QXT_SPLIT_UNITS != 0;
#ifndef QXT_WIDE_SPLIT
#define QXT_WIDE_SPLIT 1
#endif
constexpr bool kWideSplit = QXT_WIDE_SPLIT != 0;

#ifndef QXT_MFMA4_SPLIT
#define QXT_MFMA4_SPLIT 1
#endif
constexpr bool kMfma4Split = QXT_MFMA4_SPLIT != 0;
#ifndef QXT_MFMA4_SPLIT_WAVES
#define QXT_MFMA4_SPLIT_WAVES 2
#endif
constexpr int kMfma4SplitWaves = QXT_MFMA4_SPLIT_WAVES;

#ifndef QXT_SPLIT_SINGLE
#define QXT_SPLIT_SINGLE 1
#endif
constexpr bool kSplitSingle = QXT_SPLIT_SINGLE != 0;

#ifndef QXT_ARG_BATCH
#define QXT_ARG_BATCH 1
#endif

#ifndef QXT_Q8_ROW_PREFETCH
#define QXT_Q8_ROW_PREFETCH 1
#endif
constexpr bool kQ8RowPrefetchBatches = QXT_Q8_ROW_PREFETCH != 0;
constexpr bool kArgBatches = QXT_ARG_BATCH != 0;

static_assert(kPrefetchUnits >= 1 && kPrefetchUnits <= units_per_thread(1),
              "a prefetch plan must fit the one-row batch kernel it falls back to");

bool fast_path(const Q4Task &t) { return t.blocks % 8 == 0 && aligned(t.w, 16) && t.w_stride % 16 == 0; }

// Bytes of the lane layout of `columns` x `blocks` (whole groups), or 0 when
// blocks % 8 != 0.
size_t lanes_bytes(uint64_t columns, uint64_t blocks) {
    if (blocks == 0 || blocks % 8 || columns == 0) return 0;
    const uint64_t units = columns * (blocks / 8);
    return static_cast<size_t>((units + kLaneGroup - 1) / kLaneGroup * kGroupBytes);
}

// Columns per workgroup (at most `max_cpw`) and dynamic LDS bytes for a task,
// or an error status.  Normally a workgroup takes one round of units (a
// unit per thread, U per thread on the fast path) within kMaxLds; `wide`
// takes max_cpw columns, several rounds, within the whole LDS of a
// workgroup.  A K whose single-column tile exceeds kMaxLds also runs, on
// fewer workgroups per CU, up to the whole LDS (about K = 111k at one row,
// 55k at two, 37k at three and 27k at four rows).
int plan_task(Q4Task &t, int mr, bool fast, bool dots, size_t *lds, int max_cpw = 1 << 30, bool wide = false,
              int upt = 0) {
    const Q4Lds geo(t.blocks, fast);
    const int units_per_col = fast ? t.blocks / 8 : t.blocks;
    const int per_round = kThreads * (fast ? (upt > 0 ? upt : units_per_thread(mr)) : 1);
    int cpw = units_per_col >= per_round ? 1 : per_round / units_per_col;
    if (wide) cpw = max_cpw;
    cpw = std::max(1, std::min({cpw, t.ncols, max_cpw}));
    const size_t narrow = geo.words(mr, dots ? 0 : 1) * 4;
    const size_t cap = (wide || narrow > kMaxLds) ? kMaxLdsWide : kMaxLds;
    if (narrow > cap)
        return fail(QXT_CAPABILITY_MISSING, "q4_0 linear: K=%d at %d rows needs %zu bytes of LDS (> %zu)",
                    t.blocks * 32, mr, narrow, cap);
    while (cpw > 1 && geo.words(mr, dots ? 0 : cpw) * 4 > cap) --cpw;
    *lds = geo.words(mr, dots ? 0 : cpw) * 4;
    t.cpw = cpw;
    return QXT_OK;
}

template <int MR, bool DOTS>
int launch_single(Q4Task t, hipStream_t stream) {
    const bool fast = fast_path(t);
    // A single linear is latency-bound unless its grid covers the chip: cap
    // the tile width so that there are at least two workgroups per CU.  Four
    // rows on the fast path instead give each CU one wide workgroup that
    // streams its columns in rounds with the next round's weights in flight
    // (measured on MI355X, cfg2: 14.8 -> 13.4 us at N = 11008 and 8.7 -> 7.6 us
    // at N = 4096, K = 4096; the narrow tiles' LDS held N = 11008 to two
    // workgroups per CU, 1.34 rounds).
    const int row_groups = (t.rows + MR - 1) / MR;
    const bool wide = MR == 4 && fast && !DOTS;
    const long want = (wide ? 1L : 2L) * compute_units();
    const int max_cpw = static_cast<int>(std::max<long>(1, (static_cast<long>(t.ncols) * row_groups + want - 1) / want));
    size_t lds = 0;
    int rc = plan_task(t, MR, fast, DOTS, &lds, max_cpw, wide);
    if (rc != QXT_OK) return rc;
    dim3 grid((t.ncols + t.cpw - 1) / t.cpw, row_groups, 1);
    constexpr int U = units_per_thread(MR);
    const char *name = DOTS ? "q4_0_block_dots_kernel" : "q4_0_linear_kernel";
    if constexpr (!DOTS) {
        // Four rows with a block range per unit that divides 16 (K <= 4096):
        // the matrix-core tiles (measured on MI355X, cfg2 over lane-layout
        // weights back to back: 12.9 -> 9.6 us at N = 11008 and 7.4 -> 5.5 us
        // at N = 4096 against the v_dot4 wide tiles).
        const int G = t.blocks / 8;
        if constexpr (MR == 4)
            if (fast && t.x == nullptr && G <= 16 && 16 % G == 0)
            {
                // Tiles of several rounds: each unit over two waves of 512
                // (measured on MI355X, cfg2 back to back: N = 11008, three
                // rounds, 9.7 -> 9.3 us, and 10.1 us over four waves of 1024;
                // N = 4096, one round, 5.5 -> 5.65 us, so single-round tiles
                // keep one wave per unit).
                if (kMfma4Split && t.cpw * G > kMfma4Threads)
                    return t.lanes ? launch(name, q4_0_mfma4_split_kernel<kLaneLayout, kMfma4SplitWaves>, grid,
                                            dim3(kMfma4SplitWaves * kThreads), lds, stream, t)
                                   : launch(name, q4_0_mfma4_split_kernel<kNativeRows, kMfma4SplitWaves>, grid,
                                            dim3(kMfma4SplitWaves * kThreads), lds, stream, t);
                return t.lanes ? launch(name, q4_0_mfma4_kernel<kLaneLayout, kMfma4Threads>, grid,
                                        dim3(kMfma4Threads), lds, stream, t)
                               : launch(name, q4_0_mfma4_kernel<kNativeRows, kMfma4Threads>, grid,
                                        dim3(kMfma4Threads), lds, stream, t);
            }
        if constexpr (MR == 1) {
            const int units = t.cpw * G;
            if (kSplitSingle && fast && t.x == nullptr && t.blocks <= 512 && units <= 4 * kLaneGroup) {
                // Tiles of at most 64 units: 4 waves of 256 threads per unit
                // (512 threads measured 0.5 % slower on the per-linear decode
                // schedule); more: 512 threads, 4 (up to 128 units) or 2
                // waves per unit.
                if (units <= kLaneGroup)
                    return t.lanes ? launch(name, q4_0_split_kernel<kLaneLayout, 4, kThreads>, grid, dim3(kThreads),
                                            lds, stream, t)
                                   : launch(name, q4_0_split_kernel<kNativeRows, 4, kThreads>, grid, dim3(kThreads),
                                            lds, stream, t);
                if (units <= 2 * kLaneGroup)
                    return t.lanes ? launch(name, q4_0_split_kernel<kLaneLayout, 4, 2 * kThreads>, grid,
                                            dim3(2 * kThreads), lds, stream, t)
                                   : launch(name, q4_0_split_kernel<kNativeRows, 4, 2 * kThreads>, grid,
                                            dim3(2 * kThreads), lds, stream, t);
                return t.lanes ? launch(name, q4_0_split_kernel<kLaneLayout, 2, 2 * kThreads>, grid,
                                        dim3(2 * kThreads), lds, stream, t)
                               : launch(name, q4_0_split_kernel<kNativeRows, 2, 2 * kThreads>, grid,
                                        dim3(2 * kThreads), lds, stream, t);
            }
        }
        if (fast && t.lanes)
            return launch(name, q4_0_linear_kernel<MR, U, true, false, kLaneLayout>, grid, dim3(kThreads), lds, stream,
                          t);
    }
    if (fast) return launch(name, q4_0_linear_kernel<MR, U, true, DOTS>, grid, dim3(kThreads), lds, stream, t);
    return launch(name, q4_0_linear_kernel<MR, 1, false, DOTS>, grid, dim3(kThreads), lds, stream, t);
}

template <bool DOTS>
int dispatch_single(const Q4Task &t, hipStream_t stream) {
    switch (t.rows >= 4 ? 4 : t.rows) {
        case 1: return launch_single<1, DOTS>(t, stream);
        case 2: return launch_single<2, DOTS>(t, stream);
        case 3: return launch_single<3, DOTS>(t, stream);
        default: return launch_single<4, DOTS>(t, stream);
    }
}

}  // namespace

// Whether a single linear of `rows` rows and `blocks` blocks fits a workgroup's
// LDS on the v_dot4 path (the path every row count below 16 takes, and larger
// row counts when the matrix-core kernel does not apply).
int q4_0_linear_capability(uint32_t rows, uint32_t blocks) {
    Q4Task t{};
    t.blocks = static_cast<int>(blocks);
    t.ncols = 1;
    const int mr = rows >= 4 ? 4 : static_cast<int>(rows);
    size_t lds = 0;
    return plan_task(t, mr, blocks % 8 == 0, false, &lds, 1, mr == 4 && blocks % 8 == 0);
}

namespace {

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

struct qxt_q4_0_batch {
    void *device_tables = nullptr;  // [Q4Task x count][Q4Item x items][Q8Job x jobs][Q8Chunk x chunks]
    void *q8_staging = nullptr;     // Q8_0 blocks of the fp32 activations the pre-pass quantises
    const Q4Task *tasks = nullptr;
    const Q4Item *items = nullptr;
    const Q8Job *jobs = nullptr;
    const Q8Chunk *chunks = nullptr;
    uint32_t task_count = 0;
    uint32_t item_count = 0;
    uint32_t chunk_count = 0;
    uint32_t grid = 0;
    int mr = 1;
    int layout = 0;  // WeightLayout of every task (kEitherLayout when mixed)
    int prefetch = 0;  // activation chunks per thread prefetched (every task one fp32 row), kQ8RowPrefetch, or 0
    int upt = 1;       // units per thread of the batch kernel
    int split = 1;     // waves per unit (one-row prefetch batches of narrow items)
    int threads = kThreads;  // 256, or 512 / 1024 for split prefetch batches
    size_t lds = 0;
    bool in_args = false;  // tasks and items travel in the kernel arguments
    Q4ArgBatch args{};
};

namespace qxt {
namespace {

// The two forms of one batch kernel: tasks and items in device tables, or
// (at most kArgTasks tasks) in the kernel arguments.
struct BatchKernel {
    void (*tables)(const Q4Task *, const Q4Item *);
    void (*args)(Q4ArgBatch);
};

template <int MR, int U, int LAYOUT, int PC, int S, int NT>
BatchKernel batch_kernels() {
    return {q4_0_batch_kernel<MR, U, LAYOUT, PC, S, NT>, q4_0_arg_batch_kernel<MR, U, LAYOUT, PC, S, NT>};
}

template <int MR, int U, int PC, int S = 1, int NT = kThreads>
BatchKernel batch_kernel_for(int layout) {
    return layout == kLaneLayout    ? batch_kernels<MR, U, kLaneLayout, PC, S, NT>()
           : layout == kNativeRows ? batch_kernels<MR, U, kNativeRows, PC, S, NT>()
                                   : batch_kernels<MR, U, kEitherLayout, PC, S, NT>();
}

// One-row prefetch batches.  split: waves per unit; wide: 512-thread
// workgroups (the row's chunks over twice the threads).
template <int U, int PC>
BatchKernel prefetch_kernel_split(int layout, int split, int threads) {
    if constexpr (U == 1) {
        if (threads == 2 * kThreads && split == 4) return batch_kernel_for<1, 1, (PC + 1) / 2, 4, 2 * kThreads>(layout);
        if (threads == 2 * kThreads) return batch_kernel_for<1, 1, (PC + 1) / 2, 2, 2 * kThreads>(layout);
        if (split == 4) return batch_kernel_for<1, 1, PC, 4>(layout);
        if (split == 2) return batch_kernel_for<1, 1, PC, 2>(layout);
    }
    return batch_kernel_for<1, U, PC>(layout);
}

template <int U>
BatchKernel prefetch_kernel(int layout, int prefetch, int split, int threads) {
    switch (prefetch) {
        case 2: return prefetch_kernel_split<U, 2>(layout, split, threads);
        case 4: return prefetch_kernel_split<U, 4>(layout, split, threads);
        default: return prefetch_kernel_split<U, kMaxPrefetchChunks>(layout, split, threads);
    }
}

// The kernel of a batch: rows per task group, weight layout, activation
// chunks prefetched per thread (0: none), units per thread and waves per
// unit.
BatchKernel batch_kernel(int mr, int layout, int prefetch, int upt, int split, int threads) {
    if (mr != 1) return batch_kernel_for<4, units_per_thread(4), 0>(layout);
    if (prefetch == 0) return batch_kernel_for<1, units_per_thread(1), 0>(layout);
    if (prefetch == kQ8RowPrefetch) return batch_kernel_for<1, units_per_thread(1), kQ8RowPrefetch>(layout);
    return upt == 1 ? prefetch_kernel<1>(layout, prefetch, split, threads)
                    : prefetch_kernel<units_per_thread(1)>(layout, prefetch, split, threads);
}

}  // namespace
}  // namespace qxt

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
    // Prefill-sized row counts run on the int8 matrix cores (bit-identical result).
    if (q4_0_tiled_native_supported(activation_row_stride, weight_row_stride, rows, blocks, weight_column_start,
                                    column_count))
        return q4_0_tiled_native(activation, activation_row_stride, weight, weight_row_stride, destination,
                                 destination_row_stride, rows, blocks, weight_column_start, output_column_start,
                                 column_count, as_stream(stream));
    // Long rows spread their blocks over the lanes instead: more than 64
    // blocks with two or more activation rows (128 for four rows over fewer
    // than 8192 columns), more than 256 with one (measured on MI355X, event-timed: M=4
    // K=5632 8.0 -> 6.5 us, K=8192 12.5 -> 9.9, K=11008 16.2 -> 14.1,
    // K=14336 30.2 -> 14.8; M=2 K=4096 10.7 -> 9.0, K=5632 7.4 -> 5.6; one row
    // at K=11008 / 14336 11.1 -> 10.4 / 12.7 -> 11.6 us; where the other
    // kernels stay they were ahead: M=4 K=4096 N=4096 6.1 against 6.7 us,
    // one row at K=5632 / 8192 4.8 / 6.8 against 5.5 / 7.8 us).
    // Four rows over fewer than 8192 columns keep the matrix-core kernels up to
    // 128 blocks; five or more rows, and four over wider outputs, spread from
    // 65 blocks (M=4 K=4096: N=11008 10.0 -> 9.6 us, N=14336 13.3 -> 12.0 us,
    // N=8192 9.0 -> 8.4 us; M=5 / 8 K=4096 N=11008 20.6 / 20.6 -> 17.1 / 16.5
    // us; M=12 K=4096 N=4096 14.9 -> 10.2 us; M=5 / 8 N=4096 8.0 / 8.4 ->
    // 7.8 / 8.2 us; from 33 blocks, M=6 and 8 at K=2048 were no faster).
    const uint32_t spread_above = rows == 1 ? 256u : (rows != 4 || column_count >= 8192u) ? 64u : 128u;
    if (blocks > spread_above) {
        rc = q4_0_stream_native(activation, activation_row_stride, weight, weight_row_stride, destination,
                                destination_row_stride, rows, blocks, weight_column_start, output_column_start,
                                column_count, as_stream(stream));
        if (rc != QXT_CAPABILITY_MISSING) return rc;
    }
    Q4Task t{};
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
    return dispatch_single<false>(t, as_stream(stream));
}

size_t qxt_q4_0_lanes_bytes(uint32_t columns, uint32_t blocks) { return lanes_bytes(columns, blocks); }

int qxt_q4_0_pack_lanes(const void *weight, size_t weight_row_stride, void *packed, size_t packed_bytes,
                        uint32_t columns, uint32_t blocks, void *stream) {
    if (weight == nullptr || packed == nullptr) return fail(QXT_INVALID_ARGUMENT, "q4_0 pack lanes: null pointer");
    const size_t need = lanes_bytes(columns, blocks);
    if (need == 0) return fail(QXT_INVALID_ARGUMENT, "q4_0 pack lanes: needs columns > 0 and blocks %% 8 == 0");
    if (blocks > (1u << 20) || columns > (1u << 30))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 pack lanes: problem too large");
    if (!aligned(weight, 16) || !aligned(packed, 16) || weight_row_stride % 16 ||
        weight_row_stride < static_cast<size_t>(blocks) * Q4_0_BYTES)
        return fail(QXT_INVALID_ARGUMENT, "q4_0 pack lanes: weight rows and packed output must be 16-byte aligned");
    if (packed_bytes < need)
        return fail(QXT_INVALID_ARGUMENT, "q4_0 pack lanes: packed buffer holds %zu of %zu bytes", packed_bytes, need);
    int rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    const size_t chunks = need / 16;
    const size_t grid = (chunks + kThreads - 1) / kThreads;
    if (grid > 0x7FFFFFFFu) return fail(QXT_INVALID_ARGUMENT, "q4_0 pack lanes: matrix too large");
    return launch("q4_0_pack_lanes_kernel", pack_lanes_kernel, dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0,
                  as_stream(stream), static_cast<const uint8_t *>(weight), weight_row_stride,
                  static_cast<uint8_t *>(packed), static_cast<size_t>(columns) * (blocks / 8), chunks,
                  static_cast<int>(blocks / 8));
}

int qxt_ggml_q4_0_q8_0_linear_lanes(const void *activation, size_t activation_row_stride, const void *packed_weight,
                                    uint32_t weight_columns, float *destination, size_t destination_row_stride,
                                    uint32_t rows, uint32_t blocks, uint32_t weight_column_start,
                                    uint32_t output_column_start, uint32_t column_count, void *stream) {
    const size_t w_stride = static_cast<size_t>(blocks) * Q4_0_BYTES;
    int rc = validate_q4(activation, activation_row_stride, packed_weight, w_stride, rows, blocks, column_count);
    if (rc != QXT_OK) return rc;
    if (blocks % 8 || !aligned(packed_weight, 16))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 lanes linear: needs blocks %% 8 == 0 and a 16-byte aligned weight");
    if (static_cast<uint64_t>(weight_column_start) + column_count > weight_columns)
        return fail(QXT_INVALID_ARGUMENT, "q4_0 lanes linear: columns past the packed matrix");
    if (destination == nullptr || !aligned(destination, 4) || destination_row_stride % 4 ||
        destination_row_stride < (static_cast<size_t>(output_column_start) + column_count) * sizeof(float))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 lanes linear: bad destination");
    if (static_cast<uint64_t>(output_column_start) + column_count > (1ull << 31))
        return fail(QXT_INVALID_ARGUMENT, "q4_0 lanes linear: column range overflows");
    rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    Q4Task t{};
    t.act = static_cast<const uint8_t *>(activation);
    t.act_stride = activation_row_stride;
    t.w = static_cast<const uint8_t *>(packed_weight);
    t.w_stride = w_stride;
    t.lanes = 1;
    t.y = destination;
    t.y_stride = destination_row_stride;
    t.rows = static_cast<int>(rows);
    t.blocks = static_cast<int>(blocks);
    t.wcol0 = static_cast<int>(weight_column_start);
    t.ocol0 = static_cast<int>(output_column_start);
    t.ncols = static_cast<int>(column_count);
    return dispatch_single<false>(t, as_stream(stream));
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
    Q4Task t{};
    t.act = static_cast<const uint8_t *>(activation);
    t.act_stride = activation_row_stride;
    t.w = static_cast<const uint8_t *>(weight);
    t.w_stride = weight_row_stride;
    t.dots = dots;
    t.rows = static_cast<int>(rows);
    t.blocks = static_cast<int>(blocks);
    t.wcol0 = static_cast<int>(weight_column_start);
    t.ncols = static_cast<int>(column_count);
    return dispatch_single<true>(t, as_stream(stream));
}

int qxt_q4_0_batch_prepare(const qxt_q4_0_task *tasks, uint32_t count, qxt_q4_0_batch **out) {
    if (out == nullptr) return fail(QXT_INVALID_ARGUMENT, "q4_0 batch: null output handle");
    *out = nullptr;
    if (tasks == nullptr || count == 0) return fail(QXT_INVALID_ARGUMENT, "q4_0 batch: no tasks");
    std::vector<Q4Task> host(count);
    std::vector<Q8Job> jobs;
    std::vector<uint32_t> job_task;
    uint32_t max_rows = 1;
    for (uint32_t i = 0; i < count; ++i) {
        const qxt_q4_0_task &d = tasks[i];
        if ((d.x == nullptr) == (d.activation == nullptr))
            return fail(QXT_INVALID_ARGUMENT, "q4_0 batch task %u: give exactly one of x and activation", i);
        const void *act = d.x != nullptr ? static_cast<const void *>(d.x) : d.activation;
        const size_t act_stride =
            d.x != nullptr ? static_cast<size_t>(d.blocks) * Q8_0_BYTES : d.activation_row_stride;
        const size_t w_stride = d.weight_layout == QXT_Q4_0_LAYOUT_LANES ? static_cast<size_t>(d.blocks) * Q4_0_BYTES
                                                                         : d.weight_row_stride;
        int rc = validate_q4(act, act_stride, d.weight, w_stride, d.rows, d.blocks, d.column_count);
        if (rc != QXT_OK) return rc;
        if (d.rows > 4) return fail(QXT_INVALID_ARGUMENT, "q4_0 batch task %u: at most 4 rows per task", i);
        if (d.weight_layout > QXT_Q4_0_LAYOUT_LANES)
            return fail(QXT_INVALID_ARGUMENT, "q4_0 batch task %u: unknown weight layout %u", i, d.weight_layout);
        if (d.blocks / 8 > static_cast<uint32_t>(units_per_thread(4) * kThreads))
            return fail(QXT_INVALID_ARGUMENT, "q4_0 batch task %u: K = %u exceeds the batch limit of %d", i,
                        d.blocks * 32, units_per_thread(4) * kThreads * 256);
        if (d.x != nullptr && (!aligned(d.x, 16) || d.x_row_stride % 16 ||
                               d.x_row_stride < static_cast<size_t>(d.blocks) * QK * sizeof(float)))
            return fail(QXT_INVALID_ARGUMENT, "q4_0 batch task %u: fp32 activation rows must be 16-byte aligned", i);
        if (d.destination == nullptr || !aligned(d.destination, 4) || d.destination_row_stride % 4 ||
            d.destination_row_stride < (static_cast<size_t>(d.output_column_start) + d.column_count) * sizeof(float))
            return fail(QXT_INVALID_ARGUMENT, "q4_0 batch task %u: bad destination", i);
        if (static_cast<uint64_t>(d.weight_column_start) + d.column_count > (1ull << 31) ||
            static_cast<uint64_t>(d.output_column_start) + d.column_count > (1ull << 31))
            return fail(QXT_INVALID_ARGUMENT, "q4_0 batch task %u: column range overflows", i);
        Q4Task t{};
        if (d.x != nullptr) {
            // Quantised by the pre-pass into the batch's staging buffer (pointer
            // patched below), or by each workgroup in a small batch.
            jobs.push_back({d.x, d.x_row_stride, nullptr, static_cast<int>(d.rows), static_cast<int>(d.blocks)});
            job_task.push_back(i);
            t.x = d.x;
            t.x_stride = d.x_row_stride;
            t.act = nullptr;
            t.act_stride = static_cast<size_t>(d.blocks) * Q8_0_BYTES;
        } else {
            t.act = static_cast<const uint8_t *>(d.activation);
            t.act_stride = d.activation_row_stride;
        }
        t.w = static_cast<const uint8_t *>(d.weight);
        t.lanes = d.weight_layout == QXT_Q4_0_LAYOUT_LANES;
        t.w_stride = t.lanes ? static_cast<size_t>(d.blocks) * Q4_0_BYTES : d.weight_row_stride;
        t.y = d.destination;
        t.y_stride = d.destination_row_stride;
        t.rows = static_cast<int>(d.rows);
        t.blocks = static_cast<int>(d.blocks);
        t.wcol0 = static_cast<int>(d.weight_column_start);
        t.ocol0 = static_cast<int>(d.output_column_start);
        t.ncols = static_cast<int>(d.column_count);
        if (!fast_path(t))
            return fail(QXT_INVALID_ARGUMENT, "q4_0 batch task %u: needs K %% 256 == 0 and 16-byte aligned weight rows",
                        i);
        host[i] = t;
        max_rows = std::max(max_rows, d.rows);
    }
    const int mr = max_rows == 1 ? 1 : 4;
    int layout = host[0].lanes ? kLaneLayout : kNativeRows;
    for (uint32_t i = 1; i < count; ++i)
        if ((host[i].lanes ? kLaneLayout : kNativeRows) != layout) layout = kEitherLayout;
    // Tiles of one round of units each give a decode step's dependency stages
    // (a few thousand columns) only 32-176 workgroups: most CUs idle while a
    // few stream 70 KB each.  A batch whose tiles would not give every CU
    // kBatchItemsPerCu workgroups narrows them until it does.
    // Plans every task's tiles; returns the number of work items, or minus a
    // status (with the error recorded).
    auto plan_items = [&](int upt, int max_cpw, std::vector<Q4Item> *items, size_t *lds) -> int64_t {
        uint64_t count_items = 0;
        for (uint32_t i = 0; i < count; ++i) {
            size_t task_lds = 0;
            int rc = plan_task(host[i], mr, true, false, &task_lds, max_cpw, false, upt);
            if (rc != QXT_OK) return -static_cast<int64_t>(rc);
            if (lds != nullptr) *lds = std::max(*lds, task_lds);
            count_items += (static_cast<uint64_t>(host[i].ncols) + host[i].cpw - 1) / host[i].cpw;
            if (items != nullptr)
                for (int c = 0; c < host[i].ncols; c += host[i].cpw)
                    items->push_back({static_cast<int>(i), c, std::min(host[i].cpw, host[i].ncols - c)});
        }
        if (count_items > 0x7FFFFFFFu) return -static_cast<int64_t>(fail(QXT_INVALID_ARGUMENT, "q4_0 batch: too many work items"));
        return static_cast<int64_t>(count_items);
    };
    uint64_t columns = 0;
    for (uint32_t i = 0; i < count; ++i) columns += static_cast<uint64_t>(host[i].ncols);
    const uint64_t want = static_cast<uint64_t>(kBatchItemsPerCu) * compute_units();
    auto cap_for = [&](int64_t natural) {
        return static_cast<uint64_t>(natural) < want ? static_cast<int>(std::max<uint64_t>(1, columns / want))
                                                     : (1 << 30);
    };
    int64_t natural = plan_items(units_per_thread(mr), 1 << 30, nullptr, nullptr);
    if (natural < 0) return static_cast<int>(-natural);
    int max_cpw = cap_for(natural);
    const int64_t planned = plan_items(units_per_thread(mr), max_cpw, nullptr, nullptr);
    if (planned < 0) return static_cast<int>(-planned);
    // A one-row batch whose every activation is an fp32 row of K <= 6144
    // can run the prefetch kernel: each workgroup requests its row before
    // its weights and quantises it while they are in flight.  A batch whose
    // tiles were narrowed (too few columns to fill the chip) runs it with
    // kPrefetchUnits units per thread, its tiles planned for that.
    bool prefetch_candidate = mr == 1;
    for (uint32_t i = 0; i < count && prefetch_candidate; ++i) prefetch_candidate = prefetch_chunks(host[i]) > 0;
    const bool small = static_cast<size_t>(planned) <= kFusedQuantItems;
    if (!small && !kPrefetchLargeBatches) prefetch_candidate = false;
    // Every other small batch quantises its fp32 rows inside each workgroup
    // too (an L2-resident re-read per workgroup) rather than waiting for a
    // separate pre-pass launch; larger ones run the pre-pass.
    const bool fused = small || prefetch_candidate;
    const bool narrowed = max_cpw < (1 << 30);
    const int upt = prefetch_candidate && narrowed ? kPrefetchUnits : units_per_thread(mr);
    if (upt != units_per_thread(mr)) {
        natural = plan_items(upt, 1 << 30, nullptr, nullptr);
        if (natural < 0) return static_cast<int>(-natural);
        max_cpw = cap_for(natural);
    }
    if (prefetch_candidate && narrowed && kBalancePrefetchTiles) {
        // Every CU the same number of workgroups: the narrowest tiles of
        // kPrefetchUnits units per thread that give at most k workgroups per
        // CU, for the smallest k that such tiles reach (a CU holding one
        // workgroup more than the others sets the stage's time).  Measured
        // on MI355X, the 88-launch staged decode step of cfg3: q/k/v 257 ->
        // 235 workgroups and gate/up 352 -> 512, 0.428 -> 0.417 ms; two units
        // per thread to reach one workgroup per CU on gate/up instead:
        // 0.434 ms.
        auto balanced = [&](uint64_t limit) -> int {
            for (int c = static_cast<int>(std::max<uint64_t>(1, (columns + limit - 1) / limit));
                 c <= kPrefetchUnits * kThreads; ++c) {
                const int64_t n = plan_items(kPrefetchUnits, c, nullptr, nullptr);
                if (n < 0) return 0;
                if (static_cast<uint64_t>(n) <= limit) return c;
            }
            return 0;
        };
        for (uint64_t k = 1; k <= kMaxBalancedPerCu; ++k) {
            const int c = balanced(k * static_cast<uint64_t>(compute_units()));
            if (c > 0) {
                max_cpw = c;
                break;
            }
        }
    }
    size_t lds = 0;
    std::vector<Q4Item> items;
    const int64_t final_items = plan_items(upt, max_cpw, &items, &lds);
    if (final_items < 0) return static_cast<int>(-final_items);
    if (fused) {
        jobs.clear();
        job_task.clear();
    } else {
        for (uint32_t i : job_task) host[i].x = nullptr;
    }
    std::vector<Q8Chunk> chunks;
    size_t staging_bytes = 0;
    std::vector<size_t> job_offset(jobs.size());
    for (size_t j = 0; j < jobs.size(); ++j) {
        job_offset[j] = staging_bytes;
        const int nblocks = jobs[j].rows * jobs[j].blocks;
        staging_bytes += (static_cast<size_t>(nblocks) * Q8_0_BYTES + 255) & ~size_t(255);
        for (int first = 0; first < nblocks; first += kThreads / 8) chunks.push_back({static_cast<int>(j), first});
    }
    if (chunks.size() > 0x7FFFFFFFu) return fail(QXT_INVALID_ARGUMENT, "q4_0 batch: too many activation blocks");
    int rc = injected(QXT_FAIL_ALLOCATION);
    if (rc != QXT_OK) return rc;
    auto *batch = new (std::nothrow) qxt_q4_0_batch();
    if (batch == nullptr) return fail(QXT_ALLOCATION_FAILED, "q4_0 batch: host allocation failed");
    auto round = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t task_bytes = round(sizeof(Q4Task) * count);
    const size_t item_bytes = round(sizeof(Q4Item) * items.size());
    const size_t job_bytes = round(sizeof(Q8Job) * jobs.size());
    const size_t bytes = task_bytes + item_bytes + job_bytes + sizeof(Q8Chunk) * chunks.size();
    if (device_malloc(&batch->device_tables, bytes) != hipSuccess ||
        (staging_bytes > 0 && device_malloc(&batch->q8_staging, staging_bytes) != hipSuccess)) {
        if (batch->device_tables != nullptr) (void)hipFree(batch->device_tables);
        delete batch;
        return fail(QXT_ALLOCATION_FAILED, "q4_0 batch: hipMalloc of %zu + %zu bytes failed", bytes, staging_bytes);
    }
    for (size_t j = 0; j < jobs.size(); ++j) {
        uint8_t *dst = static_cast<uint8_t *>(batch->q8_staging) + job_offset[j];
        jobs[j].out = dst;
        host[job_task[j]].act = dst;
    }
    auto *base = static_cast<uint8_t *>(batch->device_tables);
    bool ok = hipMemcpy(base, host.data(), sizeof(Q4Task) * count, hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpy(base + task_bytes, items.data(), sizeof(Q4Item) * items.size(), hipMemcpyHostToDevice) ==
                  hipSuccess;
    if (ok && !jobs.empty())
        ok = hipMemcpy(base + task_bytes + item_bytes, jobs.data(), sizeof(Q8Job) * jobs.size(),
                       hipMemcpyHostToDevice) == hipSuccess &&
             hipMemcpy(base + task_bytes + item_bytes + job_bytes, chunks.data(), sizeof(Q8Chunk) * chunks.size(),
                       hipMemcpyHostToDevice) == hipSuccess;
    if (!ok) {
        (void)hipFree(batch->device_tables);
        if (batch->q8_staging != nullptr) (void)hipFree(batch->q8_staging);
        delete batch;
        return fail(QXT_IO_FAILED, "q4_0 batch: upload of the task tables failed");
    }
    batch->tasks = reinterpret_cast<const Q4Task *>(base);
    batch->items = reinterpret_cast<const Q4Item *>(base + task_bytes);
    batch->jobs = reinterpret_cast<const Q8Job *>(base + task_bytes + item_bytes);
    batch->chunks = reinterpret_cast<const Q8Chunk *>(base + task_bytes + item_bytes + job_bytes);
    batch->task_count = count;
    batch->item_count = static_cast<uint32_t>(items.size());
    batch->chunk_count = static_cast<uint32_t>(chunks.size());
    batch->grid = static_cast<uint32_t>(items.size());
    batch->mr = mr;
    batch->layout = layout;
    // The prefetch kernel runs exactly the batches planned for it.
    batch->prefetch = 0;
    batch->upt = upt;
    if (prefetch_candidate)
        for (const Q4Task &t : host) batch->prefetch = std::max(batch->prefetch, prefetch_chunks(t));
    if (kQ8RowPrefetchBatches && mr == 1 && batch->prefetch == 0 && upt == units_per_thread(1)) {
        // Every activation a native Q8_0 row (given, or written by the
        // pre-pass) of at most one block per thread: its blocks are requested
        // before the weights.
        bool q8_rows = true;
        for (const Q4Task &t : host) q8_rows = q8_rows && t.x == nullptr && t.rows == 1 && t.blocks <= kThreads;
        if (q8_rows) batch->prefetch = kQ8RowPrefetch;
    }
    if (prefetch_candidate && upt == 1 && kSplitUnits) {
        // Items of at most 64 (128) units: each unit split over 4 (2) waves.
        // Measured on MI355X, the staged decode of cfg3 (q/k/v items of 88
        // units, o of 64): 0.397 -> 0.384 ms per step.  Narrowing the gate/up
        // and down tiles (176 units) so that they split too was slower (0.404
        // ms for two waves per unit, 0.427 for four): each extra workgroup
        // quantises the whole activation row again.
        int max_units = 0;
        for (const Q4Task &t : host) max_units = std::max(max_units, t.cpw * (t.blocks / 8));
        batch->split = max_units <= kLaneGroup ? 4 : max_units <= 2 * kLaneGroup ? 2 : 1;
        // 512-thread workgroups, so that a unit still splits over two
        // (129-256 units) or four (up to 128) of their eight waves and each
        // thread quantises half as many row chunks (measured on MI355X, the
        // staged decode of cfg3, gate/up and down items of 176 units: 0.384
        // -> 0.374 ms; q/k/v items of 88 units over four of eight waves
        // instead of two of four: 0.364 -> 0.361 ms; o items of 64 units,
        // half the waves idle during the block terms: 0.370 -> 0.368 ms;
        // 1024-thread workgroups for the 176-unit items, four waves per
        // unit: 0.376 -> 0.383 ms).
        if (kWideSplit) {
            batch->threads = 2 * kThreads;
            batch->split = std::min(4, 2 * batch->split);
        }
    }
    batch->lds = lds;
    if (kArgBatches && count <= static_cast<uint32_t>(kArgTasks)) {
        batch->in_args = true;
        for (int j = 0; j < kArgTasks; ++j) batch->args.first_item[j] = std::numeric_limits<int>::max();
        int first = 0;
        for (uint32_t i = 0; i < count; ++i) {
            batch->args.task[i] = host[i];
            batch->args.first_item[i] = first;
            first += (host[i].ncols + host[i].cpw - 1) / host[i].cpw;
        }
    }
    *out = batch;
    return QXT_OK;
}

int qxt_q4_0_batch_launch(const qxt_q4_0_batch *batch, void *stream) {
    if (batch == nullptr) return fail(QXT_INVALID_ARGUMENT, "q4_0 batch: null handle");
    int rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    if (batch->chunk_count > 0) {
        rc = launch("q8_0_prepass_kernel", q8_0_prepass_kernel, dim3(batch->chunk_count), dim3(kThreads), 0,
                    as_stream(stream), batch->jobs, batch->chunks);
        if (rc != QXT_OK) return rc;
    }
    const BatchKernel kernel =
        batch_kernel(batch->mr, batch->layout, batch->prefetch, batch->upt, batch->split, batch->threads);
    const dim3 block(batch->threads);
    if (batch->in_args)
        return launch("q4_0_batch_kernel", kernel.args, dim3(batch->grid), block, batch->lds, as_stream(stream),
                      batch->args);
    return launch("q4_0_batch_kernel", kernel.tables, dim3(batch->grid), block, batch->lds, as_stream(stream),
                  batch->tasks, batch->items);
}

uint32_t qxt_q4_0_batch_work_items(const qxt_q4_0_batch *batch) { return batch == nullptr ? 0 : batch->item_count; }

void qxt_q4_0_batch_destroy(qxt_q4_0_batch *batch) {
    if (batch == nullptr) return;
    if (batch->device_tables != nullptr) (void)hipFree(batch->device_tables);
    if (batch->q8_staging != nullptr) (void)hipFree(batch->q8_staging);
    delete batch;
}

}  // extern "C"

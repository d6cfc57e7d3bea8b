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
//  * GEGLU -> Q8_0 (one block per 8 lanes): table GELU of the gate times up,
//    quantised straight to Q8_0 blocks or split planes, arithmetic of
//    ggml_geglu_q8_0_reference (src/qpu_xla/kernels/ggml_geglu_q8.py:37-59).
//
// All are HBM-streaming kernels: each input byte is read once with
// 16-byte loads; absmax reductions use cross-lane shuffles inside the wave.
// Build with -ffp-contract=off: every multiply and add rounds on its own,
// as NumPy float32 arithmetic does.
#include <cmath>
#include <cstring>

#include <type_traits>

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
    float d, inv;
    q8_0_scale(amax, d, inv);
    const int q0 = clamp127(rintf(v.x * inv));
    const int q1 = clamp127(rintf(v.y * inv));
    const int q2 = clamp127(rintf(v.z * inv));
    const int q3 = clamp127(rintf(v.w * inv));
    uint8_t *dst = out + row * out_stride + static_cast<size_t>(b) * Q8_0_BYTES;
    if (l8 == 0) *reinterpret_cast<uint16_t *>(dst) = static_cast<uint16_t>(float_to_half_bits(d));
    store_u32_at_even(dst + 2 + 4 * l8, pack_bytes(q0, q1, q2, q3));
}

// ---------------------------------------------------------- GEGLU -> Q8_0

// Where geglu_q8_0_kernel writes a block: native 34-byte blocks (LAYOUT 0),
// or split planes of int8 values and fp16 scale bits held in 2-byte
// (LAYOUT 2) or zero-extended 4-byte (LAYOUT 4) elements.
struct Q8Planes {
    uint8_t *blocks;
    size_t blocks_stride;
    uint8_t *scales;
    size_t scales_stride;
    uint8_t *values;
    size_t values_stride;
};

// The GELU table lookup of ggml_geglu_q8_0_reference
// (src/qpu_xla/kernels/ggml_geglu_q8.py:46-48): entry fp16(gate) (round to
// nearest even) of the fp16 table, as fp16 bits.  Two forms:
//
//  * TableLookup reads the 128 KB table in global memory (L1/L2 gathers);
//  * BandLookup reads gates with 2^-10 <= |x| < 8 from an LDS copy of that
//    band of the table (2 x 13312 entries, 52 KB).  Outside the band the
//    table is known in closed form: gelu(x) = x for fp16 x >= 8 and -0 for
//    x <= -8 (every entry of those ranges of the table, checked against the
//    table itself by the library's tests); tiny gates, infinities and NaNs
//    read the global table.
struct TableLookup {
    const uint16_t *__restrict__ table;
    __device__ __forceinline__ uint32_t operator()(uint32_t h) const { return table[h]; }
};

constexpr uint32_t kBandFirst = 0x1400u;  // fp16 magnitude bits of 2^-10
constexpr uint32_t kBandEnd = 0x4800u;    // fp16 magnitude bits of 8
constexpr uint32_t kBandEntries = kBandEnd - kBandFirst;
constexpr uint32_t kFp16Inf = 0x7C00u;

struct BandLookup {
    const uint16_t *band;  // LDS: positive band, then negative band
    const uint16_t *__restrict__ table;
    __device__ __forceinline__ uint32_t operator()(uint32_t h) const {
        const uint32_t mag = h & 0x7FFFu;
        if (mag - kBandFirst < kBandEntries) return band[(h >> 15) * kBandEntries + (mag - kBandFirst)];
        if (mag >= kBandEnd && mag < kFp16Inf) return (h & 0x8000u) ? 0x8000u : h;
        return table[h];
    }
};

// Blocks an 8-lane group loads before it looks any of them up: the loads of
// both are in flight together (measured on MI355X at M = 512 and 2048, K =
// 5632: 10-12 % faster than one block at a time).
constexpr int kGegluBlocks = 2;

// Blocks first, first + stride, ... (NB of them, those < total) for
// one 8-lane group: each lane reads float4 of gate and of up per block,
// v = fl32(gelu * up), and the block is quantised by the Q8_0 rule of
// ggml_geglu_q8.py:50-55: d = absmax / 127, inverse = 1 / d (0 when d is 0),
// q = clip(rint(v * inverse), +-127), d stored as fp16.
template <bool VEC, int LAYOUT, int NB, typename Lookup>
__device__ __forceinline__ void geglu_blocks(uint64_t first, uint64_t stride, uint64_t total, int l8,
                                             const float *__restrict__ gate, size_t gate_stride,
                                             const float *__restrict__ up, size_t up_stride, const Lookup &lookup,
                                             const Q8Planes &out, uint32_t blocks) {
    float4 g[NB], u[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint64_t gb = first + i * stride;
        if (gb < total) {
            const uint32_t row = static_cast<uint32_t>(gb / blocks);
            const size_t element = static_cast<size_t>(gb % blocks) * QK + l8 * 4;
            g[i] = load4<VEC>(
                reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(gate) + row * gate_stride) + element);
            u[i] = load4<VEC>(
                reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(up) + row * up_stride) + element);
        }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const uint64_t gb = first + i * stride;
        if (gb >= total) break;  // whole 8-lane groups leave together
        const uint32_t row = static_cast<uint32_t>(gb / blocks);
        const uint32_t b = static_cast<uint32_t>(gb % blocks);
        const float v0 = half_bits_to_float(lookup(float_to_half_bits(g[i].x))) * u[i].x;
        const float v1 = half_bits_to_float(lookup(float_to_half_bits(g[i].y))) * u[i].y;
        const float v2 = half_bits_to_float(lookup(float_to_half_bits(g[i].z))) * u[i].z;
        const float v3 = half_bits_to_float(lookup(float_to_half_bits(g[i].w))) * u[i].w;
        float amax = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
        amax = group8_max(amax);
        float d, inv;
        q8_0_scale(amax, d, inv);
        const uint32_t word = pack_bytes(clamp127(rintf(v0 * inv)), clamp127(rintf(v1 * inv)),
                                         clamp127(rintf(v2 * inv)), clamp127(rintf(v3 * inv)));
        const uint32_t d_bits = float_to_half_bits(d);
        if constexpr (LAYOUT == 0) {
            uint8_t *dst = out.blocks + row * out.blocks_stride + static_cast<size_t>(b) * Q8_0_BYTES;
            if (l8 == 0) *reinterpret_cast<uint16_t *>(dst) = static_cast<uint16_t>(d_bits);
            store_u32_at_even(dst + 2 + 4 * l8, word);
        } else {
            uint8_t *scale = out.scales + row * out.scales_stride + static_cast<size_t>(b) * LAYOUT;
            if (l8 == 0) {
                if constexpr (LAYOUT == 4) *reinterpret_cast<uint32_t *>(scale) = d_bits;
                else *reinterpret_cast<uint16_t *>(scale) = static_cast<uint16_t>(d_bits);
            }
            *reinterpret_cast<uint32_t *>(out.values + row * out.values_stride + static_cast<size_t>(b) * QK +
                                          l8 * 4) = word;
        }
    }
}

// Small jobs: one pass over kGegluBlocks blocks per 8-lane group, lookups
// from the global table (no set-up cost).
template <bool VEC, int LAYOUT>
__global__ __launch_bounds__(kThreads) void geglu_q8_0_kernel(const float *__restrict__ gate, size_t gate_stride,
                                                              const float *__restrict__ up, size_t up_stride,
                                                              const uint16_t *__restrict__ table, Q8Planes out,
                                                              uint32_t rows, uint32_t blocks) {
    const uint64_t groups = (static_cast<uint64_t>(gridDim.x) * kThreads) >> 3;
    const uint64_t first = (static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 3;
    geglu_blocks<VEC, LAYOUT, kGegluBlocks>(first, groups, static_cast<uint64_t>(rows) * blocks, threadIdx.x & 7, gate,
                              gate_stride, up, up_stride, TableLookup{table}, out, blocks);
}

// Large jobs: a persistent grid (kBandWorkgroupsPerCU workgroups of
// kBandThreads per CU) whose workgroups first copy the table's band into
// LDS, then stride over the blocks.  LDS lookups replace the global
// gathers, whose per-lane address processing made the gather kernel run at
// 35 % of HBM peak; measured on MI355X at K = 5632: 21.6 us against 35.5 us
// at M = 2048, even at M = 384 (the band copy costs about 1 us per launch).
constexpr int kBandThreads = 1024;
constexpr int kBandWorkgroupsPerCU = 2;       // 2 x 52 KB of the 160 KB LDS, 32 waves per CU
constexpr uint64_t kBandMinBlocks = 1u << 16;  // below this the gather kernel is as fast

// NB blocks per 8-lane group and pass: 2 for the largest jobs, 1 below
// kBandTwoBlocks (measured on MI355X at K = 5632: M = 512 9.0 -> 8.0 us with
// one, M = 2048 21.2 -> 21.6 us).
constexpr uint64_t kBandTwoBlocks = 1u << 18;

template <bool VEC, int LAYOUT, int NB>
__global__ __launch_bounds__(kBandThreads) void geglu_q8_0_band_kernel(
    const float *__restrict__ gate, size_t gate_stride, const float *__restrict__ up, size_t up_stride,
    const uint16_t *__restrict__ table, Q8Planes out, uint32_t rows, uint32_t blocks) {
    __shared__ __align__(16) uint16_t band[2 * kBandEntries];
    {
        // table is 16-byte aligned (checked on the host) and both band starts
        // are multiples of 8 entries: 16-byte copies.
        constexpr uint32_t per_sign = kBandEntries / 8;
        const uint4 *pos = reinterpret_cast<const uint4 *>(table + kBandFirst);
        const uint4 *neg = reinterpret_cast<const uint4 *>(table + 0x8000u + kBandFirst);
        uint4 *dst = reinterpret_cast<uint4 *>(band);
        for (uint32_t i = threadIdx.x; i < 2 * per_sign; i += kBandThreads)
            dst[i] = i < per_sign ? pos[i] : neg[i - per_sign];
    }
    __syncthreads();
    const uint64_t total = static_cast<uint64_t>(rows) * blocks;
    const uint64_t groups = static_cast<uint64_t>(gridDim.x) * (kBandThreads / 8);
    const uint64_t first = static_cast<uint64_t>(blockIdx.x) * (kBandThreads / 8) + (threadIdx.x >> 3);
    const BandLookup lookup{band, table};
    for (uint64_t base = first; base < total; base += groups * NB)
        geglu_blocks<VEC, LAYOUT, NB>(base, groups, total, threadIdx.x & 7, gate, gate_stride, up, up_stride, lookup,
                                      out, blocks);
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

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

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
    if constexpr (VEC) {
        // The row is read once: non-temporal 16-byte loads, all issued before
        // any is used (a lane past the row re-reads its last chunk, which
        // leaves the maximum unchanged).  Measured on MI355X at 4096 rows:
        // K = 14336 62 -> 49 us (4.7 -> 6.0 TB/s), K = 4096 19 -> 16 us,
        // against loads guarded per lane.
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = min(threadIdx.x + i * kThreads, chunks - 1);
            const v4u raw = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(src) + c);
            v[i] = make_float4(__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                               __uint_as_float(raw[3]));
        }
#pragma unroll
        for (int i = 0; i < NV; ++i)
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = threadIdx.x + i * kThreads;
            if (c < chunks) {
                v[i] = load4<VEC>(src + 4 * c);
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
            }
        }
    }
    const float s = row_scale(block_max(amax, scratch), floor);
    // Every row scale of the 1/127 floor takes the reciprocal form (measured
    // on MI355X at 4096 rows: K = 14336 50.8 -> 47.0 us, K = 4096 15.6 ->
    // 14.4 us against a division per element).
    // The choice is uniform over the workgroup: one branch around the row's
    // loop, not one per element.
    auto quantise = [&](auto recip_c) {
        constexpr bool recip = decltype(recip_c)::value;
        const float r = recip ? 1.0f / s : 0.0f;
        auto quant = [&](float x) { return recip ? quant_recip(x, s, r) : quant_div(x, s); };
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint32_t c = threadIdx.x + i * kThreads;
            if (c < chunks) {
                const uint32_t word = pack_bytes(quant(v[i].x), quant(v[i].y), quant(v[i].z), quant(v[i].w));
                if constexpr (VEC) {
                    *reinterpret_cast<uint32_t *>(dst + 4 * c) = word;
                } else {
                    for (int j = 0; j < 4; ++j) dst[4 * c + j] = static_cast<int8_t>((word >> (8 * j)) & 0xFF);
                }
            }
        }
    };
    if (s >= kRecipScaleMin)
        quantise(std::true_type{});
    else
        quantise(std::false_type{});
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

// Shared argument checks of the two GEGLU producers (gate and up: fp32 rows
// of `columns` elements; table: 65536 fp16 entries).
int check_geglu(const char *name, const float *gate, size_t gate_stride, const float *up, size_t up_stride,
                const uint16_t *table, uint32_t rows, uint32_t columns) {
    if (gate == nullptr || up == nullptr || table == nullptr) return fail(QXT_INVALID_ARGUMENT, "%s: null pointer", name);
    if (rows == 0 || columns == 0 || columns % QK)
        return fail(QXT_INVALID_ARGUMENT, "%s: rows > 0 and columns a positive multiple of 32 required", name);
    if (gate_stride < columns * sizeof(float) || gate_stride % sizeof(float) || up_stride < columns * sizeof(float) ||
        up_stride % sizeof(float) || !aligned(gate, 4) || !aligned(up, 4) || !aligned(table, 2))
        return fail(QXT_INVALID_ARGUMENT, "%s: bad strides or alignment", name);
    return QXT_OK;
}

template <int LAYOUT>
int launch_geglu(const float *gate, size_t gate_stride, const float *up, size_t up_stride, const uint16_t *table,
                 const Q8Planes &out, uint32_t rows, uint32_t blocks, void *stream) {
    const bool vec = aligned(gate, 16) && gate_stride % 16 == 0 && aligned(up, 16) && up_stride % 16 == 0;
    const uint64_t total = static_cast<uint64_t>(rows) * blocks;
    if (total >= kBandMinBlocks && aligned(table, 16)) {
        const bool two = total >= kBandTwoBlocks;
        const uint64_t per_workgroup = static_cast<uint64_t>(kBandThreads / 8) * (two ? 2 : 1);
        const uint64_t wanted = (total + per_workgroup - 1) / per_workgroup;
        const uint64_t resident = static_cast<uint64_t>(compute_units()) * kBandWorkgroupsPerCU;
        const unsigned grid = static_cast<unsigned>(wanted < resident ? wanted : resident);
        auto kernel = vec ? (two ? geglu_q8_0_band_kernel<true, LAYOUT, 2> : geglu_q8_0_band_kernel<true, LAYOUT, 1>)
                          : (two ? geglu_q8_0_band_kernel<false, LAYOUT, 2> : geglu_q8_0_band_kernel<false, LAYOUT, 1>);
        return launch("geglu_q8_0_band_kernel", kernel, dim3(grid), dim3(kBandThreads), 0, as_stream(stream), gate,
                      gate_stride, up, up_stride, table, out, rows, blocks);
    }
    const unsigned grid = grid_for_blocks((total + kGegluBlocks - 1) / kGegluBlocks);
    return launch("geglu_q8_0_kernel", vec ? geglu_q8_0_kernel<true, LAYOUT> : geglu_q8_0_kernel<false, LAYOUT>,
                  dim3(grid), dim3(kThreads), 0, as_stream(stream), gate, gate_stride, up, up_stride, table, out, rows,
                  blocks);
}

// q8_0_scale against the two IEEE divisions it replaces, for every
// non-negative fp32 amax (all 2^31 bit patterns, grid-stride): adds the
// number of patterns whose d or inv differs (NaN matches NaN) to *mismatches.
__global__ __launch_bounds__(kThreads) void q8_0_scale_check_kernel(unsigned long long *mismatches) {
    const uint32_t stride = gridDim.x * kThreads;
    unsigned int bad = 0;
    for (uint32_t bits = blockIdx.x * kThreads + threadIdx.x; bits < 0x80000000u; bits += stride) {
        const float amax = __uint_as_float(bits);
        float d, inv;
        q8_0_scale(amax, d, inv);
        const float dr = amax / 127.0f;
        const float ir = dr != 0.0f ? 1.0f / dr : 0.0f;
        const bool d_ok = __float_as_uint(d) == __float_as_uint(dr) || (d != d && dr != dr);
        const bool i_ok = __float_as_uint(inv) == __float_as_uint(ir) || (inv != inv && ir != ir);
        bad += (d_ok && i_ok) ? 0u : 1u;
        if (stride > 0x80000000u - bits) break;  // the next pattern would pass 2^31 (no wrap)
    }
    if (bad != 0) atomicAdd(mismatches, static_cast<unsigned long long>(bad));
}

}  // namespace
}  // namespace qxt

using namespace qxt;

extern "C" {

int qxt_q8_0_scale_check(uint64_t *mismatches, void *stream) {
    if (mismatches == nullptr || !aligned(mismatches, 8)) return fail(QXT_INVALID_ARGUMENT, "q8_0 scale check: bad counter");
    int rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    return launch("q8_0_scale_check_kernel", q8_0_scale_check_kernel, dim3(8192), dim3(kThreads), 0,
                  as_stream(stream), reinterpret_cast<unsigned long long *>(mismatches));
}

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

int qxt_ggml_gelu_fp16_table(uint16_t *table) {
    if (table == nullptr) return fail(QXT_INVALID_ARGUMENT, "gelu_fp16_table: null pointer");
    // Entry i: x = the fp16 value with bits i; 0.5 x (1 + erf(x / sqrt 2)) in
    // double, rounded to fp32, then to fp16 (both round to nearest even).
    const double root2 = std::sqrt(2.0);
    for (uint32_t i = 0; i < (1u << 16); ++i) {
        const uint16_t bits = static_cast<uint16_t>(i);
        _Float16 h;
        std::memcpy(&h, &bits, sizeof h);
        const double x = static_cast<double>(static_cast<float>(h));
        const float gelu = static_cast<float>(0.5 * x * (1.0 + std::erf(x / root2)));
        const _Float16 rounded = static_cast<_Float16>(gelu);
        std::memcpy(&table[i], &rounded, sizeof rounded);
    }
    return QXT_OK;
}

int qxt_ggml_geglu_q8_0(const float *gate, size_t gate_row_stride, const float *up, size_t up_row_stride,
                        const uint16_t *gelu_table, void *blocks, size_t blocks_row_stride, uint32_t rows,
                        uint32_t columns, void *stream) {
    int rc = check_geglu("geglu_q8_0", gate, gate_row_stride, up, up_row_stride, gelu_table, rows, columns);
    if (rc != QXT_OK) return rc;
    const uint32_t nb = columns / QK;
    if (blocks == nullptr) return fail(QXT_INVALID_ARGUMENT, "geglu_q8_0: null pointer");
    if (blocks_row_stride < static_cast<size_t>(nb) * Q8_0_BYTES || blocks_row_stride % 2 || !aligned(blocks, 2))
        return fail(QXT_INVALID_ARGUMENT, "geglu_q8_0: bad block stride or alignment");
    rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    Q8Planes out{static_cast<uint8_t *>(blocks), blocks_row_stride, nullptr, 0, nullptr, 0};
    return launch_geglu<0>(gate, gate_row_stride, up, up_row_stride, gelu_table, out, rows, nb, stream);
}

int qxt_ggml_geglu_q8_0_split(const float *gate, size_t gate_row_stride, const float *up, size_t up_row_stride,
                              const uint16_t *gelu_table, void *scales, size_t scales_row_stride,
                              uint32_t scale_bytes, int8_t *values, size_t values_row_stride, uint32_t rows,
                              uint32_t columns, void *stream) {
    int rc = check_geglu("geglu_q8_0_split", gate, gate_row_stride, up, up_row_stride, gelu_table, rows, columns);
    if (rc != QXT_OK) return rc;
    const uint32_t nb = columns / QK;
    if (scales == nullptr || values == nullptr) return fail(QXT_INVALID_ARGUMENT, "geglu_q8_0_split: null pointer");
    if (scale_bytes != 2 && scale_bytes != 4)
        return fail(QXT_INVALID_ARGUMENT, "geglu_q8_0_split: scale_bytes must be 2 or 4");
    if (scales_row_stride < static_cast<size_t>(nb) * scale_bytes || scales_row_stride % scale_bytes ||
        !aligned(scales, scale_bytes) || values_row_stride < columns || values_row_stride % 4 || !aligned(values, 4))
        return fail(QXT_INVALID_ARGUMENT, "geglu_q8_0_split: bad strides or alignment");
    rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    Q8Planes out{nullptr, 0, static_cast<uint8_t *>(scales), scales_row_stride, reinterpret_cast<uint8_t *>(values),
                 values_row_stride};
    if (scale_bytes == 4)
        return launch_geglu<4>(gate, gate_row_stride, up, up_row_stride, gelu_table, out, rows, nb, stream);
    return launch_geglu<2>(gate, gate_row_stride, up, up_row_stride, gelu_table, out, rows, nb, stream);
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

// Dynamic-W8A8 int8 GEMM for gfx950: LDS-tiled v_mfma_i32_32x32x32_i8 with
// exact int32 accumulation and a fused fp32 dequant (+ bias) epilogue.
//
// Arithmetic (reference src/qpu_xla/models/tinyllama/quantization.py:1073-1075,
// fused QPU store src/qpu_xla/kernels/gemm_int8.py:176-178, bias
// src/qpu_xla/models/smolvla/accelerated.py:259-261):
//     acc = sum_k a[m,k] * w[n,k]                 (int32, exact)
//     y   = fl32(fl32(float(acc) * sa[m]) * sw[n])
//     y   = fl32(y + bias[n])                     (when a bias is given)
// Built with -ffp-contract=off so the two multiplies and the add round
// separately, which makes the result bit-identical to the NumPy oracle.
//
// Tiling (w8a8_gemm_kernel): a 256-thread workgroup (4 waves, 2 x 2) owns a
// BM x BN output tile; each wave owns a (BM/2) x (BN/2) sub-tile of 32 x 32
// MFMA blocks.  K advances BKT bytes per stage; A and B tiles live in LDS
// with K contiguous per row, padded by 16 bytes so the 16-byte fragment reads
// are bank-conflict free.  The large-tile streaming kernel
// (w8a8_gemm_stream_kernel) uses eight waves of 128 x 64 instead.
// The MFMA lane layout: lane l supplies A[l % 32][k-chunk(l / 32)] and
// B[k-chunk(l / 32)][l % 32] (the same 16 k values for both operands, so the
// exact integer sum does not depend on how the chunk is ordered) and receives
// D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32] in accumulator register r.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <vector>

#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum Epilogue { EPI_I32 = 0, EPI_DEQUANT = 1, EPI_DEQUANT_BIAS = 2 };

struct GemmArgs {
    const int8_t *a;
    size_t lda;
    const uint8_t *w;
    size_t ldw;
    int32_t *acc;
    size_t ldacc;
    const float *sa;
    const float *sw;
    const float *bias;
    float *y;
    size_t ldy;
    int m, n, k;
    uint32_t a_bytes, w_bytes;  // extents of the operands (buffer-descriptor ranges)
};

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Raw buffer descriptor over `bytes` bytes at `base` (gfx9 dword3: 32-bit data
// format).  Loads at offsets >= `bytes` return zeros, which predicates the
// matrix edges without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

constexpr uint32_t kOutOfRange = 0x80000000u;  // operands are < 2 GiB, so this offset is always out of range

// Global -> register staging of one K stage (BKT bytes of K): A rows [m0, m0+BM)
// and B columns [n0, n0+BN) as 16-byte chunks, zeros outside the matrices.
template <int BM, int BN, int BKT, bool K4N>
struct StageRegs {
    static constexpr int CPR = BKT / 16;  // chunks per LDS row
    static constexpr int A_CHUNKS = BM * CPR / kThreads;
    static constexpr int B_CHUNKS = BN * CPR / kThreads;
    static constexpr int STORES = A_CHUNKS + (K4N ? 4 : 1) * B_CHUNKS;  // LDS write instructions
    v4u a[A_CHUNKS];
    v4u b[B_CHUNKS];

    __device__ __forceinline__ void load(const GemmArgs &args, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                         int m0, int n0, int k0) {
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int c = threadIdx.x + i * kThreads;
            const int row = c / CPR, kc = c % CPR;
            const int gm = m0 + row, gk = k0 + kc * 16;
            const uint32_t off = (gm < args.m && gk < args.k) ? static_cast<uint32_t>(gm) * args.lda + gk : kOutOfRange;
            a[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < B_CHUNKS; ++i) {
            const int c = threadIdx.x + i * kThreads;
            uint32_t off;
            if constexpr (!K4N) {
                const int row = c / CPR, kc = c % CPR;
                const int gn = n0 + row, gk = k0 + kc * 16;
                off = (gn < args.n && gk < args.k) ? static_cast<uint32_t>(gn) * args.ldw + gk : kOutOfRange;
            } else {
                // uint32 [K/4, N]: one chunk = k-quad k4 of 4 adjacent columns.
                const int k4 = c / (BN / 4), nq = c % (BN / 4);
                const int gn = n0 + nq * 4, gk = k0 + k4 * 4;
                off = (gn < args.n && gk < args.k) ? static_cast<uint32_t>(gk / 4) * args.ldw + gn * 4 : kOutOfRange;
            }
            b[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0);
        }
    }

    __device__ __forceinline__ void store(uint8_t *As, uint8_t *Bs) const {
        constexpr int ROW = BKT + 16;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int c = threadIdx.x + i * kThreads;
            *reinterpret_cast<v4u *>(As + (c / CPR) * ROW + (c % CPR) * 16) = a[i];
        }
#pragma unroll
        for (int i = 0; i < B_CHUNKS; ++i) {
            const int c = threadIdx.x + i * kThreads;
            if constexpr (!K4N) {
                *reinterpret_cast<v4u *>(Bs + (c / CPR) * ROW + (c % CPR) * 16) = b[i];
            } else {
                const int k4 = c / (BN / 4), nq = c % (BN / 4);
#pragma unroll
                for (int q = 0; q < 4; ++q) *reinterpret_cast<uint32_t *>(Bs + (nq * 4 + q) * ROW + k4 * 4) = b[i][q];
            }
        }
    }
};

// Copy the row scales sa[m0, m0+BM), column scales sw[n0, n0+BN) and bias of
// a workgroup's output tile into LDS (zeros past M / N).  Reading them from
// LDS in the epilogue keeps vector-memory loads out of the run of output
// stores (a load issued after a store would wait for that store).  The
// caller has finished with the LDS operand tiles.
template <int BM, int BN, int EPI>
__device__ __forceinline__ void stage_scales(const GemmArgs &args, float *lds, int m0, int n0) {
    if constexpr (EPI == EPI_I32) return;
    static_assert(BM <= kThreads && BN <= kThreads, "one scale per thread");
    const int t = threadIdx.x;
    if (t < BM) {
        const __amdgpu_buffer_rsrc_t rsa = buffer_rsrc(args.sa, static_cast<uint32_t>(args.m) * 4);
        lds[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                               rsa, m0 + t < args.m ? (m0 + t) * 4 : kOutOfRange, 0, 0));
    }
    if (t < BN) {
        const uint32_t off = n0 + t < args.n ? (n0 + t) * 4 : kOutOfRange;
        const __amdgpu_buffer_rsrc_t rsw = buffer_rsrc(args.sw, static_cast<uint32_t>(args.n) * 4);
        lds[BM + t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsw, off, 0, 0));
        float bv = 0.0f;
        if constexpr (EPI == EPI_DEQUANT_BIAS) {
            const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(args.bias, static_cast<uint32_t>(args.n) * 4);
            bv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, off, 0, 0));
        }
        lds[BM + BN + t] = bv;
    }
    __syncthreads();
}

// Write one wave's TM x TN blocks of 32 x 32 accumulators (rows from mrow0,
// columns from ncol0, i.e. tile-local rows lm0 / columns ln0): int32 as is, or
// fl32(fl32(float(acc) * sa) * sw) (+ bias) with the scales staged in LDS by
// stage_scales.  Stores go through a buffer descriptor over the output: rows
// past M are addressed out of its range and dropped; columns past N are
// masked per block column.
template <int BM, int BN, int TM, int TN, int EPI>
__device__ __forceinline__ void store_tile(const GemmArgs &args, const v16i (&acc)[TM][TN], int mrow0, int ncol0,
                                           int lm0, int ln0, int lane, const float *lds) {
    const int half = lane >> 5;
    void *base = EPI == EPI_I32 ? static_cast<void *>(args.acc) : static_cast<void *>(args.y);
    const uint32_t ld = static_cast<uint32_t>(EPI == EPI_I32 ? args.ldacc : args.ldy);
    const __amdgpu_buffer_rsrc_t ro =
        buffer_rsrc(base, static_cast<uint32_t>(args.m - 1) * ld + static_cast<uint32_t>(args.n) * 4);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int gn = ncol0 + j * 32 + (lane & 31);
        if (gn >= args.n) continue;
        float swn = 0.0f, bn = 0.0f;
        if constexpr (EPI != EPI_I32) {
            swn = lds[BM + ln0 + j * 32 + (lane & 31)];
            bn = lds[BM + BN + ln0 + j * 32 + (lane & 31)];
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float4 sa4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if constexpr (EPI != EPI_I32)
                    sa4 = *reinterpret_cast<const float4 *>(lds + lm0 + i * 32 + 8 * q + 4 * half);
                const float sar[4] = {sa4.x, sa4.y, sa4.z, sa4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * q + e;
                    const int gm = mrow0 + i * 32 + 8 * q + 4 * half + e;
                    const uint32_t off = gm < args.m ? static_cast<uint32_t>(gm) * ld + gn * 4 : kOutOfRange;
                    const int v = acc[i][j][r];
                    if constexpr (EPI == EPI_I32) {
                        __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(v), ro, off, 0, 0);
                    } else {
                        float yv = static_cast<float>(v) * sar[e];
                        yv = yv * swn;
                        if constexpr (EPI == EPI_DEQUANT_BIAS) yv = yv + bn;
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, yv), ro, off, 0, 0);
                    }
                }
            }
        }
    }
}

// Epilogue of a 256 x 256 tile held by eight waves of 128 x 64: wave w owns
// tile rows (w & 3) / 2 * 128 + [0, 128) and columns ((w & 3) % 2) * 128 +
// (w / 4) * 64 + [0, 64).  Staged through LDS so that global stores are whole
// 1 KB tile rows (16 bytes per lane) instead of 128-byte row pieces.  Two
// passes: in pass p every wave writes its 32-row blocks i = 2p, 2p + 1 (tile
// rows wm * 128 + 64p + [0, 64)) to `buf` row-major, then each wave stores 16
// of the 128 buffered rows.  Each accumulator is converted in exactly one
// pass.  Rows past M are skipped and columns past N masked (edge lanes and
// unaligned outputs store element by element).  `scales` holds what
// stage_scales wrote; `buf` takes 128 KB.
template <int EPI>
__device__ __forceinline__ void store_tile_rows(const GemmArgs &args, const v16i (&acc)[4][2], int m0, int n0,
                                                int wm, int wcol, int lane, uint8_t *buf, const float *scales) {
    constexpr int BM = 256, BN = 256;
    const int hl = lane >> 5;
    const int wave = threadIdx.x >> 6;
    float *fb = reinterpret_cast<float *>(buf);
    uint8_t *base = reinterpret_cast<uint8_t *>(EPI == EPI_I32 ? static_cast<void *>(args.acc)
                                                               : static_cast<void *>(args.y));
    const size_t ld = EPI == EPI_I32 ? args.ldacc : args.ldy;
    const int col0 = n0 + lane * 4;
    const bool vec = col0 + 3 < args.n && (((reinterpret_cast<uintptr_t>(base) | ld) & 15) == 0);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = wcol + j * 32 + (lane & 31);
            float swn = 0.0f, bn = 0.0f;
            if constexpr (EPI != EPI_I32) {
                swn = scales[BM + col];
                bn = scales[BM + BN + col];
            }
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                const int i = 2 * p + ii;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int lr = 8 * q + 4 * hl;
                    float4 sa4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if constexpr (EPI != EPI_I32)
                        sa4 = *reinterpret_cast<const float4 *>(scales + wm * 128 + i * 32 + lr);
                    const float sar[4] = {sa4.x, sa4.y, sa4.z, sa4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int v = acc[i][j][4 * q + e];
                        float out;
                        if constexpr (EPI == EPI_I32) {
                            out = __int_as_float(v);
                        } else {
                            out = static_cast<float>(v) * sar[e];
                            out = out * swn;
                            if constexpr (EPI == EPI_DEQUANT_BIAS) out = out + bn;
                        }
                        fb[(wm * 64 + ii * 32 + lr + e) * BN + col] = out;
                    }
                }
            }
        }
        __syncthreads();
        // Buffered row br holds tile row (br / 64) * 128 + 64p + br % 64.  Lane
        // l stores columns n0 + 4l .. 4l + 3 of each row: one 16-byte store when
        // all four are inside N and the address is 16-byte aligned, otherwise
        // element by element.
#pragma unroll 4
        for (int t = 0; t < 16; ++t) {
            const int br = wave * 16 + t;
            const int gm = m0 + (br >> 6) * 128 + p * 64 + (br & 63);
            if (gm < args.m) {
                const v4u v = *reinterpret_cast<const v4u *>(fb + br * BN + lane * 4);
                uint8_t *dst = base + static_cast<size_t>(gm) * ld + static_cast<size_t>(col0) * 4;
                if (vec) {
                    *reinterpret_cast<v4u *>(dst) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col0 + e < args.n) reinterpret_cast<uint32_t *>(dst)[e] = v[e];
                }
            }
        }
        __syncthreads();
    }
}

// LDS bytes the 256 x 256 epilogue uses: the 128 KB half-tile buffer and
// the staged scales behind it.
constexpr int kEpilogueLds = 128 * 1024 + 3 * 256 * 4;

// BM x BN output tile per 256-thread workgroup; waves 2 x 2, each (BM/2) x (BN/2)
// as (BM/64) x (BN/64) blocks of 32 x 32.  K advances BKT bytes per stage
// through two LDS buffers (rows padded by 16 bytes, so the 16-byte fragment
// reads of 8 consecutive rows hit distinct banks): the next stage's global
// loads are issued before the current stage's MFMAs and written to the other
// buffer after them, one barrier per stage.  Within a stage the fragments of
// the next 32-deep k step are read from LDS while the current step's MFMAs run.
template <int BM, int BN, int BKT, int DEPTH, int STORE_KS, bool K4N, int EPI>
__global__ __launch_bounds__(kThreads) void w8a8_gemm_kernel(GemmArgs args) {
    constexpr int ROW = BKT + 16;
    constexpr int STAGE = (BM + BN) * ROW;
    constexpr int KSTEPS = BKT / 32;
    static_assert(KSTEPS % 2 == 0, "fragment double buffer assumes an even number of k steps");
    static_assert(DEPTH == 1 || DEPTH == 2, "one or two register stages in flight");
    static_assert(STORE_KS >= 0 && STORE_KS < KSTEPS, "store step inside the stage");
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

    constexpr int WM = BM / 2, WN = BN / 2;    // per-wave sub-tile
    constexpr int TM = WM / 32, TN = WN / 32;  // 32x32 blocks per wave
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(args.a, args.a_bytes);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(args.w, args.w_bytes);

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    // Lane-constant parts of the fragment addresses.
    const int a_lane = (wm * WM + (lane & 31)) * ROW + (lane >> 5) * 16;
    const int b_lane = (wn * WN + (lane & 31)) * ROW + (lane >> 5) * 16;
    v4i af[2][TM], bf[2][TN];
    auto read_frags = [&](const uint8_t *As, const uint8_t *Bs, int kk, int buf) {
#pragma unroll
        for (int i = 0; i < TM; ++i) af[buf][i] = *reinterpret_cast<const v4i *>(As + a_lane + i * 32 * ROW + kk);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[buf][j] = *reinterpret_cast<const v4i *>(Bs + b_lane + j * 32 * ROW + kk);
    };

    // DEPTH register stages in flight.  DEPTH == 1: stage s+1 is loaded at the
    // start of stage s and written to LDS in k step STORE_KS of stage s.
    // DEPTH == 2: stage s+2 is loaded at the start of stage s while stage s+1
    // (loaded a full stage earlier) is written in k step STORE_KS.
    const int stages = (args.k + BKT - 1) / BKT;
    StageRegs<BM, BN, BKT, K4N> regs[DEPTH];
    regs[0].load(args, ra, rb, m0, n0, 0);
    regs[0].store(smem, smem + BM * ROW);
    if constexpr (DEPTH == 2) regs[1].load(args, ra, rb, m0, n0, BKT);
    __syncthreads();
    read_frags(smem, smem + BM * ROW, 0, 0);

    // The loop body is one basic block: past the last stages the prefetch
    // offsets are out of range (zeros, no memory traffic) and land in a
    // buffer nobody reads again, so no branch splits the schedule.
    auto stage_body = [&](int s, StageRegs<BM, BN, BKT, K4N> &prefetch, const StageRegs<BM, BN, BKT, K4N> &ready) {
        const uint8_t *As = smem + (s & 1) * STAGE;
        const uint8_t *Bs = As + BM * ROW;
        uint8_t *next = smem + ((s + 1) & 1) * STAGE;
        prefetch.load(args, ra, rb, m0, n0, (s + DEPTH) * BKT);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            // One scheduling region per k step: the TM*TN independent MFMAs of
            // this step, the LDS reads of the next step's fragments and, in
            // step STORE_KS, the LDS writes of stage s+1 (into the buffer no
            // wave reads during this stage).
            if (ks + 1 < KSTEPS) read_frags(As, Bs, (ks + 1) * 32, (ks + 1) & 1);
            if (ks == STORE_KS) ready.store(next, next + BM * ROW);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks & 1][i], bf[ks & 1][j], acc[i][j], 0, 0, 0);
            // Issue order inside the region: one MFMA, (first step: the global
            // prefetch; store step: the LDS writes), the LDS reads, then the
            // remaining MFMAs hide their latency.
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (ks == 0)
                __builtin_amdgcn_sched_group_barrier(0x020, StageRegs<BM, BN, BKT, K4N>::A_CHUNKS +
                                                                StageRegs<BM, BN, BKT, K4N>::B_CHUNKS, 0);
            if (ks == STORE_KS)
                __builtin_amdgcn_sched_group_barrier(0x200, StageRegs<BM, BN, BKT, K4N>::STORES, 0);
            if (ks + 1 < KSTEPS) __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - 1, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
        read_frags(next, next + BM * ROW, 0, 0);
    };
    if constexpr (DEPTH == 1) {
        for (int s = 0; s < stages; ++s) stage_body(s, regs[0], regs[0]);
    } else {
        int s = 0;
        for (; s + 1 < stages; s += 2) {
            stage_body(s, regs[0], regs[1]);
            stage_body(s + 1, regs[1], regs[0]);
        }
        if (s < stages) stage_body(s, regs[0], regs[1]);
    }

    __syncthreads();
    stage_scales<BM, BN, EPI>(args, reinterpret_cast<float *>(smem), m0, n0);
    store_tile<BM, BN, TM, TN, EPI>(args, acc, m0 + wm * WM, n0 + wn * WN, wm * WM, wn * WN, lane,
                                    reinterpret_cast<const float *>(smem));
}

// ----------------------------------------------------------------------------
// Large-tile streaming kernel for the common case: weight layout [N, K],
// K % 128 == 0.  A 256 x 256 output tile per workgroup of eight waves, two
// per SIMD (waves w and w + 4 share SIMD w % 4), each wave a 128 x 64
// sub-tile of 4 x 2 blocks of 32 x 32 (128 accumulators), so that while one
// wave of a SIMD waits on LDS or memory the other keeps the matrix pipe fed.
// K advances in 128-byte stages through two LDS buffers, two register stages
// in flight: every k step issues, between its 8 MFMAs, the 6 fragment reads
// of the next k step, 2 LDS writes of stage s+1 (loaded a full stage
// earlier) and 2 global loads of stage s+2.  Rows past M or N need no
// predicate: their offsets fall outside the buffer descriptor's range and
// load zeros.  Output tiles are mapped to workgroups XCD by XCD (xcd_tile)
// and written through LDS one tile row per store (store_tile_rows).
//
// Measured on MI355X (cfg4 shapes, interleaved runs in one process): against
// four waves of 128 x 128 (one wave per SIMD, the same stages) this runs
// gate_up in 240 us instead of 258 us and down in 206 us instead of 208 us;
// the matrix pipes are busier (52 / 67 % against 46 / 63 %) while the board
// lowers the clock (1.80 / 1.69 GHz against 1.90 / 1.77 GHz in the same
// profiling session), i.e. power bounds both.  Grouping each k step's MFMAs
// into one burst (with or without a raised wave priority) or leaving the
// placement to the compiler was 1-4 % slower.
namespace big {
constexpr int THREADS = 512;
constexpr int BM = 256, BN = 256, BKT = 128;
constexpr int ROW = BKT + 16;              // LDS row pitch (bytes)
constexpr int STAGE = (BM + BN) * ROW;     // one LDS buffer (A then B)
constexpr int CPR = BKT / 16;              // 16-byte chunks per row
constexpr int RPI = THREADS / CPR;         // rows covered by one load instruction
constexpr int A_CHUNKS = BM / RPI;         // 4
constexpr int B_CHUNKS = BN / RPI;         // 4
constexpr int Q = A_CHUNKS + B_CHUNKS;     // 16-byte chunks per thread per stage
constexpr int KSTEPS = BKT / 32;           // 4
constexpr int TM = 4, TN = 2;              // 32x32 blocks per wave (128 x 64)
constexpr int PER_STEP = Q / KSTEPS;       // loads (and writes) per k step
static_assert(2 * STAGE >= kEpilogueLds, "the epilogue reuses the operand buffers");
}  // namespace big

// Output tile (ty, tx) of workgroup `pid` in a tm x tn tile grid.  The
// dispatcher hands workgroups to the 8 XCDs round-robin (pid % 8), each XCD
// with its own L2.  Every XCD is given a contiguous run of a grouped tile
// order (GM tile rows at a time, column by column), so the workgroups one
// XCD runs together form a compact block whose A and B panels are shared
// through that XCD's L2 instead of being fetched by every XCD.
constexpr int kXcds = 8;
// Position `seq` of the grouped tile order: gm tile rows at a time, column by column.
__device__ __forceinline__ void grouped_tile(int seq, int tm, int tn, int gm, int &ty, int &tx) {
    const int group = seq / (gm * tn);
    const int first = group * gm;
    const int rows = min(gm, tm - first);
    const int in_group = seq - group * gm * tn;
    ty = first + in_group % rows;
    tx = in_group / rows;
}

__device__ __forceinline__ void xcd_tile(int pid, int tm, int tn, int gm, int &ty, int &tx) {
    const int total = tm * tn;
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = pid % kXcds, local = pid / kXcds;
    const int seq = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
    grouped_tile(seq, tm, tn, gm, ty, tx);
}

// Main loop of the large-tile kernel: accumulates K stages [s0, s1) of the
// output tile at (m0, n0) into `acc` (zeroed first).  Stage s + 2 is loaded
// while stage s computes; past s1 the loads read bytes nobody uses (or, past
// the operands, out of the descriptor range: zeros), so the loop body stays
// one basic block.  On return every wave is past its last LDS write, but
// waves may still read fragments: callers synchronise before reusing `smem`.
__device__ __forceinline__ void big_mainloop(const GemmArgs &args, uint8_t *smem, int m0, int n0, int s0, int s1,
                                             v16i (&acc)[big::TM][big::TN], bool zero = true) {
    using namespace big;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = (wave & 3) >> 1;                    // 128-row half of the tile
    const int wcol = (wave & 1) * 128 + (wave >> 2) * 64;  // first of the wave's 64 columns
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(args.a, args.a_bytes);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(args.w, args.w_bytes);
    const uint32_t lda = static_cast<uint32_t>(args.lda), ldw = static_cast<uint32_t>(args.ldw);

    // This thread's chunk: row tid / CPR (+ RPI per instruction), 16 bytes at (tid % CPR) * 16.
    const int crow = threadIdx.x / CPR, ccol = (threadIdx.x % CPR) * 16;
    const uint32_t a_off = static_cast<uint32_t>(m0 + crow) * lda + ccol;
    const uint32_t b_off = static_cast<uint32_t>(n0 + crow) * ldw + ccol;
    const int st_off = crow * ROW + ccol;

    if (zero) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    }

    const int a_lane = (wm * 128 + (lane & 31)) * ROW + (lane >> 5) * 16;
    const int b_lane = (wcol + (lane & 31)) * ROW + (lane >> 5) * 16;
    v4i af[2][TM], bf[2][TN];
    // Fragments in the order the MFMAs of a k step consume them.
    auto read_frags = [&](const uint8_t *As, int kk, int buf) {
        const uint8_t *Bs = As + BM * ROW;
        af[buf][0] = *reinterpret_cast<const v4i *>(As + a_lane + kk);
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[buf][j] = *reinterpret_cast<const v4i *>(Bs + b_lane + j * 32 * ROW + kk);
#pragma unroll
        for (int i = 1; i < TM; ++i) af[buf][i] = *reinterpret_cast<const v4i *>(As + a_lane + i * 32 * ROW + kk);
    };
    // Chunk q (0 .. Q-1) of a stage: A rows for q < A_CHUNKS, else B rows.
    auto load_chunk = [&](v4u &dst, int q, int k0) {
        if (q < A_CHUNKS)
            dst = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off + static_cast<uint32_t>(q * RPI) * lda + k0, 0, 0);
        else
            dst = __builtin_amdgcn_raw_buffer_load_b128(
                rb, b_off + static_cast<uint32_t>((q - A_CHUNKS) * RPI) * ldw + k0, 0, 0);
    };
    auto store_chunk = [&](uint8_t *stage, const v4u &src, int q) {
        const int row0 = q < A_CHUNKS ? q * RPI : BM + (q - A_CHUNKS) * RPI;
        *reinterpret_cast<v4u *>(stage + st_off + row0 * ROW) = src;
    };

    v4u regs0[Q], regs1[Q];
    const int k_first = s0 * BKT;
#pragma unroll
    for (int q = 0; q < Q; ++q) load_chunk(regs0[q], q, k_first);
#pragma unroll
    for (int q = 0; q < Q; ++q) load_chunk(regs1[q], q, k_first + BKT);
#pragma unroll
    for (int q = 0; q < Q; ++q) store_chunk(smem, regs0[q], q);
    __syncthreads();
    read_frags(smem, 0, 0);

    // Stage s (the r-th of this range) computes from buffer r&1, writes stage
    // s+1 (held in `ready`) to buffer (r+1)&1 and loads stage s+2 into
    // `prefetch`.
    auto stage_body = [&](int s, int r, v4u (&prefetch)[Q], const v4u (&ready)[Q]) {
        const uint8_t *As = smem + (r & 1) * STAGE;
        uint8_t *next = smem + ((r + 1) & 1) * STAGE;
        const int k2 = (s + 2) * BKT;
        auto kstep = [&](auto ksc) {
            constexpr int ks = decltype(ksc)::value;
            if constexpr (ks + 1 < KSTEPS) read_frags(As, (ks + 1) * 32, (ks + 1) & 1);
#pragma unroll
            for (int q = ks * PER_STEP; q < (ks + 1) * PER_STEP; ++q) store_chunk(next, ready[q], q);
#pragma unroll
            for (int q = ks * PER_STEP; q < (ks + 1) * PER_STEP; ++q) load_chunk(prefetch[q], q, k2);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks & 1][i], bf[ks & 1][j], acc[i][j], 0, 0, 0);
            // Issue order: after MFMA t, fragment read t (t < 6), LDS writes
            // after MFMAs 2-3, global loads after MFMAs 5-6.
            constexpr int reads = (ks + 1 < KSTEPS) ? TM + TN : 0;
#pragma unroll
            for (int t = 0; t < TM * TN; ++t) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (t < reads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                if (t >= 2 && t < 2 + PER_STEP) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                if (t >= 5 && t < 5 + PER_STEP) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        kstep(std::integral_constant<int, 0>{});
        kstep(std::integral_constant<int, 1>{});
        kstep(std::integral_constant<int, 2>{});
        kstep(std::integral_constant<int, 3>{});
        static_assert(KSTEPS == 4, "stage body is written for four k steps");
        __syncthreads();
        read_frags(next, 0, 0);
    };
    const int n = s1 - s0;
    int r = 0;
    for (; r + 1 < n; r += 2) {
        stage_body(s0 + r, r, regs0, regs1);
        stage_body(s0 + r + 1, r + 1, regs1, regs0);
    }
    if (r < n) stage_body(s0 + r, r, regs0, regs1);
}

// Fused epilogue of a finished 256 x 256 tile (LDS free: callers synchronise first).
template <int EPI>
__device__ __forceinline__ void big_epilogue(const GemmArgs &args, uint8_t *smem, int m0, int n0,
                                             const v16i (&acc)[big::TM][big::TN]) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = (wave & 3) >> 1;
    const int wcol = (wave & 1) * 128 + (wave >> 2) * 64;
    float *scales = reinterpret_cast<float *>(smem + 128 * 1024);
    stage_scales<big::BM, big::BN, EPI>(args, scales, m0, n0);
    store_tile_rows<EPI>(args, acc, m0, n0, wm, wcol, lane, smem, scales);
}

template <int EPI>
__global__ __launch_bounds__(big::THREADS) void w8a8_gemm_stream_kernel(GemmArgs args) {
    using namespace big;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];
    int ty, tx;
    xcd_tile(blockIdx.x, (args.m + BM - 1) / BM, (args.n + BN - 1) / BN, 4, ty, tx);
    const int m0 = ty * BM;
    const int n0 = tx * BN;
    v16i acc[TM][TN];
    big_mainloop(args, smem, m0, n0, 0, args.k / BKT, acc);
    // Epilogue: LDS free once every wave is past its last fragment read.
    __syncthreads();
    big_epilogue<EPI>(args, smem, m0, n0, acc);
}

// ----------------------------------------------------------------------------
// GEMV path (M <= 4): HBM-bound streaming of the weight with v_dot4_i32_i8,
// no MFMA.  The activation rows (M x K int8) are staged in LDS once per
// workgroup.  Integer sums are exact in any order, so the results equal the
// MFMA kernels' bit for bit.

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s, 64);
    return v;
}

template <int EPI>
__device__ __forceinline__ void store_one(const GemmArgs &args, int row, int col, int acc, float sa_row) {
    if constexpr (EPI == EPI_I32) {
        reinterpret_cast<int32_t *>(reinterpret_cast<uint8_t *>(args.acc) + static_cast<size_t>(row) * args.ldacc)[col] =
            acc;
    } else {
        float y = static_cast<float>(acc) * sa_row;
        y = y * args.sw[col];
        if constexpr (EPI == EPI_DEQUANT_BIAS) y = y + args.bias[col];
        reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(args.y) + static_cast<size_t>(row) * args.ldy)[col] = y;
    }
}

// fp32 activation rows quantised inside the GEMV workgroup (the dynamic
// W8A8 linear at M <= 4): same rule as qxt_quantize_rows_int8, computed by
// every workgroup; workgroup 0 also writes the int8 rows and scales to the
// caller's workspaces (args.a / args.sa), as the two-kernel path does.  A
// row is held in registers as RC 16-byte chunks per thread (RC = 4, 8, 16
// for K <= 4096, 8192, 16384).
constexpr int kGemvRowChunks = 16;

struct FusedRows {
    const float *x;
    uint32_t ldx;     // bytes
    uint32_t x_bytes; // descriptor range
    int floor;
};

// Load fp32 row r of the fused path into xv (zeros past K, and for r >= M).
template <int RC, int NT = kThreads>
__device__ __forceinline__ void load_row(const GemmArgs &args, const FusedRows &f, int r, v4u (&xv)[RC]) {
    const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(f.x, f.x_bytes);
    const int k4 = args.k / 4;
    const uint32_t base = static_cast<uint32_t>(r) * f.ldx;
#pragma unroll
    for (int u = 0; u < RC; ++u) {
        const int c = threadIdx.x + u * NT;
        xv[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, c < k4 && r < args.m ? base + c * 16 : kOutOfRange, 0, 0);
    }
}

// Stage activation rows [0, MR) (zeros past M) as 16-byte chunks in LDS;
// `row_sa` receives each row's scale (1 for stored int8 rows, whose scales
// the epilogue reads from args.sa).  Fused rows: row 0 arrives in `xv0`,
// which the caller loaded (before its weight loads, so that waiting for the
// row does not wait for them); later rows are loaded here.
template <int MR, int RC, bool FUSED, int NT = kThreads>
__device__ __forceinline__ void stage_rows(const GemmArgs &args, const FusedRows &f, v4u *act, float *row_sa,
                                           float *scratch, const v4u (&xv0)[RC]) {
    const int k16 = args.k / 16;
    if constexpr (!FUSED) {
        const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(args.a, args.a_bytes);
        for (int i = threadIdx.x; i < MR * k16; i += NT) {
            const int r = i / k16, c = i - r * k16;
            const uint32_t off = r < args.m ? static_cast<uint32_t>(r) * args.lda + c * 16 : kOutOfRange;
            act[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
        }
        if (threadIdx.x < MR)
            row_sa[threadIdx.x] = (args.sa != nullptr && threadIdx.x < args.m) ? args.sa[threadIdx.x] : 0.0f;
    } else {
        uint32_t *aw = reinterpret_cast<uint32_t *>(act);
        const int k4 = args.k / 4;
        // Rows of up to 8 chunks per thread request the next row before
        // reducing this one, so the row reads do not wait on each other
        // (measured on MI355X, M = 2: K = 14336, N = 4096 16.0 -> 14.5 us,
        // K = 4096, N = 14336 13.4 -> 12.6 us).
        constexpr bool kNextRow = RC <= 8;
        v4u xn[kNextRow ? RC : 1];
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            // Row 0 always exists (every entry point requires m >= 1).  Its
            // quantisation stays unconditional: behind an `r < m` branch the
            // compiler sank the caller's early row loads into that branch,
            // after the weight loads, and the row's first wait then waited for
            // every weight load of the workgroup.
            if (r > 0 && r >= args.m) {
                for (int c = threadIdx.x; c < k4; c += NT) aw[r * k4 + c] = 0;
                continue;
            }
            // The row is read once into registers, reduced, then quantised from them.
            v4u xv[RC];
            if (r == 0) {
#pragma unroll
                for (int u = 0; u < RC; ++u) xv[u] = xv0[u];
            } else if constexpr (kNextRow) {
#pragma unroll
                for (int u = 0; u < RC; ++u) xv[u] = xn[u];
            } else {
                load_row<RC, NT>(args, f, r, xv);
            }
            if constexpr (kNextRow)
                if (r + 1 < MR) load_row<RC, NT>(args, f, r + 1, xn);
            float amax = 0.0f;
#pragma unroll
            for (int u = 0; u < RC; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(__uint_as_float(xv[u][e])));
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
            if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = amax;
            __syncthreads();
            amax = scratch[0];
#pragma unroll
            for (int w = 1; w < NT / 64; ++w) amax = fmaxf(amax, scratch[w]);
            if (r + 1 < MR) __syncthreads();  // scratch is reused by the next row
            const float sc = row_scale(amax, f.floor != 0);
            // Through the scale's reciprocal, as rows_int8_kernel.  The choice
            // is uniform over the workgroup: one branch around the row's loop,
            // not one per element.
            auto quantise_row = [&](auto recip_c) {
                constexpr bool recip = decltype(recip_c)::value;
                const float rc = recip ? 1.0f / sc : 0.0f;
                auto quant = [&](uint32_t bits) {
                    const float x = __uint_as_float(bits);
                    return recip ? quant_recip(x, sc, rc) : quant_div(x, sc);
                };
#pragma unroll
                for (int u = 0; u < RC; ++u) {
                    const int c = threadIdx.x + u * NT;
                    if (c >= k4) break;
                    const v4u v = xv[u];
                    const uint32_t word = pack_bytes(quant(v[0]), quant(v[1]), quant(v[2]), quant(v[3]));
                    aw[r * k4 + c] = word;
                    if (blockIdx.x == 0)
                        reinterpret_cast<uint32_t *>(const_cast<int8_t *>(args.a) + static_cast<size_t>(r) * args.lda)[c] =
                            word;
                }
            };
            if (sc >= kRecipScaleMin)
                quantise_row(std::true_type{});
            else
                quantise_row(std::false_type{});
            if (threadIdx.x == 0) {
                row_sa[r] = sc;
                if (blockIdx.x == 0) const_cast<float *>(args.sa)[r] = sc;
            }
        }
    }
    __syncthreads();
}

// Weight [N, K] (K contiguous): each wave owns CPW output columns and streams
// their K bytes 1 KB per load instruction (lane l takes bytes 16 l .. 16 l + 15
// of each kilobyte), four kilobytes ahead of the one being reduced, the
// first four requested before the activation is staged (after the first
// fused fp32 row).  The weight is read once, so its loads are non-temporal
// (measured on MI355X at the cfg4 shapes, M = 1: 17.1 -> 16.0 us for
// K = 4096, N = 14336 and 18.2 -> 16.6 us for K = 14336, N = 4096; an
// eight-kilobyte ring for long rows was no faster).  A wave sum per column
// ends it.  256-thread workgroups take 16 columns (4 per wave); the fused
// 512-thread workgroups take 8, one per wave: twice the workgroups, so one
// workgroup's row quantisation overlaps another's weight stream (cfg4 at
// M = 1, rotated weights: 13.3 -> 12.9 us at K = 4096, N = 14336 and
// 12.8 -> 11.8 us at K = 14336, N = 4096, event-timed medians).
constexpr int kNonTemporal = 2;  // buffer-load cache policy bits: nt
template <int NT>
constexpr int gemv_cols_nk() {
    return NT == 2 * kThreads ? 8 : 16;
}
template <int MR, int RC, int EPI, bool FUSED, int NT = kThreads>
__global__ __launch_bounds__(NT) void w8a8_gemv_nk_kernel(GemmArgs args, FusedRows f) {
    constexpr int kGemvColsNK = gemv_cols_nk<NT>();
    constexpr int CPW = kGemvColsNK / (NT / 64);  // columns per wave
    extern __shared__ v4u act[];  // [MR][K / 16]
    __shared__ float row_sa[4];
    __shared__ float scratch[NT / 64];
    const int k16 = args.k / 16;
    const int lane = threadIdx.x & 63;
    const int n0 = blockIdx.x * kGemvColsNK + (threadIdx.x >> 6) * CPW;
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(args.w, args.w_bytes);
    uint32_t row_off[CPW];
#pragma unroll
    for (int j = 0; j < CPW; ++j) row_off[j] = n0 + j < args.n ? static_cast<uint32_t>(n0 + j) * args.ldw : kOutOfRange;
    auto load_cols = [&](v4u (&v)[CPW], int c) {
#pragma unroll
        for (int j = 0; j < CPW; ++j)
            v[j] = __builtin_amdgcn_raw_buffer_load_b128(
                rb, row_off[j] == kOutOfRange || c >= k16 ? kOutOfRange : row_off[j] + c * 16, 0, kNonTemporal);
    };
    // Four kilobytes of every column in flight: ring slot d holds chunk
    // c0 + 64 d of the current group of 256 chunks.
    constexpr int kDepth = 4;
    v4u xv0[RC];
    if constexpr (FUSED) load_row<RC, NT>(args, f, 0, xv0);
    v4u ring[kDepth][CPW];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load_cols(ring[d], lane + 64 * d);
    stage_rows<MR, RC, FUSED, NT>(args, f, act, row_sa, scratch, xv0);
    int acc[CPW][MR];
#pragma unroll
    for (int j = 0; j < CPW; ++j)
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[j][r] = 0;
    for (int c0 = lane; c0 < k16; c0 += 64 * kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const int c = c0 + 64 * d;
            if (c < k16) {
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    const v4u av = act[r * k16 + c];
#pragma unroll
                    for (int j = 0; j < CPW; ++j) {
                        int sum = acc[j][r];
                        sum = dot4(static_cast<int>(ring[d][j][0]), static_cast<int>(av[0]), sum);
                        sum = dot4(static_cast<int>(ring[d][j][1]), static_cast<int>(av[1]), sum);
                        sum = dot4(static_cast<int>(ring[d][j][2]), static_cast<int>(av[2]), sum);
                        sum = dot4(static_cast<int>(ring[d][j][3]), static_cast<int>(av[3]), sum);
                        acc[j][r] = sum;
                    }
                }
            }
            load_cols(ring[d], c + 64 * kDepth);
        }
    }
#pragma unroll
    for (int j = 0; j < CPW; ++j)
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[j][r] = wave_sum(acc[j][r]);
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < CPW; ++j)
#pragma unroll
            for (int r = 0; r < MR; ++r)
                if (n0 + j < args.n && r < args.m) store_one<EPI>(args, r, n0 + j, acc[j][r], row_sa[r]);
    }
}

// Rows over [N, K] weights, persistent form: a fixed grid of workgroups
// stages the rows once each (quantising fp32 rows in the fused linear,
// loading int8 rows otherwise), then every wave walks its columns
// gw, gw + W, gw + 2 W, ... (W waves in the grid, gw = wave * grid + block,
// so every workgroup holds the same number of columns to within one per
// wave) as one stream of kilobyte loads, D of them in flight across column
// boundaries.  A wave sum ends each column; lane j keeps the sum of the
// wave's column j and the outputs are stored after the last load (at most 64
// columns per wave): a store between the loads would leave reads and writes
// outstanding together, and the next wait would then drain every load in
// flight.  Measured on MI355X (rotated weights, back-to-back launches, against
// the one-column-per-wave kernel): M = 1, K = 4096: N = 14336 13.5 -> 11.6 us,
// N = 11008 11.1 -> 9.7 us; M = 1, K = 2048, N = 16384 11.5 -> 7.6 us; M = 2,
// K = 4096, N = 14336 20.0 -> 12.6 us; M = 2, K = 14336, N = 4096 16.0 ->
// 14.5 us; one row of one column per wave (K = 14336, N = 4096) 11.8 against
// 11.9 us, so one row takes this form from two columns per wave.  Four loads
// in flight per wave and two workgroups per CU: eight or sixteen loads were
// slower (12.5 / 14.4 us at M = 1, N = 14336), three workgroups per CU with
// three loads within 0.5 us either way, four workgroups per CU slower, and
// 1024-thread workgroups (one or two per CU) slower at every shape measured
// (M = 1, K = 14336, N = 4096 11.7 -> 12.4-12.8 us).  Unfused (int8 rows
// given, one to four rows), three workgroups per CU and three loads in
// flight, against the one-row-chunk kernel: M = 1, K = 4096, N = 14336
// 14.6 -> 11.0 us; M = 1, K = 14336, N = 4096 13.1 -> 11.9 us; M = 2, K =
// 4096, N = 14336 16.5 -> 11.6 us; M = 4 20.4 -> 13.5 us (N = 14336) and
// 17.2 -> 14.0 us (K = 14336, N = 4096); M = 1, K = 2048, N = 5632 6.3 ->
// 6.0-6.2 us (two workgroups and four loads: within 0.6 us of these).
#ifndef QXT_GEMV_RING
#define QXT_GEMV_RING 4
#endif
template <int MR, int RC, int EPI, int NT, int D, bool FUSED>
__global__ __launch_bounds__(NT) void w8a8_gemv_nk_stream_kernel(GemmArgs args, FusedRows f) {
    extern __shared__ v4u act[];  // [MR][K / 16]
    __shared__ float row_sa[4];
    __shared__ float scratch[NT / 64];
    const int k16 = args.k / 16;
    const int chunks = (k16 + 63) / 64;  // kilobyte loads per column and lane
    const int lane = threadIdx.x & 63;
    const int waves = gridDim.x * (NT / 64);
    const int gw = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) * gridDim.x + blockIdx.x);
    const int ncols = gw < args.n ? (args.n - gw + waves - 1) / waves : 0;  // <= 64 (checked by the launch)
    const int total = ncols * chunks;
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(args.w, args.w_bytes);
    int icol = gw, ichunk = 0;  // the next load: chunk `ichunk` of column `icol`
    auto issue = [&](v4u &slot, int t) {
        const int c = lane + 64 * ichunk;
        const uint32_t off =
            t < total && c < k16 ? static_cast<uint32_t>(icol) * args.ldw + static_cast<uint32_t>(c) * 16 : kOutOfRange;
        slot = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, kNonTemporal);
        if (++ichunk == chunks) {
            ichunk = 0;
            icol += waves;
        }
    };
    v4u xv0[RC];
    if constexpr (FUSED) load_row<RC, NT>(args, f, 0, xv0);
    v4u ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) issue(ring[d], d);
    stage_rows<MR, RC, FUSED, NT>(args, f, act, row_sa, scratch, xv0);
    int acc[MR], res[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = res[r] = 0;
    int j = 0, chunk = 0;  // the load being reduced: chunk `chunk` of the wave's column j
    for (int t0 = 0; t0 < total; t0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (t0 + d < total) {
                const int c = lane + 64 * chunk;
                if (c < k16) {
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        const v4u av = act[r * k16 + c];
                        int sum = acc[r];
                        sum = dot4(static_cast<int>(ring[d][0]), static_cast<int>(av[0]), sum);
                        sum = dot4(static_cast<int>(ring[d][1]), static_cast<int>(av[1]), sum);
                        sum = dot4(static_cast<int>(ring[d][2]), static_cast<int>(av[2]), sum);
                        sum = dot4(static_cast<int>(ring[d][3]), static_cast<int>(av[3]), sum);
                        acc[r] = sum;
                    }
                }
                if (++chunk == chunks) {
#pragma unroll
                    for (int r = 0; r < MR; ++r) {
                        const int s = wave_sum(acc[r]);
                        if (lane == j) res[r] = s;
                        acc[r] = 0;
                    }
                    chunk = 0;
                    ++j;
                }
            }
            issue(ring[d], t0 + d + D);
        }
    }
    if (lane < ncols) {
        const int col = gw + lane * waves;
#pragma unroll
        for (int r = 0; r < MR; ++r)
            if (r < args.m) store_one<EPI>(args, r, col, res[r], row_sa[r]);
    }
}

// Weight packed K4 [K/4, N] uint32 (pack_int8_quads(W).T): lane l of every
// wave owns column n0 + l; the four waves split K and add their exact
// partial sums through LDS.
constexpr int kGemvColsK4N = 64;
template <int MR, int RC, int EPI, bool FUSED>
__global__ __launch_bounds__(kThreads) void w8a8_gemv_k4n_kernel(GemmArgs args, FusedRows f) {
    extern __shared__ v4u act[];  // [MR][K / 16]
    __shared__ int part[4][MR][64];
    __shared__ float row_sa[4];
    __shared__ float scratch[kThreads / 64];
    v4u xv0[RC];
    if constexpr (FUSED) load_row<RC>(args, f, 0, xv0);
    stage_rows<MR, RC, FUSED>(args, f, act, row_sa, scratch, xv0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = blockIdx.x * kGemvColsK4N + lane;
    const int k4 = args.k / 4;
    const int per = (k4 + 3) / 4;
    const int q0 = wave * per, q1 = min(k4, q0 + per);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(args.w, args.w_bytes);
    const uint32_t col_off = col < args.n ? static_cast<uint32_t>(col) * 4 : kOutOfRange;
    const uint32_t *aw = reinterpret_cast<const uint32_t *>(act);
    int acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0;
#pragma unroll 8
    for (int q = q0; q < q1; ++q) {
        const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(
            rb, col_off == kOutOfRange ? kOutOfRange : static_cast<uint32_t>(q) * args.ldw + col_off, 0, 0);
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[r] = dot4(static_cast<int>(w), static_cast<int>(aw[r * k4 + q]), acc[r]);
    }
#pragma unroll
    for (int r = 0; r < MR; ++r) part[wave][r][lane] = acc[r];
    __syncthreads();
    if (wave == 0 && col < args.n) {
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const int s = part[0][r][lane] + part[1][r][lane] + part[2][r][lane] + part[3][r][lane];
            if (r < args.m) store_one<EPI>(args, r, col, s, row_sa[r]);
        }
    }
}

__global__ __launch_bounds__(kThreads) void dequantize_kernel(const int32_t *__restrict__ acc, size_t ldacc,
                                                              const float *__restrict__ sa,
                                                              const float *__restrict__ sw,
                                                              const float *__restrict__ bias, float *__restrict__ y,
                                                              size_t ldy, int m, int n) {
    const int row = blockIdx.y;
    const int32_t *src = reinterpret_cast<const int32_t *>(reinterpret_cast<const uint8_t *>(acc) + row * ldacc);
    float *dst = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(y) + row * ldy);
    const float s = sa[row];
    for (int c = blockIdx.x * kThreads + threadIdx.x; c < n; c += gridDim.x * kThreads) {
        float v = static_cast<float>(src[c]) * s;
        v = v * sw[c];
        if (bias != nullptr) v = v + bias[c];
        dst[c] = v;
    }
}

// Pipeline shape of the large-tile kernel: register stages in flight and the k
// step of a stage that writes the next stage to LDS.
#ifndef QXT_GEMM_DEPTH
#define QXT_GEMM_DEPTH 1
#endif
#ifndef QXT_GEMM_STORE_KS
#define QXT_GEMM_STORE_KS 2
#endif

template <int BM, int BN, int BKT, int DEPTH, int STORE_KS, bool K4N>
int launch_gemm(GemmArgs args, int epi, uint32_t layout, hipStream_t stream) {
    args.a_bytes = static_cast<uint32_t>(static_cast<size_t>(args.m - 1) * args.lda + args.k);
    args.w_bytes = layout == QXT_W8A8_WEIGHT_K4N
                       ? static_cast<uint32_t>(static_cast<size_t>(args.k / 4 - 1) * args.ldw + args.n * 4)
                       : static_cast<uint32_t>(static_cast<size_t>(args.n - 1) * args.ldw + args.k);
    dim3 grid((args.n + BN - 1) / BN, (args.m + BM - 1) / BM, 1);
    auto kernel = epi == EPI_I32        ? w8a8_gemm_kernel<BM, BN, BKT, DEPTH, STORE_KS, K4N, EPI_I32>
                  : epi == EPI_DEQUANT ? w8a8_gemm_kernel<BM, BN, BKT, DEPTH, STORE_KS, K4N, EPI_DEQUANT>
                                       : w8a8_gemm_kernel<BM, BN, BKT, DEPTH, STORE_KS, K4N, EPI_DEQUANT_BIAS>;
    return launch("w8a8_gemm_kernel", kernel, grid, dim3(kThreads), 0, stream, args);
}

int launch_stream(const GemmArgs &args, int epi, hipStream_t stream) {
    GemmArgs a2 = args;
    a2.a_bytes = static_cast<uint32_t>(static_cast<size_t>(args.m - 1) * args.lda + args.k);
    a2.w_bytes = static_cast<uint32_t>(static_cast<size_t>(args.n - 1) * args.ldw + args.k);
    dim3 grid(((args.n + big::BN - 1) / big::BN) * ((args.m + big::BM - 1) / big::BM), 1, 1);
    auto kernel = epi == EPI_I32        ? w8a8_gemm_stream_kernel<EPI_I32>
                  : epi == EPI_DEQUANT ? w8a8_gemm_stream_kernel<EPI_DEQUANT>
                                       : w8a8_gemm_stream_kernel<EPI_DEQUANT_BIAS>;
    return launch("w8a8_gemm_stream_kernel", kernel, grid, dim3(big::THREADS), 0, stream, a2);
}

// Device address of a file-scope __device__ array on the current device,
// looked up once per device with that device current (hipGetSymbolAddress):
// host code passes this address to kernels, never the array's name.
class DeviceSymbol {
  public:
    DeviceSymbol(const void *symbol, const char *what) : symbol_(symbol), what_(what) {}
    int address(uint8_t **out) {
        int device = -1;
        if (hipGetDevice(&device) != hipSuccess || device < 0)
            return fail(QXT_DEVICE_UNAVAILABLE, "%s: no current HIP device", what_);
        std::lock_guard<std::mutex> guard(mutex_);
        if (by_device_.size() <= static_cast<size_t>(device)) by_device_.resize(device + 1, nullptr);
        if (by_device_[device] == nullptr) {
            void *address = nullptr;
            const hipError_t err = hipGetSymbolAddress(&address, symbol_);
            if (err != hipSuccess || address == nullptr)
                return fail(QXT_DEVICE_UNAVAILABLE, "%s: address on device %d: %s", what_, device,
                            hipGetErrorString(err));
            by_device_[device] = static_cast<uint8_t *>(address);
        }
        *out = by_device_[device];
        return QXT_OK;
    }

  private:
    const void *symbol_;
    const char *what_;
    std::mutex mutex_;
    std::vector<uint8_t *> by_device_;
};

template <int MR, int RC, bool FUSED, int NT = kThreads>
int launch_gemv_rc(GemmArgs args, const FusedRows &f, int epi, uint32_t layout, hipStream_t stream) {
    args.a_bytes = static_cast<uint32_t>(static_cast<size_t>(args.m - 1) * args.lda + args.k);
    const size_t lds = static_cast<size_t>(MR) * args.k;
    if (layout == QXT_W8A8_WEIGHT_K4N) {
        args.w_bytes = static_cast<uint32_t>(static_cast<size_t>(args.k / 4 - 1) * args.ldw + args.n * 4);
        auto kernel = epi == EPI_I32        ? w8a8_gemv_k4n_kernel<MR, RC, EPI_I32, FUSED>
                      : epi == EPI_DEQUANT ? w8a8_gemv_k4n_kernel<MR, RC, EPI_DEQUANT, FUSED>
                                           : w8a8_gemv_k4n_kernel<MR, RC, EPI_DEQUANT_BIAS, FUSED>;
        return launch("w8a8_gemv_kernel", kernel, dim3((args.n + kGemvColsK4N - 1) / kGemvColsK4N), dim3(kThreads), lds,
                      stream, args, f);
    }
    args.w_bytes = static_cast<uint32_t>(static_cast<size_t>(args.n - 1) * args.ldw + args.k);
    auto kernel = epi == EPI_I32        ? w8a8_gemv_nk_kernel<MR, RC, EPI_I32, FUSED, NT>
                  : epi == EPI_DEQUANT ? w8a8_gemv_nk_kernel<MR, RC, EPI_DEQUANT, FUSED, NT>
                                       : w8a8_gemv_nk_kernel<MR, RC, EPI_DEQUANT_BIAS, FUSED, NT>;
    constexpr int cols = gemv_cols_nk<NT>();
    return launch("w8a8_gemv_kernel", kernel, dim3((args.n + cols - 1) / cols), dim3(NT), lds, stream,
                  args, f);
}

// Fused rows are held as K / (4 * threads) chunks per thread, rounded up to
// 4, 8 or 16 (fewer registers for short rows, more workgroups per CU).  The
// [N, K] weights run 512-thread workgroups of eight waves (one column each):
// every thread then holds half as much of the row, so the workgroup's
// quantisation, which no weight can be reduced before, ends sooner
// (measured on MI355X, cfg4 at M = 1 with rotated weights, two columns per
// wave: down 16.4 -> 14.9-15.1 us, gate_up 15.5-15.9 -> 15.2-15.3 us
// event-timed).
#ifndef QXT_GEMV_WIDE
#define QXT_GEMV_WIDE 1
#endif
constexpr bool kGemvWide = QXT_GEMV_WIDE != 0;
#ifndef QXT_GEMV_STREAM
#define QXT_GEMV_STREAM 1
#endif
#ifndef QXT_GEMV_STREAM_WGS
#define QXT_GEMV_STREAM_WGS 2
#endif
#ifndef QXT_GEMV_STREAM_ROWS
#define QXT_GEMV_STREAM_ROWS 2
#endif
#ifndef QXT_GEMV_STREAM_NT
#define QXT_GEMV_STREAM_NT 512
#endif
#ifndef QXT_GEMV_STREAM_MIN_COLS
#define QXT_GEMV_STREAM_MIN_COLS 2
#endif
#ifndef QXT_GEMV_STREAM_UNFUSED_ROWS
#define QXT_GEMV_STREAM_UNFUSED_ROWS 4
#endif
#ifndef QXT_GEMV_STREAM_MIN_COLS_UNFUSED
#define QXT_GEMV_STREAM_MIN_COLS_UNFUSED 0
#endif
#ifndef QXT_GEMV_STREAM_WGS_UNFUSED
#define QXT_GEMV_STREAM_WGS_UNFUSED 3
#endif
#ifndef QXT_GEMV_RING_UNFUSED
#define QXT_GEMV_RING_UNFUSED 3
#endif

// The persistent form of the fused GEMV, or QXT_CAPABILITY_MISSING where the
// one-column-per-wave kernel takes the problem: one row with fewer than two
// columns per wave, or more than 64 columns per wave.
template <int MR, int RC, bool FUSED>
int launch_gemv_stream(GemmArgs args, const FusedRows &f, int epi, hipStream_t stream) {
    constexpr int NT = QXT_GEMV_STREAM_NT, kWaves = NT / 64;
    constexpr int D = FUSED ? QXT_GEMV_RING : QXT_GEMV_RING_UNFUSED;
    constexpr long kPerCu = FUSED ? QXT_GEMV_STREAM_WGS : QXT_GEMV_STREAM_WGS_UNFUSED;
    const size_t lds = static_cast<size_t>(MR) * args.k;
    // Workgroups resident together on a CU: at most the requested count and
    // what 160 KB of LDS holds, so that the whole grid runs at once.
    const long per_cu =
        std::max<long>(1, std::min<long>(kPerCu, (160L * 1024) / static_cast<long>(lds + 1024)));
    const long wgs = std::min<long>(per_cu * compute_units(), (static_cast<long>(args.n) + kWaves - 1) / kWaves);
    const long waves = wgs * kWaves;
    const long min_cols = MR == 1 ? (FUSED ? QXT_GEMV_STREAM_MIN_COLS : QXT_GEMV_STREAM_MIN_COLS_UNFUSED) : 0;
    if (args.n < min_cols * waves || args.n > 64 * waves) return QXT_CAPABILITY_MISSING;
    args.a_bytes = static_cast<uint32_t>(static_cast<size_t>(args.m - 1) * args.lda + args.k);
    args.w_bytes = static_cast<uint32_t>(static_cast<size_t>(args.n - 1) * args.ldw + args.k);
    auto kernel = epi == EPI_DEQUANT ? w8a8_gemv_nk_stream_kernel<MR, RC, EPI_DEQUANT, NT, D, FUSED>
                                     : w8a8_gemv_nk_stream_kernel<MR, RC, EPI_DEQUANT_BIAS, NT, D, FUSED>;
    if constexpr (!FUSED)
        if (epi == EPI_I32) kernel = w8a8_gemv_nk_stream_kernel<MR, RC, EPI_I32, NT, D, FUSED>;
    return launch("w8a8_gemv_kernel", kernel, dim3(static_cast<uint32_t>(wgs)), dim3(NT), lds, stream, args, f);
}
template <int MR, bool FUSED>
int launch_gemv(const GemmArgs &args, const FusedRows &f, int epi, uint32_t layout, hipStream_t stream) {
    if constexpr (FUSED) {
        if (QXT_GEMV_STREAM && MR <= QXT_GEMV_STREAM_ROWS && layout == QXT_W8A8_WEIGHT_NK && epi != EPI_I32) {
            const int rc = args.k <= 4 * 4 * QXT_GEMV_STREAM_NT ? launch_gemv_stream<MR, 4, true>(args, f, epi, stream)
                                                                : launch_gemv_stream<MR, 8, true>(args, f, epi, stream);
            if (rc != QXT_CAPABILITY_MISSING) return rc;
        }
        if (kGemvWide && layout == QXT_W8A8_WEIGHT_NK) {
            constexpr int NT = 2 * kThreads;
            if (args.k <= 4 * 4 * NT) return launch_gemv_rc<MR, 4, true, NT>(args, f, epi, layout, stream);
            return launch_gemv_rc<MR, 8, true, NT>(args, f, epi, layout, stream);
        }
        if (args.k <= 4 * 4 * kThreads) return launch_gemv_rc<MR, 4, true>(args, f, epi, layout, stream);
        if (args.k <= 8 * 4 * kThreads) return launch_gemv_rc<MR, 8, true>(args, f, epi, layout, stream);
        return launch_gemv_rc<MR, kGemvRowChunks, true>(args, f, epi, layout, stream);
    } else {
        if (QXT_GEMV_STREAM && MR <= QXT_GEMV_STREAM_UNFUSED_ROWS && layout == QXT_W8A8_WEIGHT_NK) {
            const int rc = launch_gemv_stream<MR, 1, false>(args, f, epi, stream);
            if (rc != QXT_CAPABILITY_MISSING) return rc;
        }
        return launch_gemv_rc<MR, 1, false>(args, f, epi, layout, stream);
    }
}

template <bool FUSED>
int dispatch_gemv(const GemmArgs &args, const FusedRows &f, int epi, uint32_t layout, hipStream_t stream) {
    switch (args.m) {
        case 1: return launch_gemv<1, FUSED>(args, f, epi, layout, stream);
        case 2: return launch_gemv<2, FUSED>(args, f, epi, layout, stream);
        default: return launch_gemv<4, FUSED>(args, f, epi, layout, stream);
    }
}

// Rows up to which the GEMV path runs; its activation rows (padded to 1, 2
// or 4) must fit the 60 KB of dynamic LDS it stages them in.
constexpr int kGemvMaxRows = 4;
constexpr size_t kGemvMaxLds = 60 * 1024;

bool gemv_path(int m, int k) {
    const int rows = m <= 2 ? m : 4;
    return m <= kGemvMaxRows && static_cast<size_t>(rows) * k <= kGemvMaxLds;
}

int run_gemm(const GemmArgs &args, int epi, uint32_t layout, hipStream_t stream) {
    if (gemv_path(args.m, args.k)) return dispatch_gemv<false>(args, FusedRows{}, epi, layout, stream);
    // 256 x 256 tiles once they give every CU a workgroup; 128 x 128 below that.
    const long cus = compute_units();
    const long tm = (args.m + 255) / 256, tn = (args.n + 255) / 256;
    const bool big = tm * tn >= cus;
    constexpr int D = QXT_GEMM_DEPTH, S = QXT_GEMM_STORE_KS;
    if (big && layout == QXT_W8A8_WEIGHT_NK && args.k % big::BKT == 0) {
        // gate_up of cfg4 leaves its last round of 16 x 56 tiles half empty.
        // Measured on MI355X, nothing that fills it was faster: a second
        // launch of 256 x 128 tiles (the generic kernel needs as long for a
        // half tile as this one for a full tile); a stream-K schedule over
        // all tiles, bit-exact, 307-321 us against 240-248 us (the workgroups
        // of an XCD no longer run in lockstep over shared A and B panels); the
        // last round's tiles split in K over two workgroups, the partial sums
        // passed through the output block: 300-320 us with device-scope
        // release/acquire fences (each writes back the whole L2), equal to this
        // kernel with write-through partial rows.  The board is power-bound:
        // the same kernel reading constant operands instead of the matrices
        // (a timing-only copy) runs gate_up in 199 us and down in 152 us.
        return launch_stream(args, epi, stream);
    }
    // Fewer 128 x 128 tiles than CUs (small M and N, e.g. one GPU's row shard
    // of a down projection, M = 512, N = 4096, K = 14336): 64 x 64 tiles with
    // 128-byte K stages fill the GPU instead (measured on MI355X: 115 -> 69 us
    // for that shard; 31 -> 17 us at M = 256, K = N = 4096).
    const long t128 = ((args.m + 127) / 128) * ((args.n + 127) / 128);
    if (!big && t128 < cus) {
        if (layout == QXT_W8A8_WEIGHT_K4N) return launch_gemm<64, 64, 128, 1, 1, true>(args, epi, layout, stream);
        return launch_gemm<64, 64, 128, 1, 1, false>(args, epi, layout, stream);
    }
    if (layout == QXT_W8A8_WEIGHT_K4N)
        return big ? launch_gemm<256, 256, 128, D, S, true>(args, epi, layout, stream)
                   : launch_gemm<128, 128, 64, 1, 1, true>(args, epi, layout, stream);
    return big ? launch_gemm<256, 256, 128, D, S, false>(args, epi, layout, stream)
               : launch_gemm<128, 128, 64, 1, 1, false>(args, epi, layout, stream);
}

int validate_gemm(const int8_t *a, size_t lda, const void *w, size_t ldw, uint32_t m, uint32_t n, uint32_t k,
                  uint32_t layout) {
    if (a == nullptr || w == nullptr) return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: null operand");
    if (m == 0 || n == 0 || k == 0 || k % 16)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: m, n > 0 and k a positive multiple of 16 required");
    if (m > (1u << 30) || n > (1u << 30) || (m + 127) / 128 > 65535u)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: problem too large");
    if (static_cast<uint64_t>(k) * 127 * 127 > 2147483647ull)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: k=%u can overflow int32 accumulation", k);
    if (layout != QXT_W8A8_WEIGHT_NK && layout != QXT_W8A8_WEIGHT_K4N)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: unknown weight layout %u", layout);
    if (lda < k || lda % 16 || !aligned(a, 16) || !aligned(w, 16))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: operands need 16-byte aligned rows");
    if (layout == QXT_W8A8_WEIGHT_NK && (ldw < k || ldw % 16))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: NK weight needs 16-byte aligned rows of >= k bytes");
    if (layout == QXT_W8A8_WEIGHT_K4N && (n % 4 || ldw < static_cast<size_t>(n) * 4 || ldw % 16))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: K4N weight needs n %% 4 == 0 and 16-byte aligned rows");
    const size_t w_rows = layout == QXT_W8A8_WEIGHT_K4N ? k / 4 : n;
    if (static_cast<size_t>(m) * lda >= (1ull << 31) || w_rows * ldw >= (1ull << 31))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: operands must be smaller than 2 GiB");
    return QXT_OK;
}

int validate_epilogue(const float *sa, const float *sw, const float *bias, const float *y, size_t ldy,
                      uint32_t n) {
    if (sa == nullptr || sw == nullptr || y == nullptr)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 epilogue: null scale or output");
    if (!aligned(sa, 4) || !aligned(sw, 4) || !aligned(y, 4) || (bias != nullptr && !aligned(bias, 4)) ||
        ldy % 4 || ldy < static_cast<size_t>(n) * 4)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 epilogue: bad output stride or alignment");
    return QXT_OK;
}

// ------------------------------------------------- static workspace (no allocation)
//
// qxt_w8a8_linear_noalloc keeps the quantised activation rows (int8, row
// stride k) and their fp32 row scales in this array instead of caller or
// library allocations.  Each GPU holds its own copy from the moment the
// library's code object is loaded on it until the process ends; every call
// on a GPU reuses that GPU's copy.  Nothing in it has to start at zero: the
// row quantiser writes every byte a call reads.
constexpr size_t kScratchRowBytes = size_t(64) << 20;   // int8 activation rows: m * k <= 64 MiB
constexpr size_t kScratchScaleBytes = size_t(256) << 10;  // fp32 row scales: m <= 65,536
constexpr uint32_t kScratchMaxRows = kScratchScaleBytes / sizeof(float);

static __device__ __align__(256) uint8_t scratch[kScratchRowBytes + kScratchScaleBytes];

// Device address of `scratch` on the current device (DeviceSymbol: looked up
// once per device with that device current).  Host code never passes the
// array's name to a kernel or copy: on the host that name is only a stand-in
// for the symbol, not a device address.
int scratch_address(uint8_t **out) {
    static DeviceSymbol symbol(HIP_SYMBOL(scratch), "w8a8 linear noalloc workspace");
    return symbol.address(out);
}

}  // namespace
}  // namespace qxt

using namespace qxt;

extern "C" {

int qxt_w8a8_gemm_i32(const int8_t *a, size_t lda, const void *w, size_t ldw, int32_t *acc, size_t ldacc,
                      uint32_t m, uint32_t n, uint32_t k, uint32_t weight_layout, void *stream) {
    int rc = validate_gemm(a, lda, w, ldw, m, n, k, weight_layout);
    if (rc != QXT_OK) return rc;
    if (acc == nullptr || !aligned(acc, 4) || ldacc % 4 || ldacc < static_cast<size_t>(n) * 4)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: bad accumulator output");
    if (static_cast<uint64_t>(m) * ldacc >= (1ull << 31))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: the output must be smaller than 2 GiB");
    rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    GemmArgs args{a, lda, static_cast<const uint8_t *>(w), ldw, acc, ldacc, nullptr, nullptr, nullptr,
                  nullptr, 0, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k)};
    return run_gemm(args, EPI_I32, weight_layout, as_stream(stream));
}

int qxt_w8a8_gemm_dequantize(const int8_t *a, size_t lda, const void *w, size_t ldw, const float *row_scales,
                             const float *column_scales, const float *bias, float *y, size_t ldy, uint32_t m,
                             uint32_t n, uint32_t k, uint32_t weight_layout, void *stream) {
    int rc = validate_gemm(a, lda, w, ldw, m, n, k, weight_layout);
    if (rc != QXT_OK) return rc;
    rc = validate_epilogue(row_scales, column_scales, bias, y, ldy, n);
    if (rc != QXT_OK) return rc;
    if (static_cast<uint64_t>(m) * ldy >= (1ull << 31))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 gemm: the output must be smaller than 2 GiB");
    rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    GemmArgs args{a, lda, static_cast<const uint8_t *>(w), ldw, nullptr, 0, row_scales, column_scales, bias,
                  y, ldy, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k)};
    return run_gemm(args, bias != nullptr ? EPI_DEQUANT_BIAS : EPI_DEQUANT, weight_layout, as_stream(stream));
}

int qxt_w8a8_dequantize(const int32_t *acc, size_t ldacc, const float *row_scales, const float *column_scales,
                        const float *bias, float *y, size_t ldy, uint32_t m, uint32_t n, void *stream) {
    if (acc == nullptr || !aligned(acc, 4) || ldacc % 4 || ldacc < static_cast<size_t>(n) * 4)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 dequantize: bad accumulator input");
    if (m == 0 || n == 0 || m > 65535u) return fail(QXT_INVALID_ARGUMENT, "w8a8 dequantize: bad shape");
    int rc = validate_epilogue(row_scales, column_scales, bias, y, ldy, n);
    if (rc != QXT_OK) return rc;
    rc = injected(QXT_FAIL_SUBMISSION);
    if (rc != QXT_OK) return rc;
    const unsigned gx = static_cast<unsigned>(std::min<uint32_t>((n + kThreads - 1) / kThreads, 64u));
    return launch("w8a8_dequantize_kernel", dequantize_kernel, dim3(gx, m, 1), dim3(kThreads), 0,
                  as_stream(stream), acc, ldacc, row_scales, column_scales, bias, y, ldy, static_cast<int>(m),
                  static_cast<int>(n));
}

int qxt_w8a8_linear(const float *x, size_t ldx, int8_t *qa, size_t ldqa, float *sa, const void *w, size_t ldw,
                    const float *column_scales, const float *bias, float *y, size_t ldy, uint32_t m, uint32_t n,
                    uint32_t k, uint32_t weight_layout, uint32_t flags, void *stream) {
    int rc = validate_gemm(qa, ldqa, w, ldw, m, n, k, weight_layout);
    if (rc != QXT_OK) return rc;
    rc = validate_epilogue(sa, column_scales, bias, y, ldy, n);
    if (rc != QXT_OK) return rc;
    if (static_cast<uint64_t>(m) * ldy >= (1ull << 31))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 linear: the output must be smaller than 2 GiB");
    if (x == nullptr || ldx % 4 || ldx < static_cast<size_t>(k) * 4 || !aligned(x, 4))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 linear: bad activation input");
    if (flags & ~QXT_QUANT_NO_SCALE_FLOOR) return fail(QXT_INVALID_ARGUMENT, "w8a8 linear: unknown flags");
    // Three or four rows take the row pre-pass and the unfused GEMV (its
    // persistent form) instead of quantising every row in every workgroup,
    // except for rows longer than 4096 over at most 48 MiB of weights, where
    // the fused launch stays ahead.  Measured on MI355X, rotated weights, back
    // to back: M = 4, K = 4096, N = 14336 16.8 against 27.6 us fused; M = 4,
    // K = 14336, N = 4096 20.0 against 21.8 us; M = 4, K = N = 8192 19.0
    // against 24.3 us; M = 4, K = 11008, N = 4096 19.0 against 18.6 us; M = 3,
    // K = 5632, N = 2048 9.9 against 8.6 us.  Two rows always fuse.
    const bool fuse_rows = m <= 2 || (k > 4096 && static_cast<uint64_t>(n) * k <= (48ull << 20));
    if (fuse_rows && gemv_path(static_cast<int>(m), static_cast<int>(k)) && k <= 4u * kThreads * kGemvRowChunks &&
        aligned(x, 16) && ldx % 16 == 0 &&
        static_cast<uint64_t>(m - 1) * ldx + static_cast<uint64_t>(k) * 4 < (1ull << 31)) {
        // One launch: every GEMV workgroup quantises the rows itself.
        rc = injected(QXT_FAIL_SUBMISSION);
        if (rc != QXT_OK) return rc;
        GemmArgs args{qa, ldqa, static_cast<const uint8_t *>(w), ldw, nullptr, 0, sa, column_scales, bias,
                      y, ldy, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k)};
        const FusedRows f{x, static_cast<uint32_t>(ldx),
                          static_cast<uint32_t>(static_cast<uint64_t>(m - 1) * ldx + static_cast<uint64_t>(k) * 4),
                          (flags & QXT_QUANT_NO_SCALE_FLOOR) ? 0 : 1};
        return dispatch_gemv<true>(args, f, bias != nullptr ? EPI_DEQUANT_BIAS : EPI_DEQUANT, weight_layout,
                                   as_stream(stream));
    }
    rc = qxt_quantize_rows_int8(x, ldx, qa, ldqa, sa, m, k, k, flags, stream);
    if (rc != QXT_OK) return rc;
    GemmArgs args{qa, ldqa, static_cast<const uint8_t *>(w), ldw, nullptr, 0, sa, column_scales, bias,
                  y, ldy, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k)};
    return run_gemm(args, bias != nullptr ? EPI_DEQUANT_BIAS : EPI_DEQUANT, weight_layout, as_stream(stream));
}

int qxt_w8a8_linear_noalloc(const float *x, size_t ldx, const void *w, size_t ldw, const float *column_scales,
                            const float *bias, float *y, size_t ldy, uint32_t m, uint32_t n, uint32_t k,
                            uint32_t weight_layout, uint32_t flags, void *stream) {
    if (m == 0 || k == 0 || k % 16)
        return fail(QXT_INVALID_ARGUMENT, "w8a8 linear noalloc: m > 0 and k a positive multiple of 16 required");
    if (m > kScratchMaxRows || static_cast<uint64_t>(m) * k > kScratchRowBytes)
        return fail(QXT_INVALID_ARGUMENT,
                    "w8a8 linear noalloc: m = %u rows of k = %u exceed the static workspace (m <= %u, m * k <= %zu)",
                    m, k, kScratchMaxRows, kScratchRowBytes);
    uint8_t *base = nullptr;
    int rc = scratch_address(&base);
    if (rc != QXT_OK) return rc;
    int8_t *qa = reinterpret_cast<int8_t *>(base);
    float *sa = reinterpret_cast<float *>(base + kScratchRowBytes);
    return qxt_w8a8_linear(x, ldx, qa, k, sa, w, ldw, column_scales, bias, y, ldy, m, n, k, weight_layout, flags,
                           stream);
}

}  // extern "C"

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
// Tiling: a 256-thread workgroup (4 waves, 2 x 2) owns a BM x BN output tile;
// each wave owns a (BM/2) x (BN/2) sub-tile of 32 x 32 MFMA blocks.  K advances
// in steps of 64 bytes; A and B tiles live in LDS with K contiguous per row,
// padded to 80 bytes so the 16-byte fragment reads are bank-conflict free.
// The MFMA lane layout: lane l supplies A[l % 32][k-chunk(l / 32)] and
// B[k-chunk(l / 32)][l % 32] (the same 16 k values for both operands, so the
// exact integer sum does not depend on how the chunk is ordered) and receives
// D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32] in accumulator register r.
#include <algorithm>

#include "qxt_common.h"

namespace qxt {
namespace {

constexpr int kThreads = 256;
constexpr int BK = 64;          // K bytes per LDS stage
constexpr int LDS_ROW = BK + 16;  // padded row pitch in bytes

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
};

template <int BM, int BN, bool K4N, int EPI>
__global__ __launch_bounds__(kThreads) void w8a8_gemm_kernel(GemmArgs args) {
    __shared__ __attribute__((aligned(16))) uint8_t As[BM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[BN * LDS_ROW];

    constexpr int WM = BM / 2, WN = BN / 2;      // per-wave sub-tile
    constexpr int TM = WM / 32, TN = WN / 32;    // 32x32 blocks per wave
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    for (int k0 = 0; k0 < args.k; k0 += BK) {
        // ---- global -> LDS: A tile, 16-byte chunks (4 per row).
#pragma unroll
        for (int c = tid; c < BM * (BK / 16); c += kThreads) {
            const int row = c >> 2, kc = c & 3;
            const int gm = m0 + row, gk = k0 + kc * 16;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (gm < args.m && gk < args.k)
                v = *reinterpret_cast<const uint4 *>(args.a + static_cast<size_t>(gm) * args.lda + gk);
            *reinterpret_cast<uint4 *>(As + row * LDS_ROW + kc * 16) = v;
        }
        // ---- global -> LDS: B tile.
        if constexpr (!K4N) {
#pragma unroll
            for (int c = tid; c < BN * (BK / 16); c += kThreads) {
                const int row = c >> 2, kc = c & 3;
                const int gn = n0 + row, gk = k0 + kc * 16;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (gn < args.n && gk < args.k)
                    v = *reinterpret_cast<const uint4 *>(args.w + static_cast<size_t>(gn) * args.ldw + gk);
                *reinterpret_cast<uint4 *>(Bs + row * LDS_ROW + kc * 16) = v;
            }
        } else {
            // uint32 [K/4, N]: a 16-byte chunk holds k-quad k4 of 4 adjacent columns.
#pragma unroll
            for (int c = tid; c < (BK / 4) * (BN / 4); c += kThreads) {
                const int k4 = c / (BN / 4), nq = c % (BN / 4);
                const int gn = n0 + nq * 4, gk = k0 + k4 * 4;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (gn < args.n && gk < args.k)
                    v = *reinterpret_cast<const uint4 *>(args.w + static_cast<size_t>(gk / 4) * args.ldw +
                                                         static_cast<size_t>(gn) * 4);
                *reinterpret_cast<uint32_t *>(Bs + (nq * 4 + 0) * LDS_ROW + k4 * 4) = v.x;
                *reinterpret_cast<uint32_t *>(Bs + (nq * 4 + 1) * LDS_ROW + k4 * 4) = v.y;
                *reinterpret_cast<uint32_t *>(Bs + (nq * 4 + 2) * LDS_ROW + k4 * 4) = v.z;
                *reinterpret_cast<uint32_t *>(Bs + (nq * 4 + 3) * LDS_ROW + k4 * 4) = v.w;
            }
        }
        __syncthreads();

        // ---- MFMA over the 64-byte K stage (two 32-deep steps).
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            v4i af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const v4i *>(As + (wm * WM + i * 32 + (lane & 31)) * LDS_ROW + kk +
                                                       (lane >> 5) * 16);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *reinterpret_cast<const v4i *>(Bs + (wn * WN + j * 32 + (lane & 31)) * LDS_ROW + kk +
                                                       (lane >> 5) * 16);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // ---- epilogue.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int gn = n0 + wn * WN + j * 32 + (lane & 31);
            if (gn >= args.n) continue;
            float swn = 0.0f, bn = 0.0f;
            if constexpr (EPI != EPI_I32) swn = args.sw[gn];
            if constexpr (EPI == EPI_DEQUANT_BIAS) bn = args.bias[gn];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int gm = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (gm >= args.m) continue;
                const int v = acc[i][j][r];
                if constexpr (EPI == EPI_I32) {
                    int32_t *out = reinterpret_cast<int32_t *>(reinterpret_cast<uint8_t *>(args.acc) +
                                                               static_cast<size_t>(gm) * args.ldacc);
                    out[gn] = v;
                } else {
                    float yv = static_cast<float>(v) * args.sa[gm];
                    yv = yv * swn;
                    if constexpr (EPI == EPI_DEQUANT_BIAS) yv = yv + bn;
                    float *out = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(args.y) +
                                                           static_cast<size_t>(gm) * args.ldy);
                    out[gn] = yv;
                }
            }
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

template <int BM, int BN, bool K4N>
int launch_gemm(const GemmArgs &args, int epi, hipStream_t stream) {
    dim3 grid((args.n + BN - 1) / BN, (args.m + BM - 1) / BM, 1);
    auto kernel = epi == EPI_I32        ? w8a8_gemm_kernel<BM, BN, K4N, EPI_I32>
                  : epi == EPI_DEQUANT ? w8a8_gemm_kernel<BM, BN, K4N, EPI_DEQUANT>
                                       : w8a8_gemm_kernel<BM, BN, K4N, EPI_DEQUANT_BIAS>;
    return launch("w8a8_gemm_kernel", kernel, grid, dim3(kThreads), 0, stream, args);
}

int run_gemm(const GemmArgs &args, int epi, uint32_t layout, hipStream_t stream) {
    if (layout == QXT_W8A8_WEIGHT_K4N) return launch_gemm<128, 128, true>(args, epi, stream);
    return launch_gemm<128, 128, false>(args, epi, stream);
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
    if (x == nullptr || ldx % 4 || ldx < static_cast<size_t>(k) * 4 || !aligned(x, 4))
        return fail(QXT_INVALID_ARGUMENT, "w8a8 linear: bad activation input");
    if (flags & ~QXT_QUANT_NO_SCALE_FLOOR) return fail(QXT_INVALID_ARGUMENT, "w8a8 linear: unknown flags");
    rc = qxt_quantize_rows_int8(x, ldx, qa, ldqa, sa, m, k, k, flags, stream);
    if (rc != QXT_OK) return rc;
    GemmArgs args{qa, ldqa, static_cast<const uint8_t *>(w), ldw, nullptr, 0, sa, column_scales, bias,
                  y, ldy, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k)};
    return run_gemm(args, bias != nullptr ? EPI_DEQUANT_BIAS : EPI_DEQUANT, weight_layout, as_stream(stream));
}

}  // extern "C"

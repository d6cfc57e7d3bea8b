// llama.cpp-facing prepared Q4_0 x Q8_0 linear (include/qxt_llama_q4_0.h).
//
// Contract of the reference bridge (integrations/llama_cpp/src/qpu_llama_q4_0.c
// and the context part of qpu_llama_runtime.c), re-planned for one GPU:
//   prepare  -- validate, check the source hash, allocate every buffer once
//               (device weights/activation/output, pinned host staging),
//               upload the resident columns (CPU_REPACK groups are unpacked
//               by a kernel; decode-sized linears keep them in the lane
//               layout), then never allocate again;
//   submit   -- host rows -> pinned staging -> HBM on the context's stream,
//               CPU_REPACK Q8_0x4 rows de-interleaved by a kernel, the Q4_0
//               linear over the selected columns, the selected output columns
//               -> pinned staging, one completion event;
//   wait     -- poll the event up to the context timeout, then copy the
//               staged columns into the caller's destination.  Nothing reaches
//               the destination unless the whole submission succeeded.

#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <thread>

#include "qxt_common.h"
#include "qxt_llama_q4_0.h"

#ifndef QXT_Q4_0_SOURCE_HASH
#define QXT_Q4_0_SOURCE_HASH "unhashed-build"
#endif

namespace {

constexpr uint64_t kDefaultTimeoutNs = 10000000000ull;  // qpu_llama_runtime.c:22
constexpr uint32_t kOutputTile = 16;
constexpr uint32_t kMaxRows = 4u * 65535u;  // qpu_llama_q4_0.c:210
constexpr uint32_t kRepackGroupBytes = 4 * qxt::Q4_0_BYTES;     // block_q4_0x4: 4 x fp16 d + 64 B
constexpr uint32_t kInterleavedBlockBytes = 4 * qxt::Q8_0_BYTES; // block_q8_0x4: 4 x fp16 d + 128 B
constexpr uint32_t kKnownFailures =
    QXT_FAIL_DEVICE_OPEN | QXT_FAIL_ALLOCATION | QXT_FAIL_SUBMISSION | QXT_FAIL_WAIT | QXT_FAIL_SOURCE_HASH;

uint64_t now_ns() {
    return static_cast<uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
            .count());
}

bool mul_size(size_t a, size_t b, size_t *out) {
    if (a != 0 && b > SIZE_MAX / a) return false;
    *out = a * b;
    return true;
}

bool in_range(size_t total, size_t offset, size_t size) { return offset <= total && size <= total - offset; }

// Makes the context's device current for the scope and restores the caller's.
class DeviceScope {
  public:
    explicit DeviceScope(int device) {
        if (hipGetDevice(&previous_) != hipSuccess) previous_ = -1;
        if (previous_ != device) (void)hipSetDevice(device);
    }
    ~DeviceScope() {
        if (previous_ >= 0) (void)hipSetDevice(previous_);
    }

  private:
    int previous_ = -1;
};

// ------------------------------------------------------------------ kernels

// CPU_REPACK block_q4_0x4 -> native Q4_0 blocks (the inverse of ggml's
// make_block_q4_0x4 with a 4-byte interleave, as unpacked by the reference
// backend at ggml-qpu.cpp:250-284).  Group g, block b holds the fp16 scales
// of columns 4g..4g+3 and 16 words; word 4c + r carries bytes 4c..4c+3 of
// column r's 16 code bytes with both nibbles XOR 8.  One thread per
// (column, block); every access is 2- or 4-byte aligned.
__global__ void unpack_q4_0x4_kernel(const uint8_t *__restrict__ groups, uint8_t *__restrict__ blocks_out,
                                     uint32_t columns, uint32_t blocks) {
    const size_t item = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (item >= static_cast<size_t>(columns) * blocks) return;
    const uint32_t column = static_cast<uint32_t>(item / blocks);
    const uint32_t block = static_cast<uint32_t>(item % blocks);
    const uint32_t lane = column & 3u;
    const uint8_t *group = groups + (static_cast<size_t>(column >> 2) * blocks + block) * kRepackGroupBytes;
    uint16_t *out = reinterpret_cast<uint16_t *>(blocks_out + item * qxt::Q4_0_BYTES);
    out[0] = *reinterpret_cast<const uint16_t *>(group + 2 * lane);
    const uint32_t *words = reinterpret_cast<const uint32_t *>(group + 8);
#pragma unroll
    for (uint32_t chunk = 0; chunk < 4; ++chunk) {
        const uint32_t w = words[4 * chunk + lane] ^ 0x88888888u;
        out[1 + 2 * chunk] = static_cast<uint16_t>(w & 0xFFFFu);
        out[2 + 2 * chunk] = static_cast<uint16_t>(w >> 16);
    }
}

// CPU_REPACK block_q8_0x4 rows -> native Q8_0 rows (qpu_llama_q4_0.c:160-203).
// Rows below rows - rows % 4 come in groups of four: per block, the four fp16
// scales, then the 4 x 32 values with value i of row r at
// (i / il) * 4 * il + r * il + i % il (il = 4 or 8).  The remaining rows are
// native.  One thread per (row, block).
__global__ void deinterleave_q8_0x4_kernel(const uint8_t *__restrict__ source, uint8_t *__restrict__ rows_out,
                                           uint32_t rows, uint32_t blocks, uint32_t interleave) {
    const size_t item = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (item >= static_cast<size_t>(rows) * blocks) return;
    const uint32_t row = static_cast<uint32_t>(item / blocks);
    const uint32_t block = static_cast<uint32_t>(item % blocks);
    const size_t row_bytes = static_cast<size_t>(blocks) * qxt::Q8_0_BYTES;
    uint16_t *out = reinterpret_cast<uint16_t *>(rows_out + item * qxt::Q8_0_BYTES);
    if (row >= rows - rows % 4u) {
        const uint16_t *in = reinterpret_cast<const uint16_t *>(source + item * qxt::Q8_0_BYTES);
#pragma unroll
        for (int i = 0; i < qxt::Q8_0_BYTES / 2; ++i) out[i] = in[i];
        return;
    }
    const uint32_t lane = row & 3u;
    const uint8_t *group = source + static_cast<size_t>(row >> 2) * 4 * row_bytes +
                           static_cast<size_t>(block) * kInterleavedBlockBytes;
    out[0] = *reinterpret_cast<const uint16_t *>(group + 2 * lane);
    const uint8_t *values = group + 8;
#pragma unroll
    for (uint32_t w = 0; w < 8; ++w) {
        // Values 4w..4w+3 of this row are contiguous for both interleaves.
        const uint32_t first = 4 * w;
        const uint32_t at = (first / interleave) * 4 * interleave + lane * interleave + first % interleave;
        const uint32_t word = *reinterpret_cast<const uint32_t *>(values + at);
        out[1 + 2 * w] = static_cast<uint16_t>(word & 0xFFFFu);
        out[2 + 2 * w] = static_cast<uint16_t>(word >> 16);
    }
}

uint32_t grid_for(size_t items, uint32_t threads) { return static_cast<uint32_t>((items + threads - 1) / threads); }

}  // namespace

// ------------------------------------------------------------------ handles

struct qxt_llama_context {
    int device = 0;
    hipStream_t stream = nullptr;
    uint64_t timeout_ns = kDefaultTimeoutNs;
    std::atomic<uint32_t> failure_mask{0};
    std::mutex mutex;  // guards active / poisoned
    bool active = false;
    bool poisoned = false;
    mutable std::mutex error_mutex;
    char last_error[256] = "";

    int fail(int status, const char *fmt, ...) __attribute__((format(printf, 3, 4))) {
        std::lock_guard<std::mutex> guard(error_mutex);
        va_list args;
        va_start(args, fmt);
        vsnprintf(last_error, sizeof(last_error), fmt, args);
        va_end(args);
        return status;
    }
    bool injected(uint32_t point) const { return (failure_mask.load(std::memory_order_relaxed) & point) != 0; }
};

struct qxt_llama_q4_0_linear {
    qxt_llama_context *context = nullptr;
    uint32_t blocks = 0;
    uint32_t output_columns = 0;
    uint32_t rows = 0;
    uint32_t resident_start = 0;
    uint32_t resident_count = 0;
    size_t weight_row_bytes = 0;      // blocks * 18
    size_t activation_row_bytes = 0;  // blocks * 34
    size_t output_row_bytes = 0;      // resident_count * 4
    size_t resident_bytes = 0;
    size_t weight_bytes = 0;
    bool lanes = false;               // weight in the lane layout (decode-sized linears)
    qxt_llama_q4_0_weight_mode mode = QXT_LLAMA_Q4_0_WEIGHT_EXACT;
    // EXACT: device Q4_0 [resident_count][blocks] (native or lane layout).
    // COLUMN_W8 / ROWCOL_W8A8: int8 codes as uint32 words [blocks * 8][resident_count].
    void *weight = nullptr;
    float *column_scales = nullptr;   // approximate modes: fp32 [resident_count]
    int8_t *activation_q = nullptr;   // approximate modes: int8 [rows][blocks * 32]
    void *activation_scales = nullptr;  // COLUMN_W8: fp16 bits [rows][blocks]; ROWCOL_W8A8: fp32 [rows]
    void *activation = nullptr;       // device Q8_0 [rows][blocks]
    void *activation_packed = nullptr;  // device copy of interleaved host rows
    float *output = nullptr;          // device fp32 [rows][resident_count]
    void *host_activation = nullptr;  // pinned staging
    float *host_output = nullptr;     // pinned staging [rows][resident_count]
    hipEvent_t done = nullptr;
    std::mutex mutex;
    bool busy = false;
};

struct qxt_llama_q4_0_submission {
    qxt_llama_q4_0_linear *linear = nullptr;
    uint8_t *destination = nullptr;
    uint32_t rows = 0;
    uint32_t column_start = 0;
    uint32_t column_count = 0;
    uint32_t local_start = 0;
    uint64_t complete_start = 0;
    uint64_t input_access_end = 0;
    uint64_t input_pack_end = 0;
    uint64_t input_copy_end = 0;
    uint64_t submit_start = 0;
    uint64_t submit_end = 0;
    bool active = false;
};

namespace {

void release_buffers(qxt_llama_q4_0_linear *l) {
    if (l->done) (void)hipEventDestroy(l->done);
    for (void *p : {l->weight, l->activation, l->activation_packed, static_cast<void *>(l->output),
                    static_cast<void *>(l->column_scales), static_cast<void *>(l->activation_q), l->activation_scales})
        if (p) (void)hipFree(p);
    if (l->host_activation) (void)hipHostFree(l->host_activation);
    if (l->host_output) (void)hipHostFree(l->host_output);
    l->done = nullptr;
    l->weight = l->activation = l->activation_packed = l->activation_scales = nullptr;
    l->output = l->column_scales = nullptr;
    l->activation_q = nullptr;
    l->host_activation = nullptr;
    l->host_output = nullptr;
}

void end_submission(qxt_llama_q4_0_linear *l, bool poison) {
    qxt_llama_context *ctx = l->context;
    {
        std::lock_guard<std::mutex> guard(ctx->mutex);
        ctx->active = false;
        if (poison) ctx->poisoned = true;
    }
    std::lock_guard<std::mutex> guard(l->mutex);
    l->busy = false;
}

// Copy the resident weight columns to the device, unpacking CPU_REPACK groups
// and, for decode-sized linears, re-laying the native rows out in the lane
// layout the decode kernels stream fastest (qxt_q4_0_pack_lanes); in the
// approximate modes, re-quantising each column to int8 codes with one fp32
// scale (qpu_llama_q4_0.c:332-386).
int upload_weights(qxt_llama_q4_0_linear *l, const qxt_llama_q4_0_linear_desc *d) {
    qxt_llama_context *ctx = l->context;
    const size_t bytes = static_cast<size_t>(l->resident_count) * l->weight_row_bytes;
    // Columns [start, start + count) occupy the same byte range in both host
    // layouts (a CPU_REPACK group of 4 columns is 4 native rows long, start % 4 == 0).
    const uint8_t *src = static_cast<const uint8_t *>(d->weights) + l->resident_start * l->weight_row_bytes;
    const bool repack = d->weight_format == QXT_LLAMA_Q4_0_FORMAT_REPACK_4X4;
    const bool approximate = l->mode != QXT_LLAMA_Q4_0_WEIGHT_EXACT;
    void *raw = nullptr;     // host bytes as uploaded, when they are not yet native rows
    void *native = nullptr;  // native rows, when they are not the final layout
    hipError_t err = hipSuccess;
    if (repack) err = qxt::device_malloc(&raw, bytes);
    if (err == hipSuccess && (l->lanes || approximate)) err = qxt::device_malloc(&native, bytes);
    if (err != hipSuccess) {
        (void)hipFree(raw);
        return ctx->fail(QXT_ALLOCATION_FAILED, "weight staging: %s", hipGetErrorString(err));
    }
    void *rows = l->lanes || approximate ? native : l->weight;
    err = hipMemcpyAsync(repack ? raw : rows, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess && repack) {
        const size_t items = static_cast<size_t>(l->resident_count) * l->blocks;
        hipLaunchKernelGGL(unpack_q4_0x4_kernel, dim3(grid_for(items, 256)), dim3(256), 0, ctx->stream,
                           static_cast<const uint8_t *>(raw), static_cast<uint8_t *>(rows), l->resident_count,
                           l->blocks);
        err = hipGetLastError();
    }
    int rc = QXT_OK;
    if (err == hipSuccess && l->lanes) {
        rc = qxt_q4_0_pack_lanes(native, l->weight_row_bytes, l->weight, l->weight_bytes, l->resident_count, l->blocks,
                                 ctx->stream);
        if (rc != QXT_OK) rc = ctx->fail(rc, "weight re-layout: %s", qxt_last_error());
    }
    if (err == hipSuccess && approximate) {
        rc = qxt::q4_0_columns_w8(native, l->weight_row_bytes, l->resident_count, l->blocks,
                                  static_cast<uint32_t *>(l->weight), static_cast<size_t>(l->resident_count) * 4,
                                  l->column_scales, ctx->stream);
        if (rc != QXT_OK) rc = ctx->fail(rc, "weight re-quantisation: %s", qxt_last_error());
    }
    const hipError_t sync = hipStreamSynchronize(ctx->stream);
    (void)hipFree(raw);
    (void)hipFree(native);
    if (err == hipSuccess) err = sync;
    if (rc != QXT_OK) return rc;
    if (err != hipSuccess) return ctx->fail(QXT_IO_FAILED, "weight upload: %s", hipGetErrorString(err));
    return QXT_OK;
}

}  // namespace

// ------------------------------------------------------------------ context

extern "C" int qxt_llama_context_create(const qxt_llama_context_config *config, qxt_llama_context **result) {
    if (result == nullptr) return qxt::fail(QXT_INVALID_ARGUMENT, "llama context: null result");
    *result = nullptr;
    const int device = config ? config->device : 0;
    const uint32_t mask = config ? config->failure_mask : 0u;
    if (mask & ~kKnownFailures) return qxt::fail(QXT_INVALID_ARGUMENT, "llama context: unknown failure bits");
    if (mask & QXT_FAIL_DEVICE_OPEN) return qxt::fail(QXT_DEVICE_UNAVAILABLE, "injected device absence");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return qxt::fail(QXT_DEVICE_UNAVAILABLE, "no HIP device is available");
    if (device < 0 || device >= count)
        return qxt::fail(QXT_INVALID_ARGUMENT, "llama context: device %d out of range (%d devices)", device, count);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return qxt::fail(QXT_DEVICE_UNAVAILABLE, "device %d properties unavailable", device);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return qxt::fail(QXT_CAPABILITY_MISSING, "device %d is %s; this library is built for gfx950", device,
                         prop.gcnArchName);
    qxt_llama_context *ctx = new (std::nothrow) qxt_llama_context;
    if (ctx == nullptr) return qxt::fail(QXT_ALLOCATION_FAILED, "llama context: out of host memory");
    ctx->device = device;
    ctx->timeout_ns = config && config->timeout_ns ? config->timeout_ns : kDefaultTimeoutNs;
    ctx->failure_mask.store(mask);
    DeviceScope scope(device);
    hipError_t err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (err != hipSuccess) {
        delete ctx;
        return qxt::fail(QXT_DEVICE_UNAVAILABLE, "stream creation failed: %s", hipGetErrorString(err));
    }
    *result = ctx;
    return QXT_OK;
}

extern "C" void qxt_llama_context_destroy(qxt_llama_context *context) {
    if (context == nullptr) return;
    {
        DeviceScope scope(context->device);
        (void)hipStreamSynchronize(context->stream);
        (void)hipStreamDestroy(context->stream);
    }
    delete context;
}

extern "C" const char *qxt_llama_context_last_error(const qxt_llama_context *context) {
    return context != nullptr ? context->last_error : "no context";
}

extern "C" void qxt_llama_context_set_failure_mask(qxt_llama_context *context, uint32_t failure_mask) {
    if (context != nullptr) context->failure_mask.store(failure_mask & kKnownFailures);
}

extern "C" const char *qxt_llama_q4_0_source_hash(void) { return QXT_Q4_0_SOURCE_HASH; }

extern "C" const char *qxt_llama_status_string(int status) { return qxt_status_string(status); }

// ------------------------------------------------------------------ linear

extern "C" int qxt_llama_q4_0_linear_prepare(qxt_llama_context *context, const qxt_llama_q4_0_linear_desc *d,
                                             qxt_llama_q4_0_linear **result) {
    // Argument rules of qpu_llama_q4_0.c:208-223, plus the weight format.
    if (context == nullptr || d == nullptr || result == nullptr || d->weights == nullptr ||
        d->expected_source_hash == nullptr || d->rows == 0 || d->rows > kMaxRows || d->input_columns == 0 ||
        d->input_columns % qxt::QK != 0 || d->output_columns == 0 || d->resident_column_count == 0 ||
        d->resident_column_start % kOutputTile != 0 || d->resident_column_count % kOutputTile != 0 ||
        static_cast<uint32_t>(d->weight_mode) > QXT_LLAMA_Q4_0_WEIGHT_ROWCOL_W8A8 ||
        (d->weight_mode != QXT_LLAMA_Q4_0_WEIGHT_EXACT && d->rows <= 4) ||
        d->resident_column_start > d->output_columns ||
        d->resident_column_count > d->output_columns - d->resident_column_start ||
        static_cast<uint32_t>(d->weight_format) > QXT_LLAMA_Q4_0_FORMAT_REPACK_4X4 ||
        (d->weight_format == QXT_LLAMA_Q4_0_FORMAT_REPACK_4X4 && d->output_columns % 4 != 0)) {
        if (context) context->fail(QXT_INVALID_ARGUMENT, "q4_0 prepare: invalid descriptor");
        return QXT_INVALID_ARGUMENT;
    }
    *result = nullptr;
    const size_t blocks = d->input_columns / qxt::QK;
    size_t weight_row_bytes = 0, source_bytes = 0, resident_weight = 0, act_row = 0, act_bytes = 0, out_row = 0,
           out_bytes = 0;
    if (!mul_size(blocks, qxt::Q4_0_BYTES, &weight_row_bytes) ||
        !mul_size(d->output_columns, weight_row_bytes, &source_bytes) || d->weight_size < source_bytes ||
        !mul_size(d->resident_column_count, weight_row_bytes, &resident_weight) ||
        !mul_size(blocks, qxt::Q8_0_BYTES, &act_row) || !mul_size(d->rows, act_row, &act_bytes) ||
        !mul_size(d->resident_column_count, sizeof(float), &out_row) || !mul_size(d->rows, out_row, &out_bytes)) {
        return context->fail(QXT_INVALID_ARGUMENT, "q4_0 prepare: weight size or extents do not fit");
    }
    const bool approximate = d->weight_mode != QXT_LLAMA_Q4_0_WEIGHT_EXACT;
    if (approximate) {
        // The approximate modes run on the split-plane matrix-core kernel or
        // the W8A8 GEMM: 32-bit buffer offsets bound every operand.
        const uint64_t k = static_cast<uint64_t>(blocks) * qxt::QK;
        if (static_cast<uint64_t>(d->rows) * k >= (1ull << 31) ||
            static_cast<uint64_t>(d->resident_column_count) * k >= (1ull << 31) ||
            (d->weight_mode == QXT_LLAMA_Q4_0_WEIGHT_ROWCOL_W8A8 && k * 127 * 127 > 2147483647ull))
            return context->fail(QXT_CAPABILITY_MISSING,
                                 "q4_0 prepare: approximate weight modes need rows * K and columns * K below 2^31");
    } else if (qxt::q4_0_linear_capability(d->rows, static_cast<uint32_t>(blocks)) != QXT_OK) {
        // Every submission (any row count up to d->rows) must be runnable: reject
        // a K whose activation rows do not fit a workgroup's LDS now, not at submit.
        return context->fail(QXT_CAPABILITY_MISSING, "q4_0 prepare: %s", qxt_last_error());
    }
    if (context->injected(QXT_FAIL_SOURCE_HASH)) return context->fail(QXT_HASH_MISMATCH, "injected source hash mismatch");
    if (std::strcmp(d->expected_source_hash, QXT_Q4_0_SOURCE_HASH) != 0)
        return context->fail(QXT_HASH_MISMATCH, "expected source hash %.64s does not match this build (%s)",
                             d->expected_source_hash, QXT_Q4_0_SOURCE_HASH);
    if (context->injected(QXT_FAIL_ALLOCATION))
        return context->fail(QXT_ALLOCATION_FAILED, "injected allocation failure");

    qxt_llama_q4_0_linear *l = new (std::nothrow) qxt_llama_q4_0_linear;
    if (l == nullptr) return context->fail(QXT_ALLOCATION_FAILED, "q4_0 prepare: out of host memory");
    l->context = context;
    l->blocks = static_cast<uint32_t>(blocks);
    l->output_columns = d->output_columns;
    l->rows = d->rows;
    l->resident_start = d->resident_column_start;
    l->resident_count = d->resident_column_count;
    l->weight_row_bytes = weight_row_bytes;
    l->activation_row_bytes = act_row;
    l->output_row_bytes = out_row;
    l->mode = d->weight_mode;
    // Linears of fewer than 16 rows run on the v_dot4 decode kernel, which
    // streams the lane layout fastest; prefill-sized ones on the matrix cores
    // over native rows.
    l->lanes = !approximate && d->rows < 16 && blocks % 8 == 0;
    const size_t k = blocks * qxt::QK;
    const size_t approx_scales = d->weight_mode == QXT_LLAMA_Q4_0_WEIGHT_ROWCOL_W8A8 ? sizeof(float)
                                                                                     : blocks * sizeof(uint16_t);
    l->weight_bytes = approximate ? static_cast<size_t>(d->resident_column_count) * k
                      : l->lanes ? qxt_q4_0_lanes_bytes(d->resident_column_count, static_cast<uint32_t>(blocks))
                                 : resident_weight;
    // Device: weight, activation (+ its interleaved landing copy), output; pinned: activation, output.
    l->resident_bytes = l->weight_bytes + 2 * act_bytes + out_bytes + act_bytes + out_bytes;
    // Approximate modes: column scales, activation codes and their scales.
    if (approximate)
        l->resident_bytes += static_cast<size_t>(d->resident_column_count) * sizeof(float) +
                             static_cast<size_t>(d->rows) * (k + approx_scales);

    DeviceScope scope(context->device);
    hipError_t err = qxt::device_malloc(&l->weight, l->weight_bytes);
    if (err == hipSuccess && approximate) {
        err = qxt::device_malloc(&l->column_scales,
                        static_cast<size_t>(d->resident_column_count) * sizeof(float));
        if (err == hipSuccess) err = qxt::device_malloc(&l->activation_q, static_cast<size_t>(d->rows) * k);
        if (err == hipSuccess) err = qxt::device_malloc(&l->activation_scales, static_cast<size_t>(d->rows) * approx_scales);
    }
    if (err == hipSuccess) err = qxt::device_malloc(&l->activation, act_bytes);
    if (err == hipSuccess) err = qxt::device_malloc(&l->activation_packed, act_bytes);
    if (err == hipSuccess) err = qxt::device_malloc(&l->output, out_bytes);
    if (err == hipSuccess) err = qxt::pinned_host_malloc(&l->host_activation, act_bytes);
    if (err == hipSuccess)
        err = qxt::pinned_host_malloc(&l->host_output, out_bytes);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&l->done, hipEventDisableTiming);
    if (err != hipSuccess) {
        release_buffers(l);
        delete l;
        return context->fail(QXT_ALLOCATION_FAILED, "q4_0 prepare: %s", hipGetErrorString(err));
    }
    const int rc = upload_weights(l, d);
    if (rc != QXT_OK) {
        release_buffers(l);
        delete l;
        return rc;
    }
    *result = l;
    return QXT_OK;
}

extern "C" void qxt_llama_q4_0_linear_destroy(qxt_llama_q4_0_linear *linear) {
    if (linear == nullptr) return;
    {
        DeviceScope scope(linear->context->device);
        (void)hipStreamSynchronize(linear->context->stream);
        release_buffers(linear);
    }
    delete linear;
}

extern "C" size_t qxt_llama_q4_0_linear_resident_bytes(const qxt_llama_q4_0_linear *linear) {
    return linear != nullptr ? linear->resident_bytes : 0;
}

extern "C" int qxt_llama_q4_0_linear_submit(qxt_llama_q4_0_linear *l, const qxt_llama_q4_0_execution *e,
                                            qxt_llama_q4_0_submission **result) {
    const uint32_t rows = e != nullptr && e->rows != 0 ? e->rows : l != nullptr ? l->rows : 0;
    // Argument rules of qpu_llama_q4_0.c:464-496.
    if (l == nullptr || e == nullptr || result == nullptr || e->activation == nullptr || e->destination == nullptr ||
        e->column_count == 0 || rows == 0 || rows > l->rows || e->column_start % kOutputTile != 0 ||
        e->column_count % kOutputTile != 0 || e->column_start < l->resident_start ||
        e->column_count > l->resident_count ||
        e->column_start - l->resident_start > l->resident_count - e->column_count ||
        (e->activation_interleave != 0 && e->activation_interleave != 4 && e->activation_interleave != 8)) {
        if (l) l->context->fail(QXT_INVALID_ARGUMENT, "q4_0 submit: invalid execution");
        return QXT_INVALID_ARGUMENT;
    }
    qxt_llama_context *ctx = l->context;
    size_t act_bytes = 0, dst_elements = 0, dst_bytes = 0;
    if (!mul_size(rows, l->activation_row_bytes, &act_bytes) || !mul_size(rows, l->output_columns, &dst_elements) ||
        !mul_size(dst_elements, sizeof(float), &dst_bytes) ||
        !in_range(e->activation_size, e->activation_offset, act_bytes) ||
        !in_range(e->destination_size, e->destination_offset, dst_bytes)) {
        return ctx->fail(QXT_INVALID_ARGUMENT, "q4_0 submit: activation or destination range too small");
    }
    *result = nullptr;
    qxt_llama_q4_0_submission *s = new (std::nothrow) qxt_llama_q4_0_submission;
    if (s == nullptr) return ctx->fail(QXT_ALLOCATION_FAILED, "q4_0 submit: out of host memory");
    {
        std::lock_guard<std::mutex> guard(l->mutex);
        if (l->busy) {
            delete s;
            return ctx->fail(QXT_INTERNAL_ERROR, "q4_0 linear already has an in-flight submission");
        }
        l->busy = true;
    }
    {
        std::lock_guard<std::mutex> guard(ctx->mutex);
        int rc = QXT_OK;
        if (ctx->poisoned) rc = ctx->fail(QXT_IO_FAILED, "context is poisoned after a wait failure");
        else if (ctx->active) rc = ctx->fail(QXT_INTERNAL_ERROR, "context already has an active submission");
        else if (ctx->injected(QXT_FAIL_SUBMISSION)) rc = ctx->fail(QXT_SUBMISSION_FAILED, "injected submission failure");
        if (rc != QXT_OK) {
            std::lock_guard<std::mutex> lg(l->mutex);
            l->busy = false;
            delete s;
            return rc;
        }
        ctx->active = true;
    }

    DeviceScope scope(ctx->device);
    s->complete_start = now_ns();
    s->input_access_end = s->complete_start;  // pinned staging is always mapped
    std::memcpy(l->host_activation, static_cast<const uint8_t *>(e->activation) + e->activation_offset, act_bytes);
    s->input_pack_end = now_ns();
    const uint32_t local = e->column_start - l->resident_start;
    void *landing = e->activation_interleave ? l->activation_packed : l->activation;
    hipError_t err = hipMemcpyAsync(landing, l->host_activation, act_bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess && e->activation_interleave) {
        const size_t items = static_cast<size_t>(rows) * l->blocks;
        hipLaunchKernelGGL(deinterleave_q8_0x4_kernel, dim3(grid_for(items, 256)), dim3(256), 0, ctx->stream,
                           static_cast<const uint8_t *>(l->activation_packed), static_cast<uint8_t *>(l->activation),
                           rows, l->blocks, e->activation_interleave);
        err = hipGetLastError();
    }
    s->input_copy_end = now_ns();
    s->submit_start = s->input_copy_end;
    int rc = QXT_OK;
    if (err == hipSuccess && l->mode == QXT_LLAMA_Q4_0_WEIGHT_COLUMN_W8) {
        // Split planes of the Q8_0 rows, then the column-scale tiled linear
        // (qpu_llama_q4_0.c:572-607, 669-684).
        uint16_t *scales = static_cast<uint16_t *>(l->activation_scales);
        rc = qxt::q8_0_split_planes(l->activation, l->activation_row_bytes, rows, l->blocks, l->activation_q, scales,
                                    ctx->stream);
        if (rc == QXT_OK)
            rc = qxt::q4_0_tiled_column_w8(l->activation_q, scales, static_cast<const uint32_t *>(l->weight) + local,
                                           static_cast<size_t>(l->resident_count) * 4, l->column_scales + local,
                                           l->output + local, l->output_row_bytes, rows, l->blocks, e->column_count,
                                           ctx->stream);
        if (rc != QXT_OK) rc = ctx->fail(QXT_SUBMISSION_FAILED, "q4_0 column-w8 linear: %s", qxt_last_error());
    } else if (err == hipSuccess && l->mode == QXT_LLAMA_Q4_0_WEIGHT_ROWCOL_W8A8) {
        // Per-row int8 re-quantisation of the Q8_0 rows, then the W8A8 GEMM
        // with the row x column scale epilogue (qpu_llama_q4_0.c:526-571, 654-668).
        const uint32_t k = l->blocks * qxt::QK;
        float *row_scales = static_cast<float *>(l->activation_scales);
        rc = qxt::q8_0_rows_w8(l->activation, l->activation_row_bytes, rows, l->blocks, l->activation_q, row_scales,
                               ctx->stream);
        if (rc == QXT_OK)
            rc = qxt_w8a8_gemm_dequantize(l->activation_q, k, static_cast<const uint32_t *>(l->weight) + local,
                                          static_cast<size_t>(l->resident_count) * 4, row_scales,
                                          l->column_scales + local, nullptr, l->output + local, l->output_row_bytes,
                                          rows, e->column_count, k, QXT_W8A8_WEIGHT_K4N, ctx->stream);
        if (rc != QXT_OK) rc = ctx->fail(QXT_SUBMISSION_FAILED, "q4_0 rowcol-w8a8 linear: %s", qxt_last_error());
    } else if (err == hipSuccess) {
        rc = l->lanes ? qxt_ggml_q4_0_q8_0_linear_lanes(l->activation, l->activation_row_bytes, l->weight,
                                                        l->resident_count, l->output, l->output_row_bytes, rows,
                                                        l->blocks, local, local, e->column_count, ctx->stream)
                      : qxt_ggml_q4_0_q8_0_linear(l->activation, l->activation_row_bytes, l->weight,
                                                  l->weight_row_bytes, l->output, l->output_row_bytes, rows, l->blocks,
                                                  local, local, e->column_count, ctx->stream);
        if (rc != QXT_OK) rc = ctx->fail(QXT_SUBMISSION_FAILED, "q4_0 linear: %s", qxt_last_error());
    }
    if (rc == QXT_OK && err == hipSuccess) {
        err = hipMemcpy2DAsync(l->host_output + local, l->output_row_bytes, l->output + local, l->output_row_bytes,
                               static_cast<size_t>(e->column_count) * sizeof(float), rows, hipMemcpyDeviceToHost,
                               ctx->stream);
    }
    if (rc == QXT_OK && err == hipSuccess) err = hipEventRecord(l->done, ctx->stream);
    if (rc == QXT_OK && err != hipSuccess) rc = ctx->fail(QXT_SUBMISSION_FAILED, "q4_0 submit: %s", hipGetErrorString(err));
    if (rc != QXT_OK) {
        // Work already enqueued only touches the linear's own buffers; drain it
        // so the next submission starts from an idle stream.
        (void)hipStreamSynchronize(ctx->stream);
        end_submission(l, false);
        delete s;
        return rc;
    }
    s->submit_end = now_ns();
    s->linear = l;
    s->destination = static_cast<uint8_t *>(e->destination) + e->destination_offset;
    s->rows = rows;
    s->column_start = e->column_start;
    s->column_count = e->column_count;
    s->local_start = local;
    s->active = true;
    *result = s;
    return QXT_OK;
}

extern "C" int qxt_llama_q4_0_submission_wait(qxt_llama_q4_0_submission *s, qxt_llama_q4_0_timing *timing) {
    if (s == nullptr || !s->active || s->linear == nullptr) return QXT_INVALID_ARGUMENT;
    qxt_llama_q4_0_linear *l = s->linear;
    qxt_llama_context *ctx = l->context;
    DeviceScope scope(ctx->device);
    const uint64_t wait_start = now_ns();
    int rc = QXT_OK;
    for (uint32_t spins = 0;; ++spins) {
        const hipError_t q = hipEventQuery(l->done);
        if (q == hipSuccess) break;
        if (q != hipErrorNotReady) {
            rc = ctx->fail(QXT_IO_FAILED, "q4_0 wait: %s", hipGetErrorString(q));
            break;
        }
        if (now_ns() - wait_start > ctx->timeout_ns) {
            rc = ctx->fail(QXT_TIMEOUT, "q4_0 wait: no completion within %llu ns",
                           static_cast<unsigned long long>(ctx->timeout_ns));
            break;
        }
        // Spin briefly (decode latency), then back off.
        if (spins < 4096) std::this_thread::yield();
        else std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
    const uint64_t wait_end = now_ns();
    if (rc == QXT_OK && ctx->injected(QXT_FAIL_WAIT)) rc = ctx->fail(QXT_TIMEOUT, "injected wait timeout");
    uint64_t copy_end = wait_end;
    if (rc == QXT_OK) {
        const size_t dst_row = static_cast<size_t>(l->output_columns) * sizeof(float);
        const size_t width = static_cast<size_t>(s->column_count) * sizeof(float);
        for (uint32_t row = 0; row < s->rows; ++row) {
            std::memcpy(s->destination + row * dst_row + static_cast<size_t>(s->column_start) * sizeof(float),
                        l->host_output + static_cast<size_t>(row) * l->resident_count + s->local_start, width);
        }
        copy_end = now_ns();
    }
    if (timing != nullptr) {
        timing->input_access_ns = s->input_access_end - s->complete_start;
        timing->input_pack_ns = s->input_pack_end - s->input_access_end;
        timing->input_sync_ns = s->input_copy_end - s->input_pack_end;
        timing->input_copy_ns = s->input_copy_end - s->complete_start;
        timing->submit_ns = s->submit_end - s->submit_start;
        timing->wait_ns = wait_end - wait_start;
        timing->submit_wait_ns = wait_end - s->submit_start;
        timing->output_sync_ns = 0;  // the device-to-host copy is part of the waited stream work
        timing->output_copy_ns = copy_end - wait_end;
        timing->complete_ns = copy_end - s->complete_start;
    }
    s->active = false;
    // A failed or timed-out wait leaves the device state unknown: poison the
    // context as the reference runtime does (qpu_llama_runtime.c:705-719).
    end_submission(l, rc != QXT_OK);
    return rc;
}

extern "C" void qxt_llama_q4_0_submission_destroy(qxt_llama_q4_0_submission *submission) {
    if (submission == nullptr) return;
    if (submission->active) (void)qxt_llama_q4_0_submission_wait(submission, nullptr);
    delete submission;
}

extern "C" int qxt_llama_q4_0_linear_execute(qxt_llama_q4_0_linear *linear, const qxt_llama_q4_0_execution *execution,
                                             qxt_llama_q4_0_timing *timing) {
    qxt_llama_q4_0_submission *submission = nullptr;
    int rc = qxt_llama_q4_0_linear_submit(linear, execution, &submission);
    if (rc == QXT_OK) rc = qxt_llama_q4_0_submission_wait(submission, timing);
    qxt_llama_q4_0_submission_destroy(submission);
    return rc;
}

// No CPU compute path: the reference's fallback recomputes the submission on
// the host (qpu_llama_q4_0.c:834-946); here the caller's own CPU kernel does,
// so the destination is left exactly as it was.
extern "C" int qxt_llama_q4_0_submission_cpu_fallback(qxt_llama_q4_0_submission *submission) {
    if (submission == nullptr || submission->linear == nullptr) return QXT_INVALID_ARGUMENT;
    return submission->linear->context->fail(QXT_CAPABILITY_MISSING,
                                             "q4_0 cpu fallback: this library has no CPU compute path");
}

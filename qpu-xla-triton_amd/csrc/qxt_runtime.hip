// Status strings, per-thread last error, failure injection and device queries.
//
// The status set and failure points follow the reference's native runtime
// contract (integrations/llama_cpp/include/qpu_llama_runtime.h:16-36); the
// mechanism here is a process-wide atomic mask plus a thread-local message,
// since the library itself is stateless apart from that.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "qxt_common.h"

namespace qxt {
namespace {

thread_local char g_last_error[512] = "";
std::atomic<uint32_t> g_failure_mask{0};
std::atomic<uint64_t> g_allocations{0};

struct LaunchTiming {
    bool enabled = false;
    std::vector<hipEvent_t> pool;  // created events, reused across sessions
    size_t used = 0;               // events handed out in the current session
    struct Record {
        const char *name;
        hipEvent_t start, stop;
    };
    std::vector<Record> records;
};
thread_local LaunchTiming g_timing;

}  // namespace

int fail(int status, const char *fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
    va_end(args);
    return status;
}

int injected(uint32_t point) {
    if ((g_failure_mask.load(std::memory_order_relaxed) & point) == 0) return QXT_OK;
    switch (point) {
        case QXT_FAIL_ALLOCATION: return fail(QXT_ALLOCATION_FAILED, "injected allocation failure");
        case QXT_FAIL_SUBMISSION: return fail(QXT_SUBMISSION_FAILED, "injected submission failure");
        case QXT_FAIL_WAIT: return fail(QXT_TIMEOUT, "injected wait failure");
        case QXT_FAIL_DEVICE_OPEN: return fail(QXT_DEVICE_UNAVAILABLE, "injected device-open failure");
        default: return fail(QXT_INTERNAL_ERROR, "injected failure");
    }
}

int launch_status(const char *kernel_name) {
    hipError_t err = hipGetLastError();
    if (err == hipSuccess) return QXT_OK;
    return fail(QXT_SUBMISSION_FAILED, "%s launch failed: %s", kernel_name, hipGetErrorString(err));
}

bool timing_enabled() { return g_timing.enabled; }

void timing_events(hipEvent_t *start, hipEvent_t *stop) {
    while (g_timing.pool.size() < g_timing.used + 2) {
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) break;
        g_timing.pool.push_back(e);
    }
    if (g_timing.pool.size() < g_timing.used + 2) {
        *start = *stop = nullptr;
        return;
    }
    *start = g_timing.pool[g_timing.used++];
    *stop = g_timing.pool[g_timing.used++];
}

void timing_record(const char *kernel_name, hipEvent_t start, hipEvent_t stop) {
    if (start != nullptr && stop != nullptr) g_timing.records.push_back({kernel_name, start, stop});
}

hipError_t counted_malloc(void **ptr, size_t bytes) {
    const hipError_t err = hipMalloc(ptr, bytes);
    if (err == hipSuccess) g_allocations.fetch_add(1, std::memory_order_relaxed);
    return err;
}

hipError_t counted_host_malloc(void **ptr, size_t bytes) {
    const hipError_t err = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
    if (err == hipSuccess) g_allocations.fetch_add(1, std::memory_order_relaxed);
    return err;
}

int compute_units() {
    static std::mutex lock;
    static std::vector<int> cache;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return 256;
    std::lock_guard<std::mutex> guard(lock);
    if (static_cast<size_t>(device) >= cache.size()) cache.resize(device + 1, 0);
    if (cache[device] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cache[device] = cus;
    }
    return cache[device];
}

namespace {

// The HBM read probe: every thread of a grid of kProbeWorkgroups x 256 reads
// 16-byte chunks grid-stride with non-temporal loads (one load in flight per
// thread measured fastest on MI355X: 6.89 TB/s over 547 MB, against 5.6-6.8
// TB/s with 2 to 8 chunks per thread or other grids) and xors them; each
// workgroup stores the xor of what it read.
constexpr int kProbeWorkgroups = 2048;
typedef unsigned int probe_v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void hbm_read_probe_kernel(const probe_v4u *__restrict__ src, size_t chunks,
                                                             uint32_t *__restrict__ partials) {
    __shared__ uint32_t waves[4];
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    uint32_t acc = 0;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < chunks; i += stride) {
        const probe_v4u v = __builtin_nontemporal_load(src + i);
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) partials[blockIdx.x] = waves[0] ^ waves[1] ^ waves[2] ^ waves[3];
}

}  // namespace
}  // namespace qxt

extern "C" {

int qxt_abi_version(void) { return QXT_ABI_VERSION; }

int qxt_hbm_read_probe(const void *src, size_t bytes, uint32_t *partials, void *stream) {
    if (src == nullptr || partials == nullptr || !qxt::aligned(src, 16) || !qxt::aligned(partials, 4))
        return qxt::fail(QXT_INVALID_ARGUMENT, "hbm read probe: null or misaligned pointer");
    if (bytes == 0 || bytes % 16)
        return qxt::fail(QXT_INVALID_ARGUMENT, "hbm read probe: bytes must be a positive multiple of 16");
    return qxt::launch("hbm_read_probe_kernel", qxt::hbm_read_probe_kernel, dim3(qxt::kProbeWorkgroups), dim3(256), 0,
                       qxt::as_stream(stream), static_cast<const qxt::probe_v4u *>(src), bytes / 16, partials);
}

const char *qxt_status_string(int status) {
    switch (status) {
        case QXT_OK: return "ok";
        case QXT_INVALID_ARGUMENT: return "invalid argument";
        case QXT_DEVICE_UNAVAILABLE: return "device unavailable";
        case QXT_CAPABILITY_MISSING: return "capability missing";
        case QXT_ALLOCATION_FAILED: return "allocation failed";
        case QXT_IO_FAILED: return "I/O failed";
        case QXT_SUBMISSION_FAILED: return "submission failed";
        case QXT_TIMEOUT: return "timeout";
        case QXT_HASH_MISMATCH: return "hash mismatch";
        case QXT_INTERNAL_ERROR: return "internal error";
        default: return "unknown status";
    }
}

const char *qxt_last_error(void) { return qxt::g_last_error; }

void qxt_set_failure_mask(uint32_t mask) { qxt::g_failure_mask.store(mask, std::memory_order_relaxed); }

uint32_t qxt_get_failure_mask(void) { return qxt::g_failure_mask.load(std::memory_order_relaxed); }

uint64_t qxt_allocation_count(void) { return qxt::g_allocations.load(std::memory_order_relaxed); }

int qxt_device_query(qxt_device_info *out) {
    if (out == nullptr) return qxt::fail(QXT_INVALID_ARGUMENT, "qxt_device_query: null output");
    int rc = qxt::injected(QXT_FAIL_DEVICE_OPEN);
    if (rc != QXT_OK) return rc;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess)
        return qxt::fail(QXT_DEVICE_UNAVAILABLE, "no HIP device is available");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return qxt::fail(QXT_DEVICE_UNAVAILABLE, "hipGetDeviceProperties failed");
    std::memset(out, 0, sizeof(*out));
    std::strncpy(out->arch, prop.gcnArchName, sizeof(out->arch) - 1);
    out->compute_units = prop.multiProcessorCount;
    out->clock_khz = prop.clockRate;
    out->memory_clock_khz = prop.memoryClockRate;
    out->memory_bus_width = prop.memoryBusWidth;
    out->total_memory = static_cast<int64_t>(prop.totalGlobalMem);
    out->l2_bytes = prop.l2CacheSize;
    out->lds_bytes_per_cu = static_cast<int32_t>(prop.maxSharedMemoryPerMultiProcessor);
    return QXT_OK;
}

int qxt_timing_begin(void) {
    if (qxt::g_timing.enabled) return qxt::fail(QXT_INVALID_ARGUMENT, "launch timing is already active");
    qxt::g_timing.enabled = true;
    qxt::g_timing.used = 0;
    qxt::g_timing.records.clear();
    return QXT_OK;
}

int qxt_timing_end(qxt_launch_record *records, uint32_t capacity, uint32_t *count) {
    if (!qxt::g_timing.enabled) return qxt::fail(QXT_INVALID_ARGUMENT, "launch timing is not active");
    qxt::g_timing.enabled = false;
    int rc = QXT_OK;
    uint32_t n = 0;
    for (const auto &rec : qxt::g_timing.records) {
        if (hipEventSynchronize(rec.stop) != hipSuccess) {
            rc = qxt::fail(QXT_INTERNAL_ERROR, "hipEventSynchronize failed while collecting launch times");
            break;
        }
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, rec.start, rec.stop) != hipSuccess) {
            rc = qxt::fail(QXT_INTERNAL_ERROR, "hipEventElapsedTime failed for %s", rec.name);
            break;
        }
        if (records != nullptr && n < capacity) {
            std::memset(&records[n], 0, sizeof(records[n]));
            std::strncpy(records[n].kernel, rec.name, sizeof(records[n].kernel) - 1);
            records[n].ms = ms;
        }
        ++n;
    }
    if (count != nullptr) *count = n;
    qxt::g_timing.records.clear();
    qxt::g_timing.used = 0;
    return rc;
}

int qxt_stream_wait(void *stream) {
    int rc = qxt::injected(QXT_FAIL_WAIT);
    if (rc != QXT_OK) return rc;
    hipError_t err = hipStreamSynchronize(qxt::as_stream(stream));
    if (err != hipSuccess)
        return qxt::fail(QXT_INTERNAL_ERROR, "hipStreamSynchronize failed: %s", hipGetErrorString(err));
    return QXT_OK;
}

}  // extern "C"

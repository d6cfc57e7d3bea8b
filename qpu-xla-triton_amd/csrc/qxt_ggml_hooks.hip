// ggml CPU_REPACK M=1 Q4_0 hooks (include/qxt_ggml_hooks.h) over the prepared
// linear of the llama.cpp bridge.  Host code only: the device work is the
// bridge's (pinned copy in, decode kernel over lane-layout weights, copy out).
//
// Registry semantics follow the reference's hook implementation
// (integrations/llama_cpp/backend/ggml-qpu-up-inline.cpp:64-87,231-240,261-436):
// opt-in by environment, one context created at most once, one linear per
// tensor name, a mutex around every call, and "last executed name" plus
// "CPU columns" state for the caller's follow-up query.

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "qxt_ggml_hooks.h"
#include "qxt_llama_q4_0.h"

namespace {

struct HookRegistry {
    std::mutex mutex;
    qxt_llama_context *context = nullptr;
    bool creation_attempted = false;
    std::unordered_map<std::string, qxt_llama_q4_0_linear *> linears;
    std::unordered_map<std::string, uint64_t> shapes;  // name -> (input_columns << 32) | output_columns
    std::string last_name;
    std::atomic<uint64_t> cpu_columns{0};
    std::atomic<uint64_t> dispatches{0};
};

// Never destroyed: HIP objects are released only by ggml_qpu_m1_release, not
// by a static destructor running after the HIP runtime may have shut down.
HookRegistry &registry() {
    static HookRegistry *instance = new HookRegistry;
    return *instance;
}

bool env_flag(const char *name) {
    const char *value = std::getenv(name);
    return value != nullptr && (!std::strcmp(value, "1") || !std::strcmp(value, "true") || !std::strcmp(value, "on"));
}

// GGML_QPU_M1_TENSORS: comma-separated substrings; a tensor is selected when
// its name contains one of them.
bool tensor_selected(const char *name) {
    const char *list = std::getenv("GGML_QPU_M1_TENSORS");
    if (name == nullptr || list == nullptr || *list == '\0') return false;
    const std::string tensor(name);
    for (const char *p = list; *p != '\0';) {
        const char *comma = std::strchr(p, ',');
        const size_t length = comma ? static_cast<size_t>(comma - p) : std::strlen(p);
        if (length > 0 && tensor.find(std::string(p, length)) != std::string::npos) return true;
        if (comma == nullptr) break;
        p = comma + 1;
    }
    return false;
}

bool telemetry() {
    const char *value = std::getenv("GGML_QPU_TELEMETRY");
    return value == nullptr || std::strcmp(value, "0") != 0;
}

int ensure_context(HookRegistry &r) {
    if (r.context != nullptr) return QXT_OK;
    if (r.creation_attempted) return QXT_INTERNAL_ERROR;
    r.creation_attempted = true;
    return qxt_llama_context_create(nullptr, &r.context);
}

const char *context_error(const HookRegistry &r) {
    return r.context != nullptr ? qxt_llama_context_last_error(r.context) : "no context";
}

}  // namespace

extern "C" int ggml_qpu_m1_register_q4_0(const char *name, const void *weights, size_t weight_size,
                                         uint64_t input_columns, uint64_t output_columns) {
    if (!env_flag("GGML_QPU_M1_INLINE") || !tensor_selected(name) || weights == nullptr || input_columns == 0 ||
        input_columns > UINT32_MAX || input_columns % 32 != 0 || output_columns == 0 ||
        output_columns > UINT32_MAX || output_columns % 16 != 0)
        return 0;
    HookRegistry &r = registry();
    std::lock_guard<std::mutex> guard(r.mutex);
    if (r.linears.count(name)) return 1;
    int status = ensure_context(r);
    qxt_llama_q4_0_linear *linear = nullptr;
    if (status == QXT_OK) {
        qxt_llama_q4_0_linear_desc desc{};
        desc.weights = weights;
        desc.weight_size = weight_size;
        desc.input_columns = static_cast<uint32_t>(input_columns);
        desc.output_columns = static_cast<uint32_t>(output_columns);
        desc.rows = 1;
        desc.resident_column_start = 0;
        desc.resident_column_count = static_cast<uint32_t>(output_columns);
        desc.weight_mode = QXT_LLAMA_Q4_0_WEIGHT_EXACT;
        desc.expected_source_hash = qxt_llama_q4_0_source_hash();
        desc.weight_format = QXT_LLAMA_Q4_0_FORMAT_NATIVE;
        status = qxt_llama_q4_0_linear_prepare(r.context, &desc, &linear);
    }
    if (status != QXT_OK) {
        std::fprintf(stderr, "gfx950: could not prepare M=1 tensor %s: %s (%s)\n", name,
                     qxt_llama_status_string(status), context_error(r));
        return 0;
    }
    if (telemetry())
        std::fprintf(stderr,
                     "qpu_llama_weight_json:{\"schema_version\":1,\"operation\":\"mul_mat_q4_0_q8_0_m1\","
                     "\"backend\":\"gfx950\",\"tensor\":\"%s\",\"k\":%llu,\"n\":%llu,\"resident_bytes\":%zu}\n",
                     name, static_cast<unsigned long long>(input_columns),
                     static_cast<unsigned long long>(output_columns), qxt_llama_q4_0_linear_resident_bytes(linear));
    r.linears.emplace(name, linear);
    r.shapes.emplace(name, (input_columns << 32) | output_columns);
    return 1;
}

extern "C" int ggml_qpu_m1_weight_registered(const char *name) {
    if (name == nullptr) return 0;
    HookRegistry &r = registry();
    std::lock_guard<std::mutex> guard(r.mutex);
    return r.linears.count(name) ? 1 : 0;
}

extern "C" int ggml_qpu_m1_execute(const char *name, const void *activation_q8_0, size_t activation_size,
                                   float *destination, uint64_t rows, uint64_t input_columns,
                                   uint64_t output_columns, uint64_t activation_interleave) {
    if (name == nullptr || activation_q8_0 == nullptr || destination == nullptr || rows != 1 ||
        input_columns > UINT32_MAX || output_columns > UINT32_MAX || activation_interleave > UINT32_MAX)
        return 0;
    HookRegistry &r = registry();
    std::lock_guard<std::mutex> guard(r.mutex);
    const auto found = r.linears.find(name);
    if (found == r.linears.end()) return 0;
    if (r.shapes[name] != ((input_columns << 32) | output_columns)) return 0;
    // Until the product is known to be on the destination, the CPU owns every column.
    r.last_name = name;
    r.cpu_columns.store(output_columns, std::memory_order_release);
    if (!env_flag("GGML_QPU_M1_INLINE")) return 0;

    qxt_llama_q4_0_execution execution{};
    execution.activation = activation_q8_0;
    execution.activation_size = activation_size;
    execution.destination = destination;
    execution.destination_size = static_cast<size_t>(output_columns) * sizeof(float);
    execution.column_start = 0;
    execution.column_count = static_cast<uint32_t>(output_columns);
    execution.rows = 1;
    execution.activation_interleave = static_cast<uint32_t>(activation_interleave);
    qxt_llama_q4_0_submission *submission = nullptr;
    qxt_llama_q4_0_timing timing{};
    int status = qxt_llama_q4_0_linear_submit(found->second, &execution, &submission);
    if (status == QXT_OK) status = qxt_llama_q4_0_submission_wait(submission, &timing);
    if (status != QXT_OK && submission != nullptr) status = qxt_llama_q4_0_submission_cpu_fallback(submission);
    qxt_llama_q4_0_submission_destroy(submission);
    if (status != QXT_OK) {
        std::fprintf(stderr, "gfx950: M=1 product failed for %s: %s (%s)\n", name, qxt_llama_status_string(status),
                     context_error(r));
        return 0;
    }
    r.cpu_columns.store(0, std::memory_order_release);
    r.dispatches.fetch_add(1, std::memory_order_relaxed);
    if (telemetry())
        std::fprintf(stderr,
                     "qpu_llama_candidate_json:{\"schema_version\":1,\"backend\":\"gfx950\","
                     "\"operation\":\"mul_mat_q4_0_q8_0\",\"program\":\"q4_0_linear_kernel\","
                     "\"source_hash\":\"%s\",\"placement\":\"hybrid\","
                     "\"integration_boundary\":\"cpu-repack-inline-m1\",\"tensor\":\"%s\",\"m\":1,"
                     "\"k\":%llu,\"n\":%llu,\"dispatch_count\":1,\"input_copy_ns\":%llu,\"submit_ns\":%llu,"
                     "\"wait_ns\":%llu,\"output_copy_ns\":%llu,\"complete_ns\":%llu,\"fallback\":false}\n",
                     qxt_llama_q4_0_source_hash(), name, static_cast<unsigned long long>(input_columns),
                     static_cast<unsigned long long>(output_columns),
                     static_cast<unsigned long long>(timing.input_copy_ns),
                     static_cast<unsigned long long>(timing.submit_ns), static_cast<unsigned long long>(timing.wait_ns),
                     static_cast<unsigned long long>(timing.output_copy_ns),
                     static_cast<unsigned long long>(timing.complete_ns));
    return 1;
}

extern "C" uint64_t ggml_qpu_m1_cpu_columns_for(const char *name) {
    if (name == nullptr) return 0;
    HookRegistry &r = registry();
    std::lock_guard<std::mutex> guard(r.mutex);
    return r.last_name == name ? r.cpu_columns.load(std::memory_order_acquire) : 0;
}

extern "C" uint64_t ggml_qpu_m1_dispatch_count(void) { return registry().dispatches.load(); }

extern "C" void ggml_qpu_m1_release(void) {
    HookRegistry &r = registry();
    std::lock_guard<std::mutex> guard(r.mutex);
    for (auto &entry : r.linears) qxt_llama_q4_0_linear_destroy(entry.second);
    r.linears.clear();
    r.shapes.clear();
    r.last_name.clear();
    r.cpu_columns.store(0);
    if (r.context != nullptr) qxt_llama_context_destroy(r.context);
    r.context = nullptr;
    r.creation_attempted = false;
}

// The hyp_* C ABI (include/hyperion_hip.h). Conventions mirror the reference ABI:
// status codes and thread-local last error (native/hyperion_mlx/src/abi_error.cc:7-19),
// the no-throw abi_call wrapper (runtime.mm:79-97), magic-tagged handles with
// idempotent free (model.cc:66-68,170-207).
#include <array>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <memory>
#include <new>
#include <string>

#include "hyperion_hip.h"
#include "kernels.h"
#include "decoder.h"
#include "qlinear.h"
#include "sampling.h"
#include "step_program_host.h"

using hyperion::hip::Epilogue;
using hyperion::hip::NativeError;
using hyperion::model::DeviceBuffer;
using hyperion::model::ModelWeights;
using hyperion::model::QuantizedLinear;

namespace {

constexpr std::uint32_t kQWeightMagic = 0x48505157U;   // "HPQW"
constexpr std::uint32_t kQModelMagic = 0x4850514DU;    // "HPQM"
constexpr std::uint32_t kStreamMagic = 0x48505354U;    // "HPST"
constexpr std::uint32_t kEventMagic = 0x48504556U;     // "HPEV"
constexpr std::uint32_t kGraphMagic = 0x48504752U;     // "HPGR"
constexpr std::uint32_t kStepProgramMagic = 0x48505350U;   // "HPSP"
constexpr std::uint32_t kKvCacheMagic = 0x48504B56U;       // "HPKV"

constexpr std::size_t kLastErrorCapacity = 1024;
thread_local std::array<char, kLastErrorCapacity> g_last_error{};

HypStatus fail(HypStatus status, const char* message) noexcept {
    std::snprintf(g_last_error.data(), g_last_error.size(), "%s",
                  message != nullptr ? message : "unknown native error");
    return status;
}

HypStatus ok() noexcept {
    g_last_error[0] = '\0';
    return HYP_STATUS_OK;
}

template <typename Function>
HypStatus abi_call(const char* operation, Function&& function) noexcept {
    try {
        function();
        return ok();
    } catch (const NativeError& error) {
        return fail(error.status(), error.what());
    } catch (const std::bad_alloc&) {
        return fail(HYP_STATUS_INTERNAL, "native host allocation failed");
    } catch (const std::filesystem::filesystem_error& error) {
        return fail(HYP_STATUS_IO, error.what());
    } catch (const std::exception& error) {
        return fail(HYP_STATUS_INTERNAL, error.what());
    } catch (...) {
        std::snprintf(g_last_error.data(), g_last_error.size(), "%s failed with a non-standard exception",
                      operation != nullptr ? operation : "native operation");
        return HYP_STATUS_INTERNAL;
    }
}

#define REQUIRE_ARG(cond, msg) HYP_REQUIRE((cond), HYP_STATUS_INVALID_ARGUMENT, (msg))

// Throws UNSUPPORTED when no HIP device is usable, before any other HIP call.
void require_device() {
    int count = 0;
    const hipError_t err = hipGetDeviceCount(&count);
    if (err != hipSuccess || count <= 0) {
        throw NativeError(HYP_STATUS_UNSUPPORTED, "no HIP device is available");
    }
}

// fp32 -> nearest-even bf16 value, on the host (constants handed to kernels).
float round_to_bf16(float f) {
    std::uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return f;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

}  // namespace

struct HypQWeightOpaque {
    std::uint32_t magic = 0;
    bool owned_by_model = false;
    QuantizedLinear lin;
};

struct HypQModelOpaque {
    std::uint32_t magic = 0;
    ModelWeights weights;
    std::unique_ptr<HypQWeightOpaque> embed;
    // Per layer, per HypProj; null for a global layer's V.
    std::vector<std::array<std::unique_ptr<HypQWeightOpaque>, 7>> layers;
};

struct HypStreamOpaque {
    std::uint32_t magic = 0;
    hipStream_t stream = nullptr;
    // Device workspace of the calls that need one (greedy sampling's slice states, then the
    // temperature draw's bins and parameters from stoch_workspace_offset); work on one
    // stream is ordered, so its calls never share it concurrently.
    void* workspace = nullptr;
    size_t workspace_bytes = 0;   // the greedy part
    size_t stoch_workspace_offset = 0;
    [[nodiscard]] void* stoch_workspace() const noexcept {
        return static_cast<uint8_t*>(workspace) + stoch_workspace_offset;
    }
};

struct HypEventOpaque {
    std::uint32_t magic = 0;
    hipEvent_t event = nullptr;
};

struct HypStepProgramOpaque {
    std::uint32_t magic = 0;
    std::unique_ptr<hyperion::model::StepProgram> program;
};

struct HypKvCacheOpaque {
    std::uint32_t magic = 0;
    uint32_t capacity = 0;
    uint32_t num_kv_heads = 0;
    uint32_t head_dim = 0;
    DeviceBuffer k;
    DeviceBuffer v;
    DeviceBuffer workspace;   // decode attention's split partials
};

struct HypGraphOpaque {
    std::uint32_t magic = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

const QuantizedLinear& qweight_ref(HypQWeight w, const char* what) {
    REQUIRE_ARG(w != nullptr, std::string(what) + " handle is null");
    REQUIRE_ARG(w->magic == kQWeightMagic,
                std::string(what) + " handle magic mismatch (wrong type, freed, or corrupted)");
    return w->lin;
}

hipStream_t stream_of(HypStream s) {
    REQUIRE_ARG(s != nullptr, "stream handle is null (an explicit stream is required)");
    REQUIRE_ARG(s->magic == kStreamMagic, "stream handle magic mismatch (wrong type, freed, or corrupted)");
    return s->stream;
}

// Calls that allocate device memory (stream-ordered temporaries of the m > 4 paths) or
// clear it with hipMemsetAsync must not be recorded into a graph: a captured
// allocation or memset node would replay against memory the call no longer owns.
// Such calls check the stream first and refuse, before anything is enqueued.
void require_not_capturing(hipStream_t s, const char* what) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    HYP_HIP_CHECK(hipStreamIsCapturing(s, &st));
    REQUIRE_ARG(st == hipStreamCaptureStatusNone,
                std::string(what) + " may allocate or clear device memory and cannot be recorded into a graph "
                                    "(the stream is capturing)");
}

void validate_quant(std::uint32_t n, std::uint32_t k, std::uint32_t group_size, std::uint32_t bits) {
    if (group_size != 64 || bits != 4) {
        throw NativeError(HYP_STATUS_UNSUPPORTED, "only affine group_size=64 bits=4 is supported (got group_size=" +
                                                      std::to_string(group_size) + " bits=" + std::to_string(bits) + ")");
    }
    REQUIRE_ARG(n > 0 && k > 0, "n and k must be positive");
    REQUIRE_ARG(k % 64 == 0, "k must be a multiple of 64");
}

template <typename Handle>
HypStatus free_handle(Handle** handle, std::uint32_t magic) noexcept {
    if (handle == nullptr) return fail(HYP_STATUS_INVALID_ARGUMENT, "free requires a non-null handle pointer");
    Handle* ptr = *handle;
    if (ptr == nullptr) return ok();
    if (ptr->magic != magic) return fail(HYP_STATUS_INVALID_ARGUMENT, "handle magic mismatch (wrong type, freed, or corrupted)");
    ptr->magic = 0;
    delete ptr;
    *handle = nullptr;
    return ok();
}

}  // namespace

extern "C" {

HypStatus hyp_last_error(char* buffer, size_t buffer_len) {
    if (buffer == nullptr || buffer_len == 0) {
        return HYP_STATUS_INVALID_ARGUMENT;   // leaves the stored message intact
    }
    std::snprintf(buffer, buffer_len, "%s", g_last_error.data());
    return HYP_STATUS_OK;
}

HypStatus hyp_runtime_info(HypRuntimeInfo* out) {
    return abi_call("hyp_runtime_info", [&] {
        REQUIRE_ARG(out != nullptr, "runtime info requires a non-null out pointer");
        std::memset(out, 0, sizeof(*out));
        out->abi_version = HYP_HIP_ABI_VERSION;
        require_device();
        int count = 0;
        HYP_HIP_CHECK(hipGetDeviceCount(&count));
        int dev = 0;
        HYP_HIP_CHECK(hipGetDevice(&dev));
        hipDeviceProp_t prop{};
        HYP_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
        out->device_count = count;
        out->device = dev;
        out->compute_units = static_cast<std::uint32_t>(prop.multiProcessorCount);
        out->hbm_bytes = static_cast<std::uint64_t>(prop.totalGlobalMem);
        out->clock_khz = static_cast<std::uint32_t>(prop.clockRate);
        out->l2_bytes = static_cast<std::uint32_t>(prop.l2CacheSize);
        std::snprintf(out->arch_name, sizeof(out->arch_name), "%s", prop.gcnArchName);
        std::snprintf(out->device_name, sizeof(out->device_name), "%s", prop.name);
    });
}

HypStatus hyp_device_alloc(size_t bytes, void** out_ptr) {
    return abi_call("hyp_device_alloc", [&] {
        REQUIRE_ARG(out_ptr != nullptr, "alloc requires a non-null out pointer");
        *out_ptr = nullptr;
        REQUIRE_ARG(bytes > 0, "alloc of zero bytes");
        require_device();
        void* p = nullptr;
        const hipError_t err = hipMalloc(&p, bytes);
        if (err != hipSuccess) {
            throw NativeError(HYP_STATUS_INTERNAL, "device allocation of " + std::to_string(bytes) +
                                                       " bytes failed: " + hipGetErrorString(err));
        }
        *out_ptr = p;
    });
}

HypStatus hyp_device_free(void** ptr) {
    return abi_call("hyp_device_free", [&] {
        REQUIRE_ARG(ptr != nullptr, "free requires a non-null pointer to the allocation");
        if (*ptr == nullptr) return;
        HYP_HIP_CHECK(hipFree(*ptr));
        *ptr = nullptr;
    });
}

HypStatus hyp_stream_create(HypStream* out_stream) {
    return abi_call("hyp_stream_create", [&] {
        REQUIRE_ARG(out_stream != nullptr, "create requires a non-null out handle");
        require_device();
        auto h = std::make_unique<HypStreamOpaque>();
        h->workspace_bytes = hyperion::hip::sample_greedy_workspace_bytes();
        h->stoch_workspace_offset = (h->workspace_bytes + 255u) / 256u * 256u;
        const size_t bytes = h->stoch_workspace_offset + hyperion::hip::sample_stochastic_workspace_bytes();
        HYP_HIP_CHECK(hipMalloc(&h->workspace, bytes));
        hipError_t err = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
        if (err == hipSuccess) {
            // The draw's bins start (and stay, between calls) zero.
            hyperion::hip::init_sample_stochastic_workspace(h->stoch_workspace(), h->stream);
            err = hipStreamSynchronize(h->stream);
            if (err != hipSuccess) (void)hipStreamDestroy(h->stream);
        }
        if (err != hipSuccess) {
            (void)hipFree(h->workspace);
            HYP_HIP_CHECK(err);
        }
        h->magic = kStreamMagic;
        *out_stream = h.release();
    });
}

HypStatus hyp_stream_destroy(HypStream* stream) {
    if (stream == nullptr) return fail(HYP_STATUS_INVALID_ARGUMENT, "free requires a non-null handle pointer");
    if (*stream == nullptr) return ok();
    if ((*stream)->magic != kStreamMagic) {
        return fail(HYP_STATUS_INVALID_ARGUMENT, "handle magic mismatch (wrong type, freed, or corrupted)");
    }
    hipError_t err = hipStreamDestroy((*stream)->stream);
    // hipFree waits for the device, so work still queued on the stream finishes first.
    const hipError_t ferr = hipFree((*stream)->workspace);
    if (err == hipSuccess) err = ferr;
    (*stream)->magic = 0;
    delete *stream;
    *stream = nullptr;
    if (err != hipSuccess) return fail(HYP_STATUS_INTERNAL, hipGetErrorString(err));
    return ok();
}

HypStatus hyp_stream_synchronize(HypStream stream) {
    return abi_call("hyp_stream_synchronize", [&] { HYP_HIP_CHECK(hipStreamSynchronize(stream_of(stream))); });
}

HypStatus hyp_memcpy_htod(void* dst, const void* src, size_t bytes, HypStream stream) {
    return abi_call("hyp_memcpy_htod", [&] {
        hipStream_t s = stream_of(stream);
        if (bytes == 0) return;
        REQUIRE_ARG(dst != nullptr && src != nullptr, "memcpy requires non-null buffers");
        HYP_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
    });
}

HypStatus hyp_memcpy_dtoh(void* dst, const void* src, size_t bytes, HypStream stream) {
    return abi_call("hyp_memcpy_dtoh", [&] {
        hipStream_t s = stream_of(stream);
        if (bytes == 0) return;
        REQUIRE_ARG(dst != nullptr && src != nullptr, "memcpy requires non-null buffers");
        HYP_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
    });
}

HypStatus hyp_memcpy_dtod(void* dst, const void* src, size_t bytes, HypStream stream) {
    return abi_call("hyp_memcpy_dtod", [&] {
        hipStream_t s = stream_of(stream);
        if (bytes == 0) return;
        REQUIRE_ARG(dst != nullptr && src != nullptr, "memcpy requires non-null buffers");
        HYP_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s));
    });
}

HypStatus hyp_memset_device(void* dst, int value, size_t bytes, HypStream stream) {
    return abi_call("hyp_memset_device", [&] {
        hipStream_t s = stream_of(stream);
        if (bytes == 0) return;
        REQUIRE_ARG(dst != nullptr, "memset requires a non-null buffer");
        require_not_capturing(s, "hyp_memset_device");
        HYP_HIP_CHECK(hipMemsetAsync(dst, value, bytes, s));
    });
}

HypStatus hyp_event_create(HypEvent* out_event) {
    return abi_call("hyp_event_create", [&] {
        REQUIRE_ARG(out_event != nullptr, "create requires a non-null out handle");
        require_device();
        auto h = std::make_unique<HypEventOpaque>();
        HYP_HIP_CHECK(hipEventCreate(&h->event));
        h->magic = kEventMagic;
        *out_event = h.release();
    });
}

HypStatus hyp_event_destroy(HypEvent* event) {
    if (event == nullptr) return fail(HYP_STATUS_INVALID_ARGUMENT, "free requires a non-null handle pointer");
    if (*event == nullptr) return ok();
    if ((*event)->magic != kEventMagic) {
        return fail(HYP_STATUS_INVALID_ARGUMENT, "handle magic mismatch (wrong type, freed, or corrupted)");
    }
    const hipError_t err = hipEventDestroy((*event)->event);
    (*event)->magic = 0;
    delete *event;
    *event = nullptr;
    if (err != hipSuccess) return fail(HYP_STATUS_INTERNAL, hipGetErrorString(err));
    return ok();
}

HypStatus hyp_event_record(HypEvent event, HypStream stream) {
    return abi_call("hyp_event_record", [&] {
        REQUIRE_ARG(event != nullptr && event->magic == kEventMagic, "event handle is invalid");
        HYP_HIP_CHECK(hipEventRecord(event->event, stream_of(stream)));
    });
}

HypStatus hyp_event_elapsed_ms(HypEvent start, HypEvent end, float* out_ms) {
    return abi_call("hyp_event_elapsed_ms", [&] {
        REQUIRE_ARG(start != nullptr && start->magic == kEventMagic, "start event handle is invalid");
        REQUIRE_ARG(end != nullptr && end->magic == kEventMagic, "end event handle is invalid");
        REQUIRE_ARG(out_ms != nullptr, "elapsed requires a non-null out pointer");
        HYP_HIP_CHECK(hipEventSynchronize(end->event));
        HYP_HIP_CHECK(hipEventElapsedTime(out_ms, start->event, end->event));
    });
}

HypStatus hyp_graph_capture_begin(HypStream stream) {
    return abi_call("hyp_graph_capture_begin", [&] {
        HYP_HIP_CHECK(hipStreamBeginCapture(stream_of(stream), hipStreamCaptureModeThreadLocal));
    });
}

HypStatus hyp_graph_capture_end(HypStream stream, HypGraph* out_graph) {
    return abi_call("hyp_graph_capture_end", [&] {
        hipStream_t s = stream_of(stream);
        hipGraph_t graph = nullptr;
        const hipError_t end = hipStreamEndCapture(s, &graph);
        REQUIRE_ARG(out_graph != nullptr, "capture end requires a non-null out handle (the capture was ended)");
        if (end != hipSuccess) {
            if (graph != nullptr) (void)hipGraphDestroy(graph);
            HYP_HIP_CHECK(end);
        }
        auto h = std::make_unique<HypGraphOpaque>();
        h->graph = graph;
        const hipError_t inst = hipGraphInstantiate(&h->exec, graph, nullptr, nullptr, 0);
        if (inst != hipSuccess) {
            (void)hipGraphDestroy(graph);
            HYP_HIP_CHECK(inst);
        }
        h->magic = kGraphMagic;
        *out_graph = h.release();
    });
}

HypStatus hyp_graph_launch(HypGraph graph, HypStream stream) {
    return abi_call("hyp_graph_launch", [&] {
        REQUIRE_ARG(graph != nullptr && graph->magic == kGraphMagic, "graph handle is invalid");
        HYP_HIP_CHECK(hipGraphLaunch(graph->exec, stream_of(stream)));
    });
}

HypStatus hyp_graph_free(HypGraph* graph) {
    if (graph == nullptr) return fail(HYP_STATUS_INVALID_ARGUMENT, "free requires a non-null handle pointer");
    if (*graph == nullptr) return ok();
    if ((*graph)->magic != kGraphMagic) {
        return fail(HYP_STATUS_INVALID_ARGUMENT, "handle magic mismatch (wrong type, freed, or corrupted)");
    }
    const hipError_t e1 = hipGraphExecDestroy((*graph)->exec);
    const hipError_t e2 = hipGraphDestroy((*graph)->graph);
    (*graph)->magic = 0;
    delete *graph;
    *graph = nullptr;
    if (e1 != hipSuccess) return fail(HYP_STATUS_INTERNAL, hipGetErrorString(e1));
    if (e2 != hipSuccess) return fail(HYP_STATUS_INTERNAL, hipGetErrorString(e2));
    return ok();
}

HypStatus hyp_qweight_create(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, uint32_t n,
                             uint32_t k, uint32_t group_size, uint32_t bits, HypQWeight* out_weight) {
    return abi_call("hyp_qweight_create", [&] {
        REQUIRE_ARG(out_weight != nullptr, "create requires a non-null out handle");
        validate_quant(n, k, group_size, bits);
        REQUIRE_ARG(w != nullptr && scales != nullptr && biases != nullptr,
                    "weight, scales and biases must be non-null");
        require_device();
        auto h = std::make_unique<HypQWeightOpaque>();
        h->lin = QuantizedLinear::from_host(w, scales, biases, n, k);
        h->magic = kQWeightMagic;
        *out_weight = h.release();
    });
}

HypStatus hyp_qweight_create_device(const uint32_t* w, const void* scales, const void* biases, uint32_t n,
                                    uint32_t k, uint32_t group_size, uint32_t bits, HypStream stream,
                                    HypQWeight* out_weight) {
    return abi_call("hyp_qweight_create_device", [&] {
        REQUIRE_ARG(out_weight != nullptr, "create requires a non-null out handle");
        validate_quant(n, k, group_size, bits);
        REQUIRE_ARG(w != nullptr && scales != nullptr && biases != nullptr,
                    "weight, scales and biases must be non-null");
        hipStream_t s = stream_of(stream);
        auto h = std::make_unique<HypQWeightOpaque>();
        h->lin = QuantizedLinear::from_device(w, static_cast<const uint16_t*>(scales),
                                              static_cast<const uint16_t*>(biases), n, k, s);
        h->magic = kQWeightMagic;
        *out_weight = h.release();
    });
}

HypStatus hyp_qweight_free(HypQWeight* weight) {
    if (weight != nullptr && *weight != nullptr && (*weight)->magic == kQWeightMagic && (*weight)->owned_by_model) {
        return fail(HYP_STATUS_INVALID_ARGUMENT, "weight handle is owned by a model; free the model instead");
    }
    return free_handle(weight, kQWeightMagic);
}

HypStatus hyp_qweight_shape(HypQWeight weight, uint32_t* out_n, uint32_t* out_k) {
    return abi_call("hyp_qweight_shape", [&] {
        const QuantizedLinear& lin = qweight_ref(weight, "weight");
        REQUIRE_ARG(out_n != nullptr && out_k != nullptr, "shape requires non-null out pointers");
        *out_n = lin.mat.n;
        *out_k = lin.mat.k;
    });
}

HypStatus hyp_qweight_export(HypQWeight weight, uint32_t* w, uint16_t* scales, uint16_t* biases) {
    return abi_call("hyp_qweight_export", [&] {
        const QuantizedLinear& lin = qweight_ref(weight, "weight");
        REQUIRE_ARG(w != nullptr && scales != nullptr && biases != nullptr, "export requires non-null buffers");
        lin.export_mlx(w, scales, biases);
    });
}

HypStatus hyp_qmatmul_ex(HypQWeight weight, const void* x, uint32_t m, void* y, HypEpilogue epilogue, float cap,
                         HypStream stream) {
    return abi_call("hyp_qmatmul", [&] {
        const QuantizedLinear& lin = qweight_ref(weight, "weight");
        hipStream_t s = stream_of(stream);
        Epilogue epi = Epilogue::kNone;
        float cap_bf16 = 0.0f;
        if (epilogue == HYP_EPILOGUE_SOFTCAP) {
            REQUIRE_ARG(std::isfinite(cap) && cap > 0.0f, "softcap requires a finite positive cap");
            epi = Epilogue::kSoftcap;
            cap_bf16 = round_to_bf16(cap);
        } else {
            REQUIRE_ARG(epilogue == HYP_EPILOGUE_NONE, "unknown epilogue");
        }
        if (m == 0) return;
        REQUIRE_ARG(x != nullptr && y != nullptr, "x and y must be non-null device pointers");
        if (!hyperion::hip::skinny_supported(m, lin.mat.k, false)) require_not_capturing(s, "hyp_qmatmul on the GEMM path");
        lin.apply(static_cast<const uint16_t*>(x), m, static_cast<uint16_t*>(y), s, epi, cap_bf16);
    });
}

HypStatus hyp_qmatmul(HypQWeight weight, const void* x, uint32_t m, void* y, HypStream stream) {
    return hyp_qmatmul_ex(weight, x, m, y, HYP_EPILOGUE_NONE, 0.0f, stream);
}

HypStatus hyp_qmatmul_noalloc(HypQWeight weight, const void* x, uint32_t m, void* y, HypStream stream) {
    return abi_call("hyp_qmatmul_noalloc", [&] {
        const QuantizedLinear& lin = qweight_ref(weight, "weight");
        hipStream_t s = stream_of(stream);
        if (m == 0) return;
        REQUIRE_ARG(x != nullptr && y != nullptr, "x and y must be non-null device pointers");
        lin.apply_noalloc(static_cast<const uint16_t*>(x), m, static_cast<uint16_t*>(y), s);
    });
}

namespace {

void qmatmul_group(const HypQWeight* weights, uint32_t count, const void* x, uint32_t m, const float* rms_eps,
                   const void* norm_weight, void* const* ys, HypStream stream) {
    REQUIRE_ARG(weights != nullptr && ys != nullptr, "weights and ys must be non-null arrays");
    REQUIRE_ARG(count >= 1u && count <= HYP_QMATMUL_GROUP_MAX, "count must be 1..HYP_QMATMUL_GROUP_MAX");
    const QuantizedLinear* lins[HYP_QMATMUL_GROUP_MAX];
    uint16_t* outs[HYP_QMATMUL_GROUP_MAX];
    for (uint32_t i = 0; i < count; ++i) {
        lins[i] = &qweight_ref(weights[i], "weights[i]");
        REQUIRE_ARG(lins[i]->mat.k == lins[0]->mat.k, "grouped weights must share k");
        outs[i] = static_cast<uint16_t*>(ys[i]);
    }
    if (rms_eps != nullptr) REQUIRE_ARG(std::isfinite(*rms_eps) && *rms_eps >= 0.0f, "eps must be finite and >= 0");
    REQUIRE_ARG((reinterpret_cast<uintptr_t>(norm_weight) & 15u) == 0u, "norm_weight must be 16-byte aligned");
    hipStream_t s = stream_of(stream);
    if (m == 0) return;
    REQUIRE_ARG(x != nullptr, "x must be a non-null device pointer");
    for (uint32_t i = 0; i < count; ++i) REQUIRE_ARG(outs[i] != nullptr, "ys[i] must be non-null device pointers");
    const uint32_t k = lins[0]->mat.k;
    if (!(rms_eps != nullptr ? hyperion::hip::skinny_norm_supported(m, k) : hyperion::hip::skinny_supported(m, k, false)))
        require_not_capturing(s, "hyp_qmatmul_group on the GEMM path");
    hyperion::model::apply_group(lins, outs, count, static_cast<const uint16_t*>(x), m, rms_eps,
                                 static_cast<const uint16_t*>(norm_weight), s);
}

}  // namespace

HypStatus hyp_qmatmul_group(const HypQWeight* weights, uint32_t count, const void* x, uint32_t m,
                            void* const* ys, HypStream stream) {
    return abi_call("hyp_qmatmul_group",
                    [&] { qmatmul_group(weights, count, x, m, nullptr, nullptr, ys, stream); });
}

HypStatus hyp_qmatmul_group_rmsnorm(const HypQWeight* weights, uint32_t count, const void* x,
                                    const void* norm_weight, uint32_t m, float eps, void* const* ys,
                                    HypStream stream) {
    return abi_call("hyp_qmatmul_group_rmsnorm",
                    [&] { qmatmul_group(weights, count, x, m, &eps, norm_weight, ys, stream); });
}

HypStatus hyp_qmlp_gate_up_gelu(HypQWeight gate, HypQWeight up, const void* x, uint32_t m, void* h,
                                HypStream stream) {
    return abi_call("hyp_qmlp_gate_up_gelu", [&] {
        const QuantizedLinear& g = qweight_ref(gate, "gate");
        const QuantizedLinear& u = qweight_ref(up, "up");
        hipStream_t s = stream_of(stream);
        REQUIRE_ARG(g.mat.n == u.mat.n && g.mat.k == u.mat.k, "gate and up must have the same shape");
        if (m == 0) return;
        REQUIRE_ARG(x != nullptr && h != nullptr, "x and h must be non-null device pointers");
        if (!hyperion::hip::skinny_supported(m, g.mat.k, true)) require_not_capturing(s, "hyp_qmlp_gate_up_gelu on the GEMM path");
        hyperion::model::mlp_gate_up(g, u, static_cast<const uint16_t*>(x), m, static_cast<uint16_t*>(h), s);
    });
}

HypStatus hyp_quantize_q4g64(const void* w, uint32_t n, uint32_t k, uint32_t* w_out, void* scales_out,
                             void* biases_out, HypStream stream) {
    return abi_call("hyp_quantize_q4g64", [&] {
        hipStream_t s = stream_of(stream);
        validate_quant(n, k, 64, 4);
        REQUIRE_ARG(w != nullptr && w_out != nullptr && scales_out != nullptr && biases_out != nullptr,
                    "quantize requires non-null device buffers");
        REQUIRE_ARG((reinterpret_cast<uintptr_t>(w) & 15u) == 0u && (reinterpret_cast<uintptr_t>(w_out) & 15u) == 0u,
                    "quantize requires 16-byte aligned w and w_out");
        REQUIRE_ARG((reinterpret_cast<uintptr_t>(scales_out) & 1u) == 0u &&
                        (reinterpret_cast<uintptr_t>(biases_out) & 1u) == 0u,
                    "quantize requires 2-byte aligned scales and biases");
        hyperion::hip::launch_q4_quantize(static_cast<const uint16_t*>(w), n, k, w_out,
                                          static_cast<uint16_t*>(scales_out), static_cast<uint16_t*>(biases_out), s);
    });
}

HypStatus hyp_dequantize_q4g64(const uint32_t* w, const void* scales, const void* biases, uint32_t n_total,
                               uint32_t k, const uint32_t* rows, uint32_t n_rows, float out_scale, void* out,
                               HypStream stream) {
    return abi_call("hyp_dequantize_q4g64", [&] {
        hipStream_t s = stream_of(stream);
        validate_quant(n_total, k, 64, 4);
        REQUIRE_ARG(std::isfinite(out_scale), "out_scale must be finite");
        if (n_rows == 0) return;
        REQUIRE_ARG(w != nullptr && scales != nullptr && biases != nullptr && out != nullptr,
                    "dequantize requires non-null device buffers");
        REQUIRE_ARG(rows != nullptr || n_rows <= n_total, "n_rows exceeds the table without a row list");
        hyperion::hip::launch_q4_dequantize(w, static_cast<const uint16_t*>(scales),
                                            static_cast<const uint16_t*>(biases), n_total, k, rows, n_rows,
                                            round_to_bf16(out_scale), static_cast<uint16_t*>(out), s);
    });
}

HypStatus hyp_embed(HypQWeight table, const uint32_t* ids, uint32_t n_ids, void* out, HypStream stream) {
    return abi_call("hyp_embed", [&] {
        const QuantizedLinear& t = qweight_ref(table, "table");
        hipStream_t s = stream_of(stream);
        if (n_ids == 0) return;
        REQUIRE_ARG(ids != nullptr && out != nullptr, "ids and out must be non-null device pointers");
        const float scale = round_to_bf16(std::sqrt(static_cast<float>(t.mat.k)));
        hyperion::hip::launch_q4_dequantize_tiled(t.mat, ids, n_ids, scale, static_cast<uint16_t*>(out), s);
    });
}

HypStatus hyp_rms_normalize(const void* x, const void* weight, uint32_t m, uint32_t k, float eps, void* y,
                            HypStream stream) {
    return abi_call("hyp_rms_normalize", [&] {
        hipStream_t s = stream_of(stream);
        REQUIRE_ARG(std::isfinite(eps) && eps >= 0.0f, "eps must be finite and non-negative");
        if (m == 0 || k == 0) return;
        REQUIRE_ARG(x != nullptr && y != nullptr, "x and y must be non-null device pointers");
        REQUIRE_ARG(weight == nullptr || (reinterpret_cast<uintptr_t>(weight) & 15u) == 0u || k % 64u != 0u,
                    "the weight must be 16-byte aligned");
        hyperion::hip::launch_rms_normalize(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight), m, k,
                                            eps, static_cast<uint16_t*>(y), s);
    });
}

HypStatus hyp_rope(const void* x, uint32_t rows, uint32_t heads, uint32_t head_dim, uint32_t rotated_dims, float base,
                   uint32_t offset, void* y, HypStream stream) {
    return abi_call("hyp_rope", [&] {
        hipStream_t s = stream_of(stream);
        REQUIRE_ARG(head_dim > 0 && head_dim % 2 == 0, "head_dim must be a positive even number");
        REQUIRE_ARG(rotated_dims % 2 == 0 && rotated_dims <= head_dim, "rotated_dims must be even and <= head_dim");
        REQUIRE_ARG(std::isfinite(base) && base > 0.0f, "base must be finite and positive");
        REQUIRE_ARG(static_cast<uint64_t>(offset) + rows <= (1ull << 24),
                    "positions must stay below 2^24 (exact in fp32)");
        if (rows == 0 || heads == 0) return;
        REQUIRE_ARG(x != nullptr && y != nullptr, "x and y must be non-null device pointers");
        hyperion::hip::launch_rope(static_cast<const uint16_t*>(x), rows, heads, head_dim, rotated_dims, base, offset,
                                   static_cast<uint16_t*>(y), s);
    });
}

HypStatus hyp_sample_greedy(const void* logits, uint32_t rows, uint32_t vocab, HypGreedySample* out,
                            HypStream stream) {
    return abi_call("hyp_sample_greedy", [&] {
        hipStream_t s = stream_of(stream);
        if (rows == 0) return;
        REQUIRE_ARG(out != nullptr, "out must be a non-null device pointer");
        REQUIRE_ARG(vocab == 0 || logits != nullptr, "logits must be a non-null device pointer");
        REQUIRE_ARG(vocab <= (1u << 31), "vocab must be at most 2^31");
        REQUIRE_ARG(static_cast<uint64_t>(rows) * vocab < (1ull << 62), "logits too large");
        hyperion::hip::launch_sample_greedy(static_cast<const uint16_t*>(logits), rows, vocab, out, stream->workspace,
                                            stream->workspace_bytes, s);
    });
}

static_assert(sizeof(HypTopKSample) == 80, "HypTopKSample is 80 bytes");

HypStatus hyp_sample_greedy_topk(const void* logits, uint32_t rows, uint32_t vocab, HypTopKSample* out,
                                 HypStream stream) {
    return abi_call("hyp_sample_greedy_topk", [&] {
        hipStream_t s = stream_of(stream);
        if (rows == 0) return;
        REQUIRE_ARG(out != nullptr, "out must be a non-null device pointer");
        REQUIRE_ARG(vocab == 0 || logits != nullptr, "logits must be a non-null device pointer");
        REQUIRE_ARG(vocab <= hyperion::hip::sample_topk_max_vocab(), "vocab must be at most 2^23");
        REQUIRE_ARG(static_cast<uint64_t>(rows) * vocab < (1ull << 62), "logits too large");
        hyperion::hip::launch_sample_topk(static_cast<const uint16_t*>(logits), rows, vocab, out, stream->workspace,
                                          stream->workspace_bytes, s);
    });
}

HypStatus hyp_sample_stochastic(const void* logits, uint32_t vocab, const HypSamplingConfig* config,
                                uint64_t rng_state, HypTopKSample* out, HypStream stream) {
    return abi_call("hyp_sample_stochastic", [&] {
        hipStream_t s = stream_of(stream);
        REQUIRE_ARG(out != nullptr, "out must be a non-null device pointer");
        REQUIRE_ARG(vocab == 0 || logits != nullptr, "logits must be a non-null device pointer");
        REQUIRE_ARG(vocab <= hyperion::hip::sample_topk_max_vocab(), "vocab must be at most 2^23");
        const bool greedy = hyperion::model::sampling_is_greedy(config, vocab);
        const auto* l = static_cast<const uint16_t*>(logits);
        hyperion::hip::launch_sample_topk(l, 1, vocab, out, stream->workspace, stream->workspace_bytes, s);
        if (greedy) return;
        const hyperion::hip::SampleParams p = hyperion::model::sampling_params(*config);
        hyperion::hip::launch_sample_params(stream->stoch_workspace(), p.inv_temp, p.top_p, p.min_p, p.top_k,
                                            hyperion::model::sampling_uniform(rng_state), s);
        hyperion::hip::launch_sample_stochastic(l, vocab, stream->stoch_workspace(),
                                                hyperion::hip::sample_stochastic_workspace_bytes(), out, s);
    });
}

HypStatus hyp_kv_cache_create(uint32_t capacity, uint32_t num_kv_heads, uint32_t head_dim, HypKvCache* out_cache) {
    return abi_call("hyp_kv_cache_create", [&] {
        REQUIRE_ARG(out_cache != nullptr, "create requires a non-null out handle");
        REQUIRE_ARG(capacity > 0 && num_kv_heads > 0, "capacity and num_kv_heads must be positive");
        REQUIRE_ARG(head_dim == 64u || head_dim == 128u || head_dim == 256u || head_dim == 512u,
                    "head_dim must be 64, 128, 256 or 512");
        REQUIRE_ARG(capacity < (1u << 30), "capacity must be below 2^30 tokens");
        const uint64_t bytes = static_cast<uint64_t>(capacity) * num_kv_heads * head_dim * 2u;
        REQUIRE_ARG(bytes < (1ull << 40), "cache too large");
        require_device();
        auto c = std::make_unique<HypKvCacheOpaque>();
        c->capacity = capacity;
        c->num_kv_heads = num_kv_heads;
        c->head_dim = head_dim;
        c->k = DeviceBuffer(bytes);
        c->v = DeviceBuffer(bytes);
        c->workspace = DeviceBuffer(hyperion::hip::attention_workspace_bytes(num_kv_heads, head_dim));
        c->magic = kKvCacheMagic;
        *out_cache = c.release();
    });
}

HypStatus hyp_kv_cache_free(HypKvCache* cache) {
    return free_handle(cache, kKvCacheMagic);
}

}  // extern "C"

namespace {
HypKvCacheOpaque& kv_ref(HypKvCache c) {
    REQUIRE_ARG(c != nullptr, "kv cache handle is null");
    REQUIRE_ARG(c->magic == kKvCacheMagic, "kv cache handle magic mismatch (wrong type, freed, or corrupted)");
    return *c;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0u; }
}  // namespace

extern "C" {

HypStatus hyp_kv_cache_buffers(HypKvCache cache, void** out_k, void** out_v) {
    return abi_call("hyp_kv_cache_buffers", [&] {
        HypKvCacheOpaque& c = kv_ref(cache);
        REQUIRE_ARG(out_k != nullptr && out_v != nullptr, "out pointers must be non-null");
        *out_k = c.k.data();
        *out_v = c.v.data();
    });
}

HypStatus hyp_kv_cache_write(HypKvCache cache, const void* k, const void* v, uint32_t n_tokens, uint32_t pos0,
                             HypStream stream) {
    return abi_call("hyp_kv_cache_write", [&] {
        hipStream_t s = stream_of(stream);
        HypKvCacheOpaque& c = kv_ref(cache);
        if (n_tokens == 0) return;
        REQUIRE_ARG(k != nullptr && v != nullptr, "k and v must be non-null device pointers");
        REQUIRE_ARG(aligned16(k) && aligned16(v), "k and v must be 16-byte aligned");
        REQUIRE_ARG(static_cast<uint64_t>(pos0) + n_tokens < (1ull << 31), "positions must stay below 2^31");
        hyperion::hip::launch_kv_write(static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                                       static_cast<uint16_t*>(c.k.data()), static_cast<uint16_t*>(c.v.data()), n_tokens,
                                       pos0, c.capacity, c.num_kv_heads, c.head_dim, s);
    });
}

HypStatus hyp_attention(const void* q, const void* k, const void* v, uint32_t L, uint32_t n_heads, HypKvCache cache,
                        uint32_t offset, uint32_t prefix_len, uint32_t window, void* out, HypStream stream) {
    return abi_call("hyp_attention", [&] {
        hipStream_t s = stream_of(stream);
        HypKvCacheOpaque& c = kv_ref(cache);
        if (L == 0) return;
        REQUIRE_ARG(q != nullptr && out != nullptr, "q and out must be non-null device pointers");
        REQUIRE_ARG((k == nullptr) == (v == nullptr), "k and v must both be device pointers or both NULL");
        REQUIRE_ARG(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out),
                    "q, k, v and out must be 16-byte aligned");
        REQUIRE_ARG(n_heads > 0 && n_heads % c.num_kv_heads == 0, "n_heads must be a multiple of the cache's num_kv_heads");
        REQUIRE_ARG(prefix_len <= offset, "prefix_len must not exceed offset");
        REQUIRE_ARG(prefix_len <= c.capacity, "prefix_len must not exceed the cache capacity");
        REQUIRE_ARG(k != nullptr || static_cast<uint64_t>(prefix_len) + L <= c.capacity,
                    "with the chunk read from the cache, prefix_len + L must not exceed the cache capacity");
        REQUIRE_ARG(static_cast<uint64_t>(offset) + L < (1ull << 31), "positions must stay below 2^31");
        REQUIRE_ARG(static_cast<uint64_t>(L) * n_heads * c.head_dim < (1ull << 31), "q too large");
        hyperion::hip::AttnArgs a{};
        a.q = static_cast<const uint16_t*>(q);
        a.k = static_cast<const uint16_t*>(k);
        a.v = static_cast<const uint16_t*>(v);
        a.cache_k = static_cast<const uint16_t*>(c.k.data());
        a.cache_v = static_cast<const uint16_t*>(c.v.data());
        a.out = static_cast<uint16_t*>(out);
        a.L = L;
        a.n_heads = n_heads;
        a.n_kv_heads = c.num_kv_heads;
        a.head_dim = c.head_dim;
        a.cap = c.capacity;
        a.offset = offset;
        a.prefix_len = prefix_len;
        a.window = window;
        a.workspace = c.workspace.data();
        a.workspace_bytes = c.workspace.bytes();
        hyperion::hip::launch_attention(a, s);
    });
}

HypStatus hyp_attention_prepare(void* q, const void* k_raw, const void* v_raw, uint32_t L, uint32_t n_heads,
                                HypKvCache cache, const void* q_norm, const void* k_norm, float eps,
                                uint32_t rotated_dims, float rope_base, uint32_t offset, HypStream stream) {
    return abi_call("hyp_attention_prepare", [&] {
        hipStream_t s = stream_of(stream);
        HypKvCacheOpaque& c = kv_ref(cache);
        if (L == 0) return;
        REQUIRE_ARG(q != nullptr && k_raw != nullptr && q_norm != nullptr && k_norm != nullptr,
                    "q, k_raw, q_norm and k_norm must be non-null device pointers");
        REQUIRE_ARG(aligned16(q) && aligned16(k_raw) && aligned16(v_raw) && aligned16(q_norm) && aligned16(k_norm),
                    "q, k_raw, v_raw, q_norm and k_norm must be 16-byte aligned");
        REQUIRE_ARG(n_heads > 0 && n_heads % c.num_kv_heads == 0, "n_heads must be a multiple of the cache's num_kv_heads");
        REQUIRE_ARG(std::isfinite(eps) && eps >= 0.0f, "eps must be finite and >= 0");
        REQUIRE_ARG(rotated_dims <= c.head_dim && rotated_dims % 2u == 0u, "rotated_dims must be even and <= head_dim");
        REQUIRE_ARG(std::isfinite(rope_base) && rope_base > 0.0f, "rope_base must be finite and positive");
        REQUIRE_ARG(static_cast<uint64_t>(offset) + L < (1ull << 24), "positions must stay below 2^24");
        REQUIRE_ARG(static_cast<uint64_t>(L) * n_heads * c.head_dim < (1ull << 31), "q too large");
        hyperion::hip::AttnPrepareArgs a{};
        a.q = static_cast<uint16_t*>(q);
        a.k_raw = static_cast<const uint16_t*>(k_raw);
        a.v_raw = static_cast<const uint16_t*>(v_raw);
        a.q_norm = static_cast<const uint16_t*>(q_norm);
        a.k_norm = static_cast<const uint16_t*>(k_norm);
        a.cache_k = static_cast<uint16_t*>(c.k.data());
        a.cache_v = static_cast<uint16_t*>(c.v.data());
        a.L = L;
        a.n_heads = n_heads;
        a.n_kv_heads = c.num_kv_heads;
        a.head_dim = c.head_dim;
        a.rotated = rotated_dims;
        a.offset = offset;
        a.cap = c.capacity;
        a.base = rope_base;
        a.eps = eps;
        hyperion::hip::launch_attn_prepare(a, s);
    });
}

HypStatus hyp_residual_rms_norm(const void* branch, void* residual, const void* post_weight, const void* scalar,
                                const void* next_weight, void* next, uint32_t m, uint32_t hidden, float eps,
                                HypStream stream) {
    return abi_call("hyp_residual_rms_norm", [&] {
        hipStream_t s = stream_of(stream);
        if (m == 0) return;
        REQUIRE_ARG(branch != nullptr && residual != nullptr && post_weight != nullptr,
                    "branch, residual and post_weight must be non-null device pointers");
        REQUIRE_ARG((next_weight == nullptr) == (next == nullptr), "next_weight and next must both be given or both NULL");
        REQUIRE_ARG(aligned16(branch) && aligned16(residual) && aligned16(post_weight) && aligned16(next_weight) &&
                        aligned16(next),
                    "branch, residual, post_weight, next_weight and next must be 16-byte aligned");
        REQUIRE_ARG(hidden > 0 && hidden % 64u == 0u && hidden <= hyperion::hip::residual_norm_max_hidden(),
                    "hidden must be a positive multiple of 64, at most 16384");
        REQUIRE_ARG(std::isfinite(eps) && eps >= 0.0f, "eps must be finite and >= 0");
        REQUIRE_ARG(static_cast<uint64_t>(m) < (1ull << 31), "too many rows");
        hyperion::hip::launch_residual_norm(static_cast<const uint16_t*>(branch), static_cast<uint16_t*>(residual),
                                            static_cast<const uint16_t*>(post_weight),
                                            static_cast<const uint16_t*>(scalar),
                                            static_cast<const uint16_t*>(next_weight), static_cast<uint16_t*>(next), m,
                                            hidden, eps, s);
    });
}

HypStatus hyp_step_program_create(const HypStepOp* ops, uint32_t n_ops, uint32_t m, uint32_t spin_limit,
                                  HypStepProgram* out_program) {
    return abi_call("hyp_step_program_create", [&] {
        REQUIRE_ARG(out_program != nullptr, "create requires a non-null out handle");
        REQUIRE_ARG(ops != nullptr && n_ops > 0, "a step program needs at least one op");
        REQUIRE_ARG(m >= 1u && m <= hyperion::hip::kSkinnyMaxM, "a step program runs m = 1..4 rows");
        std::vector<hyperion::model::StepOpSpec> specs(n_ops);
        for (uint32_t i = 0; i < n_ops; ++i) {
            const HypStepOp& o = ops[i];
            hyperion::model::StepOpSpec& sp = specs[i];
            const std::string who = "op " + std::to_string(i) + ": ";
            switch (o.kind) {
                case HYP_STEP_QMATMUL: sp.form = hyperion::hip::StepForm::kPlain; break;
                case HYP_STEP_QMATMUL_RMSNORM: sp.form = hyperion::hip::StepForm::kNorm; break;
                case HYP_STEP_GATE_UP_GELU: sp.form = hyperion::hip::StepForm::kDual; break;
                default: throw NativeError(HYP_STATUS_INVALID_ARGUMENT, who + "unknown op kind");
            }
            REQUIRE_ARG(o.count >= 1u && o.count <= 3u, who + "count must be 1..3");
            REQUIRE_ARG(o.reserved == 0u, who + "reserved must be 0");
            sp.count = o.count;
            for (uint32_t q = 0; q < o.count; ++q) sp.w[q] = &qweight_ref(o.weights[q], "op weight");
            sp.x = static_cast<const uint16_t*>(o.x);
            for (uint32_t q = 0; q < 3u; ++q) sp.y[q] = static_cast<uint16_t*>(o.y[q]);
            sp.eps = o.eps;
            sp.norm_w = static_cast<const uint16_t*>(o.norm_weight);
        }
        require_device();
        auto h = std::make_unique<HypStepProgramOpaque>();
        h->program = std::make_unique<hyperion::model::StepProgram>(specs, m, spin_limit);
        h->magic = kStepProgramMagic;
        *out_program = h.release();
    });
}

HypStatus hyp_step_program_run(HypStepProgram program, HypStream stream) {
    return abi_call("hyp_step_program_run", [&] {
        REQUIRE_ARG(program != nullptr && program->magic == kStepProgramMagic, "step program handle is invalid");
        hipStream_t s = stream_of(stream);
        require_not_capturing(s, "hyp_step_program_run (a cooperative launch)");
        program->program->run(s);
    });
}

HypStatus hyp_step_program_check(HypStepProgram program) {
    return abi_call("hyp_step_program_check", [&] {
        REQUIRE_ARG(program != nullptr && program->magic == kStepProgramMagic, "step program handle is invalid");
        const std::uint32_t err = program->program->check();
        if (err != 0u) {
            throw NativeError(HYP_STATUS_INTERNAL,
                              "a step-program run gave up waiting for the other workgroups (error " +
                                  std::to_string(err) + "); its outputs are undefined and the program was reset");
        }
    });
}

HypStatus hyp_step_program_free(HypStepProgram* program) {
    return free_handle(program, kStepProgramMagic);
}

HypStatus hyp_qmodel_load(const char* dir, uint32_t num_layers, HypQModel* out_model) {
    return abi_call("hyp_qmodel_load", [&] {
        REQUIRE_ARG(out_model != nullptr, "load requires a non-null out handle");
        REQUIRE_ARG(dir != nullptr, "weights path is null");
        // Every artifact check (directory, shards, headers, names, shapes) runs on the
        // host before the first device call, so those errors surface without a GPU.
        const hyperion::model::ModelManifest manifest(dir, num_layers);
        require_device();
        auto model = std::make_unique<HypQModelOpaque>();
        model->weights = manifest.upload();
        auto wrap = [](QuantizedLinear* lin) {
            auto h = std::make_unique<HypQWeightOpaque>();
            h->magic = kQWeightMagic;
            h->owned_by_model = true;
            h->lin.mat = lin->mat;   // borrowed view; storage stays in the model
            return h;
        };
        model->embed = wrap(&model->weights.embed);
        for (auto& lw : model->weights.layers) {
            std::array<std::unique_ptr<HypQWeightOpaque>, 7> hs;
            hs[HYP_PROJ_Q] = wrap(&lw.q_proj);
            hs[HYP_PROJ_K] = wrap(&lw.k_proj);
            if (lw.v_proj) hs[HYP_PROJ_V] = wrap(&*lw.v_proj);
            hs[HYP_PROJ_O] = wrap(&lw.o_proj);
            hs[HYP_PROJ_GATE] = wrap(&lw.gate_proj);
            hs[HYP_PROJ_UP] = wrap(&lw.up_proj);
            hs[HYP_PROJ_DOWN] = wrap(&lw.down_proj);
            model->layers.push_back(std::move(hs));
        }
        model->magic = kQModelMagic;
        *out_model = model.release();
    });
}

HypStatus hyp_qmodel_free(HypQModel* model) {
    return free_handle(model, kQModelMagic);
}

HypStatus hyp_qmodel_num_layers(HypQModel model, uint32_t* out_num_layers) {
    return abi_call("hyp_qmodel_num_layers", [&] {
        REQUIRE_ARG(model != nullptr && model->magic == kQModelMagic, "model handle is invalid");
        REQUIRE_ARG(out_num_layers != nullptr, "requires a non-null out pointer");
        *out_num_layers = static_cast<uint32_t>(model->layers.size());
    });
}

HypStatus hyp_qmodel_linear(HypQModel model, uint32_t layer, HypProj proj, HypQWeight* out_weight) {
    return abi_call("hyp_qmodel_linear", [&] {
        REQUIRE_ARG(model != nullptr && model->magic == kQModelMagic, "model handle is invalid");
        REQUIRE_ARG(out_weight != nullptr, "requires a non-null out handle");
        REQUIRE_ARG(layer < model->layers.size(), "layer index out of range");
        REQUIRE_ARG(static_cast<int>(proj) >= 0 && static_cast<int>(proj) < 7, "unknown projection");
        HypQWeightOpaque* h = model->layers[layer][static_cast<int>(proj)].get();
        if (h == nullptr) {
            throw NativeError(HYP_STATUS_NOT_FOUND, "layer " + std::to_string(layer) +
                                                        " is a global (K = V) layer and has no v_proj");
        }
        *out_weight = h;
    });
}

HypStatus hyp_qmodel_embed(HypQModel model, HypQWeight* out_weight) {
    return abi_call("hyp_qmodel_embed", [&] {
        REQUIRE_ARG(model != nullptr && model->magic == kQModelMagic, "model handle is invalid");
        REQUIRE_ARG(out_weight != nullptr, "requires a non-null out handle");
        *out_weight = model->embed.get();
    });
}

}  // extern "C"

// ---- the model, its KV state and the step ABI (model.cc:359-740) ------------------------

constexpr std::uint32_t kModelMagic = 0x48504D44U;        // "HPMD"
constexpr std::uint32_t kKvStateMagic = 0x48504B53U;      // "HPKS"
constexpr std::uint32_t kStepResultMagic = 0x48505352U;   // "HPSR"

struct HypModelOpaque {
    std::uint32_t magic = 0;
    std::unique_ptr<hyperion::model::Decoder> decoder;   // null until hyp_model_load
};

struct HypKvStateOpaque {
    std::uint32_t magic = 0;
    const HypModelOpaque* model = nullptr;   // the model it was made for (compared, not used)
    hyperion::model::DecoderState state;
};

struct HypStepResultOpaque {
    std::uint32_t magic = 0;
    HypStepResultFields fields{};
};

namespace {

hyperion::model::Decoder& loaded(HypModel model) {
    REQUIRE_ARG(model != nullptr && model->magic == kModelMagic, "model handle is invalid");
    REQUIRE_ARG(model->decoder != nullptr, "model is not loaded");
    return *model->decoder;
}

hyperion::model::DecoderState& state_of(HypModel model, HypKvState kv) {
    REQUIRE_ARG(kv != nullptr && kv->magic == kKvStateMagic, "kvstate handle is invalid");
    REQUIRE_ARG(kv->model == model, "kvstate was created for another model");
    // validate_kvstate (model.cc:149-160): a state consumed by a failed decode is refused.
    HYP_REQUIRE(!kv->state.consumed, HYP_STATUS_INTERNAL,
                "KV state is unusable after an internal execution failure; free and recreate it");
    return kv->state;
}

HypStepResultOpaque& result_of(HypStepResult r) {
    REQUIRE_ARG(r != nullptr && r->magic == kStepResultMagic, "step-result handle is invalid");
    return *r;
}

// write_step_result / write_step_result_sampled (model.cc:310-356).
void write_result(HypStepResultOpaque& r, const hyperion::model::StepSample& smp,
                  const hyperion::model::DecoderState& st, bool sidecar) {
    r.fields = HypStepResultFields{};
    r.fields.token_id = smp.sample.token_id;
    r.fields.logit = smp.sample.logit;
    r.fields.local_kv_bytes = st.local_bytes;
    r.fields.global_kv_bytes = st.global_bytes;
    r.fields.governor_state = HYP_GOVERNOR_READY;
    if (sidecar) {
        r.fields.top_k_logprob_count = smp.sample.top_k_count;
        for (uint32_t i = 0; i < smp.sample.top_k_count && i < HYP_TOP_K_LOGPROBS; ++i) {
            r.fields.top_k_logprob_ids[i] = smp.sample.top_k_ids[i];
            r.fields.top_k_logprob_values[i] = smp.sample.top_k_logprobs[i];
        }
    } else {
        r.fields.near_tie_events = smp.near_tie_events;
    }
}

void check_tokens(const HypTokenStream* tokens) {
    REQUIRE_ARG(tokens != nullptr, "tokens is null");
    REQUIRE_ARG(tokens->count != 0, "prefill token count is 0");
    REQUIRE_ARG(tokens->tokens != nullptr, "tokens->tokens is null");
}

}  // namespace

extern "C" {

HypStatus hyp_model_create(HypModel* out_model) {
    return abi_call("hyp_model_create", [&] {
        REQUIRE_ARG(out_model != nullptr, "create requires a non-null out handle");
        auto m = std::make_unique<HypModelOpaque>();
        m->magic = kModelMagic;
        *out_model = m.release();
    });
}

HypStatus hyp_model_free(HypModel* model) {
    return free_handle(model, kModelMagic);
}

HypStatus hyp_model_load(HypModel model, const HypGeometryParams* geometry, const char* weights_path) {
    return abi_call("hyp_model_load", [&] {
        REQUIRE_ARG(model != nullptr && model->magic == kModelMagic, "model handle is invalid");
        REQUIRE_ARG(geometry != nullptr, "geometry is null");
        REQUIRE_ARG(weights_path != nullptr, "weights_path is null");
        REQUIRE_ARG(model->decoder == nullptr, "model is already loaded");
        hyperion::model::Geometry geo = hyperion::model::Geometry::from_abi(*geometry);
        // The artifact is resolved and checked on the host before the first device call.
        const hyperion::model::ModelManifest manifest(weights_path, geo.num_layers());
        REQUIRE_ARG(manifest.num_layers() == geo.num_layers(), "the artifact holds fewer layers than the geometry");
        require_device();
        model->decoder = std::make_unique<hyperion::model::Decoder>(std::move(geo), manifest.upload());
    });
}

HypStatus hyp_kvstate_create(HypModel model, HypKvState* out_kvstate) {
    return abi_call("hyp_kvstate_create", [&] {
        REQUIRE_ARG(model != nullptr && model->magic == kModelMagic, "model handle is invalid");
        REQUIRE_ARG(out_kvstate != nullptr, "out_kvstate is null");
        REQUIRE_ARG(model->decoder != nullptr, "model is not loaded; cannot allocate KV state");
        auto kv = std::make_unique<HypKvStateOpaque>();
        kv->model = model;
        kv->state = model->decoder->make_state();
        kv->magic = kKvStateMagic;
        *out_kvstate = kv.release();
    });
}

HypStatus hyp_kvstate_free(HypKvState* kvstate) {
    return free_handle(kvstate, kKvStateMagic);
}

HypStatus hyp_prefill_chunk(HypModel model, HypKvState kvstate, const HypTokenStream* tokens,
                            HypStepResult out_result) {
    return abi_call("hyp_prefill_chunk", [&] {
        hyperion::model::Decoder& dec = loaded(model);
        hyperion::model::DecoderState& st = state_of(model, kvstate);
        check_tokens(tokens);
        HypStepResultOpaque& r = result_of(out_result);
        const auto smp = dec.prefill(st, tokens->tokens, tokens->count);
        write_result(r, smp, st, false);
    });
}

HypStatus hyp_decode_block(HypModel model, HypKvState kvstate, uint32_t n_tokens, HypStepResult out_result) {
    return abi_call("hyp_decode_block", [&] {
        hyperion::model::Decoder& dec = loaded(model);
        hyperion::model::DecoderState& st = state_of(model, kvstate);
        HypStepResultOpaque& r = result_of(out_result);
        const auto smp = dec.decode(st, n_tokens);
        write_result(r, smp, st, false);
    });
}

HypStatus hyp_prefill_chunk_sampled(HypModel model, HypKvState kvstate, const HypTokenStream* tokens,
                                    const HypSamplingConfig* config, HypStepResult out_result) {
    return abi_call("hyp_prefill_chunk_sampled", [&] {
        hyperion::model::Decoder& dec = loaded(model);
        hyperion::model::DecoderState& st = state_of(model, kvstate);
        check_tokens(tokens);
        HypStepResultOpaque& r = result_of(out_result);
        const bool greedy = hyperion::model::sampling_is_greedy(config, dec.geometry().vocab);
        const auto smp = dec.prefill(st, tokens->tokens, tokens->count, greedy ? nullptr : config);
        write_result(r, smp, st, true);
    });
}

HypStatus hyp_decode_block_sampled(HypModel model, HypKvState kvstate, uint32_t n_tokens,
                                   const HypSamplingConfig* config, HypStepResult out_result) {
    return abi_call("hyp_decode_block_sampled", [&] {
        hyperion::model::Decoder& dec = loaded(model);
        hyperion::model::DecoderState& st = state_of(model, kvstate);
        HypStepResultOpaque& r = result_of(out_result);
        const bool greedy = hyperion::model::sampling_is_greedy(config, dec.geometry().vocab);
        const auto smp = dec.decode(st, n_tokens, greedy ? nullptr : config);
        write_result(r, smp, st, true);
    });
}

HypStatus hyp_step_result_create(HypStepResult* out_result) {
    return abi_call("hyp_step_result_create", [&] {
        REQUIRE_ARG(out_result != nullptr, "create requires a non-null out handle");
        auto r = std::make_unique<HypStepResultOpaque>();
        r->magic = kStepResultMagic;
        *out_result = r.release();
    });
}

HypStatus hyp_step_result_free(HypStepResult* result) {
    return free_handle(result, kStepResultMagic);
}

HypStatus hyp_step_result_fields(HypStepResult result, HypStepResultFields* out_fields) {
    return abi_call("hyp_step_result_fields", [&] {
        const HypStepResultOpaque& r = result_of(result);
        REQUIRE_ARG(out_fields != nullptr, "out_fields is null");
        *out_fields = r.fields;
    });
}

namespace {
void fill_report(const hyperion::model::MemoryReport& r, HypMemoryReport* out) {
    out->weight_bytes = r.weight_bytes;
    out->norm_bytes = r.norm_bytes;
    out->kv_local_bytes = r.kv_local_bytes;
    out->kv_global_bytes = r.kv_global_bytes;
    out->state_bytes = r.state_bytes;
    out->scratch_bytes = r.scratch_bytes;
    out->dense_bf16_weight_bytes = r.dense_bf16_weight_bytes;
}
}  // namespace

HypStatus hyp_geometry_memory(const HypGeometryParams* geometry, HypMemoryReport* out) {
    return abi_call("hyp_geometry_memory", [&] {
        REQUIRE_ARG(geometry != nullptr && out != nullptr, "geometry and out must be non-null");
        fill_report(hyperion::model::plan_memory(hyperion::model::Geometry::from_abi(*geometry)), out);
    });
}

HypStatus hyp_model_memory(HypModel model, HypMemoryReport* out) {
    return abi_call("hyp_model_memory", [&] {
        hyperion::model::Decoder& dec = loaded(model);
        REQUIRE_ARG(out != nullptr, "out must be non-null");
        fill_report(dec.memory(), out);
    });
}

HypStatus hyp_model_forward_hidden(HypModel model, HypKvState kvstate, const uint32_t* ids, uint32_t count,
                                   uint32_t offset, uint16_t* hidden_out) {
    return abi_call("hyp_model_forward_hidden", [&] {
        hyperion::model::Decoder& dec = loaded(model);
        hyperion::model::DecoderState& st = state_of(model, kvstate);
        REQUIRE_ARG(ids != nullptr && hidden_out != nullptr, "ids and hidden_out must be non-null host pointers");
        dec.forward_hidden(st, ids, count, offset, hidden_out);
    });
}

}  // extern "C"

// QuantizedLinear on HIP: residency in the tiled layout and dispatch between the
// skinny decode kernel (m <= 4) and the prefill MFMA GEMM (the reference leaves this
// choice to MLX's qmv/qmm routing, native/hyperion_mlx/src/weights.h:14-17).
#include "qlinear.h"

#include "q4_layout.h"

#include <utility>

namespace hyperion::hip {

uint32_t device_compute_units() {
    static thread_local int cached_device = -1;
    static thread_local uint32_t cached_cus = 0;
    int dev = 0;
    HYP_HIP_CHECK(hipGetDevice(&dev));
    if (dev != cached_device) {
        int cus = 0;
        HYP_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        cached_cus = cus > 0 ? static_cast<uint32_t>(cus) : 1u;
        cached_device = dev;
    }
    return cached_cus;
}

}  // namespace hyperion::hip

namespace hyperion::model {

using hip::NativeError;

DeviceBuffer::DeviceBuffer(size_t bytes) : bytes_(bytes) {
    if (bytes == 0) return;
    const hipError_t err = hipMalloc(&ptr_, bytes);
    if (err != hipSuccess) {
        ptr_ = nullptr;
        throw NativeError(HYP_STATUS_INTERNAL, std::string("device allocation of ") + std::to_string(bytes) +
                                                   " bytes failed: " + hipGetErrorString(err));
    }
}

DeviceBuffer::~DeviceBuffer() {
    if (ptr_ != nullptr) {
        (void)hipFree(ptr_);
    }
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept
    : ptr_(std::exchange(other.ptr_, nullptr)), bytes_(std::exchange(other.bytes_, 0)) {}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
    if (this != &other) {
        if (ptr_ != nullptr) (void)hipFree(ptr_);
        ptr_ = std::exchange(other.ptr_, nullptr);
        bytes_ = std::exchange(other.bytes_, 0);
    }
    return *this;
}

namespace {

constexpr size_t align256(size_t v) { return (v + 255u) & ~size_t{255u}; }

// MLX-layout sizes: codes uint32 [n, k/8], scales and biases bf16 [n, k/64].
struct MlxSizes {
    size_t w, s, off_s, off_b, total;
};

MlxSizes mlx_sizes(uint32_t n, uint32_t k) {
    MlxSizes z{};
    z.w = static_cast<size_t>(n) * (k / 8u) * sizeof(uint32_t);
    z.s = static_cast<size_t>(n) * (k / 64u) * sizeof(uint16_t);
    z.off_s = align256(z.w);
    z.off_b = z.off_s + align256(z.s);
    z.total = z.off_b + align256(z.s);
    return z;
}

// One allocation holding the tiled layout: codes | scales and biases.
QuantizedLinear make_storage(uint32_t n, uint32_t k) {
    const hip::TiledDims d = hip::TiledDims::of(n, k);
    const size_t off_sb = align256(d.code_bytes());
    QuantizedLinear q;
    q.storage = DeviceBuffer(off_sb + align256(d.sb_bytes()));
    auto* base = static_cast<uint8_t*>(q.storage.data());
    q.mat.codes = reinterpret_cast<const uint4*>(base);
    q.mat.sb = reinterpret_cast<const uint2*>(base + off_sb);
    q.mat.n = n;
    q.mat.k = k;
    return q;
}

void tile_into(QuantizedLinear& q, const uint32_t* w, const uint16_t* s, const uint16_t* b, hipStream_t stream) {
    hip::launch_q4_tile(w, s, b, q.mat.n, q.mat.k, const_cast<uint4*>(q.mat.codes), const_cast<uint2*>(q.mat.sb),
                        stream);
}

}  // namespace

QuantizedLinear QuantizedLinear::from_host(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                           uint32_t n, uint32_t k) {
    QuantizedLinear q = make_storage(n, k);
    // Upload in MLX layout to a staging buffer, then tile on the device.
    const MlxSizes z = mlx_sizes(n, k);
    DeviceBuffer staging(z.total);
    auto* base = static_cast<uint8_t*>(staging.data());
    HYP_HIP_CHECK(hipMemcpy(base, w, z.w, hipMemcpyHostToDevice));
    HYP_HIP_CHECK(hipMemcpy(base + z.off_s, scales, z.s, hipMemcpyHostToDevice));
    HYP_HIP_CHECK(hipMemcpy(base + z.off_b, biases, z.s, hipMemcpyHostToDevice));
    tile_into(q, reinterpret_cast<const uint32_t*>(base), reinterpret_cast<const uint16_t*>(base + z.off_s),
              reinterpret_cast<const uint16_t*>(base + z.off_b), nullptr);
    HYP_HIP_CHECK(hipStreamSynchronize(nullptr));
    return q;
}

QuantizedLinear QuantizedLinear::from_device(const uint32_t* w, const uint16_t* scales,
                                             const uint16_t* biases, uint32_t n, uint32_t k,
                                             hipStream_t stream) {
    QuantizedLinear q = make_storage(n, k);
    tile_into(q, w, scales, biases, stream);
    return q;
}

void QuantizedLinear::export_mlx(uint32_t* w, uint16_t* scales, uint16_t* biases) const {
    const MlxSizes z = mlx_sizes(mat.n, mat.k);
    DeviceBuffer staging(z.total);
    auto* base = static_cast<uint8_t*>(staging.data());
    hip::launch_q4_untile(mat.codes, mat.sb, mat.n, mat.k, reinterpret_cast<uint32_t*>(base),
                          reinterpret_cast<uint16_t*>(base + z.off_s), reinterpret_cast<uint16_t*>(base + z.off_b),
                          nullptr);
    HYP_HIP_CHECK(hipStreamSynchronize(nullptr));
    HYP_HIP_CHECK(hipMemcpy(w, base, z.w, hipMemcpyDeviceToHost));
    HYP_HIP_CHECK(hipMemcpy(scales, base + z.off_s, z.s, hipMemcpyDeviceToHost));
    HYP_HIP_CHECK(hipMemcpy(biases, base + z.off_b, z.s, hipMemcpyDeviceToHost));
}

void QuantizedLinear::apply(const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream, Epilogue epi,
                            float cap_bf16) const {
    if (m == 0) return;
    if (hip::skinny_supported(m, mat.k, false)) {
        hip::launch_q4_skinny(mat, nullptr, x, m, y, epi, cap_bf16, 0u, stream);
        return;
    }
    hip::launch_q4_gemm(mat, x, m, y, stream);
    if (epi == Epilogue::kSoftcap) {
        hip::launch_softcap(y, cap_bf16, static_cast<uint64_t>(m) * mat.n, stream);
    }
}

void QuantizedLinear::apply_noalloc(const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream) const {
    if (m == 0) return;
    if (hip::skinny_supported(m, mat.k, false)) {
        hip::launch_q4_skinny(mat, nullptr, x, m, y, Epilogue::kNone, 0.0f, 0u, stream);
        return;
    }
    hip::launch_q4_gemm_noalloc(mat, x, m, y, stream);
}

void apply_group(const QuantizedLinear* const* linears, uint16_t* const* ys, uint32_t count, const uint16_t* x,
                 uint32_t m, const float* rms_eps, const uint16_t* norm_w, hipStream_t stream) {
    if (m == 0) return;
    const uint32_t k = linears[0]->mat.k;
    const hip::Q4Matrix* mats[hip::kSkinnyMaxGroup];
    for (uint32_t i = 0; i < count; ++i) mats[i] = &linears[i]->mat;
    if (rms_eps ? hip::skinny_norm_supported(m, k) : hip::skinny_supported(m, k, false)) {
        hip::launch_q4_skinny_group(mats, ys, count, x, m, rms_eps, norm_w, stream);
        return;
    }
    if (rms_eps == nullptr) {
        hip::launch_q4_gemm_group(mats, ys, count, x, m, stream);
        return;
    }
    // The normalised rows in a stream-ordered temporary, then the grouped GEMM.
    void* xn = nullptr;
    HYP_HIP_CHECK(hipMallocAsync(&xn, static_cast<size_t>(m) * k * sizeof(uint16_t), stream));
    try {
        hip::launch_rms_normalize(x, norm_w, m, k, *rms_eps, static_cast<uint16_t*>(xn), stream);
        hip::launch_q4_gemm_group(mats, ys, count, static_cast<const uint16_t*>(xn), m, stream);
    } catch (...) {
        (void)hipFreeAsync(xn, stream);
        throw;
    }
    HYP_HIP_CHECK(hipFreeAsync(xn, stream));
}

void mlp_gate_up(const QuantizedLinear& gate, const QuantizedLinear& up, const uint16_t* x, uint32_t m,
                 uint16_t* h, hipStream_t stream) {
    if (m == 0) return;
    if (hip::skinny_supported(m, gate.mat.k, true)) {
        hip::launch_q4_skinny(gate.mat, &up.mat, x, m, h, Epilogue::kNone, 0.0f, 0u, stream);
        return;
    }
    // One dual GEMM: each wave accumulates a gate tile and the matching up tile and the
    // epilogue stores bf16(gelu(gate) * up) (no gate/up temporaries, no elementwise pass).
    hip::launch_q4_gemm_gate_up(gate.mat, up.mat, x, m, h, stream);
}

}  // namespace hyperion::model

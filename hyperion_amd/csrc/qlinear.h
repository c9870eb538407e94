// Host-side mirror of the reference's quantized-linear layer and weight
// residency, re-expressed on device-resident HIP buffers.
//
//   QuantizedLinear   native/hyperion_mlx/src/weights.h:18-37
//   LayerWeights      native/hyperion_mlx/src/weights_loader.h:24-44 (projections only)
//   ModelWeights      native/hyperion_mlx/src/weights_loader.h:49-66 (Q4 tables only)
//
// The reference keeps MLX arrays that are lazily mmapped and moved to the GPU on first
// use (weights_loader.h:70-79). Here every projection is copied to HBM once at load
// time and stored in the tiled layout of q4_layout.h, which the kernels read; MLX's
// layout stays the format at the boundary (upload, export).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace hyperion::model {

using hip::Epilogue;
using hip::Q4Matrix;

// One device allocation, freed on destruction.
class DeviceBuffer {
  public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes);
    ~DeviceBuffer();
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& other) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;

    [[nodiscard]] void* data() const noexcept { return ptr_; }
    [[nodiscard]] size_t bytes() const noexcept { return bytes_; }

  private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
};

// One Q4/g64 projection [out_features = n, in_features = k] resident in HBM.
struct QuantizedLinear {
    DeviceBuffer storage;   // tiled codes | tiled scales and biases, 256-byte aligned
    Q4Matrix mat;           // codes/sb point into storage; w/scales/biases are null
    int group_size = 64;
    int bits = 4;

    // Copy from host (MLX layout, synchronous) or from device pointers (MLX layout;
    // stream-ordered: the inputs must stay valid until the stream has run the copy).
    static QuantizedLinear from_host(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                     uint32_t n, uint32_t k);
    static QuantizedLinear from_device(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                       uint32_t n, uint32_t k, hipStream_t stream);

    // Copy back to host in MLX layout (synchronous).
    void export_mlx(uint32_t* w, uint16_t* scales, uint16_t* biases) const;

    // y[m, n] = x[m, k] . dequant(W)^T (weights.h:26-37); device pointers.
    void apply(const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream,
               Epilogue epi = Epilogue::kNone, float cap_bf16 = 0.0f) const;

    // apply() without any allocation: the same kernels and splits, with split-k partials
    // in the library's fixed device scratch (launch_q4_gemm_noalloc), so the results are
    // the same bits. Throws INVALID_ARGUMENT when a call's partials exceed the scratch.
    void apply_noalloc(const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream) const;
};

// gelu_tanh(gate(x)) * up(x) (forward.cc:338-343 minus the down projection).
void mlp_gate_up(const QuantizedLinear& gate, const QuantizedLinear& up, const uint16_t* x, uint32_t m,
                 uint16_t* h, hipStream_t stream);

// ys[i] = x . dequant(W_i)^T for up to three projections sharing x and k (the attention
// q/k/v of one layer, forward.cc:395,399,409): one launch at decode sizes. With rms_eps
// non-null, x is first rms-normalised with the bf16 weight norm_w [k] (or none, norm_w
// null; the same bits as launch_rms_normalize); at decode
// sizes inside the launch, otherwise into a stream-ordered temporary.
void apply_group(const QuantizedLinear* const* linears, uint16_t* const* ys, uint32_t count, const uint16_t* x,
                 uint32_t m, const float* rms_eps, const uint16_t* norm_w, hipStream_t stream);

enum class LayerType { Sliding, Full };

// The bf16 vectors of a layer (weights_loader.cc:142-148), device-resident: the four
// sandwich norms [hidden], q_norm and k_norm [head_dim], layer_scalar [1].
enum class LayerNorm : int {
    kInput = 0,
    kPostAttention = 1,
    kPreFeedforward = 2,
    kPostFeedforward = 3,
    kQ = 4,
    kK = 5,
    kScalar = 6,
};
constexpr int kLayerNorms = 7;

struct LayerWeights {
    QuantizedLinear q_proj;
    QuantizedLinear k_proj;
    std::optional<QuantizedLinear> v_proj;   // absent on global (K = V) layers
    QuantizedLinear o_proj;
    QuantizedLinear gate_proj;
    QuantizedLinear up_proj;
    QuantizedLinear down_proj;
    LayerType kind = LayerType::Sliding;
    DeviceBuffer norms[kLayerNorms];          // empty when the artifact has none
    uint32_t norm_len[kLayerNorms] = {};

    [[nodiscard]] const uint16_t* norm(LayerNorm which) const noexcept {
        return static_cast<const uint16_t*>(norms[static_cast<int>(which)].data());
    }
};

struct ModelWeights {
    QuantizedLinear embed;   // tied: also the LM head (forward.cc:137-152)
    std::vector<LayerWeights> layers;
    DeviceBuffer final_norm;   // [hidden] bf16 (weights_loader.cc:108); empty when absent
    uint32_t final_norm_len = 0;
    bool has_norms = false;    // every layer's vectors and the final norm were loaded
};

// Host phase of load_model_weights: maps every shard, resolves and shape-checks
// each projection. Touches no device, so artifact errors surface without a GPU.
class ModelManifest {
  public:
    ModelManifest(const std::string& dir, uint32_t num_layers);
    ~ModelManifest();
    ModelManifest(const ModelManifest&) = delete;
    ModelManifest& operator=(const ModelManifest&) = delete;
    [[nodiscard]] uint32_t num_layers() const noexcept;
    // Device phase: copy every planned projection into HBM.
    [[nodiscard]] ModelWeights upload() const;

  private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// load_model_weights (weights_loader.cc:71-153) for the Q4 projections and the
// embed table. num_layers == 0 loads every layer the shards hold.
ModelWeights load_model_weights(const std::string& dir, uint32_t num_layers);

}  // namespace hyperion::model

// Weight residency: MLX safetensors shards -> device-resident Q4 projections.
// Follows load_model_weights (native/hyperion_mlx/src/weights_loader.cc:71-153):
// every *.safetensors shard of the directory, sorted, merged into one name map;
// per-layer projections under the mlx-lm names (weights_loader.cc:13-17,132-141);
// a layer without v_proj is a global (K = V) layer (weights_loader.cc:47-49,116-129).
#include <algorithm>
#include <filesystem>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "qlinear.h"
#include "safetensors.h"

namespace hyperion::model {

using hip::NativeError;

namespace {

constexpr const char* kLayerPrefix = "language_model.model.layers.";
constexpr const char* kEmbedBase = "language_model.model.embed_tokens";

struct Located {
    const SafetensorsFile* file;
    const TensorInfo* info;
};

using NameMap = std::unordered_map<std::string, Located>;

const Located& require_tensor(const NameMap& tensors, const std::string& name) {
    const auto it = tensors.find(name);
    if (it == tensors.end()) {
        throw NativeError(HYP_STATUS_INVALID_ARGUMENT, "weight manifest is missing tensor: " + name);
    }
    return it->second;
}

std::string layer_tensor(size_t layer, const std::string& suffix) {
    return std::string(kLayerPrefix) + std::to_string(layer) + "." + suffix;
}

// One projection located and shape-checked on the host.
struct ProjPlan {
    const Located* w = nullptr;
    const Located* s = nullptr;
    const Located* b = nullptr;
    uint32_t n = 0;
    uint32_t k = 0;
};

// make_proj (weights_loader.cc:33-45) with the shape checks of weights_test.cc:76-82:
// in_features = scales.shape(1) * group_size and the packed width is in_features / 8.
ProjPlan plan_proj(const NameMap& tensors, const std::string& base) {
    const Located& w = require_tensor(tensors, base + ".weight");
    const Located& s = require_tensor(tensors, base + ".scales");
    const Located& b = require_tensor(tensors, base + ".biases");
    auto bad = [&](const std::string& why) {
        throw NativeError(HYP_STATUS_INVALID_ARGUMENT, base + ": " + why);
    };
    if (w.info->dtype != "U32") bad("weight dtype " + w.info->dtype + " is not U32 (affine Q4)");
    if (s.info->dtype != "BF16" || b.info->dtype != "BF16") bad("scales/biases must be BF16");
    if (w.info->shape.size() != 2 || s.info->shape.size() != 2 || b.info->shape != s.info->shape) {
        bad("expected 2-D weight [out, in/8] and matching 2-D scales/biases [out, in/64]");
    }
    const int64_t n = w.info->shape[0];
    const int64_t k = s.info->shape[1] * 64;
    if (s.info->shape[0] != n) bad("scales rows differ from weight rows");
    if (w.info->shape[1] * 8 != k) bad("packed width does not match group_size 64 / bits 4");
    if (n <= 0 || k <= 0 || n > 0xffffffffLL || k > 0xffffffffLL) bad("empty or oversized projection");
    return ProjPlan{&w, &s, &b, static_cast<uint32_t>(n), static_cast<uint32_t>(k)};
}

QuantizedLinear upload(const ProjPlan& p) {
    return QuantizedLinear::from_host(reinterpret_cast<const uint32_t*>(p.w->file->data(*p.w->info)),
                                      reinterpret_cast<const uint16_t*>(p.s->file->data(*p.s->info)),
                                      reinterpret_cast<const uint16_t*>(p.b->file->data(*p.b->info)), p.n, p.k);
}

// The layer's bf16 vectors, in LayerNorm order (weights_loader.cc:142-148).
constexpr const char* kNormNames[kLayerNorms] = {
    "input_layernorm.weight",          "post_attention_layernorm.weight", "pre_feedforward_layernorm.weight",
    "post_feedforward_layernorm.weight", "self_attn.q_norm.weight",         "self_attn.k_norm.weight",
    "layer_scalar",
};
constexpr const char* kFinalNorm = "language_model.model.norm.weight";

// A 1-D bf16 vector, or null when absent.
const Located* plan_vector(const NameMap& tensors, const std::string& name) {
    const auto it = tensors.find(name);
    if (it == tensors.end()) return nullptr;
    const TensorInfo& t = *it->second.info;
    if (t.dtype != "BF16" || t.shape.size() != 1 || t.shape[0] <= 0 || t.shape[0] > 0xffffffffLL) {
        throw NativeError(HYP_STATUS_INVALID_ARGUMENT, name + ": expected a non-empty 1-D BF16 vector");
    }
    return &it->second;
}

struct LayerPlan {
    ProjPlan proj[7];   // q, k, v, o, gate, up, down
    bool sliding = true;
    const Located* norm[kLayerNorms] = {};
};

DeviceBuffer upload_vector(const Located& v) {
    DeviceBuffer buf(v.info->end - v.info->begin);
    HYP_HIP_CHECK(hipMemcpy(buf.data(), v.file->data(*v.info), buf.bytes(), hipMemcpyHostToDevice));
    return buf;
}

}  // namespace

struct ModelManifest::Impl {
    std::vector<std::unique_ptr<SafetensorsFile>> files;
    NameMap tensors;
    ProjPlan embed;
    std::vector<LayerPlan> layers;
    const Located* final_norm = nullptr;
    bool has_norms = false;
};

ModelManifest::ModelManifest(const std::string& dir, uint32_t num_layers) : impl_(std::make_unique<Impl>()) {
    namespace fs = std::filesystem;
    std::error_code ec;
    if (!fs::is_directory(dir, ec)) {
        throw NativeError(HYP_STATUS_NOT_FOUND, "weights artifact directory does not exist: " + dir);
    }
    std::vector<fs::path> shards;
    for (const auto& entry : fs::directory_iterator(dir)) {
        if (entry.is_regular_file() && entry.path().extension() == ".safetensors") {
            shards.push_back(entry.path());
        }
    }
    std::sort(shards.begin(), shards.end());
    if (shards.empty()) {
        throw NativeError(HYP_STATUS_NOT_FOUND, "no .safetensors shards found in " + dir);
    }
    for (const auto& shard : shards) {
        impl_->files.push_back(std::make_unique<SafetensorsFile>(shard.string()));
        for (const auto& [name, info] : impl_->files.back()->tensors()) {
            impl_->tensors.emplace(name, Located{impl_->files.back().get(), &info});
        }
    }
    const NameMap& tensors = impl_->tensors;
    size_t available = 0;
    while (tensors.count(layer_tensor(available, "self_attn.q_proj.weight")) != 0) ++available;
    const size_t want = num_layers == 0 ? available : num_layers;
    if (want > available) {
        throw NativeError(HYP_STATUS_INVALID_ARGUMENT, "requested " + std::to_string(want) +
                                                           " layers but the shards hold " +
                                                           std::to_string(available));
    }
    impl_->embed = plan_proj(tensors, kEmbedBase);
    for (size_t i = 0; i < want; ++i) {
        LayerPlan lp;
        lp.sliding = tensors.count(layer_tensor(i, "self_attn.v_proj.weight")) != 0;
        const std::string attn = layer_tensor(i, "self_attn.");
        lp.proj[0] = plan_proj(tensors, attn + "q_proj");
        lp.proj[1] = plan_proj(tensors, attn + "k_proj");
        if (lp.sliding) lp.proj[2] = plan_proj(tensors, attn + "v_proj");
        lp.proj[3] = plan_proj(tensors, attn + "o_proj");
        lp.proj[4] = plan_proj(tensors, layer_tensor(i, "mlp.gate_proj"));
        lp.proj[5] = plan_proj(tensors, layer_tensor(i, "mlp.up_proj"));
        lp.proj[6] = plan_proj(tensors, layer_tensor(i, "mlp.down_proj"));
        for (int j = 0; j < kLayerNorms; ++j) lp.norm[j] = plan_vector(tensors, layer_tensor(i, kNormNames[j]));
        impl_->layers.push_back(lp);
    }
    impl_->final_norm = plan_vector(tensors, kFinalNorm);
    bool all = impl_->final_norm != nullptr;
    for (const LayerPlan& lp : impl_->layers) {
        for (const Located* v : lp.norm) all = all && v != nullptr;
    }
    impl_->has_norms = all;
}

ModelManifest::~ModelManifest() = default;

uint32_t ModelManifest::num_layers() const noexcept { return static_cast<uint32_t>(impl_->layers.size()); }

ModelWeights ModelManifest::upload() const {
    ModelWeights weights;
    weights.embed = hyperion::model::upload(impl_->embed);
    weights.layers.reserve(impl_->layers.size());
    for (const LayerPlan& lp : impl_->layers) {
        LayerWeights lw;
        lw.q_proj = hyperion::model::upload(lp.proj[0]);
        lw.k_proj = hyperion::model::upload(lp.proj[1]);
        if (lp.sliding) lw.v_proj = hyperion::model::upload(lp.proj[2]);
        lw.o_proj = hyperion::model::upload(lp.proj[3]);
        lw.gate_proj = hyperion::model::upload(lp.proj[4]);
        lw.up_proj = hyperion::model::upload(lp.proj[5]);
        lw.down_proj = hyperion::model::upload(lp.proj[6]);
        lw.kind = lp.sliding ? LayerType::Sliding : LayerType::Full;
        for (int j = 0; j < kLayerNorms; ++j) {
            if (lp.norm[j] == nullptr) continue;
            lw.norms[j] = upload_vector(*lp.norm[j]);
            lw.norm_len[j] = static_cast<uint32_t>(lp.norm[j]->info->shape[0]);
        }
        weights.layers.push_back(std::move(lw));
    }
    if (impl_->final_norm != nullptr) {
        weights.final_norm = upload_vector(*impl_->final_norm);
        weights.final_norm_len = static_cast<uint32_t>(impl_->final_norm->info->shape[0]);
    }
    weights.has_norms = impl_->has_norms;
    return weights;
}

ModelWeights load_model_weights(const std::string& dir, uint32_t num_layers) {
    return ModelManifest(dir, num_layers).upload();
}

}  // namespace hyperion::model

// Host side of temperature sampling: the configuration check, the uniform of the draw and
// the per-step RNG advance of the reference's sampled entry points.
#pragma once

#include <cmath>
#include <cstdint>
#include <limits>
#include <random>

#include "common.h"
#include "hyperion_hip.h"
#include "kernels.h"

namespace hyperion::model {

// validate_sampling_config (model.cc:234-257): true for the greedy path (NULL config or
// temperature 0); INVALID_ARGUMENT for a malformed config; false for a draw.
inline bool sampling_is_greedy(const HypSamplingConfig* c, uint32_t vocab) {
    using hip::NativeError;
    if (c == nullptr || c->temperature == 0.0f) return true;
    auto require = [](bool ok, const char* what) {
        if (!ok) throw NativeError(HYP_STATUS_INVALID_ARGUMENT, what);
    };
    require(!(c->temperature < 0.0f), "sampling temperature must be >= 0 (0 = greedy)");
    require(c->top_k >= 0, "sampling top_k must be >= 0 (0 = disabled)");
    require(c->top_k == 0 || static_cast<uint64_t>(c->top_k) <= vocab, "sampling top_k exceeds the vocabulary size");
    require(std::isnan(c->top_p) || (c->top_p >= 0.0f && c->top_p <= 1.0f),
            "sampling top_p must be in [0, 1] (0 = disabled)");
    require(c->min_p >= 0.0f && c->min_p < 1.0f, "sampling min_p must be in [0, 1) (0 = disabled)");
    return false;
}

// The reference draws u = std::uniform_real_distribution<float>(0, sz)(std::mt19937_64(state))
// (forward.cc:289-293); libstdc++ forms that as generate_canonical<float, 24>(rng) * sz + 0.
// The host computes the canonical value, the device scales it by its kept total sz.
inline float sampling_uniform(uint64_t state) {
    std::mt19937_64 rng(state);
    return std::generate_canonical<float, std::numeric_limits<float>::digits>(rng);
}

// hyp_decode_block_sampled's RNG state after each step (model.cc:926, :944): the block
// starts from the config's seed.
inline uint64_t advance_sampling_state(uint64_t state) {
    return state * 6364136223846793005ULL + 1442695040888963407ULL;
}

// The configuration part of SampleParams (forward.cc:225-226: t = logit * (1 / temperature)).
inline hip::SampleParams sampling_params(const HypSamplingConfig& c) {
    hip::SampleParams p{};
    p.inv_temp = 1.0f / c.temperature;
    p.top_p = c.top_p;
    p.min_p = c.min_p;
    p.top_k = c.top_k;
    p.n_uniform = 0u;
    p.step = 0u;
    return p;
}

}  // namespace hyperion::model

// TEST INFRASTRUCTURE ONLY: the reference's host sampler, ForwardPass::sample_stochastic
// (native/hyperion_mlx/src/forward.cc:225-301), restated over the C++ standard library it
// relies on (libstdc++ here): the logits scaled by 1/temperature in fp32, a std::exp
// softmax summed in index order, the nucleus by a std::sort of the probabilities, min-p
// against the largest probability, top-k by a std::partial_sort of the scaled logits, and
// the inverse-CDF draw with u from std::uniform_real_distribution<float>(0, sz) over a
// std::mt19937_64 seeded with the RNG state. The tests use it to pin the oracle's
// restatement of the HIP kernels' defined algorithm, and the RNG helpers below to pin the
// uniform the library hands those kernels.
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <numeric>
#include <random>
#include <vector>

// std::generate_canonical<float, 24> of a std::mt19937_64 seeded with `state`: the draw
// uniform_real_distribution<float> scales (libstdc++: u = canon * (b - a) + a).
extern "C" float stl_canonical_mt19937_64(uint64_t state) {
    std::mt19937_64 rng(state);
    return std::generate_canonical<float, std::numeric_limits<float>::digits>(rng);
}

// One draw of std::uniform_real_distribution<float>(0, b) from a std::mt19937_64 seeded with
// `state`, as the reference draws u.
extern "C" float stl_uniform_real_mt19937_64(uint64_t state, float b) {
    std::mt19937_64 rng(state);
    std::uniform_real_distribution<float> uni(0.0F, b);
    return uni(rng);
}

// The n-th output (n >= 1) of std::mt19937_64 seeded with `seed`.
extern "C" uint64_t stl_mt19937_64_nth(uint64_t seed, uint64_t n) {
    std::mt19937_64 rng(seed);
    uint64_t v = 0;
    for (uint64_t i = 0; i < n; ++i) v = rng();
    return v;
}

// The reference's draw over n fp32 logits. kept[i] (if non-null) = 1 where token i survives
// the three filters; *u_out (if non-null) = the uniform it draws. Returns the token.
extern "C" uint32_t stl_sample_stochastic(const float* src, uint32_t n, float temperature, int32_t top_k, float top_p,
                                          float min_p, uint64_t rng_state, uint8_t* kept, float* u_out) {
    constexpr float kNegInf = -std::numeric_limits<float>::infinity();
    std::vector<float> t(src, src + n);
    const float inv_temp = 1.0F / temperature;
    for (float& v : t) v *= inv_temp;

    float top = kNegInf;
    for (float v : t) top = std::max(top, v);
    std::vector<float> prob(n);
    float z = 0.0F;
    for (uint32_t i = 0; i < n; ++i) {
        prob[i] = std::exp(t[i] - top);
        z += prob[i];
    }
    if (z > 0.0F) {
        for (float& p : prob) p /= z;
    }

    std::vector<uint32_t> order(n);
    if (top_p > 0.0F && top_p <= 1.0F) {
        std::iota(order.begin(), order.end(), 0u);
        std::sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return prob[a] > prob[b]; });
        std::vector<uint8_t> nucleus(n, 0);
        float mass = 0.0F;
        for (uint32_t i : order) {
            nucleus[i] = 1;
            mass += prob[i];
            if (mass >= top_p) break;
        }
        for (uint32_t i = 0; i < n; ++i) {
            if (nucleus[i] == 0) t[i] = kNegInf;
        }
    }
    if (min_p > 0.0F && min_p < 1.0F) {
        float pmax = 0.0F;
        for (float p : prob) pmax = std::max(pmax, p);
        const float floor_p = min_p * pmax;
        for (uint32_t i = 0; i < n; ++i) {
            if (prob[i] < floor_p) t[i] = kNegInf;
        }
    }
    if (top_k > 0 && static_cast<uint32_t>(top_k) < n) {
        std::iota(order.begin(), order.end(), 0u);
        std::partial_sort(order.begin(), order.begin() + top_k, order.end(),
                          [&](uint32_t a, uint32_t b) { return t[a] > t[b]; });
        std::vector<uint8_t> keep(n, 0);
        for (int32_t i = 0; i < top_k; ++i) keep[order[static_cast<size_t>(i)]] = 1;
        for (uint32_t i = 0; i < n; ++i) {
            if (keep[i] == 0) t[i] = kNegInf;
        }
    }
    if (kept != nullptr) {
        for (uint32_t i = 0; i < n; ++i) kept[i] = t[i] != kNegInf ? 1 : 0;
    }

    float fmax = kNegInf;
    for (float v : t) fmax = std::max(fmax, v);
    std::vector<float> w(n);
    float sz = 0.0F;
    for (uint32_t i = 0; i < n; ++i) {
        w[i] = t[i] == kNegInf ? 0.0F : std::exp(t[i] - fmax);
        sz += w[i];
    }
    std::mt19937_64 rng(rng_state);
    std::uniform_real_distribution<float> uni(0.0F, sz);
    const float u = uni(rng);
    if (u_out != nullptr) *u_out = u;
    float run = 0.0F;
    uint32_t arg = 0;
    for (uint32_t i = 0; i < n; ++i) {
        run += w[i];
        arg = i;
        if (u <= run) break;
    }
    return arg;
}

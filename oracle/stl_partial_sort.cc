// TEST INFRASTRUCTURE ONLY: libstdc++'s std::partial_sort called the way the greedy
// epilogue calls it (native/hyperion_mlx/src/model.cc:278-288): the indices 0..n-1 of an
// fp32 row ordered by p[a] > p[b], the first min(k, n) kept. The tests use it to pin
// orc_sample_topk_bf16 to the library algorithm the reference relies on.
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <numeric>
#include <vector>

extern "C" uint32_t stl_partial_sort_topk(const float* p, int64_t n, uint32_t k, uint32_t* ids) {
    std::vector<uint32_t> idx(static_cast<size_t>(n > 0 ? n : 0));
    std::iota(idx.begin(), idx.end(), 0u);
    const size_t mid = std::min<size_t>(k, idx.size());
    std::partial_sort(idx.begin(), idx.begin() + static_cast<std::ptrdiff_t>(mid), idx.end(),
                      [&](uint32_t a, uint32_t b) { return p[a] > p[b]; });
    for (size_t i = 0; i < mid; ++i) ids[i] = idx[i];
    return static_cast<uint32_t>(mid);
}

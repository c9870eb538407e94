// Greedy sampling on the device: ForwardPass::sample_greedy
// (native/hyperion_mlx/src/forward.cc:162-189) without the host copy of the logits.
//
// The reference converts the last row of bf16 logits to fp32 on the CPU and scans it
// in index order: v > top1 moves top1 to top2 and takes (v, i); otherwise v > top2
// raises top2. So the token is the first index of the largest value, NaN values are
// skipped, an all -inf / NaN / empty row yields token 0, and top2 is the largest value
// other than the winning element (a tie at the maximum makes top2 = top1). near_tie is
// (top1 - top2) < 0.5 in fp32.
//
// Here a row is cut into up to 64 slices of whole 8-value chunks (about 4096 values each,
// one workgroup per slice): each thread scans its elements in index order with the
// reference's rule, then states merge exactly (the larger top1 wins, on equal top1 the
// lower index; the loser's top1 becomes a candidate for top2) across each wave with lane
// shuffles and across the waves in LDS; the slice states go to a small workspace and a
// second launch (one wave per row) merges them the same way. The row is read once
// (16-byte loads when the row is 16-byte aligned and vocab % 8 == 0).
//
// The greedy epilogue's top-k sidecar (native/hyperion_mlx/src/model.cc:272-288; k =
// HYP_TOP_K_LOGPROBS = 8) replaces the reference's host copy of the row and its
// std::partial_sort of the indices by p[a] > p[b]. partial_sort leaves equal values in an
// order of the library's choosing (and NaN breaks its comparator), so the order here is
// defined: larger value first (-0 == +0), then the lower index; NaN after every number,
// lower index first. A row is cut into slices of up to 65536 values (about 2048, at most
// 128 slices, one workgroup each). Within a slice each value becomes a 32-bit key that
// sorts in exactly that order - a 16-bit order image of its bf16 value (NaN lowest, -0
// folded onto +0) above 0xFFFF minus its offset in the slice - so a compare-exchange is
// one max and one min. Each thread sorts 8-value chunks with a 19-comparator network and
// merges them into its list of the 8 largest (bitonic: elementwise maximum against the
// other list reversed, then three compare-exchange layers); lists merge the same way in
// a butterfly across the wave, then across the waves, and a second launch merges the
// slices' lists. The winners' bits are re-read from the row for the values, so -0 and NaN
// payloads come back as stored. The greedy token, logit and near_tie follow from the
// first two entries (the first index of the largest value, and the largest other value).
#include <algorithm>
#include <cstdint>

#include "common.h"
#include "kernels.h"

namespace hyperion::hip {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kNone = 0xFFFFFFFFu;
constexpr uint32_t kMaxParts = 64;        // workgroups per row
constexpr uint32_t kWorkspaceRows = 64;   // rows per pair of launches

struct Top2 {
    float v1;
    uint32_t i1;   // kNone until an element > -inf is seen
    float v2;
};

__device__ __forceinline__ float bf16_to_f32(uint32_t bits) { return __uint_as_float(bits << 16); }

// The reference's per-element step (forward.cc:177-185).
__device__ __forceinline__ void scan_value(Top2& t, float v, uint32_t i) {
    if (v > t.v1) {
        t.v2 = t.v1;
        t.v1 = v;
        t.i1 = i;
    } else if (v > t.v2) {
        t.v2 = v;
    }
}

// Two disjoint index sets' states -> the state of their union (exact: no NaN is ever
// stored, and the first index of the maximum wins).
__device__ __forceinline__ Top2 merge(const Top2& a, const Top2& b) {
    const bool take_b = b.v1 > a.v1 || (b.v1 == a.v1 && b.i1 < a.i1);
    Top2 w = take_b ? b : a;
    w.v2 = fmaxf(w.v2, take_b ? a.v1 : b.v1);
    return w;
}

__device__ __forceinline__ Top2 shfl_xor(const Top2& t, int mask) {
    Top2 o;
    o.v1 = __shfl_xor(t.v1, mask, 64);
    o.i1 = static_cast<uint32_t>(__shfl_xor(static_cast<int>(t.i1), mask, 64));
    o.v2 = __shfl_xor(t.v2, mask, 64);
    return o;
}

__device__ __forceinline__ void scan_chunk(Top2& t, const uint4& c, uint32_t first) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        scan_value(t, bf16_to_f32(w[j] & 0xFFFFu), first + 2u * j);
        scan_value(t, bf16_to_f32(w[j] >> 16), first + 2u * j + 1u);
    }
}

// Pass 1: workgroup (p, r) scans elements [p span, min((p + 1) span, vocab)) of row r
// (span % 8 == 0) and stores its state in part[r * parts + p].
template <bool VEC>
__global__ __launch_bounds__(kThreads) void sample_partial_kernel(const uint16_t* __restrict__ logits, uint32_t vocab,
                                                                  uint32_t span, Top2* __restrict__ part) {
    const uint32_t p = blockIdx.x;
    const uint32_t row = blockIdx.y;
    const uint16_t* x = logits + static_cast<size_t>(row) * vocab;
    const uint32_t e0 = p * span;
    const uint32_t e1 = e0 < vocab ? min(e0 + span, vocab) : e0;
    Top2 t{-__builtin_huge_valf(), kNone, -__builtin_huge_valf()};
    if (VEC) {
        // Thread t scans chunks t, t + kThreads, ... of the slice (8 values each,
        // increasing index), all of its chunks loaded before any is scanned.
        const uint4* xv = reinterpret_cast<const uint4*>(x + e0);
        const uint32_t chunks = (e1 - e0) / 8u;
        constexpr uint32_t kBatch = 4;
        for (uint32_t base = threadIdx.x; base < chunks; base += kBatch * kThreads) {
            uint4 c[kBatch];
#pragma unroll
            for (uint32_t j = 0; j < kBatch; ++j) {
                const uint32_t ci = base + j * kThreads;
                c[j] = ci < chunks ? xv[ci] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (uint32_t j = 0; j < kBatch; ++j) {
                const uint32_t ci = base + j * kThreads;
                if (ci < chunks) scan_chunk(t, c[j], e0 + ci * 8u);
            }
        }
    } else {
        for (uint32_t i = e0 + threadIdx.x; i < e1; i += kThreads) scan_value(t, bf16_to_f32(x[i]), i);
    }

#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) t = merge(t, shfl_xor(t, mask));
    __shared__ Top2 waves[kThreads / 64];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    if (lane == 0) waves[wave] = t;
    __syncthreads();
    if (threadIdx.x == 0) {
        Top2 u = waves[0];
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) u = merge(u, waves[w]);
        part[static_cast<size_t>(row) * gridDim.x + p] = u;
    }
}

// Pass 2: one wave per row merges the row's `parts` states (parts <= 64) and writes
// the sample.
__global__ __launch_bounds__(64) void sample_merge_kernel(const Top2* __restrict__ part, uint32_t parts,
                                                          HypGreedySample* __restrict__ out) {
    const uint32_t row = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    Top2 u = lane < parts ? part[static_cast<size_t>(row) * parts + lane]
                          : Top2{-__builtin_huge_valf(), kNone, -__builtin_huge_valf()};
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) u = merge(u, shfl_xor(u, mask));
    if (lane == 0) {
        HypGreedySample r;
        r.token_id = u.i1 == kNone ? 0u : u.i1;
        r.logit = u.v1;
        r.near_tie = (u.v1 - u.v2) < 0.5f ? 1u : 0u;
        out[row] = r;
    }
}

// ---------------------------------------------------------------- top-k sidecar
constexpr uint32_t kTopKParts = 128;      // workgroups per row, at most
constexpr uint32_t kTopKSpan = 2048;      // values per workgroup aimed at (one 8-value chunk a thread)
constexpr uint32_t kTopKMaxSpan = 65536;  // local offsets fit 16 bits
constexpr uint32_t kTopKRows = 8;         // rows per pair of launches
static_assert(kTopKRows * kTopKParts * kHypTopK * sizeof(uint32_t) <= kMaxParts * kWorkspaceRows * sizeof(Top2),
              "the top-k slices must fit the stream workspace");

// Order image of a bf16 value in 1..0xFF81: NaN 1, -inf 0x80, +inf 0xFF81; -0 folded onto
// +0. 0 is left for "no element".
__device__ __forceinline__ uint32_t order_image(uint32_t b) {
    if ((b & 0x7FFFu) > 0x7F80u) return 1u;
    const uint32_t c = b == 0x8000u ? 0u : b;
    return ((c & 0x8000u) ? (~c & 0xFFFFu) : (c | 0x8000u)) + 1u;
}
constexpr uint32_t kImageNegInf = 0x80u;

// Slice key of the value with bf16 bits b at local offset off (< 2^16): larger = earlier.
__device__ __forceinline__ uint32_t slice_key(uint32_t b, uint32_t off) {
    return (order_image(b) << 16) | (0xFFFFu - off);
}

// kHypTopK distinct keys, descending; 0 = empty.
struct KeyList {
    uint32_t k[kHypTopK];
};

__device__ __forceinline__ void compare_exchange(uint32_t& a, uint32_t& b) {
    const uint32_t hi = max(a, b);
    b = min(a, b);
    a = hi;
}

// Batcher's odd-even merge sort of 8 keys, descending (19 comparators in 7 layers).
__device__ __forceinline__ void sort8(KeyList& v) {
    compare_exchange(v.k[0], v.k[1]); compare_exchange(v.k[2], v.k[3]);
    compare_exchange(v.k[4], v.k[5]); compare_exchange(v.k[6], v.k[7]);
    compare_exchange(v.k[0], v.k[2]); compare_exchange(v.k[1], v.k[3]);
    compare_exchange(v.k[4], v.k[6]); compare_exchange(v.k[5], v.k[7]);
    compare_exchange(v.k[1], v.k[2]); compare_exchange(v.k[5], v.k[6]);
    compare_exchange(v.k[0], v.k[4]); compare_exchange(v.k[3], v.k[7]);
    compare_exchange(v.k[1], v.k[5]); compare_exchange(v.k[2], v.k[6]);
    compare_exchange(v.k[1], v.k[4]); compare_exchange(v.k[3], v.k[6]);
    compare_exchange(v.k[2], v.k[4]); compare_exchange(v.k[3], v.k[5]);
    compare_exchange(v.k[3], v.k[4]);
}

// The kHypTopK largest of two descending lists of distinct keys, descending: the
// elementwise maximum of a and b reversed is a bitonic sequence holding them, and three
// half-cleaner layers sort it.
__device__ __forceinline__ KeyList merge_lists(const KeyList& a, const KeyList& b) {
    KeyList c;
#pragma unroll
    for (uint32_t i = 0; i < kHypTopK; ++i) c.k[i] = max(a.k[i], b.k[kHypTopK - 1 - i]);
#pragma unroll
    for (uint32_t stride = kHypTopK / 2; stride >= 1; stride /= 2) {
#pragma unroll
        for (uint32_t i = 0; i < kHypTopK; ++i) {
            if ((i & stride) == 0u) compare_exchange(c.k[i], c.k[i + stride]);
        }
    }
    return c;
}

// The kHypTopK largest keys over the wave's lists, in every lane: a butterfly of list
// merges (keys of different lanes are distinct, so both partners of a level hold the
// same merged list).
__device__ __forceinline__ KeyList wave_top(const KeyList& l) {
    KeyList r = l;
#pragma unroll
    for (int mask = 1; mask <= 32; mask <<= 1) {
        KeyList o;
#pragma unroll
        for (uint32_t j = 0; j < kHypTopK; ++j) {
            o.k[j] = static_cast<uint32_t>(__shfl_xor(static_cast<int>(r.k[j]), mask, 64));
        }
        r = merge_lists(r, o);
    }
    return r;
}

__device__ __forceinline__ uint32_t pick(const KeyList& l, uint32_t j) {
    uint32_t v = 0u;
#pragma unroll
    for (uint32_t q = 0; q < kHypTopK; ++q) v = q == j ? l.k[q] : v;
    return v;
}

// Pass 1: workgroup (p, r) keeps the kHypTopK largest slice keys of values
// [p span, min((p + 1) span, vocab)) of row r in part[(r * parts + p) * kHypTopK ...],
// descending. Thread t takes 8-value chunks t, t + kThreads, ...: each chunk is sorted by
// a network and merged into the thread's list.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void topk_partial_kernel(const uint16_t* __restrict__ logits, uint32_t vocab,
                                                                uint32_t span, uint32_t* __restrict__ part) {
    const uint32_t p = blockIdx.x;
    const uint32_t row = blockIdx.y;
    const uint16_t* x = logits + static_cast<size_t>(row) * vocab;
    const uint32_t e0 = p * span;
    const uint32_t n = e0 < vocab ? min(span, vocab - e0) : 0u;
    const uint32_t chunks = (n + 7u) / 8u;
    KeyList l;
#pragma unroll
    for (uint32_t j = 0; j < kHypTopK; ++j) l.k[j] = 0u;
    for (uint32_t c = threadIdx.x; c < chunks; c += kThreads) {
        KeyList v;
        const uint32_t off = c * 8u;
        if (VEC) {
            // n % 8 == 0 and x + e0 is 16-byte aligned.
            const uint4 q = reinterpret_cast<const uint4*>(x + e0)[c];
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                v.k[2 * j] = slice_key(w[j] & 0xFFFFu, off + 2u * j);
                v.k[2 * j + 1] = slice_key(w[j] >> 16, off + 2u * j + 1u);
            }
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kHypTopK; ++j) {
                v.k[j] = off + j < n ? slice_key(x[e0 + off + j], off + j) : 0u;
            }
        }
        sort8(v);
        l = merge_lists(l, v);
    }

    __shared__ uint32_t waves[kThreads / 64][kHypTopK];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const KeyList w = wave_top(l);
    if (lane < kHypTopK) waves[wave][lane] = pick(w, lane);
    __syncthreads();
    if (threadIdx.x == 0) {
        KeyList u;
#pragma unroll
        for (uint32_t j = 0; j < kHypTopK; ++j) u.k[j] = waves[0][j];
#pragma unroll
        for (uint32_t q = 1; q < kThreads / 64; ++q) {
            KeyList b;
#pragma unroll
            for (uint32_t j = 0; j < kHypTopK; ++j) b.k[j] = waves[q][j];
            u = merge_lists(u, b);
        }
        uint32_t* dst = part + (static_cast<size_t>(row) * gridDim.x + p) * kHypTopK;
#pragma unroll
        for (uint32_t j = 0; j < kHypTopK; ++j) dst[j] = u.k[j];
    }
}

// Pass 2: one wave per row merges the row's `parts` slice lists (parts <= kTopKParts) and
// writes the sample. The slice keys are re-keyed by list position (slice q, rank j ->
// 0xFFFF - (8 q + j)) under the same order image: slices cover increasing indices and a
// slice's list orders equal values by index, so for equal values position order is
// index order.
__global__ __launch_bounds__(64) void topk_merge_kernel(const uint16_t* __restrict__ logits, uint32_t vocab,
                                                        uint32_t span, const uint32_t* __restrict__ part,
                                                        uint32_t parts, HypTopKSample* __restrict__ out) {
    const uint32_t row = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    const uint16_t* x = logits + static_cast<size_t>(row) * vocab;
    const uint32_t* rp = part + static_cast<size_t>(row) * parts * kHypTopK;
    KeyList l;
#pragma unroll
    for (uint32_t j = 0; j < kHypTopK; ++j) l.k[j] = 0u;
    for (uint32_t q = lane; q < parts; q += 64u) {
        KeyList v;
#pragma unroll
        for (uint32_t j = 0; j < kHypTopK; ++j) {
            const uint32_t key = rp[q * kHypTopK + j];
            v.k[j] = key == 0u ? 0u : (key & 0xFFFF0000u) | (0xFFFFu - (q * kHypTopK + j));
        }
        l = merge_lists(l, v);
    }
    const KeyList u = wave_top(l);
    const uint32_t count = min(vocab, kHypTopK);

    // Lane j < count resolves entry j: its slice and rank, the slice key there, the index.
    const uint32_t key = pick(u, lane & (kHypTopK - 1u));
    const bool real = lane < count;
    uint32_t idx = 0u;
    float val = 0.0f;
    if (real) {
        const uint32_t pos = 0xFFFFu - (key & 0xFFFFu);
        const uint32_t off = 0xFFFFu - (rp[pos] & 0xFFFFu);
        idx = (pos / kHypTopK) * span + off;
        val = bf16_to_f32(x[idx]);
    }
    const float val1 = __shfl(val, 1, 64);
    HypTopKSample* o = out + row;
    if (lane < kHypTopK) {
        o->top_k_ids[lane] = idx;
        o->top_k_logprobs[lane] = val;
    }
    if (lane == 0) {
        // Greedy fields (forward.cc:162-189): a first entry above -inf is the winner; the
        // largest other non-NaN value is the second entry's, or -inf.
        const uint32_t image0 = u.k[0] >> 16;
        const uint32_t image1 = u.k[1] >> 16;
        const bool win = count >= 1u && image0 > kImageNegInf;
        const float top1 = win ? val : -__builtin_huge_valf();
        const float top2 = count >= 2u && image1 >= kImageNegInf ? val1 : -__builtin_huge_valf();
        o->token_id = win ? idx : 0u;
        o->logit = top1;
        o->near_tie = (top1 - top2) < 0.5f ? 1u : 0u;
        o->top_k_count = count;
    }
}

}  // namespace

size_t sample_greedy_workspace_bytes() { return kMaxParts * kWorkspaceRows * sizeof(Top2); }

void launch_sample_greedy(const uint16_t* logits, uint32_t rows, uint32_t vocab, HypGreedySample* out,
                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
    HYP_REQUIRE(workspace != nullptr && workspace_bytes >= sample_greedy_workspace_bytes(), HYP_STATUS_INTERNAL,
                "sample_greedy: workspace too small");
    // About 4096 values per workgroup, at most kMaxParts per row; slices of whole
    // 8-value chunks.
    const uint32_t parts = std::max(1u, std::min<uint32_t>(kMaxParts, (vocab + 4095u) / 4096u));
    const uint32_t span = ((vocab + parts - 1u) / parts + 7u) & ~7u;
    Top2* part = static_cast<Top2*>(workspace);
    for (uint32_t r0 = 0; r0 < rows; r0 += kWorkspaceRows) {
        const uint32_t n = std::min(kWorkspaceRows, rows - r0);
        const uint16_t* x = logits + static_cast<size_t>(r0) * vocab;
        const bool vec = vocab % 8u == 0u && (reinterpret_cast<uintptr_t>(x) & 15u) == 0u;
        if (vec) {
            hipLaunchKernelGGL(sample_partial_kernel<true>, dim3(parts, n), dim3(kThreads), 0, stream, x, vocab, span,
                               part);
        } else {
            hipLaunchKernelGGL(sample_partial_kernel<false>, dim3(parts, n), dim3(kThreads), 0, stream, x, vocab, span,
                               part);
        }
        HYP_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(sample_merge_kernel, dim3(n), dim3(64), 0, stream, part, parts, out + r0);
        HYP_HIP_CHECK(hipGetLastError());
    }
}

uint32_t sample_topk_max_vocab() { return kTopKParts * kTopKMaxSpan; }

void launch_sample_topk(const uint16_t* logits, uint32_t rows, uint32_t vocab, HypTopKSample* out, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
    HYP_REQUIRE(workspace != nullptr && workspace_bytes >= sample_greedy_workspace_bytes(), HYP_STATUS_INTERNAL,
                "sample_topk: workspace too small");
    HYP_REQUIRE(vocab <= sample_topk_max_vocab(), HYP_STATUS_INTERNAL, "sample_topk: vocab too large");
    const uint32_t parts = std::max(1u, std::min<uint32_t>(kTopKParts, (vocab + kTopKSpan - 1u) / kTopKSpan));
    const uint32_t span = ((vocab + parts - 1u) / parts + 7u) & ~7u;   // <= kTopKMaxSpan
    uint32_t* part = static_cast<uint32_t*>(workspace);
    for (uint32_t r0 = 0; r0 < rows; r0 += kTopKRows) {
        const uint32_t n = std::min(kTopKRows, rows - r0);
        const uint16_t* x = logits + static_cast<size_t>(r0) * vocab;
        const bool vec = vocab % 8u == 0u && (reinterpret_cast<uintptr_t>(x) & 15u) == 0u;
        if (vec) {
            hipLaunchKernelGGL(topk_partial_kernel<true>, dim3(parts, n), dim3(kThreads), 0, stream, x, vocab, span,
                               part);
        } else {
            hipLaunchKernelGGL(topk_partial_kernel<false>, dim3(parts, n), dim3(kThreads), 0, stream, x, vocab, span,
                               part);
        }
        HYP_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(topk_merge_kernel, dim3(n), dim3(64), 0, stream, x, vocab, span, part, parts, out + r0);
        HYP_HIP_CHECK(hipGetLastError());
    }
}

}  // namespace hyperion::hip

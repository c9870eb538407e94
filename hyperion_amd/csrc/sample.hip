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

}  // namespace hyperion::hip

// Conversion between MLX's Q4/g64 layout (the I/O format: codes uint32 [n, k/8],
// scales and biases bf16 [n, k/64], native/hyperion_mlx/src/weights.h:18-25) and the
// tiled resident layout described in q4_layout.h. One thread per 16-byte code entry or
// 8-byte scale entry; both directions are a single pass over HBM.
#include "common.h"
#include "kernels.h"
#include "q4_layout.h"

namespace hyperion::hip {
namespace {

constexpr int kThreads = 256;

struct LayoutParams {
    uint32_t n;
    uint32_t k;
    uint32_t tiles;
    uint32_t pairs;
};

// Entry e of the code array: (tile, pair, lane) with lane = kb * 16 + j.
__device__ __forceinline__ void code_entry(const LayoutParams& p, uint64_t e, uint32_t& row, uint32_t& g0,
                                           uint32_t& kb) {
    const uint32_t lane = static_cast<uint32_t>(e & 63u);
    const uint64_t tp = e >> 6;
    const uint32_t pair = static_cast<uint32_t>(tp % p.pairs);
    const uint32_t tile = static_cast<uint32_t>(tp / p.pairs);
    row = tile * kTileRows + (lane & 15u);
    g0 = 2u * pair;
    kb = lane >> 4;
}

__global__ __launch_bounds__(kThreads) void tile_codes_kernel(LayoutParams p, const uint32_t* __restrict__ w,
                                                              uint4* __restrict__ codes, uint64_t entries) {
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= entries) return;
    uint32_t row, g0, kb;
    code_entry(p, e, row, g0, kb);
    const uint32_t G = p.k / 64u;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < p.n) {
        const uint32_t* wr = w + static_cast<size_t>(row) * (p.k / 8u);
        const uint2 a = *reinterpret_cast<const uint2*>(wr + g0 * 8u + kb * 2u);
        v.x = a.x;
        v.y = a.y;
        if (g0 + 1u < G) {
            const uint2 c = *reinterpret_cast<const uint2*>(wr + (g0 + 1u) * 8u + kb * 2u);
            v.z = c.x;
            v.w = c.y;
        }
    }
    codes[e] = v;
}

__global__ __launch_bounds__(kThreads) void untile_codes_kernel(LayoutParams p, const uint4* __restrict__ codes,
                                                                uint32_t* __restrict__ w, uint64_t entries) {
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= entries) return;
    uint32_t row, g0, kb;
    code_entry(p, e, row, g0, kb);
    if (row >= p.n) return;
    const uint32_t G = p.k / 64u;
    const uint4 v = codes[e];
    uint32_t* wr = w + static_cast<size_t>(row) * (p.k / 8u);
    *reinterpret_cast<uint2*>(wr + g0 * 8u + kb * 2u) = make_uint2(v.x, v.y);
    if (g0 + 1u < G) *reinterpret_cast<uint2*>(wr + (g0 + 1u) * 8u + kb * 2u) = make_uint2(v.z, v.w);
}

// Entry e of the scale array: (tile, pair, j).
__device__ __forceinline__ void sb_entry(const LayoutParams& p, uint64_t e, uint32_t& row, uint32_t& g0) {
    const uint32_t j = static_cast<uint32_t>(e & 15u);
    const uint64_t tp = e >> 4;
    const uint32_t pair = static_cast<uint32_t>(tp % p.pairs);
    const uint32_t tile = static_cast<uint32_t>(tp / p.pairs);
    row = tile * kTileRows + j;
    g0 = 2u * pair;
}

__global__ __launch_bounds__(kThreads) void tile_sb_kernel(LayoutParams p, const uint16_t* __restrict__ s,
                                                           const uint16_t* __restrict__ b, uint2* __restrict__ sb,
                                                           uint64_t entries) {
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= entries) return;
    uint32_t row, g0;
    sb_entry(p, e, row, g0);
    const uint32_t G = p.k / 64u;
    uint2 v = make_uint2(0u, 0u);
    if (row < p.n) {
        const size_t base = static_cast<size_t>(row) * G;
        v.x = static_cast<uint32_t>(s[base + g0]) | (static_cast<uint32_t>(b[base + g0]) << 16);
        if (g0 + 1u < G) {
            v.y = static_cast<uint32_t>(s[base + g0 + 1u]) | (static_cast<uint32_t>(b[base + g0 + 1u]) << 16);
        }
    }
    sb[e] = v;
}

__global__ __launch_bounds__(kThreads) void untile_sb_kernel(LayoutParams p, const uint2* __restrict__ sb,
                                                             uint16_t* __restrict__ s, uint16_t* __restrict__ b,
                                                             uint64_t entries) {
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= entries) return;
    uint32_t row, g0;
    sb_entry(p, e, row, g0);
    if (row >= p.n) return;
    const uint32_t G = p.k / 64u;
    const uint2 v = sb[e];
    const size_t base = static_cast<size_t>(row) * G;
    s[base + g0] = static_cast<uint16_t>(v.x & 0xFFFFu);
    b[base + g0] = static_cast<uint16_t>(v.x >> 16);
    if (g0 + 1u < G) {
        s[base + g0 + 1u] = static_cast<uint16_t>(v.y & 0xFFFFu);
        b[base + g0 + 1u] = static_cast<uint16_t>(v.y >> 16);
    }
}

dim3 grid_for(uint64_t entries) {
    const uint64_t blocks = (entries + kThreads - 1) / kThreads;
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "layout: matrix too large");
    return dim3(static_cast<uint32_t>(blocks));
}

}  // namespace

void launch_q4_tile(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint32_t n, uint32_t k, uint4* codes,
                    uint2* sb, hipStream_t stream) {
    const TiledDims d = TiledDims::of(n, k);
    const LayoutParams p{n, k, d.tiles, d.pairs};
    const uint64_t ce = d.code_bytes() / 16u;
    const uint64_t se = d.sb_bytes() / 8u;
    hipLaunchKernelGGL(tile_codes_kernel, grid_for(ce), dim3(kThreads), 0, stream, p, w, codes, ce);
    hipLaunchKernelGGL(tile_sb_kernel, grid_for(se), dim3(kThreads), 0, stream, p, s, b, sb, se);
    HYP_HIP_CHECK(hipGetLastError());
}

void launch_q4_untile(const uint4* codes, const uint2* sb, uint32_t n, uint32_t k, uint32_t* w, uint16_t* s,
                      uint16_t* b, hipStream_t stream) {
    const TiledDims d = TiledDims::of(n, k);
    const LayoutParams p{n, k, d.tiles, d.pairs};
    const uint64_t ce = d.code_bytes() / 16u;
    const uint64_t se = d.sb_bytes() / 8u;
    hipLaunchKernelGGL(untile_codes_kernel, grid_for(ce), dim3(kThreads), 0, stream, p, codes, w, ce);
    hipLaunchKernelGGL(untile_sb_kernel, grid_for(se), dim3(kThreads), 0, stream, p, sb, s, b, se);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

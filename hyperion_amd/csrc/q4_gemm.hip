// Prefill GEMM for MLX-affine Q4/g64 weights on gfx950 bf16 MFMA.
//
// Replaces mlx::core::quantized_matmul(..., transpose=true, 64, 4, "affine") at
// prefill, where the reference's chunk loop (native/hyperion_mlx/src/model.cc:574-610)
// hands every projection up to 2048 rows at once.
//
// Y[m, n] = X[m, k] . dequant(W)[n, k]^T, fp32 accumulation, bf16 out.
//
// Tiling (one workgroup = 4 waves = one CU at a time, 256 x 256 output tile):
//  * K advances one quantization group (64) per step, so one (scale, bias) pair
//    covers every code a lane dequantizes in a step.
//  * X tiles (256 x 64 bf16) are staged in LDS, double-buffered, one barrier per step.
//  * Each wave owns 64 output columns (two 32-wide MFMA tiles) for all 256 rows, so
//    no two waves ever need the same dequantized weights: a lane loads 16 B of packed
//    codes for its column, dequantizes them in registers (fp32 fma of scale and code
//    plus bias, one rounding to bf16 with v_cvt_pk_bf16_f32) and feeds them straight
//    to v_mfma_f32_32x32x16_bf16 as the B operand. Within a group the lane half h
//    holds words 4h..4h+3; k-block j pairs word 4h+j with X[32h + 8j .. +7], the same
//    permutation on both operands.
//  * Workgroup ids are remapped so each XCD (ids are dealt round-robin over the 8 XCDs)
//    gets a contiguous run of tiles that share X rows, keeping the X block in that
//    XCD's L2.
#include "common.h"
#include "kernels.h"

namespace hyperion::hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 64;
constexpr int kLdsStride = kBK + 8;   // bf16 per LDS row (16 B pad against bank conflicts)
constexpr int kMTiles = kBM / 32;     // 8
constexpr int kNTiles = 2;            // per wave
constexpr int kXLoads = kBM * kBK / 8 / kThreads;   // uint4 per thread per step = 8

struct GemmParams {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    const uint16_t* x;
    uint16_t* y;
    uint32_t m;
    uint32_t n;
    uint32_t k;
    uint32_t tiles_n;
    uint32_t tiles_total;
};

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// 8 codes of one packed word -> 8 bf16 values s*q+b (single rounding), in k order.
__device__ __forceinline__ uint4 dequant_word(uint32_t word, float s, float b) {
    const uint32_t lo = word & 0x0F0F0F0Fu;          // codes 0,2,4,6 in bytes 0..3
    const uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;   // codes 1,3,5,7
    uint4 r;
    r.x = pack_bf16x2(fmaf(s, static_cast<float>(lo & 0xFFu), b), fmaf(s, static_cast<float>(hi & 0xFFu), b));
    r.y = pack_bf16x2(fmaf(s, static_cast<float>((lo >> 8) & 0xFFu), b),
                      fmaf(s, static_cast<float>((hi >> 8) & 0xFFu), b));
    r.z = pack_bf16x2(fmaf(s, static_cast<float>((lo >> 16) & 0xFFu), b),
                      fmaf(s, static_cast<float>((hi >> 16) & 0xFFu), b));
    r.w = pack_bf16x2(fmaf(s, static_cast<float>(lo >> 24), b), fmaf(s, static_cast<float>(hi >> 24), b));
    return r;
}

__global__ __launch_bounds__(kThreads) void q4_gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][kBM * kLdsStride];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t col = lane & 31u;
    const uint32_t half = lane >> 5;

    // XCD-aware tile order: XCD x = blockIdx % 8 runs tiles [start_x, start_x + count_x).
    const uint32_t b = blockIdx.x;
    const uint32_t xcd = b & 7u;
    const uint32_t slot = b >> 3;
    const uint32_t per = p.tiles_total >> 3;
    const uint32_t rem = p.tiles_total & 7u;
    const uint32_t tile = xcd * per + min(xcd, rem) + slot;
    const uint32_t tm = tile / p.tiles_n;
    const uint32_t tn = tile - tm * p.tiles_n;
    const uint32_t m0 = tm * kBM;
    const uint32_t n0 = tn * kBN;

    const uint32_t k = p.k;
    const uint32_t G = k / 64u;
    const size_t row_words = k / 8u;

    // Per-lane weight rows for the wave's two N tiles, clamped into the matrix: every
    // load is unconditional; columns past n are computed but never stored.
    uint32_t nrow[kNTiles];
    size_t wrow[kNTiles];   // row index (clamped)
#pragma unroll
    for (int t = 0; t < kNTiles; ++t) {
        nrow[t] = n0 + wave * 64u + t * 32u + col;
        wrow[t] = min(nrow[t], p.n - 1u);
    }
    // X rows this thread stages: rows (tid >> 3) + 32 i, 16-byte column (tid & 7),
    // clamped likewise (rows past m feed outputs that are never stored).
    const uint32_t xc16 = tid & 7u;
    const uint32_t xr0 = tid >> 3;
    size_t xoff[kXLoads];
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
        const uint32_t gm = min(m0 + xr0 + 32u * i, p.m - 1u);
        xoff[i] = static_cast<size_t>(gm) * k + xc16 * 8u;
    }

    f32x16_t acc[kMTiles][kNTiles];
#pragma unroll
    for (int i = 0; i < kMTiles; ++i)
#pragma unroll
        for (int t = 0; t < kNTiles; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][t][v] = 0.0f;

    uint4 xr[kXLoads];
    uint4 wv[kNTiles];
    uint32_t sraw[kNTiles];
    uint32_t braw[kNTiles];

#pragma unroll
    for (int i = 0; i < kXLoads; ++i) xr[i] = *reinterpret_cast<const uint4*>(p.x + xoff[i]);
#pragma unroll
    for (int t = 0; t < kNTiles; ++t) {
        wv[t] = *reinterpret_cast<const uint4*>(p.w + wrow[t] * row_words + half * 4u);
        sraw[t] = p.s[wrow[t] * G];
        braw[t] = p.b[wrow[t] * G];
    }
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
        *reinterpret_cast<uint4*>(&xs[0][(xr0 + 32u * i) * kLdsStride + xc16 * 8u]) = xr[i];
    }
    __syncthreads();

    for (uint32_t g = 0; g < G; ++g) {
        const uint32_t cur = g & 1u;
        bf16x8_t bfr[kNTiles][4];
#pragma unroll
        for (int t = 0; t < kNTiles; ++t) {
            const float sv = bf16_bits_to_f32(sraw[t]);
            const float bv = bf16_bits_to_f32(braw[t]);
            bfr[t][0] = __builtin_bit_cast(bf16x8_t, dequant_word(wv[t].x, sv, bv));
            bfr[t][1] = __builtin_bit_cast(bf16x8_t, dequant_word(wv[t].y, sv, bv));
            bfr[t][2] = __builtin_bit_cast(bf16x8_t, dequant_word(wv[t].z, sv, bv));
            bfr[t][3] = __builtin_bit_cast(bf16x8_t, dequant_word(wv[t].w, sv, bv));
        }
        // Prefetch the next step (the last step re-reads the current group: harmless).
        const uint32_t gn = min(g + 1u, G - 1u);
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) xr[i] = *reinterpret_cast<const uint4*>(p.x + xoff[i] + gn * 64u);
#pragma unroll
        for (int t = 0; t < kNTiles; ++t) {
            wv[t] = *reinterpret_cast<const uint4*>(p.w + wrow[t] * row_words + gn * 8u + half * 4u);
            sraw[t] = p.s[wrow[t] * G + gn];
            braw[t] = p.b[wrow[t] * G + gn];
        }
        const uint16_t* xb = xs[cur];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int i = 0; i < kMTiles; ++i) {
                const uint4 av = *reinterpret_cast<const uint4*>(
                    &xb[(i * 32u + col) * kLdsStride + half * 32u + j * 8u]);
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, av);
#pragma unroll
                for (int t = 0; t < kNTiles; ++t) {
                    acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bfr[t][j], acc[i][t], 0, 0, 0);
                }
            }
        }
        uint16_t* xn = xs[cur ^ 1u];
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            *reinterpret_cast<uint4*>(&xn[(xr0 + 32u * i) * kLdsStride + xc16 * 8u]) = xr[i];
        }
        __syncthreads();
    }

    // Epilogue: acc[i][t][v] is Y[m0 + 32i + 8(v/4) + 4*half + v%4][n0 + 64*wave + 32t + col].
#pragma unroll
    for (int t = 0; t < kNTiles; ++t) {
        const uint32_t n = nrow[t];
        const bool nok = n < p.n;
#pragma unroll
        for (int i = 0; i < kMTiles; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t m = m0 + i * 32u + 8u * (v >> 2) + 4u * half + (v & 3);
                if (nok && m < p.m) {
                    const size_t off = static_cast<size_t>(m) * p.n + n;
                    const float out = round_bf16(acc[i][t][v]);
                    p.y[off] = f32_to_bf16_bits(out);
                }
            }
        }
    }
}

}  // namespace

void launch_q4_gemm(const Q4Matrix& w, const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream) {
    GemmParams p{};
    p.w = w.w;
    p.s = w.scales;
    p.b = w.biases;
    p.x = x;
    p.y = y;
    p.m = m;
    p.n = w.n;
    p.k = w.k;
    p.tiles_n = (w.n + kBN - 1u) / kBN;
    const uint32_t tiles_m = (m + kBM - 1u) / kBM;
    p.tiles_total = p.tiles_n * tiles_m;
    hipLaunchKernelGGL(q4_gemm_kernel, dim3(p.tiles_total), dim3(kThreads), 0, stream, p);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

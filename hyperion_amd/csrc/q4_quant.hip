// Quantize / dequantize kernels for MLX-affine Q4/g64 on gfx950.
//
// quantize   = mx.quantize(w, group_size=64, bits=4, mode="affine") as the reference
//              uses it to build Q4 weights (crates/hyperion-model/fixtures/
//              build_gemma4_unified_tiny.py:54-57, scripts/nax-probe.py:74-76);
// dequantize = mx.dequantize(..., dtype=bfloat16) of gathered rows, the embed path
//              (native/hyperion_mlx/src/weights_loader.cc:53-69, forward.cc:126-131).
//
// Both are one pass over HBM with one thread per packed word (8 codes = 16 B of bf16),
// so a wave moves 1 KB of contiguous bf16 per instruction.
#include "common.h"
#include "kernels.h"
#include "q4_layout.h"

namespace hyperion::hip {
namespace {

constexpr int kThreads = 256;

template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
    const float o = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
    return fmaxf(v, o);
}
template <int CTRL>
__device__ __forceinline__ float dpp_min(float v) {
    const float o = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
    return fminf(v, o);
}

// rint((v - bias) / scale) as MLX computes it (IEEE fp32 quotient, then round half to
// even), evaluated with the group's correctly rounded reciprocal. For |q| < 64,
// |v*rcp - fl(v/scale)| < 2^-16, so both round to the same integer unless the
// quotient lies within 2^-15 of a half-integer; only then is the exact division done.
__device__ __forceinline__ float quant_code(float v, float bias, float scale, float rcp) {
    const float d = v - bias;
    float q = d * rcp;
    const float fr = q - floorf(q);
    if (fabsf(fr - 0.5f) < 3.0517578125e-05f && fabsf(q) < 64.0f) {
        q = __fdiv_rn(d, scale);
    }
    q = rintf(q);
    q = fminf(fmaxf(q, 0.0f), 15.0f);   // NaN (never produced for finite input) -> 0
    return q;
}

__global__ __launch_bounds__(kThreads) void q4_quantize_kernel(const uint16_t* __restrict__ w,
                                                               uint32_t* __restrict__ wq,
                                                               uint16_t* __restrict__ scales,
                                                               uint16_t* __restrict__ biases,
                                                               uint64_t words) {
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const bool live = t < words;
    // Dead lanes of the last wave mirror word 0 so every lane feeds the DPP reductions.
    const uint64_t src = live ? t : 0u;
    const uint4 raw = *reinterpret_cast<const uint4*>(w + src * 8u);
    float v[8];
    v[0] = bf16_bits_to_f32(raw.x & 0xFFFFu);
    v[1] = bf16_bits_to_f32(raw.x >> 16);
    v[2] = bf16_bits_to_f32(raw.y & 0xFFFFu);
    v[3] = bf16_bits_to_f32(raw.y >> 16);
    v[4] = bf16_bits_to_f32(raw.z & 0xFFFFu);
    v[5] = bf16_bits_to_f32(raw.z >> 16);
    v[6] = bf16_bits_to_f32(raw.w & 0xFFFFu);
    v[7] = bf16_bits_to_f32(raw.w >> 16);

    float w_max = -INFINITY;
    float w_min = INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        w_max = fmaxf(w_max, v[e]);
        w_min = fminf(w_min, v[e]);
    }
    // The 8 lanes of a group are lanes 8i..8i+7 of the wave.
    w_max = dpp_max<0xB1>(w_max);
    w_max = dpp_max<0x4E>(w_max);
    w_max = dpp_max<0x141>(w_max);
    w_min = dpp_min<0xB1>(w_min);
    w_min = dpp_min<0x4E>(w_min);
    w_min = dpp_min<0x141>(w_min);

    // Zero-point ("edge") rule, fp32 with IEEE division.
    const bool mask = fabsf(w_min) > fabsf(w_max);
    float scale = __fdiv_rn(w_max - w_min, 15.0f);
    scale = (scale < 1e-7f) ? 1e-7f : scale;   // std::max(scale, eps)
    scale = mask ? scale : -scale;
    const float edge = mask ? w_min : w_max;
    const float q0 = rintf(__fdiv_rn(edge, scale));
    float bias = 0.0f;
    if (q0 != 0.0f) {
        scale = __fdiv_rn(edge, q0);
        bias = edge;
    }
    const float rcp = __fdiv_rn(1.0f, scale);

    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        packed |= static_cast<uint32_t>(quant_code(v[e], bias, scale, rcp)) << (4 * e);
    }
    if (live) {
        wq[t] = packed;
        if ((t & 7u) == 0u) {
            scales[t >> 3] = f32_to_bf16_bits(scale);
            biases[t >> 3] = f32_to_bf16_bits(bias);
        }
    }
}

// The 8 bf16 outputs of one packed word: bf16(bf16(s*q) + b), optionally times a bf16
// constant with one more rounding.
__device__ __forceinline__ uint4 dequant_word_mlx(uint32_t word, float s, float b, float out_scale) {
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float q = static_cast<float>((word >> (4 * e)) & 0xFu);
        float val = round_bf16(s * q);   // s*q is exact in fp32; one rounding per MLX op
        val = round_bf16(val + b);
        if (out_scale != 0.0f) val = round_bf16(val * out_scale);
        h[e] = f32_to_bf16_bits(val);
    }
    return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

// One thread per packed word of an output row, reading the tiled layout (q4_layout.h).
__global__ __launch_bounds__(kThreads) void q4_dequantize_tiled_kernel(
    const uint4* __restrict__ codes, const uint2* __restrict__ sb, uint32_t n_total, uint32_t k, uint32_t pairs,
    const uint32_t* __restrict__ rows, uint32_t n_rows, float out_scale, uint16_t* __restrict__ out) {
    const uint32_t words_per_row = k / 8u;
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= static_cast<uint64_t>(n_rows) * words_per_row) return;
    const uint32_t i = static_cast<uint32_t>(t / words_per_row);
    const uint32_t wd = static_cast<uint32_t>(t - static_cast<uint64_t>(i) * words_per_row);
    const uint32_t r = rows ? rows[i] : i;
    uint4 res = make_uint4(0u, 0u, 0u, 0u);
    if (r < n_total) {
        const uint32_t g = wd / 8u;          // group
        const uint32_t w8 = wd % 8u;         // word within the group: entry kb = w8 / 2, half w8 % 2
        const size_t e = static_cast<size_t>(r / kTileRows) * pairs + g / 2u;
        const uint32_t j = r % kTileRows;
        const uint4 c = codes[e * 64u + (w8 / 2u) * 16u + j];
        const uint2 sbv = sb[e * 16u + j];
        const bool second = (g & 1u) != 0u;
        const uint32_t word = second ? ((w8 & 1u) ? c.w : c.z) : ((w8 & 1u) ? c.y : c.x);
        const uint32_t sbw = second ? sbv.y : sbv.x;
        res = dequant_word_mlx(word, bf16_bits_to_f32(sbw & 0xFFFFu), bf16_bits_to_f32(sbw >> 16), out_scale);
    }
    *reinterpret_cast<uint4*>(out + static_cast<size_t>(i) * k + wd * 8u) = res;
}

// One thread per packed word of an output row: bf16(bf16(s*q) + b), optionally
// times a bf16 constant.
__global__ __launch_bounds__(kThreads) void q4_dequantize_kernel(
    const uint32_t* __restrict__ wq, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, uint32_t n_total, uint32_t k,
    const uint32_t* __restrict__ rows, uint32_t n_rows, float out_scale, uint16_t* __restrict__ out) {
    const uint32_t words_per_row = k / 8u;
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= static_cast<uint64_t>(n_rows) * words_per_row) return;
    const uint32_t i = static_cast<uint32_t>(t / words_per_row);
    const uint32_t j = static_cast<uint32_t>(t - static_cast<uint64_t>(i) * words_per_row);
    const uint32_t r = rows ? rows[i] : i;
    uint4 res = make_uint4(0u, 0u, 0u, 0u);
    if (r < n_total) {
        const size_t G = k / 64u;
        const uint32_t word = wq[static_cast<size_t>(r) * words_per_row + j];
        const float s = bf16_bits_to_f32(scales[r * G + (j >> 3)]);
        const float b = bf16_bits_to_f32(biases[r * G + (j >> 3)]);
        res = dequant_word_mlx(word, s, b, out_scale);
    }
    *reinterpret_cast<uint4*>(out + static_cast<size_t>(i) * k + j * 8u) = res;
}

}  // namespace

void launch_q4_quantize(const uint16_t* w, uint32_t n, uint32_t k, uint32_t* wq, uint16_t* scales,
                        uint16_t* biases, hipStream_t stream) {
    const uint64_t words = static_cast<uint64_t>(n) * (k / 8u);
    const uint64_t blocks = (words + kThreads - 1) / kThreads;
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "quantize: matrix too large");
    hipLaunchKernelGGL(q4_quantize_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream,
                       w, wq, scales, biases, words);
    HYP_HIP_CHECK(hipGetLastError());
}

void launch_q4_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                          uint32_t n_total, uint32_t k, const uint32_t* rows, uint32_t n_rows,
                          float out_scale_bf16, uint16_t* out, hipStream_t stream) {
    const uint64_t threads = static_cast<uint64_t>(n_rows) * (k / 8u);
    const uint64_t blocks = (threads + kThreads - 1) / kThreads;
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "dequantize: output too large");
    hipLaunchKernelGGL(q4_dequantize_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream,
                       wq, scales, biases, n_total, k, rows, n_rows, out_scale_bf16, out);
    HYP_HIP_CHECK(hipGetLastError());
}

void launch_q4_dequantize_tiled(const Q4Matrix& w, const uint32_t* rows, uint32_t n_rows, float out_scale_bf16,
                                uint16_t* out, hipStream_t stream) {
    HYP_REQUIRE(w.codes != nullptr && w.sb != nullptr, HYP_STATUS_INTERNAL,
                "dequantize: weights are not in the tiled resident layout");
    const uint64_t threads = static_cast<uint64_t>(n_rows) * (w.k / 8u);
    const uint64_t blocks = (threads + kThreads - 1) / kThreads;
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "dequantize: output too large");
    hipLaunchKernelGGL(q4_dequantize_tiled_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream,
                       w.codes, w.sb, w.n, w.k, TiledDims::of(w.n, w.k).pairs, rows, n_rows, out_scale_bf16, out);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

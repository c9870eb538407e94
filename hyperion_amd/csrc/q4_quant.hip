// Quantize / dequantize kernels for MLX-affine Q4/g64 on gfx950.
//
// quantize   = mx.quantize(w, group_size=64, bits=4, mode="affine") as the reference
//              uses it to build Q4 weights (crates/hyperion-model/fixtures/
//              build_gemma4_unified_tiny.py:54-57, scripts/nax-probe.py:74-76);
// dequantize = mx.dequantize(..., dtype=bfloat16) of gathered rows, the embed path
//              (native/hyperion_mlx/src/weights_loader.cc:53-69, forward.cc:126-131).
//
// Both are one pass over HBM. Quantize runs one thread per group of 64 (the group's scale
// is derived once); dequantize one thread per packed word (8 codes = 16 B of bf16).
#include "common.h"
#include "kernels.h"
#include "q4_layout.h"

namespace hyperion::hip {
namespace {

constexpr int kThreads = 256;

// rint((v - bias) / scale) for the 8 values of one packed word, as MLX computes it (IEEE
// fp32 quotient, round half to even, clamped to 0..15), packed lowest k first. The
// quotients are formed with the group's correctly rounded reciprocal: fl(fl(d) * fl(1/s))
// is within 2^-23 relative, so for |q| < 64 within 2^-17, of the IEEE quotient, and both
// round to the same integer unless a half-integer lies within 2^-17 of the approximate
// quotient. Values whose approximate quotient lies within 2^-16 of one (twice the bound)
// are divided exactly, one by one: bf16 inputs over a scale derived from bf16 extremes
// make exact half-integer quotients common (about 0.3% of values, 2% of words on
// N(0, 0.02) weights), so the exact path is kept per value. Quotients of 64 or more clamp
// to 15 either way.
__device__ __forceinline__ uint32_t pack_codes(const float (&c)[8]) {
    // Codes 0, 2, 4, 6 as the bytes of one word and 1, 3, 5, 7 of another (v_cvt_pk_u8_f32,
    // exact for the integral 0..15), then the odd ones shifted into the high nibbles.
    const uint32_t lo01 = __builtin_amdgcn_cvt_pk_u8_f32(c[2], 1u, __builtin_amdgcn_cvt_pk_u8_f32(c[0], 0u, 0u));
    const uint32_t lo23 = __builtin_amdgcn_cvt_pk_u8_f32(c[6], 3u, __builtin_amdgcn_cvt_pk_u8_f32(c[4], 2u, 0u));
    const uint32_t hi01 = __builtin_amdgcn_cvt_pk_u8_f32(c[3], 1u, __builtin_amdgcn_cvt_pk_u8_f32(c[1], 0u, 0u));
    const uint32_t hi23 = __builtin_amdgcn_cvt_pk_u8_f32(c[7], 3u, __builtin_amdgcn_cvt_pk_u8_f32(c[5], 2u, 0u));
    return (lo01 | lo23) | ((hi01 | hi23) << 4);
}

__device__ __forceinline__ uint32_t quant_word(const float (&v)[8], float bias, float scale, float rcp) {
    constexpr float kNearTie = 0.5f - 1.52587890625e-05f;   // 2^-16 from a half-integer
    float c[8];
    float d[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float q = (v[e] - bias) * rcp;
        const float r = rintf(q);
        d[e] = fabsf(q - r);
        c[e] = fminf(fmaxf(r, 0.0f), 15.0f);   // NaN (never produced for finite input) -> 0
    }
    const float dev = fmaxf(fmaxf(fmaxf(d[0], d[1]), fmaxf(d[2], d[3])), fmaxf(fmaxf(d[4], d[5]), fmaxf(d[6], d[7])));
    if (dev > kNearTie) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (d[e] > kNearTie) c[e] = fminf(fmaxf(rintf(__fdiv_rn(v[e] - bias, scale)), 0.0f), 15.0f);
        }
    }
    return pack_codes(c);
}

// One thread per group of 64: it finds the group's extremes, derives scale and bias once
// (zero-point rule, fp32, IEEE division, rint) and forms 8 packed words plus a bf16 scale
// and bias. No cross-lane arithmetic and no redundant per-group work, so the vector ALU
// work per weight is the quantization itself.
//
// Memory: a wave's 64 groups are 8 KB of contiguous input and 2 KB of contiguous codes. The
// input is read by 8 wave-wide 16-byte loads of 1 KB each (lane-consecutive) into an LDS
// tile, from which each lane takes its own group's 8 chunks; the codes go back the same way
// (2 stores of 1 KB). In the tile chunk c of group r sits at r * 8 + (c ^ (r & 7)), so both
// the lane-consecutive writes and the per-group reads touch 16 distinct 16-byte bank groups
// per 16 lanes.
constexpr uint32_t kQuantWaves = kThreads / 64;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t tile_slot(uint32_t r, uint32_t c) { return r * 8u + (c ^ (r & 7u)); }

// Orders one wave's LDS accesses across its lanes: a wave's LDS instructions execute in
// order, so only the compiler must keep them in program order. Each wave touches only its
// own tile, so the waves of a workgroup never wait for each other.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(kThreads) void q4_quantize_kernel(const uint16_t* __restrict__ w,
                                                               uint32_t* __restrict__ wq,
                                                               uint16_t* __restrict__ scales,
                                                               uint16_t* __restrict__ biases,
                                                               uint64_t groups) {
    __shared__ uint4 tile[kQuantWaves][64 * 8];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint64_t g0 = static_cast<uint64_t>(blockIdx.x) * kThreads + wave * 64u;   // this wave's first group
    const uint64_t left = g0 < groups ? groups - g0 : 0u;                           // groups from g0 on
    const uint32_t own = static_cast<uint32_t>(left < 64u ? left : 64u);             // this wave's groups
    const uint64_t g = g0 + lane;
    const bool live = lane < own;
    uint4* t4 = tile[wave];

    const uint4* src = reinterpret_cast<const uint4*>(w) + g0 * 8u;
    if (own == 64u) {   // every load issued before the first LDS write
        uint4 in[8];
#pragma unroll
        for (int t = 0; t < 8; ++t)
            in[t] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) +
                                                                          static_cast<uint32_t>(t) * 64u + lane));
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t j = static_cast<uint32_t>(t) * 64u + lane;
            t4[tile_slot(j >> 3, j & 7u)] = in[t];
        }
    } else {   // the last, partial wave
        for (uint32_t j = lane; j < own * 8u; j += 64u) t4[tile_slot(j >> 3, j & 7u)] = src[j];
    }
    wave_lds_sync();
    uint4 raw[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) raw[t] = t4[tile_slot(lane, static_cast<uint32_t>(t))];
    wave_lds_sync();   // every lane has its chunks: the tile takes the codes next

    float w_max = -INFINITY;
    float w_min = INFINITY;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t h[4] = {raw[t].x, raw[t].y, raw[t].z, raw[t].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float lo = bf16_bits_to_f32(h[e] & 0xFFFFu);
            const float hi = __uint_as_float(h[e] & 0xFFFF0000u);
            w_max = fmaxf(w_max, fmaxf(lo, hi));
            w_min = fminf(w_min, fminf(lo, hi));
        }
    }

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

    uint32_t packed[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t h[4] = {raw[t].x, raw[t].y, raw[t].z, raw[t].w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = bf16_bits_to_f32(h[e] & 0xFFFFu);
            v[2 * e + 1] = __uint_as_float(h[e] & 0xFFFF0000u);
        }
        packed[t] = quant_word(v, bias, scale, rcp);
    }
    t4[2u * lane] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    t4[2u * lane + 1u] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    wave_lds_sync();
    uint4* dst = reinterpret_cast<uint4*>(wq) + g0 * 2u;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t j = static_cast<uint32_t>(t) * 64u + lane;
        if (j < own * 2u) __builtin_nontemporal_store(__builtin_bit_cast(u32x4, t4[j]), reinterpret_cast<u32x4*>(dst) + j);
    }
    if (live) {
        scales[g] = f32_to_bf16_bits(scale);
        biases[g] = f32_to_bf16_bits(bias);
    }
}

// The 8 bf16 outputs of one packed word: bf16(s*q + b), one rounding of the fp32 value (s*q
// is exact in fp32: 8-bit by 4-bit significands), optionally times a bf16 constant with one
// more rounding. MLX's dequantize rounds once: the reference's 12B embed golden fits this
// form in all 600 of its groups and the op-composed bf16(bf16(s*q) + b) alone in none.
__device__ __forceinline__ uint4 dequant_word_mlx(uint32_t word, float s, float b, float out_scale) {
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float q = static_cast<float>((word >> (4 * e)) & 0xFu);
        float val = round_bf16(__builtin_fmaf(s, q, b));
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

// One thread per packed word of an output row: bf16(s*q + b), optionally times a bf16
// constant.
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
    const uint64_t groups = static_cast<uint64_t>(n) * (k / 64u);
    const uint64_t blocks = (groups + kThreads - 1) / kThreads;
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "quantize: matrix too large");
    hipLaunchKernelGGL(q4_quantize_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream,
                       w, wq, scales, biases, groups);
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

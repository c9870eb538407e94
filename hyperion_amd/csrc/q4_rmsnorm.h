// Row RMS normalisation shared by the standalone kernel and the normalising prologue of
// the skinny matmul, so both produce the same bits: y = bf16(x * inv) with
// inv = 1 / sqrt(ss / k + eps), where ss is summed in one fixed order -
//   1. per 64-element unit (k ascending), a sequential fp32 fma chain;
//   2. per row, lane l of one wave adds units l, l + 64, l + 128, ... in that order,
//      then an xor butterfly over the 64 lanes (offsets 32, 16, ..., 1).
// mx::fast::rms_norm(x, weight, eps) (native/hyperion_mlx/src/forward.cc:23-26): the
// normalised value is rounded to bf16, then multiplied by the bf16 weight and rounded
// again, y = bf16(w * bf16(x * inv)); without a weight (v_norm, forward.cc:403-412) y =
// bf16(x * inv). The reference applies it with weights around every block
// (input_layernorm, post_attention_layernorm, the feed-forward norms, forward.cc:521-529)
// and to q and k per head (q_norm, k_norm, forward.cc:400-405).
#pragma once

#include "common.h"

namespace hyperion::hip {

// __shfl_xor(v, MASK, 64) for MASK < 16, whose partner lies in the lane's 16-lane row, by DPP
// moves instead of an LDS permute (register latency instead of an LDS round trip on every
// step of a butterfly): xor 1 and 2 are quad permutes, xor 4 and 8 take the row shifted
// left or right by MASK, whichever holds the partner. The same values, so the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

template <int MASK>
__device__ __forceinline__ float xor_lanes(float v, uint32_t lane) {
    static_assert(MASK == 1 || MASK == 2 || MASK == 4 || MASK == 8, "a partner in the 16-lane row");
    if constexpr (MASK == 1) {
        return dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    } else if constexpr (MASK == 2) {
        return dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    } else {
        const float up = dpp_mov<0x100 + MASK>(v);     // row_shl: lane i + MASK
        const float down = dpp_mov<0x110 + MASK>(v);   // row_shr: lane i - MASK
        return (lane & static_cast<uint32_t>(MASK)) != 0u ? down : up;
    }
}

// v + the value of lane l ^ 32 (l ^ 16): with v in both operands v_permlane32_swap
// (v_permlane16_swap) leaves each lane's own value in one register and its partner's in the
// other, and the sum of the two is v + partner (addition commutes). Inline assembly: the
// builtins, given equal inputs, compiled to an add of one output register to itself; the
// s_nop gives the swap the wait states it needs after a VALU write of its operands.
__device__ __forceinline__ float add_lane_xor32(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    uint32_t c = u;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(c));
    return __builtin_bit_cast(float, u) + __builtin_bit_cast(float, c);
}

__device__ __forceinline__ float add_lane_xor16(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    uint32_t c = u;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(u), "+v"(c));
    return __builtin_bit_cast(float, u) + __builtin_bit_cast(float, c);
}

// max(v, the value of lane l ^ 32) and of lane l ^ 16, by the same swaps.
__device__ __forceinline__ float max_lane_xor32(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    uint32_t c = u;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(c));
    return fmaxf(__builtin_bit_cast(float, u), __builtin_bit_cast(float, c));
}

__device__ __forceinline__ float max_lane_xor16(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    uint32_t c = u;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(u), "+v"(c));
    return fmaxf(__builtin_bit_cast(float, u), __builtin_bit_cast(float, c));
}

// The max over all 64 lanes by the xor butterfly 32, 16, ..., 1 (fmaxf, exact in any order).
__device__ __forceinline__ float butterfly_max64(float v, uint32_t lane) {
    v = max_lane_xor32(v);
    v = max_lane_xor16(v);
    v = fmaxf(v, xor_lanes<8>(v, lane));
    v = fmaxf(v, xor_lanes<4>(v, lane));
    v = fmaxf(v, xor_lanes<2>(v, lane));
    return fmaxf(v, xor_lanes<1>(v, lane));
}

// The xor butterfly sum with offsets TOP, TOP / 2, ..., 1 (TOP a power of two up to 32, or
// 0 for none), bit for bit `for (off = TOP; off > 0; off >>= 1) v += __shfl_xor(v, off)`,
// with no LDS permute: lane swaps for 32 and 16, DPP moves below.
template <uint32_t TOP>
__device__ __forceinline__ float butterfly_sum(float v, uint32_t lane) {
    static_assert(TOP <= 32u && (TOP & (TOP - 1u)) == 0u, "a power of two up to 32");
    if constexpr (TOP >= 32u) v = add_lane_xor32(v);
    if constexpr (TOP >= 16u) v = add_lane_xor16(v);
    if constexpr (TOP >= 8u) v += xor_lanes<8>(v, lane);
    if constexpr (TOP >= 4u) v += xor_lanes<4>(v, lane);
    if constexpr (TOP >= 2u) v += xor_lanes<2>(v, lane);
    if constexpr (TOP >= 1u) v += xor_lanes<1>(v, lane);
    return v;
}

// The unit operations below, one 16-byte chunk (8 bf16, k ascending) at a time: a unit's
// result is the same whether its chunks are taken from registers or streamed from LDS. A
// register's two bf16 values widen with one VALU op each, and each pair of results is
// rounded by one v_cvt_pk_bf16_f32 (round to nearest even per half, the bits of two
// separate conversions).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ float chunk_sumsq(const uint4& c, float ss) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float lo = bf16_lo(w[q]);
        const float hi = bf16_hi(w[q]);
        ss = fmaf(lo, lo, ss);
        ss = fmaf(hi, hi, ss);
    }
    return ss;
}

// c <- bf16(c * inv).
__device__ __forceinline__ void normalize_chunk(uint4& c, float inv) {
    uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = cvt_pk_bf16(bf16_lo(w[q]) * inv, bf16_hi(w[q]) * inv);
    c = make_uint4(w[0], w[1], w[2], w[3]);
}

// c <- bf16(w * c).
__device__ __forceinline__ void weight_chunk(uint4& c, const uint4& wc) {
    uint32_t x[4] = {c.x, c.y, c.z, c.w};
    const uint32_t w[4] = {wc.x, wc.y, wc.z, wc.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = cvt_pk_bf16(bf16_lo(w[q]) * bf16_lo(x[q]), bf16_hi(w[q]) * bf16_hi(x[q]));
    c = make_uint4(x[0], x[1], x[2], x[3]);
}

// The residual add of the Gemma sandwich (forward.cc:523-539): h <- bf16(r + h), then
// h <- bf16(h * sc) when has_scalar (the layer scalar, a bf16 value).
__device__ __forceinline__ void residual_add_chunk(uint4& h, const uint4& r, bool has_scalar, float sc) {
    uint32_t x[4] = {h.x, h.y, h.z, h.w};
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        x[q] = cvt_pk_bf16(bf16_lo(w[q]) + bf16_lo(x[q]), bf16_hi(w[q]) + bf16_hi(x[q]));
        if (has_scalar) x[q] = cvt_pk_bf16(bf16_lo(x[q]) * sc, bf16_hi(x[q]) * sc);
    }
    h = make_uint4(x[0], x[1], x[2], x[3]);
}

// unit_sumsq of a unit spread over CH consecutive lanes: lane c = lane % CH holds its
// 2 * NQ words (values [c * 4 NQ, (c + 1) * 4 NQ) of the unit, NQ = 16 / CH) in w. The fma
// chain runs in unit_sumsq's order, each lane continuing the chain of lane c - 1, which a DPP
// move hands over (CH steps, every lane computing its part each step from what it was
// handed), so the total - on lane c = CH - 1 - has unit_sumsq's bits.
template <int CH>
__device__ __forceinline__ float scan_sumsq(const uint32_t (&w)[32 / CH], uint32_t c) {
    static_assert(CH == 2 || CH == 4 || CH == 8, "a unit over 2, 4 or 8 lanes");
    constexpr int NW = 32 / CH;
    float f[2 * NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) {
        f[2 * q] = bf16_lo(w[q]);
        f[2 * q + 1] = bf16_hi(w[q]);
    }
    float in = 0.0f;
    float t = 0.0f;
#pragma unroll
    for (int s = 0; s < CH; ++s) {
        t = in;
#pragma unroll
        for (int i = 0; i < 2 * NW; ++i) t = fmaf(f[i], f[i], t);
        if (s + 1 < CH) {
            const float prev = dpp_mov<0x111>(t);   // row_shr 1: lane i - 1
            in = c == 0u ? 0.0f : prev;
        }
    }
    return t;
}

// Sum of squares of one 64-element unit (8 x 16 bytes of bf16, k ascending).
__device__ __forceinline__ float unit_sumsq(const uint4 (&xv)[8]) {
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) ss = chunk_sumsq(xv[t], ss);
    return ss;
}

// Step 2 for one row whose unit partials are part[0 .. units): every lane gets the total.
__device__ __forceinline__ float row_sumsq(const float* part, uint32_t units, uint32_t lane) {
    float ss = 0.0f;
    for (uint32_t i = lane; i < units; i += 64u) ss += part[i];
    return butterfly_sum<32>(ss, lane);
}

__device__ __forceinline__ float rms_inverse(float ss, uint32_t k, float eps) {
    return 1.0f / sqrtf(ss / static_cast<float>(k) + eps);
}

// x <- bf16(x * inv) for the 64 values of a unit.
__device__ __forceinline__ void normalize_unit(uint4 (&xv)[8], float inv) {
#pragma unroll
    for (int t = 0; t < 8; ++t) normalize_chunk(xv[t], inv);
}

// x <- bf16(w * x) for the 64 values of a unit (the learned scale after normalize_unit).
__device__ __forceinline__ void weight_unit(uint4 (&xv)[8], const uint4 (&wv)[8]) {
#pragma unroll
    for (int t = 0; t < 8; ++t) weight_chunk(xv[t], wv[t]);
}

// A head row of D <= 512 values held 8 per lane (lane l: values [8l, 8l + 8), one 16-byte
// chunk; lanes l >= D / 8 hold zeros): c <- bf16(w * bf16(c * inv)) (no weight: bf16(c *
// inv)) with the bits of the unit-per-lane form. Each unit's fma chain runs over its 8 lanes
// (scan_sumsq), its total goes to all 8, and the units meet in the xor butterfly's order
// (offsets D / 128 .. 1 units apart, 8 lanes per unit; the unit-per-lane butterfly's steps
// below them add zeros). Every lane takes part.
__device__ __forceinline__ void norm_row_lanes8(uint4& c, const uint4* w, uint32_t D, float eps, uint32_t lane) {
    const uint32_t words[4] = {c.x, c.y, c.z, c.w};
    float ss = scan_sumsq<8>(words, lane & 7u);
    ss = dpp_mov<0xFF>(ss);                     // quad_perm [3, 3, 3, 3]: lane 4q + 3's
    const float up = dpp_mov<0x104>(ss);        // row_shl 4: lane i + 4
    ss = (lane & 4u) != 0u ? ss : up;           // lane 8u + 7's total on all 8 lanes
    const uint32_t units = D / 64u;
    if (units >= 8u) ss = add_lane_xor32(ss);
    if (units >= 4u) ss = add_lane_xor16(ss);
    if (units >= 2u) ss += xor_lanes<8>(ss, lane);
    if (lane < D / 8u) {
        normalize_chunk(c, rms_inverse(ss, D, eps));
        if (w != nullptr) weight_chunk(c, *w);
    }
}

}  // namespace hyperion::hip

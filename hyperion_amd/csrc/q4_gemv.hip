// Decode GEMV for MLX-affine Q4/g64 weights on gfx950 (m <= 4 activation rows).
//
// Replaces mlx::core::quantized_matmul(x, w, scales, biases, transpose=true, 64, 4,
// "affine") at decode (native/hyperion_mlx/src/weights.h:26-37, called from
// forward.cc:395,399,409,507 for q/k/v/o, forward.cc:338-343 for the MLP and
// forward.cc:137-152 for the tied LM head).
//
// HBM-bound design (0.5625 B per weight streamed once):
//  * A wave owns whole rows of W. Lane l reads half-groups (32 codes = 16 B) l and
//    l+64 of the row, so each dwordx4 load instruction covers 1 KB of contiguous
//    row bytes. Rows of W are contiguous, so a wave's consecutive rows stream
//    consecutive memory.
//  * Codes become bf16 pairs (128+q_a, 128+q_b) with one AND-OR on the packed word
//    (0x4300 is bf16 128.0 whose ulp is 1, so OR-ing a nibble into the mantissa
//    adds it exactly) and meet x through v_dot2c_f32_bf16: two MACs per VALU op with
//    fp32 accumulation. The +128 offset is removed per half-group with the
//    precomputed sum of x: part = s * (acc - 128*sum(x)) + b * sum(x).
//  * x lives in registers for the whole kernel, pre-permuted into the pairs the
//    nibble extraction produces ((x0,x4),(x1,x5),(x2,x6),(x3,x7) per word).
//  * Rows are reduced across the wave with DPP (quad perms, row mirrors,
//    row_bcast15/31), no LDS. For k > 4096 the row is split across 2 or 4 waves of
//    the workgroup and the partials meet in LDS.
#include "common.h"
#include "kernels.h"

namespace hyperion::hip {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
#ifndef HYP_GEMV_BLOCKS_PER_CU
#define HYP_GEMV_BLOCKS_PER_CU 2
#endif
constexpr uint32_t kGemvBlocksPerCU = HYP_GEMV_BLOCKS_PER_CU;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// (128 + nibble(shift), 128 + nibble(shift + 16)) as a bf16 pair.
__device__ __forceinline__ uint32_t code_pair(uint32_t w, int shift) {
    return ((w >> shift) & 0x000F000Fu) | 0x43004300u;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
    return v + __int_as_float(t);
}

// Sum over the 64 lanes; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xF>(v);   // row_half_mirror
    v = dpp_add<0x140, 0xF>(v);   // row_mirror
    v = dpp_add<0x142, 0xA>(v);   // row_bcast15 into rows 1 and 3
    v = dpp_add<0x143, 0xC>(v);   // row_bcast31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

struct GemvParams {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    const uint32_t* w2;   // fused gate/up: the up projection (same n, k)
    const uint16_t* s2;
    const uint16_t* b2;
    const uint16_t* x;
    uint16_t* y;
    uint32_t n;
    uint32_t k;
    uint32_t splits;      // waves sharing one row: 1, 2 or 4
    float cap;            // bf16 softcap constant
};

// Load the lane's x slice for half-group h and permute it into code-pair order.
template <int M>
__device__ __forceinline__ void load_x_half(const uint16_t* __restrict__ x, uint32_t k, uint32_t h,
                                            bool active, uint32_t (&xp)[M][2][16], float (&sx)[M][2],
                                            int slot) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // h is clamped into the row; inactive lanes zero what they loaded.
            uint4 v = *reinterpret_cast<const uint4*>(x + static_cast<size_t>(m) * k + h * 32u + j * 8u);
            if (!active) v = make_uint4(0u, 0u, 0u, 0u);
            xp[m][slot][4 * j + 0] = (v.x & 0xFFFFu) | (v.z << 16);
            xp[m][slot][4 * j + 1] = (v.x >> 16) | (v.z & 0xFFFF0000u);
            xp[m][slot][4 * j + 2] = (v.y & 0xFFFFu) | (v.w << 16);
            xp[m][slot][4 * j + 3] = (v.y >> 16) | (v.w & 0xFFFF0000u);
            sum += bf16_bits_to_f32(v.x & 0xFFFFu) + bf16_bits_to_f32(v.x >> 16);
            sum += bf16_bits_to_f32(v.y & 0xFFFFu) + bf16_bits_to_f32(v.y >> 16);
            sum += bf16_bits_to_f32(v.z & 0xFFFFu) + bf16_bits_to_f32(v.z >> 16);
            sum += bf16_bits_to_f32(v.w & 0xFFFFu) + bf16_bits_to_f32(v.w >> 16);
        }
        sx[m][slot] = sum;
    }
}

// One half-group (four packed words) against the permuted x of one row m.
__device__ __forceinline__ float half_group_dot(const uint4& wv, const uint32_t* xp) {
    float a0 = 0.0f;
    float a1 = 0.0f;
    a0 = dot2_bf16(code_pair(wv.x, 0), xp[0], a0);
    a1 = dot2_bf16(code_pair(wv.x, 4), xp[1], a1);
    a0 = dot2_bf16(code_pair(wv.x, 8), xp[2], a0);
    a1 = dot2_bf16(code_pair(wv.x, 12), xp[3], a1);
    a0 = dot2_bf16(code_pair(wv.y, 0), xp[4], a0);
    a1 = dot2_bf16(code_pair(wv.y, 4), xp[5], a1);
    a0 = dot2_bf16(code_pair(wv.y, 8), xp[6], a0);
    a1 = dot2_bf16(code_pair(wv.y, 12), xp[7], a1);
    a0 = dot2_bf16(code_pair(wv.z, 0), xp[8], a0);
    a1 = dot2_bf16(code_pair(wv.z, 4), xp[9], a1);
    a0 = dot2_bf16(code_pair(wv.z, 8), xp[10], a0);
    a1 = dot2_bf16(code_pair(wv.z, 12), xp[11], a1);
    a0 = dot2_bf16(code_pair(wv.w, 0), xp[12], a0);
    a1 = dot2_bf16(code_pair(wv.w, 4), xp[13], a1);
    a0 = dot2_bf16(code_pair(wv.w, 8), xp[14], a0);
    a1 = dot2_bf16(code_pair(wv.w, 12), xp[15], a1);
    return a0 + a1;
}

// Rows a wave has in flight per iteration: enough bytes in flight to cover HBM
// latency, within the register budget left by x.
template <int M, bool DUAL>
constexpr int rows_per_stream() {
    return (M * (DUAL ? 2 : 1) <= 2) ? 4 : ((M * (DUAL ? 2 : 1) <= 4) ? 2 : 1);
}

template <int NW, int RB>
struct RowRegs {
    uint4 w[NW][RB][2];
    uint32_t s[NW][RB][2];
    uint32_t b[NW][RB][2];
};

// Loads for rows base+stream*RB .. +RB-1. Indices are clamped into the matrix so every
// load is unconditional (no exec-masked loads, no forced waits); rows past n are never
// stored and lanes past the row's half-groups are zeroed at use.
template <int NW, int RB>
__device__ __forceinline__ void load_rows(const GemvParams& p, uint32_t first_row, uint32_t h0c, uint32_t h1c,
                                          RowRegs<NW, RB>& r) {
    const size_t row_words = p.k / 8u;
    const uint32_t G = p.k / 64u;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const uint32_t row = min(first_row + rb, p.n - 1u);
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            const uint32_t* wrow = (q == 0 ? p.w : p.w2) + static_cast<size_t>(row) * row_words;
            const uint16_t* srow = (q == 0 ? p.s : p.s2) + static_cast<size_t>(row) * G;
            const uint16_t* brow = (q == 0 ? p.b : p.b2) + static_cast<size_t>(row) * G;
            r.w[q][rb][0] = *reinterpret_cast<const uint4*>(wrow + h0c * 4u);
            r.w[q][rb][1] = *reinterpret_cast<const uint4*>(wrow + h1c * 4u);
            r.s[q][rb][0] = srow[h0c >> 1];
            r.s[q][rb][1] = srow[h1c >> 1];
            r.b[q][rb][0] = brow[h0c >> 1];
            r.b[q][rb][1] = brow[h1c >> 1];
        }
    }
}

template <int M, bool DUAL, int EPI>
__global__ __launch_bounds__(kThreads) void q4_gemv_kernel(GemvParams p) {
    constexpr int NW = DUAL ? 2 : 1;
    constexpr int RB = rows_per_stream<M, DUAL>();
    __shared__ float red[2][kWaves][RB][NW][M];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t S = p.splits;
    const uint32_t split = wave % S;
    const uint32_t stream = wave / S;
    const uint32_t streams = kWaves / S;
    const uint32_t k = p.k;
    const uint32_t HG = k / 32u;
    const uint32_t HGs = (HG + S - 1u) / S;
    const uint32_t hbase = split * HGs;
    const uint32_t hend = min(HG, hbase + HGs);
    const uint32_t h0 = hbase + lane;
    const uint32_t h1 = h0 + 64u;
    const bool act0 = h0 < hend;
    const bool act1 = h1 < hend;
    const uint32_t h0c = act0 ? h0 : hbase;
    const uint32_t h1c = act1 ? h1 : hbase;

    const uint32_t rows_per_iter = streams * RB;
    const uint32_t stride = gridDim.x * rows_per_iter;
    uint32_t base = blockIdx.x * rows_per_iter;

    // x first: loads retire in issue order, so x can be consumed while the first
    // rows are still in flight.
    uint32_t xp[M][2][16];
    float sx[M][2];
    load_x_half<M>(p.x, k, h0c, act0, xp, sx, 0);
    load_x_half<M>(p.x, k, h1c, act1, xp, sx, 1);

    RowRegs<NW, RB> cur;
    load_rows<NW, RB>(p, base + stream * RB, h0c, h1c, cur);

    uint32_t parity = 0;
    while (true) {
        const uint32_t next = base + stride;
        const bool more = next < p.n;   // uniform across the workgroup
        RowRegs<NW, RB> nxt;
        if (more) load_rows<NW, RB>(p, next + stream * RB, h0c, h1c, nxt);

        float tot[NW][RB][M];
#pragma unroll
        for (int q = 0; q < NW; ++q) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float sc[2], bi[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const bool act = hh == 0 ? act0 : act1;
                    sc[hh] = act ? bf16_bits_to_f32(cur.s[q][rb][hh]) : 0.0f;
                    bi[hh] = act ? bf16_bits_to_f32(cur.b[q][rb][hh]) : 0.0f;
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float part = 0.0f;
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const float acc = half_group_dot(cur.w[q][rb][hh], xp[m][hh]);
                        const float sxv = sx[m][hh];
                        part = fmaf(sc[hh], acc - 128.0f * sxv, part);
                        part = fmaf(bi[hh], sxv, part);
                    }
                    tot[q][rb][m] = wave_sum(part);
                }
            }
        }

        if (S > 1u) {
            if (lane == 0u) {
#pragma unroll
                for (int q = 0; q < NW; ++q)
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int m = 0; m < M; ++m) red[parity][wave][rb][q][m] = tot[q][rb][m];
            }
            __syncthreads();
            if (split == 0u) {
#pragma unroll
                for (int q = 0; q < NW; ++q)
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            float v = 0.0f;
                            for (uint32_t s2 = 0; s2 < S; ++s2) v += red[parity][wave + s2][rb][q][m];
                            tot[q][rb][m] = v;
                        }
            }
            parity ^= 1u;
        }

        if (split == 0u && lane < static_cast<uint32_t>(RB * M)) {
            // Lane (rb * M + m) stores one output.
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    if (lane != static_cast<uint32_t>(rb * M + m)) continue;
                    const uint32_t r = base + stream * RB + rb;
                    if (r >= p.n) continue;
                    float out = round_bf16(tot[0][rb][m]);
                    if constexpr (DUAL) {
                        const float up = round_bf16(tot[NW - 1][rb][m]);
                        out = round_bf16(gelu_tanh_bf16_chain(out) * up);
                    } else if constexpr (EPI == static_cast<int>(Epilogue::kSoftcap)) {
                        out = softcap_bf16(out, p.cap);
                    }
                    p.y[static_cast<size_t>(m) * p.n + r] = f32_to_bf16_bits(out);
                }
            }
        }
        if (!more) break;
        cur = nxt;
        base = next;
    }
}

template <int M>
void launch_m(const GemvParams& p, bool dual, Epilogue epi, uint32_t max_blocks, hipStream_t stream) {
    const uint32_t streams = kWaves / p.splits;
    auto grid_for = [&](int rb) {
        const uint32_t rpi = streams * static_cast<uint32_t>(rb);
        return dim3(min((p.n + rpi - 1u) / rpi, max_blocks));
    };
    if (dual) {
        hipLaunchKernelGGL((q4_gemv_kernel<M, true, 0>), grid_for(rows_per_stream<M, true>()), dim3(kThreads), 0,
                           stream, p);
    } else if (epi == Epilogue::kSoftcap) {
        hipLaunchKernelGGL((q4_gemv_kernel<M, false, 1>), grid_for(rows_per_stream<M, false>()), dim3(kThreads), 0,
                           stream, p);
    } else {
        hipLaunchKernelGGL((q4_gemv_kernel<M, false, 0>), grid_for(rows_per_stream<M, false>()), dim3(kThreads), 0,
                           stream, p);
    }
}

}  // namespace

void launch_q4_gemv(const Q4Matrix& w, const Q4Matrix* up, const uint16_t* x, uint32_t m,
                    uint16_t* y, Epilogue epi, float cap_bf16, hipStream_t stream) {
    GemvParams p{};
    p.w = w.w;
    p.s = w.scales;
    p.b = w.biases;
    p.w2 = up ? up->w : nullptr;
    p.s2 = up ? up->scales : nullptr;
    p.b2 = up ? up->biases : nullptr;
    p.x = x;
    p.y = y;
    p.n = w.n;
    p.k = w.k;
    p.cap = cap_bf16;
    const uint32_t hg = w.k / 32u;
    p.splits = hg <= 128u ? 1u : (hg <= 256u ? 2u : 4u);
    // Persistent grid: kGemvBlocksPerCU workgroups per CU loop over the rows.
    const uint32_t max_blocks = device_compute_units() * kGemvBlocksPerCU;
    const bool dual = up != nullptr;
    switch (m) {
        case 1: launch_m<1>(p, dual, epi, max_blocks, stream); break;
        case 2: launch_m<2>(p, dual, epi, max_blocks, stream); break;
        case 3: launch_m<3>(p, dual, epi, max_blocks, stream); break;
        case 4: launch_m<4>(p, dual, epi, max_blocks, stream); break;
        default: throw NativeError(HYP_STATUS_INTERNAL, "gemv launched with m outside 1..4");
    }
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

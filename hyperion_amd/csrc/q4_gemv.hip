// Decode GEMV for MLX-affine Q4/g64 weights on gfx950 (m <= 4 activation rows).
//
// Replaces mlx::core::quantized_matmul(x, w, scales, biases, transpose=true, 64, 4,
// "affine") at decode (native/hyperion_mlx/src/weights.h:26-37, called from
// forward.cc:395,399,409,507 for q/k/v/o, forward.cc:338-343 for the MLP and
// forward.cc:137-152 for the tied LM head).
//
// HBM-bound design (0.5625 B per weight streamed exactly once):
//  * A wave owns R consecutive rows of W (R * 1920 contiguous bytes at k = 3840), or
//    one K-slice of them when S waves split a row. Lane l reads half-groups
//    (32 codes = 16 B) l and l+64 of its slice, so each dwordx4 load instruction
//    covers 1 KB of contiguous row bytes.
//  * Every load of the wave is issued before any arithmetic: x first (it is L2
//    resident), then the rows in order. Loads retire in issue order, so the math of
//    row r waits only for row r's bytes while rows r+1.. are still in flight, and a
//    whole CU's share of W is requested at once. The grid is one wave per R rows
//    (no persistent loop), thousands of waves, so the tail of one wave's arithmetic
//    overlaps other waves' loads.
//  * Codes become bf16 pairs (128+q_a, 128+q_b) with one AND-OR on the packed word
//    (0x4300 is bf16 128.0 whose ulp is 1, so OR-ing a nibble into the mantissa
//    adds it exactly) and meet x through v_dot2_f32_bf16: two MACs per VALU op with
//    fp32 accumulation. The +128 offset is removed per half-group with the
//    precomputed sum of x: part = s * (acc - 128*sum(x)) + b * sum(x).
//  * x lives in registers, pre-permuted into the pairs the nibble extraction
//    produces ((x0,x4),(x1,x5),(x2,x6),(x3,x7) per word).
//  * Rows are reduced across the wave with DPP (quad perms, row mirrors,
//    row_bcast15/31), no LDS. When S > 1 waves share a row, their partials meet
//    in LDS.
#include "common.h"
#include "kernels.h"

namespace hyperion::hip {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// (w & mask) | bits. With mask and bits held in VGPRs (see the kernel), this is one
// v_and_or_b32; as literals it would split into two VOP2 ops, because GFX9 VOP3
// encodings take no literal constants and read at most one SGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t mask, uint32_t bits) {
    return (w & mask) | bits;
}

// (128 + nibble(shift), 128 + nibble(shift + 16)) as a bf16 pair: 0x4300 is bf16
// 128.0, whose ulp is 1, so OR-ing a nibble into the mantissa adds it exactly.
__device__ __forceinline__ uint32_t code_pair(uint32_t w, int shift, uint32_t mask, uint32_t bits) {
    return and_or(shift == 0 ? w : (w >> shift), mask, bits);
}

constexpr uint32_t kNibbleMask = 0x000F000Fu;
constexpr uint32_t kMagic128 = 0x43004300u;   // bf16 pair (128.0, 128.0)
constexpr uint32_t kOnePair = 0x3F803F80u;    // bf16 pair (1.0, 1.0)

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

// One half-group (four packed words) against the permuted x of one row m.
__device__ __forceinline__ float half_group_dot(const uint4& wv, const uint32_t* xp, uint32_t mask, uint32_t bits) {
    float a0 = 0.0f;
    float a1 = 0.0f;
    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a0 = dot2_bf16(code_pair(words[i], 0, mask, bits), xp[4 * i + 0], a0);
        a1 = dot2_bf16(code_pair(words[i], 4, mask, bits), xp[4 * i + 1], a1);
        a0 = dot2_bf16(code_pair(words[i], 8, mask, bits), xp[4 * i + 2], a0);
        a1 = dot2_bf16(code_pair(words[i], 12, mask, bits), xp[4 * i + 3], a1);
    }
    return a0 + a1;
}

// y[m, row0 .. row0+R) for one wave: R rows (NW matrices) x H half-groups per lane.
template <int M, int R, int H, bool DUAL, int EPI>
__global__ __launch_bounds__(kThreads) void q4_gemv_kernel(GemvParams p) {
    constexpr int NW = DUAL ? 2 : 1;
    __shared__ float red[kWaves][NW][R][M];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t S = p.splits;
    const uint32_t split = wave % S;
    const uint32_t set = wave / S;
    const uint32_t row0 = (blockIdx.x * (kWaves / S) + set) * R;
    const uint32_t k = p.k;
    const uint32_t HG = k / 32u;
    const uint32_t HGs = (HG + S - 1u) / S;
    const uint32_t hbase = split * HGs;
    const uint32_t hend = min(HG, hbase + HGs);
    bool act[H];
    uint32_t hc[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
        const uint32_t hh = hbase + lane + 64u * h;
        act[h] = hh < hend;
        hc[h] = act[h] ? hh : HG - 1u;   // clamped: every load stays inside the row
    }

    // x first (L2 resident), then the rows in order.
    uint32_t xp[H][M][16];
    float sx[H][M];
    uint4 xv[H][M][4];
#pragma unroll
    for (int h = 0; h < H; ++h)
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xv[h][m][j] = *reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(m) * k + hc[h] * 32u + j * 8u);

    const size_t row_words = k / 8u;
    const uint32_t G = k / 64u;
    uint4 wv[R][NW][H];
    uint32_t sr[R][NW][H];
    uint32_t br[R][NW][H];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = min(row0 + r, p.n - 1u);   // rows past n are loaded, never stored
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            const uint32_t* wrow = (q == 0 ? p.w : p.w2) + static_cast<size_t>(row) * row_words;
            const uint16_t* srow = (q == 0 ? p.s : p.s2) + static_cast<size_t>(row) * G;
            const uint16_t* brow = (q == 0 ? p.b : p.b2) + static_cast<size_t>(row) * G;
#pragma unroll
            for (int h = 0; h < H; ++h) {
                wv[r][q][h] = *reinterpret_cast<const uint4*>(wrow + hc[h] * 4u);
                sr[r][q][h] = srow[hc[h] >> 1];
                br[r][q][h] = brow[hc[h] >> 1];
            }
        }
    }

#pragma unroll
    for (int h = 0; h < H; ++h) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            // (x0,x4),(x1,x5),(x2,x6),(x3,x7) of each 8-element word, one v_perm_b32 each;
            // sum(x) through the same dot2 unit against (1, 1).
            float s0 = 0.0f;
            float s1 = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint4 q = xv[h][m][j];
                if (!act[h]) q = make_uint4(0u, 0u, 0u, 0u);
                xp[h][m][4 * j + 0] = __builtin_amdgcn_perm(q.z, q.x, 0x05040100u);
                xp[h][m][4 * j + 1] = __builtin_amdgcn_perm(q.z, q.x, 0x07060302u);
                xp[h][m][4 * j + 2] = __builtin_amdgcn_perm(q.w, q.y, 0x05040100u);
                xp[h][m][4 * j + 3] = __builtin_amdgcn_perm(q.w, q.y, 0x07060302u);
                s0 = dot2_bf16(q.x, kOnePair, s0);
                s1 = dot2_bf16(q.y, kOnePair, s1);
                s0 = dot2_bf16(q.z, kOnePair, s0);
                s1 = dot2_bf16(q.w, kOnePair, s1);
            }
            sx[h][m] = s0 + s1;
        }
    }

    // Opaque VGPR values, so (w & mask) | bits selects v_and_or_b32 (see and_or).
    uint32_t mask = kNibbleMask;
    uint32_t bits = kMagic128;
    asm volatile("" : "+v"(mask), "+v"(bits));

    float tot[R][NW][M];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            float sc[H], bi[H];
#pragma unroll
            for (int h = 0; h < H; ++h) {
                sc[h] = act[h] ? bf16_bits_to_f32(sr[r][q][h]) : 0.0f;
                bi[h] = act[h] ? bf16_bits_to_f32(br[r][q][h]) : 0.0f;
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float part = 0.0f;
#pragma unroll
                for (int h = 0; h < H; ++h) {
                    const float acc = half_group_dot(wv[r][q][h], xp[h][m], mask, bits);
                    part = fmaf(sc[h], acc - 128.0f * sx[h][m], part);
                    part = fmaf(bi[h], sx[h][m], part);
                }
                tot[r][q][m] = wave_sum(part);
            }
        }
    }

    if (S > 1u) {
        if (lane == 0u) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int q = 0; q < NW; ++q)
#pragma unroll
                    for (int m = 0; m < M; ++m) red[wave][q][r][m] = tot[r][q][m];
        }
        __syncthreads();
        if (split == 0u) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int q = 0; q < NW; ++q)
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float v = 0.0f;
                        for (uint32_t s2 = 0; s2 < S; ++s2) v += red[wave + s2][q][r][m];
                        tot[r][q][m] = v;
                    }
        }
    }

    if (split == 0u && lane < static_cast<uint32_t>(R * M)) {
        // Lane (r * M + m) stores one output.
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if (lane != static_cast<uint32_t>(r * M + m)) continue;
                const uint32_t row = row0 + r;
                if (row >= p.n) continue;
                float out = round_bf16(tot[r][0][m]);
                if constexpr (DUAL) {
                    const float up = round_bf16(tot[r][NW - 1][m]);
                    out = round_bf16(gelu_tanh_bf16_chain(out) * up);
                } else if constexpr (EPI == static_cast<int>(Epilogue::kSoftcap)) {
                    out = softcap_bf16(out, p.cap);
                }
                p.y[static_cast<size_t>(m) * p.n + row] = f32_to_bf16_bits(out);
            }
        }
    }
}

template <int M, int R, int H>
void launch_mrh(const GemvParams& p, bool dual, Epilogue epi, hipStream_t stream) {
    const uint32_t rows_per_block = static_cast<uint32_t>(R) * (kWaves / p.splits);
    const dim3 grid((p.n + rows_per_block - 1u) / rows_per_block);
    if (dual) {
        hipLaunchKernelGGL((q4_gemv_kernel<M, R, H, true, 0>), grid, dim3(kThreads), 0, stream, p);
    } else if (epi == Epilogue::kSoftcap) {
        hipLaunchKernelGGL((q4_gemv_kernel<M, R, H, false, 1>), grid, dim3(kThreads), 0, stream, p);
    } else {
        hipLaunchKernelGGL((q4_gemv_kernel<M, R, H, false, 0>), grid, dim3(kThreads), 0, stream, p);
    }
}

template <int M, int R>
void launch_mr(const GemvParams& p, uint32_t h, bool dual, Epilogue epi, hipStream_t stream) {
    if (h == 1u) {
        launch_mrh<M, R, 1>(p, dual, epi, stream);
    } else {
        launch_mrh<M, R, 2>(p, dual, epi, stream);
    }
}

template <int M>
void launch_m(const GemvParams& p, const GemvConfig& c, bool dual, Epilogue epi, hipStream_t stream) {
    switch (c.rows) {
        case 1: launch_mr<M, 1>(p, c.halves, dual, epi, stream); break;
        case 2: launch_mr<M, 2>(p, c.halves, dual, epi, stream); break;
        case 4: launch_mr<M, 4>(p, c.halves, dual, epi, stream); break;
        case 8:
            if constexpr (M <= 2) {
                launch_mr<M, 8>(p, c.halves, dual, epi, stream);
                break;
            }
            [[fallthrough]];
        default: throw NativeError(HYP_STATUS_INTERNAL, "gemv: unsupported rows per wave");
    }
}

}  // namespace

GemvConfig choose_gemv_config(uint32_t m, uint32_t n, uint32_t k, bool dual) {
    const uint32_t hg = k / 32u;
    GemvConfig c{};
    // Rows per wave: enough bytes in flight per wave, within the registers x leaves.
    const uint32_t weight_rows = m * (dual ? 2u : 1u);
    c.rows = weight_rows <= 1u ? 4u : (weight_rows <= 2u ? 4u : 2u);
    // Waves per row: the fewest whose half-groups fit 2 per lane; more when n is
    // too small to give every CU several waves.
    c.splits = hg <= 128u ? 1u : (hg <= 256u ? 2u : 4u);
    const uint32_t target_waves = device_compute_units() * 8u;
    while (c.splits < 4u && (n / c.rows) * c.splits < target_waves) c.splits *= 2u;
    const uint32_t per_split = (hg + c.splits - 1u) / c.splits;
    c.halves = per_split <= 64u ? 1u : 2u;
    return c;
}

void launch_q4_gemv_config(const Q4Matrix& w, const Q4Matrix* up, const uint16_t* x, uint32_t m, uint16_t* y,
                           Epilogue epi, float cap_bf16, const GemvConfig& c, hipStream_t stream) {
    const uint32_t hg = w.k / 32u;
    HYP_REQUIRE(c.splits == 1u || c.splits == 2u || c.splits == 4u, HYP_STATUS_INTERNAL, "gemv: bad split count");
    HYP_REQUIRE(c.halves == 1u || c.halves == 2u, HYP_STATUS_INTERNAL, "gemv: bad half-groups per lane");
    HYP_REQUIRE((hg + c.splits - 1u) / c.splits <= 64u * c.halves, HYP_STATUS_INTERNAL,
                "gemv: k does not fit the split configuration");
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
    p.splits = c.splits;
    const bool dual = up != nullptr;
    switch (m) {
        case 1: launch_m<1>(p, c, dual, epi, stream); break;
        case 2: launch_m<2>(p, c, dual, epi, stream); break;
        case 3: launch_m<3>(p, c, dual, epi, stream); break;
        case 4: launch_m<4>(p, c, dual, epi, stream); break;
        default: throw NativeError(HYP_STATUS_INTERNAL, "gemv launched with m outside 1..4");
    }
    HYP_HIP_CHECK(hipGetLastError());
}

void launch_q4_gemv(const Q4Matrix& w, const Q4Matrix* up, const uint16_t* x, uint32_t m, uint16_t* y,
                    Epilogue epi, float cap_bf16, hipStream_t stream) {
    launch_q4_gemv_config(w, up, x, m, y, epi, cap_bf16, choose_gemv_config(m, w.n, w.k, up != nullptr), stream);
}

}  // namespace hyperion::hip

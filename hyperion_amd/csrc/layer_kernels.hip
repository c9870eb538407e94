// The per-token work of a decoder layer between its projections, on gfx950:
//
//  * attn_prepare_kernel - ForwardPass::attention from the q/k/v projections to the cache
//    append (native/hyperion_mlx/src/forward.cc:395-459): q <- rope(q_norm(q)) in place;
//    K slot <- rope(k_norm(k_raw)); V slot <- v_norm(v_raw), v_raw = k_raw on K = V global
//    layers (forward.cc:403-412). A wave takes 64 / (D/64) head rows (q, K or V rows of any
//    tokens): D/64 lanes normalise a row (lane owns a 64-value unit, the order of
//    q4_rmsnorm.h), the q and K rows are staged in LDS and their pairs (i, i + D/2) rotated
//    with (cos, sin) computed in place or read from a table that rope_table_kernel filled
//    with the same arithmetic (chunks of up to 16 tokens: attn_prepare_head_kernel, one wave
//    per head). Bits: those of rms_norm_rows_kernel followed by rope_kernel and
//    kv_write_kernel.
//
//  * residual_norm_kernel - the Gemma sandwich around a block (forward.cc:518-529):
//    residual <- bf16(residual + rms_norm(branch, w_post)), then optionally
//    residual <- bf16(residual * layer_scalar), then optionally next <- rms_norm(residual,
//    w_next) (the following block's input norm). One workgroup per row, thread u owning unit
//    u (for rows of at most 64 units, residual_norm_lanes_kernel spreads each unit over four
//    lanes; from 64 rows on, residual_norm_tiled_kernel, the unit-per-thread arithmetic behind
//    coalesced loads and stores through LDS); both statistics in the order of q4_rmsnorm.h,
//    so each norm has the bits of launch_rms_normalize and of the skinny matmul's
//    normalising prologue.
#include "common.h"
#include "kernels.h"
#include "q4_rmsnorm.h"

namespace hyperion::hip {
namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kWaves = kThreads / 64u;
constexpr uint32_t kMaxHeadDim = 512;
// Chunks of at most this many tokens take attn_prepare_head_kernel (measured on a 12B global
// layer, one token: 7.1 us against 11.5 for the packed rows; 1024-token chunks: 20.5 us packed
// against 37.6).
constexpr uint32_t kPrepareHeadMaxTokens = 16;

struct PrepareParams {
    const uint32_t* pos;      // non-null: offset = *pos
    const float2* rope_cs;    // non-null: (cos, sin) [positions][D/2], rope_table_kernel's values
    uint16_t* q;              // [L][H][D], in place
    const uint16_t* k_raw;    // [L][KVH][D]
    const uint16_t* v_raw;    // [L][KVH][D] or null (K = V: v_norm of k_raw)
    const uint16_t* q_w;      // [D]
    const uint16_t* k_w;      // [D]
    uint16_t* cache_k;        // [cap][KVH][D]
    uint16_t* cache_v;
    uint32_t L, H, KVH, D, rotated, offset, cap, first_cached;
    double base;
    float eps;
};

// rope_kernel's angle arithmetic: inv_freq in double rounded to fp32, theta in fp32, cos and
// sin in double rounded to fp32.
__device__ __forceinline__ float2 rope_angle(uint32_t pos, uint32_t i, uint32_t D, uint32_t rotated, double base) {
    const float inv = 2u * i < rotated ? static_cast<float>(pow(base, -2.0 * i / static_cast<double>(D))) : 0.0f;
    const float theta = static_cast<float>(pos) * inv;
    return make_float2(static_cast<float>(cos(static_cast<double>(theta))),
                       static_cast<float>(sin(static_cast<double>(theta))));
}

// Short chunks (a decode step: a few dozen rows, which attn_prepare_kernel would give to a
// few waves): grid (L, ceil((H + KVH) / 4)), wave w of workgroup (t, y) takes head 4y + w
// of token t (q heads first, then kv heads), 8 values per lane in its norms
// (norm_row_lanes8) and all 64 lanes in its RoPE. The same bits.
__global__ __launch_bounds__(kThreads) void attn_prepare_head_kernel(PrepareParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t head[kWaves][kMaxHeadDim];
    const uint32_t t = blockIdx.x;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t D = p.D;
    const uint32_t half = D / 2u;
    const uint32_t pos = (p.pos != nullptr ? *p.pos : p.offset) + t;
    const uint32_t hh = blockIdx.y * kWaves + wave;
    const bool is_q = hh < p.H;
    const bool active = hh < p.H + p.KVH && (is_q || t >= p.first_cached);   // wave-uniform
    const size_t slot = static_cast<size_t>(pos % p.cap);
    uint16_t* hb = head[wave];
    uint16_t* dst = nullptr;

    // This lane's pairs i = lane + 64 j: their (cos, sin), looked up or computed.
    float2 cs[kMaxHeadDim / 128];
#pragma unroll
    for (uint32_t j = 0; j < kMaxHeadDim / 128; ++j) {
        const uint32_t i = lane + 64u * j;
        cs[j] = make_float2(1.0f, 0.0f);
        if (active && i < half) {
            cs[j] = p.rope_cs != nullptr ? p.rope_cs[static_cast<size_t>(pos) * half + i]
                                         : rope_angle(pos, i, D, p.rotated, p.base);
        }
    }
    if (active) {
        // 8 values per lane (norm_row_lanes8): every lane of the wave in the norm.
        const bool has = lane < D / 8u;
        uint4 xc = make_uint4(0u, 0u, 0u, 0u);
        uint4 wc = make_uint4(0u, 0u, 0u, 0u);
        const uint32_t kh = hh - p.H;
        const size_t kv_row = (static_cast<size_t>(t) * p.KVH + kh) * D;
        if (is_q) {
            dst = p.q + (static_cast<size_t>(t) * p.H + hh) * D;
            if (has) {
                xc = reinterpret_cast<const uint4*>(dst)[lane];
                wc = reinterpret_cast<const uint4*>(p.q_w)[lane];
            }
        } else {
            // V: the weightless norm straight into the cache slot; its loads and K's are
            // issued together.
            uint4 vc = make_uint4(0u, 0u, 0u, 0u);
            if (has) {
                vc = reinterpret_cast<const uint4*>(p.v_raw != nullptr ? p.v_raw + kv_row : p.k_raw + kv_row)[lane];
                xc = reinterpret_cast<const uint4*>(p.k_raw + kv_row)[lane];
                wc = reinterpret_cast<const uint4*>(p.k_w)[lane];
            }
            norm_row_lanes8(vc, nullptr, D, p.eps, lane);
            if (has) reinterpret_cast<uint4*>(p.cache_v + (slot * p.KVH + kh) * D)[lane] = vc;
            dst = p.cache_k + (slot * p.KVH + kh) * D;
        }
        norm_row_lanes8(xc, &wc, D, p.eps, lane);
        if (has) reinterpret_cast<uint4*>(hb)[lane] = xc;
    }
    __syncthreads();   // the staged head is visible to every lane of its wave
    if (active) {
#pragma unroll
        for (uint32_t j = 0; j < kMaxHeadDim / 128; ++j) {
            const uint32_t i = lane + 64u * j;
            if (i >= half) break;
            const float x1 = bf16_bits_to_f32(hb[i]);
            const float x2 = bf16_bits_to_f32(hb[i + half]);
            const float a1 = x1 * cs[j].x;
            const float a2 = x2 * cs[j].y;
            const float b1 = x1 * cs[j].y;
            const float b2 = x2 * cs[j].x;
            dst[i] = f32_to_bf16_bits(a1 - a2);
            dst[i + half] = f32_to_bf16_bits(b1 + b2);
        }
    }
}

// Rows of the flattened [token][H + 2 KVH] space (q heads, then each kv head's K, then its V),
// D/64 lanes per row, one 64-value unit per lane: a wave takes 64 / (D/64) rows (16 at
// head_dim 256) instead of one head, so its lanes and loads are all busy (a 1024-token
// chunk of a 12B sliding layer: 37 us with one wave per head). Per row: the unit sums of
// squares of q4_rmsnorm.h met in a butterfly over the row's D/64 lanes (a 64-lane butterfly
// with the other lanes at zero adds the same partial sums in the same order), bf16(x * inv),
// bf16(w * x), then the RoPE of rope_kernel on the q and K rows. Q rows are
// normalised and rotated in place, K rows into their cache slot, V rows normalised (no
// weight) into theirs.
template <uint32_t D>
__global__ __launch_bounds__(kThreads) void attn_prepare_kernel(PrepareParams p) {
    constexpr uint32_t kU = D / 64u;            // lanes (units) per row
    constexpr uint32_t kR = 64u / kU;           // rows per wave
    constexpr uint32_t kHalf = D / 2u;
    constexpr uint32_t kHalfChunks = kHalf / 8u;
    constexpr uint32_t kRopeRows = 64u / kHalfChunks;   // rows one RoPE pass covers
    __shared__ __attribute__((aligned(16))) uint16_t stage[kWaves][kR * D];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t per_tok = p.H + 2u * p.KVH;
    const uint32_t total = p.L * per_tok;   // < 2^31 (checked on the host)
    const uint32_t row0 = (blockIdx.x * kWaves + wave) * kR;
    if (row0 >= total) return;   // wave-uniform; no workgroup barrier below
    const uint32_t base_pos = p.pos != nullptr ? *p.pos : p.offset;
    uint16_t* sw = stage[wave];

    // Row idx: its token, kind (0 q, 1 K, 2 V), head, and whether it is written.
    const auto row_of = [&](uint32_t idx, uint32_t& t, uint32_t& kind, uint32_t& hd, bool& active) {
        const bool live = idx < total;
        t = live ? idx / per_tok : 0u;
        const uint32_t hh = live ? idx - t * per_tok : 0u;
        kind = hh < p.H ? 0u : (hh < p.H + p.KVH ? 1u : 2u);
        hd = kind == 0u ? hh : (kind == 1u ? hh - p.H : hh - p.H - p.KVH);
        active = live && (kind == 0u || t >= p.first_cached);
    };
    const uint32_t r = lane / kU;
    const uint32_t u = lane - r * kU;
    uint32_t t, kind, hd;
    bool active;
    row_of(row0 + r, t, kind, hd, active);
    const size_t kv_row = (static_cast<size_t>(t) * p.KVH + hd) * D;
    const uint16_t* src = kind == 0u ? p.q + (static_cast<size_t>(t) * p.H + hd) * D
                          : kind == 1u ? p.k_raw + kv_row
                                       : (p.v_raw != nullptr ? p.v_raw : p.k_raw) + kv_row;
    const uint16_t* w = kind == 0u ? p.q_w : (kind == 1u ? p.k_w : nullptr);
    uint4 xv[8];
    uint4 wv[8];
    if (active) {
        const uint4* s4 = reinterpret_cast<const uint4*>(src + u * 64u);
#pragma unroll
        for (int q = 0; q < 8; ++q) xv[q] = s4[q];
        if (w != nullptr) {
            const uint4* w4 = reinterpret_cast<const uint4*>(w + u * 64u);
#pragma unroll
            for (int q = 0; q < 8; ++q) wv[q] = w4[q];
        }
    }
    float ss = active ? unit_sumsq(xv) : 0.0f;
    ss = butterfly_sum<kU / 2u>(ss, lane);
    const size_t slot_row = (static_cast<size_t>((base_pos + t) % p.cap) * p.KVH + hd) * D;
    if (active) {
        normalize_unit(xv, rms_inverse(ss, D, p.eps));
        if (w != nullptr) weight_unit(xv, wv);
        uint4* dst = kind == 2u ? reinterpret_cast<uint4*>(p.cache_v + slot_row + u * 64u)
                                : reinterpret_cast<uint4*>(sw + r * D + u * 64u);
#pragma unroll
        for (int q = 0; q < 8; ++q) dst[q] = xv[q];
    }
    // The wave's LDS instructions execute in order: only the compiler must keep the RoPE's
    // reads after the writes above (and the stores below after the RoPE's writes).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // RoPE of the staged q and K rows: a lane takes 8 consecutive pairs (i, i + D/2).
    {
        const uint32_t c = lane % kHalfChunks;
        for (uint32_t rr = lane / kHalfChunks; rr < kR; rr += kRopeRows) {
            uint32_t tr, kr, hr;
            bool ar;
            row_of(row0 + rr, tr, kr, hr, ar);
            if (!ar || kr == 2u) continue;
            const uint32_t pos = base_pos + tr;
            float2 cs8[8];
            if (p.rope_cs != nullptr) {
                const float4* t4 = reinterpret_cast<const float4*>(p.rope_cs + static_cast<size_t>(pos) * kHalf + c * 8u);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float4 v = t4[e];
                    cs8[2 * e] = make_float2(v.x, v.y);
                    cs8[2 * e + 1] = make_float2(v.z, v.w);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) cs8[e] = rope_angle(pos, c * 8u + e, D, p.rotated, p.base);
            }
            uint4* lo = reinterpret_cast<uint4*>(sw + rr * D + c * 8u);
            uint4* hi = reinterpret_cast<uint4*>(sw + rr * D + kHalf + c * 8u);
            const uint4 a = *lo;
            const uint4 b = *hi;
            const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
            const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
            uint32_t ow[4];
            uint32_t pw[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t o2[2];
                uint32_t p2[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float2 cs = cs8[2 * q + h];
                    const float x1 = bf16_bits_to_f32((aw[q] >> (16 * h)) & 0xFFFFu);
                    const float x2 = bf16_bits_to_f32((bw[q] >> (16 * h)) & 0xFFFFu);
                    const float a1 = x1 * cs.x;
                    const float a2 = x2 * cs.y;
                    const float b1 = x1 * cs.y;
                    const float b2 = x2 * cs.x;
                    o2[h] = f32_to_bf16_bits(a1 - a2);
                    p2[h] = f32_to_bf16_bits(b1 + b2);
                }
                ow[q] = o2[0] | (o2[1] << 16);
                pw[q] = p2[0] | (p2[1] << 16);
            }
            *lo = make_uint4(ow[0], ow[1], ow[2], ow[3]);
            *hi = make_uint4(pw[0], pw[1], pw[2], pw[3]);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (active && kind != 2u) {
        uint4* dst = kind == 0u ? reinterpret_cast<uint4*>(p.q + (static_cast<size_t>(t) * p.H + hd) * D + u * 64u)
                                : reinterpret_cast<uint4*>(p.cache_k + slot_row + u * 64u);
        const uint4* st4 = reinterpret_cast<const uint4*>(sw + r * D + u * 64u);
#pragma unroll
        for (int q = 0; q < 8; ++q) dst[q] = st4[q];
    }
}

__global__ __launch_bounds__(kThreads) void rope_table_kernel(float2* table, uint32_t positions, uint32_t D,
                                                              uint32_t rotated, double base) {
    const uint32_t half = D / 2u;
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= static_cast<uint64_t>(positions) * half) return;
    const uint32_t pos = static_cast<uint32_t>(e / half);
    const uint32_t i = static_cast<uint32_t>(e - static_cast<uint64_t>(pos) * half);
    table[e] = rope_angle(pos, i, D, rotated, base);
}

// residual and next are [m][hidden]; hidden = 64 * units, units <= kThreads.
__global__ __launch_bounds__(kThreads) void residual_norm_kernel(const uint16_t* __restrict__ branch,
                                                                 uint16_t* __restrict__ residual,
                                                                 const uint16_t* __restrict__ w_post,
                                                                 const uint16_t* __restrict__ scalar,
                                                                 const uint16_t* __restrict__ w_next,
                                                                 uint16_t* __restrict__ next, uint32_t hidden,
                                                                 float eps) {
    __shared__ float part[kThreads + 1];
    const uint32_t units = hidden / 64u;
    const uint32_t tid = threadIdx.x;
    const size_t row = static_cast<size_t>(blockIdx.x) * hidden;
    const uint4* b4 = reinterpret_cast<const uint4*>(branch + row) + tid * 8u;
    uint4* r4 = reinterpret_cast<uint4*>(residual + row) + tid * 8u;
    const bool mine = tid < units;

    uint4 xv[8];
    uint4 rv[8];
    uint4 wv[8];
    uint4 nv[8];
    if (mine) {
        const uint4* w4 = reinterpret_cast<const uint4*>(w_post) + tid * 8u;
        const uint4* n4 = reinterpret_cast<const uint4*>(w_next != nullptr ? w_next : w_post) + tid * 8u;
#pragma unroll
        for (int t = 0; t < 8; ++t) {   // every load of the row issued before the first use
            xv[t] = b4[t];
            rv[t] = r4[t];
            wv[t] = w4[t];
            nv[t] = n4[t];
        }
        part[tid] = unit_sumsq(xv);
    }
    __syncthreads();
    if (tid < 64u) {
        const float ss = row_sumsq(part, units, tid);
        if (tid == 0u) part[kThreads] = rms_inverse(ss, hidden, eps);
    }
    __syncthreads();
    const float inv = part[kThreads];
    const float sc = scalar != nullptr ? bf16_bits_to_f32(*scalar) : 1.0f;
    float ss2 = 0.0f;
    if (mine) {
        normalize_unit(xv, inv);
        weight_unit(xv, wv);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            residual_add_chunk(xv[t], rv[t], scalar != nullptr, sc);
            r4[t] = xv[t];
        }
        if (w_next != nullptr) ss2 = unit_sumsq(xv);
    }
    if (w_next == nullptr) return;   // uniform over the launch
    __syncthreads();                 // every lane has read part[kThreads]
    if (mine) part[tid] = ss2;
    __syncthreads();
    if (tid < 64u) {
        const float ss = row_sumsq(part, units, tid);
        if (tid == 0u) part[kThreads] = rms_inverse(ss, hidden, eps);
    }
    __syncthreads();
    if (mine) {
        normalize_unit(xv, part[kThreads]);
        weight_unit(xv, nv);
        uint4* n4 = reinterpret_cast<uint4*>(next + row) + tid * 8u;
#pragma unroll
        for (int t = 0; t < 8; ++t) n4[t] = xv[t];
    }
}

// residual_norm_kernel for rows of at most 64 units, one row per workgroup, each 64-value
// unit spread over kUnitLanes lanes (kUnitLanes waves): a lane widens, normalises, weights
// and adds its 64 / kUnitLanes values; the fma chains of the unit sums are handed from lane
// to lane in the unit's order (scan_sumsq), and the unit sums meet in LDS for the row's
// butterfly in one wave. The bits of residual_norm_kernel, with a quarter of the vector-ALU
// instructions per wave of a unit-per-lane form (5.6 -> about 4 us per decode row of 3840
// in the model's step) and coalesced 32-byte accesses per lane.
constexpr uint32_t kUnitLanes = 4;
constexpr uint32_t kUnitChunks = 8u / kUnitLanes;   // 16-byte chunks per lane

__global__ __launch_bounds__(64 * kUnitLanes) void residual_norm_lanes_kernel(
    const uint16_t* __restrict__ branch, uint16_t* __restrict__ residual, const uint16_t* __restrict__ w_post,
    const uint16_t* __restrict__ scalar, const uint16_t* __restrict__ w_next, uint16_t* __restrict__ next,
    uint32_t hidden, float eps) {
    __shared__ float part[64 + 2];
    const uint32_t units = hidden / 64u;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t u = tid / kUnitLanes;
    const uint32_t c = tid % kUnitLanes;
    const bool mine = u < units;
    const size_t off = static_cast<size_t>(blockIdx.x) * hidden + u * 64u + c * (64u / kUnitLanes);
    const uint4* b4 = reinterpret_cast<const uint4*>(branch + off);
    uint4* r4 = reinterpret_cast<uint4*>(residual + off);

    uint4 xv[kUnitChunks];
    uint4 rv[kUnitChunks];
    uint4 wv[kUnitChunks];
    uint4 nv[kUnitChunks];
    if (mine) {
        const size_t woff = u * 64u + c * (64u / kUnitLanes);
        const uint4* w4 = reinterpret_cast<const uint4*>(w_post + woff);
        const uint4* n4 = reinterpret_cast<const uint4*>((w_next != nullptr ? w_next : w_post) + woff);
#pragma unroll
        for (uint32_t t = 0; t < kUnitChunks; ++t) {   // every load of the row issued before the first use
            xv[t] = b4[t];
            rv[t] = r4[t];
            wv[t] = w4[t];
            nv[t] = n4[t];
        }
    } else {
#pragma unroll
        for (uint32_t t = 0; t < kUnitChunks; ++t) xv[t] = make_uint4(0u, 0u, 0u, 0u);
    }
    const float sc = scalar != nullptr ? bf16_bits_to_f32(*scalar) : 1.0f;
    // The row's inverse rms from the lanes' chunks: unit sums to LDS, one wave's butterfly.
    const auto row_inverse = [&](const uint4 (&v)[kUnitChunks], uint32_t slot) {
        uint32_t w[4 * kUnitChunks];
#pragma unroll
        for (uint32_t t = 0; t < kUnitChunks; ++t) {
            w[4 * t] = v[t].x;
            w[4 * t + 1] = v[t].y;
            w[4 * t + 2] = v[t].z;
            w[4 * t + 3] = v[t].w;
        }
        const float t = scan_sumsq<kUnitLanes>(w, c);
        if (mine && c == kUnitLanes - 1u) part[u] = t;
        __syncthreads();
        if (wave == 0u) {
            const float ss = row_sumsq(part, units, lane);
            if (lane == 0u) part[slot] = rms_inverse(ss, hidden, eps);
        }
        __syncthreads();
        return part[slot];
    };
    const float inv = row_inverse(xv, 64u);
    if (mine) {
#pragma unroll
        for (uint32_t t = 0; t < kUnitChunks; ++t) {
            normalize_chunk(xv[t], inv);
            weight_chunk(xv[t], wv[t]);
            residual_add_chunk(xv[t], rv[t], scalar != nullptr, sc);
            r4[t] = xv[t];
        }
    }
    if (w_next == nullptr) return;   // uniform over the launch
    const float inv2 = row_inverse(xv, 65u);
    if (mine) {
        uint4* n4 = reinterpret_cast<uint4*>(next + off);
#pragma unroll
        for (uint32_t t = 0; t < kUnitChunks; ++t) {
            normalize_chunk(xv[t], inv2);
            weight_chunk(xv[t], nv[t]);
            n4[t] = xv[t];
        }
    }
}

// residual_norm_kernel for many rows (prefill chunks), with the same per-lane
// arithmetic (lane u owns unit u) but coalesced memory access: the wave kernel's lanes each
// read 128 contiguous bytes, so every 16-byte load instruction touches 64 cache lines. Here a
// wave's loads and stores move 1 KB of consecutive bytes per instruction, and the row and
// the workgroup's two weights pass through LDS tiles in which chunk t of unit u sits at slot
// 8u + (t ^ (u % 8)) (the lanes reading their units' chunk t hit distinct banks). One row per
// wave, kTiledRows rows per workgroup.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
constexpr uint32_t kTiledRows = 4;
constexpr uint32_t kResidualTiledMinRows = 64;

__device__ __forceinline__ uint32_t unit_slot(uint32_t u, uint32_t t) { return u * 8u + (t ^ (u & 7u)); }

// Orders one wave's LDS accesses across its lanes (a wave's LDS instructions execute in
// order; only the compiler must keep them in program order).
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(64 * kTiledRows) void residual_norm_tiled_kernel(
    const uint16_t* __restrict__ branch, uint16_t* __restrict__ residual, const uint16_t* __restrict__ w_post,
    const uint16_t* __restrict__ scalar, const uint16_t* __restrict__ w_next, uint16_t* __restrict__ next,
    uint32_t m, uint32_t hidden, float eps) {
    __shared__ uint4 wt[2][512];            // w_post, w_next: 64 units x 8 chunks at most
    __shared__ uint4 rt[kTiledRows][512];   // one row per wave
    const uint32_t units = hidden / 64u;
    const uint32_t chunks = units * 8u;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t row = blockIdx.x * kTiledRows + wave;
    const bool live = row < m;
    const size_t base = static_cast<size_t>(live ? row : 0u) * hidden;
    const uint4* b4 = reinterpret_cast<const uint4*>(branch + base);
    uint4* r4 = reinterpret_cast<uint4*>(residual + base);

    u32x4_t bc[8];   // native vectors: held in registers (uint4 arrays here went to scratch)
    u32x4_t rc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {   // the row's loads, issued before the weights are staged;
        // chunks past the row re-read its last one (unused), so no load sits behind a branch
        const uint32_t c = min(lane + 64u * t, chunks - 1u);
        bc[t] = *reinterpret_cast<const u32x4_t*>(b4 + c);
        rc[t] = *reinterpret_cast<const u32x4_t*>(r4 + c);
    }
    const uint4* wp4 = reinterpret_cast<const uint4*>(w_post);
    const uint4* wn4 = reinterpret_cast<const uint4*>(w_next != nullptr ? w_next : w_post);
#pragma unroll
    for (uint32_t i = 0; i < 512u / (64u * kTiledRows); ++i) {   // at most 512 chunks
        const uint32_t c = tid + 64u * kTiledRows * i;
        if (c < chunks) {
            wt[0][unit_slot(c >> 3, c & 7u)] = wp4[c];
            wt[1][unit_slot(c >> 3, c & 7u)] = wn4[c];
        }
    }
    __syncthreads();
    if (!live) return;   // no workgroup barrier below

    const bool mine = lane < units;
    uint4* tile = rt[wave];
    uint4 xv[8];
    uint4 rv[8];
    uint4 wv[8];   // w_post, then w_next, read from their tile where used
#pragma unroll
    for (int t = 0; t < 8; ++t) {   // lanes past the row write the last chunk's own value again
        const uint32_t c = min(lane + 64u * t, chunks - 1u);
        tile[unit_slot(c >> 3, c & 7u)] = __builtin_bit_cast(uint4, bc[t]);
    }
    wave_lds_order();
    if (mine) {
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[t] = tile[unit_slot(lane, t)];
    }
    wave_lds_order();
#pragma unroll
    for (int t = 0; t < 8; ++t) {   // lanes past the row write the last chunk's own value again
        const uint32_t c = min(lane + 64u * t, chunks - 1u);
        tile[unit_slot(c >> 3, c & 7u)] = __builtin_bit_cast(uint4, rc[t]);
    }
    wave_lds_order();
    if (mine) {
#pragma unroll
        for (int t = 0; t < 8; ++t) rv[t] = tile[unit_slot(lane, t)];
    }

    // residual_norm_kernel's arithmetic, unit by unit.
    const float sc = scalar != nullptr ? bf16_bits_to_f32(*scalar) : 1.0f;
    float ss = mine ? unit_sumsq(xv) : 0.0f;
    ss = butterfly_sum<32>(ss, lane);
    if (mine) {
        normalize_unit(xv, rms_inverse(ss, hidden, eps));
#pragma unroll
        for (int t = 0; t < 8; ++t) wv[t] = wt[0][unit_slot(lane, t)];
        weight_unit(xv, wv);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            residual_add_chunk(xv[t], rv[t], scalar != nullptr, sc);
        }
    }

    // The new residual out through the tile (after every lane's reads of the row).
    wave_lds_order();
    if (mine) {
#pragma unroll
        for (int t = 0; t < 8; ++t) tile[unit_slot(lane, t)] = xv[t];
    }
    wave_lds_order();
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t c = lane + 64u * t;
        if (c < chunks) r4[c] = tile[unit_slot(c >> 3, c & 7u)];
    }
    if (w_next == nullptr) return;   // uniform over the launch

    float ss2 = mine ? unit_sumsq(xv) : 0.0f;
    ss2 = butterfly_sum<32>(ss2, lane);
    if (mine) {
        normalize_unit(xv, rms_inverse(ss2, hidden, eps));
#pragma unroll
        for (int t = 0; t < 8; ++t) wv[t] = wt[1][unit_slot(lane, t)];
        weight_unit(xv, wv);
    }
    wave_lds_order();
    if (mine) {
#pragma unroll
        for (int t = 0; t < 8; ++t) tile[unit_slot(lane, t)] = xv[t];
    }
    wave_lds_order();
    uint4* n4 = reinterpret_cast<uint4*>(next + base);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t c = lane + 64u * t;
        if (c < chunks) n4[c] = tile[unit_slot(c >> 3, c & 7u)];
    }
}

__global__ void decode_advance_kernel(uint32_t* pos, uint32_t* ties, const HypTopKSample* sample) {
    if (threadIdx.x == 0u) {
        pos[0] += 1u;
        ties[0] += sample->near_tie != 0u ? 1u : 0u;
    }
}

}  // namespace

void launch_decode_advance(uint32_t* pos, uint32_t* ties, const HypTopKSample* sample, hipStream_t stream) {
    hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(64), 0, stream, pos, ties, sample);
    HYP_HIP_CHECK(hipGetLastError());
}

void launch_attn_prepare(const AttnPrepareArgs& a, hipStream_t stream) {
    if (a.L == 0) return;
    HYP_REQUIRE(a.head_dim % 64u == 0u && a.head_dim <= kMaxHeadDim, HYP_STATUS_UNSUPPORTED,
                "attention prepare: head_dim must be a multiple of 64, at most 512");
    PrepareParams p{};
    p.pos = a.pos;
    p.rope_cs = a.rope_cs;
    p.q = a.q;
    p.k_raw = a.k_raw;
    p.v_raw = a.v_raw;
    p.q_w = a.q_norm;
    p.k_w = a.k_norm;
    p.cache_k = a.cache_k;
    p.cache_v = a.cache_v;
    p.L = a.L;
    p.H = a.n_heads;
    p.KVH = a.n_kv_heads;
    p.D = a.head_dim;
    p.rotated = a.rotated;
    p.offset = a.offset;
    p.cap = a.cap;
    p.first_cached = a.L > a.cap ? a.L - a.cap : 0u;
    p.base = static_cast<double>(a.base);
    p.eps = a.eps;
    if (a.L <= kPrepareHeadMaxTokens) {
        const uint32_t groups = (a.n_heads + a.n_kv_heads + kWaves - 1u) / kWaves;
        hipLaunchKernelGGL(attn_prepare_head_kernel, dim3(a.L, groups), dim3(kThreads), 0, stream, p);
        HYP_HIP_CHECK(hipGetLastError());
        return;
    }
    const uint64_t rows = static_cast<uint64_t>(a.L) * (a.n_heads + 2u * a.n_kv_heads);
    const uint64_t per_block = static_cast<uint64_t>(kWaves) * (64u / (a.head_dim / 64u));
    const uint64_t blocks = (rows + per_block - 1u) / per_block;
    HYP_REQUIRE(rows + per_block < (1ull << 31), HYP_STATUS_INVALID_ARGUMENT, "attention prepare: too many rows");
    const dim3 grid(static_cast<uint32_t>(blocks));
    switch (a.head_dim) {
        case 64: hipLaunchKernelGGL(attn_prepare_kernel<64>, grid, dim3(kThreads), 0, stream, p); break;
        case 128: hipLaunchKernelGGL(attn_prepare_kernel<128>, grid, dim3(kThreads), 0, stream, p); break;
        case 256: hipLaunchKernelGGL(attn_prepare_kernel<256>, grid, dim3(kThreads), 0, stream, p); break;
        case 512: hipLaunchKernelGGL(attn_prepare_kernel<512>, grid, dim3(kThreads), 0, stream, p); break;
        default:
            throw NativeError(HYP_STATUS_UNSUPPORTED, "attention prepare: head_dim must be 64, 128, 256 or 512");
    }
    HYP_HIP_CHECK(hipGetLastError());
}

void launch_rope_table(float2* table, uint32_t positions, uint32_t head_dim, uint32_t rotated, float base,
                       hipStream_t stream) {
    const uint64_t n = static_cast<uint64_t>(positions) * (head_dim / 2u);
    if (n == 0) return;
    const uint64_t blocks = (n + kThreads - 1u) / kThreads;
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "rope table: too large");
    hipLaunchKernelGGL(rope_table_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream, table,
                       positions, head_dim, rotated, static_cast<double>(base));
    HYP_HIP_CHECK(hipGetLastError());
}

uint32_t residual_norm_max_hidden() { return 64u * kThreads; }

void launch_residual_norm(const uint16_t* branch, uint16_t* residual, const uint16_t* w_post, const uint16_t* scalar,
                          const uint16_t* w_next, uint16_t* next, uint32_t m, uint32_t hidden, float eps,
                          hipStream_t stream) {
    if (m == 0) return;
    HYP_REQUIRE(hidden % 64u == 0u && hidden <= residual_norm_max_hidden(), HYP_STATUS_UNSUPPORTED,
                "residual norm: hidden must be a multiple of 64, at most 16384");
    if (hidden <= 64u * 64u && m >= kResidualTiledMinRows) {
        hipLaunchKernelGGL(residual_norm_tiled_kernel, dim3((m + kTiledRows - 1u) / kTiledRows),
                           dim3(64u * kTiledRows), 0, stream, branch, residual, w_post, scalar, w_next, next, m,
                           hidden, eps);
    } else if (hidden <= 64u * 64u) {
        hipLaunchKernelGGL(residual_norm_lanes_kernel, dim3(m), dim3(64u * kUnitLanes), 0, stream, branch, residual,
                           w_post, scalar, w_next, next, hidden, eps);
    } else {
        hipLaunchKernelGGL(residual_norm_kernel, dim3(m), dim3(kThreads), 0, stream, branch, residual, w_post, scalar,
                           w_next, next, hidden, eps);
    }
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

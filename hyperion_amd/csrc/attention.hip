// Attention of the Gemma-4 decoder layer on gfx950: ForwardPass::attention's
// mx::fast::scaled_dot_product_attention (native/hyperion_mlx/src/forward.cc:376-508) over a
// KV cache prefix and the current chunk, and the cache writes (LocalKvCache /
// GlobalKvCache::append, kv_cache.h:33,143).
//
// Semantics (the reference's): scale 1.0 (Gemma 4 drops 1/sqrt(d)); query token t of the
// chunk sits at position offset + t and sees key position p when p <= offset + t and, for
// a sliding layer, p > offset + t - window (build_mask, forward.cc:345-373); query head h
// reads kv head h / (H / KVH). Keys are the cache's positions [offset - prefix, offset)
// (slot p % capacity) followed by the chunk's L positions, read from the chunk's k/v or,
// when those are null, from the cache (the decoder appends the chunk first; it sizes its
// rings to hold prefix + L positions).
//
// One kernel serves prefill and decode, flash-attention style on v_mfma_f32_16x16x32_bf16:
//  * A workgroup (4 waves) takes a tile of 64 query rows of one kv head - row r is token
//    r / G, head-in-group r % G (G = H / KVH) - and walks its visible keys in blocks of 32.
//    A block's K rows and V go through LDS (AttnLds); each wave computes its 16
//    rows' scores S = Q K^T (Q rows read from LDS), masks them, and updates the online
//    softmax in fp32: m = running row maximum (log2 domain), l = running sum, O = O * 2^(m_old
//    - m) + P V, with P rounded to bf16 for the PV MFMAs (written to LDS and read back in the
//    A-operand layout).
//  * Decode (one row tile per kv head) splits the keys over several workgroups; each writes
//    its unnormalised O with m and l to a workspace, and attn_combine_kernel merges them.
//  * LDS rows are padded by 16 bytes so the 16 rows (or keys, or dims) an operand read
//    touches start on different banks.
#include <algorithm>
#include <string>

#include "common.h"
#include "kernels.h"
#include "q4_rmsnorm.h"

namespace hyperion::hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kAttnThreads = 256;
constexpr uint32_t kRowsPerTile = 64;   // 4 waves x 16 rows
constexpr uint32_t kKeyBlock = 32;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
    const uint16_t* q;      // [L][H][D]
    const uint16_t* k;      // [L][KVH][D]: the chunk, or null when it is in the cache
    const uint16_t* v;
    const uint16_t* ck;     // [cap][KVH][D]: the cache
    const uint16_t* cv;
    uint16_t* out;          // [L][H][D]
    float* part_o;          // split partials: [splits][L * H][D]
    float* part_ml;         // [splits][L * H][2]
    uint32_t L, H, KVH, G, cap, offset, prefix, window;
    uint32_t splits, keys_per_split;
    const uint32_t* pos;    // non-null: offset = *pos, read on the device (graph replays)
    // The decode form with the prepare folded in (L = 1): q is the raw projection; each
    // wave normalises and rotates its query rows, and the wave whose keys hold the new
    // token forms its K/V from k_raw/v_raw and writes them to the cache slot.
    const float2* rope_cs;  // (cos, sin) [positions][D / 2]
    const uint16_t* q_w;    // [D]
    const uint16_t* k_w;    // [D]
    const uint16_t* k_raw;  // [KVH][D]
    const uint16_t* v_raw;  // [KVH][D], or null: V = v_norm(k_raw)
    uint16_t* ck_out;       // the cache, written at the new token's slot
    uint16_t* cv_out;
    float eps;
};

// Graph-replay form: the position comes from device memory, the prefix and the split
// length follow from it as the host computes them (prefix = min(window, offset) with a
// window, offset without; keys split evenly in whole key blocks over the fixed grid).
__device__ __forceinline__ void resolve_position(AttnParams& p) {
    if (p.pos == nullptr) return;
    p.offset = *p.pos;
    p.prefix = p.window != 0u ? min(p.window, p.offset) : p.offset;
    const uint32_t T = p.prefix + p.L;
    p.keys_per_split = ((T + p.splits - 1u) / p.splits + kKeyBlock - 1u) / kKeyBlock * kKeyBlock;
}

// Max and sum over the 16 lanes of a row, in the order of the xor butterfly 1, 2, 4, 8.
__device__ __forceinline__ float row16_max(float v, uint32_t lane) {
    v = fmaxf(v, xor_lanes<1>(v, lane));
    v = fmaxf(v, xor_lanes<2>(v, lane));
    v = fmaxf(v, xor_lanes<4>(v, lane));
    return fmaxf(v, xor_lanes<8>(v, lane));
}

__device__ __forceinline__ float row16_sum(float v, uint32_t lane) {
    v += xor_lanes<1>(v, lane);
    v += xor_lanes<2>(v, lane);
    v += xor_lanes<4>(v, lane);
    return v + xor_lanes<8>(v, lane);
}

template <uint32_t D>
struct AttnLds {
    static constexpr uint32_t kRow = D * 2u + 16u;           // Q and K rows (bytes)
    // V: at head_dim 512 rows as loaded, read by transposing reads; below, transposed on the
    // way in ([d][32 keys], 16-bit writes in an order rotated by the lane), which measured
    // faster there (1024-token sliding layer 77 against 112 us; 179 against 203 at 512).
    static constexpr bool kTrV = D >= 512u;
    static constexpr uint32_t kVRow = D * 2u + 16u;           // V rows (bytes), kTrV
    static constexpr uint32_t kVtRow = kKeyBlock * 2u + 16u;  // V^T rows, !kTrV
    static constexpr uint32_t kPRow = kKeyBlock * 2u + 16u;   // P rows
    static constexpr uint32_t kQ = 0;
    static constexpr uint32_t kK = kQ + kRowsPerTile * kRow;
    static constexpr uint32_t kV = kK + kKeyBlock * kRow;
    static constexpr uint32_t kP = kV + (kTrV ? kKeyBlock * kVRow : D * kVtRow);
    static constexpr uint32_t kBytes = kP + (kAttnThreads / 64u) * 16u * kPRow;
};

__device__ __forceinline__ const uint16_t* key_row(const AttnParams& p, const uint16_t* chunk, const uint16_t* cache,
                                                   uint32_t j, uint32_t hk, uint32_t D) {
    // Key index j (0 .. prefix + L) -> its row: the cache for the prefix, the chunk after
    // (the cache too when the chunk has already been appended: chunk == null).
    if (j < p.prefix || chunk == nullptr) {
        const uint32_t pos = p.offset - p.prefix + j;
        return cache + (static_cast<size_t>(pos % p.cap) * p.KVH + hk) * D;
    }
    return chunk + (static_cast<size_t>(j - p.prefix) * p.KVH + hk) * D;
}

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef short short8_t __attribute__((ext_vector_type(8)));

// The B operand (keys 8kb .. 8kb + 7 of one dim per lane) of a 16-dim tile of V rows kept
// [key][dim] in LDS with `row` bytes between keys: two ds_read_b64_tr_b16, keys 8kb + e
// then 8kb + 4 + e; p is this lane's address in the first (row 8kb + (j / 4), dims
// 4 (j % 4) of the tile).
__device__ __forceinline__ bf16x8_t v_operand_tr(uint8_t* p, uint32_t row) {
    const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) short4_t*>(reinterpret_cast<uintptr_t>(p)));
    const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) short4_t*>(reinterpret_cast<uintptr_t>(p + 4u * row)));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <uint32_t D>
__global__ __launch_bounds__(kAttnThreads) void attn_kernel(AttnParams p) {
    resolve_position(p);
    using Lds = AttnLds<D>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t j16 = lane & 15u;
    const uint32_t kb = lane >> 4;
    const uint32_t hk = blockIdx.y;
    const uint32_t split = blockIdx.z;
    const uint32_t rows = p.L * p.G;                     // query rows of this kv head
    // Workgroups are dispatched x first, then z: the second key split takes the tiles in
    // reverse, so its longest causal halves start first, on the compute units the first
    // split's short tiles free early.
    const uint32_t tile = (split & 1u) != 0u ? gridDim.x - 1u - blockIdx.x : blockIdx.x;
    const uint32_t row0 = tile * kRowsPerTile;           // first row of the tile
    const uint32_t T = p.prefix + p.L;

    // The tile's token range and the keys any of its rows can see, within this split.
    const uint32_t t_lo = row0 / p.G;
    const uint32_t t_hi = (min(row0 + kRowsPerTile, rows) - 1u) / p.G;
    uint32_t j_begin = split * p.keys_per_split;
    uint32_t j_end = min(j_begin + p.keys_per_split, T);
    j_end = min(j_end, p.prefix + t_hi + 1u);                 // causal: keys up to the last query
    if (p.window != 0u) {
        // keys at positions > offset + t_lo - window, i.e. j > prefix + t_lo - window
        const int64_t lo = static_cast<int64_t>(p.prefix) + t_lo - p.window + 1;
        if (lo > static_cast<int64_t>(j_begin)) j_begin = static_cast<uint32_t>(lo);
    }

    // Q tile -> LDS: thread t copies 16-byte chunks (row = c / (D/8), chunk c % (D/8)).
    constexpr uint32_t kChunks = D / 8u;
    for (uint32_t c = tid; c < kRowsPerTile * kChunks; c += kAttnThreads) {
        const uint32_t r = c / kChunks;
        const uint32_t ch = c - r * kChunks;
        const uint32_t gr = row0 + r;
        uint4 val = make_uint4(0u, 0u, 0u, 0u);
        if (gr < rows) {
            const uint32_t t = gr / p.G;
            const uint32_t h = hk * p.G + (gr - t * p.G);
            val = *reinterpret_cast<const uint4*>(p.q + (static_cast<size_t>(t) * p.H + h) * D + ch * 8u);
        }
        *reinterpret_cast<uint4*>(lds + Lds::kQ + r * Lds::kRow + ch * 16u) = val;
    }

    // Per lane: rows 4 kb + i (i < 4) of the wave's 16; O tiles of 16 dims.
    constexpr uint32_t kDTiles = D / 16u;
    f32x4_t o[kDTiles];
#pragma unroll
    for (uint32_t t = 0; t < kDTiles; ++t) o[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m[4], l[4];
    int32_t qpos[4];   // -1: a padding row (never visible)
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        m[i] = -__builtin_huge_valf();
        l[i] = 0.0f;
        const uint32_t gr = row0 + wave * 16u + 4u * kb + i;
        qpos[i] = gr < rows ? static_cast<int32_t>(p.offset + gr / p.G) : -1;
    }
    const uint8_t* qrow = lds + Lds::kQ + (wave * 16u + j16) * Lds::kRow;   // A operand row (i = j16)
    uint8_t* prow_w = lds + Lds::kP + wave * 16u * Lds::kPRow;             // this wave's P [16][32]

    // K and V of a key block: thread tid takes chunks tid + 256 u (key c / (D/8), chunk c %
    // (D/8): coalesced rows). The next block's chunks are loaded into registers while the
    // current block computes; staging writes the K rows as loaded and V as AttnLds says.
    constexpr uint32_t kPer = kKeyBlock * kChunks / kAttnThreads;
    uint4 kn[kPer];
    uint4 vn[kPer];
    const auto fetch = [&](uint32_t jb_) {
        const uint32_t nk_ = min(kKeyBlock, j_end - jb_);
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            const uint32_t c = tid + kAttnThreads * u;
            const uint32_t r = c / kChunks;
            const uint32_t ch = c - r * kChunks;
            kn[u] = make_uint4(0u, 0u, 0u, 0u);
            vn[u] = make_uint4(0u, 0u, 0u, 0u);
            if (r < nk_) {
                kn[u] = *reinterpret_cast<const uint4*>(key_row(p, p.k, p.ck, jb_ + r, hk, D) + ch * 8u);
                vn[u] = *reinterpret_cast<const uint4*>(key_row(p, p.v, p.cv, jb_ + r, hk, D) + ch * 8u);
            }
        }
    };
    if (j_begin < j_end) fetch(j_begin);

    for (uint32_t jb = j_begin; jb < j_end; jb += kKeyBlock) {
        const uint32_t nk = min(kKeyBlock, j_end - jb);
        __syncthreads();   // the previous block's K/V reads are done (and Q is staged)
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            const uint32_t c = tid + kAttnThreads * u;
            const uint32_t r = c / kChunks;
            const uint32_t ch = c - r * kChunks;
            *reinterpret_cast<uint4*>(lds + Lds::kK + r * Lds::kRow + ch * 16u) = kn[u];
            if constexpr (Lds::kTrV) {
                *reinterpret_cast<uint4*>(lds + Lds::kV + r * Lds::kVRow + ch * 16u) = vn[u];
            } else {
                const uint4 vv = vn[u];
                uint8_t* col = lds + Lds::kV + (ch * 8u) * Lds::kVtRow + r * 2u;
#pragma unroll
                for (uint32_t s2 = 0; s2 < 8u; ++s2) {
                    const uint32_t e = (s2 + lane) & 7u;
                    const uint32_t d01 = (e & 2u) ? vv.y : vv.x;
                    const uint32_t d23 = (e & 2u) ? vv.w : vv.z;
                    const uint32_t dw = (e & 4u) ? d23 : d01;
                    *reinterpret_cast<uint16_t*>(col + e * Lds::kVtRow) =
                        static_cast<uint16_t>((e & 1u) ? (dw >> 16) : (dw & 0xFFFFu));
                }
            }
        }
        __syncthreads();
        if (jb + kKeyBlock < j_end) fetch(jb + kKeyBlock);   // in flight during this block

        // S = Q K^T for the wave's 16 rows x 32 keys (two column tiles of 16 keys).
        f32x4_t s[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll 4
        for (uint32_t st = 0; st < D / 32u; ++st) {
            const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(qrow + (st * 32u + kb * 8u) * 2u);
#pragma unroll
            for (uint32_t c = 0; c < 2; ++c) {
                const bf16x8_t b = *reinterpret_cast<const bf16x8_t*>(lds + Lds::kK + (16u * c + j16) * Lds::kRow +
                                                                      (st * 32u + kb * 8u) * 2u);
                s[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, s[c], 0, 0, 0);
            }
        }

        // Mask, online softmax (log2 domain), P -> LDS as bf16.
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            float sv[2];
            float bmax = -__builtin_huge_valf();
#pragma unroll
            for (uint32_t c = 0; c < 2; ++c) {
                const uint32_t key = 16u * c + j16;
                const int32_t kpos = static_cast<int32_t>(p.offset - p.prefix + jb + key);
                const bool vis = key < nk && qpos[i] >= 0 && kpos <= qpos[i] &&
                                 (p.window == 0u || kpos > qpos[i] - static_cast<int32_t>(p.window));
                sv[c] = vis ? s[c][i] * kLog2e : -__builtin_huge_valf();
                bmax = fmaxf(bmax, sv[c]);
            }
            bmax = row16_max(bmax, lane);
            const float m_new = fmaxf(m[i], bmax);
            const bool any = m_new > -__builtin_huge_valf();
            const float alpha = any ? exp2f(m[i] - m_new) : 1.0f;   // m[i] = -inf -> 0
            float psum = 0.0f;
#pragma unroll
            for (uint32_t c = 0; c < 2; ++c) {
                const float pv = any && sv[c] > -__builtin_huge_valf() ? exp2f(sv[c] - m_new) : 0.0f;
                psum += pv;
                *reinterpret_cast<uint16_t*>(prow_w + (4u * kb + i) * Lds::kPRow + (16u * c + j16) * 2u) =
                    f32_to_bf16_bits(pv);
            }
            psum = row16_sum(psum, lane);
            l[i] = l[i] * alpha + psum;
            m[i] = any ? m_new : m[i];
#pragma unroll
            for (uint32_t t = 0; t < kDTiles; ++t) o[t][i] *= alpha;
        }
        // P (16 x 32 keys) as the A operand, V^T as B: O += P V.
        const bf16x8_t pa = *reinterpret_cast<const bf16x8_t*>(prow_w + j16 * Lds::kPRow + kb * 16u);
        if constexpr (Lds::kTrV) {
            uint8_t* vt = lds + Lds::kV + (8u * kb + (j16 >> 2)) * Lds::kVRow + (j16 & 3u) * 8u;
#pragma unroll
            for (uint32_t t = 0; t < kDTiles; ++t) {
                o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, v_operand_tr(vt + 32u * t, Lds::kVRow), o[t], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (uint32_t t = 0; t < kDTiles; ++t) {
                const bf16x8_t b = *reinterpret_cast<const bf16x8_t*>(lds + Lds::kV + (16u * t + j16) * Lds::kVtRow + kb * 16u);
                o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, b, o[t], 0, 0, 0);
            }
        }
    }

    // Rows 4 kb + i of the wave, dims 16 t + j16.
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t gr = row0 + wave * 16u + 4u * kb + i;
        if (gr >= rows) continue;
        const uint32_t t = gr / p.G;
        const uint32_t h = hk * p.G + (gr - t * p.G);
        const size_t orow = static_cast<size_t>(t) * p.H + h;   // [L][H] row of the output
        if (p.splits == 1u) {
            const float inv = l[i] > 0.0f ? 1.0f / l[i] : 0.0f;
#pragma unroll
            for (uint32_t tt = 0; tt < kDTiles; ++tt) p.out[orow * D + 16u * tt + j16] = f32_to_bf16_bits(o[tt][i] * inv);
        } else {
            const size_t prow = static_cast<size_t>(split) * p.L * p.H + orow;
#pragma unroll
            for (uint32_t tt = 0; tt < kDTiles; ++tt) p.part_o[prow * D + 16u * tt + j16] = o[tt][i];
            if (j16 == 0u) {
                p.part_ml[prow * 2u] = m[i];
                p.part_ml[prow * 2u + 1u] = l[i];
            }
        }
    }
}

// Decode form (at most 16 query rows per kv head: L * G <= 16, a single MFMA row tile).
// Each wave is an independent split of the keys, with nothing shared across waves:
//  * Q stays in registers as the A operand of S = Q K^T for the whole kernel;
//  * K rows load straight from memory into the B operand (lane (j, kb) holds key j's dims
//    8kb .. 8kb + 7 of a 32-dim step: 16 contiguous bytes of the row);
//  * V rows load coalesced into the wave's own LDS as they are ([32 keys][d], 16-byte
//    writes) and reach the B operand of O += P V by transposing reads (two
//    ds_read_b64_tr_b16 per 16-dim tile: lane (dim j, kb) takes keys 8kb .. 8kb + 7);
//  * the online softmax, P in bf16 and the P.V products are those of attn_kernel.
// Every split writes its unnormalised rows with (m, l); attn_combine_kernel merges them.
template <uint32_t D>
struct DecodeLds {
    static constexpr uint32_t kVRow = D * 2u + 16u;   // a V row (bytes), padded by 16
    static constexpr uint32_t kPRow = kKeyBlock * 2u + 16u;
    static constexpr uint32_t kV = 0;   // [32 keys][kVRow]; also the query rows' staging before the key loop
    static constexpr uint32_t kP = kV + kKeyBlock * kVRow;
    static constexpr uint32_t kNew = kP + 16u * kPRow;   // the new token's K and V rows (bf16)
    static constexpr uint32_t kWave = kNew + 4u * D;
    // One wave per workgroup: the few hundred waves of a decode step then spread over that
    // many compute units instead of sharing a quarter of them (and their memory queues);
    // measured 3.40 against 3.45 ms per 12B decode step with four.
    static constexpr uint32_t kWaves = 1u;
    static constexpr uint32_t kBytes = kWaves * kWave;
};

// Orders one wave's LDS accesses across its lanes (a wave's LDS instructions execute in
// order; only the compiler must keep them in program order).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// RoPE of `rows` head rows of D bf16 in LDS (row stride D), in place, with the prepare
// kernel's arithmetic: lane takes 8 consecutive pairs (i, i + D/2) of row rsub + k * rpi;
// cs8 holds (cos, sin) of its pairs.
template <uint32_t D>
__device__ __forceinline__ void rope_rows_lds(uint16_t* rows_base, uint32_t rows, uint32_t lane, const float2 (&cs8)[8]) {
    constexpr uint32_t kHalf = D / 2u;
    constexpr uint32_t kHalfChunks = kHalf / 8u;
    constexpr uint32_t kRowsPerIter = 64u / kHalfChunks;
    const uint32_t c = lane % kHalfChunks;
    for (uint32_t r = lane / kHalfChunks; r < rows; r += kRowsPerIter) {
        uint4* lo = reinterpret_cast<uint4*>(rows_base + r * D + c * 8u);
        uint4* hi = reinterpret_cast<uint4*>(rows_base + r * D + kHalf + c * 8u);
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
                const float x1 = bf16_bits_to_f32((aw[q] >> (16 * h)) & 0xFFFFu);
                const float x2 = bf16_bits_to_f32((bw[q] >> (16 * h)) & 0xFFFFu);
                const float2 cs = cs8[2 * q + h];
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

// Lanes per 64-value unit in the folded prepare's spread form (CH > 1): at most 16 / (D / 64)
// so that the row butterfly's lane offsets stay within a 16-lane row (DPP moves).
template <uint32_t D>
constexpr uint32_t kPrepLanes = D <= 128u ? 8u : 16u / (D / 64u);

// The value of lane CH - 1 of each group of CH lanes on every lane of the group.
template <uint32_t CH>
__device__ __forceinline__ float group_last(float v, uint32_t lane) {
    static_assert(CH == 2u || CH == 4u || CH == 8u, "groups of 2, 4 or 8 lanes");
    if constexpr (CH == 2u) return dpp_mov<0xF5>(v);   // quad_perm [1, 1, 3, 3]
    v = dpp_mov<0xFF>(v);                               // quad_perm [3, 3, 3, 3]
    if constexpr (CH == 8u) {
        const float up = dpp_mov<0x104>(v);             // row_shl 4: lane i + 4
        v = (lane & 4u) != 0u ? v : up;
    }
    return v;
}

template <uint32_t D, bool PREP, uint32_t CH = 1>
__global__ __launch_bounds__(DecodeLds<D>::kWaves * 64u) void attn_decode_kernel(AttnParams p) {
    resolve_position(p);
    using Lds = DecodeLds<D>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t lane = threadIdx.x & 63u;
    // Wave-uniform (a scalar): the key range, has_keys and fresh_key below follow from it,
    // and their branches then stay scalar rather than masking lanes around the loads.
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t split = blockIdx.x * Lds::kWaves + wave;
    if (split >= p.splits) return;   // no workgroup barrier below: waves are independent
    const uint32_t hk = blockIdx.y;
    const uint32_t j16 = lane & 15u;
    const uint32_t kb = lane >> 4;
    const uint32_t rows = p.L * p.G;   // <= 16
    const uint32_t T = p.prefix + p.L;
    uint8_t* my = lds + wave * Lds::kWave;

    uint32_t j_begin = split * p.keys_per_split;
    const uint32_t j_end = min(j_begin + p.keys_per_split, T);
    if (p.window != 0u) {   // keys at positions > offset - window (the first token's bound)
        const int64_t lo = static_cast<int64_t>(p.prefix) - p.window + 1;
        if (lo > static_cast<int64_t>(j_begin)) j_begin = static_cast<uint32_t>(lo);
    }

    constexpr uint32_t kSteps = D / 32u;
    constexpr uint32_t kDTiles = D / 16u;
    bf16x8_t qa[kSteps];
    // PREP: the new token's K and V rows staged for the RoPE (this wave's keys include it
    // when fresh_key).
    uint16_t* new_k = reinterpret_cast<uint16_t*>(my + Lds::kNew);
    uint16_t* new_v = new_k + D;
    bool fresh_key = false;
    if constexpr (PREP) {
        // attn_prepare_kernel's work for one token (L = 1), in its arithmetic: q_norm and
        // RoPE of this kv head's G query rows, staged in the V area; k_norm + RoPE and
        // v_norm of the new key by the wave whose range holds it.
        constexpr uint32_t kU = D / 64u;             // 64-value units per head row
        constexpr uint32_t kHalf = D / 2u;
        const bool has_keys = j_begin < j_end;       // wave-uniform
        fresh_key = has_keys && j_begin <= p.prefix && p.prefix < j_end;
        uint16_t* qs = reinterpret_cast<uint16_t*>(my + Lds::kV);   // [G][D]
        const uint32_t pos = p.offset;
        float2 cs8[8];
        {
            const uint32_t c = lane % (kHalf / 8u);
            const float4* t4 = reinterpret_cast<const float4*>(p.rope_cs + static_cast<size_t>(pos) * kHalf + c * 8u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float4 v = has_keys ? t4[e] : make_float4(1.0f, 0.0f, 1.0f, 0.0f);
                cs8[2 * e] = make_float2(v.x, v.y);
                cs8[2 * e + 1] = make_float2(v.z, v.w);
            }
        }
        if (!has_keys) {
#pragma unroll
            for (uint32_t st = 0; st < kSteps; ++st) qa[st] = bf16x8_t{};
        } else {
            // One 64-value unit per CH lanes (lane sl = lane % CH of unit slot lane / CH holds
            // its values [64 / CH * sl, 64 / CH * (sl + 1))): slot row r = slot / kU is query
            // row r (r < G), the new key's K (r == G) or its V (r == G + 1); the host folds
            // only when they fit.
            constexpr uint32_t kCC = 8u / CH;   // 16-byte chunks per lane
            const uint32_t sl = lane % CH;
            const uint32_t u = (lane / CH) % kU;
            const uint32_t r = lane / CH / kU;
            const bool is_q = r < p.G;
            const bool is_k = fresh_key && r == p.G;
            const bool is_v = fresh_key && r == p.G + 1u;
            const size_t slot_row = (static_cast<size_t>(p.offset % p.cap) * p.KVH + hk) * D;
            const uint16_t* src = nullptr;
            const uint16_t* w = nullptr;
            if (is_q) {
                src = p.q + (static_cast<size_t>(hk) * p.G + r) * D;
                w = p.q_w;
            } else if (is_k) {
                src = p.k_raw + static_cast<size_t>(hk) * D;
                w = p.k_w;
            } else if (is_v) {
                src = (p.v_raw != nullptr ? p.v_raw : p.k_raw) + static_cast<size_t>(hk) * D;
            }
            const uint32_t voff = u * 64u + sl * (64u / CH);   // this lane's first value in the row
            uint4 xv[kCC];
            uint4 wv[kCC];
#pragma unroll
            for (uint32_t t = 0; t < kCC; ++t) xv[t] = make_uint4(0u, 0u, 0u, 0u);
            if (src != nullptr) {
                const uint4* s4 = reinterpret_cast<const uint4*>(src + voff);
#pragma unroll
                for (uint32_t t = 0; t < kCC; ++t) xv[t] = s4[t];
            }
            if (w != nullptr) {
                const uint4* w4 = reinterpret_cast<const uint4*>(w + voff);
#pragma unroll
                for (uint32_t t = 0; t < kCC; ++t) wv[t] = w4[t];
            }
            // One dword of every 128-byte line of the first key block's K and V rows, requested
            // behind this prologue's loads and consumed at its end: their HBM fetch overlaps
            // the prologue, and the key loop's loads of them hit the cache.
            uint32_t touch = 0u;
            asm volatile("" ::: "memory");   // these requests after the prologue's own
            {
                constexpr uint32_t kLines = D * 2u / 128u;   // lines per row
                constexpr uint32_t kTouch = 2u * kKeyBlock * kLines;
                const uint32_t nk0 = min(kKeyBlock, j_end - j_begin);
                if (j_begin != p.prefix) {   // (a block that starts at the new key holds only it)
#pragma unroll
                    for (uint32_t i = 0; i < kTouch / 64u; ++i) {
                        const uint32_t li = lane + 64u * i;
                        const uint32_t half = li / (kKeyBlock * kLines);   // 0: K, 1: V
                        const uint32_t rest = li - half * kKeyBlock * kLines;
                        const uint32_t r = rest / kLines;
                        // past the block or the new key's row (not read before its store): row 0
                        const uint32_t rr = r < nk0 && j_begin + r != p.prefix ? r : 0u;
                        const uint16_t* row = key_row(p, nullptr, half == 0u ? p.ck : p.cv, j_begin + rr, hk, D);
                        touch |= *reinterpret_cast<const uint32_t*>(row + (rest - r * kLines) * 64u);
                    }
                }
            }
            // The prepare's 64-lane butterfly over a row's kU units (the rest of its lanes add
            // zeros there): each unit's sum (its fma chain handed across its CH lanes) on all of
            // its lanes, then the xor steps kU / 2, ..., 1 between units.
            float ss;
            if constexpr (CH == 1u) {
                ss = src != nullptr ? unit_sumsq(xv) : 0.0f;
            } else {
                uint32_t ws[4 * kCC];
#pragma unroll
                for (uint32_t t = 0; t < kCC; ++t) {
                    ws[4 * t] = xv[t].x;
                    ws[4 * t + 1] = xv[t].y;
                    ws[4 * t + 2] = xv[t].z;
                    ws[4 * t + 3] = xv[t].w;
                }
                ss = group_last<CH>(scan_sumsq<CH>(ws, sl), lane);
            }
            if constexpr (kU >= 8u) ss += xor_lanes<4u * CH>(ss, lane);
            if constexpr (kU >= 4u) ss += xor_lanes<2u * CH>(ss, lane);
            if constexpr (kU >= 2u) ss += xor_lanes<1u * CH>(ss, lane);
            if (src != nullptr) {
                const float inv = rms_inverse(ss, D, p.eps);
                uint16_t* dst = is_q ? qs + r * D : (is_k ? new_k : new_v);
                uint4* d4 = reinterpret_cast<uint4*>(dst + voff);
                uint4* vg = reinterpret_cast<uint4*>(p.cv_out + slot_row + voff);
#pragma unroll
                for (uint32_t t = 0; t < kCC; ++t) {
                    normalize_chunk(xv[t], inv);
                    if (w != nullptr) weight_chunk(xv[t], wv[t]);
                    d4[t] = xv[t];
                    if (is_v) vg[t] = xv[t];
                }
            }
            wave_lds_sync();
            rope_rows_lds<D>(qs, p.G, lane, cs8);
            if (fresh_key) rope_rows_lds<D>(new_k, 1u, lane, cs8);
            wave_lds_sync();
            if (fresh_key && lane < kU) {
                const uint4* kl = reinterpret_cast<const uint4*>(new_k + lane * 64u);
                uint4* kg = reinterpret_cast<uint4*>(p.ck_out + slot_row + lane * 64u);
#pragma unroll
                for (int t = 0; t < 8; ++t) kg[t] = kl[t];
            }
            asm volatile("" ::"v"(touch));
            // The new key's cache slot is written (above, by this wave): once those stores are
            // complete the key loop's ordinary loads read it (no other wave reads that slot,
            // and nothing on this compute unit has read it in this launch).
            __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
            for (uint32_t st = 0; st < kSteps; ++st) {
                uint4 v = make_uint4(0u, 0u, 0u, 0u);
                if (j16 < p.G) v = *reinterpret_cast<const uint4*>(qs + j16 * D + kb * 8u + st * 32u);
                qa[st] = __builtin_bit_cast(bf16x8_t, v);
            }
        }
    } else {
        const bool valid = j16 < rows;
        const uint32_t t = valid ? j16 / p.G : 0u;
        const uint32_t h = hk * p.G + (j16 - t * p.G);
        const uint16_t* src = p.q + (static_cast<size_t>(t) * p.H + h) * D + kb * 8u;
#pragma unroll
        for (uint32_t st = 0; st < kSteps; ++st) {
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (valid) v = *reinterpret_cast<const uint4*>(src + st * 32u);
            qa[st] = __builtin_bit_cast(bf16x8_t, v);
        }
    }

    f32x4_t o[kDTiles];
#pragma unroll
    for (uint32_t t = 0; t < kDTiles; ++t) o[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m[4], l[4];
    int32_t qpos[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        m[i] = -__builtin_huge_valf();
        l[i] = 0.0f;
        const uint32_t r = 4u * kb + i;
        qpos[i] = r < rows ? static_cast<int32_t>(p.offset + r / p.G) : -1;
    }

    // Per 16-key column tile c: K rows into the B operands, V rows (coalesced, lane cidx takes
    // chunk cidx % (D/8) of key cidx / (D/8)) into registers, every load of the tile issued
    // before its first use; with D <= 256 both tiles' loads are issued together.
    constexpr uint32_t kChunks = D / 8u;
    constexpr uint32_t kVPer = 16u * kChunks / 64u;   // V chunks per lane per 16-key tile
    constexpr uint32_t kTilesUpFront = D <= 256u ? 2u : 1u;
    for (uint32_t jb = j_begin; jb < j_end; jb += kKeyBlock) {
        const uint32_t nk = min(kKeyBlock, j_end - jb);
        f32x4_t sc[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (uint32_t c0 = 0; c0 < 2u; c0 += kTilesUpFront) {
            uint4 kr[kTilesUpFront][kSteps];
            uint4 vr[kTilesUpFront][kVPer];
#pragma unroll
            for (uint32_t u = 0; u < kTilesUpFront; ++u) {
                const uint32_t c = c0 + u;
                const uint32_t key = 16u * c + j16;
                const uint16_t* row = key < nk ? key_row(p, p.k, p.ck, jb + key, hk, D) + kb * 8u : nullptr;
#pragma unroll
                for (uint32_t st = 0; st < kSteps; ++st) {
                    kr[u][st] = row != nullptr ? *reinterpret_cast<const uint4*>(row + st * 32u)
                                               : make_uint4(0u, 0u, 0u, 0u);
                }
#pragma unroll
                for (uint32_t it = 0; it < kVPer; ++it) {
                    const uint32_t cidx = lane + 64u * it;
                    const uint32_t r = 16u * c + cidx / kChunks;
                    const uint32_t ch = cidx % kChunks;
                    vr[u][it] = r < nk ? *reinterpret_cast<const uint4*>(key_row(p, p.v, p.cv, jb + r, hk, D) + ch * 8u)
                                       : make_uint4(0u, 0u, 0u, 0u);
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < kTilesUpFront; ++u) {
                const uint32_t c = c0 + u;
                // V rows into LDS as loaded.
#pragma unroll
                for (uint32_t it = 0; it < kVPer; ++it) {
                    const uint32_t cidx = lane + 64u * it;
                    const uint32_t r = 16u * c + cidx / kChunks;
                    const uint32_t ch = cidx % kChunks;
                    *reinterpret_cast<uint4*>(my + Lds::kV + r * Lds::kVRow + ch * 16u) = vr[u][it];
                }
                // S for this tile's 16 keys.
#pragma unroll
                for (uint32_t st = 0; st < kSteps; ++st) {
                    sc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[st], __builtin_bit_cast(bf16x8_t, kr[u][st]),
                                                                    sc[c], 0, 0, 0);
                }
            }
        }
        // Mask, online softmax (log2 domain), P -> LDS as bf16.
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            float sv[2];
            float bmax = -__builtin_huge_valf();
#pragma unroll
            for (uint32_t c = 0; c < 2; ++c) {
                const uint32_t key = 16u * c + j16;
                const int32_t kpos = static_cast<int32_t>(p.offset - p.prefix + jb + key);
                const bool vis = key < nk && qpos[i] >= 0 && kpos <= qpos[i] &&
                                 (p.window == 0u || kpos > qpos[i] - static_cast<int32_t>(p.window));
                sv[c] = vis ? sc[c][i] * kLog2e : -__builtin_huge_valf();
                bmax = fmaxf(bmax, sv[c]);
            }
            bmax = row16_max(bmax, lane);
            const float m_new = fmaxf(m[i], bmax);
            const bool any = m_new > -__builtin_huge_valf();
            const float alpha = any ? exp2f(m[i] - m_new) : 1.0f;
            float psum = 0.0f;
#pragma unroll
            for (uint32_t c = 0; c < 2; ++c) {
                const float pv = any && sv[c] > -__builtin_huge_valf() ? exp2f(sv[c] - m_new) : 0.0f;
                psum += pv;
                *reinterpret_cast<uint16_t*>(my + Lds::kP + (4u * kb + i) * Lds::kPRow + (16u * c + j16) * 2u) =
                    f32_to_bf16_bits(pv);
            }
            psum = row16_sum(psum, lane);
            l[i] = l[i] * alpha + psum;
            m[i] = any ? m_new : m[i];
#pragma unroll
            for (uint32_t t = 0; t < kDTiles; ++t) o[t][i] *= alpha;
        }
        // O += P V: the B operand of dim tile t by transposing reads of the V rows (the
        // lanes 4e .. 4e + 3 of a 16-lane group address key 8kb + e at dims 16t + 4(j % 4),
        // and lane j receives V[8kb + e][16t + j] as element e).
        const bf16x8_t pa = *reinterpret_cast<const bf16x8_t*>(my + Lds::kP + j16 * Lds::kPRow + kb * 16u);
        uint8_t* vt = my + Lds::kV + (8u * kb + (j16 >> 2)) * Lds::kVRow + (j16 & 3u) * 8u;
#pragma unroll
        for (uint32_t t = 0; t < kDTiles; ++t) {
            o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, v_operand_tr(vt + 32u * t, Lds::kVRow), o[t], 0, 0, 0);
        }
    }

    // Rows 4 kb + i, dims 16 t + j16.
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t r = 4u * kb + i;
        if (r >= rows) continue;
        const uint32_t t = r / p.G;
        const uint32_t h = hk * p.G + (r - t * p.G);
        const size_t orow = static_cast<size_t>(t) * p.H + h;
        if (p.splits == 1u) {
            const float inv = l[i] > 0.0f ? 1.0f / l[i] : 0.0f;
#pragma unroll
            for (uint32_t tt = 0; tt < kDTiles; ++tt) p.out[orow * D + 16u * tt + j16] = f32_to_bf16_bits(o[tt][i] * inv);
        } else {
            const size_t prow = static_cast<size_t>(split) * p.L * p.H + orow;
#pragma unroll
            for (uint32_t tt = 0; tt < kDTiles; ++tt) p.part_o[prow * D + 16u * tt + j16] = o[tt][i];
            if (j16 == 0u) {
                p.part_ml[prow * 2u] = m[i];
                p.part_ml[prow * 2u + 1u] = l[i];
            }
        }
    }
}

// Merge the splits of each output row: weights 2^(m_s - max m), sum of l_s, divided sums.
// One workgroup per row and 256 dims (two per row at head_dim 512: 10.8 -> 4.x us for the
// 12B's global rows), every load issued at once: each wave reads all (m, l) (lane s holds
// split s) and the partial rows of splits w, w + 4, ... (lane-owned dims); the four wave
// sums meet in LDS and are added in wave order.
template <uint32_t D>
__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(AttnParams p) {
    constexpr uint32_t kWaves = kAttnThreads / 64u;
    constexpr uint32_t kDW = D < 256u ? D : 256u;   // dims of this workgroup: [d0, d0 + kDW)
    constexpr uint32_t kPer = kDW / 64u;
    constexpr uint32_t kMaxPerWave = kAttnMaxSplits / kWaves;
    __shared__ float acc[kWaves][kDW];
    __shared__ float dens[kWaves];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint64_t rows = static_cast<uint64_t>(p.L) * p.H;
    const uint64_t row = blockIdx.x;
    const uint32_t d0 = blockIdx.y * kDW;
    float ms = -__builtin_huge_valf();
    float ls = 0.0f;
    if (lane < p.splits) {
        ms = p.part_ml[(lane * rows + row) * 2u];
        ls = p.part_ml[(lane * rows + row) * 2u + 1u];
    }
    float part[kMaxPerWave][kPer];
#pragma unroll
    for (uint32_t u = 0; u < kMaxPerWave; ++u) {
        const uint32_t sp = wave + kWaves * u;
        const float* o = p.part_o + (sp * rows + row) * D + d0 + lane * kPer;
#pragma unroll
        for (uint32_t e = 0; e < kPer; ++e) part[u][e] = sp < p.splits ? o[e] : 0.0f;
    }
    const float mx = butterfly_max64(ms, lane);
    const float w = ms == -__builtin_huge_valf() || mx == -__builtin_huge_valf() ? 0.0f : exp2f(ms - mx);
    float num[kPer];
#pragma unroll
    for (uint32_t e = 0; e < kPer; ++e) num[e] = 0.0f;
    float den = 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < kMaxPerWave; ++u) {
        const uint32_t sp = wave + kWaves * u;
        // Split sp's weight and l from lane sp (sp is uniform: a scalar read of one lane).
        const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), static_cast<int>(sp & 63u)));
        const float lw = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ls), static_cast<int>(sp & 63u)));
        if (sp >= p.splits || ws == 0.0f) continue;   // uniform: past the splits, or an empty split
        den += ws * lw;
#pragma unroll
        for (uint32_t e = 0; e < kPer; ++e) num[e] += ws * part[u][e];
    }
#pragma unroll
    for (uint32_t e = 0; e < kPer; ++e) acc[wave][lane * kPer + e] = num[e];
    if (lane == 0u) dens[wave] = den;
    __syncthreads();
    if (wave != 0u) return;
    float dt = 0.0f;
#pragma unroll
    for (uint32_t wv = 0; wv < kWaves; ++wv) dt += dens[wv];
    uint16_t* out = p.out + row * D + d0 + lane * kPer;
#pragma unroll
    for (uint32_t e = 0; e < kPer; ++e) {
        float v = 0.0f;
#pragma unroll
        for (uint32_t wv = 0; wv < kWaves; ++wv) v += acc[wv][lane * kPer + e];
        out[e] = f32_to_bf16_bits(dt > 0.0f ? v / dt : 0.0f);
    }
}

// The chunk form's merge of its key splits (at most kChunkMaxSplits): thread c takes the 8
// dims ch = c % (D/8) of row c / (D/8), the splits weighted as in attn_combine_kernel
// (2^(m_s - max m), the sum of l_s, the divided sum).
constexpr uint32_t kChunkMaxSplits = 2;
template <uint32_t D>
__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(AttnParams p) {
    constexpr uint32_t kCh = D / 8u;
    const uint64_t rows = static_cast<uint64_t>(p.L) * p.H;
    const uint64_t c = static_cast<uint64_t>(blockIdx.x) * kAttnThreads + threadIdx.x;
    if (c >= rows * kCh) return;
    const uint64_t row = c / kCh;
    const uint32_t ch = static_cast<uint32_t>(c - row * kCh);
    float ms[kChunkMaxSplits];
    float ls[kChunkMaxSplits];
    float4 lo[kChunkMaxSplits];
    float4 hi[kChunkMaxSplits];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (uint32_t s = 0; s < kChunkMaxSplits; ++s) {
        const bool live = s < p.splits;
        ms[s] = live ? p.part_ml[(s * rows + row) * 2u] : -__builtin_huge_valf();
        ls[s] = live ? p.part_ml[(s * rows + row) * 2u + 1u] : 0.0f;
        const float4* o4 = reinterpret_cast<const float4*>(p.part_o + (s * rows + row) * D + ch * 8u);
        lo[s] = live ? o4[0] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        hi[s] = live ? o4[1] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        mx = fmaxf(mx, ms[s]);
    }
    float den = 0.0f;
    float num[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t s = 0; s < kChunkMaxSplits; ++s) {
        const float w = ms[s] == -__builtin_huge_valf() || mx == -__builtin_huge_valf() ? 0.0f : exp2f(ms[s] - mx);
        if (w == 0.0f) continue;
        den += w * ls[s];
        const float v[8] = {lo[s].x, lo[s].y, lo[s].z, lo[s].w, hi[s].x, hi[s].y, hi[s].z, hi[s].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) num[e] += w * v[e];
    }
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = f32_to_bf16_bits(den > 0.0f ? num[e] / den : 0.0f);
    *reinterpret_cast<uint4*>(p.out + row * D + ch * 8u) =
        make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

// Tokens pos0 .. pos0 + n - 1 of k/v [n][KVH][D] -> cache slots pos % cap (only the last
// `cap` of them when n > cap: earlier ones would be overwritten in the same slots).
__global__ __launch_bounds__(kAttnThreads) void kv_write_kernel(const uint16_t* __restrict__ k,
                                                               const uint16_t* __restrict__ v, uint16_t* ck,
                                                               uint16_t* cv, uint32_t n_skip, uint32_t n,
                                                               uint32_t pos0, uint32_t cap, uint32_t row_elems) {
    const uint64_t c = static_cast<uint64_t>(blockIdx.x) * kAttnThreads + threadIdx.x;   // 16-byte chunk
    const uint32_t per_tok = row_elems / 8u;
    const uint64_t total = static_cast<uint64_t>(n - n_skip) * per_tok;
    if (c >= total) return;
    const uint32_t t = n_skip + static_cast<uint32_t>(c / per_tok);
    const uint32_t ch = static_cast<uint32_t>(c % per_tok);
    const uint32_t slot = (pos0 + t) % cap;
    const size_t src = static_cast<size_t>(t) * row_elems + ch * 8u;
    const size_t dst = static_cast<size_t>(slot) * row_elems + ch * 8u;
    *reinterpret_cast<uint4*>(ck + dst) = *reinterpret_cast<const uint4*>(k + src);
    *reinterpret_cast<uint4*>(cv + dst) = *reinterpret_cast<const uint4*>(v + src);
}

template <uint32_t D>
void launch_decode_d(const AttnParams& p, bool prep, hipStream_t stream) {
    using Lds = DecodeLds<D>;
    constexpr size_t lds = Lds::kBytes;
    static_assert(lds <= 160u * 1024u, "decode attention LDS");
    if (lds > 65536u) {
        static thread_local int configured_device = -1;
        int dev = 0;
        HYP_HIP_CHECK(hipGetDevice(&dev));
        if (configured_device != dev) {
            for (const void* f : {reinterpret_cast<const void*>(attn_decode_kernel<D, false>),
                                  reinterpret_cast<const void*>(attn_decode_kernel<D, true>),
                                  reinterpret_cast<const void*>(attn_decode_kernel<D, true, kPrepLanes<D>>)}) {
                HYP_HIP_CHECK(
                    hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
            }
            configured_device = dev;
        }
    }
    const dim3 grid((p.splits + Lds::kWaves - 1u) / Lds::kWaves, p.KVH);
    // The folded prepare spread over kPrepLanes<D> lanes per unit where the G query rows, K and
    // V of a kv head fit one wave that way.
    const bool spread = prep && (p.G + 2u) * (D / 64u) * kPrepLanes<D> <= 64u;
    auto kernel = !prep ? attn_decode_kernel<D, false>
                        : (spread ? attn_decode_kernel<D, true, kPrepLanes<D>> : attn_decode_kernel<D, true>);
    hipLaunchKernelGGL(kernel, grid, dim3(Lds::kWaves * 64u), lds, stream, p);
    HYP_HIP_CHECK(hipGetLastError());
}

template <uint32_t D>
void launch_attn_d(const AttnParams& p, hipStream_t stream) {
    constexpr size_t lds = AttnLds<D>::kBytes;
    static_assert(lds <= 160u * 1024u, "attention LDS");
    if (lds > 65536u) {
        static thread_local int configured_device = -1;
        int dev = 0;
        HYP_HIP_CHECK(hipGetDevice(&dev));
        if (configured_device != dev) {
            HYP_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(attn_kernel<D>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
            configured_device = dev;
        }
    }
    const uint32_t tiles = (p.L * p.G + kRowsPerTile - 1u) / kRowsPerTile;
    hipLaunchKernelGGL(attn_kernel<D>, dim3(tiles, p.KVH, p.splits), dim3(kAttnThreads), lds, stream, p);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace

namespace {

// The chunk form at most one workgroup per compute unit (a prefill chunk of up to about
// 1024 tokens on the 12B's layers): one wave per SIMD leaves every LDS and MFMA dependency
// exposed and the causal tiles' lengths run 1 .. L / 32 blocks. Two key splits give two
// resident workgroups per compute unit and halve the longest tile; attn_combine_kernel
// merges them (measured below).
bool chunk_split_pays(uint32_t L, uint32_t n_heads, uint32_t n_kv_heads, uint32_t keys) {
    const uint32_t G = n_heads / n_kv_heads;
    const uint64_t tiles = (static_cast<uint64_t>(L) * G + kRowsPerTile - 1u) / kRowsPerTile * n_kv_heads;
    return tiles <= device_compute_units() && keys >= 8u * kKeyBlock;
}

size_t chunk_split_bytes(uint32_t L, uint32_t n_heads, uint32_t head_dim) {
    return 2u * static_cast<size_t>(L) * n_heads * (static_cast<size_t>(head_dim) * 4u + 8u);
}

}  // namespace

size_t attention_chunk_workspace_bytes(uint32_t max_L, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim) {
    // The longest chunk that still splits (its tiles fit the compute units), within max_L,
    // for MI355X's 256 compute units (a plan needs no device; on a larger part the chunks
    // this does not cover run unsplit).
    constexpr uint64_t kPlanComputeUnits = 256;
    const uint32_t G = n_heads / n_kv_heads;
    const uint64_t fit = static_cast<uint64_t>(kRowsPerTile) * (kPlanComputeUnits / n_kv_heads) / G;
    const uint32_t L = static_cast<uint32_t>(std::min<uint64_t>(max_L, fit));
    return L > kRowsPerTile / G ? chunk_split_bytes(L, n_heads, head_dim) : 0u;
}

size_t attention_workspace_bytes(uint32_t n_kv_heads, uint32_t head_dim) {
    // Split partials for decode: at most kAttnMaxSplits splits of one row tile per kv head.
    const size_t rows = static_cast<size_t>(kRowsPerTile) * n_kv_heads;
    return kAttnMaxSplits * rows * (static_cast<size_t>(head_dim) * 4u + 8u);
}

void launch_kv_write(const uint16_t* k, const uint16_t* v, uint16_t* ck, uint16_t* cv, uint32_t n, uint32_t pos0,
                     uint32_t cap, uint32_t n_kv_heads, uint32_t head_dim, hipStream_t stream) {
    if (n == 0) return;
    const uint32_t skip = n > cap ? n - cap : 0u;
    const uint32_t row_elems = n_kv_heads * head_dim;
    const uint64_t chunks = static_cast<uint64_t>(n - skip) * (row_elems / 8u);
    const uint64_t blocks = (chunks + kAttnThreads - 1u) / kAttnThreads;
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "kv write: too many tokens");
    hipLaunchKernelGGL(kv_write_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kAttnThreads), 0, stream, k, v, ck,
                       cv, skip, n, pos0, cap, row_elems);
    HYP_HIP_CHECK(hipGetLastError());
}

bool attention_prep_fits(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim) {
    // Only the decode form folds the prepare, and one token takes it when its G query rows fit
    // the single row tile (G <= 16); the G query rows, K and V of one kv head must also fit
    // one wave as 64-value units, one per lane.
    if (n_kv_heads == 0u || n_heads % n_kv_heads != 0u) return false;
    const uint32_t G = n_heads / n_kv_heads;
    return G <= 16u && (G + 2u) * (head_dim / 64u) <= 64u;
}

// The decode form's splits: one wave per block of 32 keys (each wave then makes a single
// round trip to memory for its keys), within kAttnMaxSplits.
uint32_t decode_splits(uint32_t n_kv_heads, uint32_t keys) {
    (void)n_kv_heads;
    return std::max(1u, std::min(kAttnMaxSplits, (keys + kKeyBlock - 1u) / kKeyBlock));
}

uint32_t attention_splits(uint32_t L, uint32_t n_heads, uint32_t n_kv_heads, uint32_t keys) {
    if (static_cast<uint64_t>(L) * (n_heads / n_kv_heads) <= 16u) return decode_splits(n_kv_heads, keys);
    // One row tile per kv head (decode): split the keys so the grid covers the compute
    // units, at least 64 keys per split.
    const uint32_t G = n_heads / n_kv_heads;
    if (static_cast<uint64_t>(L) * G > kRowsPerTile) return chunk_split_pays(L, n_heads, n_kv_heads, keys) ? 2u : 1u;
    const uint32_t cus = device_compute_units();
    uint32_t s = 1u;
    while (s < kAttnMaxSplits && n_kv_heads * s * 2u <= cus && keys >= 64u * (s * 2u)) s *= 2u;
    return s;
}

void launch_attention(const AttnArgs& a, hipStream_t stream) {
    AttnParams p{};
    p.q = a.q;
    p.k = a.k;
    p.v = a.v;
    p.ck = a.cache_k;
    p.cv = a.cache_v;
    p.out = a.out;
    p.L = a.L;
    p.H = a.n_heads;
    p.KVH = a.n_kv_heads;
    p.G = a.n_heads / a.n_kv_heads;
    p.cap = a.cap;
    p.offset = a.offset;
    p.prefix = a.prefix_len;
    p.window = a.window;
    const uint32_t T = a.prefix_len + a.L;
    p.pos = a.pos;
    if (a.pos != nullptr) {
        // A grid fixed for every position the captured launch will see (the kernel
        // derives its key ranges from *pos; splits past the keys write empty partials).
        p.splits = std::max(1u, std::min(a.fixed_splits, kAttnMaxSplits));
        p.keys_per_split = kKeyBlock;
    } else {
        p.splits = attention_splits(a.L, a.n_heads, a.n_kv_heads, T);
        const bool chunk = static_cast<uint64_t>(a.L) * p.G > kRowsPerTile;
        // The chunk form splits into a workspace that holds it.
        if (chunk && p.splits > 1u &&
            (a.workspace == nullptr || a.workspace_bytes < chunk_split_bytes(a.L, a.n_heads, a.head_dim)))
            p.splits = 1u;
        p.keys_per_split = ((T + p.splits - 1u) / p.splits + kKeyBlock - 1u) / kKeyBlock * kKeyBlock;
        p.splits = std::max(1u, (T + p.keys_per_split - 1u) / p.keys_per_split);   // no empty split
    }
    if (p.splits > 1u && static_cast<uint64_t>(a.L) * p.G > kRowsPerTile) {
        // chunk form: checked above
        const size_t rows = static_cast<size_t>(a.L) * a.n_heads;
        p.part_o = static_cast<float*>(a.workspace);
        p.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(a.workspace) +
                                             static_cast<size_t>(p.splits) * rows * a.head_dim * 4u);
    } else if (p.splits > 1u) {
        HYP_REQUIRE(a.workspace != nullptr &&
                        a.workspace_bytes >= attention_workspace_bytes(a.n_kv_heads, a.head_dim),
                    HYP_STATUS_INTERNAL, "attention: split workspace too small");
        const size_t rows = static_cast<size_t>(a.L) * a.n_heads;
        p.part_o = static_cast<float*>(a.workspace);
        p.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(a.workspace) +
                                             static_cast<size_t>(p.splits) * rows * a.head_dim * 4u);
    }
    const bool decode = static_cast<uint64_t>(a.L) * p.G <= 16u;
    const bool prep = a.prep != nullptr;
    if (prep) {
        const AttnPrepareArgs& pa = *a.prep;
        HYP_REQUIRE(decode && a.L == 1u && a.k == nullptr && a.v == nullptr && pa.rope_cs != nullptr &&
                        pa.L == 1u && pa.head_dim == a.head_dim && pa.n_heads == a.n_heads &&
                        pa.n_kv_heads == a.n_kv_heads && pa.cap == a.cap && pa.pos == a.pos &&
                        (a.pos != nullptr || pa.offset == a.offset) && pa.q == a.q &&
                        pa.cache_k == a.cache_k && pa.cache_v == a.cache_v && attention_prep_fits(a.n_heads, a.n_kv_heads, a.head_dim),
                    HYP_STATUS_INTERNAL, "attention: the folded prepare needs one token, the cache form and a RoPE table");
        p.rope_cs = pa.rope_cs;
        p.q_w = pa.q_norm;
        p.k_w = pa.k_norm;
        p.k_raw = pa.k_raw;
        p.v_raw = pa.v_raw;
        p.ck_out = pa.cache_k;
        p.cv_out = pa.cache_v;
        p.eps = pa.eps;
    }
    switch (a.head_dim) {
        case 64: decode ? launch_decode_d<64>(p, prep, stream) : launch_attn_d<64>(p, stream); break;
        case 128: decode ? launch_decode_d<128>(p, prep, stream) : launch_attn_d<128>(p, stream); break;
        case 256: decode ? launch_decode_d<256>(p, prep, stream) : launch_attn_d<256>(p, stream); break;
        case 512: decode ? launch_decode_d<512>(p, prep, stream) : launch_attn_d<512>(p, stream); break;
        default: throw NativeError(HYP_STATUS_UNSUPPORTED, "attention: head_dim must be 64, 128, 256 or 512");
    }
    if (p.splits > 1u && static_cast<uint64_t>(a.L) * p.G > kRowsPerTile) {
        // chunk form: many rows, two splits; a thread per 8 dims of a row
        const uint64_t threads = static_cast<uint64_t>(a.L) * a.n_heads * (a.head_dim / 8u);
        const uint64_t blocks = (threads + kAttnThreads - 1u) / kAttnThreads;
        HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "attention: too many rows to merge");
        switch (a.head_dim) {
            case 64: hipLaunchKernelGGL(attn_merge_kernel<64>, dim3(blocks), dim3(kAttnThreads), 0, stream, p); break;
            case 128: hipLaunchKernelGGL(attn_merge_kernel<128>, dim3(blocks), dim3(kAttnThreads), 0, stream, p); break;
            case 256: hipLaunchKernelGGL(attn_merge_kernel<256>, dim3(blocks), dim3(kAttnThreads), 0, stream, p); break;
            default: hipLaunchKernelGGL(attn_merge_kernel<512>, dim3(blocks), dim3(kAttnThreads), 0, stream, p); break;
        }
        HYP_HIP_CHECK(hipGetLastError());
    } else if (p.splits > 1u) {
        const uint64_t rows = static_cast<uint64_t>(a.L) * a.n_heads;
        HYP_REQUIRE(rows <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "attention: too many rows to combine");
        const dim3 grid(static_cast<uint32_t>(rows), a.head_dim > 256u ? a.head_dim / 256u : 1u);
        switch (a.head_dim) {
            case 64: hipLaunchKernelGGL(attn_combine_kernel<64>, grid, dim3(kAttnThreads), 0, stream, p); break;
            case 128: hipLaunchKernelGGL(attn_combine_kernel<128>, grid, dim3(kAttnThreads), 0, stream, p); break;
            case 256: hipLaunchKernelGGL(attn_combine_kernel<256>, grid, dim3(kAttnThreads), 0, stream, p); break;
            default: hipLaunchKernelGGL(attn_combine_kernel<512>, grid, dim3(kAttnThreads), 0, stream, p); break;
        }
        HYP_HIP_CHECK(hipGetLastError());
    }
}

}  // namespace hyperion::hip

// Skinny quantized matmul (decode, m <= 4 activation rows) on gfx950 MFMA.
//
// Replaces mlx::core::quantized_matmul(x, w, scales, biases, transpose=true, 64, 4,
// "affine") at decode (native/hyperion_mlx/src/weights.h:26-37, called from
// forward.cc:395,399,409,507 for q/k/v/o, forward.cc:338-343 for the MLP and
// forward.cc:137-152 for the tied LM head).
//
// The op is HBM-bound (0.5625 B per weight, read once), so the design keeps the
// vector-ALU work per weight far below what the memory stream allows:
//  * The dot products run on the matrix cores. One v_mfma_f32_16x16x32_bf16 covers
//    16 weight rows x 32 k: the weights are its B operand (lane j = l % 16 holds row
//    j), the activations its A operand, and only A rows i < m carry data (rows
//    i >= m read a copy of x row m-1; their outputs are never stored).
//  * A packed word (8 codes, lowest k in the lowest nibble) becomes a lane's 8 bf16
//    B values with 3 shifts and 4 v_and_or_b32: (w >> 4s) & 0x000F000F | 0x43004300
//    is the bf16 pair (128 + q_s, 128 + q_{s+4}) exactly (bf16 128.0 has ulp 1). For
//    one matrix, two adjacent words share each shift as one 64-bit shift.
//  * One matrix, whole range in flight: the scale and bias are applied once per lane for
//    four groups instead of per group, because each 4-row block of the MFMA output
//    accumulates the m rows of one group of every two pairs (its A rows read x in that
//    group's MFMAs and a zero row in the others); the blocks are added across lanes at the end.
//    The A values use the same slot order: x is staged in LDS once per workgroup as
//    (x0,x4),(x1,x5),(x2,x6),(x3,x7) per 8-element word, next to the per-group sums
//    of x that remove the +128 offset.
//  * The weights are read in the tiled resident layout (q4_layout.h): per 16-row tile
//    and pair of groups, lane (j, kb = l / 16) loads one contiguous 16-byte entry
//    holding words 2kb and 2kb+1 of row j for both groups (the wave reads 1 KB of
//    contiguous bytes per instruction), and lane j one 8-byte entry with both groups'
//    scale and bias (128 contiguous bytes). A group is 2 MFMAs (words {0,2,4,6}, then
//    {1,3,5,7}) into a fresh accumulator, after which lane j < 16 applies the group's
//    bf16 scale and bias:
//        y[i][j] += s * (acc[i][j] - 128 * sum_g(x_i)) + b * sum_g(x_i).
//    Every partial product is exact in fp32 and accumulation is fp32. The two groups
//    of a pair are independent accumulator chains, so the matrix core and the VALU
//    overlap.
//  * A wave owns 16 rows and a contiguous range of pairs of groups (S waves of a
//    workgroup share the rows and meet in LDS at the end). Loads go through buffer
//    resources with the non-temporal policy (the weights are streamed once): the lane's
//    offset is a VGPR, the pair offset a scalar, so addressing costs no VALU.
//  * A compute unit accepts new loads only as fast as earlier ones return, so the order
//    of issue decides what arrives first. x is requested first by the waves that stage
//    it, a raw barrier (no memory wait) puts every weight load of the workgroup behind
//    those requests, and then each wave issues its weights (all of them when they fit in
//    two register batches). The staging waves publish x through an LDS counter that the
//    others poll, so no wave waits for another wave's loads to be issued.
#include "common.h"
#include "kernels.h"
#include "q4_layout.h"
#include "q4_rmsnorm.h"

namespace hyperion::hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kMaxSegments = 3;   // projections sharing x in one grouped launch
constexpr int kSkinnyWaves = 16;        // waves per workgroup (the softcap head uses 4)
constexpr uint32_t kSkinnyPairsUpFront = 8;   // two batches of 4 pairs: a wave's whole range at once
constexpr int kSkinnyDualWaves = 8;     // the fused gate/up: two accumulator sets per wave

constexpr uint32_t kNibbleMask = 0x000F000Fu;
constexpr uint32_t kMagic128 = 0x43004300u;   // bf16 pair (128.0, 128.0)
constexpr uint32_t kOnePair = 0x3F803F80u;    // bf16 pair (1.0, 1.0)

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

// The 8 codes of a packed word as MFMA B values (128+q0, 128+q4, 128+q1, 128+q5, ...).
__device__ __forceinline__ bf16x8_t code_frag(uint32_t w, uint32_t mask, uint32_t bits) {
    uint4 r;
    r.x = and_or(w, mask, bits);
    r.y = and_or(w >> 4, mask, bits);
    r.z = and_or(w >> 8, mask, bits);
    r.w = and_or(w >> 12, mask, bits);
    return __builtin_bit_cast(bf16x8_t, r);
}

// code_frag of two adjacent words (lo, hi) with one 64-bit shift per step instead of a
// 32-bit shift per word (v_lshrrev_b64 runs at full rate on gfx950): the bits of hi that
// the shift moves into lo's top (bits 20..31 at most) lie outside the mask.
__device__ __forceinline__ void code_frag2(uint32_t lo, uint32_t hi, uint32_t mask, uint32_t bits, bf16x8_t& f_lo,
                                           bf16x8_t& f_hi) {
    const uint64_t v = (static_cast<uint64_t>(hi) << 32) | lo;
    uint64_t s4, s8, s12;
    // As plain C++ the compiler narrows each shift back to two 32-bit ones.
    asm("v_lshrrev_b64 %0, 4, %1" : "=v"(s4) : "v"(v));
    asm("v_lshrrev_b64 %0, 8, %1" : "=v"(s8) : "v"(v));
    asm("v_lshrrev_b64 %0, 12, %1" : "=v"(s12) : "v"(v));
    uint4 a, b;
    a.x = and_or(lo, mask, bits);
    a.y = and_or(static_cast<uint32_t>(s4), mask, bits);
    a.z = and_or(static_cast<uint32_t>(s8), mask, bits);
    a.w = and_or(static_cast<uint32_t>(s12), mask, bits);
    b.x = and_or(hi, mask, bits);
    b.y = and_or(static_cast<uint32_t>(s4 >> 32), mask, bits);
    b.z = and_or(static_cast<uint32_t>(s8 >> 32), mask, bits);
    b.w = and_or(static_cast<uint32_t>(s12 >> 32), mask, bits);
    f_lo = __builtin_bit_cast(bf16x8_t, a);
    f_hi = __builtin_bit_cast(bf16x8_t, b);
}

// The four B fragments of one pair's words: 64-bit shifts for a single matrix; the
// two-matrix (gate/up) form keeps 32-bit shifts, which measured faster there.
template <int NW>
__device__ __forceinline__ void pair_frags(const uint4& w, uint32_t mask, uint32_t bits, bf16x8_t (&b)[4]) {
    if constexpr (NW == 1) {
        code_frag2(w.x, w.y, mask, bits, b[0], b[1]);
        code_frag2(w.z, w.w, mask, bits, b[2], b[3]);
    } else {
        b[0] = code_frag(w.x, mask, bits);
        b[1] = code_frag(w.y, mask, bits);
        b[2] = code_frag(w.z, mask, bits);
        b[3] = code_frag(w.w, mask, bits);
    }
}

// v + the values of lanes l ^ 16, l ^ 32 and l ^ 48, in the same order on all four lanes.
// With v in both operands, v_permlane32_swap leaves each lane's own value in one register
// and the value of lane l ^ 32 in the other (v_permlane16_swap likewise for l ^ 16): two
// VALU swaps instead of LDS permutes. Inline assembly, because the builtins, given equal
// inputs, compiled to an add of one output register to itself. The s_nop gives the two
// wait states a permlane swap needs after a VALU write of its operands.
__device__ __forceinline__ float sum_lane_blocks(float v) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    uint32_t c = u;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(c));
    v = __builtin_bit_cast(float, u) + __builtin_bit_cast(float, c);
    u = __builtin_bit_cast(uint32_t, v);
    c = u;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(u), "+v"(c));
    return __builtin_bit_cast(float, u) + __builtin_bit_cast(float, c);
}

// 128-bit buffer resource over [base, base + bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

// One projection of a (possibly grouped) launch: its 16-row tiles are global tiles
// [tile_begin, tile_begin + ceil(n / 16)).
struct SkinnySegment {
    const uint4* codes;   // tiled codes (q4_layout.h)
    const uint2* sb;      // tiled scales and biases
    uint16_t* y;          // [m, n]
    uint32_t n;
    uint32_t tile_begin;
};

// The fields every launch reads before its first load come first (one 64-byte line).
struct SkinnyParams {
    const uint16_t* x;
    uint32_t nseg;
    uint32_t k;
    uint32_t pairs;       // ceil(k / 128)
    uint32_t splits;      // waves sharing one 16-row tile (divides the workgroup's waves)
    uint32_t split_shift; // log2(splits): splits is a power of two
    float cap;            // bf16 softcap constant
    SkinnySegment seg[kMaxSegments];   // segments past nseg are unused
    const uint4* codes2;               // fused gate/up: the up projection (same n, k as seg[0])
    const uint2* sb2;
    float eps;            // NORM: rms normalisation epsilon
};

// One matrix as seen by one lane: buffer resources and the lane's offsets into them.
struct LaneMatrix {
    __amdgpu_buffer_rsrc_t codes;
    __amdgpu_buffer_rsrc_t sb;
    uint32_t c_off;    // (tile * pairs * 64 + lane) * 16 bytes
    uint32_t sb_off;   // (tile * pairs * 16 + j) * 8 bytes
};

// P pairs of groups of one matrix for one lane.
template <int P>
struct Batch {
    uint4 w[P];    // words 2kb, 2kb+1 of the pair's two groups
    uint2 sb[P];   // (scale | bias << 16) of the pair's two groups
};

// Cache policy of the weight loads: non-temporal (each byte is read once per launch).
constexpr int kStreamPolicy = 2;

// Pairs first, first + 1, ... (wave-uniform, so the clamp is a scalar op); indices past
// `last` are clamped to it, so every byte read lies inside the tile.
template <int P, bool SB = true>
__device__ __forceinline__ void load_batch(const LaneMatrix& lm, uint32_t first, uint32_t last, Batch<P>& bt) {
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const uint32_t gp = min(first + i, last);
        bt.w[i] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(lm.codes, lm.c_off, gp * 1024u, kStreamPolicy));
        if constexpr (SB)
            bt.sb[i] = __builtin_bit_cast(
                uint2, __builtin_amdgcn_raw_buffer_load_b64(lm.sb, lm.sb_off, gp * 128u, kStreamPolicy));
    }
}

// The row of staging unit u (units are row-major, G per row), without a division.
template <int M>
__device__ __forceinline__ uint32_t unit_row(uint32_t u, uint32_t G) {
    uint32_t m = 0u;
#pragma unroll
    for (int r = 1; r < M; ++r) m += u >= static_cast<uint32_t>(r) * G ? 1u : 0u;
    return m;
}

// Spin (bounded) until the LDS counter reaches `target`. The waves that raise it are in
// the same workgroup and never wait on the polling waves, so the bound is never reached
// in a correct launch; it only guarantees that every wave terminates.
__device__ __forceinline__ void wait_counter(const uint32_t* ctr, uint32_t target) {
    for (uint32_t spin = 0; spin < (1u << 24); ++spin) {
        if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// This wave's LDS writes become visible, then the counter is raised once.
__device__ __forceinline__ void raise_counter(uint32_t* ctr, uint32_t lane) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0u) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// y += s * (acc - 128 * sum(x)) + b * sum(x) for one group (acc[m] is D[i = m][j] on
// lanes j < 16 for m < 4; sxg has the group's sums of x rows 0..3).
template <int M>
__device__ __forceinline__ void group_scale(const f32x4_t& acc, uint32_t sbw, const float4& sxg, float (&y)[M]) {
    const float sc = bf16_bits_to_f32(sbw & 0xFFFFu);
    const float bi = bf16_bits_to_f32(sbw >> 16);
    const float sxv[4] = {sxg.x, sxg.y, sxg.z, sxg.w};
#pragma unroll
    for (int m = 0; m < M; ++m) {
        y[m] = fmaf(sc, fmaf(-128.0f, sxv[m], acc[m]), y[m]);
        y[m] = fmaf(bi, sxv[m], y[m]);
    }
}

// Operands of one pair: the 4 B fragments per matrix (groups g0, g1 x two MFMA
// steps) and the 4 A fragments they meet.
template <int NW>
struct PairOperands {
    bf16x8_t b[NW][4];
    uint4 a[4];
};

template <int NW, int P>
__device__ __forceinline__ void load_operands(const Batch<P> (&bt)[NW], int i, const uint4* xa, uint32_t g0,
                                              uint32_t G, uint32_t mask, uint32_t bits, PairOperands<NW>& op) {
#pragma unroll
    for (int q = 0; q < NW; ++q) {
        pair_frags<NW>(bt[q].w[i], mask, bits, op.b[q]);
    }
    const uint32_t g1 = min(g0 + 1u, G - 1u);   // an odd group count leaves the last pair half empty
    op.a[0] = xa[g0 * 8u];
    op.a[1] = xa[g0 * 8u + 1u];
    op.a[2] = xa[g1 * 8u];
    op.a[3] = xa[g1 * 8u + 1u];
}

// The valid pairs of batch `bt` (its first pair is the wave's pair number `base`),
// software-pipelined: pair i's MFMAs are issued, then pair i+1's operands are
// converted and read from LDS while they run, then pair i is scaled.
template <int M, int NW, int P>
__device__ __forceinline__ void compute_batch(const Batch<P> (&bt)[NW], uint32_t base, uint32_t cnt,
                                              uint32_t first, uint32_t G, const uint4* xa, const float4* sx,
                                              uint32_t mask, uint32_t bits, float (&y)[NW][M]) {
    PairOperands<NW> op;
    load_operands<NW, P>(bt, 0, xa, 2u * (first + base), G, mask, bits, op);
#pragma unroll
    for (int i = 0; i < P; ++i) {
        if (base + i >= cnt) break;   // wave-uniform
        const uint32_t gp = first + base + i;
        const uint32_t g0 = 2u * gp;
        const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
        f32x4_t acc0[NW], acc1[NW];
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            acc0[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, op.a[0]), op.b[q][0],
                                                              zero, 0, 0, 0);
            acc1[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, op.a[2]), op.b[q][2],
                                                              zero, 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            acc0[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, op.a[1]), op.b[q][1],
                                                              acc0[q], 0, 0, 0);
            acc1[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, op.a[3]), op.b[q][3],
                                                              acc1[q], 0, 0, 0);
        }
        uint2 sbw[NW];
#pragma unroll
        for (int q = 0; q < NW; ++q) sbw[q] = bt[q].sb[i];
        if (i + 1 < P && base + i + 1 < cnt) load_operands<NW, P>(bt, i + 1, xa, 2u * (gp + 1u), G, mask, bits, op);
        const float4 sx0 = sx[g0];
#pragma unroll
        for (int q = 0; q < NW; ++q) group_scale<M>(acc0[q], sbw[q].x, sx0, y[q]);
        if (g0 + 1u < G) {
            const float4 sx1 = sx[g0 + 1u];
#pragma unroll
            for (int q = 0; q < NW; ++q) group_scale<M>(acc1[q], sbw[q].y, sx1, y[q]);
        }
    }
}

// One pair of groups, in order: its B fragments, A fragments from LDS, four MFMAs per
// matrix, then the two groups' scales. Used where the whole range is in flight, so each
// pair waits only for its own loads.
template <int M, int NW>
__device__ __forceinline__ void compute_pair(const uint4 (&w)[NW], const uint2 (&sbw)[NW], uint32_t gp, uint32_t G,
                                             const uint4* xa, const float4* sx, uint32_t mask, uint32_t bits,
                                             float (&y)[NW][M]) {
    const uint32_t g0 = 2u * gp;
    const uint32_t g1 = min(g0 + 1u, G - 1u);   // an odd group count leaves the last pair half empty
    const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, xa[g0 * 8u]);
    const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, xa[g0 * 8u + 1u]);
    const bf16x8_t a2 = __builtin_bit_cast(bf16x8_t, xa[g1 * 8u]);
    const bf16x8_t a3 = __builtin_bit_cast(bf16x8_t, xa[g1 * 8u + 1u]);
    f32x4_t acc0[NW], acc1[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) {
        bf16x8_t b[4];
        pair_frags<NW>(w[q], mask, bits, b);
        acc0[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[0], zero, 0, 0, 0);
        acc1[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[2], zero, 0, 0, 0);
        acc0[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[1], acc0[q], 0, 0, 0);
        acc1[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b[3], acc1[q], 0, 0, 0);
    }
    const float4 sx0 = sx[g0];
#pragma unroll
    for (int q = 0; q < NW; ++q) group_scale<M>(acc0[q], sbw[q].x, sx0, y[q]);
    if (g0 + 1u < G) {
        const float4 sx1 = sx[g0 + 1u];
#pragma unroll
        for (int q = 0; q < NW; ++q) group_scale<M>(acc1[q], sbw[q].y, sx1, y[q]);
    }
}

// NORM: x rows are first rms-normalised (q4_rmsnorm.h) in LDS; the matmul then runs on
// the normalised rows, which are not written back.
//
// Staging: thread u < M * G owns the 64-element unit (row u / G, group u % G) while
// M * G <= threads; the staging waves are the waves holding units (at least M of them
// with NORM, which forms one row's inverse rms per wave). LDS counters: ctr[0] counts
// staging waves done with x, ctr[1] staging waves done with the NORM partials.
// LOOP: a wave's range may exceed two batches (refilled in a loop); otherwise it fits.
template <int M, bool DUAL, int EPI, int P, int NWAVE, bool NORM, bool LOOP>
__global__ __launch_bounds__(64 * NWAVE) void q4_skinny_kernel(SkinnyParams p) {
    constexpr int NW = DUAL ? 2 : 1;
    constexpr uint32_t kThreads = 64u * NWAVE;
    extern __shared__ __attribute__((aligned(16))) uint4 smem[];

    const uint32_t k = p.k;
    const uint32_t W = k / 8u;    // packed words per row
    const uint32_t G = k / 64u;   // groups per row
    // x rows in LDS are W + 1 chunks apart: W is a multiple of 16 chunks (256 bytes, all 64
    // banks), so unpadded the m rows an A read touches would all start on the same bank.
    const uint32_t WS = W + 1u;
    // Single matrix, whole range in flight: lane blocks take one group each (below). The
    // fused gate/up form measured slower this way (15.3-15.5 against 14.5 us at m = 1).
    constexpr bool kZeroRow = !DUAL;   // as skinny_lds_bytes allocates
    constexpr bool kLaneGroups = kZeroRow && !LOOP;
    uint4* xs = smem;                                              // [M][WS] permuted x
    uint4* zs = smem + M * WS;                                     // kZeroRow: [WS] zeros
    float4* sx = reinterpret_cast<float4*>(zs + (kZeroRow ? WS : 0u));   // [G] group sums of x rows 0..3
    float* red = reinterpret_cast<float*>(sx + G);                 // [NWAVE][NW][M][16]
    uint32_t* ctr = reinterpret_cast<uint32_t*>(red + NWAVE * NW * M * kTileRows);   // [4]
    float* part = reinterpret_cast<float*>(ctr + 4);               // NORM: [M][G] unit partials, [M] inverses

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Shifts, not divisions: everything up to the first weight load is on the critical path.
    const uint32_t S = p.splits;
    const uint32_t sh = p.split_shift;
    const uint32_t split = wave & (S - 1u);
    const uint32_t gtile = (blockIdx.x << (__builtin_ctz(NWAVE) - sh)) + (wave >> sh);   // tile over all segments
    const uint32_t j = lane & 15u;
    const uint32_t kb = lane >> 4;
    const uint32_t pairs = p.pairs;

    // This wave's segment (a wave-uniform branch, no indexed parameter access; a single
    // projection reads only segment 0).
    const uint4* seg_codes = p.seg[0].codes;
    const uint2* seg_sb = p.seg[0].sb;
    uint16_t* seg_y = p.seg[0].y;
    uint32_t seg_n = p.seg[0].n;
    uint32_t tile = gtile;
    if (p.nseg > 1u) {
        const bool in1 = gtile >= p.seg[1].tile_begin;
        const bool in2 = p.nseg > 2u && gtile >= p.seg[2].tile_begin;
        if (in2) {
            seg_codes = p.seg[2].codes;
            seg_sb = p.seg[2].sb;
            seg_y = p.seg[2].y;
            seg_n = p.seg[2].n;
            tile = gtile - p.seg[2].tile_begin;
        } else if (in1) {
            seg_codes = p.seg[1].codes;
            seg_sb = p.seg[1].sb;
            seg_y = p.seg[1].y;
            seg_n = p.seg[1].n;
            tile = gtile - p.seg[1].tile_begin;
        }
    }
    const uint32_t tiles = (seg_n + kTileRows - 1u) / kTileRows;
    const uint32_t ltile = min(tile, tiles - 1u);   // tiles past the matrix are loaded, never stored

    // This wave's pairs: [first, first + cnt), the S ranges as equal as possible
    // (cnt >= 1 since pairs >= S).
    const uint32_t per = pairs >> sh;
    const uint32_t rem = pairs & (S - 1u);
    const uint32_t first = split * per + min(split, rem);
    const uint32_t cnt = per + (split < rem ? 1u : 0u);
    const uint32_t last = first + cnt - 1u;

    const uint32_t units = M * G;
    const uint32_t nstage = max((min(units, kThreads) + 63u) / 64u, NORM ? static_cast<uint32_t>(M) : 1u);
    const bool stager = wave < nstage;

    // x first: thread u's unit is requested before any weight load of the workgroup.
    const uint32_t xu0 = threadIdx.x;   // first (row, group) unit this thread stages
    uint4 xv[8];
    if (xu0 < units) {
        const uint32_t m = unit_row<M>(xu0, G);
        const uint32_t g = xu0 - m * G;
        const uint4* src = reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(m) * k + g * 64u);
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[t] = src[t];
    }
    if (threadIdx.x < 4u) ctr[threadIdx.x] = 0u;
    if constexpr (kLaneGroups)
        for (uint32_t t = threadIdx.x; t < WS; t += kThreads) zs[t] = uint4{0u, 0u, 0u, 0u};
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the counters are cleared
    __builtin_amdgcn_s_barrier();         // no memory wait: only orders the issue

    const uint32_t c_bytes = tiles * pairs * 1024u;
    const uint32_t s_bytes = tiles * pairs * 128u;
    LaneMatrix lm[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) {
        lm[q].codes = buffer_rsrc(q == 0 ? seg_codes : p.codes2, c_bytes);
        lm[q].sb = buffer_rsrc(q == 0 ? seg_sb : p.sb2, s_bytes);
        lm[q].c_off = (ltile * pairs * 64u + lane) * 16u;
        lm[q].sb_off = (ltile * pairs * 16u + j) * 8u;
    }

    // kLaneGroups: lane block ob = lane / 16 scales group 2 (first + 2 b) + ob of each two
    // pairs b: one dword of scale and bias per lane and block (past the wave's range the
    // load reads a neighbour's, or zeros past the buffer; such lanes are masked). They are
    // requested before the codes: loads complete in issue order for the wait counters, so
    // behind the codes the first scaling would wait for every code load of the wave.
    const uint32_t ob = lane >> 4;
    uint32_t sbl[NW][P];
    if constexpr (kLaneGroups) {
        const uint32_t off = (ltile * pairs * 16u + (ob >> 1) * 16u + j) * 8u + (ob & 1u) * 4u;
#pragma unroll
        for (int q = 0; q < NW; ++q)
#pragma unroll
            for (int b = 0; b < P; ++b)
                sbl[q][b] = __builtin_amdgcn_raw_buffer_load_b32(lm[q].sb, off, (first + 2u * b) * 128u, kStreamPolicy);
    }
    // Two batches of weights in flight before the first arithmetic.
    Batch<P> ba[NW], bb[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) load_batch<P, !kLaneGroups>(lm[q], first, last, ba[q]);
#pragma unroll
    for (int q = 0; q < NW; ++q) load_batch<P, !kLaneGroups>(lm[q], first + P, last, bb[q]);

    if (stager) {
        if constexpr (NORM) {
            // Per-unit sums of squares, then one wave per row forms its inverse rms.
            for (uint32_t u = xu0; u < units; u += kThreads) {
                if (u != xu0) {
                    const uint32_t m = unit_row<M>(u, G);
                    const uint32_t g = u - m * G;
                    const uint4* src = reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(m) * k + g * 64u);
#pragma unroll
                    for (int t = 0; t < 8; ++t) xv[t] = src[t];
                }
                part[u] = unit_sumsq(xv);
            }
            raise_counter(ctr + 1, lane);
            wait_counter(ctr + 1, nstage);
            if (wave < static_cast<uint32_t>(M)) {
                const float ss = row_sumsq(part + wave * G, G, lane);
                if (lane == 0u) part[units + wave] = rms_inverse(ss, k, p.eps);
            }
            raise_counter(ctr + 2, lane);
            wait_counter(ctr + 2, nstage);
        }

        // Stage x: each thread permutes whole groups (8 words) and sums them.
        for (uint32_t u = xu0; u < units; u += kThreads) {
            const uint32_t m = unit_row<M>(u, G);
            const uint32_t g = u - m * G;
            if (u != xu0 || (NORM && units > kThreads)) {
                const uint4* src = reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(m) * k + g * 64u);
#pragma unroll
                for (int t = 0; t < 8; ++t) xv[t] = src[t];
            }
            if constexpr (NORM) normalize_unit(xv, part[units + m]);
            float s0 = 0.0f;
            float s1 = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                uint4 o;
                o.x = __builtin_amdgcn_perm(xv[t].z, xv[t].x, 0x05040100u);   // (x0, x4)
                o.y = __builtin_amdgcn_perm(xv[t].z, xv[t].x, 0x07060302u);   // (x1, x5)
                o.z = __builtin_amdgcn_perm(xv[t].w, xv[t].y, 0x05040100u);   // (x2, x6)
                o.w = __builtin_amdgcn_perm(xv[t].w, xv[t].y, 0x07060302u);   // (x3, x7)
                xs[m * WS + g * 8u + t] = o;
                s0 = dot2_bf16(xv[t].x, kOnePair, s0);
                s1 = dot2_bf16(xv[t].y, kOnePair, s1);
                s0 = dot2_bf16(xv[t].z, kOnePair, s0);
                s1 = dot2_bf16(xv[t].w, kOnePair, s1);
            }
            reinterpret_cast<float*>(sx)[g * 4u + m] = s0 + s1;
        }
        raise_counter(ctr, lane);
    }
    wait_counter(ctr, nstage);

    // Opaque VGPR values, so (w & mask) | bits selects v_and_or_b32 (see and_or).
    uint32_t mask = kNibbleMask;
    uint32_t bits = kMagic128;
    asm volatile("" : "+v"(mask), "+v"(bits));

    const uint32_t arow = min(j, static_cast<uint32_t>(M - 1));   // A row this lane supplies
    const uint4* xa = xs + arow * WS + kb * 2u;

    float y[NW][M];
#pragma unroll
    for (int q = 0; q < NW; ++q)
#pragma unroll
        for (int m = 0; m < M; ++m) y[q][m] = 0.0f;

    if constexpr (kLaneGroups) {
        // m <= 4 rows of x fill only A rows 0..m-1 (the rest repeat row m-1), so output
        // blocks 1..3 (rows 4..15) would carry no new sums. Instead A row block r holds the
        // m rows only in the MFMAs of group slot r of each two pairs (the other lanes read
        // the zero row), so output block r accumulates rows 0..m-1 of group
        // 2 (first + 2 b) + r alone, and each lane scales one group per two pairs: 2 + 4 m
        // VALU per lane where four per-group scalings take 4 (2 + 3 m).
        const uint32_t ablk = (lane & 15u) >> 2;   // A row block this lane supplies
        const uint32_t brow = min(lane & 3u, static_cast<uint32_t>(M - 1));   // its x row
        const uint4* src[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) src[r] = (ablk == static_cast<uint32_t>(r) ? xs + brow * WS : zs) + kb * 2u;
        const float4* sxl = sx + 2u * first + ob;
        const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
        f32x4_t acc0[NW], acc1[NW];
#pragma unroll
        for (int i = 0; i < 2 * P; ++i) {
            if (static_cast<uint32_t>(i) >= cnt) break;   // wave-uniform
            const uint32_t g0 = 2u * (first + i);
            const uint32_t g1 = min(g0 + 1u, G - 1u);   // an odd group count leaves the last pair half empty
            const uint4* pa = src[2 * (i & 1)];
            const uint4* pb = src[2 * (i & 1) + 1];
            const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, pa[g0 * 8u]);
            const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, pa[g0 * 8u + 1u]);
            const bf16x8_t a2 = __builtin_bit_cast(bf16x8_t, pb[g1 * 8u]);
            const bf16x8_t a3 = __builtin_bit_cast(bf16x8_t, pb[g1 * 8u + 1u]);
#pragma unroll
            for (int q = 0; q < NW; ++q) {
                bf16x8_t b[4];
                pair_frags<NW>(i < P ? ba[q].w[i % P] : bb[q].w[i % P], mask, bits, b);
                // The first pair of two starts fresh chains (a literal zero accumulator).
                acc0[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[0], (i & 1) == 0 ? zero : acc0[q], 0, 0, 0);
                acc1[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[2], (i & 1) == 0 ? zero : acc1[q], 0, 0, 0);
                acc0[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[1], acc0[q], 0, 0, 0);
                acc1[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, b[3], acc1[q], 0, 0, 0);
            }
            if ((i & 1) == 1 || static_cast<uint32_t>(i) + 1u >= cnt) {
                // Two pairs done: acc0 holds blocks 0 and 2 (zero rows elsewhere), acc1 1 and 3.
                const int bi = i >> 1;
                const uint32_t g = 2u * (first + 2u * bi) + ob;
                const bool valid = 2u * bi + (ob >> 1) < cnt && g < G;
                const float4 sx4 = sxl[bi * 4];
                const float sxv[4] = {sx4.x, sx4.y, sx4.z, sx4.w};
#pragma unroll
                for (int q = 0; q < NW; ++q) {
                    const float sc = bf16_bits_to_f32(sbl[q][bi] & 0xFFFFu);
                    const float bs = bf16_bits_to_f32(sbl[q][bi] >> 16);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float t = acc0[q][m] + acc1[q][m];
                        float yn = fmaf(sc, fmaf(-128.0f, sxv[m], t), y[q][m]);
                        yn = fmaf(bs, sxv[m], yn);
                        y[q][m] = valid ? yn : y[q][m];
                    }
                }
            }
        }
        // Blocks 0..3 hold the sums over disjoint groups: add lanes j, j + 16, j + 32, j + 48.
#pragma unroll
        for (int q = 0; q < NW; ++q)
#pragma unroll
            for (int m = 0; m < M; ++m) y[q][m] = sum_lane_blocks(y[q][m]);
    } else if constexpr (!LOOP) {
        // The whole range is in flight (cnt <= 2P): straight-line code, so each pair waits
        // only for its own loads (a loop waits for the loads of every iteration).
#pragma unroll
        for (int i = 0; i < 2 * P; ++i) {
            if (static_cast<uint32_t>(i) >= cnt) break;   // wave-uniform
            uint4 w[NW];
            uint2 sbw[NW];
#pragma unroll
            for (int q = 0; q < NW; ++q) {
                w[q] = i < P ? ba[q].w[i % P] : bb[q].w[i % P];
                sbw[q] = i < P ? ba[q].sb[i % P] : bb[q].sb[i % P];
            }
            compute_pair<M, NW>(w, sbw, first + i, G, xa, sx, mask, bits, y);
        }
    } else {
    // Ping-pong over two register batches: compute one, refill it two batches ahead.
    for (uint32_t base = 0; base < cnt; base += 2 * P) {
        compute_batch<M, NW, P>(ba, base, cnt, first, G, xa, sx, mask, bits, y);
        if (base + 2 * P < cnt) {
#pragma unroll
            for (int q = 0; q < NW; ++q) load_batch<P>(lm[q], first + base + 2 * P, last, ba[q]);
        }
        if (base + P >= cnt) break;
        compute_batch<M, NW, P>(bb, base + P, cnt, first, G, xa, sx, mask, bits, y);
        if (base + 3 * P < cnt) {
#pragma unroll
            for (int q = 0; q < NW; ++q) load_batch<P>(lm[q], first + base + 3 * P, last, bb[q]);
        }
    }
    }

    if (S > 1u) {
        if (kb == 0u) {
#pragma unroll
            for (int q = 0; q < NW; ++q)
#pragma unroll
                for (int m = 0; m < M; ++m) red[((wave * NW + q) * M + m) * kTileRows + j] = y[q][m];
        }
        __syncthreads();
        if (split == 0u) {
#pragma unroll
            for (int q = 0; q < NW; ++q)
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float v = y[q][m];
                    for (uint32_t s2 = 1; s2 < S; ++s2)
                        v += red[(((wave + s2) * NW + q) * M + m) * kTileRows + j];
                    y[q][m] = v;
                }
        }
    }

    const uint32_t out_row = tile * kTileRows + j;
    if (split == 0u && kb == 0u && out_row < seg_n) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float out = round_bf16(y[0][m]);
            if constexpr (DUAL) {
                const float up = round_bf16(y[NW - 1][m]);
                out = round_bf16(gelu_tanh_bf16_chain(out) * up);
            } else if constexpr (EPI == static_cast<int>(Epilogue::kSoftcap)) {
                out = softcap_bf16(out, p.cap);
            }
            seg_y[static_cast<size_t>(m) * seg_n + out_row] = f32_to_bf16_bits(out);
        }
    }
}

size_t skinny_lds_bytes(uint32_t m, uint32_t k, bool dual, uint32_t nwave, bool norm = false) {
    const size_t W = k / 8u;
    const size_t G = k / 64u;
    // Single-matrix kernels keep a zero row beside x (their straight-line form uses it).
    return (m + (dual ? 0u : 1u)) * (W + 1u) * 16u + G * 16u +
           static_cast<size_t>(nwave) * (dual ? 2u : 1u) * m * kTileRows * 4u + 16u + (norm ? (m * G + m) * 4u : 0u);
}

size_t max_lds_per_block();

template <int M, bool DUAL, int EPI, int NWAVE, bool NORM = false>
void launch_skinny_t(const SkinnyParams& p, uint32_t tiles_total, hipStream_t stream) {
    // Pairs per register batch (two batches in flight): 4, so that a wave's whole range
    // (at most kSkinnyPairsUpFront pairs) is requested at once; 2 for the fused gate/up,
    // which holds two matrices' batches, and for the softcap head, whose waves loop.
    constexpr int P = (DUAL || EPI != 0) ? 2 : 4;
    const uint32_t per_wave = (p.pairs + p.splits - 1u) / p.splits;
    auto kernel = per_wave <= 2u * P ? q4_skinny_kernel<M, DUAL, EPI, P, NWAVE, NORM, false>
                                     : q4_skinny_kernel<M, DUAL, EPI, P, NWAVE, NORM, true>;
    const size_t lds = skinny_lds_bytes(M, p.k, DUAL, NWAVE, NORM);
    HYP_REQUIRE(lds <= max_lds_per_block(), HYP_STATUS_INTERNAL, "skinny: x staging exceeds the device's LDS");
    if (lds > 65536u) {
        static thread_local int configured_device = -1;
        int dev = 0;
        HYP_HIP_CHECK(hipGetDevice(&dev));
        if (configured_device != dev) {
            for (const void* f : {reinterpret_cast<const void*>(q4_skinny_kernel<M, DUAL, EPI, P, NWAVE, NORM, false>),
                                  reinterpret_cast<const void*>(q4_skinny_kernel<M, DUAL, EPI, P, NWAVE, NORM, true>)}) {
                HYP_HIP_CHECK(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  static_cast<int>(max_lds_per_block())));
            }
            configured_device = dev;
        }
    }
    const uint32_t tiles_per_block = NWAVE / p.splits;
    const dim3 grid((tiles_total + tiles_per_block - 1u) / tiles_per_block);
    hipLaunchKernelGGL(kernel, grid, dim3(64 * NWAVE), lds, stream, p);
}

// Workgroups of 16 waves (16 / splits row tiles each), so that one workgroup per compute
// unit stages x once; the fused gate/up uses 8 (its registers) unless 16 waves share a
// tile, and the softcap head, whose grid is many workgroups per compute unit, 4.
template <int M>
void launch_skinny_m(const SkinnyParams& p, uint32_t tiles_total, bool dual, Epilogue epi, bool norm,
                     hipStream_t stream) {
    if (dual) {
        if (p.splits > static_cast<uint32_t>(kSkinnyDualWaves)) {
            launch_skinny_t<M, true, 0, kSkinnyWaves>(p, tiles_total, stream);
        } else {
            launch_skinny_t<M, true, 0, kSkinnyDualWaves>(p, tiles_total, stream);
        }
    } else if (epi == Epilogue::kSoftcap) {
        launch_skinny_t<M, false, 1, 4>(p, tiles_total, stream);
    } else if (norm) {
        launch_skinny_t<M, false, 0, kSkinnyWaves, true>(p, tiles_total, stream);
    } else {
        launch_skinny_t<M, false, 0, kSkinnyWaves>(p, tiles_total, stream);
    }
}

void launch_skinny(SkinnyParams& p, uint32_t tiles_total, uint32_t m, bool dual, Epilogue epi, bool norm,
                   hipStream_t stream) {
    switch (m) {
        case 1: launch_skinny_m<1>(p, tiles_total, dual, epi, norm, stream); break;
        case 2: launch_skinny_m<2>(p, tiles_total, dual, epi, norm, stream); break;
        case 3: launch_skinny_m<3>(p, tiles_total, dual, epi, norm, stream); break;
        case 4: launch_skinny_m<4>(p, tiles_total, dual, epi, norm, stream); break;
        default: throw NativeError(HYP_STATUS_INTERNAL, "skinny launched with m outside 1..4");
    }
    HYP_HIP_CHECK(hipGetLastError());
}

size_t max_lds_per_block() {
    static thread_local int cached_device = -1;
    static thread_local size_t cached = 0;
    int dev = 0;
    HYP_HIP_CHECK(hipGetDevice(&dev));
    if (dev != cached_device) {
        int v = 0;
        HYP_HIP_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
        cached = static_cast<size_t>(v);
        cached_device = dev;
    }
    return cached;
}

}  // namespace

uint32_t choose_skinny_splits(uint32_t tiles, uint32_t pairs, uint32_t m, SkinnyForm form) {
    // Measured on the decode shapes of a 12B layer (MI355X, cold weights, every split):
    //  * plain and grouped launches (16-wave workgroups, S waves share a 16-row tile): the
    //    smallest power of two that leaves every wave at most kSkinnyPairsUpFront pairs
    //    (all its loads issued at once), doubled while the grid is short of one workgroup
    //    per compute unit, up to 16: [15360,3840] 4; q/k/v grouped 8; o, q, k, down 16;
    //    at m = 4 o and q measured 8 and 16 within 0.4 us of each other, either way round
    //    on different boxes;
    //  * the softcap head (262144 rows, 4-wave workgroups, many per compute unit): 1
    //    (95 vs 100 us at m = 1, 111 vs 123 us at m = 4 with 2);
    //  * the fused gate/up (two matrices, 2-pair batches): at m = 1 the smallest split that
    //    keeps every wave's range in its two batches ([15360,3840]: 8, 14.5 us against
    //    16.8 us at 4); at m >= 2, 2 (17.7 us against 24.2 us at 4 for m = 4).
    const uint32_t cus = device_compute_units();
    uint32_t s = 1u;
    if (form == SkinnyForm::kHead) {
        s = 1u;
    } else if (form == SkinnyForm::kDual) {
        if (m == 1u) {
            while (s < 16u && pairs > s * (kSkinnyPairsUpFront / 2u)) s *= 2u;
        } else {
            s = 2u;
        }
    } else {
        while (s < 16u && pairs > s * kSkinnyPairsUpFront) s *= 2u;
        while (s < 16u && tiles * s < static_cast<uint32_t>(kSkinnyWaves) * cus * 9u / 10u && pairs >= 2u * s) s *= 2u;
    }
    while (s > 1u && pairs < s) s /= 2u;
    return s;
}

bool skinny_supported(uint32_t m, uint32_t k, bool dual) {
    return m >= 1u && m <= kSkinnyMaxM && k % 64u == 0u && k > 0u &&
           skinny_lds_bytes(m, k, dual, kSkinnyWaves) <= max_lds_per_block();
}

bool skinny_norm_supported(uint32_t m, uint32_t k) {
    return m >= 1u && m <= kSkinnyMaxM && k % 64u == 0u && k > 0u &&
           skinny_lds_bytes(m, k, false, kSkinnyWaves, true) <= max_lds_per_block();
}

void launch_q4_skinny(const Q4Matrix& w, const Q4Matrix* up, const uint16_t* x, uint32_t m, uint16_t* y,
                      Epilogue epi, float cap_bf16, uint32_t splits, hipStream_t stream) {
    const TiledDims d = TiledDims::of(w.n, w.k);
    const bool dual = up != nullptr;
    HYP_REQUIRE(w.codes != nullptr && w.sb != nullptr && (!dual || (up->codes != nullptr && up->sb != nullptr)),
                HYP_STATUS_INTERNAL, "skinny: weights are not in the tiled resident layout");
    HYP_REQUIRE(!dual || (up->n == w.n && up->k == w.k), HYP_STATUS_INTERNAL, "skinny: gate and up differ in shape");
    HYP_REQUIRE(skinny_supported(m, w.k, dual), HYP_STATUS_INTERNAL, "skinny: shape exceeds LDS");
    HYP_REQUIRE(d.code_bytes() < (1ull << 31), HYP_STATUS_INTERNAL, "skinny: matrix exceeds 2 GiB of packed codes");
    const bool head = epi == Epilogue::kSoftcap;
    if (splits == 0u) {
        splits = choose_skinny_splits(d.tiles, d.pairs, m,
                                      head ? SkinnyForm::kHead : (dual ? SkinnyForm::kDual : SkinnyForm::kPlain));
    }
    HYP_REQUIRE(splits == 1u || splits == 2u || splits == 4u || (!head && (splits == 8u || splits == 16u)),
                HYP_STATUS_INTERNAL, "skinny: bad split count");
    HYP_REQUIRE(d.pairs >= splits, HYP_STATUS_INTERNAL, "skinny: fewer group pairs than splits");
    SkinnyParams p{};
    p.seg[0] = SkinnySegment{w.codes, w.sb, y, w.n, 0u};
    p.nseg = 1u;
    p.codes2 = dual ? up->codes : nullptr;
    p.sb2 = dual ? up->sb : nullptr;
    p.x = x;
    p.k = w.k;
    p.pairs = d.pairs;
    p.cap = cap_bf16;
    p.splits = splits;
    p.split_shift = static_cast<uint32_t>(__builtin_ctz(splits));
    launch_skinny(p, d.tiles, m, dual, epi, false, stream);
}

void launch_q4_skinny_group(const Q4Matrix* const* ws, uint16_t* const* ys, uint32_t count, const uint16_t* x,
                            uint32_t m, const float* rms_eps, hipStream_t stream) {
    HYP_REQUIRE(count >= 1u && count <= kSkinnyMaxGroup, HYP_STATUS_INTERNAL, "skinny: bad group size");
    const uint32_t k = ws[0]->k;
    const bool norm = rms_eps != nullptr;
    HYP_REQUIRE(norm ? skinny_norm_supported(m, k) : skinny_supported(m, k, false), HYP_STATUS_INTERNAL,
                "skinny: shape exceeds LDS");
    SkinnyParams p{};
    uint32_t tiles_total = 0u;
    for (uint32_t i = 0; i < count; ++i) {
        const Q4Matrix& w = *ws[i];
        HYP_REQUIRE(w.k == k, HYP_STATUS_INTERNAL, "skinny: grouped projections differ in k");
        HYP_REQUIRE(w.codes != nullptr && w.sb != nullptr, HYP_STATUS_INTERNAL,
                    "skinny: weights are not in the tiled resident layout");
        const TiledDims d = TiledDims::of(w.n, w.k);
        HYP_REQUIRE(d.code_bytes() < (1ull << 31), HYP_STATUS_INTERNAL,
                    "skinny: matrix exceeds 2 GiB of packed codes");
        p.seg[i] = SkinnySegment{w.codes, w.sb, ys[i], w.n, tiles_total};
        tiles_total += d.tiles;
    }
    p.nseg = count;
    p.x = x;
    p.k = k;
    p.pairs = TiledDims::of(16u, k).pairs;
    p.cap = 0.0f;
    p.eps = norm ? *rms_eps : 0.0f;
    p.splits = choose_skinny_splits(tiles_total, p.pairs, m, SkinnyForm::kPlain);
    p.split_shift = static_cast<uint32_t>(__builtin_ctz(p.splits));
    launch_skinny(p, tiles_total, m, false, Epilogue::kNone, norm, stream);
}

}  // namespace hyperion::hip

// Device building blocks of the skinny (decode, m <= 4) quantized matmul on gfx950 MFMA,
// shared by the per-call kernel (q4_gemv_mfma.hip) and the persistent step-program kernel
// (q4_step_program.hip), so both run the same arithmetic and give the same bits. The
// scheme is described at the top of q4_gemv_mfma.hip.
#pragma once

#include "common.h"
#include "kernels.h"
#include "q4_layout.h"

namespace hyperion::hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kMaxSegments = 3;   // projections sharing x in one grouped launch
constexpr int kSkinnyWaves = 16;        // waves per workgroup (the softcap head uses 4)
constexpr int kSkinnyDualWaves = 8;     // the fused gate/up: two workgroups per compute unit
constexpr uint32_t kSkinnyPairsUpFront = 8;   // two batches of 4 pairs: a wave's whole range at once

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

// s_waitcnt operand for vmcnt(n) with the other counters left at their maxima (gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt in 6:4, lgkmcnt in 11:8).
constexpr uint32_t waitcnt_vm(uint32_t n) { return (n & 15u) | ((n >> 4) << 14) | 0x70u | 0xF00u; }

// Bytes of LDS that copy_to_lds fills for `bytes` of source: whole KiB.
constexpr uint32_t lds_copy_bytes(uint32_t bytes) { return (bytes + 1023u) / 1024u * 1024u; }

// One wave copies [src, src + bytes) into LDS at dst with direct buffer-to-LDS loads, no
// registers: load t moves bytes [1024 t, 1024 t + 1024), lane l its 16 bytes at
// 1024 t + 16 l; bytes past `bytes` read as zeros (the buffer's bound) into the rest of
// lds_copy_bytes(bytes). The loads count in vmcnt in issue order: the data is in LDS once
// the count has drained past them.
__device__ __forceinline__ void copy_to_lds(const void* src, uint32_t bytes, void* dst, uint32_t lane) {
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(src, bytes);
    for (uint32_t t = 0; t * 1024u < bytes; ++t) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r, (__attribute__((address_space(3))) void*)(static_cast<uint8_t*>(dst) + t * 1024u), 16,
            static_cast<int>(lane * 16u), static_cast<int>(t * 1024u), 0, 0);
    }
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
    const uint16_t* norm_w;   // NORM: the norm's learned weight [k] (bf16), or null
    // NORM with a residual (the sandwich closing the previous block, forward.cc:518-539):
    // the rows normalised are x = bf16(res_in + rms_norm(res_branch, res_w)), times
    // res_scalar (bf16 [1]) when non-null, with the same bits as residual_norm_kernel;
    // workgroup 0 writes them to res_out (not res_in, which the other workgroups still read).
    const uint16_t* res_branch;
    const uint16_t* res_in;
    uint16_t* res_out;
    const uint16_t* res_w;
    const uint16_t* res_scalar;
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

// The lane-group form: one matrix, the wave's whole range in flight (cnt <= 2P). m <= 4
// rows of x fill only A rows 0..m-1 (the rest repeat row m-1), so output blocks 1..3
// (rows 4..15) would carry no new sums. Instead A row block r holds the m rows only in
// the MFMAs of group slot r of each two pairs (the other lanes read the zero row zs), so
// output block r accumulates rows 0..m-1 of group 2 (first + 2 b) + r alone, and each lane
// scales one group per two pairs (its scale and bias word sbl[q][b]): 2 + 4 m VALU per lane
// where four per-group scalings take 4 (2 + 3 m). xs: x rows in LDS, WS chunks apart.
template <int M, int NW, int P>
__device__ __forceinline__ void compute_lane_groups(const Batch<P> (&ba)[NW], const Batch<P> (&bb)[NW],
                                                    const uint32_t (&sbl)[NW][P], uint32_t first, uint32_t cnt,
                                                    uint32_t G, const uint4* xs, const uint4* zs, uint32_t WS,
                                                    const float4* sx, uint32_t lane, uint32_t mask, uint32_t bits,
                                                    float (&y)[NW][M]) {
    const uint32_t kb = lane >> 4;
    const uint32_t ob = lane >> 4;
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
}

// The whole range is in flight (cnt <= 2P): straight-line code, so each pair waits only
// for its own loads (a loop waits for the loads of every iteration). xa: this lane's A row.
template <int M, int NW, int P>
__device__ __forceinline__ void compute_straight(const Batch<P> (&ba)[NW], const Batch<P> (&bb)[NW], uint32_t first,
                                                 uint32_t cnt, uint32_t G, const uint4* xa, const float4* sx,
                                                 uint32_t mask, uint32_t bits, float (&y)[NW][M]) {
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
}

// Ranges longer than two batches: ping-pong over the two register batches, computing one
// and refilling it two batches ahead.
template <int M, int NW, int P>
__device__ __forceinline__ void compute_loop(Batch<P> (&ba)[NW], Batch<P> (&bb)[NW], const LaneMatrix (&lm)[NW],
                                             uint32_t first, uint32_t last, uint32_t cnt, uint32_t G,
                                             const uint4* xa, const float4* sx, uint32_t mask, uint32_t bits,
                                             float (&y)[NW][M]) {
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

// The S waves sharing a tile meet in LDS (red: [waves][NW][M][16] floats): waves of split
// s > 0 publish their sums, and split 0 adds them in split order. Contains a workgroup
// barrier, so every wave of the workgroup must call it.
template <int M, int NW>
__device__ __forceinline__ void reduce_splits(float (&y)[NW][M], float* red, uint32_t wave, uint32_t split,
                                              uint32_t S, uint32_t kb, uint32_t j) {
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
}

// Output m of a lane's row: bf16 of the sum, then the softcap (EPI), each op rounded to
// bf16 as the reference does.
template <int EPI, int M, int NW>
__device__ __forceinline__ float output_value(const float (&y)[NW][M], int m, float cap) {
    float out = round_bf16(y[0][m]);
    if constexpr (EPI == static_cast<int>(Epilogue::kSoftcap)) out = softcap_bf16(out, cap);
    return out;
}

// The fused MLP gating of one output: bf16(gelu_tanh(bf16(gate)) * up), up already bf16
// (ForwardPass::mlp, forward.cc:338-343, with the op-by-op GELU chain of forward.cc:324-336).
__device__ __forceinline__ float gate_up_value(float gate_sum, float up_bf16) {
    return round_bf16(gelu_tanh_bf16_chain(round_bf16(gate_sum)) * up_bf16);
}

}  // namespace
}  // namespace hyperion::hip

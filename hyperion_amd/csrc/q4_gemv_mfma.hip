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
//    it, then each wave issues its weights (all of them when they fit in two register
//    batches). In 16-wave workgroups a raw barrier (no memory wait) puts every weight load
//    of the workgroup behind the x requests and the staging waves publish x through an LDS
//    counter that the others poll; in smaller workgroups no wave waits before issuing its
//    weights, and x is published by a barrier the staging waves reach once it is staged.
#include "common.h"
#include "kernels.h"
#include "q4_layout.h"
#include "q4_rmsnorm.h"
#include "q4_skinny_core.h"

#include <algorithm>

namespace hyperion::hip {
namespace {

// Lanes per 64-value unit in the normalising prologue's spread form.
constexpr int kSpreadLanes = 4;

// scan_sumsq over a lane's chunks (words in order).
template <int CH>
__device__ __forceinline__ float scan_sumsq_chunks(const uint4 (&v)[8 / CH], uint32_t sl) {
    uint32_t w[32 / CH];
#pragma unroll
    for (int t = 0; t < 8 / CH; ++t) {
        w[4 * t] = v[t].x;
        w[4 * t + 1] = v[t].y;
        w[4 * t + 2] = v[t].z;
        w[4 * t + 3] = v[t].w;
    }
    return scan_sumsq<CH>(w, sl);
}

// A chunk of x (8 values) in the A operand's slot order: (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ __forceinline__ uint4 permute_chunk(const uint4& c) {
    uint4 o;
    o.x = __builtin_amdgcn_perm(c.z, c.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(c.z, c.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(c.w, c.y, 0x05040100u);
    o.w = __builtin_amdgcn_perm(c.w, c.y, 0x07060302u);
    return o;
}

// The group sum of x of a unit spread over CH lanes (lane sl holding chunks 8 / CH * sl ..):
// the staging's two dot2 chains (words x, z of each chunk into s0, y, w into s1, chunks in
// order) handed from lane to lane by DPP moves, as scan_sumsq hands its chain; s0 and s1
// are complete on lane sl = CH - 1.
template <int CH>
__device__ __forceinline__ void scan_group_sums(const uint4 (&xc)[8 / CH], uint32_t sl, float& s0, float& s1) {
    float in0 = 0.0f;
    float in1 = 0.0f;
#pragma unroll
    for (int s = 0; s < CH; ++s) {
        s0 = in0;
        s1 = in1;
#pragma unroll
        for (int t = 0; t < 8 / CH; ++t) {
            s0 = dot2_bf16(xc[t].x, kOnePair, s0);
            s1 = dot2_bf16(xc[t].y, kOnePair, s1);
            s0 = dot2_bf16(xc[t].z, kOnePair, s0);
            s1 = dot2_bf16(xc[t].w, kOnePair, s1);
        }
        if (s + 1 < CH) {
            const float p0 = dpp_mov<0x111>(s0);   // row_shr 1: lane i - 1
            const float p1 = dpp_mov<0x111>(s1);
            in0 = sl == 0u ? 0.0f : p0;
            in1 = sl == 0u ? 0.0f : p1;
        }
    }
}

// NORM 1: x rows are first rms-normalised (q4_rmsnorm.h) in LDS; the matmul then runs on
// the normalised rows, which are not written back.
// NORM 2: the sandwich close of the previous block first: x = in + rms(branch) * res_w
// (times res_scalar when given), in residual_norm_kernel's arithmetic, recomputed by every
// workgroup from the same inputs; workgroup 0 writes x to res_out, and the matmul runs on
// rms(x) as with NORM 1. ctr[3..5] order the branch's statistics.
//
// Staging: thread u < M * G owns the 64-element unit (row u / G, group u % G) while
// M * G <= threads; the staging waves are the waves holding units (at least M of them
// with NORM, which forms one row's inverse rms per wave). LDS counters: ctr[0] counts
// staging waves done with x, ctr[1] staging waves done with the NORM partials.
// LOOP: a wave's range may exceed two batches (refilled in a loop); otherwise it fits.
// DUAL (the fused gate/up): the launch's 16-row tiles alternate gate, up, gate, up, ...
// (virtual tile 2t is gate tile t, 2t + 1 up tile t), so both halves of a row tile are
// in one workgroup; each wave computes one matrix exactly as a plain launch does, and the
// gate tile's waves combine with the up tile's rows in LDS for the GELU epilogue.
// The 8-wave residual form is held to 128 VGPRs (four waves per SIMD): its grids run two
// workgroups on some compute units (the 12B's global q/k: 272 workgroups), and at more
// registers the second would wait for the first (13.4 against 17.0 us at 134 VGPRs).
template <int M, bool DUAL, int EPI, int P, int NWAVE, int NORM, bool LOOP, int CH>
__global__ __launch_bounds__(64 * NWAVE, NWAVE == 8 && NORM == 2 ? 4 : 1) void q4_skinny_kernel(SkinnyParams p) {
    constexpr int NW = 1;
    constexpr uint32_t kThreads = 64u * NWAVE;
    extern __shared__ __attribute__((aligned(16))) uint4 smem[];

    const uint32_t k = p.k;
    const uint32_t W = k / 8u;    // packed words per row
    const uint32_t G = k / 64u;   // groups per row
    // x rows in LDS are W + 1 chunks apart: W is a multiple of 16 chunks (256 bytes, all 64
    // banks), so unpadded the m rows an A read touches would all start on the same bank.
    const uint32_t WS = W + 1u;
    // Whole range in flight: lane blocks take one group each (compute_lane_groups).
    constexpr bool kLaneGroups = !LOOP;
    // NORM: the norm's weight (and with a residual the branch norm's weight) copied into LDS
    // whole, KW chunks each.
    const uint32_t KW = NORM ? lds_copy_bytes(2u * k) / 16u : 0u;
    uint4* xs = smem;                                              // [M][WS] permuted x
    uint4* zs = smem + M * WS;                                     // [WS] zeros
    uint4* nwl = zs + WS;                                          // NORM: [KW] norm weight
    uint4* rwl = nwl + KW;                                         // NORM 2: [KW] branch norm weight
    float4* sx = reinterpret_cast<float4*>(rwl + (NORM == 2 ? KW : 0u));   // [G] group sums of x rows 0..3
    float* red = reinterpret_cast<float*>(sx + G);                 // [NWAVE][M][16]
    uint32_t* ctr = reinterpret_cast<uint32_t*>(red + NWAVE * M * kTileRows);   // [8]
    float* part = reinterpret_cast<float*>(ctr + 8);               // NORM: [M][G] unit partials, [M] inverses
    float* comb = part + (NORM ? M * G + M : 0u);                  // DUAL: [NWAVE / 2][M][16] up rows

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
    if constexpr (DUAL) {
        tile = gtile >> 1;
        if (gtile & 1u) {
            seg_codes = p.codes2;
            seg_sb = p.sb2;
        }
    } else if (p.nseg > 1u) {
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
    const uint32_t nstage = max((min(units * CH, kThreads) + 63u) / 64u, NORM ? static_cast<uint32_t>(M) : 1u);
    const bool stager = wave < nstage;

    // x first: thread u's unit is requested before its wave's weight loads (with the early
    // barrier below, before every weight load of the workgroup). With a residual (NORM 2)
    // the branch and residual units are requested there instead, and the staging waves run
    // the whole prologue before issuing their weight loads, so that those units are never
    // live beside two weight batches (the registers of both would halve the waves per
    // SIMD). The norms' weights (and the layer scalar) are requested there too, by wave 0
    // straight into LDS: behind the weight loads each would cost the prologue a round trip
    // through the compute unit's queue of weight requests.
    const uint32_t xu0 = threadIdx.x;   // first (row, group) unit this thread stages
    constexpr bool resid = NORM == 2;
    uint4 xv[8];
    uint4 rv[8];
    uint16_t res_sc = 0u;   // NORM 2: the layer scalar (bf16)
    // CH > 1 (the normalising forms when CH units' lanes fit the workgroup): unit su = thread
    // / CH is spread over CH lanes, lane sl = thread % CH holding its values [64 / CH * sl,
    // 64 / CH * (sl + 1)) as kCC 16-byte chunks (xc, and the residual's in rc).
    constexpr uint32_t kCC = 8u / CH;
    const uint32_t su = threadIdx.x / CH;
    const uint32_t sl = threadIdx.x % CH;
    const bool sown = su < units;
    uint4 xc[kCC];
    uint4 rc[kCC];
    if constexpr (CH > 1) {
#pragma unroll
        for (uint32_t t = 0; t < kCC; ++t) xc[t] = rc[t] = make_uint4(0u, 0u, 0u, 0u);
        if (sown) {
            const uint32_t m = unit_row<M>(su, G);
            const size_t off = static_cast<size_t>(m) * k + (su - m * G) * 64u + sl * (64u / CH);
            if constexpr (!resid) {
                const uint4* src = reinterpret_cast<const uint4*>(p.x + off);
#pragma unroll
                for (uint32_t t = 0; t < kCC; ++t) xc[t] = src[t];
            } else {
                const uint4* bsrc = reinterpret_cast<const uint4*>(p.res_branch + off);
                const uint4* rsrc = reinterpret_cast<const uint4*>(p.res_in + off);
#pragma unroll
                for (uint32_t t = 0; t < kCC; ++t) xc[t] = bsrc[t];
#pragma unroll
                for (uint32_t t = 0; t < kCC; ++t) rc[t] = rsrc[t];
            }
        }
    } else if constexpr (!resid) {
        if (xu0 < units) {
            const uint32_t m = unit_row<M>(xu0, G);
            const uint32_t g = xu0 - m * G;
            const uint4* src = reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(m) * k + g * 64u);
#pragma unroll
            for (int t = 0; t < 8; ++t) xv[t] = src[t];
        }
    } else if (stager) {
        if (xu0 < units) {   // the branch first: its statistics need only it
            const uint32_t m = unit_row<M>(xu0, G);
            const uint32_t g = xu0 - m * G;
            const size_t off = static_cast<size_t>(m) * k + g * 64u;
            const uint4* bsrc = reinterpret_cast<const uint4*>(p.res_branch + off);
            const uint4* rsrc = reinterpret_cast<const uint4*>(p.res_in + off);
#pragma unroll
            for (int t = 0; t < 8; ++t) xv[t] = bsrc[t];
#pragma unroll
            for (int t = 0; t < 8; ++t) rv[t] = rsrc[t];
        }
    }
    if constexpr (resid) {
        // By every thread, from a valid address either way (the value is used only with a
        // scalar): outside any branch, nothing consumes it before it is needed.
        res_sc = *(p.res_scalar != nullptr ? p.res_scalar : p.res_w);
    }
    if (threadIdx.x < 8u) ctr[threadIdx.x] = 0u;
    if constexpr (kLaneGroups)
        for (uint32_t t = threadIdx.x; t < WS; t += kThreads) zs[t] = uint4{0u, 0u, 0u, 0u};
    // Two ways to publish x. 16-wave workgroups (one per compute unit) and the normalising
    // forms: a raw barrier (no memory wait) right after the x requests puts every weight load
    // of the workgroup behind them and orders the clearing of the LDS counters, through which
    // the staging waves then publish x (and the rms statistics) without blocking the others.
    // Smaller workgroups: no barrier before the weight loads; the staging waves publish x by
    // arriving at a barrier after staging it, the other waves once their loads are issued.
    // Measured (cold weights, one process): [15360,3840] in 8-wave workgroups 7.69 against
    // 7.95 us, o [3840,4096] in 4-wave workgroups 4.30 against 4.63 us, the fused gate/up
    // 13.74 against 14.39 us; in 16-wave workgroups the early barrier, 8.17 against 8.65 us
    // (the late barrier waits for the last of 16 waves to issue its loads).
    constexpr bool kEarly = NORM != 0 || NWAVE >= 16;
    if constexpr (NORM) {
        // After the LDS clearing above, which would otherwise have to wait for these writes.
        if (wave == 0u) {
            if (p.norm_w != nullptr) copy_to_lds(p.norm_w, 2u * k, nwl, lane);
            if constexpr (resid) copy_to_lds(p.res_w, 2u * k, rwl, lane);
        }
    }
    if constexpr (kEarly) {
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the counters are cleared
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");        // no load of the weights above the barrier
    }
    // Vector-memory instructions a staging wave issues after the barrier before it reads the
    // LDS copies: the scale-and-bias loads and two batches (with lane groups), two batches of
    // codes and scales otherwise; none with a residual.
    constexpr uint32_t kAfterCopy = resid ? 0u : (kLaneGroups ? 3u * P : 4u * P);

    const uint32_t c_bytes = tiles * pairs * 1024u;
    const uint32_t s_bytes = tiles * pairs * 128u;
    LaneMatrix lm[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) {
        lm[q].codes = buffer_rsrc(seg_codes, c_bytes);
        lm[q].sb = buffer_rsrc(seg_sb, s_bytes);
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
    Batch<P> ba[NW], bb[NW];
    if constexpr (!resid) {
        if constexpr (kLaneGroups) {
            const uint32_t off = (ltile * pairs * 16u + (ob >> 1) * 16u + j) * 8u + (ob & 1u) * 4u;
#pragma unroll
            for (int q = 0; q < NW; ++q)
#pragma unroll
                for (int b = 0; b < P; ++b)
                    sbl[q][b] = __builtin_amdgcn_raw_buffer_load_b32(lm[q].sb, off, (first + 2u * b) * 128u, kStreamPolicy);
        }
        // Two batches of weights in flight before the first arithmetic.
#pragma unroll
        for (int q = 0; q < NW; ++q) load_batch<P, !kLaneGroups>(lm[q], first, last, ba[q]);
#pragma unroll
        for (int q = 0; q < NW; ++q) load_batch<P, !kLaneGroups>(lm[q], first + P, last, bb[q]);
    }

    if constexpr (CH > 1) {
        if (stager) {
            // The prologue of the spread form: the unit-per-thread form's operations per value and
            // its sums in the same order (scan_sumsq, scan_group_sums), so the same bits.
            const uint32_t m = unit_row<M>(min(su, units - 1u), G);
            const uint32_t c0 = (su - m * G) * 8u + sl * kCC;   // this lane's first chunk in x's row
            if constexpr (resid) {
                const float tb = scan_sumsq_chunks<CH>(xc, sl);
                if (sown && sl == CH - 1u) part[su] = tb;
                if (wave == 0u) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kAfterCopy));
                raise_counter(ctr + 3, lane);
                wait_counter(ctr + 3, nstage);
                if (wave < static_cast<uint32_t>(M)) {
                    const float ss = row_sumsq(part + wave * G, G, lane);
                    if (lane == 0u) part[units + wave] = rms_inverse(ss, k, p.eps);
                }
                raise_counter(ctr + 4, lane);
                wait_counter(ctr + 4, nstage);
                if (sown) {
                    const float inv = part[units + m];
                    const float sc = bf16_bits_to_f32(res_sc);
    #pragma unroll
                    for (uint32_t t = 0; t < kCC; ++t) {
                        normalize_chunk(xc[t], inv);
                        weight_chunk(xc[t], rwl[c0 + t]);
                        residual_add_chunk(xc[t], rc[t], p.res_scalar != nullptr, sc);
                    }
                    if (blockIdx.x == 0u) {
                        uint4* dst = reinterpret_cast<uint4*>(p.res_out + static_cast<size_t>(m) * k) + c0;
    #pragma unroll
                        for (uint32_t t = 0; t < kCC; ++t) dst[t] = xc[t];
                    }
                }
                const float tx = scan_sumsq_chunks<CH>(xc, sl);
                raise_counter(ctr + 5, lane);   // every wave has read its inverse
                wait_counter(ctr + 5, nstage);
                if (sown && sl == CH - 1u) part[su] = tx;
            } else {
                const float t = scan_sumsq_chunks<CH>(xc, sl);
                if (sown && sl == CH - 1u) part[su] = t;
                if (wave == 0u) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kAfterCopy));
            }
            raise_counter(ctr + 1, lane);
            wait_counter(ctr + 1, nstage);
            if (wave < static_cast<uint32_t>(M)) {
                const float ss = row_sumsq(part + wave * G, G, lane);
                if (lane == 0u) part[units + wave] = rms_inverse(ss, k, p.eps);
            }
            raise_counter(ctr + 2, lane);
            wait_counter(ctr + 2, nstage);
            if (sown) {
                const float inv = part[units + m];
    #pragma unroll
                for (uint32_t t = 0; t < kCC; ++t) {
                    normalize_chunk(xc[t], inv);
                    if (p.norm_w != nullptr) weight_chunk(xc[t], nwl[c0 + t]);
                    xs[m * WS + c0 + t] = permute_chunk(xc[t]);
                }
            }
            float s0, s1;
            scan_group_sums<CH>(xc, sl, s0, s1);
            if (sown && sl == CH - 1u) reinterpret_cast<float*>(sx)[(su - m * G) * 4u + m] = s0 + s1;
            raise_counter(ctr, lane);   // kEarly: every normalising form
        }
    } else if (stager) {
        if constexpr (NORM) {
            if constexpr (resid) {
                // The branch's norm (phases 3, 4), the residual add, then x's statistics
                // below; each row's inverse is formed by one wave, in residual_norm_kernel's
                // order. Every unit is held by one thread (checked on the host).
                if (xu0 < units) part[xu0] = unit_sumsq(xv);
                // Wave 0's copies are in LDS (it has issued no other loads since).
                if (wave == 0u) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kAfterCopy));
                raise_counter(ctr + 3, lane);
                wait_counter(ctr + 3, nstage);
                if (wave < static_cast<uint32_t>(M)) {
                    const float ss = row_sumsq(part + wave * G, G, lane);
                    if (lane == 0u) part[units + wave] = rms_inverse(ss, k, p.eps);
                }
                raise_counter(ctr + 4, lane);
                wait_counter(ctr + 4, nstage);
                float ssx = 0.0f;
                if (xu0 < units) {
                    const uint32_t m = unit_row<M>(xu0, G);
                    const uint32_t g = xu0 - m * G;
                    uint4 wrv[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) wrv[t] = rwl[g * 8u + t];
                    normalize_unit(xv, part[units + m]);
                    weight_unit(xv, wrv);
                    const float sc = bf16_bits_to_f32(res_sc);
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        residual_add_chunk(xv[t], rv[t], p.res_scalar != nullptr, sc);
                    }
                    if (blockIdx.x == 0u) {
                        uint4* dst = reinterpret_cast<uint4*>(p.res_out + static_cast<size_t>(m) * k + g * 64u);
#pragma unroll
                        for (int t = 0; t < 8; ++t) dst[t] = xv[t];
                    }
                    ssx = unit_sumsq(xv);
                }
                raise_counter(ctr + 5, lane);   // every wave has read its inverse
                wait_counter(ctr + 5, nstage);
                if (xu0 < units) part[xu0] = ssx;
            } else {
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
            // Wave 0's copy is in LDS once no more than the loads issued after it are pending.
            if (wave == 0u) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kAfterCopy));
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

        // Stage x: each thread permutes whole groups (8 words) and sums them. The 16-wave
        // normalising form scales one 16-byte chunk at a time (the same operations per value):
        // with the whole unit's weights in registers beside x and two weight batches it spilled
        // (123 VGPRs chunk by chunk), while the 8-wave form measured faster unit by unit
        // (7.3-7.5 against 7.9 us on the 12B's q/k/v).
        constexpr bool kChunked = NORM == 1 && NWAVE >= 16;
        for (uint32_t u = xu0; u < units; u += kThreads) {
            const uint32_t m = unit_row<M>(u, G);
            const uint32_t g = u - m * G;
            if (u != xu0 || (NORM && units > kThreads)) {   // never with a residual
                const uint4* src = reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(m) * k + g * 64u);
#pragma unroll
                for (int t = 0; t < 8; ++t) xv[t] = src[t];
            }
            if constexpr (NORM && !kChunked) {
                normalize_unit(xv, part[units + m]);
                if (p.norm_w != nullptr) {
                    uint4 wv[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) wv[t] = nwl[g * 8u + t];
                    weight_unit(xv, wv);
                }
            }
            float s0 = 0.0f;
            float s1 = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                uint4 c = xv[t];
                if constexpr (kChunked) {
                    normalize_chunk(c, part[units + m]);
                    if (p.norm_w != nullptr) weight_chunk(c, nwl[g * 8u + t]);
                }
                uint4 o;
                o.x = __builtin_amdgcn_perm(c.z, c.x, 0x05040100u);   // (x0, x4)
                o.y = __builtin_amdgcn_perm(c.z, c.x, 0x07060302u);   // (x1, x5)
                o.z = __builtin_amdgcn_perm(c.w, c.y, 0x05040100u);   // (x2, x6)
                o.w = __builtin_amdgcn_perm(c.w, c.y, 0x07060302u);   // (x3, x7)
                xs[m * WS + g * 8u + t] = o;
                s0 = dot2_bf16(c.x, kOnePair, s0);
                s1 = dot2_bf16(c.y, kOnePair, s1);
                s0 = dot2_bf16(c.z, kOnePair, s0);
                s1 = dot2_bf16(c.w, kOnePair, s1);
            }
            reinterpret_cast<float*>(sx)[g * 4u + m] = s0 + s1;
        }
        if constexpr (kEarly) raise_counter(ctr, lane);
    }
    if constexpr (resid) {   // the same loads, after the prologue
        if constexpr (kLaneGroups) {
            const uint32_t off = (ltile * pairs * 16u + (ob >> 1) * 16u + j) * 8u + (ob & 1u) * 4u;
#pragma unroll
            for (int q = 0; q < NW; ++q)
#pragma unroll
                for (int b = 0; b < P; ++b)
                    sbl[q][b] = __builtin_amdgcn_raw_buffer_load_b32(lm[q].sb, off, (first + 2u * b) * 128u, kStreamPolicy);
        }
        // Two batches of weights in flight before the first arithmetic.
#pragma unroll
        for (int q = 0; q < NW; ++q) load_batch<P, !kLaneGroups>(lm[q], first, last, ba[q]);
#pragma unroll
        for (int q = 0; q < NW; ++q) load_batch<P, !kLaneGroups>(lm[q], first + P, last, bb[q]);
    }
    if constexpr (kEarly) {
        wait_counter(ctr, nstage);
    } else {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");   // x, its sums and the zero row
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }

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
        compute_lane_groups<M, NW, P>(ba, bb, sbl, first, cnt, G, xs, zs, WS, sx, lane, mask, bits, y);
    } else if constexpr (!LOOP) {
        compute_straight<M, NW, P>(ba, bb, first, cnt, G, xa, sx, mask, bits, y);
    } else {
        compute_loop<M, NW, P>(ba, bb, lm, first, last, cnt, G, xa, sx, mask, bits, y);
    }

    reduce_splits<M, NW>(y, red, wave, split, S, kb, j);

    const uint32_t out_row = tile * kTileRows + j;
    if constexpr (DUAL) {
        // The up tile's rows meet the gate tile's in LDS (one slot per row tile of the block).
        const bool up_tile = (gtile & 1u) != 0u;
        float* cs = comb + ((wave >> sh) >> 1) * M * kTileRows;
        if (split == 0u && kb == 0u && up_tile) {
#pragma unroll
            for (int m = 0; m < M; ++m) cs[m * kTileRows + j] = round_bf16(y[0][m]);
        }
        __syncthreads();
        if (split == 0u && kb == 0u && !up_tile && out_row < seg_n) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float out = gate_up_value(y[0][m], cs[m * kTileRows + j]);
                seg_y[static_cast<size_t>(m) * seg_n + out_row] = f32_to_bf16_bits(out);
            }
        }
    } else if (split == 0u && kb == 0u && out_row < seg_n) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float out = output_value<EPI, M, NW>(y, m, p.cap);
            seg_y[static_cast<size_t>(m) * seg_n + out_row] = f32_to_bf16_bits(out);
        }
    }
}

size_t skinny_lds_bytes(uint32_t m, uint32_t k, bool dual, uint32_t nwave, int norm = 0) {
    const size_t W = k / 8u;
    const size_t G = k / 64u;
    // x rows and a zero row, the norms' weights, group sums, the split reduction, counters,
    // the rms partials, the gate/up combine.
    const size_t copies = static_cast<size_t>(norm == 2 ? 2 : (norm != 0 ? 1 : 0)) * lds_copy_bytes(2u * k);
    return (m + 1u) * (W + 1u) * 16u + copies + G * 16u + static_cast<size_t>(nwave) * m * kTileRows * 4u + 32u +
           (norm ? (m * G + m) * 4u : 0u) + (dual ? static_cast<size_t>(nwave / 2u) * m * kTileRows * 4u : 0u);
}

size_t max_lds_per_block();

template <int M, bool DUAL, int EPI, int NWAVE, int NORM = 0, int CH = 1>
void launch_skinny_t(const SkinnyParams& p, uint32_t tiles_total, hipStream_t stream) {
    // Pairs per register batch (two batches in flight): 4, so that a wave's whole range
    // (at most kSkinnyPairsUpFront pairs) is requested at once; 2 for the softcap head,
    // whose waves loop.
    constexpr int P = EPI != 0 ? 2 : 4;
    const uint32_t per_wave = (p.pairs + p.splits - 1u) / p.splits;
    auto kernel = per_wave <= 2u * P ? q4_skinny_kernel<M, DUAL, EPI, P, NWAVE, NORM, false, CH>
                                     : q4_skinny_kernel<M, DUAL, EPI, P, NWAVE, NORM, true, CH>;
    const size_t lds = skinny_lds_bytes(M, p.k, DUAL, NWAVE, NORM);
    HYP_REQUIRE(lds <= max_lds_per_block(), HYP_STATUS_INTERNAL, "skinny: x staging exceeds the device's LDS");
    if (lds > 65536u) {
        static thread_local int configured_device = -1;
        int dev = 0;
        HYP_HIP_CHECK(hipGetDevice(&dev));
        if (configured_device != dev) {
            for (const void* f : {reinterpret_cast<const void*>(q4_skinny_kernel<M, DUAL, EPI, P, NWAVE, NORM, false, CH>),
                                  reinterpret_cast<const void*>(q4_skinny_kernel<M, DUAL, EPI, P, NWAVE, NORM, true, CH>)}) {
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

// Waves per workgroup of a plain or normalising launch of `ts` = tiles x splits waves (the
// fused gate/up runs 8-wave workgroups, the softcap head 4). Measured on the decode shapes of
// a 12B layer (MI355X, cold weights, every waves x splits pair with the splits of
// choose_skinny_splits fixed): a workgroup holds the fewest waves that keep the grid at about
// one workgroup per compute unit or more - [15360,3840] at m = 1 8 waves (7.69 us against
// 8.17 with 16), o [3840,4096] 4 (4.30 against 5.76 with 16 waves at 16 splits), the
// normalised q/k/v 8 when one round of them covers the grid (7.71 against 9.04 with 16 when
// that form still spilled); 16 when the splits need them (down [3840,15360], 16 splits),
// for a normalising grid larger than one round of 8-wave workgroups, and for a plain
// launch of m >= 2 rows whose grid fills
// the compute units with 16-wave workgroups ([15360,3840] at m = 4: 9.07 against 9.36 us),
// which stage x once per compute unit.
uint32_t choose_skinny_waves(uint32_t tiles_total, uint32_t splits, uint32_t m, uint32_t k, int norm) {
    const uint64_t ts = static_cast<uint64_t>(tiles_total) * splits;
    const uint64_t cus = device_compute_units();
    uint32_t w;
    if (splits >= 16u) {
        w = 16u;
    } else if (norm == 2) {
        // The residual prologue (run by the staging waves before their own weight loads):
        // 8-wave workgroups when one round of them covers the grid, else 16-wave ones, which
        // leave some compute units idle rather than give some two workgroups (the 12B's
        // sliding q/k/v, 512 tiles at 4 splits: 9.48 us in 8-wave workgroups against 9.56 in
        // 16-wave ones at 8 splits; its global q/k, 544 tiles: 10.48 us in 136 16-wave
        // workgroups against 13.15 in 272 8-wave ones).
        w = ts <= 8u * cus ? std::max(splits, 8u) : 16u;
    } else if (norm == 0 && m >= 2u && ts >= 16u * cus * 9u / 10u) {
        w = 16u;
    } else if (norm == 1) {
        // As the residual form: 8 waves for one round, else 16 (the 12B's global q/k,
        // 544 tiles at 4 splits: 8.6 us in 136 16-wave workgroups against 10.6 in 272 8-wave
        // ones; 7.3-7.5 against 7.7 us at 16 x 8 for its sliding q/k/v, 512 tiles).
        w = ts <= 8u * cus ? std::max(splits, 8u) : 16u;
    } else if (ts >= 8u * cus * 9u / 10u) {
        w = std::max(splits, 8u);
    } else {
        w = std::max(splits, 4u);
    }
    // A residual prologue holds every (row, group) unit in one thread.
    if (norm == 2 && static_cast<uint64_t>(m) * (k / 64u) > 64u * w) w = 16u;
    return w;
}

template <int M>
void launch_skinny_m(const SkinnyParams& p, uint32_t tiles_total, bool dual, Epilogue epi, int norm,
                     hipStream_t stream) {
    if (dual) {
        launch_skinny_t<M, true, 0, kSkinnyDualWaves>(p, tiles_total, stream);
    } else if (epi == Epilogue::kSoftcap) {
        launch_skinny_t<M, false, 1, 4>(p, tiles_total, stream);
    } else {
        const uint32_t w = choose_skinny_waves(tiles_total, p.splits, M, p.k, norm);
        // The normalising prologue with each unit over kSpreadLanes lanes where the spread units
        // fit four waves, one per SIMD (at most 64 units: one row up to k = 4096). Beyond that the
        // unit-per-thread form already has a staging wave on every SIMD, and spreading would put
        // several on each.
        const bool spread = static_cast<uint64_t>(M) * (p.k / 64u) * kSpreadLanes <= 256u;
        if (norm == 2) {
            if (spread) {
                w == 8u ? launch_skinny_t<M, false, 0, 8, 2, kSpreadLanes>(p, tiles_total, stream)
                        : launch_skinny_t<M, false, 0, 16, 2, kSpreadLanes>(p, tiles_total, stream);
            } else {
                w == 8u ? launch_skinny_t<M, false, 0, 8, 2>(p, tiles_total, stream)
                        : launch_skinny_t<M, false, 0, 16, 2>(p, tiles_total, stream);
            }
        } else if (norm == 1) {
            if (spread) {
                w == 8u ? launch_skinny_t<M, false, 0, 8, 1, kSpreadLanes>(p, tiles_total, stream)
                        : launch_skinny_t<M, false, 0, 16, 1, kSpreadLanes>(p, tiles_total, stream);
            } else {
                w == 8u ? launch_skinny_t<M, false, 0, 8, 1>(p, tiles_total, stream)
                        : launch_skinny_t<M, false, 0, 16, 1>(p, tiles_total, stream);
            }
        } else if (w == 4u) {
            launch_skinny_t<M, false, 0, 4>(p, tiles_total, stream);
        } else if (w == 8u) {
            launch_skinny_t<M, false, 0, 8>(p, tiles_total, stream);
        } else {
            launch_skinny_t<M, false, 0, 16>(p, tiles_total, stream);
        }
    }
}

void launch_skinny(SkinnyParams& p, uint32_t tiles_total, uint32_t m, bool dual, Epilogue epi, int norm,
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
    // The fewest splits (a power of two) that leave every wave at most kSkinnyPairsUpFront
    // pairs, all its loads issued at once; doubled only while the launch has fewer than two
    // waves per compute unit. Measured on the decode shapes of a 12B layer (MI355X, cold
    // weights, every waves x splits pair): more splits of a short range cost more in x
    // staging and the split reduction than the extra waves gain - o [3840,4096] 4 splits in
    // 4-wave workgroups 4.30 us, 16 splits (16 waves) 5.76 us; [15360,3840] 4 (8 waves)
    // 7.69 us, 8 splits 9.93 us. The softcap head (262144 rows, 4-wave workgroups, many per
    // compute unit): 1 (95 vs 100 us at m = 1, 111 vs 123 us at m = 4 with 2). The fused
    // gate/up: at most 4, so that an 8-wave workgroup holds both halves of a row tile.
    (void)m;   // the measured choices did not depend on the row count
    const uint32_t cus = device_compute_units();
    const uint32_t cap = form == SkinnyForm::kDual ? kSkinnyDualWaves / 2u : kSkinnyWaves;
    uint32_t s = 1u;
    if (form == SkinnyForm::kHead) {
        s = 1u;
    } else {
        while (s < cap && pairs > s * kSkinnyPairsUpFront) s *= 2u;
        while (s < cap && tiles * s < 2u * cus && pairs >= 2u * s) s *= 2u;
    }
    while (s > 1u && pairs < s) s /= 2u;
    return s;
}

bool skinny_supported(uint32_t m, uint32_t k, bool dual) {
    return m >= 1u && m <= kSkinnyMaxM && k % 64u == 0u && k > 0u &&
           skinny_lds_bytes(m, k, dual, dual ? kSkinnyDualWaves : kSkinnyWaves) <= max_lds_per_block();
}

bool skinny_norm_supported(uint32_t m, uint32_t k) {
    return m >= 1u && m <= kSkinnyMaxM && k % 64u == 0u && k > 0u &&
           skinny_lds_bytes(m, k, false, kSkinnyWaves, 1) <= max_lds_per_block();
}

bool skinny_resid_supported(uint32_t m, uint32_t k) {
    return m >= 1u && m <= kSkinnyMaxM && k % 64u == 0u && k > 0u && m * (k / 64u) <= 64u * kSkinnyWaves &&
           skinny_lds_bytes(m, k, false, kSkinnyWaves, 2) <= max_lds_per_block();
}

namespace {
void set_residual(SkinnyParams& p, const SkinnyResidual* res) {
    if (res == nullptr) return;
    p.res_branch = res->branch;
    p.res_in = res->in;
    p.res_out = res->out;
    p.res_w = res->w;
    p.res_scalar = res->scalar;
    p.x = res->in;
}
}  // namespace

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
        splits = choose_skinny_splits(dual ? 2u * d.tiles : d.tiles, d.pairs, m,
                                      head ? SkinnyForm::kHead : (dual ? SkinnyForm::kDual : SkinnyForm::kPlain));
    }
    HYP_REQUIRE(splits == 1u || splits == 2u || splits == 4u || (!head && !dual && (splits == 8u || splits == 16u)),
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
    launch_skinny(p, dual ? 2u * d.tiles : d.tiles, m, dual, epi, 0, stream);
}

void launch_q4_skinny_group(const Q4Matrix* const* ws, uint16_t* const* ys, uint32_t count, const uint16_t* x,
                            uint32_t m, const float* rms_eps, const uint16_t* norm_w, hipStream_t stream,
                            const SkinnyResidual* res) {
    HYP_REQUIRE(count >= 1u && count <= kSkinnyMaxGroup, HYP_STATUS_INTERNAL, "skinny: bad group size");
    const uint32_t k = ws[0]->k;
    const bool norm = rms_eps != nullptr;
    HYP_REQUIRE(res == nullptr || (norm && skinny_resid_supported(m, k)), HYP_STATUS_INTERNAL,
                "skinny: residual prologue needs the norm and one unit per thread");
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
    p.norm_w = norm ? norm_w : nullptr;
    p.splits = choose_skinny_splits(tiles_total, p.pairs, m, SkinnyForm::kPlain);
    p.split_shift = static_cast<uint32_t>(__builtin_ctz(p.splits));
    set_residual(p, res);
    launch_skinny(p, tiles_total, m, false, Epilogue::kNone, res != nullptr ? 2 : (norm ? 1 : 0), stream);
}

}  // namespace hyperion::hip

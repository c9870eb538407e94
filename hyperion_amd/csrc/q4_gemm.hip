// Prefill GEMM for MLX-affine Q4/g64 weights on gfx950 bf16 MFMA.
//
// Replaces mlx::core::quantized_matmul(..., transpose=true, 64, 4, "affine") at
// prefill, where the reference's chunk loop (native/hyperion_mlx/src/model.cc:574-610)
// hands every projection up to 2048 rows at once.
//
// Y[m, n] = X[m, k] . dequant(W)[n, k]^T, fp32 accumulation, bf16 out.
//
// The contraction runs on v_mfma_f32_16x16x32_bf16, whose B operand lane layout is the
// tiled resident layout's (q4_layout.h): for a 16-column tile and a pair of groups,
// lane (j, kb) loads one 16-byte entry holding words 2kb, 2kb+1 of row j for both
// groups, i.e. exactly its B values for the pair's four 32-k MFMA steps. So:
//  * A workgroup (4 waves) computes a (16*MT) x (64*NT) output tile; wave w owns
//    columns [16*NT*w, 16*NT*(w+1)) for every row, so each weight is dequantized by
//    exactly one wave, in registers: code -> fp32 -> fma(scale, q, bias) -> one
//    rounding to bf16 (v_cvt_pk_bf16_f32), the MLX dequantized value.
//  * The k loop advances one pair of groups (128 k) per iteration. X tiles of
//    (16*MT) x 128 bf16 go straight from HBM to LDS (16-byte buffer loads with the LDS
//    as destination, no VGPRs), double buffered with one barrier per iteration; the
//    next tile and the next pair's weights are in flight while the current pair
//    computes. LDS rows are 256 bytes with their 16-byte chunks XOR-swizzled by
//    (row % 16), so the 16 rows an A-fragment read touches hit distinct banks.
//  * Within an iteration the B fragments of k-step s+1 are dequantized while the
//    MFMAs of step s run, and each step's A fragments are read from LDS in one
//    batch ahead of its MFMAs.
//  * Workgroup ids are remapped so each XCD (ids are dealt round-robin over the 8 XCDs)
//    gets a contiguous run of tiles that share X rows, keeping the X block in that
//    XCD's L2.
#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>

#include "common.h"
#include "kernels.h"
#include "q4_dequant.h"
#include "q4_layout.h"

namespace hyperion::hip {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPairK = 128;                 // k per iteration (two groups)
constexpr int kRowBytes = kPairK * 2;       // one LDS row of an X tile

// One projection of a (possibly grouped) launch: its workgroup column tiles are the
// global column tiles [tn_begin, tn_begin + ceil(n / 128)).
struct GemmSegment {
    const uint4* codes;   // tiled codes (q4_layout.h)
    const uint2* sb;      // tiled scales and biases
    uint16_t* y;          // [m, n]
    uint32_t n;
    uint32_t row_tiles;   // ceil(n / 16)
    uint32_t code_bytes;
    uint32_t sb_bytes;
    uint32_t tn_begin;
    uint32_t col_begin;   // first column of this segment in the split-k workspace rows
};

constexpr uint32_t kMaxGemmSegments = 3;

struct GemmParams {
    GemmSegment seg[kMaxGemmSegments];   // segments past nseg are unused
    uint32_t nseg;
    const uint16_t* x;    // m x k bf16 (m * k * 2 < 2^31 bytes)
    uint32_t m;
    uint32_t k;
    uint32_t pairs;       // ceil(k / 128)
    uint32_t tiles_n;     // workgroup column tiles over all segments
    uint32_t tiles_total;
    // Split k (pair-step kernel): ksplit workgroups share an output tile, each covering
    // pairs_per_split pairs, and write fp32 partials to partial[ksplit][m][n_total].
    uint32_t ksplit;
    uint32_t pairs_per_split;
    uint32_t n_total;
    float* partial;
    // Host dispatch only: the launch is a fused gate/up (seg[0] gate with the output,
    // seg[1] up), run by the DUAL kernels.
    uint32_t dual;
};

// The segment of global column tile tn (workgroup-uniform selects, no indexed parameter
// access) and tn's index within it.
struct SegView {
    const uint4* codes;
    const uint2* sb;
    uint16_t* y;
    uint32_t n;
    uint32_t row_tiles;
    uint32_t code_bytes;
    uint32_t sb_bytes;
    uint32_t col_begin;
    uint32_t tn;
};

__device__ __forceinline__ SegView segment_of(const GemmParams& p, uint32_t tn) {
    const bool in1 = p.nseg > 1u && tn >= p.seg[1].tn_begin;
    const bool in2 = p.nseg > 2u && tn >= p.seg[2].tn_begin;
    const GemmSegment& a = p.seg[0];
    const GemmSegment& b = p.seg[1];
    const GemmSegment& c = p.seg[2];
    SegView v;
    v.codes = in2 ? c.codes : (in1 ? b.codes : a.codes);
    v.sb = in2 ? c.sb : (in1 ? b.sb : a.sb);
    v.y = in2 ? c.y : (in1 ? b.y : a.y);
    v.n = in2 ? c.n : (in1 ? b.n : a.n);
    v.row_tiles = in2 ? c.row_tiles : (in1 ? b.row_tiles : a.row_tiles);
    v.code_bytes = in2 ? c.code_bytes : (in1 ? b.code_bytes : a.code_bytes);
    v.sb_bytes = in2 ? c.sb_bytes : (in1 ? b.sb_bytes : a.sb_bytes);
    v.col_begin = in2 ? c.col_begin : (in1 ? b.col_begin : a.col_begin);
    v.tn = tn - (in2 ? c.tn_begin : (in1 ? b.tn_begin : 0u));
    return v;
}

// Raw weights of one pair for one lane: NT code entries and NT scale entries.
template <int NT>
struct BRaw {
    uint4 c[NT];
    uint2 sb[NT];
};

// B fragments of k-step s (s = 0..3: group s/2, MFMA step s%2) from the raw entries.
template <int NT, int S>
__device__ __forceinline__ void dequant_step(const BRaw<NT>& raw, bf16x8_t (&b)[NT]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t sbw = S < 2 ? raw.sb[nt].x : raw.sb[nt].y;
        const float sc = bf16_bits_to_f32(sbw & 0xFFFFu);
        const float bi = bf16_bits_to_f32(sbw >> 16);
        const uint32_t word = S == 0 ? raw.c[nt].x : (S == 1 ? raw.c[nt].y : (S == 2 ? raw.c[nt].z : raw.c[nt].w));
        b[nt] = dequant_word(word, sc, bi);
    }
}

// Raw weights of pair `pair` for this lane: the 16-byte code entry and 8-byte scale
// entry of each of its NT column tiles (offsets set up once, the pair is a scalar offset).
template <int NT, typename R>
__device__ __forceinline__ void load_b(const R& wr, const uint32_t (&c_off)[NT], const uint32_t (&s_off)[NT],
                                       uint32_t pair, BRaw<NT>& raw) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        raw.c[nt] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(wr.c[nt & 1], c_off[nt], pair * 1024u, 0));
        raw.sb[nt] = __builtin_bit_cast(
            uint2, __builtin_amdgcn_raw_buffer_load_b64(wr.s[nt & 1], s_off[nt], pair * 128u, 0));
    }
}

// The MFMAs of k-step S over all M tiles; A fragments come from the LDS tile
// (swizzled rows: logical chunk c of row r sits at chunk c ^ (r % 16)).
template <int MT, int NT, int S>
__device__ __forceinline__ void mfma_step(const uint8_t* xb, uint32_t lane, const bf16x8_t (&b)[NT],
                                          f32x4_t (&acc)[MT][NT]) {
    const uint32_t i = lane & 15u;
    const uint32_t kb = lane >> 4;
    // This lane's 8 values: group S/2, word 2kb + S%2 of the pair, i.e. logical chunk c.
    const uint32_t c = (S / 2) * 8u + 2u * kb + (S % 2);
    const uint8_t* row = xb + i * kRowBytes + ((c ^ i) << 4);
    constexpr int kHalf = MT / 2;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        bf16x8_t a[kHalf];
#pragma unroll
        for (int mt = 0; mt < kHalf; ++mt)
            a[mt] = *reinterpret_cast<const bf16x8_t*>(row + (h * kHalf + mt) * 16u * kRowBytes);
#pragma unroll
        for (int mt = 0; mt < kHalf; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
                acc[h * kHalf + mt][nt] =
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt], b[nt], acc[h * kHalf + mt][nt], 0, 0, 0);
    }
    // Scheduling hint for this region (the dequantization of the next step, issued just
    // before, and these MFMAs): the first half's A reads, then one MFMA followed by
    // kValu VALU ops throughout, with the second half's A reads after the first MFMAs.
    constexpr int kMfma = MT * NT;
    constexpr int kValu = (NT * 25 + kMfma - 1) / kMfma;   // dequant ops of a step per MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, kHalf, 0);   // DS read
#pragma unroll
    for (int t = 0; t < kMfma; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);   // VALU
        if (t == 1) __builtin_amdgcn_sched_group_barrier(0x100, kHalf, 0);
    }
}

// The fused MLP gating of one output (forward.cc:338-343 without the down projection):
// the gate and up sums rounded to bf16 as a separate launch stores them, then
// bf16(gelu_chain(gate) * up) (the split-k reduce's form; the GEMM epilogues use the
// tabulated gated_bits_table, which gives the same bits).
__device__ __forceinline__ uint16_t gated_bits(float gate_sum, float up_sum) {
    const float g = bf16_bits_to_f32(f32_to_bf16_bits(gate_sum));
    const float u = bf16_bits_to_f32(f32_to_bf16_bits(up_sum));
    return f32_to_bf16_bits(gelu_tanh_bf16_chain(g) * u);
}

// The GELU chain of a bf16 input x is a function of its 16 bits with closed forms outside
// 2^-10 <= |x| < 8: tanh's argument is then either below 2^-9 in magnitude (1 + t rounds
// to 1, so the chain gives bf16(x / 2)) or at least 4 in magnitude (t = +-1, so it gives x
// for finite x >= 8, -0 for finite x <= -8). A DUAL epilogue tabulates the band and the
// 256 non-finite inputs (+-inf, NaN) in LDS with the chain itself (a few values per
// thread) and looks outputs up.
constexpr uint32_t kGeluLo = 0x3A80u;                  // bf16 bits of 2^-10 (magnitude)
constexpr uint32_t kGeluHi = 0x4100u;                  // bf16 bits of 8
constexpr uint32_t kGeluSpan = kGeluHi - kGeluLo;      // band values of one sign
constexpr uint32_t kGeluInf = 0x7F80u;                 // magnitudes from here on: inf, NaN
constexpr uint32_t kGeluSpecial = 0x8000u - kGeluInf;  // non-finite values of one sign
constexpr uint32_t kGeluEntries = 2u * kGeluSpan + 2u * kGeluSpecial;
constexpr uint32_t kGeluTableBytes = kGeluEntries * 2u;

// The bf16 bits tabulated at entry i: the positive band, the negative band, then the
// non-finite values of each sign.
__device__ __forceinline__ uint32_t gelu_table_bits(uint32_t i) {
    if (i < 2u * kGeluSpan) {
        const uint32_t neg = i >= kGeluSpan ? 1u : 0u;
        return (neg << 15) | (kGeluLo + i - neg * kGeluSpan);
    }
    const uint32_t j = i - 2u * kGeluSpan;
    const uint32_t neg = j >= kGeluSpecial ? 1u : 0u;
    return (neg << 15) | (kGeluInf + j - neg * kGeluSpecial);
}

__device__ __forceinline__ void build_gelu_table(uint16_t* tab, uint32_t tid, uint32_t nthreads) {
    for (uint32_t i = tid; i < kGeluEntries; i += nthreads)
        tab[i] = f32_to_bf16_bits(gelu_tanh_bf16_chain(bf16_bits_to_f32(gelu_table_bits(i))));
}

// gelu_tanh_bf16_chain(x) for a bf16 value x, from the table and the closed forms; the
// table is read for every x (entry 0 when x is outside it), so no branch is taken.
__device__ __forceinline__ float gelu_lookup(const uint16_t* tab, float x) {
    const uint32_t b = __float_as_uint(x) >> 16;
    const uint32_t a = b & 0x7FFFu;
    const uint32_t neg = b >> 15;
    const bool band = a - kGeluLo < kGeluSpan;
    const bool special = a >= kGeluInf;
    const uint32_t idx = band ? neg * kGeluSpan + a - kGeluLo
                              : (special ? 2u * kGeluSpan + neg * kGeluSpecial + a - kGeluInf : 0u);
    const float tabulated = bf16_bits_to_f32(tab[idx]);
    const float half = round_bf16(0.5f * x);
    const float large = neg ? -0.0f : x;
    return (band || special) ? tabulated : (a < kGeluLo ? half : large);
}

__device__ __forceinline__ uint16_t gated_bits_table(const uint16_t* tab, float gate_sum, float up_sum) {
    const uint32_t gu = cvt_pk_bf16(gate_sum, up_sum);   // both rounded by one instruction
    const float g = __uint_as_float(gu << 16);
    const float u = __uint_as_float(gu & 0xFFFF0000u);
    return f32_to_bf16_bits(gelu_lookup(tab, g) * u);
}

// Buffer resources of column tile nt: in a DUAL launch tile 0 is the gate's, tile 1 the
// up projection's (seg[1]); otherwise all come from the segment in view.
struct WeightRsrc {
    __amdgpu_buffer_rsrc_t c[2];
    __amdgpu_buffer_rsrc_t s[2];
};

template <bool DUAL>
__device__ __forceinline__ WeightRsrc weight_rsrc(const GemmParams& p, const SegView& sv) {
    WeightRsrc r;
    r.c[0] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4*>(sv.codes), static_cast<short>(0),
                                               static_cast<int>(sv.code_bytes), 0x00020000);
    r.s[0] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2*>(sv.sb), static_cast<short>(0),
                                               static_cast<int>(sv.sb_bytes), 0x00020000);
    if (DUAL) {
        r.c[1] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4*>(p.seg[1].codes), static_cast<short>(0),
                                                   static_cast<int>(p.seg[1].code_bytes), 0x00020000);
        r.s[1] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint2*>(p.seg[1].sb), static_cast<short>(0),
                                                   static_cast<int>(p.seg[1].sb_bytes), 0x00020000);
    } else {
        r.c[1] = r.c[0];
        r.s[1] = r.s[0];
    }
    return r;
}

// The view of a workgroup's column tile tn: in a DUAL launch always the gate's segment
// (the up projection rides along as column tile 1 of every wave).
template <bool DUAL>
__device__ __forceinline__ SegView view_of(const GemmParams& p, uint32_t tn) {
    SegView sv = segment_of(p, DUAL ? 0u : tn);
    if (DUAL) sv.tn = tn;
    return sv;
}

// Split k: this workgroup's fp32 partials of k split kz, summed by the split-k reduce
// kernels. acc[mt][nt][r] is (row 16 mt + 4 kb + r, column 16 (kOut wave + nt) + j) of
// the tile (DUAL: column 16 wave + j of the gate for nt = 0, of up for nt = 1, which sits
// seg[1].col_begin further along the workspace row).
template <int MT, int NT, int kOut, bool DUAL>
__device__ __forceinline__ void store_partials(const GemmParams& p, const SegView& sv, uint32_t kz, uint32_t m0,
                                               uint32_t n0, uint32_t wave, uint32_t lane,
                                               const f32x4_t (&acc)[MT][NT]) {
    const uint32_t j = lane & 15u;
    const uint32_t kb = lane >> 4;
    float* part = p.partial + static_cast<size_t>(kz) * p.m * p.n_total;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t col = n0 + (wave * kOut + (DUAL ? 0 : nt)) * 16u + j;
        const uint32_t base = DUAL && nt == 1 ? p.seg[1].col_begin : sv.col_begin;
        if (col >= sv.n) continue;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t row = m0 + mt * 16u + kb * 4u + r;
                if (row < p.m) part[static_cast<size_t>(row) * p.n_total + base + col] = acc[mt][nt][r];
            }
    }
}

// The tile's bf16 outputs into LDS rows of out_row bytes: column 16 (kOut wave + nt) + j
// gets bf16(acc[.][nt]); DUAL: column 16 wave + j gets the gated value of acc[.][0] (gate)
// and acc[.][1] (up), through the GELU table `tab` (built in LDS past the rows).
template <int MT, int NT, int kOut, bool DUAL>
__device__ __forceinline__ void stage_out(uint8_t* xs, uint32_t out_row, uint32_t wave, uint32_t lane,
                                          const f32x4_t (&acc)[MT][NT], const uint16_t* tab) {
    const uint32_t j = lane & 15u;
    const uint32_t kb = lane >> 4;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kOut; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t row = mt * 16u + kb * 4u + r;
                const uint32_t col = (wave * kOut + nt) * 16u + j;
                const uint16_t v =
                    DUAL ? gated_bits_table(tab, acc[mt][0][r], acc[mt][NT - 1][r])
                         : f32_to_bf16_bits(acc[mt][nt][r]);
                *reinterpret_cast<uint16_t*>(xs + row * out_row + col * 2u) = v;
            }
}

template <int MT, int NT, bool ODD, bool DUAL>
__global__ __launch_bounds__(kThreads) void q4_gemm_kernel(GemmParams p) {
    static_assert(!DUAL || NT == 2, "a dual launch pairs one gate and one up tile per wave");
    constexpr int kOut = DUAL ? 1 : NT;   // output column tiles per wave
    constexpr int BM = 16 * MT;
    constexpr int kTileBytes = BM * kRowBytes;
    constexpr int kXLoads = BM / 4 / kWaves;   // 1 KB direct loads per wave per X tile
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];   // [2][BM][256 B]

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // XCD-aware tile order: XCD x = blockIdx % 8 runs tiles [start_x, start_x + count_x).
    const uint32_t bid = blockIdx.x;
    const uint32_t xcd = bid & 7u;
    const uint32_t slot = bid >> 3;
    const uint32_t ext_total = p.tiles_total * p.ksplit;
    const uint32_t per = ext_total >> 3;
    const uint32_t rem = ext_total & 7u;
    const uint32_t ext = xcd * per + min(xcd, rem) + slot;
    const uint32_t kz = ext / p.tiles_total;          // this workgroup's k split
    const uint32_t tile = ext - kz * p.tiles_total;
    const uint32_t tm = tile / p.tiles_n;
    const SegView sv = view_of<DUAL>(p, tile - tm * p.tiles_n);
    const uint32_t m0 = tm * BM;
    const uint32_t n0 = sv.tn * (kWaves * 16u * kOut);
    const uint32_t tile16_0 = n0 / 16u + wave * kOut;

    const uint32_t k = p.k;
    const uint32_t pairs = p.pairs;

    // X staging: load t of wave w covers tile rows 4 (w kXLoads + t) .. +3; lane l fills
    // LDS chunk (l % 16) of row r = 4 (w kXLoads + t) + l / 16 with the row's logical
    // chunk (l % 16) ^ (r % 16). kXLoads is a multiple of 4, so r % 16 = (4 t + l / 16)
    // % 16. Each load's lane offset is set up once; the pair is a scalar offset. Rows past
    // m get an offset past the buffer resource (m * k * 2 bytes) and load zeros; so do the
    // chunks past k of an odd group count (ODD: the last pair's second group).
    static_assert(kXLoads % 4 == 0, "swizzle period");
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.x), static_cast<short>(0), static_cast<int>(p.m * k * 2u), 0x00020000);
    const uint32_t lh = lane >> 4;
    uint32_t xoff[kXLoads];
    uint32_t xchunk[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) xchunk[t] = (lane & 15u) ^ ((4u * t + lh) & 15u);
#pragma unroll
    for (int t = 0; t < kXLoads; ++t) {
        const uint32_t row = m0 + 4u * (wave * kXLoads + t) + lh;
        xoff[t] = row < p.m ? row * k * 2u + xchunk[t % 4] * 16u : 0x80000000u;
    }
    auto load_x = [&](uint32_t pair, uint8_t* buf) {
#pragma unroll
        for (int t = 0; t < kXLoads; ++t) {
            uint32_t off = xoff[t];
            if (ODD && pair * kPairK + xchunk[t % 4] * 8u >= k) off = 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void*)(buf + (wave * kXLoads + t) * 1024u), 16,
                static_cast<int>(off), static_cast<int>(pair * kPairK * 2u), 0, 0);
        }
    };

    // Weights: column tile (tile16_0 + nt) (DUAL: tile tile16_0 of the gate, then of up),
    // clamped to the last tile (columns past n are computed, never stored).
    const WeightRsrc wr = weight_rsrc<DUAL>(p, sv);
    uint32_t c_off[NT];
    uint32_t s_off[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t t16 = min(tile16_0 + (DUAL ? 0u : static_cast<uint32_t>(nt)), sv.row_tiles - 1u);
        c_off[nt] = (t16 * pairs * 64u + lane) * 16u;
        s_off[nt] = (t16 * pairs * 16u + (lane & 15u)) * 8u;
    }

    f32x4_t acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // This workgroup's pairs [p0, p1) (all of them without split k).
    const uint32_t p0 = kz * p.pairs_per_split;
    const uint32_t p1 = min(p0 + p.pairs_per_split, pairs);

    BRaw<NT> braw, bnext;
    load_x(p0, xs);
    load_b<NT>(wr, c_off, s_off, p0, braw);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    bf16x8_t b0[NT], b1[NT];
    dequant_step<NT, 0>(braw, b0);

    // The loop body has no branches (branches split the accumulators' live ranges and
    // cost AGPR copies); the last iteration prefetches its own pair again, harmlessly.
    for (uint32_t pair = p0; pair < p1; ++pair) {
        const uint8_t* xb = xs + ((pair - p0) & 1u) * kTileBytes;
        const uint32_t pn = min(pair + 1u, p1 - 1u);
        load_x(pn, xs + ((pair - p0 + 1u) & 1u) * kTileBytes);
        load_b<NT>(wr, c_off, s_off, pn, bnext);

        dequant_step<NT, 1>(braw, b1);
        mfma_step<MT, NT, 0>(xb, lane, b0, acc);
        dequant_step<NT, 2>(braw, b0);
        mfma_step<MT, NT, 1>(xb, lane, b1, acc);
        dequant_step<NT, 3>(braw, b1);
        mfma_step<MT, NT, 2>(xb, lane, b0, acc);
        braw = bnext;
        dequant_step<NT, 0>(braw, b0);
        mfma_step<MT, NT, 3>(xb, lane, b1, acc);

        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }

    if (p.ksplit > 1u) {
        store_partials<MT, NT, kOut, DUAL>(p, sv, kz, m0, n0, wave, lane, acc);
        return;
    }

    // Epilogue: the workgroup's (16 MT) x (64 kOut) tile goes through LDS (rows of
    // 128 kOut bytes plus 32 bytes of padding, so the four row groups a write touches hit
    // distinct banks) and leaves as 16-byte row segments. acc[mt][nt][r] is tile element
    // (16 mt + 4 kb + r, 16 kOut wave + 16 nt + j) (DUAL: nt = 0 gate, 1 up of column
    // 16 wave + j).
    constexpr uint32_t kOutRow = 128u * kOut + 32u;
    static_assert(BM * kOutRow + (DUAL ? kGeluTableBytes : 0u) <= 2u * kTileBytes,
                  "output staging exceeds the X buffers");
    uint16_t* tab = reinterpret_cast<uint16_t*>(xs + BM * kOutRow);
    __syncthreads();
    if constexpr (DUAL) {
        build_gelu_table(tab, tid, kThreads);
        __syncthreads();
    }
    stage_out<MT, NT, kOut, DUAL>(xs, kOutRow, wave, lane, acc, tab);
    __syncthreads();
    constexpr uint32_t kCols = 64u * kOut;
    constexpr uint32_t kChunks = kCols / 8u;                  // 16-byte chunks per row
    constexpr uint32_t kRowsPerPass = kThreads / kChunks;
    const uint32_t ch = threadIdx.x % kChunks;
    const uint32_t col0 = n0 + ch * 8u;
    if ((sv.n & 7u) == 0u && (reinterpret_cast<uintptr_t>(sv.y) & 15u) == 0u) {
        for (uint32_t r = threadIdx.x / kChunks; r < BM; r += kRowsPerPass) {
            const uint32_t row = m0 + r;
            if (row < p.m && col0 < sv.n)
                *reinterpret_cast<uint4*>(sv.y + static_cast<size_t>(row) * sv.n + col0) =
                    *reinterpret_cast<const uint4*>(xs + r * kOutRow + ch * 16u);
        }
    } else {
        for (uint32_t r = threadIdx.x / kChunks; r < BM; r += kRowsPerPass) {
            const uint32_t row = m0 + r;
            if (row >= p.m) continue;
            for (uint32_t c = 0; c < 8u; ++c)
                if (col0 + c < sv.n)
                    sv.y[static_cast<size_t>(row) * sv.n + col0 + c] =
                        *reinterpret_cast<const uint16_t*>(xs + r * kOutRow + ch * 16u + c * 2u);
        }
    }
}

// ---- group-step variant: 256-row tiles, one group (64 k) per iteration ---------------
//
// The same scheme with 16 row tiles per wave (each dequantized B fragment feeds 16 MFMAs
// instead of 8) and 64-k iterations, so two workgroups still fit a CU: X stages of
// 256 rows x 128 bytes (chunks swizzled by row % 16, see g_read_a), double buffered; the raw weights of
// a group are half of each 16-byte entry (plus its scale word), loaded two groups ahead.
// k-step s of a group uses word 2 kb + s of the lane's entry, and the A fragments the
// same k chunk.

constexpr uint32_t kGRowBytes = 128u;   // one group of one X row
// Waves of the group-step kernel's workgroup: each wave owns 16 NT columns, so the
// workgroup tile is 256 x (16 NT W); the W waves share one X stage.
constexpr int kGroupWaves = 8;

template <int NT>
struct GRaw {
    uint2 c[NT];       // words 2 kb, 2 kb + 1 of the group
    uint32_t sb[NT];   // scale | bias << 16 of the group
};

template <int NT, typename R>
__device__ __forceinline__ void load_graw(const R& wr, const uint32_t (&c_off)[NT], const uint32_t (&s_off)[NT],
                                          uint32_t g, GRaw<NT>& raw) {
    const uint32_t pair = g >> 1;
    const uint32_t h = g & 1u;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        raw.c[nt] = __builtin_bit_cast(
            uint2, __builtin_amdgcn_raw_buffer_load_b64(wr.c[nt & 1], c_off[nt], pair * 1024u + h * 8u, 0));
        raw.sb[nt] = __builtin_amdgcn_raw_buffer_load_b32(wr.s[nt & 1], s_off[nt], pair * 128u + h * 4u, 0);
    }
}

template <int NT, int S>
__device__ __forceinline__ void gdequant(const GRaw<NT>& raw, bf16x8_t (&b)[NT]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float sc = bf16_bits_to_f32(raw.sb[nt] & 0xFFFFu);
        const float bi = bf16_bits_to_f32(raw.sb[nt] >> 16);
        b[nt] = dequant_word(S == 0 ? raw.c[nt].x : raw.c[nt].y, sc, bi);
    }
}

// Column tile NTI's B fragment of k-step S (gdequant for one tile).
template <int NT, int S, int NTI>
__device__ __forceinline__ void gdequant_one(const GRaw<NT>& raw, bf16x8_t (&b)[NT]) {
    const float sc = bf16_bits_to_f32(raw.sb[NTI] & 0xFFFFu);
    const float bi = bf16_bits_to_f32(raw.sb[NTI] >> 16);
    b[NTI] = dequant_word(S == 0 ? raw.c[NTI].x : raw.c[NTI].y, sc, bi);
}

// f(integral_constant<int, U>) for U in the sequence, in order.
template <typename F, int... U>
__device__ __forceinline__ void static_for(F&& f, std::integer_sequence<int, U...>) {
    (f(std::integral_constant<int, U>{}), ...);
}

// A fragments of k-step S, row tiles [Q MT/P, (Q + 1) MT/P), from an X stage. Rows are
// 128 bytes; logical chunk c of row r sits at chunk c ^ swz(r % 16), swz(i) = (i ^ (i / 8))
// % 8. Measured on gfx950 with ds_read_b128 in this lane pattern (lane (i, kb) reads row
// i): zero bank conflicts and 167 B/clk per CU, against 2-way conflicts (107 B/clk) for
// both i % 8 and (i / 2) % 8.
template <int MT, int P, int S, int Q>
__device__ __forceinline__ void g_read_a(const uint8_t* xb, uint32_t lane, bf16x8_t (&a)[MT / P]) {
    const uint32_t i = lane & 15u;
    const uint32_t kb = lane >> 4;
    const uint32_t c = 2u * kb + S;   // this lane's logical k chunk of the group
    const uint8_t* row = xb + i * kGRowBytes + ((c ^ ((i ^ (i >> 3)) & 7u)) << 4);
#pragma unroll
    for (int mt = 0; mt < MT / P; ++mt)
        a[mt] = *reinterpret_cast<const bf16x8_t*>(row + (Q * (MT / P) + mt) * 16u * kGRowBytes);
}

// The MFMAs of one part of a k-step (MT/P row tiles x NT column tiles), with the
// scheduling hint: the next part's A reads (issued just before) go first, then one MFMA
// followed by kValu VALU ops (the dequantization of the next k-step) throughout.
template <int MT, int NT, int P, int Q, int kValu>
__device__ __forceinline__ void g_mfma_part(const bf16x8_t (&a)[MT / P], const bf16x8_t (&b)[NT],
                                            f32x4_t (&acc)[MT][NT], bool reads_ahead) {
    constexpr int kRows = MT / P;
#pragma unroll
    for (int mt = 0; mt < kRows; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
            acc[Q * kRows + mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt], b[nt], acc[Q * kRows + mt][nt], 0, 0, 0);
    if (reads_ahead) __builtin_amdgcn_sched_group_barrier(0x100, kRows, 0);   // DS read
#pragma unroll
    for (int t = 0; t < kRows * NT; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                 // MFMA
        if constexpr (kValu > 0) __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);   // VALU
    }
}

// Groups between barriers of the group-step kernel: its X ring holds 2 of them stages of
// 16 MT rows x 128 B (128 KB for both tile heights).
template <int MT>
constexpr uint32_t g_sync_groups() { return MT >= 16 ? 2u : 4u; }

template <int MT, int NT, int W>
constexpr size_t g_lds_bytes() {
    return 2u * g_sync_groups<MT>() * 16u * MT * kGRowBytes > 16u * MT * (32u * NT * W + 32u)
               ? 2u * g_sync_groups<MT>() * 16u * MT * kGRowBytes
               : 16u * MT * (32u * NT * W + 32u);
}

// A DUAL launch keeps its GELU table past the X ring.
template <int MT, int NT, int W, bool DUAL>
constexpr size_t g_lds_total() { return g_lds_bytes<MT, NT, W>() + (DUAL ? kGeluTableBytes : 0u); }

template <int MT, int NT, int W, bool DUAL>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2))) void q4_gemm_g_kernel(GemmParams p) {
    static_assert(!DUAL || NT == 2, "a dual launch pairs one gate and one up tile per wave");
    constexpr int kOut = DUAL ? 1 : NT;   // output column tiles per wave
    constexpr uint32_t BM = 16u * MT;
    constexpr uint32_t kStage = BM * kGRowBytes;
    constexpr uint32_t kSync = g_sync_groups<MT>();   // groups per barrier; X ring of 2 kSync stages
    constexpr uint32_t kRing = 2u * kSync - 1u;
    constexpr int kXLoads = static_cast<int>(BM / 8u / W);   // 1 KB (8 rows) direct loads per wave
    static_assert(kXLoads % 2 == 0, "swizzle period");
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];   // [2 kSync][BM][128 B], reused by the epilogue

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const uint32_t bid = blockIdx.x;
    const uint32_t xcd = bid & 7u;
    const uint32_t slot = bid >> 3;
    const uint32_t ext_total = p.tiles_total * p.ksplit;
    const uint32_t per = ext_total >> 3;
    const uint32_t rem = ext_total & 7u;
    const uint32_t ext = xcd * per + min(xcd, rem) + slot;
    const uint32_t kz = ext / p.tiles_total;          // this workgroup's k split
    const uint32_t tile = ext - kz * p.tiles_total;
    const uint32_t tm = tile / p.tiles_n;
    const SegView sv = view_of<DUAL>(p, tile - tm * p.tiles_n);
    const uint32_t m0 = tm * BM;
    const uint32_t n0 = sv.tn * (W * 16u * kOut);
    const uint32_t tile16_0 = n0 / 16u + wave * kOut;
    const uint32_t k = p.k;
    // This workgroup's groups [g0, g1): whole pairs of its split (all groups without split k).
    const uint32_t g0 = 2u * kz * p.pairs_per_split;
    const uint32_t g1 = min(g0 + 2u * p.pairs_per_split, k / 64u);

    // X: load t of wave w fills LDS rows 8 (w kXLoads + t) .. +7; lane l writes physical
    // chunk l % 8 of row r = 8 (w kXLoads + t) + l / 8 with logical chunk
    // (l % 8) ^ swz(r % 16) = (l % 8) ^ (l / 8) ^ (t % 2) (kXLoads is even, so
    // r % 16 = 8 (t % 2) + l / 8).
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.x), static_cast<short>(0), static_cast<int>(p.m * k * 2u), 0x00020000);
    uint32_t xoff[kXLoads];
#pragma unroll
    for (int t = 0; t < kXLoads; ++t) {
        const uint32_t row = m0 + 8u * (wave * kXLoads + t) + (lane >> 3);
        const uint32_t chunk = (lane & 7u) ^ (lane >> 3) ^ static_cast<uint32_t>(t & 1);
        xoff[t] = row < p.m ? row * k * 2u + chunk * 16u : 0x80000000u;
    }
    auto load_x = [&](uint32_t g, uint8_t* buf) {
#pragma unroll
        for (int t = 0; t < kXLoads; ++t)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void*)(buf + (wave * kXLoads + t) * 1024u), 16,
                static_cast<int>(xoff[t]), static_cast<int>(g * 128u), 0, 0);
    };

    const WeightRsrc wr = weight_rsrc<DUAL>(p, sv);
    uint32_t c_off[NT];
    uint32_t s_off[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t t16 = min(tile16_0 + (DUAL ? 0u : static_cast<uint32_t>(nt)), sv.row_tiles - 1u);
        c_off[nt] = (t16 * p.pairs * 64u + lane) * 16u;
        s_off[nt] = (t16 * p.pairs * 16u + (lane & 15u)) * 8u;
    }

    f32x4_t acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    GRaw<NT> r[3];
#pragma unroll
    for (uint32_t i = 0; i < kSync; ++i) load_x(min(g0 + i, g1 - 1u), xs + i * kStage);
    load_graw<NT>(wr, c_off, s_off, g0, r[0]);
    load_graw<NT>(wr, c_off, s_off, min(g0 + 1u, g1 - 1u), r[1]);
    // A DUAL epilogue's GELU table (past the X ring) is computed while the first loads are
    // in flight, instead of after the last MFMA (256-row tile at m = 2048: 7 chains per
    // thread per tile, about 4 tiles per compute unit).
    uint16_t* tab = reinterpret_cast<uint16_t*>(xs + g_lds_bytes<MT, NT, W>());
    if constexpr (DUAL) {
        if (p.ksplit == 1u) build_gelu_table(tab, tid, 64u * W);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    bf16x8_t b0[NT], b1[NT];
    gdequant<NT, 0>(r[0], b0);

    // Each group runs as 2 kParts units (k-step 0 row tiles [0, MT/kParts), then the next
    // MT/kParts, ..., then k-step 1); a unit's A fragments are read from LDS while the
    // previous unit's MFMAs run (two register sets), and the dequantization of the next
    // k-step (or the next group's first) is spread over a k-step's MFMAs. The raw weights
    // of groups g, g + 1 are in r[s], r[(s + 1) % 3] and those of g + 2 load into
    // r[(s + 2) % 3] (s = (g - g0) % 3, unrolled, so no register copies wait on loads in
    // flight). Past the last group the loads repeat the last group (unused).
    //
    // X of group g sits in ring stage (g - g0) % (2 kSync) and is loaded kSync groups ahead;
    // a barrier ends every kSync-th group. Any kSync consecutive groups hold one barrier,
    // so a stage is complete and visible (its wave's vmcnt wait, then the barrier) before
    // its group starts, and every wave has left group g before stage (g - g0) % (2 kSync)
    // is loaded again for group g + 2 kSync. Fewer barriers let the waves drift apart and
    // overlap each other's MFMA and dequantization work.
    // Units per k-step: 8 (2 row tiles each) for the 256-row tile, 2 (4 row tiles each)
    // for the 128-row one. Measured on random data against 4 units: gate at m = 2048
    // 231-234 -> 221-225 us with 8; gate at m = 512 70.5 -> 67.3 us and o at m = 2048
    // 72.9 -> 69.3 us with 2 (8 made the 128-row kernel 1-2% slower).
    constexpr int kParts = MT >= 16 ? 8 : 2;
    static_assert(NT <= kParts, "one column tile's dequantization per unit");
    constexpr int kValu = (26 + MT / kParts * NT - 1) / (MT / kParts * NT);   // one tile's dequantization per MFMA
    bf16x8_t a[2][MT / kParts];
    g_read_a<MT, kParts, 0, 0>(xs, lane, a[0]);
    auto group = [&](auto slot, auto sync, uint32_t g) {
        constexpr int s = decltype(slot)::value;
        const uint8_t* xb = xs + ((g - g0) & kRing) * kStage;
        load_x(min(g + kSync, g1 - 1u), xs + ((g - g0 + kSync) & kRing) * kStage);
        __builtin_amdgcn_sched_barrier(0);   // the raw loads below issue after the X loads
        load_graw<NT>(wr, c_off, s_off, min(g + 2u, g1 - 1u), r[(s + 2) % 3]);
        static_for(
            [&](auto uc) {
                constexpr int u = decltype(uc)::value;
                constexpr int q = u % kParts;
                // Each unit is its own scheduling region: the next unit's A reads go out
                // first, then this unit's MFMAs with one column tile's dequantization.
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (u + 1 < 2 * kParts)
                    g_read_a<MT, kParts, (u + 1) / kParts, (u + 1) % kParts>(xb, lane, a[(u + 1) & 1]);
                if constexpr (u < NT) gdequant_one<NT, 1, u>(r[s], b1);
                if constexpr (u >= kParts && u < kParts + NT) gdequant_one<NT, 0, u - kParts>(r[(s + 1) % 3], b0);
                constexpr bool deq = u < NT || (u >= kParts && u < kParts + NT);
                if constexpr (u < kParts)
                    g_mfma_part<MT, NT, kParts, q, deq ? kValu : 0>(a[u & 1], b0, acc, true);
                else
                    g_mfma_part<MT, NT, kParts, q, deq ? kValu : 0>(a[u & 1], b1, acc, u + 1 < 2 * kParts);
            },
            std::make_integer_sequence<int, 2 * kParts>{});
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(sync)::value) {
            // The X stages of the next two groups have landed once at most this group's
            // 2 NT raw loads remain.
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NT) : "memory");
            __syncthreads();
        }
        g_read_a<MT, kParts, 0, 0>(xs + ((g - g0 + 1u) & kRing) * kStage, lane, a[0]);
    };
    // Unrolled by 3 kSync groups, so the raw-weight slot and the barrier are compile-time.
    constexpr int kUnroll = 3 * static_cast<int>(kSync);
    auto step = [&](auto jc, uint32_t gj) {
        constexpr int j = decltype(jc)::value;
        group(std::integral_constant<int, j % 3>{},
              std::integral_constant<bool, j % static_cast<int>(kSync) == static_cast<int>(kSync) - 1>{}, gj);
    };
    uint32_t g = g0;
    for (; g + kUnroll <= g1; g += kUnroll)
        static_for([&](auto jc) { step(jc, g + decltype(jc)::value); }, std::make_integer_sequence<int, kUnroll>{});
    static_for(
        [&](auto jc) {
            if (g + decltype(jc)::value < g1) step(jc, g + decltype(jc)::value);
        },
        std::make_integer_sequence<int, kUnroll - 1>{});
    // X loads of the last groups may still be in flight; they write LDS the epilogue reuses.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    if (p.ksplit > 1u) {
        store_partials<MT, NT, kOut, DUAL>(p, sv, kz, m0, n0, wave, lane, acc);
        return;
    }

    // Epilogue through LDS as in q4_gemm_kernel (rows of 32 kOut W bytes plus 32 of padding).
    constexpr uint32_t kOutRow = 32u * kOut * W + 32u;
    static_assert(BM * kOutRow <= g_lds_bytes<MT, NT, W>(), "output staging exceeds the X ring");
    __syncthreads();
    stage_out<MT, NT, kOut, DUAL>(xs, kOutRow, wave, lane, acc, tab);
    __syncthreads();
    constexpr uint32_t kChunks = 16u * kOut * W / 8u;
    constexpr uint32_t kRowsPerPass = 64u * W / kChunks;
    const uint32_t ch = threadIdx.x % kChunks;
    const uint32_t col0 = n0 + ch * 8u;
    if ((sv.n & 7u) == 0u && (reinterpret_cast<uintptr_t>(sv.y) & 15u) == 0u) {
        for (uint32_t r = threadIdx.x / kChunks; r < BM; r += kRowsPerPass) {
            const uint32_t row = m0 + r;
            if (row < p.m && col0 < sv.n)
                *reinterpret_cast<uint4*>(sv.y + static_cast<size_t>(row) * sv.n + col0) =
                    *reinterpret_cast<const uint4*>(xs + r * kOutRow + ch * 16u);
        }
    } else {
        for (uint32_t r = threadIdx.x / kChunks; r < BM; r += kRowsPerPass) {
            const uint32_t row = m0 + r;
            if (row >= p.m) continue;
            for (uint32_t c = 0; c < 8u; ++c)
                if (col0 + c < sv.n)
                    sv.y[static_cast<size_t>(row) * sv.n + col0 + c] =
                        *reinterpret_cast<const uint16_t*>(xs + r * kOutRow + ch * 16u + c * 2u);
        }
    }
}


// The same with 8 consecutive workspace columns per thread (two 16-byte loads per split,
// one 16-byte store), for grids where every segment's width and first column are
// multiples of 8 and its output is 16-byte aligned (so 8 columns never straddle two
// segments and each output row segment is 16-byte aligned).
__global__ __launch_bounds__(kThreads) void q4_splitk_reduce8_kernel(GemmParams p) {
    const uint64_t e = (static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x) * 8u;
    const uint64_t total = static_cast<uint64_t>(p.m) * p.n_total;
    if (e >= total) return;
    const uint32_t row = static_cast<uint32_t>(e / p.n_total);
    const uint32_t c = static_cast<uint32_t>(e - static_cast<uint64_t>(row) * p.n_total);
    f32x4_t lo = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4_t hi = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t z = 0; z < p.ksplit; ++z) {
        const f32x4_t* src = reinterpret_cast<const f32x4_t*>(p.partial + z * total + e);
        lo += src[0];
        hi += src[1];
    }
    const bool in1 = p.nseg > 1u && c >= p.seg[1].col_begin;
    const bool in2 = p.nseg > 2u && c >= p.seg[2].col_begin;
    uint16_t* y = in2 ? p.seg[2].y : (in1 ? p.seg[1].y : p.seg[0].y);
    const uint32_t n = in2 ? p.seg[2].n : (in1 ? p.seg[1].n : p.seg[0].n);
    const uint32_t c0 = in2 ? p.seg[2].col_begin : (in1 ? p.seg[1].col_begin : 0u);
    uint4 out;
    out.x = pack_bf16x2(lo[0], lo[1]);
    out.y = pack_bf16x2(lo[2], lo[3]);
    out.z = pack_bf16x2(hi[0], hi[1]);
    out.w = pack_bf16x2(hi[2], hi[3]);
    *reinterpret_cast<uint4*>(y + static_cast<size_t>(row) * n + (c - c0)) = out;
}

// y_seg[row][col] = bf16(sum over splits z = 0, 1, ... of partial[z][row][col_begin + col]),
// one thread per element of the m x n_total workspace row block.
__global__ __launch_bounds__(kThreads) void q4_splitk_reduce_kernel(GemmParams p) {
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(p.m) * p.n_total;
    if (e >= total) return;
    const uint32_t row = static_cast<uint32_t>(e / p.n_total);
    const uint32_t c = static_cast<uint32_t>(e - static_cast<uint64_t>(row) * p.n_total);
    float sum = 0.0f;
    for (uint32_t z = 0; z < p.ksplit; ++z) sum += p.partial[z * total + e];
    const bool in1 = p.nseg > 1u && c >= p.seg[1].col_begin;
    const bool in2 = p.nseg > 2u && c >= p.seg[2].col_begin;
    uint16_t* y = in2 ? p.seg[2].y : (in1 ? p.seg[1].y : p.seg[0].y);
    const uint32_t n = in2 ? p.seg[2].n : (in1 ? p.seg[1].n : p.seg[0].n);
    const uint32_t c0 = in2 ? p.seg[2].col_begin : (in1 ? p.seg[1].col_begin : 0u);
    y[static_cast<size_t>(row) * n + (c - c0)] = f32_to_bf16_bits(sum);
}

// The split-k reduce of a DUAL launch: y[row][col] = gated(sum over z of the gate
// partial at workspace column col, the same of up at column seg[1].col_begin + col), one
// thread per output, the sums in the order of q4_splitk_reduce_kernel.
__global__ __launch_bounds__(kThreads) void q4_splitk_reduce_dual_kernel(GemmParams p) {
    const uint32_t n = p.seg[0].n;
    const uint64_t e = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t outs = static_cast<uint64_t>(p.m) * n;
    if (e >= outs) return;
    const uint32_t row = static_cast<uint32_t>(e / n);
    const uint32_t c = static_cast<uint32_t>(e - static_cast<uint64_t>(row) * n);
    const uint64_t total = static_cast<uint64_t>(p.m) * p.n_total;
    const uint64_t at = static_cast<uint64_t>(row) * p.n_total + c;
    float g = 0.0f;
    float u = 0.0f;
    for (uint32_t z = 0; z < p.ksplit; ++z) {
        g += p.partial[z * total + at];
        u += p.partial[z * total + at + p.seg[1].col_begin];
    }
    p.seg[0].y[static_cast<size_t>(row) * n + c] = gated_bits(g, u);
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

constexpr uint32_t kTileCols = 128u;   // workgroup tile width of the pair-step kernel (NT = 2)

// Column tiles of `tile_cols` output columns: each segment's first global tile and the
// total (a dual launch tiles the gate's columns only; up rides along).
void retile(GemmParams& p, uint32_t tile_cols) {
    if (p.dual != 0u) {
        p.seg[0].tn_begin = 0u;
        p.tiles_n = (p.seg[0].n + tile_cols - 1u) / tile_cols;
        return;
    }
    uint32_t tn = 0;
    for (uint32_t i = 0; i < p.nseg; ++i) {
        p.seg[i].tn_begin = tn;
        tn += (p.seg[i].n + tile_cols - 1u) / tile_cols;
    }
    p.tiles_n = tn;
}

template <int MT, int NT, bool DUAL>
void launch_t(GemmParams p, hipStream_t stream) {
    retile(p, kWaves * 16u * (DUAL ? 1u : NT));
    const bool odd = ((p.k / 64u) & 1u) != 0u;
    auto kernel = odd ? q4_gemm_kernel<MT, NT, true, DUAL> : q4_gemm_kernel<MT, NT, false, DUAL>;
    const size_t lds = 2u * 16u * MT * kRowBytes;
    HYP_REQUIRE(lds <= max_lds_per_block(), HYP_STATUS_INTERNAL, "gemm: X tiles exceed the device's LDS");
    if (lds > 65536u) {
        static thread_local int configured_device = -1;
        int dev = 0;
        HYP_HIP_CHECK(hipGetDevice(&dev));
        if (configured_device != dev) {
            HYP_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(q4_gemm_kernel<MT, NT, true, DUAL>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
            HYP_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(q4_gemm_kernel<MT, NT, false, DUAL>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
            configured_device = dev;
        }
    }
    const uint32_t tiles_m = (p.m + 16u * MT - 1u) / (16u * MT);
    p.tiles_total = p.tiles_n * tiles_m;
    hipLaunchKernelGGL(kernel, dim3(p.tiles_total * p.ksplit), dim3(kThreads), lds, stream, p);
}

template <int MT, int NT, int W, bool DUAL>
void launch_g(GemmParams p, hipStream_t stream) {
    retile(p, 16u * (DUAL ? 1u : NT) * W);
    auto kernel = q4_gemm_g_kernel<MT, NT, W, DUAL>;
    constexpr size_t lds = g_lds_total<MT, NT, W, DUAL>();
    HYP_REQUIRE(lds <= max_lds_per_block(), HYP_STATUS_INTERNAL, "gemm: X tiles exceed the device's LDS");
    if (lds > 65536u) {
        static thread_local int configured_device = -1;
        int dev = 0;
        HYP_HIP_CHECK(hipGetDevice(&dev));
        if (configured_device != dev) {
            HYP_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
            configured_device = dev;
        }
    }
    const uint32_t tiles_m = (p.m + 16u * MT - 1u) / (16u * MT);
    p.tiles_total = p.tiles_n * tiles_m;
    hipLaunchKernelGGL(kernel, dim3(p.tiles_total * p.ksplit), dim3(64 * W), lds, stream, p);
}

// Parameters of a grouped launch; tiles_total is set by the launcher of the chosen kernel.
GemmParams group_params(const Q4Matrix* const* ws, uint16_t* const* ys, uint32_t count, const uint16_t* x,
                        uint32_t m) {
    HYP_REQUIRE(count >= 1u && count <= kMaxGemmSegments, HYP_STATUS_INTERNAL, "gemm: bad group size");
    const uint32_t k = ws[0]->k;
    HYP_REQUIRE(static_cast<uint64_t>(m) * k * 2u < (1ull << 31), HYP_STATUS_INVALID_ARGUMENT,
                "gemm: x is 2 GiB or larger");
    GemmParams p{};
    uint32_t tn = 0;
    uint32_t n_total = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const Q4Matrix& w = *ws[i];
        HYP_REQUIRE(w.codes != nullptr && w.sb != nullptr, HYP_STATUS_INTERNAL,
                    "gemm: weights are not in the tiled resident layout");
        HYP_REQUIRE(w.k == k, HYP_STATUS_INTERNAL, "gemm: grouped projections differ in k");
        const TiledDims d = TiledDims::of(w.n, w.k);
        HYP_REQUIRE(d.code_bytes() < (1ull << 31), HYP_STATUS_INVALID_ARGUMENT, "gemm: weights of 2 GiB or more");
        p.seg[i] = GemmSegment{w.codes, w.sb, ys[i], w.n, d.tiles, static_cast<uint32_t>(d.code_bytes()),
                               static_cast<uint32_t>(d.sb_bytes()), tn, n_total};
        tn += (w.n + kTileCols - 1u) / kTileCols;
        n_total += w.n;
    }
    p.nseg = count;
    p.x = x;
    p.m = m;
    p.k = k;
    p.pairs = TiledDims::of(16u, k).pairs;
    p.tiles_n = tn;
    p.ksplit = 1u;
    p.pairs_per_split = p.pairs;
    p.n_total = n_total;
    p.partial = nullptr;
    p.dual = 0u;
    return p;
}

// The three GEMM kernels by workgroup tile.
enum class GemmKernel : uint32_t {
    kPair128 = 0,    // q4_gemm_kernel<8, 2>: 128 x 128, pair step, two workgroups per CU
    kGroup128 = 1,   // q4_gemm_g_kernel<8, 2, 8>: 128 x 256, group step, one per CU
    kGroup256 = 2,   // q4_gemm_g_kernel<16, 2, 8>: 256 x 256, group step, one per CU
};

struct GemmChoice {
    GemmKernel kernel;
    uint32_t ksplit;
};

template <bool DUAL>
void launch_kernel(GemmParams& p, GemmKernel kernel, hipStream_t stream) {
    switch (kernel) {
        case GemmKernel::kPair128: launch_t<8, 2, DUAL>(p, stream); break;
        case GemmKernel::kGroup128: launch_g<8, 2, kGroupWaves, DUAL>(p, stream); break;
        case GemmKernel::kGroup256: launch_g<16, 2, kGroupWaves, DUAL>(p, stream); break;
        default: throw NativeError(HYP_STATUS_INTERNAL, "gemm: unsupported kernel");
    }
}

void launch_params(GemmParams& p, GemmKernel kernel, hipStream_t stream) {
    if (p.dual != 0u) {
        launch_kernel<true>(p, kernel, stream);
    } else {
        launch_kernel<false>(p, kernel, stream);
    }
    HYP_HIP_CHECK(hipGetLastError());
}

// Workgroups of one k split: (rows / tile rows) x (column tiles over the segments).
uint64_t gemm_tiles(const GemmParams& p, uint32_t rows, uint32_t cols) {
    uint64_t tn = 0;
    for (uint32_t i = 0; i < p.nseg; ++i) tn += (p.seg[i].n + cols - 1u) / cols;
    return static_cast<uint64_t>((p.m + rows - 1u) / rows) * tn;
}

// Smallest split (<= 4, at least 6 pairs in each) whose grid of `tiles` x split reaches
// 90% of the CUs.
uint32_t fill_split(const GemmParams& p, uint64_t tiles, uint64_t cus) {
    uint32_t s = 1u;
    while (s < 4u && tiles * s * 10u < cus * 9u && (p.pairs + s) / (s + 1u) >= 6u) ++s;
    return s;
}

// Kernel and split per call. From a sweep of the seven projections and the grouped q/k/v
// at m = 512, 1024 and 2048 on seeded random data (all three kernels, 1-4 splits), these
// rules pick the fastest configuration or one within 5% of it:
//  * the 256 x 256 kernel when its grid fills 90% of the CUs (gate/up at m >= 1024, the
//    grouped q/k/v at 2048), or does so split when k is long (down at m = 1024: 4 splits,
//    125 us against 192 on the pair-step kernel; at 2048: 2 splits, 215 against 226);
//  * else the 128 x 256 kernel, split to fill the CUs, when that reaches 60% of them
//    (gate at m = 512: 71 us against 81; o at 2048: 67 against 76);
//  * else the 128 x 128 pair-step kernel, split likewise (k [2048, 3840] at m = 512, 4
//    splits: 33 us against 34-36).
GemmChoice choose_gemm(const GemmParams& p) {
    const uint64_t cus = device_compute_units();
    const uint64_t big = gemm_tiles(p, 256u, 256u);
    if (big * 10u >= cus * 9u) return {GemmKernel::kGroup256, 1u};
    if (p.pairs >= 64u) {
        const uint32_t s = fill_split(p, big, cus);
        if (big * s * 10u >= cus * 9u) return {GemmKernel::kGroup256, s};
    }
    const uint64_t mid = gemm_tiles(p, 128u, 256u);
    const uint32_t s = fill_split(p, mid, cus);
    if (mid * s * 10u >= cus * 6u) return {GemmKernel::kGroup128, s};
    const uint64_t pair = gemm_tiles(p, 128u, 128u);
    return {GemmKernel::kPair128, fill_split(p, pair, cus)};
}

// Where the split-k partials of one call live: a stream-ordered temporary
// (hipMallocAsync / hipFreeAsync around the call), or `fixed`, caller-provided device
// memory of `fixed_bytes` that the call only writes and reads (no allocation).
struct SplitWorkspace {
    float* fixed = nullptr;
    size_t fixed_bytes = 0;
};

void launch_split(GemmParams& p, GemmKernel kernel, uint32_t ksplit, hipStream_t stream,
                  const SplitWorkspace& wsp = SplitWorkspace{}) {
    p.ksplit = ksplit;
    p.pairs_per_split = (p.pairs + ksplit - 1u) / ksplit;
    p.ksplit = (p.pairs + p.pairs_per_split - 1u) / p.pairs_per_split;   // no empty split
    if (p.ksplit == 1u) {
        launch_params(p, kernel, stream);
        return;
    }
    const uint64_t elems = static_cast<uint64_t>(p.m) * p.n_total;
    const uint64_t bytes = elems * p.ksplit * sizeof(float);
    // Every split writes each (row, column) of its partial, so the buffer needs no clearing.
    void* ws = nullptr;
    if (wsp.fixed != nullptr) {
        HYP_REQUIRE(bytes <= wsp.fixed_bytes, HYP_STATUS_INVALID_ARGUMENT,
                    "gemm: this call splits k " + std::to_string(p.ksplit) + " ways and needs " +
                        std::to_string(bytes) + " bytes of partial sums; the no-allocation scratch holds " +
                        std::to_string(wsp.fixed_bytes) + " bytes");
        ws = wsp.fixed;
    } else {
        HYP_HIP_CHECK(hipMallocAsync(&ws, bytes, stream));
    }
    p.partial = static_cast<float*>(ws);
    try {
        launch_params(p, kernel, stream);
        if (p.dual != 0u) {
            const uint64_t outs = static_cast<uint64_t>(p.m) * p.seg[0].n;
            const uint64_t blocks = (outs + kThreads - 1u) / kThreads;
            HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "gemm: output too large");
            hipLaunchKernelGGL(q4_splitk_reduce_dual_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                               stream, p);
        } else {
            bool vec = true;
            for (uint32_t i = 0; i < p.nseg; ++i)
                vec = vec && p.seg[i].n % 8u == 0u && p.seg[i].col_begin % 8u == 0u &&
                      (reinterpret_cast<uintptr_t>(p.seg[i].y) & 15u) == 0u;
            const uint64_t per_thread = vec ? 8u : 1u;
            const uint64_t blocks = (elems / per_thread + kThreads - 1u) / kThreads;
            HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "gemm: output too large");
            hipLaunchKernelGGL(vec ? q4_splitk_reduce8_kernel : q4_splitk_reduce_kernel,
                               dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream, p);
        }
        HYP_HIP_CHECK(hipGetLastError());
    } catch (...) {
        if (wsp.fixed == nullptr) (void)hipFreeAsync(ws, stream);
        throw;
    }
    if (wsp.fixed == nullptr) HYP_HIP_CHECK(hipFreeAsync(ws, stream));
}

// The scratch of launch_q4_gemm_noalloc: split-k partials in a file-scope device array,
// so that path allocates nothing. Each device holds its own copy (64 MiB) from module
// load until the process ends; every call on one device shares it, so calls that
// overlap on one device (e.g. on two streams) race.
constexpr size_t kNoAllocScratchBytes = size_t{64} << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`. The array's name in host code is only a
// host-side stand-in, so the device address is looked up once per device (with that
// device current) and kept; kernels and copies take this pointer, never the name.
float* noalloc_scratch() {
    int dev = 0;
    HYP_HIP_CHECK(hipGetDevice(&dev));
    HYP_REQUIRE(dev >= 0 && dev < kMaxDevices, HYP_STATUS_UNSUPPORTED, "device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        HYP_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        HYP_REQUIRE(ptr != nullptr, HYP_STATUS_INTERNAL, "no device address for the no-allocation scratch");
        g_scratch_ptr[dev] = ptr;
    }
    return static_cast<float*>(g_scratch_ptr[dev]);
}

}  // namespace

void launch_q4_gemm_group(const Q4Matrix* const* ws, uint16_t* const* ys, uint32_t count, const uint16_t* x,
                          uint32_t m, hipStream_t stream) {
    GemmParams p = group_params(ws, ys, count, x, m);
    const GemmChoice c = choose_gemm(p);
    launch_split(p, c.kernel, c.ksplit, stream);
}

void launch_q4_gemm_gate_up(const Q4Matrix& gate, const Q4Matrix& up, const uint16_t* x, uint32_t m, uint16_t* y,
                            hipStream_t stream) {
    HYP_REQUIRE(gate.n == up.n && gate.k == up.k, HYP_STATUS_INVALID_ARGUMENT, "gate and up must have the same shape");
    const Q4Matrix* ws[2] = {&gate, &up};
    uint16_t* ys[2] = {y, nullptr};
    GemmParams p = group_params(ws, ys, 2u, x, m);
    const GemmChoice c = choose_gemm(p);   // the kernel and split of the grouped gate/up launch
    p.dual = 1u;
    launch_split(p, c.kernel, c.ksplit, stream);
}

void launch_q4_gemm(const Q4Matrix& w, const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream) {
    const Q4Matrix* ws[1] = {&w};
    uint16_t* ys[1] = {y};
    launch_q4_gemm_group(ws, ys, 1u, x, m, stream);
}

void launch_q4_gemm_noalloc(const Q4Matrix& w, const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream) {
    const Q4Matrix* ws[1] = {&w};
    uint16_t* ys[1] = {y};
    GemmParams p = group_params(ws, ys, 1u, x, m);
    const GemmChoice c = choose_gemm(p);   // the same kernel and split as launch_q4_gemm
    SplitWorkspace wsp;
    wsp.fixed = noalloc_scratch();
    wsp.fixed_bytes = kNoAllocScratchBytes;
    launch_split(p, c.kernel, c.ksplit, stream, wsp);
}

}  // namespace hyperion::hip

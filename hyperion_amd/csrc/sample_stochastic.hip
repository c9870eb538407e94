// Temperature sampling on the device: ForwardPass::sample_stochastic
// (native/hyperion_mlx/src/forward.cc:192-310) without the host copy of the logits.
//
// The reference scales the last row of logits by 1/temperature, takes the softmax, masks to
// -inf the tokens outside the top-p nucleus (by probability, descending), below min_p times
// the largest probability, and outside the top-k (by scaled logit, descending), then draws
// u = uniform_real_distribution<float>(0, sz) from std::mt19937_64 and returns the first index
// whose running sum of the kept exp(t - max) reaches u. The reference sets a statistical bar
// for this path (hyperion_mlx.h:125-140); its host sums and std::sort tie order are not
// reproducible across C++ libraries, so the orders here are defined:
//
//  * The logits are bf16, so t = bf16 value * (1/temperature) and the softmax weight are
//    functions of the 16 bits: tokens are binned by value (65536 bins, bin 0 the largest
//    value; -0 counts as +0; -inf, +inf and NaN get no bin). Every filter keeps a prefix of
//    the order (value descending, index ascending): the nucleus by probability, min-p by a
//    probability threshold and top-k by value are all monotonic in the value, and equal
//    values are taken lowest index first. The kept set is the shortest of the three
//    prefixes, cut inside one bin after c tokens.
//  * Rows the reference's arithmetic does not carry through: where a scaled logit is +inf
//    or NaN (a +inf or NaN logit, 1/temperature NaN, -inf times 1/temperature 0, or the
//    largest value times 1/temperature overflowing) its draw total is NaN, no running sum
//    reaches u and it returns the last index; here too. Where no scaled logit is finite and none of those is
//    present (every logit -inf, or 1/temperature +inf over negative values) its draw total
//    is 0, u = 0 and it returns index 0; here too.
//  * exp is det_exp below, the same float operations as the oracle's restatement, so the two
//    give the same bits. Sums run in defined orders. The cut, over 1024 blocks of 64 bins
//    (wave w of 16 taking blocks 16 i + w): z = the 16 waves' sums in order, each adding in
//    order the 64-lane butterflies of count * e over its blocks; the probability mass before
//    a bin = its block's start (the blocks' masses, each a Hillis-Steele scan over its bins,
//    scanned in block order: within waves of 64 blocks, plus the earlier waves' totals in
//    order) + the scan of its block's masses before it. The draw: the row is cut into chunks of 256 tokens, a wave each, lane l holding
//    tokens 4l..4l+3; a lane sums its kept weights in token order, a Hillis-Steele scan over
//    the 64 lanes gives each lane's running sum before it and the chunk total; the chunk
//    totals are scanned the same way in groups of 64 chunks, the group totals added in order;
//    the running sum at a token is chunk start + (lanes before + the lane's sum so far).
//  * The uniform in [0, 1) is std::generate_canonical<float> of std::mt19937_64 (the host
//    computes it from the request's RNG state, as the reference's uniform_real_distribution
//    does under libstdc++), and u = sz * it, sz the kept total.
//
// Seven launches per row, each of them short: a histogram (per workgroup in LDS, two 16-bit
// counts per word, then added to the global bins; +inf/NaN and -inf logits set bits of a flag
// word); one workgroup that reads the bins into LDS, decides the cut and clears them; then, one wave per
// chunk, the cut bin's tokens per chunk (only when the cut falls inside a bin: its first
// tokens in index order are kept), each chunk's kept total, one workgroup scanning the chunk
// totals, one wave per chunk finding its first token whose running sum reaches u (the lowest
// over the row by an atomic minimum), and one wave writing the token. The top-8 logprob
// sidecar of the pre-filter logits (forward.cc:303-319) is launch_sample_topk's.
//
// Workspace: bins [65536] uint32, the flag word and the totals of the 1024 blocks of 64 bins
// (zero between launches: the decision clears them), the decision, the parameters
// (SampleParams), per-chunk cut counts and totals, per-group cut counts, per-chunk starts,
// the draw's result word.
#include <algorithm>
#include <cstdint>

#include "common.h"
#include "kernels.h"

namespace hyperion::hip {
namespace {

constexpr uint32_t kBins = 65536;
constexpr uint32_t kNoBin = kBins;
constexpr uint32_t kNone = 0xFFFFFFFFu;                // no position: above every index and count
constexpr uint32_t kMaxVocab = 1u << 23;
constexpr uint32_t kThreads = 1024;                    // the decision and the chunk scan: one workgroup
constexpr uint32_t kWaves = kThreads / 64u;
constexpr uint32_t kHistThreads = 1024;
constexpr uint32_t kHistSpan = 8192;                   // tokens per histogram workgroup (< 2^16)
constexpr uint32_t kHistLds = kBins / 2u * 4u + 16u;   // 128 KB: two 16-bit counts per word; the flags
constexpr uint32_t kChunk = 256;                       // tokens per chunk: 4 per lane of one wave
constexpr uint32_t kMaxChunks = kMaxVocab / kChunk;    // 32768
constexpr uint32_t kMaxGroups = kMaxChunks / 64u;      // 512 groups of 64 chunks
constexpr uint32_t kChunkWaves = 4;                    // waves (chunks) per workgroup of the chunk kernels
constexpr size_t kBinsBytes = (kBins + 64u) * 4u;      // the bins, the flag word at [kBins], padding
constexpr size_t kDecisionOffset = kBinsBytes;
constexpr size_t kParamsOffset = kDecisionOffset + 256u;
constexpr size_t kParamsBytes = ((sizeof(SampleParams) + 255u) / 256u) * 256u;
constexpr size_t kCutCountOffset = kParamsOffset + kParamsBytes;          // uint32 [kMaxChunks]
constexpr size_t kGroupCountOffset = kCutCountOffset + kMaxChunks * 4u;   // uint32 [kMaxGroups]
constexpr size_t kTotalOffset = kGroupCountOffset + kMaxGroups * 4u;      // float [kMaxChunks]
constexpr size_t kStartOffset = kTotalOffset + kMaxChunks * 4u;           // float [kMaxChunks]
constexpr size_t kResultOffset = kStartOffset + kMaxChunks * 4u;          // uint32 (+ padding)
constexpr size_t kBlockTotalOffset = kResultOffset + 256u;                // uint32 [kBins / 64]
constexpr size_t kWorkspaceBytes = kBlockTotalOffset + (kBins / 64u) * 4u;

enum : uint32_t { kDrawKept = 0u, kDrawFirst = 1u, kDrawLast = 2u };
enum : uint32_t { kFlagInfNan = 1u, kFlagNegInf = 2u };   // bits of the flag word

// The decision of the second launch, read by the later ones.
struct StochDecision {
    float max_t;         // t of the largest finite value
    uint32_t cut_bin;    // bins < cut_bin are kept whole
    uint32_t cut_count;  // and the first cut_count tokens (index order) of bin cut_bin
    uint32_t mode;       // kDrawKept, or a row drawn without weights: index 0 or the last
    uint32_t partial;    // cut_count is below the cut bin's token count (ranks are needed)
    float u;             // the draw's target, sz * uniform (written by the chunk scan)
    float sz;            // the kept total
};

struct ChunkArrays {
    uint32_t* cut_count;   // [chunks] tokens of the cut bin per chunk
    uint32_t* group_count; // [groups] the same per group of 64 chunks
    float* total;          // [chunks] kept total per chunk
    float* start;          // [chunks] running sum before each chunk
    uint32_t* result;      // the lowest drawn index (atomic minimum)
};

ChunkArrays chunk_arrays(void* workspace) {
    uint8_t* b = static_cast<uint8_t*>(workspace);
    return ChunkArrays{reinterpret_cast<uint32_t*>(b + kCutCountOffset), reinterpret_cast<uint32_t*>(b + kGroupCountOffset),
                       reinterpret_cast<float*>(b + kTotalOffset), reinterpret_cast<float*>(b + kStartOffset),
                       reinterpret_cast<uint32_t*>(b + kResultOffset)};
}

__device__ __forceinline__ uint32_t bin_of(uint32_t b) {
    b &= 0xFFFFu;
    if (b == 0x8000u) b = 0u;                        // -0 -> +0
    if ((b & 0x7F80u) == 0x7F80u) return kNoBin;     // inf, NaN
    const uint32_t ok = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);   // ascending order image
    return 0xFFFFu - ok;
}

__device__ __forceinline__ float bin_value(uint32_t d) {
    const uint32_t ok = 0xFFFFu - d;
    const uint32_t b = (ok & 0x8000u) ? (ok & 0x7FFFu) : (~ok & 0xFFFFu);
    return __uint_as_float(b << 16);
}

// exp(x) for x <= 0 as a fixed sequence of fp32 operations (no fused multiply-add: the file
// is built with -ffp-contract=off): Cody-Waite reduction by ln 2, a degree-7 Taylor polynomial
// on |r| <= 0.35 (relative error below 2^-24 before rounding), scaling by 2^k. At or below
// -86 (where exp is under 2^-124, so every result stays a normal number) it is 0. exp(0) = 1
// exactly. The oracle restates it.
__device__ __forceinline__ float det_exp(float x) {
    if (!(x > -86.0f)) return 0.0f;
    const float kf = rintf(x * 1.44269502f);
    const float r = (x - kf * 0.693145751953125f) - kf * 1.42860677e-06f;
    float p = 1.98412701e-04f;             // 1/5040
    p = p * r + 1.38888892e-03f;           // 1/720
    p = p * r + 8.33333377e-03f;           // 1/120
    p = p * r + 4.16666679e-02f;           // 1/24
    p = p * r + 1.66666672e-01f;           // 1/6
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const int k = static_cast<int>(kf);    // -124 .. 0
    return p * __uint_as_float(static_cast<uint32_t>(k + 127) << 23);
}

__device__ __forceinline__ float butterfly_sum(float v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v = min(v, static_cast<uint32_t>(__shfl_xor(v, m, 64)));
    return v;
}

// Inclusive Hillis-Steele scan over the 64 lanes: in step d (1, 2, 4, ..., 32) lane l >= d
// adds the value lane l - d held before the step (fp32 addition is commutative, so the
// operand order does not matter).
__device__ __forceinline__ float hs_scan(float v, uint32_t lane) {
#pragma unroll
    for (uint32_t d = 1; d < 64u; d <<= 1) {
        const float y = __shfl_up(v, d, 64);
        if (lane >= d) v = v + y;
    }
    return v;
}

__device__ __forceinline__ uint32_t hs_scan_u(uint32_t v, uint32_t lane) {
#pragma unroll
    for (uint32_t d = 1; d < 64u; d <<= 1) {
        const uint32_t y = __shfl_up(v, d, 64);
        if (lane >= d) v += y;
    }
    return v;
}

// The exclusive value of an inclusive scan: lane l - 1's (0 on lane 0).
__device__ __forceinline__ float exclusive_of(float incl, uint32_t lane) {
    const float y = __shfl_up(incl, 1u, 64);
    return lane == 0u ? 0.0f : y;
}

// Block totals too (blocks of 64 bins): a wave's 64 words cover two blocks, one per half.
__global__ __launch_bounds__(kHistThreads) void stoch_hist_kernel(const uint16_t* __restrict__ logits, uint32_t vocab,
                                                                  uint32_t* __restrict__ bins,
                                                                  uint32_t* __restrict__ block_total) {
    extern __shared__ __attribute__((aligned(16))) uint32_t h[];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    for (uint32_t w = tid; w <= kBins / 2u; w += kHistThreads) h[w] = 0u;   // h[kBins / 2]: the flags
    __syncthreads();
    const uint32_t begin = blockIdx.x * kHistSpan;
    const uint32_t end = min(vocab, begin + kHistSpan);
    for (uint32_t i = begin + tid; i < end; i += kHistThreads) {
        const uint32_t bits = logits[i];
        const uint32_t d = bin_of(bits);
        if (d < kBins) {
            atomicAdd(&h[d >> 1], (d & 1u) ? 0x10000u : 1u);
        } else {
            atomicOr(&h[kBins / 2u], bits == 0xFF80u ? kFlagNegInf : kFlagInfNan);
        }
    }
    __syncthreads();
    for (uint32_t w = tid; w < kBins / 2u; w += kHistThreads) {   // w = 64 j + lane: blocks 2j, 2j + 1
        const uint32_t v = h[w];
        if (v & 0xFFFFu) atomicAdd(&bins[2u * w], v & 0xFFFFu);
        if (v >> 16) atomicAdd(&bins[2u * w + 1u], v >> 16);
        uint32_t t = (v & 0xFFFFu) + (v >> 16);
        if (__any(t != 0u)) {
#pragma unroll
            for (int m = 16; m > 0; m >>= 1) t += __shfl_xor(t, m, 64);   // within each half
            if ((lane & 31u) == 0u && t != 0u) atomicAdd(&block_total[w >> 5], t);
        }
    }
    if (tid == 0u && h[kBins / 2u] != 0u) atomicOr(&bins[kBins], h[kBins / 2u]);
}

// The decision runs over 1024 blocks of 64 bins, lane l of a wave holding bin 64 b + l of
// block b; wave w takes blocks 16 i + w (i = 0..63), so the blocks a row's values occupy
// (usually a few dozen neighbours) spread over all 16 waves. The histogram's block totals
// give each wave the mask of its non-empty blocks, which are the only ones it reads and
// visits; their counts go to LDS as 16-bit values (65535 standing for "read the count from
// device memory", a bin holding 65535 tokens or more).
constexpr uint32_t kBlocks = kBins / 64u;               // 1024
constexpr uint32_t kSat = 0xFFFFu;
constexpr uint32_t kDecideLds = kBins * 2u + 4u * kBlocks * 4u;   // counts, totals, masses, two starts

__device__ __forceinline__ uint32_t block_of(uint32_t i, uint32_t wave) { return kWaves * i + wave; }

// Visit the set bits i of a wave-uniform 64-bit mask in increasing order.
template <typename F>
__device__ __forceinline__ void for_each_block(uint64_t mask, F&& f) {
    while (mask != 0ull) {
        const uint32_t i = static_cast<uint32_t>(__builtin_ctzll(mask));
        mask &= mask - 1ull;
        f(i);
    }
}

__global__ __launch_bounds__(kThreads) void stoch_decide_kernel(uint32_t* __restrict__ bins, uint32_t vocab,
                                                                const SampleParams* __restrict__ prm,
                                                                StochDecision* __restrict__ dec, ChunkArrays ca,
                                                                uint32_t* __restrict__ block_total) {
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    uint16_t* c16 = reinterpret_cast<uint16_t*>(lds);            // [kBins]
    uint32_t* btot = lds + kBins / 2u;                           // [kBlocks] tokens per block
    float* bm = reinterpret_cast<float*>(btot + kBlocks);        // [kBlocks] probability mass per block
    float* bsm = bm + kBlocks;                                   // [kBlocks] mass before each block
    uint32_t* bsc = reinterpret_cast<uint32_t*>(bsm + kBlocks);  // [kBlocks] tokens before each block
    __shared__ float wf[kWaves];
    __shared__ uint32_t wu[kWaves];
    __shared__ uint32_t red;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const float inv_temp = prm->inv_temp;

    // The per-group cut counts start at zero and no token is drawn yet.
    for (uint32_t g = tid; g < kMaxGroups; g += kThreads) ca.group_count[g] = 0u;
    if (tid == 0u) {
        *ca.result = kNone;
        red = kNoBin;
    }
    const uint32_t flags = bins[kBins];
    btot[tid] = block_total[tid];   // kThreads == kBlocks
    bm[tid] = 0.0f;
    __syncthreads();
    const uint64_t active = __ballot(btot[block_of(lane, wave)] != 0u);   // bit i: block 16 i + wave

    // Counts of the non-empty blocks into LDS (a batch of up to 8 blocks' loads in flight),
    // the first non-empty bin.
    uint32_t first = kNoBin;
    {
        uint64_t rest = active;
        while (rest != 0ull) {   // uniform
            uint32_t bi[8];
#pragma unroll
            for (uint32_t j = 0; j < 8u; ++j) {
                bi[j] = rest != 0ull ? static_cast<uint32_t>(__builtin_ctzll(rest)) : 64u;   // 64: none
                rest &= rest - 1ull;   // 0 stays 0
            }
            uint32_t c[8];
#pragma unroll
            for (uint32_t j = 0; j < 8u; ++j) c[j] = bi[j] < 64u ? bins[64u * block_of(bi[j], wave) + lane] : 0u;
#pragma unroll
            for (uint32_t j = 0; j < 8u; ++j) {
                if (bi[j] >= 64u) continue;
                const uint32_t d = 64u * block_of(bi[j], wave) + lane;
                c16[d] = static_cast<uint16_t>(min(c[j], kSat));
                if (c[j] != 0u) first = min(first, d);
            }
        }
    }
    first = wave_min_u(first);
    if (lane == 0u) atomicMin(&red, first);
    __syncthreads();
    const uint32_t top = red;
    const float max_t = top != kNoBin ? bin_value(top) * inv_temp : 0.0f;
    // Rows drawn without weights (uniform branch: every thread sees the same values).
    uint32_t mode = kDrawKept;
    if ((flags & kFlagInfNan) != 0u || ((flags & kFlagNegInf) != 0u && inv_temp == 0.0f) ||
        __builtin_isnan(inv_temp) || __builtin_isnan(max_t) || max_t == __builtin_huge_valf()) {
        mode = kDrawLast;
    } else if (top == kNoBin || max_t == -__builtin_huge_valf()) {
        mode = kDrawFirst;
    }
    auto count_of = [&](uint32_t d) {
        const uint32_t c = c16[d];
        return c == kSat ? bins[d] : c;
    };
    auto weight = [&](uint32_t d) { return det_exp(bin_value(d) * inv_temp - max_t); };
    // Clears the non-empty blocks' bins and totals for the next row (each bin by the lane
    // that read it).
    auto clear_bins = [&]() {
        for_each_block(active, [&](uint32_t i) { bins[64u * block_of(i, wave) + lane] = 0u; });
        block_total[tid] = 0u;
        if (tid == 0u) bins[kBins] = 0u;
    };
    if (mode != kDrawKept) {
        if (tid == 0u) *dec = StochDecision{0.0f, 0u, 0u, mode, 0u, 0.0f, 0.0f};
        clear_bins();
        return;
    }

    // z: per block a butterfly over its 64 bins of count * e, each wave adding its blocks in
    // order (an empty block adds 0), the 16 waves' sums in order.
    float zw = 0.0f;
    for_each_block(active, [&](uint32_t i) {
        const uint32_t d = 64u * block_of(i, wave) + lane;
        const uint32_t c = count_of(d);
        zw = zw + butterfly_sum(c != 0u ? static_cast<float>(c) * weight(d) : 0.0f);
    });
    if (lane == 0u) wf[wave] = zw;
    __syncthreads();
    float z = 0.0f;
    for (uint32_t w = 0; w < kWaves; ++w) z = z + wf[w];
    __syncthreads();   // wf is reused below

    // Each block's probability mass (a scan over its bins, the last lane's value; 0 when empty).
    auto mass = [&](uint32_t d, uint32_t c) { return c != 0u ? static_cast<float>(c) * (weight(d) / z) : 0.0f; };
    for_each_block(active, [&](uint32_t i) {
        const uint32_t b = block_of(i, wave);
        const uint32_t d = 64u * b + lane;
        const float m = hs_scan(mass(d, count_of(d)), lane);
        if (lane == 63u) bm[b] = m;
    });
    __syncthreads();
    // The mass and the tokens before each block, in block order: wave w scans blocks
    // 64 w .. 64 w + 63, the earlier waves' totals added in order.
    {
        const uint32_t b = 64u * wave + lane;
        const float incl = hs_scan(bm[b], lane);
        const float excl = exclusive_of(incl, lane);
        const uint32_t cnt = btot[b];
        const uint32_t uincl = hs_scan_u(cnt, lane);
        if (lane == 63u) {
            wf[wave] = incl;
            wu[wave] = uincl;
        }
        __syncthreads();
        float off = 0.0f;
        uint32_t uoff = 0u;
        for (uint32_t w = 0; w < wave; ++w) {
            off = off + wf[w];
            uoff += wu[w];
        }
        bsm[b] = off + excl;
        bsc[b] = uoff + uincl - cnt;
    }
    uint32_t total = 0u;
    for (uint32_t w = 0; w < kWaves; ++w) total += wu[w];
    if (tid == 0u) red = kNone;
    __syncthreads();

    // top-p: the first position (in the order) whose running mass reaches top_p.
    uint32_t np = total;
    const float top_p = prm->top_p;
    if (top_p > 0.0f && top_p <= 1.0f) {   // uniform
        uint32_t cand = kNone;
        for_each_block(active, [&](uint32_t i) {
            const uint32_t b = block_of(i, wave);
            const uint32_t d = 64u * b + lane;
            const uint32_t c = count_of(d);
            const float cb = bsm[b] + exclusive_of(hs_scan(mass(d, c), lane), lane);
            const uint32_t seen = bsc[b] + hs_scan_u(c, lane) - c;
            if (c != 0u) {
                const float p = weight(d) / z;
                if (cb + static_cast<float>(c) * p >= top_p) {
                    uint32_t lo = 1u, hi = c;   // the smallest t in [1, c] with cb + t p >= top_p
                    while (lo < hi) {
                        const uint32_t mid = (lo + hi) >> 1;
                        if (cb + static_cast<float>(mid) * p >= top_p) hi = mid; else lo = mid + 1u;
                    }
                    cand = min(cand, seen + lo);
                }
            }
        });
        cand = wave_min_u(cand);
        if (lane == 0u) atomicMin(&red, cand);
        __syncthreads();
        if (red != kNone) np = red;
        __syncthreads();   // every thread has read red before it is reused
    }
    // min-p: tokens whose probability is at least min_p times the largest (1/z).
    uint32_t nm = total;
    const float min_p = prm->min_p;
    if (min_p > 0.0f && min_p < 1.0f) {   // uniform
        const float thr = min_p * (1.0f / z);
        uint32_t kept = 0u;
        for_each_block(active, [&](uint32_t i) {
            const uint32_t d = 64u * block_of(i, wave) + lane;
            const uint32_t c = count_of(d);
            if (c != 0u && weight(d) / z >= thr) kept += c;
        });
        kept = wave_sum_u(kept);
        if (tid == 0u) red = 0u;
        __syncthreads();
        if (lane == 0u) atomicAdd(&red, kept);
        __syncthreads();
        nm = red;
    }
    const int32_t top_k = prm->top_k;
    const uint32_t nk = top_k > 0 && static_cast<uint32_t>(top_k) < vocab ? static_cast<uint32_t>(top_k) : total;
    const uint32_t n = min(min(np, nm), min(nk, total));   // >= 1: every filter keeps the top token

    // The bin where the first n tokens end (one lane of one block holds it).
    for_each_block(active, [&](uint32_t i) {
        const uint32_t b = block_of(i, wave);
        if (!(bsc[b] < n && n <= bsc[b] + btot[b])) return;   // uniform
        const uint32_t d = 64u * b + lane;
        const uint32_t c = count_of(d);
        const uint32_t seen = bsc[b] + hs_scan_u(c, lane) - c;
        if (c != 0u && seen < n && n <= seen + c) {
            *dec = StochDecision{max_t, d, n - seen, kDrawKept, n - seen < c ? 1u : 0u, 0.0f, 0.0f};
        }
    });
    clear_bins();
}

// Tokens of the cut bin per chunk (and per group of 64 chunks), when the cut falls inside
// the bin. One wave per chunk.
__global__ __launch_bounds__(64 * kChunkWaves) void stoch_count_kernel(const uint16_t* __restrict__ logits,
                                                                       uint32_t vocab,
                                                                       const StochDecision* __restrict__ dec,
                                                                       ChunkArrays ca) {
    const StochDecision dc = *dec;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c = blockIdx.x * kChunkWaves + (threadIdx.x >> 6);
    if (dc.mode != kDrawKept || dc.partial == 0u || c * kChunk >= vocab) return;   // wave-uniform
    uint32_t n = 0u;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        const uint32_t i = c * kChunk + 4u * lane + k;
        if (i < vocab && bin_of(logits[i]) == dc.cut_bin) ++n;
    }
    n = wave_sum_u(n);
    if (lane == 0u) {
        ca.cut_count[c] = n;
        if (n != 0u) atomicAdd(&ca.group_count[c >> 6], n);
    }
}

// One chunk's tokens as one wave sees them: lane l holds tokens 4l..4l+3; kept[k] and the
// kept weights w[k], and the lane's sum of its kept weights in token order.
struct ChunkLane {
    float w[4];
    bool kept[4];
    float sum;
};

__device__ __forceinline__ ChunkLane chunk_lane(const uint16_t* __restrict__ logits, uint32_t vocab, uint32_t c,
                                                uint32_t lane, const StochDecision& dc, float inv_temp,
                                                const ChunkArrays& ca) {
    uint32_t d[4];
    float x[4];
    uint32_t ncut = 0u;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        const uint32_t i = c * kChunk + 4u * lane + k;
        const uint32_t bits = i < vocab ? logits[i] : 0xFF80u;   // past the row: no token (-inf)
        d[k] = i < vocab ? bin_of(bits) : kNoBin;
        x[k] = __uint_as_float(bits << 16);
        ncut += d[k] == dc.cut_bin ? 1u : 0u;
    }
    // The rank (index order) of this lane's first cut-bin token among the row's cut-bin tokens.
    uint32_t rank = 0u;
    if (dc.partial != 0u) {   // uniform
        const uint32_t g = c >> 6;
        uint32_t before = 0u;
        for (uint32_t j = lane; j < g; j += 64u) before += ca.group_count[j];
        for (uint32_t j = 64u * g + lane; j < c; j += 64u) before += ca.cut_count[j];
        rank = wave_sum_u(before) + hs_scan_u(ncut, lane) - ncut;
    }
    ChunkLane r;
    r.sum = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        const bool cut = d[k] == dc.cut_bin;
        r.kept[k] = d[k] < dc.cut_bin || (cut && (dc.partial == 0u || rank < dc.cut_count));
        rank += cut ? 1u : 0u;
        r.w[k] = r.kept[k] ? det_exp(x[k] * inv_temp - dc.max_t) : 0.0f;
        if (r.kept[k]) r.sum = r.sum + r.w[k];
    }
    return r;
}

__global__ __launch_bounds__(64 * kChunkWaves) void stoch_chunk_kernel(const uint16_t* __restrict__ logits,
                                                                       uint32_t vocab,
                                                                       const SampleParams* __restrict__ prm,
                                                                       const StochDecision* __restrict__ dec,
                                                                       ChunkArrays ca) {
    const StochDecision dc = *dec;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c = blockIdx.x * kChunkWaves + (threadIdx.x >> 6);
    if (dc.mode != kDrawKept || c * kChunk >= vocab) return;   // wave-uniform
    const ChunkLane cl = chunk_lane(logits, vocab, c, lane, dc, prm->inv_temp, ca);
    const float incl = hs_scan(cl.sum, lane);
    if (lane == 63u) ca.total[c] = incl;
}

// The running sum before each chunk: groups of 64 chunks scanned by a wave each, the group
// totals added in order; the kept total sz and u = sz * uniform into the decision.
__global__ __launch_bounds__(kThreads) void stoch_scan_kernel(uint32_t vocab, SampleParams* __restrict__ prm,
                                                              StochDecision* __restrict__ dec, ChunkArrays ca) {
    __shared__ float gt[kMaxGroups];
    __shared__ float gs[kMaxGroups + 1];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    if (dec->mode != kDrawKept) return;   // uniform
    const uint32_t chunks = (vocab + kChunk - 1u) / kChunk;
    const uint32_t groups = (chunks + 63u) / 64u;
    for (uint32_t g = wave; g < groups; g += kWaves) {
        const uint32_t c = 64u * g + lane;
        const float incl = hs_scan(c < chunks ? ca.total[c] : 0.0f, lane);
        const float excl = exclusive_of(incl, lane);
        if (c < chunks) ca.start[c] = excl;
        if (lane == 63u) gt[g] = incl;
    }
    __syncthreads();
    if (tid == 0u) {
        float run = 0.0f;
        for (uint32_t g = 0; g < groups; ++g) {
            gs[g] = run;
            run = run + gt[g];
        }
        gs[groups] = run;
    }
    __syncthreads();
    // Each wave adds its own groups' starts (the lanes that wrote them).
    for (uint32_t g = wave; g < groups; g += kWaves) {
        const uint32_t c = 64u * g + lane;
        if (c < chunks) ca.start[c] = gs[g] + ca.start[c];
    }
    if (tid == 0u) {
        const uint32_t step = prm->step;
        const uint32_t nu = min(max(prm->n_uniform, 1u), kMaxSampledSteps);
        const float canon = prm->uniform[min(step, nu - 1u)];
        const float sz = gs[groups];
        dec->sz = sz;
        dec->u = sz * canon + 0.0f;   // uniform_real_distribution<float>(0, sz)
    }
}

// Each chunk's first kept token whose running sum reaches u; the lowest index over the row.
__global__ __launch_bounds__(64 * kChunkWaves) void stoch_find_kernel(const uint16_t* __restrict__ logits,
                                                                      uint32_t vocab,
                                                                      const SampleParams* __restrict__ prm,
                                                                      const StochDecision* __restrict__ dec,
                                                                      ChunkArrays ca) {
    const StochDecision dc = *dec;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t c = blockIdx.x * kChunkWaves + (threadIdx.x >> 6);
    if (dc.mode != kDrawKept || c * kChunk >= vocab) return;   // wave-uniform
    if (!(dc.u > 0.0f)) {   // u <= 0 (or NaN: no running sum reaches it, the last index)
        if (c == 0u && lane == 0u && dc.u <= 0.0f) atomicMin(ca.result, 0u);
        return;
    }
    const ChunkLane cl = chunk_lane(logits, vocab, c, lane, dc, prm->inv_temp, ca);
    const float incl = hs_scan(cl.sum, lane);
    const float before = exclusive_of(incl, lane);
    const float sc = ca.start[c];
    uint32_t cand = kNone;
    float part = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 4u; ++k) {
        if (!cl.kept[k] || cand != kNone) continue;
        part = part + cl.w[k];
        if (dc.u <= sc + (before + part)) cand = c * kChunk + 4u * lane + k;
    }
    cand = wave_min_u(cand);
    if (lane == 0u && cand != kNone) atomicMin(ca.result, cand);
}

// The drawn token (the reference's fallback, the last index, when no running sum reached u)
// and the next step's uniform.
__global__ __launch_bounds__(64) void stoch_final_kernel(const uint16_t* __restrict__ logits, uint32_t vocab,
                                                         SampleParams* __restrict__ prm,
                                                         const StochDecision* __restrict__ dec, ChunkArrays ca,
                                                         HypTopKSample* __restrict__ out) {
    if (threadIdx.x != 0u) return;
    const StochDecision dc = *dec;
    prm->step = prm->step + 1u;
    uint32_t arg;
    if (dc.mode != kDrawKept || vocab == 0u) {
        arg = dc.mode == kDrawLast && vocab != 0u ? vocab - 1u : 0u;
    } else {
        const uint32_t r = *ca.result;
        arg = r < vocab ? r : vocab - 1u;
    }
    out->token_id = arg;
    out->logit = vocab != 0u ? __uint_as_float(static_cast<uint32_t>(logits[arg]) << 16) : -__builtin_huge_valf();
    out->near_tie = 0u;
    *ca.result = kNone;
}

}  // namespace

size_t sample_stochastic_workspace_bytes() { return kWorkspaceBytes; }

SampleParams* sample_stochastic_params(void* workspace) {
    return reinterpret_cast<SampleParams*>(static_cast<uint8_t*>(workspace) + kParamsOffset);
}

void init_sample_stochastic_workspace(void* workspace, hipStream_t stream) {
    HYP_HIP_CHECK(hipMemsetAsync(workspace, 0, kWorkspaceBytes, stream));
}

namespace {

__global__ void stoch_params_kernel(SampleParams* __restrict__ prm, float inv_temp, float top_p, float min_p,
                                    int32_t top_k, float canon) {
    if (threadIdx.x == 0u) {
        prm->inv_temp = inv_temp;
        prm->top_p = top_p;
        prm->min_p = min_p;
        prm->top_k = top_k;
        prm->n_uniform = 1u;
        prm->step = 0u;
        prm->uniform[0] = canon;
    }
}

}  // namespace

void launch_sample_params(void* workspace, float inv_temp, float top_p, float min_p, int32_t top_k, float canon,
                          hipStream_t stream) {
    hipLaunchKernelGGL(stoch_params_kernel, dim3(1), dim3(64), 0, stream, sample_stochastic_params(workspace),
                       inv_temp, top_p, min_p, top_k, canon);
    HYP_HIP_CHECK(hipGetLastError());
}

void launch_sample_stochastic(const uint16_t* logits, uint32_t vocab, void* workspace, size_t workspace_bytes,
                              HypTopKSample* out, hipStream_t stream) {
    HYP_REQUIRE(workspace != nullptr && workspace_bytes >= kWorkspaceBytes &&
                    (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0u,
                HYP_STATUS_INTERNAL, "sample_stochastic: workspace too small or misaligned");
    HYP_REQUIRE(vocab <= kMaxVocab, HYP_STATUS_INVALID_ARGUMENT, "sample_stochastic: vocab must be at most 2^23");
    uint32_t* bins = static_cast<uint32_t*>(workspace);
    auto* dec = reinterpret_cast<StochDecision*>(static_cast<uint8_t*>(workspace) + kDecisionOffset);
    static_assert(sizeof(StochDecision) <= 256u, "decision slot");
    SampleParams* params = sample_stochastic_params(workspace);
    const ChunkArrays ca = chunk_arrays(workspace);
    uint32_t* block_total = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(workspace) + kBlockTotalOffset);
    static_assert(kThreads == kBins / 64u, "one block total per thread of the decision");
    static thread_local int configured_device = -1;
    int dev = 0;
    HYP_HIP_CHECK(hipGetDevice(&dev));
    if (configured_device != dev) {
        HYP_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(stoch_hist_kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kHistLds)));
        HYP_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(stoch_decide_kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kDecideLds)));
        configured_device = dev;
    }
    if (vocab != 0u) {
        const uint32_t groups = (vocab + kHistSpan - 1u) / kHistSpan;
        hipLaunchKernelGGL(stoch_hist_kernel, dim3(groups), dim3(kHistThreads), kHistLds, stream, logits, vocab, bins,
                           block_total);
        HYP_HIP_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(stoch_decide_kernel, dim3(1), dim3(kThreads), kDecideLds, stream, bins, vocab, params, dec, ca,
                       block_total);
    HYP_HIP_CHECK(hipGetLastError());
    if (vocab != 0u) {
        const uint32_t chunks = (vocab + kChunk - 1u) / kChunk;
        const dim3 grid((chunks + kChunkWaves - 1u) / kChunkWaves);
        hipLaunchKernelGGL(stoch_count_kernel, grid, dim3(64 * kChunkWaves), 0, stream, logits, vocab, dec, ca);
        HYP_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(stoch_chunk_kernel, grid, dim3(64 * kChunkWaves), 0, stream, logits, vocab, params, dec,
                           ca);
        HYP_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(stoch_scan_kernel, dim3(1), dim3(kThreads), 0, stream, vocab, params, dec, ca);
        HYP_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(stoch_find_kernel, grid, dim3(64 * kChunkWaves), 0, stream, logits, vocab, params, dec,
                           ca);
        HYP_HIP_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(stoch_final_kernel, dim3(1), dim3(64), 0, stream, logits, vocab, params, dec, ca, out);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

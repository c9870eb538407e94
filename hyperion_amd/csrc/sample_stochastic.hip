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
//    give the same bits. Sums run in defined orders: z = the sum over 16 waves (in order) of
//    a 64-lane butterfly of per-lane sums over 64 bins (each bin adding count * e); running
//    sums over bins and tokens go chunk by chunk (a sequential sum within a thread's chunk,
//    added to the sequential prefix of the earlier chunks).
//  * The uniform in [0, 1) is std::generate_canonical<float> of std::mt19937_64 (the host
//    computes it from the request's RNG state, as the reference's uniform_real_distribution
//    does under libstdc++), and u = sz * it.
//
// Three launches per row: a histogram (per workgroup in LDS, two 16-bit counts per word,
// then added to the global bins; +inf/NaN and -inf logits set bits of a flag word), one
// workgroup that reads and clears the bins and decides the cut, one workgroup that sums
// the kept weights in index order and draws. The top-8 logprob sidecar of the pre-filter
// logits (forward.cc:303-319) is launch_sample_topk's.
//
// Workspace: bins [65536] uint32 and the flag word (zero between launches: the decision
// clears them), the decision, the parameters (SampleParams).
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
constexpr uint32_t kThreads = 1024;                    // decide and draw: one workgroup
constexpr uint32_t kBinsPerThread = kBins / kThreads;  // 64
constexpr uint32_t kHistThreads = 1024;
constexpr uint32_t kHistSpan = 8192;                   // tokens per histogram workgroup (< 2^16)
constexpr uint32_t kHistLds = kBins / 2u * 4u + 16u;   // 128 KB: two 16-bit counts per word; the flags
constexpr size_t kBinsBytes = (kBins + 64u) * 4u;      // the bins, the flag word at [kBins], padding
constexpr size_t kDecisionOffset = kBinsBytes;
constexpr size_t kParamsOffset = kDecisionOffset + 256u;
constexpr size_t kWorkspaceBytes = kParamsOffset + ((sizeof(SampleParams) + 255u) / 256u) * 256u;

enum : uint32_t { kDrawKept = 0u, kDrawFirst = 1u, kDrawLast = 2u };
enum : uint32_t { kFlagInfNan = 1u, kFlagNegInf = 2u };   // bits of the flag word

// The decision of the second launch, read by the third.
struct StochDecision {
    float max_t;         // t of the largest finite value
    uint32_t cut_bin;    // bins < cut_bin are kept whole
    uint32_t cut_count;  // and the first cut_count tokens (index order) of bin cut_bin
    uint32_t mode;       // kDrawKept, or a row drawn without weights: index 0 or the last
};

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

__global__ __launch_bounds__(kHistThreads) void stoch_hist_kernel(const uint16_t* __restrict__ logits, uint32_t vocab,
                                                                  uint32_t* __restrict__ bins) {
    extern __shared__ __attribute__((aligned(16))) uint32_t h[];
    const uint32_t tid = threadIdx.x;
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
    for (uint32_t w = tid; w < kBins / 2u; w += kHistThreads) {
        const uint32_t v = h[w];
        if (v & 0xFFFFu) atomicAdd(&bins[2u * w], v & 0xFFFFu);
        if (v >> 16) atomicAdd(&bins[2u * w + 1u], v >> 16);
    }
    if (tid == 0u && h[kBins / 2u] != 0u) atomicOr(&bins[kBins], h[kBins / 2u]);
}

// Exclusive prefix of a[0..kThreads) in index order by thread 0 (sequential: the defined
// order of the float sums); a[kThreads] receives the total.
template <typename T>
__device__ __forceinline__ void serial_prefix(T* a, uint32_t tid) {
    __syncthreads();
    if (tid == 0u) {
        T run = T(0);
        for (uint32_t j = 0; j < kThreads; ++j) {
            const T v = a[j];
            a[j] = run;
            run = run + v;
        }
        a[kThreads] = run;
    }
    __syncthreads();
}

// Each thread owns bins [64 tid, 64 tid + 64) and walks them in order once per pass,
// reading them from device memory (a pass holds 4 at a time; they are cleared after the last
// pass for the next row).
template <typename F>
__device__ __forceinline__ void for_each_bin(const uint32_t* bins, uint32_t d0, F&& f) {
    const uint4* b4 = reinterpret_cast<const uint4*>(bins + d0);
    for (uint32_t q = 0; q < kBinsPerThread / 4u; ++q) {
        const uint4 v = b4[q];
        f(d0 + 4u * q, v.x);
        f(d0 + 4u * q + 1u, v.y);
        f(d0 + 4u * q + 2u, v.z);
        f(d0 + 4u * q + 3u, v.w);
    }
}

__global__ __launch_bounds__(kThreads) void stoch_decide_kernel(uint32_t* __restrict__ bins, uint32_t vocab,
                                                                const SampleParams* __restrict__ prm,
                                                                StochDecision* __restrict__ dec) {
    __shared__ float fs[kThreads + 1];
    __shared__ uint32_t us[kThreads + 1];
    __shared__ float wz[kThreads / 64u];
    __shared__ uint32_t red;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t d0 = tid * kBinsPerThread;
    const float inv_temp = prm->inv_temp;

    const uint32_t flags = bins[kBins];
    uint32_t first = kNoBin;
    uint32_t total_l = 0u;
    for_each_bin(bins, d0, [&](uint32_t d, uint32_t c) {
        if (c != 0u && first == kNoBin) first = d;
        total_l += c;
    });
    if (tid == 0u) red = kNoBin;
    __syncthreads();
    atomicMin(&red, first);
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
    if (mode != kDrawKept) {
        __syncthreads();   // every thread has read the flag word
        if (tid == 0u) {
            *dec = StochDecision{0.0f, 0u, 0u, mode};
            bins[kBins] = 0u;
        }
        uint4* b4 = reinterpret_cast<uint4*>(bins + d0);
        for (uint32_t q = 0; q < kBinsPerThread / 4u; ++q) b4[q] = make_uint4(0u, 0u, 0u, 0u);
        return;
    }
    auto weight = [&](uint32_t d) { return det_exp(bin_value(d) * inv_temp - max_t); };

    // z: per-lane sums over the lane's bins, a butterfly per wave, the waves in order.
    float zl = 0.0f;
    for_each_bin(bins, d0, [&](uint32_t d, uint32_t c) {
        if (c != 0u) zl = zl + static_cast<float>(c) * weight(d);
    });
    const float zw = butterfly_sum(zl);
    if (lane == 0u) wz[wave] = zw;
    __syncthreads();
    float z = 0.0f;
    for (uint32_t w = 0; w < kThreads / 64u; ++w) z = z + wz[w];

    // Counts and probability masses before each thread's bins.
    float pl = 0.0f;
    for_each_bin(bins, d0, [&](uint32_t d, uint32_t c) {
        if (c != 0u) pl = pl + static_cast<float>(c) * (weight(d) / z);
    });
    fs[tid] = pl;
    us[tid] = total_l;
    serial_prefix(fs, tid);
    serial_prefix(us, tid);
    const uint32_t total = us[kThreads];
    const uint32_t before = us[tid];

    // top-p: the first position (in the order) whose running mass reaches top_p.
    uint32_t np = total;
    const float top_p = prm->top_p;
    if (top_p > 0.0f && top_p <= 1.0f) {   // uniform
        const float start = fs[tid];
        float part = 0.0f;
        uint32_t seen = before;
        uint32_t cand = kNone;
        for_each_bin(bins, d0, [&](uint32_t d, uint32_t c) {
            if (c == 0u || cand != kNone) return;
            const float p = weight(d) / z;
            const float cb = start + part;
            if (cb + static_cast<float>(c) * p >= top_p) {
                uint32_t lo = 1u, hi = c;   // the smallest t in [1, c] with cb + t p >= top_p
                while (lo < hi) {
                    const uint32_t mid = (lo + hi) >> 1;
                    if (cb + static_cast<float>(mid) * p >= top_p) hi = mid; else lo = mid + 1u;
                }
                cand = seen + lo;
            }
            part = part + static_cast<float>(c) * p;
            seen += c;
        });
        if (tid == 0u) red = kNone;
        __syncthreads();
        atomicMin(&red, cand);
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
        for_each_bin(bins, d0, [&](uint32_t d, uint32_t c) {
            if (c != 0u && weight(d) / z >= thr) kept += c;
        });
        if (tid == 0u) red = 0u;
        __syncthreads();
        atomicAdd(&red, kept);
        __syncthreads();
        nm = red;
    }
    const int32_t top_k = prm->top_k;
    const uint32_t nk = top_k > 0 && static_cast<uint32_t>(top_k) < vocab ? static_cast<uint32_t>(top_k) : total;
    const uint32_t n = min(min(np, nm), min(nk, total));   // >= 1: every filter keeps the top token

    // The bin where the first n tokens end (one thread's range holds it).
    if (before < n && n <= before + total_l) {
        uint32_t seen = before;
        bool done = false;
        for_each_bin(bins, d0, [&](uint32_t d, uint32_t c) {
            if (!done && seen + c >= n) {
                *dec = StochDecision{max_t, d, n - seen, kDrawKept};
                done = true;
            }
            seen += c;
        });
    }
    // Clear this thread's bins for the next row (only this thread reads them; every thread
    // read the flag word before the barriers above).
    if (tid == 0u) bins[kBins] = 0u;
    uint4* b4 = reinterpret_cast<uint4*>(bins + d0);
    for (uint32_t q = 0; q < kBinsPerThread / 4u; ++q) b4[q] = make_uint4(0u, 0u, 0u, 0u);
}

__device__ __forceinline__ float kept_weight(uint32_t d, uint32_t& rank, const StochDecision& dc, float x,
                                             float inv_temp) {
    const bool keep = d < dc.cut_bin || (d == dc.cut_bin && rank++ < dc.cut_count);
    return keep ? det_exp(x * inv_temp - dc.max_t) : -1.0f;
}

__global__ __launch_bounds__(kThreads) void stoch_draw_kernel(const uint16_t* __restrict__ logits, uint32_t vocab,
                                                              SampleParams* __restrict__ prm,
                                                              const StochDecision* __restrict__ dec,
                                                              HypTopKSample* __restrict__ out) {
    __shared__ float fs[kThreads + 1];
    __shared__ uint32_t us[kThreads + 1];
    __shared__ uint32_t red;
    const uint32_t tid = threadIdx.x;
    const StochDecision dc = *dec;
    const uint32_t step = prm->step;
    const uint32_t nu = min(max(prm->n_uniform, 1u), kMaxSampledSteps);
    const float canon = prm->uniform[min(step, nu - 1u)];
    const float inv_temp = prm->inv_temp;
    __syncthreads();
    if (tid == 0u) prm->step = step + 1u;
    if (dc.mode != kDrawKept || vocab == 0u) {
        if (tid == 0u) {
            const uint32_t arg = dc.mode == kDrawLast && vocab != 0u ? vocab - 1u : 0u;
            out->token_id = arg;
            out->logit = vocab != 0u ? __uint_as_float(static_cast<uint32_t>(logits[arg]) << 16) : -__builtin_huge_valf();
            out->near_tie = 0u;
        }
        return;
    }
    const uint32_t chunk = (vocab + kThreads - 1u) / kThreads;
    const uint32_t begin = min(vocab, tid * chunk);
    const uint32_t end = min(vocab, begin + chunk);

    // Ranks of the cut bin's tokens before this chunk.
    uint32_t ncut = 0u;
    for (uint32_t i = begin; i < end; ++i) ncut += bin_of(logits[i]) == dc.cut_bin ? 1u : 0u;
    us[tid] = ncut;
    serial_prefix(us, tid);
    const uint32_t rank0 = us[tid];

    // Kept weight of the chunk in index order, then the prefix over chunks.
    float s = 0.0f;
    uint32_t rank = rank0;
    for (uint32_t i = begin; i < end; ++i) {
        const uint32_t bits = logits[i];
        const float w = kept_weight(bin_of(bits), rank, dc, __uint_as_float(bits << 16), inv_temp);
        if (w >= 0.0f) s = s + w;
    }
    fs[tid] = s;
    serial_prefix(fs, tid);
    const float sz = fs[kThreads];
    const float u = sz * canon + 0.0f;   // uniform_real_distribution<float>(0, sz)

    // The first index whose running sum reaches u.
    uint32_t cand = kNone;   // above any index
    if (u <= 0.0f) {
        cand = 0u;
    } else {
        const float start = fs[tid];
        float part = 0.0f;
        rank = rank0;
        for (uint32_t i = begin; i < end; ++i) {
            const uint32_t bits = logits[i];
            const float w = kept_weight(bin_of(bits), rank, dc, __uint_as_float(bits << 16), inv_temp);
            if (w < 0.0f) continue;
            part = part + w;
            if (u <= start + part) {
                cand = i;
                break;
            }
        }
    }
    if (tid == 0u) red = kNone;
    __syncthreads();
    atomicMin(&red, cand);
    __syncthreads();
    if (tid == 0u) {
        const uint32_t arg = red < vocab ? red : vocab - 1u;   // the reference's fallback: the last index
        out->token_id = arg;
        out->logit = __uint_as_float(static_cast<uint32_t>(logits[arg]) << 16);
        out->near_tie = 0u;
    }
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
    SampleParams* params = sample_stochastic_params(workspace);
    static thread_local int configured_device = -1;
    int dev = 0;
    HYP_HIP_CHECK(hipGetDevice(&dev));
    if (configured_device != dev) {
        HYP_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(stoch_hist_kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kHistLds)));
        configured_device = dev;
    }
    if (vocab != 0u) {
        const uint32_t groups = (vocab + kHistSpan - 1u) / kHistSpan;
        hipLaunchKernelGGL(stoch_hist_kernel, dim3(groups), dim3(kHistThreads), kHistLds, stream, logits, vocab, bins);
        HYP_HIP_CHECK(hipGetLastError());
    }
    hipLaunchKernelGGL(stoch_decide_kernel, dim3(1), dim3(kThreads), 0, stream, bins, vocab, params, dec);
    HYP_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(stoch_draw_kernel, dim3(1), dim3(kThreads), 0, stream, logits, vocab, params, dec, out);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

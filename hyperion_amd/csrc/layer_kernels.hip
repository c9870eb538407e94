// The per-token work of a decoder layer between its projections, on gfx950:
//
//  * attn_prepare_kernel - ForwardPass::attention from the q/k/v projections to the cache
//    append (native/hyperion_mlx/src/forward.cc:395-459): q <- rope(q_norm(q)) in place;
//    K slot <- rope(k_norm(k_raw)); V slot <- v_norm(v_raw), v_raw = k_raw on K = V global
//    layers (forward.cc:403-412). One workgroup per token: the token's cos/sin table is
//    computed once into LDS and shared by all its heads; each wave normalises one head at
//    a time (lane u owns 64-value unit u, the order of q4_rmsnorm.h), stages it in LDS and
//    rotates pairs (i, i + D/2). Bits: those of rms_norm_rows_kernel followed by
//    rope_kernel and kv_write_kernel.
//
//  * residual_norm_kernel - the Gemma sandwich around a block (forward.cc:518-529):
//    residual <- bf16(residual + rms_norm(branch, w_post)), then optionally
//    residual <- bf16(residual * layer_scalar), then optionally next <- rms_norm(residual,
//    w_next) (the following block's input norm). One workgroup per row, thread u owning unit
//    u; both statistics in the order of q4_rmsnorm.h, so each norm has the bits of
//    launch_rms_normalize and of the skinny matmul's normalising prologue.
#include "common.h"
#include "kernels.h"
#include "q4_rmsnorm.h"

namespace hyperion::hip {
namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kWaves = kThreads / 64u;
constexpr uint32_t kMaxHeadDim = 512;

struct PrepareParams {
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

// Lanes u < D/64 load head `src` unit u and leave bf16(w * bf16(x * inv)) (w null: bf16(x *
// inv)) in xv; every lane takes part in the butterfly.
__device__ __forceinline__ void norm_head(const uint16_t* src, const uint16_t* w, uint32_t D, float eps,
                                          uint32_t lane, uint4 (&xv)[8]) {
    const uint32_t units = D / 64u;
    float ss = 0.0f;
    if (lane < units) {
        const uint4* s4 = reinterpret_cast<const uint4*>(src) + lane * 8u;
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[t] = s4[t];
        ss = unit_sumsq(xv);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float inv = rms_inverse(ss, D, eps);
    if (lane < units) {
        normalize_unit(xv, inv);
        if (w != nullptr) {
            const uint4* w4 = reinterpret_cast<const uint4*>(w) + lane * 8u;
            uint4 wv[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) wv[t] = w4[t];
            weight_unit(xv, wv);
        }
    }
}

__global__ __launch_bounds__(kThreads) void attn_prepare_kernel(PrepareParams p) {
    __shared__ float2 cs[kMaxHeadDim / 2];                        // (cos, sin) per pair
    __shared__ __attribute__((aligned(16))) uint16_t head[kWaves][kMaxHeadDim];
    const uint32_t t = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t D = p.D;
    const uint32_t half = D / 2u;
    const uint32_t pos = p.offset + t;

    // rope_kernel's angle arithmetic: inv_freq in double rounded to fp32, theta in fp32,
    // cos and sin in double rounded to fp32.
    for (uint32_t i = tid; i < half; i += kThreads) {
        const float inv = 2u * i < p.rotated ? static_cast<float>(pow(p.base, -2.0 * i / static_cast<double>(D))) : 0.0f;
        const float theta = static_cast<float>(pos) * inv;
        cs[i] = make_float2(static_cast<float>(cos(static_cast<double>(theta))),
                            static_cast<float>(sin(static_cast<double>(theta))));
    }
    __syncthreads();

    const bool cached = t >= p.first_cached;   // a chunk longer than the ring keeps its last cap tokens
    const size_t slot = static_cast<size_t>(pos % p.cap);
    const uint32_t total = p.H + p.KVH;
    const uint32_t rounds = (total + kWaves - 1u) / kWaves;
    uint16_t* hb = head[wave];
    for (uint32_t r = 0; r < rounds; ++r) {
        const uint32_t hh = r * kWaves + wave;
        const bool is_q = hh < p.H;
        const bool active = hh < total && (is_q || cached);
        uint16_t* dst = nullptr;
        uint4 xv[8];
        if (active) {
            const uint16_t* src;
            const uint16_t* w;
            if (is_q) {
                src = p.q + (static_cast<size_t>(t) * p.H + hh) * D;
                w = p.q_w;
                dst = p.q + (static_cast<size_t>(t) * p.H + hh) * D;
            } else {
                const uint32_t kh = hh - p.H;
                const size_t row = (static_cast<size_t>(t) * p.KVH + kh) * D;
                // V: the weightless norm straight into the cache slot.
                norm_head(p.v_raw != nullptr ? p.v_raw + row : p.k_raw + row, nullptr, D, p.eps, lane, xv);
                if (lane < D / 64u) {
                    uint4* v4 = reinterpret_cast<uint4*>(p.cache_v + (slot * p.KVH + kh) * D) + lane * 8u;
#pragma unroll
                    for (int u = 0; u < 8; ++u) v4[u] = xv[u];
                }
                src = p.k_raw + row;
                w = p.k_w;
                dst = p.cache_k + (slot * p.KVH + kh) * D;
            }
            norm_head(src, w, D, p.eps, lane, xv);
            if (lane < D / 64u) {
                uint4* h4 = reinterpret_cast<uint4*>(hb) + lane * 8u;
#pragma unroll
                for (int u = 0; u < 8; ++u) h4[u] = xv[u];
            }
        }
        __syncthreads();   // the staged head is visible to every lane of its wave
        if (active) {
            for (uint32_t i = lane; i < half; i += 64u) {
                const float x1 = bf16_bits_to_f32(hb[i]);
                const float x2 = bf16_bits_to_f32(hb[i + half]);
                const float c = cs[i].x;
                const float s = cs[i].y;
                const float a1 = x1 * c;
                const float a2 = x2 * s;
                const float b1 = x1 * s;
                const float b2 = x2 * c;
                dst[i] = f32_to_bf16_bits(a1 - a2);
                dst[i + half] = f32_to_bf16_bits(b1 + b2);
            }
        }
        __syncthreads();   // the rotation has read the staged head before the next round
    }
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
    if (mine) {
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[t] = b4[t];
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
        uint4 wv[8];
        const uint4* w4 = reinterpret_cast<const uint4*>(w_post) + tid * 8u;
#pragma unroll
        for (int t = 0; t < 8; ++t) wv[t] = w4[t];
        weight_unit(xv, wv);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint4 rv = r4[t];
            const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
            uint32_t hw[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float lo = round_bf16(bf16_bits_to_f32(rw[q] & 0xFFFFu) + bf16_bits_to_f32(hw[q] & 0xFFFFu));
                float hi = round_bf16(bf16_bits_to_f32(rw[q] >> 16) + bf16_bits_to_f32(hw[q] >> 16));
                if (scalar != nullptr) {
                    lo = round_bf16(lo * sc);
                    hi = round_bf16(hi * sc);
                }
                hw[q] = cvt_pk_bf16(lo, hi);
            }
            xv[t] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
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
        uint4 wv[8];
        const uint4* w4 = reinterpret_cast<const uint4*>(w_next) + tid * 8u;
#pragma unroll
        for (int t = 0; t < 8; ++t) wv[t] = w4[t];
        weight_unit(xv, wv);
        uint4* n4 = reinterpret_cast<uint4*>(next + row) + tid * 8u;
#pragma unroll
        for (int t = 0; t < 8; ++t) n4[t] = xv[t];
    }
}

}  // namespace

void launch_attn_prepare(const AttnPrepareArgs& a, hipStream_t stream) {
    if (a.L == 0) return;
    HYP_REQUIRE(a.head_dim % 64u == 0u && a.head_dim <= kMaxHeadDim, HYP_STATUS_UNSUPPORTED,
                "attention prepare: head_dim must be a multiple of 64, at most 512");
    PrepareParams p{};
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
    hipLaunchKernelGGL(attn_prepare_kernel, dim3(a.L), dim3(kThreads), 0, stream, p);
    HYP_HIP_CHECK(hipGetLastError());
}

uint32_t residual_norm_max_hidden() { return 64u * kThreads; }

void launch_residual_norm(const uint16_t* branch, uint16_t* residual, const uint16_t* w_post, const uint16_t* scalar,
                          const uint16_t* w_next, uint16_t* next, uint32_t m, uint32_t hidden, float eps,
                          hipStream_t stream) {
    if (m == 0) return;
    HYP_REQUIRE(hidden % 64u == 0u && hidden <= residual_norm_max_hidden(), HYP_STATUS_UNSUPPORTED,
                "residual norm: hidden must be a multiple of 64, at most 16384");
    hipLaunchKernelGGL(residual_norm_kernel, dim3(m), dim3(kThreads), 0, stream, branch, residual, w_post, scalar,
                       w_next, next, hidden, eps);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

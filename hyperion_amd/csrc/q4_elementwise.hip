// Elementwise bf16 epilogue for the prefill path (m > 4), where the GEMM writes plain
// bf16 outputs and this kernel finishes them:
//   softcap:  y = bf16(tanh(y / cap) * cap)     ForwardPass::softcap, forward.cc:154-160
// and the row RMS norm (mx::fast::rms_norm with or without its learned weight):
//   rms_normalize: y[r] = bf16(w * bf16(x[r] / sqrt(mean(x[r]^2) + eps))), fp32 statistics
// Eight bf16 per thread (16-byte loads and stores; the pointers are 16-byte aligned).
#include "common.h"
#include "kernels.h"
#include "q4_rmsnorm.h"

namespace hyperion::hip {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}

__global__ __launch_bounds__(kThreads) void softcap_kernel(uint16_t* __restrict__ y, float cap, uint64_t count) {
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t e0 = t * 8u;
    if (e0 >= count) return;
    if (e0 + 8u <= count) {
        uint4 v = reinterpret_cast<const uint4*>(y)[t];
        uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = pack2(softcap_bf16(bf16_bits_to_f32(w[i] & 0xFFFFu), cap),
                         softcap_bf16(bf16_bits_to_f32(w[i] >> 16), cap));
        }
        reinterpret_cast<uint4*>(y)[t] = v;
    } else {
        for (uint64_t e = e0; e < count; ++e) {
            y[e] = f32_to_bf16_bits(softcap_bf16(bf16_bits_to_f32(y[e]), cap));
        }
    }
}

// One workgroup per row; each thread sums squares over a strided slice, the wave sums
// meet in LDS, then the row is scaled in place or into y (k not a multiple of 64).
__global__ __launch_bounds__(kThreads) void rms_normalize_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ y, uint32_t k, float eps) {
    __shared__ float partial[kThreads / 64];
    const uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * k;
    uint16_t* yr = y + static_cast<size_t>(blockIdx.x) * k;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < k; i += kThreads) {
        const float v = bf16_bits_to_f32(xr[i]);
        ss = fmaf(v, v, ss);
    }
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((threadIdx.x & 63u) == 0u) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int wv = 0; wv < kThreads / 64; ++wv) total += partial[wv];
    const float inv = 1.0f / sqrtf(total / static_cast<float>(k) + eps);
    for (uint32_t i = threadIdx.x; i < k; i += kThreads) {
        float v = round_bf16(bf16_bits_to_f32(xr[i]) * inv);
        if (w != nullptr) v = bf16_bits_to_f32(w[i]) * v;
        yr[i] = f32_to_bf16_bits(v);
    }
}

dim3 grid_for(uint64_t count) {
    const uint64_t blocks = (count + 8u * kThreads - 1) / (8u * kThreads);
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "elementwise: tensor too large");
    return dim3(static_cast<uint32_t>(blocks));
}

}  // namespace

void launch_softcap(uint16_t* y, float cap_bf16, uint64_t count, hipStream_t stream) {
    if (count == 0) return;
    hipLaunchKernelGGL(softcap_kernel, grid_for(count), dim3(kThreads), 0, stream, y, cap_bf16, count);
    HYP_HIP_CHECK(hipGetLastError());
}

namespace {

// k a multiple of 64: one workgroup per row, a thread per 64-element unit (16-byte loads,
// the unit kept in registers between the two passes), the summation order of
// q4_rmsnorm.h - the same bits as the skinny matmul's normalising prologue.
__global__ __launch_bounds__(kThreads) void rms_normalize_units_kernel(const uint16_t* __restrict__ x,
                                                                       const uint16_t* __restrict__ w,
                                                                       uint16_t* __restrict__ y, uint32_t k,
                                                                       float eps) {
    extern __shared__ float part[];   // [k / 64] unit partials, then the row's inverse
    const uint32_t units = k / 64u;
    const uint4* xr = reinterpret_cast<const uint4*>(x + static_cast<size_t>(blockIdx.x) * k);
    uint4* yr = reinterpret_cast<uint4*>(y + static_cast<size_t>(blockIdx.x) * k);
    const uint4* wr = reinterpret_cast<const uint4*>(w);
    const uint32_t tid = threadIdx.x;
    uint4 xv[8];
    for (uint32_t u = tid; u < units; u += kThreads) {
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[t] = xr[u * 8u + t];
        part[u] = unit_sumsq(xv);
    }
    __syncthreads();
    if (tid < 64u) {
        const float ss = row_sumsq(part, units, tid);
        if (tid == 0u) part[units] = rms_inverse(ss, k, eps);
    }
    __syncthreads();
    const float inv = part[units];
    for (uint32_t u = tid; u < units; u += kThreads) {
        if (units > static_cast<uint32_t>(kThreads)) {   // more than one unit per thread: load it again
#pragma unroll
            for (int t = 0; t < 8; ++t) xv[t] = xr[u * 8u + t];
        }
        normalize_unit(xv, inv);
        if (wr != nullptr) {
            uint4 wv[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) wv[t] = wr[u * 8u + t];
            weight_unit(xv, wv);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) yr[u * 8u + t] = xv[t];
    }
}

// Short rows (k a multiple of 64, at most 64 units): one wave per row, lane l owning
// unit l. Each lane has at most one unit, so the order of q4_rmsnorm.h (lane l adds units
// l, l + 64, ..., then the butterfly) is the same as rms_normalize_units_kernel's: the
// same bits, for the many head-sized rows of q_norm / k_norm / v_norm.
__global__ __launch_bounds__(kThreads) void rms_norm_rows_kernel(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ w,
                                                                 uint16_t* __restrict__ y, uint32_t rows,
                                                                 uint32_t k, float eps) {
    const uint32_t row = blockIdx.x * (kThreads / 64u) + (threadIdx.x >> 6);
    if (row >= rows) return;   // wave-uniform
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t units = k / 64u;
    const uint4* xr = reinterpret_cast<const uint4*>(x + static_cast<size_t>(row) * k);
    uint4* yr = reinterpret_cast<uint4*>(y + static_cast<size_t>(row) * k);
    uint4 xv[8];
    float ss = 0.0f;
    if (lane < units) {
#pragma unroll
        for (int t = 0; t < 8; ++t) xv[t] = xr[lane * 8u + t];
        ss = unit_sumsq(xv);
    }
    ss = butterfly_sum<32>(ss, lane);
    const float inv = rms_inverse(ss, k, eps);
    if (lane < units) {
        normalize_unit(xv, inv);
        if (w != nullptr) {
            const uint4* wr = reinterpret_cast<const uint4*>(w);
            uint4 wv[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) wv[t] = wr[lane * 8u + t];
            weight_unit(xv, wv);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) yr[lane * 8u + t] = xv[t];
    }
}

}  // namespace

void launch_rms_normalize(const uint16_t* x, const uint16_t* w, uint32_t m, uint32_t k, float eps, uint16_t* y,
                          hipStream_t stream) {
    if (m == 0 || k == 0) return;
    if (k % 64u == 0u && k <= 64u * 64u) {
        const uint32_t per_block = kThreads / 64u;
        hipLaunchKernelGGL(rms_norm_rows_kernel, dim3((m + per_block - 1u) / per_block), dim3(kThreads), 0, stream,
                           x, w, y, m, k, eps);
    } else if (k % 64u == 0u && k / 64u + 1u <= 16384u) {
        const size_t lds = (k / 64u + 1u) * sizeof(float);
        hipLaunchKernelGGL(rms_normalize_units_kernel, dim3(m), dim3(kThreads), lds, stream, x, w, y, k, eps);
    } else {
        hipLaunchKernelGGL(rms_normalize_kernel, dim3(m), dim3(kThreads), 0, stream, x, w, y, k, eps);
    }
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

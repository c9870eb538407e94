// Elementwise bf16 epilogues for the prefill path (m > 4), where the GEMM writes plain
// bf16 outputs and these kernels finish them:
//   gelu_mul: h = bf16(gelu_chain(h) * u)      ForwardPass::mlp, forward.cc:338-343
//   softcap:  y = bf16(tanh(y / cap) * cap)     ForwardPass::softcap, forward.cc:154-160
// Eight bf16 per thread (16-byte loads and stores; the pointers are 16-byte aligned).
#include "common.h"
#include "kernels.h"

namespace hyperion::hip {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}

__device__ __forceinline__ float gelu_mul1(float h, float u) { return gelu_tanh_bf16_chain(h) * u; }

// Thread t owns elements [8t, 8t + 8); a full octet moves as 16-byte vectors, the
// ragged tail element by element.
__global__ __launch_bounds__(kThreads) void gelu_mul_kernel(uint16_t* __restrict__ h, const uint16_t* __restrict__ u,
                                                            uint64_t count) {
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const uint64_t e0 = t * 8u;
    if (e0 >= count) return;
    if (e0 + 8u <= count) {
        uint4 hv = reinterpret_cast<const uint4*>(h)[t];
        const uint4 uv = reinterpret_cast<const uint4*>(u)[t];
        uint32_t* hw = reinterpret_cast<uint32_t*>(&hv);
        const uint32_t* uw = reinterpret_cast<const uint32_t*>(&uv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hw[i] = pack2(gelu_mul1(bf16_bits_to_f32(hw[i] & 0xFFFFu), bf16_bits_to_f32(uw[i] & 0xFFFFu)),
                          gelu_mul1(bf16_bits_to_f32(hw[i] >> 16), bf16_bits_to_f32(uw[i] >> 16)));
        }
        reinterpret_cast<uint4*>(h)[t] = hv;
    } else {
        for (uint64_t e = e0; e < count; ++e) {
            h[e] = f32_to_bf16_bits(gelu_mul1(bf16_bits_to_f32(h[e]), bf16_bits_to_f32(u[e])));
        }
    }
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

dim3 grid_for(uint64_t count) {
    const uint64_t blocks = (count + 8u * kThreads - 1) / (8u * kThreads);
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "elementwise: tensor too large");
    return dim3(static_cast<uint32_t>(blocks));
}

}  // namespace

void launch_gelu_mul(uint16_t* h, const uint16_t* u, uint64_t count, hipStream_t stream) {
    if (count == 0) return;
    hipLaunchKernelGGL(gelu_mul_kernel, grid_for(count), dim3(kThreads), 0, stream, h, u, count);
    HYP_HIP_CHECK(hipGetLastError());
}

void launch_softcap(uint16_t* y, float cap_bf16, uint64_t count, hipStream_t stream) {
    if (count == 0) return;
    hipLaunchKernelGGL(softcap_kernel, grid_for(count), dim3(kThreads), 0, stream, y, cap_bf16, count);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

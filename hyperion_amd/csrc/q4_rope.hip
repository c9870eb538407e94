// Rotary position embedding on the device: mx::fast::rope(x, dims = head_dim,
// traditional = false, base | freqs, scale = 1, offset) as the reference applies it to q
// and k after their norms (native/hyperion_mlx/src/rope.cc:16-75, forward.cc:417-418).
//
// x is [rows, heads, head_dim] bf16 (a projection's output rows, row r at position
// offset + r). Pair (i, i + head_dim/2) of each head rotates by theta = fp32(pos) *
// inv_freq_i, inv_freq_i = fp32(base^(-2i / head_dim)) for i < rotated/2 and 0 above: the
// local layers' default scheme rotates everything (rotated = head_dim, theta 1e4); the
// global layers' proportional scheme rotates the first rotated/2 pairs with exponents over
// the full head_dim and leaves the rest (rotated = 128 of 512, theta 1e6). inv_freq, cos
// and sin are evaluated in double and rounded to fp32 once, so the result does not depend
// on the single-precision library; the rotation itself is fp32 without fusion, then bf16.
#include "common.h"
#include "kernels.h"

namespace hyperion::hip {
namespace {

constexpr int kThreads = 256;

// One thread per (row, pair index i): it rotates pair i of every head of its row.
__global__ __launch_bounds__(kThreads) void rope_kernel(const uint16_t* x, uint16_t* y, uint32_t rows, uint32_t heads,
                                                        uint32_t head_dim, uint32_t rotated, double base,
                                                        uint32_t offset) {
    const uint32_t half = head_dim / 2u;
    const uint64_t t = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= static_cast<uint64_t>(rows) * half) return;
    const uint32_t r = static_cast<uint32_t>(t / half);
    const uint32_t i = static_cast<uint32_t>(t - static_cast<uint64_t>(r) * half);
    const float pos = static_cast<float>(offset + r);
    const float inv = 2u * i < rotated ? static_cast<float>(pow(base, -2.0 * i / static_cast<double>(head_dim))) : 0.0f;
    const float theta = pos * inv;
    const float c = static_cast<float>(cos(static_cast<double>(theta)));
    const float s = static_cast<float>(sin(static_cast<double>(theta)));
    for (uint32_t h = 0; h < heads; ++h) {
        const size_t b = (static_cast<size_t>(r) * heads + h) * head_dim;
        const float x1 = bf16_bits_to_f32(x[b + i]);
        const float x2 = bf16_bits_to_f32(x[b + i + half]);
        const float a1 = x1 * c;
        const float a2 = x2 * s;
        const float b1 = x1 * s;
        const float b2 = x2 * c;
        y[b + i] = f32_to_bf16_bits(a1 - a2);
        y[b + i + half] = f32_to_bf16_bits(b1 + b2);
    }
}

}  // namespace

void launch_rope(const uint16_t* x, uint32_t rows, uint32_t heads, uint32_t head_dim, uint32_t rotated, float base,
                 uint32_t offset, uint16_t* y, hipStream_t stream) {
    const uint64_t threads = static_cast<uint64_t>(rows) * (head_dim / 2u);
    if (threads == 0) return;
    const uint64_t blocks = (threads + kThreads - 1u) / kThreads;
    HYP_REQUIRE(blocks <= 0x7fffffffull, HYP_STATUS_INVALID_ARGUMENT, "rope: tensor too large");
    hipLaunchKernelGGL(rope_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream, x, y, rows, heads,
                       head_dim, rotated, static_cast<double>(base), offset);
    HYP_HIP_CHECK(hipGetLastError());
}

}  // namespace hyperion::hip

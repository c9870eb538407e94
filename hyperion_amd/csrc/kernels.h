// Host-side launchers of the gfx950 kernels. All pointers are device pointers,
// all launches are asynchronous on `stream`. Callers validate shapes first.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace hyperion::hip {

// A resident Q4/g64 projection in MLX layout: w uint32 [n, k/8], scales and
// biases bf16 [n, k/64] (native/hyperion_mlx/src/weights.h:18-25).
struct Q4Matrix {
    const uint32_t* w = nullptr;
    const uint16_t* scales = nullptr;
    const uint16_t* biases = nullptr;
    uint32_t n = 0;
    uint32_t k = 0;
};

enum class Epilogue : int {
    kNone = 0,
    kSoftcap = 1,   // y = softcap(bf16(acc)), forward.cc:154-160
};

// Largest m the decode GEMV handles; larger m goes to the MFMA GEMM.
constexpr uint32_t kGemvMaxM = 4;
// Largest k the decode GEMV handles (64 lanes x 2 half-groups x 4 waves x 32).
constexpr uint32_t kGemvMaxK = 16384;

// Decode GEMV (m <= kGemvMaxM): y[m, n] = x[m, k] . dequant(W)^T.
// With `up` non-null it is the fused gate/up: y = gelu_chain(x.G^T) * (x.U^T).
void launch_q4_gemv(const Q4Matrix& w, const Q4Matrix* up, const uint16_t* x, uint32_t m,
                    uint16_t* y, Epilogue epi, float cap_bf16, hipStream_t stream);

// Prefill GEMM on bf16 MFMA: Q4 tiles dequantized in registers, x tiles in LDS.
// Plain bf16 output; epilogues for m > kGemvMaxM run as the elementwise kernels below.
void launch_q4_gemm(const Q4Matrix& w, const uint16_t* x, uint32_t m, uint16_t* y, hipStream_t stream);

// h = bf16(gelu_chain(h) * u) over `count` bf16 elements (in place on h).
void launch_gelu_mul(uint16_t* h, const uint16_t* u, uint64_t count, hipStream_t stream);
// y = softcap(y) over `count` bf16 elements (in place).
void launch_softcap(uint16_t* y, float cap_bf16, uint64_t count, hipStream_t stream);

// mx.quantize(w, 64, 4, "affine") of bf16 [n, k].
void launch_q4_quantize(const uint16_t* w, uint32_t n, uint32_t k, uint32_t* wq,
                        uint16_t* scales, uint16_t* biases, hipStream_t stream);

// mx.dequantize(..., bf16) of gathered rows; out_scale_bf16 != 0 multiplies each
// value by that bf16 constant with one more rounding.
void launch_q4_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                          uint32_t n_total, uint32_t k, const uint32_t* rows, uint32_t n_rows,
                          float out_scale_bf16, uint16_t* out, hipStream_t stream);

}  // namespace hyperion::hip

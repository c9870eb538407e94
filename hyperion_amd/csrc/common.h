// Shared host/device helpers for the gfx950 Q4/g64 engine.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "hyperion_hip.h"

namespace hyperion::hip {

// An error that carries the HypStatus it maps to at the C boundary (the
// reference's NativeError, runtime.mm:79-97 catches it by type).
class NativeError : public std::runtime_error {
  public:
    NativeError(HypStatus status, const std::string& message)
        : std::runtime_error(message), status_(status) {}
    [[nodiscard]] HypStatus status() const noexcept { return status_; }

  private:
    HypStatus status_;
};

[[noreturn]] inline void throw_hip(hipError_t err, const char* what, const char* file, int line) {
    throw NativeError(HYP_STATUS_INTERNAL, std::string(what) + " failed: " + hipGetErrorString(err) +
                                               " (" + file + ":" + std::to_string(line) + ")");
}

#define HYP_HIP_CHECK(expr)                                                    \
    do {                                                                       \
        hipError_t hyp_err_ = (expr);                                          \
        if (hyp_err_ != hipSuccess) {                                          \
            ::hyperion::hip::throw_hip(hyp_err_, #expr, __FILE__, __LINE__);   \
        }                                                                      \
    } while (0)

#define HYP_REQUIRE(cond, status, msg)                                         \
    do {                                                                       \
        if (!(cond)) {                                                         \
            throw ::hyperion::hip::NativeError((status), (msg));               \
        }                                                                      \
    } while (0)

// Compute units of the current device (queried once per device, then cached).
uint32_t device_compute_units();

constexpr uint32_t kGroupSize = 64;   // the locked quantization: group 64,
constexpr uint32_t kBits = 4;         // 4 bits, affine (model.cc:73-74)

// ---- device-side bf16 helpers ------------------------------------------------

// Two fp32 values -> one register of two bf16 (lo in bits 0-15), v_cvt_pk_bf16_f32: round
// to nearest even, a NaN kept quiet as (bits >> 16) | 0x40. On gfx950, with the flags these
// kernels are built with, the instruction gives exactly the bits of that definition for
// every one of the 2^32 fp32 inputs (denormals included), checked exhaustively on the
// device.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return static_cast<uint16_t>(cvt_pk_bf16(f, f) & 0xFFFFu);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// Round an fp32 value to bf16 precision and return it as fp32.
__device__ __forceinline__ float round_bf16(float f) {
    return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// The reference's gelu_pytorch_tanh (forward.cc:324-336): every MLX op rounds
// its bf16 result, constants are bf16 arrays. Input and output are bf16 values.
__device__ __forceinline__ float gelu_tanh_bf16_chain(float x) {
    const float c_coeff = 0.044677734375f;   // bf16(0.044715)
    const float c_inner = 0.796875f;         // bf16(0.7978845608)
    const float sq = round_bf16(x * x);
    const float x3 = round_bf16(x * sq);
    float inner = round_bf16(c_coeff * x3);
    inner = round_bf16(inner + x);
    inner = round_bf16(c_inner * inner);
    const float t = round_bf16(tanhf(inner));
    const float half_x = round_bf16(0.5f * x);
    const float one_t = round_bf16(1.0f + t);
    return round_bf16(half_x * one_t);
}

// The reference's softcap (forward.cc:154-160) on a bf16 logit with a bf16 cap.
__device__ __forceinline__ float softcap_bf16(float y, float cap_bf16) {
    const float d = round_bf16(__fdiv_rn(y, cap_bf16));
    const float t = round_bf16(tanhf(d));
    return round_bf16(t * cap_bf16);
}

}  // namespace hyperion::hip

// Register-level dequantization of MLX-affine Q4/g64 codes to bf16, shared by the
// prefill GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace hyperion::hip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// Two fp32 values -> one register of two bf16 (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

// The 8 codes of one packed word (lowest k in the lowest nibble) -> 8 bf16 values
// bf16(fma(s, q, b)) in k order: one rounding of the exact s * q + b.
__device__ __forceinline__ bf16x8_t dequant_word(uint32_t word, float s, float b) {
    uint32_t lo = word & 0x0F0F0F0Fu;          // codes 0,2,4,6 in bytes 0..3
    uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;   // codes 1,3,5,7
    // Opaque to the optimizer, so each byte converts with v_cvt_f32_ubyte{0..3} instead
    // of being re-extracted from the word with v_bfe_u32 first.
    asm volatile("" : "+v"(lo), "+v"(hi));
    uint4 r;
    r.x = pack_bf16x2(fmaf(s, static_cast<float>(lo & 0xFFu), b), fmaf(s, static_cast<float>(hi & 0xFFu), b));
    r.y = pack_bf16x2(fmaf(s, static_cast<float>((lo >> 8) & 0xFFu), b),
                      fmaf(s, static_cast<float>((hi >> 8) & 0xFFu), b));
    r.z = pack_bf16x2(fmaf(s, static_cast<float>((lo >> 16) & 0xFFu), b),
                      fmaf(s, static_cast<float>((hi >> 16) & 0xFFu), b));
    r.w = pack_bf16x2(fmaf(s, static_cast<float>(lo >> 24), b), fmaf(s, static_cast<float>(hi >> 24), b));
    return __builtin_bit_cast(bf16x8_t, r);
}

}  // namespace hyperion::hip

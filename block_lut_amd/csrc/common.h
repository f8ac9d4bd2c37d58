// Shared device helpers for the gfx950 LUT-MoE kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lutmoe.h"

namespace lutmoe {

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

constexpr int kBlockBL = 64;   // BL4 / nested: weights per codebook block
constexpr int kWave = 64;      // CDNA wavefront size

__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// IEEE round-to-nearest-even float -> bf16 bits (NaN -> 0x7fc0), the rule
// torch's .to(torch.bfloat16) applies.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// Two floats -> packed bf16 bits (a in the low half) by the hardware
// conversion (v_cvt_pk_bf16_f32): round to nearest even with fp32 denormals
// kept (the kernels' default float mode), the rule of f32_to_bf16 for every
// non-NaN input.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// float -> fp16 bits, round to nearest even (the hardware conversion).
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// REF: expert e's bf16[256] codebook (codebook_stride 0: one for all experts).
__device__ __forceinline__ const uint16_t* ref_codebook(const lutmoe_weights& w, int e) {
    return (const uint16_t*)w.codebook + (int64_t)e * w.codebook_stride;
}

// silu(g) * u = g * u / (1 + exp(-g)), with the hardware reciprocal (1 ulp in
// fp32; callers round the result to bf16).
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// Sum over the 64 lanes of a wave (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Orders this wave's LDS writes before its later LDS reads (the hardware
// keeps one wave's LDS operations in order; this stops the compiler moving
// the reads up).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace lutmoe

// Host-side launch helpers (defined in api.cpp).
namespace lutmoe_host {
hipStream_t stream_of(void* s);
int check_launch();
}  // namespace lutmoe_host

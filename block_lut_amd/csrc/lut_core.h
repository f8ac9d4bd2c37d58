// Inner loops shared by the LUT-GEMV kernels (gfx950).
#pragma once
#include "common.h"

namespace lutmoe {

// base + byte j of w, in one v_add_u32 with an SDWA byte select on src1
// (pure VALU; no memory access).
template <int J>
__device__ __forceinline__ uint32_t add_byte(uint32_t base, uint32_t w) {
    uint32_t r;
    if constexpr (J == 0)
        asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
            : "=v"(r) : "v"(base), "v"(w));
    else if constexpr (J == 1)
        asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
            : "=v"(r) : "v"(base), "v"(w));
    else if constexpr (J == 2)
        asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
            : "=v"(r) : "v"(base), "v"(w));
    else
        asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
            : "=v"(r) : "v"(base), "v"(w));
    return r;
}

typedef __attribute__((address_space(3))) const uint16_t lds_u16_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

__device__ __forceinline__ uint32_t lds_ld16(uint32_t a) { return *(lds_u16_t*)a; }

// One BL4 code dword (8 nibbles = 8 consecutive weights of one row) against
// its block's bf16 table at LDS byte address `tab`:
//   pair j = (table[nibble 2j], table[nibble 2j+1]) -> dot2 with x pair j.
template <int TB>
__device__ __forceinline__ void bl4_dot8(uint32_t w, uint32_t tab, const uint32_t (&x)[TB][4],
                                         int nt, float (&acc)[TB]) {
    const uint32_t we = (w << 1) & 0x1e1e1e1eu;   // byte j = 2 * code(2j)
    const uint32_t wo = (w >> 3) & 0x1e1e1e1eu;   // byte j = 2 * code(2j+1)
    uint32_t pr[4];
    pr[0] = lds_ld16(add_byte<0>(tab, we)) | (lds_ld16(add_byte<0>(tab, wo)) << 16);
    pr[1] = lds_ld16(add_byte<1>(tab, we)) | (lds_ld16(add_byte<1>(tab, wo)) << 16);
    pr[2] = lds_ld16(add_byte<2>(tab, we)) | (lds_ld16(add_byte<2>(tab, wo)) << 16);
    pr[3] = lds_ld16(add_byte<3>(tab, we)) | (lds_ld16(add_byte<3>(tab, wo)) << 16);
#pragma unroll
    for (int t = 0; t < TB; ++t) {
        if (t < nt) {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t] = dot2_bf16(pr[j], x[t][j], acc[t]);
        }
    }
}

// Full-wave sum with DPP (quad perms, half-row / row mirrors, row broadcasts);
// the total is returned uniformly (read from lane 63).
__device__ __forceinline__ float wave_reduce(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

template <int CTRL, int RMASK>
__device__ __forceinline__ float dpp_or_neg_inf(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        __builtin_bit_cast(int, -INFINITY), __builtin_bit_cast(int, x), CTRL, RMASK, 0xf, false));
}

__device__ __forceinline__ float wave_reduce_max(float v) {
    v = fmaxf(v, dpp_or_neg_inf<0xb1, 0xf>(v));
    v = fmaxf(v, dpp_or_neg_inf<0x4e, 0xf>(v));
    v = fmaxf(v, dpp_or_neg_inf<0x141, 0xf>(v));
    v = fmaxf(v, dpp_or_neg_inf<0x140, 0xf>(v));
    v = fmaxf(v, dpp_or_neg_inf<0x142, 0xa>(v));
    v = fmaxf(v, dpp_or_neg_inf<0x143, 0xc>(v));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Inclusive prefix sum over the 64 lanes (row shifts within 16-lane rows,
// then row broadcasts across rows).
__device__ __forceinline__ int wave_scan_incl(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

}  // namespace lutmoe

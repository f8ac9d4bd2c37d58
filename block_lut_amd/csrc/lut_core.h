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

// base + 16-bit field j of w (SDWA word select on src1).
template <int J>
__device__ __forceinline__ uint32_t add_word(uint32_t base, uint32_t w) {
    uint32_t r;
    if constexpr (J == 0)
        asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
            : "=v"(r) : "v"(base), "v"(w));
    else
        asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
            : "=v"(r) : "v"(base), "v"(w));
    return r;
}

typedef __attribute__((address_space(3))) const uint16_t lds_u16_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

__device__ __forceinline__ uint32_t lds_ld16(uint32_t a) { return *(lds_u16_t*)a; }

typedef __attribute__((address_space(3))) const uint32_t lds_u32_t;
__device__ __forceinline__ uint32_t lds_ld32(uint32_t a) { return *(lds_u32_t*)a; }

// 32 REF byte codes (8 dwords, code j of the lane's 32 columns in byte j%4 of
// dword j/4) against the bf16[256] codebook at LDS byte address `cbase`:
// g[t] += sum_j x_t[j] * cb[code j], products exact in fp32 (bf16 x bf16),
// two per v_dot2_f32_bf16.  x dword i holds columns 2i, 2i+1.
template <int TB>
__device__ __forceinline__ void ref_dot32(const u32x4_t (&cw)[2], uint32_t cbase, const uint32_t (&x)[TB][16],
                                          int nt, float (&g)[TB]) {
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        const uint32_t w = cw[d >> 2][d & 3];
        const uint32_t we = (w & 0x00ff00ffu) << 1;   // 2*code of columns 4d, 4d+2 (16-bit fields)
        const uint32_t wo = (w >> 7) & 0x01fe01feu;   // 2*code of columns 4d+1, 4d+3
        const uint32_t p0 = lds_ld16(add_word<0>(cbase, we)) | (lds_ld16(add_word<0>(cbase, wo)) << 16);
        const uint32_t p1 = lds_ld16(add_word<1>(cbase, we)) | (lds_ld16(add_word<1>(cbase, wo)) << 16);
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            if (t < nt) {
                g[t] = dot2_bf16(p0, x[t][2 * d], g[t]);
                g[t] = dot2_bf16(p1, x[t][2 * d + 1], g[t]);
            }
        }
    }
}

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

// One BL4 code dword (8 nibbles = 8 consecutive weights of one row, even
// weight in the low nibble) -> 8 bf16 weights in column order, looked up in
// the row's bf16[16] LDS table at byte address `tab` (one SDWA add and one
// ds_read_u16 per weight).  Split in two so the reads can be issued well
// before the combining ops that wait for them.
struct Lookup8 {
    uint32_t e[4], o[4];   // table entries of columns 2j and 2j+1
};

__device__ __forceinline__ Lookup8 lookup8_issue(uint32_t w, uint32_t tab) {
    const uint32_t we = (w << 1) & 0x1e1e1e1eu;   // byte j = 2 * code(2j)
    const uint32_t wo = (w >> 3) & 0x1e1e1e1eu;   // byte j = 2 * code(2j+1)
    Lookup8 r;
    r.e[0] = lds_ld16(add_byte<0>(tab, we));
    r.o[0] = lds_ld16(add_byte<0>(tab, wo));
    r.e[1] = lds_ld16(add_byte<1>(tab, we));
    r.o[1] = lds_ld16(add_byte<1>(tab, wo));
    r.e[2] = lds_ld16(add_byte<2>(tab, we));
    r.o[2] = lds_ld16(add_byte<2>(tab, wo));
    r.e[3] = lds_ld16(add_byte<3>(tab, we));
    r.o[3] = lds_ld16(add_byte<3>(tab, wo));
    return r;
}

__device__ __forceinline__ u32x4_t lookup8_combine(const Lookup8& l) {
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = l.e[j] | (l.o[j] << 16);
    return r;
}

// Register tables: a row's bf16 table of 2^B entries (B = 2, 3, 4; dwords
// T[i] = entries 2i, 2i+1) as two byte planes, lo[k] / hi[k] byte i = low /
// high byte of entry 4k+i, so that v_perm_b32 looks up four codes at once.
template <int B>
__device__ __forceinline__ void table_planes(const uint32_t* T, uint32_t* lo, uint32_t* hi) {
#pragma unroll
    for (int k = 0; k < (1 << B) / 4; ++k) {
        lo[k] = __builtin_amdgcn_perm(T[2 * k + 1], T[2 * k], 0x06040200u);
        hi[k] = __builtin_amdgcn_perm(T[2 * k + 1], T[2 * k], 0x07050301u);
    }
}
// Plane bytes of the four codes in the bytes of s (each < 2^B).  Eight
// entries are one v_perm_b32 (byte selects 0-7); sixteen are two, of the
// low and high halves, and a third that picks per byte by the code's bit 3.
template <int B>
__device__ __forceinline__ uint32_t plane_lookup4(const uint32_t* pl, uint32_t s, uint32_t s7, uint32_t sel8) {
    if constexpr (B == 2) return __builtin_amdgcn_perm(pl[0], pl[0], s);
    else if constexpr (B == 3) return __builtin_amdgcn_perm(pl[1], pl[0], s);
    else {
        const uint32_t p0 = __builtin_amdgcn_perm(pl[1], pl[0], s7);
        const uint32_t p1 = __builtin_amdgcn_perm(pl[3], pl[2], s7);
        return __builtin_amdgcn_perm(p1, p0, sel8);
    }
}
// The 8 codes of one BL4 code dword (nibble j = code of weight j) looked up
// in register planes: dword j = bf16(w_2j) | bf16(w_2j+1) << 16, as
// lookup8_combine(lookup8_issue(w, ...)).
template <int B>
__device__ __forceinline__ u32x4_t regtab_lookup8(const uint32_t* lo, const uint32_t* hi, uint32_t w) {
    const uint32_t se = w & 0x0f0f0f0fu, so = (w >> 4) & 0x0f0f0f0fu;
    uint32_t se7 = se, so7 = so, sel_e = 0, sel_o = 0;
    if constexpr (B == 4) {
        se7 = se & 0x07070707u;
        so7 = so & 0x07070707u;
        sel_e = ((se >> 1) & 0x04040404u) | 0x03020100u;   // byte j: j, or j + 4 for codes >= 8
        sel_o = ((so >> 1) & 0x04040404u) | 0x03020100u;
    }
    const uint32_t le = plane_lookup4<B>(lo, se, se7, sel_e), he = plane_lookup4<B>(hi, se, se7, sel_e);
    const uint32_t lo_ = plane_lookup4<B>(lo, so, so7, sel_o), ho = plane_lookup4<B>(hi, so, so7, sel_o);
    // even weights 0, 2 | 4, 6 and odd weights 1, 3 | 5, 7 as bf16 pairs
    const uint32_t e01 = __builtin_amdgcn_perm(he, le, 0x05010400u), e23 = __builtin_amdgcn_perm(he, le, 0x07030602u);
    const uint32_t o01 = __builtin_amdgcn_perm(ho, lo_, 0x05010400u), o23 = __builtin_amdgcn_perm(ho, lo_, 0x07030602u);
    u32x4_t r;
    r[0] = __builtin_amdgcn_perm(o01, e01, 0x05040100u);
    r[1] = __builtin_amdgcn_perm(o01, e01, 0x07060302u);
    r[2] = __builtin_amdgcn_perm(o23, e23, 0x05040100u);
    r[3] = __builtin_amdgcn_perm(o23, e23, 0x07060302u);
    return r;
}

// regtab_lookup8 without its last step: the 8 weights in the order
// w0, w2, w4, w6, w1, w3, w5, w7 (an MFMA operand whose partner operand holds
// its 8 k-values in the same order gives the same products)
template <int B>
__device__ __forceinline__ u32x4_t regtab_lookup8_eo(const uint32_t* lo, const uint32_t* hi, uint32_t w) {
    const uint32_t se = w & 0x0f0f0f0fu, so = (w >> 4) & 0x0f0f0f0fu;
    uint32_t se7 = se, so7 = so, sel_e = 0, sel_o = 0;
    if constexpr (B == 4) {
        se7 = se & 0x07070707u;
        so7 = so & 0x07070707u;
        sel_e = ((se >> 1) & 0x04040404u) | 0x03020100u;
        sel_o = ((so >> 1) & 0x04040404u) | 0x03020100u;
    }
    const uint32_t le = plane_lookup4<B>(lo, se, se7, sel_e), he = plane_lookup4<B>(hi, se, se7, sel_e);
    const uint32_t lo_ = plane_lookup4<B>(lo, so, so7, sel_o), ho = plane_lookup4<B>(hi, so, so7, sel_o);
    u32x4_t r;
    r[0] = __builtin_amdgcn_perm(he, le, 0x05010400u);    // w0, w2
    r[1] = __builtin_amdgcn_perm(he, le, 0x07030602u);    // w4, w6
    r[2] = __builtin_amdgcn_perm(ho, lo_, 0x05010400u);   // w1, w3
    r[3] = __builtin_amdgcn_perm(ho, lo_, 0x07030602u);   // w5, w7
    return r;
}
// 8 bf16 in column order (dword j = columns 2j, 2j+1) -> the order of
// regtab_lookup8_eo
__device__ __forceinline__ u32x4_t eo_order(const u32x4_t& a) {
    u32x4_t r;
    r[0] = __builtin_amdgcn_perm(a[1], a[0], 0x05040100u);
    r[1] = __builtin_amdgcn_perm(a[3], a[2], 0x05040100u);
    r[2] = __builtin_amdgcn_perm(a[1], a[0], 0x07060302u);
    r[3] = __builtin_amdgcn_perm(a[3], a[2], 0x07060302u);
    return r;
}

__device__ __forceinline__ u32x4_t lookup8_lds(uint32_t w, uint32_t tab) {
    return lookup8_combine(lookup8_issue(w, tab));
}

// A NestedLUT expert in the device layout: each 32 consecutive weights (flat
// row-major [rows][K] order; w_j = code of weight j of the group) as 4b bytes,
// four little-endian words of which a tier-b group holds the first b:
//   f0: nibble n = (w_n & 3) | (w_{n+8} & 3) << 2
//   f1: nibble n = (w_{n+16} & 3) | (w_{n+24} & 3) << 2
//   b2: nibble n bit q = bit 2 of w_{n+8q}       (b >= 3)
//   b3: nibble n bit q = bit 3 of w_{n+8q}       (b = 4)
// so the codes of weights 8q .. 8q+7 are one shift and mask per word away from
// a BL4 code dword (nested_code8).  Tables bf16 [rows][K/64][2^b].  Both are
// read through bounds-checked buffer descriptors (bytes past the end read as
// zero).
constexpr int kBufWord3 = 0x00020000;   // raw buffer, dword format (gfx9)

struct NestedView {
    __amdgpu_buffer_rsrc_t codes, table;
    int bits;
};

__device__ __forceinline__ NestedView nested_view(const lutmoe_weights& w, int e) {
    const uint8_t* cd = ((const uint8_t* const*)w.codes)[e];
    const uint16_t* tb = ((const uint16_t* const*)w.tables)[e];
    const int b = __builtin_amdgcn_readfirstlane((int)w.tier_bits[e]);   // uniform: scalar branches on it
    const uint32_t n = (uint32_t)w.rows * (uint32_t)w.cols;   // < 2^32 (checked on the host)
    NestedView v;
    v.codes = __builtin_amdgcn_make_buffer_rsrc((void*)cd, 0, (int)(n / 8 * (uint32_t)b), kBufWord3);
    v.table = __builtin_amdgcn_make_buffer_rsrc((void*)tb, 0, (int)(((n / 64) << b) * 2), kBufWord3);
    v.bits = b;
    return v;
}

// The BL4 code dword (nibble j = code of weight 8q + j) of weights
// 8q .. 8q+7 of a device-layout group (f0, f1 = its 2-bit field words, b2 /
// b3 = its bit-2 / bit-3 words, zero for lower tiers): one shift and mask
// per word.  kBits (2, 3 or 4; 0 = not known at compile time): words a tier
// does not have are skipped.
template <int kBits = 0>
__device__ __forceinline__ uint32_t nested_code8(uint32_t f0, uint32_t f1, uint32_t b2, uint32_t b3, int q) {
    const uint32_t f = q < 2 ? f0 : f1;
    const uint32_t x = (q & 1 ? f >> 2 : f) & 0x33333333u;
    if constexpr (kBits == 2) return x;
    const uint32_t y = (q < 3 ? b2 << (2 - q) : b2 >> 1) & 0x44444444u;
    if constexpr (kBits == 3) return x | y;
    return x | y | ((b3 << (3 - q)) & 0x88888888u);
}

// The code of weight j (0..31) of a device-layout group.
__device__ __forceinline__ uint32_t nested_code1(uint32_t f0, uint32_t f1, uint32_t b2, uint32_t b3, int j) {
    const int n = j & 7, q = j >> 3;
    const uint32_t f = q < 2 ? f0 : f1;
    return ((f >> (4 * n + 2 * (q & 1))) & 3u) | (((b2 >> (4 * n + q)) & 1u) << 2) |
           (((b3 >> (4 * n + q)) & 1u) << 3);
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

// sigmoid(x . g) over H bf16 values with fp32 accumulation (Qwen's shared-
// expert gate, customized/qwen.py:99-100).  Whole wave; the result is
// uniform.  H % 8 == 0 and both pointers 16-byte aligned.
__device__ __forceinline__ float shared_gate_weight(const uint16_t* __restrict__ x, const uint16_t* __restrict__ g,
                                                    int H) {
    const int lane = threadIdx.x & 63;
    float s = 0.f;
    for (int c = lane * 8; c < H; c += 512) {
        const uint4 xv = *reinterpret_cast<const uint4*>(x + c);
        const uint4 gv = *reinterpret_cast<const uint4*>(g + c);
        s = dot2_bf16(xv.x, gv.x, s);
        s = dot2_bf16(xv.y, gv.y, s);
        s = dot2_bf16(xv.z, gv.z, s);
        s = dot2_bf16(xv.w, gv.w, s);
    }
    const float z = wave_reduce(s);
    return 1.0f / (1.0f + __expf(-z));
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

// The two results of a swap are copied out by value: a bit cast of a
// vector element lvalue reads element 0 with this compiler.
__device__ __forceinline__ float swap_sum32(float a, float b) {
    const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                    false, false);
    const uint32_t s0 = s[0], s1 = s[1];
    return __uint_as_float(s0) + __uint_as_float(s1);
}
__device__ __forceinline__ float swap_sum16(float a, float b) {
    const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                    false, false);
    const uint32_t s0 = s[0], s1 = s[1];
    return __uint_as_float(s0) + __uint_as_float(s1);
}

// Reduce-scatter of 8 per-lane partial sums over the wave: lane l returns the
// wave total of v[l >> 3].  Halves of the wave trade values 4..7 for 0..3
// (permlane32 swap: lane l of the upper half gets the lower half's lane l,
// and the other way round, so swapped + kept is the pair sum), then 16-lane
// rows trade 2 of their 4 (permlane16 swap), then the two 8-lane halves of a
// row trade 1 of 2 (row mirror), and each 8-lane group sums its value (two
// quad permutes and a half-row mirror).  19 cross-lane/add steps instead of
// eight full reductions.
__device__ __forceinline__ float wave_reduce8(const float (&v)[8]) {
    const int lane = threadIdx.x & 63;
    float a[4], b[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = swap_sum32(v[i], v[i + 4]);
#pragma unroll
    for (int i = 0; i < 2; ++i) b[i] = swap_sum16(a[i], a[i + 2]);
    const bool hi = (lane >> 3) & 1;
    const float send = hi ? b[0] : b[1];
    float c = (hi ? b[1] : b[0]) +
              __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, send), 0x140, 0xf, 0xf,
                                                                    false));   // row_mirror
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0xb1, 0xf, 0xf, false));
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x4e, 0xf, 0xf, false));
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x141, 0xf, 0xf, false));
    return c;
}

// Reduce-scatter of 4 per-lane partial sums over the wave: lane l returns the
// wave total of v[l >> 4] (uniform within each 16-lane row).  The halves trade
// v2, v3 for v0, v1 (permlane32 swap), 16-lane rows trade one of two
// (permlane16 swap), then each row sums its value with four DPP adds.
__device__ __forceinline__ float wave_reduce4(float v0, float v1, float v2, float v3) {
    const float a0 = swap_sum32(v0, v2), a1 = swap_sum32(v1, v3);
    float c = swap_sum16(a0, a1);
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0xb1, 0xf, 0xf, false));
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x4e, 0xf, 0xf, false));
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x141, 0xf, 0xf, false));
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x140, 0xf, 0xf, false));
    return c;
}

// The value of lane l + 32 in lanes l < 32 (permlane32 swap).
__device__ __forceinline__ float from_upper_half(float v) {
    const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    const uint32_t s1 = s[1];
    return __uint_as_float(s1);
}

// Lanes of this wave holding the same id as this lane (ids < 2^nbits;
// invalid lanes match nobody and get 0): one ballot per id bit.
__device__ __forceinline__ uint64_t match_lanes(int id, bool ok, int nbits) {
    uint64_t m = __ballot(ok);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (id >> b) & 1;
        const uint64_t bal = __ballot(ok && bit);
        m &= bit ? bal : ~bal;
    }
    return ok ? m : 0ull;
}

// Order-preserving int key of a float: larger float -> larger key, -0 and +0
// equal (v + 0 turns -0 into +0), NaN -> INT_MIN (never selected, as a float
// comparison never selects it).
__device__ __forceinline__ int float_key(float v) {
    const int b = __builtin_bit_cast(int, v + 0.0f);
    return v != v ? INT_MIN : b ^ ((b >> 31) & 0x7fffffff);
}

template <int CTRL, int RMASK>
__device__ __forceinline__ int dpp_max_i32(int v) {
    return max(v, __builtin_amdgcn_update_dpp(INT_MIN, v, CTRL, RMASK, 0xf, false));
}

// Wave maximum of an int (every lane gets it).
__device__ __forceinline__ int wave_max_i32(int v) {
    v = dpp_max_i32<0xb1, 0xf>(v);    // quad_perm [1,0,3,2]
    v = dpp_max_i32<0x4e, 0xf>(v);    // quad_perm [2,3,0,1]
    v = dpp_max_i32<0x141, 0xf>(v);   // row_half_mirror
    v = dpp_max_i32<0x140, 0xf>(v);   // row_mirror
    v = dpp_max_i32<0x142, 0xa>(v);   // row_bcast:15
    v = dpp_max_i32<0x143, 0xc>(v);   // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
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

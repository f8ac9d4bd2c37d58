// Dequantisation and code-unpack kernels (memory-bound byte work).
//
//  ref_dequant   : REF codes -> bf16, out = bf16(f32(cb[c]) * f32(absmax[blk]))
//                  (csrc/kernels/tensor_recover.cu:101-142 rule; batched over
//                  experts like lut_decompress_kernel.cu:87-120).
//  bl4_dequant   : BL4 codes -> bf16 through per-block bf16 tables staged in LDS.
//  nested_dequant: NestedLUT tier-b device-layout codes -> bf16.
//  nested_group_planes: NestedLUT plane sections -> the device layout.
//  unpack_4bit   : in-place low-nibble unpack (tensor_recover.cu:161-192),
//                  done as a race-free halving sequence instead of the
//                  reference's copy-to-upper-half + expand.
//  unpack_6bit   : the 6-bit tier unpack the reference runs on the CPU
//                  (csrc/tensor_engine/tensor_engine.cpp:535-548).
//  pack_bitplanes: one-byte codes -> the three bit-plane sections (the
//                  inverse of the unpacks; convert_lut.py:95-110).
//  merge_bitplane: in-place tier upgrade of resident codes by one 2-bit
//                  section (the delta a tier promotion reads,
//                  tensor_engine.cpp:504-510).
#include "common.h"
#include "kernels.h"
#include "lut_core.h"

using namespace lutmoe;

namespace {

constexpr int kRefVec = 16;   // codes per thread in ref_dequant

__global__ __launch_bounds__(256) void ref_dequant_kernel(
    uint16_t* __restrict__ out, const uint8_t* __restrict__ idx,
    const uint16_t* __restrict__ absmax, const uint16_t* __restrict__ cb, int64_t cb_stride, int n, int nb,
    int bs, int64_t out_stride, int64_t idx_stride, int vec_ok) {
    __shared__ float s_cb[256];
    const int e = blockIdx.y;
    s_cb[threadIdx.x] = bf16_to_f32(cb[e * cb_stride + threadIdx.x]);
    __syncthreads();
    const uint8_t* ip = idx + e * idx_stride;
    const uint16_t* ap = absmax + (int64_t)e * nb;
    uint16_t* op = out + e * out_stride;
    const int i0 = (blockIdx.x * 256 + threadIdx.x) * kRefVec;
    if (i0 >= n) return;
    if (vec_ok && i0 + kRefVec <= n) {
        const uint4 c = *reinterpret_cast<const uint4*>(ip + i0);
        const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
        uint32_t o[8];
        int b = i0 / bs;
        int next = (b + 1) * bs;
        float am = bf16_to_f32(ap[min(b, nb - 1)]);
#pragma unroll
        for (int j = 0; j < kRefVec; ++j) {
            if (i0 + j == next) {            // crossed into the next absmax block
                ++b;
                next += bs;
                am = bf16_to_f32(ap[min(b, nb - 1)]);
            }
            const uint32_t code = (cw[j >> 2] >> (8 * (j & 3))) & 0xffu;
            const uint32_t v = f32_to_bf16(s_cb[code] * am);
            if (j & 1) o[j >> 1] |= v << 16; else o[j >> 1] = v;
        }
        uint4* dst = reinterpret_cast<uint4*>(op + i0);
        dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
        dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    } else {
        const int end = min(n, i0 + kRefVec);
        for (int i = i0; i < end; ++i) {
            const int b = min(i / bs, nb - 1);
            op[i] = (uint16_t)f32_to_bf16(s_cb[ip[i]] * bf16_to_f32(ap[b]));
        }
    }
}

// 256 threads handle 128 blocks of 64 weights; tables staged in LDS.
__global__ __launch_bounds__(256) void bl4_dequant_kernel(
    uint16_t* __restrict__ out, const uint8_t* __restrict__ codes,
    const uint16_t* __restrict__ tables, int64_t nblocks) {
    __shared__ uint16_t s_tab[128 * 16];
    const int64_t b0 = (int64_t)blockIdx.x * 128;
    const int t = threadIdx.x;
    const int64_t nloc = min((int64_t)128, nblocks - b0);
    // table load: thread t loads entries [8t, 8t+8) of the CTA's 128*16 entries
    if (t < nloc * 2) {
        *reinterpret_cast<uint4*>(&s_tab[t * 8]) =
            *reinterpret_cast<const uint4*>(tables + b0 * 16 + t * 8);
    }
    __syncthreads();
    const int lb = t >> 1, h = t & 1;
    if (lb >= nloc) return;
    const uint4 c = *reinterpret_cast<const uint4*>(codes + (b0 + lb) * 32 + h * 16);
    const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
    const uint16_t* tab = &s_tab[lb * 16];
    uint32_t o[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t byte = (cw[j >> 2] >> (8 * (j & 3))) & 0xffu;
        o[j] = (uint32_t)tab[byte & 15u] | ((uint32_t)tab[byte >> 4] << 16);
    }
    uint4* dst = reinterpret_cast<uint4*>(out + (b0 + lb) * 64 + h * 32);
    dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
    dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    dst[2] = make_uint4(o[8], o[9], o[10], o[11]);
    dst[3] = make_uint4(o[12], o[13], o[14], o[15]);
}

// Nested: thread handles one 32-weight group of the device layout (half a
// 64-block): 4b code bytes.
__global__ __launch_bounds__(256) void nested_dequant_kernel(
    uint16_t* __restrict__ out, const uint8_t* const* __restrict__ code_ptrs,
    const uint16_t* const* __restrict__ table_ptrs, const int8_t* __restrict__ bits,
    int e0, int64_t n_per_expert) {
    const int e = e0 + blockIdx.y;
    const int b = bits[e];
    const uint16_t* tab = table_ptrs[e];
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t i0 = g * 32;
    if (i0 >= n_per_expert) return;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(code_ptrs[e] + g * 4 * b);
    const uint32_t f0 = q[0], f1 = q[1];
    const uint32_t b2 = b >= 3 ? q[2] : 0u;
    const uint32_t b3 = b >= 4 ? q[3] : 0u;
    const uint16_t* t = tab + (i0 / kBlockBL) * (1 << b);
    uint32_t o[16];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const uint32_t v = t[nested_code1(f0, f1, b2, b3, j)];
        if (j & 1) o[j >> 1] |= v << 16; else o[j >> 1] = v;
    }
    uint4* dst = reinterpret_cast<uint4*>(out + (int64_t)blockIdx.y * n_per_expert + i0);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) dst[q4] = make_uint4(o[4 * q4], o[4 * q4 + 1], o[4 * q4 + 2], o[4 * q4 + 3]);
}

// NestedLUT plane sections [p01 n/4 | p2 n/8 | p3 n/8] (the tier's prefix;
// p01: weight i's 2-bit field at bits 2(i%4) of byte i/4; p2 / p3: its bit 2
// / bit 3 at bit i%8 of byte i/8) -> the device layout (NestedView,
// lut_core.h).  One thread per 32-weight group; n % 64 == 0 keeps every
// section and group 4-byte aligned.
__device__ __forceinline__ uint32_t spread_fields8(uint32_t f) {   // 2-bit field j -> bits 4j..4j+1
    uint32_t x = f & 0xffffu;
    x = (x | (x << 8)) & 0x00ff00ffu;
    x = (x | (x << 4)) & 0x0f0f0f0fu;
    return (x | (x << 2)) & 0x33333333u;
}
__device__ __forceinline__ uint32_t spread_bits8(uint32_t v) {     // bit j -> bit 4j
    uint32_t y = v & 0xffu;
    y = (y | (y << 12)) & 0x000f000fu;
    y = (y | (y << 6)) & 0x03030303u;
    return (y | (y << 3)) & 0x11111111u;
}
__global__ __launch_bounds__(256) void nested_group_planes_kernel(const uint32_t* __restrict__ planes, int b,
                                                                  int64_t n, uint32_t* __restrict__ out) {
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g * 32 >= n) return;
    const uint32_t p0 = planes[2 * g], p1 = planes[2 * g + 1];   // fields of weights 0-15, 16-31
    uint32_t* o = out + g * b;
    o[0] = spread_fields8(p0) | (spread_fields8(p0 >> 16) << 2);
    o[1] = spread_fields8(p1) | (spread_fields8(p1 >> 16) << 2);
    for (int s = 2; s < b; ++s) {
        const uint32_t w = planes[n / 16 + (int64_t)(s - 2) * (n / 32) + g];   // bit s of weights 0-31
        o[s] = spread_bits8(w) | (spread_bits8(w >> 8) << 1) | (spread_bits8(w >> 16) << 2) |
               (spread_bits8(w >> 24) << 3);
    }
}

__global__ __launch_bounds__(256) void f16_to_bf16_kernel(const uint16_t* __restrict__ in,
                                                          uint16_t* __restrict__ out, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i + 8 <= n) {
        const uint4 v = *reinterpret_cast<const uint4*>(in + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            o[j] = f32_to_bf16(f16_to_f32(w[j] & 0xffffu)) |
                   (f32_to_bf16(f16_to_f32(w[j] >> 16)) << 16);
        *reinterpret_cast<uint4*>(out + i) = make_uint4(o[0], o[1], o[2], o[3]);
    } else {
        for (int64_t j = i; j < n; ++j) out[j] = (uint16_t)f32_to_bf16(f16_to_f32(in[j]));
    }
}

// out[2i] = src[i] & 15, out[2i+1] = src[i] >> 4 for i in [0, nsrc); src and
// dst ranges are disjoint.
__global__ __launch_bounds__(256) void expand_nibbles_kernel(uint8_t* __restrict__ dst,
                                                             const uint8_t* __restrict__ src,
                                                             int64_t nsrc) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const int64_t end = min(nsrc, i + 4);
    for (int64_t j = i; j < end; ++j) {
        const uint8_t p = src[j];
        dst[2 * j] = p & 0x0f;
        dst[2 * j + 1] = p >> 4;
    }
}

constexpr int kUnpackBase = 8192;   // outputs finished by one CTA

// Final in-place step on a region of m <= kUnpackBase outputs: every packed
// byte is read before the CTA barrier, every output written after it.
__global__ __launch_bounds__(1024) void unpack_base_kernel(uint8_t* data, int m) {
    uint8_t v[kUnpackBase / 2 / 1024];
    const int np = m / 2;
#pragma unroll
    for (int q = 0; q < kUnpackBase / 2 / 1024; ++q) {
        const int i = threadIdx.x + q * 1024;
        v[q] = i < np ? data[i] : 0;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kUnpackBase / 2 / 1024; ++q) {
        const int i = threadIdx.x + q * 1024;
        if (i < np) {
            data[2 * i] = v[q] & 0x0f;
            data[2 * i + 1] = v[q] >> 4;
        }
    }
}

__global__ __launch_bounds__(256) void unpack_6bit_kernel(const uint8_t* __restrict__ packed,
                                                          uint8_t* __restrict__ out, int64_t n) {
    const int64_t e0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;
    if (e0 >= n) return;
    const int64_t end = min(n, e0 + 16);
    const uint8_t* low = packed;
    const uint8_t* mid = packed + n / 2;
    for (int64_t e = e0; e < end; ++e) {
        const uint8_t lb = low[e >> 1];
        const uint8_t nib = (e & 1) ? (lb >> 4) : (lb & 0x0f);
        const uint8_t m2 = (mid[e >> 2] >> (2 * (e & 3))) & 0x03;
        out[e] = nib | (m2 << 4);
    }
}

// In place: code i takes the 2-bit field (plane[i/4] >> 2*(i%4)) & 3 at bits
// [shift, shift+2), replacing what was there (so a merge is idempotent).
// The plane layout is the mid/high section of a BLOCKLUT8 bit-plane file
// (convert_lut.py:95-110: 4 codes per byte, code 4i in bits 0-1); shift 4
// merges the mid section (the field rule of tensor_engine.cpp:535-548),
// shift 6 the high one.  A thread handles 16 codes: one plane dword, one
// code dwordx4 read-modify-write.
__global__ __launch_bounds__(256) void merge_bitplane_kernel(uint8_t* __restrict__ codes,
                                                             const uint8_t* __restrict__ plane, int64_t n,
                                                             int shift, int vec_ok) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t i0 = q * 16;
    if (i0 >= n) return;
    if (vec_ok && i0 + 16 <= n) {
        const uint32_t p = *reinterpret_cast<const uint32_t*>(plane + q * 4);
        uint4 c = *reinterpret_cast<const uint4*>(codes + i0);
        uint32_t cw[4] = {c.x, c.y, c.z, c.w};
        const uint32_t keep = ~(0x03030303u << shift);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t b = (p >> (8 * k)) & 0xffu;
            // field j of the byte -> bits 0-1 of byte j
            const uint32_t f = (b & 0x03u) | ((b & 0x0cu) << 6) | ((b & 0x30u) << 12) | ((b & 0xc0u) << 18);
            cw[k] = (cw[k] & keep) | (f << shift);
        }
        *reinterpret_cast<uint4*>(codes + i0) = make_uint4(cw[0], cw[1], cw[2], cw[3]);
    } else {
        const int64_t end = min(n, i0 + 16);
        const uint32_t keep = ~(0x03u << shift);
        for (int64_t i = i0; i < end; ++i)
            codes[i] = (uint8_t)((codes[i] & keep) | (((plane[i >> 2] >> (2 * (i & 3))) & 0x03u) << shift));
    }
}

// One-byte codes [n] -> [low nibbles n/2 | bits 4-5 n/4 | bits 6-7 n/4]
// (llama-cpp-port/scripts/convert_lut.py:95-110, runtime/model_offload.py:
// 747-766): low byte i = code 2i | code 2i+1 << 4; mid / high byte i holds
// codes 4i..4i+3, code 4i+k in bits 2k, 2k+1.  A thread packs 16 codes (one
// dwordx4 load; 8 + 4 + 4 bytes stored).
__device__ __forceinline__ uint32_t fields4(uint32_t f) {   // bytes' 2-bit fields -> one byte
    return (f & 0x3u) | ((f >> 6) & 0xcu) | ((f >> 12) & 0x30u) | ((f >> 18) & 0xc0u);
}

__global__ __launch_bounds__(256) void pack_bitplanes_kernel(const uint8_t* __restrict__ codes, int64_t n,
                                                             uint8_t* __restrict__ out, int vec_ok) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t i0 = q * 16;
    if (i0 >= n) return;
    uint8_t* low = out;
    uint8_t* mid = out + n / 2;
    uint8_t* high = out + n / 2 + n / 4;
    if (vec_ok && i0 + 16 <= n) {
        const uint4 c = *reinterpret_cast<const uint4*>(codes + i0);
        const uint32_t w[4] = {c.x, c.y, c.z, c.w};
        uint32_t lo[2] = {0u, 0u}, m = 0u, h = 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t t = w[k] & 0x0f0f0f0fu;   // nibbles of codes 4k..4k+3
            const uint32_t b = (t & 0xfu) | ((t >> 4) & 0xf0u) | ((t >> 8) & 0xf00u) | ((t >> 12) & 0xf000u);
            lo[k >> 1] |= b << (16 * (k & 1));
            m |= fields4((w[k] >> 4) & 0x03030303u) << (8 * k);
            h |= fields4((w[k] >> 6) & 0x03030303u) << (8 * k);
        }
        *reinterpret_cast<uint2*>(low + i0 / 2) = make_uint2(lo[0], lo[1]);
        *reinterpret_cast<uint32_t*>(mid + i0 / 4) = m;
        *reinterpret_cast<uint32_t*>(high + i0 / 4) = h;
    } else {
        const int64_t end = min(n, i0 + 16);
        for (int64_t i = i0; i < end; i += 4) {
            uint32_t m = 0u, h = 0u;
            for (int k = 0; k < 4; ++k) {
                const uint32_t v = codes[i + k];
                m |= ((v >> 4) & 3u) << (2 * k);
                h |= ((v >> 6) & 3u) << (2 * k);
            }
            low[i / 2] = (uint8_t)((codes[i] & 0xfu) | ((codes[i + 1] & 0xfu) << 4));
            low[i / 2 + 1] = (uint8_t)((codes[i + 2] & 0xfu) | ((codes[i + 3] & 0xfu) << 4));
            mid[i / 4] = (uint8_t)m;
            high[i / 4] = (uint8_t)h;
        }
    }
}

inline int grid1(int64_t work, int per_cta) { return (int)((work + per_cta - 1) / per_cta); }

}  // namespace

namespace lutmoe_host {

int launch_ref_dequant(uint16_t* out, const uint8_t* idx, const uint16_t* absmax,
                       const uint16_t* cb, int64_t n_per_expert, int64_t nb_per_expert,
                       int block_size, int num_experts, int64_t out_stride,
                       int64_t idx_stride, hipStream_t s, int64_t cb_stride) {
    const int vec_ok = ((uintptr_t)idx % 16 == 0) && ((uintptr_t)out % 16 == 0) &&
                       (idx_stride % 16 == 0) && (out_stride % 8 == 0);
    dim3 grid(grid1(n_per_expert, 256 * kRefVec), num_experts);
    hipLaunchKernelGGL(ref_dequant_kernel, grid, dim3(256), 0, s, out, idx, absmax, cb, cb_stride,
                       (int)n_per_expert, (int)nb_per_expert, block_size, out_stride,
                       idx_stride, vec_ok);
    return check_launch();
}

int launch_bl4_dequant(uint16_t* out, const uint8_t* codes, const uint16_t* tables,
                       int64_t nblocks, hipStream_t s) {
    hipLaunchKernelGGL(bl4_dequant_kernel, dim3(grid1(nblocks, 128)), dim3(256), 0, s, out,
                       codes, tables, nblocks);
    return check_launch();
}

int launch_nested_group_planes(const uint8_t* planes, int bits, int64_t n, uint8_t* out, hipStream_t s) {
    hipLaunchKernelGGL(nested_group_planes_kernel, dim3(grid1(n / 32, 256)), dim3(256), 0, s,
                       (const uint32_t*)planes, bits, n, (uint32_t*)out);
    return check_launch();
}

int launch_nested_dequant(uint16_t* out, const lutmoe_weights* w, int e0, int ne,
                          hipStream_t s) {
    const int64_t n = (int64_t)w->rows * w->cols;
    dim3 grid(grid1(n, 256 * 32), ne);
    hipLaunchKernelGGL(nested_dequant_kernel, grid, dim3(256), 0, s, out,
                       (const uint8_t* const*)w->codes, (const uint16_t* const*)w->tables,
                       w->tier_bits, e0, n);
    return check_launch();
}

int launch_f16_to_bf16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(f16_to_bf16_kernel, dim3(grid1(n, 256 * 8)), dim3(256), 0, s, in, out,
                       n);
    return check_launch();
}

int launch_unpack_4bit_inplace(uint8_t* data, int64_t n, hipStream_t s) {
    // Region [0, m) holds its packed bytes in [0, m/2).  Peel the upper
    // outputs [h, m) from the packed bytes [h/2, m/2) (disjoint from the
    // writes since h >= m/2), then continue on [0, h).
    int64_t m = n;
    while (m > kUnpackBase) {
        const int64_t h = ((m / 2) + 1) & ~(int64_t)1;
        const int64_t nsrc = m / 2 - h / 2;
        hipLaunchKernelGGL(expand_nibbles_kernel, dim3(grid1(nsrc, 1024)), dim3(256), 0, s,
                           data + h, data + h / 2, nsrc);
        const int rc = check_launch();
        if (rc) return rc;
        m = h;
    }
    hipLaunchKernelGGL(unpack_base_kernel, dim3(1), dim3(1024), 0, s, data, (int)m);
    return check_launch();
}

int launch_pack_bitplanes(const uint8_t* codes, int64_t n, uint8_t* out, hipStream_t s) {
    const int vec_ok = ((uintptr_t)codes % 16 == 0) && ((uintptr_t)out % 8 == 0) && (n % 16 == 0);
    hipLaunchKernelGGL(pack_bitplanes_kernel, dim3(grid1(n, 256 * 16)), dim3(256), 0, s, codes, n, out, vec_ok);
    return check_launch();
}

int launch_merge_bitplane(uint8_t* codes, const uint8_t* plane, int64_t n, int shift, hipStream_t s) {
    const int vec_ok = ((uintptr_t)codes % 16 == 0) && ((uintptr_t)plane % 4 == 0);
    hipLaunchKernelGGL(merge_bitplane_kernel, dim3(grid1(n, 256 * 16)), dim3(256), 0, s, codes, plane, n,
                       shift, vec_ok);
    return check_launch();
}

int launch_unpack_6bit(const uint8_t* packed, uint8_t* out, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(unpack_6bit_kernel, dim3(grid1(n, 256 * 16)), dim3(256), 0, s, packed,
                       out, n);
    return check_launch();
}

}  // namespace lutmoe_host

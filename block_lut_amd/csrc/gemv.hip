// Decode-time LUT-GEMV kernels (HBM-bound).
//
// Work unit: one wavefront owns 8 weight rows ("octet") and walks K in
// chunks of 512 columns.  In a chunk, lane l = 8*g + q covers 8 consecutive
// columns 64*g + 8*q .. +7 of block g, i.e.
//   BL4: one code dword (8 nibbles) per row and one dword of the block's
//        32-byte bf16 table -- codes and tables have the same byte offset
//        (K/2 bytes per row each), so both loads are 256-byte coalesced;
//   REF: one code dwordx2 (8 bytes) per row; the 256-entry codebook is
//        staged once per CTA in LDS as fp32 and the 128-element absmax is
//        factored out per lane ((sum x*cb) * absmax).
// BL4 tables go through a per-wave LDS slot (8 rows x 256 B) so that the
// lookup is one ds_read_u16 per weight at  slot + 32*g + 2*code; the two
// looked-up bf16 values of an element pair feed one v_dot2_f32_bf16 with the
// activation pair.  Partial sums are reduced across the wave at the end.
// These serve the single-matrix entry points (lutmoe_gemv, lut_gemv and
// launch_lut_gemv_kernel); the MoE layer's decode kernels are in decode.hip.
//
// Reference behaviour restated: lut_gemv_kernel
// (vllm_lut/cuda_lut_gemv.py:23-80).
#include "common.h"
#include "kernels.h"

using namespace lutmoe;

namespace {

constexpr int kChunk = 512;          // columns per wave chunk
constexpr int kRows = 8;             // rows per wave
constexpr int kSlot = kRows * 256;   // LDS bytes per wave for BL4 tables

// ------------------------------------------------------------------ decoders

struct Bl4Dec {
    const uint8_t* codes;
    const uint8_t* tabs;
    int K;
    uint32_t cw[kRows], tw[kRows];

    __device__ __forceinline__ void set_expert(const lutmoe_weights& w, int e) {
        const int64_t per = (int64_t)w.rows * (w.cols / 2);
        codes = (const uint8_t*)w.codes + e * per;
        tabs = (const uint8_t*)w.tables + e * per;
        K = w.cols;
    }
    __device__ __forceinline__ void load(const int (&rows)[kRows], int c, int lane, bool ok) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const int64_t off = (int64_t)rows[r] * (K / 2) + c * 256 + 4 * lane;
            cw[r] = ok ? *reinterpret_cast<const uint32_t*>(codes + off) : 0u;
            tw[r] = ok ? *reinterpret_cast<const uint32_t*>(tabs + off) : 0u;
        }
    }
    __device__ __forceinline__ void stage(uint8_t* slot, int lane) const {
#pragma unroll
        for (int r = 0; r < kRows; ++r) *reinterpret_cast<uint32_t*>(slot + r * 256 + 4 * lane) = tw[r];
    }
    template <int TB>
    __device__ __forceinline__ void dot(int r, const uint8_t* slot, int lane, const uint4 (&xq)[TB],
                                        int nt, float (&acc)[TB]) const {
        const uint8_t* tb = slot + r * 256 + ((lane >> 3) << 5);
        const uint32_t w = cw[r];
        const uint32_t we = (w << 1) & 0x1e1e1e1eu;
        const uint32_t wo = (w >> 3) & 0x1e1e1e1eu;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = *reinterpret_cast<const uint16_t*>(tb + ((we >> (8 * j)) & 0xffu));
            const uint32_t hi = *reinterpret_cast<const uint16_t*>(tb + ((wo >> (8 * j)) & 0xffu));
            const uint32_t pr = lo | (hi << 16);
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                if (t < nt) {
                    const uint32_t xv = j == 0 ? xq[t].x : j == 1 ? xq[t].y : j == 2 ? xq[t].z : xq[t].w;
                    acc[t] = dot2_bf16(pr, xv, acc[t]);
                }
            }
        }
    }
    // fp32 activations: each looked-up entry widened to fp32 (exact) and
    // multiplied with its activation by an fp32 FMA
    template <int TB>
    __device__ __forceinline__ void dot_f32(int r, const uint8_t* slot, int lane, const float (&xv)[TB][8],
                                            int nt, float (&acc)[TB]) const {
        const uint8_t* tb = slot + r * 256 + ((lane >> 3) << 5);
        const uint32_t w = cw[r];
        const uint32_t we = (w << 1) & 0x1e1e1e1eu;
        const uint32_t wo = (w >> 3) & 0x1e1e1e1eu;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float lo = bf16_to_f32(*reinterpret_cast<const uint16_t*>(tb + ((we >> (8 * j)) & 0xffu)));
            const float hi = bf16_to_f32(*reinterpret_cast<const uint16_t*>(tb + ((wo >> (8 * j)) & 0xffu)));
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                if (t < nt) {
                    acc[t] = fmaf(xv[t][2 * j], lo, acc[t]);
                    acc[t] = fmaf(xv[t][2 * j + 1], hi, acc[t]);
                }
            }
        }
    }
};

struct RefDec {
    const uint8_t* codes;
    const uint16_t* absmax;
    const float* s_cb;   // LDS fp32 codebook
    int K;
    int64_t nb;          // absmax entries per expert
    int bs;
    uint2 cw[kRows];
    float am[kRows];

    __device__ __forceinline__ void set_expert(const lutmoe_weights& w, int e) {
        codes = (const uint8_t*)w.codes + (int64_t)e * w.rows * w.cols;
        absmax = (const uint16_t*)w.tables + (int64_t)e * w.absmax_per_expert;
        nb = w.absmax_per_expert;
        bs = w.block_size;
        K = w.cols;
    }
    __device__ __forceinline__ void load(const int (&rows)[kRows], int c, int lane, bool ok) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const int64_t flat = (int64_t)rows[r] * K + c * kChunk + 8 * lane;
            cw[r] = ok ? *reinterpret_cast<const uint2*>(codes + flat) : make_uint2(0u, 0u);
            int64_t b = flat / bs;
            b = b < nb ? b : nb - 1;
            am[r] = ok ? bf16_to_f32(absmax[b]) : 0.f;
        }
    }
    __device__ __forceinline__ void stage(uint8_t*, int) const {}
    // kDeq: the dequantised weight bf16(cb * absmax) times x (fused_lut_gemv,
    // vllm_lut/fused_kernel.py:13-46); otherwise lut_gemv's (x * cb) * absmax
    template <int TB, bool kDeq = false>
    __device__ __forceinline__ void dot(int r, const uint8_t*, int, const uint4 (&xq)[TB], int nt,
                                        float (&acc)[TB]) const {
        float s[TB];
#pragma unroll
        for (int t = 0; t < TB; ++t) s[t] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t word = j < 4 ? cw[r].x : cw[r].y;
            const float cv = s_cb[(word >> (8 * (j & 3))) & 0xffu];
            const float v = kDeq ? bf16_to_f32(f32_to_bf16(cv * am[r])) : cv;
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                if (t < nt) {
                    const uint32_t xp = (j >> 1) == 0 ? xq[t].x : (j >> 1) == 1 ? xq[t].y
                                       : (j >> 1) == 2 ? xq[t].z : xq[t].w;
                    const float xv = (j & 1) ? __uint_as_float(xp & 0xffff0000u) : __uint_as_float(xp << 16);
                    s[t] = fmaf(xv, v, s[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TB; ++t) acc[t] = kDeq ? acc[t] + s[t] : fmaf(s[t], am[r], acc[t]);
    }
    // fp32 activations, lut_gemv's product order (x * cb) * absmax
    template <int TB>
    __device__ __forceinline__ void dot_f32(int r, const uint8_t*, int, const float (&xv)[TB][8], int nt,
                                            float (&acc)[TB]) const {
        float s[TB];
#pragma unroll
        for (int t = 0; t < TB; ++t) s[t] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t word = j < 4 ? cw[r].x : cw[r].y;
            const float cv = s_cb[(word >> (8 * (j & 3))) & 0xffu];
#pragma unroll
            for (int t = 0; t < TB; ++t)
                if (t < nt) s[t] = fmaf(xv[t][j], cv, s[t]);
        }
#pragma unroll
        for (int t = 0; t < TB; ++t) acc[t] = fmaf(s[t], am[r], acc[t]);
    }
};

template <class Dec>
__device__ __forceinline__ void init_cb(const lutmoe_weights&, int, float*) {}
template <>
__device__ __forceinline__ void init_cb<RefDec>(const lutmoe_weights& w, int e, float* s_cb) {
    const uint16_t* cb = ref_codebook(w, e);
    for (int i = threadIdx.x; i < 256; i += blockDim.x) s_cb[i] = bf16_to_f32(cb[i]);
}

template <class Dec>
__device__ __forceinline__ void bind_cb(Dec&, const float*) {}
template <>
__device__ __forceinline__ void bind_cb<RefDec>(RefDec& d, const float* s_cb) { d.s_cb = s_cb; }

// One chunk for the wave's 8 rows: load, stage, dot.
template <class Dec, int TB>
__device__ __forceinline__ void octet_chunk(Dec& dec, const int (&rows)[kRows], int c, int nblk_k,
                                            int lane, uint8_t* slot, const uint16_t* const (&xrow)[TB],
                                            int nt, float (&acc)[kRows][TB]) {
    const bool ok = (c * 8 + (lane >> 3)) < nblk_k;
    uint4 xq[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t)
        xq[t] = (ok && t < nt) ? *reinterpret_cast<const uint4*>(xrow[t] + c * kChunk + 8 * lane)
                               : make_uint4(0u, 0u, 0u, 0u);
    dec.load(rows, c, lane, ok);
    dec.stage(slot, lane);
    wave_lds_sync();
    if (ok) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) dec.template dot<TB>(r, slot, lane, xq, nt, acc[r]);
    }
    wave_lds_sync();
}

// The same for fp32 activations (8 floats a lane, two 16-byte loads).
template <class Dec, int TB>
__device__ __forceinline__ void octet_chunk_f32(Dec& dec, const int (&rows)[kRows], int c, int nblk_k,
                                                int lane, uint8_t* slot, const float* const (&xrow)[TB],
                                                int nt, float (&acc)[kRows][TB]) {
    const bool ok = (c * 8 + (lane >> 3)) < nblk_k;
    float xv[TB][8];
#pragma unroll
    for (int t = 0; t < TB; ++t) {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
        if (ok && t < nt) {
            a = *reinterpret_cast<const float4*>(xrow[t] + c * kChunk + 8 * lane);
            b = *reinterpret_cast<const float4*>(xrow[t] + c * kChunk + 8 * lane + 4);
        }
        xv[t][0] = a.x; xv[t][1] = a.y; xv[t][2] = a.z; xv[t][3] = a.w;
        xv[t][4] = b.x; xv[t][5] = b.y; xv[t][6] = b.z; xv[t][7] = b.w;
    }
    dec.load(rows, c, lane, ok);
    dec.stage(slot, lane);
    wave_lds_sync();
    if (ok) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) dec.template dot_f32<TB>(r, slot, lane, xv, nt, acc[r]);
    }
    wave_lds_sync();
}

// -------------------------------------------------------- single-matrix GEMV

// y[t][row] for one expert; CTA = 4 waves, wave w owns rows 8*(4*bx + w) ..
// kXF32: x is fp32 [T][K] (else bf16).
template <class Dec, int TB, bool kXF32>
__global__ __launch_bounds__(256) void gemv_kernel(lutmoe_weights w, int expert,
                                                   const void* __restrict__ x, int T,
                                                   void* __restrict__ y, int y_dtype) {
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[4 * kSlot];
    __shared__ float s_cb[256];
    init_cb<Dec>(w, expert, s_cb);
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int M = w.rows, K = w.cols;
    const int row0 = (blockIdx.x * 4 + wv) * kRows;
    if (row0 >= M) return;
    int rows[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) rows[r] = min(row0 + r, M - 1);
    Dec dec;
    bind_cb(dec, s_cb);
    dec.set_expert(w, expert);
    const int nblk_k = K / kBlockBL;
    const int nch = (K + kChunk - 1) / kChunk;
    uint8_t* slot = s_slot + wv * kSlot;
    for (int tb = 0; tb < T; tb += TB) {
        const int nt = min(TB, T - tb);
        float acc[kRows][TB];
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int t = 0; t < TB; ++t) acc[r][t] = 0.f;
        if constexpr (kXF32) {
            const float* xrow[TB];
#pragma unroll
            for (int t = 0; t < TB; ++t) xrow[t] = (const float*)x + (int64_t)(tb + min(t, nt - 1)) * K;
            for (int c = 0; c < nch; ++c) octet_chunk_f32<Dec, TB>(dec, rows, c, nblk_k, lane, slot, xrow, nt, acc);
        } else {
            const uint16_t* xrow[TB];
#pragma unroll
            for (int t = 0; t < TB; ++t) xrow[t] = (const uint16_t*)x + (int64_t)(tb + min(t, nt - 1)) * K;
            for (int c = 0; c < nch; ++c) octet_chunk<Dec, TB>(dec, rows, c, nblk_k, lane, slot, xrow, nt, acc);
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                const float v = wave_sum(acc[r][t]);
                if (lane == 0 && t < nt && row0 + r < M) {
                    const int64_t o = (int64_t)(tb + t) * M + row0 + r;
                    if (y_dtype == LUTMOE_DTYPE_F32) ((float*)y)[o] = v;
                    else ((uint16_t*)y)[o] = (uint16_t)f32_to_bf16(v);
                }
            }
        }
    }
}

// Reference-shaped single-vector GEMV on REF weights for any K / block size:
// one wave per row, scalar lanes, exact reference product order
// (x * cb) * absmax per element.  Used when the vector path's alignment
// preconditions do not hold.
template <bool kDeq>
__global__ __launch_bounds__(256) void ref_gemv_generic_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ idx, const uint16_t* __restrict__ cbh,
    const float* __restrict__ cbf, const uint16_t* __restrict__ absmax, void* __restrict__ y, int M,
    int K, int T, int nb, int bs, int y_dtype) {
    __shared__ float s_cb[256];
    for (int i = threadIdx.x; i < 256; i += 256) s_cb[i] = cbf ? cbf[i] : bf16_to_f32(cbh[i]);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    for (int t = 0; t < T; ++t) {
        float acc = 0.f;
        for (int c = lane; c < K; c += 64) {
            const int64_t flat = (int64_t)row * K + c;
            int64_t b = flat / bs;
            b = b < nb ? b : nb - 1;
            const float xv = bf16_to_f32(x[(int64_t)t * K + c]);
            const float cv = s_cb[idx[flat]], av = bf16_to_f32(absmax[b]);
            acc += kDeq ? xv * bf16_to_f32(f32_to_bf16(cv * av)) : xv * cv * av;
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            const int64_t o = (int64_t)t * M + row;
            if (y_dtype == LUTMOE_DTYPE_F32) ((float*)y)[o] = acc;
            else ((uint16_t*)y)[o] = (uint16_t)f32_to_bf16(acc);
        }
    }
}

// REF fast path through the octet machinery: wraps the raw reference tensors
// in a one-expert weight description.
template <int TB, bool kDeq>
__global__ __launch_bounds__(256) void ref_gemv_fast_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ idx, const uint16_t* __restrict__ cbh,
    const float* __restrict__ cbf, const uint16_t* __restrict__ absmax, void* __restrict__ y, int M,
    int K, int T, int nb, int bs, int y_dtype) {
    __shared__ float s_cb[256];
    for (int i = threadIdx.x; i < 256; i += 256) s_cb[i] = cbf ? cbf[i] : bf16_to_f32(cbh[i]);
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wv) * kRows;
    if (row0 >= M) return;
    int rows[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) rows[r] = min(row0 + r, M - 1);
    RefDec dec;
    dec.codes = idx;
    dec.absmax = absmax;
    dec.s_cb = s_cb;
    dec.K = K;
    dec.nb = nb;
    dec.bs = bs;
    const int nch = (K + kChunk - 1) / kChunk;
    for (int tb = 0; tb < T; tb += TB) {
        const int nt = min(TB, T - tb);
        const uint16_t* xrow[TB];
#pragma unroll
        for (int t = 0; t < TB; ++t) xrow[t] = x + (int64_t)(tb + min(t, nt - 1)) * K;
        float acc[kRows][TB];
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int t = 0; t < TB; ++t) acc[r][t] = 0.f;
        for (int c = 0; c < nch; ++c) {
            // lane covers columns c*512 + 8*lane .. +7; valid when inside K
            const bool ok = c * kChunk + 8 * lane < K;
            uint4 xq[TB];
#pragma unroll
            for (int t = 0; t < TB; ++t)
                xq[t] = (ok && t < nt) ? *reinterpret_cast<const uint4*>(xrow[t] + c * kChunk + 8 * lane)
                                       : make_uint4(0u, 0u, 0u, 0u);
            dec.load(rows, c, lane, ok);
            if (ok) {
#pragma unroll
                for (int r = 0; r < kRows; ++r) dec.template dot<TB, kDeq>(r, nullptr, lane, xq, nt, acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                const float v = wave_sum(acc[r][t]);
                if (lane == 0 && t < nt && row0 + r < M) {
                    const int64_t o = (int64_t)(tb + t) * M + row0 + r;
                    if (y_dtype == LUTMOE_DTYPE_F32) ((float*)y)[o] = v;
                    else ((uint16_t*)y)[o] = (uint16_t)f32_to_bf16(v);
                }
            }
    }
}


inline int tb_for(int T) { return T <= 1 ? 1 : T <= 2 ? 2 : 4; }

}  // namespace

namespace lutmoe_host {

template <bool kDeq>
static int ref_gemv_dispatch(const uint16_t* x, const uint8_t* idx, const uint16_t* cb_bf16,
                             const float* cb_f32, const uint16_t* absmax, void* y, int M, int K, int T,
                             int num_blocks, int block_size, int y_dtype, hipStream_t s) {
    const bool fast = (K % 8 == 0) && (block_size % 8 == 0) && ((uintptr_t)idx % 8 == 0) &&
                      ((uintptr_t)x % 16 == 0);
    if (!fast) {
        hipLaunchKernelGGL(ref_gemv_generic_kernel<kDeq>, dim3((M + 3) / 4), dim3(256), 0, s, x, idx,
                           cb_bf16, cb_f32, absmax, y, M, K, T, num_blocks, block_size, y_dtype);
        return check_launch();
    }
    const dim3 grid((M + 4 * kRows - 1) / (4 * kRows));
    switch (tb_for(T)) {
        case 1: hipLaunchKernelGGL((ref_gemv_fast_kernel<1, kDeq>), grid, dim3(256), 0, s, x, idx, cb_bf16, cb_f32, absmax, y, M, K, T, num_blocks, block_size, y_dtype); break;
        case 2: hipLaunchKernelGGL((ref_gemv_fast_kernel<2, kDeq>), grid, dim3(256), 0, s, x, idx, cb_bf16, cb_f32, absmax, y, M, K, T, num_blocks, block_size, y_dtype); break;
        default: hipLaunchKernelGGL((ref_gemv_fast_kernel<4, kDeq>), grid, dim3(256), 0, s, x, idx, cb_bf16, cb_f32, absmax, y, M, K, T, num_blocks, block_size, y_dtype); break;
    }
    return check_launch();
}

int launch_ref_gemv(const uint16_t* x, const uint8_t* idx, const uint16_t* cb_bf16,
                    const float* cb_f32, const uint16_t* absmax, void* y, int M, int K, int T,
                    int num_blocks, int block_size, int y_dtype, hipStream_t s, bool dequant) {
    if (dequant)
        return ref_gemv_dispatch<true>(x, idx, cb_bf16, cb_f32, absmax, y, M, K, T, num_blocks, block_size, y_dtype, s);
    return ref_gemv_dispatch<false>(x, idx, cb_bf16, cb_f32, absmax, y, M, K, T, num_blocks, block_size, y_dtype, s);
}

template <class Dec, bool kXF32>
static int gemv_dispatch(const lutmoe_weights* w, int expert, const void* x, int T, void* y,
                         int y_dtype, hipStream_t s) {
    const dim3 grid((w->rows + 4 * kRows - 1) / (4 * kRows));
    switch (tb_for(T)) {
        case 1: hipLaunchKernelGGL((gemv_kernel<Dec, 1, kXF32>), grid, dim3(256), 0, s, *w, expert, x, T, y, y_dtype); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<Dec, 2, kXF32>), grid, dim3(256), 0, s, *w, expert, x, T, y, y_dtype); break;
        default: hipLaunchKernelGGL((gemv_kernel<Dec, 4, kXF32>), grid, dim3(256), 0, s, *w, expert, x, T, y, y_dtype); break;
    }
    return check_launch();
}

int launch_bl4_gemv(const lutmoe_weights* w, int expert, const void* x, bool x_f32, int T, void* y,
                    int y_dtype, hipStream_t s) {
    if (w->format == LUTMOE_FMT_REF)
        return x_f32 ? gemv_dispatch<RefDec, true>(w, expert, x, T, y, y_dtype, s)
                     : gemv_dispatch<RefDec, false>(w, expert, x, T, y, y_dtype, s);
    return x_f32 ? gemv_dispatch<Bl4Dec, true>(w, expert, x, T, y, y_dtype, s)
                 : gemv_dispatch<Bl4Dec, false>(w, expert, x, T, y, y_dtype, s);
}


}  // namespace lutmoe_host

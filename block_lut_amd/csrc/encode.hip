// BL4 encoder on the GPU: per-64-weight-block k-means (k = 16), one
// wavefront per block, lane j holding weight j.
//
// The procedure is LUTQuantizer._train_kmeans (vllm_lut/quantizer.py:120-178)
// applied per block: Lloyd iterations with argmin |x - c| (first minimum),
// mean update leaving empty clusters unchanged, final sort, cast to the
// storage dtype (fp16), codes re-assigned against the stored codebook
// (quantize(), quantizer.py:292-296); in the final 16-means an empty cluster
// is re-seeded at the farthest member instead of being left in place.  Initialisation is a binary-splitting
// tree (4-means from the quantile start sorted[16i+8], then every cell split
// by 2-means twice) instead of a random pick, so CPU and GPU agree exactly.
// Cluster sums are the xor-butterfly over the 64 lanes (non-members add +0)
// and every lane divides the same uniform sum by the same count, so the
// result is bit-identical to the CPU restatement run in the same order.
#include "common.h"
#include "kernels.h"
#include "lut_core.h"

using namespace lutmoe;

namespace {

__device__ __forceinline__ float butterfly(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, kWave);
    return v;
}

template <int K>
__device__ __forceinline__ int argmin_abs(float x, const float (&c)[K]) {
    int best = 0;
    float bd = fabsf(x - c[0]);
#pragma unroll
    for (int i = 1; i < K; ++i) {
        const float dd = fabsf(x - c[i]);
        if (dd < bd) { bd = dd; best = i; }
    }
    return best;
}

template <int K>
__device__ __forceinline__ float pick(const float (&c)[K], int i) {
    float v = c[0];
#pragma unroll
    for (int q = 1; q < K; ++q) v = (i == q) ? c[q] : v;
    return v;
}

// Lloyd on the member lanes; c[] is uniform across the wave.  kReseed: after
// each mean update every empty cluster (index order) moves to the member
// farthest from its own centroid (lowest lane on ties, each lane once per
// iteration) when that distance is > 0.
template <int K, bool kReseed = false>
__device__ void lloyd(float x, bool member, float (&c)[K], int n_iter, int& assign) {
    const int lane = threadIdx.x & 63;
    assign = -1;
    for (int it = 0; it < n_iter; ++it) {
        const int a = member ? argmin_abs<K>(x, c) : -1;
        const bool changed = member && a != assign;
        assign = a;
        if (!__any(changed)) break;
        uint32_t empty = 0;
#pragma unroll
        for (int i = 0; i < K; ++i) {
            const bool in = member && assign == i;
            const float s = butterfly(in ? x : 0.0f);
            const int cnt = __popcll(__ballot(in));
            if (cnt) c[i] = s / (float)cnt;
            else empty |= 1u << i;
        }
        if (kReseed && empty) {
            bool taken = false;
#pragma unroll
            for (int i = 0; i < K; ++i) {
                if (!((empty >> i) & 1u)) continue;
                const float d = (member && !taken) ? fabsf(x - pick(c, assign)) : -1.0f;
                const float mx = wave_reduce_max(d);
                if (!(mx > 0.0f)) break;
                const int j = (int)__builtin_ctzll(__ballot(d == mx));
                c[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), j));
                if (lane == j) taken = true;
            }
        }
    }
}

template <int K>
__device__ __forceinline__ void sort_small(float (&c)[K]) {
#pragma unroll
    for (int i = 1; i < K; ++i) {
        const float v = c[i];
        int j = i - 1;
        while (j >= 0 && c[j] > v) { c[j + 1] = c[j]; --j; }
        c[j + 1] = v;
    }
}

__device__ void split2(float x, bool member, float parent, int n_iter, float (&ch)[2]) {
    const bool any = __any(member);
    if (!any) { ch[0] = ch[1] = parent; return; }
    float lo = member ? x : INFINITY, hi = member ? x : -INFINITY;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        lo = fminf(lo, __shfl_xor(lo, off, kWave));
        hi = fmaxf(hi, __shfl_xor(hi, off, kWave));
    }
    ch[0] = lo;
    ch[1] = hi;
    int a;
    lloyd<2>(x, member, ch, n_iter, a);
    if (ch[1] < ch[0]) { const float t = ch[0]; ch[0] = ch[1]; ch[1] = t; }
}


__global__ __launch_bounds__(256) void bl4_encode_kernel(const float* __restrict__ w,
                                                         int64_t nblocks, int n_iter,
                                                         uint8_t* __restrict__ codes,
                                                         uint16_t* __restrict__ tables) {
    __shared__ float s_x[4][64];
    __shared__ float s_sorted[4][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int64_t b = (int64_t)blockIdx.x * 4 + wv; b < nblocks; b += (int64_t)gridDim.x * 4) {
        const float x = w[b * 64 + lane];
        s_x[wv][lane] = x;
        wave_lds_sync();
        int r = 0;
        for (int i = 0; i < 64; ++i) {
            const float xi = s_x[wv][i];
            r += (xi < x) || (xi == x && i < lane);
        }
        s_sorted[wv][r] = x;
        wave_lds_sync();
        float c2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c2[i] = s_sorted[wv][16 * i + 8];
        wave_lds_sync();
        int a2;
        lloyd<4>(x, true, c2, n_iter, a2);
        // order level-2 cells by centroid (stable insertion order of indices)
        int order[4] = {0, 1, 2, 3};
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            const int v = order[i];
            int j = i - 1;
            while (j >= 0 && pick(c2, order[j]) > pick(c2, v)) { order[j + 1] = order[j]; --j; }
            order[j + 1] = v;
        }
        float c2s[4];
        int rank = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c2s[i] = pick(c2, order[i]);
            rank = (order[i] == a2) ? i : rank;
        }
        a2 = rank;
        float c3[8];
#pragma unroll
        for (int j2 = 0; j2 < 4; ++j2) {
            float ch[2];
            split2(x, a2 == j2, c2s[j2], n_iter, ch);
            c3[j2] = ch[0];
            c3[j2 | 4] = ch[1];
        }
        int cell3;
        {
            const float two[2] = {pick(c3, a2), pick(c3, a2 | 4)};
            cell3 = a2 | (argmin_abs<2>(x, two) << 2);
        }
        float c[16];
#pragma unroll
        for (int k3 = 0; k3 < 8; ++k3) {
            float ch[2];
            split2(x, cell3 == k3, c3[k3], n_iter, ch);
            c[k3] = ch[0];
            c[k3 | 8] = ch[1];
        }
        int a16;
        lloyd<16, true>(x, true, c, n_iter, a16);
        sort_small<16>(c);
        float cf[16];
        uint32_t h_mine = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t h = f32_to_f16(c[i]);
            cf[i] = f16_to_f32(h);
            if (lane == i) h_mine = h;
        }
        const uint32_t code = (uint32_t)argmin_abs<16>(x, cf);
        const uint32_t nb = (uint32_t)__shfl_down((int)code, 1, kWave);
        if ((lane & 1) == 0) codes[b * 32 + (lane >> 1)] = (uint8_t)(code | (nb << 4));
        if (lane < 16) tables[b * 16 + lane] = (uint16_t)h_mine;
    }
}

// REF encoder (the reference's encode_blocklut_kernel,
// vllm_lut/fast_encode.py:22-72): bf16 weights, one fp32[256] codebook,
// blocks of block_size consecutive weights.  Per block: absmax = max |w|
// (fp32, at least 1e-10); each weight w / absmax (IEEE fp32 division) gets
// the index of the nearest codebook entry, the first one on equal distances
// (a scan of all 256 entries: the codebook need not be sorted); absmax is
// stored as bf16 (round to nearest even).  One wave per block; the codebook
// sits in LDS and every lane reads the same entry (a broadcast).
__global__ __launch_bounds__(256) void ref_encode_kernel(const uint16_t* __restrict__ w,
                                                         const float* __restrict__ codebook, int64_t n,
                                                         int block_size, int64_t nblocks,
                                                         uint8_t* __restrict__ codes,
                                                         uint16_t* __restrict__ absmax) {
    __shared__ float s_cb[256];
    s_cb[threadIdx.x] = codebook[threadIdx.x];
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int64_t b = (int64_t)blockIdx.x * 4 + wv; b < nblocks; b += (int64_t)gridDim.x * 4) {
        const int64_t start = b * block_size;
        const int len = (int)min((int64_t)block_size, n - start);
        float mx = 0.f;
        for (int i = lane; i < len; i += 64) mx = fmaxf(mx, fabsf(bf16_to_f32(w[start + i])));
        mx = fmaxf(wave_reduce_max(mx), 1e-10f);
        for (int i = lane; i < len; i += 64) {
            const float v = bf16_to_f32(w[start + i]) / mx;
            float bd = fabsf(v - s_cb[0]);
            int best = 0;
#pragma unroll 8
            for (int c = 1; c < 256; ++c) {
                const float dd = fabsf(v - s_cb[c]);
                if (dd < bd) {
                    bd = dd;
                    best = c;
                }
            }
            codes[start + i] = (uint8_t)best;
        }
        if (lane == 0) absmax[b] = (uint16_t)f32_to_bf16(mx);
    }
}

// The reference's two other REF encoding rules, one wave per block of
// block_size weights, the codebook (or its midpoints) in LDS:
//   kRule 0, LUTQuantizer.quantize (vllm_lut/quantizer.py:242-306, the
//     BLOCKLUT / NESTEDLUT branch; block_size = n is its global "LUT"
//     branch): absmax = max |w| in the weights' dtype, at least 1e-10 in that
//     dtype (:282-283); v = w / absmax, rounded to bf16 for bf16 weights (torch
//     divides bf16 tensors in fp32 and rounds the result, :284); code = the
//     first nearest of the ncb entries by |v - c| in fp32 (argmin, :293-296;
//     the codebook need not be sorted).
//   kRule 1, the offload runtime's encoder (runtime/model_offload.py:
//     897-907): weights as fp32; absmax at least fp32(1e-12); v = w / absmax in
//     fp32; code = the number of midpoints fl32(fl32(c_i + c_{i+1}) / 2) of the
//     ascending codebook below v (np.searchsorted, side "left": a value on a
//     midpoint takes the lower entry, NaN the last).
// absmax is stored as bf16 (round to nearest even).
template <int kRule, bool kBf16In>
__global__ __launch_bounds__(256) void ref_quantize_kernel(const void* __restrict__ w, const float* __restrict__ cb,
                                                           int ncb, int64_t n, int block_size, int64_t nblocks,
                                                           uint8_t* __restrict__ codes,
                                                           uint16_t* __restrict__ absmax) {
    __shared__ float s_c[256];
    const int t = threadIdx.x;
    if (kRule == 0 && t < ncb) s_c[t] = cb[t];
    if (kRule == 1 && t + 1 < ncb) {
        const float sum = cb[t] + cb[t + 1];
        s_c[t] = sum * 0.5f;   // exact halving: equals numpy's fp32 sum / 2.0
    }
    __syncthreads();
    const int lane = t & 63, wv = t >> 6;
    auto load = [&](int64_t i) __attribute__((always_inline)) {
        return kBf16In ? bf16_to_f32(reinterpret_cast<const uint16_t*>(w)[i]) : reinterpret_cast<const float*>(w)[i];
    };
    // the clamp's bound in the dtype the reference clamps in
    const float lo = kRule == 1 ? 1e-12f : kBf16In ? bf16_to_f32(f32_to_bf16(1e-10f)) : 1e-10f;
    for (int64_t b = (int64_t)blockIdx.x * 4 + wv; b < nblocks; b += (int64_t)gridDim.x * 4) {
        const int64_t start = b * block_size;
        const int len = (int)min((int64_t)block_size, n - start);
        float mx = 0.f;
        for (int i = lane; i < len; i += 64) mx = fmaxf(mx, fabsf(load(start + i)));
        mx = fmaxf(wave_reduce_max(mx), lo);
        for (int i = lane; i < len; i += 64) {
            float v = load(start + i) / mx;
            int code;
            if constexpr (kRule == 0) {
                if (kBf16In) v = bf16_to_f32(f32_to_bf16(v));
                float bd = fabsf(v - s_c[0]);
                code = 0;
                for (int c = 1; c < ncb; ++c) {
                    const float dd = fabsf(v - s_c[c]);
                    if (dd < bd) {
                        bd = dd;
                        code = c;
                    }
                }
            } else {
                code = 0;
                for (int c = 0; c + 1 < ncb; ++c) code += s_c[c] < v ? 1 : 0;
                if (v != v) code = ncb - 1;
            }
            codes[start + i] = (uint8_t)code;
        }
        if (lane == 0) absmax[b] = (uint16_t)f32_to_bf16(mx);
    }
}

// 1-D Lloyd k-means (LUTQuantizer._train_kmeans iterations,
// vllm_lut/quantizer.py:158-173): every sample joins its nearest centroid by
// |x - c| (the first one on equal distances, as argmin), then every centroid
// with members becomes their mean (one without members keeps its value).
// The assignment runs one thread per sample with the k <= 256 centroids in
// LDS; the update one CTA per centroid, which sums its members in a fixed
// order (strided by thread, then a fixed tree), so results do not depend on
// scheduling.
__global__ __launch_bounds__(256) void kmeans1d_assign_kernel(const float* __restrict__ x, int64_t n,
                                                              const float* __restrict__ cent, int k,
                                                              int32_t* __restrict__ asg) {
    __shared__ float s_c[256];
    if ((int)threadIdx.x < k) s_c[threadIdx.x] = cent[threadIdx.x];
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float bd = fabsf(v - s_c[0]);
    int bj = 0;
    for (int j = 1; j < k; ++j) {
        const float d = fabsf(v - s_c[j]);
        if (d < bd) {
            bd = d;
            bj = j;
        }
    }
    asg[i] = bj;
}

__global__ __launch_bounds__(256) void kmeans1d_update_kernel(const float* __restrict__ x, int64_t n,
                                                              const int32_t* __restrict__ asg,
                                                              float* __restrict__ cent) {
    __shared__ float s_sum[256];
    __shared__ int s_cnt[256];
    const int j = blockIdx.x, t = threadIdx.x;
    float sum = 0.f;
    int cnt = 0;
    for (int64_t i = t; i < n; i += 256) {
        if (asg[i] == j) {
            sum += x[i];
            ++cnt;
        }
    }
    s_sum[t] = sum;
    s_cnt[t] = cnt;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (t < h) {
            s_sum[t] += s_sum[t + h];
            s_cnt[t] += s_cnt[t + h];
        }
        __syncthreads();
    }
    if (t == 0 && s_cnt[0] > 0) cent[j] = s_sum[0] / (float)s_cnt[0];
}

}  // namespace

namespace lutmoe_host {

int launch_bl4_encode(const float* w, int64_t nblocks, int n_iter, uint8_t* codes,
                      uint16_t* tables, hipStream_t s) {
    int64_t ctas = (nblocks + 3) / 4;
    if (ctas > 65536) ctas = 65536;
    hipLaunchKernelGGL(bl4_encode_kernel, dim3((unsigned)ctas), dim3(256), 0, s, w, nblocks,
                       n_iter, codes, tables);
    return check_launch();
}

int launch_kmeans_1d(const float* x, int64_t n, float* cent, int k, int n_iter, int32_t* asg, hipStream_t s) {
    const unsigned grid = (unsigned)((n + 255) / 256);
    for (int it = 0; it < n_iter; ++it) {
        hipLaunchKernelGGL(kmeans1d_assign_kernel, dim3(grid), dim3(256), 0, s, x, n, cent, k, asg);
        int rc = check_launch();
        if (rc) return rc;
        hipLaunchKernelGGL(kmeans1d_update_kernel, dim3((unsigned)k), dim3(256), 0, s, x, n, asg, cent);
        if ((rc = check_launch())) return rc;
    }
    return LUTMOE_OK;
}

int launch_ref_quantize(const void* w, bool bf16_in, const float* codebook, int ncb, int64_t n, int block_size,
                        int rule, uint8_t* codes, uint16_t* absmax, hipStream_t s) {
    const int64_t nblocks = (n + block_size - 1) / block_size;
    int64_t ctas = (nblocks + 3) / 4;
    if (ctas > 65536) ctas = 65536;
    const dim3 grid((unsigned)ctas), block(256);
    if (rule == 0 && bf16_in)
        hipLaunchKernelGGL((ref_quantize_kernel<0, true>), grid, block, 0, s, w, codebook, ncb, n, block_size, nblocks,
                           codes, absmax);
    else if (rule == 0)
        hipLaunchKernelGGL((ref_quantize_kernel<0, false>), grid, block, 0, s, w, codebook, ncb, n, block_size,
                           nblocks, codes, absmax);
    else if (bf16_in)
        hipLaunchKernelGGL((ref_quantize_kernel<1, true>), grid, block, 0, s, w, codebook, ncb, n, block_size, nblocks,
                           codes, absmax);
    else
        hipLaunchKernelGGL((ref_quantize_kernel<1, false>), grid, block, 0, s, w, codebook, ncb, n, block_size,
                           nblocks, codes, absmax);
    return check_launch();
}

int launch_ref_encode(const uint16_t* w, const float* codebook, int64_t n, int block_size, uint8_t* codes,
                      uint16_t* absmax, hipStream_t s) {
    const int64_t nblocks = (n + block_size - 1) / block_size;
    int64_t ctas = (nblocks + 3) / 4;
    if (ctas > 65536) ctas = 65536;
    hipLaunchKernelGGL(ref_encode_kernel, dim3((unsigned)ctas), dim3(256), 0, s, w, codebook, n, block_size,
                       nblocks, codes, absmax);
    return check_launch();
}

}  // namespace lutmoe_host

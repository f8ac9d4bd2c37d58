// Routing and token permutation (integer/index work).
//
//  route_topk   : softmax(fp32) -> top-k sorted descending (ties to the lower
//                 expert id) -> optional renorm -> x scaling
//                 (vllm_lut/moe_layer.py:358-376; customized/qwen.py:44-54;
//                 models/deepseek/modeling_deepseek.py MoEGate.forward).
//  build_pairs  : (token, slot) pairs with num_shared always-on slots appended.
//  permute      : expert-major, pair-ascending stable order, the order the
//                 llama.cpp mul_mat_id patch builds on the host
//                 (llama-cpp-port/patches/0001:96-110), plus its inverse and
//                 the active-expert list.  One CTA per expert, no atomics on
//                 global memory, deterministic.  Pairs whose expert id is out
//                 of range are dropped (inv = -1) and contribute nothing.
//  combine      : out[t] = sum over slots of y[pos(t, slot)] in slot order
//                 (the un-permute scatter of patches/0001:210-219 plus the
//                 weighted sum of quant_method.py:257-277).
#include "common.h"
#include "kernels.h"

using namespace lutmoe;

namespace {

// One wave per token: lane l holds logits l, l+64, ...; softmax in fp32;
// top-k by logit (softmax is monotone), ties to the lower expert id.
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits,
                                                         int T, int E, int k, int renorm,
                                                         float scaling, float* __restrict__ w,
                                                         int32_t* __restrict__ ids) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const float* l = logits + (int64_t)t * E;
    float mx = -INFINITY;
    for (int e = lane; e < E; e += 64) mx = fmaxf(mx, l[e]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    float sum = 0.f;
    for (int e = lane; e < E; e += 64) sum += expf(l[e] - mx);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, kWave);
    uint64_t taken = 0;
    float wsel = 0.f, wsum = 0.f;
    int isel = 0;
    for (int j = 0; j < k; ++j) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        int q = 0;
        for (int e = lane; e < E; e += 64, ++q) {
            const float v = l[e];
            if (!((taken >> q) & 1ull) && (v > bv || (v == bv && e < bi))) { bv = v; bi = e; }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, kWave);
            const int oi = __shfl_xor(bi, off, kWave);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if ((bi & 63) == lane) taken |= 1ull << (bi >> 6);
        const float p = expf(bv - mx) / sum;
        wsum += p;
        if (lane == j) { wsel = p; isel = bi; }
    }
    if (lane < k) {
        const float v = renorm ? wsel / wsum : wsel;
        w[(int64_t)t * k + lane] = v * scaling;
        ids[(int64_t)t * k + lane] = isel;
    }
}

__global__ __launch_bounds__(256) void build_pairs_kernel(const int32_t* __restrict__ topk_ids,
                                                          const float* __restrict__ topk_w,
                                                          int T, int k, int E, int S,
                                                          int32_t* __restrict__ pair_ids,
                                                          float* __restrict__ pair_w) {
    const int ke = k + S;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= T * ke) return;
    const int t = i / ke, s = i % ke;
    if (s < k) {
        pair_ids[i] = topk_ids[(int64_t)t * k + s];
        pair_w[i] = topk_w[(int64_t)t * k + s];
    } else {
        pair_ids[i] = E + (s - k);
        pair_w[i] = 1.0f;
    }
}

// One CTA per expert id e.  Every CTA builds the full histogram in LDS
// (redundantly; P is small), derives offsets[e] and e's rank among active
// experts, then stably compacts the pairs routed to e.
__global__ __launch_bounds__(256) void permute_kernel(const int32_t* __restrict__ pair_ids,
                                                      int P, int E_tot,
                                                      int32_t* __restrict__ offsets,
                                                      int32_t* __restrict__ perm,
                                                      int32_t* __restrict__ inv,
                                                      int32_t* __restrict__ active) {
    extern __shared__ int32_t s_hist[];          // [E_tot]
    __shared__ int32_t s_wave[4];
    __shared__ int32_t s_base;
    const int e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int i = tid; i < E_tot; i += 256) s_hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < P; i += 256) {
        const int id = pair_ids[i];
        if (id >= 0 && id < E_tot) atomicAdd(&s_hist[id], 1);
        else if (e == 0) inv[i] = -1;     // out-of-range id: the pair is dropped
    }
    __syncthreads();
    if (tid == 0) {
        int off = 0, rank = 0;
        for (int q = 0; q < e; ++q) { off += s_hist[q]; rank += s_hist[q] > 0; }
        offsets[e] = off;
        if (e == E_tot - 1) {
            offsets[E_tot] = off + s_hist[e];
            active[0] = rank + (s_hist[e] > 0);
        }
        if (s_hist[e] > 0) active[1 + rank] = e;
        s_base = off;
    }
    __syncthreads();
    for (int i0 = 0; i0 < P; i0 += 256) {
        const int i = i0 + tid;
        const bool f = i < P && pair_ids[i] == e;
        const uint64_t m = __ballot(f);
        const int before = __popcll(m & ((1ull << lane) - 1ull));
        if (lane == 0) s_wave[wv] = __popcll(m);
        __syncthreads();
        int wbase = s_base;
        for (int q = 0; q < wv; ++q) wbase += s_wave[q];
        if (f) {
            const int pos = wbase + before;
            perm[pos] = i;
            inv[i] = pos;
        }
        __syncthreads();
        if (tid == 0) s_base += s_wave[0] + s_wave[1] + s_wave[2] + s_wave[3];
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y, const int32_t* __restrict__ inv,
                                                      int T, int ke, int H, void* __restrict__ out,
                                                      int out_dtype) {
    const int hq = H / 4;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)T * hq) return;
    const int t = (int)(i / hq), h = (int)(i % hq) * 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int q = 0; q < ke; ++q) {
        const int p = inv[(int64_t)t * ke + q];
        if (p < 0) continue;
        const float4 v = *reinterpret_cast<const float4*>(y + (int64_t)p * H + h);
        s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    if (out_dtype == LUTMOE_DTYPE_F32) {
        *reinterpret_cast<float4*>((float*)out + (int64_t)t * H + h) = s;
    } else {
        const uint32_t a = f32_to_bf16(s.x) | (f32_to_bf16(s.y) << 16);
        const uint32_t b = f32_to_bf16(s.z) | (f32_to_bf16(s.w) << 16);
        *reinterpret_cast<uint2*>((uint16_t*)out + (int64_t)t * H + h) = make_uint2(a, b);
    }
}

}  // namespace

namespace lutmoe_host {

int launch_route_topk(const float* logits, int T, int E, int k, int renorm, float scaling,
                      float* w, int32_t* ids, hipStream_t s) {
    hipLaunchKernelGGL(route_topk_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E,
                       k, renorm, scaling, w, ids);
    return check_launch();
}

int launch_build_pairs(const int32_t* topk_ids, const float* topk_w, int T, int k, int E,
                       int S, int32_t* pair_ids, float* pair_w, hipStream_t s) {
    const int n = T * (k + S);
    hipLaunchKernelGGL(build_pairs_kernel, dim3((n + 255) / 256), dim3(256), 0, s, topk_ids,
                       topk_w, T, k, E, S, pair_ids, pair_w);
    return check_launch();
}

int launch_permute(const int32_t* pair_ids, int T, int k_eff, int E_tot, int32_t* offsets,
                   int32_t* perm, int32_t* inv, int32_t* active, hipStream_t s) {
    const int P = T * k_eff;
    hipLaunchKernelGGL(permute_kernel, dim3(E_tot), dim3(256), E_tot * sizeof(int32_t), s,
                       pair_ids, P, E_tot, offsets, perm, inv, active);
    return check_launch();
}

int launch_combine(const float* y_pos, const int32_t* inv, int T, int k_eff, int H, void* out,
                   int out_dtype, hipStream_t s) {
    const int64_t n = (int64_t)T * (H / 4);
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y_pos,
                       inv, T, k_eff, H, out, out_dtype);
    return check_launch();
}

}  // namespace lutmoe_host

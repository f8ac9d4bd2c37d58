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
//                 the active-expert list.  One CTA per 1024 pairs (E_tot <=
//                 512; one CTA per expert above that), no atomics on global
//                 memory, deterministic.  Pairs whose expert id is out of
//                 range are dropped (inv = -1) and contribute nothing.
//  combine      : out[t] = sum over slots of y[pos(t, slot)] in slot order
//                 (the un-permute scatter of patches/0001:210-219 plus the
//                 weighted sum of quant_method.py:257-277).
#include "common.h"
#include "kernels.h"
#include "lut_core.h"

using namespace lutmoe;

namespace {

// One wave per token: lane l holds logits l, l+64, ... (E <= 4096: one bit
// per held logit in a 64-bit mask); softmax in fp32; top-k by logit (softmax
// is monotone), ties to the lower expert id.
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
        // only NaN left (nothing selectable): id -1, weight 0, as the E <= 64 kernel
        const bool none = bi == 0x7fffffff;
        if (!none && (bi & 63) == lane) taken |= 1ull << (bi >> 6);
        const float p = none ? 0.f : expf(bv - mx) / sum;
        wsum += p;
        if (lane == j) { wsel = p; isel = none ? -1 : bi; }
    }
    if (lane < k) {
        const float v = renorm ? wsel / wsum : wsel;
        w[(int64_t)t * k + lane] = v * scaling;
        ids[(int64_t)t * k + lane] = isel;
    }
}

// E <= 64: lane e holds logit e; max, softmax sum and each of the k top-k
// rounds are DPP wave reductions (no LDS round trips).  A round takes the
// largest order-preserving key; the lowest lane holding it wins (ties ->
// lower expert id; -0 == +0; NaN is never selected, and a round with only
// NaN left yields id -1 and weight 0).
__global__ __launch_bounds__(256) void route_topk_wave_kernel(const float* __restrict__ logits, int T, int E,
                                                              int k, int renorm, float scaling,
                                                              float* __restrict__ w, int32_t* __restrict__ ids) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const float v = lane < E ? logits[(int64_t)t * E + lane] : -INFINITY;
    const float mx = wave_reduce_max(v);
    const float sum = wave_reduce(lane < E ? expf(v - mx) : 0.f);
    int key = lane < E ? float_key(v) : INT_MIN;
    float wsel = 0.f, wsum = 0.f;
    int isel = -1;
    for (int j = 0; j < k; ++j) {
        const int m = wave_max_i32(key);
        const uint64_t b = __ballot(lane < E && key == m && m != INT_MIN);
        const int sel = b ? (int)__builtin_ctzll(b) : -1;
        float p = 0.f;
        if (sel >= 0) {
            const float vs = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), sel));
            p = expf(vs - mx) / sum;
        }
        wsum += p;
        if (lane == j) { wsel = p; isel = sel; }
        if (lane == sel) key = INT_MIN;
    }
    if (lane < k) {
        const float x = renorm ? wsel / wsum : wsel;
        w[(int64_t)t * k + lane] = x * scaling;
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

// Qwen's gated shared expert (customized/qwen.py:99-100): the shared slots
// k..k+S-1 of token t weigh sigmoid(x_t . g).  One wave per token.
__global__ __launch_bounds__(256) void shared_gate_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ g, int T, int H,
                                                          int k, int S, float* __restrict__ pair_w) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= T) return;   // wave-uniform
    const float sw = shared_gate_weight(x + (int64_t)t * H, g, H);
    if (lane < S) pair_w[(int64_t)t * (k + S) + k + lane] = sw;
}

// Router gate (MoEGate.forward, models/deepseek/modeling_deepseek.py:423-470;
// vLLM's bf16 ReplicatedLinear gate in vllm_lut/moe_layer.py:301-304):
// logits[t][e] = x[t] . gate[e] with fp32 accumulation, optionally rounded to
// bf16 (the gate's output dtype in the vLLM layer).  Wave w of CTA (x, t) takes
// expert 4x + w of token t: H/512 rounds of 16-byte loads of x and of the gate
// row, v_dot2_f32_bf16, one wave reduction.  Sized for decode (few tokens).
__global__ __launch_bounds__(256) void router_logits_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ gate, int H, int E,
                                                            float* __restrict__ logits, int round_bf16) {
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y;
    if (e >= E) return;   // wave-uniform
    const uint16_t* xr = x + (int64_t)t * H;
    const uint16_t* gr = gate + (int64_t)e * H;
    float s = 0.f;
    for (int c = lane * 8; c < H; c += 512) {
        const uint4 xv = *reinterpret_cast<const uint4*>(xr + c);
        const uint4 gv = *reinterpret_cast<const uint4*>(gr + c);
        s = dot2_bf16(xv.x, gv.x, s);
        s = dot2_bf16(xv.y, gv.y, s);
        s = dot2_bf16(xv.z, gv.z, s);
        s = dot2_bf16(xv.w, gv.w, s);
    }
    s = wave_reduce(s);
    if (lane == 0) logits[(int64_t)t * E + e] = round_bf16 ? bf16_to_f32(f32_to_bf16(s)) : s;
}

// One CTA per expert id e.  Every CTA builds the full histogram in LDS
// (redundantly; P is small), derives offsets[e] and e's rank among active
// experts, then stably compacts the pairs routed to e.
__global__ __launch_bounds__(256) void permute_kernel(const int32_t* __restrict__ pair_ids,
                                                      int P, int E_tot,
                                                      int32_t* __restrict__ offsets,
                                                      int32_t* __restrict__ perm,
                                                      int32_t* __restrict__ inv,
                                                      int32_t* __restrict__ active,
                                                      int32_t* __restrict__ sched) {
    extern __shared__ int32_t s_hist[];          // [E_tot]
    if (sched && blockIdx.x == 0 && threadIdx.x < 4) sched[threadIdx.x] = 0;
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

// The same permutation as permute_kernel, built from the top-k ids directly:
// pair i = (token i / ke, slot i % ke) is routed expert topk_ids[t][s] for
// s < k and shared expert E + s - k after that.  One CTA of 16 waves per
// 1024 consecutive pairs, no global scratch and no waiting between CTAs.
// Each CTA
//   (a) histograms all P pairs and the pairs before its chunk: the T*k
//       routed ids are read as one flat array, 16 independent loads per
//       thread before any is used, one LDS atomic each (routed id q is pair
//       (q/k)*ke + q%k, and it lies before the chunk exactly when q is below
//       a threshold computed once); the S shared experts' counts are closed
//       forms,
//   (b) wave w counts sub-chunk w (64 pairs) per expert and ranks each pair
//       among the equal ids before it (stable),
//   (c) offsets = exclusive scan of the totals; per expert, an exclusive scan
//       over the 16 sub-chunks starting at offset + pairs before the chunk,
//   (d) pos = that base + rank -> perm, inv; and writes its pairs' ids and
//       weights (pair_ids / pair_w, when given) for the kernels that follow.
// CTA 0 also writes offsets and the active-expert list.  Requires E_tot <= 512.
constexpr int kPermChunk = 1024;
constexpr int kPermSub = kPermChunk / 64;   // = waves per CTA
constexpr int kPermLoads = 16;              // routed ids in flight per thread in (a)

struct PairSrc {
    const int32_t* topk_ids;   // [T][k]
    const float* topk_w;       // [T][k] (nullable)
    int T, k, ke, E;           // ke = k + S; shared expert s has id E + s
};

// Expert of pair i; routed ids outside [0, E) -> -1 (the pair is dropped).
__device__ __forceinline__ int pair_expert(const PairSrc& ps, int i) {
    const int t = i / ps.ke, s = i - t * ps.ke;
    if (s >= ps.k) return ps.E + (s - ps.k);
    const int id = ps.topk_ids[(int64_t)t * ps.k + s];
    return id >= 0 && id < ps.E ? id : -1;
}

__global__ __launch_bounds__(1024) void permute_chunk_kernel(PairSrc ps, int P, int E_tot, int nbits,
                                                             int32_t* __restrict__ offsets,
                                                             int32_t* __restrict__ perm, int32_t* __restrict__ inv,
                                                             int32_t* __restrict__ active,
                                                             int32_t* __restrict__ pair_ids,
                                                             float* __restrict__ pair_w,
                                                             int32_t* __restrict__ sched) {
    extern __shared__ int32_t sm[];   // h_all[E_tot] | h_bef[E_tot] | off[E_tot+1] | sub[kPermSub][E_tot]
    int32_t* h_all = sm;
    int32_t* h_bef = sm + E_tot;
    int32_t* off = sm + 2 * E_tot;
    int32_t* sub = sm + 3 * E_tot + 1;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c0 = blockIdx.x * kPermChunk;
    if (sched && blockIdx.x == 0 && tid < 4) sched[tid] = 0;
    const uint64_t lt = (1ull << lane) - 1ull;
    for (int i = tid; i < (3 + kPermSub) * E_tot + 1; i += blockDim.x) sm[i] = 0;
    __syncthreads();
    // (a) routed ids q < qc are pairs before the chunk: tokens below c0/ke
    // entirely, and of token c0/ke its slots below c0 % ke
    const int nq = ps.T * ps.k;
    const int qc = (c0 / ps.ke) * ps.k + min(c0 % ps.ke, ps.k);
    for (int q0 = tid; q0 < nq; q0 += kPermLoads * (int)blockDim.x) {
        int idv[kPermLoads];
#pragma unroll
        for (int u = 0; u < kPermLoads; ++u) {
            const int q = q0 + u * (int)blockDim.x;
            idv[u] = q < nq ? ps.topk_ids[q] : -1;
        }
#pragma unroll
        for (int u = 0; u < kPermLoads; ++u) {
            const int id = idv[u];
            if (id >= 0 && id < ps.E) {
                atomicAdd(&h_all[id], 1);
                if (q0 + u * (int)blockDim.x < qc) atomicAdd(&h_bef[id], 1);
            }
        }
    }
    // shared expert s: slot k + s of every token; pairs before the chunk are
    // the tokens t with t*ke + k + s < c0
    for (int s = tid; s < ps.ke - ps.k; s += blockDim.x) {
        const int64_t lim = (int64_t)c0 - ps.k - s;
        h_all[ps.E + s] = ps.T;
        h_bef[ps.E + s] = lim <= 0 ? 0 : (int)min((int64_t)ps.T, (lim + ps.ke - 1) / ps.ke);
    }
    // (b) wave wv: sub-chunk wv
    const int i = c0 + wv * 64 + lane;
    const int id = i < P ? pair_expert(ps, i) : -1;
    const bool ok = id >= 0;
    const uint64_t m = match_lanes(id, ok, nbits);
    const int rk = __popcll(m & lt);
    if (ok && rk == 0) sub[wv * E_tot + id] = __popcll(m);
    if (i < P) {
        if (!ok) inv[i] = -1;                  // out-of-range id: the pair is dropped
        if (pair_ids) {
            const int t = i / ps.ke, s = i - t * ps.ke;
            pair_ids[i] = id;
            pair_w[i] = s < ps.k ? ps.topk_w[(int64_t)t * ps.k + s] : 1.0f;
        }
    }
    __syncthreads();
    // (c) offsets (wave 0: lane l owns experts [l*per, l*per+per)), active list
    if (wv == 0) {
        const int per = (E_tot + 63) / 64;
        int c = 0, a = 0;
        for (int q = 0; q < per; ++q) {
            const int e = lane * per + q;
            if (e < E_tot) { c += h_all[e]; a += h_all[e] > 0; }
        }
        int oc = wave_scan_incl(c) - c, oa = wave_scan_incl(a) - a;
        for (int q = 0; q < per; ++q) {
            const int e = lane * per + q;
            if (e < E_tot) {
                off[e] = oc;
                if (blockIdx.x == 0) {
                    offsets[e] = oc;
                    if (h_all[e] > 0) active[1 + oa] = e;
                }
                oc += h_all[e];
                oa += h_all[e] > 0;
            }
        }
        if (lane == 63) {
            off[E_tot] = oc;
            if (blockIdx.x == 0) { offsets[E_tot] = oc; active[0] = oa; }
        }
    }
    __syncthreads();
    for (int e = tid; e < E_tot; e += blockDim.x) {
        int run = off[e] + h_bef[e];
        for (int sc = 0; sc < kPermSub; ++sc) {
            const int v = sub[sc * E_tot + e];
            sub[sc * E_tot + e] = run;
            run += v;
        }
    }
    __syncthreads();
    // (d)
    if (ok) {
        const int pos = sub[wv * E_tot + id] + rk;
        perm[pos] = i;
        inv[i] = pos;
    }
}

// out[t] = sum over the token's positions p (slot order) of y[p], each y[p]
// itself the sum of nsplit partial rows (K-split down projection) at stride
// sstride, added in split order; plus addend[t] when given; one rounding to
// the output dtype.  CTA (t, x) covers columns [1024x, 1024x + 1024) of token
// t, 4 a thread: the token's positions are the same in the whole CTA (scalar
// loads), and a thread issues the loads of all its positions' rows before it
// adds them (in slot order, as one pass over the positions would).  The rows
// are read once: non-temporal loads.
constexpr int kCombineMaxKe = 16;   // k + shared experts (the entry points check it)

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y, const int32_t* __restrict__ inv,
                                                      int T, int ke, int H, void* __restrict__ out,
                                                      int out_dtype, int nsplit, int64_t sstride,
                                                      const float* __restrict__ addend) {
    const int t = blockIdx.x;
    const int h = blockIdx.y * 1024 + threadIdx.x * 4;
    if (h >= H) return;
    int pos[kCombineMaxKe];
#pragma unroll
    for (int q = 0; q < kCombineMaxKe; ++q) pos[q] = q < ke ? inv[(int64_t)t * ke + q] : -1;
    f32x4_t v[kCombineMaxKe];
#pragma unroll
    for (int q = 0; q < kCombineMaxKe; ++q) {
        v[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (pos[q] >= 0) v[q] = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(y + (int64_t)pos[q] * H + h));
    }
    for (int sp = 1; sp < nsplit; ++sp) {
#pragma unroll
        for (int q = 0; q < kCombineMaxKe; ++q)
            if (pos[q] >= 0)
                v[q] += __builtin_nontemporal_load(
                    reinterpret_cast<const f32x4_t*>(y + sp * sstride + (int64_t)pos[q] * H + h));
    }
    f32x4_t sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < kCombineMaxKe; ++q)
        if (pos[q] >= 0) sum += v[q];
    if (addend) sum += *reinterpret_cast<const f32x4_t*>(addend + (int64_t)t * H + h);
    if (out_dtype == LUTMOE_DTYPE_F32) {
        *reinterpret_cast<f32x4_t*>((float*)out + (int64_t)t * H + h) = sum;
    } else {
        const uint32_t a = f32_to_bf16(sum[0]) | (f32_to_bf16(sum[1]) << 16);
        const uint32_t b = f32_to_bf16(sum[2]) | (f32_to_bf16(sum[3]) << 16);
        *reinterpret_cast<uint2*>((uint16_t*)out + (int64_t)t * H + h) = make_uint2(a, b);
    }
}

}  // namespace

namespace lutmoe_host {

int launch_route_topk(const float* logits, int T, int E, int k, int renorm, float scaling,
                      float* w, int32_t* ids, hipStream_t s) {
    if (E <= 64 && k <= 64)
        hipLaunchKernelGGL(route_topk_wave_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, k, renorm,
                           scaling, w, ids);
    else
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

int launch_shared_gate(const uint16_t* x, const uint16_t* gate, int T, int H, int k, int S, float* pair_w,
                       hipStream_t s) {
    hipLaunchKernelGGL(shared_gate_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x, gate, T, H, k, S, pair_w);
    return check_launch();
}

int launch_router_logits(const uint16_t* x, const uint16_t* gate, int T, int H, int E, float* logits,
                         int round_bf16, hipStream_t s) {
    hipLaunchKernelGGL(router_logits_kernel, dim3((E + 3) / 4, T), dim3(256), 0, s, x, gate, H, E, logits,
                       round_bf16);
    return check_launch();
}

int launch_permute(const int32_t* pair_ids, int T, int k_eff, int E_tot, int32_t* offsets,
                   int32_t* perm, int32_t* inv, int32_t* active, hipStream_t s) {
    // pairs = the given ids (k_eff per token, no shared slots)
    return launch_route_pairs(pair_ids, nullptr, T, k_eff, E_tot, 0, offsets, perm, inv, active, nullptr,
                              nullptr, s);
}

int launch_route_pairs(const int32_t* topk_ids, const float* topk_w, int T, int k, int E, int S,
                       int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* active, int32_t* pair_ids,
                       float* pair_w, hipStream_t s, int32_t* sched) {
    const int ke = k + S, E_tot = E + S;
    const int P = T * ke;
    if (E_tot <= 512) {
        int nbits = 1;
        while ((1 << nbits) < E_tot) ++nbits;
        const int nchunk = P > 0 ? (P + kPermChunk - 1) / kPermChunk : 1;
        const size_t lds = ((size_t)(3 + kPermSub) * E_tot + 1) * sizeof(int32_t);
        const PairSrc ps{topk_ids, topk_w, T, k, ke, E};
        hipLaunchKernelGGL(permute_chunk_kernel, dim3(nchunk), dim3(64 * kPermSub), lds, s, ps, P, E_tot, nbits,
                           offsets, perm, inv, active, pair_ids, pair_w, sched);
        return check_launch();
    }
    int rc;
    if (pair_ids) {
        if ((rc = launch_build_pairs(topk_ids, topk_w, T, k, E, S, pair_ids, pair_w, s))) return rc;
    } else if (S != 0) {
        return LUTMOE_EINVAL;
    }
    hipLaunchKernelGGL(permute_kernel, dim3(E_tot), dim3(256), E_tot * sizeof(int32_t), s,
                       pair_ids ? pair_ids : topk_ids, P, E_tot, offsets, perm, inv, active, sched);
    return check_launch();
}

int launch_combine(const float* y_pos, const int32_t* inv, int T, int k_eff, int H, void* out,
                   int out_dtype, hipStream_t s, int nsplit, int64_t split_stride,
                   const float* addend) {
    if (k_eff > kCombineMaxKe) return LUTMOE_EUNSUPPORTED;
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)T, (unsigned)((H + 1023) / 1024)), dim3(256), 0, s, y_pos,
                       inv, T, k_eff, H, out, out_dtype, nsplit, split_stride, addend);
    return check_launch();
}

}  // namespace lutmoe_host

// Decode-time fused MoE layer on BL4 / REF / NestedLUT weights: a gate/up
// kernel and a down kernel per layer (with a routing kernel before them and a
// combine kernel after them when many tokens are routed).
//
//   gate/up : routing -> grouped LUT-GEMV over W13 rows of every active
//             expert -> SwiGLU -> act[position][I] (bf16)
//   down    : grouped LUT-GEMV over W2 rows of every active expert -> each
//             position's rows times its routing weight -> per-token sum in
//             slot order (in LDS, or y[position][H] + combine_kernel)
// One or two tokens whose pairs fit one wave (top-k from logits needs
// E <= 64): every gate/up wave routes in registers (one token: only its own
// slot's expert, from a top-k bitmask) and one wave publishes the routing
// copy to the workspace, which the down kernel reads in place.  Otherwise
// decode_route_kernel routes once into the workspace copy.
//
// Reference behaviour: LUTFusedMoEMethod.apply, decode branch
// (vllm_lut/quant_method.py:250-260), routing of moe_layer._routing
// (vllm_lut/moe_layer.py:358-376), shared experts added with weight 1
// (customized/deepseek.py:111-115).
//
// GEMV layout (lut_core.h): a wave owns 4 or 8 weight rows and walks K in
// 2048-column chunks; codes and tables are both K/2 bytes per row, and a
// row's tables are staged in the wave's LDS slot (block g at 32g), where each
// nibble is looked up.  Lane maps: interleaved (lane l takes the code dwords
// l + 64q of the chunk: every lookup step reads 8 blocks' tables in 8
// distinct bank groups) or contiguous (lane l takes 32 columns).  A chunk's
// loads are all issued (routing inputs, activations, then the weights) before
// any is consumed.
#include <algorithm>

#include "common.h"
#include "kernels.h"
#include "lut_core.h"

using namespace lutmoe;

namespace {

constexpr int kWChunk = 2048;            // columns per lane pass (64 lanes x 32)
constexpr int kRows = 8;
constexpr int kSlot = kRows * 1024;      // LDS bytes per wave: 8 rows' tables of a chunk
constexpr int kMaxEtot = 320;
constexpr int kGuWaves = 1;              // waves per gate/up CTA (4 intermediate indices each)
constexpr int kMaxP = 512;

// Routing result: active experts (ascending), per-expert position offsets,
// the expert-major position -> pair map and its inverse, pair weights.  Lives
// in LDS; the same layout is the global copy written by decode_route_kernel.
struct RouteOut {
    int nact;
    int act[kMaxEtot];                  // active expert ids, ascending
    int aoff[kMaxEtot];                 // first position of active slot a
    int an[kMaxEtot];                   // positions (pairs) of active slot a
    int off[kMaxEtot + 1];
    int perm[kMaxP];
    int inv[kMaxP];
    float pw[kMaxP];
};

// Work items of the precomputed-routing kernels (gate/up CTA rows, down_y
// waves): an active slot's positions cut into chunks of at most C, so one
// heavily routed expert does not hold the layer up behind many passes of
// TB tokens.  C = TB * round(mean positions per active slot / TB), at least
// TB: routing where every expert gets about as many positions keeps one chunk
// per slot.  NestedLUT at two tokens a pass: C = TB (one pass a chunk; its
// register lookups make a chunk's weights cheaper to read again than to look
// up twice).  Stored in the workspace right after the RouteOut copy.
struct RouteChunks {
    int nchunk;
    int ce[kMaxP];                      // expert of chunk c
    int cp0[kMaxP];                     // its first position
    int cn[kMaxP];                      // its positions
};

// The routing weight of each position (pw[perm[p]]), stored after the
// RouteChunks of the global copy: a down-projection wave that knows its first
// position loads its weight in the same round trip as its activations,
// instead of the pair index and then the weight.
struct RoutePosW {
    float w[kMaxP];
};
__device__ __forceinline__ float* route_pos_w(RouteOut* g) {
    return reinterpret_cast<RoutePosW*>(reinterpret_cast<RouteChunks*>(g + 1) + 1)->w;
}
__device__ __forceinline__ const float* route_pos_w(const RouteOut* g) {
    return reinterpret_cast<const RoutePosW*>(reinterpret_cast<const RouteChunks*>(g + 1) + 1)->w;
}

struct RouteScratch {
    int pid[kMaxP];                     // expert of each pair (-1: dropped)
    int rin[kMaxP];                     // rank among same-expert pairs of its 64-pair chunk
    int ccnt[kMaxP / 64][kMaxEtot];     // per chunk, per expert count -> exclusive prefix
};

struct DecodeArgs {
    lutmoe_moe_desc d;
    const uint16_t* x;         // [T][H] bf16
    const float* topk_w;       // [T][k] (ids mode)
    const int32_t* topk_ids;   // [T][k] (ids mode)
    const float* logits;       // [T][E] fp32 (logits mode: topk_ids == nullptr)
    int T, k, renorm;
    int tb;                    // tokens per pass of the expert loops (1, 2 or 4)
    float scaling;
    uint16_t* act;             // [P][I] bf16
    void* out;
    int out_dtype;
    RouteOut* route;           // global copy (precomputed-routing mode)
    const float* addend;       // NULL or fp32 [T][H]: the dense shared expert's rows
};

// out[o] = sum (+ addend[o]), one rounding to the output dtype (o = t * H + h).
__device__ __forceinline__ void store_out(const DecodeArgs& A, int64_t o, float sum) {
    if (A.addend) sum += A.addend[o];
    if (A.out_dtype == LUTMOE_DTYPE_F32) ((float*)A.out)[o] = sum;
    else ((uint16_t*)A.out)[o] = (uint16_t)f32_to_bf16(sum);
}

// Routing + permutation of all T*(k+S) pairs into LDS; identical in every CTA
// that runs it.  Cross-lane work is readlane/DPP only (no LDS round trips in
// the rank loops).
__device__ void cta_route(const DecodeArgs& A, RouteOut& R, RouteScratch& X) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int E = A.d.num_routed, S = A.d.num_shared, E_tot = E + S;
    const int k = A.k, ke = k + S, T = A.T, P = T * ke;
    const int nchunk = (P + 63) / 64;
    for (int i = tid; i < nchunk * E_tot; i += blockDim.x) X.ccnt[i / E_tot][i % E_tot] = 0;
    if (A.topk_ids) {
        for (int p = tid; p < P; p += blockDim.x) {
            const int t = p / ke, s = p - t * ke;
            int e;
            float w;
            if (s < k) {
                e = A.topk_ids[t * k + s];
                w = A.topk_w[t * k + s];
                if (e < 0 || e >= E) e = -1;
            } else {
                e = E + s - k;
                w = 1.0f;
            }
            X.pid[p] = e;
            if (s < k || !A.d.shared_gate) R.pw[p] = w;   // gated shared slots: below
        }
        if (A.d.shared_gate && S > 0) {
            for (int t = wv; t < T; t += (int)(blockDim.x >> 6)) {
                const float sw = shared_gate_weight(A.x + (int64_t)t * A.d.hidden,
                                                    (const uint16_t*)A.d.shared_gate, A.d.hidden);
                if (lane < S) R.pw[t * ke + k + lane] = sw;
            }
        }
    } else {
        // logits mode, wave per token: softmax in fp32; top-k by logit (softmax
        // is monotone): rank(e) = #{e' : l[e'] > l[e] or (l[e'] == l[e], e' < e)}.
        for (int t = wv; t < T; t += (int)(blockDim.x >> 6)) {
            const float* src = A.logits + (int64_t)t * E;
            // E <= 64: one logit per lane, read once for the softmax and the top-k
            const float v = E <= 64 && lane < E ? src[lane] : -INFINITY;
            float mx = fmaxf(-INFINITY, v);   // (a NaN logit drops out, as in the loop)
            for (int e = lane; E > 64 && e < E; e += 64) mx = fmaxf(mx, src[e]);
            mx = wave_reduce_max(mx);
            float ps = E <= 64 && lane < E ? expf(v - mx) : 0.f;
            for (int e = lane; E > 64 && e < E; e += 64) ps += expf(src[e] - mx);
            const float sum = wave_reduce(ps);
            float wsum = 0.f;
            if (E <= 64) {
                // k rounds of a DPP max over int keys (ties -> lowest lane =
                // lower expert id; NaN never selected)
                int key = lane < E ? float_key(v) : INT_MIN;
                for (int j = 0; j < k; ++j) {
                    const int m = wave_max_i32(key);
                    const uint64_t b = __ballot(lane < E && key == m && m != INT_MIN);
                    const int sel = b ? (int)__builtin_ctzll(b) : -1;
                    const float vm = __builtin_bit_cast(
                        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), sel < 0 ? 0 : sel));
                    const float pj = sel < 0 ? 0.f : expf(vm - mx) / sum;
                    wsum += pj;
                    if (lane == 0) {
                        X.pid[t * ke + j] = sel;
                        R.pw[t * ke + j] = pj;
                    }
                    if (lane == sel) key = INT_MIN;
                }
                wave_lds_sync();
                if (lane < k) {
                    const float pj = R.pw[t * ke + lane];
                    R.pw[t * ke + lane] = (A.renorm ? pj / wsum : pj) * A.scaling;
                }
            } else {
                float lsum = 0.f;
                for (int e = lane; e < E; e += 64) {
                    const float v = src[e];
                    int r = 0;
#pragma unroll 8
                    for (int q = 0; q < E; ++q) {
                        const float u = src[q];
                        r += (u > v) || (u == v && q < e);
                    }
                    if (r < k) {
                        const float pj = expf(v - mx) / sum;
                        X.pid[t * ke + r] = e;
                        R.pw[t * ke + r] = pj;
                        lsum += pj;
                    }
                }
                wsum = wave_reduce(lsum);
                wave_lds_sync();
                if (lane < k) {
                    const float pj = R.pw[t * ke + lane];
                    R.pw[t * ke + lane] = (A.renorm ? pj / wsum : pj) * A.scaling;
                }
            }
            const float sw = A.d.shared_gate && S > 0
                                 ? shared_gate_weight(A.x + (int64_t)t * A.d.hidden,
                                                      (const uint16_t*)A.d.shared_gate, A.d.hidden)
                                 : 1.0f;
            if (lane < S) {
                X.pid[t * ke + k + lane] = E + lane;
                R.pw[t * ke + k + lane] = sw;
            }
        }
    }
    __syncthreads();
    // stable ranks inside 64-pair chunks + per-chunk expert counts (equal ids
    // grouped with one ballot per id bit)
    int nbits = 1;
    while ((1 << nbits) < E_tot) ++nbits;
    const uint64_t lt = (1ull << lane) - 1ull;
    for (int c = wv; c < nchunk; c += (int)(blockDim.x >> 6)) {
        const int p = c * 64 + lane;
        const int e = p < P ? X.pid[p] : -1;
        const uint64_t m = match_lanes(e, e >= 0, nbits);
        const int before = __popcll(m & lt), after = __popcll(m & ~lt) - 1;
        if (p < P) X.rin[p] = before;
        if (e >= 0 && after == 0) X.ccnt[c][e] = before + 1;
    }
    __syncthreads();
    if (wv == 0) {
        // lane l owns experts [l*per, l*per+per): totals, chunk prefixes
        const int per = (E_tot + 63) / 64;
        int c = 0, a = 0;
        for (int q = 0; q < per; ++q) {
            const int e = lane * per + q;
            if (e < E_tot) {
                int run = 0;
                for (int ch = 0; ch < nchunk; ++ch) {
                    const int v = X.ccnt[ch][e];
                    X.ccnt[ch][e] = run;
                    run += v;
                }
                c += run;
                a += run > 0;
                R.off[e] = run;   // total for now
            }
        }
        const int ic = wave_scan_incl(c), ia = wave_scan_incl(a);
        int oc = ic - c, oa = ia - a;
        for (int q = 0; q < per; ++q) {
            const int e = lane * per + q;
            if (e < E_tot) {
                const int n = R.off[e];
                R.off[e] = oc;
                if (n > 0) R.act[oa++] = e;
                oc += n;
            }
        }
        if (lane == 63) { R.off[E_tot] = ic; R.nact = ia; }
    }
    __syncthreads();
    for (int a = tid; a < R.nact; a += blockDim.x) {
        const int e = R.act[a];
        R.aoff[a] = R.off[e];
        R.an[a] = R.off[e + 1] - R.off[e];
    }
    for (int p = tid; p < P; p += blockDim.x) {
        const int e = X.pid[p];
        if (e < 0) { R.inv[p] = -1; continue; }
        const int pos = R.off[e] + X.ccnt[p >> 6][e] + X.rin[p];
        R.perm[pos] = p;
        R.inv[p] = pos;
    }
    __syncthreads();
}

// Routing of P = T*(k+S) <= 64 pairs in one wave's registers (the decode
// case).  Lane p holds pair p = t*(k+S) + s: its expert (-1 when dropped or
// p >= P), its weight, and its position in the expert-major order (experts
// ascending, pairs in pair order inside an expert).  Top-k from logits needs
// E <= 64 (lane = expert): k rounds of a DPP wave max, the lowest lane
// holding it wins (ties -> lower id).  Positions come from runtime-bounded
// readlane loops over the P pairs.  Every wave that needs the routing
// computes it itself: no LDS copy, no CTA barrier.
struct WaveRoute {
    int e;        // this lane's pair: expert, -1 if dropped
    float w;      // its weight
    int pos;      // its position, -1 if dropped
    int cnt;      // pairs routed to its expert
    int arank;    // rank of its expert among the active experts
    bool first;   // first pair of its expert
    int nact;     // active experts (wave-uniform)
};

__device__ __forceinline__ bool wave_route_fits(const DecodeArgs& A) {
    const int P = A.T * (A.k + A.d.num_shared);
    return P <= 64 && (A.topk_ids != nullptr || A.d.num_routed <= 64);
}

// kWeights = false: expert ids and positions only (the gate/up CTAs that do
// not publish the routing skip the softmax).
template <bool kWeights>
__device__ __forceinline__ WaveRoute wave_pairs(const DecodeArgs& A) {
    const int lane = threadIdx.x & 63;
    const int E = A.d.num_routed, S = A.d.num_shared;
    const int k = A.k, ke = k + S, T = A.T, P = T * ke;
    int e = -1;
    float w = 0.f;
    if (A.topk_ids) {
        if (lane < P) {
            const int t = lane / ke, sl = lane - t * ke;
            if (sl < k) {
                e = A.topk_ids[t * k + sl];
                if (kWeights) w = A.topk_w[t * k + sl];
                if (e < 0 || e >= E) e = -1;
            } else {
                e = E + sl - k;
                w = 1.0f;
            }
        }
    } else {
        // the first two tokens' logits in flight together (clamped indices,
        // in bounds: E <= 64 here), not one round trip per token
        const int li = min(lane, E - 1);
        const float v0 = A.logits[li];
        const float v1 = A.logits[(int64_t)min(1, T - 1) * E + li];
        for (int t = 0; t < T; ++t) {
            const float raw = t == 0 ? v0 : t == 1 ? v1 : A.logits[(int64_t)t * E + li];
            const float v = lane < E ? raw : -INFINITY;
            int key = lane < E ? float_key(v) : INT_MIN;
            float mx = 0.f, sum = 1.f;
            if (kWeights) {
                mx = wave_reduce_max(v);
                sum = wave_reduce(lane < E ? expf(v - mx) : 0.f);
            }
            float wsum = 0.f;
            for (int j = 0; j < k; ++j) {
                const int m = wave_max_i32(key);
                const uint64_t b = __ballot(lane < E && key == m && m != INT_MIN);
                const int sel = b ? (int)__builtin_ctzll(b) : -1;   // none: NaN logits
                if (lane == t * ke + j) e = sel;
                if (kWeights) {
                    const float vm = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                                   __builtin_bit_cast(int, v), sel < 0 ? 0 : sel));
                    const float pj = expf(vm - mx) / sum;
                    wsum += pj;
                    if (lane == t * ke + j) w = pj;
                }
                if (lane == sel) key = INT_MIN;
            }
            if (kWeights && lane >= t * ke && lane < t * ke + k) w = (A.renorm ? w / wsum : w) * A.scaling;
            if (lane >= t * ke + k && lane < (t + 1) * ke) { e = E + lane - t * ke - k; w = 1.0f; }
        }
    }
    if (kWeights && A.d.shared_gate && S > 0) {
        // Qwen's gated shared expert: its slots of token t weigh sigmoid(x_t . g)
        for (int t = 0; t < T; ++t) {
            const float sw = shared_gate_weight(A.x + (int64_t)t * A.d.hidden, (const uint16_t*)A.d.shared_gate,
                                                A.d.hidden);
            if (lane >= t * ke + k && lane < (t + 1) * ke) w = sw;
        }
    }
    int less = 0, before = 0, cnt = 0;
    for (int q = 0; q < P; ++q) {
        const int u = __builtin_amdgcn_readlane(e, q);
        less += (u >= 0) & (u < e);
        before += (u == e) & (q < lane);
        cnt += (u == e);
    }
    const bool valid = lane < P && e >= 0;
    const uint64_t fm = __ballot(valid && before == 0);
    int arank = 0;
    for (int q = 0; q < P; ++q) {
        const int u = __builtin_amdgcn_readlane(e, q);
        arank += (int)((fm >> q) & 1ull) & (u < e);
    }
    WaveRoute r;
    r.e = valid ? e : -1;
    r.w = w;
    r.pos = valid ? less + before : -1;
    r.cnt = cnt;
    r.arank = arank;
    r.first = valid && before == 0;
    r.nact = __popcll(fm);
    return r;
}

// Active slot a of a routing: expert, first position, number of positions.
struct SlotRef {
    int e, p0, n;
};

// Read access to a routing result, either in this wave's registers
// (WaveRoute) or in LDS (RouteOut), with the same calls.
struct WaveRouteView {
    WaveRoute r;
    __device__ int nact() const { return r.nact; }
    __device__ SlotRef slot(int a) const {
        const uint64_t b = __ballot(r.first && r.arank == a);
        if (!b) return {-1, 0, 0};
        const int L = (int)__builtin_ctzll(b);
        return {__builtin_amdgcn_readlane(r.e, L), __builtin_amdgcn_readlane(r.pos, L),
                __builtin_amdgcn_readlane(r.cnt, L)};
    }
    __device__ SlotRef work(int a) const { return slot(a); }
    // pair at position p (wave-uniform p)
    __device__ int pair_at(int p) const {
        const uint64_t b = __ballot(r.pos == p);
        return b ? (int)__builtin_ctzll(b) : 0;
    }
    __device__ float weight_at(int p) const {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r.w), pair_at(p)));
    }
    // position of pair q (lane-varying q; whole wave must call)
    __device__ int pos_of(int q) const { return __shfl(r.pos, q, 64); }
};

struct LdsRouteView {
    const RouteOut* R;
    __device__ int nact() const { return R->nact; }
    __device__ SlotRef slot(int a) const {
        if (a >= R->nact) return {-1, 0, 0};
        return {R->act[a], R->aoff[a], R->an[a]};
    }
    __device__ SlotRef work(int a) const { return slot(a); }
    __device__ int pair_at(int p) const { return R->perm[p]; }
    __device__ float weight_at(int p) const { return R->pw[R->perm[p]]; }
    __device__ int pos_of(int q) const { return R->inv[q]; }
};

// The routing copy in global memory read in place: a wave reads only its
// slot's expert / first position / count and its positions' pairs and
// weights (wave-uniform indices), with no LDS copy and no CTA barrier.
struct GlobalRouteView {
    const RouteOut* R;
    __device__ int nact() const { return R->nact; }
    __device__ SlotRef slot(int a) const {
        if (a >= R->nact) return {-1, 0, 0};
        return {R->act[a], R->aoff[a], R->an[a]};
    }
    // work item c (a chunk of an active slot's positions)
    __device__ SlotRef work(int c) const {
        const RouteChunks* C = reinterpret_cast<const RouteChunks*>(R + 1);
        if (c >= C->nchunk) return {-1, 0, 0};
        return {C->ce[c], C->cp0[c], C->cn[c]};
    }
    __device__ int pair_at(int p) const { return R->perm[p]; }
    __device__ float weight_at(int p) const { return route_pos_w(R)[p]; }
    __device__ int pos_of(int q) const { return R->inv[q]; }
};

// The wave routing -> the LDS layout (wave 0 writes; callers then barrier).
__device__ __forceinline__ void wave_route_to_lds(const DecodeArgs& A, RouteOut& R) {
    const int lane = threadIdx.x & 63;
    const int P = A.T * (A.k + A.d.num_shared);
    const WaveRoute r = wave_pairs<true>(A);
    if (r.first) {
        R.act[r.arank] = r.e;
        R.aoff[r.arank] = r.pos;
        R.an[r.arank] = r.cnt;
    }
    if (lane < P) {
        R.inv[lane] = r.pos;
        R.pw[lane] = r.w;
        if (r.pos >= 0) R.perm[r.pos] = lane;
    }
    if (lane == 0) R.nact = r.nact;
}

// One wave's register routing -> the global copy (the layout
// decode_route_kernel writes), for the down kernel of the same layer.
__device__ __forceinline__ void wave_route_publish(const DecodeArgs& A, const WaveRoute& r) {
    const int lane = threadIdx.x & 63;
    const int P = A.T * (A.k + A.d.num_shared);
    RouteOut* g = A.route;
    if (r.first) {
        g->act[r.arank] = r.e;
        g->aoff[r.arank] = r.pos;
        g->an[r.arank] = r.cnt;
    }
    if (lane < P) {
        g->inv[lane] = r.pos;
        g->pw[lane] = r.w;
        if (r.pos >= 0) {
            g->perm[r.pos] = lane;
            route_pos_w(g)[r.pos] = r.w;
        }
    }
    if (lane == 0) g->nact = r.nact;
    // one work item per slot
    RouteChunks* c = reinterpret_cast<RouteChunks*>(g + 1);
    if (r.first) {
        c->ce[r.arank] = r.e;
        c->cp0[r.arank] = r.pos;
        c->cn[r.arank] = r.cnt;
    }
    if (lane == 0) c->nchunk = r.nact;
}

// The precomputed routing (decode_route_kernel's global copy) -> LDS.
__device__ __forceinline__ void load_route(const DecodeArgs& A, RouteOut& R) {
    const int E_tot = A.d.num_routed + A.d.num_shared;
    const int P = A.T * (A.k + A.d.num_shared);
    const RouteOut* g = A.route;
    for (int i = threadIdx.x; i < E_tot; i += blockDim.x) {
        R.act[i] = g->act[i];
        R.aoff[i] = g->aoff[i];
        R.an[i] = g->an[i];
    }
    for (int i = threadIdx.x; i < P; i += blockDim.x) {
        R.perm[i] = g->perm[i];
        R.inv[i] = g->inv[i];
        R.pw[i] = g->pw[i];
    }
    if (threadIdx.x == 0) R.nact = g->nact;
    __syncthreads();
}

// Routing into LDS: computed here, or copied from the precomputed global copy.
template <bool kPre>
__device__ __forceinline__ void get_route(const DecodeArgs& A, RouteOut& R, RouteScratch& X) {
    if constexpr (kPre) {
        load_route(A, R);
    } else {
        if (wave_route_fits(A)) {
            if (threadIdx.x < 64) wave_route_to_lds(A, R);
            __syncthreads();
        } else {
            cta_route(A, R, X);
        }
    }
}

// The routing result in LDS -> its global copy (read by later kernels of the
// same layer through get_route<true>).
__device__ __forceinline__ void put_route(const DecodeArgs& A, const RouteOut& R) {
    const int E_tot = A.d.num_routed + A.d.num_shared;
    const int P = A.T * (A.k + A.d.num_shared);
    RouteOut* g = A.route;
    for (int i = threadIdx.x; i < E_tot; i += blockDim.x) {
        g->act[i] = R.act[i];
        g->aoff[i] = R.aoff[i];
        g->an[i] = R.an[i];
    }
    float* pos_w = route_pos_w(g);
    for (int i = threadIdx.x; i < P; i += blockDim.x) {
        g->perm[i] = R.perm[i];
        g->inv[i] = R.inv[i];
        g->pw[i] = R.pw[i];
        if (R.inv[i] >= 0) pos_w[R.inv[i]] = R.pw[i];   // pair i's position
    }
    if (threadIdx.x == 0) g->nact = R.nact;
}

// The slots of R (LDS, complete) -> chunk work items in the global copy.
// Thread a < nact takes slot a (nact <= kMaxEtot <= blockDim.x); chunk
// indices are a block-wide exclusive scan of the per-slot chunk counts.
__device__ __forceinline__ void put_chunks(const DecodeArgs& A, const RouteOut& R) {
    __shared__ int s_wsum[32];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nact = R.nact;
    const int TB = A.tb;   // tokens per pass
    const int pv = nact > 0 ? R.aoff[nact - 1] + R.an[nact - 1] : 0;
    const int navg = nact > 0 ? (pv + nact - 1) / nact : 1;
    const int C = A.d.w13.format == LUTMOE_FMT_NESTED && TB == 2 ? TB : TB * max(1, (navg + TB / 2) / TB);
    const int n = tid < nact ? R.an[tid] : 0;
    const int nc = (n + C - 1) / C;
    const int incl = wave_scan_incl(nc);
    if (lane == 63) s_wsum[wv] = incl;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wv; ++w) base += s_wsum[w];
    RouteChunks* g = reinterpret_cast<RouteChunks*>(A.route + 1);
    const int first = base + incl - nc;
    for (int j = 0; j < nc; ++j) {
        g->ce[first + j] = R.act[tid];
        g->cp0[first + j] = R.aoff[tid] + j * C;
        g->cn[first + j] = min(C, n - j * C);
    }
    if (tid == (int)blockDim.x - 1) g->nchunk = base + incl;
}

// One CTA of 16 waves (one token per wave in the top-k loop for T <= 16).
__global__ __launch_bounds__(1024) void decode_route_kernel(DecodeArgs A) {
    __shared__ RouteOut R;
    __shared__ RouteScratch X;
    cta_route(A, R, X);
    put_route(A, R);
    put_chunks(A, R);
}

// One wave, 8 BL4 rows, one 2048-column chunk cc of K.  Codes and tables
// are both K/2 bytes per row.  Tables: lane l loads bytes [1024cc + 16l, +16)
// of each row's tables (half of block l/2's bf16[16]) and stages them at 16l
// of the row's 1 KB of LDS (block g at 32g).  Codes, in one of two lane maps:
//  * contiguous (two tokens a pass or fewer): lane l takes the row's 16 bytes
//    at 16l, columns [2048cc + 32l, +32) of its own block's half; one load;
//  * interleaved (four tokens a pass): lane l takes the chunk's code dwords
//    d = l, l + 64, l + 128, l + 192 (columns [2048cc + 8d, +8)), so in each
//    lookup step the 64 lanes use the tables of 8 consecutive blocks, which
//    sit in 8 distinct LDS bank groups (no bank conflicts), and a row of
//    K = 1408 (176 dwords) keeps 44 of 48 lane steps busy.  Four dword loads
//    a row: with four tokens they pay (T = 32: 155 -> 151 us a layer); with
//    two the extra loads and registers cost more than the conflicts (T = 8:
//    70 -> 86 us).
// Code loads past K read nothing (interleaved: lane-conditional loads, which
// keep the 256-byte step in the instruction offset; the 4-row loop instead
// clamps them) or the chunk start (contiguous); their lookups meet zero
// tables and, interleaved, zeroed activations.
template <int TB>
constexpr bool bl4_interleaved() { return TB >= 4; }

struct Rows8 {
    uint32_t cw[kRows][4];   // the lane's 4 code dwords of each row
    u32x4_t tw[kRows];
};

__device__ __forceinline__ int chunk_dwords(int K, int cc) { return min(K - cc * kWChunk, kWChunk) / 8; }

template <int TB>
__device__ __forceinline__ void load_rows8(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ tabs,
                                           const int (&rows)[kRows], int K, int cc, int lane, Rows8& b) {
    const int nd = chunk_dwords(K, cc);
    const bool okt = cc * kWChunk + 32 * lane < K;
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        // 32-bit offsets from the expert's (wave-uniform) bases
        const uint32_t ro = (uint32_t)rows[r] * (uint32_t)(K / 2) + cc * (kWChunk / 2);
        if constexpr (bl4_interleaved<TB>()) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                b.cw[r][q] = 0u;
                if (lane + 64 * q < nd)
                    b.cw[r][q] = *reinterpret_cast<const uint32_t*>(codes + (ro + 4 * lane + 256 * q));
            }
        } else {
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(codes + (ro + (okt ? 16 * lane : 0)));
#pragma unroll
            for (int q = 0; q < 4; ++q) b.cw[r][q] = v[q];
        }
        b.tw[r] = *reinterpret_cast<const u32x4_t*>(tabs + (ro + (okt ? 16 * lane : 0)));
    }
}

// The activations of the lane's BL4 code dwords in the interleaved map, up
// to TB vectors: xs[t][4q + i] = columns 8d + 2i, 8d + 2i + 1 of chunk cc
// (d = l + 64q); zero past K, where the codes meet zero tables.  Vectors past
// nt are dropped.  Lane-conditional loads, which keep the 512-column step in
// the instruction offset (the 8-row loop's registers are tight).
template <int TB>
__device__ __forceinline__ void load_xi(const uint16_t* const (&xrow)[TB], int K, int cc, int lane,
                                        uint32_t (&xs)[TB][16]) {
    const int nd = chunk_dwords(K, cc);
#pragma unroll
    for (int t = 0; t < TB; ++t) {
        const uint16_t* p = xrow[t] + cc * kWChunk + 8 * lane;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 v = {0u, 0u, 0u, 0u};
            if (lane + 64 * q < nd) v = *reinterpret_cast<const uint4*>(p + 512 * q);
            xs[t][4 * q + 0] = v.x;
            xs[t][4 * q + 1] = v.y;
            xs[t][4 * q + 2] = v.z;
            xs[t][4 * q + 3] = v.w;
        }
    }
}

// As load_xi, with every load issued (past K the chunk's last 8 columns,
// zeroed by mask_xi once the weight loads are issued; masking here would make
// the weight loads wait for these): no load sits under a lane condition, so
// the compiler's waits cover each row's own loads only (the 4-row loop).
template <int TB>
__device__ __forceinline__ void load_xi_all(const uint16_t* const (&xrow)[TB], int K, int cc, int lane,
                                            uint32_t (&xs)[TB][16]) {
    const int nd = chunk_dwords(K, cc);
#pragma unroll
    for (int t = 0; t < TB; ++t) {
        const uint16_t* p = xrow[t] + cc * kWChunk;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 v = *reinterpret_cast<const uint4*>(p + 8 * min(lane + 64 * q, nd - 1));
            xs[t][4 * q + 0] = v.x;
            xs[t][4 * q + 1] = v.y;
            xs[t][4 * q + 2] = v.z;
            xs[t][4 * q + 3] = v.w;
        }
    }
}

// Zero the activations load_xi_all read past K (their codes meet zero tables; a
// zero activation keeps an infinite one out of the sum).
template <int TB>
__device__ __forceinline__ void mask_xi(int K, int cc, int lane, uint32_t (&xs)[TB][16]) {
    const int nd = chunk_dwords(K, cc);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t m = lane + 64 * q < nd ? 0xffffffffu : 0u;
#pragma unroll
        for (int t = 0; t < TB; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) xs[t][4 * q + i] &= m;
    }
}

// The lane's 32 activations of up to TB vectors (dword 4j+i = columns 8j+2i,
// 8j+2i+1 of its 32).  Lanes past K (and vectors past nt) read valid
// activations that meet zero tables (past K) or are dropped (past nt).
template <int TB>
__device__ __forceinline__ void load_x8(const uint16_t* const (&xrow)[TB], int K, int cc, int lane, int nt,
                                        uint32_t (&xs)[TB][16]) {
    const bool ok = cc * kWChunk + 32 * lane < K;
#pragma unroll
    for (int t = 0; t < TB; ++t) {
        const uint16_t* p = xrow[t] + (ok ? cc * kWChunk + 32 * lane : 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 v = *reinterpret_cast<const uint4*>(p + 8 * q);
            xs[t][4 * q + 0] = v.x;
            xs[t][4 * q + 1] = v.y;
            xs[t][4 * q + 2] = v.z;
            xs[t][4 * q + 3] = v.w;
        }
    }
}

// Row by row: stage row r's tables of the chunk in its 1 KB of the wave's LDS
// slot (block g at r*1024 + 32g), then look its codes up there and
// accumulate (code dword q: block l/2 contiguous, l/8 + 8q interleaved); row
// r only waits for its own loads, so the first rows are done while the later
// ones are still arriving.  `ok`: the lane's table bytes lie inside K; `nd`:
// the chunk's code dwords per row (interleaved: steps q with 64q >= nd hold
// no code and are skipped, e.g. q = 3 at K = 1408).
template <int TB>
__device__ __forceinline__ void compute_rows8(const Rows8& b, const uint32_t (&xs)[TB][16], bool ok, int lane,
                                              int nd, uint8_t* slot, int nt, float (&acc)[kRows][TB]) {
    constexpr bool kInter = bl4_interleaved<TB>();
    const uint32_t tab = lds_addr(slot) + (kInter ? (lane >> 3) << 5 : (lane >> 1) << 5);
    const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        // lanes past K stage zero tables (their loads read the row start)
        *reinterpret_cast<u32x4_t*>(slot + r * 1024 + 16 * lane) = ok ? b.tw[r] : z;
        wave_lds_sync();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (kInter && 64 * q >= nd) break;
            uint32_t xj[TB][4];
#pragma unroll
            for (int t = 0; t < TB; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) xj[t][i] = xs[t][4 * q + i];
            bl4_dot8<TB>(b.cw[r][q], tab + r * 1024 + (kInter ? 256 * q : 0), xj, nt, acc[r]);
        }
    }
    wave_lds_sync();
}

// All of K, chunk by chunk: activations first (small), then the weights.
template <int TB>
__device__ __forceinline__ void bl4_rows8(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ tabs,
                                          const int (&rows)[kRows], int K, int lane, uint8_t* slot,
                                          const uint16_t* const (&xrow)[TB], int nt, float (&acc)[kRows][TB]) {
    const int nch = (K + kWChunk - 1) / kWChunk;
    for (int cc = 0; cc < nch; ++cc) {
        Rows8 b;
        uint32_t xs[TB][16];
        if constexpr (bl4_interleaved<TB>()) load_xi<TB>(xrow, K, cc, lane, xs);
        else load_x8<TB>(xrow, K, cc, lane, nt, xs);
        __builtin_amdgcn_sched_barrier(0);
        load_rows8<TB>(codes, tabs, rows, K, cc, lane, b);
        // every load in flight before the first row is consumed
        __builtin_amdgcn_sched_barrier(0);
        compute_rows8<TB>(b, xs, cc * kWChunk + 32 * lane < K, lane, chunk_dwords(K, cc), slot, nt, acc);
    }
}

// ---- NestedLUT experts (NestedView, lut_core.h).
// The lane's 32 columns [2048cc + 32l, +32) of 8 rows: one 32-weight group
// of the device layout per row (two 2-bit field words, the bit-2 and bit-3
// words: the tier's 4b bytes, one load), and 16 bytes of the row's tables
// starting at this lane's share of its block's table (2^b bytes: entries
// 2^(b-1)*(l%2) ..).
struct Rows8N {
    uint32_t f01[kRows][2], f2[kRows], f3[kRows];
    u32x4_t tw[kRows];
};

// kRegTab: each lane loads its block's whole table (b <= 3: 2^(b+1) <= 16
// bytes) for register lookups instead of its share of it.
template <int kBits, bool kRegTab = false>
__device__ __forceinline__ void load_rows8n(const NestedView& v, const int (&rows)[kRows], int K, int cc,
                                            int lane, Rows8N& b) {
    const bool ok = cc * kWChunk + 32 * lane < K;
    const uint32_t c0 = ok ? cc * kWChunk + 32 * lane : 0;
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const uint32_t i0 = (uint32_t)rows[r] * (uint32_t)K + c0;
        const int go = (int)(i0 / 32 * (4 * kBits));   // the group's bytes: the tier's only
        if constexpr (kBits == 4) {
            const auto q = __builtin_amdgcn_raw_buffer_load_b128(v.codes, go, 0, 0);
            b.f01[r][0] = q[0];
            b.f01[r][1] = q[1];
            b.f2[r] = q[2];
            b.f3[r] = q[3];
        } else if constexpr (kBits == 3) {
            const auto q = __builtin_amdgcn_raw_buffer_load_b96(v.codes, go, 0, 0);
            b.f01[r][0] = q[0];
            b.f01[r][1] = q[1];
            b.f2[r] = q[2];
            b.f3[r] = 0u;
        } else {
            const auto q = __builtin_amdgcn_raw_buffer_load_b64(v.codes, go, 0, 0);
            b.f01[r][0] = q[0];
            b.f01[r][1] = q[1];
            b.f2[r] = 0u;
            b.f3[r] = 0u;
        }
        const uint32_t tofs = ((i0 >> 6) << (v.bits + 1)) + (kRegTab ? 0u : (uint32_t)(lane & 1) << v.bits);
        if constexpr (kRegTab && kBits == 2) {   // the 8-byte table only
            const auto q = __builtin_amdgcn_raw_buffer_load_b64(v.table, (int)tofs, 0, 0);
            b.tw[r] = u32x4_t{q[0], q[1], 0u, 0u};
        } else {
            b.tw[r] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(v.table, (int)tofs, 0, 0));
        }
    }
}

// Row by row: the 16 table bytes go to the block's 32-byte LDS slot at this
// lane's share (for b < 4 the two lanes of a block write overlapping bytes
// with the same values, and a lookup only reads the first 2^(b+1) bytes);
// codes are rebuilt as BL4 nibbles and looked up as for BL4.
template <int TB, int kBits>
__device__ __forceinline__ void compute_rows8n(const Rows8N& b, const uint32_t (&xs)[TB][16], bool ok, int bits,
                                               int lane, uint8_t* slot, int nt, float (&acc)[kRows][TB]) {
    const uint32_t tab = lds_addr(slot) + ((lane >> 1) << 5);
    const int woff = ((lane >> 1) << 5) + ((lane & 1) << bits);
    const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        *reinterpret_cast<u32x4_t*>(slot + r * 1024 + woff) = ok ? b.tw[r] : z;
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t w = nested_code8<kBits>(b.f01[r][0], b.f01[r][1], b.f2[r], b.f3[r], j);
            uint32_t xj[TB][4];
#pragma unroll
            for (int t = 0; t < TB; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) xj[t][i] = xs[t][4 * j + i];
            bl4_dot8<TB>(w, tab + r * 1024, xj, nt, acc[r]);
        }
    }
    wave_lds_sync();
}

template <int TB, int kBits>
__device__ __forceinline__ void nested_rows8_tier(const NestedView& v, const int (&rows)[kRows], int K, int lane,
                                                  uint8_t* slot, const uint16_t* const (&xrow)[TB], int nt,
                                                  float (&acc)[kRows][TB]) {
    const int nch = (K + kWChunk - 1) / kWChunk;
    for (int cc = 0; cc < nch; ++cc) {
        Rows8N b;
        uint32_t xs[TB][16];
        load_x8<TB>(xrow, K, cc, lane, nt, xs);
        __builtin_amdgcn_sched_barrier(0);
        load_rows8n<kBits>(v, rows, K, cc, lane, b);
        __builtin_amdgcn_sched_barrier(0);
        compute_rows8n<TB, kBits>(b, xs, cc * kWChunk + 32 * lane < K, kBits, lane, slot, nt, acc);
    }
}

// the expert's tier is wave-uniform: one code path per tier
template <int TB>
__device__ __forceinline__ void nested_rows8(const NestedView& v, const int (&rows)[kRows], int K, int lane,
                                             uint8_t* slot, const uint16_t* const (&xrow)[TB], int nt,
                                             float (&acc)[kRows][TB]) {
    if (v.bits == 2) nested_rows8_tier<TB, 2>(v, rows, K, lane, slot, xrow, nt, acc);
    else if (v.bits == 3) nested_rows8_tier<TB, 3>(v, rows, K, lane, slot, xrow, nt, acc);
    else nested_rows8_tier<TB, 4>(v, rows, K, lane, slot, xrow, nt, acc);
}

// Tiers of 2 and 3 bits looked up in registers: the lane's block table (at
// most 8 entries; a 2-bit table's upper four are zero and never selected) as
// byte planes, one v_perm_b32 per plane and four codes, so these experts use
// no LDS.  The weights come in regtab_lookup8_eo's order (w0, w2 | w4, w6 |
// w1, w3 | w5, w7: four v_perm fewer per 8 weights than column order) and
// meet activations put in the same order once per chunk (xe).
// Every token of the pass is computed (a token past the pass's count repeats
// its last one and is not stored): per-token guards here become branches
// that keep the lookups' results live across them, and the four-token pass
// then spills.
template <int TB, int kBits>
__device__ __forceinline__ void compute_rows8n_reg(const Rows8N& b, const uint32_t (&xe)[TB][16], bool ok,
                                                   float (&acc)[kRows][TB]) {
    const uint32_t m = ok ? ~0u : 0u;   // lanes past K: zero tables
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        __builtin_amdgcn_sched_barrier(0);   // row by row, as the LDS path (register pressure)
        const uint32_t T[4] = {b.tw[r][0] & m, b.tw[r][1] & m, b.tw[r][2] & m, b.tw[r][3] & m};
        uint32_t lo[2], hi[2];
        table_planes<kBits>(T, lo, hi);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4_t pr =
                regtab_lookup8_eo<kBits>(lo, hi, nested_code8<kBits>(b.f01[r][0], b.f01[r][1], b.f2[r], 0u, j));
#pragma unroll
            for (int t = 0; t < TB; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[r][t] = dot2_bf16(pr[i], xe[t][4 * j + i], acc[r][t]);
        }
    }
}

// The 2- and 3-bit tiers looked up in registers (no LDS), one code path per
// tier (codes and planes of the tier's own width: T = 16 90-92 -> 87-90 us
// against one path for both; the loads read nothing past the expert's
// bytes); the 4-bit tier keeps the LDS lookups.
template <int TB, int kBits>
__device__ __forceinline__ void nested_rows8_reg(const NestedView& v, const int (&rows)[kRows], int K, int lane,
                                                 const uint16_t* const (&xrow)[TB], int nt, float (&acc)[kRows][TB]) {
    const int nch = (K + kWChunk - 1) / kWChunk;
    for (int cc = 0; cc < nch; ++cc) {
        Rows8N b;
        uint32_t xs[TB][16];
        load_x8<TB>(xrow, K, cc, lane, nt, xs);
        __builtin_amdgcn_sched_barrier(0);
        load_rows8n<kBits, true>(v, rows, K, cc, lane, b);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t xe[TB][16];   // the activations in regtab_lookup8_eo's order
#pragma unroll
        for (int t = 0; t < TB; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4_t o = eo_order(u32x4_t{xs[t][4 * j], xs[t][4 * j + 1], xs[t][4 * j + 2], xs[t][4 * j + 3]});
#pragma unroll
                for (int i = 0; i < 4; ++i) xe[t][4 * j + i] = o[i];
            }
        compute_rows8n_reg<TB, kBits>(b, xe, cc * kWChunk + 32 * lane < K, acc);
    }
}

template <int TB>
__device__ __forceinline__ void nested_rows8_any(const NestedView& v, const int (&rows)[kRows], int K, int lane,
                                                 uint8_t* slot, const uint16_t* const (&xrow)[TB], int nt,
                                                 float (&acc)[kRows][TB]) {
    if (v.bits == 4) nested_rows8_tier<TB, 4>(v, rows, K, lane, slot, xrow, nt, acc);
    else if (v.bits == 3) nested_rows8_reg<TB, 3>(v, rows, K, lane, xrow, nt, acc);
    else nested_rows8_reg<TB, 2>(v, rows, K, lane, xrow, nt, acc);
}

// ---- REF experts (the reference's uint8 codes, bf16 absmax per block_size
// flat elements, one bf16[256] codebook).  The lane's 32 columns
// [2048cc + 32l, +32) of 8 rows: 32 code bytes and the absmax of their block
// (block_size % 32 == 0, so 32 aligned columns share one block; block
// indices are clamped to the last entry as the reference's dequant does).
// Per row the lane sums x * cb over its 32 columns and scales the sum by the
// absmax: the reference GEMV's fp32 (x * cb) * absmax, factored per 32
// columns.  The codebook sits in the first 512 bytes of the wave's LDS slot.
struct Rows8R {
    u32x4_t cw[kRows][2];
    uint32_t am[kRows];
};

// The absmax block of the 32 aligned columns starting at flat element 32u of
// an expert: u / (block_size / 32), clamped to the last block.  32-bit (the
// host keeps REF experts on these kernels below 2^37 elements); a 64-bit
// division per row cost ~140 instructions between the rows' loads.
__device__ __forceinline__ uint32_t ref_block32(uint32_t u, uint32_t q32, uint32_t nb) {
    return min(u / q32, nb - 1u);
}

__device__ __forceinline__ void load_rows8r(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ am,
                                            int64_t nb, int bs, const int (&rows)[kRows], int K, int cc, int lane,
                                            Rows8R& b) {
    const bool ok = cc * kWChunk + 32 * lane < K;
    const uint32_t q32 = (uint32_t)bs / 32u;
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int64_t off = (int64_t)rows[r] * K + (ok ? cc * kWChunk + 32 * lane : 0);
        b.cw[r][0] = *reinterpret_cast<const u32x4_t*>(codes + off);
        b.cw[r][1] = *reinterpret_cast<const u32x4_t*>(codes + off + 16);
        const uint32_t u = (uint32_t)rows[r] * (uint32_t)(K / 32) + (ok ? (uint32_t)(cc * (kWChunk / 32) + lane) : 0u);
        b.am[r] = am[ref_block32(u, q32, (uint32_t)nb)];
    }
}

// 32 REF byte codes against the fp32[256] codebook at LDS byte address
// `cbase`, with the weights the reference's dequantisation produces:
// w = bf16_rne(cb[c] * absmax) (the product of two bf16 values is exact in
// fp32; v_cvt_pk_bf16_f32 rounds to nearest even), then g[t] += x_t . w with
// one v_dot2_f32_bf16 per weight pair.
template <int TB>
__device__ __forceinline__ void ref_dot32_deq(const u32x4_t (&cw)[2], uint32_t cbase, float a,
                                              const uint32_t (&x)[TB][16], int nt, float (&g)[TB]) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        const uint32_t w = cw[d >> 2][d & 3];
        const uint32_t we = (w << 2) & 0x03fc03fcu;   // 4 * code of columns 4d, 4d+2 (16-bit fields)
        const uint32_t wo = (w >> 6) & 0x03fc03fcu;   // 4 * code of columns 4d+1, 4d+3
        const float c0 = __uint_as_float(lds_ld32(add_word<0>(cbase, we)));
        const float c1 = __uint_as_float(lds_ld32(add_word<0>(cbase, wo)));
        const float c2 = __uint_as_float(lds_ld32(add_word<1>(cbase, we)));
        const float c3 = __uint_as_float(lds_ld32(add_word<1>(cbase, wo)));
        const f32x2_t q0 = {c0 * a, c1 * a}, q1 = {c2 * a, c3 * a};
        const uint32_t p0 = __builtin_bit_cast(uint32_t, __builtin_convertvector(q0, bf16x2v_t));
        const uint32_t p1 = __builtin_bit_cast(uint32_t, __builtin_convertvector(q1, bf16x2v_t));
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            if (t < nt) {
                g[t] = dot2_bf16(p0, x[t][2 * d], g[t]);
                g[t] = dot2_bf16(p1, x[t][2 * d + 1], g[t]);
            }
        }
    }
}

// REF rows of one expert.  One token per pass (TB == 1, i.e. T == 1) follows
// the reference's decode GEMV (vllm_lut/quant_method.py:250-260 ->
// cuda_lut_gemv.py:50-57): fp32 (x * cb) * absmax, factored per 32 columns.
// Several tokens (TB > 1, T >= 2) follow its other branch (quant_method.py:
// 261-277): the dequantised bf16 weights bf16(cb * absmax), then the matmul.
template <int TB>
__device__ __forceinline__ void ref_rows8(const lutmoe_weights& w, int e, const int (&rows)[kRows], int K, int lane,
                                          uint8_t* slot, const uint16_t* const (&xrow)[TB], int nt,
                                          float (&acc)[kRows][TB]) {
    constexpr bool kDeq = TB > 1;
    const uint8_t* codes = (const uint8_t*)w.codes + (int64_t)e * w.rows * w.cols;
    const uint16_t* am = (const uint16_t*)w.tables + (int64_t)e * w.absmax_per_expert;
    const int64_t nb = w.absmax_per_expert;
    const int bs = w.block_size;
    // codebook -> the slot (4 entries per lane: bf16, or fp32 for the
    // dequantising branch), issued with the first chunk's loads
    const uint2 cbv = reinterpret_cast<const uint2*>(ref_codebook(w, e))[lane];
    const uint32_t cbase = lds_addr(slot);
    const int nch = (K + kWChunk - 1) / kWChunk;
    for (int cc = 0; cc < nch; ++cc) {
        Rows8R b;
        uint32_t xs[TB][16];
        load_x8<TB>(xrow, K, cc, lane, nt, xs);
        __builtin_amdgcn_sched_barrier(0);
        load_rows8r(codes, am, nb, bs, rows, K, cc, lane, b);
        __builtin_amdgcn_sched_barrier(0);
        if (cc == 0) {
            if constexpr (kDeq) {
                const u32x4_t f = {cbv.x << 16, cbv.x & 0xffff0000u, cbv.y << 16, cbv.y & 0xffff0000u};
                *reinterpret_cast<u32x4_t*>(slot + 16 * lane) = f;
            } else {
                *reinterpret_cast<uint2*>(slot + 8 * lane) = cbv;
            }
            wave_lds_sync();
        }
        const bool ok = cc * kWChunk + 32 * lane < K;
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const float a = ok ? bf16_to_f32(b.am[r]) : 0.f;   // lanes past K contribute nothing
            if constexpr (kDeq) {
                ref_dot32_deq<TB>(b.cw[r], cbase, a, xs, nt, acc[r]);
            } else {
                float g[TB];
#pragma unroll
                for (int t = 0; t < TB; ++t) g[t] = 0.f;
                ref_dot32<TB>(b.cw[r], cbase, xs, nt, g);
#pragma unroll
                for (int t = 0; t < TB; ++t) acc[r][t] = fmaf(a, g[t], acc[r][t]);
            }
        }
    }
    wave_lds_sync();
}

// Rows of expert e of a stack in any decode format.
template <int kFmt, int TB>
__device__ __forceinline__ void expert_rows8(const lutmoe_weights& w, int e, const int (&rows)[kRows], int K,
                                             int lane, uint8_t* slot, const uint16_t* const (&xrow)[TB], int nt,
                                             float (&acc)[kRows][TB]) {
    if constexpr (kFmt == LUTMOE_FMT_NESTED) {
        nested_rows8_any<TB>(nested_view(w, e), rows, K, lane, slot, xrow, nt, acc);
    } else if constexpr (kFmt == LUTMOE_FMT_REF) {
        ref_rows8<TB>(w, e, rows, K, lane, slot, xrow, nt, acc);
    } else {
        const int64_t per = (int64_t)w.rows * (K / 2);
        bl4_rows8<TB>((const uint8_t*)w.codes + e * per, (const uint8_t*)w.tables + e * per, rows, K, lane, slot,
                      xrow, nt, acc);
    }
}

// Pass width: f(PassW<N>{}, n) runs one pass of n tokens with register
// arrays for N.  The dot products of a token past n would otherwise still be
// computed (the compiler turns the per-token guard into selects), and in
// skewed routing most chunks hold one or two tokens.  Modes:
//   kPassAll  N = TB always: REF, whose rows compute the reference's
//             one-token product order at N = 1 and its dequantised-weight
//             order above, chosen by the layer's token count;
//   kPass14   N = 1 for one token, else TB with n as it was (NestedLUT: a
//             third width made its kernels too large for the instruction
//             cache, and a wave-uniform n turned the per-token guards of the
//             LDS path into branches, both slower);
//   kPass124  N = 1 or 2 for exactly that many tokens, else TB, with n made
//             wave-uniform (BL4, same box: T = 8/16/32 62.4/94.7/150.6 ->
//             61.2/93.7/147.7 us).
// The choice is one scalar branch per pass.
template <int N>
struct PassW {
    static constexpr int value = N;
};
enum { kPassAll, kPass14, kPass124 };
template <int TB, int kMode, class F>
__device__ __forceinline__ void by_pass_width(int nt, F&& f) {
    if constexpr (kMode == kPassAll || TB == 1) {
        f(PassW<TB>{}, nt);
    } else if constexpr (kMode == kPass14) {
        if (__builtin_amdgcn_readfirstlane(nt) == 1) f(PassW<1>{}, 1);
        else f(PassW<TB>{}, nt);
    } else {
        nt = __builtin_amdgcn_readfirstlane(nt);
        if (nt == 1) f(PassW<1>{}, 1);
        else if (TB >= 4 && nt == 2) f(PassW<(TB >= 4 ? 2 : TB)>{}, 2);
        else f(PassW<TB>{}, nt);
    }
}
template <int kFmt>
constexpr int pass_mode() {
    return kFmt == LUTMOE_FMT_BL4 ? kPass124 : kFmt == LUTMOE_FMT_NESTED ? kPass14 : kPassAll;
}

// Gate/up for one routing view: CTA (x, y) covers 4*kGuWaves intermediate
// indices of active slot y, wave wv 4 of them (4 gate rows + 4 up rows);
// SwiGLU of the two projections -> act (bf16).  One-wave CTAs (16 KB of
// weights each) spread a layer's work evenly over the CUs: a CU streams at
// most ~40 GB/s, so a CU holding a CTA more than the others sets the tail.
template <int TB, int kFmt, class RV>
__device__ __forceinline__ void gate_up_body(const DecodeArgs& A, const RV& rv, uint8_t* s_slot) {
    const SlotRef sl = rv.work(blockIdx.y);
    if (sl.e < 0) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int I = A.d.inter, H = A.d.hidden, ke = A.k + A.d.num_shared;
    const int i0 = (blockIdx.x * kGuWaves + wv) * 4;
    if (i0 >= I) return;
    int rows[kRows];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = min(i0 + j, I - 1);
        rows[j] = i;
        rows[4 + j] = I + i;
    }
    uint8_t* slot = s_slot + wv * kSlot;
    for (int tb = 0; tb < sl.n; tb += TB) {
        by_pass_width<TB, pass_mode<kFmt>()>(min(TB, sl.n - tb), [&](auto W, int nt) __attribute__((always_inline)) {
            constexpr int N = decltype(W)::value;
            const uint16_t* xrow[N];
#pragma unroll
            for (int t = 0; t < N; ++t) {
                const int tok = rv.pair_at(sl.p0 + tb + min(t, nt - 1)) / ke;
                xrow[t] = A.x + (int64_t)min(max(tok, 0), A.T - 1) * H;   // in bounds whatever the routing holds
            }
            float acc[kRows][N];
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int t = 0; t < N; ++t) acc[r][t] = 0.f;
            expert_rows8<kFmt, N>(A.d.w13, sl.e, rows, H, lane, slot, xrow, nt, acc);
            const int j = lane >> 3;
#pragma unroll
            for (int t = 0; t < N; ++t) {
                float v[kRows];
#pragma unroll
                for (int r = 0; r < kRows; ++r) v[r] = acc[r][t];
                const float g = wave_reduce8(v);       // lane l: row l >> 3 (gate j for l < 32)
                const float u = from_upper_half(g);    // up row j
                if (lane < 32 && (lane & 7) == 0 && t < nt && i0 + j < I)
                    A.act[(int64_t)(sl.p0 + tb + t) * I + i0 + j] = (uint16_t)f32_to_bf16(silu_mul(g, u));
            }
        });
    }
}

// BL4 gate/up with 2 intermediate indices per wave (2 gate + 2 up rows): twice
// the waves of gate_up_body, each with half the serial work.  At one token
// per pass the kernel is bound by each wave's instruction and latency chain
// at about 1.4 waves per SIMD, and twice the waves shorten it (T=1 gate/up
// 10.5 -> 9.6 us).  gu2_for: the down kernel's 4-row body (down_body4), one
// token a pass; gu2_gate_up_for: the gate/up body.
static_assert(kGuWaves == 1, "gate_up_body4 assumes one wave per CTA");
template <int TB>
constexpr bool gu2_for() { return TB == 1; }
// gate/up with 2 indices a wave (gate_up_body4): one token a pass, and two or
// four when a routing kernel ran (T >= 3: 4 rows a wave in the interleaved
// map keep 44 of 48 lane steps busy at H = 2048 and look up without bank
// conflicts, each row waiting for its own loads; T = 8: 68 -> 65 us a layer,
// T = 17: 119 -> 115 us).  Where every wave routes in registers (T = 2),
// twice the waves means twice the routing (29.4 -> 30.3 us), and the 8-row
// body stays.
template <int TB, bool kPre>
constexpr bool gu2_gate_up_for() { return TB == 1 || (kPre && (TB == 2 || TB == 4)); }

// Four BL4 rows over all of K (as bl4_rows8 for 8, in its interleaved lane
// map: conflict-free lookups, which for one token a pass measured faster,
// as in bl4_decode_gate_up_t1): per 2048-column chunk the activations, then
// the loads of every row (all issued, none under a lane condition: code
// loads past K clamped to the chunk's last dword, activations zeroed once
// the weight loads are issued, so each row waits for its own loads only),
// then row by row the table staging and the lookups; the wave's LDS slot
// holds 4 rows' tables (4 KB).
template <int TB>
__device__ __forceinline__ void bl4_rows4(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ tabs,
                                          const int (&rows)[4], int K, int lane, uint8_t* slot,
                                          const uint16_t* const (&xrow)[TB], int nt, float (&acc)[4][TB]) {
    const uint32_t tab = lds_addr(slot) + ((lane >> 3) << 5);
    const u32x4_t z = {0u, 0u, 0u, 0u};
    const int nch = (K + kWChunk - 1) / kWChunk;
    for (int cc = 0; cc < nch; ++cc) {
        uint32_t xs[TB][16];
        load_xi_all<TB>(xrow, K, cc, lane, xs);
        __builtin_amdgcn_sched_barrier(0);
        const int nd = chunk_dwords(K, cc);
        const bool ok = cc * kWChunk + 32 * lane < K;
        uint32_t cw[4][4];
        u32x4_t tw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t ro = (uint32_t)rows[r] * (uint32_t)(K / 2) + cc * (kWChunk / 2);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                cw[r][q] = *reinterpret_cast<const uint32_t*>(codes + (ro + 4u * (uint32_t)min(lane + 64 * q, nd - 1)));
            tw[r] = *reinterpret_cast<const u32x4_t*>(tabs + (ro + (ok ? 16 * lane : 0)));
        }
        __builtin_amdgcn_sched_barrier(0);
        mask_xi<TB>(K, cc, lane, xs);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            *reinterpret_cast<u32x4_t*>(slot + r * 1024 + 16 * lane) = ok ? tw[r] : z;
            wave_lds_sync();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (64 * q >= nd) break;   // no code dword (K = 1408: q = 3)
                uint32_t xj[TB][4];
#pragma unroll
                for (int t = 0; t < TB; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i) xj[t][i] = xs[t][4 * q + i];
                bl4_dot8<TB>(cw[r][q], tab + r * 1024 + 256 * q, xj, nt, acc[r]);
            }
        }
        wave_lds_sync();
    }
}

template <int TB, class RV>
__device__ __forceinline__ void gate_up_body4(const DecodeArgs& A, const RV& rv, uint8_t* slot,
                                              int xcol = -1) {
    const SlotRef sl = rv.work(blockIdx.y);
    if (sl.e < 0) return;
    const int lane = threadIdx.x & 63;
    const int I = A.d.inter, H = A.d.hidden, ke = A.k + A.d.num_shared;
    const int i0 = (xcol < 0 ? (int)blockIdx.x : xcol) * 2;
    if (i0 >= I) return;
    const int i1 = min(i0 + 1, I - 1);
    const int rows[4] = {i0, i1, I + i0, I + i1};
    const int64_t per = (int64_t)A.d.w13.rows * (H / 2);
    const uint8_t* codes = (const uint8_t*)A.d.w13.codes + sl.e * per;
    const uint8_t* tabs = (const uint8_t*)A.d.w13.tables + sl.e * per;
    for (int tb = 0; tb < sl.n; tb += TB) {
        by_pass_width<TB, kPass124>(min(TB, sl.n - tb), [&](auto W, int nt) __attribute__((always_inline)) {
            constexpr int N = decltype(W)::value;
            // the positions' pairs first, all in flight together
            int pr[N];
#pragma unroll
            for (int t = 0; t < N; ++t) pr[t] = rv.pair_at(sl.p0 + tb + min(t, nt - 1));
            __builtin_amdgcn_sched_barrier(0);
            const uint16_t* xrow[N];
#pragma unroll
            for (int t = 0; t < N; ++t) xrow[t] = A.x + (int64_t)min(max(pr[t] / ke, 0), A.T - 1) * H;
            float acc[4][N];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int t = 0; t < N; ++t) acc[r][t] = 0.f;
            bl4_rows4<N>(codes, tabs, rows, H, lane, slot, xrow, nt, acc);
#pragma unroll
            for (int t = 0; t < N; ++t) {
                const float g0 = wave_reduce(acc[0][t]), g1 = wave_reduce(acc[1][t]);
                const float u0 = wave_reduce(acc[2][t]), u1 = wave_reduce(acc[3][t]);
                if (lane == 0 && t < nt) {
                    uint16_t* a = A.act + (int64_t)(sl.p0 + tb + t) * I;
                    a[i0] = (uint16_t)f32_to_bf16(silu_mul(g0, u0));
                    if (i0 + 1 < I) a[i0 + 1] = (uint16_t)f32_to_bf16(silu_mul(g1, u1));
                }
            }
        });
    }
}

// One token (T = 1): the expert of active slot y, for the gate/up CTAs that
// do not publish the routing.  The slots are the token's distinct routed
// experts in ascending id order, then the shared experts; the top-k set is a
// 64-bit mask chosen as wave_pairs chooses it (k rounds of a DPP wave max,
// ties to the lower id, NaN never selected), so the slot order matches the
// routing copy the publishing CTA writes.  A few dozen instructions where the
// general routing takes a few hundred, run by every one of the layer's
// thousands of one-wave CTAs.  Returns -1 past the last slot and -2 where
// this path does not apply (more than 64 routed experts, or ids that repeat:
// the caller then takes the general routing).
// The lane's routing input for t1_slot_expert: top-k id `lane` (lane < k)
// or router logit `lane` (lane < E) as raw bits.  One load for every lane
// (clamped index), issued before the activation loads so that the routing
// does not wait for them.
__device__ __forceinline__ uint32_t t1_route_input(const DecodeArgs& A) {
    const int lane = threadIdx.x & 63;
    const uint32_t* src = A.topk_ids ? reinterpret_cast<const uint32_t*>(A.topk_ids)
                                     : reinterpret_cast<const uint32_t*>(A.logits);
    const int n = A.topk_ids ? A.k : A.d.num_routed;
    return src[min(lane, n - 1)];
}

__device__ __forceinline__ int t1_slot_expert(const DecodeArgs& A, int y, uint32_t rin) {
    const int lane = threadIdx.x & 63;
    const int E = A.d.num_routed, S = A.d.num_shared, k = A.k;
    if (E > 64) return -2;
    uint64_t sel = 0;
    if (A.topk_ids) {
        const int id = lane < k ? (int)rin : -1;
        const bool ok = lane < k && id >= 0 && id < E;
        for (int j = 0; j < k; ++j) {
            const int e = __builtin_amdgcn_readlane(id, j);
            if (e >= 0 && e < E) sel |= 1ull << e;
        }
        if (__popcll(sel) != __popcll(__ballot(ok))) return -2;   // a repeated id
    } else {
        const float v = lane < E ? __builtin_bit_cast(float, rin) : -INFINITY;
        int key = lane < E ? float_key(v) : INT_MIN;
        for (int j = 0; j < k; ++j) {
            const int m = wave_max_i32(key);
            const uint64_t b = __ballot(lane < E && key == m && m != INT_MIN);
            if (b) {
                const int s = (int)__builtin_ctzll(b);
                sel |= 1ull << s;
                if (lane == s) key = INT_MIN;
            }
        }
    }
    const int nsel = __popcll(sel);
    if (y < nsel) {
        for (int i = 0; i < y; ++i) sel &= sel - 1;
        return (int)__builtin_ctzll(sel);
    }
    return y < nsel + S ? E + (y - nsel) : -1;
}

// One token, BL4, K = H <= 2048 (one chunk): gate/up rows i0, i0 + 1 of
// expert e (slot y, position y) with the token's activations xs loaded
// before the routing; SwiGLU -> act[y][i0 .. i0 + 1].
__device__ __forceinline__ void gate_up_t1(const DecodeArgs& A, const uint32_t (&xs)[16], const uint8_t* wcodes,
                                           const uint8_t* wtabs, int64_t per, int e, int y, int xcol, uint8_t* slot) {
    const int lane = threadIdx.x & 63;
    const int I = A.d.inter, H = A.d.hidden;
    const int i0 = xcol * 2;
    const int i1 = min(i0 + 1, I - 1);
    const int rows[4] = {i0, i1, I + i0, I + i1};
    const uint8_t* codes = wcodes + e * per;
    const uint8_t* tabs = wtabs + e * per;
    // code dwords l + 64q of each row and the lane's 16 table bytes, as
    // load_rows8 takes them (conflict-free lookups)
    const bool ok = 32 * lane < H;
    uint32_t cw[4][4];
    u32x4_t tw[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t ro = (uint32_t)rows[r] * (uint32_t)(H / 2);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            cw[r][q] = *reinterpret_cast<const uint32_t*>(codes + (ro + 4u * (uint32_t)min(lane + 64 * q, H / 8 - 1)));
        tw[r] = *reinterpret_cast<const u32x4_t*>(tabs + (ro + (ok ? 16 * lane : 0)));
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t tab = lds_addr(slot) + ((lane >> 3) << 5);
    const u32x4_t z = {0u, 0u, 0u, 0u};
    float acc[4][1] = {{0.f}, {0.f}, {0.f}, {0.f}};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        *reinterpret_cast<u32x4_t*>(slot + r * 1024 + 16 * lane) = ok ? tw[r] : z;
        wave_lds_sync();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t xj[1][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) xj[0][i] = xs[4 * q + i];
            bl4_dot8<1>(cw[r][q], tab + r * 1024 + 256 * q, xj, 1, acc[r]);
        }
    }
    // reduce-scatter of the 4 row sums: lane 16j holds row j's total
    const float v = wave_reduce4(acc[0][0], acc[1][0], acc[2][0], acc[3][0]);
    const float up = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float up1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    const float g1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    if (lane == 0) {
        uint16_t* a = A.act + (int64_t)y * I;
        a[i0] = (uint16_t)f32_to_bf16(silu_mul(v, up));
        if (i0 + 1 < I) a[i0 + 1] = (uint16_t)f32_to_bf16(silu_mul(g1, up1));
    }
}

// One token, BL4, H <= 2048: CTAs of 4 independent waves (one dispatch for
// four, no barrier); wave w of CTA (x, y) takes intermediate indices
// 2(4x + w), +1 of slot y with its own short slot routing.  The first wave of
// CTA (0, 0) also computes the full routing with the pair weights and,
// after its own rows, publishes it for the down kernel.
__global__ __launch_bounds__(256, 3) void bl4_decode_gate_up_t1(DecodeArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[4][4 * 1024];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int xcol = blockIdx.x * 4 + wv;
    const uint8_t* wcodes = (const uint8_t*)A.d.w13.codes;
    const uint8_t* wtabs = (const uint8_t*)A.d.w13.tables;
    const int64_t per = (int64_t)A.d.w13.rows * (A.d.hidden / 2);
    asm volatile("" ::"s"(wcodes), "s"(wtabs), "s"(per));
    const uint32_t rin = t1_route_input(A);
    __builtin_amdgcn_sched_barrier(0);
    // the activations of the lane's code dwords l + 64q (8 columns each):
    // every load issued (past H: the last 8 columns, then zeroed), so none
    // waits for another (a load under a lane condition made the compiler
    // wait for it before issuing the next)
    uint32_t xs[16];
    const int nd = A.d.hidden / 8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int d = lane + 64 * q;
        const uint4 v = *reinterpret_cast<const uint4*>(A.x + 8 * min(d, nd - 1));
        const uint32_t m = d < nd ? 0xffffffffu : 0u;
        xs[4 * q + 0] = v.x & m;
        xs[4 * q + 1] = v.y & m;
        xs[4 * q + 2] = v.z & m;
        xs[4 * q + 3] = v.w & m;
    }
    if (2 * xcol < A.d.inter) {
        const int e = t1_slot_expert(A, blockIdx.y, rin);
        if (e >= 0) {
            gate_up_t1(A, xs, wcodes, wtabs, per, e, blockIdx.y, xcol, s_slot[wv]);
        } else if (e == -2) {
            // ids that repeat: the general routing
            gate_up_body4<1>(A, WaveRouteView{wave_pairs<false>(A)}, s_slot[wv], xcol);
        }
    }
    // after the wave's own rows (the down kernel reads the copy only after
    // this kernel ends): publishing first put its loads ahead of every
    // wave's routing wait
    if (blockIdx.x == 0 && blockIdx.y == 0 && wv == 0) wave_route_publish(A, wave_pairs<true>(A));
}

// One token, REF, K = H <= 2048 (one chunk): gate rows i0, i0 + 1 and up
// rows I + i0, I + i0 + 1 of expert e.  The lane's 32 codes of a row (32
// bytes) against the expert's bf16[256] codebook in the wave's LDS slot, times
// the absmax of their block: the reference's one-token products,
// fp32 (x * cb) * absmax factored per 32 columns, as ref_rows8 computes them.
// SwiGLU -> act[p][i0 .. i0 + 1] for the slot's positions p0 .. p0 + n - 1
// (more than one only when the token lists the expert twice: one token, the
// same values).
__device__ __forceinline__ void ref_gate_up_t1(const DecodeArgs& A, const uint32_t (&xs)[16], int e, int p0, int n,
                                               int xcol, uint8_t* slot) {
    const int lane = threadIdx.x & 63;
    const int I = A.d.inter, H = A.d.hidden;
    const lutmoe_weights& w = A.d.w13;
    const int i0 = xcol * 2;
    const int i1 = min(i0 + 1, I - 1);
    const int rows[4] = {i0, i1, I + i0, I + i1};
    const uint8_t* codes = (const uint8_t*)w.codes + (int64_t)e * w.rows * w.cols;
    const uint16_t* am = (const uint16_t*)w.tables + (int64_t)e * w.absmax_per_expert;
    const int64_t nb = w.absmax_per_expert;
    const bool ok = 32 * lane < H;
    const uint2 cbv = reinterpret_cast<const uint2*>(ref_codebook(w, e))[lane];
    const uint32_t q32 = (uint32_t)w.block_size / 32u;
    u32x4_t cw[4][2];
    uint32_t av[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t off = (int64_t)rows[r] * H + (ok ? 32 * lane : 0);
        cw[r][0] = *reinterpret_cast<const u32x4_t*>(codes + off);
        cw[r][1] = *reinterpret_cast<const u32x4_t*>(codes + off + 16);
        const uint32_t u = (uint32_t)rows[r] * (uint32_t)(H / 32) + (ok ? (uint32_t)lane : 0u);
        av[r] = am[ref_block32(u, q32, (uint32_t)nb)];
    }
    __builtin_amdgcn_sched_barrier(0);
    *reinterpret_cast<uint2*>(slot + 8 * lane) = cbv;
    wave_lds_sync();
    const uint32_t cbase = lds_addr(slot);
    const uint32_t (&x1)[1][16] = reinterpret_cast<const uint32_t (&)[1][16]>(xs);
    float acc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float g[1] = {0.f};
        ref_dot32<1>(cw[r], cbase, x1, 1, g);
        acc[r] = ok ? bf16_to_f32(av[r]) * g[0] : 0.f;   // lanes past K contribute nothing
    }
    const float v = wave_reduce4(acc[0], acc[1], acc[2], acc[3]);   // lane 16j: row j
    const float up = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float up1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    const float g1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    if (lane == 0) {
        const uint16_t a0 = (uint16_t)f32_to_bf16(silu_mul(v, up));
        const uint16_t a1 = (uint16_t)f32_to_bf16(silu_mul(g1, up1));
        for (int q = 0; q < n; ++q) {
            uint16_t* a = A.act + (int64_t)(p0 + q) * I;
            a[i0] = a0;
            if (i0 + 1 < I) a[i0 + 1] = a1;
        }
    }
}

// One token, REF, H <= 2048: the CTA shape of bl4_decode_gate_up_t1 (four
// independent waves, intermediate indices 2(4x + w), +1 of slot y, the slot's
// expert from the token's top-k mask; the general routing where ids repeat),
// each wave with the expert's codebook in its own 512 bytes of LDS.  The
// first wave of CTA (0, 0) publishes the routing for the down kernel.
__global__ __launch_bounds__(256, 3) void ref_decode_gate_up_t1(DecodeArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t s_cb[4][512];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int xcol = blockIdx.x * 4 + wv;
    const uint32_t rin = t1_route_input(A);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t xs[16];
    const uint16_t* xp = A.x + (32 * lane < A.d.hidden ? 32 * lane : 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 v = *reinterpret_cast<const uint4*>(xp + 8 * q);
        xs[4 * q + 0] = v.x;
        xs[4 * q + 1] = v.y;
        xs[4 * q + 2] = v.z;
        xs[4 * q + 3] = v.w;
    }
    if (2 * xcol < A.d.inter) {
        int e = t1_slot_expert(A, blockIdx.y, rin), p0 = blockIdx.y, n = 1;
        if (e == -2) {
            // ids that repeat: the general routing (a slot may hold two positions)
            const SlotRef sl = WaveRouteView{wave_pairs<false>(A)}.work(blockIdx.y);
            e = sl.e;
            p0 = sl.p0;
            n = sl.n;
        }
        if (e >= 0) ref_gate_up_t1(A, xs, e, p0, n, xcol, s_cb[wv]);
    }
    // after the wave's own rows, as in bl4_decode_gate_up_t1
    if (blockIdx.x == 0 && blockIdx.y == 0 && wv == 0) wave_route_publish(A, wave_pairs<true>(A));
}

template <int TB, bool kPre, int kFmt>
__global__ __launch_bounds__(64 * kGuWaves, TB <= 2 ? 3 : 2) void bl4_decode_gate_up(DecodeArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[kGuWaves * kSlot];
    if constexpr (gu2_gate_up_for<TB, kPre>() && kFmt == LUTMOE_FMT_BL4) {
        if constexpr (kPre) {
            gate_up_body4<TB>(A, GlobalRouteView{A.route}, s_slot);
        } else {
            // (one token with H <= 2048 runs bl4_decode_gate_up_t1 instead)
            const bool pub = blockIdx.x == 0 && blockIdx.y == 0;
            const WaveRoute r = pub ? wave_pairs<true>(A) : wave_pairs<false>(A);
            if (pub && threadIdx.x < 64) wave_route_publish(A, r);
            gate_up_body4<TB>(A, WaveRouteView{r}, s_slot);
        }
    } else if constexpr (kPre) {
        gate_up_body<TB, kFmt>(A, GlobalRouteView{A.route}, s_slot);
    } else {
        // the first CTA also publishes the routing (with the pair weights)
        // for the down kernel; one copy of the body for all CTAs keeps the
        // kernel's code small
        const bool pub = blockIdx.x == 0 && blockIdx.y == 0;
        const WaveRoute r = pub ? wave_pairs<true>(A) : wave_pairs<false>(A);
        if (pub && threadIdx.x < 64) wave_route_publish(A, r);
        gate_up_body<TB, kFmt>(A, WaveRouteView{r}, s_slot);
    }
}

// Down for one routing view: CTA x covers 8 output rows; wave wv runs the
// active slots wv, wv+4, ..; per-position results (times the pair weight)
// meet in LDS and are summed per token in slot order.
template <int TB, int kFmt, class RV>
__device__ __forceinline__ void down_body(const DecodeArgs& A, const RV& rv, uint8_t* s_slot, float* s_y) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int I = A.d.inter, H = A.d.hidden, ke = A.k + A.d.num_shared;
    const int h0 = blockIdx.x * kRows;
    int rows[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) rows[r] = min(h0 + r, H - 1);
    uint8_t* slot = s_slot + wv * kSlot;
    const int nact = rv.nact();
    for (int a = wv; a < nact; a += (int)(blockDim.x >> 6)) {
        const SlotRef sl = rv.slot(a);
        for (int tb = 0; tb < sl.n; tb += TB) {
            const int nt = min(TB, sl.n - tb);
            const uint16_t* xrow[TB];
#pragma unroll
            for (int t = 0; t < TB; ++t) xrow[t] = A.act + (int64_t)(sl.p0 + tb + min(t, nt - 1)) * I;
            float acc[kRows][TB];
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int t = 0; t < TB; ++t) acc[r][t] = 0.f;
            expert_rows8<kFmt, TB>(A.d.w2, sl.e, rows, I, lane, slot, xrow, nt, acc);
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                const int p = sl.p0 + tb + min(t, nt - 1);
                const float pw = rv.weight_at(p);
                float v[kRows];
#pragma unroll
                for (int r = 0; r < kRows; ++r) v[r] = acc[r][t];
                const float y = wave_reduce8(v);   // lane l: row l >> 3
                if ((lane & 7) == 0 && t < nt) s_y[p * kRows + (lane >> 3)] = y * pw;
            }
        }
    }
    __syncthreads();
    const int T = A.T;
    // every thread runs the same trip counts (pos_of may be a wave operation)
    for (int base = 0; base < T * kRows; base += blockDim.x) {
        const int idx = base + threadIdx.x;
        const int t = min(idx / kRows, T - 1), r = idx % kRows;
        float sum = 0.f;
        for (int q = 0; q < ke; ++q) {
            const int pos = rv.pos_of(t * ke + q);
            if (pos >= 0) sum += s_y[pos * kRows + r];
        }
        if (idx < T * kRows && h0 + r < H) {
            const int64_t o = (int64_t)t * H + h0 + r;
            store_out(A, o, sum);
        }
    }
}

// BL4 down at one token per pass with 4 output rows per CTA (twice the CTAs
// of down_body, half the serial work per wave; the reason as for
// gate_up_body4).  Wave wv runs the active slots wv, wv+4, ..
template <class RV>
__device__ __forceinline__ void down_body4(const DecodeArgs& A, const RV& rv, uint8_t* s_slot, float* s_y) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int I = A.d.inter, H = A.d.hidden, ke = A.k + A.d.num_shared;
    const int h0 = blockIdx.x * 4;
    int rows[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rows[r] = min(h0 + r, H - 1);
    uint8_t* slot = s_slot + wv * kSlot;
    const int64_t per = (int64_t)A.d.w2.rows * (I / 2);
    const int nact = rv.nact();
    for (int a = wv; a < nact; a += (int)(blockDim.x >> 6)) {
        const SlotRef sl = rv.slot(a);
        for (int p = sl.p0; p < sl.p0 + sl.n; ++p) {
            const uint16_t* xrow[1] = {A.act + (int64_t)p * I};
            float acc[4][1] = {{0.f}, {0.f}, {0.f}, {0.f}};
            bl4_rows4<1>((const uint8_t*)A.d.w2.codes + sl.e * per, (const uint8_t*)A.d.w2.tables + sl.e * per,
                         rows, I, lane, slot, xrow, 1, acc);
            const float pw = rv.weight_at(p);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float y = wave_reduce(acc[r][0]);
                if (lane == r) s_y[p * 4 + r] = y * pw;
            }
        }
    }
    __syncthreads();
    const int T = A.T;
    for (int base = 0; base < T * 4; base += blockDim.x) {
        const int idx = base + threadIdx.x;
        const int t = min(idx / 4, T - 1), r = idx % 4;
        float sum = 0.f;
        for (int q = 0; q < ke; ++q) {
            const int pos = rv.pos_of(t * ke + q);
            if (pos >= 0) sum += s_y[pos * 4 + r];
        }
        if (idx < T * 4 && h0 + r < H) {
            const int64_t o = (int64_t)t * H + h0 + r;
            store_out(A, o, sum);
        }
    }
}

template <int TB, bool kPre, int kFmt>
__global__ __launch_bounds__(256, TB <= 2 ? 3 : 2) void bl4_decode_down(DecodeArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[4 * kSlot];
    extern __shared__ float s_y[];   // [P][8] ([P][4] for down_body4)
    if constexpr (kPre) {
        __shared__ RouteOut R;
        load_route(A, R);
        if constexpr (gu2_for<TB>() && kFmt == LUTMOE_FMT_BL4) down_body4(A, LdsRouteView{&R}, s_slot, s_y);
        else down_body<TB, kFmt>(A, LdsRouteView{&R}, s_slot, s_y);
    } else {
        down_body<TB, kFmt>(A, WaveRouteView{wave_pairs<true>(A)}, s_slot, s_y);
    }
}

// One or two tokens (TB), BL4: CTA x covers output rows [4x, 4x + 4); wave
// wv takes the active slots wv, wv + 4, .. (a slot holds one position per
// token that routes to its expert, more when a token lists it twice).  A
// slot's 4 rows run through bl4_rows4 (interleaved code dwords: every LDS
// lookup conflict-free, and at K = 1408, 176 dwords a row, 44 of 48 lane
// steps busy), then one 4-value reduce-scatter gives each row's sum.  The
// routing is read from the workspace copy in place: no LDS copy and no
// barrier before the weight loads.
constexpr int kD1Rows = 4;

template <int TB>
__global__ __launch_bounds__(256, 2) void bl4_decode_down1(DecodeArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[4][kD1Rows * 1024];
    __shared__ float s_y[16 * TB][kD1Rows];   // [position][row]: at most T (k + S) <= 16 T positions
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int K = A.d.inter, H = A.d.hidden, ke = A.k + A.d.num_shared;
    const int h0 = blockIdx.x * kD1Rows;   // H % 64 == 0: all 4 rows exist
    const int rows[kD1Rows] = {h0, h0 + 1, h0 + 2, h0 + 3};
    const RouteOut* R = A.route;
    const float* pos_w = route_pos_w(R);
    // the routing fields this wave needs, in one round trip: the count, the
    // first slot's expert and position (in bounds for any count), and the
    // positions of the tokens' pairs for the combine
    const int nact = R->nact;
    int e_next = R->act[wv], p_next = R->aoff[wv], n_next = R->an[wv];
    const int inv_l = (wv == 0 && lane < ke * TB) ? R->inv[lane] : -1;
    const int64_t per = (int64_t)A.d.w2.rows * (K / 2);
    const uint8_t* wcodes = (const uint8_t*)A.d.w2.codes;
    const uint8_t* wtabs = (const uint8_t*)A.d.w2.tables;
    // the weight bases come from the kernel arguments while the routing loads
    // are in flight (not after them)
    asm volatile("" ::"s"(wcodes), "s"(wtabs), "s"(per));
    for (int a = wv; a < nact; a += 4) {
        const int e = e_next, p0 = p_next, n = n_next;
        // one token: a single pass (a slot's positions are the same token);
        // two tokens: passes of up to 2 positions
        for (int tb = 0; tb < (TB == 1 ? 1 : n); tb += TB) {
            const int nt = TB == 1 ? 1 : min(TB, n - tb);
            // the routing weights from the positions' weight array, loaded
            // with the activations
            const uint16_t* xrow[TB];
            float pw[TB];
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                xrow[t] = A.act + (int64_t)(p0 + tb + min(t, nt - 1)) * K;
                pw[t] = pos_w[p0 + tb + min(t, nt - 1)];
            }
            float acc[kD1Rows][TB];
#pragma unroll
            for (int r = 0; r < kD1Rows; ++r)
#pragma unroll
                for (int t = 0; t < TB; ++t) acc[r][t] = 0.f;
            bl4_rows4<TB>(wcodes + e * per, wtabs + e * per, rows, K, lane, s_slot[wv], xrow, nt, acc);
            if (tb == 0 && a + 4 < kMaxEtot) {
                e_next = R->act[a + 4];
                p_next = R->aoff[a + 4];
                n_next = R->an[a + 4];
            }
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                if (t >= nt) break;
                const float v = wave_reduce4(acc[0][t], acc[1][t], acc[2][t], acc[3][t]);   // lane 16r: row r
                if ((lane & 15) == 0) {
                    const int r = lane >> 4;
                    s_y[p0 + tb + t][r] = v * pw[t];
                    // one token listing an expert more than once: its other
                    // positions hold the same activations, each with its own weight
                    if constexpr (TB == 1)
                        for (int q = 1; q < n; ++q) s_y[p0 + q][r] = v * pos_w[p0 + q];
                }
            }
        }
    }
    __syncthreads();
    // each token's slots in slot order (pair q of token t sits at position
    // inv[t (k + S) + q])
    if (wv == 0) {
        float sum = 0.f;
        if constexpr (TB == 1) {
            for (int q = 0; q < ke; ++q) {
                const int pos = __builtin_amdgcn_readlane(inv_l, q);
                if (pos >= 0 && lane < kD1Rows) sum += s_y[pos][lane];
            }
        } else {
            // lane 4t + r: token t, row r
            const int t = lane / kD1Rows, r = lane % kD1Rows;
            for (int q = 0; q < ke; ++q) {
                const int pos = __shfl(inv_l, min(t, TB - 1) * ke + q, 64);
                if (pos >= 0 && t < A.T) sum += s_y[pos][r];
            }
        }
        if (lane < kD1Rows * (TB == 1 ? 1 : A.T)) {
            const int64_t o = TB == 1 ? h0 + lane : (int64_t)(lane / kD1Rows) * H + h0 + lane % kD1Rows;
            store_out(A, o, sum);
        }
    }
}

// One token (T = 1), REF: the scheme of bl4_decode_down1 (CTA x: output rows
// [4x, 4x + 4); wave wv: active slots wv, wv + 4, ..; the routing read from
// the workspace copy in place) over REF rows.  An expert's 4 rows are K
// contiguous code bytes each, walked as one flat array of 32-byte units
// (unit u: columns [32g, 32g + 32) of row u / NU, NU = K/32, g = u % NU;
// lane l takes units l, l + 64, ..); a unit lies inside one absmax block
// (block_size % 64 == 0), and its sum x . cb[codes] times that absmax is the
// reference's one-token product, fp32 (x * cb) * absmax, as ref_rows8 forms
// it per 32 columns.  The expert's bf16[256] codebook sits in the wave's LDS.
template <int kPass>
__global__ __launch_bounds__(256, 2) void ref_decode_down1(DecodeArgs A) {
    __shared__ __attribute__((aligned(16))) uint8_t s_cb[4][512];
    __shared__ float s_part[4][kPass * 64];
    __shared__ float s_y[16][kD1Rows];   // [position][row], T = 1: at most k + S <= 16 positions
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int K = A.d.inter, ke = A.k + A.d.num_shared;
    const int NU = K / 32, U = kD1Rows * NU;
    const int h0 = blockIdx.x * kD1Rows;   // H % 64 == 0: all 4 rows exist
    const lutmoe_weights& w = A.d.w2;
    const RouteOut* R = A.route;
    const int nact = R->nact;
    int e_next = R->act[wv], p_next = R->aoff[wv], n_next = R->an[wv];
    const int inv_l = (wv == 0 && lane < ke) ? R->inv[lane] : -1;
    const int64_t per = (int64_t)w.rows * w.cols;
    const int64_t nb = w.absmax_per_expert;
    const uint32_t cbase = lds_addr(s_cb[wv]);
    float* part = s_part[wv];
    for (int a = wv; a < nact; a += 4) {
        const int e = e_next, p0 = p_next, n = n_next;
        const int pair = R->perm[p0];   // its weight is loaded after the weight loads
        const uint8_t* codes = (const uint8_t*)w.codes + e * per + (int64_t)h0 * K;
        const uint16_t* am = (const uint16_t*)w.tables + e * nb;
        const uint16_t* xr = A.act + (int64_t)p0 * K;
        const uint2 cbv = reinterpret_cast<const uint2*>(ref_codebook(w, e))[lane];
        uint32_t xs[kPass][1][16];
#pragma unroll
        for (int p = 0; p < kPass; ++p) {
            const int u = 64 * p + lane;
            const int g = u < U ? u % NU : 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = *reinterpret_cast<const uint4*>(xr + 32 * g + 8 * q);
                xs[p][0][4 * q + 0] = v.x;
                xs[p][0][4 * q + 1] = v.y;
                xs[p][0][4 * q + 2] = v.z;
                xs[p][0][4 * q + 3] = v.w;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        u32x4_t cw[kPass][2];
        uint32_t av[kPass];
#pragma unroll
        for (int p = 0; p < kPass; ++p) {
            const int u = 64 * p + lane;
            const int64_t off = u < U ? 32 * u : 0;
            cw[p][0] = *reinterpret_cast<const u32x4_t*>(codes + off);
            cw[p][1] = *reinterpret_cast<const u32x4_t*>(codes + off + 16);
            const uint32_t u32 = (uint32_t)h0 * (uint32_t)(K / 32) + (u < U ? (uint32_t)u : 0u);
            av[p] = am[ref_block32(u32, (uint32_t)w.block_size / 32u, (uint32_t)nb)];
        }
        __builtin_amdgcn_sched_barrier(0);
        // behind the weight loads: the pair weight and the next slot's fields
        const float pw = R->pw[pair];
        if (a + 4 < kMaxEtot) {
            e_next = R->act[a + 4];
            p_next = R->aoff[a + 4];
            n_next = R->an[a + 4];
        }
        *reinterpret_cast<uint2*>(s_cb[wv] + 8 * lane) = cbv;
        wave_lds_sync();
#pragma unroll
        for (int p = 0; p < kPass; ++p) {
            float g[1] = {0.f};
            ref_dot32<1>(cw[p], cbase, xs[p], 1, g);
            // units past the 4 rows (their loads read the first unit) add nothing
            part[64 * p + lane] = 64 * p + lane < U ? bf16_to_f32(av[p]) * g[0] : 0.f;
        }
        wave_lds_sync();
        // per-row sums: lane 16r + j adds units r*NU + j, + 16, .. and the 16
        // lanes of row r reduce with DPP
        const int r = lane >> 4, j = lane & 15;
        float v = 0.f;
        for (int u = j; u < NU; u += 16) v += part[r * NU + u];
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false));
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false));
        if (j == 0) {
            s_y[p0][r] = v * pw;
            // an expert the token lists more than once: the same activations
            for (int q = 1; q < n; ++q) s_y[p0 + q][r] = v * route_pos_w(R)[p0 + q];
        }
        wave_lds_sync();   // the codebook and the partials are restaged by the next slot
    }
    __syncthreads();
    if (wv == 0) {
        float sum = 0.f;
        for (int q = 0; q < ke; ++q) {
            const int pos = __builtin_amdgcn_readlane(inv_l, q);
            if (pos >= 0 && lane < kD1Rows) sum += s_y[pos][lane];
        }
        if (lane < kD1Rows) {
            const int64_t o = h0 + lane;
            store_out(A, o, sum);
        }
    }
}

// Down projection when many experts are active (more than 8 slots would be
// walked one after another by the 4 waves of bl4_decode_down): CTA (x, g)
// covers output rows 8x..8x+7 of active slots 4g..4g+3, one slot per wave;
// each position's result times its pair weight goes to y[pos][h] (fp32) and
// combine_kernel sums each token's slots in slot order.
template <int TB, int kFmt>
__global__ __launch_bounds__(256, TB <= 2 ? 3 : 2) void bl4_decode_down_y(DecodeArgs A, float* __restrict__ y) {
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[4 * kSlot];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int a = blockIdx.y * 4 + wv;
    const GlobalRouteView rv{A.route};
    const SlotRef sl = rv.work(a);
    if (sl.e < 0) return;
    const int I = A.d.inter, H = A.d.hidden;
    const int h0 = blockIdx.x * kRows;
    int rows[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) rows[r] = min(h0 + r, H - 1);
    uint8_t* slot = s_slot + wv * kSlot;
    for (int tb = 0; tb < sl.n; tb += TB) {
        by_pass_width<TB, pass_mode<kFmt>()>(min(TB, sl.n - tb), [&](auto W, int nt) __attribute__((always_inline)) {
            constexpr int N = decltype(W)::value;
            const uint16_t* xrow[N];
#pragma unroll
            for (int t = 0; t < N; ++t) xrow[t] = A.act + (int64_t)(sl.p0 + tb + min(t, nt - 1)) * I;
            float acc[kRows][N];
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int t = 0; t < N; ++t) acc[r][t] = 0.f;
            // the positions' routing weights (one load each, from the positions'
            // weight array) issued ahead of the weight loads, which hide them
            float pwv[N];
#pragma unroll
            for (int t = 0; t < N; ++t) pwv[t] = rv.weight_at(sl.p0 + tb + min(t, nt - 1));
            expert_rows8<kFmt, N>(A.d.w2, sl.e, rows, I, lane, slot, xrow, nt, acc);
#pragma unroll
            for (int t = 0; t < N; ++t) {
                const int p = sl.p0 + tb + min(t, nt - 1);
                const float pw = pwv[t];
                float v[kRows];
#pragma unroll
                for (int r = 0; r < kRows; ++r) v[r] = acc[r][t];
                const float yv = wave_reduce8(v);   // lane l: row l >> 3
                const int r = lane >> 3;
                if ((lane & 7) == 0 && t < nt && h0 + r < H) y[(int64_t)p * H + h0 + r] = yv * pw;
            }
        });
    }
}

// BL4 down when many experts are active, 4 output rows a wave: CTA (x, g)
// covers output rows 4x..4x+3 of work items 4g..4g+3, one per wave, through
// the interleaved 4-row loop (bl4_rows4: conflict-free lookups, and at
// K = 1408 44 of 48 lane steps busy, where 8 rows of one 32-column unit a
// lane leave 20 of 64 lanes idle); y[pos][h] as bl4_decode_down_y.
template <int TB>
// (one or two tokens a pass: 4 CTAs a CU, 128 VGPRs: T = 8 64.3 -> 62.4 us,
// T = 16 92.4 -> 88.5 us a layer against 2 CTAs a CU)
__global__ __launch_bounds__(256, TB <= 2 ? 4 : 2) void bl4_decode_down_y4(DecodeArgs A, float* __restrict__ y) {
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[4][4 * 1024];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const GlobalRouteView rv{A.route};
    const SlotRef sl = rv.work(blockIdx.y * 4 + wv);
    if (sl.e < 0) return;
    const int I = A.d.inter, H = A.d.hidden;
    const int h0 = blockIdx.x * 4;
    int rows[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rows[r] = min(h0 + r, H - 1);
    const int64_t per = (int64_t)A.d.w2.rows * (I / 2);
    const uint8_t* codes = (const uint8_t*)A.d.w2.codes + sl.e * per;
    const uint8_t* tabs = (const uint8_t*)A.d.w2.tables + sl.e * per;
    for (int tb = 0; tb < sl.n; tb += TB) {
        by_pass_width<TB, kPass124>(min(TB, sl.n - tb), [&](auto W, int nt) __attribute__((always_inline)) {
            constexpr int N = decltype(W)::value;
            const uint16_t* xrow[N];
#pragma unroll
            for (int t = 0; t < N; ++t) xrow[t] = A.act + (int64_t)(sl.p0 + tb + min(t, nt - 1)) * I;
            float acc[4][N];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int t = 0; t < N; ++t) acc[r][t] = 0.f;
            float pwv[N];
#pragma unroll
            for (int t = 0; t < N; ++t) pwv[t] = rv.weight_at(sl.p0 + tb + min(t, nt - 1));
            bl4_rows4<N>(codes, tabs, rows, I, lane, s_slot[wv], xrow, nt, acc);
#pragma unroll
            for (int t = 0; t < N; ++t) {
                const float yv = wave_reduce4(acc[0][t], acc[1][t], acc[2][t], acc[3][t]);   // lane 16r: row r
                const int r = lane >> 4;
                if ((lane & 15) == 0 && t < nt && h0 + r < H)
                    y[(int64_t)(sl.p0 + tb + t) * H + h0 + r] = yv * pwv[t];
            }
        });
    }
}

// Single-matrix NestedLUT GEMV (lutmoe_gemv): y[t][m] = sum_k x[t][k] W_e[m][k]
// for T vectors, TB at a time; a wave owns 8 rows, a CTA 32.
template <int TB>
__global__ __launch_bounds__(256, 2) void nested_gemv_kernel(lutmoe_weights w, int e, const uint16_t* __restrict__ x,
                                                             int T, void* __restrict__ y, int y_dtype) {
    __shared__ __attribute__((aligned(16))) uint8_t s_slot[4 * kSlot];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int M = w.rows, K = w.cols;
    const int m0 = (blockIdx.x * 4 + wv) * kRows;
    if (m0 >= M) return;
    int rows[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) rows[r] = min(m0 + r, M - 1);
    const NestedView v = nested_view(w, e);
    uint8_t* slot = s_slot + wv * kSlot;
    for (int t0 = 0; t0 < T; t0 += TB) {
        const int nt = min(TB, T - t0);
        const uint16_t* xrow[TB];
#pragma unroll
        for (int t = 0; t < TB; ++t) xrow[t] = x + (int64_t)(t0 + min(t, nt - 1)) * K;
        float acc[kRows][TB];
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int t = 0; t < TB; ++t) acc[r][t] = 0.f;
        nested_rows8<TB>(v, rows, K, lane, slot, xrow, nt, acc);
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                const float s = wave_reduce(acc[r][t]);
                if (lane == r * TB + t && t < nt && m0 + r < M) {
                    const int64_t o = (int64_t)(t0 + t) * M + m0 + r;
                    if (y_dtype == LUTMOE_DTYPE_F32) ((float*)y)[o] = s;
                    else ((uint16_t*)y)[o] = (uint16_t)f32_to_bf16(s);
                }
            }
    }
}

// The HBM floor of the one-token BL4 layer, for measurement: one launch
// whose CTAs issue exactly the weight loads of the two one-token kernels for
// the experts ids[y] of the slots y (which & 1: the gate/up kernel's CTAs,
// bl4_decode_gate_up_t1's grid and per-wave rows; which & 2: the down
// kernel's, bl4_decode_down1's grid, 4 rows of every slot a CTA) and fold the
// loaded words into one word per CTA (sink[blockIdx.x]): no routing, lookups
// or stores, so its time is what streaming the step's bytes in those load
// patterns costs.  H, I <= 2048.
__global__ __launch_bounds__(256, 3) void decode_stream_probe(lutmoe_moe_desc d, const int32_t* __restrict__ ids,
                                                              int ns, int which, uint32_t* __restrict__ sink) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int H = d.hidden, I = d.inter;
    const int gcols = (I + 7) / 8;
    const int ng = (which & 1) ? gcols * ns : 0;
    const int bx = blockIdx.x;
    uint32_t acc = 0;
    if (bx < ng) {
        // bl4_decode_gate_up_t1: CTA (x, y), wave wv: gate rows i0, i0 + 1 and up rows of slot y
        const int y = bx / gcols, xcol = (bx - y * gcols) * 4 + wv;
        const int e = min(max(ids[y], 0), d.w13.num_experts - 1);
        const int i0 = 2 * xcol;
        if (i0 < I) {
            const int i1 = min(i0 + 1, I - 1);
            const int rows[4] = {i0, i1, I + i0, I + i1};
            const int64_t per = (int64_t)d.w13.rows * (H / 2);
            const uint8_t* codes = (const uint8_t*)d.w13.codes + e * per;
            const uint8_t* tabs = (const uint8_t*)d.w13.tables + e * per;
            const bool ok = 32 * lane < H;
            uint32_t cw[4][4];
            u32x4_t tw[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t ro = (uint32_t)rows[r] * (uint32_t)(H / 2);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    cw[r][q] = *reinterpret_cast<const uint32_t*>(codes +
                                                                  (ro + 4u * (uint32_t)min(lane + 64 * q, H / 8 - 1)));
                tw[r] = *reinterpret_cast<const u32x4_t*>(tabs + (ro + (ok ? 16 * lane : 0)));
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc ^= cw[r][0] ^ cw[r][1] ^ cw[r][2] ^ cw[r][3] ^ tw[r][0] ^ tw[r][1] ^ tw[r][2] ^ tw[r][3];
        }
    } else {
        // bl4_decode_down1: CTA = output rows h0 .. h0 + 3; wave wv: slots wv, wv + 4, ..
        const int h0 = (bx - ng) * kD1Rows;
        const int K = I, nd = K / 8;
        const int64_t per = (int64_t)d.w2.rows * (K / 2);
        const bool ok = 32 * lane < K;
        for (int a = wv; a < ns; a += 4) {
            const int e = min(max(ids[a], 0), d.w2.num_experts - 1);
            const uint8_t* codes = (const uint8_t*)d.w2.codes + e * per;
            const uint8_t* tabs = (const uint8_t*)d.w2.tables + e * per;
            uint32_t cw[4][4];
            u32x4_t tw[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t ro = (uint32_t)(h0 + r) * (uint32_t)(K / 2);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    cw[r][q] = *reinterpret_cast<const uint32_t*>(codes + (ro + 4u * (uint32_t)min(lane + 64 * q, nd - 1)));
                tw[r] = *reinterpret_cast<const u32x4_t*>(tabs + (ro + (ok ? 16 * lane : 0)));
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc ^= cw[r][0] ^ cw[r][1] ^ cw[r][2] ^ cw[r][3] ^ tw[r][0] ^ tw[r][1] ^ tw[r][2] ^ tw[r][3];
        }
    }
    acc = (uint32_t)wave_max_i32((int)(acc & 0x7fffffffu));
    __shared__ uint32_t s_acc[4];
    if (lane == 0) s_acc[wv] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sink[bx] = s_acc[0] ^ s_acc[1] ^ s_acc[2] ^ s_acc[3];
}

// tokens per pass: T=1 and T=2 recompute routing per CTA, larger T read it
// Tokens per pass of the expert loops (fmt_idx: 0 BL4, 1 nested, 2 REF).  Up
// to 32 tokens most active experts hold a few of them, and a 4-token BL4 pass
// would spend its FMAs and activation loads on empty positions (Qwen shape,
// MI355X: 2-token passes take T=4/8/16 from 58/85/121 to 50/72/108 us per
// layer; with the 4-row loops T=17/24/32 from 115/131/150 to 99/121/146 us).
// Past 16 tokens that holds while the positions per expert stay few (at most
// 3 on average, P / min(P, E_tot)); few experts holding many tokens each
// (top-2 of 8) and more than 32 tokens (the GEMV path forced) take 4.
// NestedLUT takes 2 up to 16 tokens, with chunks of one pass each (the
// routing kernel's chunking): its kernels then fit three waves a SIMD
// (T = 16 tier workload 95.6 -> 92.8 us; 2-token passes over 4-token chunks,
// which look every weight up twice, took 95.5 -> 99.5 us).  REF keeps 4.
inline int tb_for(int T, int fmt_idx, int P, int E_tot) {
    if (T <= 1) return 1;
    if (fmt_idx == 1) return T <= 16 ? 2 : 4;
    if (fmt_idx != 0) return T <= 2 ? 2 : 4;
    return T <= 16 || (T <= 32 && P <= 3 * std::min(P, E_tot)) ? 2 : 4;
}

}  // namespace

namespace lutmoe_host {

bool decode_v2_supported(const lutmoe_moe_desc* d, int T, int k) {
    const int E_tot = d->num_routed + d->num_shared;
    const int P = T * (k + d->num_shared);
    if (d->w13.format == LUTMOE_FMT_NESTED &&
        ((int64_t)d->w13.rows * d->w13.cols >= (int64_t(1) << 32) ||
         (int64_t)d->w2.rows * d->w2.cols >= (int64_t(1) << 32)))
        return false;
    if (d->w13.format == LUTMOE_FMT_REF &&
        (d->w13.block_size <= 0 || d->w13.block_size % 32 || d->w2.block_size <= 0 || d->w2.block_size % 32 ||
         (int64_t)d->w13.rows * d->w13.cols >= (int64_t(1) << 37) ||
         (int64_t)d->w2.rows * d->w2.cols >= (int64_t(1) << 37)))   // 32-bit block indices (ref_block32)
        return false;
    return E_tot <= kMaxEtot && P <= kMaxP;
}

int launch_nested_gemv(const lutmoe_weights* w, int expert, const uint16_t* x, int T, void* y, int y_dtype,
                       hipStream_t s) {
    if ((int64_t)w->rows * w->cols >= (int64_t(1) << 32)) return LUTMOE_EUNSUPPORTED;
    const dim3 grid((w->rows + 4 * kRows - 1) / (4 * kRows));
    if (T <= 1)
        hipLaunchKernelGGL((nested_gemv_kernel<1>), grid, dim3(256), 0, s, *w, expert, x, T, y, y_dtype);
    else if (T == 2)
        hipLaunchKernelGGL((nested_gemv_kernel<2>), grid, dim3(256), 0, s, *w, expert, x, T, y, y_dtype);
    else
        hipLaunchKernelGGL((nested_gemv_kernel<4>), grid, dim3(256), 0, s, *w, expert, x, T, y, y_dtype);
    return check_launch();
}

size_t decode_route_bytes() { return sizeof(RouteOut) + sizeof(RouteChunks) + sizeof(RoutePosW); }

size_t decode_stream_probe_ctas(const lutmoe_moe_desc* d, int ns, int which) {
    return (size_t)((which & 1) ? (d->inter + 7) / 8 * ns : 0) + ((which & 2) ? d->hidden / kD1Rows : 0);
}

int launch_decode_stream_probe(const lutmoe_moe_desc* d, const int32_t* ids, int ns, int which, uint32_t* sink,
                               hipStream_t s) {
    const size_t n = decode_stream_probe_ctas(d, ns, which);
    hipLaunchKernelGGL(decode_stream_probe, dim3((unsigned)n), dim3(256), 0, s, *d, ids, ns, which, sink);
    return check_launch();
}
int launch_decode_v2(const lutmoe_moe_desc* d, const uint16_t* x, const float* topk_w,
                     const int32_t* topk_ids, const float* logits, int T, int k, int renorm,
                     float scaling, uint16_t* act, void* route_ws, float* y_ws, void* out,
                     int out_dtype, int stages, hipStream_t s, const float* addend) {
    DecodeArgs A{};
    A.addend = addend;
    A.d = *d;
    A.x = x;
    A.topk_w = topk_w;
    A.topk_ids = topk_ids;
    A.logits = logits;
    A.T = T;
    A.k = k;
    A.renorm = renorm;
    A.scaling = scaling;
    A.act = act;
    A.out = out;
    A.out_dtype = out_dtype;
    A.route = (RouteOut*)route_ws;
    const int E_tot = d->num_routed + d->num_shared;
    const int P = T * (k + d->num_shared);
    const int max_active = P < E_tot ? P : E_tot;
    // T <= 2 with the pairs in one wave: both kernels route in registers; else
    // one routing kernel writes the workspace copy both kernels read.
    const bool pre = T > 2 || !(P <= 64 && (topk_ids != nullptr || d->num_routed <= 64));
    const bool nested = d->w13.format == LUTMOE_FMT_NESTED;
    const int fmt_idx = nested ? 1 : d->w13.format == LUTMOE_FMT_REF ? 2 : 0;
    const int tb = tb_for(T, fmt_idx, P, E_tot);
    A.tb = tb;   // before the routing launch: its chunking reads it
    int rc;
    if (pre && (stages & LUTMOE_STAGE_ROUTE)) {
        hipLaunchKernelGGL(decode_route_kernel, dim3(1), dim3(1024), 0, s, A);
        if ((rc = check_launch())) return rc;
    }
#define LUTMOE_DECODE_CASE(N, TB, PRE, FMT, KERNEL, GRID, BLOCK, LDS) \
    case N: hipLaunchKernelGGL((KERNEL<TB, PRE, FMT>), GRID, BLOCK, LDS, s, A); break;
#define LUTMOE_DECODE_FMTS(N, TB, PRE, KERNEL, GRID, BLOCK, LDS)                    \
    LUTMOE_DECODE_CASE(N, TB, PRE, LUTMOE_FMT_BL4, KERNEL, GRID, BLOCK, LDS)        \
    LUTMOE_DECODE_CASE(N + 1, TB, PRE, LUTMOE_FMT_NESTED, KERNEL, GRID, BLOCK, LDS) \
    LUTMOE_DECODE_CASE(N + 2, TB, PRE, LUTMOE_FMT_REF, KERNEL, GRID, BLOCK, LDS)
#define LUTMOE_DECODE_LAUNCH(KERNEL, PRE, GRID, BLOCK, LDS)                 \
    switch (tb * 8 + ((PRE) ? 4 : 0) + fmt_idx) {                    \
        LUTMOE_DECODE_FMTS(8, 1, false, KERNEL, GRID, BLOCK, LDS)           \
        LUTMOE_DECODE_FMTS(12, 1, true, KERNEL, GRID, BLOCK, LDS)           \
        LUTMOE_DECODE_FMTS(16, 2, false, KERNEL, GRID, BLOCK, LDS)          \
        LUTMOE_DECODE_FMTS(20, 2, true, KERNEL, GRID, BLOCK, LDS)           \
        LUTMOE_DECODE_FMTS(36, 4, true, KERNEL, GRID, BLOCK, LDS)           \
        default: return LUTMOE_EINVAL;                                      \
    }
    // work items: the active slots, cut into chunks by decode_route_kernel
    // (at most P, and at most one more per slot than ceil(P / TB))
    const int max_work = pre ? std::min(P, max_active + (P + tb - 1) / tb) : max_active;
    if ((stages & LUTMOE_STAGE_GATE_UP) && fmt_idx != 1 && tb == 1 && !pre && T == 1 && d->hidden <= kWChunk) {
        const dim3 grid((d->inter + 7) / 8, max_work);   // 4 waves x 2 intermediate indices
        if (fmt_idx == 0) hipLaunchKernelGGL(bl4_decode_gate_up_t1, grid, dim3(256), 0, s, A);
        else hipLaunchKernelGGL(ref_decode_gate_up_t1, grid, dim3(256), 0, s, A);
        if ((rc = check_launch())) return rc;
    } else if (stages & LUTMOE_STAGE_GATE_UP) {
        // intermediate indices per CTA (gu2_gate_up_for: 2)
        const int per_cta = (fmt_idx == 0 && (tb == 1 || (pre && (tb == 2 || tb == 4)))) ? 2 : 4 * kGuWaves;
        const dim3 grid((d->inter + per_cta - 1) / per_cta, max_work);
        LUTMOE_DECODE_LAUNCH(bl4_decode_gate_up, pre, grid, dim3(64 * kGuWaves), 0)
        if ((rc = check_launch())) return rc;
    }
    if (stages & LUTMOE_STAGE_DOWN) {
        const int hrows = (fmt_idx == 0 && tb == 1) ? 4 : kRows;   // output rows per CTA (down_body4: 4)
        const dim3 grid((d->hidden + hrows - 1) / hrows);
        const size_t lds = (size_t)P * kRows * sizeof(float);
        // the routing comes from the copy in the workspace (written by the
        // gate/up kernel's first CTA, or by decode_route_kernel)
        if (max_active > 8) {
            // many experts: y + combine, every slot in parallel
            const dim3 gy((d->hidden + kRows - 1) / kRows, (max_work + 3) / 4);
#define LUTMOE_DOWN_Y(TB, FMT) hipLaunchKernelGGL((bl4_decode_down_y<TB, FMT>), gy, dim3(256), 0, s, A, y_ws)
            // BL4 passes of one or two tokens: 4 rows a wave (bl4_decode_down_y4;
            // T = 8: 72 -> 68 us a layer); four-token passes keep 8 rows a
            // wave (T = 32: 152 against 169 us with 4)
            const dim3 gy4((d->hidden + 3) / 4, (max_work + 3) / 4);
            switch (tb * 4 + fmt_idx + (fmt_idx == 0 && tb <= 2 ? 64 : 0)) {
                case 68: hipLaunchKernelGGL((bl4_decode_down_y4<1>), gy4, dim3(256), 0, s, A, y_ws); break;
                case 72: hipLaunchKernelGGL((bl4_decode_down_y4<2>), gy4, dim3(256), 0, s, A, y_ws); break;
                case 5: LUTMOE_DOWN_Y(1, LUTMOE_FMT_NESTED); break;
                case 6: LUTMOE_DOWN_Y(1, LUTMOE_FMT_REF); break;
                case 9: LUTMOE_DOWN_Y(2, LUTMOE_FMT_NESTED); break;
                case 10: LUTMOE_DOWN_Y(2, LUTMOE_FMT_REF); break;
                case 16: LUTMOE_DOWN_Y(4, LUTMOE_FMT_BL4); break;
                case 17: LUTMOE_DOWN_Y(4, LUTMOE_FMT_NESTED); break;
                case 18: LUTMOE_DOWN_Y(4, LUTMOE_FMT_REF); break;
                default: return LUTMOE_EINVAL;
            }
#undef LUTMOE_DOWN_Y
            if ((rc = check_launch())) return rc;
            const int32_t* inv = ((const RouteOut*)route_ws)->inv;
            return launch_combine(y_ws, inv, T, k + d->num_shared, d->hidden, out, out_dtype, s, 1, 0, addend);
        }
        if (fmt_idx == 0 && (tb == 1 || (tb == 2 && T == 2)) && T * (k + d->num_shared) <= 16 * tb) {
            // one or two tokens, BL4: 4 output rows a CTA, one slot a wave, the
            // routing read in place (s_y holds up to 16 positions a token)
            const dim3 g1(d->hidden / kD1Rows);
            if (tb == 1) hipLaunchKernelGGL((bl4_decode_down1<1>), g1, dim3(256), 0, s, A);
            else hipLaunchKernelGGL((bl4_decode_down1<2>), g1, dim3(256), 0, s, A);
            return check_launch();
        }
        if (fmt_idx == 2 && tb == 1 && d->inter <= 2048) {
            // one token, REF: flat 32-byte units over 4 rows
            const dim3 g1(d->hidden / kD1Rows);
            switch ((d->inter + 511) / 512) {
                case 1: hipLaunchKernelGGL(ref_decode_down1<1>, g1, dim3(256), 0, s, A); break;
                case 2: hipLaunchKernelGGL(ref_decode_down1<2>, g1, dim3(256), 0, s, A); break;
                case 3: hipLaunchKernelGGL(ref_decode_down1<3>, g1, dim3(256), 0, s, A); break;
                default: hipLaunchKernelGGL(ref_decode_down1<4>, g1, dim3(256), 0, s, A); break;
            }
            return check_launch();
        }
        LUTMOE_DECODE_LAUNCH(bl4_decode_down, true, grid, dim3(256), lds)
        return check_launch();
    }
#undef LUTMOE_DECODE_CASE
#undef LUTMOE_DECODE_FMTS
#undef LUTMOE_DECODE_LAUNCH
    return LUTMOE_OK;
}

}  // namespace lutmoe_host

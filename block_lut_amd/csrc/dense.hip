// Dense bf16 shared expert of the MoE layer (gfx950).
//
// The reference keeps a model's shared experts unquantised: DeepseekV2MoE_LUT
// holds them as bf16 ColumnParallelLinear / RowParallelLinear layers and adds
// their output to the routed experts' (vllm_lut/moe_layer.py:186-200,
// 348-353); the HF blocks use dense DeepseekV2MLP / Qwen2MoeMLP
// (customized/deepseek.py:52-58, 111-115; customized/qwen.py:40-43, 96-100).
// Here that MLP runs beside the LUT experts on the same activations:
//   act_s[t] = bf16(silu(x[t] . Wg^T) * (x[t] . Wu^T))     W13s = [Wg; Wu] bf16 [2 Is][H]
//   y_s[t]   = w[t] * (act_s[t] . W2s^T)                    W2s bf16 [H][Is], fp32
// with w[t] = 1, or sigmoid(x[t] . shared_gate) (Qwen's shared_expert_gate),
// and y_s is added to each token's sum of routed experts by the kernel that
// writes the layer's output, before its one rounding.
//
// Decode (few tokens): HBM-bound GEMVs.  A wave owns 4 weight rows; lane l
// takes columns 8l .. 8l + 7 of every 512-column step, 16-byte loads of the
// rows (four steps in flight per row) and of the activations, v_dot2_f32_bf16,
// one 4-value reduce-scatter per token (lane 16r: row r).  Gate/up waves take
// intermediate indices i0, i0 + 1 (rows i0, i0 + 1, Is + i0, Is + i0 + 1), so
// the SwiGLU pairs meet in one wave.  Tokens go in passes of up to 4.
// Prefill: the register-staged MFMA tile of the grouped LUT-GEMM with dense B
// fragments (a lane's 32 columns of its weight row, straight from global
// memory) in place of the table lookups; tiles of 256 tokens x 256 weight rows
// (gate/up: 128 intermediate indices, gate and up rows), K step 64.
#include "common.h"
#include "kernels.h"
#include "lut_core.h"

using namespace lutmoe;

namespace {

constexpr int kDStep = 512;     // columns per lane step (64 lanes x 8)
constexpr int kDSteps = 4;      // steps in flight per row

// w[t] = sigmoid(x[t] . g) (fp32 sum of bf16 products), or 1 without a gate;
// one wave per token.
__global__ __launch_bounds__(256) void dense_token_weights_kernel(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ g, int T, int H,
                                                                  float* __restrict__ w) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const float v = g ? shared_gate_weight(x + (int64_t)t * H, g, H) : 1.0f;
    if ((threadIdx.x & 63) == 0) w[t] = v;
}

// TB tokens a pass.  kSwiGLU: W = W13s [2I][K], out = act_s bf16 [T][I];
// else W = W2s [M][K], out = y_s fp32 [T][M] times tokw[t].
template <int TB, bool kSwiGLU>
__global__ __launch_bounds__(256, 2) void dense_gemv_kernel(const uint16_t* __restrict__ W, int M, int K, int I,
                                                            const uint16_t* __restrict__ x, int T,
                                                            const float* __restrict__ tokw, void* __restrict__ out) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int unit = blockIdx.x * 4 + wv;
    int rows[4];
    if constexpr (kSwiGLU) {
        const int i0 = 2 * unit;
        if (i0 >= I) return;
        rows[0] = i0;
        rows[1] = i0 + 1;
        rows[2] = I + i0;
        rows[3] = I + i0 + 1;
    } else {
        const int r0 = 4 * unit;
        if (r0 >= M) return;
#pragma unroll
        for (int r = 0; r < 4; ++r) rows[r] = min(r0 + r, M - 1);
    }
    const int nstep = (K + kDStep - 1) / kDStep;
    for (int t0 = 0; t0 < T; t0 += TB) {
        const int nt = min(TB, T - t0);
        float acc[4][TB];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < TB; ++t) acc[r][t] = 0.f;
        for (int s0 = 0; s0 < nstep; s0 += kDSteps) {
            // every load of kDSteps steps issued before any is used (columns
            // past K: the row's last 8 columns, their activations zeroed)
            u32x4_t wr[kDSteps][4], xr[kDSteps][TB];
#pragma unroll
            for (int s = 0; s < kDSteps; ++s) {
                const int col = min((s0 + s) * kDStep + 8 * lane, K - 8);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    wr[s][r] = *reinterpret_cast<const u32x4_t*>(W + (int64_t)rows[r] * K + col);
#pragma unroll
                for (int t = 0; t < TB; ++t)
                    xr[s][t] = *reinterpret_cast<const u32x4_t*>(x + (int64_t)(t0 + min(t, nt - 1)) * K + col);
            }
#pragma unroll
            for (int s = 0; s < kDSteps; ++s) {
                const bool ok = (s0 + s) * kDStep + 8 * lane < K;
#pragma unroll
                for (int t = 0; t < TB; ++t) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t xv = ok ? xr[s][t][j] : 0u;
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[r][t] = dot2_bf16(wr[s][r][j], xv, acc[r][t]);
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TB; ++t) {
            if (t >= nt) break;
            const float v = wave_reduce4(acc[0][t], acc[1][t], acc[2][t], acc[3][t]);   // lane 16r: row r
            if constexpr (kSwiGLU) {
                const float u = from_upper_half(v);   // lanes 0 / 16: up rows 2 / 3
                if (lane == 0 || lane == 16)
                    ((uint16_t*)out)[(int64_t)(t0 + t) * I + rows[lane >> 4]] = (uint16_t)f32_to_bf16(silu_mul(v, u));
            } else {
                const int r = lane >> 4;
                if ((lane & 15) == 0 && 4 * unit + r < M)
                    ((float*)out)[(int64_t)(t0 + t) * M + 4 * unit + r] = v * tokw[t0 + t];
            }
        }
    }
}

// ---------------------------------------------------------------- prefill
constexpr int kBM = 256;          // tokens per tile
constexpr int kBN = 256;          // weight rows per tile
constexpr int kBK = 64;           // K step
constexpr int kAStride = 72;      // bf16 per LDS A row (64 + 8 pad)

// One lane's B operand for one K step: its two weight rows (n-tiles), columns
// 32h .. 32h + 31 of the step, 8 per k-substep.
struct DenseBStep {
    u32x4_t b[2][4];
    __device__ __forceinline__ void load(const uint16_t* W, const int (&row)[2], int K, int kb, int bh) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const uint16_t* p = W + (int64_t)row[nt] * K + kb * kBK + 32 * bh;
#pragma unroll
            for (int q = 0; q < 4; ++q) b[nt][q] = *reinterpret_cast<const u32x4_t*>(p + 8 * q);
        }
    }
};

// Tile (blockIdx.x: weight-row block, blockIdx.y: 256 tokens), NMT m-tiles
// of 32 tokens.  kGateUp: A = x [T][H], out = act_s [T][I]; else A = act_s
// [T][I], out = y_s [T][H] fp32 times tokw[t].  The k-substep column map is
// the grouped LUT-GEMM's: lane half h takes columns 32h + 8ks .. +7 in both
// operands (a consistent permutation of k).
template <bool kGateUp, int NMT>
__device__ __forceinline__ void dense_tile(const uint16_t* __restrict__ W, const uint16_t* __restrict__ src,
                                           int T, int H, int I, const float* __restrict__ tokw,
                                           void* __restrict__ dst, uint16_t (*s_a)[kBM * kAStride]) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int K = kGateUp ? H : I;
    const int nkb = K / kBK;
    const int n0 = blockIdx.x * (kGateUp ? kBN / 2 : kBN);
    const int m0 = blockIdx.y * kBM;
    const int nvalid = min(kBM, T - m0);
    const uint16_t* a_src = src + (int64_t)(m0 + min(tid, nvalid - 1)) * K;
    const int bn = lane & 31, bh = lane >> 5;
    int b_row[2];
    if (kGateUp) {
        const int i = min(n0 + 32 * wv + bn, I - 1);
        b_row[0] = i;
        b_row[1] = I + i;
    } else {
        b_row[0] = min(n0 + 64 * wv + bn, H - 1);
        b_row[1] = min(n0 + 64 * wv + 32 + bn, H - 1);
    }
    u32x4_t ra[8];
    auto load_a = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 8; ++q) ra[q] = *reinterpret_cast<const u32x4_t*>(a_src + kb * kBK + 8 * q);
    };
    auto store_a = [&](int buf) __attribute__((always_inline)) {
        uint16_t* ad = &s_a[buf][tid * kAStride];
#pragma unroll
        for (int q = 0; q < 8; ++q) *reinterpret_cast<u32x4_t*>(ad + 8 * q) = ra[q];
    };
    f32x16_t acc[NMT][2];
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][nt][i] = 0.f;
    auto frag_a = [&](int buf, int ks, bf16x8_t (&af)[NMT]) __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt)
            af[mt] = *reinterpret_cast<const bf16x8_t*>(&s_a[buf][(mt * 32 + bn) * kAStride + 32 * bh + 8 * ks]);
    };
    // Entering step kb: A(kb) in LDS buffer kb & 1, A(kb + 1) in flight to
    // registers, B of step kb in bcur and of step kb + 1 in flight to bnext.
    DenseBStep bcur, bnext;
    load_a(0);
    bcur.load(W, b_row, K, 0, bh);
    store_a(0);
    load_a(min(1, nkb - 1));
    bnext.load(W, b_row, K, min(1, nkb - 1), bh);
    __syncthreads();
    bf16x8_t af[NMT];
    frag_a(0, 0, af);
    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        store_a(buf ^ 1);
        load_a(min(kb + 2, nkb - 1));
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8_t af_n[NMT];
            if (ks < 3) frag_a(buf, ks + 1, af_n);
            __builtin_amdgcn_sched_barrier(0);
            const bf16x8_t b0 = __builtin_bit_cast(bf16x8_t, bcur.b[0][ks]);
            const bf16x8_t b1 = __builtin_bit_cast(bf16x8_t, bcur.b[1][ks]);
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt) {
                acc[mt][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], b0, acc[mt][0], 0, 0, 0);
                acc[mt][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], b1, acc[mt][1], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (ks < 3) {
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt) af[mt] = af_n[mt];
            }
        }
        bcur = bnext;
        bnext.load(W, b_row, K, min(kb + 2, nkb - 1), bh);
        __syncthreads();
        frag_a(buf ^ 1, 0, af);
    }
    // ---- epilogue.  D layout: lane (n = lane % 32, h = lane / 32), element
    // i -> row m = 8 (i / 4) + 4h + (i % 4), column n.
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = mt * 32 + 8 * (i >> 2) + 4 * bh + (i & 3);
            if (m >= nvalid) continue;
            const int t = m0 + m;
            if (kGateUp) {
                const int ii = n0 + 32 * wv + bn;
                if (ii < I)
                    ((uint16_t*)dst)[(int64_t)t * I + ii] =
                        (uint16_t)f32_to_bf16(silu_mul(acc[mt][0][i], acc[mt][1][i]));
            } else {
                const float w = tokw[t];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const int h = n0 + 64 * wv + 32 * nt + bn;
                    if (h < H) ((float*)dst)[(int64_t)t * H + h] = acc[mt][nt][i] * w;
                }
            }
        }
    }
}

template <bool kGateUp>
__global__ __launch_bounds__(256, 1) void dense_mfma_kernel(const uint16_t* __restrict__ W,
                                                            const uint16_t* __restrict__ src, int T, int H, int I,
                                                            const float* __restrict__ tokw, void* __restrict__ dst) {
    __shared__ __attribute__((aligned(16))) uint16_t s_a[2][kBM * kAStride];
    const int nmt = (min(kBM, T - (int)blockIdx.y * kBM) + 31) / 32;
    switch (nmt) {
#define LUTMOE_DENSE_CASE(n) \
    case n: dense_tile<kGateUp, n>(W, src, T, H, I, tokw, dst, s_a); break;
        LUTMOE_DENSE_CASE(1) LUTMOE_DENSE_CASE(2) LUTMOE_DENSE_CASE(3) LUTMOE_DENSE_CASE(4)
        LUTMOE_DENSE_CASE(5) LUTMOE_DENSE_CASE(6) LUTMOE_DENSE_CASE(7) LUTMOE_DENSE_CASE(8)
#undef LUTMOE_DENSE_CASE
        default: break;
    }
}

template <bool kSwiGLU>
int dense_gemv_launch(const uint16_t* W, int M, int K, int I, const uint16_t* x, int T, const float* tokw,
                      void* out, hipStream_t s) {
    const int units = kSwiGLU ? (I + 1) / 2 : (M + 3) / 4;
    const dim3 grid((units + 3) / 4);
    if (T <= 1)
        hipLaunchKernelGGL((dense_gemv_kernel<1, kSwiGLU>), grid, dim3(256), 0, s, W, M, K, I, x, T, tokw, out);
    else if (T == 2)
        hipLaunchKernelGGL((dense_gemv_kernel<2, kSwiGLU>), grid, dim3(256), 0, s, W, M, K, I, x, T, tokw, out);
    else
        hipLaunchKernelGGL((dense_gemv_kernel<4, kSwiGLU>), grid, dim3(256), 0, s, W, M, K, I, x, T, tokw, out);
    return lutmoe_host::check_launch();
}

}  // namespace

namespace lutmoe_host {

int launch_dense_gate_up(const lutmoe_moe_desc* d, const uint16_t* x, int T, bool mfma, uint16_t* act,
                         float* tokw, hipStream_t s) {
    const int H = d->hidden, I = d->dense_inter;
    hipLaunchKernelGGL(dense_token_weights_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x,
                       (const uint16_t*)d->shared_gate, T, H, tokw);
    int rc = check_launch();
    if (rc) return rc;
    const uint16_t* W = (const uint16_t*)d->dense_w13;
    if (!mfma) return dense_gemv_launch<true>(W, 2 * I, H, I, x, T, tokw, act, s);
    const dim3 grid((I + kBN / 2 - 1) / (kBN / 2), (T + kBM - 1) / kBM);
    hipLaunchKernelGGL((dense_mfma_kernel<true>), grid, dim3(256), 0, s, W, x, T, H, I, (const float*)tokw,
                       (void*)act);
    return check_launch();
}

int launch_dense_down(const lutmoe_moe_desc* d, const uint16_t* act, int T, bool mfma, const float* tokw, float* y,
                      hipStream_t s) {
    const int H = d->hidden, I = d->dense_inter;
    const uint16_t* W = (const uint16_t*)d->dense_w2;
    if (!mfma) return dense_gemv_launch<false>(W, H, I, I, act, T, tokw, y, s);
    const dim3 grid((H + kBN - 1) / kBN, (T + kBM - 1) / kBM);
    hipLaunchKernelGGL((dense_mfma_kernel<false>), grid, dim3(256), 0, s, W, act, T, H, I, tokw, (void*)y);
    return check_launch();
}

}  // namespace lutmoe_host

// Prefill grouped LUT-GEMM on MFMA (v_mfma_f32_32x32x16_bf16, gfx950).
//
// Positions (permuted (token, slot) pairs) of one expert are contiguous, so
// the grouped GEMM walks tiles of 128 positions of one expert at a time
// (tile -> expert found by a scan of the expert offsets; no host sync).
//
// CTA = 4 waves, tile = 128 positions x 256 weight rows, K step = 64 (one
// BL4 codebook block per row).  Per K step:
//   A (activations, bf16) 128 x 64 -> LDS (row stride padded to 144 B);
//     stage 1 gathers the rows x[token(perm[p])] directly (fused permute).
//   B tables: the 256 rows' 32-byte bf16 tables of block kb -> LDS.
//   B codes: each lane reads its own 16 bytes (32 codes) of its row straight
//     from global memory into registers; the four 16-wide k-substeps of the
//     MFMA take bytes 4ks..4ks+3, i.e. lane half h covers columns
//     32h + 8ks .. +7 of the block.  A fragments use the same column map, so
//     the contraction is unchanged (any consistent permutation of k is).
//   The lookup (LDS table[row][code]) yields the bf16 dequantised weights
//   (bit-exact rule) that form the MFMA B fragment.
// Wave w owns 64 weight rows = 2 MFMA n-tiles and all 4 m-tiles of 32
// positions: 8 accumulators of 16 fp32.
//   stage 1 (gate_up): n-tile 0 = gate rows i0+32w.., n-tile 1 = up rows
//     I+i0+32w..; epilogue act = bf16(silu(g) * u) written per position.
//   stage 2 (down): n-tiles = rows h0+64w.., +32; epilogue y_pos[p][h] =
//     acc * routing weight (fp32), summed per token by the combine kernel.
// Restates the prefill branch of LUTFusedMoEMethod.apply
// (vllm_lut/quant_method.py:261-277) and the per-expert GEMMs of the
// llama.cpp mul_mat_id patch (llama-cpp-port/patches/0001:151-208), with the
// routed tokens only instead of all T tokens.
#include "common.h"
#include "kernels.h"

using namespace lutmoe;
using lutmoe_host::MoeRouting;

namespace {

constexpr int kBM = 128;          // positions per tile
constexpr int kBN = 256;          // weight rows per tile
constexpr int kBK = 64;           // K step
constexpr int kAStride = 72;      // bf16 per LDS A row (64 + 8 pad)

struct TileInfo {
    int e, m0, p0, n;
};

// blockIdx.y -> (expert, first position of the tile); e = -1 when past the end.
__device__ __forceinline__ TileInfo find_tile(const MoeRouting& rt, int j) {
    __shared__ TileInfo s_tile;
    if (threadIdx.x == 0) {
        TileInfo ti{-1, 0, 0, 0};
        int rem = j;
        for (int e = 0; e < rt.num_experts_total; ++e) {
            const int p0 = rt.offsets[e], n = rt.offsets[e + 1] - p0;
            const int nt = (n + kBM - 1) / kBM;
            if (rem < nt) { ti = TileInfo{e, rem * kBM, p0, n}; break; }
            rem -= nt;
        }
        s_tile = ti;
    }
    __syncthreads();
    return s_tile;
}

__device__ __forceinline__ bf16x8_t lookup8(uint32_t w, const uint16_t* tab) {
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t b = (w >> (8 * j)) & 0xffu;
        o[j] = (uint32_t)tab[b & 15u] | ((uint32_t)tab[b >> 4] << 16);
    }
    return __builtin_bit_cast(bf16x8_t, make_uint4(o[0], o[1], o[2], o[3]));
}

__device__ __forceinline__ bf16x8_t lookup8_ref(uint2 w, const float* cb, float am) {
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t word = j < 2 ? w.x : w.y;
        const uint32_t c0 = (word >> (16 * (j & 1))) & 0xffu;
        const uint32_t c1 = (word >> (16 * (j & 1) + 8)) & 0xffu;
        o[j] = f32_to_bf16(cb[c0] * am) | (f32_to_bf16(cb[c1] * am) << 16);
    }
    return __builtin_bit_cast(bf16x8_t, make_uint4(o[0], o[1], o[2], o[3]));
}

template <bool kGateUp, int kFmt>
__global__ __launch_bounds__(256, 2) void prefill_kernel(lutmoe_moe_desc d,
                                                         const uint16_t* __restrict__ src,
                                                         MoeRouting rt, void* __restrict__ dst) {
    __shared__ __attribute__((aligned(16))) uint16_t s_a[kBM * kAStride];
    __shared__ __attribute__((aligned(16))) uint16_t s_t[kFmt == LUTMOE_FMT_BL4 ? kBN * 16 : 8];
    __shared__ float s_cb[kFmt == LUTMOE_FMT_REF ? 256 : 1];
    const TileInfo ti = find_tile(rt, blockIdx.y);
    if (ti.e < 0) return;
    const lutmoe_weights& w = kGateUp ? d.w13 : d.w2;
    if (kFmt == LUTMOE_FMT_REF) {
        const uint16_t* cb = (const uint16_t*)w.codebook;
        s_cb[threadIdx.x] = bf16_to_f32(cb[threadIdx.x]);
    }
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int I = d.inter, H = d.hidden;
    const int K = kGateUp ? H : I;
    const int nkb = K / kBK;
    const int n0 = blockIdx.x * (kGateUp ? kBN / 2 : kBN);   // first intermediate idx / h row
    const int nmax = kGateUp ? I : H;                        // bound on n0 + offset

    // ---- rows owned by this thread for A staging and table staging
    const int a_row = tid >> 1, a_half = tid & 1;
    int a_pos = ti.p0 + ti.m0 + a_row;
    a_pos = min(a_pos, ti.p0 + ti.n - 1);
    const uint16_t* a_src;
    if (kGateUp) a_src = src + (int64_t)(rt.perm[a_pos] / rt.k_eff) * H;
    else a_src = src + (int64_t)a_pos * I;
    a_src += 32 * a_half;

    auto wrow = [&](int local) -> int {   // weight row of local tile row 0..255
        if (kGateUp) {
            const int i = min(n0 + (local & 127), I - 1);
            return local < 128 ? i : I + i;
        }
        return min(n0 + local, H - 1);
    };
    const int t_row = wrow(tid);

    // ---- B rows of this lane: n-tile 0/1
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
    const int b_local[2] = {kGateUp ? 32 * wv + bn : 64 * wv + bn,
                            kGateUp ? 128 + 32 * wv + bn : 64 * wv + 32 + bn};

    const uint8_t* codes;
    const uint16_t* tables;
    const uint16_t* absmax = nullptr;
    if (kFmt == LUTMOE_FMT_BL4) {
        const int64_t per = (int64_t)w.rows * (w.cols / 2);
        codes = (const uint8_t*)w.codes + ti.e * per;
        tables = (const uint16_t*)((const uint8_t*)w.tables + ti.e * per);
    } else {
        codes = (const uint8_t*)w.codes + (int64_t)ti.e * w.rows * w.cols;
        tables = nullptr;
        absmax = (const uint16_t*)w.tables + (int64_t)ti.e * w.absmax_per_expert;
    }

    // ---- register staging for the next K step
    uint4 ra[4];
    uint4 rt2[2];
    uint4 rc[2][2];   // BL4: [ntile][0] = 16 B codes; REF: [ntile][0..1] = 32 B codes
    float ram[2];

    auto load_step = [&](int kb) {
#pragma unroll
        for (int q = 0; q < 4; ++q) ra[q] = *reinterpret_cast<const uint4*>(a_src + kb * kBK + 8 * q);
        if (kFmt == LUTMOE_FMT_BL4) {
            const uint16_t* tp = tables + (int64_t)t_row * (K / 2 / 2) + kb * 16;
            rt2[0] = *reinterpret_cast<const uint4*>(tp);
            rt2[1] = *reinterpret_cast<const uint4*>(tp + 8);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                rc[nt][0] = *reinterpret_cast<const uint4*>(codes + (int64_t)b_row[nt] * (K / 2) + kb * 32 + 16 * bh);
        } else {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const int64_t flat = (int64_t)b_row[nt] * K + kb * kBK + 32 * bh;
                rc[nt][0] = *reinterpret_cast<const uint4*>(codes + flat);
                rc[nt][1] = *reinterpret_cast<const uint4*>(codes + flat + 16);
                int64_t b = ((int64_t)b_row[nt] * K + kb * kBK) / w.block_size;
                b = b < w.absmax_per_expert ? b : w.absmax_per_expert - 1;
                ram[nt] = bf16_to_f32(absmax[b]);
            }
        }
    };

    f32x16_t acc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][nt][i] = 0.f;

    load_step(0);
    for (int kb = 0; kb < nkb; ++kb) {
        // registers -> LDS
        uint16_t* ad = s_a + a_row * kAStride + 32 * a_half;
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4*>(ad + 8 * q) = ra[q];
        if (kFmt == LUTMOE_FMT_BL4) {
            *reinterpret_cast<uint4*>(s_t + tid * 16) = rt2[0];
            *reinterpret_cast<uint4*>(s_t + tid * 16 + 8) = rt2[1];
        }
        uint4 cc[2][2];
        float cam[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            cc[nt][0] = rc[nt][0];
            cc[nt][1] = rc[nt][1];
            cam[nt] = ram[nt];
        }
        __syncthreads();
        if (kb + 1 < nkb) load_step(kb + 1);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8_t bf[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                if (kFmt == LUTMOE_FMT_BL4) {
                    const uint32_t wd = ks == 0 ? cc[nt][0].x : ks == 1 ? cc[nt][0].y : ks == 2 ? cc[nt][0].z : cc[nt][0].w;
                    bf[nt] = lookup8(wd, s_t + b_local[nt] * 16);
                } else {
                    const uint4 q4 = cc[nt][ks >> 1];
                    const uint2 wd = (ks & 1) ? make_uint2(q4.z, q4.w) : make_uint2(q4.x, q4.y);
                    bf[nt] = lookup8_ref(wd, s_cb, cam[nt]);
                }
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(
                    s_a + (mt * 32 + bn) * kAStride + 32 * bh + 8 * ks);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf[nt], acc[mt][nt], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // ---- epilogue.  D layout: lane (n = lane%32, h = lane/32), element i ->
    // row m = 8*(i/4) + 4*h + (i%4), column n.
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = mt * 32 + 8 * (i >> 2) + 4 * bh + (i & 3);
            if (ti.m0 + m >= ti.n) continue;
            const int p = ti.p0 + ti.m0 + m;
            if (kGateUp) {
                const int ii = n0 + 32 * wv + bn;
                if (ii < I)
                    ((uint16_t*)dst)[(int64_t)p * I + ii] =
                        (uint16_t)f32_to_bf16(silu_mul(acc[mt][0][i], acc[mt][1][i]));
            } else {
                const float pw = rt.pair_w[rt.perm[p]];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const int h = n0 + 64 * wv + 32 * nt + bn;
                    if (h < H) ((float*)dst)[(int64_t)p * H + h] = acc[mt][nt][i] * pw;
                }
            }
        }
    }
}

inline int max_tiles(int P, int E_tot) { return (P + kBM - 1) / kBM + E_tot; }

}  // namespace

namespace lutmoe_host {

int launch_prefill_gate_up(const lutmoe_moe_desc* d, const uint16_t* x, const MoeRouting& r,
                           uint16_t* act, int P, hipStream_t s) {
    const dim3 grid((d->inter + kBN / 2 - 1) / (kBN / 2), max_tiles(P, r.num_experts_total));
    if (d->w13.format == LUTMOE_FMT_REF)
        hipLaunchKernelGGL((prefill_kernel<true, LUTMOE_FMT_REF>), grid, dim3(256), 0, s, *d, x, r, (void*)act);
    else
        hipLaunchKernelGGL((prefill_kernel<true, LUTMOE_FMT_BL4>), grid, dim3(256), 0, s, *d, x, r, (void*)act);
    return check_launch();
}

int launch_prefill_down(const lutmoe_moe_desc* d, const uint16_t* act, const MoeRouting& r,
                        float* y_pos, int P, hipStream_t s) {
    const dim3 grid((d->hidden + kBN - 1) / kBN, max_tiles(P, r.num_experts_total));
    if (d->w2.format == LUTMOE_FMT_REF)
        hipLaunchKernelGGL((prefill_kernel<false, LUTMOE_FMT_REF>), grid, dim3(256), 0, s, *d, act, r, (void*)y_pos);
    else
        hipLaunchKernelGGL((prefill_kernel<false, LUTMOE_FMT_BL4>), grid, dim3(256), 0, s, *d, act, r, (void*)y_pos);
    return check_launch();
}

}  // namespace lutmoe_host

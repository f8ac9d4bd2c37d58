// Prefill grouped LUT-GEMM on MFMA (v_mfma_f32_32x32x16_bf16, gfx950).
//
// Positions (permuted (token, slot) pairs) of one expert are contiguous, so a
// tile is up to 256 positions of one expert and 256 weight rows; K step = 64
// (one BL4 codebook block per row).  Wave w owns 64 weight rows (2 MFMA
// n-tiles) and ALL m-tiles of 32 positions: up to 8 x 2 accumulators of 16
// fp32 (256 per lane, held in AGPRs); m-tiles past the expert's position count
// are skipped, so a tile costs what its positions need.
//
// prefill_ring_kernel is persistent: one CTA per CU takes tiles one after
// another, longest first from a launch counter (no host sync).  Operands go global -> LDS by direct loads
// through a ring of stages (3 of 48 KB; 6 of 24 KB for tiles of at most 64
// positions), and the next tile's first stages are issued as soon as a K loop
// ends, so that they land while the epilogue stores straight from the
// accumulators.  B fragments are the rows' bf16 tables looked up per code (an
// SDWA add and a ds_read_u16 per weight; tiles of at most 64 positions look
// the tables up in registers instead).
//   stage 1 (gate_up): n-tile 0 = gate rows i0+32w.., n-tile 1 = up rows
//     I+i0+32w..; epilogue act = bf16(silu(g) * u) per position.  Its MFMAs
//     take the weights as the A operand, so a lane's accumulators hold runs
//     of 4 output columns of one position (8-byte bf16 stores).
//   stage 2 (down): n-tiles = rows h0+64w.., +32; epilogue y_pos[p][h] =
//     acc * routing weight (fp32), summed per token by the combine kernel.
// prefill_ref_kernel (REF stacks the ring cannot address) stages its
// operands through registers, one tile per CTA (find_tile).
// Restates the prefill branch of LUTFusedMoEMethod.apply
// (vllm_lut/quant_method.py:261-277) and the per-expert GEMMs of the
// llama.cpp mul_mat_id patch (llama-cpp-port/patches/0001:151-208), over the
// routed tokens only instead of all T tokens.
#include <atomic>

#include "common.h"
#include "kernels.h"
#include "lut_core.h"

using namespace lutmoe;
using lutmoe_host::MoeRouting;

namespace {

constexpr int kBM = 256;          // positions per tile (max)
constexpr int kBN = 256;          // weight rows per tile
constexpr int kBK = 64;           // K step
constexpr int kAStride = 72;      // bf16 per LDS A row (64 + 8 pad)

struct TileInfo {
    int e, m0, p0, n;   // tile = positions [p0 + m0, p0 + min(n, m0 + 256)) of expert e
};

// blockIdx.y -> tile; e = -1 past the end.  Experts are walked from the last
// id down so the always-on shared experts (stored last, every token) are
// scheduled first; an expert of n positions has ceil(n / 256) tile rows, and
// every tile row runs as gridDim.x CTAs (one per weight-row block).
//
// Tail split: CTAs start in blockIdx order as CUs free up, one per CU, so the
// last (Ttot * gridDim.x) mod ncu CTAs form a partial final round.  When that
// round's tile rows, cut in two 128-position halves, still fit the CUs, they
// are cut: the final round then runs half-height tiles (same weight work,
// half the activation work) and ends sooner.  The host sizes the grid for the
// extra rows (tail_rows_max).
//
// Wave 0 does it 64 experts at a time: per-expert tile counts, an inclusive
// wave scan, and a ballot for the expert whose tile range holds the row.
__device__ __forceinline__ int tail_split_rows(int ttot, int nx, int ncu) {
    if (ncu <= 0) return 0;
    const int rem = (int)(((int64_t)ttot * nx) % ncu);
    if (rem == 0) return 0;
    const int r = (rem + nx - 1) / nx;
    return 2 * r * nx <= ncu ? r : 0;
}

__device__ __forceinline__ TileInfo find_tile(const MoeRouting& rt, int j, int ncu) {
    __shared__ TileInfo s_tile;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int et = rt.num_experts_total;
        // total tile rows
        int ttot = 0;
        for (int c0 = 0; c0 < et; c0 += 64) {
            const int e = c0 + lane;
            const int n = e < et ? rt.offsets[e + 1] - rt.offsets[e] : 0;
            ttot += __builtin_amdgcn_readlane(wave_scan_incl((n + kBM - 1) / kBM), 63);
        }
        const int split = tail_split_rows(ttot, (int)gridDim.x, ncu);
        const int s0 = ttot - split;   // first split row
        int row = j, half = -1;
        if (j >= s0) {
            row = s0 + (j - s0) / 2;
            half = (j - s0) & 1;
        }
        int base = 0;   // tiles of the experts in earlier chunks
        bool found = false;
        for (int c0 = 0; c0 < et && !found && row < ttot; c0 += 64) {
            const int e = et - 1 - (c0 + lane);
            int p0 = 0, n = 0;
            if (e >= 0) {
                p0 = rt.offsets[e];
                n = rt.offsets[e + 1] - p0;
            }
            const int nt = (n + kBM - 1) / kBM;
            const int incl = wave_scan_incl(nt);
            const int excl = incl - nt;
            const bool hit = e >= 0 && row >= base + excl && row < base + incl;
            if (hit) {
                int m0 = (row - base - excl) * kBM, nn = n;
                if (half >= 0) {
                    m0 += half * (kBM / 2);
                    nn = min(n, m0 + kBM / 2);
                }
                s_tile = m0 < nn ? TileInfo{e, m0, p0, nn} : TileInfo{-1, 0, 0, 0};
            }
            found = __ballot(hit) != 0;
            base += __builtin_amdgcn_readlane(incl, 63);
        }
        if (!found && lane == 0) s_tile = TileInfo{-1, 0, 0, 0};
    }
    __syncthreads();
    return s_tile;
}

// REF: 8 byte codes -> 8 bf16 weights bf16(cb[c] * absmax) (bit-exact dequant).
__device__ __forceinline__ bf16x8_t lookup8_ref(uint32_t w0, uint32_t w1, const float* cb, float am) {
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t word = j < 2 ? w0 : w1;
        const uint32_t c0 = (word >> (16 * (j & 1))) & 0xffu;
        const uint32_t c1 = (word >> (16 * (j & 1) + 8)) & 0xffu;
        o[j] = f32_to_bf16(cb[c0] * am) | (f32_to_bf16(cb[c1] * am) << 16);
    }
    return __builtin_bit_cast(bf16x8_t, make_uint4(o[0], o[1], o[2], o[3]));
}

// One lane's REF B operand for one K step: its two weight rows (n-tiles),
// the 32 columns 32h .. 32h+31 of the 64-column block kb.
struct RefBStep {
    u32x4_t codes[2][2];  // 32 byte codes per row
    float am[2];          // absmax of the row's 128-block holding these columns
    __device__ __forceinline__ void load(const uint8_t* codes_e, const uint16_t* absmax_e, const int (&row)[2],
                                         int K, int kb, int bh, int block_size, int64_t nabs) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int64_t flat = (int64_t)row[nt] * K + kb * kBK + 32 * bh;
            codes[nt][0] = *reinterpret_cast<const u32x4_t*>(codes_e + flat);
            codes[nt][1] = *reinterpret_cast<const u32x4_t*>(codes_e + flat + 16);
            int64_t b = ((int64_t)row[nt] * K + kb * kBK) / block_size;
            b = b < nabs ? b : nabs - 1;
            am[nt] = bf16_to_f32(absmax_e[b]);
        }
    }
};

// One REF tile with register-staged operands (for REF stacks the ring cannot
// address: an odd absmax count per expert, or tables not 4-byte aligned),
// NMT m-tiles of work (a compile-time count, so the K loop is one basic block
// with no per-m-tile branches).
template <bool kGateUp, int NMT>
__device__ __forceinline__ void prefill_tile_ref(const lutmoe_moe_desc& d, const uint16_t* __restrict__ src,
                                             const MoeRouting& rt, void* __restrict__ dst,
                                             const TileInfo ti, uint16_t (*s_a)[kBM * kAStride],
                                             const float* s_cb) {
    const lutmoe_weights& w = kGateUp ? d.w13 : d.w2;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int I = d.inter, H = d.hidden;
    const int K = kGateUp ? H : I;
    const int nkb = K / kBK;
    const int n0 = blockIdx.x * (kGateUp ? kBN / 2 : kBN);   // first intermediate idx / h row
    const int nvalid = min(kBM, ti.n - ti.m0);               // positions in this tile

    // ---- A staging: thread t owns tile row t (64 bf16 = 8 x 16 B per step);
    // rows past the tile's positions repeat its last position (never read).
    const int a_pos = ti.p0 + ti.m0 + min(tid, nvalid - 1);
    const uint16_t* a_src;
    if (kGateUp) a_src = src + (int64_t)(rt.perm[a_pos] / rt.k_eff) * H;
    else a_src = src + (int64_t)a_pos * I;

    // ---- B rows of this lane: n-tiles 0/1
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
    const uint8_t* codes = (const uint8_t*)w.codes + (int64_t)ti.e * w.rows * w.cols;
    const uint16_t* absmax = (const uint16_t*)w.tables + (int64_t)ti.e * w.absmax_per_expert;
    auto load_b = [&](RefBStep& b, int kb) __attribute__((always_inline)) {
        b.load(codes, absmax, b_row, K, kb, bh, w.block_size, w.absmax_per_expert);
    };
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

    auto frag_b = [&](const RefBStep& b, int ks, bf16x8_t (&bf)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
            bf[nt] = lookup8_ref(b.codes[nt][ks >> 1][2 * (ks & 1)], b.codes[nt][ks >> 1][2 * (ks & 1) + 1], s_cb,
                                 b.am[nt]);
    };
    auto frag_a = [&](int buf, int ks, bf16x8_t (&af)[NMT]) __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt)
            af[mt] = *reinterpret_cast<const bf16x8_t*>(&s_a[buf][(mt * 32 + bn) * kAStride + 32 * bh + 8 * ks]);
    };

    // Software pipeline.  Entering step kb: A(kb) in LDS buffer kb&1 (visible
    // after the last barrier), A(kb+1) in flight to registers `ra`, the B
    // operand of step kb in `bcur`, of step kb+1 in flight to `bnext`, and the
    // step-kb fragments of k-substep 0 in bf/af.  Each k-substep computes the
    // next substep's fragments while its MFMAs issue; substep 3 prepares step
    // kb+1's B side.
    RefBStep bcur, bnext;
    load_a(0);
    load_b(bcur, 0);
    store_a(0);
    load_a(min(1, nkb - 1));
    load_b(bnext, min(1, nkb - 1));
    bf16x8_t bf[2], af[NMT];
    frag_b(bcur, 0, bf);
    __syncthreads();
    frag_a(0, 0, af);

    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        // A(kb+1) -> the other buffer (last read in step kb-1, before the
        // previous barrier), then A(kb+2) -> registers.  Past the end these
        // repeat the last step, harmlessly.
        store_a(buf ^ 1);
        load_a(min(kb + 2, nkb - 1));
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            // the next substep's A fragments are read first, a whole substep
            // of MFMAs ahead of their use (the fences keep the scheduler from
            // sinking them next to their MFMAs)
            bf16x8_t bf_n[2], af_n[NMT];
            if (ks < 3) frag_a(buf, ks + 1, af_n);
            __builtin_amdgcn_sched_barrier(0);
            if (ks < 3) frag_b(bcur, ks + 1, bf_n);
            else frag_b(bnext, 0, bf_n);
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bf[nt], acc[mt][nt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            bf[0] = bf_n[0];
            bf[1] = bf_n[1];
            if (ks < 3) {
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt) af[mt] = af_n[mt];
            }
        }
        bcur = bnext;
        load_b(bnext, min(kb + 2, nkb - 1));
        __syncthreads();
        frag_a(buf ^ 1, 0, af);
    }

    // ---- epilogue.  D layout: lane (n = lane%32, h = lane/32), element i ->
    // row m = 8*(i/4) + 4*h + (i%4), column n.  The down projection's rows'
    // routing weights go to LDS first (the A buffers are free once every
    // fragment read is done), so the stores wait on no global load.
    float* s_pw = reinterpret_cast<float*>(&s_a[0][0]);
    if constexpr (!kGateUp) {
        __syncthreads();
        if (tid < nvalid) s_pw[tid] = rt.pair_w[rt.perm[ti.p0 + ti.m0 + tid]];
        __syncthreads();
    }
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = mt * 32 + 8 * (i >> 2) + 4 * bh + (i & 3);
            if (m >= nvalid) continue;
            const int p = ti.p0 + ti.m0 + m;
            if (kGateUp) {
                const int ii = n0 + 32 * wv + bn;
                if (ii < I)
                    ((uint16_t*)dst)[(int64_t)p * I + ii] =
                        (uint16_t)f32_to_bf16(silu_mul(acc[mt][0][i], acc[mt][1][i]));
            } else {
                const float pw = s_pw[m];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const int h = n0 + 64 * wv + 32 * nt + bn;
                    if (h < H) ((float*)dst)[(int64_t)p * H + h] = acc[mt][nt][i] * pw;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// BL4 tiles: operands staged global -> LDS by direct loads (global_load_lds,
// no staging registers) through a ring of 3 stages of one K step each:
//   A      [256 rows] x 128 B             (32 KB; 16-byte chunk c = columns
//          8c..8c+7 of row r stored at chunk c ^ swz(r), so the 32 rows of a
//          fragment read hit distinct LDS banks)
//   codes  [256 rows] x 32 B             ( 8 KB; bytes 16h.. = columns 32h..32h+31)
//   tables [256 rows] x 32 B             ( 8 KB; the rows' bf16[16] tables)
// The activation loads read whole 128-byte lines (8 lanes per row), the weight
// loads each row's 32-byte piece of the K step (2 lanes per row; NestedLUT
// tiers below 4 bits pack their shorter rows densely, see RingLoader).  Only
// the tile's NMT*32 activation rows are loaded.  Every thread issues the same kDma loads per
// stage (NMT + 4 for BL4 and NestedLUT, NMT + 5 for REF), so
// `s_waitcnt vmcnt(kDma)` means "all but the newest stage have landed".  Per step kb: k-substeps 0-2 run from slot kb%3; then a barrier
// (stage kb+1 landed everywhere, slot kb%3 no longer read), the refill of slot
// kb%3 with stage kb+3, and k-substep 3's MFMAs overlapped with reading and
// looking up step kb+1's operands.
constexpr int kSlotA = kBM * kBK * 2;              // 32 KB
constexpr int kSlotB = kBN * 32;                   // 8 KB
constexpr int kStages = 3;
// Tiles of at most 64 positions (BL4 / NestedLUT): their stages are 24 KB
// (64 activation rows), so the same LDS holds 6, and 5 stages are in flight
// while one is read -- a short K step needs that many to cover the latency
// of its loads.
constexpr int kSlotAs = 64 * kBK * 2;              // 8 KB
constexpr int kSlotBytesS = kSlotAs + 2 * kSlotB;  // 24 KB
constexpr int kStagesS = 6;
// A tile's CTA claims its next item (longest first from the launch counter)
// right after the barrier of its second-to-last K step: that barrier waits
// for every ring load and no stage is issued after it, so the atomic is the
// only memory operation in flight (no ring wait counts it), and the CTA that
// frees up first takes the next item
constexpr int kClaimLead = 2;

// A-row chunk swizzle: distinct for any 8 consecutive rows, and (r&1, swz)
// distinct for any 16 consecutive rows.
__device__ __forceinline__ int a_swz(int r) { return ((r >> 1) ^ (r << 2)) & 7; }

// 16 bytes per lane from sbase + voff into LDS at m0 + 16 * lane
// (global_load_lds_dwordx4 with a scalar base, so per-step address updates
// are scalar adds).  Issued as inline asm so the compiler does not track it:
// the ring's explicit vmcnt waits and barriers order it, and no
// compiler-visible global load is in flight between the first of these and
// the final vmcnt(0).  The load reads sbase as an SGPR pair, which needs 5
// wait states after a VALU write of it (or of a dead carry the compiler put
// there just before computing the base with SALU adds); the compiler does not
// insert them in front of inline asm, so the load carries them (s_nop 4:
// DeepSeek T=2048 534.5-544.8 us with it against 534.9-545.3 us without,
// same box; a build that moved the prefill K loop into a lambda had placed
// such a carry write four instructions before a ring load).
__device__ __forceinline__ void dma16(uint32_t voff, const void* sbase, uint32_t m0) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

// Wait until at most `after` ring loads of this thread are in flight (the
// stages issued after the one needed next), and all of its LDS reads are
// done, then barrier.  Memory clobber: no LDS access moves across it.
template <int kAfter>
__device__ __forceinline__ void ring_wait_barrier_n() {
    static_assert(kAfter >= 0 && kAfter <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kAfter) : "memory");
}
// kDma = ring loads per stage per thread (A loads + weight loads)
template <int kDma>
__device__ __forceinline__ void ring_wait_barrier(int stages_after) {
    if (stages_after >= 2) ring_wait_barrier_n<2 * kDma>();
    else if (stages_after == 1) ring_wait_barrier_n<kDma>();
    else ring_wait_barrier_n<0>();
}
// the same for up to 4 stages after the one needed next
template <int kDma>
__device__ __forceinline__ void ring_wait_barrier4(int stages_after) {
    if (stages_after >= 4) ring_wait_barrier_n<4 * kDma>();
    else if (stages_after == 3) ring_wait_barrier_n<3 * kDma>();
    else ring_wait_barrier<kDma>(stages_after);
}

// 4 bytes per lane from sbase + voff into LDS at m0 + 4 * lane.  The load
// reads sbase as an SGPR pair; a VALU write of an SGPR (v_readlane of a
// spilled pointer, v_readfirstlane) needs 5 wait states before a VMEM
// instruction reads it, and the compiler does not insert them in front of
// inline asm: this load carries them itself (s_nop 4), as dma16 does; the
// build's ISA check (block_lut_amd/csrc/isa_check.py) verifies every LDS-DMA
// load of the library.
__device__ __forceinline__ void dma4(uint32_t voff, const void* sbase, uint32_t m0) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const T*)(((uint64_t)hi << 32) | lo);
}

// Ring slot geometry per format: A, then codes, then tables.  REF: codes
// 256 rows x 64 B (one byte per weight) and one absmax dword per row.
template <int kFmt>
struct RingSlot {
    static constexpr int kCodes = kFmt == LUTMOE_FMT_REF ? kBN * 64 : kSlotB;
    static constexpr int kTabs = kFmt == LUTMOE_FMT_REF ? kBN * 4 : kSlotB;
    static constexpr int kBytes = kSlotA + kCodes + kTabs;
    // LDS of a ring kernel: the stages, and REF's fp32 codebook after them
    static constexpr int kLds = kStages * kBytes + (kFmt == LUTMOE_FMT_REF ? 1024 : 0);
};

// REF lookups: 8 byte codes (two dwords, code j in byte j%4 of dword j/4)
// against the fp32[256] codebook at LDS byte address cbase; entries of
// columns 2j / 2j+1 in e[j] / o[j], as lookup8_issue.
__device__ __forceinline__ Lookup8 lookup8_ref_issue(uint32_t w0, uint32_t w1, uint32_t cbase) {
    Lookup8 r;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t w = d ? w1 : w0;
        const uint32_t we = (w << 2) & 0x03fc03fcu;   // 4 * codes 0, 2 (16-bit fields)
        const uint32_t wo = (w >> 6) & 0x03fc03fcu;   // 4 * codes 1, 3
        r.e[2 * d] = lds_ld32(add_word<0>(cbase, we));
        r.e[2 * d + 1] = lds_ld32(add_word<1>(cbase, we));
        r.o[2 * d] = lds_ld32(add_word<0>(cbase, wo));
        r.o[2 * d + 1] = lds_ld32(add_word<1>(cbase, wo));
    }
    return r;
}

// bf16(cb[c] * absmax) for the 8 looked-up entries: the product of two bf16
// values is exact in fp32; v_cvt_pk_bf16_f32 rounds to nearest even (as the
// reference's dequantisation; finite values and infinities round alike).
__device__ __forceinline__ u32x4_t lookup8_ref_combine(const Lookup8& l, float am) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f32x2_t p = {__uint_as_float(l.e[j]) * am, __uint_as_float(l.o[j]) * am};
        r[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2_t));
    }
    return r;
}

// ---------------------------------------------------------------------------
// Persistent ring kernel: one CTA per CU takes tile items -- a tile row
// (up to 256 positions of one expert) times one weight-row block x, times
// one K split z -- from a counter shared by the launch, heaviest first, so
// the CTA that finishes early takes the next item (greedy longest-first).
// Every wave finds its items itself from LDS copies of the expert offsets
// and tier widths (no barrier).  When a tile's K loop ends the ring is free:
// the next tile's first stages are issued at once and land while this
// tile's epilogue stores its results straight from the accumulators (no LDS
// staging).
struct RingTile {
    int e, m0, p0, n;   // positions [p0 + m0, p0 + min(n, m0 + 256)) of expert e; e < 0: none
    int x, z;           // weight-row block, K split
};

__device__ __forceinline__ int ring_nmt(const RingTile& t) { return (min(kBM, t.n - t.m0) + 31) / 32; }

// A tile is the same in every lane; this says so to the compiler (whose
// divergence analysis does not follow the wave-wide searches that found it),
// so that the addresses derived from it stay scalar.
__device__ __forceinline__ RingTile uniform_tile(const RingTile& t) {
    return RingTile{__builtin_amdgcn_readfirstlane(t.e), __builtin_amdgcn_readfirstlane(t.m0),
                    __builtin_amdgcn_readfirstlane(t.p0), __builtin_amdgcn_readfirstlane(t.n),
                    __builtin_amdgcn_readfirstlane(t.x), __builtin_amdgcn_readfirstlane(t.z)};
}

// Tile classes in hand-out order: estimated cost descending.  A class is
// (m-tiles, tier bits); a tile's time grows by about as much per m-tile as
// per code bit (NestedLUT tiers), so the 24 NestedLUT classes are ordered by
// m-tiles + bits, then m-tiles; the formats of one code width use the 8
// classes m-tiles = 8 .. 1.
constexpr int kMaxClasses = 24;

__device__ __forceinline__ int tile_class(bool nested, int nmt, int bits) {
    if (!nested) return 8 - nmt;
    const int est = nmt + bits;   // 3 .. 12
    // the classes of every larger estimate come first
    int start = 0;
    for (int v = 12; v > est; --v) start += min(8, v - 2) - max(1, v - 4) + 1;
    return start + (min(8, est - 2) - nmt);
}
__device__ __forceinline__ void class_params(bool nested, int c, int& nmt, int& bits) {
    if (!nested) {
        nmt = 8 - c;
        bits = 0;
        return;
    }
    for (int v = 12; v >= 3; --v) {
        const int hi = min(8, v - 2), lo = max(1, v - 4), k = hi - lo + 1;
        if (c < k) {
            nmt = hi - c;
            bits = v - nmt;
            return;
        }
        c -= k;
    }
    nmt = 1;
    bits = 2;
}

// Tiles of expert e (n positions) in class (cn, cb): its whole 256-position
// tiles and its last tile of fewer positions each fall in the class of
// their m-tiles and the expert's tier.
__device__ __forceinline__ int class_tiles(int n, int bits_e, bool nested, int cn, int cb) {
    if (nested && bits_e != cb) return 0;
    const int full = n >> 8, rn = ((n & (kBM - 1)) + 31) >> 5;
    return cn == 8 ? full + (rn == 8 ? 1 : 0) : (rn == cn ? 1 : 0);
}

// The items of one launch: tile rows in class order, the last `split` of
// them (the lightest) cut into two 128-position halves when they hold more
// than 128 positions; nsub sub-rows x nx weight-row blocks x ns K splits.
// Per class c (LDS, written once per CTA by wave 0): its first sub-row
// sub0[c], its sub-rows nsubc[c], its whole rows before the split whole[c],
// and (m-tiles | bits << 8) prm[c].
struct ClassTable {
    int sub0[kMaxClasses], nsubc[kMaxClasses], whole[kMaxClasses], prm[kMaxClasses];
    int nsub;
};

__device__ __forceinline__ void class_table(ClassTable& t, const int* cls, bool nested, int nx, int ncu) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const int nc = nested ? kMaxClasses : 8;
    int cn = 1, cb = 0, cnt = 0;
    if (lane < nc) {
        class_params(nested, lane, cn, cb);
        cnt = cls[lane];
    }
    const int r_incl = wave_scan_incl(cnt);
    const int ttot = __builtin_amdgcn_readlane(r_incl, 63);
    const int s0 = ttot - tail_split_rows(ttot, nx, ncu);
    const int a = min(max(s0 - (r_incl - cnt), 0), cnt);   // whole rows of the class
    const int w = a + (cnt - a) * (cn > 4 ? 2 : 1);
    const int w_incl = wave_scan_incl(w);
    if (lane < nc) {
        t.sub0[lane] = w_incl - w;
        t.nsubc[lane] = w;
        t.whole[lane] = a;
        t.prm[lane] = cn | (cb << 8);
    }
    if (lane == 0) t.nsub = __builtin_amdgcn_readlane(w_incl, 63);
}

struct ItemMap {
    const int* off;        // expert offsets (LDS, or global past kOffLds - 1 experts)
    const int8_t* bits;    // NestedLUT tier of each expert (LDS, or global)
    const ClassTable* ct;  // (LDS)
    int et, nc, nsub, nx, ns, nitems;
    bool nested;
};

__device__ __forceinline__ ItemMap item_map(const int* off, const int8_t* bits, const ClassTable* ct, int et,
                                            bool nested, int nx, int ns) {
    ItemMap m;
    m.off = off;
    m.bits = bits;
    m.ct = ct;
    m.et = et;
    m.nested = nested;
    m.nc = nested ? kMaxClasses : 8;
    m.nx = nx;
    m.ns = ns;
    m.nsub = __builtin_amdgcn_readfirstlane(ct->nsub);
    m.nitems = m.nsub * nx * ns;
    return m;
}

// Item -> tile, by the calling wave alone (uniform result); e < 0 past the end.
__device__ __forceinline__ RingTile map_item(const ItemMap& m, int item) {
    RingTile t{-1, 0, 0, 0, 0, 0};
    if (item >= m.nitems) return t;
    t.x = item % m.nx;
    int u = item / m.nx;
    t.z = u / m.nsub;
    u -= t.z * m.nsub;
    const int lane = threadIdx.x & 63;
    // the class holding sub-row u: lane c checks class c
    int sub0 = 0, nsc = 0;
    if (lane < m.nc) {
        sub0 = m.ct->sub0[lane];
        nsc = m.ct->nsubc[lane];
    }
    const uint64_t chit = __ballot(lane < m.nc && u >= sub0 && u < sub0 + nsc);
    if (!chit) return t;
    const int c = (int)__builtin_ctzll(chit);
    const int uu = u - __builtin_amdgcn_readlane(sub0, c);
    const int a = __builtin_amdgcn_readfirstlane(m.ct->whole[c]);
    const int prm = __builtin_amdgcn_readfirstlane(m.ct->prm[c]);
    const int cn = prm & 0xff, cb = prm >> 8;
    const int sp = cn > 4 ? 2 : 1;
    int r = uu, half = -1;
    if (uu >= a) {
        r = a + (uu - a) / sp;
        if (sp == 2) half = (uu - a) & 1;
    }
    // the r-th tile of the class, experts from the last id down
    int base = 0;
    for (int c0 = 0; c0 < m.et; c0 += 64) {
        const int e = m.et - 1 - (c0 + lane);
        int p0 = 0, n = 0, k = 0;
        if (e >= 0) {
            p0 = m.off[e];
            n = m.off[e + 1] - p0;
            k = class_tiles(n, m.nested ? m.bits[e] : 0, m.nested, cn, cb);
        }
        const int incl = wave_scan_incl(k);
        const int excl = incl - k;
        const uint64_t hit = __ballot(k > 0 && r >= base + excl && r < base + incl);
        if (hit) {
            const int src = (int)__builtin_ctzll(hit);
            const int q = r - base - excl;
            int m0 = cn == 8 ? q * kBM : (n >> 8) * kBM;
            int nn = cn == 8 ? min(n, m0 + kBM) : n;
            if (half >= 0) {
                m0 += half * (kBM / 2);
                nn = min(nn, m0 + kBM / 2);
            }
            t.e = __builtin_amdgcn_readlane(e, src);
            t.m0 = __builtin_amdgcn_readlane(m0, src);
            t.p0 = __builtin_amdgcn_readlane(p0, src);
            t.n = __builtin_amdgcn_readlane(nn, src);
            return t;
        }
        base += __builtin_amdgcn_readlane(incl, 63);
    }
    return t;
}

// K steps [kb0, kb0 + nkb) of a tile: all of K, or split z of ns (down
// projection only; partial results go to separate y buffers).
__device__ __forceinline__ void ring_k_range(int K, int z, int ns, int& kb0, int& nkb) {
    kb0 = (K / kBK) * z / ns;
    nkb = (K / kBK) * (z + 1) / ns - kb0;
}

// Loader side of one tile (all offsets 32-bit, from scalar bases; the host
// checks the sizes).  The tile's first nmt*32 activation rows are loaded:
// load j of wave w covers rows 8*nmt*w + 8j .. +7, lane l reads the
// (l%8 ^ swz)-th 16 bytes of row 8*nmt*w + 8j + l/8.  Rows past the tile's
// positions repeat its last position (never read back).
//
// BL4 codes / tables: load h of wave w covers tile rows 64w+32h .. +31, two
// lanes per row (16 B each), so a row's 32 bytes land contiguous in LDS.
// NestedLUT tier b: a row's K step is 8b code bytes (its two 32-weight
// groups) and 2^(b+1) table bytes, both contiguous in HBM:
//   codes  b=4: as BL4 (LDS row stride 32, groups at 0 and 16); b=3: as
//          BL4 with the second lane reading bytes 8..23, so the groups land
//          at 0 and 20 of the 32-byte LDS row and nothing past the row's
//          bytes is read; b=2: load 0 covers rows 64w .. +63, one lane
//          (16 B) per row (LDS row stride 16), load 1 repeats it
//   tables b=4: as BL4; b=3: load 0 covers rows 64w .. +63, one lane (16 B)
//          per row, load 1 repeats it; b=2: as BL4 with 4-byte loads (LDS
//          row stride 2^(b+1))
// so every tier issues four weight loads per stage.  REF: codes 256 rows x
// 64 B (load h of wave w covers tile rows 64w+16h .. +15, four lanes per
// row) and one absmax dword per row (lane l of wave w fetches the aligned
// dword holding row 64w+l's entry for the step).
template <bool kGateUp, int kFmt>
struct RingLoader {
    static constexpr bool kNested = kFmt == LUTMOE_FMT_NESTED;
    static constexpr bool kRef = kFmt == LUTMOE_FMT_REF;
    static constexpr int kCodesB = RingSlot<kFmt>::kCodes;
    const uint8_t* a_base;
    const uint8_t* c_base;
    const uint8_t* t_base;
    uint32_t a_off[8];
    uint32_t w_off[kRef || kNested ? 4 : 2];
    uint32_t c_step, t_step;
    uint32_t q, nb, am_row64;   // REF: absmax block of step kb of row r = min((r*K/64 + kb) / q, nb - 1)
    int bits, wvu, nmt;

    __device__ __forceinline__ void init(const lutmoe_moe_desc& d, const uint16_t* src, const MoeRouting& rt,
                                         const RingTile& ti, int nmt_) {
        int tid;
        asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
        const int lane = tid & 63, wv = tid >> 6;
        const int I = d.inter, H = d.hidden;
        const int K = kGateUp ? H : I;
        const int n0 = ti.x * (kGateUp ? kBN / 2 : kBN);
        const int nvalid = min(kBM, ti.n - ti.m0);
        const lutmoe_weights& ww = kGateUp ? d.w13 : d.w2;
        nmt = nmt_;
        wvu = __builtin_amdgcn_readfirstlane(wv);
        a_base = (const uint8_t*)src;
        // (gate/up: every row's pair index is loaded, also past nmt, and all
        // loads are issued before the first use, so that they overlap)
        int pr[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = 8 * nmt * wv + 8 * j + (lane >> 3);
            pr[j] = ti.p0 + ti.m0 + min(r, nvalid - 1);
            if constexpr (kGateUp) pr[j] = rt.perm[pr[j]];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = 8 * nmt * wv + 8 * j + (lane >> 3);
            const uint32_t row =
                kGateUp ? (uint32_t)(pr[j] / rt.k_eff) * (uint32_t)H : (uint32_t)pr[j] * (uint32_t)I;
            a_off[j] = 2u * (row + 8u * (uint32_t)((lane & 7) ^ a_swz(r)));
        }
        // weight row of tile row tr (gate/up: rows 0..127 gate, 128..255 up)
        auto tile_row = [&](int tr) __attribute__((always_inline)) {
            if (kGateUp) {
                const int i = min(n0 + (tr & 127), I - 1);
                return tr < 128 ? i : I + i;
            }
            return min(n0 + tr, H - 1);
        };
        c_step = 32;
        t_step = 32;
        bits = 4;
        q = kRef ? (uint32_t)(ww.block_size / 64) : 1u;
        nb = kRef ? (uint32_t)ww.absmax_per_expert : 1u;
        am_row64 = 0;
        if constexpr (kRef) {
            c_base = uniform_ptr((const uint8_t*)ww.codes + (int64_t)ti.e * ww.rows * ww.cols);
            t_base = uniform_ptr((const uint8_t*)((const uint16_t*)ww.tables + (int64_t)ti.e * ww.absmax_per_expert));
#pragma unroll
            for (int h = 0; h < 4; ++h)
                w_off[h] = (uint32_t)tile_row(64 * wv + 16 * h + (lane >> 2)) * (uint32_t)K + 16u * (uint32_t)(lane & 3);
            am_row64 = (uint32_t)tile_row(64 * wv + lane) * (uint32_t)(K / 64);
        } else if constexpr (kNested) {
            c_base = uniform_ptr(((const uint8_t* const*)ww.codes)[ti.e]);
            t_base = uniform_ptr((const uint8_t*)((const uint16_t* const*)ww.tables)[ti.e]);
            bits = __builtin_amdgcn_readfirstlane((int)ww.tier_bits[ti.e]);
            c_step = 8u * (uint32_t)bits;     // code bytes of a row's K step
            t_step = 2u << bits;              // table bytes of a row's K step
            const uint32_t kq = (uint32_t)(K / 64);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t pr = (uint32_t)tile_row(64 * wv + 32 * h + (lane >> 1)) * kq;   // lane pairs
                const uint32_t sr = (uint32_t)tile_row(64 * wv + lane) * kq;                   // one lane per row
                w_off[h] = bits == 2 ? sr * 16u : pr * c_step + (uint32_t)(lane & 1) * (bits == 4 ? 16u : 8u);
                w_off[2 + h] = bits == 3 ? sr * 16u : pr * t_step + (uint32_t)(lane & 1) * (t_step / 2u);
            }
        } else {
            const int64_t per = (int64_t)ww.rows * (ww.cols / 2);
            c_base = uniform_ptr((const uint8_t*)ww.codes + ti.e * per);
            t_base = uniform_ptr((const uint8_t*)ww.tables + ti.e * per);
#pragma unroll
            for (int h = 0; h < 2; ++h)
                w_off[h] = (uint32_t)tile_row(64 * wv + 32 * h + (lane >> 1)) * (uint32_t)(K / 2) +
                           16u * (uint32_t)(lane & 1);
        }
    }

    // the weight loads of step kb into the slot at LDS address l0 (SA: the
    // slot's activation bytes, the weights after them)
    template <int SA>
    __device__ __forceinline__ void issue_w(int kb, uint32_t l0) const {
        if constexpr (kRef) {
            const uint8_t* cb = c_base + kb * 64;
#pragma unroll
            for (int h = 0; h < 4; ++h) dma16(w_off[h], cb, l0 + SA + (64 * wvu + 16 * h) * 64);
            const uint32_t idx = min((am_row64 + (uint32_t)kb) / q, nb - 1u);
            dma4((idx & ~1u) * 2u, t_base, l0 + SA + kCodesB + 256 * wvu);
        } else if constexpr (kNested) {
            const uint32_t cs = (uint32_t)kb * c_step, ts = (uint32_t)kb * t_step;
            const uint32_t tl = l0 + SA + kCodesB + (uint32_t)wvu * 64u * t_step;
            if (bits == 4) {
                const uint32_t cl = l0 + SA + (uint32_t)wvu * 2048u;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    dma16(w_off[h] + cs, c_base, cl + h * 1024);
                    dma16(w_off[2 + h] + ts, t_base, tl + h * 1024);
                }
            } else if (bits == 3) {
                const uint32_t cl = l0 + SA + (uint32_t)wvu * 2048u;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    dma16(w_off[h] + cs, c_base, cl + h * 1024);
                    dma16(w_off[2 + h] + ts, t_base, tl);
                }
            } else {
                const uint32_t cl = l0 + SA + (uint32_t)wvu * 1024u;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    dma16(w_off[h] + cs, c_base, cl);
                    dma4(w_off[2 + h] + ts, t_base, tl + h * 256);
                }
            }
        } else {
            const uint8_t* cb = c_base + kb * 32;
            const uint8_t* tbp = t_base + kb * 32;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                dma16(w_off[h], cb, l0 + SA + wvu * 2048 + h * 1024);
                dma16(w_off[h], tbp, l0 + SA + kCodesB + wvu * 2048 + h * 1024);
            }
        }
    }
    // stage kb into slot sl, NMT activation loads (NMT == nmt)
    template <int NMT, int SA = kSlotA>
    __device__ __forceinline__ void issue(int kb, const uint8_t* sl) const {
        const uint32_t l0 = lds_addr(sl);
        const uint8_t* ab = a_base + kb * (kBK * 2);
#pragma unroll
        for (int j = 0; j < NMT; ++j) dma16(a_off[j], ab, l0 + (8 * NMT * wvu + 8 * j) * 128);
        issue_w<SA>(kb, l0);
    }
    // the same with the tile's activation-load count known at run time
    template <int SA = kSlotA>
    __device__ __forceinline__ void issue_rt(int kb, const uint8_t* sl) const {
        const uint32_t l0 = lds_addr(sl);
        const uint8_t* ab = a_base + kb * (kBK * 2);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < nmt) dma16(a_off[j], ab, l0 + (8 * nmt * wvu + 8 * j) * 128);
        issue_w<SA>(kb, l0);
    }
};

// A tile's first stages into the ring (and REF's fp32 codebook after them);
// the ring and the codebook must no longer be read.
template <bool kGateUp, int kFmt>
__device__ __forceinline__ void ring_prologue(const lutmoe_moe_desc& d, const uint16_t* src, const MoeRouting& rt,
                                              const RingTile& t, int ns, uint8_t* ring) {
    // REF: the expert's codebook entry of this thread, loaded beside the
    // activation row indices (the compiler's wait for them then covers no
    // ring load)
    float cbv = 0.f;
    if constexpr (kFmt == LUTMOE_FMT_REF) cbv = bf16_to_f32(ref_codebook(kGateUp ? d.w13 : d.w2, t.e)[threadIdx.x]);
    RingLoader<kGateUp, kFmt> L;
    L.init(d, src, rt, t, ring_nmt(t));
    if constexpr (kFmt == LUTMOE_FMT_REF)
        reinterpret_cast<float*>(ring + kStages * RingSlot<kFmt>::kBytes)[threadIdx.x] = cbv;
    int kb0, nkb;
    ring_k_range(kGateUp ? d.hidden : d.inter, t.z, ns, kb0, nkb);
    if (kFmt != LUTMOE_FMT_REF && ring_nmt(t) <= 2) {
        // the small-tile ring geometry
        for (int st = 0; st < min(kStagesS, nkb); ++st)
            L.template issue_rt<kSlotAs>(kb0 + st, ring + st * kSlotBytesS);
    } else {
        for (int st = 0; st < min(kStages, nkb); ++st) L.issue_rt(kb0 + st, ring + st * RingSlot<kFmt>::kBytes);
    }
}

// One tile whose first stages are in the ring (issued by ring_prologue).
// Thread 0 claims the next item from the launch's counter after the barrier
// of the second-to-last K step (kClaimLead; the returned index is published
// through s_claim in the last K step), so that the items go out longest
// first to whichever CTA frees up first; on return `next` is that item's
// tile and its first stages are issued (when there is one).
template <bool kGateUp, int kFmt, int NMT, typename NextFn>
__device__ __forceinline__ void ring_tile_body(const lutmoe_moe_desc& d, const uint16_t* __restrict__ src,
                                               const MoeRouting& rt, void* __restrict__ dst, const RingTile& ti,
                                               NextFn next_of, RingTile& next, int* ctr, int* s_claim,
                                               uint8_t* ring, float* s_pw, int ns, int64_t split_stride) {
    constexpr bool kNested = kFmt == LUTMOE_FMT_NESTED;
    constexpr bool kRef = kFmt == LUTMOE_FMT_REF;
    constexpr int kCodesB = RingSlot<kFmt>::kCodes, kSlot = RingSlot<kFmt>::kBytes;
    constexpr int kNC = kRef ? 4 : 2;   // code registers (u32x4) per lane per K step
    // ring loads per thread per stage: the tile's NMT activation loads (only
    // its NMT*32 rows are loaded) and the weight loads
    constexpr int kDma = NMT + (kRef ? 5 : 4);
    // the lane index through an opaque move, so that nothing derived from it
    // is hoisted out of the persistent loop (and kept live across K loops)
    int tid;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
    const int lane = tid & 63, wv = tid >> 6;
    const int I = d.inter, H = d.hidden;
    const int K = kGateUp ? H : I;
    int kb0, nkb;
    ring_k_range(K, ti.z, ns, kb0, nkb);
    const int n0 = ti.x * (kGateUp ? kBN / 2 : kBN);
    const int nvalid = min(kBM, ti.n - ti.m0);

    // every stage issued so far landed (the previous tile's epilogue stores
    // are done too), the REF codebook is written
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    int claim = 0;
    const int kc = max(0, nkb - kClaimLead);   // the K step that claims the next item
    RingLoader<kGateUp, kFmt> L;
    L.init(d, src, rt, ti, NMT);
    // down projection: tile row tid's routing weight, by its pair index
    // (loaded now) in K step 0 (when that index is back), so that the K loop
    // hides both loads
    int pair = 0;
    float pw_row = 0.f;
    if constexpr (!kGateUp) {
        if (tid < nvalid) pair = rt.perm[ti.p0 + ti.m0 + tid];
    }

    // ---- compute side: lane (n = lane%32, h = lane/32), n-tiles 0/1
    const int bn = lane & 31, bh = lane >> 5;
    const int L0 = kGateUp ? 32 * wv + bn : 64 * wv + bn;
    const int L1 = kGateUp ? 128 + 32 * wv + bn : 64 * wv + 32 + bn;
    const int bits = L.bits;
    const uint32_t t_step = L.t_step;
    const uint32_t q = L.q, nb = L.nb;
    auto tile_row = [&](int tr) __attribute__((always_inline)) {
        if (kGateUp) {
            const int i = min(n0 + (tr & 127), I - 1);
            return tr < 128 ? i : I + i;
        }
        return min(n0 + tr, H - 1);
    };

    // BL4: codes[nt] = the lane's 16 code bytes of row Lnt.  NestedLUT:
    // codes[nt] = the lane half's 32-weight group: its 2-bit field words (.x,
    // .y), bit-2 and bit-3 words (.z, .w; zero for tiers without them): see
    // nested_code below.
    // REF: codes[2nt], codes[2nt+1] = the lane's 32 code bytes of row Lnt; am[nt]
    // = that row's absmax for K step kb (the aligned dword holds it in the
    // half its index parity selects)
    uint32_t row64[2] = {0u, 0u};
    // NestedLUT: LDS offsets of the lane half's code group and of the rows'
    // tables within the slot's code / table regions
    uint32_t c_grp[2] = {0u, 0u}, t_row[2] = {(uint32_t)L0 * 32u, (uint32_t)L1 * 32u};
    if constexpr (kNested) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const uint32_t Lr = (uint32_t)(nt ? L1 : L0);
            c_grp[nt] = bits == 2 ? Lr * 16u + (uint32_t)bh * 8u : Lr * 32u + (uint32_t)bh * (bits == 4 ? 16u : 20u);
            t_row[nt] = Lr * t_step;
        }
    }
    if constexpr (kRef) {
        row64[0] = (uint32_t)tile_row(L0) * (uint32_t)(K / 64);
        row64[1] = (uint32_t)tile_row(L1) * (uint32_t)(K / 64);
    }
    auto read_am = [&](const uint8_t* sl, int kb, float (&am)[2]) __attribute__((always_inline)) {
        if constexpr (kRef) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t idx = min((row64[nt] + (uint32_t)kb) / q, nb - 1u);
                const uint32_t wd = *reinterpret_cast<const uint32_t*>(sl + kSlotA + kCodesB + 4 * (nt ? L1 : L0));
                am[nt] = bf16_to_f32((wd >> (16 * (idx & 1u))) & 0xffffu);
            }
        }
    };
    auto read_codes = [&](const uint8_t* sl, u32x4_t (&codes)[kNC]) __attribute__((always_inline)) {
        if constexpr (kRef) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint8_t* rb = sl + kSlotA + (nt ? L1 : L0) * 64 + 32 * bh;
                codes[2 * nt] = *reinterpret_cast<const u32x4_t*>(rb);
                codes[2 * nt + 1] = *reinterpret_cast<const u32x4_t*>(rb + 16);
            }
        } else if constexpr (kNested) {
            // dword reads (a tier-3 group is only 4-byte aligned); the words
            // past the tier's group are other bytes and are dropped
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t* g = reinterpret_cast<const uint32_t*>(sl + kSlotA + c_grp[nt]);
                codes[nt] = u32x4_t{g[0], g[1], bits >= 3 ? g[2] : 0u, bits >= 4 ? g[3] : 0u};
            }
        } else {
            const uint8_t* cb = sl + kSlotA + bh * 16;
            codes[0] = *reinterpret_cast<const u32x4_t*>(cb + L0 * 32);
            codes[1] = *reinterpret_cast<const u32x4_t*>(cb + L1 * 32);
        }
    };
    // the 8 codes of k-substep ks (columns 32bh + 8ks .. +7 of the block) as
    // BL4 nibbles
    auto nested_code = [&](const u32x4_t& c, int ks) __attribute__((always_inline)) {
        if constexpr (kNested)
            return nested_code8(c[0], c[1], c[2], c[3], ks);
        else
            return c[ks];
    };
    // the same for a tier known at compile time (Bt: 2, 3 or 4): the words
    // the tier does not have are not read
    auto nested_code_b = [&](auto Bt, const u32x4_t& c, int ks) __attribute__((always_inline)) {
        if constexpr (kNested)
            return nested_code8<decltype(Bt)::value>(c[0], c[1], c[2], c[3], ks);
        else
            return c[ks];
    };
    const int sw = a_swz(bn);   // = a_swz(mt * 32 + bn) for every m-tile
    // A fragments of m-tiles [mt0, mt1) of k-substep ks
    auto frag_a = [&](const uint8_t* sl, int ks, bf16x8_t (&af)[NMT], int mt0, int mt1) __attribute__((always_inline)) {
        const uint8_t* p = sl + bn * 128 + 16 * ((4 * bh + ks) ^ sw);
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt)
            if (mt >= mt0 && mt < mt1) af[mt] = *reinterpret_cast<const bf16x8_t*>(p + mt * 4096);
    };
    // B lookups of n-tile nt, k-substep ks (reads issued here, combined later)
    auto frag_b = [&](const uint8_t* sl, const u32x4_t (&codes)[kNC], int ks, int nt) __attribute__((always_inline)) {
        if constexpr (kRef) {
            // the 8 codes (bytes 8ks .. of the lane's 32) looked up in the fp32 codebook
            const u32x4_t& c = codes[2 * nt + (ks >> 1)];
            return lookup8_ref_issue(c[2 * (ks & 1)], c[2 * (ks & 1) + 1], lds_addr(ring + kStages * kSlot));
        } else {
            const uint32_t tbase = lds_addr(sl + kSlotA + kCodesB);
            return lookup8_issue(nested_code(codes[nt], ks), tbase + t_row[nt]);
        }
    };
    // looked-up entries -> bf16x8 B fragment (REF: times the row's absmax,
    // rounded to bf16: the reference's dequantised weight)
    auto combine = [&](const Lookup8& lk, float am) __attribute__((always_inline)) {
        if constexpr (kRef) return __builtin_bit_cast(bf16x8_t, lookup8_ref_combine(lk, am));
        else return __builtin_bit_cast(bf16x8_t, lookup8_combine(lk));
    };

    // One MFMA of activation fragment a and weight fragment w.  Gate/up puts
    // the weights in the A operand, so that its accumulators hold output
    // columns of one position (see the epilogue); down keeps the activations
    // in A, so that a store writes whole 128-byte rows of fp32 output.
    auto mma = [&](const bf16x8_t& a, const bf16x8_t& w, const f32x16_t& c) __attribute__((always_inline)) {
        if constexpr (kGateUp) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(w, a, c, 0, 0, 0);
        else return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, w, c, 0, 0, 0);
    };
    f32x16_t acc[NMT][2];
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][nt][i] = 0.f;

    // Tiles of at most 64 positions (BL4 / NestedLUT): the table lookups,
    // not the MFMAs, set the pace, and the LDS serves the random 16-bit
    // lookups into 32 rows' tables with bank conflicts.  Here each lane
    // loads its two rows' tables once per K step and looks its codes up in
    // registers (v_perm_b32 over byte planes).  A step's operand reads are
    // issued one step ahead of its MFMAs (two register sets), right after
    // the barrier that lands their stage.
    auto regtab_loop = [&](auto BC) __attribute__((always_inline)) {
        constexpr int B = decltype(BC)::value;
        constexpr int ND = (1 << B) / 2;    // table dwords per row
        constexpr int NP = (1 << B) / 4;    // plane dwords
        u32x4_t cds[2][kNC];
        uint32_t tab[2][2][ND];
        bf16x8_t afs[2][4][NMT];
        auto issue_step = [&](const uint8_t* sl, auto Bf) __attribute__((always_inline)) {
            constexpr int b = decltype(Bf)::value;
            read_codes(sl + (kSlotAs - kSlotA), cds[b]);   // (read_codes adds kSlotA)
            const uint8_t* tb = sl + kSlotAs + kCodesB;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t* tp = reinterpret_cast<const uint32_t*>(tb + t_row[nt]);
                if constexpr (ND >= 4) {
#pragma unroll
                    for (int q = 0; q < ND; q += 4) {
                        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(tp + q);
                        tab[b][nt][q] = v[0];
                        tab[b][nt][q + 1] = v[1];
                        tab[b][nt][q + 2] = v[2];
                        tab[b][nt][q + 3] = v[3];
                    }
                } else {
                    tab[b][nt][0] = tp[0];
                    tab[b][nt][1] = tp[1];
                }
            }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) frag_a(sl, ks, afs[b][ks], 0, NMT);
        };
        int slot = 0;
        auto step = [&](int kb, auto Bf) __attribute__((always_inline)) {
            constexpr int b = decltype(Bf)::value;
            uint8_t* sl = ring + slot * kSlotBytesS;
            const int nslot = slot == kStagesS - 1 ? 0 : slot + 1;
            // step kb's reads are done (this wait also tells the compiler),
            // stage kb+1 landed everywhere (stages kb+2 .. kb+5 may still be
            // in flight) and slot kb%6 is no longer read -> refill it with
            // stage kb+6, issue step kb+1's reads, then step kb's lookups and
            // MFMAs from registers
            __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
            ring_wait_barrier4<kDma>(min(4, nkb - 2 - kb));
            if (ctr && kb == kc && threadIdx.x == 0) claim = atomicAdd(ctr, 1);
            if constexpr (!kGateUp) {
                if (kb == 0 && tid < nvalid) pw_row = rt.pair_w[pair];
            }
            if (kb == nkb - 1 && threadIdx.x == 0) *s_claim = claim;
            if (kb + kStagesS < nkb) L.template issue<NMT, kSlotAs>(kb0 + kb + kStagesS, sl);
            if (kb + 1 < nkb) issue_step(ring + nslot * kSlotBytesS, std::integral_constant<int, 1 - b>{});
            uint32_t lo[2][NP], hi[2][NP];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) table_planes<B>(tab[b][nt], lo[nt], hi[nt]);
            // one m-tile: its activation fragment put in regtab_lookup8_eo's
            // order (4 v_perm) spares the two B fragments' last 4 v_perm each
            // (Mixtral B=64 398 -> 391 us, NestedLUT tier prefill 270 -> 266 us)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                if constexpr (NMT == 1) {
                    const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, eo_order(__builtin_bit_cast(u32x4_t, afs[b][ks][0])));
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        const bf16x8_t bfr = __builtin_bit_cast(
                            bf16x8_t, regtab_lookup8_eo<B>(lo[nt], hi[nt], nested_code_b(BC, cds[b][nt], ks)));
                        acc[0][nt] = mma(a0, bfr, acc[0][nt]);
                    }
                } else {
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        const bf16x8_t bfr = __builtin_bit_cast(
                            bf16x8_t, regtab_lookup8<B>(lo[nt], hi[nt], nested_code_b(BC, cds[b][nt], ks)));
#pragma unroll
                        for (int mt = 0; mt < NMT; ++mt)
                            acc[mt][nt] = mma(afs[b][ks][mt], bfr, acc[mt][nt]);
                    }
                }
            }
            slot = nslot;
        };
        issue_step(ring, std::integral_constant<int, 0>{});
        int kb = 0;
        for (; kb + 1 < nkb; kb += 2) {
            step(kb, std::integral_constant<int, 0>{});
            step(kb + 1, std::integral_constant<int, 1>{});
        }
        if (kb < nkb) step(kb, std::integral_constant<int, 0>{});
    };
    if constexpr (NMT <= 2 && !kRef) {
        if (!kNested || bits == 4) regtab_loop(std::integral_constant<int, 4>{});
        else if (bits == 3) regtab_loop(std::integral_constant<int, 3>{});
        else regtab_loop(std::integral_constant<int, 2>{});
    } else {
    // k-substep 0's fragment reads (every stage in the ring landed)
    u32x4_t codes[kNC];
    float am[2] = {0.f, 0.f};
    bf16x8_t bf[2], af[NMT];
    read_codes(ring, codes);
    read_am(ring, kb0, am);
    Lookup8 lk0 = frag_b(ring, codes, 0, 0), lk1 = frag_b(ring, codes, 0, 1);
    frag_a(ring, 0, af, 0, NMT);

    // Software pipeline, per k-substep and n-tile nt: combine the n-tile's
    // looked-up entries (issued one half-substep earlier) into its B
    // fragment, then its NMT MFMAs interleaved with the next substep's LDS
    // reads: that substep's n-tile-nt lookups and half of its A fragments,
    // one or two reads per MFMA, so the LDS queue drains while the MFMAs
    // run and every read has a half-substep of MFMAs to land.  Per step kb:
    // k-substeps 0-2 run from slot kb%3; then a barrier (stage kb+1 landed
    // everywhere, slot kb%3 no longer read), the refill of slot kb%3 with
    // stage kb+3, and k-substep 3's MFMAs overlapped with reading and looking
    // up step kb+1's operands.
    constexpr int kHalfA = (NMT + 1) / 2;
    int slot = 0;
    for (int kb = 0; kb < nkb; ++kb) {
        uint8_t* sl = ring + slot * kSlot;
        const int nslot = slot == kStages - 1 ? 0 : slot + 1;
        const uint8_t* nsl = ring + nslot * kSlot;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8_t af_n[NMT];
            u32x4_t codes_n[kNC];
            float am_n[2] = {0.f, 0.f};
            const uint8_t* rs = ks < 3 ? sl : nsl;      // slot of the next substep's operands
            const int ksn = (ks + 1) & 3;
            // ---- n-tile 0
            bf[0] = combine(lk0, am[0]);
            __builtin_amdgcn_sched_barrier(0);
            if (ks == 3) {
                // stage kb+1 landed everywhere (only stage kb+2 may still be
                // in flight) and every read of this slot is done (its values
                // are in registers) -> refill it with stage kb+3
                ring_wait_barrier<kDma>(kb + 2 < nkb ? 1 : 0);
                if (ctr && kb == kc && threadIdx.x == 0) claim = atomicAdd(ctr, 1);
                if constexpr (!kGateUp) {
                    if (kb == 0 && tid < nvalid) pw_row = rt.pair_w[pair];
                }
                if (kb == nkb - 1 && threadIdx.x == 0) *s_claim = claim;
                if (kb + 3 < nkb) L.template issue<NMT>(kb0 + kb + 3, sl);
                read_codes(nsl, codes_n);
                read_am(nsl, kb0 + kb + 1, am_n);
                frag_a(nsl, 0, af_n, 0, kHalfA);
                lk0 = frag_b(nsl, codes_n, 0, 0);
            } else {
                lk0 = frag_b(sl, codes, ksn, 0);
                frag_a(sl, ksn, af_n, 0, kHalfA);
            }
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt)
                acc[mt][0] = mma(af[mt], bf[0], acc[mt][0]);
#pragma unroll
            for (int i = 0; i < NMT; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                            // 1 MFMA
                if (!kNested) __builtin_amdgcn_sched_group_barrier(0x002, NMT <= 6 ? 3 : 2, 0);   // VALU
                __builtin_amdgcn_sched_group_barrier(0x100, (8 + kHalfA + 2 + NMT - 1) / NMT, 0);   // LDS reads
            }
            __builtin_amdgcn_sched_barrier(0);
            // ---- n-tile 1
            bf[1] = combine(lk1, am[1]);
            __builtin_amdgcn_sched_barrier(0);
            lk1 = frag_b(rs, ks == 3 ? codes_n : codes, ksn, 1);
            frag_a(rs, ksn, af_n, kHalfA, NMT);
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt)
                acc[mt][1] = mma(af[mt], bf[1], acc[mt][1]);
#pragma unroll
            for (int i = 0; i < NMT; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (!kNested) __builtin_amdgcn_sched_group_barrier(0x002, NMT <= 6 ? 3 : 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, (8 + NMT - kHalfA + NMT - 1) / NMT, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt) af[mt] = af_n[mt];
            if (ks == 3) {
#pragma unroll
                for (int c = 0; c < kNC; ++c) codes[c] = codes_n[c];
                am[0] = am_n[0];
                am[1] = am_n[1];
            }
        }
        slot = nslot;
    }
    }
    // All loads landed (none may still write LDS) and all ring reads are
    // done -> the ring is free; the rows' routing weights are in s_pw.
    if constexpr (!kGateUp) s_pw[tid] = pw_row;
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    next = next_of(*s_claim);
    if (next.e >= 0) ring_prologue<kGateUp, kFmt>(d, src, rt, next, ns, ring);

    // ---- epilogue, straight from the accumulators, through buffer
    // descriptors over the tile's rows (32-bit offsets; rows past the tile's
    // positions fall outside them and are dropped).
    if constexpr (kGateUp) {
        // act[p][i] = bf16(silu(gate) * up).  The weights are the MFMAs' A
        // operand, so D is the tile transposed: lane (m = lane%32, h =
        // lane/32), element i -> tile position 32*mt + m, weight row
        // 8*(i/4) + 4*h + (i%4) of the n-tile; a lane holds four runs of 4
        // consecutive columns of one position, stored 8 bytes at a time with
        // the hardware's pair conversion to bf16.  I is a multiple of 64, so
        // a wave's 32 columns (from a multiple of 32) are in range all or
        // none: one wave-uniform test (a lane-dependent one around each store
        // makes the compiler take the tile for divergent).
        const int wvs = __builtin_amdgcn_readfirstlane(wv);
        const int i0 = n0 + 32 * wvs;             // the wave's first column; lane runs at +4h+8g
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)((uint16_t*)dst + (int64_t)(ti.p0 + ti.m0) * I), 0, nvalid * I * 2, kBufWord3);
        if (i0 < I) {
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt) {
                const uint32_t ro = ((uint32_t)(mt * 32 + bn) * (uint32_t)I + (uint32_t)(i0 + 4 * bh)) * 2u;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    float a[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) a[r] = silu_mul(acc[mt][0][4 * g + r], acc[mt][1][4 * g + r]);
                    const u32x2_t v = {f32x2_to_bf16x2(a[0], a[1]), f32x2_to_bf16x2(a[2], a[3])};
                    __builtin_amdgcn_raw_buffer_store_b64(v, rs, (int)(ro + 16u * (uint32_t)g), 0, 0);
                }
            }
        }
    } else {
        // y[p][h] = acc * routing weight (fp32), K split z into its own y.  D
        // layout: lane (n = lane%32, h = lane/32), element i -> row m =
        // 8*(i/4) + 4*h + (i%4), column n: each store writes 32 consecutive
        // columns (128 bytes) of two rows.
        const int h0 = n0 + 64 * wv + bn;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)((float*)dst + ti.z * split_stride + (int64_t)(ti.p0 + ti.m0) * H), 0, nvalid * H * 4, kBufWord3);
        const uint32_t vo = (uint32_t)(4 * bh * H + h0) * 4u;
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int mrow = mt * 32 + 8 * (i >> 2) + (i & 3);
                const float pw = s_pw[min(mrow + 4 * bh, kBM - 1)];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    if (h0 + 32 * nt < H)
                        __builtin_amdgcn_raw_buffer_store_b32(
                            __float_as_uint(acc[mt][nt][i] * pw), rs,
                            (int)(vo + (uint32_t)mrow * (uint32_t)H * 4u + 128u * (uint32_t)nt), 0, 0);
            }
    }
}

constexpr int kOffLds = 1024;   // expert offsets held in LDS: E + S + 1 at most (more: read in place)

// sched: this launch's item counter and finished-CTA counter, zero at launch
// (the routing zeroes them; the last CTA to finish zeroes them again).
template <bool kGateUp, int kFmt>
__global__ __launch_bounds__(256, 1) void prefill_ring_kernel(lutmoe_moe_desc d, const uint16_t* __restrict__ src,
                                                              MoeRouting rt, void* __restrict__ dst, int ncu,
                                                              int nx, int ns, int64_t split_stride, int* sched) {
    constexpr bool kNested = kFmt == LUTMOE_FMT_NESTED;
    __shared__ __attribute__((aligned(16))) uint8_t ring[RingSlot<kFmt>::kLds];
    __shared__ int s_off[kOffLds];
    __shared__ int8_t s_bits[kNested ? kOffLds : 1];
    __shared__ int s_cls[kMaxClasses];
    __shared__ ClassTable s_ct;
    __shared__ float s_pw[kBM];
    __shared__ int s_claim;
    const int et = rt.num_experts_total;
    const int tid = threadIdx.x;
    // the expert offsets (and NestedLUT tier widths) in LDS, or, past
    // kOffLds - 1 experts, read in place (generic pointers)
    const bool in_lds = et < kOffLds;
    const int* off = in_lds ? (const int*)s_off : rt.offsets;
    const int8_t* bits = kNested ? (in_lds ? (const int8_t*)s_bits : (kGateUp ? d.w13 : d.w2).tier_bits) : s_bits;
    if (in_lds) {
        for (int i = tid; i <= et; i += blockDim.x) s_off[i] = rt.offsets[i];
        if constexpr (kNested) {
            const int8_t* tb = (kGateUp ? d.w13 : d.w2).tier_bits;
            for (int i = tid; i < et; i += blockDim.x) s_bits[i] = tb[i];
        }
    }
    if (tid < kMaxClasses) s_cls[tid] = 0;
    __syncthreads();
    // tile rows per class
    for (int e = tid; e < et; e += blockDim.x) {
        const int n = off[e + 1] - off[e];
        const int full = n >> 8, rn = ((n & (kBM - 1)) + 31) >> 5;
        const int b = kNested ? (int)bits[e] : 0;
        if (full + (rn == 8 ? 1 : 0) > 0) atomicAdd(&s_cls[tile_class(kNested, 8, b)], full + (rn == 8 ? 1 : 0));
        if (rn > 0 && rn < 8) atomicAdd(&s_cls[tile_class(kNested, rn, b)], 1);
    }
    __syncthreads();
    class_table(s_ct, s_cls, kNested, nx, ncu);
    __syncthreads();
    const ItemMap im = item_map(off, bits, &s_ct, et, kNested, nx, ns);
    const int G = gridDim.x, c = blockIdx.x;
    // Item order: longest first, the first G items to the CTAs in order, then
    // one item per claim from the launch counter.  With the claim at a tile's
    // end this also beats a snake order over the expert-ordered items where
    // the tiles are about equal (DeepSeek T=2048 by 0.6-1 %, Mixtral T=4096
    // by 5 %).
    int* ctr = sched;
    auto next_of = [&](int v) __attribute__((always_inline)) {
        return uniform_tile(map_item(im, G + __builtin_amdgcn_readfirstlane(v)));
    };
    RingTile cur = uniform_tile(map_item(im, c));
    if (cur.e >= 0) {
        ring_prologue<kGateUp, kFmt>(d, src, rt, cur, ns, ring);
        for (;;) {
            RingTile nxt;
            switch (ring_nmt(cur)) {
#define LUTMOE_TILE_CASE(n)                                                                                      \
    case n:                                                                                                      \
        ring_tile_body<kGateUp, kFmt, n>(d, src, rt, dst, cur, next_of, nxt, ctr, &s_claim, ring, s_pw, ns,   \
                                         split_stride);                                                          \
        break;
                LUTMOE_TILE_CASE(1) LUTMOE_TILE_CASE(2) LUTMOE_TILE_CASE(3) LUTMOE_TILE_CASE(4)
                LUTMOE_TILE_CASE(5) LUTMOE_TILE_CASE(6) LUTMOE_TILE_CASE(7) LUTMOE_TILE_CASE(8)
#undef LUTMOE_TILE_CASE
                default: nxt.e = -1; break;
            }
            if (nxt.e < 0) break;
            cur = nxt;
        }
    }
    // every claim of this CTA has returned: count it finished; the last one
    // zeroes both counters for the next launch
    if (tid == 0 && atomicAdd(sched + 1, 1) == G - 1) {
        atomicExch(sched, 0);
        atomicExch(sched + 1, 0);
    }
    // no load may still write LDS when the CTA ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <bool kGateUp>
__global__ __launch_bounds__(256, 1) void prefill_ref_kernel(lutmoe_moe_desc d, const uint16_t* __restrict__ src,
                                                             MoeRouting rt, void* __restrict__ dst, int ncu) {
    __shared__ __attribute__((aligned(16))) uint16_t s_a[2][kBM * kAStride];
    __shared__ float s_cb[256];
    const TileInfo ti = find_tile(rt, blockIdx.y, ncu);
    if (ti.e < 0) return;
    const uint16_t* cb = ref_codebook(kGateUp ? d.w13 : d.w2, ti.e);
    s_cb[threadIdx.x] = bf16_to_f32(cb[threadIdx.x]);
    const int nmt = (min(kBM, ti.n - ti.m0) + 31) / 32;
    switch (nmt) {
#define LUTMOE_TILE_CASE(n) \
    case n: prefill_tile_ref<kGateUp, n>(d, src, rt, dst, ti, s_a, s_cb); break;
        LUTMOE_TILE_CASE(1) LUTMOE_TILE_CASE(2) LUTMOE_TILE_CASE(3) LUTMOE_TILE_CASE(4)
        LUTMOE_TILE_CASE(5) LUTMOE_TILE_CASE(6) LUTMOE_TILE_CASE(7) LUTMOE_TILE_CASE(8)
#undef LUTMOE_TILE_CASE
        default: break;
    }
}

inline int max_tiles(int P, int E_tot) { return (P + kBM - 1) / kBM + E_tot; }
// extra grid rows for the tail split (find_tile cuts at most ncu / (2 nx) rows)
inline int tail_rows_max(int nx, int ncu) { return ncu / (2 * nx) + 1; }
// persistent ring grid: one CTA per compute unit, at most one per item
inline int persistent_ctas(int ncu, int64_t items) {
    const int64_t g = ncu > 0 ? ncu : 256;
    return (int)(items < g ? (items > 0 ? items : 1) : g);
}

}  // namespace

namespace lutmoe_host {

// Compute units of the current device (a per-device property cache).
static int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 0;
    cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

// The ring kernels address activations and one expert's codes / tables (or
// NestedLUT planes / tables) with 32-bit byte offsets from a scalar base.
static bool ring_offsets_fit(const lutmoe_moe_desc* d, const MoeRouting& r, int P) {
    const int64_t lim = int64_t(1) << 32;
    if ((int64_t)r.T * d->hidden * 2 >= lim || (int64_t)P * d->inter * 2 >= lim) return false;
    if (d->w13.format == LUTMOE_FMT_REF) {
        // one expert's codes and absmax by 32-bit offsets; absmax read as
        // aligned dwords (an even count per expert keeps them inside it)
        for (const lutmoe_weights* w : {&d->w13, &d->w2}) {
            if ((int64_t)w->rows * w->cols >= lim || w->absmax_per_expert % 2 || (uintptr_t)w->tables % 4)
                return false;
            if (w->block_size % 64 || w->cols % 64) return false;
        }
        return true;
    }
    if (d->w13.format == LUTMOE_FMT_NESTED)
        return (int64_t)d->w13.rows * d->w13.cols < lim && (int64_t)d->w2.rows * d->w2.cols < lim;
    return (int64_t)d->w13.rows * (d->w13.cols / 2) < lim && (int64_t)d->w2.rows * (d->w2.cols / 2) < lim;
}

int launch_prefill_gate_up(const lutmoe_moe_desc* d, const uint16_t* x, const MoeRouting& r,
                           uint16_t* act, int P, hipStream_t s) {
    const bool ring = ring_offsets_fit(d, r, P);
    if (d->w13.format != LUTMOE_FMT_REF && !ring) return LUTMOE_EUNSUPPORTED;
    const int nx = (d->inter + kBN / 2 - 1) / (kBN / 2), ncu = cu_count();
    const int rows = max_tiles(P, r.num_experts_total) + tail_rows_max(nx, ncu);
    if (d->w13.format == LUTMOE_FMT_REF && !ring) {
        const dim3 grid(nx, rows);
        hipLaunchKernelGGL((prefill_ref_kernel<true>), grid, dim3(256), 0, s, *d, x, r, (void*)act, ncu);
        return check_launch();
    }
    const dim3 grid(persistent_ctas(ncu, (int64_t)rows * nx));
    if (d->w13.format == LUTMOE_FMT_REF)
        hipLaunchKernelGGL((prefill_ring_kernel<true, LUTMOE_FMT_REF>), grid, dim3(256), 0, s, *d, x, r, (void*)act,
                           ncu, nx, 1, (int64_t)0, r.sched);
    else if (d->w13.format == LUTMOE_FMT_NESTED)
        hipLaunchKernelGGL((prefill_ring_kernel<true, LUTMOE_FMT_NESTED>), grid, dim3(256), 0, s, *d, x, r,
                           (void*)act, ncu, nx, 1, (int64_t)0, r.sched);
    else
        hipLaunchKernelGGL((prefill_ring_kernel<true, LUTMOE_FMT_BL4>), grid, dim3(256), 0, s, *d, x, r, (void*)act,
                           ncu, nx, 1, (int64_t)0, r.sched);
    return check_launch();
}

int launch_prefill_down(const lutmoe_moe_desc* d, const uint16_t* act, const MoeRouting& r,
                        float* y_pos, int P, int max_split, int* nsplit, hipStream_t s) {
    const bool ring = ring_offsets_fit(d, r, P);
    if (d->w2.format != LUTMOE_FMT_REF && !ring) return LUTMOE_EUNSUPPORTED;
    const int nx = (d->hidden + kBN - 1) / kBN, ncu = cu_count();
    // K split in two when the tiles (at most ceil(P/256) + active experts rows
    // of nx CTAs) would leave CUs idle: each half accumulates into its own y
    const int E_tot = r.num_experts_total;
    const int64_t rows_est = (P + kBM - 1) / kBM + (P < E_tot ? P : E_tot);
    const int ns = ring && max_split >= 2 && ncu > 0 && (int64_t)nx * rows_est < ncu &&
                           d->w2.cols / kBK >= 2 * kStages ? 2 : 1;
    *nsplit = ns;
    const int ncu_tail = ns > 1 ? 0 : ncu;   // one round: no tail split
    const int rows = max_tiles(P, E_tot) + tail_rows_max(nx, ncu_tail);
    const int64_t stride = (int64_t)P * d->hidden;
    if (d->w2.format == LUTMOE_FMT_REF && !ring) {
        const dim3 grid(nx, rows, ns);
        hipLaunchKernelGGL((prefill_ref_kernel<false>), grid, dim3(256), 0, s, *d, act, r, (void*)y_pos, ncu);
        return check_launch();
    }
    const dim3 grid(persistent_ctas(ncu, (int64_t)rows * nx * ns));
    if (d->w2.format == LUTMOE_FMT_REF)
        hipLaunchKernelGGL((prefill_ring_kernel<false, LUTMOE_FMT_REF>), grid, dim3(256), 0, s, *d, act, r,
                           (void*)y_pos, ncu_tail, nx, ns, stride, r.sched + 2);
    else if (d->w2.format == LUTMOE_FMT_NESTED)
        hipLaunchKernelGGL((prefill_ring_kernel<false, LUTMOE_FMT_NESTED>), grid, dim3(256), 0, s, *d, act, r,
                           (void*)y_pos, ncu_tail, nx, ns, stride, r.sched + 2);
    else
        hipLaunchKernelGGL((prefill_ring_kernel<false, LUTMOE_FMT_BL4>), grid, dim3(256), 0, s, *d, act, r,
                           (void*)y_pos, ncu_tail, nx, ns, stride, r.sched + 2);
    return check_launch();
}

}  // namespace lutmoe_host

/*
 * CPU oracle (test infrastructure only) for the LUT-dequant MoE expert path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only to check results against.  The product path never
 * calls it.
 *
 * What lives here (the parts that must be bit-exact with the HIP kernels and
 * are too slow in numpy at test sizes):
 *   - IEEE float32 -> float16 / bfloat16 round-to-nearest-even conversion;
 *   - the BL4 per-64-weight-block k-means encoder (k = 16, fp16 codebook);
 *   - the NestedLUT tree encoder (2 -> 3 -> 4 bit nested cells);
 *   - the reference REF decode GEMV restated in its own fp32 operation order.
 *
 * Reference procedure followed by the encoders: LUTQuantizer._train_kmeans
 * (vllm_lut/quantizer.py:120-178): init centroids from samples, Lloyd
 * iterations with assignment argmin|x-c| (first minimum wins, torch argmin),
 * mean update that leaves empty clusters unchanged (:170-173), final sort
 * (:176) and cast to the storage dtype (:177).  The reference quantizes codes
 * against the *stored* (rounded) codebook (quantize(), :292-296); so do we.
 *
 * Per-block deviations, fixed here because BL4 has no reference implementation:
 *   - initialisation is a binary-splitting tree (Linde-Buzo-Gray style, see
 *     tree_centroids) instead of a torch.randperm draw: deterministic and
 *     identical on CPU and GPU, and it escapes the poor local optima an
 *     equal-count start falls into on 64 samples;
 *   - every cluster sum is the 64-lane xor-butterfly sum over the block
 *     (non-members contribute +0), which is the order a wave64 reduction uses;
 *   - iterations stop early once the assignment no longer changes (a fixed
 *     point, so the result equals running all n_iter iterations);
 *   - in the final 16-means an empty cluster is re-seeded at the member
 *     farthest from its centroid (the reference leaves empty clusters where
 *     they are, which wastes codebook entries on blocks with repeated values).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define BL_BLOCK 64

/* ---------------------------------------------------------------- rounding */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;          /* NaN */
    u += 0x7fffu + ((u >> 16) & 1u);                             /* RNE */
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t oracle_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);      /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);     /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                       /* result subnormal or zero */
        if (a < 0x33000000u) return (uint16_t)sign;              /* < 2^-25 rounds to 0 */
        uint32_t e = a >> 23;                                     /* biased f32 exponent */
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        /* value = m * 2^(e-150); f16 subnormal unit = 2^-24 -> q = m >> (126 - e) */
        uint32_t shift = 126u - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal: rebias exponent 127 -> 15, keep 10 mantissa bits with RNE */
    uint32_t r = a - 0x38000000u;                                 /* (127-15) << 23 */
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1fu) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * (1.0f / 16777216.0f);                /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void oracle_f32_to_bf16_array(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_bf16(x[i]);
}
void oracle_f32_to_f16_array(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_f16(x[i]);
}

/* ------------------------------------------------------- block primitives */

/* 64-lane xor butterfly sum: level `off` pairs lane j with lane j^off. */
static float butterfly_sum64(const float* v) {
    float s[BL_BLOCK], t[BL_BLOCK];
    memcpy(s, v, sizeof(s));
    for (int off = 32; off >= 1; off >>= 1) {
        for (int j = 0; j < BL_BLOCK; ++j) t[j] = s[j] + s[j ^ off];
        memcpy(s, t, sizeof(s));
    }
    return s[0];
}

/* Stable rank of each element: #{i : x_i < x_j or (x_i == x_j and i < j)}. */
static void sort64(const float* x, float* sorted) {
    for (int j = 0; j < BL_BLOCK; ++j) {
        int r = 0;
        for (int i = 0; i < BL_BLOCK; ++i)
            r += (x[i] < x[j]) || (x[i] == x[j] && i < j);
        sorted[r] = x[j];
    }
}

static inline int argmin_abs(float v, const float* c, int k) {
    int best = 0;
    float bd = fabsf(v - c[0]);
    for (int i = 1; i < k; ++i) {
        float d = fabsf(v - c[i]);
        if (d < bd) { bd = d; best = i; }
    }
    return best;
}

/* Lloyd iterations on the members of one cell (mask) with k centroids.
 * assign[] holds the cluster of every member lane; non-members are ignored. */
/* Lloyd iterations on the members of one cell (mask) with k centroids.
 * assign[] holds the cluster of every member lane; non-members are ignored.
 * reseed != 0: after each mean update, every cluster left empty (in index
 * order) moves to the member farthest from its own centroid (lowest index on
 * ties; each point used once per iteration), when that distance is > 0. */
static void lloyd_ex(const float* x, const uint8_t* member, int k, float* c,
                     int n_iter, int* assign, int reseed) {
    for (int j = 0; j < BL_BLOCK; ++j) assign[j] = -1;
    for (int it = 0; it < n_iter; ++it) {
        int changed = 0;
        for (int j = 0; j < BL_BLOCK; ++j) {
            if (!member[j]) continue;
            int a = argmin_abs(x[j], c, k);
            if (a != assign[j]) { changed = 1; assign[j] = a; }
        }
        if (!changed) break;
        int empty[16], nempty = 0;
        for (int i = 0; i < k; ++i) {
            float v[BL_BLOCK];
            int cnt = 0;
            for (int j = 0; j < BL_BLOCK; ++j) {
                int in = member[j] && assign[j] == i;
                v[j] = in ? x[j] : 0.0f;
                cnt += in;
            }
            if (cnt) c[i] = butterfly_sum64(v) / (float)cnt;
            else if (nempty < 16) empty[nempty++] = i;
        }
        if (reseed && nempty) {
            uint8_t taken[BL_BLOCK] = {0};
            for (int q = 0; q < nempty; ++q) {
                int best = -1;
                float bd = 0.0f;
                for (int j = 0; j < BL_BLOCK; ++j) {
                    if (!member[j] || taken[j]) continue;
                    float d = fabsf(x[j] - c[assign[j]]);
                    if (d > bd) { bd = d; best = j; }
                }
                if (best < 0) break;
                c[empty[q]] = x[best];
                taken[best] = 1;
            }
        }
    }
}

static void lloyd(const float* x, const uint8_t* member, int k, float* c,
                  int n_iter, int* assign) {
    lloyd_ex(x, member, k, c, n_iter, assign, 0);
}

static void sort_small(float* c, int k) {
    for (int i = 1; i < k; ++i) {
        float v = c[i];
        int j = i - 1;
        while (j >= 0 && c[j] > v) { c[j + 1] = c[j]; --j; }
        c[j + 1] = v;
    }
}

/* ------------------------------------------------------------- tree init */

/* Split the members of one cell into 2 children with 2-means.
 * Init: child 0 = min member, child 1 = max member; an empty cell keeps the
 * parent centroid for both children.  Children are returned sorted. */
static void split2(const float* x, const uint8_t* member, float parent,
                   int n_iter, float* child) {
    int any = 0;
    float lo = 0.f, hi = 0.f;
    for (int j = 0; j < BL_BLOCK; ++j) {
        if (!member[j]) continue;
        if (!any) { lo = hi = x[j]; any = 1; }
        else { if (x[j] < lo) lo = x[j]; if (x[j] > hi) hi = x[j]; }
    }
    if (!any) { child[0] = child[1] = parent; return; }
    child[0] = lo; child[1] = hi;
    int assign[BL_BLOCK];
    lloyd(x, member, 2, child, n_iter, assign);
    sort_small(child, 2);
}

/* Binary-splitting tree of one 64-weight block (Linde-Buzo-Gray style):
 * level 2: 4-means from the quantile init sorted[16i+8], cells ordered by
 * centroid -> c2[4]; level 3: each level-2 cell j split by 2-means ->
 * c3[j | bit<<2]; level 4: each level-3 cell split -> c4[k | bit<<3].
 * Training cells are the final Lloyd assignments against float centroids. */
static void tree_centroids(const float* x, int n_iter, float* c2s, float* c3, float* c4) {
    float s[BL_BLOCK], c2[4];
    uint8_t member[BL_BLOCK];
    int a2[BL_BLOCK], cell3[BL_BLOCK];
    sort64(x, s);
    for (int i = 0; i < 4; ++i) c2[i] = s[16 * i + 8];
    memset(member, 1, sizeof(member));
    lloyd(x, member, 4, c2, n_iter, a2);
    int order[4] = {0, 1, 2, 3};
    for (int i = 1; i < 4; ++i) {
        int v = order[i]; int j = i - 1;
        while (j >= 0 && c2[order[j]] > c2[v]) { order[j + 1] = order[j]; --j; }
        order[j + 1] = v;
    }
    int rank[4];
    for (int i = 0; i < 4; ++i) { rank[order[i]] = i; c2s[i] = c2[order[i]]; }
    for (int j = 0; j < BL_BLOCK; ++j) a2[j] = rank[a2[j]];
    for (int j2 = 0; j2 < 4; ++j2) {
        uint8_t m[BL_BLOCK];
        for (int j = 0; j < BL_BLOCK; ++j) m[j] = (a2[j] == j2);
        float ch[2];
        split2(x, m, c2s[j2], n_iter, ch);
        c3[j2] = ch[0]; c3[j2 | 4] = ch[1];
    }
    for (int j = 0; j < BL_BLOCK; ++j) {
        int j2 = a2[j];
        float two[2] = {c3[j2], c3[j2 | 4]};
        cell3[j] = j2 | (argmin_abs(x[j], two, 2) << 2);
    }
    for (int k3 = 0; k3 < 8; ++k3) {
        uint8_t m[BL_BLOCK];
        for (int j = 0; j < BL_BLOCK; ++j) m[j] = (cell3[j] == k3);
        float ch[2];
        split2(x, m, c3[k3], n_iter, ch);
        c4[k3] = ch[0]; c4[k3 | 8] = ch[1];
    }
}

/* ---------------------------------------------------------------- BL4 */

/* Encode nblocks blocks of 64 fp32 weights: tree init (16 leaves), then
 * n_iter Lloyd iterations with k = 16 (empty clusters re-seeded at the
 * farthest point), sort, fp16, argmin codes.
 * codes: one code (0..15) per weight, unpacked, [nblocks*64].
 * table: fp16 bits of the sorted 16-entry codebook, [nblocks*16]. */
void oracle_bl4_encode(const float* w, int64_t nblocks, int n_iter,
                       uint8_t* codes, uint16_t* table) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const float* x = w + b * BL_BLOCK;
        float c2[4], c3[8], c[16], cf[16];
        uint8_t member[BL_BLOCK];
        int assign[BL_BLOCK];
        tree_centroids(x, n_iter, c2, c3, c);
        memset(member, 1, sizeof(member));
        lloyd_ex(x, member, 16, c, n_iter, assign, 1);
        sort_small(c, 16);
        for (int i = 0; i < 16; ++i) {
            table[b * 16 + i] = oracle_f32_to_f16(c[i]);
            cf[i] = oracle_f16_to_f32(table[b * 16 + i]);
        }
        for (int j = 0; j < BL_BLOCK; ++j)
            codes[b * BL_BLOCK + j] = (uint8_t)argmin_abs(x[j], cf, 16);
    }
}

/* ------------------------------------------------------------- NestedLUT */

/* Nested tree encoder.  Tier-b code of a weight = low b bits of its 4-bit code.
 * Tables are the tree's levels: T2[4] = c2, T3[8] = c3, T4[16] = c4 (fp16).
 * The stored code is a descent through the fp16 tables (argmin at each
 * level, first minimum wins), so the tier-b reconstruction T_b[code & (2^b-1)]
 * only uses the low b bits.
 * codes [nblocks*64] (0..15); t2 [nblocks*4]; t3 [nblocks*8]; t4 [nblocks*16]
 * (fp16 bits). */
void oracle_nested_encode(const float* w, int64_t nblocks, int n_iter,
                          uint8_t* codes, uint16_t* t2, uint16_t* t3, uint16_t* t4) {
    for (int64_t b = 0; b < nblocks; ++b) {
        const float* x = w + b * BL_BLOCK;
        float c2[4], c3[8], c4[16];
        tree_centroids(x, n_iter, c2, c3, c4);
        float f2[4], f3[8], f4[16];
        for (int i = 0; i < 4; ++i) { t2[b * 4 + i] = oracle_f32_to_f16(c2[i]); f2[i] = oracle_f16_to_f32(t2[b * 4 + i]); }
        for (int i = 0; i < 8; ++i) { t3[b * 8 + i] = oracle_f32_to_f16(c3[i]); f3[i] = oracle_f16_to_f32(t3[b * 8 + i]); }
        for (int i = 0; i < 16; ++i) { t4[b * 16 + i] = oracle_f32_to_f16(c4[i]); f4[i] = oracle_f16_to_f32(t4[b * 16 + i]); }
        for (int j = 0; j < BL_BLOCK; ++j) {
            int q2 = argmin_abs(x[j], f2, 4);
            float p3[2] = {f3[q2], f3[q2 | 4]};
            int q3 = q2 | (argmin_abs(x[j], p3, 2) << 2);
            float p4[2] = {f4[q3], f4[q3 | 8]};
            codes[b * BL_BLOCK + j] = (uint8_t)(q3 | (argmin_abs(x[j], p4, 2) << 3));
        }
    }
}

/* --------------------------------------------------------------- REF GEMV */

/* The reference decode kernel's arithmetic (vllm_lut/cuda_lut_gemv.py:23-80):
 * per element accum += (x * cb_f32[idx]) * absmax_f32[min((rK+c)/128, nb-1)],
 * in fp32.  Returned per row in double (sum of the fp32 products) so the
 * result does not depend on the GPU's reduction order; the kernels are held
 * to a tolerance against it. */
void oracle_ref_gemv(const uint16_t* x_bf16, const uint8_t* idx, const uint16_t* cb_bf16,
                     const uint16_t* absmax_bf16, int64_t M, int64_t K, int64_t nb,
                     double* y) {
    float cb[256];
    for (int i = 0; i < 256; ++i) cb[i] = oracle_bf16_to_f32(cb_bf16[i]);
    for (int64_t r = 0; r < M; ++r) {
        double acc = 0.0;
        for (int64_t c = 0; c < K; ++c) {
            int64_t flat = r * K + c;
            int64_t blk = flat / 128;
            if (blk >= nb) blk = nb - 1;
            float p = oracle_bf16_to_f32(x_bf16[c]) * cb[idx[flat]];
            p = p * oracle_bf16_to_f32(absmax_bf16[blk]);
            acc += (double)p;
        }
        y[r] = acc;
    }
}

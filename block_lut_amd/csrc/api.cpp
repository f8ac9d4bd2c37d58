// extern "C" entry points of liblutmoe.so: argument validation (before any
// HIP call, so every rejection is testable without a GPU), workspace
// carving, and dispatch to the kernel launchers.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <cstdio>

#include "../../include/lutmoe.h"
#include "kernels.h"

namespace lutmoe_host {

hipStream_t stream_of(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Per-thread text of the last failure (lutmoe_last_error).
thread_local char g_last_error[256] = "";

// A failed launch names its HIP error in the last-error text.
int check_launch() {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return LUTMOE_OK;
    snprintf(g_last_error, sizeof(g_last_error), "HIP runtime error: %s (%s)", hipGetErrorName(e),
             hipGetErrorString(e));
    return LUTMOE_EHIP;
}

}  // namespace lutmoe_host

using namespace lutmoe_host;

namespace {

void set_last_error(const char* fn, int code) {
    if (code == LUTMOE_OK) { g_last_error[0] = 0; return; }
    if (code == LUTMOE_EHIP && strncmp(g_last_error, "HIP runtime error: ", 19) == 0) {
        char hip[256];
        snprintf(hip, sizeof(hip), "%s", g_last_error);
        snprintf(g_last_error, sizeof(g_last_error), "%s: %s", fn, hip);
        return;
    }
    snprintf(g_last_error, sizeof(g_last_error), "%s: %s", fn, lutmoe_strerror(code));
}

inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int validate_weights(const lutmoe_weights* w) {
    if (!w || !w->codes || !w->tables) return LUTMOE_EINVAL;
    if (w->num_experts <= 0 || w->rows <= 0 || w->cols <= 0) return LUTMOE_EINVAL;
    switch (w->format) {
        case LUTMOE_FMT_REF:
            if (!w->codebook || w->block_size <= 0 || w->absmax_per_expert <= 0) return LUTMOE_EINVAL;
            if (w->codebook_stride != 0 && w->codebook_stride < 256) return LUTMOE_EINVAL;
            if ((int64_t)w->rows * w->cols >= (1ll << 31)) return LUTMOE_EUNSUPPORTED;
            return LUTMOE_OK;
        case LUTMOE_FMT_BL4:
            if (w->cols % 64) return LUTMOE_EINVAL;
            if (!aligned(w->codes, 16) || !aligned(w->tables, 16)) return LUTMOE_EALIGN;
            return LUTMOE_OK;
        case LUTMOE_FMT_NESTED:
            if (w->cols % 64 || !w->tier_bits) return LUTMOE_EINVAL;
            return LUTMOE_OK;
        default:
            return LUTMOE_EINVAL;
    }
}

// Preconditions of the vectorised REF paths (grouped GEMV / MFMA): whole
// 64-column blocks and absmax blocks made of whole 64-column steps.
int validate_ref_vector(const lutmoe_weights* w) {
    if (w->cols % 64 || w->block_size % 64) return LUTMOE_EUNSUPPORTED;
    if (!aligned(w->codes, 16)) return LUTMOE_EALIGN;
    return LUTMOE_OK;
}

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

struct MoeLayout {
    size_t route, topk_w, topk_ids, pair_ids, pair_w, offsets, perm, inv, active, sched, act, y, dact, dy, dw, total;
};

// Room for two K-split partial results of the down projection when that is
// small (the split fills the GPU when the grouped down GEMM has few tiles).
size_t prefill_y_splits(size_t P, int H) { return P * (size_t)H * 4 <= (size_t(32) << 20) ? 2 : 1; }

MoeLayout moe_layout(const lutmoe_moe_desc* d, int T, int k) {
    const int E_tot = d->num_routed + d->num_shared;
    const size_t P = (size_t)T * (k + d->num_shared);
    MoeLayout L{};
    size_t o = 0;
    L.route = o;    o = align_up(o + decode_route_bytes());
    L.topk_w = o;   o = align_up(o + (size_t)T * k * 4);
    L.topk_ids = o; o = align_up(o + (size_t)T * k * 4);
    L.pair_ids = o; o = align_up(o + P * 4);
    L.pair_w = o;   o = align_up(o + P * 4);
    L.offsets = o;  o = align_up(o + (E_tot + 1) * 4);
    L.perm = o;     o = align_up(o + P * 4);
    L.inv = o;      o = align_up(o + P * 4);
    L.active = o;   o = align_up(o + (E_tot + 1) * 4);
    L.sched = o;    o = align_up(o + 4 * 4);
    L.act = o;      o = align_up(o + P * d->inter * 2);
    L.y = o;        o = align_up(o + P * d->hidden * 4 * prefill_y_splits(P, d->hidden));
    // the dense shared expert: its activations, its weighted rows, token weights
    const size_t Is = d->dense_inter > 0 ? (size_t)d->dense_inter : 0;
    L.dact = o;     o = align_up(o + (Is ? (size_t)T * Is * 2 : 0));
    L.dy = o;       o = align_up(o + (Is ? (size_t)T * d->hidden * 4 : 0));
    L.dw = o;       o = align_up(o + (Is ? (size_t)T * 4 : 0));
    L.total = o;
    return L;
}

int validate_moe(const lutmoe_moe_desc* d) {
    if (!d) return LUTMOE_EINVAL;
    int rc = validate_weights(&d->w13);
    if (rc) return rc;
    rc = validate_weights(&d->w2);
    if (rc) return rc;
    const int H = d->hidden, I = d->inter;
    if (H <= 0 || I <= 0 || d->num_routed <= 0 || d->num_shared < 0) return LUTMOE_EINVAL;
    if (d->w13.rows != 2 * I || d->w13.cols != H || d->w2.rows != H || d->w2.cols != I)
        return LUTMOE_EINVAL;
    const int E_tot = d->num_routed + d->num_shared;
    if (d->w13.num_experts < E_tot || d->w2.num_experts < E_tot) return LUTMOE_EINVAL;
    if (d->w13.format != d->w2.format) return LUTMOE_EUNSUPPORTED;
    if (H % 64 || I % 64) return LUTMOE_EUNSUPPORTED;
    if (d->shared_gate && !aligned(d->shared_gate, 16)) return LUTMOE_EALIGN;
    if (d->dense_inter < 0 || d->dense_reserved != 0) return LUTMOE_EINVAL;
    if (d->dense_inter > 0) {
        if (!d->dense_w13 || !d->dense_w2) return LUTMOE_EINVAL;
        if (d->dense_inter % 64) return LUTMOE_EUNSUPPORTED;
        if (!aligned(d->dense_w13, 16) || !aligned(d->dense_w2, 16)) return LUTMOE_EALIGN;
        if ((int64_t)2 * d->dense_inter * H >= (1ll << 31)) return LUTMOE_EUNSUPPORTED;
    }
    if (d->w13.format == LUTMOE_FMT_REF) {
        if ((rc = validate_ref_vector(&d->w13)) || (rc = validate_ref_vector(&d->w2))) return rc;
    }
    return LUTMOE_OK;
}

}  // namespace

extern "C" {

const char* lutmoe_strerror(int code) {
    switch (code) {
        case LUTMOE_OK: return "ok";
        case LUTMOE_EINVAL: return "invalid argument";
        case LUTMOE_EUNSUPPORTED: return "unsupported shape or format combination";
        case LUTMOE_EHIP: return "HIP runtime error";
        case LUTMOE_EWORKSPACE: return "workspace too small";
        case LUTMOE_EALIGN: return "pointer not aligned for vector access";
        default: return "unknown error";
    }
}

const char* lutmoe_version(void) { return "lutmoe 0.1.0 gfx950"; }

const char* lutmoe_last_error(void) { return g_last_error; }

// ------------------------------------------------------ reference-compatible

int launch_blocklut_decompress(void* output, const void* indices, const void* absmax,
                               const void* codebook, int N, int block_size, void* stream) {
    if (N < 0 || block_size <= 0 || (N > 0 && (!output || !indices || !absmax || !codebook)))
        return -1;
    if (N == 0) return 0;
    const int64_t nb = ((int64_t)N + block_size - 1) / block_size;
    const int rc = launch_ref_dequant((uint16_t*)output, (const uint8_t*)indices,
                                      (const uint16_t*)absmax, (const uint16_t*)codebook, N, nb,
                                      block_size, 1, 0, 0, stream_of(stream));
    return rc == LUTMOE_OK ? 0 : -1;
}

int launch_batch_blocklut_decompress(void* output, const void* indices, const void* absmax,
                                     const void* codebook, int num_experts,
                                     int elements_per_expert, int blocks_per_expert,
                                     int block_size, void* stream) {
    if (num_experts < 0 || elements_per_expert < 0 || blocks_per_expert <= 0 || block_size <= 0)
        return -1;
    if (num_experts == 0 || elements_per_expert == 0) return 0;
    if (!output || !indices || !absmax || !codebook) return -1;
    // The reference kernel leaves elements whose block index reaches
    // blocks_per_expert unwritten; callers size absmax so that never happens,
    // which is the only case accepted here.
    if (((int64_t)elements_per_expert + block_size - 1) / block_size > blocks_per_expert) return -1;
    const int rc = launch_ref_dequant((uint16_t*)output, (const uint8_t*)indices,
                                      (const uint16_t*)absmax, (const uint16_t*)codebook,
                                      elements_per_expert, blocks_per_expert, block_size,
                                      num_experts, elements_per_expert, elements_per_expert,
                                      stream_of(stream));
    return rc == LUTMOE_OK ? 0 : -1;
}

void lut_moe_launch_blocklut_recover(uint16_t* out, const uint8_t* idx, const uint16_t* absmax,
                                     const uint16_t* lut, size_t n, void* stream) {
    int rc = LUTMOE_OK;
    if (n == 0) { set_last_error(__func__, rc); return; }
    if (!out || !idx || !absmax || !lut || n >= (1ull << 31)) rc = LUTMOE_EINVAL;
    else rc = launch_ref_dequant(out, idx, absmax, lut, (int64_t)n, ((int64_t)n + 127) / 128, 128,
                                 1, 0, 0, stream_of(stream));
    set_last_error(__func__, rc);
}

void lut_moe_launch_unpack_4bit(uint8_t* data, size_t n, void* stream) {
    int rc = LUTMOE_OK;
    if (n == 0) { set_last_error(__func__, rc); return; }
    if (!data || (n & 1)) rc = LUTMOE_EINVAL;
    else rc = launch_unpack_4bit_inplace(data, (int64_t)n, stream_of(stream));
    set_last_error(__func__, rc);
}

void launch_lut_gemv_kernel(const void* input, const void* indices, const void* codebook,
                            const void* absmax, void* output, int M, int K, int num_blocks) {
    int rc = LUTMOE_OK;
    if (M <= 0 || K <= 0 || num_blocks <= 0 || !input || !indices || !codebook || !absmax || !output)
        rc = LUTMOE_EINVAL;
    else
        rc = launch_ref_gemv((const uint16_t*)input, (const uint8_t*)indices, nullptr,
                             (const float*)codebook, (const uint16_t*)absmax, output, M, K, 1,
                             num_blocks, 128, LUTMOE_DTYPE_BF16, nullptr);
    set_last_error(__func__, rc);
}

// ------------------------------------------------------------------- REF

int lutmoe_ref_gemv(const void* x, const void* indices, const void* codebook, const void* absmax,
                    void* y, int M, int K, int T, int num_blocks, int block_size, int y_dtype,
                    void* stream) {
    if (M <= 0 || K <= 0 || T < 0 || num_blocks <= 0 || block_size <= 0) return LUTMOE_EINVAL;
    if (y_dtype != LUTMOE_DTYPE_BF16 && y_dtype != LUTMOE_DTYPE_F32) return LUTMOE_EINVAL;
    if (!x || !indices || !codebook || !absmax || !y) return LUTMOE_EINVAL;
    if ((int64_t)M * K >= (1ll << 31)) return LUTMOE_EUNSUPPORTED;
    if (T == 0) return LUTMOE_OK;
    return launch_ref_gemv((const uint16_t*)x, (const uint8_t*)indices, (const uint16_t*)codebook,
                           nullptr, (const uint16_t*)absmax, y, M, K, T, num_blocks, block_size,
                           y_dtype, stream_of(stream));
}

int lutmoe_fused_lut_gemv(const void* x, const void* indices, const void* codebook, const void* absmax,
                          void* y, int M, int K, int T, int num_blocks, int block_size, int y_dtype,
                          void* stream) {
    if (M <= 0 || K <= 0 || T < 0 || num_blocks <= 0 || block_size <= 0) return LUTMOE_EINVAL;
    if (y_dtype != LUTMOE_DTYPE_BF16 && y_dtype != LUTMOE_DTYPE_F32) return LUTMOE_EINVAL;
    if (!x || !indices || !codebook || !absmax || !y) return LUTMOE_EINVAL;
    if ((int64_t)M * K >= (1ll << 31)) return LUTMOE_EUNSUPPORTED;
    if (T == 0) return LUTMOE_OK;
    return launch_ref_gemv((const uint16_t*)x, (const uint8_t*)indices, (const uint16_t*)codebook,
                           nullptr, (const uint16_t*)absmax, y, M, K, T, num_blocks, block_size,
                           y_dtype, stream_of(stream), true);
}

int lutmoe_pack_bitplanes(const uint8_t* codes, int64_t n, uint8_t* packed, void* stream) {
    if (n < 0 || (n % 4)) return LUTMOE_EINVAL;
    if (n == 0) return LUTMOE_OK;
    if (!codes || !packed) return LUTMOE_EINVAL;
    return launch_pack_bitplanes(codes, n, packed, stream_of(stream));
}

int lutmoe_merge_bitplane(uint8_t* codes, const uint8_t* plane, int64_t n, int shift, void* stream) {
    if (n < 0 || (n % 4) || shift < 0 || shift > 6 || (shift & 1)) return LUTMOE_EINVAL;
    if (n == 0) return LUTMOE_OK;
    if (!codes || !plane) return LUTMOE_EINVAL;
    return launch_merge_bitplane(codes, plane, n, shift, stream_of(stream));
}

int lutmoe_unpack_6bit(const uint8_t* packed, uint8_t* out, int64_t n, void* stream) {
    if (n < 0 || (n % 4)) return LUTMOE_EINVAL;
    if (n == 0) return LUTMOE_OK;
    if (!packed || !out) return LUTMOE_EINVAL;
    return launch_unpack_6bit(packed, out, n, stream_of(stream));
}

int lutmoe_nested_group_planes(const uint8_t* planes, int bits, int64_t n, uint8_t* out, void* stream) {
    if (n < 0 || (n % 64) || bits < 2 || bits > 4) return LUTMOE_EINVAL;
    if (n == 0) return LUTMOE_OK;
    if (!planes || !out) return LUTMOE_EINVAL;
    if (!aligned(planes, 4) || !aligned(out, 4)) return LUTMOE_EALIGN;
    return launch_nested_group_planes(planes, bits, n, out, stream_of(stream));
}

// ---------------------------------------------------------------- generic

int lutmoe_dequant(const lutmoe_weights* w, int e0, int ne, void* out, void* stream) {
    int rc = validate_weights(w);
    if (rc) return rc;
    if (!out || e0 < 0 || ne < 0 || e0 + ne > w->num_experts) return LUTMOE_EINVAL;
    if (ne == 0) return LUTMOE_OK;
    const int64_t n = (int64_t)w->rows * w->cols;
    switch (w->format) {
        case LUTMOE_FMT_REF:
            return launch_ref_dequant((uint16_t*)out, (const uint8_t*)w->codes + e0 * n,
                                      (const uint16_t*)w->tables + e0 * w->absmax_per_expert,
                                      (const uint16_t*)w->codebook + (int64_t)e0 * w->codebook_stride, n,
                                      w->absmax_per_expert, w->block_size, ne, n, n, stream_of(stream),
                                      w->codebook_stride);
        case LUTMOE_FMT_BL4: {
            if (!aligned(out, 16)) return LUTMOE_EALIGN;
            const int64_t nbl = n / 64;
            return launch_bl4_dequant((uint16_t*)out, (const uint8_t*)w->codes + e0 * (n / 2),
                                      (const uint16_t*)w->tables + e0 * (n / 4), ne * nbl,
                                      stream_of(stream));
        }
        default:
            if (!aligned(out, 16)) return LUTMOE_EALIGN;
            return launch_nested_dequant((uint16_t*)out, w, e0, ne, stream_of(stream));
    }
}

int lutmoe_gemv_ex(const lutmoe_weights* w, int expert, const void* x, int x_dtype, int T, void* y, int y_dtype,
                   void* stream) {
    int rc = validate_weights(w);
    if (rc) return rc;
    if (!x || !y || T < 0 || expert < 0 || expert >= w->num_experts) return LUTMOE_EINVAL;
    if (y_dtype != LUTMOE_DTYPE_BF16 && y_dtype != LUTMOE_DTYPE_F32) return LUTMOE_EINVAL;
    if (x_dtype != LUTMOE_DTYPE_BF16 && x_dtype != LUTMOE_DTYPE_F32) return LUTMOE_EINVAL;
    if (!aligned(x, 16) || w->cols % 8) return LUTMOE_EALIGN;
    if (T == 0) return LUTMOE_OK;
    if (w->format == LUTMOE_FMT_NESTED) {
        if (x_dtype == LUTMOE_DTYPE_F32) return LUTMOE_EUNSUPPORTED;
        return launch_nested_gemv(w, expert, (const uint16_t*)x, T, y, y_dtype, stream_of(stream));
    }
    if (w->format == LUTMOE_FMT_REF && (rc = validate_ref_vector(w))) return rc;
    return launch_bl4_gemv(w, expert, x, x_dtype == LUTMOE_DTYPE_F32, T, y, y_dtype, stream_of(stream));
}

int lutmoe_gemv(const lutmoe_weights* w, int expert, const void* x, int T, void* y, int y_dtype,
                void* stream) {
    return lutmoe_gemv_ex(w, expert, x, LUTMOE_DTYPE_BF16, T, y, y_dtype, stream);
}

int lutmoe_bl4_tables_from_f16(const uint16_t* f16, uint16_t* bf16, int64_t n, void* stream) {
    if (n < 0) return LUTMOE_EINVAL;
    if (n == 0) return LUTMOE_OK;
    if (!f16 || !bf16) return LUTMOE_EINVAL;
    if (!aligned(f16, 16) || !aligned(bf16, 16)) return LUTMOE_EALIGN;
    return launch_f16_to_bf16(f16, bf16, n, stream_of(stream));
}

// ---------------------------------------------------------------- routing

int lutmoe_route_topk(const float* logits, int T, int E, int k, int renormalize, float scaling,
                      float* topk_w, int32_t* topk_ids, void* stream) {
    if (T < 0 || E <= 0 || k <= 0 || k > E || k > 16) return LUTMOE_EINVAL;
    if (E > 4096) return LUTMOE_EUNSUPPORTED;
    if (T == 0) return LUTMOE_OK;
    if (!logits || !topk_w || !topk_ids) return LUTMOE_EINVAL;
    return launch_route_topk(logits, T, E, k, renormalize, scaling, topk_w, topk_ids,
                             stream_of(stream));
}

int lutmoe_router_logits(const void* x, const void* gate, int T, int H, int E, float* logits, int round_bf16,
                         void* stream) {
    if (T < 0 || H <= 0 || E <= 0 || (H % 8) || T > 65535) return LUTMOE_EINVAL;
    if (T == 0) return LUTMOE_OK;
    if (!x || !gate || !logits) return LUTMOE_EINVAL;
    if (!aligned(x, 16) || !aligned(gate, 16)) return LUTMOE_EALIGN;
    return launch_router_logits((const uint16_t*)x, (const uint16_t*)gate, T, H, E, logits, round_bf16 ? 1 : 0,
                                stream_of(stream));
}

int lutmoe_permute(const int32_t* topk_ids, int T, int k, int E, int32_t* offsets, int32_t* perm,
                   int32_t* inv, int32_t* active, void* stream) {
    if (T < 0 || k <= 0 || E <= 0 || E > 4096) return LUTMOE_EINVAL;
    if (!topk_ids || !offsets || !perm || !inv || !active) return LUTMOE_EINVAL;
    if ((int64_t)T * k >= (1ll << 31)) return LUTMOE_EUNSUPPORTED;
    return launch_permute(topk_ids, T, k, E, offsets, perm, inv, active, stream_of(stream));
}

// -------------------------------------------------------------- MoE layer

size_t lutmoe_decode_stream_probe_sink_words(const lutmoe_moe_desc* d, int k, int which) {
    if (validate_moe(d) || k <= 0 || which < 1 || which > 3) return 0;
    return decode_stream_probe_ctas(d, k + d->num_shared, which);
}

int lutmoe_decode_stream_probe(const lutmoe_moe_desc* d, const int32_t* ids_dev, int k, int which,
                               uint32_t* sink_dev, void* stream) {
    int rc = validate_moe(d);
    if (rc) return rc;
    if (!ids_dev || !sink_dev || k <= 0 || which < 1 || which > 3) return LUTMOE_EINVAL;
    if (d->w13.format != LUTMOE_FMT_BL4 || d->hidden > 2048 || d->inter > 2048 || k + d->num_shared > 64)
        return LUTMOE_EUNSUPPORTED;
    return launch_decode_stream_probe(d, ids_dev, k + d->num_shared, which, sink_dev, stream_of(stream));
}

size_t lutmoe_moe_workspace_size(const lutmoe_moe_desc* d, int T, int k) {
    if (!d || T < 0 || k <= 0) return 0;
    return moe_layout(d, T, k).total;
}

}  // extern "C"

namespace lutmoe_host {

// Shared body of the MoE entry points.  Exactly one of (topk_w, topk_ids) and
// logits is given.
int moe_forward_impl(const lutmoe_moe_desc* d, const void* x, const float* topk_w,
                     const int32_t* topk_ids, const float* logits, int T, int k, int renorm,
                     float scaling, void* out, int out_dtype, void* workspace, size_t ws_bytes,
                     int force_path, int stages, void* stream) {
    if (stages <= 0 || stages > LUTMOE_STAGE_ALL) return LUTMOE_EINVAL;
    int rc = validate_moe(d);
    if (rc) return rc;
    if (T < 0 || k <= 0 || k > d->num_routed || k + d->num_shared > 16) return LUTMOE_EINVAL;
    if (out_dtype != LUTMOE_DTYPE_BF16 && out_dtype != LUTMOE_DTYPE_F32) return LUTMOE_EINVAL;
    if (force_path < 0 || force_path > 2) return LUTMOE_EINVAL;
    if (T == 0) return LUTMOE_OK;
    const bool by_logits = logits != nullptr;
    if (!x || !out || !workspace || (!by_logits && (!topk_w || !topk_ids))) return LUTMOE_EINVAL;
    if (by_logits && d->num_routed > 320) return LUTMOE_EUNSUPPORTED;
    if (!aligned(x, 16) || !aligned(out, 16) || !aligned(workspace, 256)) return LUTMOE_EALIGN;
    const MoeLayout L = moe_layout(d, T, k);
    if (ws_bytes < L.total) return LUTMOE_EWORKSPACE;
    const int S = d->num_shared, E = d->num_routed, E_tot = E + S, ke = k + S;
    const int64_t P = (int64_t)T * ke;
    if (P >= (1ll << 31) / (d->hidden > d->inter ? d->hidden : d->inter)) return LUTMOE_EUNSUPPORTED;
    const bool lds_ok = P * 8 * 4 <= 48 * 1024;
    bool gemv = force_path == 1 || (force_path == 0 && T <= 32 && lds_ok);
    if (gemv && !lds_ok) return LUTMOE_EUNSUPPORTED;
    // the decode-layer kernels take up to 320 experts and 512 (token, slot)
    // pairs; anything else runs on the grouped MFMA path
    if (gemv && !decode_v2_supported(d, T, k)) {
        if (force_path == 1) return LUTMOE_EUNSUPPORTED;
        gemv = false;
    }

    char* ws = (char*)workspace;
    uint16_t* act = (uint16_t*)(ws + L.act);
    hipStream_t s = stream_of(stream);
    // the dense shared expert: gate/up with the gate/up stage, its weighted
    // rows with the down stage, before the kernels that write the output
    // (which add them)
    const bool dense = d->dense_inter > 0;
    const float* addend = dense ? (const float*)(ws + L.dy) : nullptr;
    if (dense && (stages & LUTMOE_STAGE_GATE_UP) &&
        (rc = launch_dense_gate_up(d, (const uint16_t*)x, T, !gemv, (uint16_t*)(ws + L.dact), (float*)(ws + L.dw), s)))
        return rc;
    if (dense && (stages & LUTMOE_STAGE_DOWN) &&
        (rc = launch_dense_down(d, (const uint16_t*)(ws + L.dact), T, !gemv, (const float*)(ws + L.dw),
                                (float*)(ws + L.dy), s)))
        return rc;
    if (gemv) {
        // routing + permutation happen inside both decode kernels
        return launch_decode_v2(d, (const uint16_t*)x, topk_w, topk_ids, logits, T, k, renorm,
                                scaling, act, ws + L.route, (float*)(ws + L.y), out, out_dtype, stages, s, addend);
    }
    int32_t* pair_ids = (int32_t*)(ws + L.pair_ids);
    float* pair_w = (float*)(ws + L.pair_w);
    MoeRouting r;
    r.offsets = (int32_t*)(ws + L.offsets);
    r.perm = (int32_t*)(ws + L.perm);
    r.inv = (int32_t*)(ws + L.inv);
    r.active = (int32_t*)(ws + L.active);
    r.pair_w = pair_w;
    r.T = T;
    r.k_eff = ke;
    r.num_experts_total = E_tot;
    r.sched = (int32_t*)(ws + L.sched);
    float* y = (float*)(ws + L.y);
    if (stages & LUTMOE_STAGE_ROUTE) {
        if (by_logits) {
            float* tw = (float*)(ws + L.topk_w);
            int32_t* ti = (int32_t*)(ws + L.topk_ids);
            if ((rc = launch_route_topk(logits, T, E, k, renorm, scaling, tw, ti, s))) return rc;
            topk_w = tw;
            topk_ids = ti;
        }
        if ((rc = launch_route_pairs(topk_ids, topk_w, T, k, E, S, (int32_t*)r.offsets, (int32_t*)r.perm,
                                     (int32_t*)r.inv, (int32_t*)r.active, pair_ids, pair_w, s, r.sched)))
            return rc;
        if (d->shared_gate && S > 0 &&
            (rc = launch_shared_gate((const uint16_t*)x, (const uint16_t*)d->shared_gate, T, d->hidden, k, S,
                                     pair_w, s)))
            return rc;
    }
    if ((stages & LUTMOE_STAGE_GATE_UP) &&
        (rc = launch_prefill_gate_up(d, (const uint16_t*)x, r, act, (int)P, s)))
        return rc;
    if (stages & LUTMOE_STAGE_DOWN) {
        int nsplit = 1;
        if ((rc = launch_prefill_down(d, act, r, y, (int)P, (int)prefill_y_splits(P, d->hidden), &nsplit, s)))
            return rc;
        return launch_combine(y, r.inv, T, ke, d->hidden, out, out_dtype, s, nsplit, (int64_t)P * d->hidden,
                              addend);
    }
    return LUTMOE_OK;
}

void set_last_error_text(const char* text) { snprintf(g_last_error, sizeof(g_last_error), "%s", text); }

}  // namespace lutmoe_host

extern "C" {

int lutmoe_moe_forward(const lutmoe_moe_desc* d, const void* x, const float* topk_w,
                       const int32_t* topk_ids, int T, int k, void* out, int out_dtype,
                       void* workspace, size_t ws_bytes, int force_path, void* stream) {
    if (!topk_w || !topk_ids) return T == 0 ? LUTMOE_OK : LUTMOE_EINVAL;
    return moe_forward_impl(d, x, topk_w, topk_ids, nullptr, T, k, 0, 1.0f, out, out_dtype,
                            workspace, ws_bytes, force_path, LUTMOE_STAGE_ALL, stream);
}

int lutmoe_moe_forward_stages(const lutmoe_moe_desc* d, const void* x, const float* topk_w,
                              const int32_t* topk_ids, int T, int k, void* out, int out_dtype,
                              void* workspace, size_t ws_bytes, int force_path, int stages,
                              void* stream) {
    if (!topk_w || !topk_ids) return T == 0 ? LUTMOE_OK : LUTMOE_EINVAL;
    return moe_forward_impl(d, x, topk_w, topk_ids, nullptr, T, k, 0, 1.0f, out, out_dtype,
                            workspace, ws_bytes, force_path, stages, stream);
}

int lutmoe_moe_forward_logits(const lutmoe_moe_desc* d, const void* x, const float* logits,
                              int T, int k, int renormalize, float scaling, void* out,
                              int out_dtype, void* workspace, size_t ws_bytes, int force_path,
                              int stages, void* stream) {
    if (!logits) return T == 0 ? LUTMOE_OK : LUTMOE_EINVAL;
    return moe_forward_impl(d, x, nullptr, nullptr, logits, T, k, renormalize, scaling, out,
                            out_dtype, workspace, ws_bytes, force_path, stages, stream);
}

// --------------------------------------------------------------- encoders

int lutmoe_bl4_encode(const float* w, int64_t nblocks, int n_iter, uint8_t* codes,
                      uint16_t* tables_f16, void* stream) {
    if (nblocks < 0 || n_iter < 1 || n_iter > 1000) return LUTMOE_EINVAL;
    if (nblocks == 0) return LUTMOE_OK;
    if (!w || !codes || !tables_f16) return LUTMOE_EINVAL;
    return launch_bl4_encode(w, nblocks, n_iter, codes, tables_f16, stream_of(stream));
}

int lutmoe_kmeans_1d(const float* data, int64_t n, float* centroids, int k, int n_iter, int32_t* assign_ws,
                     void* stream) {
    if (n <= 0 || n >= (1ll << 31) || k < 1 || k > 256 || n_iter < 0) return LUTMOE_EINVAL;
    if (!data || !centroids || !assign_ws) return LUTMOE_EINVAL;
    return launch_kmeans_1d(data, n, centroids, k, n_iter, assign_ws, stream_of(stream));
}

int lutmoe_ref_encode(const void* w_bf16, const float* codebook, int64_t n, int block_size, uint8_t* codes,
                      void* absmax_bf16, void* stream) {
    if (n < 0 || block_size <= 0) return LUTMOE_EINVAL;
    if (n == 0) return LUTMOE_OK;
    if (!w_bf16 || !codebook || !codes || !absmax_bf16) return LUTMOE_EINVAL;
    return launch_ref_encode((const uint16_t*)w_bf16, codebook, n, block_size, codes, (uint16_t*)absmax_bf16,
                             stream_of(stream));
}

int lutmoe_ref_quantize(const void* w, int w_dtype, const float* codebook, int n_entries, int64_t n, int block_size,
                        int rule, uint8_t* codes, void* absmax_bf16, void* stream) {
    if (n < 0 || block_size <= 0) return LUTMOE_EINVAL;
    if (w_dtype != LUTMOE_DTYPE_BF16 && w_dtype != LUTMOE_DTYPE_F32) return LUTMOE_EINVAL;
    if (rule != LUTMOE_QRULE_QUANTIZER && rule != LUTMOE_QRULE_MIDPOINTS) return LUTMOE_EINVAL;
    if (n_entries < (rule == LUTMOE_QRULE_MIDPOINTS ? 2 : 1) || n_entries > 256) return LUTMOE_EINVAL;
    if (n == 0) return LUTMOE_OK;
    if (!w || !codebook || !codes || !absmax_bf16) return LUTMOE_EINVAL;
    if (!aligned(w, w_dtype == LUTMOE_DTYPE_F32 ? 4 : 2) || !aligned(codebook, 4) || !aligned(absmax_bf16, 2))
        return LUTMOE_EALIGN;
    return launch_ref_quantize(w, w_dtype == LUTMOE_DTYPE_BF16, codebook, n_entries, n, block_size, rule, codes,
                               (uint16_t*)absmax_bf16, stream_of(stream));
}

}  // extern "C"

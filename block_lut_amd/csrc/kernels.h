// Launchers of the gfx950 kernels (one translation unit per kernel family).
// Arguments are validated by api.cpp before any of these is called.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lutmoe.h"

namespace lutmoe_host {

// dequant.hip
int launch_ref_dequant(uint16_t* out, const uint8_t* idx, const uint16_t* absmax,
                       const uint16_t* cb, int64_t n_per_expert, int64_t nb_per_expert,
                       int block_size, int num_experts, int64_t out_stride,
                       int64_t idx_stride, hipStream_t s, int64_t cb_stride = 0);
int launch_merge_bitplane(uint8_t* codes, const uint8_t* plane, int64_t n, int shift, hipStream_t s);
int launch_pack_bitplanes(const uint8_t* codes, int64_t n, uint8_t* out, hipStream_t s);
int launch_bl4_dequant(uint16_t* out, const uint8_t* codes, const uint16_t* tables,
                       int64_t nblocks, hipStream_t s);
int launch_nested_dequant(uint16_t* out, const lutmoe_weights* w, int e0, int ne,
                          hipStream_t s);
int launch_ref_quantize(const void* w, bool bf16_in, const float* codebook, int ncb, int64_t n, int block_size,
                        int rule, uint8_t* codes, uint16_t* absmax, hipStream_t s);
int launch_nested_group_planes(const uint8_t* planes, int bits, int64_t n, uint8_t* out, hipStream_t s);
int launch_f16_to_bf16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t s);
int launch_unpack_4bit_inplace(uint8_t* data, int64_t n, hipStream_t s);
int launch_unpack_6bit(const uint8_t* packed, uint8_t* out, int64_t n, hipStream_t s);

// gemv.hip
// dequant: y = x . bf16(cb * absmax) (fused_lut_gemv); else lut_gemv's
// (x * cb) * absmax products
int launch_ref_gemv(const uint16_t* x, const uint8_t* idx, const uint16_t* cb_bf16,
                    const float* cb_f32, const uint16_t* absmax, void* y, int M, int K,
                    int T, int num_blocks, int block_size, int y_dtype, hipStream_t s,
                    bool dequant = false);
// BL4 and REF weights; x bf16, or fp32 when x_f32
int launch_bl4_gemv(const lutmoe_weights* w, int expert, const void* x, bool x_f32, int T, void* y,
                    int y_dtype, hipStream_t s);
int launch_nested_gemv(const lutmoe_weights* w, int expert, const uint16_t* x, int T,
                       void* y, int y_dtype, hipStream_t s);

// Routing of the grouped MFMA path.  Pairs are (token, slot) with k_eff =
// k + num_shared slots per token; positions are permuted pairs.
struct MoeRouting {
    const int32_t* offsets;   // [E_tot+1]
    const int32_t* perm;      // [P] pair index at each position
    const int32_t* inv;       // [P] position of each pair
    const int32_t* active;    // [1 + E_tot]: count, then active expert ids
    const float* pair_w;      // [P] routing weight of each pair (by pair index)
    int T;
    int k_eff;
    int num_experts_total;    // E + S
    int32_t* sched;           // [4] item and finished-CTA counters of the gate/up and down ring kernels
                              // (zeroed by the routing, and by each ring launch's last CTA)
};

// api.cpp: the body shared by the MoE layer entry points (arguments as
// lutmoe_moe_forward_stages, logits instead of topk_w/topk_ids when given),
// and the calling thread's lutmoe_last_error text.
int moe_forward_impl(const lutmoe_moe_desc* d, const void* x, const float* topk_w,
                     const int32_t* topk_ids, const float* logits, int T, int k, int renorm,
                     float scaling, void* out, int out_dtype, void* workspace, size_t ws_bytes,
                     int force_path, int stages, void* stream);
void set_last_error_text(const char* text);

// decode.hip (BL4 decode layer, routing recomputed inside each CTA)
bool decode_v2_supported(const lutmoe_moe_desc* d, int T, int k);
size_t decode_route_bytes();
// addend: NULL or fp32 [T][H] added to each output before its rounding
int launch_decode_v2(const lutmoe_moe_desc* d, const uint16_t* x, const float* topk_w,
                     const int32_t* topk_ids, const float* logits, int T, int k, int renorm,
                     float scaling, uint16_t* act, void* route_ws, float* y_ws, void* out,
                     int out_dtype, int stages, hipStream_t s, const float* addend = nullptr);

// dense.hip: a dense bf16 shared expert (d->dense_inter > 0).  gate_up:
// tokw[t] = the shared weight of token t, act [T][Is] bf16; down: y [T][H]
// fp32 = tokw[t] * (act[t] . W2s^T).  mfma: the MFMA tiles, else GEMVs.
int launch_dense_gate_up(const lutmoe_moe_desc* d, const uint16_t* x, int T, bool mfma, uint16_t* act,
                         float* tokw, hipStream_t s);
int launch_dense_down(const lutmoe_moe_desc* d, const uint16_t* act, int T, bool mfma, const float* tokw, float* y,
                      hipStream_t s);

// decode.hip: the one-token layer's weight loads alone (HBM floor measurement)
size_t decode_stream_probe_ctas(const lutmoe_moe_desc* d, int ns, int which);
int launch_decode_stream_probe(const lutmoe_moe_desc* d, const int32_t* ids, int ns, int which, uint32_t* sink,
                               hipStream_t s);

// route.hip
int launch_route_topk(const float* logits, int T, int E, int k, int renorm, float scaling,
                      float* w, int32_t* ids, hipStream_t s);
int launch_build_pairs(const int32_t* topk_ids, const float* topk_w, int T, int k,
                       int E, int S, int32_t* pair_ids, float* pair_w, hipStream_t s);
int launch_permute(const int32_t* pair_ids, int T, int k_eff, int E_tot, int32_t* offsets,
                   int32_t* perm, int32_t* inv, int32_t* active, hipStream_t s);
// pairs built from top-k ids (+ S shared slots per token), permuted, and
// their ids / weights written to pair_ids / pair_w
int launch_route_pairs(const int32_t* topk_ids, const float* topk_w, int T, int k, int E, int S,
                       int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* active, int32_t* pair_ids,
                       float* pair_w, hipStream_t s, int32_t* sched = nullptr);
// shared slots k..k+S-1 of every token t: pair_w = sigmoid(x_t . gate)
int launch_shared_gate(const uint16_t* x, const uint16_t* gate, int T, int H, int k, int S, float* pair_w,
                       hipStream_t s);
// router logits[t][e] = x[t] . gate[e] (fp32 accumulation; round_bf16: the
// sum rounded to bf16, stored as fp32)
int launch_router_logits(const uint16_t* x, const uint16_t* gate, int T, int H, int E, float* logits,
                         int round_bf16, hipStream_t s);
// nsplit > 1: y_pos holds nsplit partial results (K splits of the down
// projection), split_stride floats apart, summed per position first.
// addend: NULL or fp32 [T][H] added to each token's sum before the rounding.
int launch_combine(const float* y_pos, const int32_t* inv, int T, int k_eff, int H,
                   void* out, int out_dtype, hipStream_t s, int nsplit = 1, int64_t split_stride = 0,
                   const float* addend = nullptr);

// gemm.hip (prefill, MFMA)
int launch_prefill_gate_up(const lutmoe_moe_desc* d, const uint16_t* x, const MoeRouting& r,
                           uint16_t* act, int P, hipStream_t s);
// y_pos holds room for max_split partial results of P x H floats; *nsplit
// returns how many K splits ran (combine sums them).
int launch_prefill_down(const lutmoe_moe_desc* d, const uint16_t* act, const MoeRouting& r,
                        float* y_pos, int P, int max_split, int* nsplit, hipStream_t s);

// encode.hip
int launch_bl4_encode(const float* w, int64_t nblocks, int n_iter, uint8_t* codes,
                      uint16_t* tables, hipStream_t s);
int launch_kmeans_1d(const float* x, int64_t n, float* cent, int k, int n_iter, int32_t* asg, hipStream_t s);
int launch_ref_encode(const uint16_t* w, const float* codebook, int64_t n, int block_size, uint8_t* codes,
                      uint16_t* absmax, hipStream_t s);

}  // namespace lutmoe_host

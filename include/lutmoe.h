/*
 * lutmoe.h -- C ABI of the MI355X (gfx950) LUT-dequant MoE expert library
 * (block_lut_amd/liblutmoe.so).
 *
 * Plain pointers and sizes only.  Every pointer argument named *_dev is a
 * device pointer; `stream` is a hipStream_t passed as void* (NULL = the
 * default stream).  All entry points are asynchronous on `stream` and never
 * synchronise the device.  Argument validation happens before any HIP call,
 * so an invalid call returns an error code without touching the GPU.
 *
 * Return convention of the int-returning functions: 0 = success, negative =
 * one of the LUTMOE_E* codes below (lutmoe_strerror gives the text).
 *
 * Formats (device layouts):
 *   REF  : codes uint8 [E][M][K] (one code per weight), absmax bf16 [E][nb]
 *          with nb = ceil(M*K/block_size) per expert, codebook bf16[256].
 *   BL4  : codes uint8 [E][M][K/2] (two 4-bit codes per byte, even element in
 *          the low nibble), tables bf16 [E][M][K/64][16] (the dequantised
 *          entries; lutmoe_bl4_tables_from_f16 converts the fp16 codebooks).
 *   NL   : NestedLUT tier b in {2,3,4} per expert.  Stored (and loaded
 *          progressively) as bit-plane sections [p01 M*K/4 | p2 M*K/8 |
 *          p3 M*K/8] (a tier-b expert holds the first 2, 3 or all sections);
 *          on the device the codes are grouped: each 32 consecutive weights
 *          of the flat row-major [M][K] order (w_j = code of weight j) are
 *          the first b of four little-endian uint32 words -- f0: nibble n =
 *          (w_n & 3) | (w_{n+8} & 3) << 2; f1: the same for w_{n+16},
 *          w_{n+24}; b2: nibble n bit q = bit 2 of w_{n+8q} (b >= 3); b3:
 *          bit 3 likewise (b = 4) -- 4b bytes per group, M*K*b/8 per expert
 *          (lutmoe_nested_group_planes converts).  Tables bf16 [M][K/64][2^b].
 */
#ifndef LUTMOE_H
#define LUTMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes ---------------------------------------------------- */
#define LUTMOE_OK             0
#define LUTMOE_EINVAL        -1   /* bad argument (null pointer, size, dtype) */
#define LUTMOE_EUNSUPPORTED  -2   /* valid but unsupported combination        */
#define LUTMOE_EHIP          -3   /* a HIP runtime call failed                */
#define LUTMOE_EWORKSPACE    -4   /* workspace too small                      */
#define LUTMOE_EALIGN        -5   /* pointer misaligned for vector access     */

/* ---- formats and dtypes ---------------------------------------------- */
#define LUTMOE_FMT_REF        0
#define LUTMOE_FMT_BL4        1
#define LUTMOE_FMT_NESTED     2

#define LUTMOE_DTYPE_BF16     0
#define LUTMOE_DTYPE_F32      1

/* One stack of per-expert LUT-quantised matrices W[e] of shape [rows, cols]
 * (rows = output features, cols = K = input features). */
typedef struct lutmoe_weights {
    int32_t format;            /* LUTMOE_FMT_*                                   */
    int32_t num_experts;       /* E                                              */
    int32_t rows;              /* M                                              */
    int32_t cols;              /* K                                              */
    const void* codes;         /* REF/BL4: device base of [E] code arrays.
                                  NL: device array of E pointers (uint8_t*) to
                                  each expert's grouped codes (M*K*b/8 bytes).   */
    const void* tables;        /* REF: bf16 absmax [E][absmax_per_expert].
                                  BL4: bf16 tables [E][M][K/64][16].
                                  NL: device array of E pointers (uint16_t*) to
                                  each expert's bf16 table [M][K/64][2^b].       */
    const void* codebook;      /* REF: bf16[256] codebook(s); else NULL.         */
    const int8_t* tier_bits;   /* NL: device int8 [E] with b in {2,3,4}.         */
    int64_t absmax_per_expert; /* REF: absmax entries per expert.                */
    int32_t block_size;        /* REF: absmax block (reference default 128).     */
    int32_t codebook_stride;   /* REF: 0 = one codebook for every expert (the
                                  reference's model._codebook); else >= 256:
                                  expert e uses codebook + e*codebook_stride,
                                  i.e. the table of its own tier
                                  (csrc/tensor_engine/tensor_engine.hpp:287-291
                                  selects it per expert node).                 */
} lutmoe_weights;

/* Fused-MoE layer description: routed experts 0..E-1, plus num_shared
 * always-on expert slots stored after them (expert ids E..E+S-1 of the same
 * stacks).  A shared expert whose intermediate size is m*I occupies m slots
 * (gate/up rows and down columns split at multiples of I: SwiGLU acts per
 * intermediate index, so the slots' outputs sum to the expert's).  Every
 * shared slot of token t is applied with weight 1.0 (DeepSeek,
 * customized/deepseek.py:111-115), or, when shared_gate is set, with
 * sigmoid(x[t] . shared_gate) computed in fp32 (Qwen's shared_expert_gate,
 * customized/qwen.py:42-43, 99-100). */
typedef struct lutmoe_moe_desc {
    lutmoe_weights w13;        /* [E+S][2I][H]: gate rows [0,I), up rows [I,2I) */
    lutmoe_weights w2;         /* [E+S][H][I]                                   */
    int32_t hidden;            /* H                                             */
    int32_t inter;             /* I                                             */
    int32_t num_routed;        /* E                                             */
    int32_t num_shared;        /* S                                             */
    const void* shared_gate;   /* bf16 [H] (device) or NULL                     */
    /* Optional dense bf16 shared expert, as the reference keeps a model's
     * shared experts (bf16 linears beside the LUT experts,
     * vllm_lut/moe_layer.py:186-200, 348-353; customized/qwen.py:40-43,
     * 96-100): dense_inter = its intermediate size Is (0 = none; Is % 64 ==
     * 0), dense_w13 bf16 [2 Is][H] (gate rows [0, Is), up rows [Is, 2 Is)),
     * dense_w2 bf16 [H][Is], both row-major and 16-byte aligned.  Every token
     * adds w * W2s . bf16(silu(Wg x) * (Wu x)) with w = 1, or
     * sigmoid(x . shared_gate) when shared_gate is set (it then weighs the
     * LUT shared slots too), to its sum of expert outputs before the one
     * rounding of the result.  Decode runs it as bf16 GEMVs, prefill on MFMA. */
    int32_t dense_inter;
    int32_t dense_reserved;    /* 0 */
    const void* dense_w13;
    const void* dense_w2;
} lutmoe_moe_desc;

/* ---- library ---------------------------------------------------------- */
const char* lutmoe_strerror(int code);
const char* lutmoe_version(void);
/* Last error text recorded on the calling thread by a void-returning
 * reference-compatible entry point or by lutmoe_moe_forward_noalloc ("" when
 * none).  After any entry point returns LUTMOE_EHIP it names the HIP error
 * ("HIP runtime error: hipErrorName (description)"). */
const char* lutmoe_last_error(void);

/* ---- reference-compatible entry points --------------------------------
 * Same names, argument meaning and error behaviour as the reference's
 * native surface (asynchronous here: no device synchronisation). */

/* vllm_lut/cuda/lut_decompress_kernel.cu:125-154.
 * out[i] = bf16(cb[idx[i]] * absmax[i / block_size]); 0 ok, -1 on error. */
int launch_blocklut_decompress(void* output, const void* indices, const void* absmax,
                               const void* codebook, int N, int block_size, void* stream);

/* vllm_lut/cuda/lut_decompress_kernel.cu:156-180 (any elements_per_expert;
 * the reference's one-thread-per-element launch is limited to 1024). */
int launch_batch_blocklut_decompress(void* output, const void* indices, const void* absmax,
                                     const void* codebook, int num_experts,
                                     int elements_per_expert, int blocks_per_expert,
                                     int block_size, void* stream);

/* csrc/kernels/tensor_recover.hpp (lut_moe_launch_blocklut_recover,
 * tensor_recover.cu:144-159): 128-element absmax blocks, bf16 out. */
void lut_moe_launch_blocklut_recover(uint16_t* gpu_output_tensor,
                                     const uint8_t* gpu_indices_ptr,
                                     const uint16_t* gpu_absmax_ptr,
                                     const uint16_t* gpu_lut_ptr,
                                     size_t num_elements, void* tensor_stream);

/* csrc/kernels/tensor_recover.hpp (lut_moe_launch_unpack_4bit,
 * tensor_recover.cu:182-192): in place, the first n/2 bytes (low nibble
 * section) become n one-byte codes. */
void lut_moe_launch_unpack_4bit(uint8_t* gpu_data, size_t num_elements, void* tensor_stream);

/* vllm_lut/cuda_lut_gemv.py:119-135 (launch_lut_gemv_kernel): fp32 codebook
 * [256], bf16 input [K], uint8 indices [M][K], bf16 absmax [num_blocks]
 * (128-element blocks), bf16 output [M]; default stream. */
void launch_lut_gemv_kernel(const void* input, const void* indices, const void* codebook,
                            const void* absmax, void* output, int M, int K, int num_blocks);

/* ---- REF format ----------------------------------------------------------- */

/* lut_gemv (vllm_lut/cuda_lut_gemv.py:153-169) with a bf16 codebook and an
 * explicit stream.  y[T][M] (dtype y_dtype) = sum_k x[T][K] * cb[idx]*absmax,
 * fp32 accumulation in the reference's (x*cb)*absmax product order. */
int lutmoe_ref_gemv(const void* x_dev, const void* indices_dev, const void* codebook_dev,
                    const void* absmax_dev, void* y_dev, int M, int K, int T,
                    int num_blocks, int block_size, int y_dtype, void* stream);

/* fused_lut_gemv (vllm_lut/fused_kernel.py:13-46): the dequantised weights
 * W = bf16(cb[idx] * absmax[min(i / block_size, num_blocks - 1)]) (i the
 * flat row-major index) times each of the T vectors: y[T][M] (y_dtype) =
 * x[T][K] . W^T with fp32 accumulation.  Arguments as lutmoe_ref_gemv. */
int lutmoe_fused_lut_gemv(const void* x_dev, const void* indices_dev, const void* codebook_dev,
                          const void* absmax_dev, void* y_dev, int M, int K, int T, int num_blocks,
                          int block_size, int y_dtype, void* stream);

/* CPU-side tier unpack of the reference, on the GPU (csrc/tensor_engine/
 * tensor_engine.cpp:535-548): 6-bit codes = low nibble | mid 2 bits << 4 from
 * the [low | mid] sections of `packed`, written to `out` (n bytes). */
int lutmoe_unpack_6bit(const uint8_t* packed_dev, uint8_t* out_dev, int64_t n, void* stream);

/* Bit-plane packing (llama-cpp-port/scripts/convert_lut.py:95-110,
 * runtime/model_offload.py:747-766), the inverse of the unpacks above:
 * codes_dev[n] (one byte per code) -> packed_dev[n] = [low nibbles n/2 |
 * bits 4-5 n/4 | bits 6-7 n/4]; low byte i = code 2i | code 2i+1 << 4, mid /
 * high byte i holds code 4i+k in bits 2k..2k+1.  n % 4 == 0. */
int lutmoe_pack_bitplanes(const uint8_t* codes_dev, int64_t n, uint8_t* packed_dev, void* stream);

/* NestedLUT plane sections of one tier-b expert (planes_dev: the tier's
 * prefix of [p01 n/4 | p2 n/8 | p3 n/8]) -> its device codes out_dev
 * (n*b/8 bytes, the group words described at the top of this file).
 * n = M*K weights, n % 64 == 0; both pointers 4-byte aligned.  No
 * counterpart in the reference, whose 4/6/8-bit sections are merged into
 * byte codes on load (csrc/tensor_engine/tensor_engine.cpp:535-548): the
 * grouped order lets a kernel read a weight group in one load and turn 8 of
 * its codes into a 4-bit code word with one shift and mask per word. */
int lutmoe_nested_group_planes(const uint8_t* planes_dev, int bits, int64_t n, uint8_t* out_dev, void* stream);

/* Progressive tier upgrade of resident codes (the reference reloads the whole
 * expert on a promotion, csrc/topology/model_topology.cpp:74-80, reading
 * the tier's prefix of the bit-plane file, tensor_engine.cpp:504-510): in
 * place, code i of codes_dev[n] takes the 2-bit field
 * (plane[i/4] >> 2*(i%4)) & 3 at bits [shift, shift+2), replacing them.
 * plane_dev holds n/4 bytes laid out as a BLOCKLUT8 mid/high section
 * (llama-cpp-port/scripts/convert_lut.py:95-110).  shift 4: tier 2 -> 1
 * (the mid section; same field rule as tensor_engine.cpp:535-548), shift 6:
 * tier 1 -> 0 (the high section).  n % 4 == 0; shift in {0, 2, 4, 6}. */
int lutmoe_merge_bitplane(uint8_t* codes_dev, const uint8_t* plane_dev, int64_t n, int shift, void* stream);

/* ---- generic (all formats) --------------------------------------------- */

/* Dequantise experts [e0, e0+ne) of a weight stack to bf16 [ne][M][K]. */
int lutmoe_dequant(const lutmoe_weights* w, int e0, int ne, void* out_dev, void* stream);

/* y[T][M] = x[T][K] . W[expert]^T for one expert (fp32 accumulation); x bf16. */
int lutmoe_gemv(const lutmoe_weights* w, int expert, const void* x_dev, int T,
                void* y_dev, int y_dtype, void* stream);

/* lutmoe_gemv with the activations' dtype given: x_dtype LUTMOE_DTYPE_BF16 or
 * LUTMOE_DTYPE_F32 (BL4 and REF weights; fp32 x: each weight widened to fp32
 * and multiplied by an fp32 FMA, REF in lut_gemv's (x * cb) * absmax order --
 * the reference's CPU dequant + F.linear on fp32 inputs,
 * vllm_lut/quantizer.py:449-477).  NestedLUT takes bf16 x only
 * (LUTMOE_EUNSUPPORTED). */
int lutmoe_gemv_ex(const lutmoe_weights* w, int expert, const void* x_dev, int x_dtype, int T,
                   void* y_dev, int y_dtype, void* stream);

/* BL4 repack: fp16 codebook entries -> bf16 dequantised entries. */
int lutmoe_bl4_tables_from_f16(const uint16_t* f16_dev, uint16_t* bf16_dev, int64_t n,
                               void* stream);

/* ---- routing and permutation ------------------------------------------ */

/* softmax(fp32 logits [T][E]) -> top-k (sorted descending, ties to the lower
 * id), optional renormalisation, times `scaling`; weights fp32 [T][k],
 * ids int32 [T][k] (vllm_lut/moe_layer.py:358-376).  NaN logits are never
 * selected; a round with only NaN left gives id -1 and weight 0.
 * E <= 4096 (larger E: LUTMOE_EUNSUPPORTED). */
int lutmoe_route_topk(const float* logits_dev, int T, int E, int k, int renormalize,
                      float scaling, float* topk_w_dev, int32_t* topk_ids_dev, void* stream);

/* Router gate (MoEGate.forward, models/deepseek/modeling_deepseek.py:423-470;
 * the bf16 gate linear of vllm_lut/moe_layer.py:301-304): logits[t][e] =
 * x[t] . gate[e] over H with fp32 accumulation; round_bf16 != 0 rounds each
 * logit to bf16 (the vLLM layer's logits dtype), stored as fp32.  x bf16
 * [T][H], gate bf16 [E][H] (both 16-byte aligned, H % 8 == 0), logits fp32
 * [T][E]; T <= 65535.  Sized for decode batches (one wave per logit). */
int lutmoe_router_logits(const void* x_dev, const void* gate_dev, int T, int H, int E, float* logits_dev,
                         int round_bf16, void* stream);

/* Expert-major, pair-ascending permutation of the T*k (token, slot) pairs.
 * offsets int32 [E+1], perm int32 [T*k] (pair index t*k+slot at each
 * position), inv int32 [T*k] (position of each pair), active int32 [E+1]
 * (active[0] = number of experts with tokens, then their ids ascending). */
int lutmoe_permute(const int32_t* topk_ids_dev, int T, int k, int E, int32_t* offsets_dev,
                   int32_t* perm_dev, int32_t* inv_dev, int32_t* active_dev, void* stream);

/* ---- fused MoE layer ------------------------------------------------------ */

/* Workspace bytes lutmoe_moe_forward needs for T tokens and top-k.
 * The workspace is device memory, 256-byte aligned, owned by the caller; its
 * contents need no initialisation (every kernel writes what it reads within
 * the call).  Calls that overlap in time must not share a workspace. */
size_t lutmoe_moe_workspace_size(const lutmoe_moe_desc* d, int T, int k);

/* out[T][H] (out_dtype) = sum_k topk_w[t][k] * FFN_{ids[t][k]}(x[t])
 *                         + sum_s FFN_{E+s}(x[t]),
 * FFN(x) = W2 . bf16(silu(W13_gate x) * (W13_up x)), fp32 accumulation.
 * x bf16 [T][H]; topk_w fp32 [T][k]; topk_ids int32 [T][k] in [0, E).
 * Decode (small T) uses the grouped LUT-GEMV kernels, prefill the grouped
 * MFMA LUT-GEMM; `force_path` 0 = auto, 1 = GEMV, 2 = MFMA. */
int lutmoe_moe_forward(const lutmoe_moe_desc* d, const void* x_dev, const float* topk_w_dev,
                       const int32_t* topk_ids_dev, int T, int k, void* out_dev,
                       int out_dtype, void* workspace_dev, size_t workspace_bytes,
                       int force_path, void* stream);

/* lutmoe_moe_forward without a workspace argument: the layer's scratch is a
 * file-scope device array of the library, 32 MiB per GPU, held until the
 * process ends; the call allocates nothing (no hipMalloc, hipFree or
 * allocating library routine).  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  A layer whose
 * workspace (lutmoe_moe_workspace_size) exceeds 32 MiB is rejected with
 * LUTMOE_EWORKSPACE and a lutmoe_last_error text giving the sizes.  Every call
 * on one GPU shares that GPU's scratch, which keeps the last call's contents:
 * calls that overlap in time on one GPU race (serialise them, e.g. on one
 * stream).  The scratch's address on a device is looked up once, by
 * lutmoe_noalloc_prepare or else by the first call there; that lookup may load
 * the library's code object, so code that captures calls into a HIP graph
 * calls lutmoe_noalloc_prepare (or one lutmoe_moe_forward_noalloc) on the
 * device before it starts capturing. */
int lutmoe_noalloc_prepare(void);   /* current device; 0 or LUTMOE_EHIP */
int lutmoe_moe_forward_noalloc(const lutmoe_moe_desc* d, const void* x_dev, const float* topk_w_dev,
                               const int32_t* topk_ids_dev, int T, int k, void* out_dev, int out_dtype,
                               int force_path, void* stream);

/* Stage bits of lutmoe_moe_forward_stages. */
#define LUTMOE_STAGE_ROUTE    1   /* pair build + permutation into the workspace   */
#define LUTMOE_STAGE_GATE_UP  2   /* gate/up LUT-GEMV or GEMM + SwiGLU -> act      */
#define LUTMOE_STAGE_DOWN     4   /* down projection + weighted combine -> out     */
#define LUTMOE_STAGE_ALL      7

/* lutmoe_moe_forward restricted to some stages; a later stage reads what an
 * earlier call left in the same workspace (same T, k, routing).  Used to time
 * each kernel family on its own. */
int lutmoe_moe_forward_stages(const lutmoe_moe_desc* d, const void* x_dev, const float* topk_w_dev,
                              const int32_t* topk_ids_dev, int T, int k, void* out_dev,
                              int out_dtype, void* workspace_dev, size_t workspace_bytes,
                              int force_path, int stages, void* stream);

/* The MoE block forward from router logits (DeepseekV2MoE_LUT.forward,
 * vllm_lut/moe_layer.py:281-355): softmax(fp32 logits [T][E]) -> top-k
 * (ties to the lower id) -> optional renormalisation -> x scaling -> the
 * layer of lutmoe_moe_forward.  On the decode path the routing runs inside
 * decode layer kernel (one launch per layer at T <= 2). */
int lutmoe_moe_forward_logits(const lutmoe_moe_desc* d, const void* x_dev, const float* logits_dev,
                              int T, int k, int renormalize, float scaling, void* out_dev,
                              int out_dtype, void* workspace_dev, size_t workspace_bytes,
                              int force_path, int stages, void* stream);

/* ---- measurement ---------------------------------------------------------- */

/* The HBM floor of the one-token BL4 layer (no counterpart in the reference;
 * for benchmarks): one launch whose CTAs issue the same weight loads as the
 * one-token kernels (which = 1: the gate/up kernel's grid and W13 rows,
 * 2: the down kernel's grid and W2 rows, 3: both in one launch) for expert
 * ids_dev[y] of each slot (int32 [k + num_shared], shared slots included;
 * clamped into the stacks) and only fold the loaded words into
 * sink_dev[lutmoe_decode_stream_probe_sink_words(d, k, which)] (uint32).
 * BL4, H and I <= 2048, k + num_shared <= 64. */
size_t lutmoe_decode_stream_probe_sink_words(const lutmoe_moe_desc* d, int k, int which);
int lutmoe_decode_stream_probe(const lutmoe_moe_desc* d, const int32_t* ids_dev, int k, int which,
                               uint32_t* sink_dev, void* stream);

/* ---- encoders (format producers) ----------------------------------------- */

/* BL4 per-64-block k-means encoder on the GPU: w fp32 [nblocks*64] ->
 * packed codes [nblocks*32] and fp16 tables [nblocks*16]. */
int lutmoe_bl4_encode(const float* w_dev, int64_t nblocks, int n_iter, uint8_t* codes_dev,
                      uint16_t* tables_f16_dev, void* stream);

/* REF encoder, replacing encode_blocklut_kernel / launch_encode
 * (vllm_lut/fast_encode.py:22-72, 80-99): bf16 weights [n] and an fp32[256]
 * codebook -> uint8 codes [n] (nearest entry of w / absmax, first index on
 * equal distances) and bf16 absmax [ceil(n / block_size)] (max |w| of each
 * block of block_size weights, at least 1e-10).  Asynchronous on `stream`
 * (the reference synchronises the device after the launch); IEEE division
 * (the reference builds with fast math). */
int lutmoe_ref_encode(const void* w_bf16_dev, const float* codebook_dev, int64_t n, int block_size,
                      uint8_t* codes_dev, void* absmax_bf16_dev, void* stream);

/* The reference's other two REF encoding rules (codes and bf16 absmax as
 * lutmoe_ref_encode; blocks of block_size weights, the last one shorter):
 *   LUTMOE_QRULE_QUANTIZER: LUTQuantizer.quantize (vllm_lut/quantizer.py:
 *     242-306; block_size = n gives its global "LUT" branch): absmax = max |w|
 *     in the weights' dtype, at least 1e-10; w / absmax rounded to bf16 when
 *     the weights are bf16 (:284); code = first nearest of the n_entries
 *     codebook values (fp32 [n_entries], any order) by |v - c|.
 *   LUTMOE_QRULE_MIDPOINTS: the offload runtime's encoder
 *     (runtime/model_offload.py:897-907): fp32 division, absmax at least
 *     1e-12; code = number of fp32 midpoints (c_i + c_{i+1}) / 2 of the
 *     ascending codebook (fp32 [n_entries], n_entries >= 2) below v (a value
 *     on a midpoint takes the lower entry, NaN the last).
 * w_dev: bf16 or fp32 [n] (w_dtype); n_entries <= 256. */
#define LUTMOE_QRULE_QUANTIZER 0
#define LUTMOE_QRULE_MIDPOINTS 1
int lutmoe_ref_quantize(const void* w_dev, int w_dtype, const float* codebook_dev, int n_entries, int64_t n,
                        int block_size, int rule, uint8_t* codes_dev, void* absmax_bf16_dev, void* stream);

/* The Lloyd iterations of LUTQuantizer._train_kmeans (vllm_lut/quantizer.py:
 * 158-173) on the device: n_iter rounds of "each sample joins its nearest
 * centroid by |x - c| (first on equal distances), each centroid with members
 * becomes their mean".  data: fp32 [n] (the training samples, already
 * subsampled); centroids: fp32 [k] in (the initial pick) and out; k <= 256;
 * assign_ws: int32 [n] scratch.  Sums run in a fixed order (results do not
 * depend on scheduling); they differ from torch's own summation order in the
 * last bits.  Sorting and the bf16 store (:176-177) are left to the caller. */
int lutmoe_kmeans_1d(const float* data_dev, int64_t n, float* centroids_dev, int k, int n_iter,
                     int32_t* assign_ws_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LUTMOE_H */

/*
 * qlin.h -- C ABI of the MI355X (gfx950) GGUF quantized-linear library (libqlin.so).
 *
 * Drop-in boundary for the quantized-linear launchers of the reference engine
 * (AI/codes/local-llm/src/backend/cuda/ops/kernel.cuh).  Each entry point keeps the reference
 * launcher's argument list and meaning, with three deliberate differences:
 *   - the weight format is an int ggml type code instead of the C++ DType enum (same values,
 *     src/tensor/TensorCommon.h:15-33);
 *   - every call returns a qlin_status (0 = launched) where the reference returns void and silently
 *     does nothing for an unsupported type (src/backend/cuda/ops/launch.cu:57);
 *   - the stream is the library's current stream, set with qlin_set_stream (the reference's
 *     set_current_cuda_stream, src/backend/cuda/common.cpp:13-17).
 *
 * Conventions (as the reference's):
 *   - all data pointers are device pointers owned by the caller; weights are resident packed GGUF
 *     bytes, row-major [out_dim, in_dim], row r at weight + r * row_bytes; activations and outputs
 *     are f32 row-major [m, in_dim] / [m, out_dim];
 *   - launches are asynchronous on the current stream; no entry point allocates device memory,
 *     synchronises or reads device data back, so all of them may be captured into a HIP graph;
 *   - validation happens on the host before any launch and needs no GPU.
 *
 * Supported weight types: Q4_0 (2), Q5_0 (6), Q8_0 (8), Q4_K (12), Q6_K (14).
 */
#ifndef QLIN_H
#define QLIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QLIN_TYPE_Q4_0 2
#define QLIN_TYPE_Q5_0 6
#define QLIN_TYPE_Q8_0 8
#define QLIN_TYPE_Q8_1 9
#define QLIN_TYPE_Q4_K 12
#define QLIN_TYPE_Q6_K 14

typedef enum qlin_status {
    QLIN_OK = 0,
    QLIN_ERR_UNSUPPORTED_TYPE = 1, /* weight type not supported by this entry point */
    QLIN_ERR_SHAPE = 2,            /* negative dimension, or in_dim not a multiple of the block */
    QLIN_ERR_NULL = 3,             /* required pointer is NULL while there is work to do */
    QLIN_ERR_ROW_BYTES = 4,        /* row / expert stride smaller than the packed data it holds */
    QLIN_ERR_LIMIT = 5,            /* argument beyond a documented limit (e.g. n_experts > 256) */
    QLIN_ERR_LAUNCH = 6,           /* the HIP runtime rejected the launch */
    QLIN_ERR_ALIGN = 7,            /* pointer misaligned for its element type */
    QLIN_ERR_IO = 8,               /* GGUF reader: the file cannot be opened or mapped */
    QLIN_ERR_FORMAT = 9,           /* GGUF reader: malformed or unsupported file contents */
    QLIN_ERR_NOT_FOUND = 10,       /* GGUF reader: no such tensor, key or index, or another value type */
    QLIN_ERR_ALLOC = 11            /* weight pool: device allocation or copy failed */
} qlin_status;

/* Human-readable name of a status code. */
const char *qlin_status_string(int status);

/* Library version, and the gfx target it was built for ("gfx950"). */
const char *qlin_version(void);

/* Stream used by every launch (a hipStream_t; NULL = the default stream).
 * Mirrors set_current_cuda_stream / get_current_cuda_stream (common.cpp:13-17). */
int qlin_set_stream(void *stream);
void *qlin_get_stream(void);

/* Block geometry of a ggml type (GgufFile.cpp:35-55); 0 for an unknown type. */
int qlin_block_elems(int type);
int qlin_block_bytes(int type);
/* Packed bytes of one row of in_dim elements; 0 if the type is unknown or in_dim is indivisible. */
size_t qlin_row_bytes(int type, int in_dim);

/* ---- decode / prefill linear (kernel.cuh:33-42) ------------------------------------------------ */

/* y[r, o] = sum_k W[o, k] x[r, k], r < m.  Replaces launch_quant_gemv (launch.cu:42-60). */
int qlin_launch_quant_gemv(int type, const uint8_t *weight, size_t row_bytes, const float *x, float *y,
                           int out_dim, int in_dim, int m);

/* y[o] += sum_k W[o, k] x[k].  Replaces launch_quant_gemv_add (launch.cu:71-89). */
int qlin_launch_quant_gemv_add(int type, const uint8_t *weight, size_t row_bytes, const float *x,
                               float *y, int out_dim, int in_dim);

/* Same contraction as qlin_launch_quant_gemv, for m > 1 (prefill with f32 activations).
 * Replaces launch_quant_matmul (launch.cu:101-119). */
int qlin_launch_quant_matmul(int type, const uint8_t *weight, size_t row_bytes, const float *x, float *y,
                             int out_dim, int in_dim, int m);

/* y[r, o] += sum_k W[o, k] x[r, k], r < m.  For m == 1 the same as qlin_launch_quant_gemv_add; for
 * m > 1 it replaces the gemm into a scratch tensor followed by TensorTool::add that the shared
 * experts run for a batch of tokens (SharedExperts.cpp:42-48). */
int qlin_launch_quant_matmul_add(int type, const uint8_t *weight, size_t row_bytes, const float *x, float *y,
                                 int out_dim, int in_dim, int m);

/* n_mats (1..4) GEMVs that share x, as one launch: ys[i][o] = W_i[o] . x for o < out_dims[i].
 * weights, ys and out_dims are host arrays of n_mats entries (the pointers they hold are device
 * pointers); all weights have the same type, in_dim and row_bytes.  No reference counterpart: the
 * reference issues one launch_quant_gemv per matrix (e.g. q, k and v of a layer); on MI355X a
 * launch costs about 2 us even when empty, so matrices that read the same x are batched. */
int qlin_launch_quant_gemv_multi(int type, int n_mats, const uint8_t *const *weights, size_t row_bytes,
                                 const float *x, float *const *ys, const int *out_dims, int in_dim);

/* ---- Q8_1 activations (kernel.cuh:46-54) ------------------------------------------------------ */

/* Bytes of one Q8_1 activation row: ceil(in_dim / 32) * 36.  Replaces q8_1_row_bytes. */
size_t qlin_q8_1_row_bytes(int in_dim);

/* Quantize m rows of in_dim f32 values to Q8_1 blocks (d f16, s f16, int8 q[32]); s = d * sum(q),
 * or the raw f32 sum when store_raw_sum != 0.  Replaces launch_quantize_q8_1 (launch.cu:201-207). */
int qlin_launch_quantize_q8_1(const float *x, uint8_t *x_q8_1, int in_dim, int m, int store_raw_sum);

/* y[r, o] = W[o] . x_q8_1[r] with block-dot semantics (kernel.cu:2305-2402).
 * Replaces launch_quant_matmul_q8_1 (launch.cu:500-531). */
int qlin_launch_quant_matmul_q8_1(int type, const uint8_t *weight, size_t row_bytes, const uint8_t *x_q8_1,
                                  float *y, int out_dim, int in_dim, int m);

/* qlin_launch_quant_matmul_q8_1 for one row.  Replaces launch_quant_gemv_q8_1 (launch.cu:226-246). */
int qlin_launch_quant_gemv_q8_1(int type, const uint8_t *weight, size_t row_bytes, const uint8_t *x_q8_1, float *y,
                                int out_dim, int in_dim);

/* Q8_1 blocks in the group-major MMQ layout: the ceil(in_dim / 128) groups of 128 values of row r
 * at (g * m + r) * 144 bytes = 4 x (d f16, s f16) then 4 x 32 int8 (values past in_dim are 0).
 * Replaces launch_quantize_q8_1_mmq (launch.cu:209-215). */
int qlin_launch_quantize_q8_1_mmq(const float *x, uint8_t *x_q8_1, int in_dim, int m, int store_raw_sum);

/* y[r, o] = W[o] . x_q8_1[r] from the MMQ layout, block-dot semantics; Q4_K and Q6_K.
 * Replaces launch_quant_matmul_q8_1_mmq (launch.cu:546-560). */
int qlin_launch_quant_matmul_q8_1_mmq(int type, const uint8_t *weight, size_t row_bytes, const uint8_t *x_q8_1,
                                      float *y, int out_dim, int in_dim, int m);

/* ---- MoE decode (kernel.cuh:62-129, 335-336) --------------------------------------------------- */

/* act[o] = silu(Wg[o].x) * (Wu[o].x).  Replaces launch_quant_swiglu (launch.cu:132-154). */
int qlin_launch_quant_swiglu(int type, const uint8_t *gate_weight, const uint8_t *up_weight,
                             size_t gate_row_bytes, size_t up_row_bytes, const float *x, float *act,
                             int ffn_dim, int in_dim);

/* act[r, o] = silu(Wg[o].x[r]) * (Wu[o].x[r]) for m rows of x ([m, in_dim]) into act ([m, ffn_dim]).
 * For m == 1 the same as qlin_launch_quant_swiglu; for m > 1 it replaces the two gemms and silu_mul
 * of the shared experts over a batch of tokens (SharedExperts.cpp:34-40). */
int qlin_launch_quant_swiglu_rows(int type, const uint8_t *gate_weight, const uint8_t *up_weight,
                                  size_t gate_row_bytes, size_t up_row_bytes, const float *x, float *act,
                                  int ffn_dim, int in_dim, int m);

/* act[r, o] for route r on expert expert_ids[r] (device array; id < 0 writes 0).
 * Replaces launch_quant_swiglu_indexed (launch.cu:170-189). */
int qlin_launch_quant_swiglu_indexed(int type, const uint8_t *gate_weight, const uint8_t *up_weight,
                                     size_t gate_expert_bytes, size_t up_expert_bytes,
                                     size_t gate_row_bytes, size_t up_row_bytes, const float *x,
                                     const int *expert_ids, float *act, int k, int ffn_dim, int in_dim);

/* The reference's block-factored form of qlin_launch_quant_swiglu_indexed (the same contraction,
 * Q4_K and Q6_K; fast_silu is ignored, as the reference kernel ignores it).
 * Replaces launch_quant_swiglu_indexed_block (launch.cu:262-283). */
int qlin_launch_quant_swiglu_indexed_block(int type, const uint8_t *gate_weight, const uint8_t *up_weight,
                                           size_t gate_expert_bytes, size_t up_expert_bytes, size_t gate_row_bytes,
                                           size_t up_row_bytes, const float *x, const int *expert_ids, float *act,
                                           int k, int ffn_dim, int in_dim, int fast_silu);

/* act[r, o] = silu(Wg[e_r][o] . x_q8_1) * (Wu[e_r][o] . x_q8_1) (block-dot semantics, one Q8_1 row
 * x shared by the routes; id < 0 writes 0); Q4_K and Q6_K.
 * Replaces launch_quant_swiglu_indexed_q8_1 (launch.cu:298-318). */
int qlin_launch_quant_swiglu_indexed_q8_1(int type, const uint8_t *gate_weight, const uint8_t *up_weight,
                                          size_t gate_expert_bytes, size_t up_expert_bytes, size_t gate_row_bytes,
                                          size_t up_row_bytes, const uint8_t *x_q8_1, const int *expert_ids,
                                          float *act, int k, int ffn_dim, int in_dim);

/* out[h] += route_weights[r] * (Wd[e_r][h] . act_q8_1[r]) for each route with e_r >= 0, act_q8_1 k
 * Q8_1 rows of ffn_dim; the routes are added in route order (the reference adds them with atomics
 * in any order, of which this is one).  Replaces launch_quant_down_q8_1_indexed_accum (launch.cu:333-364). */
int qlin_launch_quant_down_q8_1_indexed_accum(int type, const uint8_t *down_weight, size_t down_expert_bytes,
                                              size_t down_row_bytes, const uint8_t *act_q8_1, const int *expert_ids,
                                              const float *route_weights, float *out, int k, int hidden_size,
                                              int ffn_dim);

/* The same contraction.  Replaces launch_quant_down_q8_1_indexed_accum_shared (launch.cu:379-409). */
int qlin_launch_quant_down_q8_1_indexed_accum_shared(int type, const uint8_t *down_weight, size_t down_expert_bytes,
                                                     size_t down_row_bytes, const uint8_t *act_q8_1,
                                                     const int *expert_ids, const float *route_weights, float *out,
                                                     int k, int hidden_size, int ffn_dim);

/* The same from f32 act [k, ffn_dim]: each route's act is quantized to Q8_1 (s = d * sum(q)) and
 * then dotted; (ffn_dim / 32) * 36 bytes must fit the 160 KiB of LDS.
 * Replaces launch_quant_down_f32_indexed_accum (launch.cu:425-455). */
int qlin_launch_quant_down_f32_indexed_accum(int type, const uint8_t *down_weight, size_t down_expert_bytes,
                                             size_t down_row_bytes, const float *act, const int *expert_ids,
                                             const float *route_weights, float *out, int k, int hidden_size,
                                             int ffn_dim);

/* out[h] += sum_r route_weights[r] * (Wd[e_r][h] . act[r]), routes in order, negative ids skipped.
 * Replaces launch_quant_down_f32_indexed_accum_ordered (launch.cu:469-498). */
int qlin_launch_quant_down_f32_indexed_accum_ordered(int type, const uint8_t *down_weight,
                                                     size_t down_expert_bytes, size_t down_row_bytes,
                                                     const float *act, const int *expert_ids,
                                                     const float *route_weights, float *out, int k,
                                                     int hidden_size, int ffn_dim);

/* Softmax top-k router: top_idx[t, r], top_w[t, r] = p * routed_scaling (n_experts <= 256).
 * Replaces launch_moe_router_topk (kernel.cu:3463-3511). */
int qlin_launch_moe_router_topk(const float *router_logits, int *top_idx, float *top_w, int tokens,
                                int n_experts, int k, float routed_scaling);

/* out[i] += weight * expert_out[i] (one expert's output into the MoE sum).
 * Replaces launch_moe_accumulate (kernel.cuh:339, kernel.cu:3514-3518). */
int qlin_launch_moe_accumulate(const float *expert_out, float weight, float *out, int n);

/* The same with the weight read on the device (*weight), so routing weights need not come back to
 * the host.  Replaces launch_moe_accumulate_device (kernel.cuh:342, kernel.cu:3522-3526). */
int qlin_launch_moe_accumulate_device(const float *expert_out, const float *weight, float *out, int n);

/* out_idx[0] = the index of the largest of logits[0 .. n), the lowest index on ties (greedy decode;
 * the result stays on the device).  Replaces launch_argmax (kernel.cuh:347, kernel.cu:3531-3592). */
int qlin_launch_argmax(const float *logits, int n, int *out_idx);

/* ---- dequantization (kernel.cuh:237-252) -------------------------------------------------------- */

/* num_elements values of a contiguous block stream to f16 bit patterns (RNE of the exact f32 value).
 * Generic form of launch_dequantize_{q4k,q80,q50,q6k}_to_f16 (launch.cu:803-828). */
int qlin_launch_dequantize_to_f16(int type, const uint8_t *src, uint16_t *out, int64_t num_elements);
/* The reference's per-type names. */
int qlin_launch_dequantize_q4k_to_f16(const uint8_t *src, uint16_t *out, int64_t num_elements);
int qlin_launch_dequantize_q80_to_f16(const uint8_t *src, uint16_t *out, int64_t num_elements);
int qlin_launch_dequantize_q50_to_f16(const uint8_t *src, uint16_t *out, int64_t num_elements);
int qlin_launch_dequantize_q6k_to_f16(const uint8_t *src, uint16_t *out, int64_t num_elements);
/* Same values as f32 (no reference counterpart; the exact values the GEMV consumes). */
int qlin_launch_dequantize_to_f32(int type, const uint8_t *src, float *out, int64_t num_elements);

/* ---- op facade (TensorTool, src/tensor/TensorTool.cpp) ----------------------------------------- */

/* TensorTool::gemm for a quantized weight (TensorTool.cpp:87-98, 146-173): row_bytes is derived as
 * weight_bytes / out_dim, m == 1 runs the decode GEMV, m > 1 the f32-activation matmul. */
int qlin_gemm(int type, const uint8_t *weight, size_t weight_bytes, const float *x, float *y, int out_dim,
              int in_dim, int m);

/* TensorTool::moe_routed_decode_indexed (TensorTool.cpp:271-336) for one token: expert tensors are
 * packed [n_experts, rows, cols] with strides derived from their byte sizes; act_scratch holds
 * k * ffn_dim floats.  Returns QLIN_OK when launched and a QLIN_ERR_* code where the reference
 * returns false (caller falls back). */
int qlin_moe_routed_decode_indexed(int gate_up_type, const uint8_t *gate_exps, const uint8_t *up_exps,
                                   size_t gate_up_bytes, int down_type, const uint8_t *down_exps,
                                   size_t down_bytes, int n_experts, int ffn_dim, int in_dim,
                                   int hidden_size, const float *x, const int *expert_ids,
                                   const float *route_weights, float *act_scratch, float *out, int k);

/* No counterpart in the reference: qlin_launch_moe_router_topk of one token's router_logits
 * [n_experts] followed by qlin_moe_routed_decode_indexed with its picks, in one call.  expert_ids and
 * route_weights [k] receive the router's picks and weights (times routed_scaling) exactly as
 * qlin_launch_moe_router_topk writes them; up to 64 experts, where the routed matrix-core SwiGLU takes
 * the layout, that launch picks the routes itself (one launch fewer), otherwise the router runs first.
 * Arguments and checks otherwise as qlin_moe_routed_decode_indexed's, and n_experts <= 256 (else
 * QLIN_ERR_LIMIT). */
int qlin_moe_routed_decode_indexed_logits(int gate_up_type, const uint8_t *gate_exps, const uint8_t *up_exps,
                                          size_t gate_up_bytes, int down_type, const uint8_t *down_exps,
                                          size_t down_bytes, int n_experts, int ffn_dim, int in_dim, int hidden_size,
                                          const float *x, const float *router_logits, float routed_scaling,
                                          int *expert_ids, float *route_weights, float *act_scratch, float *out,
                                          int k);

/* MoE::forward for one decode token after its norm and before its residual add (MoE.cpp:29-52 with
 * SharedExperts.cpp:25-55), from the router logits: out [hidden_size] gets (out + the routed sum) + the
 * shared experts' down projection of SiLU(shared gate x) * (shared up x), exactly the result of
 * qlin_moe_routed_decode_indexed_logits followed by qlin_launch_quant_swiglu and
 * qlin_launch_quant_gemv_add on the shared weights.  When the shared gate and up have gate_up_type and
 * the routed row stride, shared_ffn is a multiple of ffn_dim with k + shared_ffn / ffn_dim <= 16, and
 * n_experts <= 64, the routed SwiGLU launch also computes the shared SwiGLU (3 launches instead of 4).
 * Shared weights as qlin_moe_ffn_decode_grouped_logits's; shared_ffn = 0 runs the routed part alone.
 * act_scratch: at least k * ffn_dim + shared_ffn floats (the routes' activations, then the shared
 * ones).  Other arguments and checks as qlin_moe_routed_decode_indexed_logits's. */
int qlin_moe_ffn_decode_indexed_logits(int gate_up_type, const uint8_t *gate_exps, const uint8_t *up_exps,
                                       size_t gate_up_bytes, int down_type, const uint8_t *down_exps,
                                       size_t down_bytes, int n_experts, int ffn_dim, int in_dim, int hidden_size,
                                       int shared_type, const uint8_t *shared_gate, const uint8_t *shared_up,
                                       size_t shared_gate_up_row_bytes, const uint8_t *shared_down,
                                       size_t shared_down_row_bytes, int shared_ffn, const float *x,
                                       const float *router_logits, float routed_scaling, int *expert_ids,
                                       float *route_weights, float *act_scratch, float *out, int k);

/* No reference counterpart (the reference decodes one token at a time): moe_routed_decode_indexed
 * for a batch of tokens, each selected expert's weights read once for all the routes that chose it.
 * x [tokens, in_dim], expert_ids / route_weights [tokens, k], out [tokens, hidden_size] (+=); per
 * token the result is that of qlin_moe_routed_decode_indexed.  workspace: device memory of at least
 * qlin_moe_grouped_workspace_bytes(...) bytes, 256-byte aligned, not used by anything else while the
 * call runs; n_experts <= 1024 and tokens * k < 2^21 (else QLIN_ERR_LIMIT). */
size_t qlin_moe_grouped_workspace_bytes(int tokens, int k, int n_experts, int ffn_dim, int hidden_size);
int qlin_moe_routed_decode_grouped(int gate_up_type, const uint8_t *gate_exps, const uint8_t *up_exps,
                                   size_t gate_up_bytes, int down_type, const uint8_t *down_exps,
                                   size_t down_bytes, int n_experts, int ffn_dim, int in_dim, int hidden_size,
                                   const float *x, const int *expert_ids, const float *route_weights,
                                   void *workspace, size_t workspace_bytes, float *out, int tokens, int k);

/* No counterpart in the reference: qlin_launch_moe_router_topk of router_logits [tokens, n_experts]
 * followed by qlin_moe_routed_decode_grouped with its picks, in one call.  expert_ids and
 * route_weights [tokens, k] receive the router's picks and weights (times routed_scaling) exactly as
 * qlin_launch_moe_router_topk writes them; up to 64 experts the routing runs inside the batched
 * decode's gate/up launch (one launch fewer), otherwise as its own launch first.  Arguments and limits
 * otherwise as qlin_moe_routed_decode_grouped's, and n_experts <= 256 (else QLIN_ERR_LIMIT). */
int qlin_moe_routed_decode_grouped_logits(int gate_up_type, const uint8_t *gate_exps, const uint8_t *up_exps,
                                          size_t gate_up_bytes, int down_type, const uint8_t *down_exps,
                                          size_t down_bytes, int n_experts, int ffn_dim, int in_dim, int hidden_size,
                                          const float *x, const float *router_logits, float routed_scaling,
                                          int *expert_ids, float *route_weights, void *workspace,
                                          size_t workspace_bytes, float *out, int tokens, int k);

/* The routed and shared experts of one MoE FFN layer for a batch of decode tokens: MoE::forward after
 * its norm and before its residual add (MoE.cpp:29-52 with SharedExperts.cpp:25-55), from the router
 * logits.  out [tokens, hidden_size] gets (out + the routed sum) + the shared experts' down projection
 * of SiLU(shared gate x) * (shared up x), each token's result exactly that of
 * qlin_moe_routed_decode_grouped_logits followed by qlin_launch_quant_swiglu_rows and
 * qlin_launch_quant_matmul_add on the shared weights, which is what the call runs when the shared
 * down projection cannot take the m > 1 matrix-core kernel; when it can (tokens > 1), that launch
 * also adds the routed sum, so the separate combine launch is not needed.  Shared weights:
 * gate and up [shared_ffn, in_dim] of shared_type with rows of shared_gate_up_row_bytes, down
 * [hidden_size, shared_ffn] with rows of shared_down_row_bytes; shared_ffn = 0 runs the routed part
 * alone.  workspace: at least qlin_moe_ffn_workspace_bytes(...) bytes, 256-byte aligned (the routed
 * part's workspace, then the shared activations).  Other arguments and limits as
 * qlin_moe_routed_decode_grouped_logits's; k = 0 runs the shared experts alone. */
size_t qlin_moe_ffn_workspace_bytes(int tokens, int k, int n_experts, int ffn_dim, int hidden_size, int shared_ffn);
int qlin_moe_ffn_decode_grouped_logits(int gate_up_type, const uint8_t *gate_exps, const uint8_t *up_exps,
                                       size_t gate_up_bytes, int down_type, const uint8_t *down_exps,
                                       size_t down_bytes, int n_experts, int ffn_dim, int in_dim, int hidden_size,
                                       int shared_type, const uint8_t *shared_gate, const uint8_t *shared_up,
                                       size_t shared_gate_up_row_bytes, const uint8_t *shared_down,
                                       size_t shared_down_row_bytes, int shared_ffn, const float *x,
                                       const float *router_logits, float routed_scaling, int *expert_ids,
                                       float *route_weights, void *workspace, size_t workspace_bytes, float *out,
                                       int tokens, int k);

/* No counterpart in the reference: qlin_moe_routed_decode_grouped for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid it).  The same arguments
 * without the workspace: the call runs on a scratch array the library keeps on each GPU for the
 * life of the process, QLIN_MOE_NOALLOC_SCRATCH_BYTES long, and allocates nothing.  A batch whose
 * qlin_moe_grouped_workspace_bytes(...) exceeds that size is refused with QLIN_ERR_LIMIT before
 * anything runs.  Every call on a GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other host threads) race and must be serialised by the caller. */
#define QLIN_MOE_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int qlin_moe_routed_decode_grouped_noalloc(int gate_up_type, const uint8_t *gate_exps, const uint8_t *up_exps,
                                           size_t gate_up_bytes, int down_type, const uint8_t *down_exps,
                                           size_t down_bytes, int n_experts, int ffn_dim, int in_dim,
                                           int hidden_size, const float *x, const int *expert_ids,
                                           const float *route_weights, float *out, int tokens, int k);

/* launch_quant_embedding (kernel.cuh:141-142): output[t, :] = the dequantized row input[t] of a
 * quantized table [vocab, hidden_size] (Q4_K, Q6_K, Q5_0 or Q8_0; bit-exact element values).  As in
 * the reference, the ids must be rows of the table; they are device data and are not checked. */
int qlin_launch_quant_embedding(int type, const int *input, float *output, const uint8_t *table, size_t row_bytes,
                                int hidden_size, int input_size);

/* MLA latent absorption over kv_b [n_heads * (qk_nope + v_head), kv_lora] (kernel.cuh:300-305, 328-330):
 *   q_nope:     q_abs[h, l] = sum_{d < qk_nope} W[h*(qk_nope+v_head) + d, l] * q[h*(qk_nope+qk_rope) + d]
 *   xsum_delta: (Q4_K kv_b) delta[h, b] = sum_{d < qk_nope} q[h, d] * (-dmin * m) of 32-block b of row
 *               h*(qk_nope+v_head) + d, for b < ceil(kv_lora / 32)
 *   v:          attn[h, v] = sum_k W[h*(qk_nope+v_head) + qk_nope + v, k] * attn_latent[h*kv_lora + k],
 *               plus, for Q4_K, sum_b (-dmin * m)(that row, b) * attn_xsum_delta[h, b]. */
int qlin_launch_mla_absorb_q_nope(int type, const float *q, const uint8_t *kv_b_weight, size_t row_bytes,
                                  float *q_abs, int n_heads, int qk_nope, int qk_rope, int v_head, int kv_lora);
int qlin_launch_mla_absorb_q4_xsum_delta(const float *q, const uint8_t *kv_b_weight, size_t row_bytes,
                                         float *q_abs_xsum_delta, int n_heads, int qk_nope, int qk_rope,
                                         int v_head, int kv_lora);
int qlin_launch_mla_absorb_v(int type, const uint8_t *kv_b_weight, size_t row_bytes, const float *attn_latent,
                             const float *attn_xsum_delta, float *attn, int n_heads, int qk_nope, int v_head,
                             int kv_lora);

/* ---- MLA decode over the Q8_1 latent cache (kernel.cuh:297-327) -------------------------------
 * The cache holds one Q8_1 row of latent_row_bytes (>= ceil(kv_lora / 32) * 36, a multiple of 4)
 * per position; kv_cache rows are f32 [kv_lora + qk_rope] (latent, then k_rope).  pos = *d_pos is
 * read on the device (d_pos a device int); the score / context entry points clamp it to
 * max_seq_len - 1, and a negative pos means no positions. */

/* cache[pos] = Q8_1 of kv_cache[pos, 0 .. kv_lora), zero-padded to row_bytes / 36 blocks, s = d * sum(q).
 * Replaces launch_mla_store_latent_q8_1_device_pos (launch.cu:911-917). */
int qlin_launch_mla_store_latent_q8_1_device_pos(const float *kv_cache, uint8_t *latent_q8_1_cache, int kv_lora,
                                                 int qk_rope, size_t row_bytes, const int *d_pos);

/* scores[h * max_seq_len + t] = softmax_scale * (q_abs[h] . latent(t) + q_rope[h] . k_rope(t)
 *   + sum_b q_abs_xsum_delta[h, b] * (stored_sum(t, b) - dequantized_sum(t, b))) for t <= pos; q
 * rows are [qk_nope + qk_rope] per head.  Replaces launch_mla_absorb_scores_device_pos (launch.cu:977-989). */
int qlin_launch_mla_absorb_scores_device_pos(const float *q_abs, const float *q, const uint8_t *latent_q8_1_cache,
                                             size_t latent_row_bytes, const float *q_abs_xsum_delta,
                                             const float *kv_cache, float *scores, int n_heads, int qk_nope,
                                             int qk_rope, int kv_lora, const int *d_pos, int max_seq_len,
                                             float softmax_scale);

/* p = softmax over t <= pos of scores[h] (denominator + 1e-9); attn_latent[h, k] = sum_t p_t latent(t, k),
 * attn_xsum_delta[h, b] = sum_t p_t (stored_sum(t, b) - dequantized_sum(t, b)).
 * Replaces launch_mla_absorb_context_device_pos (launch.cu:991-1000). */
int qlin_launch_mla_absorb_context_device_pos(const float *scores, const uint8_t *latent_q8_1_cache,
                                              size_t latent_row_bytes, float *attn_xsum_delta, float *attn_latent,
                                              int n_heads, int kv_lora, const int *d_pos, int max_seq_len);

/* The scores, softmax and context above in one launch, with the fast exp (__expf) and no 1e-9 in the
 * denominator; the scores of every position stay on chip, so max_seq_len <= 32768 (and the LDS of
 * max_seq_len + kv_lora + qk_rope + ceil(kv_lora / 32) floats fits).
 * Replaces launch_mla_absorb_attend_device_pos (launch.cu:964-975). */
int qlin_launch_mla_absorb_attend_device_pos(const float *q_abs, const float *q, const uint8_t *latent_q8_1_cache,
                                             size_t latent_row_bytes, const float *q_abs_xsum_delta,
                                             float *attn_xsum_delta, const float *kv_cache, float *attn_latent,
                                             int n_heads, int qk_nope, int qk_rope, int kv_lora, const int *d_pos,
                                             int max_seq_len, float softmax_scale);

/* kv_b_cache[pos, r] = W_kv_b[r] . cache[pos] (Q8_1 block-dot semantics of quant_matmul_q8_1) for the
 * v rows r = h * (qk_nope + v_head) + qk_nope + v of every head.  Types Q4_K, Q6_K, Q5_0, Q8_0.
 * Replaces launch_mla_project_v_device_pos (launch.cu:1015-1040). */
int qlin_launch_mla_project_v_device_pos(int type, const uint8_t *kv_b_weight, size_t row_bytes,
                                         const uint8_t *latent_q8_1_cache, size_t latent_row_bytes,
                                         float *kv_b_cache, int n_heads, int qk_nope, int v_head, int kv_lora,
                                         const int *d_pos);

/* attn[h, v] = sum_t p_t kv_b_cache[t, h * (qk_nope + v_head) + qk_nope + v], p the softmax of
 * scores[h] as above; v_head <= 256.  Replaces launch_mla_absorb_context_v_device_pos (launch.cu:1042-1049). */
int qlin_launch_mla_absorb_context_v_device_pos(const float *scores, const float *kv_b_cache, float *attn,
                                                int n_heads, int qk_nope, int v_head, const int *d_pos,
                                                int max_seq_len);

#ifdef __cplusplus
}
#endif
#endif /* QLIN_H */

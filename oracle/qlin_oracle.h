/*
 * qlin_oracle.h -- CPU restatement of the reference's GGUF quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (blog_amd/, include/) may link, load or
 * call this code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the checker.  It is plain C99, compiled with -ffp-contract=off so every
 * floating-point expression is evaluated exactly as written (no fused multiply-add).
 *
 * Reference being restated (paths relative to AI/codes/local-llm/ in the reference repo):
 *   block codecs   src/backend/cuda/ops/kernel.cu:913-921 (q4k_scale_min), 1090-1119 (q4k_at),
 *                  1122-1156 (q6k_at), 1159-1175 (q50_at), 1178-1185 (q80_at)
 *   dequant->f16   kernel.cu:954-1063 (dequantize_{q4k,q80,q50,q6k}_to_f16_kernel)
 *   GEMV / matmul  kernel.cu:1192-1279 (quant_gemv_kernel, quant_gemv_add_kernel, quant_matmul_kernel)
 *   Q8_1           kernel.cu:1679-1720 (quantize_q8_1_kernel), 2305-2402 (quant_matmul_q8_1_kernel)
 *   MoE            kernel.cu:1289-1385 (quant_swiglu[_indexed]_kernel),
 *                  2253-2287 (quant_down_f32_indexed_accum_ordered_kernel),
 *                  3463-3511 (moe_router_topk_kernel), 3531-3592 (argmax, lowest index on ties)
 *   embedding, MLA kernel.cu:2678-2693 (quant_embedding_kernel), 3004-3075 (q4k_min_coeff_at,
 *                  mla_absorb_q_nope_kernel, mla_absorb_q4_xsum_delta_kernel), 3417-3453
 *                  (mla_absorb_v_kernel)
 *   block traits   src/format/gguf/GgufFile.cpp:35-55; dtype codes src/tensor/TensorCommon.h:15-33
 *   Q4_0           not implemented by the reference (trait only, GgufFile.cpp:40); restated from
 *                  the published ggml block_q4_0 format (d f16, 16 bytes of split-half nibbles,
 *                  w = d * (q - 8)).
 *
 * How each part is pinned (tests/test_oracle.py):
 *   f16 <-> f32     exhaustive over all 65536 halves and RNE-encoded against numpy's float16.
 *   Q4_K, Q6_K      the reference's own known-answer blocks (LaunchAddTest.cpp:711-756 -> 2212,
 *                   758-803 -> 948) plus every scale/min field and bit position against an
 *                   independent encoder (tests/qgen.py).
 *   Q8_0            the reference's two-row closed form (LaunchAddTest.cpp:186-240).
 *   Q8_1            the reference's sums (LaunchAddTest.cpp:679-709: 158/127 and raw 1.31) and
 *                   the quantizer's invariants (|q| <= 127, RNE, d = amax/127).
 *   GEMV / matmul   double-precision truth against closed forms, linearity, and f32 orders.
 *   router, SwiGLU, brute force on tiny inputs, the tie (lowest index) and NaN rules, numpy.
 *   down-accumulate
 *   embedding, MLA  the dequantized rows (pinned above) against numpy restatements of each sum
 *                   (transposed per-head products, the -dmin*m block coefficients from the scale
 *                   bytes); no reference test covers these kernels.
 *   Q5_0            parity unpinned: the reference has the codec (kernel.cu:1159-1175) but no test;
 *                   checked only against that formula as read and an independent encoder.
 *   Q4_0            parity unpinned: the reference has no implementation; checked only against the
 *                   ggml closed form and an independent encoder.
 *   The last ulp of the reference's f32 summation order and of its expf/__expf cannot be pinned
 *   without running its CUDA code; those are bounded by tolerance, not bits.
 */
#ifndef QLIN_ORACLE_H
#define QLIN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type codes (TensorCommon.h:15-33). */
enum {
    ORC_F32 = 0,
    ORC_F16 = 1,
    ORC_Q4_0 = 2,
    ORC_Q5_0 = 6,
    ORC_Q8_0 = 8,
    ORC_Q8_1 = 9,
    ORC_Q4_K = 12,
    ORC_Q6_K = 14,
};

/* Elements and bytes per block; 0 for an unknown type (GgufFile.cpp:35-55). */
int orc_block_elems(int type);
int orc_block_bytes(int type);

/* IEEE-754 binary16 <-> binary32.  f16->f32 is exact; f32->f16 rounds to nearest, ties to even. */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_array(const uint16_t *h, float *out, int64_t n);
void orc_f32_to_f16_array(const float *f, uint16_t *out, int64_t n);

/* Q4_K 6-bit (scale, min) of sub-block j in [0,8) (kernel.cu:913-921). */
void orc_q4k_scale_min(int j, const uint8_t *scales, int *sc, int *m);

/* Dequantize n elements (n a multiple of the block size) of one contiguous block stream.
 * f32 values use the canonical non-contracted formulas; the f16 variant is RNE of the f32 value.
 * Returns 0, or -1 for an unsupported type / indivisible n. */
int orc_dequant_f32(int type, const uint8_t *src, int64_t n, float *out);
int orc_dequant_f16(int type, const uint8_t *src, int64_t n, uint16_t *out);

/* y[r, o] = sum_k w(o, k) * x[r, k] over m activation rows, double accumulation (the truth).
 * W is [out_dim, in_dim] in row_bytes-strided rows.  Returns 0 or -1. */
int orc_matmul_f64(int type, const uint8_t *w, size_t row_bytes, const float *x, double *y,
                   int out_dim, int in_dim, int m);

/* Same contraction with f32 accumulation, parallel over output rows with nthreads OpenMP
 * threads (<= 0 means the OpenMP default).  This is the timed CPU path. */
int orc_matmul_f32(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y,
                   int out_dim, int in_dim, int m, int nthreads);

/* The reference kernel's own f32 order: 32 lanes, lane-strided fmaf, then a shuffle-down tree
 * (kernel.cu:1192-1215).  Used to bound the fp32 deviation expected of any GPU order. */
int orc_matmul_lane32(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y,
                      int out_dim, int in_dim, int m);

/* y[o] += sum_k w(o,k) x[k]  (kernel.cu:1223-1244), double accumulation then one f32 add. */
int orc_gemv_add(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y,
                 int out_dim, int in_dim);

/* Q8_1 activation blocks: per 32 values, 36 bytes = d f16 | s f16 | q int8[32]
 * (kernel.cu:1679-1720).  A trailing partial block is zero padded.  Bit-exact target. */
size_t orc_q8_1_row_bytes(int in_dim);
void orc_quantize_q8_1(const float *x, uint8_t *xq, int in_dim, int m, int store_raw_sum);

/* Quantized weight x Q8_1 activation, block-dot semantics of kernel.cu:2305-2402, computed in
 * double (the truth for the int8 prefill path).  Returns 0 or -1. */
int orc_matmul_q8_1(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, double *y,
                    int out_dim, int in_dim, int m);
/* the same with `threads` OpenMP threads over the rows (<= 0: all); every output is summed in
 * the same order whatever the count */
int orc_matmul_q8_1_mt(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, double *y,
                       int out_dim, int in_dim, int m, int threads);

/* MoE router: softmax over n_experts (non-finite -> -inf), k picks with strict '>' (lowest index
 * wins ties), w = p * routed_scaling, no renormalisation (kernel.cu:3463-3511). */
void orc_router_topk(const float *logits, int *top_idx, float *top_w, int tokens, int n_experts,
                     int k, float routed_scaling);

/* act[o] = silu(Wg[o].x) * (Wu[o].x)  (kernel.cu:1289-1328). */
int orc_swiglu(int type, const uint8_t *wg, const uint8_t *wu, size_t g_row_bytes,
               size_t u_row_bytes, const float *x, float *act, int ffn_dim, int in_dim);

/* act[r, o] for route r with expert_ids[r] (< 0 -> 0)  (kernel.cu:1340-1385). */
int orc_swiglu_indexed(int type, const uint8_t *wg, const uint8_t *wu, size_t g_expert_bytes,
                       size_t u_expert_bytes, size_t g_row_bytes, size_t u_row_bytes,
                       const float *x, const int *expert_ids, float *act, int k, int ffn_dim,
                       int in_dim);

/* out[h] += sum_r w_r * (Wd[e_r][h] . act[r]), routes in order, negative ids skipped
 * (kernel.cu:2253-2287). */
int orc_down_indexed_ordered(int type, const uint8_t *wd, size_t d_expert_bytes,
                             size_t d_row_bytes, const float *act, const int *expert_ids,
                             const float *route_w, float *out, int k, int hidden, int ffn_dim);

/* Q8_1-activation variants, sums in double.
 * quantize_q8_1_mmq: the group-major MMQ layout (kernel.cu:1724-1765): group g of row r at
 *   (g * m + r) * 144 = 4 x (d f16, s f16), then 4 x 32 int8; the blocks are those of orc_quantize_q8_1.
 * matmul_q8_1_mmq: orc_matmul_q8_1 over that layout (kernel.cu:2405-2660).
 * swiglu_indexed_q8_1: silu(g) * u with g, u the block-dot rows against one Q8_1 x (kernel.cu:1532-1666).
 * down_q8_1_indexed_accum: out[h] += sum_r rw_r * (Wd_e[h] . act_q8_1[r]) (kernel.cu:1873-2097);
 * down_f32_indexed_accum: the same after orc_quantize_q8_1 of each route's act (kernel.cu:2112-2242). */
void orc_quantize_q8_1_mmq(const float *x, uint8_t *xq, int in_dim, int m, int store_raw_sum);
int orc_matmul_q8_1_mmq(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, double *y, int out_dim,
                        int in_dim, int m);
int orc_swiglu_indexed_q8_1(int type, const uint8_t *wg, const uint8_t *wu, size_t g_expert_bytes,
                            size_t u_expert_bytes, size_t g_row_bytes, size_t u_row_bytes, const uint8_t *xq,
                            const int *expert_ids, double *act, int k, int ffn_dim, int in_dim);
int orc_down_q8_1_indexed_accum(int type, const uint8_t *wd, size_t d_expert_bytes, size_t d_row_bytes,
                                const uint8_t *act_q8_1, const int *expert_ids, const float *route_w, double *out,
                                int k, int hidden, int ffn_dim);
int orc_down_f32_indexed_accum(int type, const uint8_t *wd, size_t d_expert_bytes, size_t d_row_bytes,
                               const float *act, const int *expert_ids, const float *route_w, double *out, int k,
                               int hidden, int ffn_dim);

/* Index of the maximum, lowest index on ties (kernel.cu:3531-3592). */
int orc_argmax(const float *v, int n);

/* Embedding rows and MLA absorption (kernel.cu:2678-2693, 3004-3075, 3417-3453), sums in double. */
int orc_quant_embedding(int type, const int *ids, int n, const uint8_t *table, size_t row_bytes, int hidden,
                        float *out);
int orc_mla_absorb_q_nope(int type, const float *q, const uint8_t *w, size_t row_bytes, double *q_abs, int n_heads,
                          int qk_nope, int qk_rope, int v_head, int kv_lora);
int orc_mla_absorb_q4_xsum_delta(const float *q, const uint8_t *w, size_t row_bytes, double *out, int n_heads,
                                 int qk_nope, int qk_rope, int v_head, int kv_lora);
int orc_mla_absorb_v(int type, const uint8_t *w, size_t row_bytes, const float *latent, const float *delta,
                     double *attn, int n_heads, int qk_nope, int v_head, int kv_lora);

/* MLA decode over the Q8_1 latent cache (kernel.cu:2945-3415) at position pos; sums in double.
 * store: cache row pos from kv_cache row pos (row_bytes / 36 blocks, zero past kv_lora).
 * scores: scores[h * max_seq + t] for t <= pos (other entries untouched).
 * context: the softmax-weighted latent rows and block-sum corrections per head.
 * project_v: kv_b_cache[pos * n_heads * (qk_nope + v_head) + r] for the v rows r of every head.
 * context_v: the softmax-weighted v rows of kv_b_cache per head. */
int orc_mla_store_latent_q8_1(const float *kv_cache, uint8_t *cache, int kv_lora, int qk_rope, size_t row_bytes,
                              int pos);
int orc_mla_absorb_scores(const float *q_abs, const float *q, const uint8_t *cache, size_t cache_row_bytes,
                          const float *delta, const float *kv_cache, double *scores, int n_heads, int qk_nope,
                          int qk_rope, int kv_lora, int pos, int max_seq, float scale);
int orc_mla_absorb_context(const float *scores, const uint8_t *cache, size_t cache_row_bytes, double *delta_out,
                           double *latent_out, int n_heads, int kv_lora, int pos, int max_seq);
/* attend: scores, then the softmax without the 1e-9 term, then the context (kernel.cu:3078-3155). */
int orc_mla_absorb_attend(const float *q_abs, const float *q, const uint8_t *cache, size_t cache_row_bytes,
                          const float *delta, double *delta_out, const float *kv_cache, double *latent_out,
                          int n_heads, int qk_nope, int qk_rope, int kv_lora, int pos, int max_seq, float scale);
int orc_mla_project_v(int type, const uint8_t *w, size_t row_bytes, const uint8_t *cache, size_t cache_row_bytes,
                      double *kv_b_cache, int n_heads, int qk_nope, int v_head, int kv_lora, int pos);
int orc_mla_absorb_context_v(const float *scores, const float *kv_b_cache, double *attn, int n_heads, int qk_nope,
                             int v_head, int pos, int max_seq);

/* The CPU twin of the config-3 decoder harness (blog_amd/decoder.py): a Qwen2-architecture decoder
 * with quantized linears, restating the layer's glue from the reference (kernel.cu:112-150 RMSNorm,
 * 186-226 rotary pairs (i, i + d/2), 345-420 causal GQA attention; SwiGLU as quant_swiglu, 1289-1328)
 * and the Qwen2 layer order: x -> RMSNorm -> q, k, v -> rotary -> attention -> o added to the
 * residual -> RMSNorm -> SiLU(gate) * up -> down added to the residual; then the final RMSNorm and the
 * tied embedding table as the output head.  No q/k/v biases.  Every sum and the whole hidden state
 * in double.  tokens[0..n) are processed at positions 0..n-1 (teacher forcing); the logits of
 * positions first..n-1 are written to logits [(n - first) * vocab].  Linears and the table share the
 * type `wtype`; norm weights are f32 values.  `threads` OpenMP threads share each matrix's rows. */
typedef struct {
    int layers, hidden, n_heads, kv_heads, head_dim, ffn, vocab, wtype;
    double eps, theta;
} orc_qwen2_cfg;
typedef struct {
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd; /* [out, in] rows, in = hidden (wd: ffn) */
    const float *attn_norm, *ffn_norm;                /* [hidden] */
} orc_qwen2_layer;
int orc_qwen2_logits(const orc_qwen2_cfg *cfg, const orc_qwen2_layer *layers, const float *final_norm,
                     const uint8_t *table, const int *tokens, int n, int first, float *logits, int threads);

#ifdef __cplusplus
}
#endif
#endif /* QLIN_ORACLE_H */

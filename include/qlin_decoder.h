/*
 * qlin_decoder.h -- the glue around the quantized linears of a Qwen2-architecture decoder layer:
 * RMSNorm, rotary embedding with the KV-cache store, and causal grouped-query attention.
 *
 * These are not part of the quantized-linear path.  They let a whole decoder (benchmark configuration
 * C3, Qwen2.5-0.5B architecture with every linear in Q8_0) run its greedy decode on the path's kernels;
 * the linears, the embedding lookup and the argmax are the entry points of qlin.h.  Conventions as
 * in qlin.h: caller-owned device pointers, asynchronous on qlin_set_stream's stream, nothing
 * allocated, a qlin_status returned.
 *
 * Semantics restated from the reference engine (AI/codes/local-llm/src/backend/cuda/ops/):
 *   qlin_launch_rms_norm       launch_rms_norm (kernel.cuh:147-150, kernel.cu:112-150), same arguments:
 *                              y[r, j] = x[r, j] * rsqrt(mean_j x^2 + eps) * w[j], w bf16 (weight_type 0)
 *                              or f16 (1), plus one if one_plus.
 *   qlin_launch_rope_store_kv  the Qwen2 counterpart of launch_full_attention_q / _kv (kernel.cuh:162-184,
 *                              kernel.cu:186-340) without their q/k norms: rows at positions
 *                              *start_pos_dev + r; each head's pairs (i, i + head_dim/2) rotated by
 *                              pos / theta^(2i / head_dim); q in place, k rotated and v copied into the
 *                              caches [max_seq_len, kv_heads * head_dim] (f32) at the row's position.
 *   qlin_launch_attend         launch_full_attention_attend (kernel.cuh:186-189, kernel.cu:345-420) without
 *                              its output gate: attn[r, h] = softmax_j(q[r, h] . k[j, h / (n_heads /
 *                              kv_heads)] / sqrt(head_dim)) v[j, .] over positions j <= the row's.
 * A row's position is clamped to [0, max_seq_len - 1]; head_dim <= 256 and max_seq_len <= 32768
 * (else QLIN_ERR_LIMIT); n_heads a multiple of kv_heads and head_dim of 4 (else QLIN_ERR_SHAPE);
 * qlin_launch_attend reads q, the caches and attn as 16-byte vectors (16-byte aligned, else
 * QLIN_ERR_ALIGN).
 *
 * The RMSNorm fused into the decode linear that consumes it (no counterpart in the reference, whose
 * decode step runs launch_rms_norm and then launch_quant_gemv / launch_quant_swiglu on its output):
 *   qlin_launch_rms_norm_quant_gemv_multi  qlin_launch_quant_gemv_multi (one row, n_mats matrices that
 *                              share x) of rms_norm(x), the norm's arguments as qlin_launch_rms_norm's;
 *   qlin_launch_rms_norm_quant_swiglu      qlin_launch_quant_swiglu (gate and up of one row stride) of
 *                              rms_norm(x).
 * The decode kernels normalize x as they stage it (the normalized vector is not written), in one
 * launch instead of two.  They take the shapes of the matrix-core decode kernels (every format, in_dim
 * a multiple of 256, or 128 for Q8_0 and Q5_0, x 16-byte aligned); other shapes return
 * QLIN_ERR_LIMIT, for the two-launch form.
 *   qlin_launch_rope_attend    qlin_launch_rope_store_kv then qlin_launch_attend for one row (a decode
 *                              step), in one launch, with the same results: the rotated key and the
 *                              value are stored in the caches at the row's position as before, but q is
 *                              left as it is (the rotated q lives only in the launch).  Alignment as
 *                              qlin_launch_attend's for q, the caches and attn; k and v 4-byte aligned.
 *   qlin_launch_quant_gemv_argmax  the output head and the greedy pick: logits = W x, or W rms_norm(x) when
 *                              norm_weight is non-null, as qlin_launch_quant_gemv / ..._rms_norm_quant_gemv_multi
 *                              give them, then *out_idx as qlin_launch_argmax gives it for those logits (the
 *                              largest, the lowest index among equals, NaN never; 0 when nothing beats -inf).
 *                              Each workgroup of the GEMV reduces its own rows to one (value, index) pair in
 *                              scratch (QLIN_GEMV_ARGMAX_SCRATCH_BYTES of device memory, 4-byte aligned, used
 *                              by nothing else while the launches run), and one small launch reduces the pairs:
 *                              two launches instead of a GEMV and a one-workgroup scan of every logit.  Shapes
 *                              as the fused RMSNorm launches' (else QLIN_ERR_LIMIT); out_dim >= 1.
 */
#ifndef QLIN_DECODER_H
#define QLIN_DECODER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int qlin_launch_rms_norm(const float *input, float *output, const uint16_t *weight, int weight_type, int rows,
                         int hidden_size, float eps, int one_plus);
int qlin_launch_rope_store_kv(float *q, const float *k, const float *v, float *key_cache, float *value_cache, int rows,
                              int n_heads, int kv_heads, int head_dim, int max_seq_len, const int *start_pos_dev,
                              float rope_theta);
int qlin_launch_attend(const float *q, const float *key_cache, const float *value_cache, float *attn, int rows,
                       int n_heads, int kv_heads, int head_dim, int max_seq_len, const int *start_pos_dev);
int qlin_launch_rope_attend(const float *q, const float *k, const float *v, float *key_cache, float *value_cache,
                            float *attn, int n_heads, int kv_heads, int head_dim, int max_seq_len,
                            const int *start_pos_dev, float rope_theta);
int qlin_launch_rms_norm_quant_gemv_multi(int type, int n_mats, const uint8_t *const *weights, size_t row_bytes,
                                          const float *x, const uint16_t *norm_weight, int norm_type, float eps,
                                          int one_plus, float *const *ys, const int *out_dims, int in_dim);
int qlin_launch_rms_norm_quant_swiglu(int type, const uint8_t *w_gate, const uint8_t *w_up, size_t row_bytes,
                                      const float *x, const uint16_t *norm_weight, int norm_type, float eps,
                                      int one_plus, float *act, int ffn_dim, int in_dim);
#define QLIN_GEMV_ARGMAX_SCRATCH_BYTES 8192
int qlin_launch_quant_gemv_argmax(int type, const uint8_t *weights, size_t row_bytes, const float *x,
                                  const uint16_t *norm_weight, int norm_type, float eps, int one_plus, float *logits,
                                  int out_dim, int in_dim, void *scratch, int *out_idx);

#ifdef __cplusplus
}
#endif

#endif /* QLIN_DECODER_H */

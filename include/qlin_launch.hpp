// qlin_launch.hpp -- header-only C++ shim that restores the reference engine's launcher names and
// DType-typed signatures on top of the C ABI (qlin.h), so a caller of
// AI/codes/local-llm/src/backend/cuda/ops/kernel.cuh switches by changing its include.
//
// Differences from the reference, on purpose:
//   - an unsupported type or bad shape throws qlin_ref::QlinError (the reference silently does
//     nothing, launch.cu:57);
//   - the launch stream is the one set with set_current_stream (common.cpp:13-17 keeps a global).
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "qlin.h"

namespace qlin_ref {

// Same values as the reference's DType (src/tensor/TensorCommon.h:15-33) = ggml type codes.
enum class DType : int32_t {
    F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q8_1 = 9,
    Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, Q8_K = 15, I32 = 24, BF16 = 30, UNKNOWN = -1,
};

class QlinError : public std::runtime_error {
public:
    QlinError(const char *fn, int status)
        : std::runtime_error(std::string(fn) + ": " + qlin_status_string(status)), status_(status) {}
    int status() const { return status_; }

private:
    int status_;
};

inline void check(int status, const char *fn) {
    if (status != QLIN_OK) throw QlinError(fn, status);
}

inline void set_current_stream(void *hip_stream) { check(qlin_set_stream(hip_stream), "set_current_stream"); }
inline void *get_current_stream() { return qlin_get_stream(); }

// kernel.cuh:33-42
inline void launch_quant_gemv(DType t, const uint8_t *weight, size_t row_bytes, const float *x, float *y,
                              int out_dim, int in_dim, int m) {
    check(qlin_launch_quant_gemv(static_cast<int>(t), weight, row_bytes, x, y, out_dim, in_dim, m),
          "launch_quant_gemv");
}
inline void launch_quant_gemv_add(DType t, const uint8_t *weight, size_t row_bytes, const float *x, float *y,
                                  int out_dim, int in_dim) {
    check(qlin_launch_quant_gemv_add(static_cast<int>(t), weight, row_bytes, x, y, out_dim, in_dim),
          "launch_quant_gemv_add");
}
inline void launch_quant_matmul(DType t, const uint8_t *weight, size_t row_bytes, const float *x, float *y,
                                int out_dim, int in_dim, int m) {
    check(qlin_launch_quant_matmul(static_cast<int>(t), weight, row_bytes, x, y, out_dim, in_dim, m),
          "launch_quant_matmul");
}
// The batched forms of launch_quant_gemv_add and launch_quant_swiglu (SharedExperts.cpp:34-48 for m > 1).
inline void launch_quant_matmul_add(DType t, const uint8_t *weight, size_t row_bytes, const float *x, float *y,
                                    int out_dim, int in_dim, int m) {
    check(qlin_launch_quant_matmul_add(static_cast<int>(t), weight, row_bytes, x, y, out_dim, in_dim, m),
          "launch_quant_matmul_add");
}
inline void launch_quant_swiglu_rows(DType t, const uint8_t *gate_weight, const uint8_t *up_weight,
                                     size_t gate_row_bytes, size_t up_row_bytes, const float *x, float *act,
                                     int ffn_dim, int in_dim, int m) {
    check(qlin_launch_quant_swiglu_rows(static_cast<int>(t), gate_weight, up_weight, gate_row_bytes, up_row_bytes,
                                        x, act, ffn_dim, in_dim, m),
          "launch_quant_swiglu_rows");
}

// No reference counterpart: q, k and v (or any matrices reading the same x) in one launch.
inline void launch_quant_gemv_multi(DType t, int n_mats, const uint8_t *const *weights, size_t row_bytes,
                                    const float *x, float *const *ys, const int *out_dims, int in_dim) {
    check(qlin_launch_quant_gemv_multi(static_cast<int>(t), n_mats, weights, row_bytes, x, ys, out_dims, in_dim),
          "launch_quant_gemv_multi");
}

// kernel.cuh:46-54
inline size_t q8_1_row_bytes(int in_dim) { return qlin_q8_1_row_bytes(in_dim); }
inline void launch_quantize_q8_1(const float *x, uint8_t *x_q8_1, int in_dim, int m, bool store_raw_sum = false) {
    check(qlin_launch_quantize_q8_1(x, x_q8_1, in_dim, m, store_raw_sum ? 1 : 0), "launch_quantize_q8_1");
}
inline void launch_quant_matmul_q8_1(DType t, const uint8_t *weight, size_t row_bytes, const uint8_t *x_q8_1,
                                     float *y, int out_dim, int in_dim, int m) {
    check(qlin_launch_quant_matmul_q8_1(static_cast<int>(t), weight, row_bytes, x_q8_1, y, out_dim, in_dim, m),
          "launch_quant_matmul_q8_1");
}
inline void launch_quant_gemv_q8_1(DType t, const uint8_t *weight, size_t row_bytes, const uint8_t *x_q8_1, float *y,
                                   int out_dim, int in_dim) {
    check(qlin_launch_quant_gemv_q8_1(static_cast<int>(t), weight, row_bytes, x_q8_1, y, out_dim, in_dim),
          "launch_quant_gemv_q8_1");
}
inline void launch_quantize_q8_1_mmq(const float *x, uint8_t *x_q8_1, int in_dim, int m, bool store_raw_sum = false) {
    check(qlin_launch_quantize_q8_1_mmq(x, x_q8_1, in_dim, m, store_raw_sum ? 1 : 0), "launch_quantize_q8_1_mmq");
}
inline void launch_quant_matmul_q8_1_mmq(DType t, const uint8_t *weight, size_t row_bytes, const uint8_t *x_q8_1,
                                         float *y, int out_dim, int in_dim, int m) {
    check(qlin_launch_quant_matmul_q8_1_mmq(static_cast<int>(t), weight, row_bytes, x_q8_1, y, out_dim, in_dim, m),
          "launch_quant_matmul_q8_1_mmq");
}

// kernel.cuh:62-129
inline void launch_quant_swiglu(DType t, const uint8_t *gate_weight, const uint8_t *up_weight,
                                size_t gate_row_bytes, size_t up_row_bytes, const float *x, float *act,
                                int ffn_dim, int in_dim) {
    check(qlin_launch_quant_swiglu(static_cast<int>(t), gate_weight, up_weight, gate_row_bytes, up_row_bytes, x,
                                   act, ffn_dim, in_dim),
          "launch_quant_swiglu");
}
inline void launch_quant_swiglu_indexed(DType t, const uint8_t *gate_weight, const uint8_t *up_weight,
                                        size_t gate_expert_bytes, size_t up_expert_bytes, size_t gate_row_bytes,
                                        size_t up_row_bytes, const float *x, const int *expert_ids, float *act,
                                        int k, int ffn_dim, int in_dim) {
    check(qlin_launch_quant_swiglu_indexed(static_cast<int>(t), gate_weight, up_weight, gate_expert_bytes,
                                           up_expert_bytes, gate_row_bytes, up_row_bytes, x, expert_ids, act, k,
                                           ffn_dim, in_dim),
          "launch_quant_swiglu_indexed");
}
inline void launch_quant_down_f32_indexed_accum_ordered(DType t, const uint8_t *down_weight,
                                                        size_t down_expert_bytes, size_t down_row_bytes,
                                                        const float *act, const int *expert_ids,
                                                        const float *route_weights, float *out, int k,
                                                        int hidden_size, int ffn_dim) {
    check(qlin_launch_quant_down_f32_indexed_accum_ordered(static_cast<int>(t), down_weight, down_expert_bytes,
                                                           down_row_bytes, act, expert_ids, route_weights, out, k,
                                                           hidden_size, ffn_dim),
          "launch_quant_down_f32_indexed_accum_ordered");
}
inline void launch_quant_swiglu_indexed_block(DType t, const uint8_t *gate_weight, const uint8_t *up_weight,
                                              size_t gate_expert_bytes, size_t up_expert_bytes, size_t gate_row_bytes,
                                              size_t up_row_bytes, const float *x, const int *expert_ids, float *act,
                                              int k, int ffn_dim, int in_dim, bool fast_silu = false) {
    check(qlin_launch_quant_swiglu_indexed_block(static_cast<int>(t), gate_weight, up_weight, gate_expert_bytes,
                                                 up_expert_bytes, gate_row_bytes, up_row_bytes, x, expert_ids, act, k,
                                                 ffn_dim, in_dim, fast_silu ? 1 : 0),
          "launch_quant_swiglu_indexed_block");
}
inline void launch_quant_swiglu_indexed_q8_1(DType t, const uint8_t *gate_weight, const uint8_t *up_weight,
                                             size_t gate_expert_bytes, size_t up_expert_bytes, size_t gate_row_bytes,
                                             size_t up_row_bytes, const uint8_t *x_q8_1, const int *expert_ids,
                                             float *act, int k, int ffn_dim, int in_dim) {
    check(qlin_launch_quant_swiglu_indexed_q8_1(static_cast<int>(t), gate_weight, up_weight, gate_expert_bytes,
                                                up_expert_bytes, gate_row_bytes, up_row_bytes, x_q8_1, expert_ids, act,
                                                k, ffn_dim, in_dim),
          "launch_quant_swiglu_indexed_q8_1");
}
inline void launch_quant_down_q8_1_indexed_accum(DType t, const uint8_t *down_weight, size_t down_expert_bytes,
                                                 size_t down_row_bytes, const uint8_t *act_q8_1,
                                                 const int *expert_ids, const float *route_weights, float *out, int k,
                                                 int hidden_size, int ffn_dim) {
    check(qlin_launch_quant_down_q8_1_indexed_accum(static_cast<int>(t), down_weight, down_expert_bytes,
                                                    down_row_bytes, act_q8_1, expert_ids, route_weights, out, k,
                                                    hidden_size, ffn_dim),
          "launch_quant_down_q8_1_indexed_accum");
}
inline void launch_quant_down_q8_1_indexed_accum_shared(DType t, const uint8_t *down_weight, size_t down_expert_bytes,
                                                        size_t down_row_bytes, const uint8_t *act_q8_1,
                                                        const int *expert_ids, const float *route_weights, float *out,
                                                        int k, int hidden_size, int ffn_dim) {
    check(qlin_launch_quant_down_q8_1_indexed_accum_shared(static_cast<int>(t), down_weight, down_expert_bytes,
                                                           down_row_bytes, act_q8_1, expert_ids, route_weights, out, k,
                                                           hidden_size, ffn_dim),
          "launch_quant_down_q8_1_indexed_accum_shared");
}
inline void launch_quant_down_f32_indexed_accum(DType t, const uint8_t *down_weight, size_t down_expert_bytes,
                                                size_t down_row_bytes, const float *act, const int *expert_ids,
                                                const float *route_weights, float *out, int k, int hidden_size,
                                                int ffn_dim) {
    check(qlin_launch_quant_down_f32_indexed_accum(static_cast<int>(t), down_weight, down_expert_bytes, down_row_bytes,
                                                   act, expert_ids, route_weights, out, k, hidden_size, ffn_dim),
          "launch_quant_down_f32_indexed_accum");
}

// kernel.cuh:339-347
inline void launch_moe_accumulate(const float *expert_out, float weight, float *out, int n) {
    check(qlin_launch_moe_accumulate(expert_out, weight, out, n), "launch_moe_accumulate");
}
inline void launch_moe_accumulate_device(const float *expert_out, const float *weight, float *out, int n) {
    check(qlin_launch_moe_accumulate_device(expert_out, weight, out, n), "launch_moe_accumulate_device");
}
inline void launch_argmax(const float *logits, int n, int *out_idx) {
    check(qlin_launch_argmax(logits, n, out_idx), "launch_argmax");
}

// kernel.cuh:335-336
inline void launch_moe_router_topk(const float *router_logits, int *top_idx, float *top_w, int tokens,
                                   int n_experts, int k, float routed_scaling) {
    check(qlin_launch_moe_router_topk(router_logits, top_idx, top_w, tokens, n_experts, k, routed_scaling),
          "launch_moe_router_topk");
}

// kernel.cuh:237-248 (the reference takes the element count as int64_t)
inline void launch_dequantize_q4k_to_f16(const uint8_t *src, uint16_t *out, int64_t n) {
    check(qlin_launch_dequantize_q4k_to_f16(src, out, n), "launch_dequantize_q4k_to_f16");
}
inline void launch_dequantize_q80_to_f16(const uint8_t *src, uint16_t *out, int64_t n) {
    check(qlin_launch_dequantize_q80_to_f16(src, out, n), "launch_dequantize_q80_to_f16");
}
inline void launch_dequantize_q50_to_f16(const uint8_t *src, uint16_t *out, int64_t n) {
    check(qlin_launch_dequantize_q50_to_f16(src, out, n), "launch_dequantize_q50_to_f16");
}
inline void launch_dequantize_q6k_to_f16(const uint8_t *src, uint16_t *out, int64_t n) {
    check(qlin_launch_dequantize_q6k_to_f16(src, out, n), "launch_dequantize_q6k_to_f16");
}

// kernel.cuh:141-142
inline void launch_quant_embedding(DType quant_type, const int *input, float *output, const uint8_t *table,
                                   size_t row_bytes, int hidden_size, int input_size) {
    check(qlin_launch_quant_embedding(static_cast<int>(quant_type), input, output, table, row_bytes, hidden_size,
                                      input_size),
          "launch_quant_embedding");
}

// kernel.cuh:300-305, 328-330
inline void launch_mla_absorb_q_nope(DType quant_type, const float *q, const uint8_t *kv_b_weight, size_t row_bytes,
                                     float *q_abs, int n_heads, int qk_nope, int qk_rope, int v_head, int kv_lora) {
    check(qlin_launch_mla_absorb_q_nope(static_cast<int>(quant_type), q, kv_b_weight, row_bytes, q_abs, n_heads,
                                        qk_nope, qk_rope, v_head, kv_lora),
          "launch_mla_absorb_q_nope");
}
inline void launch_mla_absorb_q4_xsum_delta(const float *q, const uint8_t *kv_b_weight, size_t row_bytes,
                                            float *q_abs_xsum_delta, int n_heads, int qk_nope, int qk_rope,
                                            int v_head, int kv_lora) {
    check(qlin_launch_mla_absorb_q4_xsum_delta(q, kv_b_weight, row_bytes, q_abs_xsum_delta, n_heads, qk_nope,
                                               qk_rope, v_head, kv_lora),
          "launch_mla_absorb_q4_xsum_delta");
}
inline void launch_mla_absorb_v(DType quant_type, const uint8_t *kv_b_weight, size_t row_bytes,
                                const float *attn_latent, const float *attn_xsum_delta, float *attn, int n_heads,
                                int qk_nope, int v_head, int kv_lora) {
    check(qlin_launch_mla_absorb_v(static_cast<int>(quant_type), kv_b_weight, row_bytes, attn_latent, attn_xsum_delta,
                                   attn, n_heads, qk_nope, v_head, kv_lora),
          "launch_mla_absorb_v");
}

// kernel.cuh:297-327 -- the Q8_1 latent cache
inline void launch_mla_store_latent_q8_1_device_pos(const float *kv_cache, uint8_t *latent_q8_1_cache, int kv_lora,
                                                    int qk_rope, size_t row_bytes, const int *d_pos) {
    check(qlin_launch_mla_store_latent_q8_1_device_pos(kv_cache, latent_q8_1_cache, kv_lora, qk_rope, row_bytes, d_pos),
          "launch_mla_store_latent_q8_1_device_pos");
}
inline void launch_mla_absorb_scores_device_pos(const float *q_abs, const float *q, const uint8_t *latent_q8_1_cache,
                                                size_t latent_q8_1_row_bytes, const float *q_abs_xsum_delta,
                                                const float *kv_cache, float *scores, int n_heads, int qk_nope,
                                                int qk_rope, int kv_lora, const int *d_pos, int max_seq_len,
                                                float softmax_scale) {
    check(qlin_launch_mla_absorb_scores_device_pos(q_abs, q, latent_q8_1_cache, latent_q8_1_row_bytes, q_abs_xsum_delta,
                                                   kv_cache, scores, n_heads, qk_nope, qk_rope, kv_lora, d_pos,
                                                   max_seq_len, softmax_scale),
          "launch_mla_absorb_scores_device_pos");
}
inline void launch_mla_absorb_context_device_pos(const float *scores, const uint8_t *latent_q8_1_cache,
                                                 size_t latent_q8_1_row_bytes, float *attn_xsum_delta,
                                                 float *attn_latent, int n_heads, int kv_lora, const int *d_pos,
                                                 int max_seq_len) {
    check(qlin_launch_mla_absorb_context_device_pos(scores, latent_q8_1_cache, latent_q8_1_row_bytes, attn_xsum_delta,
                                                    attn_latent, n_heads, kv_lora, d_pos, max_seq_len),
          "launch_mla_absorb_context_device_pos");
}
inline void launch_mla_absorb_attend_device_pos(const float *q_abs, const float *q, const uint8_t *latent_q8_1_cache,
                                                size_t latent_q8_1_row_bytes, const float *q_abs_xsum_delta,
                                                float *attn_xsum_delta, const float *kv_cache, float *attn_latent,
                                                int n_heads, int qk_nope, int qk_rope, int kv_lora, const int *d_pos,
                                                int max_seq_len, float softmax_scale) {
    check(qlin_launch_mla_absorb_attend_device_pos(q_abs, q, latent_q8_1_cache, latent_q8_1_row_bytes,
                                                   q_abs_xsum_delta, attn_xsum_delta, kv_cache, attn_latent, n_heads,
                                                   qk_nope, qk_rope, kv_lora, d_pos, max_seq_len, softmax_scale),
          "launch_mla_absorb_attend_device_pos");
}
inline void launch_mla_project_v_device_pos(DType quant_type, const uint8_t *kv_b_weight, size_t row_bytes,
                                            const uint8_t *latent_q8_1_cache, size_t latent_q8_1_row_bytes,
                                            float *kv_b_cache, int n_heads, int qk_nope, int v_head, int kv_lora,
                                            const int *d_pos) {
    check(qlin_launch_mla_project_v_device_pos(static_cast<int>(quant_type), kv_b_weight, row_bytes, latent_q8_1_cache,
                                               latent_q8_1_row_bytes, kv_b_cache, n_heads, qk_nope, v_head, kv_lora,
                                               d_pos),
          "launch_mla_project_v_device_pos");
}
inline void launch_mla_absorb_context_v_device_pos(const float *scores, const float *kv_b_cache, float *attn,
                                                   int n_heads, int qk_nope, int v_head, const int *d_pos,
                                                   int max_seq_len) {
    check(qlin_launch_mla_absorb_context_v_device_pos(scores, kv_b_cache, attn, n_heads, qk_nope, v_head, d_pos,
                                                      max_seq_len),
          "launch_mla_absorb_context_v_device_pos");
}

}  // namespace qlin_ref

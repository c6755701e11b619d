// qlin_internal.hpp -- launchers shared between the kernel translation units and the C-ABI layer.
// All launchers are asynchronous on the given stream, allocate nothing and never synchronise, so a
// caller may capture them into a HIP graph.  Arguments are validated by the C-ABI layer first.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qlin {

struct DeviceInfo {
    int cu_count = 256;
};
const DeviceInfo &device_info();

// y[r, o] (=|+=) sum_k W[o, k] x[r, k] for r < m.
hipError_t gemv(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y, int out_dim,
                int in_dim, int m, bool add, hipStream_t s);

// Several GEMVs that share x (same type, in_dim and row_bytes), as one launch when possible.
constexpr int kMaxStreamMats = 4;
hipError_t gemv_multi(int type, const uint8_t *const *w, float *const *y, const int *rows, int nmat,
                      size_t row_bytes, const float *x, int in_dim, hipStream_t s);

// Streaming Q4_K kernels (m == 1): preconditions, several matrices sharing x, fused SwiGLU.
bool q4k_stream_ok(const uint8_t *const *w, int nmat, size_t row_bytes, const float *x, int total, int in_dim,
                   bool swiglu);
hipError_t q4k_stream_gemv(const uint8_t *const *w, float *const *y, const int *rows, int nmat, size_t row_bytes,
                           const float *x, int in_dim, bool add, hipStream_t s);
hipError_t q4k_stream_swiglu(const uint8_t *wg, const uint8_t *wu, size_t row_bytes, const float *x, float *act,
                             int ffn_dim, int in_dim, hipStream_t s);

// The router's inputs and outputs when a MoE decode also routes (logits [tokens, n_experts] in, ids
// and weights [tokens, k] out, as router_topk writes them).
struct MoeRouter {
    const float *logits;
    float scaling;
    int *ids;
    float *w;
};
// The routed part of a batched MoE decode handed to a later launch instead of the combine launch:
// per-route results yr [tokens * k, hidden] and the routes' ids and weights [tokens, k].  A launch
// that applies it adds, per (token t, hidden row h), the routes in route order as the combine does:
// total = fmaf(yr[t k + r][h], rw[t k + r], total) over the routes with 0 <= id < n_experts, from 0.
struct RouteCombine {
    const float *yr;
    const int *ids;
    const float *rw;
    int k, n_experts;
};
// An RMSNorm applied to x as the decode kernels stage it: x[j] * rsqrt(mean x^2 + eps) * w[j], w bf16
// (type 0) or f16 (1), plus one if one_plus.
struct RmsNorm {
    const uint16_t *w;
    int type;
    float eps;
    int one_plus;
};
// Matrix-core decode kernels (m == 1) for Q4_K, Q4_0, Q8_0, Q5_0 and Q6_K, same contracts as the streaming ones;
// with norm, x is first normalized (in the staging, not in memory).
bool mfma_ok(int type, const uint8_t *const *w, int nmat, size_t row_bytes, const float *x, int total, int in_dim,
             bool swiglu);
// One matrix's decode GEMV (optionally normalizing x) and the argmax of its outputs, as qlin_launch_argmax
// gives it: every workgroup writes its pick to pairs_v / pairs_i (mfma_gemv_pairs(...) entries: the
// launch's workgroup count, 0 when the matrix-core kernel does not take the shape), and one more launch
// reduces them into *out_idx.
int mfma_gemv_pairs(int type, const uint8_t *w, size_t row_bytes, const float *x, int out_dim, int in_dim);
hipError_t mfma_gemv_argmax(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y, int out_dim,
                            int in_dim, const RmsNorm *norm, float *pairs_v, int *pairs_i, int *out_idx,
                            hipStream_t s);
hipError_t mfma_gemv(int type, const uint8_t *const *w, float *const *y, const int *rows, int nmat,
                     size_t row_bytes, const float *x, int in_dim, bool add, hipStream_t s,
                     const RmsNorm *norm = nullptr);
hipError_t mfma_swiglu(int type, const uint8_t *wg, const uint8_t *wu, size_t row_bytes, const float *x, float *act,
                       int ffn_dim, int in_dim, hipStream_t s, const RmsNorm *norm = nullptr);
// The routed-expert forms (qlin_mfma_gemv.hip): route r's weights are expert ids[r]'s (negative: none).
// SwiGLU: act[r, o] = silu(Wg[e_r] x) (Wu[e_r] x), 0 for no expert.  Down: out[h] += the routes' dots
// Wd[e_r][h] . act[r] added in route order as fmaf(dot, rw[r], total).  mfma_routed_ok takes the
// SwiGLU's (rows = ffn, k = in_dim) or the down projection's (rows = hidden, k = ffn) shape.
bool mfma_routed_ok(int type, bool swiglu, const uint8_t *w0, const uint8_t *w1, size_t expert_bytes,
                    size_t row_bytes, const float *x, int routes, int rows, int k);
// router: the routes are router_topk's picks of the token's logits (n_experts <= 64), made in the
// launch and written to router->ids / router->w; ids is then not read.  sh_routes > 0: sh_routes more
// routes after them, the consecutive ffn_dim-row blocks of the shared gate and up matrices sh_wg / sh_wu
// (same format and row stride), written after the routes' rows in act.
hipError_t mfma_swiglu_routed(int type, const uint8_t *wg, const uint8_t *wu, size_t expert_bytes, size_t row_bytes,
                              const float *x, const int *ids, float *act, int routes, int ffn_dim, int in_dim,
                              hipStream_t s, const MoeRouter *router = nullptr, int n_experts = 0,
                              const uint8_t *sh_wg = nullptr, const uint8_t *sh_wu = nullptr, int sh_routes = 0);
hipError_t mfma_down_routed(int type, const uint8_t *wd, size_t expert_bytes, size_t row_bytes, const float *act,
                            const int *ids, const float *rw, float *out, int routes, int hidden, int ffn_dim,
                            hipStream_t s);

// m > 1 rows of f32 activations (qlin_dense.hip), for fewer than kF32GemmMinRows rows or the other
// formats: Q4_K on the bf16 matrix cores with x as bf16 hi + lo (x to about 2^-17 of itself, products
// exact, f32 accumulation), the other formats on the f32 matrix cores with the reference's f32 operands.
// Mode 0 stores y[r, o], 1 adds into it, 2 writes act[r, o] = silu(gate . x_r) * (up . x_r) with w1 the up
// matrix.
bool dense_ok(int type, const uint8_t *w0, const uint8_t *w1, size_t row_bytes, const float *x, int in_dim);
// mode 1 (y +=) with combine: y = (y + the routed total) + the product, as the combine launch and then
// the plain mode 1 give it
hipError_t dense_matmul(int type, const uint8_t *w0, const uint8_t *w1, size_t row_bytes, const float *x, float *y,
                        int out_dim, int in_dim, int m, int mode, hipStream_t s, const RouteCombine *combine = nullptr);

// MLA over the Q8_1 latent cache (qlin_mla_latent.hip); pos is read from d_pos on the device.
hipError_t mla_store_latent_q8_1(const float *kv_cache, uint8_t *cache, int kv_lora, int qk_rope, size_t row_bytes,
                                 const int *d_pos, hipStream_t s);
hipError_t mla_absorb_scores(const float *q_abs, const float *q, const uint8_t *cache, size_t cache_row_bytes,
                             const float *delta, const float *kv_cache, float *scores, int n_heads, int qk_nope,
                             int qk_rope, int kv_lora, const int *d_pos, int max_seq, float scale, hipStream_t s);
hipError_t mla_absorb_context(const float *scores, const uint8_t *cache, size_t cache_row_bytes, float *delta_out,
                              float *latent_out, int n_heads, int kv_lora, const int *d_pos, int max_seq,
                              hipStream_t s);
// The fused scores + softmax + context of one head per workgroup (scores of every position in LDS).
bool mla_attend_ok(int max_seq, int kv_lora, int qk_rope);
hipError_t mla_absorb_attend(const float *q_abs, const float *q, const uint8_t *cache, size_t cache_row_bytes,
                             const float *delta, float *delta_out, const float *kv_cache, float *latent_out,
                             int n_heads, int qk_nope, int qk_rope, int kv_lora, const int *d_pos, int max_seq,
                             float scale, hipStream_t s);
hipError_t mla_project_v(int type, const uint8_t *w, size_t row_bytes, const uint8_t *cache, size_t cache_row_bytes,
                         float *kv_b_cache, int n_heads, int qk_nope, int v_head, int kv_lora, const int *d_pos,
                         hipStream_t s);
hipError_t mla_absorb_context_v(const float *scores, const float *kv_b_cache, float *attn, int n_heads, int qk_nope,
                                int v_head, const int *d_pos, int max_seq, hipStream_t s);

// The per-element fallback used for any type / alignment (exposed for tests of the fast paths).
hipError_t gemv_generic(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y,
                        int out_dim, int in_dim, int m, bool add, hipStream_t s);

// Whole-stream dequantization: n elements to f32 or to f16 bit patterns (RNE of the f32 value).
hipError_t dequant(int type, const uint8_t *src, void *out, int64_t n, bool to_f16, hipStream_t s);

// Q8_1 activation quantizer (36 B per 32 values) and the weight x Q8_1 matmul.
hipError_t quantize_q8_1(const float *x, uint8_t *xq, int in_dim, int m, bool raw_sum, hipStream_t s);
// Q8_0 / Q5_0 / Q4_0 x Q8_1 prefill GEMM on the fp16 matrix cores (qlin_qblk_gemm.hip).
bool qblk_gemm_ok(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, int in_dim);
hipError_t qblk_gemm_q8_1(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, float *y, int out_dim,
                          int in_dim, int m, hipStream_t s);
// Q4_K / Q6_K x f32 activations, the prefill GEMM of quant_matmul for m >= kF32GemmMinRows rows, on the
// fp16 matrix cores (qlin_f32_gemm.hip); fewer rows take dense_matmul.  add: y += the product.
#ifndef QLIN_F32_GEMM_MIN_ROWS
#define QLIN_F32_GEMM_MIN_ROWS 64
#endif
constexpr int kF32GemmMinRows = QLIN_F32_GEMM_MIN_ROWS;
bool f32_gemm_ok(int type, const uint8_t *w, size_t row_bytes, const float *x, int in_dim);
hipError_t f32_gemm(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y, int out_dim, int in_dim,
                    int m, bool add, hipStream_t s);
// Q4_K x Q8_1 prefill GEMM on the fp16 matrix cores (qlin_q4k_gemm.hip).
bool q4k_gemm_ok(const uint8_t *w, size_t row_bytes, const uint8_t *xq, int in_dim);
hipError_t q4k_gemm_q8_1(const uint8_t *w, size_t row_bytes, const uint8_t *xq, float *y, int out_dim, int in_dim,
                         int m, hipStream_t s);
hipError_t matmul_q8_1(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, float *y,
                       int out_dim, int in_dim, int m, hipStream_t s);

// Q8_1-activation variants (qlin_q8_1_moe.hip): the MMQ layout, the MoE SwiGLU over one Q8_1 x and
// the routed down projections over Q8_1 (or f32, quantized on the fly) activations.
hipError_t quantize_q8_1_mmq(const float *x, uint8_t *xq, int in_dim, int m, bool raw_sum, hipStream_t s);
hipError_t matmul_q8_1_mmq(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, float *y, int out_dim,
                           int in_dim, int m, hipStream_t s);
hipError_t swiglu_indexed_q8_1(int type, const uint8_t *wg, const uint8_t *wu, size_t g_expert_bytes,
                               size_t u_expert_bytes, size_t g_row_bytes, size_t u_row_bytes, const uint8_t *xq,
                               const int *expert_ids, float *act, int k, int ffn_dim, int in_dim, hipStream_t s);
hipError_t down_q8_1_indexed_accum(int type, bool f32_act, const uint8_t *wd, size_t d_expert_bytes,
                                   size_t d_row_bytes, const void *act, const int *expert_ids, const float *route_w,
                                   float *out, int k, int hidden, int ffn_dim, hipStream_t s);

// MoE.
hipError_t moe_accumulate(const float *expert_out, float weight, const float *weight_dev, float *out, int n,
                          hipStream_t s);
hipError_t argmax(const float *logits, int n, int *out_idx, hipStream_t s);
hipError_t router_topk(const float *logits, int *top_idx, float *top_w, int tokens, int n_experts,
                       int k, float routed_scaling, hipStream_t s);
hipError_t swiglu(int type, const uint8_t *wg, const uint8_t *wu, size_t g_row_bytes,
                  size_t u_row_bytes, const float *x, float *act, int ffn_dim, int in_dim,
                  hipStream_t s);
hipError_t swiglu_indexed(int type, const uint8_t *wg, const uint8_t *wu, size_t g_expert_bytes,
                          size_t u_expert_bytes, size_t g_row_bytes, size_t u_row_bytes,
                          const float *x, const int *expert_ids, float *act, int k, int ffn_dim,
                          int in_dim, hipStream_t s);
hipError_t down_indexed_ordered(int type, const uint8_t *wd, size_t d_expert_bytes,
                                size_t d_row_bytes, const float *act, const int *expert_ids,
                                const float *route_w, float *out, int k, int hidden, int ffn_dim,
                                hipStream_t s);

// Batched routed decode, each selected expert read once per pass over its routes (qlin_moe_grouped.hip).
size_t moe_grouped_workspace(int tokens, int k, int n_experts, int ffn_dim, int hidden);
// The per-device scratch of the allocation-free batched entry point (kMoeStaticScratchBytes), its
// address resolved once per device; nullptr when it cannot be.
constexpr size_t kMoeStaticScratchBytes = size_t{8} << 20;
void *moe_static_scratch();
bool moe_grouped_shape_ok(int n_experts, int64_t routes);
bool moe_grouped_up_ok(int type, const uint8_t *wg, const uint8_t *wu, size_t expert_bytes, size_t row_bytes,
                       const float *x, int in_dim, int ffn_dim, int n_experts, int routes);
// router non-null: ids and rw are ignored, the routes are router_topk's of the logits (inside the gate/up
// launch for n_experts <= 64 when its LDS allows, else one router launch first).  defer non-null: out is
// not touched; the combine is left to the caller, whose launch applies *defer (filled here).
// The shared experts' SwiGLU over the batch, handed to the batched MoE decode's gate/up launch:
// act [tokens, rows] = SiLU(wg x) * (wu x) for Q4_K gate and up matrices of row stride rb (K = the
// routed in_dim), as q4k_dense_kernel computes it.  moe_grouped sets *done when its launch took it.
struct SharedUp {
    const uint8_t *wg, *wu;
    size_t rb;
    float *act;
    int rows;
    bool *done;
};
hipError_t moe_grouped(int gu_type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t g_rb, int d_type,
                       const uint8_t *wd, size_t d_eb, size_t d_rb, int n_experts, int ffn_dim, int in_dim,
                       int hidden, const float *x, const int *ids, const float *rw, void *workspace, float *out,
                       int tokens, int k, hipStream_t s, const MoeRouter *router = nullptr,
                       RouteCombine *defer = nullptr, const SharedUp *shared = nullptr);

// Quantized embedding rows and the MLA latent-absorption products over kv_b (qlin_embed_mla.hip).
hipError_t quant_embedding(int type, const int *ids, float *out, const uint8_t *table, size_t row_bytes, int hidden,
                           int n, hipStream_t s);
hipError_t mla_absorb_q_nope(int type, const float *q, const uint8_t *w, size_t row_bytes, float *q_abs, int n_heads,
                             int qk_nope, int qk_rope, int v_head, int kv_lora, hipStream_t s);
hipError_t mla_absorb_q4_xsum_delta(const float *q, const uint8_t *w, size_t row_bytes, float *delta, int n_heads,
                                    int qk_nope, int qk_rope, int v_head, int kv_lora, hipStream_t s);
hipError_t mla_absorb_v(int type, const uint8_t *w, size_t row_bytes, const float *latent, const float *delta,
                        float *attn, int n_heads, int qk_nope, int v_head, int kv_lora, hipStream_t s);

}  // namespace qlin

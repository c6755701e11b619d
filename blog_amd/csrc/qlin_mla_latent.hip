// qlin_mla_latent.hip -- the MLA decode kernels over the Q8_1 latent cache, gfx950.
//
// The latent cache holds one Q8_1 row (kernel.cu:1679-1720 blocks, 36 bytes per 32 values) per
// position: the RMS-normed latent of kv_a.  With pos = *d_pos (device memory, as the reference's
// device-pos launchers read it) and L(t, k) = d * q the dequantized latent element k of row t:
//
//   store      cache[pos] = Q8_1(kv_cache[pos, 0 .. kv_lora))             (kernel.cu:2945-2978)
//   scores     s[h, t] = scale * ( sum_k q_abs[h, k] L(t, k) + sum_r q_rope[h, r] k_rope(t, r)
//                        + sum_b delta[h, b] (S(t, b) - sum_l L(t, 32b + l)) ),  t <= pos
//                                                                            (kernel.cu:3157-3196)
//   context    p[h, t] = exp(s[h, t] - max_t s[h]) / (sum_t exp(...) + 1e-9);
//              latent[h, k] = sum_t p[h, t] L(t, k);  delta[h, b] = sum_t p[h, t] (S(t, b) - ...)
//                                                                            (kernel.cu:3198-3257)
//   attend     scores, softmax (fast exp, no 1e-9) and context in one launch   (kernel.cu:3078-3155)
//   project_v  kv_b_cache[pos, v row r of head h] = W_kv_b[r] . cache[pos] with the Q8_1 block-dot
//              semantics of quant_matmul_q8_1                               (kernel.cu:3259-3361)
//   context_v  attn[h, v] = sum_t p[h, t] kv_b_cache[t, v row of head h]   (kernel.cu:3368-3415)
//
// S(t, b) is the block's stored f16 sum and the inner sum is the block's dequantized values added in
// order.  The products run on v_mfma_f32_16x16x4_f32 where heads meet positions (scores: heads x
// positions; context: heads x latent columns over positions); operands are the reference's f32 values
// and only the summation order differs.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "qlin_mfma.hpp"
#include "qlin_q8_1.hpp"

namespace qlin {
namespace {

// S(t, b) - sum_l L(t, 32b + l) of the block at blk (l over the kv_lora - 32b valid values).
__device__ __forceinline__ float block_sum_delta(const uint8_t *blk, int valid) {
    const float d = f16_bits_to_f32(ld_u16(blk));
    const int8_t *q = reinterpret_cast<const int8_t *>(blk + 4);
    float sum = 0.0f;
    for (int l = 0; l < 32 && l < valid; ++l) sum = __fadd_rn(sum, __fmul_rn(d, static_cast<float>(q[l])));
    return __fsub_rn(f16_bits_to_f32(ld_u16(blk + 2)), sum);
}

__global__ __launch_bounds__(64) void store_latent_kernel(const float *__restrict__ kv_cache, uint8_t *cache,
                                                          int kv_lora, int qk_rope, size_t row_bytes, int nblk,
                                                          const int *__restrict__ d_pos) {
    const int b = blockIdx.x * 64 + threadIdx.x;
    const int pos = *d_pos;
    if (b >= nblk || pos < 0) return;
    const float *src = kv_cache + static_cast<size_t>(pos) * (kv_lora + qk_rope) + b * 32;
    quantize_block_q8_1(src, kv_lora - b * 32, cache + static_cast<size_t>(pos) * row_bytes + b * 36, false);
}

struct ScoreArgs {
    const float *q_abs, *q;
    const uint8_t *cache;
    size_t crb;
    const float *delta, *kv_cache;
    float *scores;
    int n_heads, qk_nope, qk_rope, kv_lora, max_seq;
    const int *d_pos;
    float scale;
};

// One wave per (16 positions, 16 heads): lane l supplies head l % 16 (A) and position l % 16 (B);
// the 8 MFMAs of a 32-value block take its values 8g .. 8g+7 in k-slot g = l / 16.
__global__ __launch_bounds__(64) void scores_kernel(const ScoreArgs a) {
    const int pos = min(*a.d_pos, a.max_seq - 1);
    const int t0 = blockIdx.x * 16;
    if (t0 > pos) return;  // uniform (also pos < 0)
    const int lane = threadIdx.x, n = lane & 15, g = lane >> 4;
    const int h0 = blockIdx.y * 16;
    const int hn = min(h0 + n, a.n_heads - 1), tn = min(t0 + n, pos);
    const int nb = (a.kv_lora + 31) / 32;
    const float *qa = a.q_abs + static_cast<size_t>(hn) * a.kv_lora;
    const uint8_t *row = a.cache + static_cast<size_t>(tn) * a.crb;

    f32x4 D = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + static_cast<size_t>(b) * 36;
        const float d = f16_bits_to_f32(ld_u16(blk));
        const uint32_t w0 = *reinterpret_cast<const uint32_t *>(blk + 4 + 8 * g);
        const uint32_t w1 = *reinterpret_cast<const uint32_t *>(blk + 8 + 8 * g);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int k = b * 32 + 8 * g + i;
            const int qv = static_cast<int8_t>(((i < 4 ? w0 : w1) >> (8 * (i & 3))) & 0xffu);
            const bool in = k < a.kv_lora;
            D = mfma_f32(in ? qa[k] : 0.0f, in ? __fmul_rn(d, static_cast<float>(qv)) : 0.0f, D);
        }
    }
    const float *qr = a.q + static_cast<size_t>(hn) * (a.qk_nope + a.qk_rope) + a.qk_nope;
    const float *kr = a.kv_cache + static_cast<size_t>(tn) * (a.kv_lora + a.qk_rope) + a.kv_lora;
    for (int r0 = 0; r0 < a.qk_rope; r0 += 32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = r0 + 8 * g + i;
            const bool in = r < a.qk_rope;
            D = mfma_f32(in ? qr[r] : 0.0f, in ? kr[r] : 0.0f, D);
        }
    }
    const float *dl = a.delta + static_cast<size_t>(hn) * nb;
    for (int b0 = 0; b0 < nb; b0 += 4) {
        const int b = b0 + g;
        const bool in = b < nb;
        D = mfma_f32(in ? dl[b] : 0.0f, in ? block_sum_delta(row + static_cast<size_t>(b) * 36, a.kv_lora - 32 * b) : 0.0f,
                     D);
    }
    const int t = t0 + n;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int h = h0 + 4 * g + r;
        if (h < a.n_heads && t <= pos) a.scores[static_cast<size_t>(h) * a.max_seq + t] = __fmul_rn(D[r], a.scale);
    }
}

constexpr int kCWaves = 16, kCThreads = kCWaves * 64;
constexpr int kCBatch = 8;  // MFMAs (4 positions each) whose operands a wave loads together

struct ContextArgs {
    const float *scores;
    const uint8_t *cache;
    size_t crb;
    float *delta_out, *latent_out;
    int n_heads, kv_lora, max_seq;
    const int *d_pos;
};

// max_t s[h] and sum_t exp(s[h, t] - max) + 1e-9 for heads h0 .. h0+15 into s_max / s_den (wave w
// takes head h0 + w).  Heads past n_heads get (-inf, 1e-9); pos < 0 the same for every head.
__device__ __forceinline__ void softmax_stats(const float *scores, int max_seq, int n_heads, int h0, int pos,
                                              float *s_max, float *s_den) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = h0 + wave;
    const float *sh = scores + static_cast<size_t>(min(h, n_heads - 1)) * max_seq;
    float m = -INFINITY;
    if (h < n_heads)
        for (int t = lane; t <= pos; t += 64) m = fmaxf(m, sh[t]);
    m = wave_max(m);
    float s = 0.0f;
    if (h < n_heads)
        for (int t = lane; t <= pos; t += 64) s += expf(sh[t] - m);
    s = wave_sum(s);
    if (lane == 0) {
        s_max[wave] = m;
        s_den[wave] = s + 1e-9f;
    }
}

// A workgroup per (16 output columns, 16 heads); columns 0 .. kv_lora-1 are latent values, the last
// tiles the per-block sum corrections.  Wave w takes positions 4(w + 16 i) .. +3; lane l supplies
// head l % 16 (A = probability) and column l % 16 (B = latent value) at position 4i' + l / 16.
__global__ __launch_bounds__(kCThreads) void context_kernel(const ContextArgs a) {
    static_assert(kCWaves == 16, "one head per wave in the softmax statistics");
    __shared__ float s_max[16], s_den[16];
    __shared__ f32x4 part[kCWaves][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 15, g = lane >> 4;
    const int pos = min(*a.d_pos, a.max_seq - 1);
    const int h0 = blockIdx.y * 16;
    const int nb = (a.kv_lora + 31) / 32, lat_tiles = (a.kv_lora + 15) / 16;
    const bool corr = static_cast<int>(blockIdx.x) >= lat_tiles;
    const int col = (corr ? blockIdx.x - lat_tiles : blockIdx.x) * 16 + n;
    const bool col_in = corr ? col < nb : col < a.kv_lora;

    softmax_stats(a.scores, a.max_seq, a.n_heads, h0, pos, s_max, s_den);
    __syncthreads();
    const int hn = h0 + n;
    const bool h_in = hn < a.n_heads;
    const float mx = s_max[n], den = s_den[n];
    const float *sh = a.scores + static_cast<size_t>(min(hn, a.n_heads - 1)) * a.max_seq;

    f32x4 D = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int base = 4 * wave; base <= pos; base += 4 * kCWaves * kCBatch) {
        float av[kCBatch], bv[kCBatch];
#pragma unroll
        for (int u = 0; u < kCBatch; ++u) {
            const int t = base + u * 4 * kCWaves + g;
            av[u] = 0.0f;
            bv[u] = 0.0f;
            if (t <= pos) {
                if (h_in) av[u] = expf(sh[t] - mx) / den;
                const uint8_t *row = a.cache + static_cast<size_t>(t) * a.crb;
                if (col_in) {
                    if (corr) {
                        bv[u] = block_sum_delta(row + static_cast<size_t>(col) * 36, a.kv_lora - 32 * col);
                    } else {
                        const uint8_t *blk = row + static_cast<size_t>(col >> 5) * 36;
                        bv[u] = __fmul_rn(f16_bits_to_f32(ld_u16(blk)),
                                          static_cast<float>(reinterpret_cast<const int8_t *>(blk + 4)[col & 31]));
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kCBatch; ++u) D = mfma_f32(av[u], bv[u], D);
    }
    part[wave][lane] = D;
    __syncthreads();
    if (tid < 256) {  // (head, column) of the tile; lane (column, g) of D holds heads 4g .. 4g+3
        const int hl = tid >> 4, cl = tid & 15;
        const int l = (hl >> 2) * 16 + cl, r = hl & 3;
        float v = 0.0f;
        for (int w = 0; w < kCWaves; ++w) v += part[w][l][r];
        const int h = h0 + hl, c = (corr ? blockIdx.x - lat_tiles : blockIdx.x) * 16 + cl;
        if (h < a.n_heads) {
            if (corr && c < nb) a.delta_out[static_cast<size_t>(h) * nb + c] = v;
            else if (!corr && c < a.kv_lora) a.latent_out[static_cast<size_t>(h) * a.kv_lora + c] = v;
        }
    }
}

// One wave per (head, v row): kv_b row h * (qk_nope + v_head) + qk_nope + v against the latent row.
template <int T>
__global__ __launch_bounds__(256) void project_v_kernel(const uint8_t *__restrict__ w, size_t rb,
                                                        const uint8_t *__restrict__ cache, size_t crb,
                                                        float *__restrict__ kvb_cache, int n_heads, int qk_nope,
                                                        int v_head, int kv_lora, const int *__restrict__ d_pos) {
    const int wv = static_cast<int>((blockIdx.x * 256 + threadIdx.x) >> 6), lane = threadIdx.x & 63;
    const int pos = *d_pos;
    if (wv >= n_heads * v_head || pos < 0) return;  // whole waves
    const int h = wv / v_head, v = wv - h * v_head;
    const int r = h * (qk_nope + v_head) + qk_nope + v;
    const uint8_t *wr = w + static_cast<size_t>(r) * rb;
    const uint8_t *xr = cache + static_cast<size_t>(pos) * crb;
    float acc = 0.0f;
    for (int qb = lane; qb < kv_lora / 32; qb += 64) acc += block_dot_q8_1<T>(wr, qb, xr + static_cast<size_t>(qb) * 36);
    acc = wave_sum(acc);
    if (lane == 0) kvb_cache[static_cast<size_t>(pos) * n_heads * (qk_nope + v_head) + r] = acc;
}

constexpr int kVMax = 4;  // v_head <= 64 * kVMax

// A workgroup per head: wave w takes positions w, w + 16, ...; lane l columns l, l + 64, ...
__global__ __launch_bounds__(kCThreads) void context_v_kernel(const float *__restrict__ scores,
                                                              const float *__restrict__ kvb_cache,
                                                              float *__restrict__ attn, int n_heads, int qk_nope,
                                                              int v_head, const int *__restrict__ d_pos,
                                                              int max_seq) {
    __shared__ float s_part[2][kCWaves];
    __shared__ float s_acc[kCWaves][64 * kVMax];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x;
    const int pos = min(*d_pos, max_seq - 1);
    const float *sh = scores + static_cast<size_t>(h) * max_seq;
    // statistics over the whole workgroup: per-wave max, then per-wave sums of exp(s - max)
    float m = -INFINITY;
    for (int t = tid; t <= pos; t += kCThreads) m = fmaxf(m, sh[t]);
    m = wave_max(m);
    if (lane == 0) s_part[0][wave] = m;
    __syncthreads();
    m = -INFINITY;
    for (int w = 0; w < kCWaves; ++w) m = fmaxf(m, s_part[0][w]);
    float s = 0.0f;
    for (int t = tid; t <= pos; t += kCThreads) s += expf(sh[t] - m);
    s = wave_sum(s);
    if (lane == 0) s_part[1][wave] = s;
    __syncthreads();
    s = 0.0f;
    for (int w = 0; w < kCWaves; ++w) s += s_part[1][w];
    const float den = s + 1e-9f;

    const int stride = n_heads * (qk_nope + v_head);
    const float *vbase = kvb_cache + static_cast<size_t>(h) * (qk_nope + v_head) + qk_nope;
    float acc[kVMax] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int t = wave; t <= pos; t += kCWaves) {
        const float p = expf(sh[t] - m) / den;
        const float *vr = vbase + static_cast<size_t>(t) * stride;
#pragma unroll
        for (int c = 0; c < kVMax; ++c)
            if (lane + 64 * c < v_head) acc[c] = fmaf(p, vr[lane + 64 * c], acc[c]);
    }
#pragma unroll
    for (int c = 0; c < kVMax; ++c) s_acc[wave][lane + 64 * c] = acc[c];
    __syncthreads();
    for (int v = tid; v < v_head; v += kCThreads) {
        float o = 0.0f;
        for (int w = 0; w < kCWaves; ++w) o += s_acc[w][v];
        attn[static_cast<size_t>(h) * v_head + v] = o;
    }
}

constexpr int kAMaxSeq = 32768;  // attend: scores of every position in LDS
constexpr size_t kMaxLds = 160 * 1024;

// Scores, softmax and context of one head in one workgroup (the fused form): the scores of all
// positions stay in LDS.  exp is the fast __expf and the denominator has no 1e-9 term, as in
// kernel.cu:3078-3155.
__global__ __launch_bounds__(kCThreads) void attend_kernel(const ScoreArgs a, float *delta_out, float *latent_out) {
    extern __shared__ float s_sc[];  // [max_seq] scores, then q_abs [kv_lora], q_rope [qk_rope], delta [nb]
    __shared__ float s_red[2][kCWaves];
    __shared__ float s_out[kCWaves][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x;
    const int pos = min(*a.d_pos, a.max_seq - 1);
    const int nb = (a.kv_lora + 31) / 32;
    float *s_qa = s_sc + a.max_seq, *s_qr = s_qa + a.kv_lora, *s_dl = s_qr + a.qk_rope;
    for (int i = tid; i < a.kv_lora; i += kCThreads) s_qa[i] = a.q_abs[static_cast<size_t>(h) * a.kv_lora + i];
    for (int i = tid; i < a.qk_rope; i += kCThreads)
        s_qr[i] = a.q[static_cast<size_t>(h) * (a.qk_nope + a.qk_rope) + a.qk_nope + i];
    for (int i = tid; i < nb; i += kCThreads) s_dl[i] = a.delta[static_cast<size_t>(h) * nb + i];
    __syncthreads();

    // scores: a wave per position, lanes over the latent values, the rope pair and the block sums
    float m = -INFINITY;
    for (int t = wave; t <= pos; t += kCWaves) {
        const uint8_t *row = a.cache + static_cast<size_t>(t) * a.crb;
        const float *kr = a.kv_cache + static_cast<size_t>(t) * (a.kv_lora + a.qk_rope) + a.kv_lora;
        float dot = 0.0f;
        for (int k = lane; k < a.kv_lora; k += 64) {
            const uint8_t *blk = row + static_cast<size_t>(k >> 5) * 36;
            dot = fmaf(s_qa[k], __fmul_rn(f16_bits_to_f32(ld_u16(blk)),
                                          static_cast<float>(reinterpret_cast<const int8_t *>(blk + 4)[k & 31])), dot);
        }
        for (int r = lane; r < a.qk_rope; r += 64) dot = fmaf(s_qr[r], kr[r], dot);
        for (int b = lane; b < nb; b += 64)
            dot = fmaf(s_dl[b], block_sum_delta(row + static_cast<size_t>(b) * 36, a.kv_lora - 32 * b), dot);
        dot = wave_sum(dot);
        const float sc = __fmul_rn(dot, a.scale);
        if (lane == 0) s_sc[t] = sc;
        m = fmaxf(m, sc);
    }
    if (lane == 0) s_red[0][wave] = m;
    __syncthreads();
    m = -INFINITY;
    for (int w = 0; w < kCWaves; ++w) m = fmaxf(m, s_red[0][w]);
    float den = 0.0f;
    for (int t = tid; t <= pos; t += kCThreads) {
        const float e = __expf(s_sc[t] - m);
        s_sc[t] = e;
        den += e;
    }
    den = wave_sum(den);
    if (lane == 0) s_red[1][wave] = den;
    __syncthreads();
    den = 0.0f;
    for (int w = 0; w < kCWaves; ++w) den += s_red[1][w];

    // context: a column per lane, the positions split over the waves, wave partials added in order
    const int ncol = a.kv_lora + nb;
    for (int c0 = 0; c0 < ncol; c0 += 64) {
        const int c = c0 + lane;
        float acc = 0.0f;
        if (c < ncol)
            for (int t = wave; t <= pos; t += kCWaves) {
                const uint8_t *row = a.cache + static_cast<size_t>(t) * a.crb;
                float v;
                if (c < a.kv_lora) {
                    const uint8_t *blk = row + static_cast<size_t>(c >> 5) * 36;
                    v = __fmul_rn(f16_bits_to_f32(ld_u16(blk)),
                                  static_cast<float>(reinterpret_cast<const int8_t *>(blk + 4)[c & 31]));
                } else {
                    const int b = c - a.kv_lora;
                    v = block_sum_delta(row + static_cast<size_t>(b) * 36, a.kv_lora - 32 * b);
                }
                acc = fmaf(s_sc[t] / den, v, acc);
            }
        s_out[wave][lane] = acc;
        __syncthreads();
        if (tid < 64 && c < ncol) {
            float o = 0.0f;
            for (int w = 0; w < kCWaves; ++w) o += s_out[w][tid];
            if (c < a.kv_lora) latent_out[static_cast<size_t>(h) * a.kv_lora + c] = o;
            else delta_out[static_cast<size_t>(h) * nb + (c - a.kv_lora)] = o;
        }
        __syncthreads();
    }
}

template <int T> struct ProjectV {
    static void run(const uint8_t *w, size_t rb, const uint8_t *cache, size_t crb, float *kvb, int nh, int qn, int vh,
                    int kl, const int *d_pos, hipStream_t s) {
        hipLaunchKernelGGL(project_v_kernel<T>, dim3((nh * vh + 3) / 4), dim3(256), 0, s, w, rb, cache, crb, kvb, nh,
                           qn, vh, kl, d_pos);
    }
};

}  // namespace

hipError_t mla_store_latent_q8_1(const float *kv_cache, uint8_t *cache, int kv_lora, int qk_rope, size_t row_bytes,
                                 const int *d_pos, hipStream_t s) {
    const int nblk = static_cast<int>(row_bytes / 36);
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(store_latent_kernel, dim3((nblk + 63) / 64), dim3(64), 0, s, kv_cache, cache, kv_lora, qk_rope,
                       row_bytes, nblk, d_pos);
    return hipGetLastError();
}

hipError_t mla_absorb_scores(const float *q_abs, const float *q, const uint8_t *cache, size_t crb,
                             const float *delta, const float *kv_cache, float *scores, int n_heads, int qk_nope,
                             int qk_rope, int kv_lora, const int *d_pos, int max_seq, float scale, hipStream_t s) {
    if (n_heads == 0 || max_seq == 0) return hipSuccess;
    const ScoreArgs a{q_abs, q, cache, crb, delta, kv_cache, scores, n_heads, qk_nope, qk_rope, kv_lora, max_seq,
                      d_pos, scale};
    hipLaunchKernelGGL(scores_kernel, dim3((max_seq + 15) / 16, (n_heads + 15) / 16), dim3(64), 0, s, a);
    return hipGetLastError();
}

hipError_t mla_absorb_context(const float *scores, const uint8_t *cache, size_t crb, float *delta_out,
                              float *latent_out, int n_heads, int kv_lora, const int *d_pos, int max_seq,
                              hipStream_t s) {
    if (n_heads == 0 || kv_lora == 0) return hipSuccess;
    const ContextArgs a{scores, cache, crb, delta_out, latent_out, n_heads, kv_lora, max_seq, d_pos};
    const int nb = (kv_lora + 31) / 32;
    const dim3 grid((kv_lora + 15) / 16 + (nb + 15) / 16, (n_heads + 15) / 16);
    hipLaunchKernelGGL(context_kernel, grid, dim3(kCThreads), 0, s, a);
    return hipGetLastError();
}

size_t mla_attend_lds(int max_seq, int kv_lora, int qk_rope) {
    return sizeof(float) * (static_cast<size_t>(max_seq) + kv_lora + qk_rope + (kv_lora + 31) / 32);
}

bool mla_attend_ok(int max_seq, int kv_lora, int qk_rope) {
    return max_seq <= kAMaxSeq && mla_attend_lds(max_seq, kv_lora, qk_rope) + sizeof(float) * 2 * kCWaves +
                                          sizeof(float) * kCWaves * 64 <= kMaxLds;
}

hipError_t mla_absorb_attend(const float *q_abs, const float *q, const uint8_t *cache, size_t crb, const float *delta,
                             float *delta_out, const float *kv_cache, float *latent_out, int n_heads, int qk_nope,
                             int qk_rope, int kv_lora, const int *d_pos, int max_seq, float scale, hipStream_t s) {
    if (n_heads == 0) return hipSuccess;
    const ScoreArgs a{q_abs, q, cache, crb, delta, kv_cache, nullptr, n_heads, qk_nope, qk_rope, kv_lora, max_seq,
                      d_pos, scale};
    hipLaunchKernelGGL(attend_kernel, dim3(n_heads), dim3(kCThreads), mla_attend_lds(max_seq, kv_lora, qk_rope), s, a,
                       delta_out, latent_out);
    return hipGetLastError();
}

hipError_t mla_project_v(int type, const uint8_t *w, size_t rb, const uint8_t *cache, size_t crb, float *kvb_cache,
                         int n_heads, int qk_nope, int v_head, int kv_lora, const int *d_pos, hipStream_t s) {
    if (n_heads == 0 || v_head == 0) return hipSuccess;
    switch (type) {
        case T_Q4_K: ProjectV<T_Q4_K>::run(w, rb, cache, crb, kvb_cache, n_heads, qk_nope, v_head, kv_lora, d_pos, s); break;
        case T_Q6_K: ProjectV<T_Q6_K>::run(w, rb, cache, crb, kvb_cache, n_heads, qk_nope, v_head, kv_lora, d_pos, s); break;
        case T_Q5_0: ProjectV<T_Q5_0>::run(w, rb, cache, crb, kvb_cache, n_heads, qk_nope, v_head, kv_lora, d_pos, s); break;
        case T_Q8_0: ProjectV<T_Q8_0>::run(w, rb, cache, crb, kvb_cache, n_heads, qk_nope, v_head, kv_lora, d_pos, s); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t mla_absorb_context_v(const float *scores, const float *kvb_cache, float *attn, int n_heads, int qk_nope,
                                int v_head, const int *d_pos, int max_seq, hipStream_t s) {
    if (n_heads == 0 || v_head == 0) return hipSuccess;
    hipLaunchKernelGGL(context_v_kernel, dim3(n_heads), dim3(kCThreads), 0, s, scores, kvb_cache, attn, n_heads,
                       qk_nope, v_head, d_pos, max_seq);
    return hipGetLastError();
}

}  // namespace qlin

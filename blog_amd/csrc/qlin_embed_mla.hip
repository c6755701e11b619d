// qlin_embed_mla.hip -- the remaining quantized-weight consumers of the DeepSeek layer, gfx950:
// the quantized embedding lookup and the three MLA latent-absorption products over kv_b.
//
//   embedding  out[t, k] = w(ids[t], k)                  (kernel.cu:2678-2693, quant_embedding_kernel)
//   q_nope     q_abs[h, l] = sum_{d < qk_nope} w(r_h + d, l) * q[h, d]        (kernel.cu:3018-3045)
//   xsum_delta delta[h, b] = sum_{d < qk_nope} q[h, d] * (-dmin * m)(r_h + d, b)  (Q4_K, 3052-3075)
//   v          attn[h, v] = sum_k w(r_h + qk_nope + v, k) * latent[h, k]
//                           (+ for Q4_K: sum_b (-dmin * m)(row, b) * xsum_delta[h, b])   (3417-3453)
// with r_h = h * (qk_nope + v_head) the first kv_b row of head h, q rows of qk_nope + qk_rope, and
// w(row, k) the canonical dequantized element.  These are small (DeepSeek-V2-Lite: 16 heads, kv_b
// [4096, 512]) and latency-bound, so each output is one thread (or one wave for the v product) with
// the sums in index order.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

namespace qlin {
namespace {

template <int T>
__global__ __launch_bounds__(256) void embedding_kernel(const int *__restrict__ ids, float *__restrict__ out,
                                                        const uint8_t *__restrict__ table, size_t rb, int hidden) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    const int t = blockIdx.x;
    const uint8_t *row = table + static_cast<size_t>(ids[t]) * rb;
    float *o = out + static_cast<size_t>(t) * hidden;
    for (int k = blockIdx.y * 256 + threadIdx.x; k < hidden; k += gridDim.y * 256)
        o[k] = block_value<T>(row + static_cast<size_t>(k / BE) * BB, k % BE);
}

template <int T>
__global__ __launch_bounds__(256) void absorb_q_nope_kernel(const float *__restrict__ q, const uint8_t *__restrict__ w,
                                                            size_t rb, float *__restrict__ q_abs, int n_heads,
                                                            int qk_nope, int qk_rope, int v_head, int kv_lora) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_heads * kv_lora) return;
    const int h = i / kv_lora, l = i - h * kv_lora;
    const float *qh = q + static_cast<size_t>(h) * (qk_nope + qk_rope);
    const uint8_t *col = w + static_cast<size_t>(h) * (qk_nope + v_head) * rb + static_cast<size_t>(l / BE) * BB;
    float acc = 0.0f;
    for (int d = 0; d < qk_nope; ++d) acc = fmaf(block_value<T>(col + static_cast<size_t>(d) * rb, l % BE), qh[d], acc);
    q_abs[i] = acc;
}

// -dmin * m of 32-block b of a Q4_K row (the min term of every element of that block)
__device__ __forceinline__ float q4k_min_coeff(const uint8_t *row, int b) {
    const uint8_t *sb = row + static_cast<size_t>(b >> 3) * 144;
    const uint32_t s0 = sb[4] | (sb[5] << 8) | (sb[6] << 16) | (static_cast<uint32_t>(sb[7]) << 24);
    const uint32_t s1 = sb[8] | (sb[9] << 8) | (sb[10] << 16) | (static_cast<uint32_t>(sb[11]) << 24);
    const uint32_t s2 = sb[12] | (sb[13] << 8) | (sb[14] << 16) | (static_cast<uint32_t>(sb[15]) << 24);
    int sc, m;
    q4k_scale_min(b & 7, s0, s1, s2, sc, m);
    return -mul_rn(f16_bits_to_f32(ld_u16(sb + 2)), static_cast<float>(m));
}

__global__ __launch_bounds__(256) void absorb_xsum_delta_kernel(const float *__restrict__ q,
                                                                const uint8_t *__restrict__ w, size_t rb,
                                                                float *__restrict__ delta, int n_heads, int qk_nope,
                                                                int qk_rope, int v_head, int nblk) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_heads * nblk) return;
    const int h = i / nblk, b = i - h * nblk;
    const float *qh = q + static_cast<size_t>(h) * (qk_nope + qk_rope);
    const uint8_t *rows = w + static_cast<size_t>(h) * (qk_nope + v_head) * rb;
    float acc = 0.0f;
    for (int d = 0; d < qk_nope; ++d) acc = fmaf(qh[d], q4k_min_coeff(rows + static_cast<size_t>(d) * rb, b), acc);
    delta[i] = acc;
}

template <int T>
__global__ __launch_bounds__(256) void absorb_v_kernel(const uint8_t *__restrict__ w, size_t rb,
                                                       const float *__restrict__ latent,
                                                       const float *__restrict__ delta, float *__restrict__ attn,
                                                       int n_heads, int qk_nope, int v_head, int kv_lora) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (i >= n_heads * v_head) return;  // whole waves
    const int h = i / v_head, v = i - h * v_head;
    const uint8_t *row = w + (static_cast<size_t>(h) * (qk_nope + v_head) + qk_nope + v) * rb;
    const float *x = latent + static_cast<size_t>(h) * kv_lora;
    float acc = 0.0f;
    for (int k = lane; k < kv_lora; k += 64)
        acc = fmaf(block_value<T>(row + static_cast<size_t>(k / BE) * BB, k % BE), x[k], acc);
    acc = wave_sum(acc);
    if (lane == 0) {
        if constexpr (T == T_Q4_K) {
            const int nblk = (kv_lora + 31) / 32;
            const float *dh = delta + static_cast<size_t>(h) * nblk;
            for (int b = 0; b < nblk; ++b) acc = fmaf(q4k_min_coeff(row, b), dh[b], acc);
        }
        attn[i] = acc;
    }
}

template <template <int> class K, typename... Args>
bool by_type(int type, Args... args) {
    switch (type) {
        case T_Q4_K: K<T_Q4_K>::run(args...); return true;
        case T_Q6_K: K<T_Q6_K>::run(args...); return true;
        case T_Q5_0: K<T_Q5_0>::run(args...); return true;
        case T_Q8_0: K<T_Q8_0>::run(args...); return true;
        default: return false;
    }
}

template <int T> struct Embed {
    static void run(const int *ids, float *out, const uint8_t *table, size_t rb, int hidden, int n, hipStream_t s) {
        const dim3 grid(n, (hidden + 255) / 256 < 8 ? (hidden + 255) / 256 : 8);
        hipLaunchKernelGGL(embedding_kernel<T>, grid, dim3(256), 0, s, ids, out, table, rb, hidden);
    }
};
template <int T> struct QNope {
    static void run(const float *q, const uint8_t *w, size_t rb, float *q_abs, int nh, int qn, int qr, int vh, int kl,
                    hipStream_t s) {
        hipLaunchKernelGGL(absorb_q_nope_kernel<T>, dim3((nh * kl + 255) / 256), dim3(256), 0, s, q, w, rb, q_abs,
                           nh, qn, qr, vh, kl);
    }
};
template <int T> struct AbsorbV {
    static void run(const uint8_t *w, size_t rb, const float *latent, const float *delta, float *attn, int nh, int qn,
                    int vh, int kl, hipStream_t s) {
        hipLaunchKernelGGL(absorb_v_kernel<T>, dim3((nh * vh + 3) / 4), dim3(256), 0, s, w, rb, latent, delta, attn,
                           nh, qn, vh, kl);
    }
};

}  // namespace

hipError_t quant_embedding(int type, const int *ids, float *out, const uint8_t *table, size_t rb, int hidden,
                           int n, hipStream_t s) {
    if (n == 0 || hidden == 0) return hipSuccess;
    if (!by_type<Embed>(type, ids, out, table, rb, hidden, n, s)) return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t mla_absorb_q_nope(int type, const float *q, const uint8_t *w, size_t rb, float *q_abs, int n_heads,
                             int qk_nope, int qk_rope, int v_head, int kv_lora, hipStream_t s) {
    if (n_heads == 0 || kv_lora == 0) return hipSuccess;
    if (!by_type<QNope>(type, q, w, rb, q_abs, n_heads, qk_nope, qk_rope, v_head, kv_lora, s))
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t mla_absorb_q4_xsum_delta(const float *q, const uint8_t *w, size_t rb, float *delta, int n_heads,
                                    int qk_nope, int qk_rope, int v_head, int kv_lora, hipStream_t s) {
    const int nblk = (kv_lora + 31) / 32;
    if (n_heads == 0 || nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(absorb_xsum_delta_kernel, dim3((n_heads * nblk + 255) / 256), dim3(256), 0, s, q, w, rb,
                       delta, n_heads, qk_nope, qk_rope, v_head, nblk);
    return hipGetLastError();
}

hipError_t mla_absorb_v(int type, const uint8_t *w, size_t rb, const float *latent, const float *delta, float *attn,
                        int n_heads, int qk_nope, int v_head, int kv_lora, hipStream_t s) {
    if (n_heads == 0 || v_head == 0) return hipSuccess;
    if (!by_type<AbsorbV>(type, w, rb, latent, delta, attn, n_heads, qk_nope, v_head, kv_lora, s))
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace qlin

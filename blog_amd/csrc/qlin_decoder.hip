// qlin_decoder.hip -- the glue of a Qwen2-architecture decoder layer around the quantized linears,
// gfx950: RMSNorm, rotary embedding with the KV-cache store, and causal grouped-query attention.
//
// These are not on the quantized-linear path; they exist so that a whole decoder (benchmark
// configuration C3: Qwen2.5-0.5B architecture, all linears Q8_0) can run its greedy decode on the
// path's kernels.
// Semantics, restated from the reference engine (AI/codes/local-llm/src/backend/cuda/ops/kernel.cu):
//   rms_norm      112-150   y = x * rsqrt(mean(x^2) + eps) * w, w from bf16 / f16 (1 + w if one_plus)
//   rope          186-226   pairs (i, i + d/2), inv_freq = 1 / theta^(2i / d), angle = pos * inv_freq
//                           (the reference's full-attention kernels, without their q/k norms)
//   attention     345-420   causal over positions 0..pos, scale 1 / sqrt(d), GQA head h -> h / (H / Hkv),
//                           softmax with the maximum subtracted (without the reference's output gate)
// The KV cache is f32 [max_seq_len, kv_heads * head_dim] per layer, as the reference lays it out.
// Positions come from a device int (start_pos_dev), so a captured decode step replays at the next
// position once that int is advanced; a row's position is clamped to [0, max_seq_len - 1], which
// keeps every cache and LDS access in bounds whatever that int holds.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "qlin.h"
#include "qlin_decoder.h"

namespace qlin {
namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float norm_weight(const uint16_t *w, int j, int type, int one_plus) {
    const uint32_t b = w[j];
    const float v = type == 0 ? __builtin_bit_cast(float, b << 16)
                              : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
    return one_plus ? v + 1.0f : v;
}

// Sum over the workgroup (blockDim.x a multiple of 64, at most 1024), the same in every thread.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < nw; ++w) t += red[w];
    return t;
}
__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int w = 0; w < nw; ++w) t = fmaxf(t, red[w]);
    return t;
}

// One workgroup per row.
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                                const uint16_t *__restrict__ w, int type, int hidden,
                                                                float eps, int one_plus) {
    __shared__ float red[kNormThreads / 64];
    const float *x = in + static_cast<size_t>(blockIdx.x) * hidden;
    float *y = out + static_cast<size_t>(blockIdx.x) * hidden;
    float ss = 0.0f;
    for (int j = threadIdx.x; j < hidden; j += kNormThreads) ss += x[j] * x[j];
    const float inv = rsqrtf(block_sum(ss, red) / static_cast<float>(hidden) + eps);
    for (int j = threadIdx.x; j < hidden; j += kNormThreads) y[j] = x[j] * inv * norm_weight(w, j, type, one_plus);
}

// One wave per (row, head): query heads rotated in place; key heads rotated into the cache at the
// row's position, with the row's value head beside them.
__global__ __launch_bounds__(64) void rope_store_kernel(float *__restrict__ q, const float *__restrict__ k,
                                                        const float *__restrict__ v, float *__restrict__ kc,
                                                        float *__restrict__ vc, int n_heads, int kv_heads, int hd,
                                                        int max_seq, const int *__restrict__ start_pos, float theta) {
    const int row = blockIdx.x, head = blockIdx.y;
    const int pos = min(max(*start_pos + row, 0), max_seq - 1);
    const int half = hd / 2;
    auto rotate = [&](const float *src, float *dst) {
        for (int i = threadIdx.x; i < half; i += 64) {
            const float inv_freq = 1.0f / powf(theta, static_cast<float>(2 * i) / static_cast<float>(hd));
            const float angle = static_cast<float>(pos) * inv_freq;
            const float c = cosf(angle), s = sinf(angle);
            const float x1 = src[i], x2 = src[i + half];
            dst[i] = x1 * c - x2 * s;
            dst[i + half] = x2 * c + x1 * s;
        }
    };
    if (head < n_heads) {
        float *qh = q + (static_cast<size_t>(row) * n_heads + head) * hd;
        rotate(qh, qh);
    } else {
        const int kh = head - n_heads;
        const size_t src = (static_cast<size_t>(row) * kv_heads + kh) * hd;
        const size_t dst = (static_cast<size_t>(pos) * kv_heads + kh) * hd;
        rotate(k + src, kc + dst);
        for (int d = threadIdx.x; d < hd; d += 64) vc[dst + d] = v[src + d];
    }
}

constexpr int kAttnThreads = 256;

// One workgroup per (row, query head).  Scores: one thread per position, its key row read as
// independent float4 loads (all in flight together); the scores of positions 0..pos sit in LDS for
// the softmax.  Output: thread (class c, float4 column d4) adds the weighted value rows of positions
// c, c + C, ... (C = 256 / (head_dim / 4) classes), 8 rows' loads in flight at a time; the classes'
// sums are added in class order.
// ROPE (one decode row): the rotary embedding and the cache store of rope_store_kernel done here as
// well -- q and the row's key rotated into LDS, the row's position scored and weighted from LDS (so
// no workgroup reads the cache row written in this launch), and the first query head of each key
// head's group writing the rotated key and the value into the caches for the later rows.  Every value
// is computed as the two kernels compute it, in the same order.
template <bool ROPE>
__global__ __launch_bounds__(kAttnThreads) void attend_kernel(const float *__restrict__ q, const float *__restrict__ kc,
                                                              const float *__restrict__ vc, float *__restrict__ out,
                                                              int n_heads, int kv_heads, int hd, int max_seq,
                                                              const int *__restrict__ start_pos,
                                                              const float *__restrict__ k_row,
                                                              const float *__restrict__ v_row, float *__restrict__ kc_w,
                                                              float *__restrict__ vc_w, float theta) {
    extern __shared__ float4 smem4[];
    __shared__ float red[kAttnThreads / 64];
    __shared__ float4 s_krow[ROPE ? 64 : 1], s_vrow[ROPE ? 64 : 1];  // the row's key and value (head_dim <= 256)
    const int n4 = hd / 4;
    float4 *qs = smem4;                                       // [n4]
    float *sc = reinterpret_cast<float *>(smem4 + n4);        // [max(max_seq, 4 * ... class sums)]
    const int row = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int pos = min(max(*start_pos + row, 0), max_seq - 1), n = pos + 1;
    const int kh = h / (n_heads / kv_heads);
    const size_t stride4 = static_cast<size_t>(kv_heads) * n4;
    const float4 *kb = reinterpret_cast<const float4 *>(kc) + static_cast<size_t>(kh) * n4;
    const float4 *vb = reinterpret_cast<const float4 *>(vc) + static_cast<size_t>(kh) * n4;
    const float4 *qh = reinterpret_cast<const float4 *>(q) + (static_cast<size_t>(row) * n_heads + h) * n4;
    if constexpr (ROPE) {
        // pairs (i, i + hd/2) rotated by pos / theta^(2i / hd), as rope_store_kernel
        const int half = hd / 2;
        float *qf = reinterpret_cast<float *>(qs), *kf = reinterpret_cast<float *>(s_krow);
        const float *qsrc = reinterpret_cast<const float *>(qh);
        const float *ksrc = k_row + static_cast<size_t>(kh) * hd, *vsrc = v_row + static_cast<size_t>(kh) * hd;
        if (tid < half) {
            const float inv_freq = 1.0f / powf(theta, static_cast<float>(2 * tid) / static_cast<float>(hd));
            const float angle = static_cast<float>(pos) * inv_freq;
            const float c = cosf(angle), sn = sinf(angle);
            const float q1 = qsrc[tid], q2 = qsrc[tid + half], k1 = ksrc[tid], k2 = ksrc[tid + half];
            qf[tid] = q1 * c - q2 * sn;
            qf[tid + half] = q2 * c + q1 * sn;
            kf[tid] = k1 * c - k2 * sn;
            kf[tid + half] = k2 * c + k1 * sn;
        }
        for (int d = tid; d < hd; d += kAttnThreads) reinterpret_cast<float *>(s_vrow)[d] = vsrc[d];
        __syncthreads();
        if (h % (n_heads / kv_heads) == 0) {
            const size_t dst = (static_cast<size_t>(pos) * kv_heads + kh) * hd;
            for (int d = tid; d < hd; d += kAttnThreads) {
                kc_w[dst + d] = reinterpret_cast<const float *>(s_krow)[d];
                vc_w[dst + d] = reinterpret_cast<const float *>(s_vrow)[d];
            }
        }
    } else {
        for (int d = tid; d < n4; d += kAttnThreads) qs[d] = qh[d];
        __syncthreads();
    }
    const float scale = rsqrtf(static_cast<float>(hd));
    float mx = -INFINITY;
    for (int j = tid; j < n; j += kAttnThreads) {
        const float4 *kj = kb + static_cast<size_t>(j) * stride4;
        float dot = 0.0f;
        if (ROPE && j == pos) {
            for (int c = 0; c < n4; ++c) {
                const float4 a = qs[c], kv = s_krow[c];
                dot += a.x * kv.x + a.y * kv.y + a.z * kv.z + a.w * kv.w;
            }
        } else {
            for (int c = 0; c < n4; c += 16) {
                float4 kv[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) kv[u] = c + u < n4 ? kj[c + u] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    if (c + u < n4) {
                        const float4 a = qs[c + u];
                        dot += a.x * kv[u].x + a.y * kv[u].y + a.z * kv[u].z + a.w * kv[u].w;
                    }
                }
            }
        }
        const float s = dot * scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max(mx, red);
    float sum = 0.0f;
    for (int j = tid; j < n; j += kAttnThreads) {
        const float p = expf(sc[j] - mx);
        sc[j] = p;
        sum += p;
    }
    sum = block_sum(sum, red);  // (its barriers also order the sc writes before the reads below)
    const int C = kAttnThreads / n4, cls = tid / n4, d4 = tid % n4;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (cls < C) {
        for (int j0 = cls; j0 < n; j0 += 8 * C) {
            float4 vv[8];
            float pp[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int j = j0 + u * C;
                vv[u] = j >= n                 ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                        : (ROPE && j == pos) ? s_vrow[d4]
                                             : vb[static_cast<size_t>(j) * stride4 + d4];
                pp[u] = j < n ? sc[j] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc.x += pp[u] * vv[u].x;
                acc.y += pp[u] * vv[u].y;
                acc.z += pp[u] * vv[u].z;
                acc.w += pp[u] * vv[u].w;
            }
        }
    }
    __syncthreads();  // (the probabilities are no longer read: their LDS takes the classes' sums)
    float4 *cs = reinterpret_cast<float4 *>(sc);
    if (cls < C) cs[cls * n4 + d4] = acc;
    __syncthreads();
    float4 *o4 = reinterpret_cast<float4 *>(out) + (static_cast<size_t>(row) * n_heads + h) * n4;
    for (int d = tid; d < n4; d += kAttnThreads) {
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int c = 0; c < C; ++c) {
            const float4 v = cs[c * n4 + d];
            o.x += v.x;
            o.y += v.y;
            o.z += v.z;
            o.w += v.w;
        }
        o4[d] = make_float4(o.x / sum, o.y / sum, o.z / sum, o.w / sum);
    }
}

hipStream_t current_stream() { return static_cast<hipStream_t>(qlin_get_stream()); }
int launched(hipError_t e) { return e == hipSuccess ? QLIN_OK : QLIN_ERR_LAUNCH; }
bool al4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace qlin

extern "C" {

int qlin_launch_rms_norm(const float *input, float *output, const uint16_t *weight, int weight_type, int rows,
                         int hidden_size, float eps, int one_plus) {
    if (rows < 0 || hidden_size < 0 || (weight_type != 0 && weight_type != 1)) return QLIN_ERR_SHAPE;
    if (rows == 0 || hidden_size == 0) return QLIN_OK;
    if (!input || !output || !weight) return QLIN_ERR_NULL;
    if (!qlin::al4(input) || !qlin::al4(output) || (reinterpret_cast<uintptr_t>(weight) & 1u)) return QLIN_ERR_ALIGN;
    hipLaunchKernelGGL(qlin::rms_norm_kernel, dim3(rows), dim3(qlin::kNormThreads), 0, qlin::current_stream(), input,
                       output, weight, weight_type, hidden_size, eps, one_plus);
    return qlin::launched(hipGetLastError());
}

static int check_heads(int rows, int n_heads, int kv_heads, int head_dim, int max_seq_len) {
    if (rows < 0 || n_heads <= 0 || kv_heads <= 0 || n_heads % kv_heads || head_dim <= 0 || head_dim % 4 ||
        max_seq_len <= 0)
        return QLIN_ERR_SHAPE;
    if (head_dim > 256 || max_seq_len > 32768) return QLIN_ERR_LIMIT;
    return QLIN_OK;
}

int qlin_launch_rope_store_kv(float *q, const float *k, const float *v, float *key_cache, float *value_cache, int rows,
                              int n_heads, int kv_heads, int head_dim, int max_seq_len, const int *start_pos_dev,
                              float rope_theta) {
    int rc = check_heads(rows, n_heads, kv_heads, head_dim, max_seq_len);
    if (rc || rows == 0) return rc;
    if (!q || !k || !v || !key_cache || !value_cache || !start_pos_dev) return QLIN_ERR_NULL;
    if (!qlin::al4(q) || !qlin::al4(k) || !qlin::al4(v) || !qlin::al4(key_cache) || !qlin::al4(value_cache) ||
        !qlin::al4(start_pos_dev))
        return QLIN_ERR_ALIGN;
    hipLaunchKernelGGL(qlin::rope_store_kernel, dim3(rows, n_heads + kv_heads), dim3(64), 0, qlin::current_stream(), q,
                       k, v, key_cache, value_cache, n_heads, kv_heads, head_dim, max_seq_len, start_pos_dev, rope_theta);
    return qlin::launched(hipGetLastError());
}

int qlin_launch_attend(const float *q, const float *key_cache, const float *value_cache, float *attn, int rows,
                       int n_heads, int kv_heads, int head_dim, int max_seq_len, const int *start_pos_dev) {
    int rc = check_heads(rows, n_heads, kv_heads, head_dim, max_seq_len);
    if (rc || rows == 0) return rc;
    if (!q || !key_cache || !value_cache || !attn || !start_pos_dev) return QLIN_ERR_NULL;
    if (!qlin::al16(q) || !qlin::al16(key_cache) || !qlin::al16(value_cache) || !qlin::al16(attn) ||
        !qlin::al4(start_pos_dev))
        return QLIN_ERR_ALIGN;
    // q, then the scores of every position up to max_seq_len, later the classes' output sums (at most
    // 256 threads' float4s), in LDS
    const size_t slots = static_cast<size_t>(qlin::kAttnThreads) * 4;
    const size_t lds = static_cast<size_t>(head_dim) * sizeof(float) +
                       (static_cast<size_t>(max_seq_len) > slots ? max_seq_len : slots) * sizeof(float);
    hipLaunchKernelGGL(qlin::attend_kernel<false>, dim3(rows, n_heads), dim3(qlin::kAttnThreads), lds,
                       qlin::current_stream(), q, key_cache, value_cache, attn, n_heads, kv_heads, head_dim,
                       max_seq_len, start_pos_dev, nullptr, nullptr, nullptr, nullptr, 0.0f);
    return qlin::launched(hipGetLastError());
}

int qlin_launch_rope_attend(const float *q, const float *k, const float *v, float *key_cache, float *value_cache,
                            float *attn, int n_heads, int kv_heads, int head_dim, int max_seq_len,
                            const int *start_pos_dev, float rope_theta) {
    int rc = check_heads(1, n_heads, kv_heads, head_dim, max_seq_len);
    if (rc) return rc;
    if (!q || !k || !v || !key_cache || !value_cache || !attn || !start_pos_dev) return QLIN_ERR_NULL;
    if (!qlin::al16(q) || !qlin::al4(k) || !qlin::al4(v) || !qlin::al16(key_cache) || !qlin::al16(value_cache) ||
        !qlin::al16(attn) || !qlin::al4(start_pos_dev))
        return QLIN_ERR_ALIGN;
    const size_t slots = static_cast<size_t>(qlin::kAttnThreads) * 4;
    const size_t lds = static_cast<size_t>(head_dim) * sizeof(float) +
                       (static_cast<size_t>(max_seq_len) > slots ? max_seq_len : slots) * sizeof(float);
    hipLaunchKernelGGL(qlin::attend_kernel<true>, dim3(1, n_heads), dim3(qlin::kAttnThreads), lds,
                       qlin::current_stream(), q, key_cache, value_cache, attn, n_heads, kv_heads, head_dim,
                       max_seq_len, start_pos_dev, k, v, key_cache, value_cache, rope_theta);
    return qlin::launched(hipGetLastError());
}

}  // extern "C"

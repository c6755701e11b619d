// qlin_moe.hip -- routed-expert decode pieces, gfx950.
//
// Semantics (AI/codes/local-llm/src/backend/cuda/ops/kernel.cu):
//   router_topk            3463-3511  softmax over n_experts (non-finite -> -inf), k picks by strict
//                                     '>' (lowest index wins ties), w = p * routed_scaling.
//   swiglu                 1289-1328  act[o] = g / (1 + exp(-g)) * u, g = Wg[o].x, u = Wu[o].x
//   swiglu_indexed         1340-1385  the same per route r on expert expert_ids[r]; id < 0 -> 0.
//   down_indexed_ordered   2253-2287  out[h] += sum_r fmaf(Wd[e_r][h].act[r], w_r, .) in route order
// swiglu_indexed and down_indexed_ordered run on the matrix-core decode kernel's routed forms
// (qlin_mfma_gemv.hip) when the layout meets its alignment; otherwise, and for the rest here, one
// wave64 per output row, the dot products decoding weights per element (any alignment).
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

#ifndef QLIN_Q4K_MFMA
#define QLIN_Q4K_MFMA 1
#endif

namespace qlin {
namespace {

constexpr int kBlock = 256;

template <int T>
__device__ __forceinline__ float row_dot(const uint8_t *row, const float *x, int in_dim, int lane) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    float acc = 0.0f;
    for (int k = lane; k < in_dim; k += 64) acc = fmaf(block_value<T>(row + (k / BE) * BB, k % BE), x[k], acc);
    return wave_sum(acc);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// One wave per token: lanes hold the logits of experts lane, lane + 64, ...  The maximum is
// order-free; the softmax denominator is summed by lane 0 in expert order, as the reference does;
// each of the k picks is a wave argmax that prefers the lower index on equal values, which is the
// first maximum of the reference's strict '>' scan.
__global__ __launch_bounds__(64) void router_kernel(const float *__restrict__ logits, int *__restrict__ idx,
                                                    float *__restrict__ wout, int tokens, int ne, int k,
                                                    float scaling) {
    const int t = blockIdx.x, lane = threadIdx.x;
    const float *lg = logits + static_cast<size_t>(t) * ne;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        const float l = e < ne ? lg[e] : -INFINITY;
        v[j] = isfinite(l) ? l : -INFINITY;
    }
    float maxv = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    maxv = wave_max(maxv);
    __shared__ __attribute__((aligned(16))) float ex[256];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (lane + 64 * j < ne) ex[lane + 64 * j] = isfinite(maxv) ? expf(v[j] - maxv) : 0.0f;
    __syncthreads();
    __shared__ float denom_s;
    if (lane == 0) {
        // summed in expert order, as the reference's one thread per token does; the reads go 4 at a
        // time, so that the adds wait on few LDS round trips
        float denom = 0.0f;
        if (isfinite(maxv)) {
            const int n4 = ne >> 2;
            for (int i = 0; i < n4; ++i) {
                const float4 q = reinterpret_cast<const float4 *>(ex)[i];
                denom += q.x;
                denom += q.y;
                denom += q.z;
                denom += q.w;
            }
            for (int e = 4 * n4; e < ne; ++e) denom += ex[e];
        }
        denom_s = denom;
    }
    __syncthreads();
    const float denom = denom_s;
    bool used[4] = {false, false, false, false};
    for (int r = 0; r < k; ++r) {
        float bv = -INFINITY;
        int be = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            if (e < ne && !used[j] && (v[j] > bv || (v[j] == bv && e < be))) {
                bv = v[j];
                be = e;
            }
        }
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) {
            const float ov = __shfl_xor(bv, m, 64);
            const int oe = __shfl_xor(be, m, 64);
            if (ov > bv || (ov == bv && oe < be)) {
                bv = ov;
                be = oe;
            }
        }
        // every remaining logit is -inf: the reference falls back to expert r (or 0)
        const int best_e = bv == -INFINITY ? (r < ne ? r : 0) : be;
#pragma unroll
        for (int j = 0; j < 4; ++j) used[j] = used[j] || (lane + 64 * j == best_e);
        if (lane == 0) {
            const float prob = (denom > 0.0f && isfinite(bv)) ? expf(bv - maxv) / denom : 0.0f;
            idx[static_cast<size_t>(t) * k + r] = best_e;
            wout[static_cast<size_t>(t) * k + r] = prob * scaling;
        }
    }
}

// At most 64 experts, one wave per token (route_token_rank): router_kernel's k successive wave
// argmaxes on the logits held one per lane, with router_kernel's weights and fallback for picks past
// the finite logits.
__global__ __launch_bounds__(64) void router_rank_kernel(const float *__restrict__ logits, int *__restrict__ idx,
                                                         float *__restrict__ wout, int ne, int k, float scaling) {
    __shared__ __attribute__((aligned(16))) float ex[64];
    const size_t t = blockIdx.x;
    route_token_rank(true, logits + t * ne, ne, k, scaling, ex, [&](int r, int e, float w) {
        idx[t * k + r] = e;
        wout[t * k + r] = w;
    });
}

template <int T>
__global__ __launch_bounds__(kBlock) void swiglu_kernel(const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu,
                                                        size_t g_eb, size_t u_eb, size_t g_rb, size_t u_rb,
                                                        const float *__restrict__ x, const int *__restrict__ ids,
                                                        float *__restrict__ act, int k, int ffn, int in_dim) {
    const int wave = static_cast<int>((blockIdx.x * kBlock + threadIdx.x) >> 6);
    const int lane = threadIdx.x & 63;
    if (wave >= k * ffn) return;
    const int route = wave / ffn, row = wave - route * ffn;
    const int e = ids ? ids[route] : 0;
    float *dst = act + static_cast<size_t>(route) * ffn + row;
    if (e < 0) {
        if (lane == 0) *dst = 0.0f;
        return;
    }
    const float g = row_dot<T>(wg + static_cast<size_t>(e) * g_eb + static_cast<size_t>(row) * g_rb, x, in_dim, lane);
    const float u = row_dot<T>(wu + static_cast<size_t>(e) * u_eb + static_cast<size_t>(row) * u_rb, x, in_dim, lane);
    if (lane == 0) *dst = silu_mul(g, u);
}

template <int T>
__global__ __launch_bounds__(kBlock) void down_kernel(const uint8_t *__restrict__ wd, size_t d_eb, size_t d_rb,
                                                      const float *__restrict__ act, const int *__restrict__ ids,
                                                      const float *__restrict__ rw, float *__restrict__ out,
                                                      int k, int hidden, int ffn) {
    const int h = static_cast<int>((blockIdx.x * kBlock + threadIdx.x) >> 6);
    const int lane = threadIdx.x & 63;
    if (h >= hidden) return;
    float total = 0.0f;
    for (int r = 0; r < k; ++r) {
        const int e = ids[r];
        if (e < 0) continue;
        const float a = row_dot<T>(wd + static_cast<size_t>(e) * d_eb + static_cast<size_t>(h) * d_rb,
                                   act + static_cast<size_t>(r) * ffn, ffn, lane);
        total = fmaf(a, rw[r], total);
    }
    if (lane == 0) out[h] += total;
}

// out[i] += w * expert_out[i], w from the host or read on the device (kernel.cu:3514-3526).
__global__ __launch_bounds__(256) void accumulate_kernel(const float *__restrict__ e, float w, const float *wp,
                                                         float *__restrict__ out, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = fmaf(wp ? *wp : w, e[i], out[i]);
}

// Index of the largest logit, the lowest index among equals; NaN never wins and index 0 is the
// answer when nothing beats -inf (kernel.cu:3531-3592).  One workgroup: strided scans, then the
// (value, index) pairs are reduced across lanes and waves with the same rule.
constexpr int kArgThreads = 1024;

__device__ __forceinline__ void better(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float *__restrict__ logits, int n,
                                                            int *__restrict__ out_idx) {
    __shared__ float s_v[kArgThreads / 64];
    __shared__ int s_i[kArgThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float v = -INFINITY;
    int idx = 0;
    // float4 loads, 8 in flight per thread (a strided loop of single loads waits on each in turn:
    // 51 us over a 151936-entry vocabulary), when logits is 16-byte aligned; the tail and any other
    // layout element by element.  Every element meets the same comparison, so the order is immaterial.
    int head = 0;
    if ((reinterpret_cast<uintptr_t>(logits) & 15u) == 0) {
        const int n4 = n / 4;
        const float4 *l4 = reinterpret_cast<const float4 *>(logits);
        constexpr int U = 8;
        for (int i0 = tid; i0 < n4; i0 += U * kArgThreads) {
            float4 q[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = i0 + u * kArgThreads;
                q[u] = i < n4 ? l4[i] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = 4 * (i0 + u * kArgThreads);
                better(v, idx, q[u].x, i);
                better(v, idx, q[u].y, i + 1);
                better(v, idx, q[u].z, i + 2);
                better(v, idx, q[u].w, i + 3);
            }
        }
        head = 4 * n4;
    }
    for (int i = head + tid; i < n; i += kArgThreads) better(v, idx, logits[i], i);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) better(v, idx, __shfl_xor(v, off, 64), __shfl_xor(idx, off, 64));
    if (lane == 0) {
        s_v[wave] = v;
        s_i[wave] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kArgThreads / 64; ++w) better(v, idx, s_v[w], s_i[w]);
        *out_idx = idx;
    }
}

}  // namespace

hipError_t moe_accumulate(const float *expert_out, float weight, const float *weight_dev, float *out, int n,
                          hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(accumulate_kernel, dim3((n + 255) / 256), dim3(256), 0, s, expert_out, weight, weight_dev, out, n);
    return hipGetLastError();
}

hipError_t argmax(const float *logits, int n, int *out_idx, hipStream_t s) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgThreads), 0, s, logits, n, out_idx);
    return hipGetLastError();
}

hipError_t router_topk(const float *logits, int *top_idx, float *top_w, int tokens, int n_experts, int k,
                       float routed_scaling, hipStream_t s) {
    if (tokens == 0) return hipSuccess;
    if (n_experts <= 64)
        hipLaunchKernelGGL(router_rank_kernel, dim3(tokens), dim3(64), 0, s, logits, top_idx, top_w, n_experts, k,
                           routed_scaling);
    else
        hipLaunchKernelGGL(router_kernel, dim3(tokens), dim3(64), 0, s, logits, top_idx, top_w, tokens,
                           n_experts, k, routed_scaling);
    return hipGetLastError();
}

#define QLIN_TYPE_SWITCH(type, CALL)            \
    switch (type) {                             \
        case T_Q4_0: { constexpr int TT = T_Q4_0; CALL; break; } \
        case T_Q5_0: { constexpr int TT = T_Q5_0; CALL; break; } \
        case T_Q8_0: { constexpr int TT = T_Q8_0; CALL; break; } \
        case T_Q4_K: { constexpr int TT = T_Q4_K; CALL; break; } \
        case T_Q6_K: { constexpr int TT = T_Q6_K; CALL; break; } \
        default: return hipErrorInvalidValue;   \
    }

hipError_t swiglu_indexed(int type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t u_eb,
                          size_t g_rb, size_t u_rb, const float *x, const int *ids, float *act, int k,
                          int ffn, int in_dim, hipStream_t s) {
    const int64_t waves = static_cast<int64_t>(k) * ffn;
    if (waves == 0) return hipSuccess;
    // the k routes' gate/up pairs as one matrix-core SwiGLU launch when the layout allows
    if (ids && g_eb == u_eb && g_rb == u_rb && mfma_routed_ok(type, true, wg, wu, g_eb, g_rb, x, k, ffn, in_dim))
        return mfma_swiglu_routed(type, wg, wu, g_eb, g_rb, x, ids, act, k, ffn, in_dim, s);
    const int blocks = static_cast<int>((waves + 3) / 4);
    QLIN_TYPE_SWITCH(type, hipLaunchKernelGGL((swiglu_kernel<TT>), dim3(blocks), dim3(kBlock), 0, s, wg, wu,
                                              g_eb, u_eb, g_rb, u_rb, x, ids, act, k, ffn, in_dim));
    return hipGetLastError();
}

hipError_t swiglu(int type, const uint8_t *wg, const uint8_t *wu, size_t g_rb, size_t u_rb, const float *x,
                  float *act, int ffn, int in_dim, hipStream_t s) {
    const uint8_t *gu[2] = {wg, wu};
    if ((QLIN_Q4K_MFMA || type != T_Q4_K) && g_rb == u_rb && mfma_ok(type, gu, 2, g_rb, x, ffn, in_dim, true))
        return mfma_swiglu(type, wg, wu, g_rb, x, act, ffn, in_dim, s);
    if (type == T_Q4_K && g_rb == u_rb && q4k_stream_ok(gu, 2, g_rb, x, ffn, in_dim, true))
        return q4k_stream_swiglu(wg, wu, g_rb, x, act, ffn, in_dim, s);
    return swiglu_indexed(type, wg, wu, 0, 0, g_rb, u_rb, x, nullptr, act, 1, ffn, in_dim, s);
}

hipError_t down_indexed_ordered(int type, const uint8_t *wd, size_t d_eb, size_t d_rb, const float *act,
                                const int *ids, const float *rw, float *out, int k, int hidden, int ffn,
                                hipStream_t s) {
    if (hidden == 0) return hipSuccess;
    // the k routes' down rows as one matrix-core GEMV over their activations end to end
    if (k > 0 && mfma_routed_ok(type, false, wd, wd, d_eb, d_rb, act, k, hidden, ffn))
        return mfma_down_routed(type, wd, d_eb, d_rb, act, ids, rw, out, k, hidden, ffn, s);
    const int blocks = (hidden + 3) / 4;
    QLIN_TYPE_SWITCH(type, hipLaunchKernelGGL((down_kernel<TT>), dim3(blocks), dim3(kBlock), 0, s, wd, d_eb, d_rb,
                                              act, ids, rw, out, k, hidden, ffn));
    return hipGetLastError();
}

}  // namespace qlin

// qlin_dense.hip -- quantized matmul over a few rows of f32 activations on the matrix cores, gfx950.
//
//   y[r, o] = sum_k w(o, k) * x[r, k]          (kernel.cu:1254-1279, quant_matmul_kernel; m > 1)
//   y[r, o] += ...                              (the gemm + add of SharedExperts.cpp:42-48)
//   act[r, o] = g / (1 + expf(-g)) * u,  g, u the rows of the gate and up matrices
//                                               (the gemm, gemm, silu_mul of SharedExperts.cpp:34-40)
//
// Q4_K (the shared experts) on v_mfma_f32_16x16x32_bf16 with the tokens as the MFMA rows
// (q4k_rows_dot, qlin_rows.hpp): the nibble q enters as the exact bf16 128 + q and x as the bf16 pair
// hi = bf16(x), lo = bf16(x - hi), so every product is exact and accumulates in f32; per sub-block
// and 16-token tile one MFMA pair gives sum x (128 + q) for 16 weight rows and another pair sum x,
// and two fmas per output apply the scales.  The other formats multiply the canonical f32 element values (decoded as the
// reference decodes them) on v_mfma_f32_16x16x4_f32: the contraction the reference runs one warp
// per (r, o), with the same f32 operands and only the summation order changed.
//
// Layout.  A workgroup owns a tile of 16 output rows and all of K; its 8 waves take the chunks of K in
// turn (wave w: w, w + 8, ...; Q4_K super-blocks, eight 32-element blocks otherwise).  Lane l supplies output row l % 16 and token l % 16 of the current
// 16-token tile, and k-slots of group g = l / 16 of each MFMA (Q4_K: elements 8g .. 8g+7 of a
// sub-block).  D holds tokens 4g .. 4g+3 of row l % 16.  The waves' partials meet in LDS and are
// summed in wave order.  A grid row per 64 tokens.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "qlin_mfma.hpp"
#include "qlin_rows.hpp"

namespace qlin {
namespace {

constexpr int kDWaves = 8, kDThreads = kDWaves * 64;
constexpr int kDTokens = 64;  // tokens per grid row (4 tiles of 16)

enum : int { kStore = 0, kAdd = 1, kSwiGLU = 2 };

struct DenseArgs {
    const uint8_t *w0, *w1;  // w1: the up matrix of kSwiGLU
    size_t rb;
    const float *x;
    float *y;
    int n, k, m;
    RouteCombine c;  // kAdd: a batched MoE decode's deferred combine (c.yr non-null), added before the product
};

// The deferred combine's routed total of (token t, row h): the routes in route order from 0, as the
// combine launch forms it (qlin_moe_grouped.hip).
__device__ __forceinline__ float routed_total(const RouteCombine &c, int t, int h, int hidden) {
    constexpr int kLoadsFirst = 16;
    float total = 0.0f;
    if (c.k <= kLoadsFirst) {  // uniform
        // every route's id, weight and result requested at once (one round trip), then the same sum
        // (a route without an expert has no result written; its value is read but not used)
        int e[kLoadsFirst];
        float y[kLoadsFirst], w[kLoadsFirst];
#pragma unroll
        for (int r = 0; r < kLoadsFirst; ++r) {
            if (r < c.k) {
                const int route = t * c.k + r;
                e[r] = c.ids[route];
                w[r] = c.rw[route];
                y[r] = c.yr[static_cast<size_t>(route) * hidden + h];
            }
        }
#pragma unroll
        for (int r = 0; r < kLoadsFirst; ++r)
            if (r < c.k && e[r] >= 0 && e[r] < c.n_experts) total = fmaf(y[r], w[r], total);
        return total;
    }
    for (int r = 0; r < c.k; ++r) {
        const int route = t * c.k + r, e = c.ids[route];
        if (e < 0 || e >= c.n_experts) continue;
        total = fmaf(c.yr[static_cast<size_t>(route) * hidden + h], c.rw[route], total);
    }
    return total;
}
// y = (y + routed total) + v: the combine launch's y += total, then the plain add
__device__ __forceinline__ void add_out(const DenseArgs &a, float *yo, int t, int h, float v) {
    float y = *yo;
    if (a.c.yr) y += routed_total(a.c, t, h, a.n);  // uniform
    *yo = y + v;
}

template <int MODE>
__global__ __launch_bounds__(kDThreads) void q4k_dense_kernel(const DenseArgs a) {
    constexpr int NW = MODE == kSwiGLU ? 2 : 1;
    __shared__ f32x4 part[kDWaves][NW][4][64];  // [wave][matrix][token tile][lane]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int K = a.k, nsb = K / 256;
    const int row0 = blockIdx.x * 16;
    const int row = min(row0 + n, a.n - 1);
    const int t0 = blockIdx.y * kDTokens;
    const int ntt = min(4, (a.m - t0 + 15) / 16);  // token tiles of this grid row
    const uint8_t *rp[2] = {a.w0 + static_cast<size_t>(row) * a.rb, a.w1 + static_cast<size_t>(row) * a.rb};
    const int rows = min(16, a.n - row0);

    // kAdd over at most two token tiles (thread i writes output i alone): what is added before the
    // product -- the output's current value and a batched MoE decode's routed results with their
    // ids and weights -- depends on nothing this launch computes, so it is requested here, ahead of
    // the weights, and the same adds in the same order run at the end (one round trip fewer after the
    // sums)
    constexpr int kPreRoutes = MODE == kAdd ? 8 : 1;
    const bool pre = MODE == kAdd && ntt <= 2 && a.c.k <= kPreRoutes;  // uniform
    const int ptl = tid >> 4, po = tid & 15, pt = t0 + ptl;
    const bool pown = pre && tid < ntt * 256 && po < rows && pt < a.m;
    float pre_y = 0.0f, pre_v[kPreRoutes], pre_w[kPreRoutes];
    int pre_e[kPreRoutes];
    if constexpr (MODE == kAdd) {
        if (pown) {
            pre_y = a.y[static_cast<size_t>(pt) * a.n + row0 + po];
            if (a.c.yr) {  // uniform
#pragma unroll
                for (int r = 0; r < kPreRoutes; ++r) {
                    if (r < a.c.k) {
                        const int route = pt * a.c.k + r;
                        pre_e[r] = a.c.ids[route];
                        pre_w[r] = a.c.rw[route];
                        pre_v[r] = a.c.yr[static_cast<size_t>(route) * a.n + row0 + po];
                    }
                }
            }
        }
    }

    // one 16-token tile at a time (a tile's weights come again from the cache for the next one)
    for (int tt = 0; tt < ntt; ++tt) {
        // token of this lane's A row (tokens past m read the last one; their D rows are dropped)
        const int tok = min(t0 + tt * 16 + n, a.m - 1);
        const float *xrow = a.x + static_cast<size_t>(tok) * K + 8 * g;
        f32x4 D[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) D[w] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // wave w takes super-blocks w, w + 8, ...
        q4k_rows_dot<NW>(rp, xrow, wave, kDWaves, nsb, g, D);
#pragma unroll
        for (int w = 0; w < NW; ++w) part[wave][w][tt][lane] = D[w];
    }
    __syncthreads();

    // outputs: row o = row0 + (i % 16), token t0 + i / 16; D element r of lane l is token 4(l/16) + r
    for (int i = tid; i < ntt * 256; i += kDThreads) {
        const int tl = i >> 4, o = i & 15;  // token within the grid row, row within the tile
        const int t = t0 + tl;
        if (o >= rows || t >= a.m) continue;
        const int tt = tl >> 4, l = ((tl & 15) >> 2) * 16 + o, r = tl & 3;
        float v0 = 0.0f, v1 = 0.0f;
        for (int wv = 0; wv < kDWaves; ++wv) {
            v0 += part[wv][0][tt][l][r];
            if constexpr (NW == 2) v1 += part[wv][NW - 1][tt][l][r];
        }
        float *yo = a.y + static_cast<size_t>(t) * a.n + row0 + o;
        if constexpr (MODE == kSwiGLU) {
            *yo = v0 / (1.0f + expf(-v0)) * v1;
        } else if constexpr (MODE == kAdd) {
            if (pre) {  // (then i == tid)
                float y = pre_y;
                if (a.c.yr) {
                    float total = 0.0f;  // routed_total's sum from the preloaded values
#pragma unroll
                    for (int r = 0; r < kPreRoutes; ++r)
                        if (r < a.c.k && pre_e[r] >= 0 && pre_e[r] < a.c.n_experts) total = fmaf(pre_v[r], pre_w[r], total);
                    y += total;
                }
                *yo = y + v0;
            } else {
                add_out(a, yo, t, row0 + o, v0);
            }
        } else {
            *yo = v0;
        }
    }
}

// 8 bytes at a 2-byte aligned address, as two dwords.
__device__ __forceinline__ void ld8_a2(const uint8_t *p, uint32_t &lo, uint32_t &hi) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    lo = h[0] | (static_cast<uint32_t>(h[1]) << 16);
    hi = h[2] | (static_cast<uint32_t>(h[3]) << 16);
}
__device__ __forceinline__ uint32_t byte_of(uint32_t lo, uint32_t hi, int i) {
    return ((i < 4 ? lo : hi) >> (8 * (i & 3))) & 0xffu;
}

// Elements k0 .. k0+7 of a row (k0 a multiple of 8: one block, one scale group), canonical values
// as the per-element decoders give them (kernel.cu:1122-1185, ggml's Q4_0): the raw words first
// (so that a wave can have several blocks' loads in flight), then the values.
template <int T>
__device__ __forceinline__ void raw8(const uint8_t *row, int k0, uint32_t (&w)[5]) {
    if constexpr (T == T_Q8_0) {
        const uint8_t *b = row + static_cast<size_t>(k0 >> 5) * 34;
        w[0] = ld_u16(b);
        ld8_a2(b + 2 + (k0 & 31), w[1], w[2]);
    } else if constexpr (T == T_Q4_0 || T == T_Q5_0) {
        constexpr int BB = T == T_Q4_0 ? 18 : 22, QS = T == T_Q4_0 ? 2 : 6;
        const uint8_t *b = row + static_cast<size_t>(k0 >> 5) * BB;
        w[0] = ld_u16(b);
        ld8_a2(b + QS + (k0 & 15), w[1], w[2]);
        if constexpr (T == T_Q5_0) w[3] = ld_u16(b + 2) | (ld_u16(b + 4) << 16);
    } else {  // Q6_K: half h, group g of 32, lanes l0 .. l0+7 (one 16-element scale)
        const uint8_t *b = row + static_cast<size_t>(k0 >> 8) * 210;
        const int e = k0 & 255, half = e >> 7, grp = (e & 127) >> 5, l0 = e & 31;
        ld8_a2(b + half * 64 + l0 + 32 * (grp & 1), w[0], w[1]);
        ld8_a2(b + 128 + half * 32 + l0, w[2], w[3]);
        w[4] = ld_u16(b + 208) | (static_cast<uint32_t>(b[192 + half * 8 + l0 / 16 + 2 * grp]) << 16);
    }
}

template <int T>
__device__ __forceinline__ void values8(const uint32_t (&w)[5], int k0, float (&v)[8]) {
    if constexpr (T == T_Q8_0) {
        const float d = f16_bits_to_f32(w[0]);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = mul_rn(d, static_cast<float>(static_cast<int8_t>(byte_of(w[1], w[2], i))));
    } else if constexpr (T == T_Q4_0 || T == T_Q5_0) {
        const int e0 = k0 & 31, sh = e0 >= 16 ? 4 : 0;
        const float d = f16_bits_to_f32(w[0]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int q = static_cast<int>((byte_of(w[1], w[2], i) >> sh) & 15u);
            if constexpr (T == T_Q5_0) q |= static_cast<int>(((w[3] >> (e0 + i)) & 1u) << 4);
            v[i] = mul_rn(d, static_cast<float>(q - (T == T_Q4_0 ? 8 : 16)));
        }
    } else {
        const int grp = ((k0 & 255) & 127) >> 5;
        const int sc = static_cast<int8_t>(w[4] >> 16);
        const float dsc = mul_rn(f16_bits_to_f32(w[4] & 0xffffu), static_cast<float>(sc));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lb = byte_of(w[0], w[1], i), hb = byte_of(w[2], w[3], i);
            const int q = static_cast<int>(((grp < 2 ? lb : lb >> 4) & 15u) | (((hb >> (2 * grp)) & 3u) << 4)) - 32;
            v[i] = mul_rn(dsc, static_cast<float>(q));
        }
    }
}

// The other formats (Q4_0, Q5_0, Q8_0, Q6_K): the waves take 32-element blocks in turn (wave w: w,
// w + 8, ...); a lane's 8 values of a block are decoded once and serve every token tile.
template <int T, int MODE>
__global__ __launch_bounds__(kDThreads) void dense_generic_kernel(const DenseArgs a) {
    constexpr int NW = MODE == kSwiGLU ? 2 : 1;
    __shared__ f32x4 part[kDWaves][NW][1][64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int K = a.k, nb32 = K / 32;
    const int row0 = blockIdx.x * 16;
    const int row = min(row0 + n, a.n - 1);
    const int t0 = blockIdx.y * 16;  // one 16-token tile per grid row
    constexpr int ntt = 1;
    const uint8_t *rp[2] = {a.w0 + static_cast<size_t>(row) * a.rb, a.w1 + static_cast<size_t>(row) * a.rb};
    const float *xrow = a.x + static_cast<size_t>(min(t0 + n, a.m - 1)) * K;  // past m: the last token

    f32x4 D[NW][1];
#pragma unroll
    for (int w = 0; w < NW; ++w) D[w][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // groups of U consecutive blocks, wave w: groups w, w + 8, ...; a group's weight words and
    // activations are all requested before its first block is used
    constexpr int U = 4;
    for (int b0 = wave * U; b0 < nb32; b0 += kDWaves * U) {
        uint32_t raw[NW][U][5];
        float4 xq[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k0 = 32 * min(b0 + u, nb32 - 1) + 8 * g;
#pragma unroll
            for (int w = 0; w < NW; ++w) raw8<T>(rp[w], k0, raw[w][u]);
            xq[u][0] = *reinterpret_cast<const float4 *>(xrow + k0);
            xq[u][1] = *reinterpret_cast<const float4 *>(xrow + k0 + 4);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the group's loads ahead of its first use
        // straight-line over the group (no branch lets the compiler sink a load to its use): a block
        // past the end repeats the last one with zero activations
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool in = b0 + u < nb32;
            const int k0 = 32 * min(b0 + u, nb32 - 1) + 8 * g;
            const float xv[8] = {in ? xq[u][0].x : 0.0f, in ? xq[u][0].y : 0.0f, in ? xq[u][0].z : 0.0f,
                                 in ? xq[u][0].w : 0.0f, in ? xq[u][1].x : 0.0f, in ? xq[u][1].y : 0.0f,
                                 in ? xq[u][1].z : 0.0f, in ? xq[u][1].w : 0.0f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                float v[8];
                values8<T>(raw[w][u], k0, v);
#pragma unroll
                for (int i = 0; i < 8; ++i) D[w][0] = mfma_f32(xv[i], v[i], D[w][0]);
            }
        }
    }

#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
            if (tt < ntt) part[wave][w][tt][lane] = D[w][tt];
    __syncthreads();
    const int rows = min(16, a.n - row0);
    for (int i = tid; i < ntt * 256; i += kDThreads) {
        const int tl = i >> 4, o = i & 15;
        const int t = t0 + tl;
        if (o >= rows || t >= a.m) continue;
        const int tt = tl >> 4, l = ((tl & 15) >> 2) * 16 + o, r = tl & 3;
        float v0 = 0.0f, v1 = 0.0f;
        for (int wv = 0; wv < kDWaves; ++wv) {
            v0 += part[wv][0][tt][l][r];
            if constexpr (NW == 2) v1 += part[wv][NW - 1][tt][l][r];
        }
        float *yo = a.y + static_cast<size_t>(t) * a.n + row0 + o;
        if constexpr (MODE == kSwiGLU) *yo = v0 / (1.0f + expf(-v0)) * v1;
        else if constexpr (MODE == kAdd) add_out(a, yo, t, row0 + o, v0);
        else *yo = v0;
    }
}

template <int T>
hipError_t launch_dense(const DenseArgs &a, int mode, hipStream_t s) {
    const dim3 grid((a.n + 15) / 16, (a.m + 15) / 16);
    switch (mode) {
        case kStore: hipLaunchKernelGGL((dense_generic_kernel<T, kStore>), grid, dim3(kDThreads), 0, s, a); break;
        case kAdd: hipLaunchKernelGGL((dense_generic_kernel<T, kAdd>), grid, dim3(kDThreads), 0, s, a); break;
        case kSwiGLU: hipLaunchKernelGGL((dense_generic_kernel<T, kSwiGLU>), grid, dim3(kDThreads), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool dense_ok(int type, const uint8_t *w0, const uint8_t *w1, size_t rb, const float *x, int k) {
    const auto al = [](const void *p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
    if (type == T_Q4_K) return k % 256 == 0 && rb % 16 == 0 && al(w0, 16) && (!w1 || al(w1, 16)) && al(x, 16);
    if (type != T_Q4_0 && type != T_Q5_0 && type != T_Q8_0 && type != T_Q6_K) return false;
    // the per-element decoder reads 16-bit fields: 2-byte aligned blocks
    return k % 32 == 0 && rb % 2 == 0 && al(w0, 2) && (!w1 || al(w1, 2)) && al(x, 16);
}

hipError_t dense_matmul(int type, const uint8_t *w0, const uint8_t *w1, size_t rb, const float *x, float *y, int n,
                        int k, int m, int mode, hipStream_t s, const RouteCombine *combine) {
    if (n == 0 || m == 0) return hipSuccess;
    DenseArgs a{w0, w1 ? w1 : w0, rb, x, y, n, k, m, RouteCombine{}};
    if (combine && mode == kAdd) a.c = *combine;
    const dim3 grid((n + 15) / 16, (m + kDTokens - 1) / kDTokens);
    switch (type) {
        case T_Q4_K: break;
        case T_Q4_0: return launch_dense<T_Q4_0>(a, mode, s);
        case T_Q5_0: return launch_dense<T_Q5_0>(a, mode, s);
        case T_Q8_0: return launch_dense<T_Q8_0>(a, mode, s);
        case T_Q6_K: return launch_dense<T_Q6_K>(a, mode, s);
        default: return hipErrorInvalidValue;
    }
    switch (mode) {
        case kStore: hipLaunchKernelGGL(q4k_dense_kernel<kStore>, grid, dim3(kDThreads), 0, s, a); break;
        case kAdd: hipLaunchKernelGGL(q4k_dense_kernel<kAdd>, grid, dim3(kDThreads), 0, s, a); break;
        case kSwiGLU: hipLaunchKernelGGL(q4k_dense_kernel<kSwiGLU>, grid, dim3(kDThreads), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qlin

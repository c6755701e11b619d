// qlin_moe_grouped.hip -- routed-expert decode for a batch of tokens, each selected expert read
// once for all the routes that chose it, gfx950.
//
// Per token t the result is the reference's routed sum (TensorTool::moe_routed_decode_indexed,
// AI/codes/local-llm/src/tensor/TensorTool.cpp:271-336, with kernel.cu:1340-1385 and 2253-2287):
//   act_r  = silu(Wg[e_r] x_t) * (Wu[e_r] x_t)               for routes r of t with 0 <= e_r < E
//   out[t] += sum_r fmaf(Wd[e_r] act_r, w_r, .)  in route order r = 0 .. k-1
// The reference decodes one token at a time, so an expert chosen by several tokens of a batch is
// read once per token; here the routes are first grouped by expert (a stable counting sort on the
// device), then
//   gate/up: one workgroup per (expert, 64 rows) reads those rows of Wg and Wu once and applies
//     them to up to kGroup routes' x vectors per pass (Q4_K on the matrix cores, the same operands
//     as the decode GEMV);
//   down: one wave per (expert, row) decodes the row once and dots it with up to kGroup
//     activations per pass;
//   combine: per (token, hidden row), the route results in route order.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "qlin_mfma.hpp"

namespace qlin {
namespace {

constexpr int kGroup = 4;  // routes of one expert per pass
constexpr int kMaxExperts = 1024;

struct Groups {
    int *offset;  // [E + 1] first position of expert e in list
    int *list;    // [R] route indices grouped by expert, increasing within an expert
};

// Stable counting sort of the R = tokens * k routes by expert id (invalid ids are left out).  One
// workgroup: thread e counts and then lists expert e's routes, which keeps them in route order.
__global__ __launch_bounds__(256) void group_kernel(const int *__restrict__ ids, int R, int E, Groups gr) {
    __shared__ int cnt[kMaxExperts + 1];
    for (int e = threadIdx.x; e < E; e += 256) {
        int c = 0;
        for (int r = 0; r < R; ++r) c += ids[r] == e;
        cnt[e] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {  // exclusive prefix sum in place
        int acc = 0;
        for (int e = 0; e < E; ++e) {
            const int c = cnt[e];
            cnt[e] = acc;
            acc += c;
        }
        cnt[E] = acc;
    }
    __syncthreads();
    for (int e = threadIdx.x; e <= E; e += 256) gr.offset[e] = cnt[e];
    for (int e = threadIdx.x; e < E; e += 256) {
        int pos = cnt[e];
        for (int r = 0; r < R; ++r)
            if (ids[r] == e) gr.list[pos++] = r;
    }
}

struct UpArgs {
    const uint8_t *wg, *wu;
    size_t eb, rb;       // expert and row bytes (gate and up alike)
    const float *x;      // [tokens, K]
    Groups gr;
    float *act;          // [R, ffn]
    int ffn, K, k;       // k = routes per token
};

// Q4_K gate/up of one expert for its routes: 4 waves x 16 rows, kGroup x vectors per pass.
__global__ __launch_bounds__(256) void up_kernel(const UpArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int e = blockIdx.x;
    const int beg = a.gr.offset[e], cnt = a.gr.offset[e + 1] - beg;
    if (cnt == 0) return;  // uniform per workgroup
    const int K = a.K, nsb = K / 256;
    uint16_t *xpart = reinterpret_cast<uint16_t *>(smem);                      // [kGroup][2][K]
    float *xsum = reinterpret_cast<float *>(smem + kGroup * 4 * static_cast<size_t>(K));  // [kGroup][K/32]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int row = min(blockIdx.y * 64 + wave * 16 + n, a.ffn - 1);
    const uint8_t *rg = a.wg + static_cast<size_t>(e) * a.eb + static_cast<size_t>(row) * a.rb;
    const uint8_t *ru = a.wu + static_cast<size_t>(e) * a.eb + static_cast<size_t>(row) * a.rb;
    const ScaleDecoder dec(g);
    const bool a_active = (n >> 2) == g;
    const bool a_high = (n >> 1) & 1;
    const int a_part = n & 1;

    for (int q0 = 0; q0 < cnt; q0 += kGroup) {
        const int nq = min(kGroup, cnt - q0);
        // stage the x vectors of this pass's routes: bf16 hi / lo and sums per 32 (as the GEMV)
        __syncthreads();
        for (int q = 0; q < kGroup; ++q) {
            const int route = a.gr.list[beg + min(q0 + q, cnt - 1)];
            const float4 *xs = reinterpret_cast<const float4 *>(a.x + static_cast<size_t>(route / a.k) * K);
            uint16_t *xp = xpart + static_cast<size_t>(q) * 2 * K;
            for (int i0 = 0; i0 < K / 4; i0 += 256) {  // K / 4 is a multiple of 64: whole waves
                const int i = i0 + tid;
                const float4 v = xs[min(i, K / 4 - 1)];
                const float xe[4] = {v.x, v.y, v.z, v.w};
                uint32_t hb[4], lb[4];
                float sm = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    hb[c] = bf16_rne(xe[c]);
                    lb[c] = bf16_rne(xe[c] - bf16_val(hb[c]));
                    sm += bf16_val(hb[c]) + bf16_val(lb[c]);
                }
                sm += __shfl_xor(sm, 1, 64);
                sm += __shfl_xor(sm, 2, 64);
                sm += __shfl_xor(sm, 4, 64);
                if (i < K / 4) {
                    reinterpret_cast<uint2 *>(xp)[i] = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
                    reinterpret_cast<uint2 *>(xp + K)[i] = make_uint2(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16));
                    if ((i & 7) == 0) xsum[q * (K / 32) + (i >> 3)] = sm;
                }
            }
        }
        __syncthreads();

        float accg[kGroup], accu[kGroup];
#pragma unroll
        for (int q = 0; q < kGroup; ++q) accg[q] = accu[q] = 0.0f;
        for (int sb = 0; sb < nsb; ++sb) {
            const uint8_t *pg = rg + static_cast<size_t>(sb) * 144, *pu = ru + static_cast<size_t>(sb) * 144;
            const u32x4 hg = ld16(pg), ag = ld16(pg + 16 + 32 * g), bg = ld16(pg + 32 + 32 * g);
            const u32x4 hu = ld16(pu), au = ld16(pu + 16 + 32 * g), bu = ld16(pu + 32 + 32 * g);
            const uint32_t qg[8] = {ag.x, ag.y, ag.z, ag.w, bg.x, bg.y, bg.z, bg.w};
            const uint32_t qu[8] = {au.x, au.y, au.z, au.w, bu.x, bu.y, bu.z, bu.w};
            u32x4 Bg[8], Bu[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                Bg[t] = weights_operand(qg[t]);
                Bu[t] = weights_operand(qu[t]);
            }
            // per-lane scales of sub-blocks 2g, 2g+1 of both matrices
            uint32_t scg, mg, scu, mu;
            dec(hg.y, hg.z, hg.w, scg, mg);
            dec(hu.y, hu.z, hu.w, scu, mu);
            const float dg = f16_bits_to_f32(hg.x & 0xffffu), dmg = f16_bits_to_f32(hg.x >> 16);
            const float du = f16_bits_to_f32(hu.x & 0xffffu), dmu = f16_bits_to_f32(hu.x >> 16);
#pragma unroll
            for (int q = 0; q < kGroup; ++q) {
                if (q >= nq) break;  // uniform
                const uint16_t *xp = xpart + static_cast<size_t>(q) * 2 * K;
                uint32_t dw[16];
                if (a_active) {
                    const uint4 *src = reinterpret_cast<const uint4 *>(xp + a_part * K + sb * 256 + (n >> 1) * 32);
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const uint4 v = src[c];
                        dw[4 * c] = v.x; dw[4 * c + 1] = v.y; dw[4 * c + 2] = v.z; dw[4 * c + 3] = v.w;
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 16; ++c) dw[c] = 0u;
                }
                f32x4 Dg = {0.0f, 0.0f, 0.0f, 0.0f}, Du = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    u32x4 ao;
                    ao.x = a_high ? 0u : dw[2 * t];
                    ao.y = a_high ? 0u : dw[2 * t + 1];
                    ao.z = a_high ? dw[2 * t] : 0u;
                    ao.w = a_high ? dw[2 * t + 1] : 0u;
                    Dg = mfma(ao, Bg[t], Dg);
                    Du = mfma(ao, Bu[t], Du);
                }
                const float2 xs = *reinterpret_cast<const float2 *>(xsum + q * (K / 32) + sb * 8 + 2 * g);
                auto epi = [&](const f32x4 &D, float dd, float dm, uint32_t sc, uint32_t mn, float acc) {
                    acc = fmaf(dd * static_cast<float>(sc & 0xffu), (D[0] + D[1]) - 128.0f * xs.x, acc);
                    acc = fmaf(dd * static_cast<float>((sc >> 8) & 0xffu), (D[2] + D[3]) - 128.0f * xs.y, acc);
                    acc = fmaf(-dm * static_cast<float>(mn & 0xffu), xs.x, acc);
                    return fmaf(-dm * static_cast<float>((mn >> 8) & 0xffu), xs.y, acc);
                };
                accg[q] = epi(Dg, dg, dmg, scg, mg, accg[q]);
                accu[q] = epi(Du, du, dmu, scu, mu, accu[q]);
            }
        }
        const int orow = blockIdx.y * 64 + wave * 16 + n;
#pragma unroll
        for (int q = 0; q < kGroup; ++q) {
            float gq = accg[q], uq = accu[q];
            gq += __shfl_xor(gq, 16, 64);
            gq += __shfl_xor(gq, 32, 64);
            uq += __shfl_xor(uq, 16, 64);
            uq += __shfl_xor(uq, 32, 64);
            if (q < nq && g == 0 && orow < a.ffn) {
                const int route = a.gr.list[beg + q0 + q];
                a.act[static_cast<size_t>(route) * a.ffn + orow] = gq / (1.0f + expf(-gq)) * uq;
            }
        }
    }
}

struct DownArgs {
    const uint8_t *w;
    size_t eb, rb;
    const float *act;    // [R, ffn]
    Groups gr;
    float *yr;           // [R, hidden] per-route results
    int hidden, ffn;
};

// Waves take hidden rows of one expert (64 per workgroup); each row is decoded once per pass and
// dotted with kGroup activations.
template <int T>
__global__ __launch_bounds__(256) void down_kernel(const DownArgs a) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    const int e = blockIdx.x;
    const int beg = a.gr.offset[e], cnt = a.gr.offset[e + 1] - beg;
    if (cnt == 0) return;
    const int lane = threadIdx.x & 63;
    const int h_end = min(a.hidden, (blockIdx.y + 1) * 64);
    for (int h = blockIdx.y * 64 + (threadIdx.x >> 6); h < h_end; h += 4)  // whole waves
    for (int q0 = 0; q0 < cnt; q0 += kGroup) {
        const uint8_t *row = a.w + static_cast<size_t>(e) * a.eb + static_cast<size_t>(h) * a.rb;
        const int nq = min(kGroup, cnt - q0);
        const float *xr[kGroup];
#pragma unroll
        for (int q = 0; q < kGroup; ++q)
            xr[q] = a.act + static_cast<size_t>(a.gr.list[beg + min(q0 + q, cnt - 1)]) * a.ffn;
        float acc[kGroup] = {};
        for (int i = lane; i < a.ffn; i += 64) {
            const float wv = block_value<T>(row + (i / BE) * BB, i % BE);
#pragma unroll
            for (int q = 0; q < kGroup; ++q) acc[q] = fmaf(wv, xr[q][i], acc[q]);
        }
#pragma unroll
        for (int q = 0; q < kGroup; ++q) {
            const float v = wave_sum(acc[q]);
            if (q < nq && lane == 0) a.yr[static_cast<size_t>(a.gr.list[beg + q0 + q]) * a.hidden + h] = v;
        }
    }
}

// 32-weight formats: each lane decodes a pair of blocks (Q4_0 36 B, Q5_0 44 B, Q8_0 68 B, all
// multiples of 4, so the pair is read as aligned dwords, exactly in bounds) into 64 weights and dots
// them with the pass's activations held in LDS.  32 lanes per row, two rows per wave, 64 rows per
// workgroup.  The activations are stored in 64-float segments padded to 68 floats, so that the
// lanes, which read one segment each at the same offset, fall in different LDS banks.
template <int T> struct Pair;
template <> struct Pair<T_Q4_0> { static constexpr int dw = 9; };
template <> struct Pair<T_Q5_0> { static constexpr int dw = 11; };
template <> struct Pair<T_Q8_0> { static constexpr int dw = 17; };

// weight e (0..31) of block j (0, 1) of a pair held in dwords w
template <int T>
__device__ __forceinline__ void pair_block(const uint32_t *w, int j, float &d, float q[32]) {
    if constexpr (T == T_Q8_0) {
        d = f16_bits_to_f32(j ? w[8] >> 16 : w[0] & 0xffffu);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t v = j ? w[9 + c] : __builtin_amdgcn_alignbyte(w[c + 1], w[c], 2);
#pragma unroll
            for (int b = 0; b < 4; ++b) q[4 * c + b] = static_cast<float>(static_cast<int8_t>((v >> (8 * b)) & 0xffu));
        }
    } else {
        uint32_t qs[4], qh = 0;
        if constexpr (T == T_Q5_0) {
            d = f16_bits_to_f32(j ? w[5] >> 16 : w[0] & 0xffffu);
            qh = j ? w[6] : __builtin_amdgcn_alignbyte(w[1], w[0], 2);
#pragma unroll
            for (int c = 0; c < 4; ++c) qs[c] = j ? w[7 + c] : __builtin_amdgcn_alignbyte(w[c + 2], w[c + 1], 2);
        } else {
            d = f16_bits_to_f32(j ? w[4] >> 16 : w[0] & 0xffffu);
#pragma unroll
            for (int c = 0; c < 4; ++c) qs[c] = j ? w[5 + c] : __builtin_amdgcn_alignbyte(w[c + 1], w[c], 2);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t byte = (qs[e >> 2] >> (8 * (e & 3))) & 0xffu;
            int lo = static_cast<int>(byte & 0xfu), hi = static_cast<int>(byte >> 4);
            if constexpr (T == T_Q5_0) {
                lo |= static_cast<int>((qh >> e) & 1u) << 4;
                hi |= static_cast<int>((qh >> (e + 16)) & 1u) << 4;
                q[e] = static_cast<float>(lo - 16);
                q[e + 16] = static_cast<float>(hi - 16);
            } else {
                q[e] = static_cast<float>(lo - 8);
                q[e + 16] = static_cast<float>(hi - 8);
            }
        }
    }
}

template <int T>
__global__ __launch_bounds__(256) void down_pair_kernel(const DownArgs a) {
    extern __shared__ __attribute__((aligned(16))) float xa[];  // [kGroup][ffn / 64][68]
    const int e = blockIdx.x;
    const int beg = a.gr.offset[e], cnt = a.gr.offset[e + 1] - beg;
    if (cnt == 0) return;  // uniform per workgroup
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l32 = lane & 31;
    const int npairs = a.ffn / 64, qstride = npairs * 68;
    for (int q0 = 0; q0 < cnt; q0 += kGroup) {
        const int nq = min(kGroup, cnt - q0);
        __syncthreads();
        for (int i = tid; i < kGroup * a.ffn; i += 256) {
            const int q = i / a.ffn, c = i - q * a.ffn;
            xa[q * qstride + (c >> 6) * 68 + (c & 63)] =
                a.act[static_cast<size_t>(a.gr.list[beg + min(q0 + q, cnt - 1)]) * a.ffn + c];
        }
        __syncthreads();
        for (int rr = 0; rr < 16; rr += 2) {
            const int h = blockIdx.y * 64 + wave * 16 + rr + (lane >> 5);
            const int hc = min(h, a.hidden - 1);
            const uint8_t *row = a.w + static_cast<size_t>(e) * a.eb + static_cast<size_t>(hc) * a.rb;
            float acc[kGroup] = {};
            for (int p = l32; p < npairs; p += 32) {
                uint32_t w[Pair<T>::dw];
                const uint8_t *pp = row + static_cast<size_t>(p) * 2 * Block<T>::bytes;
#pragma unroll
                for (int c = 0; c < Pair<T>::dw; ++c) w[c] = *reinterpret_cast<const uint32_t *>(pp + 4 * c);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    float d, q[32];
                    pair_block<T>(w, j, d, q);
                    const int base = 68 * p + 32 * j;
#pragma unroll
                    for (int c = 0; c < 32; c += 4) {
                        float wv[4];
#pragma unroll
                        for (int b = 0; b < 4; ++b) wv[b] = d * q[c + b];
#pragma unroll
                        for (int qq = 0; qq < kGroup; ++qq) {
                            const float4 xv = *reinterpret_cast<const float4 *>(xa + qq * qstride + base + c);
                            acc[qq] = fmaf(wv[0], xv.x, acc[qq]);
                            acc[qq] = fmaf(wv[1], xv.y, acc[qq]);
                            acc[qq] = fmaf(wv[2], xv.z, acc[qq]);
                            acc[qq] = fmaf(wv[3], xv.w, acc[qq]);
                        }
                    }
                }
            }
#pragma unroll
            for (int qq = 0; qq < kGroup; ++qq) {
                float v = acc[qq];
#pragma unroll
                for (int m = 1; m < 32; m <<= 1) v += __shfl_xor(v, m, 64);
                if (qq < nq && l32 == 0 && h < a.hidden)
                    a.yr[static_cast<size_t>(a.gr.list[beg + q0 + qq]) * a.hidden + h] = v;
            }
        }
    }
}

// out[t, h] += sum over t's routes in order of fmaf(yr, w, .), skipping invalid experts.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ yr, const int *__restrict__ ids,
                                                      const float *__restrict__ rw, float *__restrict__ out,
                                                      int tokens, int k, int hidden, int E) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<int64_t>(tokens) * hidden) return;
    const int t = static_cast<int>(i / hidden), h = static_cast<int>(i % hidden);
    float total = 0.0f;
    for (int r = 0; r < k; ++r) {
        const int route = t * k + r, e = ids[route];
        if (e < 0 || e >= E) continue;
        total = fmaf(yr[static_cast<size_t>(route) * hidden + h], rw[route], total);
    }
    out[i] += total;
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// the pair kernel reads whole block pairs as aligned dwords and keeps kGroup activations in LDS
bool down_pairs_ok(int type, const uint8_t *w, size_t eb, size_t rb, int ffn) {
    if (type != T_Q4_0 && type != T_Q5_0 && type != T_Q8_0) return false;
    return ffn % 64 == 0 && rb % 4 == 0 && eb % 4 == 0 && (reinterpret_cast<uintptr_t>(w) & 3u) == 0 &&
           static_cast<size_t>(kGroup) * (ffn / 64) * 68 * sizeof(float) <= 160 * 1024;
}

}  // namespace

size_t moe_grouped_workspace(int tokens, int k, int n_experts, int ffn, int hidden) {
    const size_t R = static_cast<size_t>(tokens) * k;
    return align256((n_experts + 1) * sizeof(int)) + align256(R * sizeof(int)) +
           align256(R * ffn * sizeof(float)) + align256(R * hidden * sizeof(float));
}

bool moe_grouped_shape_ok(int n_experts) { return n_experts <= kMaxExperts; }

bool moe_grouped_up_ok(int type, const uint8_t *wg, const uint8_t *wu, size_t eb, size_t rb, const float *x, int K) {
    const auto al = [](const void *p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
    return type == T_Q4_K && K % 256 == 0 && rb % 16 == 0 && eb % 16 == 0 && al(wg, 16) && al(wu, 16) && al(x, 16) &&
           static_cast<size_t>(kGroup) * (4 * K + K / 8) <= 160 * 1024;
}

hipError_t moe_grouped(int gu_type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t g_rb, int d_type,
                       const uint8_t *wd, size_t d_eb, size_t d_rb, int E, int ffn, int K, int hidden,
                       const float *x, const int *ids, const float *rw, void *ws, float *out, int tokens, int k,
                       hipStream_t s) {
    const int R = tokens * k;
    if (R == 0 || hidden == 0) return hipSuccess;
    uint8_t *p = static_cast<uint8_t *>(ws);
    Groups gr;
    gr.offset = reinterpret_cast<int *>(p);
    p += align256((E + 1) * sizeof(int));
    gr.list = reinterpret_cast<int *>(p);
    p += align256(static_cast<size_t>(R) * sizeof(int));
    float *act = reinterpret_cast<float *>(p);
    p += align256(static_cast<size_t>(R) * ffn * sizeof(float));
    float *yr = reinterpret_cast<float *>(p);

    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(256), 0, s, ids, R, E, gr);
    UpArgs ua{wg, wu, g_eb, g_rb, x, gr, act, ffn, K, k};
    const size_t lds = static_cast<size_t>(kGroup) * (4 * K + K / 8);
    hipLaunchKernelGGL(up_kernel, dim3(E, (ffn + 63) / 64), dim3(256), lds, s, ua);
    DownArgs da{wd, d_eb, d_rb, act, gr, yr, hidden, ffn};
    const dim3 dgrid(E, (hidden + 63) / 64);
    const bool pairs = down_pairs_ok(d_type, wd, d_eb, d_rb, ffn);
    const size_t plds = static_cast<size_t>(kGroup) * (ffn / 64) * 68 * sizeof(float);
    switch (d_type) {
        case T_Q4_0:
            if (pairs) hipLaunchKernelGGL(down_pair_kernel<T_Q4_0>, dgrid, dim3(256), plds, s, da);
            else hipLaunchKernelGGL(down_kernel<T_Q4_0>, dgrid, dim3(256), 0, s, da);
            break;
        case T_Q5_0:
            if (pairs) hipLaunchKernelGGL(down_pair_kernel<T_Q5_0>, dgrid, dim3(256), plds, s, da);
            else hipLaunchKernelGGL(down_kernel<T_Q5_0>, dgrid, dim3(256), 0, s, da);
            break;
        case T_Q8_0:
            if (pairs) hipLaunchKernelGGL(down_pair_kernel<T_Q8_0>, dgrid, dim3(256), plds, s, da);
            else hipLaunchKernelGGL(down_kernel<T_Q8_0>, dgrid, dim3(256), 0, s, da);
            break;
        case T_Q4_K: hipLaunchKernelGGL(down_kernel<T_Q4_K>, dgrid, dim3(256), 0, s, da); break;
        case T_Q6_K: hipLaunchKernelGGL(down_kernel<T_Q6_K>, dgrid, dim3(256), 0, s, da); break;
        default: return hipErrorInvalidValue;
    }
    const int64_t outs = static_cast<int64_t>(tokens) * hidden;
    hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>((outs + 255) / 256)), dim3(256), 0, s, yr, ids, rw,
                       out, tokens, k, hidden, E);
    return hipGetLastError();
}

}  // namespace qlin

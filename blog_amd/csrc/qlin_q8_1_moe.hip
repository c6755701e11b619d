// qlin_q8_1_moe.hip -- the Q8_1-activation variants of the prefill matmul and the MoE decode, gfx950.
//
//   quantize_mmq   Q8_1 blocks in the group-major MMQ layout: group g of 128 values of row r at
//                  (g * m + r) * 144 = 4 x (d f16, s f16), then 4 x 32 int8   (kernel.cu:1724-1765)
//   matmul_mmq     y[r, o] = W[o] . x_q8_1[r] from that layout              (kernel.cu:2405-2660)
//   swiglu_q8_1    act[route, o] = silu(Wg_e[o] . x) * (Wu_e[o] . x), x one Q8_1 row
//                                                                             (kernel.cu:1532-1666)
//   down_q8_1      out[h] += rw_r * (Wd_e[h] . act_q8_1[r]) over routes with e_r >= 0
//                                                                             (kernel.cu:1873-2097)
//   down_f32       the same from f32 act, each route's act quantized to Q8_1 (s = d * sum(q)) first
//                                                                             (kernel.cu:2112-2242)
//
// Every dot is the Q8_1 block-dot of quant_matmul_q8_1 (qlin_q8_1.hpp).  The reference adds each
// route's down product into out with atomicAdd in whatever order the warps finish; here one wave
// owns a row and adds the routes in route order, one of the orders the reference can produce, so
// repeated calls give identical bits.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "qlin_q8_1.hpp"

namespace qlin {
namespace {

__global__ __launch_bounds__(256) void quantize_mmq_kernel(const float *__restrict__ x, uint8_t *__restrict__ xq,
                                                           int in_dim, int m, int bpr, int raw) {
    const int gb = blockIdx.x * 256 + threadIdx.x;  // block b of row r, b < 4 * groups
    if (gb >= m * bpr) return;
    const int r = gb / bpr, b = gb - r * bpr, g = b >> 2, sub = b & 3;
    uint8_t *grp = xq + (static_cast<size_t>(g) * m + r) * 144;
    quantize_block_q8_1(x + static_cast<size_t>(r) * in_dim + b * 32, in_dim - b * 32,
                        reinterpret_cast<uint32_t *>(grp + 4 * sub), reinterpret_cast<uint32_t *>(grp + 16 + 32 * sub),
                        raw != 0);
}

// One wave per (activation row, output row); lanes over the 32-wide blocks.
template <int T>
__global__ __launch_bounds__(256) void matmul_mmq_kernel(const uint8_t *__restrict__ w, size_t rb,
                                                         const uint8_t *__restrict__ xq, float *__restrict__ y,
                                                         int out_dim, int in_dim, int m) {
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= static_cast<int64_t>(m) * out_dim) return;
    const int r = static_cast<int>(wave / out_dim), o = static_cast<int>(wave - static_cast<int64_t>(r) * out_dim);
    const uint8_t *row = w + static_cast<size_t>(o) * rb;
    float acc = 0.0f;
    for (int qb = lane; qb < in_dim / 32; qb += 64) {
        const uint8_t *grp = xq + (static_cast<size_t>(qb >> 2) * m + r) * 144;
        const int sub = qb & 3;
        acc += block_dot_q8_1<T>(row, qb, f16_bits_to_f32(ld_u16(grp + 4 * sub)),
                                 f16_bits_to_f32(ld_u16(grp + 4 * sub + 2)),
                                 reinterpret_cast<const int8_t *>(grp + 16 + 32 * sub));
    }
    acc = wave_sum(acc);
    if (lane == 0) y[static_cast<size_t>(r) * out_dim + o] = acc;
}

// One wave per (route, ffn row): both dots over the shared Q8_1 x, then SiLU(gate) * up.
template <int T>
__global__ __launch_bounds__(256) void swiglu_q8_1_kernel(const uint8_t *__restrict__ wg, const uint8_t *__restrict__ wu,
                                                          size_t g_eb, size_t u_eb, size_t g_rb, size_t u_rb,
                                                          const uint8_t *__restrict__ xq, const int *__restrict__ ids,
                                                          float *__restrict__ act, int k, int ffn, int in_dim) {
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= static_cast<int64_t>(k) * ffn) return;
    const int route = static_cast<int>(wave / ffn), o = static_cast<int>(wave - static_cast<int64_t>(route) * ffn);
    const int e = ids[route];
    float g = 0.0f, u = 0.0f;
    if (e >= 0) {  // uniform
        const uint8_t *gr = wg + static_cast<size_t>(e) * g_eb + static_cast<size_t>(o) * g_rb;
        const uint8_t *ur = wu + static_cast<size_t>(e) * u_eb + static_cast<size_t>(o) * u_rb;
        for (int qb = lane; qb < in_dim / 32; qb += 64) {
            g += block_dot_q8_1<T>(gr, qb, xq + static_cast<size_t>(qb) * 36);
            u += block_dot_q8_1<T>(ur, qb, xq + static_cast<size_t>(qb) * 36);
        }
        g = wave_sum(g);
        u = wave_sum(u);
    }
    if (lane == 0) act[static_cast<size_t>(route) * ffn + o] = e >= 0 ? g / (1.0f + expf(-g)) * u : 0.0f;
}

constexpr int kDnWaves = 16, kDnThreads = kDnWaves * 64;

// A workgroup per 16 hidden rows, a wave per row.  Routes in order; with QUANT the route's f32 act
// is quantized into LDS by the workgroup first (one thread per block), otherwise the Q8_1 act is
// read in place.
template <int T, bool QUANT>
__global__ __launch_bounds__(kDnThreads) void down_q8_1_kernel(const uint8_t *__restrict__ wd, size_t d_eb,
                                                               size_t d_rb, const void *__restrict__ act,
                                                               const int *__restrict__ ids,
                                                               const float *__restrict__ rw, float *__restrict__ out,
                                                               int k, int hidden, int ffn) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_act[];  // QUANT: one route's Q8_1 row
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x * kDnWaves + wave;
    const int bpr = ffn / 32;
    float total = h < hidden ? out[h] : 0.0f;
    for (int r = 0; r < k; ++r) {
        const int e = ids[r];
        if (e < 0) continue;  // uniform
        const uint8_t *xr;
        if constexpr (QUANT) {
            __syncthreads();  // the previous route's blocks are no longer read
            const float *a = static_cast<const float *>(act) + static_cast<size_t>(r) * ffn;
            for (int b = tid; b < bpr; b += kDnThreads) quantize_block_q8_1(a + b * 32, 32, s_act + b * 36, false);
            __syncthreads();
            xr = s_act;
        } else {
            xr = static_cast<const uint8_t *>(act) + static_cast<size_t>(r) * bpr * 36;
        }
        if (h < hidden) {
            const uint8_t *row = wd + static_cast<size_t>(e) * d_eb + static_cast<size_t>(h) * d_rb;
            float acc = 0.0f;
            for (int qb = lane; qb < bpr; qb += 64) acc += block_dot_q8_1<T>(row, qb, xr + static_cast<size_t>(qb) * 36);
            acc = wave_sum(acc);
            total = __fadd_rn(total, __fmul_rn(acc, rw[r]));
        }
    }
    if (h < hidden && lane == 0) out[h] = total;
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

template <int T> struct MatmulMmq {
    static void run(const uint8_t *w, size_t rb, const uint8_t *xq, float *y, int out_dim, int in_dim, int m,
                    hipStream_t s) {
        const int64_t waves = static_cast<int64_t>(m) * out_dim;
        hipLaunchKernelGGL(matmul_mmq_kernel<T>, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, s, w, rb,
                           xq, y, out_dim, in_dim, m);
    }
};
template <int T> struct SwigluQ8 {
    static void run(const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t u_eb, size_t g_rb, size_t u_rb,
                    const uint8_t *xq, const int *ids, float *act, int k, int ffn, int in_dim, hipStream_t s) {
        const int64_t waves = static_cast<int64_t>(k) * ffn;
        hipLaunchKernelGGL(swiglu_q8_1_kernel<T>, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, s, wg,
                           wu, g_eb, u_eb, g_rb, u_rb, xq, ids, act, k, ffn, in_dim);
    }
};
template <int T> struct DownQ8 {
    static void run(bool quant, const uint8_t *wd, size_t d_eb, size_t d_rb, const void *act, const int *ids,
                    const float *rw, float *out, int k, int hidden, int ffn, hipStream_t s) {
        const dim3 grid((hidden + kDnWaves - 1) / kDnWaves);
        if (quant)
            hipLaunchKernelGGL((down_q8_1_kernel<T, true>), grid, dim3(kDnThreads), static_cast<size_t>(ffn / 32) * 36, s,
                               wd, d_eb, d_rb, act, ids, rw, out, k, hidden, ffn);
        else
            hipLaunchKernelGGL((down_q8_1_kernel<T, false>), grid, dim3(kDnThreads), 0, s, wd, d_eb, d_rb, act, ids, rw,
                               out, k, hidden, ffn);
    }
};

}  // namespace

hipError_t quantize_q8_1_mmq(const float *x, uint8_t *xq, int in_dim, int m, bool raw_sum, hipStream_t s) {
    const int bpr = (in_dim + 127) / 128 * 4;
    const int64_t n = static_cast<int64_t>(m) * bpr;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_mmq_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, x, xq,
                       in_dim, m, bpr, raw_sum ? 1 : 0);
    return hipGetLastError();
}

hipError_t matmul_q8_1_mmq(int type, const uint8_t *w, size_t rb, const uint8_t *xq, float *y, int out_dim,
                           int in_dim, int m, hipStream_t s) {
    if (static_cast<int64_t>(m) * out_dim == 0) return hipSuccess;
    if (!by_type<MatmulMmq>(type, w, rb, xq, y, out_dim, in_dim, m, s)) return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t swiglu_indexed_q8_1(int type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t u_eb, size_t g_rb,
                               size_t u_rb, const uint8_t *xq, const int *ids, float *act, int k, int ffn, int in_dim,
                               hipStream_t s) {
    if (static_cast<int64_t>(k) * ffn == 0) return hipSuccess;
    if (!by_type<SwigluQ8>(type, wg, wu, g_eb, u_eb, g_rb, u_rb, xq, ids, act, k, ffn, in_dim, s))
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t down_q8_1_indexed_accum(int type, bool f32_act, const uint8_t *wd, size_t d_eb, size_t d_rb,
                                   const void *act, const int *ids, const float *rw, float *out, int k, int hidden,
                                   int ffn, hipStream_t s) {
    if (hidden == 0 || k == 0) return hipSuccess;
    if (!by_type<DownQ8>(type, f32_act, wd, d_eb, d_rb, act, ids, rw, out, k, hidden, ffn, s)) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace qlin

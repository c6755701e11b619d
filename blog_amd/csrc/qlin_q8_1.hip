// qlin_q8_1.hip -- Q8_1 activation quantizer and the quantized-weight x Q8_1 matmul (prefill), gfx950.
// The block quantizer and the per-type block dots (kernel.cu:1679-1720, 2305-2402) are in qlin_q8_1.hpp.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "qlin_q8_1.hpp"

namespace qlin {
namespace {

__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float *__restrict__ x, uint8_t *__restrict__ xq,
                                                            int in_dim, int m, int bpr, int raw) {
    const int gb = blockIdx.x * 256 + threadIdx.x;
    if (gb >= m * bpr) return;
    const int r = gb / bpr, b = gb - r * bpr;
    // 36-byte blocks: 4-aligned
    quantize_block_q8_1(x + static_cast<size_t>(r) * in_dim + b * 32, min(32, in_dim - b * 32),
                        xq + static_cast<size_t>(gb) * 36, raw != 0);
}

// One wave per (activation row, output row); lanes over 32-wide blocks.
template <int T>
__global__ __launch_bounds__(256) void matmul_q8_1_kernel(const uint8_t *__restrict__ w, size_t rb,
                                                          const uint8_t *__restrict__ xq, float *__restrict__ y,
                                                          int out_dim, int in_dim, int m) {
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= static_cast<int64_t>(m) * out_dim) return;
    const int r = static_cast<int>(wave / out_dim), o = static_cast<int>(wave - static_cast<int64_t>(r) * out_dim);
    const int bpr = in_dim / 32;
    const uint8_t *row = w + static_cast<size_t>(o) * rb;
    const uint8_t *xr = xq + static_cast<size_t>(r) * bpr * 36;
    float acc = 0.0f;
    for (int qb = lane; qb < bpr; qb += 64) acc += block_dot_q8_1<T>(row, qb, xr + static_cast<size_t>(qb) * 36);
    acc = wave_sum(acc);
    if (lane == 0) y[static_cast<size_t>(r) * out_dim + o] = acc;
}

}  // namespace

hipError_t quantize_q8_1(const float *x, uint8_t *xq, int in_dim, int m, bool raw_sum, hipStream_t s) {
    const int bpr = (in_dim + 31) / 32;
    const int64_t nblk = static_cast<int64_t>(m) * bpr;
    if (nblk == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_1_kernel, dim3(static_cast<unsigned>((nblk + 255) / 256)), dim3(256), 0, s, x,
                       xq, in_dim, m, bpr, raw_sum ? 1 : 0);
    return hipGetLastError();
}

hipError_t matmul_q8_1(int type, const uint8_t *w, size_t rb, const uint8_t *xq, float *y, int out_dim,
                       int in_dim, int m, hipStream_t s) {
    const int64_t waves = static_cast<int64_t>(m) * out_dim;
    if (waves == 0) return hipSuccess;
    if (type == T_Q4_K && q4k_gemm_ok(w, rb, xq, in_dim)) return q4k_gemm_q8_1(w, rb, xq, y, out_dim, in_dim, m, s);
    if (qblk_gemm_ok(type, w, rb, xq, in_dim)) return qblk_gemm_q8_1(type, w, rb, xq, y, out_dim, in_dim, m, s);
    const dim3 grid(static_cast<unsigned>((waves + 3) / 4));
    switch (type) {
        case T_Q4_0: hipLaunchKernelGGL((matmul_q8_1_kernel<T_Q4_0>), grid, dim3(256), 0, s, w, rb, xq, y, out_dim, in_dim, m); break;
        case T_Q5_0: hipLaunchKernelGGL((matmul_q8_1_kernel<T_Q5_0>), grid, dim3(256), 0, s, w, rb, xq, y, out_dim, in_dim, m); break;
        case T_Q8_0: hipLaunchKernelGGL((matmul_q8_1_kernel<T_Q8_0>), grid, dim3(256), 0, s, w, rb, xq, y, out_dim, in_dim, m); break;
        case T_Q4_K: hipLaunchKernelGGL((matmul_q8_1_kernel<T_Q4_K>), grid, dim3(256), 0, s, w, rb, xq, y, out_dim, in_dim, m); break;
        case T_Q6_K: hipLaunchKernelGGL((matmul_q8_1_kernel<T_Q6_K>), grid, dim3(256), 0, s, w, rb, xq, y, out_dim, in_dim, m); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qlin

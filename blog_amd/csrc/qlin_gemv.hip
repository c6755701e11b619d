// qlin_gemv.hip -- dequant-fused GEMV for decode (m small), gfx950.
//
// Semantics: y[r, o] = sum_k w(o, k) * x[r, k] with f32 activations and f32 accumulation, as the
// reference's quant_gemv_kernel / quant_gemv_add_kernel (AI/codes/local-llm/src/backend/cuda/ops/
// kernel.cu:1192-1244).  The summation order is ours (results agree within fp32 rounding).
//
// m == 1 goes to the matrix-core decode kernels (qlin_mfma_gemv.hip) or the streaming Q4_K kernel
// (qlin_q4k_stream.hip), Q4_K with m > 1 to the f32 matrix-core kernel (qlin_dense.hip); everything
// else takes the generic per-element kernel below, which decodes each weight with the reference's
// per-element formula.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

#ifndef QLIN_Q4K_MFMA
#define QLIN_Q4K_MFMA 1  // Q4_K decode on the matrix cores (0: the VALU streaming kernel)
#endif

namespace qlin {

namespace {

constexpr int kBlock = 256;   // 4 waves
constexpr int kWaves = kBlock / 64;

// ---- generic per-element path (any supported type, any 2-byte alignment) ---------------------

template <int T, int MT>
__global__ __launch_bounds__(kBlock) void gemv_generic_kernel(const uint8_t *__restrict__ w,
                                                              size_t row_bytes,
                                                              const float *__restrict__ x,
                                                              float *__restrict__ y, int out_dim,
                                                              int in_dim, int m, int add) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    const int row = static_cast<int>((blockIdx.x * kBlock + threadIdx.x) >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= out_dim) return;  // uniform per wave
    const uint8_t *rp = w + static_cast<size_t>(row) * row_bytes;
    for (int r0 = 0; r0 < m; r0 += MT) {
        float acc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
        for (int k = lane; k < in_dim; k += 64) {
            const float wv = block_value<T>(rp + (k / BE) * BB, k % BE);
#pragma unroll
            for (int t = 0; t < MT; ++t)
                if (r0 + t < m) acc[t] = fmaf(wv, x[static_cast<size_t>(r0 + t) * in_dim + k], acc[t]);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const float s = wave_sum(acc[t]);
            if (lane == 0 && r0 + t < m) {
                float *dst = y + static_cast<size_t>(r0 + t) * out_dim + row;
                *dst = add ? *dst + s : s;
            }
        }
    }
}

template <int T>
hipError_t launch_generic_t(const uint8_t *w, size_t rb, const float *x, float *y, int n, int k,
                            int m, bool add, hipStream_t s) {
    const int blocks = (n + kWaves - 1) / kWaves;
    hipLaunchKernelGGL((gemv_generic_kernel<T, 4>), dim3(blocks), dim3(kBlock), 0, s, w, rb, x, y, n,
                       k, m, add ? 1 : 0);
    return hipGetLastError();
}

}  // namespace

hipError_t gemv_generic(int type, const uint8_t *w, size_t rb, const float *x, float *y, int n,
                        int k, int m, bool add, hipStream_t s) {
    switch (type) {
        case T_Q4_0: return launch_generic_t<T_Q4_0>(w, rb, x, y, n, k, m, add, s);
        case T_Q5_0: return launch_generic_t<T_Q5_0>(w, rb, x, y, n, k, m, add, s);
        case T_Q8_0: return launch_generic_t<T_Q8_0>(w, rb, x, y, n, k, m, add, s);
        case T_Q4_K: return launch_generic_t<T_Q4_K>(w, rb, x, y, n, k, m, add, s);
        case T_Q6_K: return launch_generic_t<T_Q6_K>(w, rb, x, y, n, k, m, add, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t gemv(int type, const uint8_t *w, size_t rb, const float *x, float *y, int n, int k, int m,
                bool add, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    if (m == 1 && (QLIN_Q4K_MFMA || type != T_Q4_K) && mfma_ok(type, &w, 1, rb, x, n, k, false))
        return mfma_gemv(type, &w, &y, &n, 1, rb, x, k, add, s);
    if (type == T_Q4_K && m == 1 && q4k_stream_ok(&w, 1, rb, x, n, k, false))
        return q4k_stream_gemv(&w, &y, &n, 1, rb, x, k, add, s);
    if (m >= kF32GemmMinRows && f32_gemm_ok(type, w, rb, x, k)) return f32_gemm(type, w, rb, x, y, n, k, m, add, s);
    if (m > 1 && dense_ok(type, w, nullptr, rb, x, k)) return dense_matmul(type, w, nullptr, rb, x, y, n, k, m, add, s);
    return gemv_generic(type, w, rb, x, y, n, k, m, add, s);
}

hipError_t gemv_multi(int type, const uint8_t *const *w, float *const *y, const int *rows, int nmat, size_t rb,
                      const float *x, int k, hipStream_t s) {
    int total = 0;
    for (int i = 0; i < nmat; ++i) total += rows[i];
    if (total == 0) return hipSuccess;
    if ((QLIN_Q4K_MFMA || type != T_Q4_K) && mfma_ok(type, w, nmat, rb, x, total, k, false))
        return mfma_gemv(type, w, y, rows, nmat, rb, x, k, false, s);
    if (type == T_Q4_K && q4k_stream_ok(w, nmat, rb, x, total, k, false))
        return q4k_stream_gemv(w, y, rows, nmat, rb, x, k, false, s);
    for (int i = 0; i < nmat; ++i) {
        const hipError_t e = gemv(type, w[i], rb, x, y[i], rows[i], k, 1, false, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace qlin

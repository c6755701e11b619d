// qlin_q8_1.hip -- Q8_1 activation quantizer and the quantized-weight x Q8_1 matmul (prefill), gfx950.
//
// Q8_1 block (kernel.cu:1679-1720): 36 bytes per 32 activations = d f16 | s f16 | int8 q[32] with
// d = max|x| / 127, q = round-half-even(x * (1/d)) clamped to +-127, s = d * sum(q) (or the raw
// f32 sum of x in shuffle-down order when raw_sum).  Every step is an IEEE-exact f32 operation, so
// the bytes are bit-identical to any correct evaluation.
//
// Matmul block-dot semantics (kernel.cu:2305-2402), per 32-wide activation block:
//   Q4_K: acc = fma(dw*sc*dx, sum(qw*qx), acc) - dmin*m*s
//   Q6_K: acc = fma(dw*dx, sc0*sum16(qw*qx) + sc1*sum16'(qw*qx), acc)
//   Q8_0 / Q5_0 / Q4_0: acc = fma(w, dx*qx, acc) per element
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

namespace qlin {
namespace {

__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float *__restrict__ x, uint8_t *__restrict__ xq,
                                                            int in_dim, int m, int bpr, int raw) {
    const int gb = blockIdx.x * 256 + threadIdx.x;
    if (gb >= m * bpr) return;
    const int r = gb / bpr, b = gb - r * bpr;
    float v[32], t[32];
    float amax = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
        const int k = b * 32 + l;
        v[l] = k < in_dim ? x[static_cast<size_t>(r) * in_dim + k] : 0.0f;
        amax = fmaxf(amax, fabsf(v[l]));
        t[l] = v[l];
    }
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
#pragma unroll
        for (int i = 0; i < off; ++i) t[i] = t[i] + t[i + off];
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t packed[8];
    int qsum = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int q = static_cast<int>(rintf(__fmul_rn(v[4 * w + i], id)));
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            qsum += q;
            word |= (static_cast<uint32_t>(q) & 0xffu) << (8 * i);
        }
        packed[w] = word;
    }
    const float sum = raw ? t[0] : __fmul_rn(d, static_cast<float>(qsum));
    const uint32_t head = f32_to_f16_bits(d) | (f32_to_f16_bits(sum) << 16);
    uint32_t *dst = reinterpret_cast<uint32_t *>(xq + static_cast<size_t>(gb) * 36);  // 36-byte blocks: 4-aligned
    dst[0] = head;
#pragma unroll
    for (int w = 0; w < 8; ++w) dst[1 + w] = packed[w];
}

template <int T>
__device__ __forceinline__ float block_dot_q8_1(const uint8_t *row, int qb, const uint8_t *xb) {
    const float dx = f16_bits_to_f32(ld_u16(xb));
    const float sx = f16_bits_to_f32(ld_u16(xb + 2));
    const int8_t *qx = reinterpret_cast<const int8_t *>(xb + 4);
    if constexpr (T == T_Q4_K) {
        const uint8_t *sb = row + static_cast<size_t>(qb >> 3) * 144;
        const int j = qb & 7;
        const uint32_t s0 = sb[4] | (sb[5] << 8) | (sb[6] << 16) | (static_cast<uint32_t>(sb[7]) << 24);
        const uint32_t s1 = sb[8] | (sb[9] << 8) | (sb[10] << 16) | (static_cast<uint32_t>(sb[11]) << 24);
        const uint32_t s2 = sb[12] | (sb[13] << 8) | (sb[14] << 16) | (static_cast<uint32_t>(sb[15]) << 24);
        int sc, mn;
        q4k_scale_min(j, s0, s1, s2, sc, mn);
        int qdot = 0;
        for (int l = 0; l < 32; ++l) {
            const uint8_t byte = sb[16 + (j >> 1) * 32 + l];
            qdot += ((j & 1) ? (byte >> 4) : (byte & 15)) * qx[l];
        }
        const float dw = f16_bits_to_f32(ld_u16(sb));
        const float dmin = f16_bits_to_f32(ld_u16(sb + 2));
        return fmaf(dw * static_cast<float>(sc) * dx, static_cast<float>(qdot), 0.0f) -
               dmin * static_cast<float>(mn) * sx;
    } else if constexpr (T == T_Q6_K) {
        const uint8_t *sb = row + static_cast<size_t>(qb >> 3) * 210;
        const int sub = qb & 7, half = sub >> 2, g = sub & 3;
        int dot0 = 0, dot1 = 0;
        for (int l = 0; l < 32; ++l) {
            const uint8_t lo_byte = sb[half * 64 + l + 32 * (g & 1)];
            const int lo = (g < 2) ? (lo_byte & 15) : (lo_byte >> 4);
            const int hi = (sb[128 + half * 32 + l] >> (2 * g)) & 3;
            const int qw = (lo | (hi << 4)) - 32;
            if (l < 16) dot0 += qw * qx[l]; else dot1 += qw * qx[l];
        }
        const int8_t *sc = reinterpret_cast<const int8_t *>(sb + 192) + half * 8;
        const float dw = f16_bits_to_f32(ld_u16(sb + 208));
        return fmaf(dw * dx, static_cast<float>(sc[2 * g]) * static_cast<float>(dot0) +
                                 static_cast<float>(sc[2 * g + 1]) * static_cast<float>(dot1), 0.0f);
    } else {
        constexpr int BB = Block<T>::bytes;
        const uint8_t *b = row + static_cast<size_t>(qb) * BB;
        float acc = 0.0f;
        for (int l = 0; l < 32; ++l) acc = fmaf(block_value<T>(b, l), dx * static_cast<float>(qx[l]), acc);
        return acc;
    }
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

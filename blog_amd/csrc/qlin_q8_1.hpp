// qlin_q8_1.hpp -- the Q8_1 block routines shared by the quantizer, the Q8_1 matmul and the MLA
// latent-cache kernels (gfx950 device code).
//
// Q8_1 block (kernel.cu:1679-1720): 36 bytes per 32 activations = d f16 | s f16 | int8 q[32] with
// d = max|x| / 127, q = round-half-even(x * (1/d)) clamped to +-127, s = d * sum(q) (or the raw
// f32 sum of x in shuffle-down order when raw_sum).  Every step is an IEEE-exact f32 operation, so
// the bytes are bit-identical to any correct evaluation.
//
// Block-dot semantics against a quantized weight row (kernel.cu:2305-2402), per 32-wide block:
//   Q4_K: acc = fma(dw*sc*dx, sum(qw*qx), acc) - dmin*m*s
//   Q6_K: acc = fma(dw*dx, sc0*sum16(qw*qx) + sc1*sum16'(qw*qx), acc)
//   Q8_0 / Q5_0 / Q4_0: acc = fma(w, dx*qx, acc) per element
#pragma once

#include "qlin_device.hpp"

namespace qlin {

// One Q8_1 block from src[0 .. valid) (values past valid are 0): (d, s) as two f16 into the dword at
// ds, the 32 int8 q into the 8 dwords at q8 (the contiguous 36-byte block has q8 = ds + 1; the
// group-major MMQ layout keeps them apart).
__device__ __forceinline__ void quantize_block_q8_1(const float *src, int valid, uint32_t *ds, uint32_t *q8,
                                                    bool raw) {
    float v[32], t[32];
    float amax = 0.0f;
#pragma unroll
    for (int l = 0; l < 32; ++l) {
        v[l] = l < valid ? src[l] : 0.0f;
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
    *ds = f32_to_f16_bits(d) | (f32_to_f16_bits(sum) << 16);
#pragma unroll
    for (int w = 0; w < 8; ++w) q8[w] = packed[w];
}

// The same into a contiguous 36-byte block at dst (4-aligned).
__device__ __forceinline__ void quantize_block_q8_1(const float *src, int valid, uint8_t *dst, bool raw) {
    uint32_t *out = reinterpret_cast<uint32_t *>(dst);
    quantize_block_q8_1(src, valid, out, out + 1, raw);
}

// Block qb of a weight row against activation block (dx, sx, qx[32]).
template <int T>
__device__ __forceinline__ float block_dot_q8_1(const uint8_t *row, int qb, float dx, float sx, const int8_t *qx) {
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

// ... against the contiguous 36-byte block at xb.
template <int T>
__device__ __forceinline__ float block_dot_q8_1(const uint8_t *row, int qb, const uint8_t *xb) {
    return block_dot_q8_1<T>(row, qb, f16_bits_to_f32(ld_u16(xb)), f16_bits_to_f32(ld_u16(xb + 2)),
                             reinterpret_cast<const int8_t *>(xb + 4));
}

}  // namespace qlin

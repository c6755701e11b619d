// qlin_mfma.hpp -- operand builders shared by the matrix-core decode kernels (gfx950).
//
// A weight nibble q (or any 7-bit value) becomes the bf16 value 128 + q exactly: bytes (q, 0x43)
// assembled by v_perm_b32.  Activations x are split as hi = bf16(x), lo = bf16(x - hi), so products
// with weights are exact and hi + lo equals x to 2^-18 |x|; v_mfma_f32_16x16x32_bf16 accumulates in
// f32.  Lane l of an MFMA supplies row / column l % 16 and k-slots 8*(l/16) .. 8*(l/16)+7.
#pragma once

#include "qlin_device.hpp"

namespace qlin {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// bf16 bits of f (round to nearest even; finite inputs).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_val(uint32_t b) { return __builtin_bit_cast(float, b << 16); }
// value of the bf16 in the upper half of p
__device__ __forceinline__ float bf16_hi_val(uint32_t p) { return __builtin_bit_cast(float, p & 0xffff0000u); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// hi = bf16(x), lo = bf16(x - hi) of two values, each as a packed pair (first value in the low half),
// by v_cvt_pk_bf16_f32 (round to nearest even, as bf16_rne for finite values).
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t &hi, uint32_t &lo) {
    const f32x2 v = {a, b};
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    const f32x2 r = {a - bf16_val(hi & 0xffffu), b - bf16_hi_val(hi)};
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));
}

// Lane-constant (scale, min) decode of sub-blocks 2p and 2p+1 (kernel.cu:913-921), packed in bytes
// 0 and 1 of the results.
struct ScaleDecoder {
    bool upper;
    int sh, m_shift;
    uint32_t lo_mask, hi_mask;
    __device__ explicit ScaleDecoder(int p)
        : upper(p >= 2), sh(p >= 2 ? 16 * (p - 2) : 16 * p), m_shift(p >= 2 ? 4 : 0),
          lo_mask(p >= 2 ? 0x0f0fu : 0x3f3fu), hi_mask(p >= 2 ? 0x0303u : 0u) {}
    __device__ __forceinline__ void operator()(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &scp,
                                               uint32_t &mp) const {
        const uint32_t a_sc = upper ? s2 : s0;
        const uint32_t a_m = upper ? s2 : s1;
        scp = ((a_sc >> sh) & lo_mask) | (((s0 >> (sh + 6)) & hi_mask) << 4);
        mp = ((a_m >> (sh + m_shift)) & lo_mask) | (((s1 >> (sh + 6)) & hi_mask) << 4);
    }
};

__device__ __forceinline__ u32x4 ld16(const uint8_t *p) { return *reinterpret_cast<const u32x4 *>(p); }

// Loads from dword-aligned addresses of 16, 12 and 8 bytes, one instruction each (the HSA runtime runs
// gfx950 with unaligned access enabled).  A 16-byte load on a dword boundary runs at the rate of an
// aligned one; off a dword boundary the same load is much slower, so pieces that are only 2-byte
// aligned are read from the dword before them and realigned in registers.
__device__ __forceinline__ u32x4 ld16_a4(const uint8_t *p) {
    u32x4 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 4), 16);
    return v;
}
typedef uint32_t u32x3_a4 __attribute__((ext_vector_type(3), aligned(4)));
__device__ __forceinline__ void ld12_a4(const uint8_t *p, uint32_t (&v)[3]) {
    const u32x3_a4 t = *reinterpret_cast<const u32x3_a4 *>(__builtin_assume_aligned(p, 4));
    v[0] = t.x;
    v[1] = t.y;
    v[2] = t.z;
}
__device__ __forceinline__ uint2 ld8_a4(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, __builtin_assume_aligned(p, 4), 8);
    return v;
}
// N consecutive dwords from a dword-aligned address: 16-byte loads, then one of 12, 8 or 4 bytes
template <int N>
__device__ __forceinline__ void ld_dwords_a4(const uint8_t *p, uint32_t *w) {
#pragma unroll
    for (int i = 0; i + 4 <= N; i += 4) {
        const u32x4 v = ld16_a4(p + 4 * i);
        w[i] = v.x;
        w[i + 1] = v.y;
        w[i + 2] = v.z;
        w[i + 3] = v.w;
    }
    constexpr int B = N - N % 4;
    if constexpr (N % 4 == 3) {
        uint32_t t[3];
        ld12_a4(p + 4 * B, t);
        w[B] = t[0];
        w[B + 1] = t[1];
        w[B + 2] = t[2];
    } else if constexpr (N % 4 == 2) {
        const uint2 t = ld8_a4(p + 4 * B);
        w[B] = t.x;
        w[B + 1] = t.y;
    } else if constexpr (N % 4 == 1) {
        w[B] = *reinterpret_cast<const uint32_t *>(__builtin_assume_aligned(p + 4 * B, 4));
    }
}

// bits 0..3 of b to bit 0 of bytes 0..3 (the four shifted copies of b do not overlap): the fifth
// bits of four Q5_0 elements, ready to join their nibbles
__device__ __forceinline__ uint32_t spread4(uint32_t b) { return __umul24(b & 0xfu, 0x204081u) & 0x01010101u; }

// B operand of MFMA t from qs dword v: bf16(128 + q) for the 4 low nibbles, then the 4 high ones.
// bf16 128 + q has bytes (q, 0x43); v_perm_b32 interleaves the nibble bytes with 0x43 bytes taken
// from a constant register.
__device__ __forceinline__ u32x4 weights_operand(uint32_t v) {
    const uint32_t lo = v & 0x0f0f0f0fu;
    const uint32_t hi = (v >> 4) & 0x0f0f0f0fu;
    const uint32_t k43 = 0x43434343u;
    u32x4 r;
    r.x = __builtin_amdgcn_perm(k43, lo, 0x04010400u);  // (q0, 43, q1, 43)
    r.y = __builtin_amdgcn_perm(k43, lo, 0x04030402u);  // (q2, 43, q3, 43)
    r.z = __builtin_amdgcn_perm(k43, hi, 0x04010400u);
    r.w = __builtin_amdgcn_perm(k43, hi, 0x04030402u);
    return r;
}
// The same from ready 7-bit values: 4 bytes for slots 0..3 and 4 for slots 4..7.
__device__ __forceinline__ u32x4 weights_operand2(uint32_t lo, uint32_t hi) {
    const uint32_t k43 = 0x43434343u;
    u32x4 r;
    r.x = __builtin_amdgcn_perm(k43, lo, 0x04010400u);  // (q0, 43, q1, 43)
    r.y = __builtin_amdgcn_perm(k43, lo, 0x04030402u);  // (q2, 43, q3, 43)
    r.z = __builtin_amdgcn_perm(k43, hi, 0x04010400u);
    r.w = __builtin_amdgcn_perm(k43, hi, 0x04030402u);
    return r;
}

// v summed over lanes n, n+16, n+32, n+48 (the four lane-groups of an MFMA), in lanes 0..15: the
// gfx950 half-wave and row swaps, (v_n + v_n+32) + (v_n+16 + v_n+48).
__device__ __forceinline__ float sum_lane_groups(float v) {
    const auto s32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                      false, false);
    const float a = v + __builtin_bit_cast(float, static_cast<uint32_t>(s32[1]));
    const auto s16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, a),
                                                      false, false);
    return a + __builtin_bit_cast(float, static_cast<uint32_t>(s16[1]));
}

__device__ __forceinline__ f32x4 mfma(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// x as int8 digits, for the int8 matrix cores.  Called by the 8 consecutive lanes that hold the 4
// elements each of one 32-element block: with e such that max|x| < 2^(e+6), t = x / 2^e is below 64
// in magnitude and x = 2^e (d1 + d2 / 128 + d3 / 16384) to within 2^(e-15), the digits
//   d1 = rint(t), d2 = rint(128 (t - d1)), d3 = rint(128 (128 (t - d1) - d2))
// each in [-64, 64] (rint is the low byte of t + 1.5 * 2^23: round to nearest even, exact for
// |t| < 2^22; every residual above is exact).  Gives the lane's 4 digits of each kind packed in a
// dword, and the block's scale 2^e (NaN if any of its x is not finite), sum of x and the sum of
// the lane's 16-element half.
__device__ __forceinline__ void x_digits4(const float4 &v, uint32_t &p1, uint32_t &p2, uint32_t &p3, float &scale,
                                          float &sum, float &sum16) {
    constexpr float kMagic = 12582912.0f;
    const float xe[4] = {v.x, v.y, v.z, v.w};
    float mx = fmaxf(fmaxf(fabsf(xe[0]), fabsf(xe[1])), fmaxf(fabsf(xe[2]), fabsf(xe[3])));
    float sm = ((xe[0] + xe[1]) + xe[2]) + xe[3];
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
    sm += __shfl_xor(sm, 1, 64);
    sm += __shfl_xor(sm, 2, 64);
    sum16 = sm;  // the sum of the lane's 16-element half of the block
    sm += __shfl_xor(sm, 4, 64);
    int ex;
    (void)frexpf(mx, &ex);
    const int e = ex - 6;
    uint32_t b[3][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float t = ldexpf(xe[k], -e);
        const float f1 = t + kMagic, r1 = t - (f1 - kMagic);
        const float u = r1 * 128.0f;
        const float f2 = u + kMagic, r2 = u - (f2 - kMagic);
        const float f3 = r2 * 128.0f + kMagic;
        b[0][k] = __builtin_bit_cast(uint32_t, f1);
        b[1][k] = __builtin_bit_cast(uint32_t, f2);
        b[2][k] = __builtin_bit_cast(uint32_t, f3);
    }
    uint32_t pk[3];
#pragma unroll
    for (int d = 0; d < 3; ++d)
        pk[d] = __builtin_amdgcn_perm(b[d][1], b[d][0], 0x0c0c0400u) | __builtin_amdgcn_perm(b[d][3], b[d][2], 0x04000c0cu);
    p1 = pk[0];
    p2 = pk[1];
    p3 = pk[2];
    scale = isfinite(sm) && isfinite(mx) ? ldexpf(1.0f, e) : __builtin_nanf("");
    sum = sm;
}
// the value of a unit's three digit dots (exact integers) in units of its scale
__device__ __forceinline__ float digits_value(const i32x4 &d) {
    return static_cast<float>(d[0]) + (static_cast<float>(d[1]) * 0.0078125f + static_cast<float>(d[2]) * 6.103515625e-05f);
}
// v_mfma_i32_16x16x64_i8: 16 int8 k-slots per lane in A and B alike, exact int32 accumulation.
__device__ __forceinline__ i32x4 mfma_i8(const i32x4 &a, const i32x4 &b, const i32x4 &c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]; D as above.
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

}  // namespace qlin

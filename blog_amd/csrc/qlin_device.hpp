// qlin_device.hpp -- device-side building blocks shared by the gfx950 kernels.
//
// GGUF block layouts (ggml type codes, little-endian fields), as the reference engine stores them
// (AI/codes/local-llm/src/format/gguf/GgufFile.cpp:35-55, kernel.cu:1090-1185):
//   Q4_0  32 elems / 18 B : d f16 | qs[16]            w = d*(q-8),  q = nibble (e<16 low, else high)
//   Q5_0  32 elems / 22 B : d f16 | qh u32 | qs[16]   w = d*(q-16), q = nibble | bit e of qh << 4
//   Q8_0  32 elems / 34 B : d f16 | int8 qs[32]       w = d*q
//   Q4_K 256 elems / 144 B: d f16 | dmin f16 | scales[12] | qs[128]   w = d*sc*q - dmin*m
//   Q6_K 256 elems / 210 B: ql[128] | qh[64] | int8 sc[16] | d f16    w = d*sc*q
// Every per-element value below is computed with the canonical, non-contracted order
// (no fused multiply-add), which is what makes the dequant kernels bit-exact.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qlin {

enum : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q8_1 = 9, T_Q4_K = 12, T_Q6_K = 14 };

template <int T> struct Block;
template <> struct Block<T_Q4_0> { static constexpr int elems = 32, bytes = 18; };
template <> struct Block<T_Q5_0> { static constexpr int elems = 32, bytes = 22; };
template <> struct Block<T_Q8_0> { static constexpr int elems = 32, bytes = 34; };
template <> struct Block<T_Q4_K> { static constexpr int elems = 256, bytes = 144; };
template <> struct Block<T_Q6_K> { static constexpr int elems = 256, bytes = 210; };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (nontemporal: the weight stream is read once).
__device__ __forceinline__ u32x4 ld_stream16(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// f32 -> binary16 bits, round to nearest even, f16 subnormals kept (the kernels' FP16 denorm mode
// is "preserve").  Pinned to the scalar v_cvt_f16_f32: the packed v_cvt_pk_f16_f32 that the
// compiler forms from two adjacent conversions does not give the same bits for every input.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float v) {
    uint32_t r;
    asm volatile("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(v));
    return r & 0xffffu;
}

// Exact IEEE products / differences that the compiler may not fuse.
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float sub_rn(float a, float b) { return __fsub_rn(a, b); }

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    return *reinterpret_cast<const uint16_t *>(p);
}

// Q4_K 6-bit (scale, min) of sub-block j from the 12 scale bytes packed in three dwords
// (kernel.cu:913-921).
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                              int &sc, int &m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63;
        m = (s1 >> (8 * j)) & 63;
    } else {
        const int jj = 8 * (j - 4);
        sc = ((s2 >> jj) & 0x0f) | (((s0 >> (jj + 6)) & 3) << 4);
        m = ((s2 >> (jj + 4)) & 0x0f) | (((s1 >> (jj + 6)) & 3) << 4);
    }
}

// ---- per-element decoders (canonical values; used by dequant and the generic paths) ----------

// Q4_K element e (0..255) of the super-block at b.
__device__ __forceinline__ float q4k_value(const uint8_t *b, int e) {
    const float d = f16_bits_to_f32(ld_u16(b));
    const float dmin = f16_bits_to_f32(ld_u16(b + 2));
    const int j = e >> 5;
    const uint32_t s0 = b[4] | (b[5] << 8) | (b[6] << 16) | (static_cast<uint32_t>(b[7]) << 24);
    const uint32_t s1 = b[8] | (b[9] << 8) | (b[10] << 16) | (static_cast<uint32_t>(b[11]) << 24);
    const uint32_t s2 = b[12] | (b[13] << 8) | (b[14] << 16) | (static_cast<uint32_t>(b[15]) << 24);
    int sc, m;
    q4k_scale_min(j, s0, s1, s2, sc, m);
    const uint8_t byte = b[16 + (j >> 1) * 32 + (e & 31)];
    const int q = (j & 1) ? (byte >> 4) : (byte & 0x0f);
    return sub_rn(mul_rn(mul_rn(d, static_cast<float>(sc)), static_cast<float>(q)),
                  mul_rn(dmin, static_cast<float>(m)));
}

// Q6_K element e (0..255): half h = e/128; group g = (e%128)/32, lane l = e%32.
__device__ __forceinline__ float q6k_value(const uint8_t *b, int e) {
    const int half = e >> 7, within = e & 127, g = within >> 5, l = within & 31;
    const uint8_t lo_byte = b[half * 64 + l + 32 * (g & 1)];
    const int lo = (g < 2) ? (lo_byte & 0x0f) : (lo_byte >> 4);
    const int hi = (b[128 + half * 32 + l] >> (2 * g)) & 3;
    const int q = (lo | (hi << 4)) - 32;
    const int sc = static_cast<int8_t>(b[192 + half * 8 + l / 16 + 2 * g]);
    const float d = f16_bits_to_f32(ld_u16(b + 208));
    return mul_rn(mul_rn(d, static_cast<float>(sc)), static_cast<float>(q));
}

__device__ __forceinline__ float q50_value(const uint8_t *b, int e) {
    const float d = f16_bits_to_f32(ld_u16(b));
    const uint32_t qh = ld_u16(b + 2) | (ld_u16(b + 4) << 16);
    const int lo = (e < 16) ? (b[6 + e] & 0x0f) : (b[6 + e - 16] >> 4);
    const int q = lo | static_cast<int>(((qh >> e) & 1u) << 4);
    return mul_rn(d, static_cast<float>(q - 16));
}

__device__ __forceinline__ float q80_value(const uint8_t *b, int e) {
    const float d = f16_bits_to_f32(ld_u16(b));
    return mul_rn(d, static_cast<float>(static_cast<int8_t>(b[2 + e])));
}

__device__ __forceinline__ float q40_value(const uint8_t *b, int e) {
    const float d = f16_bits_to_f32(ld_u16(b));
    const int q = (e < 16) ? (b[2 + e] & 0x0f) : (b[2 + e - 16] >> 4);
    return mul_rn(d, static_cast<float>(q - 8));
}

template <int T>
__device__ __forceinline__ float block_value(const uint8_t *b, int e) {
    if constexpr (T == T_Q4_K) return q4k_value(b, e);
    else if constexpr (T == T_Q6_K) return q6k_value(b, e);
    else if constexpr (T == T_Q5_0) return q50_value(b, e);
    else if constexpr (T == T_Q8_0) return q80_value(b, e);
    else return q40_value(b, e);
}

// ---- prefill GEMM tile order ---------------------------------------------------------------------
// The tile (weight tile bx of nx, token tile by of ny) of workgroup L of a one-dimensional grid of
// nx * ny.  Workgroups go to the 8 XCDs in turn (L % 8), and each XCD has its own L2: XCD x takes
// weight tiles x, x + 8, ... and runs a weight tile's ny token tiles one after another, so each
// weight tile is fetched once into the L2 that all its workgroups read.  Weight tiles past the last
// multiple of 8 follow in the same token-tile-minor order.
#ifndef QLIN_GEMM_XCD
#define QLIN_GEMM_XCD 1
#endif
__device__ __forceinline__ void gemm_tile(int nx, int ny, int &bx, int &by) {
#if QLIN_GEMM_XCD
    const int L = blockIdx.x, nx8 = nx & ~7, head = nx8 * ny;
    if (L < head) {
        const int i = L >> 3, u = i / ny;
        bx = u * 8 + (L & 7);
        by = i - u * ny;
    } else {
        const int r = L - head, u = r / ny;
        bx = nx8 + u;
        by = r - u * ny;
    }
#else
    bx = blockIdx.x;
    by = blockIdx.y;
#endif
}
inline dim3 gemm_grid(int nx, int ny) { return QLIN_GEMM_XCD ? dim3(nx * ny) : dim3(nx, ny); }

// ---- wave64 reductions ------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Wave maximum in register moves (every lane active, wave-uniform control flow): DPP within each
// row of 16 lanes (quads, then the other quad of each 8, then the other 8), then the gfx950 lane
// swaps between rows 2r and 2r + 1 and between the two halves of the wave.  Every lane gets the
// maximum; fmaxf is exact, so the result is the same as any other order's.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_move<0xb1>(v));   // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, dpp_move<0x4e>(v));   // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_move<0x140>(v));  // row_mirror
    const auto s16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                      false, false);
    // (the two results hold rows 0, 0, 2, 2 and 1, 1, 3, 3: their maximum is the row pair's)
    v = fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(s16[0])),
              __builtin_bit_cast(float, static_cast<uint32_t>(s16[1])));
    const auto s32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                      false, false);
    return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(s32[0])),
                 __builtin_bit_cast(float, static_cast<uint32_t>(s32[1])));
}

// ---- router top-k of one token by one wave (at most 64 experts) --------------------------------
// Lane e holds expert e's logit (non-finite as -inf).  Pick r is the expert with exactly r experts
// ahead of it -- a larger logit, or an equal one at a lower index -- which is the order of k
// successive argmaxes that prefer the lower index, the reference's strict-'>' first maximum; they are
// taken here as k wave maxima, each pick the lowest lane holding the maximum, which then drops out.
// Picks past the finite logits fall back to expert r (0 past ne) with weight 0; a pick's weight is
// exp(l - max) / (the exponentials summed in expert order) times scaling.
// Wave-local: no workgroup barrier.  live is uniform per wave; only live waves read logits (row of ne
// floats), use ex (64 floats, 16-byte aligned, of LDS that no other wave uses) and put their picks,
// through put(r, expert, weight), called by one lane per pick.
template <class Put>
__device__ __forceinline__ void route_token_rank(bool live, const float *row, int ne, int k, float scaling, float *ex,
                                                 Put put) {
    if (!live) return;
    const int lane = threadIdx.x & 63;
    const float l = lane < ne ? row[lane] : -INFINITY;
    const float v = isfinite(l) ? l : -INFINITY;
    const float maxv = wave_max_dpp(v);
    ex[lane] = isfinite(maxv) ? expf(v - maxv) : 0.0f;  // 0 for -inf and past ne
    // The wave's LDS accesses run in program order, so every lane reads all 64 values just written.
    __builtin_amdgcn_wave_barrier();
    // in expert order (every lane alike); past ne the exponentials are 0 and leave the sum as it is
    float denom = 0.0f;
    if (isfinite(maxv)) {
        float4 q[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = reinterpret_cast<const float4 *>(ex)[i];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            denom += q[i].x;
            denom += q[i].y;
            denom += q[i].z;
            denom += q[i].w;
        }
    }
    const bool fin = v != -INFINITY;
    const int nf = static_cast<int>(__popcll(__ballot(fin)));
    float cur = v;  // the finite logits not yet picked
    const int kf = min(k, nf);
    for (int r = 0; r < kf; ++r) {
        const float m = wave_max_dpp(cur);  // finite: nf - r finite logits remain
        const int p = static_cast<int>(__ffsll(static_cast<long long>(__ballot(cur == m)))) - 1;
        if (lane == p) {
            put(r, lane, (denom > 0.0f ? expf(v - maxv) / denom : 0.0f) * scaling);
            cur = -INFINITY;
        }
    }
    for (int r = nf + lane; r < k; r += 64) put(r, r < ne ? r : 0, 0.0f);
}

}  // namespace qlin

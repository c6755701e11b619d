// qlin_rows.hpp -- one wave's Q4_K dot of 16 weight rows against a 16-token tile of f32 activations on
// the bf16 matrix cores (the tokens as the MFMA rows), shared by q4k_dense_kernel (qlin_dense.hip) and
// the shared-expert tiles of the grouped MoE gate/up launch (qlin_moe_grouped.hip), so that both give
// the same bits.
//
// The element value of sub-block j is w = dsc*q - dm (dsc = d*sc_j, dm = dmin*m_j, kernel.cu:913-930),
// so  sum_k w x = dsc * sum x (128 + q) - (128 dsc + dm) * sum x,  where the nibble q enters as the
// exact bf16 128 + q and x as the bf16 pair hi = bf16(x), lo = bf16(x - hi).  Per sub-block one MFMA
// pair gives sum x (128 + q) for the 16 rows, and one more pair against an all-ones B gives sum x in
// the same D layout; two fmas per output apply the scales.  Lane l supplies weight row l % 16 and
// token l % 16, and k-slots 8g .. 8g+7 (g = l / 16) of each sub-block; D holds tokens 4g .. 4g+3 of
// row l % 16.
#pragma once

#include "qlin_device.hpp"
#include "qlin_mfma.hpp"

namespace qlin {

// The raw bytes a lane needs of one Q4_K super-block: the header (d, dmin, 12 scale bytes) and,
// for each pair c of sub-blocks, qs bytes 32c + 8g .. 32c + 8g + 7 (low nibbles: sub-block 2c,
// high nibbles: sub-block 2c + 1).
struct Q4KRaw {
    u32x4 h;
    uint32_t q[8];
};

__device__ __forceinline__ void load_q4k(Q4KRaw &r, const uint8_t *sb, int g) {
    r.h = ld16(sb);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint2 v = *reinterpret_cast<const uint2 *>(sb + 16 + 32 * c + 8 * g);
        r.q[2 * c] = v.x;
        r.q[2 * c + 1] = v.y;
    }
}

// x of super-block sb for this lane: elements 8g .. 8g+7 of each of the 8 sub-blocks (xr = the lane's
// token row at offset 8g, plus sb * 256)
__device__ __forceinline__ void load_x_sb(float4 (&xs)[16], const float *xr) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        xs[2 * j] = *reinterpret_cast<const float4 *>(xr + 32 * j);
        xs[2 * j + 1] = *reinterpret_cast<const float4 *>(xr + 32 * j + 4);
    }
}

// D[w] += one super-block's dots of the rows whose raw bytes are cur[w], sub-block by sub-block in order.
template <int NW>
__device__ __forceinline__ void q4k_sb_math(const Q4KRaw (&cur)[NW], const float4 (&xs)[16], f32x4 (&D)[NW]) {
    const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};  // bf16 1.0 in every slot
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 x0 = xs[2 * j], x1 = xs[2 * j + 1];
        uint32_t h[4], l[4];
        split_bf16x2(x0.x, x0.y, h[0], l[0]);
        split_bf16x2(x0.z, x0.w, h[1], l[1]);
        split_bf16x2(x1.x, x1.y, h[2], l[2]);
        split_bf16x2(x1.z, x1.w, h[3], l[3]);
        const u32x4 ahi = {h[0], h[1], h[2], h[3]}, alo = {l[0], l[1], l[2], l[3]};
        const f32x4 X = mfma(alo, ones, mfma(ahi, ones, f32x4{0.0f, 0.0f, 0.0f, 0.0f}));
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            // this lane's row: dsc and the coefficient of sum x for sub-block j
            int sc, mn;
            q4k_scale_min(j, cur[w].h.y, cur[w].h.z, cur[w].h.w, sc, mn);
            const float dsc = mul_rn(f16_bits_to_f32(cur[w].h.x & 0xffffu), static_cast<float>(sc));
            const float cx = -(128.0f * dsc + mul_rn(f16_bits_to_f32(cur[w].h.x >> 16), static_cast<float>(mn)));
            // elements 8g .. 8g+7 of sub-block j: the low (j even) or high nibbles of the lane's
            // bytes of sub-block pair j / 2
            const int sh = 4 * (j & 1);
            const u32x4 B = weights_operand2((cur[w].q[2 * (j >> 1)] >> sh) & 0x0f0f0f0fu,
                                             (cur[w].q[2 * (j >> 1) + 1] >> sh) & 0x0f0f0f0fu);
            const f32x4 Dj = mfma(alo, B, mfma(ahi, B, f32x4{0.0f, 0.0f, 0.0f, 0.0f}));
#pragma unroll
            for (int r = 0; r < 4; ++r) D[w][r] = fmaf(cx, X[r], fmaf(dsc, Dj[r], D[w][r]));
        }
    }
}

// D[w] += the dots of rows rp[w] (this lane's row of matrix w) over super-blocks sb0, sb0 + step, ...
// below nsb, for the tile's tokens whose x rows start at xrow (this lane's token, offset 8g).  Each
// super-block's x is requested first, then the next super-block's weights, then the math: a wait for
// x never waits for the weight prefetch (loads complete in issue order), and x's 16 loads share one
// round trip.  cur holds super-block sb0's weights (when sb0 < nsb), requested by the caller.
template <int NW>
__device__ __forceinline__ void q4k_rows_dot_from(Q4KRaw (&cur)[NW], const uint8_t *const *rp, const float *xrow,
                                                  int sb0, int step, int nsb, int g, f32x4 (&D)[NW]) {
    int sb = sb0;
    while (sb < nsb) {  // uniform
        float4 xs[16];
        load_x_sb(xs, xrow + sb * 256);
        __builtin_amdgcn_sched_barrier(0);
        const int sb2 = sb + step;
        Q4KRaw nxt[NW];
        if (sb2 < nsb) {  // uniform
#pragma unroll
            for (int w = 0; w < NW; ++w) load_q4k(nxt[w], rp[w] + static_cast<size_t>(sb2) * 144, g);
        }
        __builtin_amdgcn_sched_barrier(0);
        q4k_sb_math<NW>(cur, xs, D);
        if (sb2 >= nsb) break;
#pragma unroll
        for (int w = 0; w < NW; ++w) cur[w] = nxt[w];
        sb = sb2;
    }
}

template <int NW>
__device__ __forceinline__ void q4k_rows_dot(const uint8_t *const *rp, const float *xrow, int sb0, int step, int nsb,
                                             int g, f32x4 (&D)[NW]) {
    Q4KRaw cur[NW];
    if (sb0 < nsb) {
#pragma unroll
        for (int w = 0; w < NW; ++w) load_q4k(cur[w], rp[w] + static_cast<size_t>(sb0) * 144, g);
    }
    q4k_rows_dot_from<NW>(cur, rp, xrow, sb0, step, nsb, g, D);
}

// The same dot for nt <= NT 16-row tiles of one matrix, one after another (D[t] for tile t, rows
// rp[t]), each over super-blocks sb0, sb0 + step, ...: the weights one step ahead run on across the
// tiles, so the next tile's first weights travel while the last super-block of a tile is computed.
// cur holds tile 0's super-block sb0 (when sb0 < nsb).  Each D[t] takes the adds q4k_rows_dot<1>
// gives it.
template <int NT>
__device__ __forceinline__ void q4k_tiles_dot(Q4KRaw (&cur)[1], const uint8_t *const (&rp)[NT], int nt,
                                              const float *xrow, int sb0, int step, int nsb, int g,
                                              f32x4 (&D)[NT]) {
    if (sb0 >= nsb) return;  // uniform
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (t >= nt) break;  // uniform
        f32x4 Dt[1] = {D[t]};
        for (int sb = sb0; sb < nsb; sb += step) {  // uniform
            float4 xs[16];
            load_x_sb(xs, xrow + sb * 256);
            __builtin_amdgcn_sched_barrier(0);
            const int sb2 = sb + step;
            Q4KRaw nxt[1];
            const uint8_t *np = sb2 < nsb ? rp[t] + static_cast<size_t>(sb2) * 144
                                          : (t + 1 < NT && t + 1 < nt ? rp[t + 1 < NT ? t + 1 : t] + static_cast<size_t>(sb0) * 144
                                                                      : nullptr);
            if (np) load_q4k(nxt[0], np, g);  // uniform
            __builtin_amdgcn_sched_barrier(0);
            q4k_sb_math<1>(cur, xs, Dt);
            if (np) cur[0] = nxt[0];
        }
        D[t] = Dt[0];
    }
}

}  // namespace qlin

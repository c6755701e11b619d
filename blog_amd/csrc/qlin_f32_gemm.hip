// qlin_f32_gemm.hip -- Q4_K and Q6_K weights x f32 activations, the prefill GEMM behind quant_matmul
// (m > 1), on the fp16 matrix cores of gfx950 (Q6_K: see compute_q6 below).
//
// Computes y[r, o] (=|+=) sum_k w(o, k) x[r, k] with w(o, k) = d*sc_j*q - dmin*m_j (kernel.cu:913-930)
// and f32 activations x, the reference's quant_matmul_kernel (AI/codes/local-llm/src/backend/cuda/
// ops/kernel.cu:1254-1279) that TensorTool::quant_direct_gemm runs for every m > 1 product
// (TensorTool.cpp:163-168).  Per super-block and output,
//   sum_k w x = d * sum_j sc_j sum_{k in j} q_k x_k  -  dmin * sum_j m_j X_j,    X_j = sum_{k in j} x_k.
//
// Operands (v_mfma_f32_16x16x32_f16, products exact, f32 accumulation):
//   A (activations): per token and super-block, x is scaled by a power of two 2^s so that its largest
//     magnitude lies in [2^14, 2^15), and split into fp16 hi = fp16(x 2^s), lo = fp16(x 2^s - hi):
//     hi + lo equals x 2^s to within 2^-22 of that largest magnitude.  The two parts are two MFMAs
//     into the same accumulator.
//   B (weights): sc_j*q, an integer <= 63*15 = 945, exact in fp16 (as in the Q8_1 GEMM).
// So the 8 sub-blocks of a super-block accumulate in one MFMA result per tile (16 MFMAs), with no
// per-block scaling; the min term takes two more MFMAs against the sums X_j 2^s / 32 (hi and lo) and
// B = 32 m_j.  Per output and super-block the epilogue is ldexp(d*D - dmin*Dm, -s) added to the
// total: the x scale is a power of two, so it is exact, and it never needs the whole row.
//
// Tiling (as the Q8_1 GEMM).  A workgroup of 8 waves computes 64 tokens x 256 weight rows, each wave
// 32 rows (two 16-row tiles) for all 64 tokens (four 16-token tiles).  Per super-block the
// workgroup stages its 64 x 256 activations once into the A layout in LDS (double-buffered, the next
// super-block's x requested while the current one is multiplied): lane (token, sub-block) of the
// staging holds the token's 32 values of one sub-block, and the token's 8 lanes find its scale by
// three shuffles.  Each wave decodes its own weight rows from global memory into B operands, the
// register set reloaded part by part with the next super-block as in the Q8_1 GEMM.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

#include <type_traits>

namespace qlin {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#ifndef QLIN_F32_GEMM_SMALL
#define QLIN_F32_GEMM_SMALL 1  // the 4-wave, 32-token geometry for launches that would leave half the CUs idle
#endif
constexpr int kNT = 2;  // 16-row weight tiles per wave
// A workgroup's geometry: W waves of 32 rows each for MT 16-token tiles.  The default (8 waves, 64
// tokens: 256 rows) covers large grids; a launch that would leave more than half the CUs idle (short
// prompts) takes 4 waves and 32 tokens (128 rows), four times as many workgroups.
template <int W, int MT>
struct Geo {
    static constexpr int kWaves = W, kThreads = W * 64;
    static constexpr int kBN = W * kNT * 16;       // weight rows per workgroup
    static constexpr int kMT = MT, kBM = MT * 16;  // 16-token tiles and tokens per workgroup
    static_assert(kBM == W * 8, "staging: each wave stages 8 tokens, one lane per (token, sub-block)");
    // One LDS buffer (uint4 units): the hi plane [mt][j][lane], the lo plane, the min-term rows hi
    // [mt][lane] and lo (lanes >= 16 stay zero), then the tokens' scale exponents s (ints).  Two buffers
    // (145 KB for the default).
    static constexpr int kPlane = MT * 8 * 64;
    static constexpr int kRows = MT * 64;
    static constexpr int kExp = kBM / 4;
    static constexpr int kBuf = 2 * kPlane + 2 * kRows + kExp;
    static constexpr size_t kLdsBytes = 2 * kBuf * sizeof(uint4);
    static_assert(kLdsBytes <= 160 * 1024, "fits the CU's LDS");
};
using GeoLarge = Geo<8, 4>;
using GeoSmall = Geo<4, 2>;

struct F32GemmArgs {
    const uint8_t *w;
    size_t rb;  // weight row bytes
    const float *x;
    float *y;
    int n, m, k, nsb, add;
};

__device__ __forceinline__ f32x4 mfma(const uint4 &a, const uint4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}
__device__ __forceinline__ uint32_t h2u(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ f16x2 u2h(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ f16x2 splat(float v) {
    const _Float16 h = static_cast<_Float16>(v);
    return f16x2{h, h};
}

// B operand of sub-block J for this lane: 8 nibbles (k = 8g .. 8g+7 of the sub-block) times sc, as
// fp16 integers: bytes (q, 0x64) are the fp16 1024 + q, and (1024 + q) sc - 1024 sc = q sc exactly.
template <int J>
__device__ __forceinline__ uint4 weights_b(const uint2 &q, f16x2 sc2, f16x2 c2) {
    const uint32_t v0 = (J & 1) ? (q.x >> 4) & 0x0f0f0f0fu : q.x & 0x0f0f0f0fu;
    const uint32_t v1 = (J & 1) ? (q.y >> 4) & 0x0f0f0f0fu : q.y & 0x0f0f0f0fu;
    const uint32_t k64 = 0x64646464u;
    uint4 r;
    r.x = h2u(__builtin_elementwise_fma(u2h(__builtin_amdgcn_perm(k64, v0, 0x04010400u)), sc2, c2));
    r.y = h2u(__builtin_elementwise_fma(u2h(__builtin_amdgcn_perm(k64, v0, 0x04030402u)), sc2, c2));
    r.z = h2u(__builtin_elementwise_fma(u2h(__builtin_amdgcn_perm(k64, v1, 0x04010400u)), sc2, c2));
    r.w = h2u(__builtin_elementwise_fma(u2h(__builtin_amdgcn_perm(k64, v1, 0x04030402u)), sc2, c2));
    return r;
}

// (hi, lo) fp16 parts of v, packed two values per dword (first value in the low half)
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
    const _Float16 ha = static_cast<_Float16>(a), hb = static_cast<_Float16>(b);
    const _Float16 la = static_cast<_Float16>(a - static_cast<float>(ha));
    const _Float16 lb = static_cast<_Float16>(b - static_cast<float>(hb));
    hi = h2u(f16x2{ha, hb});
    lo = h2u(f16x2{la, lb});
}

template <int V> using ic = std::integral_constant<int, V>;

// Q6_K (210-byte super-blocks: ql[128], qh[64], int8 scales[16], d f16; kernel.cu:1122-1156): element l
// of 32-block j = 4 h + g6 is q = (nibble g6 / 2 of ql[64 h + 32 (g6 % 2) + l]) | (bits 2 g6 .. 2 g6 + 1
// of qh[32 h + l]) << 4, value d * sc[8 h + 2 g6 + l / 16] * (q - 32).  Lane group g holds elements
// 8g .. 8g+7 of a block, all under scale 2 g6 + g / 2, so B = sc (q - 32) carries the block's two
// scales; |sc (q - 32)| <= 4096 is not exact in fp16, so it is split as B1 = fp16(sc (q - 32)) and
// B2 = fma(q - 32, sc, -B1), both exact integers (|B2| <= 1).  A block takes hi B1, hi B2 and lo B1
// into the accumulator; lo B2 is at most 2^-22 of hi B1 and is left out.  d applies per super-block.
// Rows: 4-byte aligned with an even number of super-blocks (super-block s starts 2 past a multiple of
// 4 when s is odd); each 8-byte piece a lane needs is read as 3 aligned dwords and realigned.
struct K6Raw {
    uint32_t ql[4][3], qh[2][3], sd[5];
};
__device__ __forceinline__ void load3(uint32_t (&w)[3], const uint8_t *p) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
    w[0] = q[0];
    w[1] = q[1];
    w[2] = q[2];
}
__device__ __forceinline__ uint2 piece(const uint32_t (&w)[3], int off) {
    return make_uint2(__builtin_amdgcn_alignbyte(w[1], w[0], off), __builtin_amdgcn_alignbyte(w[2], w[1], off));
}

template <int FMT, class G>
__global__ __launch_bounds__(G::kThreads) void f32_gemm_kernel(const F32GemmArgs a) {
    constexpr int kThreads = G::kThreads, kBN = G::kBN, kMT = G::kMT, kBM = G::kBM;
    constexpr int kPlane = G::kPlane, kRows = G::kRows, kBuf = G::kBuf;
    constexpr bool Q6 = FMT == T_Q6_K;
    extern __shared__ uint4 lds[];
    auto hi_plane = [&](int buf) { return lds + buf * kBuf; };
    auto lo_plane = [&](int buf) { return lds + buf * kBuf + kPlane; };
    auto hi_rows = [&](int buf) { return lds + buf * kBuf + 2 * kPlane; };
    auto lo_rows = [&](int buf) { return lds + buf * kBuf + 2 * kPlane + kRows; };
    auto exps = [&](int buf) { return reinterpret_cast<int *>(lds + buf * kBuf + 2 * kPlane + 2 * kRows); };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    int bx, by;
    gemm_tile((a.n + kBN - 1) / kBN, (a.m + kBM - 1) / kBM, bx, by);
    const int m0 = by * kBM;
    const int o0 = bx * kBN + wave * kNT * 16;

    const uint8_t *wrow[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) wrow[t] = a.w + static_cast<size_t>(min(o0 + t * 16 + n, a.n - 1)) * a.rb;

    // staging role: token st (0..63) of the workgroup and sub-block sj; tokens past m repeat the last
    // row (their outputs are never stored)
    const int st = wave * 8 + (lane >> 3), sj = lane & 7;
    const int smt = st >> 4, sn = st & 15;
    const float *xrow = a.x + static_cast<size_t>(min(m0 + st, a.m - 1)) * a.k + 32 * sj;

    // lanes 16..63 of the min-term rows stay zero
    for (int i = tid; i < 2 * 2 * kRows; i += kThreads)
        if ((i & 63) >= 16) lds[(i / (2 * kRows)) * kBuf + 2 * kPlane + i % (2 * kRows)] = make_uint4(0u, 0u, 0u, 0u);

    f32x4 acc[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int t = 0; t < kNT; ++t) acc[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    struct WRawQ4 {
        uint4 hdr[kNT];
        uint2 qs[kNT][4];
    };
    struct WRawQ6 {
        K6Raw k[kNT];
    };
    using WRaw = std::conditional_t<Q6, WRawQ6, WRawQ4>;
    // Q6_K: super-block s of the rows (past the end the last one of the same parity), from the aligned
    // address at or 2 before it
    auto sbase = [&](int t, int sb) {
        sb = min(sb, a.nsb - 2 + (sb & 1));
        return wrow[t] + static_cast<size_t>(sb) * 210 - 2 * (sb & 1);
    };
    auto fetch_half = [&](WRawQ6 &w, int sb, int h) {
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            const uint8_t *b = sbase(t, sb);
            load3(w.k[t].ql[2 * h], b + 64 * h + 8 * g);
            load3(w.k[t].ql[2 * h + 1], b + 64 * h + 32 + 8 * g);
            load3(w.k[t].qh[h], b + 128 + 32 * h + 8 * g);
        }
    };
    auto fetch_sd = [&](WRawQ6 &w, int sb) {
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            const uint32_t *q = reinterpret_cast<const uint32_t *>(sbase(t, sb) + 192);
#pragma unroll
            for (int i = 0; i < 5; ++i) w.k[t].sd[i] = q[i];
        }
    };
    struct XRaw {
        float4 v[8];
    };
    // past the end a fetch reloads the last super-block (valid addresses, never used)
    auto fetch_hdr = [&](WRawQ4 &w, int sb) {
        sb = min(sb, a.nsb - 1);
#pragma unroll
        for (int t = 0; t < kNT; ++t) w.hdr[t] = *reinterpret_cast<const uint4 *>(wrow[t] + static_cast<size_t>(sb) * 144);
    };
    auto fetch_qs = [&](WRawQ4 &w, int sb, int pr) {
        sb = min(sb, a.nsb - 1);
#pragma unroll
        for (int t = 0; t < kNT; ++t)
            w.qs[t][pr] = *reinterpret_cast<const uint2 *>(wrow[t] + static_cast<size_t>(sb) * 144 + 16 + 32 * pr + 8 * g);
    };
    auto fetch_x = [&](XRaw &x, int sb) {
        sb = min(sb, a.nsb - 1);
        const float4 *p = reinterpret_cast<const float4 *>(xrow + static_cast<size_t>(sb) * 256);
#pragma unroll
        for (int i = 0; i < 8; ++i) x.v[i] = p[i];
    };

    // The token's 32 values of sub-block sj into buffer buf: the exponent s of the token's super-block
    // (its largest |x| below 2^15 after scaling; 0 for an all-zero or non-finite block), the hi and lo
    // planes in the A layout (lane (g, n) of tile smt: elements 8g .. 8g+7 of sub-block sj of token
    // sn), and the block sum / 32 (hi, lo) in slot sj of the token's min-term row.
    auto stage = [&](const XRaw &x, int buf) {
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            am = fmaxf(fmaxf(am, fmaxf(fabsf(x.v[i].x), fabsf(x.v[i].y))), fmaxf(fabsf(x.v[i].z), fabsf(x.v[i].w)));
        am = fmaxf(am, __shfl_xor(am, 1, 64));
        am = fmaxf(am, __shfl_xor(am, 2, 64));
        am = fmaxf(am, __shfl_xor(am, 4, 64));
        int ex = 0;
        (void)frexpf(am, &ex);
        const int s = (am > 0.0f && am <= 3.4e38f) ? 15 - ex : 0;
        float xs[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            xs[4 * i] = ldexpf(x.v[i].x, s);
            xs[4 * i + 1] = ldexpf(x.v[i].y, s);
            xs[4 * i + 2] = ldexpf(x.v[i].z, s);
            xs[4 * i + 3] = ldexpf(x.v[i].w, s);
        }
        uint4 *ph = hi_plane(buf) + (smt * 8 + sj) * 64 + sn;
        uint4 *pl = lo_plane(buf) + (smt * 8 + sj) * 64 + sn;
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
            uint32_t h[4], l[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) split2(xs[8 * gg + 2 * e], xs[8 * gg + 2 * e + 1], h[e], l[e]);
            ph[16 * gg] = make_uint4(h[0], h[1], h[2], h[3]);
            pl[16 * gg] = make_uint4(l[0], l[1], l[2], l[3]);
        }
        if constexpr (!Q6) {
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) sum += xs[i];
            sum *= 0.03125f;
            const _Float16 sh = static_cast<_Float16>(sum);
            const _Float16 sl = static_cast<_Float16>(sum - static_cast<float>(sh));
            reinterpret_cast<_Float16 *>(hi_rows(buf) + smt * 64 + sn)[sj] = sh;
            reinterpret_cast<_Float16 *>(lo_rows(buf) + smt * 64 + sn)[sj] = sl;
        }
        if (sj == 0) exps(buf)[st] = s;
    };

    // One super-block: B operands of the 8 sub-blocks against both x parts into one accumulator per
    // tile, the min term, then the scaled, exponent-corrected sum into acc.
    struct Frag {
        uint4 h[kMT], l[kMT];
    };
    auto load_frag_of = [&](Frag &f, int buf, int J) {
        const uint4 *hp = hi_plane(buf), *lp = lo_plane(buf);
#pragma unroll
        for (int i = 0; i < kMT; ++i) {
            f.h[i] = hp[(i * 8 + J) * 64 + lane];
            f.l[i] = lp[(i * 8 + J) * 64 + lane];
        }
    };
    // Q6_K: one super-block's blocks (three MFMAs each), then d and the exponent into acc
    auto compute_q6 = [&](WRawQ6 &w, int buf, int next) {
        const int off = 2 * (next - 1 & 1);
        uint32_t s4[kNT][4];
        float dw[kNT];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) s4[t][i] = __builtin_amdgcn_alignbyte(w.k[t].sd[i + 1], w.k[t].sd[i], off);
            dw[t] = f16_bits_to_f32((w.k[t].sd[4] >> (8 * off)) & 0xffffu);
        }
        fetch_sd(w, next);
        f32x4 D[kMT][kNT];
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int t = 0; t < kNT; ++t) D[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const int gb = g >> 1;
        auto block = [&](auto jc, const Frag &f) {
            constexpr int J = decltype(jc)::value, H = J >> 2, G6 = J & 3;
            uint4 B1[kNT], B2[kNT];
#pragma unroll
            for (int t = 0; t < kNT; ++t) {
                // scale 8 H + 2 G6 + g / 2 = byte 2 J + g / 2 of the 16, as the fp16 pair (sc, sc)
                const uint32_t scb = (s4[t][J >> 1] >> (8 * (2 * (J & 1) + gb))) ^ 0x80u;
                const f16x2 sc2 = u2h(__builtin_amdgcn_perm(0x64646464u, scb, 0x04000400u)) + splat(-1152.0f);
                const uint2 l2 = piece(w.k[t].ql[2 * H + (G6 & 1)], off), h2 = piece(w.k[t].qh[H], off);
                const uint32_t u0 = ((l2.x >> (4 * (G6 >> 1))) & 0x0f0f0f0fu) | (((h2.x >> (2 * G6)) & 0x03030303u) << 4);
                const uint32_t u1 = ((l2.y >> (4 * (G6 >> 1))) & 0x0f0f0f0fu) | (((h2.y >> (2 * G6)) & 0x03030303u) << 4);
                const f16x2 c32 = splat(-1056.0f);  // (q, 0x64) = 1024 + q
                f16x2 q[4];
                q[0] = u2h(__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) + c32;
                q[1] = u2h(__builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) + c32;
                q[2] = u2h(__builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) + c32;
                q[3] = u2h(__builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) + c32;
                uint32_t b1[4], b2[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const f16x2 p1 = q[e] * sc2;
                    b1[e] = h2u(p1);
                    b2[e] = h2u(__builtin_elementwise_fma(q[e], sc2, -p1));
                }
                B1[t] = make_uint4(b1[0], b1[1], b1[2], b1[3]);
                B2[t] = make_uint4(b2[0], b2[1], b2[2], b2[3]);
            }
#pragma unroll
            for (int i = 0; i < kMT; ++i)
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    D[i][t] = mfma(f.h[i], B1[t], D[i][t]);
                    D[i][t] = mfma(f.h[i], B2[t], D[i][t]);
                    D[i][t] = mfma(f.l[i], B1[t], D[i][t]);
                }
            if constexpr (J == 3) fetch_half(w, next, 0);
            if constexpr (J == 7) fetch_half(w, next, 1);
            __builtin_amdgcn_sched_barrier(0);
        };
        Frag f0, f1;
        load_frag_of(f0, buf, 0);
        load_frag_of(f1, buf, 1);
        block(ic<0>{}, f0);
        load_frag_of(f0, buf, 2);
        block(ic<1>{}, f1);
        load_frag_of(f1, buf, 3);
        block(ic<2>{}, f0);
        load_frag_of(f0, buf, 4);
        block(ic<3>{}, f1);
        load_frag_of(f1, buf, 5);
        block(ic<4>{}, f0);
        load_frag_of(f0, buf, 6);
        block(ic<5>{}, f1);
        load_frag_of(f1, buf, 7);
        block(ic<6>{}, f0);
        block(ic<7>{}, f1);
        const int *ex = exps(buf);
#pragma unroll
        for (int i = 0; i < kMT; ++i) {
            const int4 e4 = *reinterpret_cast<const int4 *>(ex + i * 16 + 4 * g);
            const int er[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
            for (int t = 0; t < kNT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i][t][r] += ldexpf(D[i][t][r] * dw[t], -er[r]);
        }
    };
    auto compute = [&](WRawQ4 &w, int buf, int next) {
        const uint4 *hp = hi_plane(buf), *lp = lo_plane(buf);
        float dd[kNT], dmin[kNT];
        uint32_t mlo[kNT], mhi[kNT];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            dd[t] = f16_bits_to_f32(w.hdr[t].x & 0xffffu);
            dmin[t] = f16_bits_to_f32(w.hdr[t].x >> 16);
            mlo[t] = w.hdr[t].z;
            mhi[t] = w.hdr[t].w;
        }
        // the 8 scales of a tile as fp16 pairs (sc_2i, sc_2i+1) (kernel.cu:913-921 on whole dwords)
        const f16x2 off = splat(-1024.0f);
        auto pairs = [&](uint32_t v, f16x2 *dst) {
            dst[0] = u2h(__builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)) + off;
            dst[1] = u2h(__builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)) + off;
        };
        f16x2 scp[kNT][4], cp[kNT][4];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            const uint32_t s0 = w.hdr[t].y, s2 = w.hdr[t].w;
            pairs(s0 & 0x3f3f3f3fu, scp[t]);
            pairs((s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u), scp[t] + 2);
#pragma unroll
            for (int i = 0; i < 4; ++i) cp[t][i] = scp[t][i] * off;
        }
        fetch_hdr(w, next);
        f32x4 D[kMT][kNT];
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int t = 0; t < kNT; ++t) D[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        struct Frag {
            uint4 h[kMT], l[kMT];
        };
        auto load_frag = [&](Frag &f, int J) {
#pragma unroll
            for (int i = 0; i < kMT; ++i) {
                f.h[i] = hp[(i * 8 + J) * 64 + lane];
                f.l[i] = lp[(i * 8 + J) * 64 + lane];
            }
        };
        auto sub_block = [&](auto jc, const Frag &f) {
            constexpr int J = decltype(jc)::value;
            uint4 B[kNT];
#pragma unroll
            for (int t = 0; t < kNT; ++t) {
                const f16x2 sc2 = __builtin_shufflevector(scp[t][J >> 1], scp[t][J >> 1], J & 1, J & 1);
                const f16x2 c2 = __builtin_shufflevector(cp[t][J >> 1], cp[t][J >> 1], J & 1, J & 1);
                B[t] = weights_b<J>(w.qs[t][J >> 1], sc2, c2);
            }
#pragma unroll
            for (int i = 0; i < kMT; ++i)
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    D[i][t] = mfma(f.h[i], B[t], D[i][t]);
                    D[i][t] = mfma(f.l[i], B[t], D[i][t]);
                }
            __builtin_amdgcn_sched_barrier(0);
        };
        // fragments of sub-block J + 1 are read while J is multiplied
        Frag f0, f1;
        load_frag(f0, 0);
        load_frag(f1, 1);
        sub_block(ic<0>{}, f0);
        load_frag(f0, 2);
        sub_block(ic<1>{}, f1);
        fetch_qs(w, next, 0);
        load_frag(f1, 3);
        sub_block(ic<2>{}, f0);
        load_frag(f0, 4);
        sub_block(ic<3>{}, f1);
        fetch_qs(w, next, 1);
        load_frag(f1, 5);
        sub_block(ic<4>{}, f0);
        load_frag(f0, 6);
        sub_block(ic<5>{}, f1);
        fetch_qs(w, next, 2);
        load_frag(f1, 7);
        sub_block(ic<6>{}, f0);
        sub_block(ic<7>{}, f1);
        fetch_qs(w, next, 3);

        // min term: sum_j (X_j 2^s / 32) (32 m_j) over k-slots 0..7 (lane-group 0; the other lanes' A
        // entries are zeros), then the exponent-corrected total
        const uint4 *hr = hi_rows(buf), *lr = lo_rows(buf);
        const int *ex = exps(buf);
        const f16x2 k32 = splat(32.0f);
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            f16x2 mp[4];
            pairs(mlo[t] & 0x3f3f3f3fu, mp);
            pairs(((mhi[t] >> 4) & 0x0f0f0f0fu) | ((mlo[t] >> 2) & 0x30303030u), mp + 2);
            const uint4 b2 = make_uint4(h2u(mp[0] * k32), h2u(mp[1] * k32), h2u(mp[2] * k32), h2u(mp[3] * k32));
#pragma unroll
            for (int i = 0; i < kMT; ++i) {
                f32x4 dm = mfma(hr[i * 64 + lane], b2, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                dm = mfma(lr[i * 64 + lane], b2, dm);
                const int4 e4 = *reinterpret_cast<const int4 *>(ex + i * 16 + 4 * g);
                const int er[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float v = fmaf(dd[t], D[i][t][r], -dmin[t] * dm[r]);
                    acc[i][t][r] += ldexpf(v, -er[r]);
                }
            }
        }
    };

    WRaw w;
    XRaw x;
    if constexpr (Q6) {
        fetch_sd(w, 0);
        fetch_half(w, 0, 0);
        fetch_half(w, 0, 1);
    } else {
        fetch_hdr(w, 0);
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) fetch_qs(w, 0, pr);
    }
    fetch_x(x, 0);
    stage(x, 0);
    fetch_x(x, 1);
    __syncthreads();
    for (int sb = 0; sb < a.nsb; ++sb) {
        const int buf = sb & 1;
        if constexpr (Q6) compute_q6(w, buf, sb + 1);
        else compute(w, buf, sb + 1);
        stage(x, buf ^ 1);  // past the end: a copy of the last super-block, never read
        fetch_x(x, sb + 2);
        __syncthreads();
    }

    // lane (g, n) holds tokens 4g .. 4g+3 of each 16-token tile, weight row n of each 16-row tile
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
        const int o = o0 + t * 16 + n;
        if (o >= a.n) continue;
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tk = m0 + i * 16 + 4 * g + r;
                if (tk < a.m) {
                    float *yp = a.y + static_cast<size_t>(tk) * a.n + o;
                    *yp = a.add ? *yp + acc[i][t][r] : acc[i][t][r];
                }
            }
    }
}

}  // namespace

bool f32_gemm_ok(int type, const uint8_t *w, size_t rb, const float *x, int in_dim) {
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return false;
    if (type == T_Q4_K) return in_dim % 256 == 0 && rb % 16 == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
    if (type == T_Q6_K) return in_dim % 512 == 0 && rb % 4 == 0 && (reinterpret_cast<uintptr_t>(w) & 3u) == 0;
    return false;
}

hipError_t f32_gemm(int type, const uint8_t *w, size_t rb, const float *x, float *y, int out_dim, int in_dim, int m,
                    bool add, hipStream_t s) {
    if (out_dim == 0 || m == 0) return hipSuccess;
    F32GemmArgs a;
    a.w = w;
    a.rb = rb;
    a.x = x;
    a.y = y;
    a.n = out_dim;
    a.m = m;
    a.k = in_dim;
    a.nsb = in_dim / 256;
    a.add = add ? 1 : 0;
    auto launch = [&](auto geo) {
        using G = decltype(geo);
        const dim3 grid = gemm_grid((out_dim + G::kBN - 1) / G::kBN, (m + G::kBM - 1) / G::kBM);
        if (type == T_Q6_K) hipLaunchKernelGGL((f32_gemm_kernel<T_Q6_K, G>), grid, dim3(G::kThreads), G::kLdsBytes, s, a);
        else hipLaunchKernelGGL((f32_gemm_kernel<T_Q4_K, G>), grid, dim3(G::kThreads), G::kLdsBytes, s, a);
    };
    // the default tiles, unless they would leave more than half the CUs idle
    const int64_t large = static_cast<int64_t>((out_dim + GeoLarge::kBN - 1) / GeoLarge::kBN) *
                          ((m + GeoLarge::kBM - 1) / GeoLarge::kBM);
    if (QLIN_F32_GEMM_SMALL && large * 2 < device_info().cu_count) launch(GeoSmall{});
    else launch(GeoLarge{});
    return hipGetLastError();
}

}  // namespace qlin

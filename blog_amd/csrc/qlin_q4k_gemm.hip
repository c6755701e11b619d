// qlin_q4k_gemm.hip -- Q4_K weights x Q8_1 activations, the prefill GEMM, on the fp16 matrix cores
// of gfx950.
//
// Computes y[r, o] = sum over 32-blocks b of  dw*sc_b*d8_b * sum_i(qw*qx) - dmin*m_b*s8_b  (the
// reference quant_matmul_q8_1_kernel for Q4_K, AI/codes/local-llm/src/backend/cuda/ops/kernel.cu:
// 2305-2345), for m tokens of Q8_1 activations (d8 f16 | s8 f16 | int8 q[32] per 32 values).
//
// Every product is exact on v_mfma_f32_16x16x32_f16:
//   A (activations): d8*qx needs at most 18 significant bits (11 of d8, 7 of q), so it is split
//     exactly into two fp16 halves, hi = f16(d8*qx) and lo = d8*qx - hi, and both are multiplied.
//   B (weights): sc_j*qw is an integer <= 63*15 = 945, exact in fp16.  A nibble becomes fp16 1024+q
//     by one v_perm_b32 per two weights (bytes (q, 0x64)); one v_pk_fma_f16 per two weights then
//     gives (1024+q)*sc - 1024*sc = q*sc, exact because the result is representable.
// So one super-block's MFMAs sum sum_j sc_j * sum_i (d8_j qx)(qw) in f32, and d is applied once
// per super-block instead of once per 32-block.  The min term sum_j m_j*s8_j (m_j <= 63 and s8 an
// f16, both exact) is one more MFMA per tile, scaled by dmin.
//
// Tiling.  A workgroup of 8 waves computes 64 tokens x 256 weight rows; each wave owns 32 rows (two
// 16-row tiles) for all 64 tokens (four 16-token tiles).  Per super-block the workgroup converts
// its 64 x 256 activations once into the A-operand layout in LDS (hi and lo planes, 64 KB), and
// each wave decodes its own weight rows straight from global memory into B operands.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

namespace qlin {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kNT = 2;                    // 16-row weight tiles per wave
constexpr int kBN = kWaves * kNT * 16;    // weight rows per workgroup (256)
constexpr int kMT = 4;                    // 16-token tiles per workgroup
constexpr int kBM = kMT * 16;             // tokens per workgroup (64)
constexpr size_t kLds = (2 * kMT * 8 * 64 + kMT * 16) * sizeof(uint4);  // A planes + s8 operands

struct GemmArgs {
    const uint8_t *w;
    size_t rb;         // weight row bytes
    const uint8_t *xq;
    size_t xrb;        // Q8_1 row bytes
    float *y;
    int n, m, nsb;
};

__device__ __forceinline__ f32x4 mfma(const uint4 &a, const uint4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

__device__ __forceinline__ uint32_t h2u(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ f16x2 u2h(uint32_t u) { return __builtin_bit_cast(f16x2, u); }

// 6-bit (scale, min) of sub-block J from scale bytes s[0..11] held in three dwords (kernel.cu:913-921).
template <int J>
__device__ __forceinline__ void scale_min(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &sc, uint32_t &mn) {
    const uint32_t s[3] = {s0, s1, s2};
    auto byte = [&](int i) { return (s[i >> 2] >> (8 * (i & 3))) & 0xffu; };
    if constexpr (J < 4) {
        sc = byte(J) & 63u;
        mn = byte(J + 4) & 63u;
    } else {
        sc = (byte(J + 4) & 0xfu) | ((byte(J - 4) >> 6) << 4);
        mn = (byte(J + 4) >> 4) | ((byte(J) >> 6) << 4);
    }
}

// B operand of sub-block J for this lane: 8 nibbles (k = 8g .. 8g+7 of the sub-block) times sc.
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

__device__ __forceinline__ f16x2 splat(float v) {
    const _Float16 h = static_cast<_Float16>(v);
    return f16x2{h, h};
}

__global__ __launch_bounds__(kThreads) void q4k_gemm_kernel(const GemmArgs a) {
    extern __shared__ uint4 lds[];
    uint4 *aplane = lds;                          // [part][mt][j][lane]
    uint4 *s8op = lds + 2 * kMT * 8 * 64;         // [mt][token]: s8 of sub-blocks 0..7

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.y * kBM;
    const int o0 = blockIdx.x * kBN + wave * kNT * 16;

    const uint8_t *wrow[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) wrow[t] = a.w + static_cast<size_t>(min(o0 + t * 16 + n, a.n - 1)) * a.rb;

    // staging role: token tile smt, slot lane sl (token si, k-group sg), sub-blocks 4*sjh .. 4*sjh+3
    const int smt = tid >> 7, sjh = (tid >> 6) & 1, sl = tid & 63, si = sl & 15, sg = sl >> 4;
    const int tok = m0 + smt * 16 + si;
    const bool tok_ok = tok < a.m;
    const uint8_t *xrow = a.xq + static_cast<size_t>(min(tok, a.m - 1)) * a.xrb;

    f32x4 acc[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int t = 0; t < kNT; ++t) acc[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (int sb = 0; sb < a.nsb; ++sb) {
        // this wave's weights for the super-block (issued before the staging so they are in flight)
        uint4 hdr[kNT];
        uint2 qs[kNT][4];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            const uint8_t *p = wrow[t] + static_cast<size_t>(sb) * 144;
            hdr[t] = *reinterpret_cast<const uint4 *>(p);
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) qs[t][pr] = *reinterpret_cast<const uint2 *>(p + 16 + 32 * pr + 8 * g);
        }

        // activations: Q8_1 blocks -> exact fp16 hi / lo A operands in LDS
        __syncthreads();  // the previous super-block's operands are no longer read
        uint32_t s8h[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int j = 4 * sjh + jj;
            const uint8_t *blk = xrow + static_cast<size_t>(sb * 8 + j) * 36;
            const uint32_t bh = *reinterpret_cast<const uint32_t *>(blk);
            const uint32_t q0 = *reinterpret_cast<const uint32_t *>(blk + 4 + 8 * sg);
            const uint32_t q1 = *reinterpret_cast<const uint32_t *>(blk + 8 + 8 * sg);
            const float d8 = f16_bits_to_f32(bh & 0xffffu);
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t w = e < 2 ? q0 : q1;
                const int sh = 16 * (e & 1);
                const float v0 = d8 * static_cast<float>(static_cast<int8_t>((w >> sh) & 0xffu));
                const float v1 = d8 * static_cast<float>(static_cast<int8_t>((w >> (sh + 8)) & 0xffu));
                const _Float16 h0 = static_cast<_Float16>(v0), h1 = static_cast<_Float16>(v1);
                const _Float16 l0 = static_cast<_Float16>(v0 - static_cast<float>(h0));
                const _Float16 l1 = static_cast<_Float16>(v1 - static_cast<float>(h1));
                hi[e] = h2u(f16x2{h0, h1});
                lo[e] = h2u(f16x2{l0, l1});
            }
            uint4 H = make_uint4(hi[0], hi[1], hi[2], hi[3]), L = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            if (!tok_ok) H = L = make_uint4(0u, 0u, 0u, 0u);
            aplane[((0 * kMT + smt) * 8 + j) * 64 + sl] = H;
            aplane[((1 * kMT + smt) * 8 + j) * 64 + sl] = L;
            s8h[jj] = tok_ok ? bh >> 16 : 0u;
        }
        // the s8 operand row of token si: halves s8_0 .. s8_7 (written by the two threads of sg == 0)
        if (sg == 0) {
            uint2 *dst = reinterpret_cast<uint2 *>(&s8op[smt * 16 + si]) + sjh;
            *dst = make_uint2(s8h[0] | (s8h[1] << 16), s8h[2] | (s8h[3] << 16));
        }
        __syncthreads();

        // weights: per tile the super-block scales, then the 8 sub-blocks' MFMAs
        float dd[kNT], dmin[kNT];
        uint32_t s0[kNT], s1[kNT], s2[kNT];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            dd[t] = f16_bits_to_f32(hdr[t].x & 0xffffu);
            dmin[t] = f16_bits_to_f32(hdr[t].x >> 16);
            s0[t] = hdr[t].y;
            s1[t] = hdr[t].z;
            s2[t] = hdr[t].w;
        }
        f32x4 D[kMT][kNT];
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int t = 0; t < kNT; ++t) D[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        uint32_t mins[kNT][8];
        auto sub_block = [&](auto jc) {
            constexpr int J = decltype(jc)::value;
            uint4 B[kNT];
#pragma unroll
            for (int t = 0; t < kNT; ++t) {
                uint32_t sc, mn;
                scale_min<J>(s0[t], s1[t], s2[t], sc, mn);
                mins[t][J] = mn;
                const float scf = static_cast<float>(sc);
                B[t] = weights_b<J>(qs[t][J >> 1], splat(scf), splat(-1024.0f * scf));
            }
#pragma unroll
            for (int i = 0; i < kMT; ++i) {
                const uint4 ah = aplane[((0 * kMT + i) * 8 + J) * 64 + lane];
                const uint4 al = aplane[((1 * kMT + i) * 8 + J) * 64 + lane];
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    D[i][t] = mfma(ah, B[t], D[i][t]);
                    D[i][t] = mfma(al, B[t], D[i][t]);
                }
            }
        };
        sub_block(std::integral_constant<int, 0>{});
        sub_block(std::integral_constant<int, 1>{});
        sub_block(std::integral_constant<int, 2>{});
        sub_block(std::integral_constant<int, 3>{});
        sub_block(std::integral_constant<int, 4>{});
        sub_block(std::integral_constant<int, 5>{});
        sub_block(std::integral_constant<int, 6>{});
        sub_block(std::integral_constant<int, 7>{});

        // min term: sum_j s8_j * m_j on one more MFMA (k-slots 0..7 carried by lane-group 0)
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            uint4 b2 = make_uint4(0u, 0u, 0u, 0u);
            if (g == 0) {
                auto mh = [&](int j) { return h2u(f16x2{static_cast<_Float16>(static_cast<float>(mins[t][j])),
                                                        static_cast<_Float16>(static_cast<float>(mins[t][j + 1]))}); };
                b2 = make_uint4(mh(0), mh(2), mh(4), mh(6));
            }
#pragma unroll
            for (int i = 0; i < kMT; ++i) {
                const uint4 a2 = g == 0 ? s8op[i * 16 + n] : make_uint4(0u, 0u, 0u, 0u);
                const f32x4 d2 = mfma(a2, b2, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[i][t][r] = fmaf(dd[t], D[i][t][r], acc[i][t][r]);
                    acc[i][t][r] = fmaf(-dmin[t], d2[r], acc[i][t][r]);
                }
            }
        }
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
                if (tk < a.m) a.y[static_cast<size_t>(tk) * a.n + o] = acc[i][t][r];
            }
    }
}

}  // namespace

bool q4k_gemm_ok(const uint8_t *w, size_t rb, const uint8_t *xq, int in_dim) {
    return in_dim % 256 == 0 && rb % 16 == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(xq) & 3u) == 0;
}

hipError_t q4k_gemm_q8_1(const uint8_t *w, size_t rb, const uint8_t *xq, float *y, int out_dim, int in_dim, int m,
                         hipStream_t s) {
    if (out_dim == 0 || m == 0) return hipSuccess;
    GemmArgs a;
    a.w = w;
    a.rb = rb;
    a.xq = xq;
    a.xrb = static_cast<size_t>(in_dim / 32) * 36;
    a.y = y;
    a.n = out_dim;
    a.m = m;
    a.nsb = in_dim / 256;
    const dim3 grid((out_dim + kBN - 1) / kBN, (m + kBM - 1) / kBM);
    hipLaunchKernelGGL(q4k_gemm_kernel, grid, dim3(kThreads), kLds, s, a);
    return hipGetLastError();
}

}  // namespace qlin

// qlin_q4k_gemm.hip -- Q4_K weights x Q8_1 activations, the prefill GEMM, on the fp16 matrix cores
// of gfx950.
//
// Computes y[r, o] = sum over 32-blocks b of  dw*sc_b*d8_b * sum_i(qw*qx) - dmin*m_b*s8_b  (the
// reference quant_matmul_q8_1_kernel for Q4_K, AI/codes/local-llm/src/backend/cuda/ops/kernel.cu:
// 2305-2345), for m tokens of Q8_1 activations (d8 f16 | s8 f16 | int8 q[32] per 32 values).
//
// The products are exact on v_mfma_f32_16x16x32_f16 (up to the 2^-22 rounding of lo):
//   A (activations): d8*qx needs at most 18 significant bits (11 of d8, 7 of q), so it is split
//     into two fp16 halves, hi (its top 11 bits) and lo (the rest, rounded to fp16: 2^-22 of the
//     value), and both are multiplied.
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

#ifndef QLIN_GEMM_WAVES
#define QLIN_GEMM_WAVES 8
#endif
#ifndef QLIN_GEMM_NT
#define QLIN_GEMM_NT 2
#endif
constexpr int kWaves = QLIN_GEMM_WAVES;
constexpr int kThreads = kWaves * 64;
constexpr int kNT = QLIN_GEMM_NT;         // 16-row weight tiles per wave
constexpr int kBN = kWaves * kNT * 16;    // weight rows per workgroup (256)
#ifndef QLIN_GEMM_SB
#define QLIN_GEMM_SB 1
#endif
#ifndef QLIN_GEMM_MT
#define QLIN_GEMM_MT 4
#endif
constexpr int kMT = QLIN_GEMM_MT;         // 16-token tiles per workgroup
constexpr int kBM = kMT * 16;             // tokens per workgroup (64)
constexpr int kPlane = 2 * kMT * 8 * 64;  // uint4s of one buffer's A planes (hi, lo): 64 KB
constexpr int kBuf = kPlane + kMT * 64;   // plus the min-term operands [mt][lane] (lanes >= 16 stay zero)
constexpr int kSJ = kThreads / kMT / 64;  // staging waves per token tile
constexpr int kJJ = 8 / kSJ;              // sub-blocks each staging thread converts
constexpr size_t kLds = 2 * kBuf * sizeof(uint4);  // two buffers

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
    // two buffers, each: A planes [part][mt][j][lane] then s8 operands [mt][token]
    auto plane = [&](int buf) { return lds + buf * kBuf; };
    auto s8ops = [&](int buf) { return lds + buf * kBuf + kPlane; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.y * kBM;
    const int o0 = blockIdx.x * kBN + wave * kNT * 16;

    const uint8_t *wrow[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) wrow[t] = a.w + static_cast<size_t>(min(o0 + t * 16 + n, a.n - 1)) * a.rb;

    // staging role: token tile smt, slot lane sl (token si, k-group sg), sub-blocks kJJ*sjh .. +kJJ-1
    const int smt = tid / (kSJ * 64), sjh = (tid >> 6) % kSJ, sl = tid & 63, si = sl & 15, sg = sl >> 4;
    const int tok = m0 + smt * 16 + si;
    const uint8_t *xrow = a.xq + static_cast<size_t>(min(tok, a.m - 1)) * a.xrb;

    // min-term operand entries of lane-groups 1..3 stay zero (staging writes lanes 0..15 only)
    for (int i = tid; i < 2 * kMT * 64; i += kThreads)
        if ((i & 63) >= 16) s8ops(i / (kMT * 64))[i % (kMT * 64)] = make_uint4(0u, 0u, 0u, 0u);

    f32x4 acc[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int t = 0; t < kNT; ++t) acc[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Raw operands of a super-block: this wave's weight bytes and this thread's activation slots.
    struct WRaw {
        uint4 hdr[kNT];
        uint2 qs[kNT][4];
    };
    struct XRaw {
        uint32_t bh[kJJ], q0[kJJ], q1[kJJ];
    };
    // past the end a fetch reloads the last super-block (valid addresses, never used)
    auto fetch_w = [&](WRaw &w, int sb) {
        sb = min(sb, a.nsb - 1);
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            const uint8_t *p = wrow[t] + static_cast<size_t>(sb) * 144;
            w.hdr[t] = *reinterpret_cast<const uint4 *>(p);
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) w.qs[t][pr] = *reinterpret_cast<const uint2 *>(p + 16 + 32 * pr + 8 * g);
        }
    };
    auto fetch_x = [&](XRaw &x, int sb) {
        sb = min(sb, a.nsb - 1);
#pragma unroll
        for (int jj = 0; jj < kJJ; ++jj) {
            const uint8_t *blk = xrow + static_cast<size_t>(sb * 8 + kJJ * sjh + jj) * 36;
            x.bh[jj] = *reinterpret_cast<const uint32_t *>(blk);
            x.q0[jj] = *reinterpret_cast<const uint32_t *>(blk + 4 + 8 * sg);
            x.q1[jj] = *reinterpret_cast<const uint32_t *>(blk + 8 + 8 * sg);
        }
    };

    // Activations of a super-block into buffer buf: q becomes fp16 exactly (bytes (q ^ 0x80, 0x64)
    // = 1152 + q, minus 1152), hi = f16(d8*q) and lo = fma(d8, q, -hi) = the exact residual of hi
    // (d8*q has at most 18 significant bits, hi keeps 11, so the residual fits an fp16).
    auto stage = [&](const XRaw &x, int buf) {
        uint4 *pl = plane(buf);
        const f16x2 off = splat(-1152.0f);
        uint32_t s8h[kJJ];
#pragma unroll
        for (int jj = 0; jj < kJJ; ++jj) {
            const int j = kJJ * sjh + jj;
            const f16x2 d2 = u2h((x.bh[jj] & 0xffffu) * 0x10001u);
            const uint32_t u[2] = {x.q0[jj] ^ 0x80808080u, x.q1[jj] ^ 0x80808080u};
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t sel = (e & 1) ? 0x04030402u : 0x04010400u;
                const f16x2 q2 = u2h(__builtin_amdgcn_perm(0x64646464u, u[e >> 1], sel)) + off;
                const f16x2 h2 = d2 * q2;
                hi[e] = h2u(h2);
                lo[e] = h2u(__builtin_elementwise_fma(d2, q2, -h2));
            }
            // tokens past m repeat the last row: their D rows are never stored
            pl[((0 * kMT + smt) * 8 + j) * 64 + sl] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            pl[((1 * kMT + smt) * 8 + j) * 64 + sl] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            s8h[jj] = x.bh[jj] >> 16;
        }
        // the s8 operand row of token si: halves s8_0 .. s8_7 (written by the threads of sg == 0)
        if (sg == 0) {
            uint16_t *dst = reinterpret_cast<uint16_t *>(&s8ops(buf)[smt * 64 + si]) + kJJ * sjh;
#pragma unroll
            for (int jj = 0; jj < kJJ; ++jj) dst[jj] = static_cast<uint16_t>(s8h[jj]);
        }
    };

    // One super-block: per 16-row tile the scales, then the 8 sub-blocks' MFMAs, then the min term.
    auto compute = [&](const WRaw &w, int buf) {
        const uint4 *pl = plane(buf);
        float dd[kNT], dmin[kNT];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            dd[t] = f16_bits_to_f32(w.hdr[t].x & 0xffffu);
            dmin[t] = f16_bits_to_f32(w.hdr[t].x >> 16);
        }
        f32x4 D[kMT][kNT];
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int t = 0; t < kNT; ++t) D[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // All 8 scales of a tile at once (kernel.cu:913-921 on whole dwords): bytes j of sl are sub-block
        // j < 4, of sh sub-block 4 + j; as fp16 pairs (sc_2i, sc_2i+1) via the bytes (v, 0x64) = 1024 + v.
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
        auto sub_block = [&](auto jc) {
            constexpr int J = decltype(jc)::value;
            uint4 B[kNT];
#pragma unroll
            for (int t = 0; t < kNT; ++t) {
                const f16x2 sc2 = __builtin_shufflevector(scp[t][J >> 1], scp[t][J >> 1], J & 1, J & 1);
                const f16x2 c2 = __builtin_shufflevector(cp[t][J >> 1], cp[t][J >> 1], J & 1, J & 1);
                B[t] = weights_b<J>(w.qs[t][J >> 1], sc2, c2);
            }
            // hi for every (token tile, row tile), then lo: consecutive MFMAs never feed each other
#pragma unroll
            for (int part = 0; part < 2; ++part)
#pragma unroll
                for (int i = 0; i < kMT; ++i) {
                    const uint4 av = pl[((part * kMT + i) * 8 + J) * 64 + lane];
#pragma unroll
                    for (int t = 0; t < kNT; ++t) D[i][t] = mfma(av, B[t], D[i][t]);
                }
            // no hoisting of the next sub-block's LDS reads above these MFMAs: the registers they
            // would hold push the kernel past its 256 VGPRs (measured 3% faster)
#if QLIN_GEMM_SB
            __builtin_amdgcn_sched_barrier(0);
#endif
        };
        sub_block(std::integral_constant<int, 0>{});
        sub_block(std::integral_constant<int, 1>{});
        sub_block(std::integral_constant<int, 2>{});
        sub_block(std::integral_constant<int, 3>{});
        sub_block(std::integral_constant<int, 4>{});
        sub_block(std::integral_constant<int, 5>{});
        sub_block(std::integral_constant<int, 6>{});
        sub_block(std::integral_constant<int, 7>{});

        // min term: sum_j s8_j * m_j on one more MFMA.  Only k-slots 0..7 (lane-group 0) carry s8; the
        // other lanes' A entries are zeros in LDS, so their B entries (finite mins) add nothing.
        const uint4 *s8 = s8ops(buf);
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            // the 8 mins of the tile, as the scales above (bytes j of ml: sub-block j < 4; of mh: 4 + j)
            const uint32_t s1 = w.hdr[t].z, s2 = w.hdr[t].w;
            f16x2 mp[4];
            pairs(s1 & 0x3f3f3f3fu, mp);
            pairs(((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u), mp + 2);
            const uint4 b2 = make_uint4(h2u(mp[0]), h2u(mp[1]), h2u(mp[2]), h2u(mp[3]));
#pragma unroll
            for (int i = 0; i < kMT; ++i) {
                const uint4 a2 = s8[i * 64 + lane];
                const f32x4 d2 = mfma(a2, b2, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[i][t][r] = fmaf(dd[t], D[i][t][r], acc[i][t][r]);
                    acc[i][t][r] = fmaf(-dmin[t], d2[r], acc[i][t][r]);
                }
            }
        }
    };

    // Pipeline: the operands of super-block sb + 2 are requested while sb is computed and sb + 1 is
    // staged into the other LDS buffer; one barrier per super-block.  Two register sets in turn (a
    // single set copied forward would make the copy wait for the loads just issued).
    WRaw w0, w1;
    XRaw x0, x1;
    fetch_w(w0, 0);
    fetch_x(x0, 0);
    fetch_w(w1, 1);
    fetch_x(x1, 1);
    stage(x0, 0);
    __syncthreads();
    // At the top of an iteration: buffer 0 holds sb's activations, w0 = sb's weights, w1 / x1 =
    // sb + 1's raw operands (buffer 1 was last read before the previous barrier).
    const int pairs = a.nsb >> 1;  // branch-free body, so the compiler waits for exactly what is used
    for (int pi = 0; pi < pairs; ++pi) {
        const int sb = 2 * pi;
        fetch_x(x0, sb + 2);
        compute(w0, 0);
        stage(x1, 1);
        fetch_w(w0, sb + 2);
        __syncthreads();
        fetch_x(x1, sb + 3);
        compute(w1, 1);
        stage(x0, 0);
        fetch_w(w1, sb + 3);
        __syncthreads();
    }
    if (a.nsb & 1) compute(w0, 0);  // odd count: the last super-block is staged in buffer 0

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

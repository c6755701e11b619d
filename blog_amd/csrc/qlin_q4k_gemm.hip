// qlin_q4k_gemm.hip -- Q4_K weights x Q8_1 activations, the prefill GEMM, on the fp16 matrix cores
// of gfx950.
//
// Computes y[r, o] = sum over 32-blocks b of  dw*sc_b*d8_b * sum_i(qw*qx) - dmin*m_b*s8_b  (the
// reference quant_matmul_q8_1_kernel for Q4_K, AI/codes/local-llm/src/backend/cuda/ops/kernel.cu:
// 2305-2345), for m tokens of Q8_1 activations (d8 f16 | s8 f16 | int8 q[32] per 32 values).
//
// The block dot is taken as the reference takes it, in integers, on v_mfma_f32_16x16x32_f16:
//   A (activations): qx, an integer of at most 8 bits, exact in fp16 (bytes (q ^ 0x80, 0x64) are the
//     fp16 1152 + q; one packed subtraction leaves q).
//   B (weights): sc_j*qw is an integer <= 63*15 = 945, exact in fp16.  A nibble becomes fp16 1024+q
//     by one v_perm_b32 per two weights (bytes (q, 0x64)); one v_pk_fma_f16 per two weights then
//     gives (1024+q)*sc - 1024*sc = q*sc, exact because the result is representable.
// One MFMA per 32-block and 16 x 16 tile gives sum_i sc_j*qw*qx exactly in f32 (|sum| < 2^22); d8_j
// is applied to it by one fma per output element, and d once per super-block.  The min term
// sum_j m_j*s8_j (m_j <= 63 and s8 an f16, both exact) is one more MFMA per tile, scaled by dmin.
//
// Two other forms measured slower.  Splitting d8*qx into fp16 hi and lo parts moves d8 into the A
// operand (no per-block fma) but doubles the MFMAs, and its operands, full fp16 mantissas, draw
// the matrix cores' power limit (150 us against 144 us here on the C4 shape).  The int8 MFMA on the
// raw bytes and nibbles needs sc and d8 applied to each int32 block result, three VALU per element
// and block (162 us).
//
// Tiling.  A workgroup of 8 waves computes 64 tokens x 256 weight rows; each wave owns 32 rows (two
// 16-row tiles) for all 64 tokens (four 16-token tiles).  Per super-block the workgroup stages its
// 64 x 256 activations once into the A-operand layout in LDS, and each wave decodes its own weight
// rows straight from global memory into B operands.  The weights live in one register set whose
// parts are reloaded with the next super-block as soon as they are decoded, and the A fragments of
// sub-block J + 2 are read while J is multiplied.
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
// One LDS buffer (uint4 units): the qx plane [mt][j][lane] (fp16 integers), then the min-term
// operands [mt][lane] (lanes >= 16 stay zero), then the block scales d8 [mt][j][token] as floats.
// Two buffers: 76 KB.
constexpr int kPlane = kMT * 8 * 64;
constexpr int kS8 = kMT * 64;
constexpr int kD8 = kMT * 8 * 16 / 4;
constexpr int kBuf = kPlane + kS8 + kD8;
constexpr size_t kLdsBytes = 2 * kBuf * sizeof(uint4);
constexpr int kSJ = kThreads / kMT / 64;  // staging waves per token tile
constexpr int kJJ = 8 / kSJ;              // sub-blocks each staging thread converts

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

template <int V> using ic = std::integral_constant<int, V>;

__global__ __launch_bounds__(kThreads) void q4k_gemm_kernel(const GemmArgs a) {
    extern __shared__ uint4 lds[];
    auto plane = [&](int buf) { return lds + buf * kBuf; };
    auto s8ops = [&](int buf) { return lds + buf * kBuf + kPlane; };
    auto d8s = [&](int buf) { return reinterpret_cast<float *>(lds + buf * kBuf + kPlane + kS8); };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    int bx, by;
    gemm_tile((a.n + kBN - 1) / kBN, (a.m + kBM - 1) / kBM, bx, by);
    const int m0 = by * kBM;
    const int o0 = bx * kBN + wave * kNT * 16;

    const uint8_t *wrow[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) wrow[t] = a.w + static_cast<size_t>(min(o0 + t * 16 + n, a.n - 1)) * a.rb;

    // staging role: token tile smt, slot lane sl (token si, k-group sg), sub-blocks kJJ*sjh .. +kJJ-1
    const int smt = tid / (kSJ * 64), sjh = (tid >> 6) % kSJ, sl = tid & 63, si = sl & 15, sg = sl >> 4;
    const int tok = m0 + smt * 16 + si;
    const uint8_t *xrow = a.xq + static_cast<size_t>(min(tok, a.m - 1)) * a.xrb;

    // min-term operand entries of lane-groups 1..3 stay zero (staging writes lanes 0..15 only)
    for (int i = tid; i < 2 * kS8; i += kThreads)
        if ((i & 63) >= 16) s8ops(i / kS8)[i % kS8] = make_uint4(0u, 0u, 0u, 0u);

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
    auto fetch_hdr = [&](WRaw &w, int sb) {
        sb = min(sb, a.nsb - 1);
#pragma unroll
        for (int t = 0; t < kNT; ++t) w.hdr[t] = *reinterpret_cast<const uint4 *>(wrow[t] + static_cast<size_t>(sb) * 144);
    };
    auto fetch_qs = [&](WRaw &w, int sb, int pr) {
        sb = min(sb, a.nsb - 1);
#pragma unroll
        for (int t = 0; t < kNT; ++t)
            w.qs[t][pr] = *reinterpret_cast<const uint2 *>(wrow[t] + static_cast<size_t>(sb) * 144 + 16 + 32 * pr + 8 * g);
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

    // Activations of a super-block into buffer buf: qx as fp16 integers, d8 as a float per (token
    // tile, block, token), s8 into the min-term operand row.  Tokens past m repeat the last row:
    // their D rows are never stored.
    auto stage = [&](const XRaw &x, int buf) {
        uint4 *pl = plane(buf);
        const f16x2 off = splat(-1152.0f);
#pragma unroll
        for (int jj = 0; jj < kJJ; ++jj) {
            const int j = kJJ * sjh + jj;
            const uint32_t u[2] = {x.q0[jj] ^ 0x80808080u, x.q1[jj] ^ 0x80808080u};
            uint32_t qh[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t sel = (e & 1) ? 0x04030402u : 0x04010400u;
                qh[e] = h2u(u2h(__builtin_amdgcn_perm(0x64646464u, u[e >> 1], sel)) + off);
            }
            pl[(smt * 8 + j) * 64 + sl] = make_uint4(qh[0], qh[1], qh[2], qh[3]);
            if (sg == 0) d8s(buf)[(smt * 8 + j) * 16 + si] = f16_bits_to_f32(x.bh[jj] & 0xffffu);
        }
        // the s8 operand row of token si: halves s8_0 .. s8_7 (written by the threads of sg == 0)
        if (sg == 0) {
            uint16_t *dst = reinterpret_cast<uint16_t *>(&s8ops(buf)[smt * 64 + si]) + kJJ * sjh;
#pragma unroll
            for (int jj = 0; jj < kJJ; ++jj) dst[jj] = static_cast<uint16_t>(x.bh[jj] >> 16);
        }
    };

    // One super-block: per 16-row tile the scales, then the 8 sub-blocks' MFMAs, then the min term.
    // Each part of w is reloaded with super-block `next` as soon as it has been used, so one register
    // set carries the weights (the loads have the rest of the super-block to land).
    auto compute = [&](WRaw &w, int buf, int next) {
        const uint4 *pl = plane(buf);
        const float *d8 = d8s(buf);
        float dd[kNT], dmin[kNT];
        uint32_t mlo[kNT], mhi[kNT];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            dd[t] = f16_bits_to_f32(w.hdr[t].x & 0xffffu);
            dmin[t] = f16_bits_to_f32(w.hdr[t].x >> 16);
            mlo[t] = w.hdr[t].z;
            mhi[t] = w.hdr[t].w;
        }
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
        fetch_hdr(w, next);
        // T = sum_j d8_j * (sc_j qw . qx)_j per output over the super-block; d applied after it
        f32x4 T[kMT][kNT];
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int t = 0; t < kNT; ++t) T[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        // A fragments of a sub-block: qx of every token tile, and d8 of the lane's 4 tokens
        struct Frag {
            uint4 a[kMT];
            float4 d8[kMT];
        };
        auto load_frag = [&](Frag &f, int J) {
#pragma unroll
            for (int i = 0; i < kMT; ++i) {
                f.a[i] = pl[(i * 8 + J) * 64 + lane];
                f.d8[i] = *reinterpret_cast<const float4 *>(d8 + (i * 8 + J) * 16 + 4 * g);
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
            for (int i = 0; i < kMT; ++i) {
                f32x4 Dj[kNT];
#pragma unroll
                for (int t = 0; t < kNT; ++t) Dj[t] = mfma(f.a[i], B[t], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                const float d8r[4] = {f.d8[i].x, f.d8[i].y, f.d8[i].z, f.d8[i].w};
#pragma unroll
                for (int t = 0; t < kNT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) T[i][t][r] = fmaf(Dj[t][r], d8r[r], T[i][t][r]);
            }
            // The block's scaling is pure arithmetic, which instruction selection would otherwise
            // sink below every later sub-block, keeping all of a super-block's MFMA results live
            // (hundreds of VGPRs spilled); consuming the sums here pins it before the next MFMAs.
            static_assert(kMT * kNT == 8, "one operand per sum");
            asm volatile("" ::"v"(T[0][0]), "v"(T[0][1]), "v"(T[1][0]), "v"(T[1][1]), "v"(T[2][0]), "v"(T[2][1]),
                         "v"(T[3][0]), "v"(T[3][1]));
            // the order as written: the next fragments' LDS reads (issued before this call) overlap
            // these MFMAs, and nothing is hoisted above them to hold more registers
            __builtin_amdgcn_sched_barrier(0);
        };
        // software pipeline over the sub-blocks: fragments of J + 1 are read while J is multiplied
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

        // min term: sum_j s8_j * m_j on one more MFMA.  Only k-slots 0..7 (lane-group 0) carry s8; the
        // other lanes' A entries are zeros in LDS, so their B entries (finite mins) add nothing.
        const uint4 *s8 = s8ops(buf);
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            // the 8 mins of the tile, as the scales above (bytes j of ml: sub-block j < 4; of mh: 4 + j)
            f16x2 mp[4];
            pairs(mlo[t] & 0x3f3f3f3fu, mp);
            pairs(((mhi[t] >> 4) & 0x0f0f0f0fu) | ((mlo[t] >> 2) & 0x30303030u), mp + 2);
            const uint4 b2 = make_uint4(h2u(mp[0]), h2u(mp[1]), h2u(mp[2]), h2u(mp[3]));
#pragma unroll
            for (int i = 0; i < kMT; ++i) {
                const f32x4 d2 = mfma(s8[i * 64 + lane], b2, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[i][t][r] = fmaf(dd[t], T[i][t][r], acc[i][t][r]);
                    acc[i][t][r] = fmaf(-dmin[t], d2[r], acc[i][t][r]);
                }
            }
        }
    };

    // Pipeline over super-blocks: sb is computed from buffer sb & 1 while its weights are replaced by
    // sb + 1's part by part; then sb + 1's activations (loaded during sb) are staged into the other
    // buffer, whose last reads were before the previous barrier, and sb + 2's requested.
    WRaw w;
    XRaw x;
    fetch_hdr(w, 0);
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) fetch_qs(w, 0, pr);
    fetch_x(x, 0);
    stage(x, 0);
    fetch_x(x, 1);
    __syncthreads();
    for (int sb = 0; sb < a.nsb; ++sb) {
        const int buf = sb & 1;
        compute(w, buf, sb + 1);
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
    const dim3 grid = gemm_grid((out_dim + kBN - 1) / kBN, (m + kBM - 1) / kBM);
    hipLaunchKernelGGL(q4k_gemm_kernel, grid, dim3(kThreads), kLdsBytes, s, a);
    return hipGetLastError();
}

}  // namespace qlin

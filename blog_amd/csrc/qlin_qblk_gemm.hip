// qlin_qblk_gemm.hip -- Q8_0, Q5_0, Q4_0 and Q6_K weights x Q8_1 activations, the prefill GEMM, on
// the fp16 matrix cores of gfx950 (Q6_K: see q6k_gemm_kernel below).
//
// Computes y[r, o] = sum over 32-blocks b of  dw_b * d8_b * sum_i (qw_i - c) qx_i  (the reference
// quant_matmul_q8_1_kernel for these formats, AI/codes/local-llm/src/backend/cuda/ops/kernel.cu:
// 2305-2402: the dequantized weight dw * (q - c) times dx * qx, summed over the block), c = 0 (Q8_0),
// 16 (Q5_0), 8 (Q4_0), for m tokens of Q8_1 activations (d8 f16 | s8 f16 | int8 q[32] per 32 values).
//
// The block dot runs on integers, on v_mfma_f32_16x16x32_f16:
//   A (activations): qx, exact in fp16 (bytes (q ^ 0x80, 0x64) are the fp16 1152 + q).
//   B (weights): q - c, exact in fp16: the bytes (q, 0x64) are 1024 + q for a nibble or 5-bit value,
//     (q ^ 0x80, 0x64) 1152 + q for an int8; one packed subtraction leaves q - c.
// One MFMA per 32-block and 16 x 16 tile gives the integer dot exactly in f32 (|dot| < 2^17); the
// block's two scales are applied by a multiply and an fma per output element.
//
// Tiling and pipeline as in qlin_q4k_gemm.hip: a workgroup of 8 waves computes 64 tokens x 256 weight
// rows, each wave 32 rows (two 16-row tiles) for all 64 tokens; per unit of 8 blocks (256 values of
// K) the workgroup stages its activations once into the A-operand layout in LDS (two buffers, one
// barrier per unit) and each wave decodes its own weight rows from global memory.  K need only be a
// multiple of 64: the last unit may hold fewer than 8 blocks (its missing A entries are zeros and
// its missing blocks are skipped).
//
// Alignment.  The blocks (34, 22, 18 bytes) are 2-byte aligned: with 4-byte aligned rows of an even
// number of blocks, block b starts at a multiple of 4 when b is even and 2 past one when b is odd, so
// every read is a dword from the aligned address at or 2 before the block, realigned by
// v_alignbyte_b32.  An even block's reads end at most 2 bytes into the next block (which exists: the
// last block of a row is odd); an odd block's start at most 2 bytes before it.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

#include <type_traits>

namespace qlin {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#ifndef QLIN_QBLK_SMALL
#define QLIN_QBLK_SMALL 1  // the 4-wave, 32-token geometry for launches that would leave half the CUs idle
#endif
constexpr int kNT = 2;  // 16-row weight tiles per wave
// A workgroup's geometry: W waves of 32 rows each, MT 16-token tiles.  The default (8 waves, 64 tokens:
// 256 rows) covers large grids; a launch that would leave more than half the CUs idle takes 4 waves and
// 32 tokens (128 rows), four times as many workgroups for the same work per output.
template <int W, int MT>
struct Geo {
    static constexpr int kWaves = W, kThreads = W * 64;
    static constexpr int kBN = W * kNT * 16;  // weight rows per workgroup
    static constexpr int kMT = MT, kBM = MT * 16;  // 16-token tiles and tokens per workgroup
    // One LDS buffer (uint4 units): the qx plane [mt][j][lane] (fp16 integers), then the block scales
    // d8 [mt][j][token] as floats.  Two buffers (68 KB for the default).
    static constexpr int kPlane = MT * 8 * 64;
    static constexpr int kD8 = MT * 8 * 16 / 4;
    static constexpr int kBuf = kPlane + kD8;
    static constexpr size_t kLdsBytes = 2 * kBuf * sizeof(uint4);
    // Q6_K: then each wave's output sums (MT x kNT tiles of 4 floats per lane), 64 KB for the default
    static constexpr size_t kLdsBytesQ6 = kLdsBytes + static_cast<size_t>(W) * MT * kNT * 64 * sizeof(uint4);
    static constexpr int kSJ = kThreads / MT / 64;  // staging waves per token tile
    static constexpr int kJJ = 8 / kSJ;             // blocks each staging thread converts
    static_assert(kSJ >= 1 && 8 % kSJ == 0, "whole waves stage whole token tiles");
};
using GeoLarge = Geo<8, 4>;
using GeoSmall = Geo<4, 2>;

template <int FMT> struct QBlk;
template <> struct QBlk<T_Q8_0> {
    static constexpr int bytes = 34;
    [[maybe_unused]] static constexpr int offset = 0;  // (the int8 path subtracts 1152 instead)
};
template <> struct QBlk<T_Q5_0> {
    static constexpr int bytes = 22, offset = 16;
};
template <> struct QBlk<T_Q4_0> {
    static constexpr int bytes = 18, offset = 8;
};

struct GemmArgs {
    const uint8_t *w;
    size_t rb;         // weight row bytes
    const uint8_t *xq;
    size_t xrb;        // Q8_1 row bytes
    float *y;
    int n, m, nblk;    // rows, tokens, 32-blocks per row (even)
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
// bytes 2 .. 5 of the 8 bytes (lo, hi)
__device__ __forceinline__ uint32_t align2(uint32_t hi, uint32_t lo) { return __builtin_amdgcn_alignbyte(hi, lo, 2); }
// bits 0..3 of b to bit 4 of bytes 0..3
__device__ __forceinline__ uint32_t bit4_of_bytes(uint32_t b) {
    return (__umul24(b & 0xfu, 0x204081u) & 0x01010101u) << 4;
}

// The bytes of one block a lane needs (see the alignment note above): d (f16, low half), the 8
// quant bytes of its k-slots (Q8_0: bytes 8g .. 8g+7 of qs; Q5_0 / Q4_0: bytes 8(g&1) .. +7 of qs,
// whose low nibbles (g < 2) or high nibbles (g >= 2) are elements 8g .. 8g+7), and Q5_0's qh.
struct BRaw {
    uint32_t d, q0, q1, qh;
};
template <int FMT, int ODD>
__device__ __forceinline__ BRaw load_block(const uint8_t *blk, int g) {
    const uint32_t *a = reinterpret_cast<const uint32_t *>(blk - 2 * ODD);
    const int h = g & 1;
    BRaw r;
    r.qh = 0;
    if constexpr (FMT == T_Q8_0) {
        if constexpr (ODD) {
            r.d = a[0] >> 16;
            r.q0 = a[1 + 2 * g];
            r.q1 = a[2 + 2 * g];
        } else {
            r.d = a[0];
            const uint32_t w0 = a[2 * g], w1 = a[2 * g + 1], w2 = a[2 * g + 2];
            r.q0 = align2(w1, w0);
            r.q1 = align2(w2, w1);
        }
    } else if constexpr (FMT == T_Q4_0) {
        if constexpr (ODD) {
            r.d = a[0] >> 16;
            r.q0 = a[1 + 2 * h];
            r.q1 = a[2 + 2 * h];
        } else {
            r.d = a[0];
            const uint32_t w0 = a[2 * h], w1 = a[2 * h + 1], w2 = a[2 * h + 2];
            r.q0 = align2(w1, w0);
            r.q1 = align2(w2, w1);
        }
    } else {  // Q5_0: d | qh | qs
        if constexpr (ODD) {
            r.d = a[0] >> 16;
            r.qh = a[1];
            r.q0 = a[2 + 2 * h];
            r.q1 = a[3 + 2 * h];
        } else {
            const uint32_t w0 = a[0], w1 = a[1];
            r.d = w0;
            r.qh = align2(w1, w0);
            // qs bytes 8h .. 8h+7 are block bytes 6 + 8h .. 13 + 8h
            const uint32_t w2 = a[2 + 2 * h], w3 = a[3 + 2 * h];
            r.q0 = align2(w2, a[1 + 2 * h]);
            r.q1 = align2(w3, w2);
        }
    }
    return r;
}

// B operand of one block for this lane: q - c at k-slots 8g .. 8g+7 as fp16 integers.
template <int FMT>
__device__ __forceinline__ uint4 weights_b(const BRaw &r, int g) {
    uint32_t u0, u1;
    f16x2 off;
    if constexpr (FMT == T_Q8_0) {
        u0 = r.q0 ^ 0x80808080u;  // (q ^ 0x80, 0x64) = 1152 + q
        u1 = r.q1 ^ 0x80808080u;
        off = splat(-1152.0f);
    } else {
        const int sh = 4 * (g >> 1);
        u0 = (r.q0 >> sh) & 0x0f0f0f0fu;
        u1 = (r.q1 >> sh) & 0x0f0f0f0fu;
        if constexpr (FMT == T_Q5_0) {
            // the fifth bits of elements 8g .. 8g+7: bits 8g .. 8g+7 of qh (g < 2 low nibbles of
            // elements 0..15, g >= 2 high nibbles of elements 16..31: bit e for element e either way)
            const uint32_t hb = r.qh >> (8 * g);
            u0 |= bit4_of_bytes(hb);
            u1 |= bit4_of_bytes(hb >> 4);
        }
        off = splat(-(1024.0f + QBlk<FMT>::offset));  // (q, 0x64) = 1024 + q
    }
    const uint32_t k64 = 0x64646464u;
    uint4 b;
    b.x = h2u(u2h(__builtin_amdgcn_perm(k64, u0, 0x04010400u)) + off);
    b.y = h2u(u2h(__builtin_amdgcn_perm(k64, u0, 0x04030402u)) + off);
    b.z = h2u(u2h(__builtin_amdgcn_perm(k64, u1, 0x04010400u)) + off);
    b.w = h2u(u2h(__builtin_amdgcn_perm(k64, u1, 0x04030402u)) + off);
    return b;
}

template <int V> using ic = std::integral_constant<int, V>;

// The Q8_1 activations of a workgroup's 64 tokens, staged per unit of 8 blocks into two LDS buffers:
// qx as fp16 integers in the A-operand layout and d8 as a float per (token tile, block, token);
// blocks past the row are zeros.  Thread roles: token tile smt, slot lane sl (token si, k-group sg),
// blocks kJJ*sjh .. +kJJ-1 of the unit.  Tokens past m repeat the last row (their D rows are never
// stored).
template <class G>
struct ActStage {
    static constexpr int kSJ = G::kSJ, kJJ = G::kJJ, kBuf = G::kBuf, kPlane = G::kPlane;
    uint4 *lds;
    const uint8_t *xrow;
    int smt, sjh, sl, si, sg, nblk, nunit;
    struct Raw {
        uint32_t bh[kJJ], q0[kJJ], q1[kJJ];
    };
    __device__ ActStage(uint4 *l, const GemmArgs &a, int tid, int m0)
        : lds(l), smt(tid / (kSJ * 64)), sjh((tid >> 6) % kSJ), sl(tid & 63), si(tid & 15), sg((tid & 63) >> 4),
          nblk(a.nblk), nunit((a.nblk + 7) / 8) {
        const int tok = m0 + smt * 16 + si;
        xrow = a.xq + static_cast<size_t>(min(tok, a.m - 1)) * a.xrb;
    }
    __device__ uint4 *plane(int buf) const { return lds + buf * kBuf; }
    __device__ float *d8s(int buf) const { return reinterpret_cast<float *>(lds + buf * kBuf + kPlane); }
    __device__ void fetch(Raw &x, int u) const {
        u = min(u, nunit - 1);
#pragma unroll
        for (int jj = 0; jj < kJJ; ++jj) {
            const int b = min(u * 8 + kJJ * sjh + jj, nblk - 1);
            const uint8_t *blk = xrow + static_cast<size_t>(b) * 36;
            x.bh[jj] = *reinterpret_cast<const uint32_t *>(blk);
            x.q0[jj] = *reinterpret_cast<const uint32_t *>(blk + 4 + 8 * sg);
            x.q1[jj] = *reinterpret_cast<const uint32_t *>(blk + 8 + 8 * sg);
        }
    }
    __device__ void stage(const Raw &x, int buf, int u) const {
        uint4 *pl = plane(buf);
        const f16x2 off = splat(-1152.0f);
#pragma unroll
        for (int jj = 0; jj < kJJ; ++jj) {
            const int j = kJJ * sjh + jj;
            const bool live = u * 8 + j < nblk;
            const uint32_t v[2] = {x.q0[jj] ^ 0x80808080u, x.q1[jj] ^ 0x80808080u};
            uint32_t q[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t sel = (e & 1) ? 0x04030402u : 0x04010400u;
                q[e] = live ? h2u(u2h(__builtin_amdgcn_perm(0x64646464u, v[e >> 1], sel)) + off) : 0u;
            }
            pl[(smt * 8 + j) * 64 + sl] = make_uint4(q[0], q[1], q[2], q[3]);
            if (sg == 0) d8s(buf)[(smt * 8 + j) * 16 + si] = live ? f16_bits_to_f32(x.bh[jj] & 0xffffu) : 0.0f;
        }
    }
};

// A fragments of block J: qx of every token tile, and d8 of the lane's 4 tokens
template <int MT>
struct Frag {
    uint4 a[MT];
    float4 d8[MT];
};
template <class G>
__device__ __forceinline__ void load_frag(Frag<G::kMT> &f, const ActStage<G> &st, int buf, int J, int lane) {
    const uint4 *pl = st.plane(buf);
    const float *d8 = st.d8s(buf);
#pragma unroll
    for (int i = 0; i < G::kMT; ++i) {
        f.a[i] = pl[(i * 8 + J) * 64 + lane];
        f.d8[i] = *reinterpret_cast<const float4 *>(d8 + (i * 8 + J) * 16 + 4 * (lane >> 4));
    }
}

// The block's scaling is pure arithmetic, which instruction selection would otherwise sink below
// every later block, keeping all of a unit's MFMA results live (spills); consuming the sums pins it
// before the next block's MFMAs.
template <int MT>
__device__ __forceinline__ void pin(f32x4 (&T)[MT][kNT]) {
    if constexpr (MT == 4) {
        asm volatile("" ::"v"(T[0][0]), "v"(T[0][1]), "v"(T[1][0]), "v"(T[1][1]), "v"(T[2][0]), "v"(T[2][1]),
                     "v"(T[3][0]), "v"(T[3][1]));
    } else {
        static_assert(MT == 2, "the geometries' token tiles");
        asm volatile("" ::"v"(T[0][0]), "v"(T[0][1]), "v"(T[1][0]), "v"(T[1][1]));
    }
}

// lane (g, n) holds tokens 4g .. 4g+3 of each 16-token tile, weight row n of each 16-row tile
template <int kMT>
__device__ __forceinline__ void store_tile(const GemmArgs &a, const f32x4 (&acc)[kMT][kNT], int o0, int m0, int n,
                                           int g) {
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

template <int FMT, class G>
__global__ __launch_bounds__(G::kThreads) void qblk_gemm_kernel(const GemmArgs a) {
    constexpr int kMT = G::kMT, kBN = G::kBN, kBM = G::kBM;
    using ActStage = qlin::ActStage<G>;
    using Frag = qlin::Frag<kMT>;
    constexpr int BB = QBlk<FMT>::bytes;
    extern __shared__ uint4 lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    int bx, by;
    gemm_tile((a.n + kBN - 1) / kBN, (a.m + kBM - 1) / kBM, bx, by);
    const int m0 = by * kBM;
    const int o0 = bx * kBN + wave * kNT * 16;
    const ActStage st(lds, a, tid, m0);
    const int nblk = a.nblk, nunit = st.nunit;

    const uint8_t *wrow[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) wrow[t] = a.w + static_cast<size_t>(min(o0 + t * 16 + n, a.n - 1)) * a.rb;

    f32x4 T[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int t = 0; t < kNT; ++t) T[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // this wave's weight bytes of one unit: block j of tile t
    struct WRaw {
        BRaw b[8][kNT];
    };
    // block J of unit u (past the end: the last block of the same parity, valid and never used)
    auto fetch_blk = [&](auto jc, WRaw &w, int u) {
        constexpr int J = decltype(jc)::value;
        const int b = min(8 * u + J, nblk - 2 + (J & 1));
#pragma unroll
        for (int t = 0; t < kNT; ++t) w.b[J][t] = load_block<FMT, J & 1>(wrow[t] + static_cast<size_t>(b) * BB, g);
    };

    // One unit from buffer buf: the blocks' MFMAs and scaling; each block's weights are reloaded
    // with unit u + 1 right after they are decoded.
    auto compute = [&](WRaw &w, int buf, int u) {
        auto block = [&](auto jc, const Frag &f) {
            constexpr int J = decltype(jc)::value;
            if (u * 8 + J < nblk) {  // uniform
                uint4 B[kNT];
                float dw[kNT];
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    B[t] = weights_b<FMT>(w.b[J][t], g);
                    dw[t] = f16_bits_to_f32(w.b[J][t].d & 0xffffu);
                }
#pragma unroll
                for (int i = 0; i < kMT; ++i) {
                    const float d8r[4] = {f.d8[i].x, f.d8[i].y, f.d8[i].z, f.d8[i].w};
#pragma unroll
                    for (int t = 0; t < kNT; ++t) {
                        const f32x4 Dj = mfma(f.a[i], B[t], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                        for (int r = 0; r < 4; ++r) T[i][t][r] = fmaf(Dj[r] * dw[t], d8r[r], T[i][t][r]);
                    }
                }
                pin(T);
            }
            fetch_blk(jc, w, u + 1);
            __builtin_amdgcn_sched_barrier(0);
        };
        // fragments of block J + 1 are read while J is multiplied
        Frag f0, f1;
        load_frag(f0, st, buf, 0, lane);
        load_frag(f1, st, buf, 1, lane);
        block(ic<0>{}, f0);
        load_frag(f0, st, buf, 2, lane);
        block(ic<1>{}, f1);
        load_frag(f1, st, buf, 3, lane);
        block(ic<2>{}, f0);
        load_frag(f0, st, buf, 4, lane);
        block(ic<3>{}, f1);
        load_frag(f1, st, buf, 5, lane);
        block(ic<4>{}, f0);
        load_frag(f0, st, buf, 6, lane);
        block(ic<5>{}, f1);
        load_frag(f1, st, buf, 7, lane);
        block(ic<6>{}, f0);
        block(ic<7>{}, f1);
    };

    // Pipeline over units: u is computed from buffer u & 1 while its weights are replaced by u + 1's
    // block by block; then u + 1's activations (loaded during u) are staged into the other buffer,
    // whose last reads were before the previous barrier, and u + 2's requested.
    WRaw w;
    typename ActStage::Raw x;
    fetch_blk(ic<0>{}, w, 0);
    fetch_blk(ic<1>{}, w, 0);
    fetch_blk(ic<2>{}, w, 0);
    fetch_blk(ic<3>{}, w, 0);
    fetch_blk(ic<4>{}, w, 0);
    fetch_blk(ic<5>{}, w, 0);
    fetch_blk(ic<6>{}, w, 0);
    fetch_blk(ic<7>{}, w, 0);
    st.fetch(x, 0);
    st.stage(x, 0, 0);
    st.fetch(x, 1);
    __syncthreads();
    for (int u = 0; u < nunit; ++u) {
        const int buf = u & 1;
        compute(w, buf, u);
        st.stage(x, buf ^ 1, u + 1);  // past the end: zeros and copies, never read
        st.fetch(x, u + 2);
        __syncthreads();
    }
    store_tile(a, T, o0, m0, n, g);
}

// Q6_K (210-byte super-blocks: ql[128], qh[64], int8 scales[16], d f16): element l of 32-block j =
// 4 h + g6 (h = j / 4, g6 = j % 4) is q = (nibble g6 / 2 of ql[64 h + 32 (g6 % 2) + l]) | (bits
// 2 g6 .. 2 g6 + 1 of qh[32 h + l]) << 4, value d * sc[8 h + 2 g6 + l / 16] * (q - 32)
// (kernel.cu:1122-1156); the block dot with Q8_1 is dw * dx * (sc0 dot(first 16) + sc1 dot(last 16))
// (kernel.cu:2305-2402).  Lane group g holds elements 8g .. 8g+7 of a block, all under scale
// 2 g6 + g / 2, so B = sc * (q - 32) carries the two scales of the block; |sc (q - 32)| <= 4096 is
// not exact in fp16, so it is split as B1 = f16(sc (q - 32)) and B2 = fma(q - 32, sc, -B1), both exact
// integers, and two MFMAs (A B1, then A B2 into the same D) give the block's integer dot exactly
// (|dot| < 2^24).  d8 is applied per block by one fma per output into the super-block's sums T, and d
// once per super-block, into sums kept in LDS (T = sum d8 dot, then acc += d T): 18% fewer VALU
// instructions than d * d8 per block (a multiply and an fma per output), lm_head [102400, 2048] at 512
// tokens 712 -> 632 us.
//
// Alignment: 210 = 2 mod 4, so with 4-byte aligned rows of an even number of super-blocks, super-
// block s starts at a multiple of 4 when s is even and 2 past one when s is odd; every 8-byte piece a
// lane needs sits at a multiple of 8 within it and is read as 3 dwords from the aligned address at or
// 2 before it, realigned by v_alignbyte_b32 with the super-block's offset.  Reads end at most 2 bytes
// into the next super-block (even s: its scale and d dwords) or start at most 2 before (odd s).
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

template <class G>
__global__ __launch_bounds__(G::kThreads) void q6k_gemm_kernel(const GemmArgs a) {
    constexpr int kMT = G::kMT, kBN = G::kBN, kBM = G::kBM;
    using ActStage = qlin::ActStage<G>;
    using Frag = qlin::Frag<kMT>;
    extern __shared__ uint4 lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4, gb = g >> 1;
    int bx, by;
    gemm_tile((a.n + kBN - 1) / kBN, (a.m + kBM - 1) / kBM, bx, by);
    const int m0 = by * kBM;
    const int o0 = bx * kBN + wave * kNT * 16;
    const ActStage st(lds, a, tid, m0);
    const int nsb = a.nblk / 8;  // super-blocks per row (even)

    const uint8_t *wrow[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) wrow[t] = a.w + static_cast<size_t>(min(o0 + t * 16 + n, a.n - 1)) * a.rb;

    // this lane's output sums, tile (i, t) at acc[(i * kNT + t) * 64], in LDS after the activation buffers:
    // a super-block's block sums T are scaled by its d once and added there, so no register set holds
    // them between super-blocks (the kernel's 225 VGPRs leave no room for a second one)
    float4 *acc = reinterpret_cast<float4 *>(lds + 2 * G::kBuf) + wave * kMT * kNT * 64 + lane;
#pragma unroll
    for (int i = 0; i < kMT * kNT; ++i) acc[i * 64] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    struct WRaw {
        K6Raw k[kNT];
    };
    // super-block s of the rows, past the end the last one of the same parity (valid, never used)
    auto sbase = [&](int t, int s) {
        s = min(s, nsb - 2 + (s & 1));
        return wrow[t] + static_cast<size_t>(s) * 210 - 2 * (s & 1);  // the aligned address at or before
    };
    auto fetch_half = [&](WRaw &w, int s, int h) {
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            const uint8_t *b = sbase(t, s);
            load3(w.k[t].ql[2 * h], b + 64 * h + 8 * g);
            load3(w.k[t].ql[2 * h + 1], b + 64 * h + 32 + 8 * g);
            load3(w.k[t].qh[h], b + 128 + 32 * h + 8 * g);
        }
    };
    auto fetch_sd = [&](WRaw &w, int s) {
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            const uint32_t *q = reinterpret_cast<const uint32_t *>(sbase(t, s) + 192);
#pragma unroll
            for (int i = 0; i < 5; ++i) w.k[t].sd[i] = q[i];
        }
    };

    auto compute = [&](WRaw &w, int buf, int u) {
        const int off = 2 * (u & 1);
        // this unit's scales (realigned) and d, then the next unit's requested
        uint32_t s4[kNT][4];
        float dw[kNT];
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) s4[t][i] = __builtin_amdgcn_alignbyte(w.k[t].sd[i + 1], w.k[t].sd[i], off);
            dw[t] = f16_bits_to_f32((w.k[t].sd[4] >> (8 * off)) & 0xffffu);
        }
        fetch_sd(w, u + 1);
        f32x4 T[kMT][kNT];  // sum over the unit's blocks of d8 times the block dot
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int t = 0; t < kNT; ++t) T[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
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
            for (int i = 0; i < kMT; ++i) {
                const float d8r[4] = {f.d8[i].x, f.d8[i].y, f.d8[i].z, f.d8[i].w};
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    const f32x4 Dj = mfma(f.a[i], B2[t], mfma(f.a[i], B1[t], f32x4{0.0f, 0.0f, 0.0f, 0.0f}));
#pragma unroll
                    for (int r = 0; r < 4; ++r) T[i][t][r] = fmaf(Dj[r], d8r[r], T[i][t][r]);
                }
            }
            pin(T);
            if constexpr (J == 3) fetch_half(w, u + 1, 0);
            if constexpr (J == 7) fetch_half(w, u + 1, 1);
            __builtin_amdgcn_sched_barrier(0);
        };
        Frag f0, f1;
        load_frag(f0, st, buf, 0, lane);
        load_frag(f1, st, buf, 1, lane);
        block(ic<0>{}, f0);
        load_frag(f0, st, buf, 2, lane);
        block(ic<1>{}, f1);
        load_frag(f1, st, buf, 3, lane);
        block(ic<2>{}, f0);
        load_frag(f0, st, buf, 4, lane);
        block(ic<3>{}, f1);
        load_frag(f1, st, buf, 5, lane);
        block(ic<4>{}, f0);
        load_frag(f0, st, buf, 6, lane);
        block(ic<5>{}, f1);
        load_frag(f1, st, buf, 7, lane);
        block(ic<6>{}, f0);
        block(ic<7>{}, f1);
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int t = 0; t < kNT; ++t) {
                float4 s = acc[(i * kNT + t) * 64];
                s.x = fmaf(dw[t], T[i][t][0], s.x);
                s.y = fmaf(dw[t], T[i][t][1], s.y);
                s.z = fmaf(dw[t], T[i][t][2], s.z);
                s.w = fmaf(dw[t], T[i][t][3], s.w);
                acc[(i * kNT + t) * 64] = s;
            }
    };

    WRaw w;
    typename ActStage::Raw x;
    fetch_sd(w, 0);
    fetch_half(w, 0, 0);
    fetch_half(w, 0, 1);
    st.fetch(x, 0);
    st.stage(x, 0, 0);
    st.fetch(x, 1);
    __syncthreads();
    for (int u = 0; u < nsb; ++u) {
        const int buf = u & 1;
        compute(w, buf, u);
        st.stage(x, buf ^ 1, u + 1);
        st.fetch(x, u + 2);
        __syncthreads();
    }
    f32x4 out[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
            const float4 v = acc[(i * kNT + t) * 64];
            out[i][t] = f32x4{v.x, v.y, v.z, v.w};
        }
    store_tile(a, out, o0, m0, n, g);
}

}  // namespace

bool qblk_gemm_ok(int type, const uint8_t *w, size_t rb, const uint8_t *xq, int in_dim) {
    if (type == T_Q6_K)
        return in_dim % 512 == 0 && rb % 4 == 0 && (reinterpret_cast<uintptr_t>(w) & 3u) == 0 &&
               (reinterpret_cast<uintptr_t>(xq) & 3u) == 0;
    if (type != T_Q8_0 && type != T_Q5_0 && type != T_Q4_0) return false;
    return in_dim % 64 == 0 && rb % 4 == 0 && (reinterpret_cast<uintptr_t>(w) & 3u) == 0 &&
           (reinterpret_cast<uintptr_t>(xq) & 3u) == 0;
}

hipError_t qblk_gemm_q8_1(int type, const uint8_t *w, size_t rb, const uint8_t *xq, float *y, int out_dim,
                          int in_dim, int m, hipStream_t s) {
    if (out_dim == 0 || m == 0) return hipSuccess;
    GemmArgs a;
    a.w = w;
    a.rb = rb;
    a.xq = xq;
    a.xrb = static_cast<size_t>(in_dim / 32) * 36;
    a.y = y;
    a.n = out_dim;
    a.m = m;
    a.nblk = in_dim / 32;
    auto launch = [&](auto geo) {
        using G = decltype(geo);
        const dim3 grid = gemm_grid((out_dim + G::kBN - 1) / G::kBN, (m + G::kBM - 1) / G::kBM);
        switch (type) {
            case T_Q8_0: hipLaunchKernelGGL((qblk_gemm_kernel<T_Q8_0, G>), grid, dim3(G::kThreads), G::kLdsBytes, s, a); break;
            case T_Q5_0: hipLaunchKernelGGL((qblk_gemm_kernel<T_Q5_0, G>), grid, dim3(G::kThreads), G::kLdsBytes, s, a); break;
            case T_Q4_0: hipLaunchKernelGGL((qblk_gemm_kernel<T_Q4_0, G>), grid, dim3(G::kThreads), G::kLdsBytes, s, a); break;
            case T_Q6_K:
                if constexpr (std::is_same_v<G, GeoLarge>) {
                    hipLaunchKernelGGL((q6k_gemm_kernel<G>), grid, dim3(G::kThreads), G::kLdsBytesQ6, s, a);
                    break;
                }
                return hipErrorInvalidValue;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    };
    // the default tiles, unless they would leave more than half the CUs idle (the Q6_K kernel keeps
    // the default: its lm_head shapes fill the chip many times).  DeepSeek-V2-Lite's Q5_0 expert down at
    // 512 tokens (64 default workgroups): 40.5 -> 23.7 us.  A Q8_0 [4864, 896] at 512 tokens (152 default
    // workgroups) ran 34.2 us on the default tiles and 45.5 us on the small ones.
    const int64_t large = static_cast<int64_t>((out_dim + GeoLarge::kBN - 1) / GeoLarge::kBN) *
                          ((m + GeoLarge::kBM - 1) / GeoLarge::kBM);
    if (QLIN_QBLK_SMALL && type != T_Q6_K && large * 2 < device_info().cu_count) return launch(GeoSmall{});
    return launch(GeoLarge{});
}

}  // namespace qlin

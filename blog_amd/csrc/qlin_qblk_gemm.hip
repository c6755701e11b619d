// qlin_qblk_gemm.hip -- Q8_0, Q5_0 and Q4_0 weights x Q8_1 activations, the prefill GEMM, on the fp16
// matrix cores of gfx950.
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
// One LDS buffer (uint4 units): the qx plane [mt][j][lane] (fp16 integers), then the block scales
// d8 [mt][j][token] as floats.  Two buffers: 68 KB.
constexpr int kPlane = kMT * 8 * 64;
constexpr int kD8 = kMT * 8 * 16 / 4;
constexpr int kBuf = kPlane + kD8;
constexpr size_t kLdsBytes = 2 * kBuf * sizeof(uint4);
constexpr int kSJ = kThreads / kMT / 64;  // staging waves per token tile
constexpr int kJJ = 8 / kSJ;              // blocks each staging thread converts

template <int FMT> struct QBlk;
template <> struct QBlk<T_Q8_0> {
    static constexpr int bytes = 34, offset = 0;
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

template <int FMT>
__global__ __launch_bounds__(kThreads) void qblk_gemm_kernel(const GemmArgs a) {
    constexpr int BB = QBlk<FMT>::bytes;
    extern __shared__ uint4 lds[];
    auto plane = [&](int buf) { return lds + buf * kBuf; };
    auto d8s = [&](int buf) { return reinterpret_cast<float *>(lds + buf * kBuf + kPlane); };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.y * kBM;
    const int o0 = blockIdx.x * kBN + wave * kNT * 16;
    const int nblk = a.nblk, nunit = (nblk + 7) / 8;

    const uint8_t *wrow[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) wrow[t] = a.w + static_cast<size_t>(min(o0 + t * 16 + n, a.n - 1)) * a.rb;

    // staging role: token tile smt, slot lane sl (token si, k-group sg), blocks kJJ*sjh .. +kJJ-1
    const int smt = tid / (kSJ * 64), sjh = (tid >> 6) % kSJ, sl = tid & 63, si = sl & 15, sg = sl >> 4;
    const int tok = m0 + smt * 16 + si;
    const uint8_t *xrow = a.xq + static_cast<size_t>(min(tok, a.m - 1)) * a.xrb;

    f32x4 T[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int t = 0; t < kNT; ++t) T[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // this wave's weight bytes of one unit: block j of tile t
    struct WRaw {
        BRaw b[8][kNT];
    };
    struct XRaw {
        uint32_t bh[kJJ], q0[kJJ], q1[kJJ];
    };
    // block J of unit u (past the end: the last block of the same parity, valid and never used)
    auto fetch_blk = [&](auto jc, WRaw &w, int u) {
        constexpr int J = decltype(jc)::value;
        const int b = min(8 * u + J, nblk - 2 + (J & 1));
#pragma unroll
        for (int t = 0; t < kNT; ++t) w.b[J][t] = load_block<FMT, J & 1>(wrow[t] + static_cast<size_t>(b) * BB, g);
    };
    auto fetch_x = [&](XRaw &x, int u) {
        u = min(u, nunit - 1);
#pragma unroll
        for (int jj = 0; jj < kJJ; ++jj) {
            const int b = min(u * 8 + kJJ * sjh + jj, nblk - 1);
            const uint8_t *blk = xrow + static_cast<size_t>(b) * 36;
            x.bh[jj] = *reinterpret_cast<const uint32_t *>(blk);
            x.q0[jj] = *reinterpret_cast<const uint32_t *>(blk + 4 + 8 * sg);
            x.q1[jj] = *reinterpret_cast<const uint32_t *>(blk + 8 + 8 * sg);
        }
    };

    // Activations of unit u into buffer buf: qx as fp16 integers, d8 as a float per (token tile,
    // block, token); blocks past the row are zeros.  Tokens past m repeat the last row: their D rows
    // are never stored.
    auto stage = [&](const XRaw &x, int buf, int u) {
        uint4 *pl = plane(buf);
        const f16x2 off = splat(-1152.0f);
#pragma unroll
        for (int jj = 0; jj < kJJ; ++jj) {
            const int j = kJJ * sjh + jj;
            const bool live = u * 8 + j < nblk;
            const uint32_t v[2] = {x.q0[jj] ^ 0x80808080u, x.q1[jj] ^ 0x80808080u};
            uint32_t qh[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t sel = (e & 1) ? 0x04030402u : 0x04010400u;
                qh[e] = live ? h2u(u2h(__builtin_amdgcn_perm(0x64646464u, v[e >> 1], sel)) + off) : 0u;
            }
            pl[(smt * 8 + j) * 64 + sl] = make_uint4(qh[0], qh[1], qh[2], qh[3]);
            if (sg == 0) d8s(buf)[(smt * 8 + j) * 16 + si] = live ? f16_bits_to_f32(x.bh[jj] & 0xffffu) : 0.0f;
        }
    };

    // One unit from buffer buf: the blocks' MFMAs and scaling; each block's weights are reloaded
    // with unit `next` right after they are decoded.
    auto compute = [&](WRaw &w, int buf, int u) {
        const uint4 *pl = plane(buf);
        const float *d8 = d8s(buf);
        const int next = u + 1;
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
                // the scaling, pinned before the next block's MFMAs (instruction selection would
                // otherwise keep every block's results live to the end of the unit)
                static_assert(kMT * kNT == 8, "one operand per sum");
                asm volatile("" ::"v"(T[0][0]), "v"(T[0][1]), "v"(T[1][0]), "v"(T[1][1]), "v"(T[2][0]),
                             "v"(T[2][1]), "v"(T[3][0]), "v"(T[3][1]));
            }
            fetch_blk(jc, w, next);
            __builtin_amdgcn_sched_barrier(0);
        };
        // fragments of block J + 1 are read while J is multiplied
        Frag f0, f1;
        load_frag(f0, 0);
        load_frag(f1, 1);
        block(ic<0>{}, f0);
        load_frag(f0, 2);
        block(ic<1>{}, f1);
        load_frag(f1, 3);
        block(ic<2>{}, f0);
        load_frag(f0, 4);
        block(ic<3>{}, f1);
        load_frag(f1, 5);
        block(ic<4>{}, f0);
        load_frag(f0, 6);
        block(ic<5>{}, f1);
        load_frag(f1, 7);
        block(ic<6>{}, f0);
        block(ic<7>{}, f1);
    };

    // Pipeline over units: u is computed from buffer u & 1 while its weights are replaced by u + 1's
    // block by block; then u + 1's activations (loaded during u) are staged into the other buffer,
    // whose last reads were before the previous barrier, and u + 2's requested.
    WRaw w;
    XRaw x;
    fetch_blk(ic<0>{}, w, 0);
    fetch_blk(ic<1>{}, w, 0);
    fetch_blk(ic<2>{}, w, 0);
    fetch_blk(ic<3>{}, w, 0);
    fetch_blk(ic<4>{}, w, 0);
    fetch_blk(ic<5>{}, w, 0);
    fetch_blk(ic<6>{}, w, 0);
    fetch_blk(ic<7>{}, w, 0);
    fetch_x(x, 0);
    stage(x, 0, 0);
    fetch_x(x, 1);
    __syncthreads();
    for (int u = 0; u < nunit; ++u) {
        const int buf = u & 1;
        compute(w, buf, u);
        stage(x, buf ^ 1, u + 1);  // past the end: zeros and copies, never read
        fetch_x(x, u + 2);
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
                if (tk < a.m) a.y[static_cast<size_t>(tk) * a.n + o] = T[i][t][r];
            }
    }
}

}  // namespace

bool qblk_gemm_ok(int type, const uint8_t *w, size_t rb, const uint8_t *xq, int in_dim) {
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
    const dim3 grid((out_dim + kBN - 1) / kBN, (m + kBM - 1) / kBM);
    switch (type) {
        case T_Q8_0: hipLaunchKernelGGL(qblk_gemm_kernel<T_Q8_0>, grid, dim3(kThreads), kLdsBytes, s, a); break;
        case T_Q5_0: hipLaunchKernelGGL(qblk_gemm_kernel<T_Q5_0>, grid, dim3(kThreads), kLdsBytes, s, a); break;
        case T_Q4_0: hipLaunchKernelGGL(qblk_gemm_kernel<T_Q4_0>, grid, dim3(kThreads), kLdsBytes, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qlin

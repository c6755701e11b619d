// qlin_moe_grouped.hip -- routed-expert decode for a batch of tokens, each selected expert read
// once for all the routes that chose it, gfx950.
//
// Per token t the result is the reference's routed sum (TensorTool::moe_routed_decode_indexed,
// AI/codes/local-llm/src/tensor/TensorTool.cpp:271-336, with kernel.cu:1340-1385 and 2253-2287):
//   act_r  = silu(Wg[e_r] x_t) * (Wu[e_r] x_t)               for routes r of t with 0 <= e_r < E
//   out[t] += sum_r fmaf(Wd[e_r] act_r, w_r, .)  in route order r = 0 .. k-1
// The reference decodes one token at a time, so an expert chosen by several tokens of a batch is
// read once per token.  Here the routes are first grouped by expert (a stable counting sort on the
// device, which also lists the selected experts), then two streaming launches read the selected
// experts' rows once per pass of up to NQ routes:
//   gate/up (Q4_K) and down (Q5_0, Q8_0), both on the bf16 matrix cores: one workgroup per
//     CU takes a contiguous range of the selected experts' 16-row tiles, and its waves claim
//     (tile, matrix, chunk) steps in memory order from an LDS counter, loading the next step while
//     computing the current one, as the decode GEMV does;
//   combine: per (token, hidden row), the route results in route order.
// Shapes or layouts outside those kernels' preconditions take per-element kernels (up_kernel,
// down_kernel) with the same results.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "qlin_mfma.hpp"
#include "qlin_plan.hpp"
#include "qlin_rows.hpp"

#include <algorithm>
#include <mutex>

namespace qlin {
namespace {

constexpr int kGroup = 4;  // routes of one expert per pass of the per-element kernels
constexpr int kMaxExperts = 1024;
constexpr int kRouteBits = 21;  // routes per call < 2^21: the expert scan packs (count, selected)
constexpr int kIdsChunk = 4096;
// The gate/up streaming launch groups the routes itself (in LDS) up to these sizes.
constexpr int kFuseRoutes = 1024;
constexpr int kFuseExperts = 256;

struct Groups {
    int *offset;  // [E + 1] first position of expert e in list
    int *list;    // [R] route indices grouped by expert, increasing within an expert
    int4 *seg;    // [E] the selected experts in increasing id order: (expert, first position, count, 0)
    int *nsel;    // number of selected experts
};

// Stable counting sort of the R = tokens * k routes by expert id (invalid ids are left out).  One
// workgroup: the ids are staged in LDS, thread e counts and then lists expert e's routes in route
// order, and a scan over the experts gives the offsets and the compacted selected-expert records.
__global__ __launch_bounds__(1024) void group_kernel(const int *__restrict__ ids, int R, int E, Groups gr) {
    __shared__ int4 s_ids4[kIdsChunk / 4];
    __shared__ int s_wave[16];
    const int *s_ids = reinterpret_cast<const int *>(s_ids4);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // a chunk of ids into LDS, padded with -1 to a multiple of 16 (read 16 at a time below)
    auto stage = [&](int base) {
        const int n = min(kIdsChunk, R - base);
        int *dst = reinterpret_cast<int *>(s_ids4);
        for (int i = tid; i < ((n + 15) & ~15); i += 1024) dst[i] = i < n ? ids[base + i] : -1;
        return n;
    };
    auto count16 = [&](int i, int e) {
        int c = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int4 v = s_ids4[i / 4 + j];
            c += (v.x == e) + (v.y == e) + (v.z == e) + (v.w == e);
        }
        return c;
    };
    int c = 0;
    for (int base = 0; base < R; base += kIdsChunk) {
        if (base) __syncthreads();
        const int n = stage(base);
        __syncthreads();
        if (tid < E)
            for (int i = 0; i < n; i += 16) c += count16(i, tid);
    }
    // exclusive scan over the experts of count | selected << kRouteBits
    const int v = tid < E ? c | (static_cast<int>(c > 0) << kRouteBits) : 0;
    int inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(inc, d, 64);
        if (lane >= d) inc += t;
    }
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += s_wave[w];
    const int excl = before + inc - v;
    constexpr int kMask = (1 << kRouteBits) - 1;
    const int pos0 = excl & kMask;
    if (tid < E) {
        gr.offset[tid] = pos0;
        if (c > 0) gr.seg[excl >> kRouteBits] = make_int4(tid, pos0, c, 0);
    }
    if (tid == 1023) {  // threads past E add nothing, so the last inclusive value is the total
        gr.offset[E] = (before + inc) & kMask;
        *gr.nsel = (before + inc) >> kRouteBits;
    }
    int pos = pos0;
    for (int base = 0; base < R; base += kIdsChunk) {
        int n = min(kIdsChunk, R - base);
        if (R > kIdsChunk) {  // the count pass left only the last chunk in LDS
            __syncthreads();
            n = stage(base);
            __syncthreads();
        }
        if (tid < E && c > 0)
            for (int i = 0; i < n; i += 16) {
                if (count16(i, tid) == 0) continue;
                for (int j = i; j < i + 16; ++j)
                    if (s_ids[j] == tid) gr.list[pos++] = base + j;
            }
    }
}

// ---- streaming grouped kernels (matrix cores) ---------------------------------------------------

// Q4_K steps on the int8 matrix cores (x as digits, see x_digits4): 2-5% faster over the grouped
// decode than the bf16 operands (4 MFMAs per route instead of 8, the nibbles taken as they are)
#ifndef QLIN_STREAM_I8
#define QLIN_STREAM_I8 1
#endif
constexpr int kSWaves = 16;
constexpr int kSThreads = kSWaves * 64;
using plan::kXPad;

// One step = 16 rows x one chunk of a row.
//   Q4_K (gate/up): a chunk is one super-block; the A operand is the decode GEMV's block-diagonal
//     layout (rows = 8 sub-blocks x hi/lo of one route), 8 MFMAs per route.
//   Q5_0 / Q8_0 (down): a chunk is 4 blocks, lane-group g decoding block g.  A rows are
//     (block b, route r of a pair, hi/lo): row i = 4b + 2r + p, nonzero only in lane-group b's
//     k-slots, so one set of tpb MFMAs serves two routes and D rows 4g .. 4g+3 of a lane hold its
//     block's dots for both.  MFMA t takes qs dword t of the block: the 4 low nibbles (elements
//     4t .. 4t+3) and the 4 high ones (elements 16+4t ..), or for Q8_0 the bytes q+128 = 16h + l
//     split into nibbles, with A slots (x, 16x) so that one D sums both.
//   Per block: sum x*w = d * (D - corr * X), X = sum of x (hi + lo) over the block, because the
//   operand is bf16(128 + u) with u = q + 16 (Q5_0), or l / h (Q8_0: 128*17 + 128).
template <int FMT> struct StepFmt;
// The workgroups split the selected experts' work by a cost: a 16-row tile costs the larger of w0 per
// pass (the weights' stream) and wc per route (the block-diagonal operand's MFMA and VALU work), plus
// w1 per route, and an expert ws per pass (the workgroup that takes part of an expert stages its
// routes' x and starts a new stream of steps).  Fitted to per-workgroup times within one launch of the
// C5 shape (16 tokens, top-6 of 64): a gate/up tile takes 1.49 us with 1, 2 or 3 routes and 1.80 us
// with 4 (workgroups that take one expert, by its route count), an expert about 4.4 us more; over all
// workgroups a down tile 0.52 us, a route on it 0.07 us, an expert 3.2 us (residual 1.0 us, no trend
// left by route count).  (A gate/up cost linear in the routes, 32 + routes, left the workgroups with
// a 4-route expert 7 us behind the median.)
template <> struct StepFmt<T_Q4_K> {
    static constexpr int ce = 256, bb = 144, cb = 144, tpb = 0, w0 = 32, wc = 10, w1 = 0, ws = 94;
};
template <> struct StepFmt<T_Q5_0> {
    static constexpr int ce = 128, bb = 22, cb = 88, nd = 5, tpb = 4, w0 = 8, wc = 0, w1 = 1, ws = 54;
    static constexpr float corr = 144.0f;
};
template <> struct StepFmt<T_Q8_0> {
    static constexpr int ce = 128, bb = 34, cb = 136, nd = 8, tpb = 8, w0 = 8, wc = 0, w1 = 1, ws = 54;
    static constexpr float corr = 2304.0f;
};

struct StreamArgs {
    const uint8_t *w0, *w1;  // gate/up: Wg, Wu; down: Wd (w1 = w0)
    size_t eb, rb;           // expert and row bytes
    const float *x;          // gate/up: x [tokens, K]; down: act [R, K]
    int x_div;               // the x row of route r is r / x_div (k for gate/up, 1 for down)
    const int *list;
    const int4 *seg;
    const int *nsel;
    float *out;              // gate/up: act [R, rows]; down: per-route results [R, rows]
    int rows, K, nchunk, tpe;  // rows per expert, inner dimension, chunks per row, 16-row tiles per expert
    int piece;                 // tiles whose step partials fit in LDS at once
    // grouping in the kernel (GRP): the routes' expert ids, their count and the expert count; the
    // groups are built in LDS from these, and workgroup 0 writes them to gr for the later launches.
    // With logits (n_experts <= 64) the kernel also routes: the ids are the router's picks, which
    // workgroup 0 writes to ids_out and w_out (weights times scaling) as router_topk does.
    const int *ids;
    int R, ne;
    Groups gr;
    const float *logits;
    float scaling;
    int *ids_out;
    float *w_out;
    // SW: the shared experts' SwiGLU in the same launch (sh_rows > 0): workgroup b computes 16-row tiles
    // b * sh_per_wg .. of the shared gate and up matrices for the sh_tokens (<= 16) rows of x before its
    // routed share, into sh_act [sh_tokens, sh_rows], and its routed share is smaller by sh_cost.
    const uint8_t *sh_wg, *sh_wu;
    size_t sh_rb;
    float *sh_act;
    int sh_rows, sh_tokens, sh_cost, sh_per_wg;
};
// LDS of the in-kernel router, after the staged ids: per wave the 64 exponentials
constexpr int kRouteWaveFloats = 64;
// Shared-expert tiles in the gate/up launch: up to kSharedMaxTiles per workgroup (one output pass of
// 256 threads each), the tokens' x and then their partials (per tile 8 super-block slots x 2 matrices
// x 64 lanes of 4 floats) in the dynamic LDS.  A workgroup's cost for them, in the units of
// StepFmt<T_Q4_K> (about 0.047 us of a workgroup's time each): staging x, then each tile
// (per-workgroup trace at 16 tokens, two tiles per workgroup: x staged 6.0 us after the start, the
// tiles done 10 us later; with x rows unpadded, staging took 5.3 us and the tiles 11.7 more, their
// 16 lanes reading one bank, and the costs were 125 and 135).
// Two tiles per workgroup halve the staging (C5 step 89.2 -> 88.2 us against one); more, in this
// kernel's 128 VGPRs, spill.
#ifndef QLIN_SHARED_TILES
#define QLIN_SHARED_TILES 2  // tiles per workgroup
#endif
constexpr int kSharedMaxTiles = 2;
constexpr size_t kSharedPartBytes = 8 * 2 * 64 * 16;
constexpr int kSharedStageCost = 140, kSharedTileCost = 115;

// 64-bit integer division is a sequence of a few hundred scalar instructions, run by every wave and
// shared by the 16 waves of a CU: both helpers take 32-bit arithmetic when the operands allow
// (wave-uniform branches), which covers every realistic cost total.
__device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) {
    constexpr int64_t lim = int64_t{1} << 30;
    if (a > -lim && a < lim && b < lim)
        return (static_cast<int>(a) + static_cast<int>(b) - 1) / static_cast<int>(b);
    return (a + b - 1) / b;
}
// floor(C * b / G) for workgroup b of G
__device__ __forceinline__ int64_t share_bound(int64_t C, int b, int G) {
    if (C < (int64_t{1} << 23) && G <= 256)
        return static_cast<int64_t>(static_cast<uint32_t>(C) * static_cast<uint32_t>(b) / static_cast<uint32_t>(G));
    return C * b / G;
}

// A value the whole wave holds alike, moved to scalar registers (LDS and vector loads give VGPRs).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni(int64_t v) {
    const uint64_t u = static_cast<uint64_t>(v);
    return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(uni(static_cast<int>(u >> 32)))) << 32) |
                                static_cast<uint32_t>(uni(static_cast<int>(u))));
}

// Cost of one 16-row tile of an expert with cnt routes (its passes and its routes), and of the
// expert's set-up per pass, which comes first in the expert's cost range.
template <int FMT, int NQ>
__device__ __forceinline__ int64_t tile_cost(int cnt) {
    using F = StepFmt<FMT>;
    const int64_t stream = static_cast<int64_t>((cnt + NQ - 1) / NQ) * F::w0, math = static_cast<int64_t>(cnt) * F::wc;
    return (stream > math ? stream : math) + static_cast<int64_t>(cnt) * F::w1;
}
template <int FMT, int NQ>
__device__ __forceinline__ int64_t setup_cost(int cnt) {
    return static_cast<int64_t>((cnt + NQ - 1) / NQ) * StepFmt<FMT>::ws;
}

// SW: gate and up matrices with SiLU(gate) * up out (Q4_K); otherwise one matrix, its dot out.
template <int FMT, int NQ, bool SW, bool GRP>
__global__ __launch_bounds__(kSThreads) void stream_kernel(const StreamArgs a) {
    using F = StepFmt<FMT>;
    constexpr bool K4 = FMT == T_Q4_K;  // super-block steps, block-diagonal A
    constexpr int NW = SW ? 2 : 1;      // matrices per output row (gate, up)
    static_assert(!SW || K4, "the SwiGLU pair is Q4_K");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int K = a.K, nblk = K / 32, nchunk = a.nchunk;
    // staging of the pass's routes: Q4_K bf16 planes [NQ][2][KX]; others slot vectors
    // [NQ][2][PS] (8 bf16 each, nblk * tpb of them and a pad); then the block sums X [NQ][nblk] and
    // the step partials [NW][NQ][nchunk][rows of the piece]
    // I8 (Q4_K): the routes' x as int8 digit planes [NQ][3][KP] and (scale, sum) per 32 elements,
    // in no more LDS than the bf16 planes (the plan is sized for those)
    // The parts and planes are kXPad bytes longer than their values: an A-operand read gathers one
    // offset of several of them, which then fall in different LDS banks.
    constexpr bool I8 = K4 && QLIN_STREAM_I8;
    const int KX = K + kXPad / 2, KP = K + kXPad, PS = nblk * F::tpb + kXPad / 16;
    const size_t stage_bytes = I8   ? static_cast<size_t>(NQ) * 3 * KP
                               : K4 ? static_cast<size_t>(NQ) * 4 * KX
                                    : static_cast<size_t>(NQ) * 2 * PS * 16;
    uint16_t *xpart = reinterpret_cast<uint16_t *>(smem);
    uint4 *slots = reinterpret_cast<uint4 *>(smem);
    int8_t *planes = reinterpret_cast<int8_t *>(smem);
    float *xsum = reinterpret_cast<float *>(smem + stage_bytes);  // I8: [NQ][nblk][2] (scale, sum)
    float *partial = xsum + NQ * nblk * (I8 ? 2 : 1);
    __shared__ int next_step;
    __shared__ int64_t s_pref[kMaxExperts + 1];  // cost of the selected experts before s
    __shared__ int64_t s_wave[kSWaves];
    __shared__ uint4 s_zero[8];  // down: the A operand of lanes whose k-slots are empty

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    if (tid < 8) s_zero[tid] = make_uint4(0u, 0u, 0u, 0u);  // before the barriers below

    // The shared experts' SwiGLU tiles of this workgroup, first (they depend on no routing): wave w takes
    // matrix w & 1 and super-blocks w / 2, w / 2 + 8, ... of each tile, the wave and order
    // q4k_dense_kernel's wave w / 2 gives that matrix, and the 8 waves' sums of a matrix are added in
    // wave order as there: the same bits as the separate launch.  The tokens' x is staged in LDS once
    // per workgroup (read from L2 by every wave, the x lines' L2 channels were the bound), after each
    // wave has requested its first weights, and serves the workgroup's sh_per_wg tiles; x and then the
    // partials use the (still unused) staging area.
    const int n_tiles = SW && a.sh_rows > 0 ? (a.sh_rows + 15) / 16 : 0;
    const int n_shared = n_tiles ? (n_tiles + a.sh_per_wg - 1) / a.sh_per_wg : 0;  // workgroups with tiles
    if constexpr (SW) {
        if (blockIdx.x < n_shared) {  // uniform
            const int m = wave & 1, slot = wave >> 1, nsb = a.K / 256;
            const int t0 = blockIdx.x * a.sh_per_wg, nt = min(a.sh_per_wg, n_tiles - t0);
            const uint8_t *wm = m ? a.sh_wu : a.sh_wg;
            const uint8_t *rp[kSharedMaxTiles];
#pragma unroll
            for (int t = 0; t < kSharedMaxTiles; ++t)
                rp[t] = wm + static_cast<size_t>(min((t0 + min(t, nt - 1)) * 16 + n, a.sh_rows - 1)) * a.sh_rb;
            Q4KRaw cur[1];
            if (slot < nsb) load_q4k(cur[0], rp[0] + static_cast<size_t>(slot) * 144, g);
            // [sh_tokens][K + 4]: the rows padded by 16 bytes, so that the 16 lanes of a lane group, one
            // token each, read the same offsets of 16 rows from different banks.  The flat copy advances
            // its (token, column) pair with the index instead of dividing it.
            float *sx = reinterpret_cast<float *>(smem);
            const int k4 = a.K / 4, nx4 = a.sh_tokens * k4;
            int xt = tid / k4, xj = tid - xt * k4;
            for (int i = tid; i < nx4; i += kSThreads) {
                reinterpret_cast<float4 *>(sx)[xt * (k4 + 1) + xj] = reinterpret_cast<const float4 *>(a.x)[i];
                xj += kSThreads;
                while (xj >= k4) {
                    xj -= k4;
                    ++xt;
                }
            }
            __syncthreads();
            const float *xrow = sx + min(n, a.sh_tokens - 1) * (a.K + 4) + 8 * g;
            f32x4 D[kSharedMaxTiles];
#pragma unroll
            for (int t = 0; t < kSharedMaxTiles; ++t) D[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            q4k_tiles_dot<kSharedMaxTiles>(cur, rp, nt, xrow, slot, 8, nsb, g, D);
            __syncthreads();  // x is read: the partials take its place
            f32x4 *part = reinterpret_cast<f32x4 *>(smem);  // [tile][slot][matrix][lane]
#pragma unroll
            for (int t = 0; t < kSharedMaxTiles; ++t)
                if (t < nt) part[((t * 8 + slot) * 2 + m) * 64 + lane] = D[t];
            __syncthreads();
            // outputs: 256 threads per tile; token tl, row row0 + o; D element r of lane l is token
            // 4 (l / 16) + r
            const int ti = tid >> 8, tl = (tid >> 4) & 15, o = tid & 15;
            if (ti < nt) {
                const int row0 = (t0 + ti) * 16;
                if (tl < a.sh_tokens && o < min(16, a.sh_rows - row0)) {
                    const int l = (tl >> 2) * 16 + o, r = tl & 3;
                    const f32x4 *pt = part + ti * 8 * 2 * 64;
                    float v0 = 0.0f, v1 = 0.0f;
                    for (int wv = 0; wv < 8; ++wv) {
                        v0 += pt[(wv * 2) * 64 + l][r];
                        v1 += pt[(wv * 2 + 1) * 64 + l][r];
                    }
                    a.sh_act[static_cast<size_t>(tl) * a.sh_rows + row0 + o] = v0 / (1.0f + expf(-v0)) * v1;
                }
            }
            __syncthreads();  // the staging area is free again
        }
    }

    // GRP: the routes grouped by expert here, as group_kernel does (a stable counting sort, invalid
    // ids left out), into LDS: one launch and two dependent reads (the count, then the records) fewer
    // before the first weights are requested.  The ids are staged in the (still unused) x staging area.
    __shared__ int s_list[GRP ? kFuseRoutes : 1];
    __shared__ int4 s_seg[GRP ? kFuseExperts : 1];
    __shared__ int s_scan[kSWaves];
    __shared__ int s_off[GRP ? kFuseExperts : 1];
    __shared__ int s_nsel;
    if constexpr (GRP) {
        const int R = a.R, E = a.ne, R16 = (R + 15) & ~15;
        int *sids = reinterpret_cast<int *>(smem);
        const int4 *sids4 = reinterpret_cast<const int4 *>(smem);
        if (a.logits) {  // uniform
            // router_rank_kernel's picks, one token per wave at a time (E <= 64: lane e holds expert e)
            const int k = a.x_div, T = R / k;
            float *ex = reinterpret_cast<float *>(smem) + R16 + wave * kRouteWaveFloats;
            for (int i = R + tid; i < R16; i += kSThreads) sids[i] = -1;
            for (int t0 = 0; t0 < T; t0 += kSWaves) {
                const int t = t0 + wave;
                route_token_rank(t < T, a.logits + static_cast<size_t>(t) * E, E, k, a.scaling, ex,
                                 [&](int r, int e, float w) {
                                     const size_t o = static_cast<size_t>(t) * k + r;
                                     sids[o] = e;
                                     if (blockIdx.x == 0) {
                                         a.ids_out[o] = e;
                                         a.w_out[o] = w;
                                     }
                                 });
            }
            __syncthreads();  // the picks are in LDS
        } else {
            for (int i = tid; i < R16; i += kSThreads) sids[i] = i < R ? a.ids[i] : -1;
            __syncthreads();
        }
        // routes i .. i + 15 (below lim) with expert e
        auto count16 = [&](int i, int e, int lim = 0x7fffffff) {
            int c = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int4 v = sids4[i / 4 + j];
                const int b = i + 4 * j;
                c += (v.x == e && b < lim) + (v.y == e && b + 1 < lim) + (v.z == e && b + 2 < lim) +
                     (v.w == e && b + 3 < lim);
            }
            return c;
        };
        int c = 0;
        if (tid < E) {
#pragma unroll 4
            for (int i = 0; i < R; i += 16) c += count16(i, tid);
        }
        // exclusive scan over the experts of count | selected << kRouteBits: the first list
        // position of each expert and the records of the selected ones
        const int v = tid < E ? c | (static_cast<int>(c > 0) << kRouteBits) : 0;
        int inc = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int t = __shfl_up(inc, d, 64);
            if (lane >= d) inc += t;
        }
        const int nw = (E + 63) / 64;  // the waves that hold experts
        if (lane == 63 && wave < nw) s_scan[wave] = inc;
        __syncthreads();
        int before = 0;
        for (int w = 0; w < min(wave, nw); ++w) before += s_scan[w];
        const int excl = before + inc - v;
        constexpr int kMask = (1 << kRouteBits) - 1;
        const int pos0 = excl & kMask;
        if (tid < E) s_off[tid] = pos0;
        if (tid < E && c > 0) s_seg[excl >> kRouteBits] = make_int4(tid, pos0, c, 0);
        if (tid == 0) {
            int total = 0;
            for (int w = 0; w < nw; ++w) total += s_scan[w];
            s_nsel = total >> kRouteBits;
            if (blockIdx.x == 0) {
                a.gr.offset[E] = total & kMask;
                *a.gr.nsel = total >> kRouteBits;
            }
        }
        if (blockIdx.x == 0 && tid < E) a.gr.offset[tid] = pos0;
        __syncthreads();
        // route r goes after the earlier routes of its expert (thread r counts them)
        if (tid < R) {
            const int e = sids[tid];
            if (e >= 0 && e < E) {
                int rank = 0;
                const int full = tid & ~15;
#pragma unroll 4
                for (int i = 0; i < full; i += 16) rank += count16(i, e);
                rank += count16(full, e, tid);
                s_list[s_off[e] + rank] = tid;
            }
        }
        __syncthreads();  // the groups are complete; the staging area is free again
        if (blockIdx.x == 0) {
            const int nsel = s_nsel;
            for (int i = tid; i < R; i += kSThreads) a.gr.list[i] = s_list[i];  // past the valid routes: unread
            if (tid < nsel) a.gr.seg[tid] = s_seg[tid];
        }
    }
    const int *lst = GRP ? s_list : a.list;
    const int4 *segs = GRP ? s_seg : a.seg;
    // (otherwise the records' counts are read with the number of them, not after it: the entries
    // past that number are not used)
    int seg_cnt = 0;
    if (!GRP && tid < a.ne) seg_cnt = a.seg[tid].z;
    const int nsel = GRP ? s_nsel : *a.nsel;
    if (nsel == 0) return;  // uniform

    // Each workgroup takes an equal share of the total cost, in tiles: tile t of selected expert s
    // starts at cost s_pref[s] + setup_cost + t * tile_cost and belongs to the workgroup whose range
    // holds that.
    {
        const int cs = GRP ? (tid < nsel ? segs[tid].z : 0) : seg_cnt;
        const int64_t v =
            tid < nsel ? setup_cost<FMT, NQ>(cs) + static_cast<int64_t>(a.tpe) * tile_cost<FMT, NQ>(cs) : 0;
        int64_t inc = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int64_t t = __shfl_up(inc, d, 64);
            if (lane >= d) inc += t;
        }
        // (up to 64 selected experts, wave 0 holds every cost: no sums across waves)
        const int nw = (nsel + 63) / 64;
        if (nw > 1 && lane == 63 && wave < nw) s_wave[wave] = inc;
        if (nw > 1) __syncthreads();  // uniform
        int64_t before = 0;
        if (nw > 1)
            for (int w = 0; w < min(wave, nw); ++w) before += s_wave[w];
        if (tid == 0) s_pref[0] = 0;
        if (tid < nsel) s_pref[tid + 1] = before + inc;
        __syncthreads();
    }
    const int64_t C = uni(s_pref[nsel]);
    const int bid = blockIdx.x, nwg = gridDim.x;
    // With the shared tiles, workgroup b's range is its equal share of the routed cost plus the shared
    // tiles' cost, less the cost of the shared tiles it took: ranges then stay ordered and cover [0, C)
    // as long as an equal share is at least one tile's cost (else the tiles are left out of the split).
    int64_t us = n_shared ? static_cast<int64_t>(a.sh_cost) : 0;
    if (us > 0 && (C + us * n_shared) / nwg < us) us = 0;
    const int64_t Ct = C + us * n_shared;
    const int64_t c0 = share_bound(Ct, bid, nwg) - us * min(bid, n_shared);
    const int64_t c1 = share_bound(Ct, bid + 1, nwg) - us * min(bid + 1, n_shared);
    if (c0 >= c1) return;  // uniform
    int s_first = 0;
    for (int hi = nsel - 1; s_first < hi;) {  // first expert whose range ends after c0
        const int mid = (s_first + hi) >> 1;
        if (s_pref[mid + 1] > c0) hi = mid;
        else s_first = mid + 1;
    }

    // A-operand role of this lane (row n of A, k-slots of lane-group g)
    const bool a_active = (n >> 2) == g;
    const int a_part = n & 1;
    const int a_pair = (n >> 1) & 1;        // Q5_0 / Q8_0: route of the pair
    // Q4_K x operands, in the decode GEMV's slot order (MFMAs 0..3 carry the low nibbles of lane
    // group g's bytes 8t..8t+7, sub-block 2g; MFMAs 4..7 the high nibbles, sub-block 2g+1): for
    // route q, operand t is the 16 bytes at a_lo (t < 4) or a_hi (t >= 4) + 16 (t & 3), offset by
    // the route and chunk where the lane's row (part n & 1 of sub-block n >> 1) belongs to that
    // sub-block, and a zero area otherwise -- LDS reads with no selects.
    const bool on_lo = (n >> 1) == 2 * g, on_hi = (n >> 1) == 2 * g + 1;
    // I8: row n is digit n & 3 (3: none) of sub-blocks 2g, 2g + 1 of lane group g = n >> 2
    const bool i8_on = (n >> 2) == g && (n & 3) < 3;
    const int8_t *a8 = planes + (n & 3) * KP + 64 * g;  // read only when i8_on
    const uint8_t *a_lo, *a_hi;
    {
        const uint8_t *xb = reinterpret_cast<const uint8_t *>(xpart + a_part * KX + (n >> 1) * 32);
        const uint8_t *zb = reinterpret_cast<const uint8_t *>(s_zero);
        a_lo = on_lo ? xb : zb;
        a_hi = on_hi ? xb : zb;
    }
    const ScaleDecoder dec(g);
    // others: lane-group g's block starts bb*g bytes into the chunk (bb = 2 mod 4), and nd + 1 dwords
    // from the one holding d cover the block: d in its low half for even g (payload 2 bytes in), its
    // high half for odd g (payload in the next dwords), so no 16-bit load is needed
    const int d_dw = (F::bb * g) >> 2;
    const bool d_hi = g & 1;

    struct Raw {
        uint32_t w[12];
    };
    struct Pos {
        int s, which, tile, ch;
        const uint8_t *rp;
    };

    for (int s = uni(s_first); s < nsel; ++s) {
        if (uni(s_pref[s]) >= c1) break;
        const int4 sg = segs[s];
        const int e = uni(sg.x), beg = uni(sg.y), cnt = uni(sg.z);
        const int64_t ps = uni(s_pref[s]) + setup_cost<FMT, NQ>(cnt);  // where the expert's tiles start
        const int64_t ct = tile_cost<FMT, NQ>(cnt);
        const int lt0 = static_cast<int>(max(ceil_div(c0 - ps, ct), int64_t{0}));
        const int lt1 = static_cast<int>(min(ceil_div(c1 - ps, ct), static_cast<int64_t>(a.tpe)));
        if (lt0 >= lt1) continue;  // uniform
        const uint8_t *we0 = a.w0 + static_cast<size_t>(e) * a.eb;
        const uint8_t *we1 = a.w1 + static_cast<size_t>(e) * a.eb;
        // the tiles are taken in pieces of at most a.piece (the LDS partials' capacity)
        int r0, r1, ntile, nrows, pstride, nsteps;
        auto set_piece = [&](int pt0) {
            const int pt1 = min(pt0 + a.piece, lt1);
            r0 = pt0 * 16;
            r1 = min(pt1 * 16, a.rows);
            ntile = pt1 - pt0;
            nrows = r1 - r0;
            pstride = ntile * 16;
            nsteps = ntile * NW * nchunk;
        };

        // step s in memory order: matrix, then tile, then chunk (past the end: the last step)
        auto at = [&](int st) {
            Pos p;
            p.s = st;
            const int c = min(st, nsteps - 1);
            const int tw = c / nchunk;
            p.ch = c - tw * nchunk;
            p.which = NW == 2 && tw >= ntile;
            p.tile = tw - p.which * ntile;
            const int row = min(r0 + p.tile * 16 + n, r1 - 1);
            p.rp = (p.which ? we1 : we0) + static_cast<size_t>(row) * a.rb;
            return p;
        };
        auto load = [&](Raw &st, const Pos &p) {
            const uint8_t *q = p.rp + static_cast<size_t>(p.ch) * F::cb;
            if constexpr (K4) {
                const u32x4 h = ld16(q), qa = ld16(q + 16 + 32 * g), qb = ld16(q + 32 + 32 * g);
                st.w[0] = h.x; st.w[1] = h.y; st.w[2] = h.z; st.w[3] = h.w;
                st.w[4] = qa.x; st.w[5] = qa.y; st.w[6] = qa.z; st.w[7] = qa.w;
                st.w[8] = qb.x; st.w[9] = qb.y; st.w[10] = qb.z; st.w[11] = qb.w;
            } else {
                // nd + 1 dwords from the one holding d (d_dw + nd is at most the chunk's last dword)
                ld_dwords_a4<F::nd + 1>(q + 4 * d_dw, st.w + 1);
            }
        };

        auto process = [&](const Raw &cur, const Pos &p, int nq) {
            float *pp = partial + (static_cast<size_t>(p.which) * NQ * nchunk + p.ch) * pstride + p.tile * 16 + n;
            const bool store = g == 0 && p.tile * 16 + n < nrows;
            if constexpr (I8) {
                // the pair's nibbles as the int8 B operand (MFMAs 0, 1: sub-block 2g; 2, 3: 2g + 1)
                constexpr uint32_t M = 0x0f0f0f0fu;
                auto nib = [&](int k0, int sh) {
                    return i32x4{static_cast<int>((cur.w[k0] >> sh) & M), static_cast<int>((cur.w[k0 + 1] >> sh) & M),
                                 static_cast<int>((cur.w[k0 + 2] >> sh) & M), static_cast<int>((cur.w[k0 + 3] >> sh) & M)};
                };
                const i32x4 b0 = nib(4, 0), b1 = nib(8, 0), b2 = nib(4, 4), b3 = nib(8, 4);
                uint32_t scp, mp;
                dec(cur.w[1], cur.w[2], cur.w[3], scp, mp);
                const float dd = f16_bits_to_f32(cur.w[0] & 0xffffu);
                const float dmin = f16_bits_to_f32(cur.w[0] >> 16);
                const float dsc0 = dd * static_cast<float>(scp & 0xffu);
                const float dsc1 = dd * static_cast<float>((scp >> 8) & 0xffu);
                const float dm0 = dmin * static_cast<float>(mp & 0xffu);
                const float dm1 = dmin * static_cast<float>((mp >> 8) & 0xffu);
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    if (q >= nq) break;  // uniform
                    const i32x4 *pa = reinterpret_cast<const i32x4 *>(
                        i8_on ? a8 + static_cast<size_t>(q) * 3 * KP + p.ch * 256 : reinterpret_cast<const int8_t *>(s_zero));
                    i32x4 de = mfma_i8(pa[0], b0, i32x4{0, 0, 0, 0});
                    de = mfma_i8(pa[1], b1, de);
                    i32x4 dq = mfma_i8(pa[2], b2, i32x4{0, 0, 0, 0});
                    dq = mfma_i8(pa[3], b3, dq);
                    const float4 sx = *reinterpret_cast<const float4 *>(xsum + 2 * (q * nblk + p.ch * 8 + 2 * g));
                    float r = dsc0 * (sx.x * digits_value(de));
                    r = fmaf(dsc1, sx.z * digits_value(dq), r);
                    r = fmaf(-dm0, sx.y, r);
                    r = fmaf(-dm1, sx.w, r);
                    r = sum_lane_groups(r);
                    if (store) pp[q * nchunk * pstride] = r;
                }
            } else if constexpr (K4) {
                u32x4 B[8];
                constexpr uint32_t M = 0x0f0f0f0fu;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int k = 2 * (t & 3), sh = 4 * (t >> 2);
                    B[t] = weights_operand2((cur.w[4 + k] >> sh) & M, (cur.w[5 + k] >> sh) & M);
                }
                uint32_t scp, mp;
                dec(cur.w[1], cur.w[2], cur.w[3], scp, mp);
                const float dd = f16_bits_to_f32(cur.w[0] & 0xffffu);
                const float dmin = f16_bits_to_f32(cur.w[0] >> 16);
                const float dsc0 = dd * static_cast<float>(scp & 0xffu);
                const float dsc1 = dd * static_cast<float>((scp >> 8) & 0xffu);
                const float dm0 = dmin * static_cast<float>(mp & 0xffu);
                const float dm1 = dmin * static_cast<float>((mp >> 8) & 0xffu);
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    if (q >= nq) break;  // uniform
                    // route q's planes start 4 KX bytes after route q-1's; a chunk is 512 bytes of a plane
                    const int off = q * 4 * KX + p.ch * 512;
                    const u32x4 *pl = reinterpret_cast<const u32x4 *>(a_lo + (on_lo ? off : 0));
                    const u32x4 *ph = reinterpret_cast<const u32x4 *>(a_hi + (on_hi ? off : 0));
                    f32x4 D = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int t = 0; t < 4; ++t) D = mfma(pl[t], B[t], D);
#pragma unroll
                    for (int t = 0; t < 4; ++t) D = mfma(ph[t], B[4 + t], D);
                    const float2 xs = *reinterpret_cast<const float2 *>(xsum + q * nblk + p.ch * 8 + 2 * g);
                    float r = dsc0 * ((D[0] + D[1]) - 128.0f * xs.x);
                    r = fmaf(dsc1, (D[2] + D[3]) - 128.0f * xs.y, r);
                    r = fmaf(-dm0, xs.x, r);
                    r = fmaf(-dm1, xs.y, r);
                    r = sum_lane_groups(r);
                    if (store) pp[q * nchunk * pstride] = r;
                }
            } else {
                uint32_t C[F::nd];
#pragma unroll
                for (int k = 0; k < F::nd; ++k)
                    C[k] = d_hi ? cur.w[2 + k] : __builtin_amdgcn_alignbyte(cur.w[2 + k], cur.w[1 + k], 2);
                const float d = f16_bits_to_f32(d_hi ? cur.w[1] >> 16 : cur.w[1] & 0xffffu);
                u32x4 B[F::tpb];
#pragma unroll
                for (int t = 0; t < F::tpb; ++t) {
                    if constexpr (FMT == T_Q5_0) {
                        const uint32_t qh = C[0], qs = C[1 + t];
                        const uint32_t lo = (qs & 0x0f0f0f0fu) | (spread4(qh >> (4 * t)) << 4);
                        const uint32_t hi = ((qs >> 4) & 0x0f0f0f0fu) | (spread4(qh >> (16 + 4 * t)) << 4);
                        B[t] = weights_operand2(lo, hi);
                    } else {
                        B[t] = weights_operand(C[t] ^ 0x80808080u);
                    }
                }
                const int blk = p.ch * 4 + g;
#pragma unroll
                for (int q = 0; q < NQ; q += 2) {
                    if (q >= nq) break;  // uniform
                    const uint4 *src = a_active ? slots + (static_cast<size_t>(q + a_pair) * 2 + a_part) * PS + blk * F::tpb
                                                : s_zero;
                    f32x4 D = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int t = 0; t < F::tpb; ++t) {
                        const uint4 v = src[t];
                        D = mfma(u32x4{v.x, v.y, v.z, v.w}, B[t], D);
                    }
                    const float r0 = sum_lane_groups(d * ((D[0] + D[1]) - F::corr * xsum[q * nblk + blk]));
                    const float r1 = sum_lane_groups(d * ((D[2] + D[3]) - F::corr * xsum[(q + 1) * nblk + blk]));
                    if (store) {
                        pp[q * nchunk * pstride] = r0;
                        if (q + 1 < nq) pp[(q + 1) * nchunk * pstride] = r1;
                    }
                }
            }
        };

        for (int q0 = 0; q0 < cnt; q0 += NQ) {
            const int nq = min(NQ, cnt - q0);
            set_piece(lt0);
            Pos cur = at(wave);
            Raw buf;
            load(buf, cur);  // the first weights are requested before the activations are staged

            // stage the pass's routes (hi = bf16(x), lo = bf16(x - hi); X sums hi + lo)
            if constexpr (I8) {
                const int per = K / 4;  // float4s per route, a multiple of 64: whole waves per route
                for (int it = tid; it < nq * per; it += kSThreads) {
                    const int q = it / per, c = it - q * per;
                    const int route = lst[beg + q0 + q];
                    const float4 v = reinterpret_cast<const float4 *>(a.x + static_cast<size_t>(route / a.x_div) * K)[c];
                    uint32_t p1, p2, p3;
                    float sc, sm, sm16;
                    x_digits4(v, p1, p2, p3, sc, sm, sm16);
                    uint32_t *pq = reinterpret_cast<uint32_t *>(planes + static_cast<size_t>(q) * 3 * KP);
                    pq[c] = p1;
                    pq[KP / 4 + c] = p2;
                    pq[KP / 2 + c] = p3;
                    if ((c & 7) == 0) reinterpret_cast<float2 *>(xsum)[q * nblk + (c >> 3)] = make_float2(sc, sm);
                }
            } else if constexpr (K4) {
                const int per = K / 4;  // float4s per route, a multiple of 64: whole waves per route
                for (int it = tid; it < nq * per; it += kSThreads) {
                    const int q = it / per, c = it - q * per;
                    const int route = lst[beg + q0 + q];
                    const float4 v = reinterpret_cast<const float4 *>(a.x + static_cast<size_t>(route / a.x_div) * K)[c];
                    uint32_t hp[2], lp[2];  // (element 2i, 2i + 1) as bf16 pairs
                    float sm = 0.0f;
                    split_bf16x2(v.x, v.y, hp[0], lp[0]);
                    split_bf16x2(v.z, v.w, hp[1], lp[1]);
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        sm += bf16_val(hp[i] & 0xffffu) + bf16_val(lp[i] & 0xffffu);
                        sm += bf16_hi_val(hp[i]) + bf16_hi_val(lp[i]);
                    }
                    sm += __shfl_xor(sm, 1, 64);
                    sm += __shfl_xor(sm, 2, 64);
                    sm += __shfl_xor(sm, 4, 64);
                    uint16_t *xp = xpart + static_cast<size_t>(q) * 2 * KX;
                    reinterpret_cast<uint2 *>(xp)[c] = make_uint2(hp[0], hp[1]);
                    reinterpret_cast<uint2 *>(xp + KX)[c] = make_uint2(lp[0], lp[1]);
                    if ((c & 7) == 0) xsum[q * nblk + (c >> 3)] = sm;
                }
            } else {
                // one thread per (route, block, t): the 8 values of slot vector t (the tpb threads of a
                // block are consecutive lanes, and the item count is a multiple of tpb)
                const int per = nblk * F::tpb;
                for (int it = tid; it < nq * per; it += kSThreads) {
                    const int q = it / per, rem = it - q * per, blk = rem / F::tpb, t = rem - blk * F::tpb;
                    const int route = lst[beg + q0 + q];
                    const float4 *xr = reinterpret_cast<const float4 *>(
                        a.x + static_cast<size_t>(route / a.x_div) * K + blk * 32);
                    float xe[8];
                    const float4 u = xr[t];
                    xe[0] = u.x; xe[1] = u.y; xe[2] = u.z; xe[3] = u.w;
                    if constexpr (FMT != T_Q8_0) {
                        const float4 u2 = xr[4 + t];
                        xe[4] = u2.x; xe[5] = u2.y; xe[6] = u2.z; xe[7] = u2.w;
                    }
                    uint32_t hb[8], lb[8];
                    float sm = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        if (FMT == T_Q8_0 && i >= 4) {
                            // 16x, exactly 16 times the parts of x
                            hb[i] = bf16_rne(16.0f * bf16_val(hb[i - 4]));
                            lb[i] = bf16_rne(16.0f * bf16_val(lb[i - 4]));
                        } else {
                            hb[i] = bf16_rne(xe[i]);
                            lb[i] = bf16_rne(xe[i] - bf16_val(hb[i]));
                            sm += bf16_val(hb[i]) + bf16_val(lb[i]);
                        }
                    }
#pragma unroll
                    for (int m = 1; m < F::tpb; m <<= 1) sm += __shfl_xor(sm, m, 64);
                    uint4 *dst = slots + static_cast<size_t>(q) * 2 * PS + blk * F::tpb + t;
                    dst[0] = make_uint4(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16), hb[4] | (hb[5] << 16),
                                        hb[6] | (hb[7] << 16));
                    dst[PS] = make_uint4(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16), lb[4] | (lb[5] << 16),
                                         lb[6] | (lb[7] << 16));
                    if (t == 0) xsum[q * nblk + blk] = sm;
                }
            }
            for (int pt0 = lt0;;) {
                if (tid == 0) next_step = kSWaves;
                __syncthreads();  // staging (and the previous piece's outputs) done

                while (cur.s < nsteps) {
                    int claimed = 0;
                    if (lane == 0) claimed = atomicAdd(&next_step, 1);
                    const Pos nxt = at(__builtin_amdgcn_readfirstlane(claimed));
                    Raw nb;
                    load(nb, nxt);
                    process(buf, cur, nq);
                    buf = nb;
                    cur = nxt;
                }
                __syncthreads();

                // the piece's outputs: chunk partials summed in chunk order, consecutive threads on
                // consecutive rows of one route
                for (int i = tid; i < nq * nrows; i += kSThreads) {
                    const int q = i / nrows, lr = i - q * nrows;
                    const float *pq = partial + static_cast<size_t>(q) * nchunk * pstride + lr;
                    float v0 = 0.0f, v1 = 0.0f;
                    for (int ch = 0; ch < nchunk; ++ch) {
                        v0 += pq[ch * pstride];
                        if constexpr (SW) v1 += pq[(static_cast<size_t>(NQ) * nchunk + ch) * pstride];
                    }
                    const int route = lst[beg + q0 + q];
                    a.out[static_cast<size_t>(route) * a.rows + r0 + lr] = SW ? v0 / (1.0f + expf(-v0)) * v1 : v0;
                }
                pt0 += a.piece;
                if (pt0 >= lt1) break;
                set_piece(pt0);
                cur = at(wave);
                load(buf, cur);
            }
            // the next pass rewrites the staging area, last read before the barrier above, and the
            // partials only after its own first barrier
        }
    }
}

struct UpArgs {
    const uint8_t *wg, *wu;
    size_t eb, rb;       // expert and row bytes (gate and up alike)
    const float *x;      // [tokens, K]
    Groups gr;
    float *act;          // [R, ffn]
    int ffn, K, k;       // k = routes per token
};

// Q4_K gate/up of one expert for its routes: 4 waves x 16 rows, kGroup x vectors per pass.
__global__ __launch_bounds__(256) void up_kernel(const UpArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int e = blockIdx.x;
    const int beg = a.gr.offset[e], cnt = a.gr.offset[e + 1] - beg;
    if (cnt == 0) return;  // uniform per workgroup
    const int K = a.K, nsb = K / 256;
    uint16_t *xpart = reinterpret_cast<uint16_t *>(smem);                      // [kGroup][2][K]
    float *xsum = reinterpret_cast<float *>(smem + kGroup * 4 * static_cast<size_t>(K));  // [kGroup][K/32]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int row = min(blockIdx.y * 64 + wave * 16 + n, a.ffn - 1);
    const uint8_t *rg = a.wg + static_cast<size_t>(e) * a.eb + static_cast<size_t>(row) * a.rb;
    const uint8_t *ru = a.wu + static_cast<size_t>(e) * a.eb + static_cast<size_t>(row) * a.rb;
    const ScaleDecoder dec(g);
    const bool a_active = (n >> 2) == g;
    const bool a_high = (n >> 1) & 1;
    const int a_part = n & 1;

    for (int q0 = 0; q0 < cnt; q0 += kGroup) {
        const int nq = min(kGroup, cnt - q0);
        // stage the x vectors of this pass's routes: bf16 hi / lo and sums per 32 (as the GEMV)
        __syncthreads();
        for (int q = 0; q < kGroup; ++q) {
            const int route = a.gr.list[beg + min(q0 + q, cnt - 1)];
            const float4 *xs = reinterpret_cast<const float4 *>(a.x + static_cast<size_t>(route / a.k) * K);
            uint16_t *xp = xpart + static_cast<size_t>(q) * 2 * K;
            for (int i0 = 0; i0 < K / 4; i0 += 256) {  // K / 4 is a multiple of 64: whole waves
                const int i = i0 + tid;
                const float4 v = xs[min(i, K / 4 - 1)];
                const float xe[4] = {v.x, v.y, v.z, v.w};
                uint32_t hb[4], lb[4];
                float sm = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    hb[c] = bf16_rne(xe[c]);
                    lb[c] = bf16_rne(xe[c] - bf16_val(hb[c]));
                    sm += bf16_val(hb[c]) + bf16_val(lb[c]);
                }
                sm += __shfl_xor(sm, 1, 64);
                sm += __shfl_xor(sm, 2, 64);
                sm += __shfl_xor(sm, 4, 64);
                if (i < K / 4) {
                    reinterpret_cast<uint2 *>(xp)[i] = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
                    reinterpret_cast<uint2 *>(xp + K)[i] = make_uint2(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16));
                    if ((i & 7) == 0) xsum[q * (K / 32) + (i >> 3)] = sm;
                }
            }
        }
        __syncthreads();

        float accg[kGroup], accu[kGroup];
#pragma unroll
        for (int q = 0; q < kGroup; ++q) accg[q] = accu[q] = 0.0f;
        for (int sb = 0; sb < nsb; ++sb) {
            const uint8_t *pg = rg + static_cast<size_t>(sb) * 144, *pu = ru + static_cast<size_t>(sb) * 144;
            const u32x4 hg = ld16(pg), ag = ld16(pg + 16 + 32 * g), bg = ld16(pg + 32 + 32 * g);
            const u32x4 hu = ld16(pu), au = ld16(pu + 16 + 32 * g), bu = ld16(pu + 32 + 32 * g);
            const uint32_t qg[8] = {ag.x, ag.y, ag.z, ag.w, bg.x, bg.y, bg.z, bg.w};
            const uint32_t qu[8] = {au.x, au.y, au.z, au.w, bu.x, bu.y, bu.z, bu.w};
            u32x4 Bg[8], Bu[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                Bg[t] = weights_operand(qg[t]);
                Bu[t] = weights_operand(qu[t]);
            }
            // per-lane scales of sub-blocks 2g, 2g+1 of both matrices
            uint32_t scg, mg, scu, mu;
            dec(hg.y, hg.z, hg.w, scg, mg);
            dec(hu.y, hu.z, hu.w, scu, mu);
            const float dg = f16_bits_to_f32(hg.x & 0xffffu), dmg = f16_bits_to_f32(hg.x >> 16);
            const float du = f16_bits_to_f32(hu.x & 0xffffu), dmu = f16_bits_to_f32(hu.x >> 16);
#pragma unroll
            for (int q = 0; q < kGroup; ++q) {
                if (q >= nq) break;  // uniform
                const uint16_t *xp = xpart + static_cast<size_t>(q) * 2 * K;
                uint32_t dw[16];
                if (a_active) {
                    const uint4 *src = reinterpret_cast<const uint4 *>(xp + a_part * K + sb * 256 + (n >> 1) * 32);
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const uint4 v = src[c];
                        dw[4 * c] = v.x; dw[4 * c + 1] = v.y; dw[4 * c + 2] = v.z; dw[4 * c + 3] = v.w;
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 16; ++c) dw[c] = 0u;
                }
                f32x4 Dg = {0.0f, 0.0f, 0.0f, 0.0f}, Du = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    u32x4 ao;
                    ao.x = a_high ? 0u : dw[2 * t];
                    ao.y = a_high ? 0u : dw[2 * t + 1];
                    ao.z = a_high ? dw[2 * t] : 0u;
                    ao.w = a_high ? dw[2 * t + 1] : 0u;
                    Dg = mfma(ao, Bg[t], Dg);
                    Du = mfma(ao, Bu[t], Du);
                }
                const float2 xs = *reinterpret_cast<const float2 *>(xsum + q * (K / 32) + sb * 8 + 2 * g);
                auto epi = [&](const f32x4 &D, float dd, float dm, uint32_t sc, uint32_t mn, float acc) {
                    acc = fmaf(dd * static_cast<float>(sc & 0xffu), (D[0] + D[1]) - 128.0f * xs.x, acc);
                    acc = fmaf(dd * static_cast<float>((sc >> 8) & 0xffu), (D[2] + D[3]) - 128.0f * xs.y, acc);
                    acc = fmaf(-dm * static_cast<float>(mn & 0xffu), xs.x, acc);
                    return fmaf(-dm * static_cast<float>((mn >> 8) & 0xffu), xs.y, acc);
                };
                accg[q] = epi(Dg, dg, dmg, scg, mg, accg[q]);
                accu[q] = epi(Du, du, dmu, scu, mu, accu[q]);
            }
        }
        const int orow = blockIdx.y * 64 + wave * 16 + n;
#pragma unroll
        for (int q = 0; q < kGroup; ++q) {
            float gq = accg[q], uq = accu[q];
            gq += __shfl_xor(gq, 16, 64);
            gq += __shfl_xor(gq, 32, 64);
            uq += __shfl_xor(uq, 16, 64);
            uq += __shfl_xor(uq, 32, 64);
            if (q < nq && g == 0 && orow < a.ffn) {
                const int route = a.gr.list[beg + q0 + q];
                a.act[static_cast<size_t>(route) * a.ffn + orow] = gq / (1.0f + expf(-gq)) * uq;
            }
        }
    }
}

struct DownArgs {
    const uint8_t *w;
    size_t eb, rb;
    const float *act;    // [R, ffn]
    Groups gr;
    float *yr;           // [R, hidden] per-route results
    int hidden, ffn;
};

// Waves take hidden rows of one expert (64 per workgroup); each row is decoded once per pass and
// dotted with kGroup activations.
template <int T>
__global__ __launch_bounds__(256) void down_kernel(const DownArgs a) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    const int e = blockIdx.x;
    const int beg = a.gr.offset[e], cnt = a.gr.offset[e + 1] - beg;
    if (cnt == 0) return;
    const int lane = threadIdx.x & 63;
    const int h_end = min(a.hidden, (blockIdx.y + 1) * 64);
    for (int h = blockIdx.y * 64 + (threadIdx.x >> 6); h < h_end; h += 4)  // whole waves
    for (int q0 = 0; q0 < cnt; q0 += kGroup) {
        const uint8_t *row = a.w + static_cast<size_t>(e) * a.eb + static_cast<size_t>(h) * a.rb;
        const int nq = min(kGroup, cnt - q0);
        const float *xr[kGroup];
#pragma unroll
        for (int q = 0; q < kGroup; ++q)
            xr[q] = a.act + static_cast<size_t>(a.gr.list[beg + min(q0 + q, cnt - 1)]) * a.ffn;
        float acc[kGroup] = {};
        for (int i = lane; i < a.ffn; i += 64) {
            const float wv = block_value<T>(row + (i / BE) * BB, i % BE);
#pragma unroll
            for (int q = 0; q < kGroup; ++q) acc[q] = fmaf(wv, xr[q][i], acc[q]);
        }
#pragma unroll
        for (int q = 0; q < kGroup; ++q) {
            const float v = wave_sum(acc[q]);
            if (q < nq && lane == 0) a.yr[static_cast<size_t>(a.gr.list[beg + q0 + q]) * a.hidden + h] = v;
        }
    }
}

// out[t, h] += sum over t's routes in order of fmaf(yr, w, .), skipping invalid experts.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ yr, const int *__restrict__ ids,
                                                      const float *__restrict__ rw, float *__restrict__ out,
                                                      int tokens, int k, int hidden, int E) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<int64_t>(tokens) * hidden) return;
    const int t = static_cast<int>(i / hidden), h = static_cast<int>(i % hidden);
    float total = 0.0f;
    for (int r = 0; r < k; ++r) {
        const int route = t * k + r, e = ids[route];
        if (e < 0 || e >= E) continue;
        total = fmaf(yr[static_cast<size_t>(route) * hidden + h], rw[route], total);
    }
    out[i] += total;
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

using plan::kMaxLds;

// The static LDS of one streaming-kernel instantiation, as compiled (cost prefix, scan totals,
// zero operands, step counter), read once; kMaxLds if it cannot be read, so no plan takes it.
template <int FMT, int NQ, bool SW, bool GRP>
size_t stream_static_lds() {
    static const size_t v = [] {
        hipFuncAttributes fa{};
        return hipFuncGetAttributes(&fa, reinterpret_cast<const void *>(&stream_kernel<FMT, NQ, SW, GRP>)) == hipSuccess
                   ? fa.sharedSizeBytes
                   : kMaxLds;
    }();
    return v;
}

// A streaming launch: one workgroup per CU, routes per pass, and the tiles whose partials fit in
// LDS at once (qlin_plan.hpp); not ok when no pass of 2 or 4 routes fits, so the per-element
// kernels take the call.
using StreamPlan = plan::Stream;

template <int FMT, bool SW, bool GRP = false>
StreamPlan stream_plan(int rows, int K, int E, int R) {
    using F = StepFmt<FMT>;
    const plan::StreamFmt f{F::ce, FMT == T_Q4_K, F::tpb};
    return plan::stream(f, SW, rows, K, E, R, device_info().cu_count, stream_static_lds<FMT, 4, SW, GRP>(),
                        stream_static_lds<FMT, 2, SW, GRP>());
}

template <int FMT, int NQ, bool SW, bool GRP>
hipError_t launch_stream_nq(const StreamPlan &p, const StreamArgs &a, hipStream_t s) {
    hipLaunchKernelGGL((stream_kernel<FMT, NQ, SW, GRP>), dim3(p.grid), dim3(kSThreads), p.lds, s, a);
    return hipGetLastError();
}
template <int FMT, bool SW, bool GRP = false>
hipError_t launch_stream(const StreamPlan &p, const StreamArgs &a, hipStream_t s) {
    return p.nq == 4 ? launch_stream_nq<FMT, 4, SW, GRP>(p, a, s) : launch_stream_nq<FMT, 2, SW, GRP>(p, a, s);
}

// The streaming down kernel reads Q5_0 / Q8_0 4-block chunks at dword boundaries (88 and 136 bytes,
// multiples of 4, so every chunk starts 4-aligned once the weights do), and Q4_K super-blocks as
// 16-byte pieces (144 bytes = 9 x 16).
bool down_stream_ok(int type, const uint8_t *w, size_t eb, size_t rb, int ffn) {
    const auto al = [](const void *p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
    if (type == T_Q4_K) return ffn % 256 == 0 && eb % 16 == 0 && rb % 16 == 0 && al(w, 16);
    if (type != T_Q5_0 && type != T_Q8_0) return false;
    return ffn % 128 == 0 && eb % 4 == 0 && rb % 4 == 0 && al(w, 4);
}

}  // namespace

// ---- the scratch of the allocation-free batched entry point --------------------------------------
// Callers that cannot allocate device memory (HIP graph capture, serving loops that forbid it) run
// the batched decode on this array instead of a workspace of their own.  Each GPU the library runs
// on holds its own copy until the process ends, and every call on that GPU shares it: calls that
// overlap on one GPU race.  Nothing in it has to start at zero: each call writes every word of it
// that it reads (group_kernel, or workgroup 0 of the gate/up launch that groups the routes itself,
// the offsets, lists and selected experts; the streaming launches the activations and route
// results they hand on).
namespace {
static __device__ __align__(256) uint8_t scratch[kMoeStaticScratchBytes];
}  // namespace

void *moe_static_scratch() {
    constexpr int kMaxDevices = 64;
    static void *ptrs[kMaxDevices] = {};
    static std::mutex m;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(m);
    if (!ptrs[dev]) {
        // this device's copy of the array (the device is current); host code uses only this address
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        ptrs[dev] = p;
    }
    return ptrs[dev];
}

size_t moe_grouped_workspace(int tokens, int k, int n_experts, int ffn, int hidden) {
    const size_t R = static_cast<size_t>(tokens) * k;
    return align256((n_experts + 1) * sizeof(int)) + align256(R * sizeof(int)) +
           align256(n_experts * sizeof(int4)) + align256(sizeof(int)) + align256(R * ffn * sizeof(float)) +
           align256(R * hidden * sizeof(float));
}

bool moe_grouped_shape_ok(int n_experts, int64_t routes) {
    return n_experts <= kMaxExperts && routes < (int64_t{1} << kRouteBits);
}

bool moe_grouped_up_ok(int type, const uint8_t *wg, const uint8_t *wu, size_t eb, size_t rb, const float *x, int K,
                       int ffn, int E, int R) {
    const auto al = [](const void *p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
    if (type != T_Q4_K || K % 256 || rb % 16 || eb % 16 || !al(wg, 16) || !al(wu, 16) || !al(x, 16)) return false;
    return stream_plan<T_Q4_K, true>(ffn, K, E, R).ok || static_cast<size_t>(kGroup) * (4 * K + K / 8) <= kMaxLds;
}

hipError_t moe_grouped(int gu_type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t g_rb, int d_type,
                       const uint8_t *wd, size_t d_eb, size_t d_rb, int E, int ffn, int K, int hidden,
                       const float *x, const int *ids, const float *rw, void *ws, float *out, int tokens, int k,
                       hipStream_t s, const MoeRouter *router, RouteCombine *defer, const SharedUp *shared) {
    (void)gu_type;  // Q4_K (moe_grouped_up_ok)
    const int R = tokens * k;
    if (R == 0 || hidden == 0) return hipSuccess;
    if (router) {
        ids = router->ids;
        rw = router->w;
    }
    uint8_t *p = static_cast<uint8_t *>(ws);
    Groups gr;
    gr.offset = reinterpret_cast<int *>(p);
    p += align256((E + 1) * sizeof(int));
    gr.list = reinterpret_cast<int *>(p);
    p += align256(static_cast<size_t>(R) * sizeof(int));
    gr.seg = reinterpret_cast<int4 *>(p);
    p += align256(static_cast<size_t>(E) * sizeof(int4));
    gr.nsel = reinterpret_cast<int *>(p);
    p += align256(sizeof(int));
    float *act = reinterpret_cast<float *>(p);
    p += align256(static_cast<size_t>(R) * ffn * sizeof(float));
    float *yr = reinterpret_cast<float *>(p);

    // The gate/up streaming launch groups the routes itself when they fit its LDS arrays and its
    // staging area holds the ids; otherwise group_kernel writes the groups first.
    // With router logits and at most 64 experts it routes as well (its LDS then also holds each wave's
    // logits); otherwise the router runs first, as its own launch.
    StreamPlan up = R <= kFuseRoutes && E <= kFuseExperts ? stream_plan<T_Q4_K, true, true>(ffn, K, E, R)
                                                          : StreamPlan{};
    const size_t ids_lds = static_cast<size_t>((R + 15) & ~15) * sizeof(int);
    const bool grp = up.ok && up.lds >= ids_lds;
    const bool route_here = router && grp && E <= 64 && up.lds >= ids_lds + kSWaves * kRouteWaveFloats * sizeof(float);
    if (router && !route_here) {
        const hipError_t e = router_topk(router->logits, router->ids, router->w, tokens, E, k, router->scaling, s);
        if (e != hipSuccess) return e;
    }
    if (!grp) {
        hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, s, ids, R, E, gr);
        up = stream_plan<T_Q4_K, true>(ffn, K, E, R);
    }
    if (up.ok) {
        StreamArgs ua{wg,  wu,  g_eb, g_rb,   x,         k,          gr.list, gr.seg,
                      gr.nsel, act, ffn, K, K / 256, (ffn + 15) / 16, up.piece};
        ua.ids = ids;
        ua.R = R;
        ua.ne = E;
        ua.gr = gr;
        if (route_here) {
            ua.logits = router->logits;
            ua.scaling = router->scaling;
            ua.ids_out = router->ids;
            ua.w_out = router->w;
        }
        // the shared experts' SwiGLU as the first tile of workgroups 0 .. (one 16-token tile, one
        // shared tile per workgroup at most, its partials in the dynamic LDS)
        const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
        const int sh_tiles = shared ? (shared->rows + 15) / 16 : 0;
        const int per_wg = std::max(1, std::min(QLIN_SHARED_TILES, kSharedMaxTiles));
        if (shared && shared->rows > 0 && tokens <= 16 && (sh_tiles + per_wg - 1) / per_wg <= up.grid &&
            shared->rb % 16 == 0 && al16(shared->wg) && al16(shared->wu) &&
            up.lds >= std::max(per_wg * kSharedPartBytes, static_cast<size_t>(tokens) * (K + 4) * sizeof(float))) {
            ua.sh_wg = shared->wg;
            ua.sh_wu = shared->wu;
            ua.sh_rb = shared->rb;
            ua.sh_act = shared->act;
            ua.sh_rows = shared->rows;
            ua.sh_tokens = tokens;
            ua.sh_cost = kSharedStageCost + per_wg * kSharedTileCost;
            ua.sh_per_wg = per_wg;
            if (shared->done) *shared->done = true;
        }
        const hipError_t e = grp ? launch_stream<T_Q4_K, true, true>(up, ua, s) : launch_stream<T_Q4_K, true>(up, ua, s);
        if (e != hipSuccess) return e;
    } else {
        const UpArgs ua{wg, wu, g_eb, g_rb, x, gr, act, ffn, K, k};
        const size_t lds = static_cast<size_t>(kGroup) * (4 * K + K / 8);
        hipLaunchKernelGGL(up_kernel, dim3(E, (ffn + 63) / 64), dim3(256), lds, s, ua);
    }

    StreamPlan dn;
    if (down_stream_ok(d_type, wd, d_eb, d_rb, ffn)) {
        if (d_type == T_Q5_0) dn = stream_plan<T_Q5_0, false>(hidden, ffn, E, R);
        else if (d_type == T_Q8_0) dn = stream_plan<T_Q8_0, false>(hidden, ffn, E, R);
        else dn = stream_plan<T_Q4_K, false>(hidden, ffn, E, R);
    }
    if (dn.ok) {
        const int nchunk = ffn / (d_type == T_Q4_K ? 256 : 128);
        StreamArgs da{wd,      wd, d_eb,   d_rb, act,    1,                  gr.list, gr.seg,
                      gr.nsel, yr, hidden, ffn,  nchunk, (hidden + 15) / 16, dn.piece};
        da.ne = E;
        const hipError_t e = d_type == T_Q5_0   ? launch_stream<T_Q5_0, false>(dn, da, s)
                             : d_type == T_Q8_0 ? launch_stream<T_Q8_0, false>(dn, da, s)
                                                : launch_stream<T_Q4_K, false>(dn, da, s);
        if (e != hipSuccess) return e;
    } else {
        const DownArgs da{wd, d_eb, d_rb, act, gr, yr, hidden, ffn};
        const dim3 dgrid(E, (hidden + 63) / 64);
        switch (d_type) {
            case T_Q5_0: hipLaunchKernelGGL(down_kernel<T_Q5_0>, dgrid, dim3(256), 0, s, da); break;
            case T_Q8_0: hipLaunchKernelGGL(down_kernel<T_Q8_0>, dgrid, dim3(256), 0, s, da); break;
            case T_Q4_K: hipLaunchKernelGGL(down_kernel<T_Q4_K>, dgrid, dim3(256), 0, s, da); break;
            case T_Q6_K: hipLaunchKernelGGL(down_kernel<T_Q6_K>, dgrid, dim3(256), 0, s, da); break;
            default: return hipErrorInvalidValue;
        }
    }
    if (defer) {
        *defer = RouteCombine{yr, ids, rw, k, E};
        return hipGetLastError();
    }
    const int64_t outs = static_cast<int64_t>(tokens) * hidden;
    hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>((outs + 255) / 256)), dim3(256), 0, s, yr, ids, rw,
                       out, tokens, k, hidden, E);
    return hipGetLastError();
}

}  // namespace qlin

// qlin_mfma_gemv.hip -- decode GEMV (m == 1) of Q4_K, Q4_0 and Q8_0 weights on the matrix cores, gfx950.
//
// Computes y[o] = sum_k w(o, k) x[k] (reference quant_gemv_kernel / quant_gemv_add_kernel,
// AI/codes/local-llm/src/backend/cuda/ops/kernel.cu:1192-1244) for up to four matrices sharing x
// (their rows form one concatenated index space), or the fused SwiGLU act[o] = g/(1+exp(-g))*u of a
// gate/up pair (quant_swiglu_kernel, kernel.cu:1289-1328).  For one matrix it can also leave each
// workgroup's greedy pick of its outputs (the argmax rule of kernel.cu:3531-3592) for
// pick_pairs_kernel, which reduces them: an output head and its argmax without a scan of the logits.
//
// Why matrix cores for a GEMV.  Without packed FP32 a CU retires about one wave64 VALU instruction
// per clock, and decoding a Q4_K weight plus an f32 multiply-add costs about three of them per
// weight: the VALU would need as long as HBM takes to deliver the bytes.  Here the multiply-adds
// run on v_mfma_f32_16x16x32_bf16 and the VALU only builds operands (about one instruction per
// weight) and applies the per-sub-block scales.
//
// Exactness.  A nibble q becomes the bf16 value 128 + q, exactly, with one v_perm_b32 and one
// v_and_or_b32 per two weights.  x is split as hi = bf16(x), lo = bf16(x - hi), so hi + lo equals x
// to within 2^-18 |x|; products are exact and accumulate in f32.  The 128 offset is removed in the
// epilogue with the sub-block sums X = sum(hi + lo).
//
// Q4_K, Q4_0 and Q8_0 with a short x (at most 2 float4s per thread, e.g. K = 3584) run on the int8
// matrix cores instead (v_mfma_i32_16x16x64_i8, half the MFMAs and about a third less VALU per step): per 32
// elements x = 2^e (d1 + d2/128 + d3/16384) with int8 digits in [-64, 64] and max|x| < 2^(e+6), so
// each element is represented to within 2^(e-15) < 2^-21 of its block's largest |x|; the stored
// integers (nibbles, Q8_0 bytes) are the int8 B operand as they are, and every digit's dot is exact
// in int32 (Q4_0's q - 8 leaves with the block sums, as the bf16 form's 128 offset does).  A long x (the down
// projection) keeps the bf16 form, whose staging costs about half.
//
// Operands of one MFMA (16 weight rows n, K = 32; lane l supplies row or column l % 16 and the
// eight k-slots 8*(l/16) .. 8*(l/16)+7, the same slots in A and B):
//   B (weights): lane (n, g = l/16) takes dword t of sub-block pair g of its row -- 4 low nibbles
//     (sub-block 2g, elements 4t..4t+3) and the 4 high nibbles of the same bytes (sub-block 2g+1).
//   A (x): row i = 2*j + part holds part (hi or lo) of sub-block j, non-zero only in the slots that
//     carry sub-block j -- a block-diagonal operand, so that after the 8 MFMAs of a super-block
//     (t = 0..7) D[2j + part][n] is the complete dot of sub-block j for row n.
//   D: lane (g, n) holds rows 4g..4g+3 = both parts of sub-blocks 2g and 2g+1 of row n, which is
//     exactly the pair whose 6-bit scale and min the lane decodes for the epilogue
//       acc += d*sc*(D_j - 128 X_j) - dmin*m*X_j.
//
// Other formats on the same machinery (a step covers 16 rows x one chunk; "sub-block" j below is
// the D-row pair of 32 weights that share one x slice and one scale):
//   Q4_0 (chunk = 8 blocks of 18 B, kernel.cu-free ggml layout): lane group g holds blocks 2g and
//     2g+1; MFMA t carries bytes 4(t%4).. of block 2g + t/4, whose low nibbles are elements 4(t%4)+e
//     and high nibbles elements 16+4(t%4)+e, so the x operand of a block fills both halves of its
//     4 MFMAs.  y += d (D - 136 X)  (q - 8, and the 128 offset).
//   Q8_0 (chunk = 4 blocks of 34 B, kernel.cu:1178-1185): q + 128 = 16 h + l splits each int8
//     weight into two nibbles, so block g becomes the nibble pair of a Q4_K sub-block pair with the
//     same x slice in both; y += d (D_l + 16 D_h - 2304 X).
//   Q6_K (chunk = one 210 B super-block, kernel.cu:1122-1156; int8 matrix cores only): lane group
//     g = 2h + s takes positions 16s..16s+15 of all four 32-element column groups c of half h (ql
//     bytes 64h + 16s and + 32, qh bytes 128 + 32h + 16s, so no byte is read by two lane groups);
//     MFMA c carries column group c, one 16-element scale group, with the 6-bit u itself as B;
//     the x sums are kept per 16; y += d sum_c sc (s_x D_c - 32 X16).
//   Q5_0 (chunk = 4 blocks of 22 B, kernel.cu:1159-1175; int8 matrix cores only): lane group g
//     decodes block g, q = nibble | (bit e of qh) << 4 as the int8 B operand; y += d (D - 16 X).
//   Their blocks are only 2-byte aligned, so each lane loads the dword-aligned window around its
//     bytes (16-byte loads on dword boundaries, which run at the rate of aligned ones; off a dword
//     boundary they are much slower) and realigns it in registers.
//
// Routed experts (the per-token MoE, TensorTool.cpp:271-336 with kernel.cu:1340-1385, 2253-2287):
// route r's weights are expert ids[r]'s.  The gate/up SwiGLU of k routes is the SwiGLU over k * ffn
// concatenated rows whose row pointers come from the ids; the down projection of k routes is one
// GEMV over the routes' activations laid end to end (chunk c of a row belongs to route c / cpr),
// and each row adds its route dots in route order, fmaf(dot_r, w_r, total), as the reference does.
//
// Work decomposition.  One workgroup per CU; workgroup b of G owns the 16-row tiles b, b + G, ...,
// so that the workgroups sweep one region of the weights together.  Its work is the flat sequence
// of steps (tile, matrix, super-block), in memory order; the waves claim the steps one at a time
// from an LDS counter, so the workgroup reads one compact window that slides along its tiles
// (waves with separate contiguous ranges each open their own window, and HBM serves many scattered
// windows measurably slower), and no wave is left with a backlog at the end.
// A wave loads the step it will compute next while it computes the current one, and parks each
// step's 16 row sums in LDS; they are added in super-block order at the end (deterministic) and
// only then is y written.
#include <cstddef>
#include <type_traits>

#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "qlin_mfma.hpp"
#include "qlin_plan.hpp"

namespace qlin {
namespace {

#ifndef QLIN_MFMA_WAVES
#define QLIN_MFMA_WAVES 16
#endif
// Waves per workgroup of the SwiGLU pair.  With bf16 operands 12 was 3-6% faster than 16 on the
// 2 x [18944, 3584] pair; with the int8 operands 16 is (15.6 against 16.1 us).
#ifndef QLIN_MFMA_SW_WAVES
#define QLIN_MFMA_SW_WAVES 16
#endif
constexpr int waves_for(bool swiglu) { return swiglu ? QLIN_MFMA_SW_WAVES : QLIN_MFMA_WAVES; }
constexpr int threads_for(bool swiglu) { return 64 * waves_for(swiglu); }
#ifndef QLIN_MFMA_DEPTH
// Steps in flight per wave while one is computed.  2 (a ring of three buffers) measured 9% slower
// over the decode step than 1: more outstanding requests per CU serve worse on this memory system.
#define QLIN_MFMA_DEPTH 1
#endif
// The same for the routed launches: 2 measured slower there too (per-token MoE at DeepSeek-V2-Lite's
// shape: SwiGLU 9.8 -> 11.0 us, down 11.9 -> 12.2 us).
#ifndef QLIN_MFMA_ROUTED_DEPTH
#define QLIN_MFMA_ROUTED_DEPTH 1
#endif
#ifndef QLIN_MFMA_LONG_DEPTH
#define QLIN_MFMA_LONG_DEPTH 1
#endif
// Equal rows per workgroup where whole tiles would leave some with one tile more (1), or whole
// tiles only (0)
#ifndef QLIN_MFMA_EVEN
#define QLIN_MFMA_EVEN 1
#endif
// Workgroup b of G takes 16-row tiles b, b + G, b + 2G, ... (1), so that all workgroups sweep one
// region of the weights together, rather than a contiguous slice each (0): 1.6% faster over the
// decode step (gate/up and lm_head, the launches with several tiles per workgroup).
#ifndef QLIN_MFMA_INTERLEAVE
#define QLIN_MFMA_INTERLEAVE 1
#endif
// Q4_K on the int8 matrix cores: 0 never, 1 the SwiGLU pair, 2 every launch, 3 launches whose
// threads stage at most 2 float4s of x.  3 is the fastest: the digit staging costs about twice the
// bf16 one, which the long x of a down projection (K = 18944) does not repay.
#ifndef QLIN_MFMA_I8
#define QLIN_MFMA_I8 3
#endif
#ifndef QLIN_MFMA_FINAL_UNROLL
#define QLIN_MFMA_FINAL_UNROLL 4  // batches the final per-row sum's LDS reads (same order of adds)
#endif
#ifndef QLIN_MFMA_FINAL_SPLIT
#define QLIN_MFMA_FINAL_SPLIT 8  // lanes per row in the final sum of rows of many chunks (1: one thread)
#endif
#ifndef QLIN_MFMA_MATMAJOR
#define QLIN_MFMA_MATMAJOR 1  // SwiGLU steps: 1 = all gate tiles, then all up tiles; 0 = tile-major
#endif
using plan::kMaxLds;
using plan::kXPad;
constexpr int kMaxXr = 10;              // float4 loads of x per thread: K <= 40 * threads

// Weights per step chunk of one row, and its bytes.
template <int FMT> struct Chunk;
template <> struct Chunk<T_Q4_K> { static constexpr int elems = 256, bytes = 144; };
template <> struct Chunk<T_Q4_0> { static constexpr int elems = 256, bytes = 144; };
template <> struct Chunk<T_Q8_0> { static constexpr int elems = 128, bytes = 136; };
template <> struct Chunk<T_Q5_0> { static constexpr int elems = 128, bytes = 88; };
template <> struct Chunk<T_Q6_K> { static constexpr int elems = 256, bytes = 210; };
// Elements per x sum kept in LDS.
template <int FMT> constexpr int kSumElems = FMT == T_Q6_K ? 16 : 32;


// The kernel argument block.  Each 64-byte line of it that a launch reads is a scalar-cache miss at the
// start of every wave: the fields every launch reads come first, then one union of the fields only the
// plain launches read and those only the routed launches read, so a plain launch reads 3 lines and a
// routed one 4 (the workgroup count is passed here rather than read from the implicit arguments that
// follow the block).  Adding 24 bytes to the earlier, flat block moved the implicit arguments into a
// fifth line and cost the plain launches 0.2-0.3 us each; this layout took the decode step from
// 1.1008 ms (the flat block before those bytes) to 1.0974 ms: q/k/v and o gained 0.25 and 0.08 us, while
// the down projection, whose instructions are the same but for the argument offsets, lost 0.2 us for a
// reason not found (the common fields keep their earlier order; padding the block back to its earlier
// size did not change it).
struct MfmaArgs {
    const uint8_t *w[kMaxStreamMats];
    float *y[kMaxStreamMats];
    int row_end[kMaxStreamMats];
    int nmat;
    size_t row_bytes;
    const float *x;
    int nsb;      // chunks per row
    int total;    // concatenated rows (SwiGLU: rows of each of gate and up)
    int add;
    // Workgroup b owns rows_q rows (+1 for b < rows_r), and a step index c splits as
    // tile = mulhi(c, nsb_magic) with nsb_magic = ceil(2^32 / nsb), exact while c * nsb < 2^32
    // (nsb = 1: tile = c, as 2^32 does not fit).  The host does these divisions, so the waves start
    // their loads without a 64-bit division sequence on the scalar unit (several hundred cycles per
    // wave, and the 16 waves of a CU share that unit).
    int rows_q, rows_r;
    uint32_t nsb_magic;
    int grid;  // workgroups in the launch
    union {
        // routed launches (first: value-initialisation zeroes the whole union)
        struct {
            // Route r's weights start at w[.] + ids[r] * eb (a negative id: no expert, its loads read
            // expert 0 and its results are dropped).  SwiGLU: route r owns concatenated rows
            // [r * route_rows, (r + 1) * route_rows); otherwise chunks [r * cpr, (r + 1) * cpr) of every
            // row, weighted by rw[r].  The magics are ceil(2^32 / divisor), exact as nsb_magic (0:
            // divisor 1).
            const int *ids;
            const float *rw;
            size_t eb;
            int routes, route_rows, cpr;
            uint32_t route_magic, cpr_magic;
            // SwiGLU from router logits (logits non-null, ne <= 64): wave 0 picks the token's routes
            // (route_token_rank) instead of reading ids, and workgroup 0 writes the picks and their
            // weights (times scaling) to ids_out and rw_out for the down launch.
            int ne;
            const float *logits;
            float scaling;
            int *ids_out;
            float *rw_out;
            // SwiGLU: the last sh_routes routes are not experts but consecutive route_rows-row blocks
            // of the shared gate and up matrices sh_w0 and sh_w1 (same format and row stride): the
            // shared experts in the same launch.  They are not routed and never empty.
            const uint8_t *sh_w0, *sh_w1;
            int sh_routes;
        };
        // plain launches
        struct {
            // RMSNorm of x fused into the staging (norm_w non-null): x is used as
            // x[j] * rsqrt(mean x^2 + eps) * w[j], w bf16 (norm_type 0) or f16 (1), plus one if one_plus
            const uint16_t *norm_w;
            int norm_type, norm_one_plus;
            float norm_eps;
            // The greedy pick of the outputs (one matrix, no add): workgroup b writes the largest of its
            // rows' outputs and its row, the lowest row among equals (NaN never wins, (-inf, 0) when
            // nothing beats -inf), to amax_v[b] and amax_i[b]; a later launch reduces the pairs by the
            // same rule, which gives the argmax of the whole output whatever the order.
            float *amax_v;
            int *amax_i;
        };
    };
};
static_assert(offsetof(MfmaArgs, amax_i) + sizeof(int *) <= 192, "the plain launches' fields fill 3 lines");
static_assert(sizeof(MfmaArgs) <= 256, "the routed launches' fields fill 4 lines");

// (v, i) becomes (v2, i2) when that is larger, or equal at a lower index: the argmax's rule
__device__ __forceinline__ void pick_better(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

constexpr int kMaxRoutes = 16;  // routes of one routed launch (top-k of one token)

// What every wave needs before its first requests (x, the first matrix, the row stride and the
// step decomposition), passed as leading scalar kernel arguments: gfx950 preloads those into SGPRs
// when it launches the wave, so the first x and weight requests wait for no scalar load of the
// argument block, which follows them (its fields: MfmaArgs).
// (13 dwords: at most 14 are preloaded, beside the argument segment's own pointer, in the 16 user SGPRs.)
struct Lead {
    const float *x;
    const uint8_t *w0;
    size_t rb;
    int nsb, total, rows_q, rows_r;
    uint32_t magic;
    int grid, nmat;
};

// The argument arrays, copied into registers once: indexing the kernel-argument struct with a
// per-lane value would compile to vector loads of the argument segment, whose completion shares the
// vmcnt counter with the weight stream and forces a full drain of the prefetched loads.
struct Mats {
    const uint8_t *w[kMaxStreamMats];
    float *y[kMaxStreamMats];
    int end[kMaxStreamMats];
    int nmat;
    __device__ Mats(const MfmaArgs &a, const Lead &ld) : nmat(ld.nmat) {
#pragma unroll
        for (int i = 0; i < kMaxStreamMats; ++i) {
            w[i] = i ? a.w[i] : ld.w0;
            y[i] = a.y[i];
            end[i] = a.row_end[i];
        }
    }
    // matrix of concatenated row gr and the row within it, by compare-and-select
    __device__ __forceinline__ void locate(int gr, const uint8_t *&wp, float *&yp, int &local) const {
        wp = w[0];
        yp = y[0];
        local = gr;
        if (nmat == 1) return;  // uniform
#pragma unroll
        for (int i = 1; i < kMaxStreamMats; ++i) {
            const bool past = i < nmat && gr >= end[i - 1];
            wp = past ? w[i] : wp;
            yp = past ? y[i] : yp;
            local = past ? gr - end[i - 1] : local;
        }
    }
};


// A lane's raw bytes of one step: Q4_K the 16-byte header and 32 bytes of nibbles; the 32-weight
// formats the 9 (Q5_0: 6) dwords from the one at or 2 bytes before the lane's blocks; Q6_K on the
// int8 matrix cores three 16-byte pieces and 12 scale bytes, on the bf16 ones 48-byte windows.
struct Raw {
    uint32_t w[27];
};
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }


// XR: float4 loads of x per thread (K/4 <= XR * kThreads).  ROUTED: the routed-expert forms (a.ids).
template <int FMT, bool SWIGLU, int XR, bool ROUTED = false>
__global__ __launch_bounds__(threads_for(SWIGLU)) void mfma_gemv_kernel(const float *lx, const uint8_t *lw0, size_t lrb,
                                                                       int lnsb, int ltotal, int lrows_q, int lrows_r,
                                                                       uint32_t lmagic, int lgrid, int lnmat,
                                                                       const MfmaArgs a) {
    const Lead ld{lx, lw0, lrb, lnsb, ltotal, lrows_q, lrows_r, lmagic, lgrid, lnmat};
    constexpr int kWaves = waves_for(SWIGLU), kThreads = threads_for(SWIGLU);
    constexpr int NW = SWIGLU ? 2 : 1;  // matrices per output row (gate, up)
    constexpr int CE = Chunk<FMT>::elems, CB = Chunk<FMT>::bytes;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int XS = kSumElems<FMT>;
    const int nsb = ld.nsb, K = nsb * CE;
    // I8 (Q4_K): x as three base-128 int8 digits per element in planes [3][K] and (scale, sum of x)
    // per 32 elements, in no more LDS than the bf16 layout takes (3 KP + K/4 against 4 KX + K/8 bytes).
    // Q5_0 has only this form.
    constexpr bool I8 = FMT == T_Q5_0 || FMT == T_Q6_K ||
                        ((FMT == T_Q4_K || FMT == T_Q4_0 || FMT == T_Q8_0) &&
                         (QLIN_MFMA_I8 == 2 || (QLIN_MFMA_I8 == 1 && SWIGLU) || (QLIN_MFMA_I8 == 3 && XR <= 2)));
    constexpr bool K32 = FMT == T_Q8_0 || FMT == T_Q5_0;  // 128-weight chunks: lane group g, block g
    // The parts (digit planes) are kXPad bytes longer than K values: an A operand read gathers
    // the same offset of 2 (3) of them, which then fall in different LDS banks.
    const int KX = K + kXPad / 2, KP = K + kXPad;                  // bf16 part, int8 plane strides
    uint16_t *xpart = reinterpret_cast<uint16_t *>(smem);          // [2][KX] bf16: hi, lo
    float *xsum = reinterpret_cast<float *>(smem + 4 * KX);        // [K/XS] sum(hi + lo) per XS elements
    float *partial = xsum + K / XS;                                // [rows][NW][nsb]
    int8_t *planes = reinterpret_cast<int8_t *>(smem);                    // I8: [3][KP]
    float *sxp = reinterpret_cast<float *>(smem + 3 * static_cast<size_t>(KP));  // I8: [K/32][2] (scale, sum)

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int bid = blockIdx.x;
#if QLIN_MFMA_INTERLEAVE
    // 16-row tiles bid, bid + G, bid + 2G, ... (G workgroups): all workgroups sweep one region
    // (rows_q, rows_r here count tiles: tiles / G and tiles % G, from the host).  rows_r < 0: every
    // workgroup takes rows_q such tiles and then -rows_r consecutive rows of the rows past them
    // (workgroup b from row 16 rows_q G + b (-rows_r)), a last tile with fewer than 16 rows: equal
    // bytes in every workgroup, where whole tiles leave some workgroups with one tile more.
    const int G = ld.grid;
    const bool even = ld.rows_r < 0;  // uniform
    const int ntl = even ? ld.rows_q + 1 : ld.rows_q + (bid < ld.rows_r ? 1 : 0);
    const int nrows = even  ? 16 * ld.rows_q - ld.rows_r
                      : ntl ? (ntl - 1) * 16 + min(16, ld.total - 16 * (bid + (ntl - 1) * G))
                            : 0;
    const int tail0 = 16 * ld.rows_q * (G - 1) - ld.rows_r * bid;  // global row of local row lr in the last tile: tail0 + lr
    auto grow = [&](int lr) {  // global row of local row lr
        return even && lr >= 16 * ld.rows_q ? tail0 + lr : 16 * (bid + (lr >> 4) * G) + (lr & 15);
    };
#else
    const int rb = bid * ld.rows_q + min(bid, ld.rows_r);
    const int nrows = ld.rows_q + (bid < ld.rows_r ? 1 : 0);
    auto grow = [&](int lr) { return rb + lr; };
#endif
    // The workgroup's work is the flat sequence of steps (16-row tile, matrix, super-block), which
    // is also the order of the bytes in memory; the waves claim them in that order, so that at any
    // time the workgroup reads one compact window of its rows.
    const int nsteps = (nrows + 15) / 16 * NW * nsb;
    const int n = lane & 15, g = lane >> 4;
    const ScaleDecoder dec(g);
    const Mats mats(a, ld);

    // bf16 A operand (Q4_K, Q4_0, Q8_0): every MFMA gives lane group g's 8 slots to 8
    // consecutive weights of one 32-weight unit ("sub-block" j of the D rows).  MFMAs 0..3 carry
    // unit 2g, 4..7 unit 2g+1:
    //   Q4_K: the low / high nibbles of the pair's bytes 8t..8t+7 (sub-blocks 2g, 2g+1);
    //   Q4_0: blocks 2g, 2g+1, each as low nibbles of bytes 0..7, 8..15, then high nibbles of the same;
    //   Q8_0: block g's bytes 8t..8t+7 as the l (units 2g) and h (unit 2g+1) nibbles of q + 128.
    // Row n of A (part n & 1 of unit n >> 1) then holds x in all 8 slots of MFMAs 0..3 when
    // n >> 1 == 2g, of MFMAs 4..7 when n >> 1 == 2g + 1, and zeros otherwise, so each A operand is
    // 16 bytes read from the staged x or from a zero area (stride 0), with no selects.
    const int a_part = n & 1;
    // I8 A operand: row n is digit n & 3 (3: none) of the 32-element units of lane group g = n >> 2:
    // Q4_K sub-blocks 2g (MFMAs 0, 1) and 2g + 1 (2, 3), Q4_0 blocks 2g and 2g + 1 likewise (their 4
    // x 16 bytes are 64 consecutive plane bytes), Q8_0 block g (MFMAs 0, 1: 32 bytes)
    const bool i8_on = (n >> 2) == g && (n & 3) < 3;
    // (Q6_K: lane group g's elements of column group c start 128 (g >> 1) + 32 c + 16 (g & 1) into the
    // chunk)
    const int8_t *a8 = planes + (n & 3) * KP +
                       (K32 ? 32 * g : FMT == T_Q6_K ? (g >> 1) * 128 + (g & 1) * 16 : 64 * g);  // when i8_on
    __shared__ u32x4 s_zero[4];
    const uint8_t *a_lo, *a_hi;
    int a_lo_st, a_hi_st;
    {
        const int j = n >> 1;
        // the unit's 32 x values: Q8_0 units 2b and 2b+1 are both block b
        const int xo = FMT == T_Q8_0 ? (j >> 1) * 32 : j * 32;
        const uint8_t *xb = reinterpret_cast<const uint8_t *>(xpart + a_part * KX + xo);
        const uint8_t *zb = reinterpret_cast<const uint8_t *>(s_zero);
        a_lo = j == 2 * g ? xb : zb;
        a_lo_st = j == 2 * g ? 2 * CE : 0;
        a_hi = j == 2 * g + 1 ? xb : zb;
        a_hi_st = j == 2 * g + 1 ? 2 * CE : 0;
    }

    // A step: tw = tile * NW + matrix, sb = super-block; s = its index in the flat sequence.
    struct Pos {
        int s, tw, sb;
        const uint8_t *rp;  // this lane's bytes of the step's chunk
    };
    // Routed launches: the routes' experts (and down weights), read before the first weight load
    __shared__ int s_ids[ROUTED ? kMaxRoutes : 1];
    __shared__ float s_rw[ROUTED ? kMaxRoutes : 1];
    // route of a concatenated SwiGLU row / of a down chunk
    auto route_of = [&](int v, int d, uint32_t magic) {
        return d == 1 ? v : static_cast<int>(__umulhi(static_cast<uint32_t>(v), magic));
    };
    // expert e's weights (a negative id reads expert 0, whose results are dropped)
    auto expert = [&](const uint8_t *w, int r) { return w + static_cast<size_t>(max(s_ids[r], 0)) * a.eb; };
    const int ntiles = (nrows + 15) / 16;
    auto split_tw = [&](int tw, int &tile, int &which) {
        if constexpr (NW == 1) {
            tile = tw;
            which = 0;
        } else if (QLIN_MFMA_MATMAJOR) {
            which = tw >= ntiles;
            tile = tw - which * ntiles;
        } else {
            tile = tw >> 1;
            which = tw & 1;
        }
    };
    // Position of step s (wave-uniform).  Past the last step the position is the last step (valid
    // addresses, loads never consumed), so that no load needs a branch.
    auto at = [&](int s) {
        Pos p;
        p.s = s;
        const int c = min(s, nsteps - 1);
        p.tw = nsb == 1 ? c : static_cast<int>(__umulhi(static_cast<uint32_t>(c), ld.magic));
        p.sb = c - p.tw * nsb;
        int tile, which;
        split_tw(p.tw, tile, which);
        const int gr = grow(min(tile * 16 + n, nrows - 1));
        if constexpr (ROUTED && SWIGLU) {
            // route of this lane's concatenated row (the 16 rows of a tile may span two routes)
            const int r = route_of(gr, a.route_rows, a.route_magic);
            const int row = gr - r * a.route_rows;
            const int rs = r - (a.routes - a.sh_routes);  // >= 0: a block of the shared matrices
            const uint8_t *base =
                rs >= 0 ? (which ? a.sh_w1 : a.sh_w0) + static_cast<size_t>(rs) * a.route_rows * ld.rb
                        : expert(which ? mats.w[1] : mats.w[0], r);
            p.rp = base + static_cast<size_t>(row) * ld.rb + static_cast<size_t>(p.sb) * CB;
        } else if constexpr (ROUTED) {
            // chunk sb of the concatenated activations is chunk cl of route r (wave-uniform)
            const int r = route_of(p.sb, a.cpr, a.cpr_magic);
            const int cl = p.sb - r * a.cpr;
            p.rp = expert(mats.w[0], r) + static_cast<size_t>(gr) * ld.rb + static_cast<size_t>(cl) * CB;
        } else if constexpr (SWIGLU) {
            p.rp = (which ? mats.w[1] : mats.w[0]) + static_cast<size_t>(gr) * ld.rb +
                   static_cast<size_t>(p.sb) * CB;
        } else {
            const uint8_t *wp;
            float *yp;
            int local;
            mats.locate(gr, wp, yp, local);
            p.rp = wp + static_cast<size_t>(local) * ld.rb + static_cast<size_t>(p.sb) * CB;
        }
        return p;
    };
    auto load = [&](Raw &st, const Pos &p) {
        const uint8_t *q = p.rp;
        if constexpr (FMT == T_Q4_K) {
            const u32x4 h = ld16(q), qa = ld16(q + 16 + 32 * g), qb = ld16(q + 32 + 32 * g);
            st.w[0] = h.x; st.w[1] = h.y; st.w[2] = h.z; st.w[3] = h.w;
            st.w[4] = qa.x; st.w[5] = qa.y; st.w[6] = qa.z; st.w[7] = qa.w;
            st.w[8] = qb.x; st.w[9] = qb.y; st.w[10] = qb.z; st.w[11] = qb.w;
        } else if constexpr (FMT == T_Q6_K && I8) {
            // Lane group g = 2h + s takes positions 16s .. 16s + 15 of all four 32-element column groups c
            // of half h: ql bytes o = 64h + 16s (c = 0, 2: low and high nibbles) and o + 32 (c = 1, 3), qh
            // bytes c0 = 128 + 32h + 16s (bits 2c, 2c + 1), and the half's scales sc[8h + 2c + s]; no byte
            // is read by two lane groups.  Rows start on dwords (row_bytes a multiple of 4), so even
            // super-blocks start on a dword and odd ones 2 bytes past one.  Every load is dword-aligned:
            // the three pieces and 12 bytes at 192 + 8h, all from 2 bytes before them in an odd
            // super-block.  The 12 bytes hold the half's 8 scales and, for h = 1, d; at their end an even
            // super-block's h = 1 lanes read the 2 bytes after it, which exist: the next super-block's, or
            // the row's padding (a packed row has an even count, so its last super-block is odd; with an
            // odd count row_bytes is at least 2 past the packed size).  An odd super-block's pieces then
            // lack their last 2 bytes: the first dword that another lane group of the row loaded (process).
            const int h = g >> 1, o = 64 * h + 16 * (g & 1), c0 = 128 + 32 * h + 16 * (g & 1);
            const uint8_t *qa = q - ((__builtin_amdgcn_readfirstlane(p.sb) & 1) ? 2 : 0);
            const u32x4 la = ld16_a4(qa + o), lb = ld16_a4(qa + o + 32), qh = ld16_a4(qa + c0);
            st.w[0] = la.x; st.w[1] = la.y; st.w[2] = la.z; st.w[3] = la.w;
            st.w[5] = lb.x; st.w[6] = lb.y; st.w[7] = lb.z; st.w[8] = lb.w;
            st.w[10] = qh.x; st.w[11] = qh.y; st.w[12] = qh.z; st.w[13] = qh.w;
            uint32_t sv[3];
            ld12_a4(qa + 192 + 8 * h, sv);
            st.w[15] = sv[0];
            st.w[16] = sv[1];
            st.w[17] = sv[2];
        } else if constexpr (FMT == T_Q5_0) {
            // block g = bytes [22g, 22g+22), from the dword at or 2 bytes before it (6 dwords, inside
            // the chunk for every g)
            const uint8_t *b = q + 22 * g - 2 * (g & 1);
            ld_dwords_a4<6>(b, st.w);
        } else {
            // Q4_0: blocks 2g, 2g+1 = bytes [36g, 36g+36).  Q8_0: block g = bytes [34g, 34g+34), read
            // from the dword at or 2 bytes before it.
            const uint8_t *b = FMT == T_Q4_0 ? q + 36 * g : q + 34 * g - 2 * (g & 1);
            ld_dwords_a4<9>(b, st.w);
        }
    };

    if (nsteps == 0) {  // uniform per workgroup
        if (!ROUTED && !SWIGLU && a.amax_v && tid == 0) {
            a.amax_v[bid] = -INFINITY;
            a.amax_i[bid] = 0;
        }
        return;
    }

    // x first: requested before any weight load of the workgroup.  Every load is branch-free, which
    // lets the compiler wait for exactly the loads a step consumes and keep the younger ones in
    // flight.
    float4 xv[XR];
#pragma unroll
    for (int r = 0; r < XR; ++r) xv[r] = reinterpret_cast<const float4 *>(ld.x)[min(tid + r * kThreads, K / 4 - 1)];
    if (!ROUTED && a.norm_w) {  // uniform
        // the norm weights are requested with x; the sum of squares over the workgroup (each thread
        // its float4s in order, then the wave, then the waves in order)
        uint32_t nw[XR][4];
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            const uint16_t *np = a.norm_w + 4 * min(tid + r * kThreads, K / 4 - 1);
#pragma unroll
            for (int c = 0; c < 4; ++c) nw[r][c] = np[c];
        }
        __shared__ float s_ss[kWaves];
        float ss = 0.0f;
#pragma unroll
        for (int r = 0; r < XR; ++r)
            if (tid + r * kThreads < K / 4)
                ss += xv[r].x * xv[r].x + xv[r].y * xv[r].y + xv[r].z * xv[r].z + xv[r].w * xv[r].w;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (lane == 0) s_ss[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) tot += s_ss[w];
        const float inv = rsqrtf(tot / static_cast<float>(K) + a.norm_eps);
        auto nv = [&](uint32_t b) {
            const float v = a.norm_type == 0 ? __builtin_bit_cast(float, b << 16)
                                             : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
            return a.norm_one_plus ? v + 1.0f : v;
        };
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            xv[r].x = xv[r].x * inv * nv(nw[r][0]);
            xv[r].y = xv[r].y * inv * nv(nw[r][1]);
            xv[r].z = xv[r].z * inv * nv(nw[r][2]);
            xv[r].w = xv[r].w * inv * nv(nw[r][3]);
        }
    }
    if constexpr (ROUTED) {
        // the routes' experts (and down weights): every weight address depends on them.  A route that
        // nothing below sets stays -1 (no expert: its loads read expert 0 and its results are dropped);
        // these writes and every later one are wave 0's, so they land in program order.
        if (tid < kMaxRoutes) s_ids[tid] = -1;
        bool routed_here = false;
        if constexpr (SWIGLU) {
            if (a.logits) {  // uniform: wave 0 routes the token (the only live wave: its LDS alone)
                __shared__ __attribute__((aligned(16))) float s_rex[64];
                route_token_rank(wave == 0, a.logits, a.ne, a.routes - a.sh_routes, a.scaling, s_rex,
                                 [&](int r, int e, float w) {
                                     s_ids[r] = e;
                                     if (blockIdx.x == 0) {
                                         a.ids_out[r] = e;
                                         a.rw_out[r] = w;
                                     }
                                 });
                routed_here = true;
            }
        }
        if (!routed_here && tid < a.routes - a.sh_routes) {
            s_ids[tid] = a.ids[tid];
            if constexpr (!SWIGLU) s_rw[tid] = a.rw[tid];
        }
        if (tid >= a.routes - a.sh_routes && tid < a.routes) s_ids[tid] = 0;  // the shared blocks
        __syncthreads();
    }

    auto stage_x_i8 = [&]() {
        // x as three int8 digit planes and (scale, sum) per 32 elements (x_digits4)
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            const int i = tid + r * kThreads;
            uint32_t p1, p2, p3;
            float sc, sm, sm16;
            x_digits4(xv[r], p1, p2, p3, sc, sm, sm16);
            if (i < K / 4) {
                reinterpret_cast<uint32_t *>(planes)[i] = p1;
                reinterpret_cast<uint32_t *>(planes + KP)[i] = p2;
                reinterpret_cast<uint32_t *>(planes + 2 * KP)[i] = p3;
                if constexpr (FMT == T_Q6_K) {
                    // scales per 32 [K/32], then x sums per 16 [K/16]
                    if ((i & 7) == 0) sxp[i >> 3] = sc;
                    if ((i & 3) == 0) sxp[K / 32 + (i >> 2)] = sm16;
                } else {
                    if ((i & 7) == 0) reinterpret_cast<float2 *>(sxp)[i >> 3] = make_float2(sc, sm);
                }
            }
        }
    };
    auto stage_x = [&]() {
        if constexpr (I8) {
            stage_x_i8();
            return;
        }
        // bf16 hi / lo parts and the per-sub-block sums of hi + lo
#pragma unroll
        for (int r = 0; r < XR; ++r) {
            const int i = tid + r * kThreads;
            const float xe[4] = {xv[r].x, xv[r].y, xv[r].z, xv[r].w};
            uint32_t hp[2], lp[2];  // (element 2e, element 2e + 1) as bf16 pairs
            float sm = 0.0f;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                split_bf16x2(xe[2 * e], xe[2 * e + 1], hp[e], lp[e]);
                sm += bf16_val(hp[e] & 0xffffu) + bf16_val(lp[e] & 0xffffu);
                sm += bf16_hi_val(hp[e]) + bf16_hi_val(lp[e]);
            }
            // the threads of a 16- or 32-element group are consecutive lanes, and K is a multiple of
            // 128, so a group is entirely below K/4 or entirely above it
            sm += __shfl_xor(sm, 1, 64);
            sm += __shfl_xor(sm, 2, 64);
            if constexpr (XS == 32) sm += __shfl_xor(sm, 4, 64);
            if (i < K / 4) {
                reinterpret_cast<uint2 *>(xpart)[i] = make_uint2(hp[0], hp[1]);
                reinterpret_cast<uint2 *>(xpart + KX)[i] = make_uint2(lp[0], lp[1]);
                if ((i & (XS / 4 - 1)) == 0) xsum[i / (XS / 4)] = sm;
            }
        }
    };

    // Steps are handed out dynamically, in memory order: wave w starts with step w, then takes the
    // next unclaimed one from an LDS counter each time it prefetches.  The waves of a CU are not
    // served equally (a wave that starts late stays behind), so a fixed share per wave leaves the
    // workgroup waiting for its slowest wave; claiming on demand ends all waves within about one step
    // of each other.
    // DEPTH 2: wave w starts with steps w and w + kWaves, both requested before the x staging
    // (Q6_K's 27-dword steps would spill with three buffers)
    constexpr int DEPTH = ROUTED && FMT != T_Q6_K ? QLIN_MFMA_ROUTED_DEPTH
                          : (!ROUTED && XR > 2 && FMT != T_Q6_K) ? QLIN_MFMA_LONG_DEPTH : QLIN_MFMA_DEPTH;
    __shared__ int next_step;
    if (tid == 0) next_step = DEPTH * kWaves;
    if (tid < 4) s_zero[tid] = u32x4{0u, 0u, 0u, 0u};
    Pos cur = at(wave);
    Raw buf;
    load(buf, cur);
    Pos second = cur;
    Raw bb;
    if constexpr (DEPTH == 2) {
        second = at(wave + kWaves);
        load(bb, second);
    }
    stage_x();
    __syncthreads();

    u32x4 aop[8];

    // One step: the 16 rows' dots with super-block sb, parked in LDS (each (row, matrix, sb) slot is
    // written by exactly one step; a global store here would share vmcnt with the weight stream).
    auto process = [&](const Raw &cur, const Pos &p) {
        if constexpr (I8) {
            // The int8 matrix cores: B takes the stored integers themselves (Q4_K / Q4_0 nibbles, Q8_0
            // bytes), A the x digits; D rows 4g + r are digit r's dots of a unit, exact in int32.
            const i32x4 *pa = reinterpret_cast<const i32x4 *>(i8_on ? a8 + p.sb * CE : reinterpret_cast<const int8_t *>(s_zero));
            constexpr uint32_t M = 0x0f0f0f0fu;
            // the 8 dwords of this lane's stored integers: Q4_K the pair's 32 bytes; Q4_0 blocks 2g,
            // 2g + 1 (16 bytes each); Q8_0 block g's 32 bytes
            uint32_t src[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
            if constexpr (FMT == T_Q6_K || FMT == T_Q5_0) {
                // decoded below
            } else if constexpr (FMT == T_Q4_K) {
#pragma unroll
                for (int k = 0; k < 8; ++k) src[k] = cur.w[4 + k];
            } else if constexpr (FMT == T_Q4_0) {
#pragma unroll
                for (int k = 0; k < 4; ++k) src[k] = __builtin_amdgcn_alignbyte(cur.w[k + 1], cur.w[k], 2);
#pragma unroll
                for (int k = 0; k < 4; ++k) src[4 + k] = cur.w[5 + k];
            } else {
                // odd blocks' bytes start at the second dword, even ones' 2 bytes into the first: one
                // byte permute per dword with a per-lane selector
                const uint32_t sel = (g & 1) ? 0x07060504u : 0x05040302u;
#pragma unroll
                for (int k = 0; k < 8; ++k) src[k] = __builtin_amdgcn_perm(cur.w[k + 1], cur.w[k], sel);
            }
            auto nib = [&](int k0, int sh) {
                return i32x4{static_cast<int>((src[k0] >> sh) & M), static_cast<int>((src[k0 + 1] >> sh) & M),
                             static_cast<int>((src[k0 + 2] >> sh) & M), static_cast<int>((src[k0 + 3] >> sh) & M)};
            };
            auto digits = [](const i32x4 &d) { return digits_value(d); };
            float r;
            if constexpr (FMT == T_Q6_K) {
                // MFMA c: the 6-bit values u of column group c at the lane group's 16 positions (elements
                // 4t..4t+3 from dword t of the ql and qh pieces), one 16-element scale group.  ODD: the
                // pieces and scales were read from 2 bytes before them (the load's layout).
                // The value of x at lane group g ^ 1 / g ^ 2 of the same row (the swap's first result holds
                // the partner's value in the odd / upper lane groups, its second in the others).  Every
                // lane must run them, so their results are selected after the call, never by a
                // conditional around it: a swap in a branch reads its partners with their lanes off.
                auto from16 = [&](uint32_t x) {
                    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
                    return static_cast<uint32_t>((g & 1) ? r[0] : r[1]);
                };
                auto from32 = [&](uint32_t x) {
                    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
                    return static_cast<uint32_t>((g >> 1) ? r[0] : r[1]);
                };
                auto q6_dot = [&](auto oddc) {
                    constexpr bool ODD = decltype(oddc)::value;
                    const int s = g & 1;
                    uint32_t tail[3] = {0u, 0u, 0u};
                    if constexpr (ODD) {
                        // the dword after each piece's window starts the window of the piece 16 bytes on
                        // (the scales' window after the last qh piece): A of g + 1 or B of g - 1 for the A
                        // pieces (lane group g ^ 1); for B and C the next lane group (g ^ 1 from an even
                        // group, g ^ 3 from an odd one), which gives B or A / C, or C / the h = 0 scales
                        const uint32_t a0 = cur.w[0], b0 = cur.w[5], c0 = cur.w[10], s0w = cur.w[15];
                        tail[0] = from16(s ? a0 : b0);
                        const uint32_t db = s ? b0 : ((g >> 1) ? a0 : c0), dc = g == 0 ? s0w : c0;
                        const uint32_t b1 = from16(db), c1 = from16(dc);
                        const uint32_t b3 = from32(b1), c3 = from32(c1);
                        tail[1] = s ? b3 : b1;
                        tail[2] = s ? c3 : c1;
                    }
                    uint32_t bq[4][4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        uint32_t la = cur.w[t], lb = cur.w[5 + t], qh = cur.w[10 + t];
                        if constexpr (ODD) {
                            la = __builtin_amdgcn_alignbyte(t < 3 ? cur.w[t + 1] : tail[0], cur.w[t], 2);
                            lb = __builtin_amdgcn_alignbyte(t < 3 ? cur.w[6 + t] : tail[1], cur.w[5 + t], 2);
                            qh = __builtin_amdgcn_alignbyte(t < 3 ? cur.w[11 + t] : tail[2], cur.w[10 + t], 2);
                        }
                        bq[0][t] = (la & M) | ((qh << 4) & 0x30303030u);
                        bq[1][t] = (lb & M) | ((qh << 2) & 0x30303030u);
                        bq[2][t] = ((la >> 4) & M) | (qh & 0x30303030u);
                        bq[3][t] = ((lb >> 4) & M) | ((qh >> 2) & 0x30303030u);
                    }
                    auto vec = [](const uint32_t *v) {
                        return i32x4{static_cast<int>(v[0]), static_cast<int>(v[1]), static_cast<int>(v[2]),
                                     static_cast<int>(v[3])};
                    };
                    // A: column group c at +32c bytes (the zero area's lanes read its first 16 bytes)
                    const i32x4 *pq = reinterpret_cast<const i32x4 *>(
                        i8_on ? a8 + p.sb * CE : reinterpret_cast<const int8_t *>(s_zero));
                    const int ast = i8_on ? 2 : 0;
                    const i32x4 d0 = mfma_i8(pq[0], vec(bq[0]), i32x4{0, 0, 0, 0});
                    const i32x4 d1 = mfma_i8(pq[ast], vec(bq[1]), i32x4{0, 0, 0, 0});
                    const i32x4 d2 = mfma_i8(pq[2 * ast], vec(bq[2]), i32x4{0, 0, 0, 0});
                    const i32x4 d3 = mfma_i8(pq[3 * ast], vec(bq[3]), i32x4{0, 0, 0, 0});
                    // the half's scales sc[8h .. 8h + 7] and d: the h = 1 lanes hold d in the last of their
                    // 12 bytes (low half, or high half after the odd super-block's 2-byte shift), the h = 0
                    // lanes take it from the lane group 2 above
                    uint32_t sw0 = cur.w[15], sw1 = cur.w[16];
                    if constexpr (ODD) {
                        sw0 = __builtin_amdgcn_alignbyte(cur.w[16], cur.w[15], 2);
                        sw1 = __builtin_amdgcn_alignbyte(cur.w[17], cur.w[16], 2);
                    }
                    const uint32_t dh = from32(cur.w[17]);
                    const uint32_t dw = (g >> 1) ? cur.w[17] : dh;
                    const uint32_t db = (ODD ? dw >> 16 : dw) & 0xffffu;
                    // x digit scales of the 32-element blocks 8 sb + 4h + c, x sums of the 16-element
                    // groups 16 sb + 8h + 2c + s, weight scales sc[8h + 2c + s]
                    const float4 sx = *reinterpret_cast<const float4 *>(sxp + p.sb * 8 + 4 * (g >> 1));
                    const float *x16 = sxp + K / 32 + p.sb * 16 + 8 * (g >> 1) + s;
                    const uint32_t sa = sw0 >> (8 * s), sb = sw1 >> (8 * s);
                    const float s0 = static_cast<float>(static_cast<int8_t>(sa & 0xffu));
                    const float s1 = static_cast<float>(static_cast<int8_t>((sa >> 16) & 0xffu));
                    const float s2 = static_cast<float>(static_cast<int8_t>(sb & 0xffu));
                    const float s3 = static_cast<float>(static_cast<int8_t>((sb >> 16) & 0xffu));
                    const float dd = f16_bits_to_f32(db);
                    // u - 32: the offset leaves with the 16-element x sums
                    float v = s0 * (sx.x * digits(d0) - 32.0f * x16[0]);
                    v = fmaf(s1, sx.y * digits(d1) - 32.0f * x16[2], v);
                    v = fmaf(s2, sx.z * digits(d2) - 32.0f * x16[4], v);
                    v = fmaf(s3, sx.w * digits(d3) - 32.0f * x16[6], v);
                    return v * dd;
                };
                if (__builtin_amdgcn_readfirstlane(p.sb) & 1)  // a scalar branch: the swaps see every lane
                    r = q6_dot(std::true_type{});
                else
                    r = q6_dot(std::false_type{});
            } else if constexpr (FMT == T_Q8_0) {
                const i32x4 b0 = {static_cast<int>(src[0]), static_cast<int>(src[1]), static_cast<int>(src[2]),
                                  static_cast<int>(src[3])};
                const i32x4 b1 = {static_cast<int>(src[4]), static_cast<int>(src[5]), static_cast<int>(src[6]),
                                  static_cast<int>(src[7])};
                i32x4 de = mfma_i8(pa[0], b0, i32x4{0, 0, 0, 0});
                de = mfma_i8(pa[1], b1, de);
                const float2 sx = *reinterpret_cast<const float2 *>(sxp + 2 * (p.sb * 4 + g));  // s of block g
                const float dq = f16_bits_to_f32((cur.w[0] >> (16 * (g & 1))) & 0xffffu);
                r = dq * (sx.x * digits(de));
            } else if constexpr (FMT == T_Q5_0) {
                // block g from its 6 dwords: d, then qh and qs (2 bytes into the window for even g)
                const bool odd = g & 1;
                const uint32_t qh = odd ? cur.w[1] : __builtin_amdgcn_alignbyte(cur.w[1], cur.w[0], 2);
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t qs = odd ? cur.w[2 + t] : __builtin_amdgcn_alignbyte(cur.w[2 + t], cur.w[1 + t], 2);
                    lo[t] = (qs & M) | (spread4(qh >> (4 * t)) << 4);              // elements 4t .. 4t+3
                    hi[t] = ((qs >> 4) & M) | (spread4(qh >> (16 + 4 * t)) << 4);  // elements 16+4t ..
                }
                const i32x4 b0 = {static_cast<int>(lo[0]), static_cast<int>(lo[1]), static_cast<int>(lo[2]),
                                  static_cast<int>(lo[3])};
                const i32x4 b1 = {static_cast<int>(hi[0]), static_cast<int>(hi[1]), static_cast<int>(hi[2]),
                                  static_cast<int>(hi[3])};
                i32x4 de = mfma_i8(pa[0], b0, i32x4{0, 0, 0, 0});
                de = mfma_i8(pa[1], b1, de);
                const float2 sx = *reinterpret_cast<const float2 *>(sxp + 2 * (p.sb * 4 + g));  // s, X of block g
                const float dq = f16_bits_to_f32((cur.w[0] >> (16 * (g & 1))) & 0xffffu);
                // q - 16: the offset leaves with the block sum
                r = dq * (sx.x * digits(de) - 16.0f * sx.y);
            } else {
                // MFMAs 0, 1 carry unit 2g (Q4_K: low nibbles of bytes 0..15, 16..31; Q4_0: block 2g's
                // low, then high nibbles), 2, 3 unit 2g + 1
                const i32x4 b0 = nib(0, 0);
                const i32x4 b1 = FMT == T_Q4_K ? nib(4, 0) : nib(0, 4);
                const i32x4 b2 = FMT == T_Q4_K ? nib(0, 4) : nib(4, 0);
                const i32x4 b3 = nib(4, 4);
                i32x4 de = mfma_i8(pa[0], b0, i32x4{0, 0, 0, 0});
                de = mfma_i8(pa[1], b1, de);
                i32x4 dq = mfma_i8(pa[2], b2, i32x4{0, 0, 0, 0});
                dq = mfma_i8(pa[3], b3, dq);
                const float4 sx = *reinterpret_cast<const float4 *>(sxp + p.sb * 16 + 4 * g);  // s, X of 2g, 2g + 1
                const float dote = sx.x * digits(de), doto = sx.z * digits(dq);
                if constexpr (FMT == T_Q4_K) {
                    uint32_t scp, mp;
                    dec(cur.w[1], cur.w[2], cur.w[3], scp, mp);
                    const float dd = f16_bits_to_f32(cur.w[0] & 0xffffu);
                    const float dmin = f16_bits_to_f32(cur.w[0] >> 16);
                    r = dd * static_cast<float>(scp & 0xffu) * dote;
                    r = fmaf(dd * static_cast<float>((scp >> 8) & 0xffu), doto, r);
                    r = fmaf(-dmin * static_cast<float>(mp & 0xffu), sx.y, r);
                    r = fmaf(-dmin * static_cast<float>((mp >> 8) & 0xffu), sx.w, r);
                } else {
                    // q - 8: the offset leaves with the block sums
                    const float d0 = f16_bits_to_f32(cur.w[0] & 0xffffu), d1 = f16_bits_to_f32(cur.w[4] >> 16);
                    r = d0 * (dote - 8.0f * sx.y);
                    r = fmaf(d1, doto - 8.0f * sx.w, r);
                }
            }
            r = sum_lane_groups(r);
            int tile, which;
            split_tw(p.tw, tile, which);
            const int lr = tile * 16 + n;
            if (g == 0 && lr < nrows) partial[(lr * NW + which) * nsb + p.sb] = r;
            return;
        }
        // A operands of this chunk (x only): the lane's 32 values of its part / sub-block (Q8_0: the
        // block both nibble sub-blocks of the pair come from).
        {
            const u32x4 *pl = reinterpret_cast<const u32x4 *>(a_lo + p.sb * a_lo_st);
            const u32x4 *ph = reinterpret_cast<const u32x4 *>(a_hi + p.sb * a_hi_st);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                aop[t] = pl[t];
                aop[4 + t] = ph[t];
            }
        }
        // the 8 dwords of nibbles this lane feeds to the MFMAs
        uint32_t qv[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
        if constexpr (FMT == T_Q4_0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) qv[k] = __builtin_amdgcn_alignbyte(cur.w[k + 1], cur.w[k], 2);
#pragma unroll
            for (int k = 0; k < 4; ++k) qv[4 + k] = cur.w[5 + k];
        } else if constexpr (FMT == T_Q8_0) {
            const bool odd = g & 1;  // odd blocks start 2 bytes into the first dword
#pragma unroll
            for (int k = 0; k < 8; ++k)
                qv[k] = (odd ? cur.w[k + 1] : __builtin_amdgcn_alignbyte(cur.w[k + 1], cur.w[k], 2)) ^ 0x80808080u;
        }
        f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (FMT == T_Q4_0) {
            // block 2g + (t >> 2): low nibbles of bytes 0..7, 8..15 (elements 0..15), then high nibbles
            constexpr uint32_t M = 0x0f0f0f0fu;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t a0 = qv[4 * (t >> 2) + 2 * (t & 1)], a1 = qv[4 * (t >> 2) + 2 * (t & 1) + 1];
                const int sh = 4 * ((t >> 1) & 1);
                d = mfma(aop[t], weights_operand2((a0 >> sh) & M, (a1 >> sh) & M), d);
            }
        } else {
            // Q4_K: the pair's bytes 8t..8t+7 (cur.w[4..11]); Q8_0: block g's (qv): low nibbles, then high
            constexpr uint32_t M = 0x0f0f0f0fu;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int k = 2 * (t & 3), sh = 4 * (t >> 2);
                const uint32_t a0 = FMT == T_Q4_K ? cur.w[4 + k] : qv[k];
                const uint32_t a1 = FMT == T_Q4_K ? cur.w[5 + k] : qv[k + 1];
                d = mfma(aop[t], weights_operand2((a0 >> sh) & M, (a1 >> sh) & M), d);
            }
        }
        float r;
        if constexpr (FMT == T_Q4_K) {
            const float2 xs = *reinterpret_cast<const float2 *>(xsum + p.sb * 8 + 2 * g);
            uint32_t scp, mp;
            dec(cur.w[1], cur.w[2], cur.w[3], scp, mp);
            const float dd = f16_bits_to_f32(cur.w[0] & 0xffffu);
            const float dmin = f16_bits_to_f32(cur.w[0] >> 16);
            const float dsc0 = dd * static_cast<float>(scp & 0xffu);
            const float dsc1 = dd * static_cast<float>((scp >> 8) & 0xffu);
            const float dm0 = dmin * static_cast<float>(mp & 0xffu);
            const float dm1 = dmin * static_cast<float>((mp >> 8) & 0xffu);
            r = dsc0 * ((d[0] + d[1]) - 128.0f * xs.x);
            r = fmaf(dsc1, (d[2] + d[3]) - 128.0f * xs.y, r);
            r = fmaf(-dm0, xs.x, r);
            r = fmaf(-dm1, xs.y, r);
        } else if constexpr (FMT == T_Q4_0) {
            const float2 xs = *reinterpret_cast<const float2 *>(xsum + p.sb * 8 + 2 * g);
            const float d0 = f16_bits_to_f32(cur.w[0] & 0xffffu), d1 = f16_bits_to_f32(cur.w[4] >> 16);
            r = d0 * ((d[0] + d[1]) - 136.0f * xs.x);
            r = fmaf(d1, (d[2] + d[3]) - 136.0f * xs.y, r);
        } else {
            const float xs = xsum[p.sb * 4 + g];
            const float dq = f16_bits_to_f32((cur.w[0] >> (16 * (g & 1))) & 0xffffu);
            r = dq * (((d[0] + d[1]) + 16.0f * (d[2] + d[3])) - 2304.0f * xs);
        }
        // add the four lane-groups (sub-block pairs), into lanes 0..15
        r = sum_lane_groups(r);
        int tile, which;
        split_tw(p.tw, tile, which);
        const int lr = tile * 16 + n;
        if (g == 0 && lr < nrows) partial[(lr * NW + which) * nsb + p.sb] = r;
    };

    auto claim = [&]() {
        int c = 0;
        if (lane == 0) c = atomicAdd(&next_step, 1);
        return at(__builtin_amdgcn_readfirstlane(c));
    };
    if constexpr (DEPTH == 2) {
    // Two steps in flight while one is computed: a ring of three buffers, unrolled so that no
    // buffer is copied (a loop-carried copy of loaded registers waits for every outstanding load).
    // Claims are monotonic per wave, so once a claimed step is past the end, so are the later ones.
    Pos pa = cur, pb = second;
    for (;;) {
        if (pa.s >= nsteps) break;
        const Pos pc = claim();
        Raw bc;
        load(bc, pc);
        __builtin_amdgcn_sched_barrier(0);
        process(buf, pa);
        if (pb.s >= nsteps) break;
        pa = claim();
        load(buf, pa);
        __builtin_amdgcn_sched_barrier(0);
        process(bb, pb);
        if (pc.s >= nsteps) break;
        pb = claim();
        load(bb, pb);
        __builtin_amdgcn_sched_barrier(0);
        process(bc, pc);
    }
    } else {
    while (cur.s < nsteps) {
        const Pos nxt = claim();
        Raw nb;
        load(nb, nxt);
        __builtin_amdgcn_sched_barrier(0);
        process(buf, cur);
        buf = nb;
        cur = nxt;
    }
    }

    __syncthreads();
    if constexpr (ROUTED && !SWIGLU) {
        // each route's dot in chunk order, one thread per (row, route), parked in the route's first
        // chunk slot; then the routes in route order: out += sum fmaf(dot, w, .)
        const int nq = a.routes, cpr = a.cpr;
        for (int i = tid; i < nrows * nq; i += kThreads) {
            float *pr = partial + (i / nq) * nsb + (i % nq) * cpr;
            float dot = 0.0f;
#pragma unroll 4
            for (int c = 0; c < cpr; ++c) dot += pr[c];
            pr[0] = dot;
        }
        __syncthreads();
        for (int r = tid; r < nrows; r += kThreads) {
            const float *pr = partial + r * nsb;
            float total = 0.0f;
            for (int q = 0; q < nq; ++q)
                if (s_ids[q] >= 0) total = fmaf(pr[q * cpr], s_rw[q], total);
            float *yp = mats.y[0] + grow(r);
            *yp += total;
        }
        return;
    }
    float best_v = -INFINITY;  // the greedy pick over the rows this thread writes (amax_v set)
    int best_i = 0;
    auto write_row = [&](int r, const float (&tot)[NW]) {
        const int gr = grow(r);
        if constexpr (ROUTED && SWIGLU) {  // (the routed down adds its routes above and never gets here)
            // a route without an expert gives 0 (kernel.cu:1340-1385)
            const bool none = s_ids[route_of(gr, a.route_rows, a.route_magic)] < 0;
            mats.y[0][gr] = none ? 0.0f : tot[0] / (1.0f + expf(-tot[0])) * tot[1];
        } else if constexpr (SWIGLU) {
            mats.y[0][gr] = tot[0] / (1.0f + expf(-tot[0])) * tot[1];
        } else {
            const uint8_t *wp;
            float *yp;
            int local;
            mats.locate(gr, wp, yp, local);
            yp[local] = a.add ? yp[local] + tot[0] : tot[0];
            pick_better(best_v, best_i, tot[0], gr);
        }
    };
    // the workgroup's pick: the threads', then the waves' (the rule does not depend on the order)
    auto write_pick = [&]() {
        if constexpr (!ROUTED && !SWIGLU) {
            if (!a.amax_v) return;  // uniform
            __shared__ float s_pv[kWaves];
            __shared__ int s_pi[kWaves];
#pragma unroll
            for (int m = 32; m > 0; m >>= 1) pick_better(best_v, best_i, __shfl_xor(best_v, m, 64), __shfl_xor(best_i, m, 64));
            if (lane == 0) {
                s_pv[wave] = best_v;
                s_pi[wave] = best_i;
            }
            __syncthreads();
            if (tid == 0) {
                for (int w = 1; w < kWaves; ++w) pick_better(best_v, best_i, s_pv[w], s_pi[w]);
                a.amax_v[bid] = best_v;
                a.amax_i[bid] = best_i;
            }
        }
    };
    // Each row's step partials added in a fixed order.  With many chunks, L consecutive lanes share
    // a row, lane j adding partials j, j + L, ..., then a butterfly over the L lanes: a thread alone
    // would wait on nsb dependent LDS reads (74 for a K = 18944 row).
    constexpr int L = QLIN_MFMA_FINAL_SPLIT;
    if (L > 1 && nsb >= 2 * L) {
        const int span = (nrows * L + 63) / 64 * 64;  // whole waves, for the shuffles
        for (int i = tid; i < span; i += kThreads) {
            const int r = i / L, j = i % L;
            const bool live = r < nrows;
            float tot[NW];
#pragma unroll
            for (int q = 0; q < NW; ++q) {
                tot[q] = 0.0f;
                if (live)
                    for (int sb = j; sb < nsb; sb += L) tot[q] += partial[(r * NW + q) * nsb + sb];
#pragma unroll
                for (int m = L / 2; m > 0; m >>= 1) tot[q] += __shfl_xor(tot[q], m, 64);
            }
            if (live && j == 0) write_row(r, tot);
        }
        write_pick();
        return;
    }
    for (int r = tid; r < nrows; r += kThreads) {
        float tot[NW];
#pragma unroll
        for (int q = 0; q < NW; ++q) {
            tot[q] = 0.0f;
#if QLIN_MFMA_FINAL_UNROLL > 1
#pragma unroll QLIN_MFMA_FINAL_UNROLL
#endif
            for (int sb = 0; sb < nsb; ++sb) tot[q] += partial[(r * NW + q) * nsb + sb];
        }
        write_row(r, tot);
    }
    write_pick();
}

using Plan = plan::Gemv;

Plan make_plan(int total, int k, int nsb, bool swiglu, int sum_elems) {
    return plan::gemv(total, k, nsb, swiglu, sum_elems, device_info().cu_count, QLIN_MFMA_INTERLEAVE != 0);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// One instantiation of the kernel, with its own (static) LDS as the compiler laid it out: a plan
// fits when that plus the plan's dynamic LDS is within the CU's 160 KB.
struct Kern {
    const void *fn = nullptr;
    size_t static_lds = kMaxLds;
    unsigned threads = 0;
};
template <int FMT, bool SW, int XR, bool R>
Kern kern() {
    const void *fn = reinterpret_cast<const void *>(&mfma_gemv_kernel<FMT, SW, XR, R>);
    static const size_t lds = [fn] {
        hipFuncAttributes fa{};
        return hipFuncGetAttributes(&fa, fn) == hipSuccess ? fa.sharedSizeBytes : kMaxLds;
    }();
    return Kern{fn, lds, static_cast<unsigned>(threads_for(SW))};
}
// x loads per thread from K; routed launches have at most 4 (K <= 16 * threads)
template <int FMT, bool SW, bool R>
Kern kern_xr(int k) {
    constexpr int kThreads = threads_for(SW);
    const int need = (k / 4 + kThreads - 1) / kThreads;
    if (need <= 1) return kern<FMT, SW, 1, R>();
    if (need <= 2) return kern<FMT, SW, 2, R>();
    if (need <= 4) return kern<FMT, SW, 4, R>();
    if constexpr (!R) {
        if (need <= 6) return kern<FMT, SW, 6, R>();
        if (need <= kMaxXr) return kern<FMT, SW, kMaxXr, R>();
    }
    return Kern{};
}
template <bool SW, bool R>
Kern kern_for(int type, int k) {
    switch (type) {
        case T_Q4_K: return kern_xr<T_Q4_K, SW, R>(k);
        case T_Q4_0: return kern_xr<T_Q4_0, SW, R>(k);
        case T_Q8_0: return kern_xr<T_Q8_0, SW, R>(k);
        case T_Q5_0: return kern_xr<T_Q5_0, SW, R>(k);
        case T_Q6_K: return kern_xr<T_Q6_K, SW, R>(k);
        default: return Kern{};
    }
}
Kern kernel_for(int type, bool swiglu, bool routed, int k) {
    if (routed) return swiglu ? kern_for<true, true>(type, k) : kern_for<false, true>(type, k);
    return swiglu ? kern_for<true, false>(type, k) : kern_for<false, false>(type, k);
}

int chunk_elems(int type) { return type == T_Q8_0 || type == T_Q5_0 ? 128 : 256; }
int sum_elems(int type) { return type == T_Q6_K ? kSumElems<T_Q6_K> : kSumElems<T_Q4_K>; }
bool mfma_type(int type) {
    return type == T_Q4_K || type == T_Q4_0 || type == T_Q8_0 || type == T_Q6_K || type == T_Q5_0;
}
// Q4_K loads 16-byte pieces at 16-byte boundaries; the 32-weight formats and Q6_K load at dword
// boundaries (16-byte loads among them)
size_t weight_align(int type) { return type == T_Q4_K ? 16 : 4; }
uint32_t magic_of(int d) { return d > 1 ? static_cast<uint32_t>(((uint64_t{1} << 32) + d - 1) / d) : 0u; }

// The launch's kernel and plan, or no kernel when the shape does not fit (callers then take the
// per-element kernels).
struct Launch {
    Kern k;
    Plan p;
    bool ok = false;
};
Launch prepare(int type, const MfmaArgs &a, int k, bool swiglu, bool routed) {
    Launch l;
    l.k = kernel_for(type, swiglu, routed, k);
    if (!l.k.fn) return l;
    l.p = make_plan(a.total, k, a.nsb, swiglu, sum_elems(type));
    l.ok = plan::gemv_fits(l.p, l.k.static_lds);
    return l;
}

hipError_t launch(int type, MfmaArgs &a, int k, bool swiglu, bool routed, hipStream_t s, int *grid = nullptr) {
    const Launch l = prepare(type, a, k, swiglu, routed);
    if (!l.ok) return hipErrorInvalidValue;  // the *_ok checks reject these shapes first
    if (grid) *grid = l.p.grid;
    const int units = QLIN_MFMA_INTERLEAVE ? (a.total + 15) / 16 : a.total;  // tiles or rows per workgroup
    a.rows_q = units / l.p.grid;
    a.rows_r = units % l.p.grid;
    // Plain launches with at least two whole tiles per workgroup and a remainder that splits evenly
    // take whole tiles and an equal share of the rest of the rows (the kernel's rows_r < 0): the
    // Qwen2-7B gate/up pair's 1184 tiles left 160 workgroups with 5 tiles and 96 with 4; now each has
    // 4 and 10 rows.
    const int whole = a.total / (16 * l.p.grid), rest = a.total - 16 * whole * l.p.grid;
    if (QLIN_MFMA_INTERLEAVE && QLIN_MFMA_EVEN && !routed && whole >= 2 && rest > 0 && rest % l.p.grid == 0) {
        a.rows_q = whole;
        a.rows_r = -(rest / l.p.grid);
    }
    a.nsb_magic = magic_of(a.nsb);
    a.grid = l.p.grid;
    const float *lx = a.x;
    const uint8_t *lw0 = a.w[0];
    size_t lrb = a.row_bytes;
    int lnsb = a.nsb, ltotal = a.total, lrows_q = a.rows_q, lrows_r = a.rows_r, lgrid = a.grid, lnmat = a.nmat;
    uint32_t lmagic = a.nsb_magic;
    void *args[] = {&lx, &lw0, &lrb, &lnsb, &ltotal, &lrows_q, &lrows_r, &lmagic, &lgrid, &lnmat, &a};
    const hipError_t e = hipLaunchKernel(l.k.fn, dim3(l.p.grid), dim3(l.k.threads), args, l.p.lds, s);
    return e != hipSuccess ? e : hipGetLastError();
}

// The workgroups' greedy picks (amax_v, amax_i of a launch of n workgroups) reduced by one workgroup
// with the same rule: the argmax of the launch's whole output.
constexpr int kPickThreads = 256;
__global__ __launch_bounds__(kPickThreads) void pick_pairs_kernel(const float *__restrict__ pv,
                                                                  const int *__restrict__ pi, int n,
                                                                  int *__restrict__ out_idx) {
    __shared__ float s_v[kPickThreads / 64];
    __shared__ int s_i[kPickThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float v = -INFINITY;
    int idx = 0;
    for (int j = tid; j < n; j += kPickThreads) pick_better(v, idx, pv[j], pi[j]);
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) pick_better(v, idx, __shfl_xor(v, m, 64), __shfl_xor(idx, m, 64));
    if (lane == 0) {
        s_v[wave] = v;
        s_i[wave] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kPickThreads / 64; ++w) pick_better(v, idx, s_v[w], s_i[w]);
        *out_idx = idx;
    }
}

MfmaArgs base_args(int type, size_t rb, const float *x, int k) {
    MfmaArgs a{};
    a.row_bytes = rb;
    a.x = x;
    a.nsb = k / chunk_elems(type);
    return a;
}

MfmaArgs swiglu_routed_args(int type, const uint8_t *wg, const uint8_t *wu, size_t eb, size_t rb, const float *x,
                            const int *ids, float *act, int routes, int ffn, int k) {
    MfmaArgs a = base_args(type, rb, x, k);
    a.w[0] = wg;
    a.w[1] = wu;
    a.y[0] = act;
    a.nmat = 1;
    a.total = routes * ffn;
    a.row_end[0] = a.total;
    a.ids = ids;
    a.eb = eb;
    a.routes = routes;
    a.route_rows = ffn;
    a.route_magic = magic_of(ffn);
    return a;
}

MfmaArgs down_routed_args(int type, const uint8_t *wd, size_t eb, size_t rb, const float *act, const int *ids,
                          const float *rw, float *out, int routes, int hidden, int ffn) {
    MfmaArgs a = base_args(type, rb, act, routes * ffn);
    a.w[0] = wd;
    a.y[0] = out;
    a.nmat = 1;
    a.total = hidden;
    a.row_end[0] = hidden;
    a.ids = ids;
    a.rw = rw;
    a.eb = eb;
    a.routes = routes;
    a.cpr = ffn / chunk_elems(type);
    a.cpr_magic = magic_of(a.cpr);
    return a;
}

}  // namespace

bool mfma_ok(int type, const uint8_t *const *w, int nmat, size_t rb, const float *x, int total, int k, bool swiglu) {
    if (!mfma_type(type)) return false;
    const size_t wal = weight_align(type);
    // whole chunks (Q8_0, Q5_0: 128 weights, the others 256); x is staged as float4s in groups of 8 lanes
    if (nmat < 1 || nmat > kMaxStreamMats || k % chunk_elems(type) || rb % wal || !aligned16(x) || total <= 0)
        return false;
    MfmaArgs a = base_args(type, rb, x, k);
    for (int i = 0; i < nmat; ++i) {
        if (reinterpret_cast<uintptr_t>(w[i]) % wal) return false;
        a.w[i] = w[i];
    }
    a.nmat = nmat;
    a.total = total;
    return prepare(type, a, k, swiglu, false).ok;
}

void set_norm(MfmaArgs &a, const RmsNorm *norm) {
    if (!norm) return;
    a.norm_w = norm->w;
    a.norm_type = norm->type;
    a.norm_one_plus = norm->one_plus;
    a.norm_eps = norm->eps;
}

hipError_t mfma_gemv(int type, const uint8_t *const *w, float *const *y, const int *rows, int nmat, size_t rb,
                     const float *x, int k, bool add, hipStream_t s, const RmsNorm *norm) {
    MfmaArgs a = base_args(type, rb, x, k);
    set_norm(a, norm);
    int total = 0;
    for (int i = 0; i < nmat; ++i) {
        a.w[i] = w[i];
        a.y[i] = y[i];
        total += rows[i];
        a.row_end[i] = total;
    }
    if (total == 0) return hipSuccess;
    a.nmat = nmat;
    a.total = total;
    a.add = add ? 1 : 0;
    return launch(type, a, k, false, false, s);
}

int mfma_gemv_pairs(int type, const uint8_t *w, size_t rb, const float *x, int n, int k) {
    MfmaArgs a = base_args(type, rb, x, k);
    a.w[0] = w;
    a.row_end[0] = n;
    a.nmat = 1;
    a.total = n;
    const Launch l = prepare(type, a, k, false, false);
    return l.ok ? l.p.grid : 0;
}

hipError_t mfma_gemv_argmax(int type, const uint8_t *w, size_t rb, const float *x, float *y, int n, int k,
                            const RmsNorm *norm, float *pairs_v, int *pairs_i, int *out_idx, hipStream_t s) {
    MfmaArgs a = base_args(type, rb, x, k);
    set_norm(a, norm);
    a.w[0] = w;
    a.y[0] = y;
    a.row_end[0] = n;
    a.nmat = 1;
    a.total = n;
    a.amax_v = pairs_v;
    a.amax_i = pairs_i;
    int grid = 0;
    const hipError_t e = launch(type, a, k, false, false, s, &grid);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(pick_pairs_kernel, dim3(1), dim3(kPickThreads), 0, s, pairs_v, pairs_i, grid, out_idx);
    return hipGetLastError();
}

hipError_t mfma_swiglu(int type, const uint8_t *wg, const uint8_t *wu, size_t rb, const float *x, float *act, int ffn,
                       int k, hipStream_t s, const RmsNorm *norm) {
    if (ffn == 0) return hipSuccess;
    MfmaArgs a = base_args(type, rb, x, k);
    set_norm(a, norm);
    a.w[0] = wg;
    a.w[1] = wu;
    a.y[0] = act;
    a.row_end[0] = ffn;
    a.nmat = 1;
    a.total = ffn;
    return launch(type, a, k, true, false, s);
}

bool mfma_routed_ok(int type, bool swiglu, const uint8_t *w0, const uint8_t *w1, size_t eb, size_t rb, const float *x,
                    int routes, int rows, int k) {
    if (!mfma_type(type) || routes < 1 || routes > kMaxRoutes || rows <= 0 || k <= 0) return false;
    const size_t wal = weight_align(type);
    const auto al = [wal](const void *p) { return reinterpret_cast<uintptr_t>(p) % wal == 0; };
    if (k % chunk_elems(type) || rb % wal || eb % wal || !al(w0) || (swiglu && !al(w1)) || !aligned16(x)) return false;
    const uint64_t lim = uint64_t{1} << 32;
    MfmaArgs a;
    if (swiglu) {
        // route_of(gr) for every concatenated row gr < routes * rows
        if (static_cast<uint64_t>(routes) * rows * rows >= lim) return false;
        a = swiglu_routed_args(type, w0, w1, eb, rb, x, nullptr, nullptr, routes, rows, k);
        return prepare(type, a, k, true, true).ok;
    }
    // the down projection: rows = hidden, k = ffn per route; route_of(chunk) for every chunk
    const int cpr = k / chunk_elems(type);
    // Q6_K's load takes a super-block's dword offset (0 or 2) from its step index, which in the routed
    // down counts the routes' chunks end to end: that is the super-block's parity in its row only when a
    // route has an even number of them (an odd one needs a padded row_bytes to pass the checks above)
    if (type == T_Q6_K && cpr % 2) return false;
    if (static_cast<uint64_t>(routes) * cpr * cpr >= lim) return false;
    a = down_routed_args(type, w0, eb, rb, x, nullptr, nullptr, nullptr, routes, rows, k);
    return prepare(type, a, routes * k, false, true).ok;
}

hipError_t mfma_swiglu_routed(int type, const uint8_t *wg, const uint8_t *wu, size_t eb, size_t rb, const float *x,
                              const int *ids, float *act, int routes, int ffn, int k, hipStream_t s,
                              const MoeRouter *router, int n_experts, const uint8_t *sh_wg, const uint8_t *sh_wu,
                              int sh_routes) {
    MfmaArgs a = swiglu_routed_args(type, wg, wu, eb, rb, x, ids, act, routes + sh_routes, ffn, k);
    a.sh_w0 = sh_wg;
    a.sh_w1 = sh_wu;
    a.sh_routes = sh_routes;
    if (router) {
        a.logits = router->logits;
        a.ne = n_experts;
        a.scaling = router->scaling;
        a.ids_out = router->ids;
        a.rw_out = router->w;
    }
    return launch(type, a, k, true, true, s);
}

hipError_t mfma_down_routed(int type, const uint8_t *wd, size_t eb, size_t rb, const float *act, const int *ids,
                            const float *rw, float *out, int routes, int hidden, int ffn, hipStream_t s) {
    MfmaArgs a = down_routed_args(type, wd, eb, rb, act, ids, rw, out, routes, hidden, ffn);
    return launch(type, a, routes * ffn, false, true, s);
}

}  // namespace qlin

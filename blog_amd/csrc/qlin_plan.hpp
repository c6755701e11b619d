// qlin_plan.hpp -- launch planning of the matrix-core streaming kernels: host-only arithmetic, no
// HIP calls, so the same code is checked on the CPU (tests/plan_check.cpp).
//
// A plan gives the workgroup count and the dynamic LDS of a launch.  The kernels' own (static) LDS
// is an input: the callers read it from the compiled kernels (hipFuncGetAttributes), and a plan is
// accepted only when static + dynamic LDS fits the CU's 160 KB.  A shape no plan fits takes the
// per-element kernels instead, so a call that passes validation never fails at launch for LDS.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>

namespace qlin {
namespace plan {

constexpr size_t kMaxLds = 160 * 1024;  // LDS per CU on gfx950
// Padding of each staged x part (bf16 hi or lo, int8 digit plane) past its K values, in bytes: an
// A-operand read gathers one offset of several parts, and a part length that is a multiple of the
// LDS bank row (256 bytes) would put them all in the same banks.  16 bytes (one b128 read) shifts
// each part by 4 banks.  Staging of a route (one x) takes 4K + 2 kXPad bytes as bf16 parts.
constexpr int kXPad = 16;

// The decode GEMV (qlin_mfma_gemv.hip): one workgroup per CU over `total` rows of nsb chunks of
// k / nsb weights.  Dynamic LDS: x in the bf16 layout (4K + 2 kXPad bytes, which the int8 digit
// planes, 3 (K + kXPad) bytes and their sums, never exceed), the x sums (one float per sum_elems elements) and one partial per (row,
// matrix, chunk) of the workgroup's rows.  interleave: workgroup b takes 16-row tiles b, b + G, ...
struct Gemv {
    int grid = 0;
    size_t lds = 0;
    bool magic_exact = false;  // every step index c of a workgroup has c * nsb < 2^32
};
inline Gemv gemv(int total, int k, int nsb, bool swiglu, int sum_elems, int cu_count, bool interleave) {
    Gemv p;
    p.grid = std::max(1, std::min(cu_count, (total + 15) / 16));
    const int rows = interleave ? ((total + 15) / 16 + p.grid - 1) / p.grid * 16 : (total + p.grid - 1) / p.grid;
    const uint64_t steps = static_cast<uint64_t>((rows + 15) / 16) * (swiglu ? 2 : 1) * static_cast<uint64_t>(nsb);
    p.magic_exact = steps * static_cast<uint64_t>(nsb) < (uint64_t{1} << 32);
    const size_t K = static_cast<size_t>(k);
    p.lds = 4 * K + 2 * kXPad + (K / static_cast<size_t>(sum_elems)) * sizeof(float) +
            static_cast<size_t>(rows) * (swiglu ? 2 : 1) * static_cast<size_t>(nsb) * sizeof(float);
    return p;
}
inline bool gemv_fits(const Gemv &p, size_t static_lds) {
    return p.magic_exact && static_lds <= kMaxLds && p.lds <= kMaxLds - static_lds;
}

// The grouped MoE streaming kernels (qlin_moe_grouped.hip): routes per pass nq (4, else 2), and the
// tiles whose partials fit in LDS at once.  Dynamic LDS: the pass's routes' staged x (Q4_K 4K +
// 2 kXPad bytes; the 32-weight formats tpb 16-byte slot vectors per block and hi / lo part, each part
// kXPad bytes longer), one x sum
// per 32 elements and route, and per tile nw * nq * nchunk * 16 partials.  The selected experts are
// only known on the device, so a piece is sized for twice an even share of min(E, R) of them.
struct StreamFmt {
    int ce;     // weights per chunk
    bool q4k;   // Q4_K staging (otherwise slot vectors)
    int tpb;    // 16-byte slot vectors per block (32-weight formats)
};
struct Stream {
    bool ok = false;
    int nq = 0, grid = 0, piece = 0;
    size_t lds = 0;
};
inline Stream stream(const StreamFmt &f, bool swiglu, int rows, int K, int E, int R, int cu_count,
                     size_t static_nq4, size_t static_nq2) {
    Stream p;
    const int nw = swiglu ? 2 : 1;
    const int nblk = K / 32, nchunk = K / f.ce, tpe = (rows + 15) / 16;
    const int grid = std::max(1, cu_count);
    const int64_t share = (static_cast<int64_t>(std::min(E, R)) * tpe + grid - 1) / grid;
    for (int nq = 4; nq >= 2; nq -= 2) {
        const size_t st = nq == 4 ? static_nq4 : static_nq2;
        if (st >= kMaxLds) continue;
        const size_t budget = kMaxLds - st;
        const size_t stage = f.q4k ? static_cast<size_t>(nq) * (4 * K + 2 * kXPad)
                                   : static_cast<size_t>(nq) * 2 * (nblk * f.tpb * 16 + kXPad);
        const size_t fixed = stage + static_cast<size_t>(nq) * nblk * sizeof(float);
        const size_t per_tile = static_cast<size_t>(nw) * nq * nchunk * 16 * sizeof(float);
        if (fixed + per_tile > budget) continue;
        const int64_t cap = static_cast<int64_t>((budget - fixed) / per_tile);
        p.ok = true;
        p.nq = nq;
        p.grid = grid;
        p.piece = static_cast<int>(std::min<int64_t>(cap, std::max<int64_t>(1, 2 * share)));
        p.lds = fixed + static_cast<size_t>(p.piece) * per_tile;
        return p;
    }
    return p;
}

}  // namespace plan
}  // namespace qlin

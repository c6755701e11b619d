// qlin_q4k_stream.hip -- persistent streaming Q4_K GEMV for decode (m == 1), gfx950.
//
// Computes y[o] = sum_k w(o, k) x[k] (reference quant_gemv_kernel / quant_gemv_add_kernel,
// AI/codes/local-llm/src/backend/cuda/ops/kernel.cu:1192-1244) for up to four matrices that share x
// (their rows are one concatenated index space), or the fused SwiGLU act[o] = g/(1+exp(-g))*u with
// g = Wg[o].x, u = Wu[o].x (reference quant_swiglu_kernel, kernel.cu:1289-1328).
//
// Work decomposition.  One workgroup of kStreamWaves waves per CU owns a contiguous slice of the
// concatenated rows.  A Q4_K row is K/256 super-blocks of 144 bytes (d, dmin, 12 scale bytes, 128
// nibble bytes).  Lane l owns sub-block pair p = l % 4 of super-block l / 4 of a 16-super-block
// step: its 32 nibble bytes are the 32 low nibbles of sub-block 2p and the 32 high nibbles of
// sub-block 2p+1, i.e. 64 weights read with two 16-byte loads plus one 16-byte header load shared
// by the 4 lanes of the super-block.  A work item is (row or gate/up row pair, step); items are
// dealt round-robin to the waves, and each wave keeps the next item's loads in flight while it
// computes the current one.
//
// x is staged into LDS once per workgroup (padded by 4 floats every 64 so that the 16-byte reads
// of 8 consecutive lanes hit distinct banks).  When K <= 4096 a row is a single step: each lane
// copies its 64 x values into registers once and reuses them for every row it touches, so the
// steady state reads nothing but the weight stream.  For longer rows the per-(row, step) sums are
// parked in LDS and added in step order at the end, which keeps the result deterministic.
//
// Per lane, row and pair the partial dot product is
//   d*sc_lo*sum(q_lo*x_lo) + (d*sc_hi/16)*sum(16*q_hi*x_hi) - dmin*(m_lo*sum(x_lo) + m_hi*sum(x_hi))
// (the high nibbles are converted without the shift; the 1/16 is exact), followed by a DPP
// reduction across the wave.  Weight loads are plain cached loads: on gfx950 the nontemporal
// variant streams measurably slower.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

namespace qlin {
namespace {

#ifndef QLIN_Q4K_STREAM_WAVES
#define QLIN_Q4K_STREAM_WAVES 16
#endif
constexpr int kStreamWaves = QLIN_Q4K_STREAM_WAVES;  // one workgroup per CU
constexpr int kStreamThreads = kStreamWaves * 64;
constexpr int kPadStride = 272;                     // floats per staged super-block (256 + 4 per 64)
constexpr size_t kMaxLds = 160 * 1024;              // gfx950 LDS per workgroup

struct StreamArgs {
    const uint8_t *w[kMaxStreamMats];
    float *y[kMaxStreamMats];
    int row_end[kMaxStreamMats];  // cumulative row counts of the concatenated matrices
    int nmat;
    size_t row_bytes;
    const float *x;
    int nsb;    // super-blocks per row
    int total;  // concatenated rows (SwiGLU: rows of the gate matrix)
    int add;    // y += instead of y =
};

__device__ __forceinline__ float cvt_b0(uint32_t v) { return static_cast<float>(v & 0xffu); }
__device__ __forceinline__ float cvt_b1(uint32_t v) { return static_cast<float>((v >> 8) & 0xffu); }
__device__ __forceinline__ float cvt_b2(uint32_t v) { return static_cast<float>((v >> 16) & 0xffu); }
__device__ __forceinline__ float cvt_b3(uint32_t v) { return static_cast<float>(v >> 24); }

// v & mask, opaque to the optimiser so that the byte conversions stay single
// v_cvt_f32_ubyte{0..3} instructions instead of being folded into bit-field extracts.
__device__ __forceinline__ uint32_t and_opaque(uint32_t v, uint32_t mask) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(mask), "v"(v));
    return r;
}

__device__ __forceinline__ float dot4(uint32_t v, const float *xv, float acc) {
    acc = fmaf(cvt_b0(v), xv[0], acc);
    acc = fmaf(cvt_b1(v), xv[1], acc);
    acc = fmaf(cvt_b2(v), xv[2], acc);
    acc = fmaf(cvt_b3(v), xv[3], acc);
    return acc;
}

__device__ __forceinline__ u32x4 ld16(const uint8_t *p) { return *reinterpret_cast<const u32x4 *>(p); }

template <int R>
struct Rows {
    u32x4 hdr[R], qa[R], qb[R];
};

// Lane-constant part of the 6-bit scale/min decode for sub-blocks j = 2p and 2p+1
// (kernel.cu:913-921): j < 4 takes 6 bits of bytes j (scale) and j+4 (min); j >= 4 takes a nibble
// of byte j+4 plus the top 2 bits of bytes j-4 (scale) and j (min).  Both j of a lane fall on the
// same side, so the two (scale, min) pairs come out packed in bytes 0 and 1.
struct ScaleDecoder {
    bool upper;
    int sh, m_shift;
    uint32_t lo_mask, hi_mask;
    __device__ explicit ScaleDecoder(int p)
        : upper(p >= 2), sh(p >= 2 ? 16 * (p - 2) : 16 * p), m_shift(p >= 2 ? 4 : 0),
          lo_mask(p >= 2 ? 0x0f0fu : 0x3f3fu), hi_mask(p >= 2 ? 0x0303u : 0u) {}
    __device__ __forceinline__ void operator()(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &scp,
                                               uint32_t &mp) const {
        const uint32_t a_sc = upper ? s2 : s0;
        const uint32_t a_m = upper ? s2 : s1;
        scp = ((a_sc >> sh) & lo_mask) | (((s0 >> (sh + 6)) & hi_mask) << 4);
        mp = ((a_m >> (sh + m_shift)) & lo_mask) | (((s1 >> (sh + 6)) & hi_mask) << 4);
    }
};

__device__ __forceinline__ float pair_dot(const u32x4 &hdr, const u32x4 &qa, const u32x4 &qb, const float *xlo,
                                          const float *xhi, float sxlo, float sxhi, const ScaleDecoder &dec) {
    const uint32_t qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    float slo0 = 0.0f, slo1 = 0.0f, shi0 = 0.0f, shi1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        slo0 = dot4(and_opaque(qv[i], 0x0f0f0f0fu), xlo + 4 * i, slo0);
        shi0 = dot4(and_opaque(qv[i], 0xf0f0f0f0u), xhi + 4 * i, shi0);
        slo1 = dot4(and_opaque(qv[i + 1], 0x0f0f0f0fu), xlo + 4 * i + 4, slo1);
        shi1 = dot4(and_opaque(qv[i + 1], 0xf0f0f0f0u), xhi + 4 * i + 4, shi1);
    }
    uint32_t scp, mp;
    dec(hdr.y, hdr.z, hdr.w, scp, mp);
    const float d = f16_bits_to_f32(hdr.x & 0xffffu);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    float a = (d * cvt_b0(scp)) * (slo0 + slo1);
    a = fmaf((d * 0.0625f) * cvt_b1(scp), shi0 + shi1, a);
    a = fmaf(-(dmin * cvt_b0(mp)), sxlo, a);
    a = fmaf(-(dmin * cvt_b1(mp)), sxhi, a);
    return a;
}

__device__ __forceinline__ void read_x(const float *xs, int s, int p, float *xlo, float *xhi, float &sxlo,
                                       float &sxhi) {
    const float *xl = xs + s * kPadStride + 68 * p;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 a = *reinterpret_cast<const float4 *>(xl + 4 * i);
        const float4 b = *reinterpret_cast<const float4 *>(xl + 32 + 4 * i);
        xlo[4 * i] = a.x; xlo[4 * i + 1] = a.y; xlo[4 * i + 2] = a.z; xlo[4 * i + 3] = a.w;
        xhi[4 * i] = b.x; xhi[4 * i + 1] = b.y; xhi[4 * i + 2] = b.z; xhi[4 * i + 3] = b.w;
    }
    sxlo = 0.0f;
    sxhi = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) { sxlo += xlo[i]; sxhi += xhi[i]; }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes without LDS: DPP within each 16-lane row (xor 1 and xor 2 by quad
// permutation, then rotations by 4 and 8), then the four row sums read back as scalars.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f32<0xb1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4e>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x124>(v);  // row_ror:4
    v += dpp_f32<0x128>(v);  // row_ror:8
    const int iv = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
    return (r0 + r1) + (r2 + r3);
}

// Matrix index and local row of concatenated row gr.
__device__ __forceinline__ void locate(const StreamArgs &a, int gr, int &mat, int &local) {
    mat = 0;
#pragma unroll
    for (int i = 0; i + 1 < kMaxStreamMats; ++i)
        if (i + 1 < a.nmat && gr >= a.row_end[i]) mat = i + 1;
    local = gr - (mat ? a.row_end[mat - 1] : 0);
}

template <bool SINGLE, bool SWIGLU>
__global__ __launch_bounds__(kStreamThreads) void q4k_stream_kernel(const StreamArgs a) {
    constexpr int R = SWIGLU ? 2 : 1;  // rows per item: one row, or the gate/up pair of one output
    extern __shared__ float smem[];
    float *xs = smem;
    float *partial = smem + a.nsb * kPadStride;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rb = static_cast<int>(static_cast<int64_t>(a.total) * blockIdx.x / gridDim.x);
    const int re = static_cast<int>(static_cast<int64_t>(a.total) * (blockIdx.x + 1) / gridDim.x);
    const int nsb = a.nsb;
    const int steps = SINGLE ? 1 : (nsb + 15) >> 4;
    const int nitems = (re - rb) * steps;
    const int p = lane & 3, sbl = lane >> 2;
    const ScaleDecoder dec(p);

    auto row_ptr = [&](int gr, int r) -> const uint8_t * {
        if constexpr (SWIGLU) {
            return a.w[r] + static_cast<size_t>(gr) * a.row_bytes;
        } else {
            int mat, local;
            locate(a, gr, mat, local);
            return a.w[mat] + static_cast<size_t>(local) * a.row_bytes;
        }
    };
    auto load_item = [&](Rows<R> &t, int i) {
        const int gr = rb + i / steps;  // i < nitems, so gr < re
        const int sb = min((i % steps) * 16 + sbl, nsb - 1);
        const size_t off = static_cast<size_t>(sb) * 144;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *sp = row_ptr(gr, r) + off;
            t.hdr[r] = ld16(sp);
            t.qa[r] = ld16(sp + 16 + 32 * p);
            t.qb[r] = ld16(sp + 32 + 32 * p);
        }
    };

    Rows<R> A, B;
    if (wave < nitems) load_item(A, wave);  // weights first: they do not depend on x
    {
        const float4 *src = reinterpret_cast<const float4 *>(a.x);
        for (int i = tid; i < nsb * 64; i += kStreamThreads) {
            const int e = i * 4;
            *reinterpret_cast<float4 *>(xs + e + 4 * (e >> 6)) = src[i];
        }
    }
    __syncthreads();

    float xlo[32], xhi[32], sxlo = 0.0f, sxhi = 0.0f;
    if constexpr (SINGLE) {
        read_x(xs, min(sbl, nsb - 1), p, xlo, xhi, sxlo, sxhi);
        if (sbl >= nsb) {  // lanes past the end of the row contribute nothing
#pragma unroll
            for (int i = 0; i < 32; ++i) { xlo[i] = 0.0f; xhi[i] = 0.0f; }
            sxlo = 0.0f;
            sxhi = 0.0f;
        }
    }

    auto process = [&](const Rows<R> &t, int i) {
        const int gr = rb + i / steps, st = i % steps;
        const int sb = st * 16 + sbl;
        if constexpr (!SINGLE) read_x(xs, min(sb, nsb - 1), p, xlo, xhi, sxlo, sxhi);
        float tot[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float part = pair_dot(t.hdr[r], t.qa[r], t.qb[r], xlo, xhi, sxlo, sxhi, dec);
            if (!SINGLE && sb >= nsb) part = 0.0f;
            tot[r] = wave_sum_dpp(part);
        }
        if (lane == 0) {
            if constexpr (!SINGLE) {
#pragma unroll
                for (int r = 0; r < R; ++r) partial[((gr - rb) * steps + st) * R + r] = tot[r];
            } else if constexpr (SWIGLU) {
                a.y[0][gr] = tot[0] / (1.0f + expf(-tot[0])) * tot[1];
            } else {
                int mat, local;
                locate(a, gr, mat, local);
                float *dst = a.y[mat] + local;
                *dst = a.add ? *dst + tot[0] : tot[0];
            }
        }
    };

    for (int i = wave; i < nitems; i += 2 * kStreamWaves) {
        const int i1 = i + kStreamWaves, i2 = i + 2 * kStreamWaves;
        if (i1 < nitems) load_item(B, i1);
        process(A, i);
        if (i2 < nitems) load_item(A, i2);
        if (i1 < nitems) process(B, i1);
    }

    if constexpr (!SINGLE) {
        __syncthreads();
        for (int r = tid; r < re - rb; r += kStreamThreads) {
            float tot[R];
#pragma unroll
            for (int q = 0; q < R; ++q) {
                tot[q] = 0.0f;
                for (int st = 0; st < steps; ++st) tot[q] += partial[(r * steps + st) * R + q];
            }
            const int gr = rb + r;
            if constexpr (SWIGLU) {
                a.y[0][gr] = tot[0] / (1.0f + expf(-tot[0])) * tot[1];
            } else {
                int mat, local;
                locate(a, gr, mat, local);
                float *dst = a.y[mat] + local;
                *dst = a.add ? *dst + tot[0] : tot[0];
            }
        }
    }
}

int stream_grid(int total) { return max(1, min(device_info().cu_count, (total + kStreamWaves - 1) / kStreamWaves)); }

size_t stream_lds(int total, int nsb, bool swiglu) {
    size_t floats = static_cast<size_t>(nsb) * kPadStride;
    if (nsb > 16) {
        const int grid = stream_grid(total);
        floats += static_cast<size_t>((total + grid - 1) / grid + 1) * ((nsb + 15) / 16) * (swiglu ? 2 : 1);
    }
    return floats * sizeof(float);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

hipError_t launch(const StreamArgs &a, bool swiglu, hipStream_t s) {
    const int grid = stream_grid(a.total);
    const size_t lds = stream_lds(a.total, a.nsb, swiglu);
    const bool single = a.nsb <= 16;
    if (swiglu) {
        if (single)
            hipLaunchKernelGGL((q4k_stream_kernel<true, true>), dim3(grid), dim3(kStreamThreads), lds, s, a);
        else
            hipLaunchKernelGGL((q4k_stream_kernel<false, true>), dim3(grid), dim3(kStreamThreads), lds, s, a);
    } else {
        if (single)
            hipLaunchKernelGGL((q4k_stream_kernel<true, false>), dim3(grid), dim3(kStreamThreads), lds, s, a);
        else
            hipLaunchKernelGGL((q4k_stream_kernel<false, false>), dim3(grid), dim3(kStreamThreads), lds, s, a);
    }
    return hipGetLastError();
}

}  // namespace

bool q4k_stream_ok(const uint8_t *const *w, int nmat, size_t rb, const float *x, int total, int k, bool swiglu) {
    if (nmat < 1 || nmat > kMaxStreamMats || k % 256 || rb % 16 || !aligned16(x)) return false;
    for (int i = 0; i < nmat; ++i)
        if (!aligned16(w[i])) return false;
    return stream_lds(total, k / 256, swiglu) <= kMaxLds;
}

hipError_t q4k_stream_gemv(const uint8_t *const *w, float *const *y, const int *rows, int nmat, size_t rb,
                           const float *x, int k, bool add, hipStream_t s) {
    StreamArgs a{};
    int total = 0;
    for (int i = 0; i < nmat; ++i) {
        a.w[i] = w[i];
        a.y[i] = y[i];
        total += rows[i];
        a.row_end[i] = total;
    }
    if (total == 0) return hipSuccess;
    a.nmat = nmat;
    a.row_bytes = rb;
    a.x = x;
    a.nsb = k / 256;
    a.total = total;
    a.add = add ? 1 : 0;
    return launch(a, false, s);
}

hipError_t q4k_stream_swiglu(const uint8_t *wg, const uint8_t *wu, size_t rb, const float *x, float *act,
                             int ffn, int k, hipStream_t s) {
    if (ffn == 0) return hipSuccess;
    StreamArgs a{};
    a.w[0] = wg;
    a.w[1] = wu;
    a.y[0] = act;
    a.row_end[0] = ffn;
    a.nmat = 1;
    a.row_bytes = rb;
    a.x = x;
    a.nsb = k / 256;
    a.total = ffn;
    return launch(a, true, s);
}

}  // namespace qlin

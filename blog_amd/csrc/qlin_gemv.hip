// qlin_gemv.hip -- dequant-fused GEMV for decode (m small), gfx950.
//
// Semantics: y[r, o] = sum_k w(o, k) * x[r, k] with f32 activations and f32 accumulation, as the
// reference's quant_gemv_kernel / quant_gemv_add_kernel (AI/codes/local-llm/src/backend/cuda/ops/
// kernel.cu:1192-1244).  The summation order is ours (results agree within fp32 rounding).
//
// Fast path, Q4_K (the decode hot spot): one wave64 owns R consecutive weight rows; lane l owns
// sub-block pair p = l % 4 of super-block 16*i + l/4, i.e. 32 qs bytes = 64 weights (32 low
// nibbles of sub-block 2p, 32 high nibbles of sub-block 2p+1).  The workgroup stages x through LDS
// once per K tile (padded by 4 floats every 64 so the lanes' 16-byte reads are bank-conflict free);
// each lane then keeps its 64 x values in registers and reuses them for all R rows, so the only
// per-row memory traffic is the weight stream itself (two 16-byte qs loads + one 16-byte header
// load that the lanes of a super-block share).  Per row and pair the lane forms
//   d*sc_lo*sum(q_lo*x_lo) + (d*sc_hi/16)*sum(16*q_hi*x_hi) - dmin*(m_lo*sum(x_lo) + m_hi*sum(x_hi))
// where sum(x_*) does not depend on the row and is computed once.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

namespace qlin {

namespace {

constexpr int kBlock = 256;   // 4 waves
constexpr int kWaves = kBlock / 64;

// ---- generic per-element path (any supported type, any 2-byte alignment) ---------------------

template <int T, int MT>
__global__ __launch_bounds__(kBlock) void gemv_generic_kernel(const uint8_t *__restrict__ w,
                                                              size_t row_bytes,
                                                              const float *__restrict__ x,
                                                              float *__restrict__ y, int out_dim,
                                                              int in_dim, int m, int add) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    const int row = static_cast<int>((blockIdx.x * kBlock + threadIdx.x) >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= out_dim) return;  // uniform per wave
    const uint8_t *rp = w + static_cast<size_t>(row) * row_bytes;
    for (int r0 = 0; r0 < m; r0 += MT) {
        float acc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
        for (int k = lane; k < in_dim; k += 64) {
            const float wv = block_value<T>(rp + (k / BE) * BB, k % BE);
#pragma unroll
            for (int t = 0; t < MT; ++t)
                if (r0 + t < m) acc[t] = fmaf(wv, x[static_cast<size_t>(r0 + t) * in_dim + k], acc[t]);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const float s = wave_sum(acc[t]);
            if (lane == 0 && r0 + t < m) {
                float *dst = y + static_cast<size_t>(r0 + t) * out_dim + row;
                *dst = add ? *dst + s : s;
            }
        }
    }
}

template <int T>
hipError_t launch_generic_t(const uint8_t *w, size_t rb, const float *x, float *y, int n, int k,
                            int m, bool add, hipStream_t s) {
    const int blocks = (n + kWaves - 1) / kWaves;
    hipLaunchKernelGGL((gemv_generic_kernel<T, 4>), dim3(blocks), dim3(kBlock), 0, s, w, rb, x, y, n,
                       k, m, add ? 1 : 0);
    return hipGetLastError();
}

// ---- Q4_K fast path (m == 1) ------------------------------------------------------------------

#ifndef QLIN_Q4K_WAVES_PER_EU
#define QLIN_Q4K_WAVES_PER_EU 0   // 0: let the compiler choose the register budget
#endif
#ifndef QLIN_Q4K_R_SINGLE
#define QLIN_Q4K_R_SINGLE 2       // rows per work item when a row is a single step (K <= 4096)
#endif
#if QLIN_Q4K_WAVES_PER_EU > 0
#define QLIN_Q4K_ATTR __attribute__((amdgpu_waves_per_eu(QLIN_Q4K_WAVES_PER_EU)))
#else
#define QLIN_Q4K_ATTR
#endif

constexpr int kPadStride = 272;              // floats per staged super-block (256 + 4 per 64)

__device__ __forceinline__ float cvt_b0(uint32_t v) { return static_cast<float>(v & 0xffu); }
__device__ __forceinline__ float cvt_b1(uint32_t v) { return static_cast<float>((v >> 8) & 0xffu); }
__device__ __forceinline__ float cvt_b2(uint32_t v) { return static_cast<float>((v >> 16) & 0xffu); }
__device__ __forceinline__ float cvt_b3(uint32_t v) { return static_cast<float>(v >> 24); }

// sum over the 4 bytes of v of byte * xv[0..3]
__device__ __forceinline__ float dot4(uint32_t v, const float *xv, float acc) {
    acc = fmaf(cvt_b0(v), xv[0], acc);
    acc = fmaf(cvt_b1(v), xv[1], acc);
    acc = fmaf(cvt_b2(v), xv[2], acc);
    acc = fmaf(cvt_b3(v), xv[3], acc);
    return acc;
}

// v & mask, opaque to the optimiser so that the byte conversions below stay single
// v_cvt_f32_ubyte{0..3} instructions instead of being folded into bit-field extracts.
__device__ __forceinline__ uint32_t and_opaque(uint32_t v, uint32_t mask) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(mask), "v"(v));
    return r;
}

template <int R>
struct Q4kRows {
    u32x4 hdr[R], qa[R], qb[R];
};

// Issue the 16-byte loads of super-block sb (pair p) for rows row0 .. row0+R-1 (clamped to
// last_row; the duplicate rows are never stored).
template <int R>
__device__ __forceinline__ void q4k_load(Q4kRows<R> &t, const uint8_t *__restrict__ w, size_t row_bytes,
                                         int row0, int last_row, int sb, int p) {
    const size_t sb_off = static_cast<size_t>(sb) * 144;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, last_row);
        const uint8_t *sp = w + static_cast<size_t>(row) * row_bytes + sb_off;
        t.hdr[r] = ld_stream16(sp);
        t.qa[r] = ld_stream16(sp + 16 + 32 * p);
        t.qb[r] = ld_stream16(sp + 32 + 32 * p);
    }
}

// Lane-constant part of the 6-bit scale/min decode for sub-blocks j = 2p and 2p+1
// (kernel.cu:913-921): j < 4 takes 6 bits of bytes j (scale) and j+4 (min); j >= 4 takes a
// nibble of byte j+4 plus the top 2 bits of bytes j-4 (scale) and j (min).  Both j of a lane
// fall on the same side, so the two (scale, min) pairs come out packed in bytes 0 and 1.
struct Q4kScaleDecoder {
    bool upper;
    int sh, m_shift;
    uint32_t lo_mask, hi_mask;
    __device__ explicit Q4kScaleDecoder(int p)
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

// Partial dot of one lane's 64 weights of one row with its x slice:
//   d*sc_lo*sum(q_lo*x_lo) + (d*sc_hi/16)*sum(16 q_hi*x_hi) - dmin*m_lo*sum(x_lo) - dmin*m_hi*sum(x_hi)
__device__ __forceinline__ float q4k_pair_dot(const u32x4 &hdr, const u32x4 &qa, const u32x4 &qb,
                                              const float *xlo, const float *xhi, float sxlo, float sxhi,
                                              const Q4kScaleDecoder &dec) {
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

// Lane l's 64 x values: pair p = l % 4 of staged super-block s (LDS layout padded by 4 floats
// every 64, so the 16-byte reads of 8 consecutive lanes hit distinct banks).
__device__ __forceinline__ void q4k_read_x(const float *xs, int s, int p, float *xlo, float *xhi, float &sxlo,
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

// Sum over the 64 lanes without LDS: DPP within each 16-lane row (xor 1, xor 2 by quad
// permutation, then rotations by 4 and 8), then the four row sums read back as scalars.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

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

#ifndef QLIN_Q4K_STREAM_WAVES
#define QLIN_Q4K_STREAM_WAVES 12
#endif
constexpr int kStreamWaves = QLIN_Q4K_STREAM_WAVES;  // one workgroup per CU
constexpr int kStreamThreads = kStreamWaves * 64;
constexpr size_t kMaxLds = 160 * 1024;              // gfx950 LDS per workgroup

int q4k_stream_grid(int n) { return max(1, min(device_info().cu_count, (n + kStreamWaves - 1) / kStreamWaves)); }

// Dynamic LDS of the streaming kernel: x padded to 272 floats per super-block, plus the
// per-(row, step) partials when a row takes more than one step.
size_t q4k_stream_lds(int n, int k) {
    const int nsb = k / 256;
    size_t floats = static_cast<size_t>(nsb) * kPadStride;
    if (nsb > 16) {
        const int grid = q4k_stream_grid(n);
        floats += static_cast<size_t>((n + grid - 1) / grid + 1) * ((nsb + 15) / 16);
    }
    return floats * sizeof(float);
}

// Persistent streaming Q4_K GEMV.  Workgroup b owns the contiguous rows
// [N*b/G, N*(b+1)/G); its work items are (group of R rows, 16-super-block step) pairs dealt
// round-robin to its waves, each wave prefetching its next item's weights while computing the
// current one.  SINGLE (K <= 4096): one step per row, the lane's x slice lives in registers for
// the whole kernel and each item's R sums go straight to y.  Otherwise every (row, step) partial is
// parked in LDS and summed in step order at the end (deterministic).
template <int R, bool SINGLE>
__global__ __launch_bounds__(kStreamThreads) QLIN_Q4K_ATTR void gemv_q4k_stream_kernel(
    const uint8_t *__restrict__ w, size_t row_bytes, const float *__restrict__ x, float *__restrict__ y,
    int out_dim, int nsb, int add) {
    extern __shared__ float smem[];
    float *xs = smem;
    float *partial = smem + nsb * kPadStride;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rb = static_cast<int>(static_cast<int64_t>(out_dim) * blockIdx.x / gridDim.x);
    const int re = static_cast<int>(static_cast<int64_t>(out_dim) * (blockIdx.x + 1) / gridDim.x);
    const int steps = SINGLE ? 1 : (nsb + 15) >> 4;
    const int nitems = (re - rb + R - 1) / R * steps;
    const int p = lane & 3, sbl = lane >> 2;
    const Q4kScaleDecoder dec(p);

    auto item_row0 = [&](int i) { return rb + (i / steps) * R; };
    auto item_step = [&](int i) { return i % steps; };
    auto load_item = [&](Q4kRows<R> &t, int i) {
        const int sb = min(item_step(i) * 16 + sbl, nsb - 1);
        q4k_load<R>(t, w, row_bytes, item_row0(i), re - 1, sb, p);
    };

    Q4kRows<R> A, B;
    if (wave < nitems) load_item(A, wave);  // weights first: they do not depend on x
    {
        const float4 *src = reinterpret_cast<const float4 *>(x);
        for (int i = tid; i < nsb * 64; i += kStreamThreads) {
            const int e = i * 4;
            *reinterpret_cast<float4 *>(xs + e + 4 * (e >> 6)) = src[i];
        }
    }
    __syncthreads();

    float xlo[32], xhi[32], sxlo = 0.0f, sxhi = 0.0f;
    if constexpr (SINGLE) {
        q4k_read_x(xs, min(sbl, nsb - 1), p, xlo, xhi, sxlo, sxhi);
        if (sbl >= nsb) {  // lanes past the row end contribute nothing
#pragma unroll
            for (int i = 0; i < 32; ++i) { xlo[i] = 0.0f; xhi[i] = 0.0f; }
            sxlo = 0.0f;
            sxhi = 0.0f;
        }
    }

    auto process = [&](const Q4kRows<R> &t, int i) {
        const int row0 = item_row0(i), st = item_step(i);
        const int sb = st * 16 + sbl;
        if constexpr (!SINGLE) q4k_read_x(xs, min(sb, nsb - 1), p, xlo, xhi, sxlo, sxhi);
        const bool valid = sb < nsb;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float part = q4k_pair_dot(t.hdr[r], t.qa[r], t.qb[r], xlo, xhi, sxlo, sxhi, dec);
            if (!SINGLE && !valid) part = 0.0f;
            const float tot = wave_sum_dpp(part);
            const int row = row0 + r;
            if (lane == 0 && row < re) {
                if constexpr (SINGLE) {
                    y[row] = add ? y[row] + tot : tot;
                } else {
                    partial[(row - rb) * steps + st] = tot;
                }
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
            float tot = 0.0f;
            for (int st = 0; st < steps; ++st) tot += partial[r * steps + st];
            y[rb + r] = add ? y[rb + r] + tot : tot;
        }
    }
}

template <int R>
hipError_t launch_q4k_stream(const uint8_t *w, size_t rb, const float *x, float *y, int n, int k, bool add,
                             hipStream_t s) {
    const int nsb = k / 256;
    const int grid = q4k_stream_grid(n);
    const size_t lds = q4k_stream_lds(n, k);
    if (nsb <= 16) {
        hipLaunchKernelGGL((gemv_q4k_stream_kernel<R, true>), dim3(grid), dim3(kStreamThreads), lds, s, w, rb, x, y,
                           n, nsb, add ? 1 : 0);
    } else {
        hipLaunchKernelGGL((gemv_q4k_stream_kernel<1, false>), dim3(grid), dim3(kStreamThreads), lds, s, w, rb, x,
                           y, n, nsb, add ? 1 : 0);
    }
    return hipGetLastError();
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t gemv_generic(int type, const uint8_t *w, size_t rb, const float *x, float *y, int n,
                        int k, int m, bool add, hipStream_t s) {
    switch (type) {
        case T_Q4_0: return launch_generic_t<T_Q4_0>(w, rb, x, y, n, k, m, add, s);
        case T_Q5_0: return launch_generic_t<T_Q5_0>(w, rb, x, y, n, k, m, add, s);
        case T_Q8_0: return launch_generic_t<T_Q8_0>(w, rb, x, y, n, k, m, add, s);
        case T_Q4_K: return launch_generic_t<T_Q4_K>(w, rb, x, y, n, k, m, add, s);
        case T_Q6_K: return launch_generic_t<T_Q6_K>(w, rb, x, y, n, k, m, add, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t gemv(int type, const uint8_t *w, size_t rb, const float *x, float *y, int n, int k, int m,
                bool add, hipStream_t s) {
    if (n == 0 || m == 0) return hipSuccess;
    if (type == T_Q4_K && m == 1 && aligned16(w) && aligned16(x) && rb % 16 == 0 && q4k_stream_lds(n, k) <= kMaxLds)
        return launch_q4k_stream<QLIN_Q4K_R_SINGLE>(w, rb, x, y, n, k, add, s);
    return gemv_generic(type, w, rb, x, y, n, k, m, add, s);
}

}  // namespace qlin

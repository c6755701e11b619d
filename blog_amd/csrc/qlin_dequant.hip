// qlin_dequant.hip -- whole-stream dequantization to f32 or f16, gfx950.
//
// Semantics of the reference's dequantize_{q4k,q80,q50,q6k}_to_f16_kernel
// (AI/codes/local-llm/src/backend/cuda/ops/kernel.cu:954-1063): every element is the canonical
// non-contracted f32 value of its block (qlin_device.hpp), and the f16 output is that value rounded
// to nearest-even (scalar v_cvt_f16_f32 under the default round-to-nearest mode, f16 subnormals
// preserved).  Results are bit-exact
// against any correct evaluation of the formulas.  Q4_0 is added from the ggml format.
//
// Layout: one thread per output element, consecutive threads on consecutive elements, so the
// stores (the dominant traffic: 4 or 2 bytes out per 0.56..1.06 bytes in) are fully coalesced; the
// block header bytes are re-read by the threads of a block and served from L1.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"

namespace qlin {
namespace {

template <int T, bool F16>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ src,
                                                      void *__restrict__ out, int64_t n) {
    constexpr int BE = Block<T>::elems, BB = Block<T>::bytes;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int64_t b = i / BE;
        const float v = block_value<T>(src + b * BB, static_cast<int>(i - b * BE));
        if constexpr (F16) {
            static_cast<uint16_t *>(out)[i] = static_cast<uint16_t>(f32_to_f16_bits(v));
        } else {
            static_cast<float *>(out)[i] = v;
        }
    }
}

template <int T>
hipError_t launch_t(const uint8_t *src, void *out, int64_t n, bool f16, hipStream_t s) {
    const int64_t want = (n + 255) / 256;
    const int blocks = static_cast<int>(want < 65536 ? want : 65536);
    if (f16)
        hipLaunchKernelGGL((dequant_kernel<T, true>), dim3(blocks), dim3(256), 0, s, src, out, n);
    else
        hipLaunchKernelGGL((dequant_kernel<T, false>), dim3(blocks), dim3(256), 0, s, src, out, n);
    return hipGetLastError();
}

}  // namespace

hipError_t dequant(int type, const uint8_t *src, void *out, int64_t n, bool to_f16, hipStream_t s) {
    if (n == 0) return hipSuccess;
    switch (type) {
        case T_Q4_0: return launch_t<T_Q4_0>(src, out, n, to_f16, s);
        case T_Q5_0: return launch_t<T_Q5_0>(src, out, n, to_f16, s);
        case T_Q8_0: return launch_t<T_Q8_0>(src, out, n, to_f16, s);
        case T_Q4_K: return launch_t<T_Q4_K>(src, out, n, to_f16, s);
        case T_Q6_K: return launch_t<T_Q6_K>(src, out, n, to_f16, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qlin

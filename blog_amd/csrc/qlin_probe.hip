// qlin_probe.hip -- a plain streaming read of a device buffer (qlin_probe.h): the bandwidth floor of
// a launch of the same bytes, for the measurements that compare the kernels against it.
#include "qlin_device.hpp"
#include "qlin_internal.hpp"
#include "qlin.h"
#include "qlin_probe.h"

namespace qlin {
namespace {

// Grid-stride 16-byte loads, 4 in flight per thread; the words' xor checksum is stored only for one
// improbable value.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4 *__restrict__ p, size_t n, float *sink) {
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n; i += 4 * stride) {
        const uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n; i += stride) {
        const uint4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = static_cast<float>(acc);
}

}  // namespace
}  // namespace qlin

extern "C" int qlin_probe_stream_read(const void *buf, size_t bytes, int workgroups, float *sink) {
    if (workgroups <= 0 || bytes % 16) return QLIN_ERR_SHAPE;
    if (!sink || (bytes && !buf)) return QLIN_ERR_NULL;
    if ((reinterpret_cast<uintptr_t>(buf) & 15u) || (reinterpret_cast<uintptr_t>(sink) & 3u)) return QLIN_ERR_ALIGN;
    hipLaunchKernelGGL(qlin::stream_read_kernel, dim3(workgroups), dim3(256), 0,
                       static_cast<hipStream_t>(qlin_get_stream()), static_cast<const uint4 *>(buf), bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? QLIN_OK : QLIN_ERR_LAUNCH;
}

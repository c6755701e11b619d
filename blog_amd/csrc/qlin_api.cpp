// qlin_api.cpp -- the C ABI (include/qlin.h): host-side argument validation and dispatch.
//
// Validation runs entirely on the host, before any HIP call, and returns a qlin_status where the
// reference launchers (AI/codes/local-llm/src/backend/cuda/ops/launch.cu) return void.  The facade
// entry points mirror TensorTool (src/tensor/TensorTool.cpp) including its rejection rules.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

#include "qlin.h"
#include "qlin_decoder.h"
#include "qlin_internal.hpp"

namespace qlin {

const DeviceInfo &device_info() {
    static DeviceInfo infos[64];
    static std::atomic<bool> ready[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        static DeviceInfo fallback;
        return fallback;
    }
    if (!ready[dev].load(std::memory_order_acquire)) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            infos[dev].cu_count = cus;
        ready[dev].store(true, std::memory_order_release);
    }
    return infos[dev];
}

}  // namespace qlin

namespace {

std::atomic<hipStream_t> g_stream{nullptr};

hipStream_t stream() { return g_stream.load(std::memory_order_relaxed); }

bool known_weight_type(int t) {
    return t == QLIN_TYPE_Q4_0 || t == QLIN_TYPE_Q5_0 || t == QLIN_TYPE_Q8_0 || t == QLIN_TYPE_Q4_K ||
           t == QLIN_TYPE_Q6_K;
}

int elems_of(int t) {
    switch (t) {
        case QLIN_TYPE_Q4_0: case QLIN_TYPE_Q5_0: case QLIN_TYPE_Q8_0: case QLIN_TYPE_Q8_1: return 32;
        case QLIN_TYPE_Q4_K: case QLIN_TYPE_Q6_K: return 256;
        default: return 0;
    }
}

int bytes_of(int t) {
    switch (t) {
        case QLIN_TYPE_Q4_0: return 18;
        case QLIN_TYPE_Q5_0: return 22;
        case QLIN_TYPE_Q8_0: return 34;
        case QLIN_TYPE_Q8_1: return 36;
        case QLIN_TYPE_Q4_K: return 144;
        case QLIN_TYPE_Q6_K: return 210;
        default: return 0;
    }
}

size_t min_row_bytes(int t, int in_dim) {
    const int be = elems_of(t);
    if (be == 0 || in_dim < 0 || in_dim % be) return 0;
    return static_cast<size_t>(in_dim / be) * static_cast<size_t>(bytes_of(t));
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int launched(hipError_t e) { return e == hipSuccess ? QLIN_OK : QLIN_ERR_LAUNCH; }

// Shared checks of a [out_dim, in_dim] weight with the given row stride.
int check_weight(int type, const uint8_t *w, size_t row_bytes, int out_dim, int in_dim) {
    if (!known_weight_type(type)) return QLIN_ERR_UNSUPPORTED_TYPE;
    if (out_dim < 0 || in_dim <= 0 || in_dim % elems_of(type)) return QLIN_ERR_SHAPE;
    if (row_bytes < min_row_bytes(type, in_dim)) return QLIN_ERR_ROW_BYTES;
    if (out_dim > 0 && !w) return QLIN_ERR_NULL;
    if (!aligned(w, 2) || (out_dim > 1 && row_bytes % 2)) return QLIN_ERR_ALIGN;
    return QLIN_OK;
}

int check_f32(const float *p, bool needed) {
    if (needed && !p) return QLIN_ERR_NULL;
    if (!aligned(p, 4)) return QLIN_ERR_ALIGN;
    return QLIN_OK;
}

int gemv_common(int type, const uint8_t *w, size_t rb, const float *x, float *y, int out_dim, int in_dim, int m,
                bool add) {
    int rc = check_weight(type, w, rb, out_dim, in_dim);
    if (rc) return rc;
    if (m < 0) return QLIN_ERR_SHAPE;
    const bool work = out_dim > 0 && m > 0;
    if ((rc = check_f32(x, work)) || (rc = check_f32(y, work))) return rc;
    if (!work) return QLIN_OK;
    return launched(qlin::gemv(type, w, rb, x, y, out_dim, in_dim, m, add, stream()));
}

}  // namespace

extern "C" {

const char *qlin_status_string(int status) {
    switch (status) {
        case QLIN_OK: return "ok";
        case QLIN_ERR_UNSUPPORTED_TYPE: return "unsupported weight type";
        case QLIN_ERR_SHAPE: return "invalid shape (negative dimension or in_dim not a multiple of the block)";
        case QLIN_ERR_NULL: return "null pointer";
        case QLIN_ERR_ROW_BYTES: return "row or expert stride smaller than its packed data";
        case QLIN_ERR_LIMIT: return "argument beyond a documented limit";
        case QLIN_ERR_LAUNCH: return "HIP launch failed";
        case QLIN_ERR_ALIGN: return "misaligned pointer";
        case QLIN_ERR_IO: return "cannot open or map the file";
        case QLIN_ERR_FORMAT: return "malformed or unsupported GGUF file";
        case QLIN_ERR_NOT_FOUND: return "no such tensor, key or index, or a value of another type";
        case QLIN_ERR_ALLOC: return "device allocation or copy failed";
        default: return "unknown status";
    }
}

const char *qlin_version(void) { return "qlin 0.1 gfx950"; }

int qlin_set_stream(void *s) {
    g_stream.store(static_cast<hipStream_t>(s), std::memory_order_relaxed);
    return QLIN_OK;
}

void *qlin_get_stream(void) { return stream(); }

int qlin_block_elems(int type) { return elems_of(type); }
int qlin_block_bytes(int type) { return bytes_of(type); }
size_t qlin_row_bytes(int type, int in_dim) { return min_row_bytes(type, in_dim); }

int qlin_launch_quant_gemv(int type, const uint8_t *w, size_t rb, const float *x, float *y, int out_dim, int in_dim,
                           int m) {
    return gemv_common(type, w, rb, x, y, out_dim, in_dim, m, false);
}

int qlin_launch_quant_gemv_add(int type, const uint8_t *w, size_t rb, const float *x, float *y, int out_dim,
                               int in_dim) {
    return gemv_common(type, w, rb, x, y, out_dim, in_dim, 1, true);
}

int qlin_launch_quant_matmul(int type, const uint8_t *w, size_t rb, const float *x, float *y, int out_dim,
                             int in_dim, int m) {
    return gemv_common(type, w, rb, x, y, out_dim, in_dim, m, false);
}

int qlin_launch_quant_matmul_add(int type, const uint8_t *w, size_t rb, const float *x, float *y, int out_dim,
                                 int in_dim, int m) {
    return gemv_common(type, w, rb, x, y, out_dim, in_dim, m, true);
}

int qlin_launch_quant_gemv_multi(int type, int n_mats, const uint8_t *const *weights, size_t rb, const float *x,
                                 float *const *ys, const int *out_dims, int in_dim) {
    if (n_mats < 0) return QLIN_ERR_SHAPE;
    if (n_mats > qlin::kMaxStreamMats) return QLIN_ERR_LIMIT;
    if (n_mats == 0) return QLIN_OK;
    if (!weights || !ys || !out_dims) return QLIN_ERR_NULL;
    bool work = false;
    for (int i = 0; i < n_mats; ++i) {
        int rc = check_weight(type, weights[i], rb, out_dims[i], in_dim);
        if (rc) return rc;
        if ((rc = check_f32(ys[i], out_dims[i] > 0))) return rc;
        work = work || out_dims[i] > 0;
    }
    int rc = check_f32(x, work);
    if (rc || !work) return rc;
    return launched(qlin::gemv_multi(type, weights, ys, out_dims, n_mats, rb, x, in_dim, stream()));
}

int qlin_launch_rms_norm_quant_gemv_multi(int type, int n_mats, const uint8_t *const *weights, size_t rb,
                                          const float *x, const uint16_t *norm_weight, int norm_type, float eps,
                                          int one_plus, float *const *ys, const int *out_dims, int in_dim) {
    if (n_mats < 0 || (norm_type != 0 && norm_type != 1)) return QLIN_ERR_SHAPE;
    if (n_mats > qlin::kMaxStreamMats) return QLIN_ERR_LIMIT;
    if (n_mats == 0) return QLIN_OK;
    if (!weights || !ys || !out_dims) return QLIN_ERR_NULL;
    bool work = false;
    int total = 0;
    for (int i = 0; i < n_mats; ++i) {
        int rc = check_weight(type, weights[i], rb, out_dims[i], in_dim);
        if (rc) return rc;
        if ((rc = check_f32(ys[i], out_dims[i] > 0))) return rc;
        work = work || out_dims[i] > 0;
        total += out_dims[i];
    }
    int rc = check_f32(x, work);
    if (rc || !work) return rc;
    if (!norm_weight) return QLIN_ERR_NULL;
    if (!aligned(norm_weight, 2)) return QLIN_ERR_ALIGN;
    if (!qlin::mfma_ok(type, weights, n_mats, rb, x, total, in_dim, false)) return QLIN_ERR_LIMIT;
    const qlin::RmsNorm norm{norm_weight, norm_type, eps, one_plus};
    return launched(qlin::mfma_gemv(type, weights, ys, out_dims, n_mats, rb, x, in_dim, false, stream(), &norm));
}

int qlin_launch_quant_gemv_argmax(int type, const uint8_t *w, size_t rb, const float *x, const uint16_t *norm_weight,
                                  int norm_type, float eps, int one_plus, float *logits, int out_dim, int in_dim,
                                  void *scratch, int *out_idx) {
    if (norm_weight && norm_type != 0 && norm_type != 1) return QLIN_ERR_SHAPE;
    int rc = check_weight(type, w, rb, out_dim, in_dim);
    if (rc) return rc;
    if (out_dim <= 0) return QLIN_ERR_SHAPE;
    if ((rc = check_f32(x, true)) || (rc = check_f32(logits, true))) return rc;
    if (!scratch || !out_idx) return QLIN_ERR_NULL;
    if (!aligned(scratch, 4) || !aligned(out_idx, 4) || !aligned(norm_weight, 2)) return QLIN_ERR_ALIGN;
    const uint8_t *ws[1] = {w};
    if (!qlin::mfma_ok(type, ws, 1, rb, x, out_dim, in_dim, false)) return QLIN_ERR_LIMIT;
    constexpr int kPairs = QLIN_GEMV_ARGMAX_SCRATCH_BYTES / 8;  // (float, int) per workgroup
    const int grid = qlin::mfma_gemv_pairs(type, w, rb, x, out_dim, in_dim);
    if (grid <= 0 || grid > kPairs) return QLIN_ERR_LIMIT;
    float *pv = static_cast<float *>(scratch);
    int *pi = reinterpret_cast<int *>(pv + kPairs);
    const qlin::RmsNorm norm{norm_weight, norm_type, eps, one_plus};
    return launched(qlin::mfma_gemv_argmax(type, w, rb, x, logits, out_dim, in_dim, norm_weight ? &norm : nullptr, pv,
                                           pi, out_idx, stream()));
}

int qlin_launch_rms_norm_quant_swiglu(int type, const uint8_t *wg, const uint8_t *wu, size_t rb, const float *x,
                                      const uint16_t *norm_weight, int norm_type, float eps, int one_plus,
                                      float *act, int ffn_dim, int in_dim) {
    if (norm_type != 0 && norm_type != 1) return QLIN_ERR_SHAPE;
    int rc = check_weight(type, wg, rb, ffn_dim, in_dim);
    if (rc || (rc = check_weight(type, wu, rb, ffn_dim, in_dim))) return rc;
    const bool work = ffn_dim > 0;
    if ((rc = check_f32(x, work)) || (rc = check_f32(act, work))) return rc;
    if (!work) return QLIN_OK;
    if (!norm_weight) return QLIN_ERR_NULL;
    if (!aligned(norm_weight, 2)) return QLIN_ERR_ALIGN;
    const uint8_t *gu[2] = {wg, wu};
    if (!qlin::mfma_ok(type, gu, 2, rb, x, ffn_dim, in_dim, true)) return QLIN_ERR_LIMIT;
    const qlin::RmsNorm norm{norm_weight, norm_type, eps, one_plus};
    return launched(qlin::mfma_swiglu(type, wg, wu, rb, x, act, ffn_dim, in_dim, stream(), &norm));
}

size_t qlin_q8_1_row_bytes(int in_dim) {
    return in_dim <= 0 ? 0 : static_cast<size_t>((in_dim + 31) / 32) * 36;
}

int qlin_launch_quantize_q8_1(const float *x, uint8_t *xq, int in_dim, int m, int store_raw_sum) {
    if (in_dim <= 0 || m < 0) return QLIN_ERR_SHAPE;
    if (m == 0) return QLIN_OK;
    int rc = check_f32(x, true);
    if (rc) return rc;
    if (!xq) return QLIN_ERR_NULL;
    if (!aligned(xq, 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::quantize_q8_1(x, xq, in_dim, m, store_raw_sum != 0, stream()));
}

int qlin_launch_quant_matmul_q8_1(int type, const uint8_t *w, size_t rb, const uint8_t *xq, float *y,
                                  int out_dim, int in_dim, int m) {
    int rc = check_weight(type, w, rb, out_dim, in_dim);
    if (rc) return rc;
    if (m < 0) return QLIN_ERR_SHAPE;
    const bool work = out_dim > 0 && m > 0;
    if (!work) return QLIN_OK;
    if (!xq) return QLIN_ERR_NULL;
    if (!aligned(xq, 2)) return QLIN_ERR_ALIGN;
    if ((rc = check_f32(y, true))) return rc;
    return launched(qlin::matmul_q8_1(type, w, rb, xq, y, out_dim, in_dim, m, stream()));
}

int qlin_launch_quant_gemv_q8_1(int type, const uint8_t *w, size_t rb, const uint8_t *xq, float *y, int out_dim,
                                int in_dim) {
    return qlin_launch_quant_matmul_q8_1(type, w, rb, xq, y, out_dim, in_dim, 1);
}

int qlin_launch_quantize_q8_1_mmq(const float *x, uint8_t *xq, int in_dim, int m, int store_raw_sum) {
    if (in_dim <= 0 || m < 0) return QLIN_ERR_SHAPE;
    if (m == 0) return QLIN_OK;
    int rc = check_f32(x, true);
    if (rc) return rc;
    if (!xq) return QLIN_ERR_NULL;
    if (!aligned(xq, 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::quantize_q8_1_mmq(x, xq, in_dim, m, store_raw_sum != 0, stream()));
}

int qlin_launch_quant_matmul_q8_1_mmq(int type, const uint8_t *w, size_t rb, const uint8_t *xq, float *y,
                                      int out_dim, int in_dim, int m) {
    if (type != QLIN_TYPE_Q4_K && type != QLIN_TYPE_Q6_K) return QLIN_ERR_UNSUPPORTED_TYPE;
    int rc = check_weight(type, w, rb, out_dim, in_dim);
    if (rc) return rc;
    if (m < 0) return QLIN_ERR_SHAPE;
    if (out_dim == 0 || m == 0) return QLIN_OK;
    if (!xq) return QLIN_ERR_NULL;
    if (!aligned(xq, 4)) return QLIN_ERR_ALIGN;
    if ((rc = check_f32(y, true))) return rc;
    return launched(qlin::matmul_q8_1_mmq(type, w, rb, xq, y, out_dim, in_dim, m, stream()));
}

int qlin_launch_quant_swiglu(int type, const uint8_t *wg, const uint8_t *wu, size_t g_rb, size_t u_rb,
                             const float *x, float *act, int ffn_dim, int in_dim) {
    int rc = check_weight(type, wg, g_rb, ffn_dim, in_dim);
    if (rc || (rc = check_weight(type, wu, u_rb, ffn_dim, in_dim))) return rc;
    const bool work = ffn_dim > 0;
    if ((rc = check_f32(x, work)) || (rc = check_f32(act, work))) return rc;
    if (!work) return QLIN_OK;
    return launched(qlin::swiglu(type, wg, wu, g_rb, u_rb, x, act, ffn_dim, in_dim, stream()));
}

int qlin_launch_quant_swiglu_rows(int type, const uint8_t *wg, const uint8_t *wu, size_t g_rb, size_t u_rb,
                                  const float *x, float *act, int ffn_dim, int in_dim, int m) {
    int rc = check_weight(type, wg, g_rb, ffn_dim, in_dim);
    if (rc || (rc = check_weight(type, wu, u_rb, ffn_dim, in_dim))) return rc;
    if (m < 0) return QLIN_ERR_SHAPE;
    const bool work = ffn_dim > 0 && m > 0;
    if ((rc = check_f32(x, work)) || (rc = check_f32(act, work))) return rc;
    if (!work) return QLIN_OK;
    if (m > 1 && g_rb == u_rb && qlin::dense_ok(type, wg, wu, g_rb, x, in_dim))
        return launched(qlin::dense_matmul(type, wg, wu, g_rb, x, act, ffn_dim, in_dim, m, 2, stream()));
    for (int r = 0; r < m; ++r) {
        const hipError_t e = qlin::swiglu(type, wg, wu, g_rb, u_rb, x + static_cast<size_t>(r) * in_dim,
                                          act + static_cast<size_t>(r) * ffn_dim, ffn_dim, in_dim, stream());
        if (e != hipSuccess) return launched(e);
    }
    return QLIN_OK;
}

int qlin_launch_quant_swiglu_indexed(int type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t u_eb,
                                     size_t g_rb, size_t u_rb, const float *x, const int *ids, float *act, int k,
                                     int ffn_dim, int in_dim) {
    int rc = check_weight(type, wg, g_rb, ffn_dim, in_dim);
    if (rc || (rc = check_weight(type, wu, u_rb, ffn_dim, in_dim))) return rc;
    if (k < 0) return QLIN_ERR_SHAPE;
    if (g_eb < g_rb * static_cast<size_t>(ffn_dim) || u_eb < u_rb * static_cast<size_t>(ffn_dim))
        return QLIN_ERR_ROW_BYTES;
    const bool work = ffn_dim > 0 && k > 0;
    if ((rc = check_f32(x, work)) || (rc = check_f32(act, work))) return rc;
    if (!work) return QLIN_OK;
    if (!ids) return QLIN_ERR_NULL;
    if (!aligned(ids, 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::swiglu_indexed(type, wg, wu, g_eb, u_eb, g_rb, u_rb, x, ids, act, k, ffn_dim, in_dim,
                                         stream()));
}

// gate/up of the experimental routed SwiGLU variants: Q4_K or Q6_K (launch.cu:262-318)
static int check_swiglu_experts(int type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t u_eb, size_t g_rb,
                                size_t u_rb, int k, int ffn_dim, int in_dim) {
    if (type != QLIN_TYPE_Q4_K && type != QLIN_TYPE_Q6_K) return QLIN_ERR_UNSUPPORTED_TYPE;
    int rc = check_weight(type, wg, g_rb, ffn_dim, in_dim);
    if (rc || (rc = check_weight(type, wu, u_rb, ffn_dim, in_dim))) return rc;
    if (k < 0) return QLIN_ERR_SHAPE;
    if (g_eb < g_rb * static_cast<size_t>(ffn_dim) || u_eb < u_rb * static_cast<size_t>(ffn_dim))
        return QLIN_ERR_ROW_BYTES;
    return QLIN_OK;
}

int qlin_launch_quant_swiglu_indexed_block(int type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t u_eb,
                                           size_t g_rb, size_t u_rb, const float *x, const int *ids, float *act, int k,
                                           int ffn_dim, int in_dim, int fast_silu) {
    (void)fast_silu;  // unused by the reference kernel as well (kernel.cu:1400)
    int rc = check_swiglu_experts(type, wg, wu, g_eb, u_eb, g_rb, u_rb, k, ffn_dim, in_dim);
    if (rc) return rc;
    return qlin_launch_quant_swiglu_indexed(type, wg, wu, g_eb, u_eb, g_rb, u_rb, x, ids, act, k, ffn_dim, in_dim);
}

int qlin_launch_quant_swiglu_indexed_q8_1(int type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t u_eb,
                                          size_t g_rb, size_t u_rb, const uint8_t *xq, const int *ids, float *act,
                                          int k, int ffn_dim, int in_dim) {
    int rc = check_swiglu_experts(type, wg, wu, g_eb, u_eb, g_rb, u_rb, k, ffn_dim, in_dim);
    if (rc) return rc;
    const bool work = ffn_dim > 0 && k > 0;
    if ((rc = check_f32(act, work))) return rc;
    if (!work) return QLIN_OK;
    if (!xq || !ids) return QLIN_ERR_NULL;
    if (!aligned(xq, 2) || !aligned(ids, 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::swiglu_indexed_q8_1(type, wg, wu, g_eb, u_eb, g_rb, u_rb, xq, ids, act, k, ffn_dim, in_dim,
                                              stream()));
}

static int down_q8_1_common(int type, bool f32_act, const uint8_t *wd, size_t d_eb, size_t d_rb, const void *act,
                            const int *ids, const float *rw, float *out, int k, int hidden, int ffn_dim) {
    if (type != QLIN_TYPE_Q4_K && type != QLIN_TYPE_Q6_K && type != QLIN_TYPE_Q5_0 && type != QLIN_TYPE_Q8_0)
        return QLIN_ERR_UNSUPPORTED_TYPE;
    int rc = check_weight(type, wd, d_rb, hidden, ffn_dim);
    if (rc) return rc;
    if (k < 0) return QLIN_ERR_SHAPE;
    if (d_eb < d_rb * static_cast<size_t>(hidden)) return QLIN_ERR_ROW_BYTES;
    if (f32_act && static_cast<size_t>(ffn_dim / 32) * 36 > 160 * 1024) return QLIN_ERR_LIMIT;
    const bool work = hidden > 0 && k > 0;
    if ((rc = check_f32(out, hidden > 0)) || (rc = check_f32(rw, work))) return rc;
    if (!work) return QLIN_OK;
    if (!act || !ids) return QLIN_ERR_NULL;
    if (!aligned(act, f32_act ? 4 : 2) || !aligned(ids, 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::down_q8_1_indexed_accum(type, f32_act, wd, d_eb, d_rb, act, ids, rw, out, k, hidden, ffn_dim,
                                                  stream()));
}

int qlin_launch_quant_down_q8_1_indexed_accum(int type, const uint8_t *wd, size_t d_eb, size_t d_rb,
                                              const uint8_t *act_q8_1, const int *ids, const float *rw, float *out,
                                              int k, int hidden, int ffn_dim) {
    return down_q8_1_common(type, false, wd, d_eb, d_rb, act_q8_1, ids, rw, out, k, hidden, ffn_dim);
}

int qlin_launch_quant_down_q8_1_indexed_accum_shared(int type, const uint8_t *wd, size_t d_eb, size_t d_rb,
                                                     const uint8_t *act_q8_1, const int *ids, const float *rw,
                                                     float *out, int k, int hidden, int ffn_dim) {
    return down_q8_1_common(type, false, wd, d_eb, d_rb, act_q8_1, ids, rw, out, k, hidden, ffn_dim);
}

int qlin_launch_quant_down_f32_indexed_accum(int type, const uint8_t *wd, size_t d_eb, size_t d_rb, const float *act,
                                             const int *ids, const float *rw, float *out, int k, int hidden,
                                             int ffn_dim) {
    return down_q8_1_common(type, true, wd, d_eb, d_rb, act, ids, rw, out, k, hidden, ffn_dim);
}

int qlin_launch_quant_down_f32_indexed_accum_ordered(int type, const uint8_t *wd, size_t d_eb, size_t d_rb,
                                                     const float *act, const int *ids, const float *rw,
                                                     float *out, int k, int hidden, int ffn_dim) {
    int rc = check_weight(type, wd, d_rb, hidden, ffn_dim);
    if (rc) return rc;
    if (k < 0) return QLIN_ERR_SHAPE;
    if (d_eb < d_rb * static_cast<size_t>(hidden)) return QLIN_ERR_ROW_BYTES;
    const bool work = hidden > 0;
    if ((rc = check_f32(out, work)) || (rc = check_f32(act, work && k > 0)) || (rc = check_f32(rw, work && k > 0)))
        return rc;
    if (!work) return QLIN_OK;
    if (k > 0 && !ids) return QLIN_ERR_NULL;
    if (!aligned(ids, 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::down_indexed_ordered(type, wd, d_eb, d_rb, act, ids, rw, out, k, hidden, ffn_dim, stream()));
}

int qlin_launch_moe_router_topk(const float *logits, int *idx, float *w, int tokens, int n_experts, int k,
                                float routed_scaling) {
    if (tokens < 0 || k < 0 || n_experts <= 0) return QLIN_ERR_SHAPE;
    if (n_experts > 256) return QLIN_ERR_LIMIT;
    if (tokens == 0 || k == 0) return QLIN_OK;
    int rc = check_f32(logits, true);
    if (rc || (rc = check_f32(w, true))) return rc;
    if (!idx) return QLIN_ERR_NULL;
    if (!aligned(idx, 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::router_topk(logits, idx, w, tokens, n_experts, k, routed_scaling, stream()));
}

int qlin_launch_moe_accumulate(const float *expert_out, float weight, float *out, int n) {
    if (n < 0) return QLIN_ERR_SHAPE;
    if (n == 0) return QLIN_OK;
    int rc;
    if ((rc = check_f32(expert_out, true)) || (rc = check_f32(out, true))) return rc;
    return launched(qlin::moe_accumulate(expert_out, weight, nullptr, out, n, stream()));
}

int qlin_launch_moe_accumulate_device(const float *expert_out, const float *weight, float *out, int n) {
    if (n < 0) return QLIN_ERR_SHAPE;
    if (n == 0) return QLIN_OK;
    int rc;
    if ((rc = check_f32(expert_out, true)) || (rc = check_f32(out, true)) || (rc = check_f32(weight, true))) return rc;
    return launched(qlin::moe_accumulate(expert_out, 0.0f, weight, out, n, stream()));
}

int qlin_launch_argmax(const float *logits, int n, int *out_idx) {
    if (n <= 0) return QLIN_ERR_SHAPE;
    int rc = check_f32(logits, true);
    if (rc) return rc;
    if (!out_idx) return QLIN_ERR_NULL;
    if (!aligned(out_idx, 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::argmax(logits, n, out_idx, stream()));
}

static int dequant_common(int type, const uint8_t *src, void *out, int64_t n, bool f16) {
    if (!known_weight_type(type)) return QLIN_ERR_UNSUPPORTED_TYPE;
    if (n < 0 || n % elems_of(type)) return QLIN_ERR_SHAPE;
    if (n == 0) return QLIN_OK;
    if (!src || !out) return QLIN_ERR_NULL;
    if (!aligned(src, 2) || !aligned(out, f16 ? 2 : 4)) return QLIN_ERR_ALIGN;
    return launched(qlin::dequant(type, src, out, n, f16, stream()));
}

int qlin_launch_dequantize_to_f16(int type, const uint8_t *src, uint16_t *out, int64_t n) {
    return dequant_common(type, src, out, n, true);
}
int qlin_launch_dequantize_q4k_to_f16(const uint8_t *src, uint16_t *out, int64_t n) {
    return dequant_common(QLIN_TYPE_Q4_K, src, out, n, true);
}
int qlin_launch_dequantize_q80_to_f16(const uint8_t *src, uint16_t *out, int64_t n) {
    return dequant_common(QLIN_TYPE_Q8_0, src, out, n, true);
}
int qlin_launch_dequantize_q50_to_f16(const uint8_t *src, uint16_t *out, int64_t n) {
    return dequant_common(QLIN_TYPE_Q5_0, src, out, n, true);
}
int qlin_launch_dequantize_q6k_to_f16(const uint8_t *src, uint16_t *out, int64_t n) {
    return dequant_common(QLIN_TYPE_Q6_K, src, out, n, true);
}
int qlin_launch_dequantize_to_f32(int type, const uint8_t *src, float *out, int64_t n) {
    return dequant_common(type, src, out, n, false);
}

int qlin_gemm(int type, const uint8_t *w, size_t weight_bytes, const float *x, float *y, int out_dim, int in_dim,
              int m) {
    if (out_dim < 0) return QLIN_ERR_SHAPE;
    const size_t rb = out_dim > 0 ? weight_bytes / static_cast<size_t>(out_dim) : min_row_bytes(type, in_dim);
    return gemv_common(type, w, rb, x, y, out_dim, in_dim, m, false);
}

int qlin_moe_routed_decode_indexed(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes,
                                   int down_type, const uint8_t *down, size_t down_bytes, int n_experts, int ffn_dim,
                                   int in_dim, int hidden, const float *x, const int *ids, const float *rw,
                                   float *act, float *out, int k) {
    // TensorTool.cpp:277-305, in the reference's order of checks.
    if (!ids || !rw) return QLIN_ERR_NULL;
    if (down_type != QLIN_TYPE_Q4_K && down_type != QLIN_TYPE_Q6_K && down_type != QLIN_TYPE_Q5_0 &&
        down_type != QLIN_TYPE_Q8_0)
        return QLIN_ERR_UNSUPPORTED_TYPE;
    if (gu_type != QLIN_TYPE_Q4_K && gu_type != QLIN_TYPE_Q6_K) return QLIN_ERR_UNSUPPORTED_TYPE;
    if (n_experts <= 0 || ffn_dim <= 0 || in_dim <= 0 || hidden <= 0 || k < 0) return QLIN_ERR_SHAPE;
    const size_t g_eb = gate_up_bytes / static_cast<size_t>(n_experts);
    const size_t d_eb = down_bytes / static_cast<size_t>(n_experts);
    const size_t g_rb = g_eb / static_cast<size_t>(ffn_dim);
    const size_t d_rb = d_eb / static_cast<size_t>(hidden);
    if (!act) return QLIN_ERR_NULL;
    // the down projection is validated before anything is launched, so a rejection launches nothing
    int rc = check_weight(down_type, down, d_rb, hidden, ffn_dim);
    if (rc) return rc;
    if ((rc = check_f32(out, true)) || (rc = check_f32(rw, k > 0))) return rc;
    rc = qlin_launch_quant_swiglu_indexed(gu_type, gate, up, g_eb, g_eb, g_rb, g_rb, x, ids, act, k, ffn_dim,
                                              in_dim);
    if (rc) return rc;
    return qlin_launch_quant_down_f32_indexed_accum_ordered(down_type, down, d_eb, d_rb, act, ids, rw, out, k,
                                                            hidden, ffn_dim);
}

// The per-token call from logits: qlin_moe_routed_decode_indexed's checks (ids and rw are written here),
// all before anything runs.
static int indexed_logits_check(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes,
                                int down_type, const uint8_t *down, size_t down_bytes, int n_experts, int ffn_dim,
                                int in_dim, int hidden, const float *x, const float *router_logits, int *ids,
                                float *rw, float *act, float *out, int k) {
    if (!ids || !rw || !router_logits) return QLIN_ERR_NULL;
    if (down_type != QLIN_TYPE_Q4_K && down_type != QLIN_TYPE_Q6_K && down_type != QLIN_TYPE_Q5_0 &&
        down_type != QLIN_TYPE_Q8_0)
        return QLIN_ERR_UNSUPPORTED_TYPE;
    if (gu_type != QLIN_TYPE_Q4_K && gu_type != QLIN_TYPE_Q6_K) return QLIN_ERR_UNSUPPORTED_TYPE;
    if (n_experts <= 0 || ffn_dim <= 0 || in_dim <= 0 || hidden <= 0 || k < 0) return QLIN_ERR_SHAPE;
    if (n_experts > 256) return QLIN_ERR_LIMIT;  // the router's limit
    const size_t g_eb = gate_up_bytes / static_cast<size_t>(n_experts);
    const size_t d_eb = down_bytes / static_cast<size_t>(n_experts);
    const size_t g_rb = g_eb / static_cast<size_t>(ffn_dim);
    const size_t d_rb = d_eb / static_cast<size_t>(hidden);
    if (!act) return QLIN_ERR_NULL;
    int rc = check_weight(down_type, down, d_rb, hidden, ffn_dim);
    if (rc || (rc = check_weight(gu_type, gate, g_rb, ffn_dim, in_dim)) ||
        (rc = check_weight(gu_type, up, g_rb, ffn_dim, in_dim)))
        return rc;
    if ((rc = check_f32(out, true)) || (rc = check_f32(rw, true)) || (rc = check_f32(x, true)) ||
        (rc = check_f32(act, true)) || (rc = check_f32(router_logits, true)))
        return rc;
    if (!aligned(ids, 4)) return QLIN_ERR_ALIGN;
    return QLIN_OK;
}

int qlin_moe_routed_decode_indexed_logits(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes,
                                          int down_type, const uint8_t *down, size_t down_bytes, int n_experts,
                                          int ffn_dim, int in_dim, int hidden, const float *x,
                                          const float *router_logits, float routed_scaling, int *ids, float *rw,
                                          float *act, float *out, int k) {
    int rc = indexed_logits_check(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes, n_experts, ffn_dim,
                                  in_dim, hidden, x, router_logits, ids, rw, act, out, k);
    if (rc || k == 0) return rc;
    const size_t g_eb = gate_up_bytes / static_cast<size_t>(n_experts);
    const size_t d_eb = down_bytes / static_cast<size_t>(n_experts);
    const size_t g_rb = g_eb / static_cast<size_t>(ffn_dim);
    const size_t d_rb = d_eb / static_cast<size_t>(hidden);
    if (n_experts <= 64 && qlin::mfma_routed_ok(gu_type, true, gate, up, g_eb, g_rb, x, k, ffn_dim, in_dim)) {
        // the routing in the gate/up launch (its workgroup 0 writes ids and rw), then the down launch
        const qlin::MoeRouter router{router_logits, routed_scaling, ids, rw};
        const hipError_t e = qlin::mfma_swiglu_routed(gu_type, gate, up, g_eb, g_rb, x, nullptr, act, k, ffn_dim,
                                                      in_dim, stream(), &router, n_experts);
        if (e != hipSuccess) return QLIN_ERR_LAUNCH;
        return qlin_launch_quant_down_f32_indexed_accum_ordered(down_type, down, d_eb, d_rb, act, ids, rw, out, k,
                                                                hidden, ffn_dim);
    }
    if ((rc = qlin_launch_moe_router_topk(router_logits, ids, rw, 1, n_experts, k, routed_scaling))) return rc;
    return qlin_moe_routed_decode_indexed(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes, n_experts,
                                          ffn_dim, in_dim, hidden, x, ids, rw, act, out, k);
}

// MoE::forward for one token (MoE.cpp:29-52 after the norm, before the residual add): the routed experts
// from the logits, then the shared experts.  Where the routed SwiGLU takes the shared gate and up rows as
// extra routes (same format and row stride, shared_ffn a multiple of ffn_dim, at most 16 routes in all,
// up to 64 experts) that is 3 launches instead of 4: routing + routed and shared SwiGLU, routed down,
// shared down-add.  Either way out gets (out + routed) + shared, bit for bit as the separate calls.
int qlin_moe_ffn_decode_indexed_logits(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes,
                                       int down_type, const uint8_t *down, size_t down_bytes, int n_experts,
                                       int ffn_dim, int in_dim, int hidden, int shared_type, const uint8_t *shared_gate,
                                       const uint8_t *shared_up, size_t shared_gate_up_rb, const uint8_t *shared_down,
                                       size_t shared_down_rb, int shared_ffn, const float *x,
                                       const float *router_logits, float routed_scaling, int *ids, float *rw,
                                       float *act, float *out, int k) {
    if (shared_ffn < 0) return QLIN_ERR_SHAPE;
    int rc = indexed_logits_check(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes, n_experts, ffn_dim,
                                  in_dim, hidden, x, router_logits, ids, rw, act, out, k);
    if (rc) return rc;
    const bool shared = shared_ffn > 0;
    if (shared) {
        if ((rc = check_weight(shared_type, shared_gate, shared_gate_up_rb, shared_ffn, in_dim)) ||
            (rc = check_weight(shared_type, shared_up, shared_gate_up_rb, shared_ffn, in_dim)) ||
            (rc = check_weight(shared_type, shared_down, shared_down_rb, hidden, shared_ffn)))
            return rc;
    }
    float *sact = act + static_cast<size_t>(k) * ffn_dim;  // the shared activations follow the routes'
    const size_t g_eb = gate_up_bytes / static_cast<size_t>(n_experts);
    const size_t g_rb = g_eb / static_cast<size_t>(ffn_dim);
    const int n_sh = shared && shared_ffn % ffn_dim == 0 ? shared_ffn / ffn_dim : 0;
    const bool fuse = k > 0 && n_sh > 0 && n_experts <= 64 && shared_type == gu_type && shared_gate_up_rb == g_rb &&
                      qlin::mfma_routed_ok(gu_type, true, gate, up, g_eb, g_rb, x, k + n_sh, ffn_dim, in_dim) &&
                      qlin::mfma_routed_ok(gu_type, true, shared_gate, shared_up, g_eb, g_rb, x, k + n_sh, ffn_dim,
                                           in_dim);
    if (fuse) {
        const size_t d_eb = down_bytes / static_cast<size_t>(n_experts);
        const size_t d_rb = d_eb / static_cast<size_t>(hidden);
        const qlin::MoeRouter router{router_logits, routed_scaling, ids, rw};
        const hipError_t e = qlin::mfma_swiglu_routed(gu_type, gate, up, g_eb, g_rb, x, nullptr, act, k, ffn_dim,
                                                      in_dim, stream(), &router, n_experts, shared_gate, shared_up,
                                                      n_sh);
        if (e != hipSuccess) return QLIN_ERR_LAUNCH;
        if ((rc = qlin_launch_quant_down_f32_indexed_accum_ordered(down_type, down, d_eb, d_rb, act, ids, rw, out, k,
                                                                    hidden, ffn_dim)))
            return rc;
        return qlin_launch_quant_gemv_add(shared_type, shared_down, shared_down_rb, sact, out, hidden, shared_ffn);
    }
    if ((rc = qlin_moe_routed_decode_indexed_logits(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes,
                                                    n_experts, ffn_dim, in_dim, hidden, x, router_logits,
                                                    routed_scaling, ids, rw, act, out, k)))
        return rc;
    if (!shared) return QLIN_OK;
    if ((rc = qlin_launch_quant_swiglu(shared_type, shared_gate, shared_up, shared_gate_up_rb, shared_gate_up_rb, x,
                                       sact, shared_ffn, in_dim)))
        return rc;
    return qlin_launch_quant_gemv_add(shared_type, shared_down, shared_down_rb, sact, out, hidden, shared_ffn);
}

static bool embed_mla_type(int t) {
    return t == QLIN_TYPE_Q4_K || t == QLIN_TYPE_Q6_K || t == QLIN_TYPE_Q5_0 || t == QLIN_TYPE_Q8_0;
}

int qlin_launch_quant_embedding(int type, const int *input, float *output, const uint8_t *table, size_t rb,
                                int hidden, int input_size) {
    if (!embed_mla_type(type)) return QLIN_ERR_UNSUPPORTED_TYPE;
    if (hidden < 0 || input_size < 0 || hidden % elems_of(type)) return QLIN_ERR_SHAPE;
    if (rb < min_row_bytes(type, hidden)) return QLIN_ERR_ROW_BYTES;
    const bool work = hidden > 0 && input_size > 0;
    if (!work) return QLIN_OK;
    if (!input || !table) return QLIN_ERR_NULL;
    int rc = check_f32(output, true);
    if (rc) return rc;
    if (!aligned(input, 4) || !aligned(table, 2) || rb % 2) return QLIN_ERR_ALIGN;
    return launched(qlin::quant_embedding(type, input, output, table, rb, hidden, input_size, stream()));
}

// kv_b of n_heads * (qk_nope + v_head) rows of kv_lora weights
static int check_kv_b(int type, const uint8_t *w, size_t rb, int n_heads, int qk_nope, int qk_rope, int v_head,
                      int kv_lora) {
    if (!embed_mla_type(type)) return QLIN_ERR_UNSUPPORTED_TYPE;
    if (n_heads < 0 || qk_nope < 0 || qk_rope < 0 || v_head < 0 || kv_lora < 0 || kv_lora % elems_of(type))
        return QLIN_ERR_SHAPE;
    if (rb < min_row_bytes(type, kv_lora)) return QLIN_ERR_ROW_BYTES;
    if (!aligned(w, 2) || rb % 2) return QLIN_ERR_ALIGN;
    return QLIN_OK;
}

int qlin_launch_mla_absorb_q_nope(int type, const float *q, const uint8_t *w, size_t rb, float *q_abs, int n_heads,
                                  int qk_nope, int qk_rope, int v_head, int kv_lora) {
    int rc = check_kv_b(type, w, rb, n_heads, qk_nope, qk_rope, v_head, kv_lora);
    if (rc) return rc;
    const bool work = n_heads > 0 && kv_lora > 0;
    if (!work) return QLIN_OK;
    if (!w) return QLIN_ERR_NULL;
    if ((rc = check_f32(q_abs, true)) || (rc = check_f32(q, qk_nope > 0))) return rc;
    return launched(qlin::mla_absorb_q_nope(type, q, w, rb, q_abs, n_heads, qk_nope, qk_rope, v_head, kv_lora,
                                            stream()));
}

int qlin_launch_mla_absorb_q4_xsum_delta(const float *q, const uint8_t *w, size_t rb, float *delta, int n_heads,
                                         int qk_nope, int qk_rope, int v_head, int kv_lora) {
    int rc = check_kv_b(QLIN_TYPE_Q4_K, w, rb, n_heads, qk_nope, qk_rope, v_head, kv_lora);
    if (rc) return rc;
    const bool work = n_heads > 0 && kv_lora > 0;
    if (!work) return QLIN_OK;
    if (!w) return QLIN_ERR_NULL;
    if ((rc = check_f32(delta, true)) || (rc = check_f32(q, qk_nope > 0))) return rc;
    return launched(qlin::mla_absorb_q4_xsum_delta(q, w, rb, delta, n_heads, qk_nope, qk_rope, v_head, kv_lora,
                                                   stream()));
}

int qlin_launch_mla_absorb_v(int type, const uint8_t *w, size_t rb, const float *latent, const float *delta,
                             float *attn, int n_heads, int qk_nope, int v_head, int kv_lora) {
    int rc = check_kv_b(type, w, rb, n_heads, qk_nope, 0, v_head, kv_lora);
    if (rc) return rc;
    const bool work = n_heads > 0 && v_head > 0;
    if (!work) return QLIN_OK;
    if (!w) return QLIN_ERR_NULL;
    if ((rc = check_f32(attn, true)) || (rc = check_f32(latent, kv_lora > 0)) ||
        (rc = check_f32(delta, type == QLIN_TYPE_Q4_K && kv_lora > 0)))
        return rc;
    return launched(qlin::mla_absorb_v(type, w, rb, latent, delta, attn, n_heads, qk_nope, v_head, kv_lora,
                                       stream()));
}

// a Q8_1 latent cache: rows of at least ceil(kv_lora / 32) blocks, 4-aligned
static int check_latent_cache(const uint8_t *cache, size_t crb, int kv_lora) {
    if (crb < qlin_q8_1_row_bytes(kv_lora)) return QLIN_ERR_ROW_BYTES;
    if (!cache) return QLIN_ERR_NULL;
    if (!aligned(cache, 4) || crb % 4) return QLIN_ERR_ALIGN;
    return QLIN_OK;
}

static int check_pos(const int *d_pos) {
    if (!d_pos) return QLIN_ERR_NULL;
    return aligned(d_pos, 4) ? QLIN_OK : QLIN_ERR_ALIGN;
}

int qlin_launch_mla_store_latent_q8_1_device_pos(const float *kv_cache, uint8_t *cache, int kv_lora, int qk_rope,
                                                 size_t row_bytes, const int *d_pos) {
    if (kv_lora <= 0 || qk_rope < 0) return QLIN_ERR_SHAPE;
    int rc = check_latent_cache(cache, row_bytes, kv_lora);
    if (rc || (rc = check_f32(kv_cache, true)) || (rc = check_pos(d_pos))) return rc;
    return launched(qlin::mla_store_latent_q8_1(kv_cache, cache, kv_lora, qk_rope, row_bytes, d_pos, stream()));
}

int qlin_launch_mla_absorb_scores_device_pos(const float *q_abs, const float *q, const uint8_t *cache, size_t crb,
                                             const float *q_abs_xsum_delta, const float *kv_cache, float *scores,
                                             int n_heads, int qk_nope, int qk_rope, int kv_lora, const int *d_pos,
                                             int max_seq_len, float softmax_scale) {
    if (n_heads < 0 || qk_nope < 0 || qk_rope < 0 || kv_lora <= 0 || max_seq_len < 0) return QLIN_ERR_SHAPE;
    if (n_heads == 0 || max_seq_len == 0) return QLIN_OK;
    int rc = check_latent_cache(cache, crb, kv_lora);
    if (rc || (rc = check_f32(q_abs, true)) || (rc = check_f32(q, qk_rope > 0)) ||
        (rc = check_f32(q_abs_xsum_delta, true)) || (rc = check_f32(kv_cache, qk_rope > 0)) ||
        (rc = check_f32(scores, true)) || (rc = check_pos(d_pos)))
        return rc;
    return launched(qlin::mla_absorb_scores(q_abs, q, cache, crb, q_abs_xsum_delta, kv_cache, scores, n_heads, qk_nope,
                                            qk_rope, kv_lora, d_pos, max_seq_len, softmax_scale, stream()));
}

int qlin_launch_mla_absorb_context_device_pos(const float *scores, const uint8_t *cache, size_t crb,
                                              float *attn_xsum_delta, float *attn_latent, int n_heads, int kv_lora,
                                              const int *d_pos, int max_seq_len) {
    if (n_heads < 0 || kv_lora <= 0 || max_seq_len <= 0) return QLIN_ERR_SHAPE;
    if (n_heads == 0) return QLIN_OK;
    int rc = check_latent_cache(cache, crb, kv_lora);
    if (rc || (rc = check_f32(scores, true)) || (rc = check_f32(attn_xsum_delta, true)) ||
        (rc = check_f32(attn_latent, true)) || (rc = check_pos(d_pos)))
        return rc;
    return launched(qlin::mla_absorb_context(scores, cache, crb, attn_xsum_delta, attn_latent, n_heads, kv_lora, d_pos,
                                             max_seq_len, stream()));
}

int qlin_launch_mla_absorb_attend_device_pos(const float *q_abs, const float *q, const uint8_t *cache, size_t crb,
                                             const float *q_abs_xsum_delta, float *attn_xsum_delta,
                                             const float *kv_cache, float *attn_latent, int n_heads, int qk_nope,
                                             int qk_rope, int kv_lora, const int *d_pos, int max_seq_len,
                                             float softmax_scale) {
    if (n_heads < 0 || qk_nope < 0 || qk_rope < 0 || kv_lora <= 0 || max_seq_len <= 0) return QLIN_ERR_SHAPE;
    if (!qlin::mla_attend_ok(max_seq_len, kv_lora, qk_rope)) return QLIN_ERR_LIMIT;
    if (n_heads == 0) return QLIN_OK;
    int rc = check_latent_cache(cache, crb, kv_lora);
    if (rc || (rc = check_f32(q_abs, true)) || (rc = check_f32(q, qk_rope > 0)) ||
        (rc = check_f32(q_abs_xsum_delta, true)) || (rc = check_f32(attn_xsum_delta, true)) ||
        (rc = check_f32(kv_cache, qk_rope > 0)) || (rc = check_f32(attn_latent, true)) || (rc = check_pos(d_pos)))
        return rc;
    return launched(qlin::mla_absorb_attend(q_abs, q, cache, crb, q_abs_xsum_delta, attn_xsum_delta, kv_cache,
                                            attn_latent, n_heads, qk_nope, qk_rope, kv_lora, d_pos, max_seq_len,
                                            softmax_scale, stream()));
}

int qlin_launch_mla_project_v_device_pos(int type, const uint8_t *w, size_t rb, const uint8_t *cache, size_t crb,
                                         float *kv_b_cache, int n_heads, int qk_nope, int v_head, int kv_lora,
                                         const int *d_pos) {
    int rc = check_kv_b(type, w, rb, n_heads, qk_nope, 0, v_head, kv_lora);
    if (rc) return rc;
    if (n_heads == 0 || v_head == 0) return QLIN_OK;
    if (kv_lora == 0) return QLIN_ERR_SHAPE;
    if (!w) return QLIN_ERR_NULL;
    if ((rc = check_latent_cache(cache, crb, kv_lora)) || (rc = check_f32(kv_b_cache, true)) || (rc = check_pos(d_pos)))
        return rc;
    return launched(qlin::mla_project_v(type, w, rb, cache, crb, kv_b_cache, n_heads, qk_nope, v_head, kv_lora, d_pos,
                                        stream()));
}

int qlin_launch_mla_absorb_context_v_device_pos(const float *scores, const float *kv_b_cache, float *attn,
                                                int n_heads, int qk_nope, int v_head, const int *d_pos,
                                                int max_seq_len) {
    if (n_heads < 0 || qk_nope < 0 || v_head < 0 || max_seq_len <= 0) return QLIN_ERR_SHAPE;
    if (v_head > 256) return QLIN_ERR_LIMIT;
    if (n_heads == 0 || v_head == 0) return QLIN_OK;
    int rc;
    if ((rc = check_f32(scores, true)) || (rc = check_f32(kv_b_cache, true)) || (rc = check_f32(attn, true)) ||
        (rc = check_pos(d_pos)))
        return rc;
    return launched(qlin::mla_absorb_context_v(scores, kv_b_cache, attn, n_heads, qk_nope, v_head, d_pos, max_seq_len,
                                               stream()));
}

size_t qlin_moe_grouped_workspace_bytes(int tokens, int k, int n_experts, int ffn_dim, int hidden_size) {
    if (tokens < 0 || k < 0 || n_experts <= 0 || ffn_dim <= 0 || hidden_size <= 0) return 0;
    return qlin::moe_grouped_workspace(tokens, k, n_experts, ffn_dim, hidden_size);
}

// The batched decode's checks: the per-token facade's rules (TensorTool.cpp:277-305) plus the batch's own.
static int grouped_check(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes, int down_type,
                         const uint8_t *down, size_t down_bytes, int n_experts, int ffn_dim, int in_dim, int hidden,
                         const float *x, const int *ids, const float *rw, const void *workspace,
                         size_t workspace_bytes, const float *out, int tokens, int k) {
    if (down_type != QLIN_TYPE_Q4_K && down_type != QLIN_TYPE_Q6_K && down_type != QLIN_TYPE_Q5_0 &&
        down_type != QLIN_TYPE_Q8_0)
        return QLIN_ERR_UNSUPPORTED_TYPE;
    if (gu_type != QLIN_TYPE_Q4_K && gu_type != QLIN_TYPE_Q6_K) return QLIN_ERR_UNSUPPORTED_TYPE;
    if (n_experts <= 0 || ffn_dim <= 0 || in_dim <= 0 || hidden <= 0 || k < 0 || tokens < 0) return QLIN_ERR_SHAPE;
    if (!qlin::moe_grouped_shape_ok(n_experts, static_cast<int64_t>(tokens) * k)) return QLIN_ERR_LIMIT;
    const bool work = tokens > 0 && k > 0;
    if (work && (!ids || !rw || !x || !out || !workspace)) return QLIN_ERR_NULL;
    if (work && workspace_bytes < qlin::moe_grouped_workspace(tokens, k, n_experts, ffn_dim, hidden))
        return QLIN_ERR_LIMIT;
    if (work && (reinterpret_cast<uintptr_t>(workspace) & 255u)) return QLIN_ERR_ALIGN;
    const size_t g_eb = gate_up_bytes / static_cast<size_t>(n_experts);
    const size_t d_eb = down_bytes / static_cast<size_t>(n_experts);
    const size_t g_rb = g_eb / static_cast<size_t>(ffn_dim);
    const size_t d_rb = d_eb / static_cast<size_t>(hidden);
    int rc = check_weight(down_type, down, d_rb, hidden, ffn_dim);
    if (rc || (rc = check_weight(gu_type, gate, g_rb, ffn_dim, in_dim)) ||
        (rc = check_weight(gu_type, up, g_rb, ffn_dim, in_dim)))
        return rc;
    if ((rc = check_f32(x, work)) || (rc = check_f32(out, work)) || (rc = check_f32(rw, work))) return rc;
    if (work && !aligned(ids, 4)) return QLIN_ERR_ALIGN;
    return QLIN_OK;
}

int qlin_moe_routed_decode_grouped(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes,
                                   int down_type, const uint8_t *down, size_t down_bytes, int n_experts, int ffn_dim,
                                   int in_dim, int hidden, const float *x, const int *ids, const float *rw,
                                   void *workspace, size_t workspace_bytes, float *out, int tokens, int k) {
    int rc = grouped_check(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes, n_experts, ffn_dim, in_dim,
                           hidden, x, ids, rw, workspace, workspace_bytes, out, tokens, k);
    if (rc || tokens == 0 || k == 0) return rc;
    const size_t g_eb = gate_up_bytes / static_cast<size_t>(n_experts);
    const size_t d_eb = down_bytes / static_cast<size_t>(n_experts);
    const size_t g_rb = g_eb / static_cast<size_t>(ffn_dim);
    const size_t d_rb = d_eb / static_cast<size_t>(hidden);
    if (qlin::moe_grouped_up_ok(gu_type, gate, up, g_eb, g_rb, x, in_dim, ffn_dim, n_experts, tokens * k))
        return launched(qlin::moe_grouped(gu_type, gate, up, g_eb, g_rb, down_type, down, d_eb, d_rb, n_experts,
                                          ffn_dim, in_dim, hidden, x, ids, rw, workspace, out, tokens, k, stream()));
    // other layouts: the per-token kernels, token by token, with act in the workspace
    float *act = static_cast<float *>(workspace);
    for (int t = 0; t < tokens; ++t) {
        const float *xt = x + static_cast<size_t>(t) * in_dim;
        const int *it = ids + static_cast<size_t>(t) * k;
        const float *wt = rw + static_cast<size_t>(t) * k;
        hipError_t e = qlin::swiglu_indexed(gu_type, gate, up, g_eb, g_eb, g_rb, g_rb, xt, it, act, k, ffn_dim,
                                            in_dim, stream());
        if (e == hipSuccess)
            e = qlin::down_indexed_ordered(down_type, down, d_eb, d_rb, act, it, wt,
                                           out + static_cast<size_t>(t) * hidden, k, hidden, ffn_dim, stream());
        if (e != hipSuccess) return QLIN_ERR_LAUNCH;
    }
    return QLIN_OK;
}

int qlin_moe_routed_decode_grouped_logits(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes,
                                          int down_type, const uint8_t *down, size_t down_bytes, int n_experts,
                                          int ffn_dim, int in_dim, int hidden, const float *x,
                                          const float *router_logits, float routed_scaling, int *ids, float *rw,
                                          void *workspace, size_t workspace_bytes, float *out, int tokens, int k) {
    int rc = grouped_check(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes, n_experts, ffn_dim, in_dim,
                           hidden, x, ids, rw, workspace, workspace_bytes, out, tokens, k);
    if (rc || tokens == 0 || k == 0) return rc;
    if (n_experts > 256) return QLIN_ERR_LIMIT;  // the router's limit
    if ((rc = check_f32(router_logits, true))) return rc;
    const size_t g_eb = gate_up_bytes / static_cast<size_t>(n_experts);
    const size_t g_rb = g_eb / static_cast<size_t>(ffn_dim);
    if (qlin::moe_grouped_up_ok(gu_type, gate, up, g_eb, g_rb, x, in_dim, ffn_dim, n_experts, tokens * k)) {
        const size_t d_eb = down_bytes / static_cast<size_t>(n_experts);
        const size_t d_rb = d_eb / static_cast<size_t>(hidden);
        const qlin::MoeRouter router{router_logits, routed_scaling, ids, rw};
        return launched(qlin::moe_grouped(gu_type, gate, up, g_eb, g_rb, down_type, down, d_eb, d_rb, n_experts,
                                          ffn_dim, in_dim, hidden, x, nullptr, nullptr, workspace, out, tokens, k,
                                          stream(), &router));
    }
    // other layouts: the router, then the batched call's per-token path
    if ((rc = qlin_launch_moe_router_topk(router_logits, ids, rw, tokens, n_experts, k, routed_scaling))) return rc;
    return qlin_moe_routed_decode_grouped(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes, n_experts,
                                          ffn_dim, in_dim, hidden, x, ids, rw, workspace, workspace_bytes, out, tokens,
                                          k);
}

int qlin_moe_routed_decode_grouped_noalloc(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes,
                                           int down_type, const uint8_t *down, size_t down_bytes, int n_experts,
                                           int ffn_dim, int in_dim, int hidden, const float *x, const int *ids,
                                           const float *rw, float *out, int tokens, int k) {
    static_assert(QLIN_MOE_NOALLOC_SCRATCH_BYTES == qlin::kMoeStaticScratchBytes, "header and library agree");
    // a batch whose workspace would not fit the library's scratch is refused before anything runs
    const size_t need = qlin_moe_grouped_workspace_bytes(tokens, k, n_experts, ffn_dim, hidden);
    if (need > qlin::kMoeStaticScratchBytes) return QLIN_ERR_LIMIT;
    void *ws = nullptr;
    if (tokens > 0 && k > 0 && need > 0) {
        ws = qlin::moe_static_scratch();
        if (!ws) return QLIN_ERR_LAUNCH;
    }
    return qlin_moe_routed_decode_grouped(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes, n_experts,
                                          ffn_dim, in_dim, hidden, x, ids, rw, ws, qlin::kMoeStaticScratchBytes, out,
                                          tokens, k);
}

size_t qlin_moe_ffn_workspace_bytes(int tokens, int k, int n_experts, int ffn_dim, int hidden_size, int shared_ffn) {
    if (shared_ffn < 0) return 0;
    const size_t routed = qlin_moe_grouped_workspace_bytes(tokens, k, n_experts, ffn_dim, hidden_size);
    if (routed == 0) return 0;
    return routed + ((static_cast<size_t>(tokens) * static_cast<size_t>(shared_ffn) * sizeof(float) + 255) & ~size_t{255});
}

// MoE::forward's routed and shared experts (MoE.cpp:29-52, after the norm, before the residual add):
// the batched routed decode from the logits, then the shared experts' SwiGLU and down-add.  When the
// shared down-add takes the m > 1 matrix-core kernel, that launch also applies the routed combine
// (one launch fewer); either way out gets (out + routed) + shared, as the three calls give it.
int qlin_moe_ffn_decode_grouped_logits(int gu_type, const uint8_t *gate, const uint8_t *up, size_t gate_up_bytes,
                                       int down_type, const uint8_t *down, size_t down_bytes, int n_experts,
                                       int ffn_dim, int in_dim, int hidden, int shared_type, const uint8_t *shared_gate,
                                       const uint8_t *shared_up, size_t shared_gate_up_rb, const uint8_t *shared_down,
                                       size_t shared_down_rb, int shared_ffn, const float *x,
                                       const float *router_logits, float routed_scaling, int *ids, float *rw,
                                       void *workspace, size_t workspace_bytes, float *out, int tokens, int k) {
    if (shared_ffn < 0) return QLIN_ERR_SHAPE;
    int rc = grouped_check(gu_type, gate, up, gate_up_bytes, down_type, down, down_bytes, n_experts, ffn_dim, in_dim,
                           hidden, x, ids, rw, workspace, workspace_bytes, out, tokens, k);
    if (rc) return rc;
    if (n_experts > 256) return QLIN_ERR_LIMIT;  // the router's limit
    const bool shared = shared_ffn > 0;
    if (shared) {
        if ((rc = check_weight(shared_type, shared_gate, shared_gate_up_rb, shared_ffn, in_dim)) ||
            (rc = check_weight(shared_type, shared_up, shared_gate_up_rb, shared_ffn, in_dim)) ||
            (rc = check_weight(shared_type, shared_down, shared_down_rb, hidden, shared_ffn)))
            return rc;
    }
    if (tokens == 0) return QLIN_OK;
    if (!x || !out || (shared && !workspace)) return QLIN_ERR_NULL;
    if ((rc = check_f32(x, true)) || (rc = check_f32(out, true))) return rc;
    if (shared && workspace_bytes < qlin_moe_ffn_workspace_bytes(tokens, k, n_experts, ffn_dim, hidden, shared_ffn))
        return QLIN_ERR_LIMIT;
    if (shared && (reinterpret_cast<uintptr_t>(workspace) & 255u)) return QLIN_ERR_ALIGN;
    if (k > 0 && (rc = check_f32(router_logits, true))) return rc;
    // the shared activations [tokens, shared_ffn] follow the routed part's workspace
    float *sact = shared ? reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) +
                                                     qlin::moe_grouped_workspace(tokens, k, n_experts, ffn_dim, hidden))
                         : nullptr;
    const size_t g_eb = gate_up_bytes / static_cast<size_t>(n_experts);
    const size_t g_rb = g_eb / static_cast<size_t>(ffn_dim);
    const bool fuse = k > 0 && shared && tokens > 1 &&
                      qlin::moe_grouped_up_ok(gu_type, gate, up, g_eb, g_rb, x, in_dim, ffn_dim, n_experts, tokens * k) &&
                      qlin::dense_ok(shared_type, shared_down, nullptr, shared_down_rb, sact, shared_ffn);
    if (fuse) {
        const size_t d_eb = down_bytes / static_cast<size_t>(n_experts);
        const size_t d_rb = d_eb / static_cast<size_t>(hidden);
        const qlin::MoeRouter router{router_logits, routed_scaling, ids, rw};
        qlin::RouteCombine routed{};
        // the shared SwiGLU rides in the routed gate/up launch when that launch can take it
        bool shared_done = false;
        const qlin::SharedUp sh{shared_gate, shared_up, shared_gate_up_rb, sact, shared_ffn, &shared_done};
        const bool sh_ok = shared_type == QLIN_TYPE_Q4_K && in_dim % 256 == 0 &&
                           qlin::dense_ok(shared_type, shared_gate, shared_up, shared_gate_up_rb, x, in_dim);
        hipError_t e = qlin::moe_grouped(gu_type, gate, up, g_eb, g_rb, down_type, down, d_eb, d_rb, n_experts, ffn_dim,
                                         in_dim, hidden, x, nullptr, nullptr, workspace, out, tokens, k, stream(),
                                         &router, &routed, sh_ok ? &sh : nullptr);
        if (e != hipSuccess) return launched(e);
        if (!shared_done && (rc = qlin_launch_quant_swiglu_rows(shared_type, shared_gate, shared_up, shared_gate_up_rb,
                                                                shared_gate_up_rb, x, sact, shared_ffn, in_dim, tokens)))
            return rc;
        return launched(qlin::dense_matmul(shared_type, shared_down, nullptr, shared_down_rb, sact, out, hidden,
                                           shared_ffn, tokens, 1, stream(), &routed));
    }
    if (k > 0 && (rc = qlin_moe_routed_decode_grouped_logits(gu_type, gate, up, gate_up_bytes, down_type, down,
                                                             down_bytes, n_experts, ffn_dim, in_dim, hidden, x,
                                                             router_logits, routed_scaling, ids, rw, workspace,
                                                             workspace_bytes, out, tokens, k)))
        return rc;
    if (!shared) return QLIN_OK;
    if ((rc = qlin_launch_quant_swiglu_rows(shared_type, shared_gate, shared_up, shared_gate_up_rb, shared_gate_up_rb,
                                            x, sact, shared_ffn, in_dim, tokens)))
        return rc;
    return qlin_launch_quant_matmul_add(shared_type, shared_down, shared_down_rb, sact, out, hidden, shared_ffn,
                                        tokens);
}

}  // extern "C"

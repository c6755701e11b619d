/*
 * qlin_oracle.c -- CPU restatement of the reference's GGUF quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).  Build with
 * -ffp-contract=off: every expression below is evaluated in the order written, with no fused
 * multiply-add except where fmaf() is called explicitly to mirror an explicit fmaf() in the
 * reference.  Function-level citations name the reference lines being restated; paths are
 * relative to AI/codes/local-llm/ in the reference repository.
 */
#include "qlin_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* block traits -- src/format/gguf/GgufFile.cpp:35-55                                           */

int orc_block_elems(int type) {
    switch (type) {
        case ORC_F32: case ORC_F16: return 1;
        case ORC_Q4_0: case ORC_Q5_0: case ORC_Q8_0: case ORC_Q8_1: return 32;
        case ORC_Q4_K: case ORC_Q6_K: return 256;
        default: return 0;
    }
}

int orc_block_bytes(int type) {
    switch (type) {
        case ORC_F32: return 4;
        case ORC_F16: return 2;
        case ORC_Q4_0: return 18;
        case ORC_Q5_0: return 22;
        case ORC_Q8_0: return 34;
        case ORC_Q8_1: return 36;
        case ORC_Q4_K: return 144;
        case ORC_Q6_K: return 210;
        default: return 0;
    }
}

/* ------------------------------------------------------------------------------------------ */
/* IEEE-754 binary16, written from the standard's definition of the format.                    */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13)); /* inf / nan, payload kept */
    if (exp != 0) return u2f(sign | ((exp + 112u) << 23) | (man << 13));
    /* zero or subnormal: man * 2^-24, exact in binary32 */
    const float mag = (float)man * 0x1p-24f;
    return sign ? -mag : mag;
}

/* Shift v right by s (1 <= s <= 31) rounding to nearest, ties to even. */
static uint32_t shr_rne(uint32_t v, int s) {
    const uint32_t q = v >> s;
    const uint32_t rem = v & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (q & 1u))) return q + 1u;
    return q;
}

uint16_t orc_f32_to_f16(float f) {
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* nan */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 (and inf) -> inf */
    const int e = (int)(ax >> 23);
    if (e >= 113) {
        /* normal half: rebias exponent, round the 23-bit mantissa to 10 bits (a carry into the
         * exponent field is the correct result) */
        const uint32_t v = ((uint32_t)(e - 112) << 23) | (ax & 0x7fffffu);
        return (uint16_t)(sign | shr_rne(v, 13));
    }
    /* subnormal half (or zero): value = mant * 2^(e-150); result k units of 2^-24 */
    if (e == 0) return sign; /* binary32 subnormals are far below half's smallest subnormal */
    const int s = 126 - e; /* >= 14 */
    if (s > 24) return sign; /* < 2^-25: rounds to zero */
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    return (uint16_t)(sign | shr_rne(mant, s)); /* k == 1024 is the smallest normal: correct */
}

void orc_f16_to_f32_array(const uint16_t *h, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(h[i]);
}

void orc_f32_to_f16_array(const float *f, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(f[i]);
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* ------------------------------------------------------------------------------------------ */
/* block codecs                                                                                 */

/* kernel.cu:913-921 */
void orc_q4k_scale_min(int j, const uint8_t *s, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q4_K super-block (144 B: d f16, dmin f16, scales[12], qs[128]) -> 256 f32.
 * kernel.cu:1090-1119: element e is in sub-block j = e/32 at inner = e%32; its nibble is
 * qs[(j/2)*32 + inner], low half for even j, high half for odd j; w = d*sc*q - dmin*m. */
static void deq_q4k(const uint8_t *b, float *out) {
    const float d = orc_f16_to_f32(rd16(b));
    const float dmin = orc_f16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4;
    const uint8_t *qs = b + 16;
    for (int j = 0; j < 8; ++j) {
        int sc, m;
        orc_q4k_scale_min(j, scales, &sc, &m);
        for (int inner = 0; inner < 32; ++inner) {
            const uint8_t byte = qs[(j >> 1) * 32 + inner];
            const int q = (j & 1) ? (byte >> 4) : (byte & 0x0f);
            out[j * 32 + inner] = d * (float)sc * (float)q - dmin * (float)m;
        }
    }
}

/* Q6_K super-block (210 B: ql[128], qh[64], int8 sc[16], d f16) -> 256 f32.  kernel.cu:1122-1156:
 * two 128-element halves; within a half, group g in [0,4) of 32 elements takes the low (g<2) or
 * high (g>=2) nibble of ql[h*64 + l + 32*(g&1)] and bits 2g..2g+1 of qh[h*32 + l];
 * q = that 6-bit value - 32; scale index h*8 + l/16 + 2g; w = d*sc*q. */
static void deq_q6k(const uint8_t *b, float *out) {
    const uint8_t *ql = b;
    const uint8_t *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d = orc_f16_to_f32(rd16(b + 208));
    for (int e = 0; e < 256; ++e) {
        const int half = e >> 7;
        const int within = e & 127;
        const int g = within >> 5;
        const int l = within & 31;
        const uint8_t lo_byte = ql[half * 64 + l + 32 * (g & 1)];
        const int lo = (g < 2) ? (lo_byte & 0x0f) : (lo_byte >> 4);
        const int hi = (qh[half * 32 + l] >> (2 * g)) & 3;
        const int q = (lo | (hi << 4)) - 32;
        const int s = sc[half * 8 + l / 16 + 2 * g];
        out[e] = d * (float)s * (float)q;
    }
}

/* Q5_0 block (22 B: d f16, qh u32, qs[16]) -> 32 f32.  kernel.cu:1159-1175: element e<16 uses the
 * low nibble of qs[e] and bit e of qh; e>=16 the high nibble of qs[e-16] and bit e of qh;
 * w = d*(q-16). */
static void deq_q50(const uint8_t *b, float *out) {
    const float d = orc_f16_to_f32(rd16(b));
    const uint32_t qh = rd32(b + 2);
    const uint8_t *qs = b + 6;
    for (int e = 0; e < 32; ++e) {
        const int lo = (e < 16) ? (qs[e] & 0x0f) : (qs[e - 16] >> 4);
        const int q = lo | (int)(((qh >> e) & 1u) << 4);
        out[e] = d * (float)(q - 16);
    }
}

/* Q8_0 block (34 B: d f16, int8 qs[32]) -> 32 f32.  kernel.cu:1178-1185: w = d*q. */
static void deq_q80(const uint8_t *b, float *out) {
    const float d = orc_f16_to_f32(rd16(b));
    const int8_t *qs = (const int8_t *)(b + 2);
    for (int e = 0; e < 32; ++e) out[e] = d * (float)qs[e];
}

/* Q4_0 block (18 B: d f16, qs[16]) -> 32 f32, ggml block_q4_0: element e<16 is the low nibble
 * of qs[e], e>=16 the high nibble of qs[e-16]; w = d*(q-8).  The reference has no decoder for it
 * (GgufFile.cpp:40 holds the trait only). */
static void deq_q40(const uint8_t *b, float *out) {
    const float d = orc_f16_to_f32(rd16(b));
    const uint8_t *qs = b + 2;
    for (int e = 0; e < 32; ++e) {
        const int q = (e < 16) ? (qs[e] & 0x0f) : (qs[e - 16] >> 4);
        out[e] = d * (float)(q - 8);
    }
}

typedef void (*deq_fn)(const uint8_t *, float *);

static deq_fn deq_for(int type) {
    switch (type) {
        case ORC_Q4_0: return deq_q40;
        case ORC_Q5_0: return deq_q50;
        case ORC_Q8_0: return deq_q80;
        case ORC_Q4_K: return deq_q4k;
        case ORC_Q6_K: return deq_q6k;
        default: return NULL;
    }
}

int orc_dequant_f32(int type, const uint8_t *src, int64_t n, float *out) {
    const deq_fn f = deq_for(type);
    if (!f) return -1;
    const int be = orc_block_elems(type), bb = orc_block_bytes(type);
    if (n % be) return -1;
    for (int64_t b = 0; b < n / be; ++b) f(src + b * bb, out + b * be);
    return 0;
}

/* kernel.cu:954-1063: the f16 output is the RNE conversion of the f32 value. */
int orc_dequant_f16(int type, const uint8_t *src, int64_t n, uint16_t *out) {
    const deq_fn f = deq_for(type);
    if (!f) return -1;
    const int be = orc_block_elems(type), bb = orc_block_bytes(type);
    if (n % be) return -1;
    float tmp[256];
    for (int64_t b = 0; b < n / be; ++b) {
        f(src + b * bb, tmp);
        for (int e = 0; e < be; ++e) out[b * be + e] = orc_f32_to_f16(tmp[e]);
    }
    return 0;
}

/* Dequantize one weight row of in_dim elements. */
static int deq_row(int type, const uint8_t *row, int in_dim, float *out) {
    return orc_dequant_f32(type, row, in_dim, out);
}

static int check_shape(int type, int in_dim) {
    const int be = orc_block_elems(type);
    if (!deq_for(type) || be == 0 || in_dim <= 0 || in_dim % be) return -1;
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* GEMV / matmul -- kernel.cu:1192-1279                                                         */

int orc_matmul_f64(int type, const uint8_t *w, size_t row_bytes, const float *x, double *y,
                   int out_dim, int in_dim, int m) {
    if (check_shape(type, in_dim) || out_dim < 0 || m < 0) return -1;
    float *wr = (float *)malloc(sizeof(float) * (size_t)in_dim);
    if (!wr) return -1;
    for (int o = 0; o < out_dim; ++o) {
        deq_row(type, w + (size_t)o * row_bytes, in_dim, wr);
        for (int r = 0; r < m; ++r) {
            const float *xr = x + (size_t)r * in_dim;
            double acc = 0.0;
            for (int k = 0; k < in_dim; ++k) acc += (double)wr[k] * (double)xr[k];
            y[(size_t)r * out_dim + o] = acc;
        }
    }
    free(wr);
    return 0;
}

int orc_matmul_f32(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y,
                   int out_dim, int in_dim, int m, int nthreads) {
    if (check_shape(type, in_dim) || out_dim < 0 || m < 0) return -1;
    int err = 0;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#else
    (void)nthreads;
#endif
    {
        float *wr = (float *)malloc(sizeof(float) * (size_t)in_dim);
        if (!wr) {
            err = -1;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int o = 0; o < out_dim; ++o) {
                deq_row(type, w + (size_t)o * row_bytes, in_dim, wr);
                for (int r = 0; r < m; ++r) {
                    const float *xr = x + (size_t)r * in_dim;
                    /* 8 independent partial sums so the compiler can vectorise the dot */
                    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                    for (int k = 0; k < in_dim; k += 8)
                        for (int t = 0; t < 8; ++t) acc[t] += wr[k + t] * xr[k + t];
                    y[(size_t)r * out_dim + o] =
                        ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
                }
            }
            free(wr);
        }
    }
    return err;
}

/* Warp-32 shuffle-down tree as seen by lane 0: a[i] += a[i+off] for off = 16, 8, 4, 2, 1. */
static float tree32(float *a) {
    for (int off = 16; off > 0; off >>= 1)
        for (int i = 0; i < off; ++i) a[i] = a[i] + a[i + off];
    return a[0];
}

int orc_matmul_lane32(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y,
                      int out_dim, int in_dim, int m) {
    if (check_shape(type, in_dim) || out_dim < 0 || m < 0) return -1;
    float *wr = (float *)malloc(sizeof(float) * (size_t)in_dim);
    if (!wr) return -1;
    for (int o = 0; o < out_dim; ++o) {
        deq_row(type, w + (size_t)o * row_bytes, in_dim, wr);
        for (int r = 0; r < m; ++r) {
            const float *xr = x + (size_t)r * in_dim;
            float lane[32];
            for (int l = 0; l < 32; ++l) {
                float acc = 0.0f;
                for (int k = l; k < in_dim; k += 32) acc = fmaf(wr[k], xr[k], acc);
                lane[l] = acc;
            }
            y[(size_t)r * out_dim + o] = tree32(lane);
        }
    }
    free(wr);
    return 0;
}

/* kernel.cu:1223-1244 */
int orc_gemv_add(int type, const uint8_t *w, size_t row_bytes, const float *x, float *y,
                 int out_dim, int in_dim) {
    double *tmp = (double *)malloc(sizeof(double) * (size_t)(out_dim > 0 ? out_dim : 1));
    if (!tmp) return -1;
    const int rc = orc_matmul_f64(type, w, row_bytes, x, tmp, out_dim, in_dim, 1);
    if (rc == 0)
        for (int o = 0; o < out_dim; ++o) y[o] = (float)((double)y[o] + tmp[o]);
    free(tmp);
    return rc;
}

/* ------------------------------------------------------------------------------------------ */
/* Q8_1 activations -- kernel.cu:1679-1720                                                      */

size_t orc_q8_1_row_bytes(int in_dim) { return (size_t)((in_dim + 31) / 32) * 36; }

void orc_quantize_q8_1(const float *x, uint8_t *xq, int in_dim, int m, int store_raw_sum) {
    const int bpr = (in_dim + 31) / 32;
    for (int r = 0; r < m; ++r) {
        for (int b = 0; b < bpr; ++b) {
            float v[32], sums[32];
            float amax = 0.0f;
            for (int l = 0; l < 32; ++l) {
                const int k = b * 32 + l;
                v[l] = (k < in_dim) ? x[(size_t)r * in_dim + k] : 0.0f;
                amax = fmaxf(amax, fabsf(v[l]));
                sums[l] = v[l];
            }
            const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            const float raw_sum = tree32(sums); /* shuffle-down order, as lane 0 sees it */
            int qsum = 0;
            uint8_t *dst = xq + ((size_t)r * bpr + b) * 36;
            for (int l = 0; l < 32; ++l) {
                int q = (int)rintf(v[l] * id); /* round half to even (default rounding mode) */
                q = q < -127 ? -127 : (q > 127 ? 127 : q);
                qsum += q;
                dst[4 + l] = (uint8_t)(int8_t)q;
            }
            const uint16_t dh = orc_f32_to_f16(d);
            const float sum = store_raw_sum ? raw_sum : d * (float)qsum;
            const uint16_t sh = orc_f32_to_f16(sum);
            dst[0] = (uint8_t)(dh & 0xff); dst[1] = (uint8_t)(dh >> 8);
            dst[2] = (uint8_t)(sh & 0xff); dst[3] = (uint8_t)(sh >> 8);
        }
    }
}

/* kernel.cu:2305-2402, in double.  Q4_K: per 32-block j, (dw*sc*dx)*sum(qw*qx) - dmin*m*s
 * with s the block's stored f16 sum; Q6_K: dw*dx*(s0*dot(first 16) + s1*dot(last 16));
 * Q8_0 / Q5_0 / Q4_0: sum of the dequantized weight times dx*qx. */
int orc_matmul_q8_1(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, double *y,
                    int out_dim, int in_dim, int m) {
    return orc_matmul_q8_1_mt(type, w, row_bytes, xq, y, out_dim, in_dim, m, 1);
}

int orc_matmul_q8_1_mt(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, double *y,
                       int out_dim, int in_dim, int m, int threads) {
    if (check_shape(type, in_dim) || out_dim < 0 || m < 0) return -1;
    const int bpr = in_dim / 32;
    /* rows in parallel, each output element summed in the same order whatever the thread count */
    const int nt = threads > 0 ? threads : omp_get_max_threads();
    float *wall = (float *)malloc(sizeof(float) * (size_t)in_dim * (size_t)nt);
    if (!wall) return -1;
#pragma omp parallel for num_threads(nt) schedule(static) if (nt > 1)
    for (int o = 0; o < out_dim; ++o) {
        float *wr = wall + (size_t)omp_get_thread_num() * (size_t)in_dim;
        const uint8_t *row = w + (size_t)o * row_bytes;
        deq_row(type, row, in_dim, wr);
        for (int r = 0; r < m; ++r) {
            const uint8_t *xr = xq + (size_t)r * bpr * 36;
            double acc = 0.0;
            for (int qb = 0; qb < bpr; ++qb) {
                const uint8_t *xb = xr + (size_t)qb * 36;
                const double dx = orc_f16_to_f32(rd16(xb));
                const double sx = orc_f16_to_f32(rd16(xb + 2));
                const int8_t *qx = (const int8_t *)(xb + 4);
                if (type == ORC_Q4_K) {
                    const uint8_t *sb = row + (size_t)(qb >> 3) * 144;
                    const int j = qb & 7;
                    int sc, mn;
                    orc_q4k_scale_min(j, sb + 4, &sc, &mn);
                    long qdot = 0;
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t byte = sb[16 + (j >> 1) * 32 + l];
                        const int qw = (j & 1) ? (byte >> 4) : (byte & 0x0f);
                        qdot += (long)qw * qx[l];
                    }
                    const double dw = orc_f16_to_f32(rd16(sb));
                    const double dmin = orc_f16_to_f32(rd16(sb + 2));
                    acc += dw * sc * dx * (double)qdot - dmin * mn * sx;
                } else if (type == ORC_Q6_K) {
                    /* the dequantized value divided by d*sc is the integer q, so the 16-wide
                     * scale groups reduce to sc*q*qx sums */
                    const uint8_t *sb = row + (size_t)(qb >> 3) * 210;
                    const double dw = orc_f16_to_f32(rd16(sb + 208));
                    const int sub = qb & 7, half = sub >> 2, g = sub & 3;
                    const int8_t *sc = (const int8_t *)(sb + 192) + half * 8;
                    long dot0 = 0, dot1 = 0;
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t lo_byte = sb[half * 64 + l + 32 * (g & 1)];
                        const int lo = (g < 2) ? (lo_byte & 0x0f) : (lo_byte >> 4);
                        const int hi = (sb[128 + half * 32 + l] >> (2 * g)) & 3;
                        const int qw = (lo | (hi << 4)) - 32;
                        if (l < 16) dot0 += (long)qw * qx[l]; else dot1 += (long)qw * qx[l];
                    }
                    acc += dw * dx * ((double)sc[g * 2] * (double)dot0 + (double)sc[g * 2 + 1] * (double)dot1);
                } else {
                    for (int l = 0; l < 32; ++l) {
                        const float xv = (float)dx * (float)qx[l];
                        acc += (double)wr[qb * 32 + l] * (double)xv;
                    }
                }
            }
            y[(size_t)r * out_dim + o] = acc;
        }
    }
    free(wall);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* MoE -- kernel.cu:3463-3511 (router), 1289-1385 (swiglu), 2253-2287 (ordered down)           */

void orc_router_topk(const float *logits, int *top_idx, float *top_w, int tokens, int n_experts,
                     int k, float routed_scaling) {
    int *used = (int *)calloc((size_t)(n_experts > 0 ? n_experts : 1), sizeof(int));
    for (int t = 0; t < tokens; ++t) {
        const float *lg = logits + (size_t)t * n_experts;
        float maxv = -INFINITY;
        for (int e = 0; e < n_experts; ++e) {
            const float v = isfinite(lg[e]) ? lg[e] : -INFINITY;
            maxv = fmaxf(maxv, v);
        }
        float denom = 0.0f;
        if (isfinite(maxv))
            for (int e = 0; e < n_experts; ++e) {
                const float v = isfinite(lg[e]) ? lg[e] : -INFINITY;
                denom += expf(v - maxv);
            }
        for (int e = 0; e < n_experts; ++e) used[e] = 0;
        for (int r = 0; r < k; ++r) {
            float best = -INFINITY;
            int best_e = -1;
            for (int e = 0; e < n_experts; ++e) {
                if (used[e]) continue;
                const float v = isfinite(lg[e]) ? lg[e] : -INFINITY;
                if (v > best) { best = v; best_e = e; }
            }
            if (best_e < 0) best_e = r < n_experts ? r : 0;
            used[best_e] = 1;
            const float prob = (denom > 0.0f && isfinite(best)) ? expf(best - maxv) / denom : 0.0f;
            top_idx[(size_t)t * k + r] = best_e;
            top_w[(size_t)t * k + r] = prob * routed_scaling;
        }
    }
    free(used);
}

static double dot_row(int type, const uint8_t *row, const float *x, int in_dim, float *scratch) {
    deq_row(type, row, in_dim, scratch);
    double acc = 0.0;
    for (int k = 0; k < in_dim; ++k) acc += (double)scratch[k] * (double)x[k];
    return acc;
}

static float silu_mul(double g, double u) { return (float)(g / (1.0 + exp(-g)) * u); }

int orc_swiglu(int type, const uint8_t *wg, const uint8_t *wu, size_t g_row_bytes,
               size_t u_row_bytes, const float *x, float *act, int ffn_dim, int in_dim) {
    if (check_shape(type, in_dim)) return -1;
    float *s = (float *)malloc(sizeof(float) * (size_t)in_dim);
    if (!s) return -1;
    for (int o = 0; o < ffn_dim; ++o) {
        const double g = dot_row(type, wg + (size_t)o * g_row_bytes, x, in_dim, s);
        const double u = dot_row(type, wu + (size_t)o * u_row_bytes, x, in_dim, s);
        act[o] = silu_mul(g, u);
    }
    free(s);
    return 0;
}

int orc_swiglu_indexed(int type, const uint8_t *wg, const uint8_t *wu, size_t g_expert_bytes,
                       size_t u_expert_bytes, size_t g_row_bytes, size_t u_row_bytes,
                       const float *x, const int *expert_ids, float *act, int k, int ffn_dim,
                       int in_dim) {
    if (check_shape(type, in_dim)) return -1;
    float *s = (float *)malloc(sizeof(float) * (size_t)in_dim);
    if (!s) return -1;
    for (int r = 0; r < k; ++r) {
        const int e = expert_ids[r];
        for (int o = 0; o < ffn_dim; ++o) {
            if (e < 0) { act[(size_t)r * ffn_dim + o] = 0.0f; continue; }
            const double g = dot_row(type, wg + (size_t)e * g_expert_bytes + (size_t)o * g_row_bytes, x, in_dim, s);
            const double u = dot_row(type, wu + (size_t)e * u_expert_bytes + (size_t)o * u_row_bytes, x, in_dim, s);
            act[(size_t)r * ffn_dim + o] = silu_mul(g, u);
        }
    }
    free(s);
    return 0;
}

int orc_down_indexed_ordered(int type, const uint8_t *wd, size_t d_expert_bytes,
                             size_t d_row_bytes, const float *act, const int *expert_ids,
                             const float *route_w, float *out, int k, int hidden, int ffn_dim) {
    if (check_shape(type, ffn_dim)) return -1;
    float *s = (float *)malloc(sizeof(float) * (size_t)ffn_dim);
    if (!s) return -1;
    for (int h = 0; h < hidden; ++h) {
        double total = 0.0;
        for (int r = 0; r < k; ++r) {
            const int e = expert_ids[r];
            if (e < 0) continue;
            const double a = dot_row(type, wd + (size_t)e * d_expert_bytes + (size_t)h * d_row_bytes,
                                     act + (size_t)r * ffn_dim, ffn_dim, s);
            total += a * (double)route_w[r];
        }
        out[h] = (float)((double)out[h] + total);
    }
    free(s);
    return 0;
}

/* kernel.cu:2678-2693 (quant_embedding_kernel): out[t, :] = the dequantized row ids[t]. */
int orc_quant_embedding(int type, const int *ids, int n, const uint8_t *table, size_t row_bytes, int hidden,
                        float *out) {
    if (check_shape(type, hidden)) return -1;
    for (int t = 0; t < n; ++t)
        if (deq_row(type, table + (size_t)ids[t] * row_bytes, hidden, out + (size_t)t * hidden)) return -1;
    return 0;
}

/* kernel.cu:3018-3045 (mla_absorb_q_nope_kernel), in double: the head's first qk_nope kv_b rows,
 * column l, against q[h, :qk_nope]. */
int orc_mla_absorb_q_nope(int type, const float *q, const uint8_t *w, size_t row_bytes, double *q_abs, int n_heads,
                          int qk_nope, int qk_rope, int v_head, int kv_lora) {
    if (check_shape(type, kv_lora)) return -1;
    float *row = (float *)malloc(sizeof(float) * (size_t)kv_lora);
    if (!row) return -1;
    for (int i = 0; i < n_heads * kv_lora; ++i) q_abs[i] = 0.0;
    for (int h = 0; h < n_heads; ++h)
        for (int d = 0; d < qk_nope; ++d) {
            deq_row(type, w + ((size_t)h * (qk_nope + v_head) + d) * row_bytes, kv_lora, row);
            const double qv = q[(size_t)h * (qk_nope + qk_rope) + d];
            for (int l = 0; l < kv_lora; ++l) q_abs[(size_t)h * kv_lora + l] += (double)row[l] * qv;
        }
    free(row);
    return 0;
}

/* -dmin * m of 32-block b of a Q4_K row, in f32 as kernel.cu:3004-3014 (q4k_min_coeff_at) forms it. */
static float q4k_min_coeff(const uint8_t *row, int b) {
    const uint8_t *sb = row + (size_t)(b >> 3) * 144;
    int sc, m;
    orc_q4k_scale_min(b & 7, sb + 4, &sc, &m);
    return -(orc_f16_to_f32(rd16(sb + 2)) * (float)m);
}

/* kernel.cu:3052-3075 (mla_absorb_q4_xsum_delta_kernel), Q4_K kv_b, in double. */
int orc_mla_absorb_q4_xsum_delta(const float *q, const uint8_t *w, size_t row_bytes, double *out, int n_heads,
                                 int qk_nope, int qk_rope, int v_head, int kv_lora) {
    if (check_shape(ORC_Q4_K, kv_lora)) return -1;
    const int nblk = (kv_lora + 31) / 32;
    for (int h = 0; h < n_heads; ++h)
        for (int b = 0; b < nblk; ++b) {
            double acc = 0.0;
            for (int d = 0; d < qk_nope; ++d)
                acc += (double)q[(size_t)h * (qk_nope + qk_rope) + d] *
                       (double)q4k_min_coeff(w + ((size_t)h * (qk_nope + v_head) + d) * row_bytes, b);
            out[(size_t)h * nblk + b] = acc;
        }
    return 0;
}

/* kernel.cu:3417-3453 (mla_absorb_v_kernel), in double: the head's v rows (after its qk_nope rows)
 * against attn_latent[h, :]; Q4_K adds sum_b (-dmin * m)(row, b) * xsum_delta[h, b]. */
int orc_mla_absorb_v(int type, const uint8_t *w, size_t row_bytes, const float *latent, const float *delta,
                     double *attn, int n_heads, int qk_nope, int v_head, int kv_lora) {
    if (check_shape(type, kv_lora)) return -1;
    float *row = (float *)malloc(sizeof(float) * (size_t)kv_lora);
    if (!row) return -1;
    const int nblk = (kv_lora + 31) / 32;
    for (int h = 0; h < n_heads; ++h)
        for (int v = 0; v < v_head; ++v) {
            const uint8_t *r = w + ((size_t)h * (qk_nope + v_head) + qk_nope + v) * row_bytes;
            deq_row(type, r, kv_lora, row);
            double acc = 0.0;
            for (int k = 0; k < kv_lora; ++k) acc += (double)row[k] * (double)latent[(size_t)h * kv_lora + k];
            if (type == ORC_Q4_K)
                for (int b = 0; b < nblk; ++b) acc += (double)q4k_min_coeff(r, b) * (double)delta[(size_t)h * nblk + b];
            attn[(size_t)h * v_head + v] = acc;
        }
    free(row);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Q8_1-activation variants -- kernel.cu:1532-1765, 1873-2242, 2405-2660                       */

void orc_quantize_q8_1_mmq(const float *x, uint8_t *xq, int in_dim, int m, int store_raw_sum) {
    /* the same blocks as orc_quantize_q8_1 over each row zero-padded to whole groups of 128 */
    const int groups = (in_dim + 127) / 128, padded = groups * 128;
    float *row = (float *)calloc((size_t)padded, sizeof(float));
    uint8_t *blk = (uint8_t *)malloc((size_t)groups * 4 * 36);
    if (!row || !blk) { free(row); free(blk); return; }
    for (int r = 0; r < m; ++r) {
        memcpy(row, x + (size_t)r * in_dim, sizeof(float) * (size_t)in_dim);
        orc_quantize_q8_1(row, blk, padded, 1, store_raw_sum);
        for (int g = 0; g < groups; ++g) {
            uint8_t *dst = xq + ((size_t)g * m + r) * 144;
            for (int sub = 0; sub < 4; ++sub) {
                const uint8_t *b = blk + (size_t)(4 * g + sub) * 36;
                memcpy(dst + 4 * sub, b, 4);
                memcpy(dst + 16 + 32 * sub, b + 4, 32);
            }
        }
    }
    free(row);
    free(blk);
}

int orc_matmul_q8_1_mmq(int type, const uint8_t *w, size_t row_bytes, const uint8_t *xq, double *y, int out_dim,
                        int in_dim, int m) {
    if (check_shape(type, in_dim) || m < 0) return -1;
    const int bpr = in_dim / 32;
    uint8_t *rows = (uint8_t *)malloc((size_t)(m > 0 ? m : 1) * bpr * 36);
    if (!rows) return -1;
    for (int r = 0; r < m; ++r)
        for (int b = 0; b < bpr; ++b) {
            const uint8_t *grp = xq + ((size_t)(b / 4) * m + r) * 144;
            uint8_t *dst = rows + ((size_t)r * bpr + b) * 36;
            memcpy(dst, grp + 4 * (b % 4), 4);
            memcpy(dst + 4, grp + 16 + 32 * (b % 4), 32);
        }
    const int rc = orc_matmul_q8_1(type, w, row_bytes, rows, y, out_dim, in_dim, m);
    free(rows);
    return rc;
}

int orc_swiglu_indexed_q8_1(int type, const uint8_t *wg, const uint8_t *wu, size_t g_eb, size_t u_eb, size_t g_rb,
                            size_t u_rb, const uint8_t *xq, const int *ids, double *act, int k, int ffn_dim,
                            int in_dim) {
    if (check_shape(type, in_dim)) return -1;
    for (int r = 0; r < k; ++r)
        for (int o = 0; o < ffn_dim; ++o) {
            double g = 0.0, u = 0.0, *dst = act + (size_t)r * ffn_dim + o;
            if (ids[r] < 0) { *dst = 0.0; continue; }
            if (orc_matmul_q8_1(type, wg + (size_t)ids[r] * g_eb + (size_t)o * g_rb, g_rb, xq, &g, 1, in_dim, 1) ||
                orc_matmul_q8_1(type, wu + (size_t)ids[r] * u_eb + (size_t)o * u_rb, u_rb, xq, &u, 1, in_dim, 1))
                return -1;
            *dst = g / (1.0 + exp(-g)) * u;
        }
    return 0;
}

int orc_down_q8_1_indexed_accum(int type, const uint8_t *wd, size_t d_eb, size_t d_rb, const uint8_t *act_q8_1,
                                const int *ids, const float *rw, double *out, int k, int hidden, int ffn_dim) {
    if (check_shape(type, ffn_dim)) return -1;
    const size_t xrb = (size_t)(ffn_dim / 32) * 36;
    for (int h = 0; h < hidden; ++h)
        for (int r = 0; r < k; ++r) {
            if (ids[r] < 0) continue;
            double y;
            if (orc_matmul_q8_1(type, wd + (size_t)ids[r] * d_eb + (size_t)h * d_rb, d_rb, act_q8_1 + (size_t)r * xrb,
                                &y, 1, ffn_dim, 1))
                return -1;
            out[h] += (double)rw[r] * y;
        }
    return 0;
}

int orc_down_f32_indexed_accum(int type, const uint8_t *wd, size_t d_eb, size_t d_rb, const float *act,
                               const int *ids, const float *rw, double *out, int k, int hidden, int ffn_dim) {
    if (check_shape(type, ffn_dim) || k < 0) return -1;
    uint8_t *q = (uint8_t *)malloc((size_t)(k > 0 ? k : 1) * (size_t)(ffn_dim / 32) * 36);
    if (!q) return -1;
    orc_quantize_q8_1(act, q, ffn_dim, k, 0);
    const int rc = orc_down_q8_1_indexed_accum(type, wd, d_eb, d_rb, q, ids, rw, out, k, hidden, ffn_dim);
    free(q);
    return rc;
}

/* ------------------------------------------------------------------------------------------ */
/* MLA over the Q8_1 latent cache -- kernel.cu:2945-3415                                       */

int orc_mla_store_latent_q8_1(const float *kv_cache, uint8_t *cache, int kv_lora, int qk_rope, size_t row_bytes,
                              int pos) {
    /* kernel.cu:2945-2978: one block of 32 per warp, values past kv_lora are 0, s = d * sum(q) --
     * the quantizer of kernel.cu:1679-1720 over the row zero-padded to row_bytes / 36 blocks */
    const int nblk = (int)(row_bytes / 36);
    if (kv_lora <= 0 || qk_rope < 0 || pos < 0) return -1;
    float *row = (float *)calloc((size_t)nblk * 32 + 1, sizeof(float));
    if (!row) return -1;
    const int n = kv_lora < nblk * 32 ? kv_lora : nblk * 32;
    memcpy(row, kv_cache + (size_t)pos * (kv_lora + qk_rope), sizeof(float) * (size_t)n);
    orc_quantize_q8_1(row, cache + (size_t)pos * row_bytes, nblk * 32, 1, 0);
    free(row);
    return 0;
}

/* d * q of latent element k of a Q8_1 row (kernel.cu:2979-2987; exact in f32) */
static float latent_at(const uint8_t *row, int k) {
    const uint8_t *blk = row + (size_t)(k >> 5) * 36;
    return orc_f16_to_f32(rd16(blk)) * (float)((const int8_t *)(blk + 4))[k & 31];
}

/* stored f16 sum minus the block's dequantized values added in order (kernel.cu:2989-3003) */
static float latent_sum_delta(const uint8_t *row, int b, int kv_lora) {
    const uint8_t *blk = row + (size_t)b * 36;
    const float d = orc_f16_to_f32(rd16(blk));
    float sum = 0.0f;
    for (int l = 0; l < 32 && b * 32 + l < kv_lora; ++l) sum += d * (float)((const int8_t *)(blk + 4))[l];
    return orc_f16_to_f32(rd16(blk + 2)) - sum;
}

int orc_mla_absorb_scores(const float *q_abs, const float *q, const uint8_t *cache, size_t crb, const float *delta,
                          const float *kv_cache, double *scores, int n_heads, int qk_nope, int qk_rope, int kv_lora,
                          int pos, int max_seq, float scale) {
    /* kernel.cu:3157-3196 */
    const int nb = (kv_lora + 31) / 32;
    if (pos >= max_seq) pos = max_seq - 1;
    for (int h = 0; h < n_heads; ++h)
        for (int t = 0; t <= pos; ++t) {
            const uint8_t *row = cache + (size_t)t * crb;
            double dot = 0.0;
            for (int k = 0; k < kv_lora; ++k) dot += (double)q_abs[(size_t)h * kv_lora + k] * latent_at(row, k);
            const float *qr = q + (size_t)h * (qk_nope + qk_rope) + qk_nope;
            const float *kr = kv_cache + (size_t)t * (kv_lora + qk_rope) + kv_lora;
            for (int r = 0; r < qk_rope; ++r) dot += (double)qr[r] * kr[r];
            for (int b = 0; b < nb; ++b) dot += (double)delta[(size_t)h * nb + b] * latent_sum_delta(row, b, kv_lora);
            scores[(size_t)h * max_seq + t] = dot * scale;
        }
    return 0;
}

/* exp(s - max) / (sum + 1e-9) over t <= pos of one head's scores (kernel.cu:3211-3235) */
static void softmax_probs(const float *s, int pos, double *p) {
    double mx = -INFINITY, den = 0.0;
    for (int t = 0; t <= pos; ++t) mx = s[t] > mx ? s[t] : mx;
    for (int t = 0; t <= pos; ++t) den += (p[t] = exp((double)s[t] - mx));
    for (int t = 0; t <= pos; ++t) p[t] /= den + 1e-9;
}

int orc_mla_absorb_context(const float *scores, const uint8_t *cache, size_t crb, double *delta_out,
                           double *latent_out, int n_heads, int kv_lora, int pos, int max_seq) {
    /* kernel.cu:3198-3257 */
    const int nb = (kv_lora + 31) / 32;
    if (pos >= max_seq) pos = max_seq - 1;
    double *p = (double *)malloc(sizeof(double) * (size_t)(pos + 2));
    if (!p) return -1;
    for (int h = 0; h < n_heads; ++h) {
        softmax_probs(scores + (size_t)h * max_seq, pos, p);
        for (int k = 0; k < kv_lora; ++k) {
            double acc = 0.0;
            for (int t = 0; t <= pos; ++t) acc += p[t] * latent_at(cache + (size_t)t * crb, k);
            latent_out[(size_t)h * kv_lora + k] = acc;
        }
        for (int b = 0; b < nb; ++b) {
            double acc = 0.0;
            for (int t = 0; t <= pos; ++t) acc += p[t] * latent_sum_delta(cache + (size_t)t * crb, b, kv_lora);
            delta_out[(size_t)h * nb + b] = acc;
        }
    }
    free(p);
    return 0;
}

int orc_mla_absorb_attend(const float *q_abs, const float *q, const uint8_t *cache, size_t crb, const float *delta,
                          double *delta_out, const float *kv_cache, double *latent_out, int n_heads, int qk_nope,
                          int qk_rope, int kv_lora, int pos, int max_seq, float scale) {
    /* kernel.cu:3078-3155: the scores of kernel.cu:3157-3196, exp(s - max) / sum (no 1e-9), the context */
    const int nb = (kv_lora + 31) / 32;
    if (pos >= max_seq) pos = max_seq - 1;
    double *sc = (double *)malloc(sizeof(double) * (size_t)n_heads * (size_t)max_seq + 1);
    if (!sc) return -1;
    orc_mla_absorb_scores(q_abs, q, cache, crb, delta, kv_cache, sc, n_heads, qk_nope, qk_rope, kv_lora, pos, max_seq,
                          scale);
    for (int h = 0; h < n_heads; ++h) {
        double *p = sc + (size_t)h * max_seq, mx = -INFINITY, den = 0.0;
        for (int t = 0; t <= pos; ++t) mx = p[t] > mx ? p[t] : mx;
        for (int t = 0; t <= pos; ++t) den += (p[t] = exp(p[t] - mx));
        for (int k = 0; k < kv_lora; ++k) {
            double acc = 0.0;
            for (int t = 0; t <= pos; ++t) acc += p[t] / den * latent_at(cache + (size_t)t * crb, k);
            latent_out[(size_t)h * kv_lora + k] = acc;
        }
        for (int b = 0; b < nb; ++b) {
            double acc = 0.0;
            for (int t = 0; t <= pos; ++t) acc += p[t] / den * latent_sum_delta(cache + (size_t)t * crb, b, kv_lora);
            delta_out[(size_t)h * nb + b] = acc;
        }
    }
    free(sc);
    return 0;
}

int orc_mla_project_v(int type, const uint8_t *w, size_t row_bytes, const uint8_t *cache, size_t crb,
                      double *kv_b_cache, int n_heads, int qk_nope, int v_head, int kv_lora, int pos) {
    /* kernel.cu:3259-3361: each v row of kv_b against the latent row, with the block-dot semantics
     * of quant_matmul_q8_1 (kernel.cu:2305-2402) */
    if (check_shape(type, kv_lora) || pos < 0) return -1;
    const size_t stride = (size_t)n_heads * (qk_nope + v_head);
    for (int h = 0; h < n_heads; ++h)
        for (int v = 0; v < v_head; ++v) {
            const size_t r = (size_t)h * (qk_nope + v_head) + qk_nope + v;
            double y;
            if (orc_matmul_q8_1(type, w + r * row_bytes, row_bytes, cache + (size_t)pos * crb, &y, 1, kv_lora, 1))
                return -1;
            kv_b_cache[(size_t)pos * stride + r] = y;
        }
    return 0;
}

int orc_mla_absorb_context_v(const float *scores, const float *kv_b_cache, double *attn, int n_heads, int qk_nope,
                             int v_head, int pos, int max_seq) {
    /* kernel.cu:3368-3415 */
    if (pos >= max_seq) pos = max_seq - 1;
    double *p = (double *)malloc(sizeof(double) * (size_t)(pos + 2));
    if (!p) return -1;
    const size_t stride = (size_t)n_heads * (qk_nope + v_head);
    for (int h = 0; h < n_heads; ++h) {
        softmax_probs(scores + (size_t)h * max_seq, pos, p);
        for (int v = 0; v < v_head; ++v) {
            double acc = 0.0;
            for (int t = 0; t <= pos; ++t)
                acc += p[t] * kv_b_cache[(size_t)t * stride + (size_t)h * (qk_nope + v_head) + qk_nope + v];
            attn[(size_t)h * v_head + v] = acc;
        }
    }
    free(p);
    return 0;
}

int orc_argmax(const float *v, int n) {
    float best = -INFINITY;
    int idx = 0;
    for (int i = 0; i < n; ++i)
        if (v[i] > best) { best = v[i]; idx = i; }
    return idx;
}

/* ---- the config-3 decoder twin (see orc_qwen2_logits in qlin_oracle.h) ---------------------- */

/* y[o] = sum_k w(o, k) x[k] in double, rows over `threads` threads (scratch: one dequantized row each) */
static int matvec_d(int type, const uint8_t *w, int out_dim, int in_dim, const double *x, double *y, int threads) {
    const size_t rb = (size_t)(in_dim / orc_block_elems(type)) * (size_t)orc_block_bytes(type);
    int bad = 0;
#pragma omp parallel num_threads(threads)
    {
        float *s = (float *)malloc(sizeof(float) * (size_t)in_dim);
        if (!s) {
#pragma omp atomic write
            bad = 1;
        } else {
#pragma omp for schedule(static)
            for (int o = 0; o < out_dim; ++o) {
                deq_row(type, w + (size_t)o * rb, in_dim, s);
                double acc = 0.0;
                for (int k = 0; k < in_dim; ++k) acc += (double)s[k] * x[k];
                y[o] = acc;
            }
            free(s);
        }
    }
    return bad ? -1 : 0;
}

/* kernel.cu:112-150: x * rsqrt(mean(x^2) + eps) * w */
static void rms_norm_d(const double *x, const float *w, int n, double eps, double *y) {
    double ss = 0.0;
    for (int j = 0; j < n; ++j) ss += x[j] * x[j];
    const double inv = 1.0 / sqrt(ss / n + eps);
    for (int j = 0; j < n; ++j) y[j] = x[j] * inv * (double)w[j];
}

/* kernel.cu:186-226: pairs (i, i + d/2) rotated by pos / theta^(2i / d) */
static void rope_d(double *v, int d, int pos, double theta) {
    const int half = d / 2;
    for (int i = 0; i < half; ++i) {
        const double ang = (double)pos / pow(theta, (double)(2 * i) / (double)d);
        const double c = cos(ang), sn = sin(ang), a = v[i], b = v[i + half];
        v[i] = a * c - b * sn;
        v[i + half] = b * c + a * sn;
    }
}

int orc_qwen2_logits(const orc_qwen2_cfg *c, const orc_qwen2_layer *layers, const float *final_norm,
                     const uint8_t *table, const int *tokens, int n, int first, float *logits, int threads) {
    const int H = c->hidden, NH = c->n_heads, NKV = c->kv_heads, D = c->head_dim, F = c->ffn, V = c->vocab;
    const int QD = NH * D, KD = NKV * D, group = NH / NKV;
    if (n <= 0 || first < 0 || first >= n || NH % NKV || check_shape(c->wtype, H) || check_shape(c->wtype, F))
        return -1;
    const size_t trb = (size_t)(H / orc_block_elems(c->wtype)) * (size_t)orc_block_bytes(c->wtype);
    double *kc = (double *)malloc(sizeof(double) * (size_t)c->layers * n * KD);
    double *vc = (double *)malloc(sizeof(double) * (size_t)c->layers * n * KD);
    double *h = (double *)malloc(sizeof(double) * H), *xn = (double *)malloc(sizeof(double) * H);
    double *q = (double *)malloc(sizeof(double) * QD), *k = (double *)malloc(sizeof(double) * KD);
    double *v = (double *)malloc(sizeof(double) * KD), *att = (double *)malloc(sizeof(double) * QD);
    double *o = (double *)malloc(sizeof(double) * (H > F ? H : F)), *g = (double *)malloc(sizeof(double) * F);
    double *u = (double *)malloc(sizeof(double) * F), *p = (double *)malloc(sizeof(double) * n);
    double *lg = (double *)malloc(sizeof(double) * V);
    float *row = (float *)malloc(sizeof(float) * H);
    int rc = 0;
    if (!kc || !vc || !h || !xn || !q || !k || !v || !att || !o || !g || !u || !p || !lg || !row) rc = -1;
    for (int pos = 0; pos < n && rc == 0; ++pos) {
        deq_row(c->wtype, table + (size_t)tokens[pos] * trb, H, row); /* the embedding row */
        for (int j = 0; j < H; ++j) h[j] = row[j];
        for (int l = 0; l < c->layers && rc == 0; ++l) {
            const orc_qwen2_layer *L = layers + l;
            double *kl = kc + (size_t)l * n * KD, *vl = vc + (size_t)l * n * KD;
            rms_norm_d(h, L->attn_norm, H, c->eps, xn);
            rc |= matvec_d(c->wtype, L->wq, QD, H, xn, q, threads);
            rc |= matvec_d(c->wtype, L->wk, KD, H, xn, k, threads);
            rc |= matvec_d(c->wtype, L->wv, KD, H, xn, v, threads);
            for (int hh = 0; hh < NH; ++hh) rope_d(q + (size_t)hh * D, D, pos, c->theta);
            for (int hh = 0; hh < NKV; ++hh) rope_d(k + (size_t)hh * D, D, pos, c->theta);
            memcpy(kl + (size_t)pos * KD, k, sizeof(double) * KD);
            memcpy(vl + (size_t)pos * KD, v, sizeof(double) * KD);
            for (int hh = 0; hh < NH; ++hh) { /* kernel.cu:345-420, without the output gate */
                const int kh = hh / group;
                double mx = -INFINITY, den = 0.0;
                for (int t = 0; t <= pos; ++t) {
                    double s = 0.0;
                    for (int d = 0; d < D; ++d) s += q[(size_t)hh * D + d] * kl[(size_t)t * KD + (size_t)kh * D + d];
                    p[t] = s / sqrt((double)D);
                    if (p[t] > mx) mx = p[t];
                }
                for (int t = 0; t <= pos; ++t) { p[t] = exp(p[t] - mx); den += p[t]; }
                for (int d = 0; d < D; ++d) {
                    double acc = 0.0;
                    for (int t = 0; t <= pos; ++t) acc += p[t] * vl[(size_t)t * KD + (size_t)kh * D + d];
                    att[(size_t)hh * D + d] = acc / den;
                }
            }
            rc |= matvec_d(c->wtype, L->wo, H, QD, att, o, threads);
            for (int j = 0; j < H; ++j) h[j] += o[j];
            rms_norm_d(h, L->ffn_norm, H, c->eps, xn);
            rc |= matvec_d(c->wtype, L->wg, F, H, xn, g, threads);
            rc |= matvec_d(c->wtype, L->wu, F, H, xn, u, threads);
            for (int j = 0; j < F; ++j) g[j] = g[j] / (1.0 + exp(-g[j])) * u[j]; /* kernel.cu:1289-1328 */
            rc |= matvec_d(c->wtype, L->wd, H, F, g, o, threads);
            for (int j = 0; j < H; ++j) h[j] += o[j];
        }
        if (rc == 0 && pos >= first) {
            rms_norm_d(h, final_norm, H, c->eps, xn);
            rc |= matvec_d(c->wtype, table, V, H, xn, lg, threads);
            for (int j = 0; j < V; ++j) logits[(size_t)(pos - first) * V + j] = (float)lg[j];
        }
    }
    free(kc); free(vc); free(h); free(xn); free(q); free(k); free(v); free(att); free(o); free(g); free(u);
    free(p); free(lg); free(row);
    return rc;
}

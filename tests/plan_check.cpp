// CPU check of the launch planners' LDS arithmetic (blog_amd/csrc/qlin_plan.hpp), built and run by
// tests/test_plan.py: every accepted plan fits the CU's 160 KB together with the kernel's static
// LDS, the edge shapes land on the right side of it, and a shape no plan fits is refused (so the
// caller takes the per-element kernels rather than a launch that would fail).
#include <cstdio>
#include <cstdlib>

#include "qlin_plan.hpp"

using namespace qlin::plan;

static int failures = 0;
#define CHECK(c)                                                          \
    do {                                                                  \
        if (!(c)) {                                                       \
            std::printf("FAIL line %d: %s\n", __LINE__, #c);              \
            ++failures;                                                   \
        }                                                                 \
    } while (0)

int main() {
    // decode GEMV: over shapes, sum sizes and static LDS, an accepted plan always fits
    const size_t statics[] = {0, 256, 512, 4096};
    long accepted = 0, refused = 0;
    for (int k = 256; k <= 65536; k += 256)
        for (int total : {1, 16, 300, 3584, 18944, 152064, 1 << 20})
            for (int se : {16, 32})
                for (bool sw : {false, true})
                    for (size_t st : statics) {
                        const Gemv p = gemv(total, k, k / 256, sw, se, 256, true);
                        if (gemv_fits(p, st)) {
                            ++accepted;
                            CHECK(p.lds + st <= kMaxLds);
                            CHECK(p.grid >= 1 && p.grid <= 256);
                        } else {
                            ++refused;
                        }
                    }
    CHECK(accepted > 0 && refused > 0);
    // the edge: one row (grid 1, one 16-row tile), K = 256 n: 4K + 2 pads + K/32 * 4 + 16 n * 4 =
    // 1120 n + 2 kXPad bytes
    {
        const size_t pad = 2 * kXPad;
        const int n_edge = static_cast<int>((kMaxLds - pad) / 1120);
        const Gemv e = gemv(1, 256 * n_edge, n_edge, false, 32, 256, true);
        CHECK(e.lds == 1120u * n_edge + pad);
        CHECK(gemv_fits(e, kMaxLds - 1120 * n_edge - pad));
        CHECK(!gemv_fits(e, kMaxLds - 1120 * n_edge - pad + 1));
        CHECK(!gemv_fits(gemv(1, 256 * (n_edge + 1), n_edge + 1, false, 32, 256, true), 0));
    }
    CHECK(!gemv_fits(gemv(16, 256, 1, false, 32, 256, true), kMaxLds));  // a kernel that cannot be read
    // the grouped MoE streaming plans: Q4_K SwiGLU, Q5_0 / Q8_0 / Q4_K down
    const StreamFmt q4k{256, true, 0}, q50{128, false, 4}, q80{128, false, 8};
    struct Case { StreamFmt f; bool sw; };
    const Case cases[] = {{q4k, true}, {q4k, false}, {q50, false}, {q80, false}};
    for (const Case &c : cases)
        for (int K = c.f.ce; K <= 24576; K += c.f.ce)
            for (int rows : {16, 1408, 2048, 2816, 7168})
                for (int R : {1, 6, 96, 4096})
                    for (size_t st : statics) {
                        const Stream p = stream(c.f, c.sw, rows, K, 64, R, 256, st, st);
                        if (!p.ok) continue;
                        CHECK(p.nq == 4 || p.nq == 2);
                        CHECK(p.piece >= 1);
                        CHECK(p.lds + st <= kMaxLds);
                    }
    // Q4_K SwiGLU at the edge of four routes per pass: fixed = 4*(4K + 2 pads) + 4*K/32*4, per tile
    // 2*4*nchunk*64
    {
        auto need4 = [](int K) { return 16L * K + 8L * kXPad + K / 2 + 2L * 4 * (K / 256) * 64; };
        int K = 256;
        while (need4(K + 256) <= static_cast<long>(kMaxLds)) K += 256;
        const size_t st_fit = kMaxLds - need4(K);
        const Stream a = stream(q4k, true, 16, K, 64, 6, 256, st_fit, st_fit);
        CHECK(a.ok && a.nq == 4 && a.lds + st_fit <= kMaxLds);
        const Stream b = stream(q4k, true, 16, K, 64, 6, 256, st_fit + 1, st_fit + 1);  // four no longer fit
        CHECK(b.ok && b.nq == 2 && b.lds + st_fit + 1 <= kMaxLds);
        const Stream c = stream(q4k, true, 16, 4 * K, 64, 6, 256, 0, 0);  // not even two routes
        CHECK(!c.ok);
        CHECK(!stream(q4k, true, 16, 256, 64, 6, 256, kMaxLds, kMaxLds).ok);  // unreadable kernels
    }
    std::printf("%s: %ld gemv plans accepted, %ld refused\n", failures ? "FAILED" : "ok", accepted, refused);
    return failures ? 1 : 0;
}

// Parses each GGUF file named on the command line with the library's reader (blog_amd/csrc/qlin_gguf.cpp)
// and touches every byte the reader hands back: tensor names and data, metadata keys, strings and array
// elements.  tests/test_gguf_fuzz.py builds it with the host sanitizers and runs it over malformed and
// mutated files, so that any read outside the mapped file or any leak on an error path is reported.
#include <sys/stat.h>

#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "qlin_gguf.h"

static unsigned long sink = 0;
static void touch(const void *p, size_t n) {
    const unsigned char *b = static_cast<const unsigned char *>(p);
    for (size_t i = 0; i < n; ++i) sink += b[i];
}

// Where the reader mapped `path`: the start of that file's mapping in /proc/self/maps (0 if none).  The
// sanitizers do not see reads past the end of a file inside its last mapped page, so the ranges the
// reader hands back are checked against [start, start + file size) here.
static uintptr_t mapping_of(const char *path) {
    char real[PATH_MAX];
    if (!realpath(path, real)) return 0;
    FILE *f = std::fopen("/proc/self/maps", "r");
    if (!f) return 0;
    char line[PATH_MAX + 256];
    uintptr_t found = 0;
    while (std::fgets(line, sizeof line, f)) {
        unsigned long lo, hi, off;
        char perms[8], dev[16], file[PATH_MAX];
        unsigned long inode;
        file[0] = 0;
        if (std::sscanf(line, "%lx-%lx %7s %lx %15s %lu %4095s", &lo, &hi, perms, &off, dev, &inode, file) >= 6 &&
            off == 0 && std::strcmp(file, real) == 0) {
            found = lo;
            break;
        }
    }
    std::fclose(f);
    return found;
}

int main(int argc, char **argv) {
    int opened = 0, refused = 0, inconsistent = 0;
    for (int a = 1; a < argc; ++a) {
        qlin_gguf *g = nullptr;
        const int rc = qlin_gguf_open(argv[a], &g);
        if (rc != QLIN_OK) {
            ++refused;
            if (rc != QLIN_ERR_FORMAT && rc != QLIN_ERR_IO) {
                std::printf("unexpected status %d: %s\n", rc, argv[a]);
                ++inconsistent;
            }
            continue;
        }
        ++opened;
        struct stat st;
        const uintptr_t lo = mapping_of(argv[a]);
        const uintptr_t hi = lo + (stat(argv[a], &st) == 0 ? static_cast<uintptr_t>(st.st_size) : 0);
        // a range [p, p + n) inside the file's mapping must end within the file
        auto inside = [&](const void *p, uint64_t n, const char *what) {
            const uintptr_t q = reinterpret_cast<uintptr_t>(p);
            if (lo && q >= lo && q < lo + (((hi - lo) + 4095) & ~uintptr_t{4095}) && (q > hi || n > hi - q)) {
                std::printf("%s ends past the file: %s\n", what, argv[a]);
                ++inconsistent;
            }
        };
        if (!lo) {
            std::printf("no mapping found for %s\n", argv[a]);
            ++inconsistent;
        }
        (void)qlin_gguf_version(g);
        (void)qlin_gguf_alignment(g);
        const int64_t nt = qlin_gguf_tensor_count(g);
        for (int64_t i = 0; i < nt; ++i) {
            qlin_gguf_tensor t;
            if (qlin_gguf_tensor_info(g, i, &t) != QLIN_OK) {
                std::printf("tensor %lld unreadable: %s\n", static_cast<long long>(i), argv[a]);
                ++inconsistent;
                continue;
            }
            touch(t.name, std::strlen(t.name) + 1);
            inside(t.data, t.nbytes, "tensor data");
            touch(t.data, static_cast<size_t>(t.nbytes));
            // a lookup by name finds a tensor of that name (names are length-prefixed in the file, so one
            // with a NUL byte inside is not found by its C-string prefix, as std::string lookups behave)
            const int64_t j = qlin_gguf_find_tensor(g, t.name);
            qlin_gguf_tensor u;
            if (j >= 0 && (qlin_gguf_tensor_info(g, j, &u) != QLIN_OK || std::strcmp(u.name, t.name) != 0)) {
                std::printf("lookup of %s gave another tensor: %s\n", t.name, argv[a]);
                ++inconsistent;
            }
        }
        const int64_t nm = qlin_gguf_metadata_count(g);
        for (int64_t i = 0; i < nm; ++i) {
            const char *k = qlin_gguf_metadata_key(g, i);
            if (!k) continue;
            touch(k, std::strlen(k) + 1);
            int64_t iv;
            double dv;
            const char *s;
            size_t len;
            (void)qlin_gguf_get_i64(g, k, &iv);
            (void)qlin_gguf_get_f64(g, k, &dv);
            if (qlin_gguf_get_str(g, k, &s, &len) == QLIN_OK) {
                inside(s, len, "string value");
                touch(s, len);
            }
            if (qlin_gguf_metadata_type(g, k) != QLIN_GGUF_ARRAY) continue;
            int et;
            int64_t cnt;
            if (qlin_gguf_get_array_info(g, k, &et, &cnt) != QLIN_OK) continue;
            for (int64_t e = 0; e < cnt && e < 4096; ++e) {
                (void)qlin_gguf_get_array_i64(g, k, e, &iv);
                (void)qlin_gguf_get_array_f64(g, k, e, &dv);
                if (qlin_gguf_get_array_str(g, k, e, &s, &len) == QLIN_OK) {
                    inside(s, len, "array string");
                    touch(s, len);
                }
            }
            if (qlin_gguf_get_array_i64(g, k, cnt, &iv) == QLIN_OK || qlin_gguf_get_array_i64(g, k, -1, &iv) == QLIN_OK) {
                std::printf("array %s read outside its %lld elements: %s\n", k, static_cast<long long>(cnt), argv[a]);
                ++inconsistent;
            }
        }
        qlin_gguf_close(g);
    }
    std::printf("opened %d refused %d inconsistent %d (%lu)\n", opened, refused, inconsistent, sink & 1);
    return inconsistent ? 1 : 0;
}

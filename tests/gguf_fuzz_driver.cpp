// Sanitizer driver for the GGUF reader (arf_amd/csrc/arfq_gguf.cpp), built by
// tests/test_gguf_sanitized.py with AddressSanitizer and UBSan on the host:
// every file named on the command line is probed, opened and, when the open
// succeeds, walked through every query of the reader's C ABI, so that a read
// past a buffer, a use after free, a leak or an overflow on malformed input
// aborts the run.  The file itself is memory-mapped, which the sanitizers do
// not watch (and a read a little past its end stays inside the last page), so
// the driver checks the ranges the reader hands out itself: a tensor's blocks
// end within the file, and an upload's row slice lies within those blocks.
// Prints one line per file: the open status and the tensor count.
#include <sys/stat.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "arfq.h"

static const int kTypes[] = {0, 1, 2, 8, 12, 13, 14, 23, 99};

static unsigned long touch(const void *p, size_t n) {
    // read every byte of a returned range (a range past the mapping faults here)
    const unsigned char *b = static_cast<const unsigned char *>(p);
    unsigned long s = 0;
    for (size_t i = 0; i < n; i++) s += b[i];
    return s;
}

// The reader's upload path hands a range of the mapping to the device
// library's upload; here the range is read in full (so a row slice past the
// mapping aborts the run) and nothing is uploaded.
static unsigned long g_uploaded = 0;
static const unsigned char *g_up_ptr = nullptr;
static size_t g_up_bytes = 0;
extern "C" int arfq_weight_upload(arfq_ctx *, int, const void *host_blocks, size_t nbytes, int64_t, int64_t,
                                  int, arfq_weight **out) {
    g_up_ptr = static_cast<const unsigned char *>(host_blocks);
    g_up_bytes = nbytes;
    g_uploaded += touch(host_blocks, nbytes);
    if (out) *out = nullptr;
    return ARFQ_E_UNSUPPORTED;
}

static void check(bool ok, const char *path, const char *what) {
    if (ok) return;
    std::fprintf(stderr, "%s: %s\n", path, what);
    std::abort();
}

int main(int argc, char **argv) {
    unsigned long sink = 0;
    for (int a = 1; a < argc; a++) {
        const char *path = argv[a];
        struct stat st;
        const uint64_t fsize = stat(path, &st) == 0 ? (uint64_t)st.st_size : 0;
        const int magic = arfq_gguf_is_gguf(path);
        arfq_gguf *g = nullptr;
        const int rc = arfq_gguf_open(path, &g);
        if (rc != ARFQ_OK) {
            sink += std::strlen(arfq_gguf_last_error(nullptr));
            std::printf("%s open=%d magic=%d\n", path, rc, magic);
            continue;
        }
        int64_t n = -1;
        arfq_gguf_tensor_count(g, &n);
        for (int64_t i = -1; i <= n; i++) {  // one index past each end
            const char *name = nullptr;
            int ty = -1, nd = 0;
            int64_t dims[8] = {0};
            uint64_t off = 0, nbytes = 0;
            if (arfq_gguf_tensor_info(g, i, &name, &ty, &nd, dims, 8, &off, &nbytes) != ARFQ_OK) continue;
            sink += std::strlen(name) + (unsigned long)nd;
            int64_t idx = -1;
            arfq_gguf_find(g, name, &idx);
            sink += (unsigned long)idx;
            const unsigned char *own = nullptr;  // the blocks at the tensor's own type
            size_t own_bytes = 0;
            for (int t : kTypes) {
                const void *blocks = nullptr;
                size_t bytes = 0;
                int64_t rows = 0, cols = 0;
                if (arfq_gguf_blocks(g, name, t, &blocks, &bytes, &rows, &cols) == ARFQ_OK) {
                    check(t == ty && bytes == nbytes, path, "blocks of another type or size");
                    check(off <= fsize && bytes <= fsize - off, path, "tensor data past the end of the file");
                    own = static_cast<const unsigned char *>(blocks);
                    own_bytes = bytes;
                    sink += touch(blocks, bytes) + (unsigned long)rows;
                }
            }
            // row slices: whole, the first row, the last row, one past the end
            int ctx_stand_in = 0;
            arfq_ctx *ctx = reinterpret_cast<arfq_ctx *>(&ctx_stand_in);  // never dereferenced
            const int64_t r = nd >= 2 ? dims[1] : 1;
            const int64_t slices[4][2] = {{0, -1}, {0, 1}, {r - 1, 1}, {r, 1}};
            for (const auto &sl : slices) {
                arfq_weight *w = nullptr;
                g_up_ptr = nullptr;
                arfq_gguf_upload(ctx, g, name, sl[0], sl[1], &w);
                if (g_up_ptr)
                    check(own && g_up_ptr >= own && g_up_bytes <= own_bytes &&
                              (size_t)(g_up_ptr - own) <= own_bytes - g_up_bytes,
                          path, "upload range outside the tensor's blocks");
                sink += std::strlen(arfq_gguf_last_error(g));
            }
        }
        int64_t idx = 0;
        arfq_gguf_find(g, "no such tensor", &idx);
        arfq_gguf_tensor_info(g, 0, nullptr, nullptr, nullptr, nullptr, 0, nullptr, nullptr);
        arfq_gguf_close(g);
        std::printf("%s open=0 magic=%d tensors=%lld\n", path, magic, (long long)n);
    }
    std::printf("sink %lu\n", (sink + g_uploaded) & 1);
    return 0;
}

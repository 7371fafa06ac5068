// The GGUF reader (hyper_amd/csrc/hy_gguf.cpp) under AddressSanitizer and UBSan: opens every file named on the command
// line, reads the metadata accessors, every byte of every tensor view it accepts, and the expert tensors of layer 0.
// Exit 0 unless a sanitizer reports (they abort).  Built by tests/sanitize/Makefile; run by tests/test_sanitize.py.
#include "../../include/hymoe.h"

#include <cstdarg>
#include <cstdio>

namespace hy {
static char g_msg[512];
void set_error(const char *fmt, ...) {   // the library's hy_capi.cpp keeps a thread-local message; one suffices here
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof g_msg, fmt, ap);
    va_end(ap);
}
} // namespace hy

int main(int argc, char **argv) {
    unsigned long long sum = 0;
    int opened = 0;
    for (int i = 1; i < argc; ++i) {
        hy_gguf *g = nullptr;
        if (hy_gguf_open(argv[i], &g) != HY_OK) continue;
        ++opened;
        int64_t iv = 0;
        double dv = 0;
        const char *sv = nullptr;
        int64_t arr[8];
        double farr[8];
        size_t n = 0;
        (void) hy_gguf_get_int(g, "general.alignment", &iv);
        (void) hy_gguf_get_float(g, "qwen3moe.eps", &dv);
        (void) hy_gguf_get_str(g, "general.architecture", &sv);
        (void) hy_gguf_get_int_arr(g, "some.int_arr", arr, 8, &n);
        (void) hy_gguf_get_float_arr(g, "some.float_arr", farr, 8, &n);
        const char *arch = hy_gguf_arch(g);
        if (arch) sum += (unsigned char) arch[0];
        const int nt = hy_gguf_n_tensors(g);
        for (int t = 0; t < nt; ++t) {
            hy_gguf_tensor_info info;
            if (hy_gguf_tensor_at(g, t, &info) != HY_OK) continue;
            for (size_t b = 0; b < info.nbytes; ++b) sum += info.data[b];
            hy_gguf_tensor_info again;
            (void) hy_gguf_tensor(g, info.name, &again);
        }
        hy_expert_tensors et;
        if (hy_gguf_expert_tensors(g, 0, 4, &et) == HY_OK) sum += et.gate[0] + et.down[et.db * et.E - 1];
        hy_gguf_close(g);
    }
    std::printf("gguf_san: %d of %d files opened, checksum %llu\n", opened, argc - 1, sum);
    return 0;
}

// Driver of the host file readers (dit_files.cpp) for the sanitizer tests:
//   test_files raw <path>
//   test_files linear <base> <has_bias>
//   test_files win <path> <txt_len>
//   test_files graph <param> <bin> <mm_layers> [weight name]
// Prints the reader's return code (and on success a checksum of what it
// returned) and exits 0; a memory error makes the sanitizer end it non-zero.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "dit_model.h"

static double sum(const float* p, long n) {
    double s = 0;
    for (long i = 0; i < n; i++) s += p[i];
    return s;
}

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    const char* mode = argv[1];
    int rc = -100;
    if (!std::strcmp(mode, "raw")) {
        float* d = nullptr;
        int64_t n = 0, shape[8];
        int nd = 0;
        rc = dit_read_raw_f(argv[2], &d, &n, shape, &nd);
        if (!rc) std::printf("n=%lld ndim=%d sum=%g\n", (long long)n, nd, sum(d, (long)n));
        if (!rc) dit_free_host(d);
    } else if (!std::strcmp(mode, "linear") && argc >= 4) {
        float *w = nullptr, *b = nullptr;
        int no = 0, ni = 0;
        const int bias = std::atoi(argv[3]);
        rc = dit_read_linear(argv[2], bias, &w, &b, &no, &ni);
        if (!rc) std::printf("out=%d in=%d sum=%g\n", no, ni, sum(w, (long)no * ni) + (b ? sum(b, no) : 0.0));
        if (!rc) {
            dit_free_host(w);
            dit_free_host(b);
        }
    } else if (!std::strcmp(mode, "win") && argc >= 4) {
        int64_t header[10];
        int32_t* sl = nullptr;
        float *vf = nullptr, *tf = nullptr;
        int64_t nv = 0, nt = 0;
        rc = dit_read_win(argv[2], std::atoi(argv[3]), header, &sl, &vf, &nv, &tf, &nt);
        if (!rc) std::printf("nwin=%lld nv=%lld nt=%lld sum=%g\n", (long long)header[9], (long long)nv, (long long)nt,
                             sum(vf, (long)nv) + sum(tf, (long)nt) + sl[0]);
        if (!rc) {
            dit_free_host(sl);
            dit_free_host(vf);
            dit_free_host(tf);
        }
    } else if (!std::strcmp(mode, "graph") && argc >= 5) {
        int nl = 0, mm = 0, nw = 0;
        rc = dit_graph_file_info(argv[2], argv[3], std::atoi(argv[4]), &nl, &mm, &nw);
        if (!rc) std::printf("layers=%d mm=%d weights=%d\n", nl, mm, nw);
        if (!rc && argc >= 6) {
            float *w = nullptr, *b = nullptr;
            int no = 0, ni = 0;
            rc = dit_read_graph_weight(argv[2], argv[3], std::atoi(argv[4]), argv[5], &w, &b, &no, &ni);
            if (!rc) std::printf("%s out=%d in=%d sum=%g\n", argv[5], no, ni, sum(w, ni ? (long)no * ni : no));
            if (!rc) {
                dit_free_host(w);
                dit_free_host(b);
            }
        }
    } else {
        return 2;
    }
    std::printf("rc=%d%s%s\n", rc, rc ? " " : "", rc ? dit_host_last_error() : "");
    return 0;
}

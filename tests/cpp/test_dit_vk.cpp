// test_dit_vk.cpp — the C++ DitVk mirror (csrc/dit_vk.hpp) on a model directory.
//
// Usage: test_dit_vk <model_dir> <n_layers> <mm_layers> <grid.f32> <txt.f32> T H W TXT <timestep> <out.f32>
// Reads the (T, H, W, 33) grid and [TXT][5120] text as raw float32, runs
// DitVk::init + forward_grid and writes the (T, H, W, 16) result as raw
// float32; tests/test_dit_gpu.py compares it with the same forward driven
// from Python.  Also checks that a second call reuses the cached geometry and
// buffers (same result) and that bad shapes are refused.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "dit_vk.hpp"

static bool read_f32(const char* path, std::vector<float>& v, size_t n) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    v.resize(n);
    const size_t got = std::fread(v.data(), 4, n, f);
    std::fclose(f);
    return got == n;
}

int main(int argc, char** argv) {
    if (argc != 12) {
        std::fprintf(stderr, "usage: %s dir n_layers mm_layers grid txt T H W TXT t out\n", argv[0]);
        return 2;
    }
    const int T = std::atoi(argv[6]), H = std::atoi(argv[7]), W = std::atoi(argv[8]), TXT = std::atoi(argv[9]);
    const float t = (float)std::atof(argv[10]);
    std::vector<float> grid, txt, out, out2, bad;
    if (!read_f32(argv[4], grid, (size_t)T * H * W * 33) || !read_f32(argv[5], txt, (size_t)TXT * 5120)) {
        std::fprintf(stderr, "cannot read inputs\n");
        return 2;
    }
    seedvr2::DitVk dit;
    if (!dit.init(argv[1], std::atoi(argv[2]), std::atoi(argv[3]))) return 1;
    if (!dit.forward_grid(grid, T, H, W, txt, TXT, t, out)) return 1;
    if (!dit.forward_grid(grid, T, H, W, txt, TXT, t, out2) || out2 != out) {
        std::fprintf(stderr, "second call differs\n");
        return 1;
    }
    if (dit.forward_grid(grid, T, H + 1, W, txt, TXT, t, bad)) {
        std::fprintf(stderr, "odd H accepted\n");
        return 1;
    }
    FILE* f = std::fopen(argv[11], "wb");
    if (!f || std::fwrite(out.data(), 4, out.size(), f) != out.size()) return 2;
    std::fclose(f);
    std::printf("DitVk forward_grid ok (%zu values)\n", out.size());
    return 0;
}

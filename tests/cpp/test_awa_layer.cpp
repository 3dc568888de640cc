// test_awa_layer.cpp — the C++ host mirror (AwaLayer / AwaVk over the C ABI)
// on a GPU, in the style of the reference's standalone test executables
// (src/test_awa_layer.cpp): prints the checks and returns non-zero on failure.
//
//  1. AwaLayer with device-built geometry vs AwaLayer with the same geometry
//     injected through set_window_geometry, and vs AwaLayer reading it from a
//     win_*.bin file (build_window_geometry, awa_layer.cpp:110-141):
//     identical outputs (fp32 and bf16).
//  2. AwaVk (host vectors) vs AwaLayer fp32: identical outputs, with the
//     geometry handle and with a reference Win record (awa_vk.h:40-45).
//  3. Error paths return -1 / false.
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <random>
#include <string>
#include <vector>

#include "awa_layer.hpp"

#define CK(x)                                                             \
    do {                                                                  \
        if ((x) != hipSuccess) {                                          \
            std::fprintf(stderr, "HIP failure at %s:%d\n", __FILE__, __LINE__); \
            return 2;                                                     \
        }                                                                 \
    } while (0)

static int fails = 0;
static void check(bool ok, const char* what) {
    std::printf("[%s] %s\n", ok ? "PASS" : "FAIL", what);
    if (!ok) fails++;
}

static uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// A window file in load_win's layout (dit_vk.cpp:74-93) from a geometry.
static bool write_win(const std::string& path, int t, int h, int w, const int32_t nw[3],
                      const std::vector<int32_t>& slices, const std::vector<float>& vf,
                      const std::vector<float>& tf) {
    std::ofstream f(path, std::ios::binary);
    const int64_t nwin = (int64_t)slices.size() / 6;
    const int64_t hdr[10] = {t, h, w, nw[0], nw[1], nw[2], 0, 0, 0, nwin};
    f.write(reinterpret_cast<const char*>(hdr), sizeof hdr);
    for (int32_t v : slices) {
        const int64_t x = v;
        f.write(reinterpret_cast<const char*>(&x), 8);
    }
    f.write(reinterpret_cast<const char*>(vf.data()), vf.size() * 4);
    f.write(reinterpret_cast<const char*>(tf.data()), tf.size() * 4);
    return (bool)f;
}

int main() {
    char tmpl[] = "/tmp/awa_win_XXXXXX";
    const char* tmpdir = mkdtemp(tmpl);
    if (!tmpdir) return 2;
    const std::string win_dir = std::string(tmpdir) + "/";
    const int t = 1, h = 12, w = 20, TXT = 9, Lv = t * h * w;
    const int32_t nw[3] = {4, 3, 3};
    std::mt19937 rng(123);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<float> vqkv((size_t)Lv * AWA_QKV), tqkv((size_t)TXT * AWA_QKV), gains(4 * 128);
    for (auto& v : vqkv) v = nd(rng);
    for (auto& v : tqkv) v = nd(rng);
    for (auto& v : gains) v = 1.f + 0.02f * nd(rng);
    std::vector<uint16_t> vqkv16(vqkv.size()), tqkv16(tqkv.size());
    for (size_t i = 0; i < vqkv.size(); i++) vqkv16[i] = to_bf16(vqkv[i]);
    for (size_t i = 0; i < tqkv.size(); i++) tqkv16[i] = to_bf16(tqkv[i]);

    float *d_v, *d_t, *d_g, *d_o1, *d_o2, *d_to1, *d_to2;
    uint16_t *d_v16, *d_t16;
    CK(hipMalloc(&d_v, vqkv.size() * 4));
    CK(hipMalloc(&d_t, tqkv.size() * 4));
    CK(hipMalloc(&d_v16, vqkv.size() * 2));
    CK(hipMalloc(&d_t16, tqkv.size() * 2));
    CK(hipMalloc(&d_g, gains.size() * 4));
    CK(hipMalloc(&d_o1, (size_t)Lv * AWA_DIM * 4));
    CK(hipMalloc(&d_o2, (size_t)Lv * AWA_DIM * 4));
    CK(hipMalloc(&d_to1, (size_t)TXT * AWA_DIM * 4));
    CK(hipMalloc(&d_to2, (size_t)TXT * AWA_DIM * 4));
    CK(hipMemcpy(d_v, vqkv.data(), vqkv.size() * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_t, tqkv.data(), tqkv.size() * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_v16, vqkv16.data(), vqkv16.size() * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_t16, tqkv16.data(), tqkv16.size() * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_g, gains.data(), gains.size() * 4, hipMemcpyHostToDevice));

    for (int win_type = 0; win_type < 2; win_type++) {
        seedvr2::AwaLayer built, injected;
        built.set_config(win_type, Lv, TXT);
        injected.set_config(win_type, Lv, TXT);
        check(built.forward(d_v, vqkv.size() * 4, d_t, tqkv.size() * 4, d_o1, d_to1, false) == -1,
              "forward before geometry returns -1");
        check(built.build_window_geometry(t, h, w, nw, TXT) == 0, "build_window_geometry");
        built.set_qk_norm_device(d_g, d_g + 128, d_g + 256, d_g + 384);
        injected.set_qk_norm_device(d_g, d_g + 128, d_g + 256, d_g + 384);

        awa_geom_info info;
        awa_geom_query(built.geometry(), &info);
        std::vector<int32_t> cumf(info.nwin + 1), vidx(info.sumf);
        std::vector<float> vf((size_t)info.sumf * AWA_ROPE_ROT), tf((size_t)info.nwin * TXT * AWA_ROPE_ROT);
        awa_geom_read(built.context(), built.geometry(), nullptr, cumf.data(), vidx.data(), vf.data(), tf.data());
        std::vector<float> fcumf(cumf.begin(), cumf.end()), fvidx(vidx.begin(), vidx.end());
        check(injected.set_window_geometry(fvidx, fcumf, vf, tf, info.nwin, Lv, TXT) == 0,
              "set_window_geometry with the device geometry's arrays");
        std::vector<int32_t> slices((size_t)info.nwin * 6);
        awa_geom_read(built.context(), built.geometry(), slices.data(), nullptr, nullptr, nullptr, nullptr);
        const std::string wpath = win_dir + (win_type == 0 ? "win_nonshifted.bin" : "win_shifted.bin");
        check(write_win(wpath, t, h, w, nw, slices, vf, tf), "write the window file");
        seedvr2::AwaLayer fromfile;
        fromfile.set_config(win_type, Lv, TXT);
        fromfile.set_win_dir(win_dir);
        fromfile.set_qk_norm_device(d_g, d_g + 128, d_g + 256, d_g + 384);
        check(fromfile.build_window_geometry() == 0, "build_window_geometry from the window file");
        seedvr2::Win win;
        check(seedvr2::load_win(wpath, TXT, win) && win.nwin == info.nwin && win.t == t && win.h == h &&
                  win.w == w, "load_win");
        seedvr2::AwaLayer nofile;
        nofile.set_config(win_type, Lv, TXT);
        nofile.set_win_dir(win_dir + "missing/");
        check(nofile.build_window_geometry() == -1, "build_window_geometry without the file returns -1");
        std::vector<float> bad = fvidx;
        bad[1] = bad[0];
        seedvr2::AwaLayer rejecting;
        check(rejecting.set_window_geometry(bad, fcumf, vf, tf, info.nwin, Lv, TXT) == -1,
              "set_window_geometry rejects a token in two windows");

        for (int bf = 0; bf < 2; bf++) {
            const size_t es = bf ? 2 : 4;
            const void* v = bf ? (const void*)d_v16 : (const void*)d_v;
            const void* tq = bf ? (const void*)d_t16 : (const void*)d_t;
            int r1 = built.forward(v, vqkv.size() * es, tq, tqkv.size() * es, d_o1, d_to1, bf);
            int r2 = injected.forward(v, vqkv.size() * es, tq, tqkv.size() * es, d_o2, d_to2, bf);
            CK(hipDeviceSynchronize());
            std::vector<uint8_t> a((size_t)Lv * AWA_DIM * es), b(a.size());
            std::vector<uint8_t> ta((size_t)TXT * AWA_DIM * es), tb(ta.size());
            CK(hipMemcpy(a.data(), d_o1, a.size(), hipMemcpyDeviceToHost));
            CK(hipMemcpy(b.data(), d_o2, b.size(), hipMemcpyDeviceToHost));
            CK(hipMemcpy(ta.data(), d_to1, ta.size(), hipMemcpyDeviceToHost));
            CK(hipMemcpy(tb.data(), d_to2, tb.size(), hipMemcpyDeviceToHost));
            char msg[128];
            std::snprintf(msg, sizeof msg, "win_type %d %s: built == injected geometry", win_type, bf ? "bf16" : "fp32");
            check(r1 == 0 && r2 == 0 && a == b && ta == tb, msg);
            int r3 = fromfile.forward(v, vqkv.size() * es, tq, tqkv.size() * es, d_o2, d_to2, bf);
            CK(hipDeviceSynchronize());
            CK(hipMemcpy(b.data(), d_o2, b.size(), hipMemcpyDeviceToHost));
            CK(hipMemcpy(tb.data(), d_to2, tb.size(), hipMemcpyDeviceToHost));
            std::snprintf(msg, sizeof msg, "win_type %d %s: built == window-file geometry", win_type,
                          bf ? "bf16" : "fp32");
            check(r3 == 0 && a == b && ta == tb, msg);
            if (!bf) {
                seedvr2::AwaVk vk;
                check(vk.init(0), "AwaVk::init");
                std::vector<float> vo, to;
                std::vector<float> g0(gains.begin(), gains.begin() + 128), g1(gains.begin() + 128, gains.begin() + 256);
                std::vector<float> g2(gains.begin() + 256, gains.begin() + 384), g3(gains.begin() + 384, gains.end());
                bool ok = vk.forward(vqkv, tqkv, built.geometry(), g0, g1, g2, g3, Lv, TXT, vo, to);
                std::snprintf(msg, sizeof msg, "win_type %d: AwaVk host vectors == AwaLayer fp32", win_type);
                check(ok && std::memcmp(vo.data(), a.data(), a.size()) == 0 &&
                          std::memcmp(to.data(), ta.data(), ta.size()) == 0, msg);
                std::vector<float> wo, wto;
                ok = vk.forward(vqkv, tqkv, win, g0, g1, g2, g3, Lv, TXT, wo, wto) &&
                     vk.forward(vqkv, tqkv, win, g0, g1, g2, g3, Lv, TXT, vo, to);  // cached geometry
                std::snprintf(msg, sizeof msg, "win_type %d: AwaVk with a Win record == AwaLayer fp32", win_type);
                check(ok && std::memcmp(wo.data(), a.data(), a.size()) == 0 &&
                          std::memcmp(wto.data(), ta.data(), ta.size()) == 0 && wo == vo && wto == to, msg);
                std::vector<float> short_v(vqkv.begin(), vqkv.end() - 1);
                check(!vk.forward(short_v, tqkv, built.geometry(), g0, g1, g2, g3, Lv, TXT, vo, to),
                      "AwaVk::forward rejects a short vqkv");
            }
        }
    }
    (void)hipFree(d_v); (void)hipFree(d_t); (void)hipFree(d_v16); (void)hipFree(d_t16); (void)hipFree(d_g);
    (void)hipFree(d_o1); (void)hipFree(d_o2); (void)hipFree(d_to1); (void)hipFree(d_to2);
    for (const char* n : {"win_nonshifted.bin", "win_shifted.bin"}) unlink((win_dir + n).c_str());
    rmdir(tmpdir);
    std::printf(fails ? "FAIL (%d)\n" : "ALL PASS\n", fails);
    return fails ? 1 : 0;
}

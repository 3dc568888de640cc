// dit_vk.hpp — header-only C++17 mirror of the reference's DitVk (dit_vk.h:24-72)
// over the C ABI (include/dit_model.h), for callers that hold the model as a
// DitVk object and exchange host vectors.
//
//   init(model_dir)   DitVk::init (dit_vk.cpp:140-203): the model directory's
//                     weights go to the device once and stay resident.
//   forward_grid(...) DitVk::forward_grid (dit_vk.cpp:752-763): (T, H, W, 33)
//                     -> (T, H, W, 16); the window geometry of each resolution
//                     (unshifted and shifted, make_windows' num_windows) is
//                     built on the device once and cached, as are the
//                     device buffers of the last shape.
//
// Differences a caller sees: the device and the window counts are arguments
// (the reference reads windows from win_*.bin or set_windows), status is a
// bool with the message on stderr, as the reference's DitVk prints its own.
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <cstdio>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "awa_capi.h"
#include "dit_model.h"

namespace seedvr2 {

class DitVk {
public:
    DitVk() = default;
    DitVk(const DitVk&) = delete;
    DitVk& operator=(const DitVk&) = delete;
    ~DitVk() { release(); }

    // n_layers / mm_layers: 32 / 10 for the reference checkpoint.
    bool init(const std::string& model_dir, int n_layers = 32, int mm_layers = 10, int hip_device = 0,
              std::array<int, 3> num_windows = {4, 3, 3}) {
        release();
        if (hipSetDevice(hip_device) != hipSuccess || awa_create(&ctx_, hip_device) != AWA_OK) {
            std::fprintf(stderr, "[DitVk] no HIP device %d\n", hip_device);
            return false;
        }
        nw_ = num_windows;
        if (dit_model_load(ctx_, model_dir.c_str(), n_layers, mm_layers, &model_, nullptr) != AWA_OK) {
            std::fprintf(stderr, "[DitVk] %s\n", awa_last_error(ctx_));
            release();
            return false;
        }
        return true;
    }
    bool ready() const { return model_ != nullptr; }

    bool forward_grid(const std::vector<float>& vid_grid, int T, int H, int W, const std::vector<float>& txt,
                      int TXT, float timestep, std::vector<float>& sr_latent) {
        if (!model_) return false;
        if (T < 1 || H < 2 || W < 2 || H % 2 || W % 2 || TXT < 1 ||
            vid_grid.size() != (size_t)T * H * W * 33 || txt.size() != (size_t)TXT * 5120) {
            std::fprintf(stderr, "[DitVk] forward_grid: bad shapes (T=%d H=%d W=%d TXT=%d)\n", T, H, W, TXT);
            return false;
        }
        awa_geom* g[2] = {nullptr, nullptr};
        if (!geometries(T, H / 2, W / 2, TXT, g)) return false;
        const size_t Lv = (size_t)T * (H / 2) * (W / 2);
        const size_t n_grid = vid_grid.size(), n_txt = txt.size(), n_x = (Lv + TXT) * 2560,
                     n_out = (size_t)T * H * W * 16;
        if (!buffers(n_grid + n_txt + n_x + n_out)) return false;
        float* d_grid = buf_;
        float* d_txt = d_grid + n_grid;
        float* d_x = d_txt + n_txt;
        float* d_out = d_x + n_x;
        sr_latent.assign(n_out, 0.f);
        hipError_t e = hipMemcpy(d_grid, vid_grid.data(), n_grid * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d_txt, txt.data(), n_txt * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail(hipGetErrorString(e));
        // the last layer's text rows attend to video only, as forward_latent runs them
        if (dit_model_forward_grid(ctx_, model_, g[0], g[1], 1, 1e-5f, timestep, d_grid, T, H, W, d_txt, TXT,
                                   d_x, d_out, nullptr) != AWA_OK)
            return fail(awa_last_error(ctx_));
        e = hipMemcpy(sr_latent.data(), d_out, n_out * 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return fail(hipGetErrorString(e));
        return true;
    }

    void release() {
        for (auto& kv : geoms_) {
            awa_geom_destroy(kv.second[0]);
            awa_geom_destroy(kv.second[1]);
        }
        geoms_.clear();
        if (buf_) (void)hipFree(buf_);
        buf_ = nullptr;
        buf_n_ = 0;
        if (model_) dit_model_destroy(ctx_, model_);
        model_ = nullptr;
        if (ctx_) awa_destroy(ctx_);
        ctx_ = nullptr;
    }

private:
    bool fail(const char* msg) {
        std::fprintf(stderr, "[DitVk] %s\n", msg);
        return false;
    }
    bool geometries(int t, int h, int w, int txt, awa_geom* (&g)[2]) {
        const auto key = std::make_tuple(t, h, w, txt);
        auto it = geoms_.find(key);
        if (it == geoms_.end()) {
            std::array<awa_geom*, 2> made = {nullptr, nullptr};
            for (int s = 0; s < 2; s++)
                if (awa_geom_build(ctx_, t, h, w, nw_.data(), txt, s, &made[s], nullptr) != AWA_OK) {
                    awa_geom_destroy(made[0]);
                    return fail(awa_last_error(ctx_));
                }
            it = geoms_.emplace(key, made).first;
        }
        g[0] = it->second[0];
        g[1] = it->second[1];
        return true;
    }
    bool buffers(size_t n) {
        if (n <= buf_n_) return true;
        if (buf_) (void)hipFree(buf_);
        buf_ = nullptr;
        buf_n_ = 0;
        if (hipMalloc(reinterpret_cast<void**>(&buf_), n * sizeof(float)) != hipSuccess)
            return fail("hipMalloc of the forward buffers failed");
        buf_n_ = n;
        return true;
    }

    awa_ctx* ctx_ = nullptr;
    dit_model* model_ = nullptr;
    std::array<int, 3> nw_{4, 3, 3};
    std::map<std::tuple<int, int, int, int>, std::array<awa_geom*, 2>> geoms_;
    float* buf_ = nullptr;
    size_t buf_n_ = 0;
};

}  // namespace seedvr2

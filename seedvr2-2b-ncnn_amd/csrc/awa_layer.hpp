// awa_layer.hpp — C++17 host mirror of the reference's AWA operator surfaces
// over the C ABI (include/awa_capi.h).  Header-only; link libseedvr2_awa.so.
//
//   AwaLayer  mirrors the ncnn custom layer (src/awa_layer.h:26-108): the same
//             params (win_type, Lv, TXT), the four 128-wide qk-norm gains,
//             host-injected geometry through set_window_geometry, and a
//             forward that takes device buffers and returns 0 / -1, recording
//             on a stream without synchronising (awa_layer.cpp:284-453).
//   AwaVk     mirrors the host-vector module (src/awa_vk.h:14-52): init on a
//             device, synchronous forward on std::vector<float>, bool result.
//   Win       the reference's window record (src/dit_vk.h:17-22) and
//             load_win (dit_vk.cpp:74-93), which both classes accept.
//
// Both are single-threaded, like the reference's classes.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "awa_capi.h"
#include "dit_model.h"

namespace seedvr2 {

// struct Win (dit_vk.h:17-22): grid, windows [st,en) x [sh,eh) x [sw,ew),
// vid_freq [sum f][126] in window order, txt_freq [nwin*txt_len][126].
struct Win {
    int t = 0, h = 0, w = 0, nwin = 0;
    std::vector<int> st, en, sh, eh, sw, ew;
    std::vector<float> vid_freq, txt_freq;
};

// load_win (dit_vk.cpp:74-93): a win_*.bin file, the float tables split by
// txt_len.  Returns false (message on stderr) on a missing or malformed file.
inline bool load_win(const std::string& path, int txt_len, Win& out) {
    int64_t hdr[10];
    int32_t* sl = nullptr;
    float *vf = nullptr, *tf = nullptr;
    int64_t nv = 0, nt = 0;
    if (dit_read_win(path.c_str(), txt_len, hdr, &sl, &vf, &nv, &tf, &nt) != 0) {
        std::fprintf(stderr, "[load_win] %s\n", dit_host_last_error());
        return false;
    }
    Win w;
    w.t = (int)hdr[0]; w.h = (int)hdr[1]; w.w = (int)hdr[2]; w.nwin = (int)hdr[9];
    for (int i = 0; i < w.nwin; i++) {
        w.st.push_back(sl[6 * i]); w.en.push_back(sl[6 * i + 1]);
        w.sh.push_back(sl[6 * i + 2]); w.eh.push_back(sl[6 * i + 3]);
        w.sw.push_back(sl[6 * i + 4]); w.ew.push_back(sl[6 * i + 5]);
    }
    w.vid_freq.assign(vf, vf + nv);
    w.txt_freq.assign(tf, tf + nt);
    dit_free_host(sl);
    dit_free_host(vf);
    dit_free_host(tf);
    out = std::move(w);
    return true;
}

// The device geometry of a Win (awa_geom_from_win); nullptr on error, with
// the message in awa_last_error(ctx).
inline awa_geom* geometry_from_win(awa_ctx* ctx, const Win& w, int txt_len,
                                   awa_stream_t stream = nullptr) {
    const size_t n = (size_t)w.nwin;
    if (w.st.size() != n || w.en.size() != n || w.sh.size() != n || w.eh.size() != n ||
        w.sw.size() != n || w.ew.size() != n || w.txt_freq.size() != n * txt_len * AWA_ROPE_ROT)
        return nullptr;
    std::vector<int32_t> sl(6 * n);
    size_t sumf = 0;
    for (size_t i = 0; i < n; i++) {
        const int32_t r[6] = {w.st[i], w.en[i], w.sh[i], w.eh[i], w.sw[i], w.ew[i]};
        std::memcpy(&sl[6 * i], r, sizeof r);
        if (r[1] > r[0] && r[3] > r[2] && r[5] > r[4])
            sumf += (size_t)(r[1] - r[0]) * (r[3] - r[2]) * (r[5] - r[4]);
    }
    if (w.vid_freq.size() != sumf * AWA_ROPE_ROT) return nullptr;
    awa_geom* g = nullptr;
    if (awa_geom_from_win(ctx, w.t, w.h, w.w, w.nwin, sl.data(), w.vid_freq.data(), w.txt_freq.data(),
                          txt_len, &g, stream) != AWA_OK)
        return nullptr;
    return g;
}

class AwaLayer {
public:
    AwaLayer() = default;
    ~AwaLayer() { release(); }
    AwaLayer(const AwaLayer&) = delete;
    AwaLayer& operator=(const AwaLayer&) = delete;

    // AwaLayer::create_pipeline: acquire the device context.
    int create(int hip_device = 0) {
        if (ctx_) return 0;
        if (awa_create(&ctx_, hip_device) != AWA_OK) {
            std::fprintf(stderr, "[AwaLayer] awa_create(%d) failed\n", hip_device);
            return -1;
        }
        return 0;
    }
    void release() {
        if (geom_) awa_geom_destroy(geom_);
        geom_ = nullptr;
        if (ctx_) awa_destroy(ctx_);
        ctx_ = nullptr;
    }

    // load_param 1..3 (awa_layer.h:11-16): window type 0 unshifted / 1 shifted.
    void set_config(int win_type, int Lv, int TXT) {
        win_type_ = win_type;
        Lv_ = Lv;
        TXT_ = TXT;
    }
    // load_model / set_qk_norm_host: nq_v, nk_v, nq_t, nk_t, 128 floats each,
    // given as DEVICE pointers (the caller owns them; they must outlive forward).
    void set_qk_norm_device(const float* nqv, const float* nkv, const float* nqt, const float* nkt) {
        g_[0] = nqv; g_[1] = nkv; g_[2] = nqt; g_[3] = nkt;
    }
    // set_window_geometry (awa_layer.cpp:73-91): float-encoded vidx/cumf and
    // the two frequency tables; replaces any previous geometry.
    int set_window_geometry(const std::vector<float>& vidx, const std::vector<float>& cumf,
                            const std::vector<float>& vfreq, const std::vector<float>& tfreq,
                            int nwin, int Lv, int TXT) {
        if (!ctx_ && create() != 0) return -1;
        if ((int)cumf.size() != nwin + 1 || vfreq.size() != vidx.size() * AWA_ROPE_ROT ||
            tfreq.size() != (size_t)nwin * TXT * AWA_ROPE_ROT) {
            std::fprintf(stderr, "[AwaLayer] set_window_geometry: inconsistent sizes\n");
            return -1;
        }
        awa_geom* g = nullptr;
        if (awa_geom_set(ctx_, vidx.data(), cumf.data(), vfreq.data(), tfreq.data(), nwin, Lv, TXT,
                         &g, nullptr) != AWA_OK) {
            std::fprintf(stderr, "[AwaLayer] %s\n", awa_last_error(ctx_));
            return -1;
        }
        if (geom_) awa_geom_destroy(geom_);
        geom_ = g;
        Lv_ = Lv;
        TXT_ = TXT;
        return 0;
    }
    // load_param 0 (awa_layer.h:11-16): the directory that holds
    // win_nonshifted.bin and win_shifted.bin.
    void set_win_dir(const std::string& dir) { win_dir_ = dir; }
    // build_window_geometry (awa_layer.cpp:110-141): the window file of this
    // layer's win_type from the directory, TXT text rows per window.
    int build_window_geometry() {
        const std::string path = win_dir_ + (win_type_ == 0 ? "win_nonshifted.bin" : "win_shifted.bin");
        Win w;
        if (!load_win(path, TXT_, w)) return -1;
        return set_window_geometry(w, TXT_);
    }
    // The geometry of a reference Win record.
    int set_window_geometry(const Win& w, int TXT) {
        if (!ctx_ && create() != 0) return -1;
        awa_geom* g = geometry_from_win(ctx_, w, TXT);
        if (!g) {
            std::fprintf(stderr, "[AwaLayer] window record rejected: %s\n", awa_last_error(ctx_));
            return -1;
        }
        if (geom_) awa_geom_destroy(geom_);
        geom_ = g;
        Lv_ = w.t * w.h * w.w;
        TXT_ = TXT;
        return 0;
    }
    // The native alternative: build the geometry on the device (awa::make_win).
    int build_window_geometry(int t, int h, int w, const int32_t num_windows[3], int TXT) {
        if (!ctx_ && create() != 0) return -1;
        awa_geom* g = nullptr;
        if (awa_geom_build(ctx_, t, h, w, num_windows, TXT, win_type_, &g, nullptr) != AWA_OK) {
            std::fprintf(stderr, "[AwaLayer] %s\n", awa_last_error(ctx_));
            return -1;
        }
        if (geom_) awa_geom_destroy(geom_);
        geom_ = g;
        Lv_ = t * h * w;
        TXT_ = TXT;
        return 0;
    }
    bool geometry_ready() const { return geom_ != nullptr; }
    int win_type() const { return win_type_; }

    // forward(bottoms {vqkv, tqkv}, tops {vattn, tattn}): device buffers of
    // [Lv][7680], [TXT][7680] in, [Lv][2560], [TXT][2560] out; bf16 selects
    // 2-byte storage (ncnn's use_bf16_storage), else fp32.  Lv and TXT are
    // inferred from the byte sizes as awa_layer.cpp:296-308 does.
    int forward(const void* vqkv, size_t vqkv_bytes, const void* tqkv, size_t tqkv_bytes,
                void* vattn, void* tattn, bool bf16, awa_stream_t stream = nullptr) const {
        if (!ctx_ || !geom_) {
            std::fprintf(stderr, "[AwaLayer] FAIL: window geometry not set\n");
            return -1;
        }
        const size_t es = bf16 ? 2 : 4;
        const int Lv = (int)(vqkv_bytes / es / AWA_QKV), TXT = (int)(tqkv_bytes / es / AWA_QKV);
        if (Lv <= 0 || TXT <= 0) {
            std::fprintf(stderr, "[AwaLayer] FAIL: input shape (%zu, %zu bytes)\n", vqkv_bytes, tqkv_bytes);
            return -1;
        }
        if (!g_[0] || !g_[1] || !g_[2] || !g_[3]) {
            std::fprintf(stderr, "[AwaLayer] FAIL: qk-norm gains not set\n");
            return -1;
        }
        const int rc = awa_forward(ctx_, geom_, bf16 ? AWA_BF16 : AWA_F32, vqkv, tqkv, Lv, TXT, g_[0],
                                   g_[1], g_[2], g_[3], eps_, vattn, tattn, stream);
        if (rc != AWA_OK) {
            std::fprintf(stderr, "[AwaLayer] %s\n", awa_last_error(ctx_));
            return -1;
        }
        return 0;
    }
    void set_eps(float eps) { eps_ = eps; }
    awa_ctx* context() const { return ctx_; }
    const awa_geom* geometry() const { return geom_; }

private:
    awa_ctx* ctx_ = nullptr;
    awa_geom* geom_ = nullptr;
    const float* g_[4] = {nullptr, nullptr, nullptr, nullptr};
    int win_type_ = 0, Lv_ = 0, TXT_ = 0;
    float eps_ = 1e-5f;  // dit_vk.cpp:17, awa_layer.cpp:20
    std::string win_dir_;
};

class AwaVk {
public:
    ~AwaVk() { release(); }
    bool init(int hip_device = 0) { return ctx_ || awa_create(&ctx_, hip_device) == AWA_OK; }
    bool ready() const { return ctx_ != nullptr; }
    void release() {
        if (win_geom_) awa_geom_destroy(win_geom_);
        win_geom_ = nullptr;
        win_key_.clear();
        if (ctx_) awa_destroy(ctx_);
        ctx_ = nullptr;
    }
    // AwaVk::forward with the reference's signature (awa_vk.h:40-45): the
    // window as a Win record.  Its device geometry is built on first use and
    // kept while the record's contents stay the same.
    bool forward(const std::vector<float>& vqkv, const std::vector<float>& tqkv, const Win& win,
                 const std::vector<float>& nq_v, const std::vector<float>& nk_v,
                 const std::vector<float>& nq_t, const std::vector<float>& nk_t, int Lv, int TXT,
                 std::vector<float>& vid_out, std::vector<float>& txt_out, float eps = 1e-5f) {
        if (!ctx_) return false;
        std::vector<uint8_t> key = win_key(win, TXT);
        if (!win_geom_ || key != win_key_) {
            if (win_geom_) awa_geom_destroy(win_geom_);
            win_key_.clear();
            win_geom_ = geometry_from_win(ctx_, win, TXT);
            if (!win_geom_) {
                std::fprintf(stderr, "[AwaVk] window record rejected: %s\n", awa_last_error(ctx_));
                return false;
            }
            win_key_ = std::move(key);
        }
        return forward(vqkv, tqkv, win_geom_, nq_v, nk_v, nq_t, nk_t, Lv, TXT, vid_out, txt_out, eps);
    }
    // AwaVk::forward (awa_vk.cpp:62-199); the window comes as make_win's
    // parameters, built on the device once per call site and cached.
    bool forward(const std::vector<float>& vqkv, const std::vector<float>& tqkv, const awa_geom* win,
                 const std::vector<float>& nq_v, const std::vector<float>& nk_v,
                 const std::vector<float>& nq_t, const std::vector<float>& nk_t, int Lv, int TXT,
                 std::vector<float>& vid_out, std::vector<float>& txt_out, float eps = 1e-5f) {
        if (!ctx_ || !win) return false;
        if (vqkv.size() != (size_t)Lv * AWA_QKV || tqkv.size() != (size_t)TXT * AWA_QKV ||
            nq_v.size() != 128 || nk_v.size() != 128 || nq_t.size() != 128 || nk_t.size() != 128)
            return false;
        vid_out.assign((size_t)Lv * AWA_DIM, 0.f);
        txt_out.assign((size_t)TXT * AWA_DIM, 0.f);
        const int rc = awa_forward_host(ctx_, win, vqkv.data(), tqkv.data(), Lv, TXT, nq_v.data(),
                                        nk_v.data(), nq_t.data(), nk_t.data(), eps, vid_out.data(),
                                        txt_out.data());
        if (rc != AWA_OK) std::fprintf(stderr, "[AwaVk] %s\n", awa_last_error(ctx_));
        return rc == AWA_OK;
    }
    awa_ctx* context() const { return ctx_; }

private:
    // The record's bytes (sizes, slices, both tables): equal keys give the
    // same geometry.
    static std::vector<uint8_t> win_key(const Win& w, int TXT) {
        std::vector<uint8_t> k;
        auto put = [&k](const void* p, size_t n) {
            const uint8_t* b = static_cast<const uint8_t*>(p);
            k.insert(k.end(), b, b + n);
        };
        const int hdr[5] = {w.t, w.h, w.w, w.nwin, TXT};
        put(hdr, sizeof hdr);
        for (const std::vector<int>* v : {&w.st, &w.en, &w.sh, &w.eh, &w.sw, &w.ew})
            put(v->data(), v->size() * sizeof(int));
        put(w.vid_freq.data(), w.vid_freq.size() * 4);
        put(w.txt_freq.data(), w.txt_freq.size() * 4);
        return k;
    }

    awa_ctx* ctx_ = nullptr;
    awa_geom* win_geom_ = nullptr;
    std::vector<uint8_t> win_key_;
};

}  // namespace seedvr2

// dit_model.cpp — the loader of a model directory or a merged graph onto the
// device (the file readers are in dit_files.cpp), and the whole-model
// forward and its captured HIP graph.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <fstream>
#include <map>
#include <exception>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "dit_files.hpp"
#include "dit_internal.hpp"
#include "dit_model.h"

using namespace awa;
using namespace dit_files;

struct dit_model {
    int device = 0;
    int n_layers = 0, mm_layers = 0, mlp = 0;
    std::vector<void*> allocs;       // every device buffer of the model
    std::vector<dit_branch> vb, tb;  // per layer (tb[i] == vb[i] for shared layers)
    dit_io* io = nullptr;
    dit_time_weights tw{};
};

extern "C" {

void dit_model_destroy(awa_ctx* ctx, dit_model* m) {
    if (!m) return;
    DeviceGuard dg(ctx ? ctx->device : m->device);
    if (m->io) dit_io_destroy(ctx, m->io);
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
}

}  // extern "C"

namespace {

// The model's weights from src onto the device: linear weights as bf16, the
// SwiGLU pair packed, vectors and the timestep MLP as float32.
int load_model_from(awa_ctx* ctx, WeightSource& src, int n_layers, int mm_layers, dit_model** out,
                    awa_stream_t stream) {
    *out = nullptr;
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    dit_model* m = new dit_model();
    m->device = ctx->device;
    m->n_layers = n_layers;
    m->mm_layers = mm_layers;
    float* stage = nullptr;  // fp32 staging of one matrix on its way to bf16
    size_t stage_n = 0;
    int rc = AWA_OK;

    auto bad = [&](const char* fmt, const char* a, long x, long y) {
        set_err(ctx, fmt, a, x, y);
        rc = AWA_EARG;
    };
    auto dev_alloc = [&](size_t bytes) -> void* {
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            set_err(ctx, "dit_model_load: hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
            rc = AWA_EHIP;
            return nullptr;
        }
        m->allocs.push_back(p);
        return p;
    };
    auto upload_f32 = [&](const std::vector<float>& v) -> float* {
        float* p = static_cast<float*>(dev_alloc(v.size() * 4));
        if (!p) return nullptr;
        hipError_t e = hipMemcpy(p, v.data(), v.size() * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            set_err(ctx, "dit_model_load: %s", hipGetErrorString(e));
            rc = AWA_EHIP;
            return nullptr;
        }
        return p;
    };
    auto upload_bf16 = [&](const std::vector<float>& v) -> uint16_t* {
        if (stage_n < v.size()) {
            if (stage) (void)hipFree(stage);
            stage = nullptr;
            stage_n = 0;
            if (hipMalloc(reinterpret_cast<void**>(&stage), v.size() * 4) != hipSuccess) {
                set_err(ctx, "dit_model_load: hipMalloc of the staging buffer failed");
                rc = AWA_EHIP;
                return nullptr;
            }
            stage_n = v.size();
        }
        uint16_t* p = static_cast<uint16_t*>(dev_alloc(v.size() * 2));
        if (!p) return nullptr;
        hipError_t e = hipMemcpy(stage, v.data(), v.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = launch_cast_f32_bf16(stage, p, (int64_t)v.size(), s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);  // the staging buffer is reused
        if (e != hipSuccess) {
            set_err(ctx, "dit_model_load: %s", hipGetErrorString(e));
            rc = AWA_EHIP;
            return nullptr;
        }
        return p;
    };
    // the readers return -1 on a bad file; an exception (memory exhausted by
    // a huge but well-formed file) is turned into the same error
    auto read_ok = [&](auto&& read) {
        try {
            return read() == 0;
        } catch (const std::exception& e) {
            fail("%s", e.what());
            return false;
        }
    };
    auto linear = [&](const std::string& name, bool bias, int n_out, int n_in, HostLinear& L) {
        if (rc != AWA_OK) return false;
        if (!read_ok([&] { return src.linear(name, bias, L); })) {
            set_err(ctx, "dit_model_load: %s", last_error().c_str());
            rc = AWA_EARG;
            return false;
        }
        if ((n_out > 0 && L.n_out != n_out) || (n_in > 0 && L.n_in != n_in)) {
            bad("dit_model_load: %s is %ld x %ld", name.c_str(), L.n_out, L.n_in);
            return false;
        }
        return true;
    };
    auto vec = [&](const std::string& name, size_t n) -> float* {
        if (rc != AWA_OK) return nullptr;
        std::vector<float> v;
        if (!read_ok([&] { return src.vec(name, v); })) {
            set_err(ctx, "dit_model_load: %s", last_error().c_str());
            rc = AWA_EARG;
            return nullptr;
        }
        if (v.size() != n) {
            bad("dit_model_load: %s holds %ld floats, expected %ld", name.c_str(), (long)v.size(), (long)n);
            return nullptr;
        }
        return upload_f32(v);
    };

    // input / output layers and the timestep MLP
    HostLinear L;
    dit_io_weights iw{};
    if (linear("vid_in_proj", true, DIM, 132, L)) { iw.vid_in_w = upload_bf16(L.w); iw.vid_in_b = upload_f32(L.b); }
    if (linear("txt_in", true, DIM, 5120, L)) { iw.txt_in_w = upload_bf16(L.w); iw.txt_in_b = upload_f32(L.b); }
    if (linear("vid_out_proj", true, 64, DIM, L)) { iw.vid_out_w = upload_bf16(L.w); iw.vid_out_b = upload_f32(L.b); }
    iw.out_norm_w = vec("vid_out_norm_w", DIM);
    iw.out_ada_shift = vec("vid_out_ada_shift", DIM);
    iw.out_ada_scale = vec("vid_out_ada_scale", DIM);
    if (linear("emb_proj_in", true, DIM, 256, L)) { m->tw.w_in = upload_f32(L.w); m->tw.b_in = upload_f32(L.b); }
    if (linear("emb_proj_hid", true, DIM, DIM, L)) { m->tw.w_hid = upload_f32(L.w); m->tw.b_hid = upload_f32(L.b); }
    if (linear("emb_proj_out", true, DIT_EMB, DIM, L)) { m->tw.w_out = upload_f32(L.w); m->tw.b_out = upload_f32(L.b); }
    if (rc == AWA_OK) rc = dit_io_create(ctx, &iw, &m->io, stream);

    // layers: dual branches below mm_layers, one shared branch above
    auto branch = [&](const std::string& b, dit_branch& br) {
        HostLinear qkv, o, mi, mg, mo;
        if (linear(b + "_qkv", false, QKV, DIM, qkv)) br.qkv_w = upload_bf16(qkv.w);
        if (linear(b + "_out", true, DIM, DIM, o)) { br.out_w = upload_bf16(o.w); br.out_b = upload_f32(o.b); }
        if (linear(b + "_mlp_in", false, m->mlp > 0 ? m->mlp : 0, DIM, mi) &&
            linear(b + "_mlp_g", false, mi.n_out, DIM, mg) && linear(b + "_mlp_out", false, DIM, mi.n_out, mo)) {
            if (mi.n_out % 128) {
                bad("dit_model_load: %s MLP width %ld (%ld) is not a multiple of 128", b.c_str(), mi.n_out, 0);
            } else {
                m->mlp = mi.n_out;
                uint16_t* win = upload_bf16(mi.w);
                uint16_t* wg = upload_bf16(mg.w);
                uint16_t* cat = static_cast<uint16_t*>(dev_alloc((size_t)2 * m->mlp * DIM * 2));
                if (rc == AWA_OK && win && wg && cat) {
                    hipError_t e = launch_pack_mlp(win, wg, m->mlp, cat, s);
                    if (e != hipSuccess) {
                        set_err(ctx, "dit_model_load: %s", hipGetErrorString(e));
                        rc = AWA_EHIP;
                    }
                }
                br.mlp_w = cat;
                br.mlp_out_w = upload_bf16(mo.w);
            }
        }
        br.nq = vec(b + "_nq", 128);
        br.nk = vec(b + "_nk", 128);
        br.attn_shift = vec(b + "_attn_shift", DIM);
        br.attn_scale = vec(b + "_attn_scale", DIM);
        br.attn_gate = vec(b + "_attn_gate", DIM);
        br.mlp_shift = vec(b + "_mlp_shift", DIM);
        br.mlp_scale = vec(b + "_mlp_scale", DIM);
        br.mlp_gate = vec(b + "_mlp_gate", DIM);
    };
    m->vb.resize(n_layers);
    m->tb.resize(n_layers);
    for (int i = 0; i < n_layers && rc == AWA_OK; i++) {
        const std::string p = "b" + std::to_string(i);
        if (i < mm_layers) {
            branch(p + "_vid", m->vb[i]);
            branch(p + "_txt", m->tb[i]);
        } else {
            branch(p + "_all", m->vb[i]);
            m->tb[i] = m->vb[i];
        }
    }
    if (rc == AWA_OK) {
        hipError_t e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            set_err(ctx, "dit_model_load: %s", hipGetErrorString(e));
            rc = AWA_EHIP;
        }
    }
    if (stage) (void)hipFree(stage);
    if (rc != AWA_OK) {
        dit_model_destroy(ctx, m);
        return rc;
    }
    *out = m;
    return AWA_OK;
}

}  // namespace

extern "C" {

int dit_model_load(awa_ctx* ctx, const char* dir, int n_layers, int mm_layers, dit_model** out,
                   awa_stream_t stream) {
    if (!ctx || !dir || !out || n_layers < 0 || mm_layers < 0 || mm_layers > n_layers) {
        set_err(ctx, "dit_model_load: bad argument (n_layers=%d mm_layers=%d)", n_layers, mm_layers);
        return AWA_EARG;
    }
    DirSource src(dir);
    return load_model_from(ctx, src, n_layers, mm_layers, out, stream);
}

int dit_model_load_graph(awa_ctx* ctx, const char* param, const char* bin, const char* dir, int mm_layers,
                         dit_model** out, awa_stream_t stream) {
    if (!ctx || !param || !bin || !out) {
        set_err(ctx, "dit_model_load_graph: null argument");
        return AWA_EARG;
    }
    *out = nullptr;
    GraphSource src;
    std::unique_ptr<DirSource> d(dir ? new DirSource(dir) : nullptr);
    src.dir = d.get();
    int bad_graph;
    try {
        bad_graph = index_graph(param, bin, mm_layers, src.G) || src.open();
    } catch (const std::exception& e) {
        bad_graph = fail("%s", e.what());
    }
    if (bad_graph) {
        set_err(ctx, "dit_model_load_graph: %s", last_error().c_str());
        return AWA_EARG;
    }
    return load_model_from(ctx, src, src.G.n_layers, src.G.mm_layers, out, stream);
}

int dit_model_info(const dit_model* m, int* n_layers, int* mm_layers, int* mlp) {
    if (!m) return AWA_EARG;
    if (n_layers) *n_layers = m->n_layers;
    if (mm_layers) *mm_layers = m->mm_layers;
    if (mlp) *mlp = m->mlp;
    return AWA_OK;
}

int dit_model_forward_grid(awa_ctx* ctx, const dit_model* m, const awa_geom* g_even, const awa_geom* g_odd,
                           int last_txt_vid_only, float eps, float t, const float* d_grid, int T, int H, int W,
                           const float* d_txt, int TXT, float* d_x, float* d_out, awa_stream_t stream) {
    if (!ctx || !m) {
        set_err(ctx, "dit_model_forward_grid: null argument");
        return AWA_EARG;
    }
    std::vector<const dit_branch*> vb(m->n_layers), tb(m->n_layers);
    for (int i = 0; i < m->n_layers; i++) {
        vb[i] = &m->vb[i];
        tb[i] = (i < m->mm_layers) ? &m->tb[i] : &m->vb[i];  // shared layers: the same branch
    }
    return dit_forward_grid(ctx, m->io, &m->tw, vb.data(), tb.data(), m->n_layers, g_even, g_odd, m->mlp,
                            last_txt_vid_only, eps, t, d_grid, T, H, W, d_txt, TXT, d_x, d_out, stream);
}

struct dit_graph {
    int device = 0;
    awa_ctx* priv = nullptr;  // owns the scratch baked into the graph
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

void dit_graph_destroy(dit_graph* g) {
    if (!g) return;
    DeviceGuard dg(g->device);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    if (g->priv) awa_destroy(g->priv);
    delete g;
}

int dit_graph_create(awa_ctx* ctx, const dit_model* m, const awa_geom* g_even, const awa_geom* g_odd,
                     int last_txt_vid_only, float eps, float t, const float* d_grid, int T, int H, int W,
                     const float* d_txt, int TXT, float* d_x, float* d_out, awa_stream_t stream, dit_graph** out) {
    if (!ctx || !m || !out || !stream) {
        set_err(ctx, "dit_graph_create: null argument (capture needs a created stream, not the null stream)");
        return AWA_EARG;
    }
    *out = nullptr;
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    dit_graph* g = new dit_graph();
    g->device = ctx->device;
    int rc = awa_create(&g->priv, ctx->device);
    if (rc != AWA_OK) {
        set_err(ctx, "dit_graph_create: private context: %s", g->priv ? awa_last_error(g->priv) : "awa_create failed");
        dit_graph_destroy(g);
        return rc;
    }
    // eager run: sizes the private context's buffers (no allocation may happen
    // while capturing) and checks every argument
    rc = dit_model_forward_grid(g->priv, m, g_even, g_odd, last_txt_vid_only, eps, t, d_grid, T, H, W, d_txt, TXT,
                                d_x, d_out, stream);
    hipError_t e = rc == AWA_OK ? hipStreamSynchronize(s) : hipSuccess;
    if (rc == AWA_OK && e == hipSuccess) {
        e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            rc = dit_model_forward_grid(g->priv, m, g_even, g_odd, last_txt_vid_only, eps, t, d_grid, T, H, W,
                                        d_txt, TXT, d_x, d_out, stream);
            hipError_t e2 = hipStreamEndCapture(s, &g->graph);
            if (rc == AWA_OK) e = e2;
        }
        if (rc == AWA_OK && e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    }
    if (rc != AWA_OK || e != hipSuccess) {
        if (rc != AWA_OK) set_err(ctx, "dit_graph_create: %s", awa_last_error(g->priv));
        else set_err(ctx, "dit_graph_create: %s", hipGetErrorString(e));
        dit_graph_destroy(g);
        return rc != AWA_OK ? rc : AWA_EHIP;
    }
    *out = g;
    return AWA_OK;
}

int dit_graph_launch(awa_ctx* ctx, dit_graph* g, awa_stream_t stream) {
    if (!ctx || !g) {
        set_err(ctx, "dit_graph_launch: null argument");
        return AWA_EARG;
    }
    DeviceGuard dg(g->device);
    hipError_t e = hipGraphLaunch(g->exec, reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        set_err(ctx, "dit_graph_launch: %s", hipGetErrorString(e));
        return AWA_EHIP;
    }
    return AWA_OK;
}

}  // extern "C"

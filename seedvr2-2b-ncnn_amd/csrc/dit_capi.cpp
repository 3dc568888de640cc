// dit_capi.cpp — C ABI of the DiT block: one layer of DitVk::forward_latent
// (dit_vk.cpp:517-632) as norm -> GEMM -> AWA -> GEMM -> norm -> GEMM -> GEMM
// on the caller's stream.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "dit_internal.hpp"

using namespace awa;

namespace {

#define HIPCK(ctx, expr)                                                                     \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess) {                                                              \
            set_err(ctx, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__,    \
                    __LINE__);                                                               \
            return AWA_EHIP;                                                                 \
        }                                                                                    \
    } while (0)

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

bool branch_ok(const dit_branch* b) {
    return b && b->qkv_w && b->out_w && b->out_b && b->mlp_w && b->mlp_out_w && b->nq && b->nk &&
           b->attn_shift && b->attn_scale && b->attn_gate && b->mlp_shift && b->mlp_scale && b->mlp_gate;
}

GemmProblem problem(const uint16_t* A, int lda, const uint16_t* W, int ldw, int M, int N, int K,
                    void* C, int ldc) {
    GemmProblem p{};
    p.A = A; p.lda = lda; p.W = W; p.ldw = ldw; p.M = M; p.N = N; p.K = K; p.C = C; p.ldc = ldc;
    p.split = M;
    return p;
}

constexpr int VID_IN = 132, VID_IN_PAD = 192;   // patch channels 33 x 2 x 2; K padded to the GEMM step (64)
constexpr int VID_OUT = 64, VID_OUT_PAD = 256;  // output channels 16 x 2 x 2; N padded to the GEMM tile

}  // namespace

struct dit_io {
    int device = 0;
    uint16_t* vid_in_w = nullptr;   // [2560][192], columns 132.. zero
    const float* vid_in_b = nullptr;
    const uint16_t* txt_in_w = nullptr;
    const float* txt_in_b = nullptr;
    const float* out_norm_w = nullptr;
    const float* out_ada_shift = nullptr;
    const float* out_ada_scale = nullptr;
    uint16_t* vid_out_w = nullptr;  // [256][2560], rows 64.. zero
    float* vid_out_b = nullptr;     // [256], 64.. zero
};

extern "C" {

int dit_io_create(awa_ctx* ctx, const dit_io_weights* w, dit_io** out, awa_stream_t stream) {
    if (!ctx || !w || !out || !w->vid_in_w || !w->vid_in_b || !w->txt_in_w || !w->txt_in_b ||
        !w->out_norm_w || !w->out_ada_shift || !w->out_ada_scale || !w->vid_out_w || !w->vid_out_b) {
        set_err(ctx, "dit_io_create: null argument");
        return AWA_EARG;
    }
    *out = nullptr;
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    dit_io* io = new dit_io();
    io->device = ctx->device;
    io->vid_in_b = w->vid_in_b; io->txt_in_w = w->txt_in_w; io->txt_in_b = w->txt_in_b;
    io->out_norm_w = w->out_norm_w; io->out_ada_shift = w->out_ada_shift; io->out_ada_scale = w->out_ada_scale;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&io->vid_in_w), (size_t)DIM * VID_IN_PAD * 2);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&io->vid_out_w), (size_t)VID_OUT_PAD * DIM * 2);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&io->vid_out_b), VID_OUT_PAD * 4);
    // zero, then copy the real rows / columns in (set-up, not in a captured sequence)
    if (e == hipSuccess) e = hipMemsetAsync(io->vid_in_w, 0, (size_t)DIM * VID_IN_PAD * 2, s);
    if (e == hipSuccess) e = hipMemsetAsync(io->vid_out_w, 0, (size_t)VID_OUT_PAD * DIM * 2, s);
    if (e == hipSuccess) e = hipMemsetAsync(io->vid_out_b, 0, VID_OUT_PAD * 4, s);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(io->vid_in_w, VID_IN_PAD * 2, w->vid_in_w, VID_IN * 2, VID_IN * 2, DIM,
                             hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(io->vid_out_w, w->vid_out_w, (size_t)VID_OUT * DIM * 2, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(io->vid_out_b, w->vid_out_b, VID_OUT * 4, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) {
        set_err(ctx, "dit_io_create: %s", hipGetErrorString(e));
        dit_io_destroy(ctx, io);
        return AWA_EHIP;
    }
    *out = io;
    return AWA_OK;
}

void dit_io_destroy(awa_ctx* ctx, dit_io* io) {
    if (!io) return;
    DeviceGuard dg(ctx ? ctx->device : io->device);
    if (io->vid_in_w) (void)hipFree(io->vid_in_w);
    if (io->vid_out_w) (void)hipFree(io->vid_out_w);
    if (io->vid_out_b) (void)hipFree(io->vid_out_b);
    delete io;
}

namespace {
// workspace bytes of each entry point (the offsets below follow the same layouts)
size_t embed_ws_bytes(int Lv, int TXT) {
    return align256((size_t)Lv * VID_IN_PAD * 2) + align256((size_t)TXT * 5120 * 2);
}
size_t final_ws_bytes(int Lv) {
    return align256(2 * DIM * 4) + align256((size_t)Lv * DIM * 2) + align256((size_t)Lv * VID_OUT_PAD * 4);
}
size_t layer_ws_bytes(int M, int mlp) {
    return align256(12 * DIM * 4) + align256((size_t)M * DIM * 2) + align256((size_t)M * QKV * 2) +
           align256((size_t)M * DIM * 2) + align256((size_t)M * mlp * 2);
}
}  // namespace

int dit_reserve(awa_ctx* ctx, const awa_geom* g, int mlp) {
    if (!ctx || !g || mlp <= 0 || mlp % 128 != 0 || mlp > DIT_MLP_MAX) {
        set_err(ctx, "dit_reserve: bad argument (mlp=%d must be a positive multiple of 128, at most %d)", mlp,
                DIT_MLP_MAX);
        return AWA_EARG;
    }
    const int Lv = g->plan.Lv, TXT = g->plan.txt_len;
    const size_t need = std::max(layer_ws_bytes(Lv + TXT, mlp), std::max(embed_ws_bytes(Lv, TXT), final_ws_bytes(Lv)));
    DeviceGuard dg(ctx->device);
    HIPCK(ctx, ensure_buffer(&ctx->ws, &ctx->ws_bytes, need));
    return awa_reserve(ctx, g, AWA_BF16);
}

int dit_embed(awa_ctx* ctx, const dit_io* io, const float* d_grid, int T, int H, int W, const float* d_txt,
              int TXT, float* d_x, awa_stream_t stream) {
    if (!ctx || !io || !d_grid || !d_txt || !d_x || T < 1 || H < 2 || W < 2 || H % 2 || W % 2 || TXT < 1) {
        set_err(ctx, "dit_embed: bad argument (T=%d H=%d W=%d TXT=%d; H and W even)", T, H, W, TXT);
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int Lv = T * (H / 2) * (W / 2), M = Lv + TXT;
    // workspace: patches [Lv][192] bf16 | text [TXT][5120] bf16
    const size_t o_t = align256((size_t)Lv * VID_IN_PAD * 2);
    HIPCK(ctx, ensure_buffer(&ctx->ws, &ctx->ws_bytes, embed_ws_bytes(Lv, TXT)));
    uint16_t* patch = static_cast<uint16_t*>(ctx->ws);
    uint16_t* txt = reinterpret_cast<uint16_t*>(static_cast<char*>(ctx->ws) + o_t);
    HIPCK(ctx, launch_patchify(d_grid, T, H, W, patch, VID_IN_PAD, s));
    HIPCK(ctx, launch_cast_f32_bf16(d_txt, txt, (int64_t)TXT * 5120, s));
    // x = A W^T + b: the residual epilogue on a zeroed x, gate 1
    HIPCK(ctx, launch_zero(d_x, (size_t)M * DIM * 4, s));
    GemmBatch b{};
    b.nprob = 2;
    b.p[0] = problem(patch, VID_IN_PAD, io->vid_in_w, VID_IN_PAD, Lv, DIM, VID_IN_PAD, d_x, DIM);
    b.p[0].bias = io->vid_in_b;
    b.p[1] = problem(txt, 5120, io->txt_in_w, 5120, TXT, DIM, 5120, d_x + (size_t)Lv * DIM, DIM);
    b.p[1].bias = io->txt_in_b;
    HIPCK(ctx, launch_gemm(EPI_RESID, b, s));
    return AWA_OK;
}

int dit_final(awa_ctx* ctx, const dit_io* io, const float* d_emb, const float* d_x, int T, int H, int W,
              float eps, float* d_out, awa_stream_t stream) {
    if (!ctx || !io || !d_emb || !d_x || !d_out || T < 1 || H < 2 || W < 2 || H % 2 || W % 2 || !(eps > 0.f)) {
        set_err(ctx, "dit_final: bad argument (T=%d H=%d W=%d; H and W even, eps > 0)", T, H, W);
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int Lv = T * (H / 2) * (W / 2);
    // workspace: scale, shift [2][2560] f32 | h [Lv][2560] bf16 | y [Lv][256] f32
    const size_t o_h = align256(2 * DIM * 4);
    const size_t o_y = o_h + align256((size_t)Lv * DIM * 2);
    HIPCK(ctx, ensure_buffer(&ctx->ws, &ctx->ws_bytes, final_ws_bytes(Lv)));
    char* ws = static_cast<char*>(ctx->ws);
    float* scale = reinterpret_cast<float*>(ws);
    float* shift = scale + DIM;
    uint16_t* h = reinterpret_cast<uint16_t*>(ws + o_h);
    float* y = reinterpret_cast<float*>(ws + o_y);
    HIPCK(ctx, launch_final_ada(d_emb, io->out_norm_w, io->out_ada_scale, io->out_ada_shift, scale, shift, s));
    NormArgs na{};
    na.x = d_x; na.h = h; na.M = Lv; na.split = Lv; na.eps = eps;
    na.scale0 = scale; na.shift0 = shift;
    HIPCK(ctx, launch_norm_ada(na, s));
    HIPCK(ctx, launch_zero(y, (size_t)Lv * VID_OUT_PAD * 4, s));
    GemmBatch b{};
    b.nprob = 1;
    b.p[0] = problem(h, DIM, io->vid_out_w, DIM, Lv, VID_OUT_PAD, DIM, y, VID_OUT_PAD);
    b.p[0].bias = io->vid_out_b;
    HIPCK(ctx, launch_gemm(EPI_RESID, b, s));
    HIPCK(ctx, launch_unpatchify(y, VID_OUT_PAD, T, H, W, d_out, s));
    return AWA_OK;
}

int dit_pack_mlp_weights(awa_ctx* ctx, const uint16_t* d_w_in, const uint16_t* d_w_gate, int mlp,
                         uint16_t* d_w_cat, awa_stream_t stream) {
    if (!ctx || !d_w_in || !d_w_gate || !d_w_cat || mlp <= 0 || mlp % 128 != 0 || mlp > DIT_MLP_MAX) {
        set_err(ctx, "dit_pack_mlp_weights: bad argument (mlp=%d must be a positive multiple of 128, at most %d)",
                mlp, DIT_MLP_MAX);
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    HIPCK(ctx, launch_pack_mlp(d_w_in, d_w_gate, mlp, d_w_cat, reinterpret_cast<hipStream_t>(stream)));
    return AWA_OK;
}

int dit_time_embedding(awa_ctx* ctx, float t, const float* d_w_in, const float* d_b_in,
                       const float* d_w_hid, const float* d_b_hid, const float* d_w_out,
                       const float* d_b_out, float* d_emb, awa_stream_t stream) {
    if (!ctx || !d_w_in || !d_b_in || !d_w_hid || !d_b_hid || !d_w_out || !d_b_out || !d_emb) {
        set_err(ctx, "dit_time_embedding: null argument");
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (!ctx->small) HIPCK(ctx, hipMalloc(reinterpret_cast<void**>(&ctx->small), 8192 * sizeof(float)));
    float* e0 = ctx->small;          // [256]
    float* e1 = e0 + 256;            // [2560]
    float* e2 = e1 + DIM;            // [2560]
    HIPCK(ctx, launch_sinusoid(t, e0, 256, s));
    HIPCK(ctx, launch_gemv_f32(d_w_in, d_b_in, e0, e1, 256, DIM, 1, s));
    HIPCK(ctx, launch_gemv_f32(d_w_hid, d_b_hid, e1, e2, DIM, DIM, 1, s));
    HIPCK(ctx, launch_gemv_f32(d_w_out, d_b_out, e2, d_emb, DIM, DIT_EMB, 0, s));
    return AWA_OK;
}

int dit_gemm_bf16(awa_ctx* ctx, const uint16_t* d_A, const uint16_t* d_W, uint16_t* d_C, int M, int N,
                  int K, awa_stream_t stream) {
    if (!ctx || !d_A || !d_W || !d_C || M < 1 || N < 256 || N % 256 || N > DIT_GEMM_NK_MAX || K < 64 || K % 64 ||
        K > DIT_GEMM_NK_MAX) {
        set_err(ctx, "dit_gemm_bf16: bad argument M=%d N=%d K=%d (N %% 256 == 0, K %% 64 == 0, N, K <= %d)", M, N, K,
                DIT_GEMM_NK_MAX);
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    GemmBatch b{};
    b.nprob = 1;
    b.p[0] = problem(d_A, K, d_W, K, M, N, K, d_C, N);
    HIPCK(ctx, launch_gemm(EPI_STORE, b, reinterpret_cast<hipStream_t>(stream)));
    return AWA_OK;
}

int dit_layer_forward(awa_ctx* ctx, const awa_geom* g, const dit_branch* vb, const dit_branch* tb,
                      const float* d_emb, int mlp, int txt_vid_only, float eps, float* d_x, int Lv,
                      int TXT, awa_stream_t stream) {
    if (!ctx || !g || !d_emb || !d_x || !branch_ok(vb) || !branch_ok(tb)) {
        set_err(ctx, "dit_layer_forward: null argument or incomplete branch");
        return AWA_EARG;
    }
    if (Lv != g->plan.Lv || TXT != g->plan.txt_len) {
        set_err(ctx, "dit_layer_forward: Lv=%d TXT=%d do not match the geometry (Lv=%d TXT=%d)", Lv,
                TXT, g->plan.Lv, g->plan.txt_len);
        return AWA_EARG;
    }
    if (mlp <= 0 || mlp % 128 != 0 || mlp > DIT_MLP_MAX || !(eps > 0.f)) {
        set_err(ctx, "dit_layer_forward: mlp=%d must be a positive multiple of 128 (at most %d), eps > 0", mlp,
                DIT_MLP_MAX);
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool dual = vb != tb;
    const int M = Lv + TXT;
    const int Mm = txt_vid_only ? Lv : M;  // rows that run the MLP

    // workspace: ada [12][2560] f32 | h [M][2560] | qkv [M][7680] | attn [M][2560] | u [M][mlp]
    const size_t o_h = align256(12 * DIM * 4);
    const size_t o_qkv = o_h + align256((size_t)M * DIM * 2);
    const size_t o_att = o_qkv + align256((size_t)M * QKV * 2);
    const size_t o_u = o_att + align256((size_t)M * DIM * 2);
    HIPCK(ctx, ensure_buffer(&ctx->ws, &ctx->ws_bytes, layer_ws_bytes(M, mlp)));
    char* ws = static_cast<char*>(ctx->ws);
    float* ada = reinterpret_cast<float*>(ws);
    uint16_t* h = reinterpret_cast<uint16_t*>(ws + o_h);
    uint16_t* qkv = reinterpret_cast<uint16_t*>(ws + o_qkv);
    uint16_t* att = reinterpret_cast<uint16_t*>(ws + o_att);
    uint16_t* u = reinterpret_cast<uint16_t*>(ws + o_u);
    auto V = [&](int f, int k) { return ada + (size_t)(f * 6 + k) * DIM; };  // a_sc a_sh a_g m_sc m_sh m_g
    auto mark = [&]() { return event_mark(ctx, ctx->dit_ev_used, s); };

    HIPCK(ctx, mark());
    AdaArgs aa{};
    aa.emb = d_emb;
    aa.out = ada;
    const dit_branch* br[2] = {vb, tb};
    for (int f = 0; f < 2; f++) {
        aa.vec[f][0] = br[f]->attn_scale; aa.vec[f][1] = br[f]->attn_shift; aa.vec[f][2] = br[f]->attn_gate;
        aa.vec[f][3] = br[f]->mlp_scale;  aa.vec[f][4] = br[f]->mlp_shift;  aa.vec[f][5] = br[f]->mlp_gate;
    }
    HIPCK(ctx, launch_ada(aa, s));
    // attention norm + ada (dit_vk.cpp:530-545); last layer: text rows unmodulated
    NormArgs na{};
    na.x = d_x; na.h = h; na.M = M; na.split = Lv; na.eps = eps;
    na.scale0 = V(0, 0); na.shift0 = V(0, 1);
    na.scale1 = txt_vid_only ? nullptr : V(1, 0);
    na.shift1 = txt_vid_only ? nullptr : V(1, 1);
    HIPCK(ctx, launch_norm_ada(na, s));
    HIPCK(ctx, mark());

    // qkv projections (dit_vk.cpp:321-322), no bias
    GemmBatch b{};
    if (!dual) {
        b.nprob = 1;
        b.p[0] = problem(h, DIM, vb->qkv_w, DIM, M, QKV, DIM, qkv, QKV);
    } else {
        b.nprob = 2;
        b.p[0] = problem(h, DIM, vb->qkv_w, DIM, Lv, QKV, DIM, qkv, QKV);
        b.p[1] = problem(h + (size_t)Lv * DIM, DIM, tb->qkv_w, DIM, TXT, QKV, DIM, qkv + (size_t)Lv * QKV, QKV);
    }
    HIPCK(ctx, launch_gemm(EPI_STORE, b, s));
    HIPCK(ctx, mark());

    // the AWA op, bf16 boundary (awa_layer.cpp:338-451)
    int rc = forward_impl(ctx, g, AWA_BF16, qkv, qkv + (size_t)Lv * QKV, vb->nq, vb->nk, tb->nq, tb->nk, eps,
                          att, att + (size_t)Lv * DIM, s);
    if (rc != AWA_OK) return rc;
    HIPCK(ctx, mark());

    // out projection + bias, attention gate, residual (dit_vk.cpp:461-462, 558-575)
    b = GemmBatch{};
    if (!dual) {
        b.nprob = 1;
        b.p[0] = problem(att, DIM, vb->out_w, DIM, M, DIM, DIM, d_x, DIM);
        b.p[0].bias = vb->out_b;
        b.p[0].gate0 = V(0, 2);
        b.p[0].gate1 = txt_vid_only ? nullptr : V(1, 2);
        b.p[0].split = Lv;
    } else {
        b.nprob = 2;
        b.p[0] = problem(att, DIM, vb->out_w, DIM, Lv, DIM, DIM, d_x, DIM);
        b.p[0].bias = vb->out_b;
        b.p[0].gate0 = V(0, 2);
        b.p[1] = problem(att + (size_t)Lv * DIM, DIM, tb->out_w, DIM, TXT, DIM, DIM, d_x + (size_t)Lv * DIM, DIM);
        b.p[1].bias = tb->out_b;
        b.p[1].gate0 = txt_vid_only ? nullptr : V(1, 2);
    }
    HIPCK(ctx, launch_gemm(EPI_RESID, b, s));
    HIPCK(ctx, mark());

    // MLP norm + ada (dit_vk.cpp:577-597); last layer: text rows skip the MLP
    na = NormArgs{};
    na.x = d_x; na.h = h; na.M = Mm; na.split = Lv; na.eps = eps;
    na.scale0 = V(0, 3); na.shift0 = V(0, 4);
    na.scale1 = V(1, 3); na.shift1 = V(1, 4);
    HIPCK(ctx, launch_norm_ada(na, s));
    HIPCK(ctx, mark());

    // SwiGLU (dit_vk.cpp:465-472): u = silu(h Wg^T) * (h Win^T), then out, gate, residual
    b = GemmBatch{};
    if (!dual || txt_vid_only) {
        b.nprob = 1;
        b.p[0] = problem(h, DIM, vb->mlp_w, DIM, dual ? Lv : Mm, 2 * mlp, DIM, u, mlp);
    } else {
        b.nprob = 2;
        b.p[0] = problem(h, DIM, vb->mlp_w, DIM, Lv, 2 * mlp, DIM, u, mlp);
        b.p[1] = problem(h + (size_t)Lv * DIM, DIM, tb->mlp_w, DIM, TXT, 2 * mlp, DIM, u + (size_t)Lv * mlp, mlp);
    }
    HIPCK(ctx, launch_gemm(EPI_SWIGLU, b, s));
    b = GemmBatch{};
    if (!dual || txt_vid_only) {
        b.nprob = 1;
        b.p[0] = problem(u, mlp, vb->mlp_out_w, mlp, dual ? Lv : Mm, DIM, mlp, d_x, DIM);
        b.p[0].gate0 = V(0, 5);
        b.p[0].gate1 = V(1, 5);
        b.p[0].split = Lv;
    } else {
        b.nprob = 2;
        b.p[0] = problem(u, mlp, vb->mlp_out_w, mlp, Lv, DIM, mlp, d_x, DIM);
        b.p[0].gate0 = V(0, 5);
        b.p[1] = problem(u + (size_t)Lv * mlp, mlp, tb->mlp_out_w, mlp, TXT, DIM, mlp, d_x + (size_t)Lv * DIM, DIM);
        b.p[1].gate0 = V(1, 5);
    }
    HIPCK(ctx, launch_gemm(EPI_RESID, b, s));
    HIPCK(ctx, mark());
    return AWA_OK;
}

int dit_forward_grid(awa_ctx* ctx, const dit_io* io, const dit_time_weights* tw, const dit_branch* const* vb,
                     const dit_branch* const* tb, int n_layers, const awa_geom* g_even, const awa_geom* g_odd,
                     int mlp, int last_txt_vid_only, float eps, float t, const float* d_grid, int T, int H,
                     int W, const float* d_txt, int TXT, float* d_x, float* d_out, awa_stream_t stream) {
    if (!ctx || !io || !tw || !vb || !tb || n_layers < 0 || !g_even || (n_layers > 1 && !g_odd)) {
        set_err(ctx, "dit_forward_grid: null argument or n_layers=%d < 0", n_layers);
        return AWA_EARG;
    }
    if (H % 2 || W % 2 || H < 2 || W < 2 || T < 1) {
        set_err(ctx, "dit_forward_grid: T=%d H=%d W=%d (H and W even)", T, H, W);
        return AWA_EARG;
    }
    const int Lv = T * (H / 2) * (W / 2);
    for (const awa_geom* g : {g_even, g_odd}) {
        if (g && (g->plan.Lv != Lv || g->plan.txt_len != TXT)) {
            set_err(ctx, "dit_forward_grid: geometry (Lv=%d TXT=%d) does not match the grid (Lv=%d TXT=%d)",
                    g->plan.Lv, g->plan.txt_len, Lv, TXT);
            return AWA_EARG;
        }
    }
    {
        DeviceGuard dg(ctx->device);
        if (!ctx->emb) HIPCK(ctx, hipMalloc(reinterpret_cast<void**>(&ctx->emb), DIT_EMB * sizeof(float)));
    }
    int rc = dit_embed(ctx, io, d_grid, T, H, W, d_txt, TXT, d_x, stream);
    if (rc == AWA_OK)
        rc = dit_time_embedding(ctx, t, tw->w_in, tw->b_in, tw->w_hid, tw->b_hid, tw->w_out, tw->b_out, ctx->emb,
                                stream);
    for (int i = 0; i < n_layers && rc == AWA_OK; i++)
        rc = dit_layer_forward(ctx, (i % 2 == 0) ? g_even : g_odd, vb[i], tb[i], ctx->emb, mlp,
                               (i == n_layers - 1) ? last_txt_vid_only : 0, eps, d_x, Lv, TXT, stream);
    if (rc == AWA_OK) rc = dit_final(ctx, io, ctx->emb, d_x, T, H, W, eps, d_out, stream);
    return rc;
}

int dit_timing_read(awa_ctx* ctx, double* ms_gemm, double* ms_awa, double* ms_eltwise, int* layers) {
    if (!ctx) return AWA_EARG;
    DeviceGuard dg(ctx->device);
    // per layer: e0 norm e1 qkv e2 awa e3 out e4 norm e5 mlp e6
    double gemm = 0, awa_ms = 0, elt = 0;
    const size_t n = ctx->dit_ev_used.size() / 7;
    int rc = AWA_OK;
    for (size_t i = 0; i < n && rc == AWA_OK; i++) {
        hipEvent_t* e = &ctx->dit_ev_used[7 * i];
        float d[6] = {0, 0, 0, 0, 0, 0};
        hipError_t r = hipEventSynchronize(e[6]);
        for (int k = 0; k < 6 && r == hipSuccess; k++) r = hipEventElapsedTime(&d[k], e[k], e[k + 1]);
        if (r != hipSuccess) {
            set_err(ctx, "dit_timing_read: %s", hipGetErrorString(r));
            rc = AWA_EHIP;
        }
        elt += d[0] + d[4];
        gemm += d[1] + d[3] + d[5];
        awa_ms += d[2];
    }
    ctx->ev_free.insert(ctx->ev_free.end(), ctx->dit_ev_used.begin(), ctx->dit_ev_used.end());
    ctx->dit_ev_used.clear();
    if (ms_gemm) *ms_gemm = gemm;
    if (ms_awa) *ms_awa = awa_ms;
    if (ms_eltwise) *ms_eltwise = elt;
    if (layers) *layers = (int)n;
    return rc;
}

}  // extern "C"

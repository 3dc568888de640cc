/*
 * dit_capi.h — C ABI of the DiT block around the AWA op on MI355X (gfx950).
 *
 * Replaces the per-layer body of DitVk::forward_latent (src/dit_vk.cpp:517-632)
 * with DitVk::awa_forward (dit_vk.cpp:312-463) and swiglu (dit_vk.cpp:465-472),
 * the AdaCompose layer (src/ada_compose.cpp:165-235) and time_embedding
 * (dit_vk.cpp:295-309), in the order of the merged graph
 * (export/export_dit_graph.py:155-226):
 *
 *   h   = RMSNorm(x) * (emb[6d+1] + attn_scale) + (emb[6d] + attn_shift)
 *   qkv = h W_qkv^T                                   (no bias)
 *   a   = AWA(qkv_vid, qkv_txt)                       (awa_capi.h)
 *   x  += (a W_out^T + b_out) * (emb[6d+2] + attn_gate)
 *   h   = RMSNorm(x) * (emb[6d+4] + mlp_scale) + (emb[6d+3] + mlp_shift)
 *   x  += ((silu(h W_gate^T) * (h W_in^T)) W_mlp_out^T) * (emb[6d+5] + mlp_gate)
 *
 * for the video rows with the video branch and the text rows with the text
 * branch (the two branches are the same weights from layer 10 on).  With
 * txt_vid_only set (forward_latent's last layer, dit_vk.cpp:523-620) the text
 * rows get no ada modulation before attention, no attention gate and no MLP.
 *
 * Precision: weights and GEMM inputs bf16, fp32 accumulation on the matrix
 * cores, fp32 residual stream x, bf16 AWA boundary as AwaLayer's.
 *
 * Conventions as awa_capi.h: device pointers, stream-ordered, 0 / AWA_EARG /
 * AWA_EHIP, messages through awa_last_error of the context.
 */
#ifndef SEEDVR2_DIT_CAPI_H
#define SEEDVR2_DIT_CAPI_H

#include <stdint.h>

#include "awa_capi.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { DIT_MLP = 6912, DIT_EMB = 15360 };

/* Size limits of the block's GEMM kernel: its operand and output rows are
 * addressed through buffer resources with 32-bit byte ranges over a tile's
 * rows, so N and K stay at or under 2^20 and the MLP width (N of the fused
 * SwiGLU GEMM is twice it) at or under 2^19; larger values are rejected
 * (AWA_EARG).  The model's widths are 2560, 7680 and 6912. */
enum { DIT_GEMM_NK_MAX = 1 << 20, DIT_MLP_MAX = 1 << 19 };

/* One branch's weights on the device (names as the reference's per-branch
 * files, dit_vk.cpp:163-177 and verify_dit.cpp:163-179). */
typedef struct {
    const uint16_t* qkv_w;      /* bf16 [7680][2560]                              */
    const uint16_t* out_w;      /* bf16 [2560][2560]                              */
    const float* out_b;         /* fp32 [2560]                                    */
    const uint16_t* mlp_w;      /* bf16 [2*mlp][2560], from dit_pack_mlp_weights  */
    const uint16_t* mlp_out_w;  /* bf16 [2560][mlp]                               */
    const float* nq;            /* fp32 [128] qk-norm gains                       */
    const float* nk;
    const float* attn_shift;    /* fp32 [2560] each                               */
    const float* attn_scale;
    const float* attn_gate;
    const float* mlp_shift;
    const float* mlp_scale;
    const float* mlp_gate;
} dit_branch;

/* Interleaves proj_in (w_in) and proj_in_gate (w_gate), each bf16 [mlp][2560],
 * into the fused SwiGLU weight [2*mlp][2560]: 32-row blocks alternate
 * in, gate, in, gate, ... (mlp a multiple of 128). */
int dit_pack_mlp_weights(awa_ctx* ctx, const uint16_t* d_w_in, const uint16_t* d_w_gate,
                         int mlp, uint16_t* d_w_cat, awa_stream_t stream);

/* time_embedding(t) (dit_vk.cpp:295-309): 256-wide sinusoid (sin half, then
 * cos), then Linear 256->2560, SiLU, Linear 2560->2560, SiLU,
 * Linear 2560->15360, fp32 weights [out][in] and biases; d_emb fp32 [15360]. */
int dit_time_embedding(awa_ctx* ctx, float t, const float* d_w_in, const float* d_b_in,
                       const float* d_w_hid, const float* d_b_hid, const float* d_w_out,
                       const float* d_b_out, float* d_emb, awa_stream_t stream);

/* One DiT layer in place on the residual stream d_x, fp32 [Lv + TXT][2560]
 * (video rows first, then the text rows).  g is the layer's window geometry
 * (unshifted on even layers, shifted on odd ones, dit_vk.cpp:518).  vb / tb
 * are the video and text branches (the same pointer for shared layers).
 * d_emb is the timestep embedding [15360].  mlp is the SwiGLU width (6912 in
 * the reference checkpoint).  Scratch comes from the context: its workspace
 * grows (hipMalloc) on the first call with a larger shape, so a caller that
 * captures this call into a graph calls dit_reserve at that shape first (or
 * runs it once eagerly, as dit_graph_create does). */
int dit_layer_forward(awa_ctx* ctx, const awa_geom* g, const dit_branch* vb,
                      const dit_branch* tb, const float* d_emb, int mlp, int txt_vid_only,
                      float eps, float* d_x, int Lv, int TXT, awa_stream_t stream);

/* Sizes the context's workspace and the AWA scratch for dit_layer_forward,
 * dit_embed and dit_final on geometry g (Lv video rows, TXT text rows) and
 * MLP width mlp, so that those calls at that shape allocate nothing: a caller
 * may then capture them into a graph without an eager run first.  No
 * counterpart in the reference (DitVk::init sizes its buffers per resolution,
 * dit_vk.cpp:140-203). */
int dit_reserve(awa_ctx* ctx, const awa_geom* g, int mlp);

/* Per-phase device timing of dit_layer_forward (HIP events on its stream):
 * GEMMs, AWA op, and norms/elementwise, summed since the last read. */
int dit_timing_read(awa_ctx* ctx, double* ms_gemm, double* ms_awa, double* ms_eltwise,
                    int* layers);

/* The DiT's input and output layers (DitVk::forward_grid, dit_vk.cpp:752-763,
 * with forward_latent's vid_in_proj / txt_in, dit_vk.cpp:494-497, and its final
 * norm, ada and vid_out_proj, dit_vk.cpp:657-675).  Linear weights [out][in]
 * as the reference's InnerProduct layers (verify_dit.cpp:354-356: all three
 * with bias), bf16 on the device; vectors fp32. */
typedef struct {
    const uint16_t* vid_in_w;     /* bf16 [2560][132], input in (ph, pw, c) patch order */
    const float* vid_in_b;        /* fp32 [2560]                                        */
    const uint16_t* txt_in_w;     /* bf16 [2560][5120]                                  */
    const float* txt_in_b;        /* fp32 [2560]                                        */
    const float* out_norm_w;      /* fp32 [2560] vid_out_norm_w (RMSNorm weight)        */
    const float* out_ada_shift;   /* fp32 [2560] vid_out_ada_shift                      */
    const float* out_ada_scale;   /* fp32 [2560] vid_out_ada_scale                      */
    const uint16_t* vid_out_w;    /* bf16 [64][2560] vid_out_proj                       */
    const float* vid_out_b;       /* fp32 [64]                                          */
} dit_io_weights;

/* Prepared input/output layers: padded device copies of vid_in_w (K 132 ->
 * 192) and vid_out_w / vid_out_b (N 64 -> 256) for the block's GEMM kernel;
 * the other pointers are borrowed and must stay valid. */
typedef struct dit_io dit_io;
int dit_io_create(awa_ctx* ctx, const dit_io_weights* w, dit_io** out, awa_stream_t stream);
void dit_io_destroy(awa_ctx* ctx, dit_io* io);

/* Input layers: patchify the latent grid d_grid fp32 (T, H, W, 33) (H, W even;
 * dit_vk.cpp:717-733), vid_in_proj to the video rows and txt_in of d_txt fp32
 * [TXT][5120] to the text rows of the residual stream d_x fp32
 * [Lv + TXT][2560], Lv = T (H/2) (W/2).  bf16 GEMM inputs, fp32 out. */
int dit_embed(awa_ctx* ctx, const dit_io* io, const float* d_grid, int T, int H, int W,
              const float* d_txt, int TXT, float* d_x, awa_stream_t stream);

/* Output layer: RMSNorm of the video rows of d_x with out_norm_w, times
 * (emb[6d+1] + out_ada_scale) plus (emb[6d] + out_ada_shift), vid_out_proj,
 * unpatchified to d_out fp32 (T, H, W, 16) (dit_vk.cpp:735-750). */
int dit_final(awa_ctx* ctx, const dit_io* io, const float* d_emb, const float* d_x, int T, int H,
              int W, float eps, float* d_out, awa_stream_t stream);

/* Timestep MLP weights of dit_time_embedding (fp32, [out][in]). */
typedef struct {
    const float* w_in;   /* [2560][256]   */
    const float* b_in;   /* [2560]        */
    const float* w_hid;  /* [2560][2560]  */
    const float* b_hid;  /* [2560]        */
    const float* w_out;  /* [15360][2560] */
    const float* b_out;  /* [15360]       */
} dit_time_weights;

/* The whole DiT, DitVk::forward_grid (dit_vk.cpp:752-763) with
 * forward_latent(0, n_layers, init, final) (dit_vk.cpp:486-691): dit_embed,
 * the timestep embedding at t, n_layers x dit_layer_forward (layer i with
 * branches vb[i] / tb[i], geometry g_even on even i and g_odd on odd i,
 * dit_vk.cpp:518; the last layer with txt_vid_only = last_txt_vid_only),
 * then dit_final into d_out fp32 (T, H, W, 16).  The geometries are built
 * on the latent grid (T, H/2, W/2) with TXT text rows.  d_x is the caller's
 * residual stream, fp32 [Lv + TXT][2560]; the embedding lives in the context. */
int dit_forward_grid(awa_ctx* ctx, const dit_io* io, const dit_time_weights* tw,
                     const dit_branch* const* vb, const dit_branch* const* tb, int n_layers,
                     const awa_geom* g_even, const awa_geom* g_odd, int mlp, int last_txt_vid_only,
                     float eps, float t, const float* d_grid, int T, int H, int W, const float* d_txt,
                     int TXT, float* d_x, float* d_out, awa_stream_t stream);

/* Plain bf16 GEMM with the block's kernel, for tests and measurement:
 * C[M][N] = A[M][K] W[N][K]^T, bf16 in, bf16 out (fp32 accumulation).
 * N a multiple of 256, K a multiple of 64, both at most DIT_GEMM_NK_MAX. */
int dit_gemm_bf16(awa_ctx* ctx, const uint16_t* d_A, const uint16_t* d_W, uint16_t* d_C, int M,
                  int N, int K, awa_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif

/*
 * oracle.h — CPU restatement of the SeedVR2 AWA path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the oracle the HIP implementation is tested against.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (seedvr2-2b-ncnn_amd/) never links or calls it.
 *
 * Every function restates a reference routine with the same float operation
 * order, so that a build with the reference's flags (-O2, no FMA contraction,
 * x86-64 baseline ISA) reproduces the reference bit for bit.  Citations are
 * relative to the reference repository root.
 *
 * Pinning status of each function (how it is checked) is listed in the header
 * of oracle.c.
 */
#ifndef SEEDVR2_ORACLE_H
#define SEEDVR2_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_HEADS = 20, ORC_HEAD_D = 128, ORC_DIM = 2560, ORC_QKV = 7680,
       ORC_ROPE_ROT = 126, ORC_MLP = 6912, ORC_EMB = 15360 };

/* ---- window geometry: src/awa_window.cpp:15-150 ---- */
/* Writes at most cap windows as [st,en,sh,eh,sw,ew] into slices; returns nwin
 * (which may exceed cap; then only cap are written). */
int orc_make_windows(int t, int h, int w, const int num_windows[3], int shifted,
                     int32_t* slices, int cap);
/* vid_freq [sumf*126], txt_freq [nwin*txt_len*126]; returns sumf. */
int orc_build_freqs(const int32_t* slices, int nwin, int txt_len,
                    float* vid_freq, float* txt_freq);
/* cumf [nwin+1], vidx [sumf] — awa_vk.cpp:73-88 (carried as int here). */
int orc_build_index(const int32_t* slices, int nwin, int H, int W,
                    int32_t* cumf, int32_t* vidx);

/* ---- per-token ops: dit_vk.cpp:48-71 ---- */
void orc_rmsnorm(const float* x, int n, const float* w, float eps, float* out);
void orc_qk_norm(const float* x, const float* w, float eps, float* out);
void orc_apply_rope(const float* freq, const float* q, float* out);

/* ---- the AWA op: dit_vk.cpp:345-462 (CPU branch of DitVk::awa_forward) ----
 * vqkv [Lv*7680], tqkv [TXT*7680] -> vattn [Lv*2560], tattn [TXT*2560].
 * nthreads > 1 splits the (window, head) loop over OpenMP threads; the
 * arithmetic of each (window, head) is unchanged, so results are identical. */
void orc_awa_forward(const float* vqkv, const float* tqkv, int Lv, int TXT,
                     int T, int H, int W, const int32_t* slices, int nwin,
                     const float* vid_freq, const float* txt_freq,
                     const float* nq_v, const float* nk_v,
                     const float* nq_t, const float* nk_t, float eps,
                     float* vattn, float* tattn, int nthreads);

/* ---- bf16 boundary: shaders/cast_f32_bf16.comp:23-24, cast_bf16_f32.comp:18-19 */
void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n);
void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n);

/* ---- block surroundings: dit_vk.cpp:270-309, 465-472, 486-675 ---- */
/* y[Ln*out] = x[Ln*in] W^T + b, fp32 sequential accumulation (LinearRaw::run,
 * verify_dit.cpp:59-72).  b may be NULL. */
void orc_linear(const float* x, const float* W, const float* b, int Ln,
                int in, int out, float* y, int nthreads);
void orc_sinusoidal(float t, int dim, float* e);
void orc_silu(float* x, int64_t n);

typedef struct {
    const float *qkv_w;              /* [7680][2560] */
    const float *out_w, *out_b;      /* [2560][2560], [2560] */
    const float *mlp_in_w, *mlp_g_w; /* [6912][2560] (mlp width given by mlp) */
    const float *mlp_out_w;          /* [2560][mlp] */
    const float *nq, *nk;            /* [128] */
    const float *attn_shift, *attn_scale, *attn_gate;   /* [2560] */
    const float *mlp_shift, *mlp_scale, *mlp_gate;      /* [2560] */
} orc_branch;

/* One DiT layer, forward_latent order (dit_vk.cpp:517-632), in place on
 * vid [Lv*2560] and txt [TXT*2560].  txt_vid_only != 0 applies the last-layer
 * vid_only semantics of dit_vk.cpp:523-620 (no txt ada/gate/MLP). */
void orc_dit_layer(float* vid, float* txt, int Lv, int TXT, const float* emb,
                   const orc_branch* vb, const orc_branch* tb, int mlp,
                   int T, int H, int W, const int32_t* slices, int nwin,
                   const float* vid_freq, const float* txt_freq, float eps,
                   int txt_vid_only, int nthreads);

/* Timestep embedding (dit_vk.cpp:295-309): emb [15360]. */
void orc_time_embedding(float t, const float* w_in, const float* b_in,
                        const float* w_hid, const float* b_hid,
                        const float* w_out, const float* b_out, float* emb);

#ifdef __cplusplus
}
#endif
#endif

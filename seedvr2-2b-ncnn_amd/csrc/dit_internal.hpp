// dit_internal.hpp — shared definitions of the DiT block kernels.
#pragma once

#include "awa_internal.hpp"
#include "dit_capi.h"

namespace awa {

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

struct GemmProblem {
    const uint16_t* A;     // [M][K] bf16, row stride lda (elements)
    const uint16_t* W;     // [N][K] bf16, row stride ldw
    int M, N, K, lda, ldw;
    void* C;               // EPI_STORE / EPI_SWIGLU: bf16; EPI_RESID: fp32 residual (in/out)
    int ldc;
    const float* bias;     // [N] or null (EPI_RESID)
    const float* gate0;    // [N] gate of rows < split, null = 1 (EPI_RESID)
    const float* gate1;    // [N] gate of rows >= split, null = 1
    int split;
    int n_tiles, m_tiles;  // filled by launch_gemm
};

struct GemmBatch {
    GemmProblem p[2];      // one or two independent problems in one launch
    int nprob;
    int tiles0, total_tiles;
};

hipError_t launch_gemm(int epi, GemmBatch& b, hipStream_t s);

// h[m] = bf16(RMSNorm(x[m]) * scale + shift); rows >= split use the second
// pair (null scale: plain RMSNorm, the last layer's text rows).
struct NormArgs {
    const float* x;
    uint16_t* h;
    int M, split;
    const float* scale0;
    const float* shift0;
    const float* scale1;
    const float* shift1;
    float eps;
};
hipError_t launch_norm_ada(const NormArgs& a, hipStream_t s);

// out[f][k][d] = emb[6d + K_MAP[k]] + branch_f[k][d] for the 6 vectors
// (a_sc, a_sh, a_g, m_sc, m_sh, m_g) of the two flows.
struct AdaArgs {
    const float* emb;
    const float* vec[2][6];  // branch vectors per flow, order as above
    float* out;              // [2][6][2560]
};
hipError_t launch_ada(const AdaArgs& a, hipStream_t s);

hipError_t launch_pack_mlp(const uint16_t* w_in, const uint16_t* w_gate, int mlp, uint16_t* w_cat,
                           hipStream_t s);

// y[out] = act(W[out][in] x[in] + b[out]) in fp32; act: 0 none, 1 SiLU.
hipError_t launch_gemv_f32(const float* W, const float* b, const float* x, float* y, int in, int out,
                           int silu, hipStream_t s);
hipError_t launch_sinusoid(float t, float* e, int dim, hipStream_t s);

// grid (T, H, W, 33) fp32 -> [T (H/2) (W/2)][kpad] bf16 patches, (ph, pw, c) order
hipError_t launch_patchify(const float* grid, int T, int H, int W, uint16_t* out, int kpad, hipStream_t s);
// [T (H/2) (W/2)][ldy] fp32 (first 64 columns) -> (T, H, W, 16) fp32
hipError_t launch_unpatchify(const float* y, int ldy, int T, int H, int W, float* out, hipStream_t s);
// output-layer modulation vectors: scale = w (emb[6d+1] + ada_scale), shift = emb[6d] + ada_shift
hipError_t launch_final_ada(const float* emb, const float* w, const float* ada_scale, const float* ada_shift,
                            float* scale, float* shift, hipStream_t s);

}  // namespace awa

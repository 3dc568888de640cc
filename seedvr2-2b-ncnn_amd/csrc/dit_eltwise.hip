// dit_eltwise.hip — row-wise and small kernels of the DiT block.
//
//   norm_ada   RMSNorm (no affine, dit_vk.cpp:48-52) then the ada modulation
//              x * scale + shift (dit_vk.cpp:532-545, 584-597), bf16 out:
//              the A operand of the next projection.  One wave64 per row,
//              HBM-bound (reads 10 KiB fp32, writes 5 KiB bf16 per row).
//   ada        AdaCompose (ada_compose.cpp:165-235): emb[6d + K_MAP[k]] +
//              branch vector, the 12 modulation vectors of a layer.
//   pack_mlp   interleave proj_in / proj_in_gate rows for the fused SwiGLU.
//   gemv_f32   the timestep MLP (M = 1 linears, dit_vk.cpp:303-309).
//   patchify / unpatchify   the DiT's input and output layouts
//              (dit_vk.cpp:717-750); final_ada   the modulation vectors of
//              the output layer (dit_vk.cpp:657-669).
#include <cmath>

#include "dit_internal.hpp"

namespace awa {

namespace {

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

constexpr int PER_LANE4 = DIM / 4 / 64;  // float4s per lane per 2560-wide row

__global__ __launch_bounds__(256) void norm_ada_kernel(NormArgs a) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= a.M) return;
    const float4* x = reinterpret_cast<const float4*>(a.x + (size_t)row * DIM);
    float4 v[PER_LANE4];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER_LANE4; i++) v[i] = x[i * 64 + lane];
    // the modulation vectors (cached, the same for every row) are loaded
    // while the row is in flight, not after the reduction
    const bool second = row >= a.split;
    const float* sc = second ? a.scale1 : a.scale0;
    const float* sh = second ? a.shift1 : a.shift0;
    float4 s[PER_LANE4], t[PER_LANE4];
    if (sc) {
#pragma unroll
        for (int i = 0; i < PER_LANE4; i++) {
            s[i] = reinterpret_cast<const float4*>(sc)[i * 64 + lane];
            t[i] = reinterpret_cast<const float4*>(sh)[i * 64 + lane];
        }
    }
#pragma unroll
    for (int i = 0; i < PER_LANE4; i++)
        ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)DIM + a.eps);
    uint2* out = reinterpret_cast<uint2*>(a.h + (size_t)row * DIM);
#pragma unroll
    for (int i = 0; i < PER_LANE4; i++) {
        float o0 = v[i].x * r, o1 = v[i].y * r, o2 = v[i].z * r, o3 = v[i].w * r;
        if (sc) {
            o0 = o0 * s[i].x + t[i].x;
            o1 = o1 * s[i].y + t[i].y;
            o2 = o2 * s[i].z + t[i].z;
            o3 = o3 * s[i].w + t[i].w;
        }
        out[i * 64 + lane] = make_uint2(bf16x2_rne(o0, o1), bf16x2_rne(o2, o3));
    }
}

// K_MAP of ada_compose.cpp:16: a_sc->1, a_sh->0, a_g->2, m_sc->4, m_sh->3, m_g->5
__constant__ int kAdaSlot[6] = {1, 0, 2, 4, 3, 5};

__global__ __launch_bounds__(256) void ada_kernel(AdaArgs a) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= 12 * DIM) return;
    const int d = i % DIM, k = (i / DIM) % 6, f = i / (6 * DIM);
    a.out[i] = a.emb[d * 6 + kAdaSlot[k]] + a.vec[f][k][d];
}

__global__ __launch_bounds__(256) void pack_mlp_kernel(const uint16_t* __restrict__ w_in,
                                                       const uint16_t* __restrict__ w_gate,
                                                       uint16_t* __restrict__ w_cat) {
    const int r = blockIdx.x;          // row of the fused weight
    const int blk = r >> 5, within = r & 31;
    const uint16_t* src = ((blk & 1) ? w_gate : w_in) + (size_t)((blk >> 1) * 32 + within) * DIM;
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    uint4* d4 = reinterpret_cast<uint4*>(w_cat + (size_t)r * DIM);
    for (int c = threadIdx.x; c < DIM / 8; c += 256) d4[c] = s4[c];
}

__global__ __launch_bounds__(256) void gemv_f32_kernel(const float* __restrict__ W,
                                                       const float* __restrict__ b,
                                                       const float* __restrict__ x,
                                                       float* __restrict__ y, int in, int out,
                                                       int silu) {
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (o >= out) return;
    const float* w = W + (size_t)o * in;
    float acc = 0.f;
    for (int i = lane; i < in; i += 64) acc += w[i] * x[i];
    acc = wave_sum(acc);
    if (lane == 0) {
        float v = acc + (b ? b[o] : 0.f);
        if (silu) v = v / (1.f + expf(-v));
        y[o] = v;
    }
}

// One row (t, hh, ww) of the patchified grid per workgroup: the 2x2 patch's
// 33-channel pixels in (ph, pw, c) order (dit_vk.cpp:717-733), bf16, zeros
// from column 132 up to kpad (the projection's K padding).
__global__ __launch_bounds__(128) void patchify_kernel(const float* __restrict__ grid, int H, int W,
                                                       uint16_t* __restrict__ out, int kpad) {
    const int row = blockIdx.x;
    const int H2 = H >> 1, W2 = W >> 1;
    const int t = row / (H2 * W2), hh = (row / W2) % H2, ww = row % W2;
    for (int j = threadIdx.x; j < kpad; j += 128) {
        float v = 0.f;
        if (j < 132) {
            const int ph = j / 66, pw = (j / 33) & 1, c = j % 33;
            v = grid[(((size_t)t * H + 2 * hh + ph) * W + 2 * ww + pw) * 33 + c];
        }
        out[(size_t)row * kpad + j] = (uint16_t)bf16_rne(v);
    }
}

// The output layer's 64 values of row (t, hh, ww) back to the 2x2 patch's
// 16-channel pixels, (ph, pw, c) order (dit_vk.cpp:735-750).
__global__ __launch_bounds__(64) void unpatchify_kernel(const float* __restrict__ y, int ldy, int H,
                                                        int W, float* __restrict__ out) {
    const int row = blockIdx.x;
    const int H2 = H >> 1, W2 = W >> 1;
    const int t = row / (H2 * W2), hh = (row / W2) % H2, ww = row % W2;
    const int j = threadIdx.x;  // 64 values
    const int ph = j >> 5, pw = (j >> 4) & 1, c = j & 15;
    out[(((size_t)t * H + 2 * hh + ph) * W + 2 * ww + pw) * 16 + c] = y[(size_t)row * ldy + j];
}

// Output layer modulation (dit_vk.cpp:657-669): RMSNorm(x) * w * (emb[6d+1] +
// ada_scale) + (emb[6d] + ada_shift), as the scale w * (emb[6d+1] + ada_scale)
// and the shift of norm_ada.
__global__ __launch_bounds__(256) void final_ada_kernel(const float* __restrict__ emb,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ ada_scale,
                                                        const float* __restrict__ ada_shift,
                                                        float* __restrict__ scale, float* __restrict__ shift) {
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= DIM) return;
    scale[d] = w[d] * (emb[6 * d + 1] + ada_scale[d]);
    shift[d] = emb[6 * d] + ada_shift[d];
}

struct Sinusoid {
    float v[256];
};

__global__ void sinusoid_kernel(Sinusoid s, float* e, int dim) {
    const int j = threadIdx.x;
    if (j < dim) e[j] = s.v[j];
}

}  // namespace

hipError_t launch_norm_ada(const NormArgs& a, hipStream_t s) {
    if (a.M <= 0) return hipSuccess;
    hipLaunchKernelGGL(norm_ada_kernel, dim3((a.M + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_ada(const AdaArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(ada_kernel, dim3((12 * DIM + 255) / 256), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_pack_mlp(const uint16_t* w_in, const uint16_t* w_gate, int mlp, uint16_t* w_cat,
                           hipStream_t s) {
    hipLaunchKernelGGL(pack_mlp_kernel, dim3(2 * mlp), dim3(256), 0, s, w_in, w_gate, w_cat);
    return hipGetLastError();
}

hipError_t launch_gemv_f32(const float* W, const float* b, const float* x, float* y, int in, int out,
                           int silu, hipStream_t s) {
    hipLaunchKernelGGL(gemv_f32_kernel, dim3((out + 3) / 4), dim3(256), 0, s, W, b, x, y, in, out, silu);
    return hipGetLastError();
}

hipError_t launch_patchify(const float* grid, int T, int H, int W, uint16_t* out, int kpad, hipStream_t s) {
    const int rows = T * (H / 2) * (W / 2);
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(patchify_kernel, dim3(rows), dim3(128), 0, s, grid, H, W, out, kpad);
    return hipGetLastError();
}

hipError_t launch_unpatchify(const float* y, int ldy, int T, int H, int W, float* out, hipStream_t s) {
    const int rows = T * (H / 2) * (W / 2);
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(unpatchify_kernel, dim3(rows), dim3(64), 0, s, y, ldy, H, W, out);
    return hipGetLastError();
}

hipError_t launch_final_ada(const float* emb, const float* w, const float* ada_scale, const float* ada_shift,
                            float* scale, float* shift, hipStream_t s) {
    hipLaunchKernelGGL(final_ada_kernel, dim3((DIM + 255) / 256), dim3(256), 0, s, emb, w, ada_scale,
                       ada_shift, scale, shift);
    return hipGetLastError();
}

hipError_t launch_sinusoid(float t, float* e, int dim, hipStream_t s) {
    // The 256 sinusoid values are formed on the host with the reference's
    // expression (dit_vk.cpp:295-302) and passed by value.
    Sinusoid v{};
    const int half = dim / 2;
    for (int j = 0; j < dim && j < 256; j++) {
        // float argument, double exp, rounded to float: as C's exp()
        const float freq = (j < half) ? (float)::exp((double)(-logf(10000.f) * j / half))
                                      : (float)::exp((double)(-logf(10000.f) * (j - half) / half));
        v.v[j] = (j < half) ? sinf(t * freq) : cosf(t * freq);
    }
    hipLaunchKernelGGL(sinusoid_kernel, dim3(1), dim3(256), 0, s, v, e, dim);
    return hipGetLastError();
}

}  // namespace awa

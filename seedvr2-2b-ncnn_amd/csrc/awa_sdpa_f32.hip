// awa_sdpa_f32.hip — varlen window attention with fp32 storage on CDNA4 matrix
// cores (v_mfma_f32_32x32x2f32).
//
// The fp32 counterpart of sdpa_bf16_kernel (awa_sdpa.hip), for AWA_F32
// storage: the reference's fp32 attention (dit_vk.cpp:406-439) at fp32
// MFMA precision.  One workgroup (4 wave64) per (work item, head): a work
// item is one window and up to two of its 64-row query tiles, each wave owns
// 32 queries; the window's K and V^T tiles stream through LDS (double
// buffered).  Scores are formed transposed, S^T = K Q^T, so that a lane owns
// one query column and the online softmax needs one cross-lane exchange;
// the probabilities leave the accumulator in the B-operand layout of
// O^T = V^T P^T.  Video query rows are scattered back to token order
// (dit_vk.cpp:445-455); text query rows go to per-window fp32 partials that
// the coalesce kernel averages in window order (dit_vk.cpp:440-444).
#include "awa_internal.hpp"

namespace awa {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The key/query tile sequence of one window: its video tiles, then the text
// tiles of its text set.
struct WinTiles {
    int vbase, nvt, tbase, ntt, f, txt;
    __device__ int tile(int kk) const { return kk < nvt ? vbase + kk : tbase + (kk - nvt); }
    __device__ int nvalid(int kk) const {
        return kk < nvt ? min(TILE, f - TILE * kk) : min(TILE, txt - TILE * (kk - nvt));
    }
};

__device__ inline WinTiles window_tiles(const SdpaArgs& a, int w) {
    WinTiles t;
    t.vbase = a.tile_base[w];
    t.nvt = a.tile_base[w + 1] - t.vbase;
    t.ntt = a.ntt;
    t.tbase = a.n_vid_tiles + (a.txt_sets == 1 ? 0 : w) * a.ntt;
    t.f = a.cumf[w + 1] - a.cumf[w];
    t.txt = a.txt_len;
    return t;
}

// Hardware dispatches workgroup b to XCD b % 8.  Remap so that each XCD gets
// a contiguous range of (head, item) ids: consecutive items of one head are
// mostly the same window and share its K/V tiles through that XCD's L2.

// Online-softmax update of one 64-key tile held as two 32x32 S^T accumulators
// (lane: query column n = lane % 32; register r: key 8(r/4) + 4(lane/32) + r%4
// of each 32-key half).  Scales and masks the scores, returns the factor that
// rescales the running output, and leaves exp2(s - m) in sacc.
__device__ inline float softmax_tile(f32x16 (&sacc)[2], int kvalid, int hb, float scale,
                                     float& m_i, float& l_i) {
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = 32 * kt + 8 * (r >> 2) + 4 * hb + (r & 3);
            const float v = key < kvalid ? sacc[kt][r] * scale : -INFINITY;
            sacc[kt][r] = v;
            mloc = fmaxf(mloc, v);
        }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_i, mloc);  // finite: every tile has a valid key
    const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
    float psum = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float p = __builtin_amdgcn_exp2f(sacc[kt][r] - m_new);
            sacc[kt][r] = p;
            psum += p;
        }
    l_i = l_i * alpha + psum;
    m_i = m_new;
    return alpha;
}

// Writes the normalised O^T accumulators of one wave (lane: query n, register
// r of d-tile dt: channel 32dt + 8(r/4) + 4(lane/32) + r%4).
__device__ inline void store_rows(const f32x16 (&oacc)[4], float inv, int hb, float* dst_row) {
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 32 * dt + 8 * g + 4 * hb;
            *reinterpret_cast<float4*>(dst_row + d0) =
                make_float4(oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv, oacc[dt][4 * g + 2] * inv,
                            oacc[dt][4 * g + 3] * inv);
        }
}

// Destination of query slot `slot` of query tile kq (nullptr: padding slot).
__device__ inline void* query_dst(const SdpaArgs& a, const WinTiles& wt, int w, int h, int kq,
                                  int slot, bool& to_text, size_t elem) {
    if (slot >= wt.nvalid(kq)) return nullptr;
    if (kq < wt.nvt) {
        to_text = false;
        const int g = a.cumf[w] + TILE * kq + slot;
        const size_t tok = (size_t)a.vidx[g];
        return reinterpret_cast<char*>(a.vattn) + (tok * DIM + (size_t)h * HEAD_D) * elem;
    }
    to_text = true;
    const int i = TILE * (kq - wt.nvt) + slot;
    return a.tpart + ((size_t)w * a.txt_len + i) * DIM + (size_t)h * HEAD_D;
}

constexpr int KP32 = 132;                 // LDS pitch of a K row (floats)
constexpr int VP32 = 68;                  // LDS pitch of a V^T row (floats)
constexpr int KS32 = TILE * KP32;
constexpr int STAGE32 = KS32 + HEAD_D * VP32;

__global__ __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
void sdpa_f32_kernel(SdpaArgs a) {
    __shared__ __align__(16) float lds[2 * STAGE32];
    const int nblk = a.n_items * HEADS;
    const int lid = xcd_remap(nblk);
    if (lid >= nblk) return;
    const int h = lid / a.n_items;
    const int item = lid % a.n_items;

    const int4 it = reinterpret_cast<const int4*>(a.items)[item];
    const int w = it.x;
    const WinTiles wt = window_tiles(a, w);
    const int nk = wt.nvt + wt.ntt;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = lane & 31, hb = lane >> 5;
    const int kq = wave < 2 ? it.y : it.z;
    const bool active = kq >= 0;
    const int qslot = (wave & 1) * 32 + n;

    const size_t head_off = (size_t)h * a.n_tiles * TILE * HEAD_D;
    const float* Qh = reinterpret_cast<const float*>(a.Qp) + head_off;
    const float* Kh = reinterpret_cast<const float*>(a.Kp) + head_off;
    const float* Vh = reinterpret_cast<const float*>(a.Vp) + head_off;

    // k-step s of S^T pairs channel s (lanes 0-31) with channel 64 + s
    // (lanes 32-63): lane (n, hb) holds Q[slot][64hb + s].
    // Loaded on every path (an idle wave reads its partner's tile): a load
    // under a condition leaves the array to scratch memory.
    float qf[64];
    {
        const float* qrow = Qh + ((size_t)wt.tile(active ? kq : it.y) * TILE + qslot) * HEAD_D + 64 * hb;
#pragma unroll
        for (int s = 0; s < 64; s += 4) {
            const float4 v = *reinterpret_cast<const float4*>(qrow + s);
            qf[s] = v.x; qf[s + 1] = v.y; qf[s + 2] = v.z; qf[s + 3] = v.w;
        }
    }

    // K and V tiles go through the same 32 staging registers one after the
    // other: K of the next tile is loaded at the top of an iteration and
    // stored to the free LDS stage after the score MFMAs, V is loaded then
    // and stored at the end (two staging sets at once made the kernel spill).
    // (a plain vector type: an array of HIP's float4 stayed in scratch memory)
    f32x4 reg[8];
    auto load_k = [&](int kk) __attribute__((always_inline)) {
        const f32x4* src = reinterpret_cast<const f32x4*>(Kh + (size_t)wt.tile(kk) * TILE * HEAD_D);
#pragma unroll
        for (int i = 0; i < 8; i++) reg[i] = src[tid + 256 * i];
    };
    auto load_v = [&](int kk) __attribute__((always_inline)) {
        const f32x4* src = reinterpret_cast<const f32x4*>(Vh + (size_t)wt.tile(kk) * TILE * HEAD_D);
#pragma unroll
        for (int i = 0; i < 8; i++) reg[i] = src[tid + 256 * i];
    };
    auto store_k = [&](int stage) __attribute__((always_inline)) {
        float* ks = lds + stage * STAGE32;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<f32x4*>(ks + (c >> 5) * KP32 + (c & 31) * 4) = reg[i];
        }
    };
    auto store_v = [&](int stage) __attribute__((always_inline)) {
        float* vs = lds + stage * STAGE32 + KS32;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<f32x4*>(vs + (c >> 4) * VP32 + (c & 15) * 4) = reg[i];
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) oacc[dt][r] = 0.f;
    float m_i = -INFINITY, l_i = 0.f;

    load_k(0);
    store_k(0);
    load_v(0);
    store_v(0);
    __syncthreads();
    for (int kk = 0; kk < nk; kk++) {
        const int stage = kk & 1;
        if (kk + 1 < nk) load_k(kk + 1);
        if (active) {
            const float* ks = lds + stage * STAGE32;
            const float* vs = ks + KS32;
            f32x16 sacc[2];
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) sacc[kt][r] = 0.f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                const float* krow = ks + (32 * kt + n) * KP32 + 64 * hb;
#pragma unroll
                for (int s = 0; s < 64; s += 4) {
                    const float4 kv = *reinterpret_cast<const float4*>(krow + s);
                    sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[s], sacc[kt], 0, 0, 0);
                    sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[s + 1], sacc[kt], 0, 0, 0);
                    sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[s + 2], sacc[kt], 0, 0, 0);
                    sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[s + 3], sacc[kt], 0, 0, 0);
                }
            }
            if (kk + 1 < nk) {
                store_k(stage ^ 1);
                load_v(kk + 1);
            }
            const float alpha = softmax_tile(sacc, wt.nvalid(kk), hb, a.scale_log2e, m_i, l_i);
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) oacc[dt][r] *= alpha;
            // O^T += V^T P^T; k-step r pairs key 8(r/4)+r%4 (lanes 0-31) with
            // key 8(r/4)+4+r%4 (lanes 32-63) of the 32-key half kt, which is
            // exactly where the S^T accumulator left P.
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int dt = 0; dt < 4; dt++) {
                    const float* vrow = vs + (32 * dt + n) * VP32 + 32 * kt + 4 * hb;
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const float4 vv = *reinterpret_cast<const float4*>(vrow + 8 * g);
                        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, sacc[kt][4 * g], oacc[dt], 0, 0, 0);
                        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, sacc[kt][4 * g + 1], oacc[dt], 0, 0, 0);
                        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, sacc[kt][4 * g + 2], oacc[dt], 0, 0, 0);
                        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, sacc[kt][4 * g + 3], oacc[dt], 0, 0, 0);
                    }
                }
        }
        if (kk + 1 < nk) {
            if (!active) {  // idle waves still carry their share of the tiles
                store_k(stage ^ 1);
                load_v(kk + 1);
            }
            store_v(stage ^ 1);
        }
        __syncthreads();
    }
    if (!active) return;
    const float l = l_i + __shfl_xor(l_i, 32);
    const float inv = 1.f / l;
    bool to_text = false;
    void* dst = query_dst(a, wt, w, h, kq, qslot, to_text, 4);
    if (dst == nullptr) return;
    store_rows(oacc, inv, hb, reinterpret_cast<float*>(dst));
}

}  // namespace

hipError_t launch_sdpa_f32(const SdpaArgs& a, hipStream_t s) {
    const int nblk = a.n_items * HEADS;
    const int grid = ((nblk + 7) >> 3) << 3;
    hipLaunchKernelGGL(sdpa_f32_kernel, dim3(grid), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace awa

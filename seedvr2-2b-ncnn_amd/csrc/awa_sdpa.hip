// awa_sdpa.hip — varlen window attention on CDNA4 matrix cores.
//
// Replaces the per-(window, head) softmax(Q K^T / sqrt(128)) V of
// dit_vk.cpp:406-439 / awa.comp:79-171 for all windows at once.  Window w's
// sequence is its f_w video rows followed by the TXT text rows (dit_vk.cpp:
// 391-405), non-causal.
//
// One workgroup (4 wave64) per (work item, head).  A work item is one window
// and up to two of its 64-row query tiles; each wave owns 32 queries.  The
// window's key/value tiles stream through LDS (double buffered).  Scores are
// formed transposed, S^T = K Q^T, so that a lane owns one query column: the
// online softmax (exp2, log2(e) folded into the scale) then needs only one
// cross-lane exchange (lane ^ 32), and the probabilities leave the MFMA
// accumulator already in the B-operand layout of O^T = V^T P^T.  V is stored
// transposed per tile by the pack kernel so that A = V^T is read from LDS with
// 8-byte loads.
//
// bf16 storage -> v_mfma_f32_32x32x16_bf16 (fp32 accumulation).
// fp32 storage -> v_mfma_f32_32x32x2f32.
//
// Video query rows are scattered back to token order (dit_vk.cpp:445-455);
// text query rows go to per-window fp32 partials that the coalesce kernel
// averages in window order (dit_vk.cpp:440-444).
#include "awa_internal.hpp"

namespace awa {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

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
template <bool kBf16Out>
__device__ inline void store_rows(const f32x16 (&oacc)[4], float inv, int hb, void* dst_row) {
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 32 * dt + 8 * g + 4 * hb;
            const float o0 = oacc[dt][4 * g] * inv, o1 = oacc[dt][4 * g + 1] * inv;
            const float o2 = oacc[dt][4 * g + 2] * inv, o3 = oacc[dt][4 * g + 3] * inv;
            if constexpr (kBf16Out) {
                uint2 u;
                u.x = bf16_rne(o0) | (bf16_rne(o1) << 16);
                u.y = bf16_rne(o2) | (bf16_rne(o3) << 16);
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(dst_row) + d0) = u;
            } else {
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(dst_row) + d0) =
                    make_float4(o0, o1, o2, o3);
            }
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

// ----------------------------------------------------------------- bf16
// Four wave64 per workgroup, 32 queries each (two 64-row query tiles), and two
// workgroups per CU so that each SIMD holds two waves: while one runs its
// softmax on the VALU the other keeps the matrix core busy.  K and V^T
// tiles are copied global -> LDS with global_load_lds_dwordx4 (lane i of a
// wave writes 16 bytes at M0 + 16 i) into a double buffer whose 16-byte
// chunks are XOR-swizzled per row (swz_k, swz_v): the 16 rows read by a
// quarter-wave then fall in distinct banks.  Online softmax keeps a stale maximum
// until a new tile's maximum exceeds it by more than 2^8 (the output is
// divided by the matching sum at the end, so the result is unchanged).
typedef __attribute__((address_space(1))) void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

constexpr int KT_E = TILE * HEAD_D;         // bf16 elements of a K (or V^T) tile
constexpr int STAGE2 = 2 * KT_E;            // K tile then V^T tile
constexpr float RESCALE_LOG2 = 8.f;

// LDS has 64 four-byte banks: a 256-byte window.  A K row is 256 bytes (16
// chunks), so chunk ^ (row & 15) gives 16 consecutive rows 16 distinct chunk
// slots.  A V^T row is 128 bytes: rows 2r and 2r+1 share a window in its two
// halves, so chunk ^ ((row >> 1) & 7) spreads 16 consecutive rows likewise.
__device__ inline int swz_k(int row, int chunk) {
    return row * HEAD_D + ((chunk ^ (row & 15)) << 3);
}
__device__ inline int swz_v(int row, int chunk) {
    return row * TILE + ((chunk ^ ((row >> 1) & 7)) << 3);
}

__global__ __launch_bounds__(256, 2) void sdpa_bf16_kernel(SdpaArgs a) {
    __shared__ __align__(16) uint16_t lds[2 * STAGE2];
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

    const size_t head_off = (size_t)h * a.n_tiles * KT_E;
    const uint16_t* Kh = reinterpret_cast<const uint16_t*>(a.Kp) + head_off;
    const uint16_t* Vh = reinterpret_cast<const uint16_t*>(a.Vp) + head_off;

    // B operand of S^T = K Q^T, k-step s: Q[slot][16s + 8hb .. +8]
    bf16x8 qf[8];
    if (active) {
        const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.Qp) + head_off +
                               (size_t)wt.tile(kq) * KT_E + qslot * HEAD_D + 8 * hb;
#pragma unroll
        for (int s = 0; s < 8; s++) qf[s] = *reinterpret_cast<const bf16x8*>(qrow + 16 * s);
    }

    // DMA of one K tile and one V^T tile: each wave fills 4 + 4 KiB.
    const int krow_l = lane >> 4, kch = lane & 15;  // K: 4 rows of 16 chunks per KiB
    const int vrow_l = lane >> 3, vch = lane & 7;   // V^T: 8 rows of 8 chunks per KiB
    auto load_tile = [&](int kk, int stage) {
        const size_t t = (size_t)wt.tile(kk) * KT_E;
        uint16_t* ks = lds + stage * STAGE2;
        uint16_t* vs = ks + KT_E;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int blk = wave * 4 + i;
            const int kr = blk * 4 + krow_l;
            const uint16_t* ksrc = Kh + t + kr * HEAD_D + ((kch ^ (kr & 15)) << 3);
            __builtin_amdgcn_global_load_lds((gptr_t)ksrc, (lptr_t)(ks + blk * 512), 16, 0, 0);
            const int vr = blk * 8 + vrow_l;
            const uint16_t* vsrc = Vh + t + vr * TILE + ((vch ^ ((vr >> 1) & 7)) << 3);
            __builtin_amdgcn_global_load_lds((gptr_t)vsrc, (lptr_t)(vs + blk * 512), 16, 0, 0);
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) oacc[dt][r] = 0.f;
    // Running maximum m (log2 units) enters the score accumulator as its
    // initial value -m, so the MFMA yields s - m directly.
    float m_i = -INFINITY, l_i = 0.f;
    f32x16 mbias;
#pragma unroll
    for (int r = 0; r < 16; r++) mbias[r] = 0.f;
    bool first = true;

    load_tile(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int kk = 0; kk < nk; kk++) {
        const int stage = kk & 1;
        if (kk + 1 < nk) load_tile(kk + 1, stage ^ 1);
        if (active) {
            const uint16_t* ks = lds + stage * STAGE2;
            const uint16_t* vs = ks + KT_E;
            f32x16 sacc[2];
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                const bf16x8 kf = *reinterpret_cast<const bf16x8*>(ks + swz_k(32 * kt + n, hb));
                sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[0], mbias, 0, 0, 0);
            }
#pragma unroll
            for (int s = 1; s < 8; s++)
#pragma unroll
                for (int kt = 0; kt < 2; kt++) {
                    const bf16x8 kf = *reinterpret_cast<const bf16x8*>(ks + swz_k(32 * kt + n, 2 * s + hb));
                    sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], sacc[kt], 0, 0, 0);
                }
            const int kvalid = wt.nvalid(kk);
            if (kvalid < TILE) {
#pragma unroll
                for (int kt = 0; kt < 2; kt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int key = 32 * kt + 8 * (r >> 2) + 4 * hb + (r & 3);
                        if (key >= kvalid) sacc[kt][r] = -INFINITY;
                    }
            }
            // tile maximum relative to m
            float mt = fmaxf(sacc[0][0], sacc[1][0]);
#pragma unroll
            for (int r = 1; r < 16; r++) mt = fmaxf(mt, fmaxf(sacc[0][r], sacc[1][r]));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            if (__any(first || mt > RESCALE_LOG2)) {
                // raise m by mt (first tile: m = tile maximum); rare after the first tiles
                const float up = first ? mt : fmaxf(mt, 0.f);
                const float alpha = first ? 0.f : __builtin_amdgcn_exp2f(-up);
                m_i = first ? mt : m_i + up;
                l_i *= alpha;
#pragma unroll
                for (int dt = 0; dt < 4; dt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) oacc[dt][r] *= alpha;
#pragma unroll
                for (int kt = 0; kt < 2; kt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) sacc[kt][r] -= up;
#pragma unroll
                for (int r = 0; r < 16; r++) mbias[r] = -m_i;
                first = false;
            }
            float ps = 0.f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float p = __builtin_amdgcn_exp2f(sacc[kt][r]);
                    sacc[kt][r] = p;
                    ps += p;
                }
            l_i += ps;
            // O^T += V^T P^T
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int c2 = 0; c2 < 2; c2++) {
                    bf16x8 pb;
#pragma unroll
                    for (int i = 0; i < 8; i++) pb[i] = (__bf16)sacc[kt][8 * c2 + i];
#pragma unroll
                    for (int dt = 0; dt < 4; dt++) {
                        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(
                            vs + swz_v(32 * dt + n, 4 * kt + 2 * c2 + hb));
                        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb, oacc[dt], 0, 0, 0);
                    }
                }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (!active) return;
    const float l = l_i + __shfl_xor(l_i, 32);
    const float inv = 1.f / l;
    bool to_text = false;
    void* dst = query_dst(a, wt, w, h, kq, qslot, to_text, 2);
    if (dst == nullptr) return;
    if (to_text) store_rows<false>(oacc, inv, hb, dst);
    else store_rows<true>(oacc, inv, hb, dst);
}

// ----------------------------------------------------------------- fp32
constexpr int KP32 = 132;                 // LDS pitch of a K row (floats)
constexpr int VP32 = 68;                  // LDS pitch of a V^T row (floats)
constexpr int KS32 = TILE * KP32;
constexpr int STAGE32 = KS32 + HEAD_D * VP32;

__global__ __launch_bounds__(256, 1) void sdpa_f32_kernel(SdpaArgs a) {
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
    float qf[64];
    if (active) {
        const float* qrow = Qh + ((size_t)wt.tile(kq) * TILE + qslot) * HEAD_D + 64 * hb;
#pragma unroll
        for (int s = 0; s < 64; s += 4) {
            const float4 v = *reinterpret_cast<const float4*>(qrow + s);
            qf[s] = v.x; qf[s + 1] = v.y; qf[s + 2] = v.z; qf[s + 3] = v.w;
        }
    }

    float4 kreg[8], vreg[8];
    auto load_tile = [&](int kk) {
        const size_t t = (size_t)wt.tile(kk) * TILE * HEAD_D;
        const float4* ksrc = reinterpret_cast<const float4*>(Kh + t);
        const float4* vsrc = reinterpret_cast<const float4*>(Vh + t);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            kreg[i] = ksrc[tid + 256 * i];
            vreg[i] = vsrc[tid + 256 * i];
        }
    };
    auto store_tile = [&](int stage) {
        float* ks = lds + stage * STAGE32;
        float* vs = ks + KS32;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = tid + 256 * i;
            *reinterpret_cast<float4*>(ks + (c >> 5) * KP32 + (c & 31) * 4) = kreg[i];
            *reinterpret_cast<float4*>(vs + (c >> 4) * VP32 + (c & 15) * 4) = vreg[i];
        }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) oacc[dt][r] = 0.f;
    float m_i = -INFINITY, l_i = 0.f;

    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kk = 0; kk < nk; kk++) {
        const int stage = kk & 1;
        if (kk + 1 < nk) load_tile(kk + 1);
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
        if (kk + 1 < nk) store_tile(stage ^ 1);
        __syncthreads();
    }
    if (!active) return;
    const float l = l_i + __shfl_xor(l_i, 32);
    const float inv = 1.f / l;
    bool to_text = false;
    void* dst = query_dst(a, wt, w, h, kq, qslot, to_text, 4);
    if (dst == nullptr) return;
    store_rows<false>(oacc, inv, hb, dst);
}

}  // namespace

hipError_t launch_sdpa(int dtype, const SdpaArgs& a, hipStream_t s) {
    const int nblk = a.n_items * HEADS;
    const int grid = ((nblk + 7) >> 3) << 3;
    if (dtype == AWA_BF16)
        hipLaunchKernelGGL(sdpa_bf16_kernel, dim3(grid), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(sdpa_f32_kernel, dim3(grid), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace awa

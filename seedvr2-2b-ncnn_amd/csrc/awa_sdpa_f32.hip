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

// Destination of query slot `slot` of query tile kq (nullptr: padding slot).
__device__ inline void* query_dst(const SdpaArgs& a, const WinTiles& wt, int w, int h, int kq,
                                  int slot, size_t elem) {
    if (slot >= wt.nvalid(kq)) return nullptr;
    if (kq < wt.nvt) {
        const int g = a.cumf[w] + TILE * kq + slot;
        const size_t tok = (size_t)a.vidx[g];
        return reinterpret_cast<char*>(a.vattn) + (tok * DIM + (size_t)h * HEAD_D) * elem;
    }
    const int i = TILE * (kq - wt.nvt) + slot;
    return a.tpart + ((size_t)w * a.txt_len + i) * DIM + (size_t)h * HEAD_D;
}

constexpr int KP32 = 132;                 // LDS pitch of a K row (floats)
constexpr int VP32 = 68;                  // LDS pitch of a V^T row (floats)
constexpr int KS32 = TILE * KP32;
constexpr int STAGE32 = KS32 + HEAD_D * VP32;  // one K and one V^T tile: 68.6 KiB

typedef float f32x4v __attribute__((ext_vector_type(4)));

// One workgroup per (64-row query tile, head).  With v_mfma_f32_16x16x4_f32 a
// wave holds 16 queries' Q (32 floats), O^T (32) and one key tile's scores (16)
// in few registers, so two waves share each SIMD:
//   kSplit = false: four waves (wave w owns the tile's queries 16 w .. + 15)
//     and one LDS tile stage (68.6 KiB): two workgroups per CU;
//   kSplit = true: eight waves in two halves of four, half 0 taking the
//     window's key tiles [0, nk0), half 1 the rest (nk0 = ceil(nk / 2)), each
//     through its own stage: one workgroup per CU, and a long window's key
//     tiles take half as long; at the end half 1 leaves its row maxima, sums
//     and O^T in its stage and half 0 merges them.
// The launch takes the split form for small grids (at most two workgroups per
// CU, where the longest query tile sets the time), else the other.
//
// Lane l = 16 g + j (j: the lane's query; g: its group of four).
//   S^T = K Q^T per 16-key block kb and k-step s (32 steps of 4 channels):
//     A: K[16 kb + j][32 g + s], B: Q[j][32 g + s] (step s pairs channel
//     32 g + s across the four lane groups: any channel order that A and B
//     share gives the same dot products), out: lane l holds keys
//     16 kb + 4 g + r (r = 0..3) of query j.
//   O^T += V^T P^T per 16-channel block db and key step (kb, r):
//     A: V^T[16 db + j][16 kb + 4 g + r], B: P[j][16 kb + 4 g + r], which is
//     exactly score register r of block kb: the probabilities never move.
//     out: lane l holds channels 16 db + 4 g + r of query j.
// A query's scores are spread over lanes j, j + 16, j + 32, j + 48: its row
// maximum and sum take two cross-lane steps.
template <bool kSplit>
__global__ __launch_bounds__(kSplit ? 512 : 256, 2) void sdpa_f32_kernel(SdpaArgs a) {
    constexpr int HALVES = kSplit ? 2 : 1;
    __shared__ __align__(16) float lds[HALVES * STAGE32];
    // Workgroup b: head b % 20 of query tile GeomPlan::f32_units[b / 20]
    // (2 item + tile of the item), the tiles of windows with more key tiles
    // first: workgroups are dispatched in index order, and window sizes can
    // differ several-fold (the slowest workgroup sets the time).
    const int lid = (int)blockIdx.x;
    if (lid >= a.n_f32_units * HEADS) return;
    const int h = lid % HEADS;
    const int unit = a.f32_units[lid / HEADS];
    const int4 it = reinterpret_cast<const int4*>(a.items)[unit >> 1];
    const int kq = (unit & 1) ? it.z : it.y;
    const int w = it.x;
    const WinTiles wt = window_tiles(a, w);
    const int nk = wt.nvt + wt.ntt;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int half = kSplit ? __builtin_amdgcn_readfirstlane(wave >> 2) : 0;
    const int htid = tid & 255;  // thread index within the half
    const int j = lane & 15, g = lane >> 4;
    const int qslot = 16 * (wave & 3) + j;
    float* stage = lds + half * STAGE32;
    const int nk0 = kSplit ? (nk + 1) >> 1 : nk;  // iterations: half 0 has nk0 tiles, half 1 nk - nk0
    const int kbeg = half ? nk0 : 0, kend = half ? nk : nk0;

    const size_t head_off = (size_t)h * a.n_tiles * TILE * HEAD_D;
    const float* Qh = reinterpret_cast<const float*>(a.Qp) + head_off;
    const float* Kh = reinterpret_cast<const float*>(a.Kp) + head_off;
    const float* Vh = reinterpret_cast<const float*>(a.Vp) + head_off;

    // B operand of S^T: Q[qslot][32 g + s], s = 0..31
    float qf[32];
    {
        const float* qrow = Qh + ((size_t)wt.tile(kq) * TILE + qslot) * HEAD_D + 32 * g;
#pragma unroll
        for (int s = 0; s < 32; s += 4) {
            const f32x4v v = *reinterpret_cast<const f32x4v*>(qrow + s);
            qf[s] = v[0]; qf[s + 1] = v[1]; qf[s + 2] = v[2]; qf[s + 3] = v[3];
        }
    }

    // The half's next tile's K and V^T travel through registers (eight
    // 16-byte pieces of each per thread) while its current tile is computed.
    f32x4v rk[8], rv[8];
    auto load_tile = [&](int kk) __attribute__((always_inline)) {
        const size_t t = (size_t)wt.tile(kk) * TILE * HEAD_D;
        const f32x4v* ks = reinterpret_cast<const f32x4v*>(Kh + t);
        const f32x4v* vs = reinterpret_cast<const f32x4v*>(Vh + t);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            rk[i] = ks[htid + 256 * i];
            rv[i] = vs[htid + 256 * i];
        }
    };
    auto store_tile = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = htid + 256 * i;
            *reinterpret_cast<f32x4v*>(stage + (c >> 5) * KP32 + (c & 31) * 4) = rk[i];      // K row c / 32
            *reinterpret_cast<f32x4v*>(stage + KS32 + (c >> 4) * VP32 + (c & 15) * 4) = rv[i];  // V^T row c / 16
        }
    };

    f32x4v oacc[8];
#pragma unroll
    for (int db = 0; db < 8; db++) oacc[db] = (f32x4v){0.f, 0.f, 0.f, 0.f};
    float m_i = -INFINITY, l_i = 0.f;

    if (kbeg < kend) {
        load_tile(kbeg);
        store_tile();
    }
    __syncthreads();
    for (int i = 0; i < nk0; i++) {  // the same iteration count in both halves
        const int kk = kbeg + i;
        const bool have = kk < kend, have_next = kk + 1 < kend;  // uniform per half
        if (have_next) load_tile(kk + 1);
        if (have) {
            // ---- scores of the tile: four 16-key blocks
            f32x4v sacc[4];
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                sacc[kb] = (f32x4v){0.f, 0.f, 0.f, 0.f};
                const float* krow = stage + (16 * kb + j) * KP32 + 32 * g;
#pragma unroll
                for (int s = 0; s < 32; s += 4) {
                    const f32x4v kv = *reinterpret_cast<const f32x4v*>(krow + s);
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        sacc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[e], qf[s + e], sacc[kb], 0, 0, 0);
                }
            }
            // ---- online softmax (scale folded into Q; keys past the tile's
            // valid count get -inf)
            const int kvalid = wt.nvalid(kk);
            float mloc = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = 16 * kb + 4 * g + r;
                    const float v = key < kvalid ? sacc[kb][r] * a.scale_log2e : -INFINITY;
                    sacc[kb][r] = v;
                    mloc = fmaxf(mloc, v);
                }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
            const float m_new = fmaxf(m_i, mloc);  // finite: every tile has a valid key
            const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
            float psum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float p = __builtin_amdgcn_exp2f(sacc[kb][r] - m_new);
                    sacc[kb][r] = p;
                    psum += p;
                }
            l_i = l_i * alpha + psum;  // this lane's keys; summed over the group at the end
            m_i = m_new;
#pragma unroll
            for (int db = 0; db < 8; db++) oacc[db] *= alpha;
            // ---- O^T += V^T P^T
#pragma unroll
            for (int db = 0; db < 8; db++) {
                const float* vrow = stage + KS32 + (16 * db + j) * VP32 + 4 * g;
#pragma unroll
                for (int kb = 0; kb < 4; kb++) {
                    const f32x4v vv = *reinterpret_cast<const f32x4v*>(vrow + 16 * kb);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r], sacc[kb][r], oacc[db], 0, 0, 0);
                }
            }
        }
        if (i + 1 < nk0) {
            __syncthreads();  // every wave is done with its half's tile
            if (have_next) store_tile();
            __syncthreads();
        }
    }
    float l = l_i + __shfl_xor(l_i, 16);
    l += __shfl_xor(l, 32);
    if constexpr (kSplit) {
        // merge: half 1 leaves its running maximum (-inf when it had no
        // tile), sum and O^T in its stage, half 0 rescales both to the common
        // maximum
        __syncthreads();
        float* pub = lds + STAGE32;
        if (half == 1) {
#pragma unroll
            for (int db = 0; db < 8; db++)
                *reinterpret_cast<f32x4v*>(pub + qslot * HEAD_D + 16 * db + 4 * g) = oacc[db];
            if (g == 0) {
                pub[TILE * HEAD_D + qslot] = m_i;
                pub[TILE * HEAD_D + TILE + qslot] = l;
            }
        }
        __syncthreads();
        if (half == 1) return;
        const float m1 = pub[TILE * HEAD_D + qslot], l1 = pub[TILE * HEAD_D + TILE + qslot];
        const float m = fmaxf(m_i, m1);
        const float a0 = __builtin_amdgcn_exp2f(m_i - m), a1 = __builtin_amdgcn_exp2f(m1 - m);
        l = l * a0 + l1 * a1;
#pragma unroll
        for (int db = 0; db < 8; db++)
            oacc[db] = oacc[db] * a0 + *reinterpret_cast<const f32x4v*>(pub + qslot * HEAD_D + 16 * db + 4 * g) * a1;
    }
    const float inv = 1.f / l;
    float* dst = reinterpret_cast<float*>(query_dst(a, wt, w, h, kq, qslot, 4));
    if (dst == nullptr) return;
#pragma unroll
    for (int db = 0; db < 8; db++)
        *reinterpret_cast<float4*>(dst + 16 * db + 4 * g) =
            make_float4(oacc[db][0] * inv, oacc[db][1] * inv, oacc[db][2] * inv, oacc[db][3] * inv);
}

}  // namespace

hipError_t launch_sdpa_f32(const SdpaArgs& a, hipStream_t s) {
    const int nblk = a.n_f32_units * HEADS;
    if (nblk == 0) return hipSuccess;
    // n_slots: two per CU (the persistent bf16 schedule's slot count); the
    // split form at most two workgroups per CU (measured: 360p 63 -> 53 us,
    // while 720p and larger grids are faster with two 4-wave workgroups per CU)
    if (nblk <= a.n_slots)
        hipLaunchKernelGGL(sdpa_f32_kernel<true>, dim3(nblk), dim3(512), 0, s, a);
    else
        hipLaunchKernelGGL(sdpa_f32_kernel<false>, dim3(nblk), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace awa

// awa_pack.hip — fused qk RMSNorm + 3-D RoPE + window partition.
//
// One workgroup per (64-row tile, head); the 20 heads of a tile are
// neighbouring work indices on one XCD, so the tile's (cos, sin) rows come
// from HBM once and from that XCD's L2 for the other heads.  It gathers the
// tile's rows from vqkv / tqkv (window order through vidx, awa_vk.cpp:73-88),
// normalises q and k per head (dit_vk.cpp:54-61: r = sqrt(sum x^2 / 128 +
// eps), y = x / r * g), rotates channel pairs (2i, 2i+1) for i < 63
// (dit_vk.cpp:62-71; pair 63 of the table is the identity) and writes the
// packed tiles the SDPA kernel reads: Qp/Kp row-major per tile and, for fp32
// storage only, Vp transposed per tile (layout in awa_internal.hpp; the bf16
// attention kernel reads V from vqkv / tqkv itself).  HBM-bound: every byte it
// needs is read once and every packed byte written once; all loads of a
// thread are issued before the first use.
#include "awa_internal.hpp"

namespace awa {

namespace {

template <typename T> struct Io;

template <> struct Io<uint16_t> {  // bf16 storage: 8 channels in one 16-byte load
    using Raw = uint4;
    static __device__ inline Raw load(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
    static __device__ inline Raw zero() { return make_uint4(0, 0, 0, 0); }
    static __device__ inline void widen(const Raw& u, float* x) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[2 * i] = __uint_as_float(w[i] << 16);
            x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    static __device__ inline void store8(uint16_t* p, const float* x) {
        uint4 u;
        u.x = bf16_rne(x[0]) | (bf16_rne(x[1]) << 16);
        u.y = bf16_rne(x[2]) | (bf16_rne(x[3]) << 16);
        u.z = bf16_rne(x[4]) | (bf16_rne(x[5]) << 16);
        u.w = bf16_rne(x[6]) | (bf16_rne(x[7]) << 16);
        *reinterpret_cast<uint4*>(p) = u;
    }
};

template <> struct Io<float> {
    struct Raw { float4 a, b; };
    static __device__ inline Raw load(const float* p) {
        return {*reinterpret_cast<const float4*>(p), *reinterpret_cast<const float4*>(p + 4)};
    }
    static __device__ inline Raw zero() { return {make_float4(0, 0, 0, 0), make_float4(0, 0, 0, 0)}; }
    static __device__ inline void widen(const Raw& r, float* x) {
        x[0] = r.a.x; x[1] = r.a.y; x[2] = r.a.z; x[3] = r.a.w;
        x[4] = r.b.x; x[5] = r.b.y; x[6] = r.b.z; x[7] = r.b.w;
    }
    static __device__ inline void store8(float* p, const float* x) {
        *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<float4*>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
    }
};

// Sum over the 16 lanes that hold one 128-channel head row.
__device__ inline float row_sum16(float v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    return v;
}

// V staging tile in LDS (fp32), [slot][d] with a row pitch of VP = 129
// 4-byte words, so that the row writes and the transposing column reads below
// both hit distinct banks.
constexpr int VP = 129;

constexpr int RPT = TILE / 16;  // rows per thread (16 rows per 256-thread pass)

// kV: also pack V (fp32 storage).
template <typename T, bool kV>
__global__ __launch_bounds__(256) void pack_kernel(PackArgs a) {
    using IO = Io<T>;
    static_assert(!kV || sizeof(T) == 4, "V is packed for fp32 storage only");
    __shared__ uint32_t vs[kV ? TILE * VP : 1];

    const int nblk = a.n_tiles * HEADS;
    const int lid = xcd_remap(nblk);
    if (lid >= nblk) return;
    const int tile = lid / HEADS;
    const int h = lid - tile * HEADS;
    const int tid = threadIdx.x;
    const int c = tid & 15;     // 8-channel chunk of the head row
    const int r0 = tid >> 4;    // first slot handled by this thread

    const bool is_txt = tile >= a.n_vid_tiles;
    int nvalid;
    size_t cs_row0;             // table row of slot 0
    const int32_t* vidx = nullptr;
    const T* src;
    if (!is_txt) {
        const int w = a.tile_win[tile];
        const int j0 = (tile - a.tile_base[w]) * TILE;
        const int g0 = a.cumf[w] + j0;
        nvalid = min(TILE, a.cumf[w + 1] - g0);
        cs_row0 = g0;
        vidx = a.vidx + g0;
        src = reinterpret_cast<const T*>(a.vqkv);
    } else {
        const int tt = tile - a.n_vid_tiles;
        const int set = tt / a.ntt;
        const int j0 = (tt % a.ntt) * TILE;
        nvalid = min(TILE, a.txt_len - j0);
        cs_row0 = (size_t)set * a.txt_len + j0;
        src = reinterpret_cast<const T*>(a.tqkv) + (size_t)j0 * QKV;
    }
    const float4* cst = reinterpret_cast<const float4*>(is_txt ? a.tcs : a.vcs);
    const float* gq = is_txt ? a.nq_t : a.nq_v;
    const float* gk = is_txt ? a.nk_t : a.nk_v;
    const int col = h * HEAD_D + c * 8;

    // Issue every load of the thread: 4 rows x (q, k, v, 4 cos/sin pairs).
    typename IO::Raw rq[RPT], rk[RPT], rv[RPT];
    float4 cs[RPT][2];
#pragma unroll
    for (int kk = 0; kk < RPT; kk++) {
        const int r = r0 + 16 * kk;
        if (r < nvalid) {  // uniform across the 16 lanes of a row
            const T* row = src + (size_t)(is_txt ? r : vidx[r]) * QKV + col;
            rq[kk] = IO::load(row);
            rk[kk] = IO::load(row + DIM);
            if constexpr (kV) rv[kk] = IO::load(row + 2 * DIM);
            const float4* p = cst + ((cs_row0 + r) * CS_STRIDE + c * 4) / 2;
            cs[kk][0] = p[0];
            cs[kk][1] = p[1];
        } else {
            rq[kk] = rk[kk] = rv[kk] = IO::zero();
            cs[kk][0] = cs[kk][1] = make_float4(1.f, 0.f, 1.f, 0.f);
        }
    }
    float gqv[8], gkv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        gqv[i] = gq[c * 8 + i];
        gkv[i] = gk[c * 8 + i];
    }

    const size_t tile_off = ((size_t)h * a.n_tiles + tile) * TILE * HEAD_D;
    T* Qt = reinterpret_cast<T*>(a.Qp) + tile_off;
    T* Kt = reinterpret_cast<T*>(a.Kp) + tile_off;
    T* Vt = kV ? reinterpret_cast<T*>(a.Vp) + tile_off : nullptr;

#pragma unroll
    for (int kk = 0; kk < RPT; kk++) {
        const int r = r0 + 16 * kk;
        float q[8], k[8];
        IO::widen(rq[kk], q);
        IO::widen(rk[kk], k);
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sq += q[i] * q[i];
            sk += k[i] * k[i];
        }
        sq = row_sum16(sq);
        sk = row_sum16(sk);
        const float nq = sqrtf(sq / (float)HEAD_D + a.eps);
        const float nk = sqrtf(sk / (float)HEAD_D + a.eps);
        const float csv[8] = {cs[kk][0].x, cs[kk][0].y, cs[kk][0].z, cs[kk][0].w,
                              cs[kk][1].x, cs[kk][1].y, cs[kk][1].z, cs[kk][1].w};
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float cn = csv[2 * p], sn = csv[2 * p + 1];
            const float q0 = q[2 * p] / nq * gqv[2 * p], q1 = q[2 * p + 1] / nq * gqv[2 * p + 1];
            const float k0 = k[2 * p] / nk * gkv[2 * p], k1 = k[2 * p + 1] / nk * gkv[2 * p + 1];
            q[2 * p] = (q0 * cn - q1 * sn) * a.qscale;
            q[2 * p + 1] = (q1 * cn + q0 * sn) * a.qscale;
            k[2 * p] = k0 * cn - k1 * sn;
            k[2 * p + 1] = k1 * cn + k0 * sn;
        }
        IO::store8(Qt + (size_t)r * HEAD_D + c * 8, q);
        IO::store8(Kt + (size_t)r * HEAD_D + c * 8, k);
        if constexpr (kV) {
            float v[8];
            IO::widen(rv[kk], v);
            uint32_t* vrow = vs + r * VP;
#pragma unroll
            for (int i = 0; i < 8; i++) vrow[c * 8 + i] = __float_as_uint(v[i]);
        }
    }
    if constexpr (!kV) return;
    __syncthreads();

    // Transposed V tile Vt[d][slot] (fp32), written as whole 256-byte rows by
    // consecutive lanes: thread unit (d, 4-slot chunk sc), 16 chunks per row.
#pragma unroll
    for (int it = 0; it < 8; it++) {
        const int u = it * 256 + tid;
        const int d = u >> 4, sc = u & 15;
        float4 o;
        o.x = __uint_as_float(vs[(sc * 4 + 0) * VP + d]);
        o.y = __uint_as_float(vs[(sc * 4 + 1) * VP + d]);
        o.z = __uint_as_float(vs[(sc * 4 + 2) * VP + d]);
        o.w = __uint_as_float(vs[(sc * 4 + 3) * VP + d]);
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(Vt) + (size_t)d * TILE + sc * 4) = o;
    }
}

}  // namespace

hipError_t launch_pack(int dtype, const PackArgs& a, hipStream_t s) {
    const dim3 grid(xcd_grid((long)a.n_tiles * HEADS)), block(256);
    if (dtype == AWA_BF16)
        hipLaunchKernelGGL((pack_kernel<uint16_t, false>), grid, block, 0, s, a);
    else
        hipLaunchKernelGGL((pack_kernel<float, true>), grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace awa

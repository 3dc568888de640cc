// awa_pack.hip — fused qk RMSNorm + 3-D RoPE + window partition.
//
// One workgroup per (64-row tile, head).  It gathers the tile's rows from
// vqkv / tqkv (window order through vidx, awa_vk.cpp:73-88), normalises q and k
// per head (dit_vk.cpp:54-61: r = sqrt(sum x^2 / 128 + eps), y = x / r * g),
// rotates channel pairs (2i, 2i+1) for i < 63 (dit_vk.cpp:62-71) with the
// (cos, sin) rows staged in LDS, and writes the packed tiles the SDPA kernel
// reads: Qp/Kp row-major per tile, Vp transposed per tile (see
// awa_internal.hpp).  HBM-bound: every input byte of q, k, v is read once.
#include "awa_internal.hpp"

namespace awa {

namespace {

template <typename T> struct Io;

template <> struct Io<uint16_t> {  // bf16 storage
    static __device__ inline void load8(const uint16_t* p, float* x) {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[2 * i] = __uint_as_float(w[i] << 16);
            x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    static __device__ inline uint32_t rne(float f) {
        // round to nearest even, cast_f32_bf16.comp:24
        const uint32_t u = __float_as_uint(f);
        return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    }
    static __device__ inline void store8(uint16_t* p, const float* x) {
        uint4 u;
        u.x = rne(x[0]) | (rne(x[1]) << 16);
        u.y = rne(x[2]) | (rne(x[3]) << 16);
        u.z = rne(x[4]) | (rne(x[5]) << 16);
        u.w = rne(x[6]) | (rne(x[7]) << 16);
        *reinterpret_cast<uint4*>(p) = u;
    }
};

template <> struct Io<float> {
    static __device__ inline void load8(const float* p, float* x) {
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
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

template <typename T>
__global__ __launch_bounds__(256) void pack_kernel(PackArgs a) {
    constexpr int VROW = 128 + 16 / (int)sizeof(T);  // LDS pitch of the V staging tile
    __shared__ __align__(16) T vs[TILE][VROW];
    __shared__ float2 cs_s[TILE][NPAIR + 1];

    const int tile = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int c = tid & 15;     // 8-channel chunk of the head row
    const int r0 = tid >> 4;    // first slot handled by this thread

    const bool is_txt = tile >= a.n_vid_tiles;
    int w = 0, set = 0, j0, nvalid;
    if (!is_txt) {
        w = a.tile_win[tile];
        j0 = (tile - a.tile_base[w]) * TILE;
        nvalid = min(TILE, a.cumf[w + 1] - a.cumf[w] - j0);
    } else {
        const int tt = tile - a.n_vid_tiles;
        set = tt / a.ntt;
        j0 = (tt % a.ntt) * TILE;
        nvalid = min(TILE, a.txt_len - j0);
    }
    const float* gq = is_txt ? a.nq_t : a.nq_v;
    const float* gk = is_txt ? a.nk_t : a.nk_v;

    // Stage the (cos, sin) rows of the tile's slots in LDS; they are shared by
    // q and k (and, across the grid, by all heads through L2).
    for (int i = tid; i < TILE * NPAIR; i += 256) {
        const int r = i / NPAIR, q = i % NPAIR;
        float2 v = make_float2(1.f, 0.f);
        if (r < nvalid) {
            const size_t row = is_txt ? (size_t)set * a.txt_len + j0 + r
                                      : (size_t)a.cumf[w] + j0 + r;
            v = (is_txt ? a.tcs : a.vcs)[row * NPAIR + q];
        }
        cs_s[r][q] = v;
    }
    float gqv[8], gkv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        gqv[i] = gq[c * 8 + i];
        gkv[i] = gk[c * 8 + i];
    }
    __syncthreads();

    const size_t tile_off = ((size_t)h * a.n_tiles + tile) * TILE * HEAD_D;
    T* Qt = reinterpret_cast<T*>(a.Qp) + tile_off;
    T* Kt = reinterpret_cast<T*>(a.Kp) + tile_off;
    T* Vt = reinterpret_cast<T*>(a.Vp) + tile_off;

#pragma unroll
    for (int kk = 0; kk < TILE / 16; kk++) {
        const int r = r0 + 16 * kk;
        float q[8], k[8], v[8];
        if (r < nvalid) {  // uniform across the 16 lanes of a row
            const T* row;
            if (!is_txt) {
                const int g = a.cumf[w] + j0 + r;
                row = reinterpret_cast<const T*>(a.vqkv) + (size_t)a.vidx[g] * QKV;
            } else {
                row = reinterpret_cast<const T*>(a.tqkv) + (size_t)(j0 + r) * QKV;
            }
            const int col = h * HEAD_D + c * 8;
            Io<T>::load8(row + col, q);
            Io<T>::load8(row + DIM + col, k);
            Io<T>::load8(row + 2 * DIM + col, v);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] = k[i] = v[i] = 0.f;
        }
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            sq += q[i] * q[i];
            sk += k[i] * k[i];
        }
        sq = row_sum16(sq);
        sk = row_sum16(sk);
        const float rq = sqrtf(sq / (float)HEAD_D + a.eps);
        const float rk = sqrtf(sk / (float)HEAD_D + a.eps);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            q[i] = q[i] / rq * gqv[i];
            k[i] = k[i] / rk * gkv[i];
        }
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int P = c * 4 + p;  // channel pair index; pair 63 passes through
            if (P < NPAIR) {
                const float2 cs = cs_s[r][P];
                const float q0 = q[2 * p], q1 = q[2 * p + 1];
                q[2 * p] = q0 * cs.x - q1 * cs.y;
                q[2 * p + 1] = q1 * cs.x + q0 * cs.y;
                const float k0 = k[2 * p], k1 = k[2 * p + 1];
                k[2 * p] = k0 * cs.x - k1 * cs.y;
                k[2 * p + 1] = k1 * cs.x + k0 * cs.y;
            }
        }
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] *= a.qscale;
        Io<T>::store8(Qt + (size_t)r * HEAD_D + c * 8, q);
        Io<T>::store8(Kt + (size_t)r * HEAD_D + c * 8, k);
        if constexpr (sizeof(T) == 2) {
            uint4 u;
            u.x = Io<uint16_t>::rne(v[0]) | (Io<uint16_t>::rne(v[1]) << 16);
            u.y = Io<uint16_t>::rne(v[2]) | (Io<uint16_t>::rne(v[3]) << 16);
            u.z = Io<uint16_t>::rne(v[4]) | (Io<uint16_t>::rne(v[5]) << 16);
            u.w = Io<uint16_t>::rne(v[6]) | (Io<uint16_t>::rne(v[7]) << 16);
            *reinterpret_cast<uint4*>(&vs[r][c * 8]) = u;
        } else {
            *reinterpret_cast<float4*>(&vs[r][c * 8]) = make_float4(v[0], v[1], v[2], v[3]);
            *reinterpret_cast<float4*>(&vs[r][c * 8 + 4]) = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
    __syncthreads();

    // Transposed V tile: Vt[d][slot]; lanes of a wave take 64 consecutive d
    // (conflict-free LDS column reads), each wave one group of slots.
    constexpr int EPC = 16 / (int)sizeof(T);        // elements per 16-byte chunk
    constexpr int CPR = TILE / EPC;                 // chunks per V^T row
    const int d = tid & 127;
#pragma unroll
    for (int sc = tid >> 7; sc < CPR; sc += 2) {
        union {
            uint4 u;
            T e[EPC];
        } tmp;
#pragma unroll
        for (int j = 0; j < EPC; j++) {
            int slot = sc * EPC + j;
            if constexpr (sizeof(T) == 2) {
                // swap quads 1 and 2 of each 16-slot group (see awa_internal.hpp)
                const int qd = (slot >> 2) & 3;
                if (qd == 1 || qd == 2) slot ^= 12;
            }
            tmp.e[j] = vs[slot][d];
        }
        *reinterpret_cast<uint4*>(Vt + (size_t)d * TILE + sc * EPC) = tmp.u;
    }
}

}  // namespace

hipError_t launch_pack(int dtype, const PackArgs& a, hipStream_t s) {
    dim3 grid(a.n_tiles, HEADS), block(256);
    if (dtype == AWA_BF16)
        hipLaunchKernelGGL(pack_kernel<uint16_t>, grid, block, 0, s, a);
    else
        hipLaunchKernelGGL(pack_kernel<float>, grid, block, 0, s, a);
    return hipGetLastError();
}

}  // namespace awa

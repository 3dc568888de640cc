// awa_pack.hip — fused qk RMSNorm + 3-D RoPE + window partition.
//
// One workgroup per (16-row quarter of a 64-row tile, head) for fp32
// storage, per (tile, two heads) for bf16; the workgroups of a tile are
// neighbouring work indices on one XCD, so the tile's (cos, sin) rows come
// from HBM once and from that XCD's L2 for the other heads, staged in LDS.  It gathers the
// tile's rows from vqkv / tqkv (window order of vidx, awa_vk.cpp:73-88, through
// the geometry's row table),
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

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

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
    // round to nearest even, two values per v_cvt_pk_bf16_f32
    static __device__ inline uint32_t pk(float lo, float hi) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
    }
    static __device__ inline void store8(uint16_t* p, const float* x) {
        *reinterpret_cast<uint4*>(p) = make_uint4(pk(x[0], x[1]), pk(x[2], x[3]), pk(x[4], x[5]), pk(x[6], x[7]));
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

// Sum over the 16 lanes that hold one 128-channel head row, a butterfly with
// DPP lane moves (no LDS round trips): partners lane ^ 1 and lane ^ 2
// (quad_perm), then the mirror lane in each half of 8 (which holds the other
// quad's sum) and in the 16 (the other half's): every lane adds the same
// two partial sums as with partners lane ^ 4 and lane ^ 8, so the result is
// the xor butterfly's, bit for bit.
__device__ inline float dpp_add(float v, int ctrl) {
    int m;
    switch (ctrl) {  // the control must be a constant
    case 0xB1: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false); break;  // [1,0,3,2]
    case 0x4E: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false); break;  // [2,3,0,1]
    case 0x141: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false); break; // row_half_mirror
    default: m = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xf, 0xf, false); break;    // row_mirror
    }
    return v + __int_as_float(m);
}
__device__ inline float row_sum16(float v) {
    v = dpp_add(v, 0xB1);
    v = dpp_add(v, 0x4E);
    v = dpp_add(v, 0x141);
    return dpp_add(v, 0x140);
}
// x / r, correctly rounded, from rinv = 1 / r (correctly rounded): q = x rinv
// is within an ulp of x / r, and one correction step with the exact residual
// fma(-q, r, x) rounds it correctly (Markstein, IBM J. Res. Dev. 34(1), 1990).
// Three instructions where the IEEE division takes about ten.
__device__ inline float div_by(float x, float r, float rinv) {
    const float q = x * rinv;
    return __builtin_fmaf(__builtin_fmaf(-q, r, x), rinv, q);
}

// V staging tile in LDS (fp32), [slot][d] with a row pitch of VP = 129
// 4-byte words, so that the row writes and the transposing column reads below
// both hit distinct banks.
constexpr int VP = 129;

constexpr int RPT = TILE / 16;  // rows per thread of the bf16 kernel (16 rows per 256-thread pass)

// The tile's (cos, sin) table rows staged in LDS: rows cs_row0 .. +63 of the
// geometry's table are contiguous (64 pairs = 32 float4 per row), so the 256
// threads read them as one coalesced 32 KiB block, eight float4 each; rows at
// or past nvalid (padding slots, whose table rows may lie past the table's
// end) hold the identity rotation.  Each thread then reads its own rows'
// pairs back from LDS: the 16 lanes of a row read its 512 contiguous bytes.
constexpr int CS_Q4 = CS_STRIDE / 2;  // float4 per table row
constexpr int CS_PT = TILE * CS_Q4 / 256;  // float4 per thread
// The loads are issued before the q/k loads (load_cs) and written to LDS after
// them (store_cs): the LDS writes then wait only for the table loads.
__device__ inline void load_cs(float4 (&t)[CS_PT], const float4* cst, size_t cs_row0, int nvalid, int tid) {
#pragma unroll
    for (int it = 0; it < CS_PT; it++) {
        const int i = it * 256 + tid, row = i / CS_Q4;
        t[it] = row < nvalid ? cst[(cs_row0 + row) * CS_Q4 + (i % CS_Q4)] : make_float4(1.f, 0.f, 1.f, 0.f);
    }
}
__device__ inline void store_cs(float4* lds_cs, const float4 (&t)[CS_PT], int tid) {
#pragma unroll
    for (int it = 0; it < CS_PT; it++) lds_cs[it * 256 + tid] = t[it];
}

// fp32 storage: one workgroup per (QR rows of a 64-row tile, head), QR / 16
// rows per thread (16 threads per row, each an 8-channel chunk).  QR = 64
// (whole tiles) when the grid fills the device; QR = 16 (four workgroups per
// tile and head) for small geometries, whose whole-tile grid has fewer
// workgroups than the device has CUs (220 at 360p).  Correctly rounded
// arithmetic (IEEE sqrt, division by div_by); V is packed transposed through
// LDS: the workgroup's QR slots of every channel row of the V^T tile.
// whole-tile workgroups from this many (tile, head) pairs on (measured: quarters
// faster up to 1,200 pairs (360p 12.0 -> 10.2 us, 720p 31 -> 26), whole tiles
// from 1,900 (1080p 79 against 86 us))
constexpr long F32_WHOLE_MIN = 1536;
template <int QR>
__global__ __launch_bounds__(256) void pack_f32_kernel(PackArgs a) {
    using IO = Io<float>;
    constexpr int NQ = TILE / QR;                 // workgroups per (tile, head)
    constexpr int RT = QR / 16;                   // rows per thread
    constexpr int NCS = QR * CS_Q4 / 256;         // table float4 per thread
    __shared__ uint32_t vs[QR * VP];
    __shared__ float4 lds_cs[QR * CS_Q4];

    const int nblk = a.n_tiles * HEADS * NQ;
    const int lid = xcd_remap(nblk);  // a tile's workgroups: neighbouring ids, one XCD
    if (lid >= nblk) return;
    const int tile = lid / (HEADS * NQ);
    const int rem = lid - tile * (HEADS * NQ);
    const int h = rem / NQ, qt = rem - (rem / NQ) * NQ;
    const int tid = threadIdx.x;
    const int c = tid & 15;                  // 8-channel chunk of the head row
    const int rl = tid >> 4;                 // first row of the thread in the workgroup

    // Two levels of loads: the tile's record (RoPE-table row of slot 0,
    // valid rows) and the thread's row indices from the row table, then every
    // data load of the thread.
    const bool is_txt = tile >= a.n_vid_tiles;
    const int2 meta = reinterpret_cast<const int2*>(a.tile_meta)[tile];
    const uint32_t* rows =
        a.vrow + (size_t)(is_txt ? a.n_vid_tiles + (tile - a.n_vid_tiles) % a.ntt : tile) * TILE;
    uint32_t ridx[RT];
#pragma unroll
    for (int kk = 0; kk < RT; kk++) ridx[kk] = rows[vrow_pos(qt * QR + rl + 16 * kk)];
    const int nvalid = meta.y;
    const size_t cs_row0 = (size_t)meta.x;  // table row of slot 0
    const float* src = reinterpret_cast<const float*>(is_txt ? a.tqkv : a.vqkv);
    const float4* cst = reinterpret_cast<const float4*>(is_txt ? a.tcs : a.vcs);
    const float* gq = is_txt ? a.nq_t : a.nq_v;
    const float* gk = is_txt ? a.nk_t : a.nk_v;
    const int col = h * HEAD_D + c * 8;

    // the workgroup's (cos, sin) rows for LDS, then the rows' q, k, v
    float4 cst_t[NCS];
#pragma unroll
    for (int it = 0; it < NCS; it++) {
        const int i = it * 256 + tid, row = qt * QR + i / CS_Q4;
        // padding slots repeat the last valid row (as the row table makes
        // them repeat the window's last token), so that every load of this
        // kernel is unconditional: under a per-row branch the compiler waited
        // for them conservatively (360p 10.6 -> 9.6 us; the bf16 kernel keeps
        // its branches, which measured faster at 1080p).  The attention
        // kernels mask padding keys by the key count (an exact zero weight)
        // and drop padding queries, so padding rows reach no output.
        cst_t[it] = cst[(cs_row0 + min(row, nvalid - 1)) * CS_Q4 + (i % CS_Q4)];
    }
    IO::Raw rq[RT], rk[RT], rv[RT];
#pragma unroll
    for (int kk = 0; kk < RT; kk++) {  // padding slots: the window's last row
        const float* row = src + (size_t)ridx[kk] + col;
        rq[kk] = IO::load(row);
        rk[kk] = IO::load(row + DIM);
        rv[kk] = IO::load(row + 2 * DIM);
    }
    float gqv[8], gkv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        gqv[i] = gq[c * 8 + i];
        gkv[i] = gk[c * 8 + i];
    }
#pragma unroll
    for (int it = 0; it < NCS; it++) lds_cs[it * 256 + tid] = cst_t[it];
    __syncthreads();

    const size_t tile_off = ((size_t)h * a.n_tiles + tile) * TILE * HEAD_D;
    float* Qt = reinterpret_cast<float*>(a.Qp) + tile_off;
    float* Kt = reinterpret_cast<float*>(a.Kp) + tile_off;
    float* Vt = reinterpret_cast<float*>(a.Vp) + tile_off;

#pragma unroll
    for (int kk = 0; kk < RT; kk++) {
        const int lr = rl + 16 * kk;       // row in the workgroup
        const int r = qt * QR + lr;        // slot in the tile
        const float4 cs0 = lds_cs[lr * CS_Q4 + 2 * c], cs1 = lds_cs[lr * CS_Q4 + 2 * c + 1];
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
        const float iq = 1.f / nq, ik = 1.f / nk;
        const float csv[8] = {cs0.x, cs0.y, cs0.z, cs0.w, cs1.x, cs1.y, cs1.z, cs1.w};
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float cn = csv[2 * p], sn = csv[2 * p + 1];
            const float q0 = div_by(q[2 * p], nq, iq) * gqv[2 * p];
            const float q1 = div_by(q[2 * p + 1], nq, iq) * gqv[2 * p + 1];
            const float k0 = div_by(k[2 * p], nk, ik) * gkv[2 * p];
            const float k1 = div_by(k[2 * p + 1], nk, ik) * gkv[2 * p + 1];
            q[2 * p] = (q0 * cn - q1 * sn) * a.qscale;
            q[2 * p + 1] = (q1 * cn + q0 * sn) * a.qscale;
            k[2 * p] = k0 * cn - k1 * sn;
            k[2 * p + 1] = k1 * cn + k0 * sn;
        }
        IO::store8(Qt + (size_t)r * HEAD_D + c * 8, q);
        IO::store8(Kt + (size_t)r * HEAD_D + c * 8, k);
        float v[8];
        IO::widen(rv[kk], v);
        uint32_t* vrow = vs + lr * VP;
#pragma unroll
        for (int i = 0; i < 8; i++) vrow[c * 8 + i] = __float_as_uint(v[i]);
    }
    __syncthreads();

    // Transposed V: Vt[d][slot] for the workgroup's QR slots, 4 QR contiguous
    // bytes per channel row (thread unit: channel d, 4-slot chunk sc).
    constexpr int NSC = QR / 4;
#pragma unroll
    for (int it = 0; it < QR * HEAD_D / 4 / 256; it++) {
        const int u = it * 256 + tid;
        const int d = u / NSC, sc = u % NSC;
        float4 o;
        o.x = __uint_as_float(vs[(sc * 4 + 0) * VP + d]);
        o.y = __uint_as_float(vs[(sc * 4 + 1) * VP + d]);
        o.z = __uint_as_float(vs[(sc * 4 + 2) * VP + d]);
        o.w = __uint_as_float(vs[(sc * 4 + 3) * VP + d]);
        *reinterpret_cast<float4*>(Vt + (size_t)d * TILE + qt * QR + sc * 4) = o;
    }
}

// bf16 storage: one workgroup per (64-row tile, group of PACK_HG heads).  A
// thread's row offsets, (cos, sin) pairs and gains are the same for every head
// of the tile, so the workgroup stages the tile's table rows in LDS once
// (load_cs, store_cs) and each thread keeps its rows' pairs, offsets and gains in
// registers for its heads; the q and k loads of the next head are in flight
// while the current head is normalised, rotated and stored.  The output is rounded to bf16, so
// the arithmetic is the short form: 1/r by v_rsq_f32 (within an ulp of the
// correctly rounded sqrt and division of the fp32 kernel) and
// y = ((x g) c -/+ (x' g') s) (1/r [* qscale]), eight operations per channel
// pair where the exact form takes fourteen.
constexpr int PACK_HG = 2;  // heads per workgroup (measured against 1, 4, 5 and 10 at 360p-1080p)

__global__ __launch_bounds__(256) void pack_bf16_kernel(PackArgs a) {
    using IO = Io<uint16_t>;
    __shared__ float4 lds_cs[TILE * CS_Q4];
    constexpr int NG = HEADS / PACK_HG;
    static_assert(HEADS % PACK_HG == 0, "head groups must tile the heads");
    const int nblk = a.n_tiles * NG;
    const int lid = xcd_remap(nblk);  // a tile's groups: neighbouring ids, one XCD
    if (lid >= nblk) return;
    const int tile = lid / NG;
    const int h0 = (lid - tile * NG) * PACK_HG;
    const int tid = threadIdx.x;
    const int c = tid & 15;
    const int r0 = tid >> 4;

    const bool is_txt = tile >= a.n_vid_tiles;
    const int2 meta = reinterpret_cast<const int2*>(a.tile_meta)[tile];
    const uint32_t* rows =
        a.vrow + (size_t)(is_txt ? a.n_vid_tiles + (tile - a.n_vid_tiles) % a.ntt : tile) * TILE;
    uint32_t ridx[RPT];
#pragma unroll
    for (int kk = 0; kk < RPT; kk++) ridx[kk] = rows[vrow_pos(r0 + 16 * kk)];
    const int nvalid = meta.y;
    const size_t cs_row0 = (size_t)meta.x;
    const uint16_t* src = reinterpret_cast<const uint16_t*>(is_txt ? a.tqkv : a.vqkv);
    const float4* cst = reinterpret_cast<const float4*>(is_txt ? a.tcs : a.vcs);
    const float* gq = is_txt ? a.nq_t : a.nq_v;
    const float* gk = is_txt ? a.nk_t : a.nk_v;

    // q and k of head h for the thread's rows (zeros for padding rows)
    auto load_head = [&](int h, IO::Raw (&q)[RPT], IO::Raw (&k)[RPT]) __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < RPT; kk++) {
            if (r0 + 16 * kk < nvalid) {  // uniform across the 16 lanes of a row
                const uint16_t* row = src + (size_t)ridx[kk] + h * HEAD_D + c * 8;
                q[kk] = IO::load(row);
                k[kk] = IO::load(row + DIM);
            } else {
                q[kk] = k[kk] = IO::zero();
            }
        }
    };
    float4 cst_t[CS_PT];
    load_cs(cst_t, cst, cs_row0, nvalid, tid);
    IO::Raw rq[2][RPT], rk[2][RPT];
    load_head(h0, rq[0], rk[0]);
    store_cs(lds_cs, cst_t, tid);
    __syncthreads();
    float4 cs[RPT][2];
#pragma unroll
    for (int kk = 0; kk < RPT; kk++) {
        const int r = r0 + 16 * kk;
        cs[kk][0] = lds_cs[r * CS_Q4 + 2 * c];
        cs[kk][1] = lds_cs[r * CS_Q4 + 2 * c + 1];
    }
    float gqv[8], gkv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        gqv[i] = gq[c * 8 + i];
        gkv[i] = gk[c * 8 + i];
    }
    // y (8 channels of one row, normalised, gained and rotated, times s)
    auto rope8 = [&](float (&x)[8], const float (&g)[8], float s, const float (&csv)[8]) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float cn = csv[2 * p], sn = csv[2 * p + 1];
            const float p0 = x[2 * p] * g[2 * p], p1 = x[2 * p + 1] * g[2 * p + 1];
            x[2 * p] = __builtin_fmaf(p0, cn, -(p1 * sn)) * s;
            x[2 * p + 1] = __builtin_fmaf(p1, cn, p0 * sn) * s;
        }
    };

#pragma unroll
    for (int j = 0; j < PACK_HG; j++) {
        const int h = h0 + j;
        if (j + 1 < PACK_HG) load_head(h + 1, rq[(j + 1) & 1], rk[(j + 1) & 1]);
        const size_t tile_off = ((size_t)h * a.n_tiles + tile) * TILE * HEAD_D;
        uint16_t* Qt = reinterpret_cast<uint16_t*>(a.Qp) + tile_off;
        uint16_t* Kt = reinterpret_cast<uint16_t*>(a.Kp) + tile_off;
#pragma unroll
        for (int kk = 0; kk < RPT; kk++) {
            const int r = r0 + 16 * kk;
            float q[8], k[8];
            IO::widen(rq[j & 1][kk], q);
            IO::widen(rk[j & 1][kk], k);
            float sq = 0.f, sk = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                sq = __builtin_fmaf(q[i], q[i], sq);
                sk = __builtin_fmaf(k[i], k[i], sk);
            }
            sq = row_sum16(sq);
            sk = row_sum16(sk);
            // sum / 128 is exact (a power of two)
            const float iq = __builtin_amdgcn_rsqf(sq * (1.f / (float)HEAD_D) + a.eps) * a.qscale;
            const float ik = __builtin_amdgcn_rsqf(sk * (1.f / (float)HEAD_D) + a.eps);
            const float csv[8] = {cs[kk][0].x, cs[kk][0].y, cs[kk][0].z, cs[kk][0].w,
                                  cs[kk][1].x, cs[kk][1].y, cs[kk][1].z, cs[kk][1].w};
            rope8(q, gqv, iq, csv);
            rope8(k, gkv, ik, csv);
            IO::store8(Qt + (size_t)r * HEAD_D + c * 8, q);
            IO::store8(Kt + (size_t)r * HEAD_D + c * 8, k);
        }
    }
}

}  // namespace

hipError_t launch_pack(int dtype, const PackArgs& a, hipStream_t s) {
    const dim3 block(256);
    if (dtype == AWA_BF16)
        hipLaunchKernelGGL(pack_bf16_kernel, dim3(xcd_grid((long)a.n_tiles * (HEADS / PACK_HG))), block, 0, s, a);
    else if ((long)a.n_tiles * HEADS >= F32_WHOLE_MIN)
        hipLaunchKernelGGL(pack_f32_kernel<TILE>, dim3(xcd_grid((long)a.n_tiles * HEADS)), block, 0, s, a);
    else
        hipLaunchKernelGGL(pack_f32_kernel<16>, dim3(xcd_grid((long)a.n_tiles * HEADS * (TILE / 16))), block, 0, s,
                           a);
    return hipGetLastError();
}

}  // namespace awa

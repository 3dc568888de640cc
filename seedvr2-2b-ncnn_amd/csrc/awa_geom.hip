// awa_geom.hip — window partition, shift and ragged index build on the device.
//
// Replaces awa::make_windows / make_shifted_windows / build_freqs
// (src/awa_window.cpp:15-131) and the vidx/cumf host loops
// (src/awa_vk.cpp:73-88, src/awa_layer.cpp:110-141).  Integer work only,
// except the RoPE angle tables: angle = float(double(pos) * base[j]) exactly
// as awa_window.cpp:94-130 forms it, plus a (cos, sin) table per channel pair
// (64 pairs per row; pair 63 is the identity for the unrotated channels
// 126-127) that the pack kernel reads.
#include "awa_internal.hpp"

namespace awa {

namespace {

__device__ inline double angle_of(const GeomParams& p, int k, int tt, int ih, int iw) {
    // channel k of a video row at window-local position (tt, ih, iw)
    if (k < 42) return (double)tt * p.base[k >> 1];
    if (k < 84) return (double)ih * p.base[(k - 42) >> 1];
    return (double)iw * p.base[(k - 84) >> 1];
}

__global__ __launch_bounds__(256) void geom_build_kernel(GeomParams p, int32_t* __restrict__ slices,
                                                         int32_t* __restrict__ cumf,
                                                         int32_t* __restrict__ vidx,
                                                         float* __restrict__ vfreq,
                                                         float* __restrict__ tfreq,
                                                         float2* __restrict__ vcs,
                                                         float2* __restrict__ tcs) {
    __shared__ int s_st[3][MAX_AXIS];
    __shared__ int s_en[3][MAX_AXIS];
    __shared__ int s_cnt[3];
    __shared__ int s_cumf[MAX_WIN + 1];

    // Non-empty slices of each axis, in increasing index order
    // (awa_window.cpp:31-33 and :65-68 skip empty ones per axis).
    if (threadIdx.x < 3) {
        const Axis ax = p.ax[threadIdx.x];
        const int n = ax.count();
        int c = 0;
        for (int i = 0; i < n && c < MAX_AXIS; i++) {
            int s, e;
            ax.slice(i, &s, &e);
            if (e > s) {
                s_st[threadIdx.x][c] = s;
                s_en[threadIdx.x][c] = e;
                c++;
            }
        }
        s_cnt[threadIdx.x] = c;
    }
    __syncthreads();
    const int ct = s_cnt[0], ch = s_cnt[1], cw = s_cnt[2];
    int nwin = ct * ch * cw;
    if (nwin > p.nwin) nwin = p.nwin;  // the host plan sized every buffer
    // Window order: w outermost, then h, then t (awa_window.cpp:30-33),
    // i.e. wi = (iw * ch + ih) * ct + it.
    if (threadIdx.x == 0) {
        int acc = 0;
        s_cumf[0] = 0;
        for (int wi = 0; wi < nwin; wi++) {
            const int it = wi % ct, ih = (wi / ct) % ch, iw = wi / (ct * ch);
            acc += (s_en[0][it] - s_st[0][it]) * (s_en[1][ih] - s_st[1][ih]) *
                   (s_en[2][iw] - s_st[2][iw]);
            s_cumf[wi + 1] = acc;
        }
    }
    __syncthreads();

    const int gtid = blockIdx.x * blockDim.x + threadIdx.x;
    const int gstride = gridDim.x * blockDim.x;

    for (int wi = gtid; wi < nwin; wi += gstride) {
        const int it = wi % ct, ih = (wi / ct) % ch, iw = wi / (ct * ch);
        int32_t* s = slices + wi * 6;
        s[0] = s_st[0][it]; s[1] = s_en[0][it];
        s[2] = s_st[1][ih]; s[3] = s_en[1][ih];
        s[4] = s_st[2][iw]; s[5] = s_en[2][iw];
    }
    for (int i = gtid; i <= nwin; i += gstride) cumf[i] = s_cumf[i];

    const int total = s_cumf[nwin] < p.sumf ? s_cumf[nwin] : p.sumf;
    for (int g = gtid; g < total; g += gstride) {
        int lo = 0, hi = nwin;  // s_cumf[lo] <= g < s_cumf[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_cumf[mid] <= g) lo = mid; else hi = mid;
        }
        const int wi = lo;
        const int it = wi % ct, ih = (wi / ct) % ch, iw = wi / (ct * ch);
        const int dh = s_en[1][ih] - s_st[1][ih];
        const int dw = s_en[2][iw] - s_st[2][iw];
        const int local = g - s_cumf[wi];
        const int lw = local % dw;
        const int lh = (local / dw) % dh;
        const int lt = local / (dw * dh);
        vidx[g] = ((s_st[0][it] + lt) * p.h + s_st[1][ih] + lh) * p.w + s_st[2][iw] + lw;
        const int tt = p.txt_len + lt;  // time positions start after the text
        float* fr = vfreq + (size_t)g * ROPE_ROT;
        for (int k = 0; k < ROPE_ROT; k++) fr[k] = (float)angle_of(p, k, tt, lh, lw);
        float2* cs = vcs + (size_t)g * CS_STRIDE;
        for (int q = 0; q < NPAIR; q++) {
            float sn, cn;
            sincosf((float)angle_of(p, 2 * q, tt, lh, lw), &sn, &cn);
            cs[q] = make_float2(cn, sn);
        }
        cs[NPAIR] = make_float2(1.f, 0.f);  // channels 126, 127 pass through
    }
    // Text rows: 1-D position ii on every axis, same table in every window
    // (awa_window.cpp:120-130).
    const int trows = nwin * p.txt_len;
    for (int r = gtid; r < trows; r += gstride) {
        const int ii = r % p.txt_len;
        float* fr = tfreq + (size_t)r * ROPE_ROT;
        for (int k = 0; k < ROPE_ROT; k++) fr[k] = (float)((double)ii * p.base[(k % 42) >> 1]);
    }
    for (int r = gtid; r < p.txt_len; r += gstride) {
        float2* cs = tcs + (size_t)r * CS_STRIDE;
        for (int q = 0; q < NPAIR; q++) {
            float sn, cn;
            sincosf((float)((double)r * p.base[(2 * q % 42) >> 1]), &sn, &cn);
            cs[q] = make_float2(cn, sn);
        }
        cs[NPAIR] = make_float2(1.f, 0.f);
    }
}

// (cos, sin) of channel 2q of every row of injected frequency tables.
__global__ __launch_bounds__(256) void geom_tables_kernel(const float* __restrict__ vfreq,
                                                          const float* __restrict__ tfreq,
                                                          int sumf, int trows,
                                                          float2* __restrict__ vcs,
                                                          float2* __restrict__ tcs) {
    const int gtid = blockIdx.x * blockDim.x + threadIdx.x;
    const int gstride = gridDim.x * blockDim.x;
    const long nv = (long)sumf * CS_STRIDE, nt = (long)trows * CS_STRIDE;
    for (long i = gtid; i < nv + nt; i += gstride) {
        const bool txt = i >= nv;
        const long j = txt ? i - nv : i;
        const long row = j / CS_STRIDE, q = j % CS_STRIDE;
        float sn = 0.f, cn = 1.f;
        if (q < NPAIR)
            sincosf(txt ? tfreq[row * ROPE_ROT + 2 * q] : vfreq[row * ROPE_ROT + 2 * q], &sn, &cn);
        (txt ? tcs : vcs)[j] = make_float2(cn, sn);
    }
}

// The row table (layout and clamping in awa_internal.hpp): entry
// [tile][w][g][j] holds the element offset (index x 7680) of row 32 w + 4 j + g
// of the tile in vqkv (video tiles, through vidx) or tqkv.
__global__ __launch_bounds__(256) void vrow_kernel(const int32_t* __restrict__ cumf,
                                                   const int32_t* __restrict__ vidx,
                                                   const int32_t* __restrict__ tile_base,
                                                   const int32_t* __restrict__ tile_win, int n_vid_tiles,
                                                   int ntt, int txt_len, uint32_t* __restrict__ vrow) {
    const long n = (long)(n_vid_tiles + ntt) * TILE;
    for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (long)gridDim.x * blockDim.x) {
        const int tile = (int)(e / TILE), pos = (int)(e % TILE);
        const int R = 32 * (pos >> 5) + 4 * (pos & 7) + ((pos >> 3) & 3);
        int row;
        if (tile < n_vid_tiles) {
            const int w = tile_win[tile];
            const int f = cumf[w + 1] - cumf[w];
            row = vidx[cumf[w] + min((tile - tile_base[w]) * TILE + R, f - 1)];
        } else {
            row = min((tile - n_vid_tiles) * TILE + R, txt_len - 1);
        }
        vrow[e] = (uint32_t)row * (uint32_t)QKV;
    }
}

}  // namespace

hipError_t launch_vrow(const int32_t* cumf, const int32_t* vidx, const int32_t* tile_base,
                       const int32_t* tile_win, int n_vid_tiles, int ntt, int txt_len, uint32_t* vrow,
                       hipStream_t s) {
    const long n = (long)(n_vid_tiles + ntt) * TILE;
    long blocks = (n + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(vrow_kernel, dim3((unsigned)blocks), dim3(256), 0, s, cumf, vidx, tile_base, tile_win,
                       n_vid_tiles, ntt, txt_len, vrow);
    return hipGetLastError();
}

hipError_t launch_geom_build(const GeomParams& p, awa_geom* g, hipStream_t s) {
    int rows = p.sumf > p.nwin * p.txt_len ? p.sumf : p.nwin * p.txt_len;
    int blocks = (rows + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(geom_build_kernel, dim3(blocks), dim3(256), 0, s, p, g->d_slices, g->d_cumf,
                       g->d_vidx, g->d_vfreq, g->d_tfreq, g->d_vcs, g->d_tcs);
    return hipGetLastError();
}

hipError_t launch_geom_tables(const float* vfreq, const float* tfreq, int sumf, int trows,
                              float2* vcs, float2* tcs, hipStream_t s) {
    long n = (long)(sumf + trows) * CS_STRIDE;
    long blocks = (n + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(geom_tables_kernel, dim3((unsigned)blocks), dim3(256), 0, s, vfreq, tfreq,
                       sumf, trows, vcs, tcs);
    return hipGetLastError();
}

}  // namespace awa

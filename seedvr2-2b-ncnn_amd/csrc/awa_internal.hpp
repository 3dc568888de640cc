// awa_internal.hpp — shared definitions of the gfx950 AWA implementation.
//
// Packed attention layout (built by the pack kernel, read by the SDPA kernel):
// every window's video rows are cut into 64-row "tiles"; the text rows form
// ceil(TXT/64) further tiles, stored once when every window uses the same text
// RoPE table (always true for make_win geometry) or once per window otherwise.
// Per head h and tile k the packed buffers hold
//   Qp[h][k][slot 0..63][d 0..127]   normalised + rotated queries
//   Kp[h][k][slot 0..63][d 0..127]   normalised + rotated keys
//   Vp[h][k][d 0..127][slot 0..63]   values, transposed inside the tile (fp32 only)
// in the storage type of the op (bf16 or fp32).  Unused slots are zero.
// Queries carry the softmax scale times log2(e), so scores come out in log2
// units.  The bf16 attention kernel reads V from vqkv / tqkv itself, through
// the geometry's row table (awa_geom::d_vrow).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "awa_capi.h"

namespace awa {

constexpr int HEADS = 20, HEAD_D = 128, DIM = 2560, QKV = 7680;
constexpr int ROPE_ROT = 126, NPAIR = 63;
constexpr int CS_STRIDE = 64;      // (cos, sin) pairs per row of the RoPE tables; pair 63 is (1, 0)
constexpr int TILE = 64;           // rows per packed tile
constexpr int MAX_AXIS = 256;      // slices per axis accepted by the geometry kernel
constexpr int MAX_WIN = 4096;      // windows accepted by the geometry kernel

// Block index -> work index such that the hardware's round-robin dispatch of
// consecutive blocks over the 8 XCDs hands each XCD one contiguous range of
// work indices (and so one L2 for the data neighbouring indices share).  The
// grid must be a multiple of 8; indices >= nblk are idle.
__device__ inline int xcd_remap(int nblk) {
    const int per = (nblk + 7) >> 3;
    return (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
}
inline unsigned xcd_grid(long nblk) { return (unsigned)(((nblk + 7) >> 3) << 3); }

// fp32 -> bf16 bits, round to nearest even (cast_f32_bf16.comp:24)
__device__ inline uint32_t bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
// Two floats -> two bf16 in one word (lo in the low half) by the hardware
// conversion (one v_cvt_pk_bf16_f32 where bf16_rne takes four instructions per
// value).  Equal to bf16_rne on every finite value: awa_cast_f32_to_bf16 uses
// it and is checked against torch's cast on all finite patterns and against
// the integer formula on a sample (NaNs stay NaNs here, which the formula can
// turn into infinities).
__device__ inline uint32_t bf16x2_rne(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// Integer restatement of awa_window.cpp:15-78 along one axis.  The reference
// forms shifted bounds as int((i - 0.5) * wX) in double; for integer i and wX
// that product is an exact half-integer, so C's truncating integer division
// of (2i - 1) * wX by 2 is identical.  Likewise ceil((X - 0.5) / wX) equals
// ceil((2X - 1) / (2 wX)) because the quotient can never be an integer.
struct Axis {
    int X;        // extent of the axis
    int wX;       // window size along the axis
    int shift;    // 1: half-window shift (shifted variant and wX < X)
    int shifted_variant;

    __host__ __device__ int count() const {
        if (!shifted_variant) return (X + wX - 1) / wX;
        if (!shift) return 1;
        int num = 2 * X - 1, den = 2 * wX;
        return (num + den - 1) / den + 1;
    }
    __host__ __device__ void slice(int i, int* s, int* e) const {
        if (!shifted_variant) {
            *s = i * wX;
            *e = (i + 1) * wX < X ? (i + 1) * wX : X;
        } else if (!shift) {
            *s = 0;
            *e = wX < X ? wX : X;
        } else {
            int a = ((2 * i - 1) * wX) / 2;  // truncates toward zero like int()
            int b = ((2 * i + 1) * wX) / 2;
            *s = a > 0 ? a : 0;
            *e = b < X ? b : X;
        }
    }
};

struct GeomParams {
    Axis ax[3];            // t, h, w
    int t, h, w;
    int txt_len;
    int nwin, sumf;
    double base[21];       // 1 / 10000^(2j/42), computed on the host in double
};

// Host plan: sizes, tiles and attention work items.
struct GeomPlan {
    int t = 0, h = 0, w = 0, txt_len = 0, nwin = 0, sumf = 0, Lv = 0, max_S = 0;
    int txt_sets = 1;      // 1: text rows shared by all windows, else nwin
    int ntt = 0;           // text tiles per set
    int n_vid_tiles = 0, n_tiles = 0, n_items = 0;
    bool covers_all = true;  // vidx is a permutation of [0, Lv)
    std::vector<int32_t> slices;     // nwin*6
    std::vector<int32_t> cumf;       // nwin+1
    std::vector<int32_t> tile_base;  // nwin+1, first video tile of window w
    std::vector<int32_t> tile_win;   // n_vid_tiles, window of each video tile
    std::vector<int32_t> tile_meta;  // n_tiles*2: RoPE-table row of slot 0, valid rows
    std::vector<int32_t> items;      // n_items*4: window, first q tile, second q tile (-1), 0
    // Work units of the fp32 attention kernel (one workgroup per unit and
    // head): 2 item + query tile of the item, units of windows with more key
    // tiles first (workgroups are dispatched in index order, and window sizes
    // can differ several-fold: the longest must start first).
    std::vector<int32_t> f32_units;
    // Persistent schedule of the bf16 attention kernel: one workgroup per
    // resident slot (two per CU); slot s runs on XCD s % 8 and processes the
    // work items sched_start[s] .. sched_start[s+1]) of sched_desc, longest
    // first.  Each item is two int4: {head | window << 8, first query tile,
    // second query tile (-1: none), cumf[window]}, {first video tile of the
    // window, its video tile count, its first text tile, its token count}.
    int n_slots = 0;
    std::vector<int32_t> sched_start;  // n_slots+1
    std::vector<int32_t> sched_desc;   // 8 per item, n_items*HEADS items
};
// Host planning (awa_capi.cpp): the tiles and work items of a geometry with
// nwin, cumf, txt_len and txt_sets set, then the attention kernel's
// schedule over n_slots workgroups (a multiple of 8 is used).
void plan_tiles(GeomPlan& P);
void plan_schedule(GeomPlan& P, int n_slots);
// Row table (awa_geom::d_vrow): per row tile (the video tiles, then ntt
// text tiles shared by all windows) the element offsets (row index x 7680) of
// its 64 rows in vqkv (video, through vidx) or tqkv (text); rows past the end
// of a window or of the text repeat its last row.  Stored so that the lane of the bf16
// attention kernel that fetches row 32 w + 4 j + g of a tile (w: wave,
// g = lane / 16) finds its eight rows at [tile][w][g][j]; vrow_pos gives the
// position of row r.  The offsets are 32-bit (VROW_MAX_OFFSET_ROWS rows),
// and so are the bf16 attention kernel's byte offsets (twice them), which
// bounds the rows of the bf16 path (VROW_MAX_ROWS).
constexpr long VROW_MAX_OFFSET_ROWS = 0xffffffffL / QKV;
constexpr long VROW_MAX_ROWS = 0xffffffffL / (2L * QKV);
__host__ __device__ inline int vrow_pos(int r) { return 32 * (r >> 5) + 8 * (r & 3) + ((r & 31) >> 2); }

// The key tiles of the bf16 attention kernel's DMA stream.  A slot's stream
// is the key tiles of its work items in order: a window's nvt video tiles,
// then the ntt text tiles.  Tile kk of an item fetches K tile kk + 2 and V
// tile kk + 1 of the stream, so past the item's end the next item's first
// two tiles; for that every item must hold at least two tiles.  A window
// without video rows and at most 64 text rows (possible for injected
// geometry) has one: it gets a second that repeats its last text tile, whose
// keys all lie past the text and are masked.
__host__ __device__ inline int stream_tiles(int nvt, int ntt) { return nvt + ntt > 2 ? nvt + ntt : 2; }
// Tile index of key tile kk (< stream_tiles) of an item: video tiles from
// vbase, text tiles from tbase (packed K: the window's text set; V row
// table: n_vid_tiles), clamped to the last text tile.
__host__ __device__ inline int stream_tile(int kk, int nvt, int vbase, int tbase, int ntt) {
    return kk < nvt ? vbase + kk : tbase + (kk - nvt < ntt - 1 ? kk - nvt : ntt - 1);
}
// The fetch of key tile kk of an item with nk stream tiles: K tile k_kk and
// V tile v_kk of the current item (*_nxt = 0) or of the next one (*_nxt = 1).
__host__ __device__ inline void stream_fetch(int kk, int nk, int* k_kk, int* k_nxt, int* v_kk, int* v_nxt) {
    *k_nxt = kk + 2 >= nk;
    *k_kk = *k_nxt ? kk + 2 - nk : kk + 2;
    *v_nxt = kk + 1 >= nk;
    *v_kk = *v_nxt ? kk + 1 - nk : kk + 1;
}

}  // namespace awa

struct awa_ctx {
    int device = 0;
    std::string err;
    hipError_t noalloc_status = hipSuccess;  // lookup of the allocation-free entry's scratch
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    // Per-phase timing (awa_timing_enable): 4 events per recorded call,
    // bracketing pack, attention and text average on the call's stream.
    bool timing = false;
    std::vector<hipEvent_t> ev_free;
    std::vector<hipEvent_t> ev_used;      // awa_forward: 4 per call
    std::vector<hipEvent_t> dit_ev_used;  // dit_layer_forward: 7 per layer
    // DiT block workspace (activations between the projections) and a small
    // buffer for the timestep MLP.
    void* ws = nullptr;
    size_t ws_bytes = 0;
    float* small = nullptr;
    float* emb = nullptr;  // dit_forward_grid: the timestep embedding [15360]
};

struct awa_geom {
    int device = 0;
    bool injected = false;
    awa::GeomPlan plan;
    int32_t* d_slices = nullptr;
    int32_t* d_cumf = nullptr;
    int32_t* d_vidx = nullptr;
    int32_t* d_tile_base = nullptr;
    int32_t* d_tile_win = nullptr;
    int32_t* d_items = nullptr;
    int32_t* d_f32_units = nullptr;  // GeomPlan::f32_units
    int32_t* d_sched_start = nullptr;
    int32_t* d_sched_desc = nullptr;
    float* d_vfreq = nullptr;
    float* d_tfreq = nullptr;
    float2* d_vcs = nullptr;   // [sumf][64] (cos, sin) per channel pair, pair 63 = (1, 0)
    float2* d_tcs = nullptr;   // [txt_sets*txt_len][64]
    int32_t* d_tile_meta = nullptr;  // GeomPlan::tile_meta
    uint32_t* d_vrow = nullptr;      // [n_vid_tiles + ntt][64] row table (layout above)
};

namespace awa {

// Host helpers shared by the C ABI translation units (awa_capi.cpp).
void set_err(awa_ctx* ctx, const char* fmt, ...);
struct DeviceGuard {
    int prev = -1;
    bool ok = false;
    explicit DeviceGuard(int dev);
    ~DeviceGuard();
};
// Grows a device buffer (freeing the old one, which waits for its users).
hipError_t ensure_buffer(void** buf, size_t* have, size_t need);
hipError_t event_mark(awa_ctx* ctx, std::vector<hipEvent_t>& list, hipStream_t s);
// Argument checks of awa_forward (and its allocation-free variant); who
// names the entry point in the error message.
int check_forward_args(const char* who, awa_ctx* ctx, const awa_geom* g, int dtype,
                       const void* d_vqkv, const void* d_tqkv, int Lv, int TXT, const float* d_nq_v,
                       const float* d_nk_v, const float* d_nq_t, const float* d_nk_t, float eps,
                       const void* d_vattn, const void* d_tattn);
// Bytes of scratch the op needs for a geometry and storage type: packed Q, K
// and V tiles, then the per-window text partials, each 256-byte aligned.
size_t op_scratch_bytes(const GeomPlan& P, int dtype);
// awa_forward without argument checks (shared with the block).  ext_scratch:
// nullptr uses the context's scratch (grown on demand, per-phase events when
// timing is on); otherwise a caller-provided device buffer of at least
// op_scratch_bytes, and nothing is allocated or recorded.
// reps > 0 (with phase_ms[3]): after the op, each of its three kernels (pack,
// attention, text average) is launched reps more times back to back between
// two events (the same inputs, so the same outputs), and phase_ms receives
// the mean time per launch of each.
int forward_impl(awa_ctx* ctx, const awa_geom* g, int dtype, const void* d_vqkv, const void* d_tqkv,
                 const float* d_nq_v, const float* d_nk_v, const float* d_nq_t, const float* d_nk_t,
                 float eps, void* d_vattn, void* d_tattn, hipStream_t s, void* ext_scratch = nullptr,
                 int reps = 0, double* phase_ms = nullptr);
// The allocation-free entry's per-device scratch (awa_noalloc.hip):
// noalloc_resolve looks up the device address of the current device's copy
// (call with that device current); noalloc_scratch returns it, or nullptr.
hipError_t noalloc_resolve(int device);
void* noalloc_scratch(int device);

// Kernel launchers (defined in the .hip files).
hipError_t launch_geom_build(const GeomParams& p, awa_geom* g, hipStream_t s);
hipError_t launch_geom_tables(const float* vfreq, const float* tfreq, int sumf, int trows,
                              float2* vcs, float2* tcs, hipStream_t s);
hipError_t launch_vrow(const int32_t* cumf, const int32_t* vidx, const int32_t* tile_base,
                       const int32_t* tile_win, int n_vid_tiles, int ntt, int txt_len, uint32_t* vrow,
                       hipStream_t s);

struct PackArgs {
    const void* vqkv;
    const void* tqkv;
    const float* nq_v;
    const float* nk_v;
    const float* nq_t;
    const float* nk_t;
    const int32_t* tile_meta;  // GeomPlan::tile_meta
    const uint32_t* vrow;      // row table
    const float2* vcs;
    const float2* tcs;
    void* Qp;
    void* Kp;
    void* Vp;              // fp32 storage only (the bf16 attention reads V from vqkv / tqkv)
    int n_vid_tiles, ntt, txt_sets, txt_len, n_tiles;
    float eps;
    float qscale;          // folded into Q: softmax scale 1/sqrt(128) times log2(e)
};
hipError_t launch_pack(int dtype, const PackArgs& a, hipStream_t s);

struct SdpaArgs {
    const void* Qp;
    const void* Kp;
    const void* Vp;              // fp32 kernel
    const uint32_t* vrow;        // bf16 kernel: V row table of the geometry
    const void* vsrc;            // bf16 kernel: vqkv and tqkv, whose V columns it reads
    const void* tsrc;
    uint32_t vsrc_bytes, tsrc_bytes;
    const int32_t* items;
    const int32_t* cumf;
    const int32_t* vidx;
    const int32_t* tile_base;
    const int32_t* sched_start;  // bf16 kernel: persistent schedule (GeomPlan)
    const int32_t* sched_desc;
    int n_slots;
    void* vattn;
    uint32_t vattn_bytes;  // bf16 kernel: size of vattn (buffer stores drop beyond it)
    float* tpart;          // [nwin][txt_len][2560] fp32 text partials
    int n_vid_tiles, ntt, txt_sets, txt_len, n_tiles, n_items, nwin;
    float scale_log2e;     // multiplier of the scores (1 when Q carries the scale)
    const int32_t* f32_units;  // fp32 kernel: GeomPlan::f32_units
    int n_f32_units;
};
hipError_t launch_sdpa(int dtype, const SdpaArgs& a, hipStream_t s);
hipError_t launch_sdpa_f32(const SdpaArgs& a, hipStream_t s);   // awa_sdpa_f32.hip

hipError_t launch_coalesce(int dtype, const float* tpart, void* tattn, int nwin, int txt_len,
                           hipStream_t s);
hipError_t launch_cast_f32_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t s);
hipError_t launch_cast_bf16_f32(const uint16_t* in, float* out, int64_t n, hipStream_t s);
hipError_t launch_zero(void* p, size_t bytes, hipStream_t s);
hipError_t launch_stream_copy(void* dst, const void* src, size_t bytes, hipStream_t s);

}  // namespace awa

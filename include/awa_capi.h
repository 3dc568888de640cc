/*
 * awa_capi.h — C ABI of the MI355X (gfx950) SeedVR2 Adaptive Window Attention.
 *
 * Drop-in for the reference's AWA operator surfaces:
 *   - the ncnn custom layer AwaLayer (src/awa_layer.h:26-108,
 *     src/awa_layer.cpp:29-453): per-block qk-norm gains, host-injected
 *     window geometry, vqkv/tqkv in, vattn/tattn out, fp32 or bf16 storage;
 *   - the host-vector module AwaVk (src/awa_vk.h:14-52, awa_vk.cpp:62-199);
 *   - the window builder awa::make_win (src/awa_window.h:26,
 *     awa_window.cpp:133-150) plus the vidx/cumf index build
 *     (awa_vk.cpp:73-88, awa_layer.cpp:110-141).
 *   - the block-level DitVk::awa_forward / forward_latent layer
 *     (src/dit_vk.h:83-92, dit_vk.cpp:312-632), see dit_capi.h.
 *
 * Conventions
 *   - Plain pointers and sizes only.  Device pointers ("d_") live on the
 *     context's HIP device; host pointers ("h_") are ordinary memory.
 *   - Row-major layouts of the reference: vqkv [Lv][7680], tqkv [TXT][7680]
 *     with each row q|k|v and head h at column h*128 of each part; vattn
 *     [Lv][2560]; tattn [TXT][2560].
 *   - Device-pointer calls are stream-ordered and asynchronous: they enqueue on
 *     `stream` and return without a host synchronisation.  Host-pointer calls
 *     (awa_forward_host, awa_geom_read) are synchronous.
 *   - Return codes follow the reference's 0 / -1 convention
 *     (awa_layer.cpp:288,304,316): 0 ok, AWA_EARG (-1) bad argument, shape or
 *     geometry, AWA_EHIP (-2) a HIP runtime error.  The message of the last
 *     failure is available from awa_last_error().
 *   - Thread-compatible, not thread-safe: use one context per host thread and
 *     stream (the reference layer is single-threaded too, awa_layer.h:86-107).
 *     Calls on one context must not overlap in time on different streams,
 *     because they share the context's scratch buffers.
 */
#ifndef SEEDVR2_AWA_CAPI_H
#define SEEDVR2_AWA_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct awa_ctx awa_ctx;
typedef struct awa_geom awa_geom;
/* hipStream_t without requiring the HIP headers; NULL = the null stream. */
typedef struct ihipStream_t* awa_stream_t;

enum { AWA_OK = 0, AWA_EARG = -1, AWA_EHIP = -2 };
/* Storage type of vqkv/tqkv/vattn/tattn.  Arithmetic is fp32 accumulation in
 * both cases; AWA_BF16 feeds bf16 MFMA, AWA_F32 fp32 MFMA. */
enum { AWA_F32 = 0, AWA_BF16 = 1 };

enum { AWA_HEADS = 20, AWA_HEAD_D = 128, AWA_DIM = 2560, AWA_QKV = 7680,
       AWA_ROPE_ROT = 126 };

/* Context: owns the scratch (packed q/k/v tiles, per-window text partials),
 * grown on demand and reused.  Replaces AwaVk::init / AwaLayer::create_pipeline
 * (awa_vk.cpp:33-60, awa_layer.cpp:143-242). */
int awa_create(awa_ctx** out, int hip_device);
void awa_destroy(awa_ctx* ctx);
const char* awa_last_error(const awa_ctx* ctx);

/* Geometry summary (host-readable). */
typedef struct {
    int32_t t, h, w;         /* token grid (0 for injected geometry)        */
    int32_t nwin;            /* windows                                      */
    int32_t sumf;            /* video rows over all windows                  */
    int32_t Lv;              /* video tokens                                 */
    int32_t txt_len;         /* text tokens appended to every window         */
    int32_t max_S;           /* largest window sequence f + txt_len          */
    int32_t n_tiles;         /* 64-row key tiles of the packed layout        */
    int32_t n_items;         /* attention work items per head                */
} awa_geom_info;

/* Host-only window planner, the slice part of awa::make_windows /
 * make_shifted_windows (awa_window.cpp:15-78) restated in integers: writes up
 * to cap windows as [st,en,sh,eh,sw,ew] and returns the window count, or
 * AWA_EARG.  Touches no device; the device builder below uses the same
 * formulas. */
int awa_plan_windows(int t, int h, int w, const int32_t num_windows[3], int shifted,
                     int32_t* h_slices, int cap);

/* awa::make_win(t, h, w, num_windows, txt_len, shifted) followed by the index
 * build, on the device: window slices (unshifted or half-window shifted),
 * cumf, vidx and the RoPE frequency tables in the reference's formats.
 * Built once per resolution and reused (dit_graph.cpp:226-229 caches it).
 * Every geometry entry point rejects (AWA_EARG) more than 559,240 video or
 * text rows: the geometry's row table holds 32-bit element offsets into the
 * 7680-wide projection rows (the bf16 op further accepts at most 279,620). */
int awa_geom_build(awa_ctx* ctx, int t, int h, int w, const int32_t num_windows[3],
                   int txt_len, int shifted, awa_geom** out, awa_stream_t stream);

/* AwaLayer::set_window_geometry(vidx, cumf, vfreq, tfreq, nwin, Lv, TXT)
 * (awa_layer.cpp:73-91): host arrays in the reference's float encoding
 * (vidx/cumf as floats read with int(x+0.5), awa.comp:88,101).  vfreq is
 * [sumf][126], tfreq [nwin*txt_len][126], sumf = vidx length = cumf[nwin].
 * Rejected (AWA_EARG): vidx entries outside [0,Lv) or repeated, cumf not
 * non-decreasing from 0, frequency rows whose channel pairs (2i,2i+1) differ
 * (make_win always repeats them, awa_window.cpp:108-112). */
int awa_geom_set(awa_ctx* ctx, const float* h_vidx, const float* h_cumf,
                 const float* h_vfreq, const float* h_tfreq, int nwin, int Lv,
                 int txt_len, awa_geom** out, awa_stream_t stream);

/* The geometry of a reference struct Win (dit_vk.h:17-22), as awa::make_win
 * returns it (awa_window.cpp:133-150) or load_win reads a win_*.bin file
 * (dit_vk.cpp:74-93): grid t, h, w; nwin windows with slices
 * [st,en,sh,eh,sw,ew] (h_slices, nwin x 6); vid_freq [sumf][126] in window
 * order; txt_freq [nwin*txt_len][126].  The index is built on the host as
 * AwaVk::forward and AwaLayer::build_window_geometry build it
 * (awa_vk.cpp:73-88, awa_layer.cpp:110-141): windows in order, a window's
 * tokens in (t, h, w) C order, sumf = the windows' token count, Lv = t*h*w.
 * Rejected (AWA_EARG): slices outside the grid, a token in two windows,
 * frequency rows whose channel pairs differ. */
int awa_geom_from_win(awa_ctx* ctx, int t, int h, int w, int nwin, const int32_t* h_slices,
                      const float* h_vid_freq, const float* h_txt_freq, int txt_len,
                      awa_geom** out, awa_stream_t stream);

int awa_geom_query(const awa_geom* g, awa_geom_info* info);

/* Synchronous copies of the device geometry for inspection; any output may be
 * NULL.  slices [nwin][6] (st,en,sh,eh,sw,ew; zeros for injected geometry),
 * cumf [nwin+1], vidx [sumf], vfreq [sumf][126], tfreq [nwin*txt_len][126]. */
int awa_geom_read(awa_ctx* ctx, const awa_geom* g, int32_t* h_slices, int32_t* h_cumf,
                  int32_t* h_vidx, float* h_vfreq, float* h_tfreq);

void awa_geom_destroy(awa_geom* g);

/* Sizes the context's scratch for awa_forward on geometry g in storage dtype,
 * so that a later call at that geometry allocates nothing (a caller capturing
 * awa_forward into a graph; awa_geom_build already reserves the bf16 size).
 * No counterpart in the reference: AwaLayer allocates its buffers in
 * create_pipeline (awa_layer.cpp:143-255), for one fixed shape. */
int awa_reserve(awa_ctx* ctx, const awa_geom* g, int dtype);

/* The AWA op, AwaLayer::forward (awa_layer.cpp:284-453): per-head qk RMSNorm
 * (gains shared across heads, eps), 3-D RoPE on 126 channels, window SDPA
 * with the text rows appended to every window, text outputs averaged over the
 * windows in window order, video rows scattered back to token order.
 *   dtype     AWA_F32 or AWA_BF16 storage for d_vqkv, d_tqkv, d_vattn, d_tattn
 *   Lv, TXT   must equal the geometry's Lv and txt_len
 *   d_nq_v .. d_nk_t  fp32 [128] device vectors
 * Tokens outside every window get zero rows, as the reference's zero-fill
 * (awa_layer.cpp:386-399). */
int awa_forward(awa_ctx* ctx, const awa_geom* g, int dtype, const void* d_vqkv,
                const void* d_tqkv, int Lv, int TXT, const float* d_nq_v,
                const float* d_nk_v, const float* d_nq_t, const float* d_nk_t,
                float eps, void* d_vattn, void* d_tattn, awa_stream_t stream);

/* awa_forward without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as awa_forward; the scratch is a fixed
 * device array of AWA_NOALLOC_SCRATCH_MIB MiB that the library holds on every
 * device it runs on until the process ends (awa_create looks up its address).
 * Geometries whose scratch exceeds it are rejected with AWA_EARG (1080p bf16
 * needs 76 MiB, the 71 x 97 grid with 77 text rows 104 MiB; fp32 storage
 * also packs V and needs about 2.6 times as much).  No per-phase timing events
 * are recorded.  All calls on one device share the array: calls that overlap
 * in time on one device race. */
enum { AWA_NOALLOC_SCRATCH_MIB = 128 };
int awa_forward_noalloc(awa_ctx* ctx, const awa_geom* g, int dtype, const void* d_vqkv,
                        const void* d_tqkv, int Lv, int TXT, const float* d_nq_v,
                        const float* d_nk_v, const float* d_nq_t, const float* d_nk_t, float eps,
                        void* d_vattn, void* d_tattn, awa_stream_t stream);

/* AwaVk::forward (awa_vk.cpp:62-199): fp32 host vectors in and out, computed
 * on the device, synchronous.  Returns 0 / error code instead of bool. */
int awa_forward_host(awa_ctx* ctx, const awa_geom* g, const float* h_vqkv,
                     const float* h_tqkv, int Lv, int TXT, const float* h_nq_v,
                     const float* h_nk_v, const float* h_nq_t, const float* h_nk_t,
                     float eps, float* h_vid_out, float* h_txt_out);

/* Per-phase device timing, the MI355X counterpart of the reference's
 * [perf] accumulators (dit_vk.cpp:23-24, 332-334) at kernel granularity.
 * While enabled, every awa_forward records HIP events on its stream around
 * the pack (qk-norm + RoPE + partition), attention and text-average kernels.
 * awa_timing_read waits for the recorded events, returns the summed
 * milliseconds of each phase and the number of calls, and clears them. */
int awa_timing_enable(awa_ctx* ctx, int enable);
/* awa_forward, then each of its three kernels (pack, attention, text
 * average) launched `reps` more times back to back on `stream` between two
 * events (same inputs, same outputs); ms_per_launch[0..2] receive the mean
 * per launch of each and the call returns after the last one.  No
 * counterpart in the reference: it times the kernels without the per-phase
 * events of awa_timing_enable between launches (the roofline figures of
 * bench.py). */
int awa_time_phases(awa_ctx* ctx, const awa_geom* g, int dtype, const void* d_vqkv, const void* d_tqkv,
                    int Lv, int TXT, const float* d_nq_v, const float* d_nk_v, const float* d_nq_t,
                    const float* d_nk_t, float eps, void* d_vattn, void* d_tattn, int reps,
                    double ms_per_launch[3], awa_stream_t stream);
int awa_timing_read(awa_ctx* ctx, double* ms_pack, double* ms_attn, double* ms_text, int* calls);

/* Casts at the bf16 boundary (cast_f32_bf16.comp:23-24, round to nearest
 * even; cast_bf16_f32.comp:18-19, exact widening).  n elements. */
int awa_cast_f32_to_bf16(awa_ctx* ctx, const float* d_in, uint16_t* d_out, int64_t n,
                         awa_stream_t stream);
int awa_cast_bf16_to_f32(awa_ctx* ctx, const uint16_t* d_in, float* d_out, int64_t n,
                         awa_stream_t stream);

/* Streaming device copy of `bytes` (a multiple of 16) from d_src to d_dst.
 * No counterpart in the reference: it is the measuring stick for the
 * HBM-bound passes (the fastest hand-written copy of those measured on the
 * MI355X, timed beside them by bench.py and used to calibrate the HBM byte
 * counters). */
int awa_stream_copy(awa_ctx* ctx, void* d_dst, const void* d_src, int64_t bytes, awa_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif

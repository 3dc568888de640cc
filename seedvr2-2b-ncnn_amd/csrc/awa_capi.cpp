// awa_capi.cpp — C ABI of the AWA op: contexts, geometry, forward.
//
// Host C++17.  Computes the geometry plan (window sizes, 64-row tiles, work
// items) with the same integer formulas the device kernel uses, owns the
// device buffers, and enqueues pack -> SDPA -> coalesce on the caller's
// stream without synchronising.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <map>
#include <vector>

#include "awa_internal.hpp"

using namespace awa;

namespace awa {

void set_err(awa_ctx* ctx, const char* fmt, ...) {
    if (!ctx) return;
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    ctx->err = buf;
}

// Makes the given device current for the scope and restores the caller's.
DeviceGuard::DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    ok = (prev == dev) || (hipSetDevice(dev) == hipSuccess);
}
DeviceGuard::~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
}

hipError_t ensure_buffer(void** buf, size_t* have, size_t need) {
    if (*have >= need) return hipSuccess;
    if (*buf) {
        hipError_t e = hipFree(*buf);
        *buf = nullptr;
        *have = 0;
        if (e != hipSuccess) return e;
    }
    hipError_t e = hipMalloc(buf, need);
    if (e == hipSuccess) *have = need;
    return e;
}

hipError_t event_mark(awa_ctx* ctx, std::vector<hipEvent_t>& list, hipStream_t s) {
    if (!ctx->timing) return hipSuccess;
    hipEvent_t e;
    if (!ctx->ev_free.empty()) {
        e = ctx->ev_free.back();
        ctx->ev_free.pop_back();
    } else {
        hipError_t r = hipEventCreate(&e);
        if (r != hipSuccess) return r;
    }
    list.push_back(e);
    return hipEventRecord(e, s);
}

}  // namespace awa

namespace {

#define HIPCK(ctx, expr)                                                                     \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess) {                                                              \
            set_err(ctx, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__,    \
                    __LINE__);                                                               \
            return AWA_EHIP;                                                                 \
        }                                                                                    \
    } while (0)

template <typename T>
hipError_t dalloc(T** p, size_t n) {
    *p = nullptr;
    if (n == 0) n = 1;
    return hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T));
}

void free_geom_buffers(awa_geom* g) {
    void* ptrs[] = {g->d_slices, g->d_cumf, g->d_vidx, g->d_tile_base, g->d_tile_win,
                    g->d_items, g->d_f32_units, g->d_sched_start, g->d_sched_desc, g->d_vfreq, g->d_tfreq,
                    g->d_vcs, g->d_tcs, g->d_tile_meta, g->d_vrow};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
}

}  // namespace

namespace awa {

// 64-row tiles of every window plus the text tiles, and the work items of the
// attention kernel (one window, two query tiles).
void plan_tiles(GeomPlan& P) {
    P.ntt = (P.txt_len + TILE - 1) / TILE;
    P.tile_base.assign(P.nwin + 1, 0);
    P.tile_win.clear();
    P.max_S = 0;
    for (int w = 0; w < P.nwin; w++) {
        const int f = P.cumf[w + 1] - P.cumf[w];
        const int nvt = (f + TILE - 1) / TILE;
        P.tile_base[w + 1] = P.tile_base[w] + nvt;
        for (int k = 0; k < nvt; k++) P.tile_win.push_back(w);
        if (f + P.txt_len > P.max_S) P.max_S = f + P.txt_len;
    }
    P.n_vid_tiles = P.tile_base[P.nwin];
    P.n_tiles = P.n_vid_tiles + P.txt_sets * P.ntt;
    P.tile_meta.clear();
    for (int w = 0; w < P.nwin; w++)
        for (int g0 = P.cumf[w]; g0 < P.cumf[w + 1]; g0 += TILE) {
            P.tile_meta.push_back(g0);
            P.tile_meta.push_back(std::min(TILE, P.cumf[w + 1] - g0));
        }
    for (int set = 0; set < P.txt_sets; set++)
        for (int j0 = 0; j0 < P.txt_len; j0 += TILE) {
            P.tile_meta.push_back(set * P.txt_len + j0);
            P.tile_meta.push_back(std::min(TILE, P.txt_len - j0));
        }
    P.items.clear();
    for (int w = 0; w < P.nwin; w++) {
        const int nq = (P.tile_base[w + 1] - P.tile_base[w]) + P.ntt;
        for (int q = 0; q < nq; q += 2) {
            P.items.push_back(w);
            P.items.push_back(q);
            P.items.push_back(q + 1 < nq ? q + 1 : -1);
            P.items.push_back(0);
        }
    }
    P.n_items = (int)P.items.size() / 4;
    // fp32 units: every query tile of every item, longest windows first
    std::vector<int> units;
    for (int i = 0; i < P.n_items; i++)
        for (int half = 0; half < 2; half++)
            if (P.items[4 * i + 1 + half] >= 0) units.push_back(2 * i + half);
    auto nkey = [&](int u) {
        const int w = P.items[4 * (u >> 1)];
        return P.tile_base[w + 1] - P.tile_base[w];
    };
    std::stable_sort(units.begin(), units.end(), [&](int x, int y) { return nkey(x) > nkey(y); });
    P.f32_units.assign(units.begin(), units.end());
}

// Static schedule of the persistent bf16 attention
// kernel over n_slots resident workgroups.  A work item costs about its
// window's key-tile count plus two and a half tiles of per-item work (first
// scores, the wait for the query tile, the epilogue), as timed per wave on
// 1080p layers.  All items of one (window, head) go to one XCD so that they
// share that window's K/V tiles through the XCD's L2; groups are spread over
// the XCDs longest first onto the least loaded XCD, then each XCD's items onto
// its slots the same way, or by first fit decreasing when that packs them
// under a smaller makespan.  Slot s is workgroup s, dispatched to XCD s % 8.
void plan_schedule(GeomPlan& P, int n_slots) {
    constexpr int XCDS = 8;
    n_slots = std::max(XCDS, n_slots - n_slots % XCDS);
    P.n_slots = n_slots;
    const int per_xcd = n_slots / XCDS;
    std::vector<int> win_cost(P.nwin);
    for (int w = 0; w < P.nwin; w++) win_cost[w] = 10 * stream_tiles(P.tile_base[w + 1] - P.tile_base[w], P.ntt) + 25;
    struct Group { long cost; int h, w; };
    std::vector<Group> groups;
    std::vector<std::vector<int>> items_of(P.nwin);
    for (int i = 0; i < P.n_items; i++) items_of[P.items[4 * i]].push_back(i);
    for (int h = 0; h < HEADS; h++)
        for (int w = 0; w < P.nwin; w++)
            groups.push_back({(long)win_cost[w] * (long)items_of[w].size(), h, w});
    std::stable_sort(groups.begin(), groups.end(), [](const Group& x, const Group& y) { return x.cost > y.cost; });
    std::vector<long> xload(XCDS, 0);
    std::vector<std::vector<int>> xwork(XCDS);  // work ids per XCD
    for (const Group& gr : groups) {
        const int x = (int)(std::min_element(xload.begin(), xload.end()) - xload.begin());
        xload[x] += gr.cost;
        for (int i : items_of[gr.w]) xwork[x].push_back(gr.h * P.n_items + i);
    }
    std::vector<std::vector<int>> slot_work(n_slots);
    auto cost = [&](int id) { return (long)win_cost[P.items[4 * (id % P.n_items)]]; };
    for (int x = 0; x < XCDS; x++) {
        auto& wl = xwork[x];
        std::stable_sort(wl.begin(), wl.end(), [&](int a, int b) { return cost(a) > cost(b); });
        // longest first onto the least loaded slot
        std::vector<std::vector<int>> best(per_xcd);
        std::vector<long> sload(per_xcd, 0);
        long total = 0, cmax = 0;
        for (int id : wl) {
            const int k = (int)(std::min_element(sload.begin(), sload.end()) - sload.begin());
            sload[k] += cost(id);
            best[k].push_back(id);
            total += cost(id);
            cmax = std::max(cmax, cost(id));
        }
        // first fit decreasing under the smallest capacity it packs, when
        // that beats the longest-first makespan (items come in a few sizes,
        // so the least-loaded rule often stacks two long items on a slot
        // that a packing avoids)
        auto ffd = [&](long cap, std::vector<std::vector<int>>* out) {
            std::vector<long> ld(per_xcd, 0);
            if (out) out->assign(per_xcd, {});
            for (int id : wl) {
                int k = 0;
                while (k < per_xcd && ld[k] + cost(id) > cap) k++;
                if (k == per_xcd) return false;
                ld[k] += cost(id);
                if (out) (*out)[k].push_back(id);
            }
            return true;
        };
        long lo = std::max(cmax, (total + per_xcd - 1) / per_xcd);
        long hi = *std::max_element(sload.begin(), sload.end());  // ffd(hi) need not hold
        if (lo < hi && ffd(hi - 1, nullptr)) {
            hi = hi - 1;
            while (lo < hi) {
                const long mid = (lo + hi) / 2;
                if (ffd(mid, nullptr)) hi = mid;
                else lo = mid + 1;
            }
            ffd(hi, &best);
            // The packing fixes each slot's sequence of item sizes; hand out
            // the items position by position over the slots (slots with equal
            // sequences adjacent), so that the items of one (window, head),
            // which have equal sizes and lie together in wl, run at the same
            // time on neighbouring slots and share the window's tiles in L2
            // rather than fetching them again at different times.
            std::vector<std::vector<long>> pat(per_xcd);
            size_t plen = 0;
            for (int k = 0; k < per_xcd; k++) {
                for (int id : best[k]) pat[k].push_back(cost(id));
                plen = std::max(plen, pat[k].size());
            }
            std::vector<int> order(per_xcd);
            for (int k = 0; k < per_xcd; k++) order[k] = k;
            std::stable_sort(order.begin(), order.end(), [&](int u, int v) { return pat[u] > pat[v]; });
            std::map<long, std::vector<int>> queue;  // size -> ids in wl order
            for (int id : wl) queue[cost(id)].push_back(id);
            std::map<long, size_t> next;
            for (int k = 0; k < per_xcd; k++) best[k].clear();
            for (size_t pos = 0; pos < plen; pos++)
                for (int k : order)
                    if (pos < pat[k].size()) {
                        const long c = pat[k][pos];
                        best[k].push_back(queue[c][next[c]++]);
                    }
        }
        for (int k = 0; k < per_xcd; k++)
            for (int id : best[k]) slot_work[x + XCDS * k].push_back(id);
    }
    P.sched_start.assign(n_slots + 1, 0);
    P.sched_desc.clear();
    int n = 0;
    for (int sl = 0; sl < n_slots; sl++) {
        for (int id : slot_work[sl]) {
            const int h = id / P.n_items, i = id % P.n_items, w = P.items[4 * i];
            const int32_t d[8] = {h | (w << 8), P.items[4 * i + 1], P.items[4 * i + 2], P.cumf[w],
                                  P.tile_base[w], P.tile_base[w + 1] - P.tile_base[w],
                                  P.n_vid_tiles + (P.txt_sets == 1 ? 0 : w) * P.ntt,
                                  P.cumf[w + 1] - P.cumf[w]};
            P.sched_desc.insert(P.sched_desc.end(), d, d + 8);
            n++;
        }
        P.sched_start[sl + 1] = n;
    }
}

}  // namespace awa

namespace {

int upload_plan(awa_ctx* ctx, awa_geom* g, hipStream_t s) {
    GeomPlan& P = g->plan;
    int n_cu = 0;
    HIPCK(ctx, hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, ctx->device));
    plan_schedule(P, 2 * n_cu);
    HIPCK(ctx, dalloc(&g->d_sched_start, P.sched_start.size()));
    HIPCK(ctx, dalloc(&g->d_sched_desc, P.sched_desc.size()));
    HIPCK(ctx, hipMemcpyAsync(g->d_sched_start, P.sched_start.data(), P.sched_start.size() * 4,
                              hipMemcpyHostToDevice, s));
    if (!P.sched_desc.empty())
        HIPCK(ctx, hipMemcpyAsync(g->d_sched_desc, P.sched_desc.data(), P.sched_desc.size() * 4,
                                  hipMemcpyHostToDevice, s));
    HIPCK(ctx, dalloc(&g->d_tile_base, P.tile_base.size()));
    HIPCK(ctx, dalloc(&g->d_tile_win, P.tile_win.size()));
    HIPCK(ctx, dalloc(&g->d_items, P.items.size()));
    HIPCK(ctx, dalloc(&g->d_f32_units, P.f32_units.size()));
    if (!P.f32_units.empty())
        HIPCK(ctx, hipMemcpyAsync(g->d_f32_units, P.f32_units.data(), P.f32_units.size() * 4,
                                  hipMemcpyHostToDevice, s));
    HIPCK(ctx, hipMemcpyAsync(g->d_tile_base, P.tile_base.data(), P.tile_base.size() * 4,
                              hipMemcpyHostToDevice, s));
    if (!P.tile_win.empty())
        HIPCK(ctx, hipMemcpyAsync(g->d_tile_win, P.tile_win.data(), P.tile_win.size() * 4,
                                  hipMemcpyHostToDevice, s));
    if (!P.items.empty())
        HIPCK(ctx, hipMemcpyAsync(g->d_items, P.items.data(), P.items.size() * 4,
                                  hipMemcpyHostToDevice, s));
    HIPCK(ctx, dalloc(&g->d_tile_meta, P.tile_meta.size()));
    HIPCK(ctx, hipMemcpyAsync(g->d_tile_meta, P.tile_meta.data(), P.tile_meta.size() * 4,
                              hipMemcpyHostToDevice, s));
    // the row table (needs d_cumf and d_vidx)
    if (P.Lv > VROW_MAX_OFFSET_ROWS || P.txt_len > VROW_MAX_OFFSET_ROWS) {
        set_err(ctx, "geometry: %d video / %d text rows exceed the row table's 32-bit offsets", P.Lv, P.txt_len);
        return AWA_EARG;
    }
    HIPCK(ctx, dalloc(&g->d_vrow, (size_t)(P.n_vid_tiles + P.ntt) * TILE));
    HIPCK(ctx, launch_vrow(g->d_cumf, g->d_vidx, g->d_tile_base, g->d_tile_win, P.n_vid_tiles, P.ntt,
                           P.txt_len, g->d_vrow, s));
    return AWA_OK;
}


// Window sizes (awa_window.cpp:21-26, in double as the reference) and the
// non-empty slices of each axis with the integer formulas of Axis.
struct AxisSlices {
    int cnt[3];
    std::vector<int> st[3], en[3];
};

int plan_axes(int t, int h, int w, const int32_t num_windows[3], int shifted, GeomParams& p,
              AxisSlices& out, awa_ctx* ctx) {
    if (t < 1 || h < 1 || w < 1 || num_windows[0] < 1 || num_windows[1] < 1 || num_windows[2] < 1) {
        set_err(ctx, "window plan: bad sizes t=%d h=%d w=%d nw=(%d,%d,%d)", t, h, w, num_windows[0],
                num_windows[1], num_windows[2]);
        return AWA_EARG;
    }
    if ((long)t * h * w > (1L << 24)) {
        set_err(ctx, "window plan: grid too large");
        return AWA_EARG;
    }
    const double scale = std::sqrt((45.0 * 80.0) / ((double)h * w));
    const int resized_h = (int)std::round(h * scale);
    const int resized_w = (int)std::round(w * scale);
    const int wh = (resized_h + num_windows[1] - 1) / num_windows[1];
    const int ww = (resized_w + num_windows[2] - 1) / num_windows[2];
    const int wt = ((t < 30 ? t : 30) + num_windows[0] - 1) / num_windows[0];
    const int ext[3] = {t, h, w}, win[3] = {wt, wh, ww};
    for (int a = 0; a < 3; a++) {
        if (win[a] < 1) {
            set_err(ctx, "window plan: empty window size on axis %d", a);
            return AWA_EARG;
        }
        p.ax[a].X = ext[a];
        p.ax[a].wX = win[a];
        p.ax[a].shifted_variant = shifted ? 1 : 0;
        p.ax[a].shift = (shifted && win[a] < ext[a]) ? 1 : 0;
        const int n = p.ax[a].count();
        out.st[a].clear();
        out.en[a].clear();
        for (int i = 0; i < n; i++) {
            int s0, e0;
            p.ax[a].slice(i, &s0, &e0);
            if (e0 > s0) {
                out.st[a].push_back(s0);
                out.en[a].push_back(e0);
            }
        }
        out.cnt[a] = (int)out.st[a].size();
        if (out.cnt[a] < 1 || out.cnt[a] > MAX_AXIS) {
            set_err(ctx, "window plan: %d windows on axis %d (limit %d)", out.cnt[a], a, MAX_AXIS);
            return AWA_EARG;
        }
    }
    const long nwin = (long)out.cnt[0] * out.cnt[1] * out.cnt[2];
    if (nwin > MAX_WIN) {
        set_err(ctx, "window plan: %ld windows (limit %d)", nwin, MAX_WIN);
        return AWA_EARG;
    }
    return AWA_OK;
}

size_t elem_size(int dtype) { return dtype == AWA_BF16 ? 2 : 4; }

int ensure_scratch(awa_ctx* ctx, size_t bytes) {
    HIPCK(ctx, ensure_buffer(&ctx->scratch, &ctx->scratch_bytes, bytes));
    return AWA_OK;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

hipError_t timing_mark(awa_ctx* ctx, hipStream_t s) { return event_mark(ctx, ctx->ev_used, s); }

}  // namespace

namespace awa {

size_t op_scratch_bytes(const GeomPlan& P, int dtype) {
    const size_t packed = (size_t)HEADS * P.n_tiles * TILE * HEAD_D * elem_size(dtype);
    const size_t n_packed = dtype == AWA_BF16 ? 2 : 3;  // Q, K (and V for fp32)
    return n_packed * align256(packed) + align256((size_t)P.nwin * P.txt_len * DIM * 4);
}

int forward_impl(awa_ctx* ctx, const awa_geom* g, int dtype, const void* d_vqkv, const void* d_tqkv,
                 const float* d_nq_v, const float* d_nk_v, const float* d_nq_t, const float* d_nk_t,
                 float eps, void* d_vattn, void* d_tattn, hipStream_t s, void* ext_scratch, int reps,
                 double* phase_ms) {
    const GeomPlan& P = g->plan;
    const int Lv = P.Lv;
    const size_t es = elem_size(dtype);
    const size_t packed = (size_t)HEADS * P.n_tiles * TILE * HEAD_D * es;
    const bool bf16 = dtype == AWA_BF16;
    const size_t off_k = align256(packed), off_v = 2 * off_k, off_t = (bf16 ? 2 : 3) * off_k;
    // the bf16 kernel addresses vattn with 32-bit buffer offsets (and marks
    // padding rows with offsets from 2^31), and vqkv / tqkv rows through the
    // geometry's 32-bit row table
    if (bf16 && ((size_t)Lv * DIM * es > 0x7fffffffu || Lv > VROW_MAX_ROWS || P.txt_len > VROW_MAX_ROWS)) {
        set_err(ctx, "awa_forward: Lv=%d video rows exceed the bf16 path's 32-bit addressing", Lv);
        return AWA_EARG;
    }
    char* base = static_cast<char*>(ext_scratch);
    if (!base) {
        int rc = ensure_scratch(ctx, op_scratch_bytes(P, dtype));
        if (rc != AWA_OK) return rc;
        base = static_cast<char*>(ctx->scratch);
    }
    // per-phase events only for the context's own scratch: creating events
    // may allocate, which the caller-provided scratch path must not
    auto mark = [&]() { return ext_scratch ? hipSuccess : timing_mark(ctx, s); };

    if (!P.covers_all) HIPCK(ctx, launch_zero(d_vattn, (size_t)Lv * DIM * es, s));
    HIPCK(ctx, mark());

    PackArgs pa{};
    pa.vqkv = d_vqkv; pa.tqkv = d_tqkv;
    pa.nq_v = d_nq_v; pa.nk_v = d_nk_v; pa.nq_t = d_nq_t; pa.nk_t = d_nk_t;
    pa.tile_meta = g->d_tile_meta; pa.vrow = g->d_vrow;
    pa.vcs = g->d_vcs; pa.tcs = g->d_tcs;
    pa.Qp = base; pa.Kp = base + off_k; pa.Vp = bf16 ? nullptr : base + off_v;
    pa.n_vid_tiles = P.n_vid_tiles; pa.ntt = P.ntt; pa.txt_sets = P.txt_sets; pa.txt_len = P.txt_len;
    pa.n_tiles = P.n_tiles; pa.eps = eps;
    pa.qscale = (1.0f / std::sqrt(128.0f)) * 1.4426950408889634f;
    HIPCK(ctx, launch_pack(dtype, pa, s));
    HIPCK(ctx, mark());

    SdpaArgs sa{};
    sa.Qp = pa.Qp; sa.Kp = pa.Kp; sa.Vp = pa.Vp;
    sa.vrow = g->d_vrow; sa.vsrc = d_vqkv; sa.tsrc = d_tqkv;
    sa.vsrc_bytes = (uint32_t)std::min<size_t>((size_t)Lv * QKV * es, 0xffffffffu);
    sa.tsrc_bytes = (uint32_t)std::min<size_t>((size_t)P.txt_len * QKV * es, 0xffffffffu);
    sa.items = g->d_items; sa.cumf = g->d_cumf; sa.vidx = g->d_vidx; sa.tile_base = g->d_tile_base;
    sa.sched_start = g->d_sched_start; sa.sched_desc = g->d_sched_desc; sa.n_slots = P.n_slots;
    sa.vattn = d_vattn; sa.vattn_bytes = (uint32_t)((size_t)Lv * DIM * es);
    sa.tpart = reinterpret_cast<float*>(base + off_t);
    sa.n_vid_tiles = P.n_vid_tiles; sa.ntt = P.ntt; sa.txt_sets = P.txt_sets; sa.txt_len = P.txt_len;
    sa.n_tiles = P.n_tiles; sa.n_items = P.n_items; sa.nwin = P.nwin;
    sa.scale_log2e = 1.0f;  // the pack kernel folded the scale into Q
    sa.f32_units = g->d_f32_units; sa.n_f32_units = (int)P.f32_units.size();
    HIPCK(ctx, launch_sdpa(dtype, sa, s));
    HIPCK(ctx, mark());

    HIPCK(ctx, launch_coalesce(dtype, sa.tpart, d_tattn, P.nwin, P.txt_len, s));
    HIPCK(ctx, mark());
    if (reps > 0 && phase_ms) {
        hipEvent_t e[2] = {nullptr, nullptr};
        hipError_t r = hipEventCreate(&e[0]);
        if (r == hipSuccess) r = hipEventCreate(&e[1]);
        for (int ph = 0; ph < 3 && r == hipSuccess; ph++) {
            r = hipEventRecord(e[0], s);
            for (int i = 0; i < reps && r == hipSuccess; i++)
                r = ph == 0 ? launch_pack(dtype, pa, s)
                  : ph == 1 ? launch_sdpa(dtype, sa, s)
                            : launch_coalesce(dtype, sa.tpart, d_tattn, P.nwin, P.txt_len, s);
            if (r == hipSuccess) r = hipEventRecord(e[1], s);
            if (r == hipSuccess) r = hipEventSynchronize(e[1]);
            float ms = 0.f;
            if (r == hipSuccess) r = hipEventElapsedTime(&ms, e[0], e[1]);
            phase_ms[ph] = (double)ms / reps;
        }
        for (hipEvent_t x : e)
            if (x) (void)hipEventDestroy(x);
        HIPCK(ctx, r);
    }
    return AWA_OK;
}

int check_forward_args(const char* who, awa_ctx* ctx, const awa_geom* g, int dtype,
                       const void* d_vqkv, const void* d_tqkv, int Lv, int TXT, const float* d_nq_v,
                       const float* d_nk_v, const float* d_nq_t, const float* d_nk_t, float eps,
                       const void* d_vattn, const void* d_tattn) {
    if (!ctx || !g || !d_vqkv || !d_tqkv || !d_nq_v || !d_nk_v || !d_nq_t || !d_nk_t || !d_vattn ||
        !d_tattn) {
        set_err(ctx, "%s: null argument", who);
        return AWA_EARG;
    }
    const GeomPlan& P = g->plan;
    if (dtype != AWA_F32 && dtype != AWA_BF16) {
        set_err(ctx, "%s: unknown dtype %d", who, dtype);
        return AWA_EARG;
    }
    if (Lv != P.Lv || TXT != P.txt_len) {
        set_err(ctx, "%s: Lv=%d TXT=%d do not match the geometry (Lv=%d TXT=%d)", who, Lv, TXT,
                P.Lv, P.txt_len);
        return AWA_EARG;
    }
    if (!(eps > 0.f)) {
        set_err(ctx, "%s: eps must be > 0 (got %g)", who, (double)eps);
        return AWA_EARG;
    }
    if (g->device != ctx->device) {
        set_err(ctx, "%s: geometry lives on device %d, context on %d", who, g->device, ctx->device);
        return AWA_EARG;
    }
    return AWA_OK;
}

}  // namespace awa

extern "C" {

int awa_create(awa_ctx** out, int hip_device) {
    if (!out) return AWA_EARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || hip_device < 0 || hip_device >= n) return AWA_EHIP;
    awa_ctx* ctx = new (std::nothrow) awa_ctx();
    if (!ctx) return AWA_EHIP;
    ctx->device = hip_device;
    {
        // the allocation-free entry's device array: its address on this
        // device, looked up once per device with the device current
        DeviceGuard dg(hip_device);
        ctx->noalloc_status = noalloc_resolve(hip_device);
    }
    *out = ctx;
    return AWA_OK;
}

void awa_destroy(awa_ctx* ctx) {
    if (!ctx) return;
    DeviceGuard dg(ctx->device);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->small) (void)hipFree(ctx->small);
    if (ctx->emb) (void)hipFree(ctx->emb);
    for (hipEvent_t e : ctx->ev_free) (void)hipEventDestroy(e);
    for (hipEvent_t e : ctx->ev_used) (void)hipEventDestroy(e);
    for (hipEvent_t e : ctx->dit_ev_used) (void)hipEventDestroy(e);
    delete ctx;
}

const char* awa_last_error(const awa_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int awa_plan_windows(int t, int h, int w, const int32_t num_windows[3], int shifted,
                     int32_t* h_slices, int cap) {
    if (!num_windows || cap < 0 || (cap > 0 && !h_slices)) return AWA_EARG;
    GeomParams p{};
    AxisSlices ax;
    if (plan_axes(t, h, w, num_windows, shifted, p, ax, nullptr) != AWA_OK) return AWA_EARG;
    const int nwin = ax.cnt[0] * ax.cnt[1] * ax.cnt[2];
    for (int wi = 0; wi < nwin && wi < cap; wi++) {
        const int it = wi % ax.cnt[0], ih = (wi / ax.cnt[0]) % ax.cnt[1];
        const int iw = wi / (ax.cnt[0] * ax.cnt[1]);
        int32_t* sl = h_slices + (size_t)wi * 6;
        sl[0] = ax.st[0][it]; sl[1] = ax.en[0][it];
        sl[2] = ax.st[1][ih]; sl[3] = ax.en[1][ih];
        sl[4] = ax.st[2][iw]; sl[5] = ax.en[2][iw];
    }
    return nwin;
}

int awa_geom_build(awa_ctx* ctx, int t, int h, int w, const int32_t num_windows[3], int txt_len,
                   int shifted, awa_geom** out, awa_stream_t stream) {
    if (!ctx || !out || !num_windows) {
        set_err(ctx, "awa_geom_build: null argument");
        return AWA_EARG;
    }
    *out = nullptr;
    if (t < 1 || h < 1 || w < 1 || txt_len < 1 || num_windows[0] < 1 || num_windows[1] < 1 ||
        num_windows[2] < 1) {
        set_err(ctx, "awa_geom_build: bad sizes t=%d h=%d w=%d txt=%d nw=(%d,%d,%d)", t, h, w,
                txt_len, num_windows[0], num_windows[1], num_windows[2]);
        return AWA_EARG;
    }
    if ((long)t * h * w > (1L << 24)) {
        set_err(ctx, "awa_geom_build: grid too large");
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);

    GeomParams p{};
    AxisSlices ax;
    int rc0 = plan_axes(t, h, w, num_windows, shifted, p, ax, ctx);
    if (rc0 != AWA_OK) return rc0;
    const int* cnt = ax.cnt;
    const std::vector<int>* st = ax.st;
    const std::vector<int>* en = ax.en;
    const long nwin = (long)cnt[0] * cnt[1] * cnt[2];
    awa_geom* g = new (std::nothrow) awa_geom();
    if (!g) return AWA_EHIP;
    g->device = ctx->device;
    GeomPlan& P = g->plan;
    P.t = t; P.h = h; P.w = w; P.txt_len = txt_len; P.nwin = (int)nwin; P.Lv = t * h * w;
    P.txt_sets = 1;
    P.cumf.assign(P.nwin + 1, 0);
    for (int wi = 0; wi < P.nwin; wi++) {
        const int it = wi % cnt[0], ih = (wi / cnt[0]) % cnt[1], iw = wi / (cnt[0] * cnt[1]);
        const int sl[6] = {st[0][it], en[0][it], st[1][ih], en[1][ih], st[2][iw], en[2][iw]};
        P.slices.insert(P.slices.end(), sl, sl + 6);
        P.cumf[wi + 1] = P.cumf[wi] + (sl[1] - sl[0]) * (sl[3] - sl[2]) * (sl[5] - sl[4]);
    }
    P.sumf = P.cumf[P.nwin];
    P.covers_all = (P.sumf == P.Lv);  // windows tile the grid (every token once)
    plan_tiles(P);

    p.t = t; p.h = h; p.w = w; p.txt_len = txt_len; p.nwin = P.nwin; p.sumf = P.sumf;
    for (int j = 0; j < 21; j++) p.base[j] = 1.0 / std::pow(10000.0, (double)(j * 2) / 42);

    int rc = AWA_OK;
    auto fail = [&](hipError_t e, const char* what) {
        set_err(ctx, "awa_geom_build: %s: %s", what, hipGetErrorString(e));
        rc = AWA_EHIP;
    };
    hipError_t e;
    if ((e = dalloc(&g->d_slices, (size_t)P.nwin * 6)) != hipSuccess) fail(e, "alloc");
    else if ((e = dalloc(&g->d_cumf, (size_t)P.nwin + 1)) != hipSuccess) fail(e, "alloc");
    else if ((e = dalloc(&g->d_vidx, (size_t)P.sumf)) != hipSuccess) fail(e, "alloc");
    else if ((e = dalloc(&g->d_vfreq, (size_t)P.sumf * ROPE_ROT)) != hipSuccess) fail(e, "alloc");
    else if ((e = dalloc(&g->d_tfreq, (size_t)P.nwin * txt_len * ROPE_ROT)) != hipSuccess) fail(e, "alloc");
    else if ((e = dalloc(&g->d_vcs, (size_t)P.sumf * CS_STRIDE)) != hipSuccess) fail(e, "alloc");
    else if ((e = dalloc(&g->d_tcs, (size_t)txt_len * CS_STRIDE)) != hipSuccess) fail(e, "alloc");
    else if ((e = launch_geom_build(p, g, s)) != hipSuccess) fail(e, "geometry kernel");
    if (rc == AWA_OK) rc = upload_plan(ctx, g, s);
    if (rc == AWA_OK) {
        // The plan vectors are pageable; make sure the copies have consumed
        // them before the caller can touch the geometry.
        if ((e = hipStreamSynchronize(s)) != hipSuccess) fail(e, "sync");
    }
    // the op's scratch for this geometry (bf16 storage), so that a first
    // awa_forward under stream capture does not allocate
    if (rc == AWA_OK) rc = ensure_scratch(ctx, op_scratch_bytes(P, AWA_BF16));
    if (rc != AWA_OK) {
        free_geom_buffers(g);
        delete g;
        return rc;
    }
    *out = g;
    return AWA_OK;
}

}  // extern "C"

namespace {

// The geometry from a decoded index: cumf [nwin+1] non-decreasing from 0,
// vidx [cumf[nwin]] distinct tokens in [0, Lv), the frequency tables
// [sumf][126] and [nwin*txt_len][126] with repeated channel pairs.  slices
// (nwin x 6) and t, h, w are kept for awa_geom_read / awa_geom_query when
// given (nullptr: zeros).  who names the entry point in error messages.
int geom_inject(awa_ctx* ctx, const char* who, const std::vector<int32_t>& cumf,
                const std::vector<int32_t>& vidx, const int32_t* slices, int t, int h, int w,
                const float* h_vfreq, const float* h_tfreq, int nwin, int Lv, int txt_len,
                awa_geom** out, hipStream_t s) {
    if (cumf[0] != 0) {
        set_err(ctx, "%s: cumf[0] = %d, expected 0", who, cumf[0]);
        return AWA_EARG;
    }
    for (int i = 0; i < nwin; i++)
        if (cumf[i + 1] < cumf[i]) {
            set_err(ctx, "%s: cumf decreases at window %d", who, i);
            return AWA_EARG;
        }
    const int sumf = cumf[nwin];
    if (sumf < 1 || sumf > Lv || (int)vidx.size() != sumf) {
        set_err(ctx, "%s: sumf=%d outside [1, Lv=%d]", who, sumf, Lv);
        return AWA_EARG;
    }
    std::vector<uint8_t> seen(Lv, 0);
    for (int g = 0; g < sumf; g++) {
        const int v = vidx[g];
        if (v < 0 || v >= Lv) {
            set_err(ctx, "%s: vidx[%d] = %d outside [0, %d)", who, g, v, Lv);
            return AWA_EARG;
        }
        if (seen[v]) {
            set_err(ctx, "%s: token %d appears in two windows", who, v);
            return AWA_EARG;
        }
        seen[v] = 1;
    }
    for (size_t r = 0; r < (size_t)sumf; r++)
        for (int q = 0; q < NPAIR; q++)
            if (h_vfreq[r * ROPE_ROT + 2 * q] != h_vfreq[r * ROPE_ROT + 2 * q + 1]) {
                set_err(ctx, "%s: vfreq row %zu channel pair %d differs", who, r, q);
                return AWA_EARG;
            }
    const size_t trows = (size_t)nwin * txt_len;
    for (size_t r = 0; r < trows; r++)
        for (int q = 0; q < NPAIR; q++)
            if (h_tfreq[r * ROPE_ROT + 2 * q] != h_tfreq[r * ROPE_ROT + 2 * q + 1]) {
                set_err(ctx, "%s: tfreq row %zu channel pair %d differs", who, r, q);
                return AWA_EARG;
            }
    // Text rows shared by all windows?  (make_win repeats one table, so yes.)
    bool shared = true;
    for (int wi = 1; wi < nwin && shared; wi++)
        shared = std::memcmp(h_tfreq, h_tfreq + (size_t)wi * txt_len * ROPE_ROT,
                             sizeof(float) * txt_len * ROPE_ROT) == 0;

    DeviceGuard dg(ctx->device);
    awa_geom* g = new (std::nothrow) awa_geom();
    if (!g) return AWA_EHIP;
    g->device = ctx->device;
    g->injected = true;
    GeomPlan& P = g->plan;
    P.nwin = nwin; P.Lv = Lv; P.txt_len = txt_len; P.sumf = sumf; P.cumf = cumf;
    if (slices) {
        P.t = t; P.h = h; P.w = w;
        P.slices.assign(slices, slices + (size_t)nwin * 6);
    } else {
        P.slices.assign((size_t)nwin * 6, 0);
    }
    P.txt_sets = shared ? 1 : nwin;
    P.covers_all = (sumf == Lv);
    plan_tiles(P);
    const size_t tcs_rows = (size_t)P.txt_sets * txt_len;

    int rc = AWA_OK;
    hipError_t e = hipSuccess;
    auto step = [&](hipError_t x) {
        if (rc == AWA_OK && x != hipSuccess) {
            e = x;
            rc = AWA_EHIP;
        }
    };
    step(dalloc(&g->d_slices, (size_t)nwin * 6));
    step(dalloc(&g->d_cumf, (size_t)nwin + 1));
    step(dalloc(&g->d_vidx, (size_t)sumf));
    step(dalloc(&g->d_vfreq, (size_t)sumf * ROPE_ROT));
    step(dalloc(&g->d_tfreq, trows * ROPE_ROT));
    step(dalloc(&g->d_vcs, (size_t)sumf * CS_STRIDE));
    step(dalloc(&g->d_tcs, tcs_rows * CS_STRIDE));
    if (rc == AWA_OK) {
        step(hipMemcpyAsync(g->d_slices, P.slices.data(), P.slices.size() * 4, hipMemcpyHostToDevice, s));
        step(hipMemcpyAsync(g->d_cumf, cumf.data(), cumf.size() * 4, hipMemcpyHostToDevice, s));
        step(hipMemcpyAsync(g->d_vidx, vidx.data(), vidx.size() * 4, hipMemcpyHostToDevice, s));
        step(hipMemcpyAsync(g->d_vfreq, h_vfreq, (size_t)sumf * ROPE_ROT * 4, hipMemcpyHostToDevice, s));
        step(hipMemcpyAsync(g->d_tfreq, h_tfreq, trows * ROPE_ROT * 4, hipMemcpyHostToDevice, s));
        step(launch_geom_tables(g->d_vfreq, g->d_tfreq, sumf, (int)tcs_rows, g->d_vcs, g->d_tcs, s));
    }
    if (rc == AWA_OK) rc = upload_plan(ctx, g, s);
    if (rc == AWA_OK) step(hipStreamSynchronize(s));
    if (rc == AWA_OK) rc = ensure_scratch(ctx, op_scratch_bytes(P, AWA_BF16));
    if (rc != AWA_OK) {
        if (e != hipSuccess) set_err(ctx, "%s: %s", who, hipGetErrorString(e));
        free_geom_buffers(g);
        delete g;
        return rc;
    }
    *out = g;
    return AWA_OK;
}

}  // namespace

extern "C" {

int awa_geom_set(awa_ctx* ctx, const float* h_vidx, const float* h_cumf, const float* h_vfreq,
                 const float* h_tfreq, int nwin, int Lv, int txt_len, awa_geom** out,
                 awa_stream_t stream) {
    if (!ctx || !out || !h_cumf || !h_vfreq || !h_tfreq || !h_vidx) {
        set_err(ctx, "awa_geom_set: null argument");
        return AWA_EARG;
    }
    *out = nullptr;
    if (nwin < 1 || nwin > MAX_WIN || Lv < 1 || txt_len < 1) {
        set_err(ctx, "awa_geom_set: bad sizes nwin=%d Lv=%d txt=%d", nwin, Lv, txt_len);
        return AWA_EARG;
    }
    // Decode the float encoding (int(x + 0.5), awa.comp:88,101).
    std::vector<int32_t> cumf(nwin + 1);
    for (int i = 0; i <= nwin; i++) cumf[i] = (int32_t)(h_cumf[i] + 0.5f);
    const int sumf = cumf[nwin];
    if (sumf < 1 || sumf > Lv) {
        set_err(ctx, "awa_geom_set: sumf=%d outside [1, Lv=%d]", sumf, Lv);
        return AWA_EARG;
    }
    std::vector<int32_t> vidx(sumf);
    for (int g = 0; g < sumf; g++) {
        const float x = h_vidx[g];
        if (!(x > -0.5f) || !(x < (float)Lv - 0.5f)) {
            set_err(ctx, "awa_geom_set: vidx[%d] = %g outside [0, %d)", g, x, Lv);
            return AWA_EARG;
        }
        vidx[g] = (int)(x + 0.5f);
    }
    return geom_inject(ctx, "awa_geom_set", cumf, vidx, nullptr, 0, 0, 0, h_vfreq, h_tfreq, nwin, Lv,
                       txt_len, out, reinterpret_cast<hipStream_t>(stream));
}

int awa_geom_from_win(awa_ctx* ctx, int t, int h, int w, int nwin, const int32_t* h_slices,
                      const float* h_vid_freq, const float* h_txt_freq, int txt_len, awa_geom** out,
                      awa_stream_t stream) {
    if (!ctx || !out || !h_slices || !h_vid_freq || !h_txt_freq) {
        set_err(ctx, "awa_geom_from_win: null argument");
        return AWA_EARG;
    }
    *out = nullptr;
    if (t < 1 || h < 1 || w < 1 || (long)t * h * w > (1L << 24) || nwin < 1 || nwin > MAX_WIN ||
        txt_len < 1) {
        set_err(ctx, "awa_geom_from_win: bad sizes t=%d h=%d w=%d nwin=%d txt=%d", t, h, w, nwin, txt_len);
        return AWA_EARG;
    }
    // The index of awa_vk.cpp:73-88 / awa_layer.cpp:116-128: windows in
    // order, tokens of a window in (t, h, w) C order.
    const int ext[3] = {t, h, w};
    std::vector<int32_t> cumf(nwin + 1, 0), vidx;
    for (int wi = 0; wi < nwin; wi++) {
        const int32_t* sl = h_slices + (size_t)wi * 6;
        for (int a = 0; a < 3; a++)
            if (sl[2 * a] < 0 || sl[2 * a] > sl[2 * a + 1] || sl[2 * a + 1] > ext[a]) {
                set_err(ctx, "awa_geom_from_win: window %d axis %d slice [%d, %d) outside [0, %d]", wi, a,
                        sl[2 * a], sl[2 * a + 1], ext[a]);
                return AWA_EARG;
            }
        const long f = (long)(sl[1] - sl[0]) * (sl[3] - sl[2]) * (sl[5] - sl[4]);
        if (cumf[wi] + f > (long)t * h * w) {
            set_err(ctx, "awa_geom_from_win: windows hold more tokens than the grid");
            return AWA_EARG;
        }
        cumf[wi + 1] = cumf[wi] + (int32_t)f;
        for (int lt = sl[0]; lt < sl[1]; lt++)
            for (int lh = sl[2]; lh < sl[3]; lh++)
                for (int lw = sl[4]; lw < sl[5]; lw++) vidx.push_back((lt * h + lh) * w + lw);
    }
    return geom_inject(ctx, "awa_geom_from_win", cumf, vidx, h_slices, t, h, w, h_vid_freq, h_txt_freq,
                       nwin, t * h * w, txt_len, out, reinterpret_cast<hipStream_t>(stream));
}

int awa_geom_query(const awa_geom* g, awa_geom_info* info) {
    if (!g || !info) return AWA_EARG;
    const GeomPlan& P = g->plan;
    info->t = P.t; info->h = P.h; info->w = P.w;
    info->nwin = P.nwin; info->sumf = P.sumf; info->Lv = P.Lv; info->txt_len = P.txt_len;
    info->max_S = P.max_S; info->n_tiles = P.n_tiles; info->n_items = P.n_items;
    return AWA_OK;
}

int awa_geom_read(awa_ctx* ctx, const awa_geom* g, int32_t* h_slices, int32_t* h_cumf,
                  int32_t* h_vidx, float* h_vfreq, float* h_tfreq) {
    if (!ctx || !g) {
        set_err(ctx, "awa_geom_read: null argument");
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    const GeomPlan& P = g->plan;
    HIPCK(ctx, hipDeviceSynchronize());
    if (h_slices) HIPCK(ctx, hipMemcpy(h_slices, g->d_slices, (size_t)P.nwin * 6 * 4, hipMemcpyDeviceToHost));
    if (h_cumf) HIPCK(ctx, hipMemcpy(h_cumf, g->d_cumf, (size_t)(P.nwin + 1) * 4, hipMemcpyDeviceToHost));
    if (h_vidx) HIPCK(ctx, hipMemcpy(h_vidx, g->d_vidx, (size_t)P.sumf * 4, hipMemcpyDeviceToHost));
    if (h_vfreq)
        HIPCK(ctx, hipMemcpy(h_vfreq, g->d_vfreq, (size_t)P.sumf * ROPE_ROT * 4, hipMemcpyDeviceToHost));
    if (h_tfreq)
        HIPCK(ctx, hipMemcpy(h_tfreq, g->d_tfreq, (size_t)P.nwin * P.txt_len * ROPE_ROT * 4,
                             hipMemcpyDeviceToHost));
    return AWA_OK;
}

void awa_geom_destroy(awa_geom* g) {
    if (!g) return;
    DeviceGuard dg(g->device);
    free_geom_buffers(g);
    delete g;
}

int awa_forward(awa_ctx* ctx, const awa_geom* g, int dtype, const void* d_vqkv, const void* d_tqkv,
                int Lv, int TXT, const float* d_nq_v, const float* d_nk_v, const float* d_nq_t,
                const float* d_nk_t, float eps, void* d_vattn, void* d_tattn, awa_stream_t stream) {
    const int rc = check_forward_args("awa_forward", ctx, g, dtype, d_vqkv, d_tqkv, Lv, TXT, d_nq_v,
                                      d_nk_v, d_nq_t, d_nk_t, eps, d_vattn, d_tattn);
    if (rc != AWA_OK) return rc;
    DeviceGuard dg(ctx->device);
    return forward_impl(ctx, g, dtype, d_vqkv, d_tqkv, d_nq_v, d_nk_v, d_nq_t, d_nk_t, eps, d_vattn,
                        d_tattn, reinterpret_cast<hipStream_t>(stream));
}

int awa_forward_host(awa_ctx* ctx, const awa_geom* g, const float* h_vqkv, const float* h_tqkv,
                     int Lv, int TXT, const float* h_nq_v, const float* h_nk_v, const float* h_nq_t,
                     const float* h_nk_t, float eps, float* h_vid_out, float* h_txt_out) {
    if (!ctx || !g || !h_vqkv || !h_tqkv || !h_nq_v || !h_nk_v || !h_nq_t || !h_nk_t ||
        !h_vid_out || !h_txt_out) {
        set_err(ctx, "awa_forward_host: null argument");
        return AWA_EARG;
    }
    if (Lv != g->plan.Lv || TXT != g->plan.txt_len) {
        set_err(ctx, "awa_forward_host: Lv=%d TXT=%d do not match the geometry", Lv, TXT);
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    const size_t nv = (size_t)Lv * QKV, nt = (size_t)TXT * QKV;
    const size_t ov = (size_t)Lv * DIM, ot = (size_t)TXT * DIM;
    float* buf = nullptr;
    const size_t total = nv + nt + ov + ot + 4 * HEAD_D;
    HIPCK(ctx, hipMalloc(reinterpret_cast<void**>(&buf), total * sizeof(float)));
    float *dv = buf, *dt = dv + nv, *dvo = dt + nt, *dto = dvo + ov, *dg4 = dto + ot;
    int rc = AWA_OK;
    auto cp = [&](void* dst, const void* src, size_t bytes, hipMemcpyKind k) {
        if (rc == AWA_OK) {
            hipError_t e = hipMemcpy(dst, src, bytes, k);
            if (e != hipSuccess) {
                set_err(ctx, "awa_forward_host: copy failed: %s", hipGetErrorString(e));
                rc = AWA_EHIP;
            }
        }
    };
    cp(dv, h_vqkv, nv * 4, hipMemcpyHostToDevice);
    cp(dt, h_tqkv, nt * 4, hipMemcpyHostToDevice);
    cp(dg4, h_nq_v, HEAD_D * 4, hipMemcpyHostToDevice);
    cp(dg4 + HEAD_D, h_nk_v, HEAD_D * 4, hipMemcpyHostToDevice);
    cp(dg4 + 2 * HEAD_D, h_nq_t, HEAD_D * 4, hipMemcpyHostToDevice);
    cp(dg4 + 3 * HEAD_D, h_nk_t, HEAD_D * 4, hipMemcpyHostToDevice);
    if (rc == AWA_OK)
        rc = awa_forward(ctx, g, AWA_F32, dv, dt, Lv, TXT, dg4, dg4 + HEAD_D, dg4 + 2 * HEAD_D,
                         dg4 + 3 * HEAD_D, eps, dvo, dto, nullptr);
    if (rc == AWA_OK) {
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            set_err(ctx, "awa_forward_host: %s", hipGetErrorString(e));
            rc = AWA_EHIP;
        }
    }
    cp(h_vid_out, dvo, ov * 4, hipMemcpyDeviceToHost);
    cp(h_txt_out, dto, ot * 4, hipMemcpyDeviceToHost);
    (void)hipFree(buf);
    return rc;
}

int awa_time_phases(awa_ctx* ctx, const awa_geom* g, int dtype, const void* d_vqkv, const void* d_tqkv,
                    int Lv, int TXT, const float* d_nq_v, const float* d_nk_v, const float* d_nq_t,
                    const float* d_nk_t, float eps, void* d_vattn, void* d_tattn, int reps,
                    double ms_per_launch[3], awa_stream_t stream) {
    const int rc = check_forward_args("awa_time_phases", ctx, g, dtype, d_vqkv, d_tqkv, Lv, TXT, d_nq_v,
                                      d_nk_v, d_nq_t, d_nk_t, eps, d_vattn, d_tattn);
    if (rc != AWA_OK) return rc;
    if (reps < 1 || !ms_per_launch) {
        set_err(ctx, "awa_time_phases: reps=%d must be positive and ms_per_launch non-null", reps);
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    return forward_impl(ctx, g, dtype, d_vqkv, d_tqkv, d_nq_v, d_nk_v, d_nq_t, d_nk_t, eps, d_vattn, d_tattn,
                        reinterpret_cast<hipStream_t>(stream), nullptr, reps, ms_per_launch);
}

int awa_reserve(awa_ctx* ctx, const awa_geom* g, int dtype) {
    if (!ctx || !g || (dtype != AWA_F32 && dtype != AWA_BF16)) {
        set_err(ctx, "awa_reserve: bad argument");
        return AWA_EARG;
    }
    if (g->device != ctx->device) {
        set_err(ctx, "awa_reserve: geometry of device %d, context of device %d", g->device, ctx->device);
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    return ensure_scratch(ctx, op_scratch_bytes(g->plan, dtype));
}

int awa_timing_enable(awa_ctx* ctx, int enable) {
    if (!ctx) return AWA_EARG;
    ctx->timing = enable != 0;
    return AWA_OK;
}

int awa_timing_read(awa_ctx* ctx, double* ms_pack, double* ms_attn, double* ms_text, int* calls) {
    if (!ctx) return AWA_EARG;
    DeviceGuard dg(ctx->device);
    double acc[3] = {0, 0, 0};
    const size_t n = ctx->ev_used.size() / 4;
    int rc = AWA_OK;
    for (size_t i = 0; i < n && rc == AWA_OK; i++) {
        hipEvent_t* e = &ctx->ev_used[4 * i];
        hipError_t r = hipEventSynchronize(e[3]);
        for (int k = 0; k < 3 && r == hipSuccess; k++) {
            float ms = 0.f;
            r = hipEventElapsedTime(&ms, e[k], e[k + 1]);
            acc[k] += ms;
        }
        if (r != hipSuccess) {
            set_err(ctx, "awa_timing_read: %s", hipGetErrorString(r));
            rc = AWA_EHIP;
        }
    }
    ctx->ev_free.insert(ctx->ev_free.end(), ctx->ev_used.begin(), ctx->ev_used.end());
    ctx->ev_used.clear();
    if (ms_pack) *ms_pack = acc[0];
    if (ms_attn) *ms_attn = acc[1];
    if (ms_text) *ms_text = acc[2];
    if (calls) *calls = (int)n;
    return rc;
}

int awa_cast_f32_to_bf16(awa_ctx* ctx, const float* d_in, uint16_t* d_out, int64_t n,
                         awa_stream_t stream) {
    if (!ctx || (n > 0 && (!d_in || !d_out)) || n < 0) {
        set_err(ctx, "awa_cast_f32_to_bf16: bad argument");
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    HIPCK(ctx, launch_cast_f32_bf16(d_in, d_out, n, reinterpret_cast<hipStream_t>(stream)));
    return AWA_OK;
}

int awa_cast_bf16_to_f32(awa_ctx* ctx, const uint16_t* d_in, float* d_out, int64_t n,
                         awa_stream_t stream) {
    if (!ctx || (n > 0 && (!d_in || !d_out)) || n < 0) {
        set_err(ctx, "awa_cast_bf16_to_f32: bad argument");
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    HIPCK(ctx, launch_cast_bf16_f32(d_in, d_out, n, reinterpret_cast<hipStream_t>(stream)));
    return AWA_OK;
}

int awa_stream_copy(awa_ctx* ctx, void* d_dst, const void* d_src, int64_t bytes, awa_stream_t stream) {
    if (!ctx || bytes < 0 || bytes % 16 != 0 || (bytes > 0 && (!d_dst || !d_src))) {
        set_err(ctx, "awa_stream_copy: bad argument (bytes must be a multiple of 16)");
        return AWA_EARG;
    }
    DeviceGuard dg(ctx->device);
    HIPCK(ctx, launch_stream_copy(d_dst, d_src, (size_t)bytes, reinterpret_cast<hipStream_t>(stream)));
    return AWA_OK;
}

}  // extern "C"

// test_plan.cpp — the host planner of the bf16 attention kernel (awa::plan_tiles,
// awa::plan_schedule in seedvr2-2b-ncnn_amd/csrc/awa_capi.cpp) on the CPU.
//
// Usage: test_plan t h w nw_t nw_h nw_w txt shifted n_slots [empty_at]
// Builds the windows with awa_plan_windows (awa_window.cpp:15-78), their
// cumulative sizes (with empty_at >= 0: an empty window, as an injected
// geometry may hold, inserted before window empty_at), the tiles and the
// schedule, then checks:
//   - every (head, work item) appears in exactly one slot, once;
//   - every descriptor matches its item (window, query tiles, tile ranges);
//   - all items of one (window, head) sit on slots of one XCD (slot % 8);
//   - the kernel's DMA stream (stream_tiles, stream_tile, stream_fetch): in
//     every slot, replaying the prologue and each tile's fetch into the K
//     ring (3 slots) and the V ring (2 slots), the tile an item reads at key
//     tile kk is the one it needs, and every fetched tile index lies inside
//     the packed K tiles and the row table;
// and prints the schedule's makespan, the plain longest-first makespan over
// the same XCD assignment and the mean slot load, in the planner's cost
// units.  The last line is "rc=0" when every check holds.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <vector>

#include "awa_internal.hpp"

using awa::GeomPlan;

static int fail(const char* what, long a, long b) {
    std::printf("FAIL %s (%ld, %ld)\nrc=1\n", what, a, b);
    return 1;
}

int main(int argc, char** argv) {
    if (argc != 10 && argc != 11) {
        std::printf("usage: test_plan t h w nw_t nw_h nw_w txt shifted n_slots [empty_at]\nrc=2\n");
        return 2;
    }
    const int empty_at = argc == 11 ? std::atoi(argv[10]) : -1;
    int v[9];
    for (int i = 0; i < 9; i++) v[i] = std::atoi(argv[i + 1]);
    const int32_t nw[3] = {v[3], v[4], v[5]};
    const int txt = v[6], shifted = v[7], n_slots = v[8];
    int nwin = awa_plan_windows(v[0], v[1], v[2], nw, shifted, nullptr, 0);
    if (nwin <= 0) return fail("window count", nwin, 0);
    std::vector<int32_t> sl((size_t)nwin * 6);
    if (awa_plan_windows(v[0], v[1], v[2], nw, shifted, sl.data(), nwin) != nwin) return fail("windows", nwin, 0);
    if (empty_at >= 0 && empty_at <= nwin) {
        const int32_t e[6] = {0, 1, 0, 0, 0, 1};  // no rows on the h axis
        sl.insert(sl.begin() + (size_t)empty_at * 6, e, e + 6);
        nwin++;
    }

    GeomPlan P;
    P.t = v[0]; P.h = v[1]; P.w = v[2];
    P.nwin = nwin;
    P.txt_len = txt;
    P.txt_sets = 1;
    P.cumf.assign(nwin + 1, 0);
    for (int w = 0; w < nwin; w++) {
        const int32_t* s = &sl[(size_t)w * 6];
        P.cumf[w + 1] = P.cumf[w] + (s[1] - s[0]) * (s[3] - s[2]) * (s[5] - s[4]);
    }
    P.sumf = P.Lv = P.cumf[nwin];
    awa::plan_tiles(P);
    awa::plan_schedule(P, n_slots);

    const int S = P.n_slots, NI = P.n_items, H = awa::HEADS;
    if (S % 8 != 0 || S < 8) return fail("slot count", S, n_slots);
    if ((int)P.sched_start.size() != S + 1 || P.sched_start[0] != 0 || P.sched_start[S] != NI * H)
        return fail("schedule extent", P.sched_start.empty() ? -1 : P.sched_start[S], (long)NI * H);
    std::vector<int> seen((size_t)NI * H, 0);
    std::map<long, int> group_xcd;  // window * HEADS + head -> XCD
    std::vector<long> load(S, 0);
    for (int s = 0; s < S; s++) {
        if (P.sched_start[s + 1] < P.sched_start[s]) return fail("slot order", s, 0);
        for (int k = P.sched_start[s]; k < P.sched_start[s + 1]; k++) {
            const int32_t* d = &P.sched_desc[(size_t)k * 8];
            const int h = d[0] & 255, w = d[0] >> 8;
            if (h < 0 || h >= H || w < 0 || w >= nwin) return fail("descriptor head/window", h, w);
            // the work item of this window with these query tiles
            int item = -1;
            for (int i = 0; i < NI; i++)
                if (P.items[4 * i] == w && P.items[4 * i + 1] == d[1] && P.items[4 * i + 2] == d[2]) item = i;
            if (item < 0) return fail("descriptor item", w, d[1]);
            if (seen[(size_t)h * NI + item]++) return fail("item scheduled twice", h, item);
            if (d[3] != P.cumf[w] || d[4] != P.tile_base[w] || d[5] != P.tile_base[w + 1] - P.tile_base[w] ||
                d[6] != P.n_vid_tiles || d[7] != P.cumf[w + 1] - P.cumf[w])
                return fail("descriptor fields", w, d[3]);
            const long g = (long)w * H + h;
            auto it = group_xcd.find(g);
            if (it == group_xcd.end()) group_xcd[g] = s % 8;
            else if (it->second != s % 8) return fail("group split over XCDs", g, s);
            load[s] += 10 * awa::stream_tiles(d[5], P.ntt) + 25;
        }
    }
    for (size_t i = 0; i < seen.size(); i++)
        if (seen[i] != 1) return fail("item not scheduled", (long)i, seen[i]);

    // The DMA stream of every slot, replayed as the kernel issues it: a ring
    // entry is (head, tile); -1 marks a fetch past the slot's last item (an
    // empty buffer: zeros, never read).
    const int vtiles = P.n_vid_tiles + P.ntt;  // tiles of the row table
    long stream_tiles_total = 0;
    for (int s = 0; s < S; s++) {
        const int i0 = P.sched_start[s], i1 = P.sched_start[s + 1];
        if (i0 == i1) continue;
        struct It { int h, nvt, vbase, tbase, nk; };
        auto item = [&](int k) {
            const int32_t* d = &P.sched_desc[(size_t)k * 8];
            return It{d[0] & 255, d[5], d[4], d[6], awa::stream_tiles(d[5], P.ntt)};
        };
        auto ktile = [&](const It& W, int kk) { return awa::stream_tile(kk, W.nvt, W.vbase, W.tbase, P.ntt); };
        auto vtile = [&](const It& W, int kk) { return awa::stream_tile(kk, W.nvt, W.vbase, P.n_vid_tiles, P.ntt); };
        long kring[3][2], vring[2][2];
        for (auto& r : kring) r[0] = r[1] = -2;
        for (auto& r : vring) r[0] = r[1] = -2;
        It cur = item(i0);
        kring[0][0] = cur.h; kring[0][1] = ktile(cur, 0);
        kring[1][0] = cur.h; kring[1][1] = ktile(cur, 1);
        vring[0][0] = cur.h; vring[0][1] = vtile(cur, 0);
        int kb = 0, vb = 0;
        for (int k = i0; k < i1; k++) {
            const bool has_next = k + 1 < i1;
            const It nxt = item(has_next ? k + 1 : k);
            for (int kk = 0; kk < cur.nk; kk++) {
                // the tiles this key tile reads
                const long* kr = kring[(kb + kk) % 3];
                const long* vr = vring[(vb + kk) & 1];
                if (kr[0] != cur.h || kr[1] != ktile(cur, kk)) return fail("K ring holds the wrong tile", s, kk);
                if (vr[0] != cur.h || vr[1] != vtile(cur, kk)) return fail("V ring holds the wrong tile", s, kk);
                if (kr[1] < 0 || kr[1] >= P.n_tiles) return fail("K tile outside the packed tiles", kr[1], P.n_tiles);
                if (vr[1] < 0 || vr[1] >= vtiles) return fail("V tile outside the row table", vr[1], vtiles);
                // its fetch
                int k_kk, k_nxt, v_kk, v_nxt;
                awa::stream_fetch(kk, cur.nk, &k_kk, &k_nxt, &v_kk, &v_nxt);
                long* kw = kring[(kb + kk + 2) % 3];
                long* vw = vring[(vb + kk + 1) & 1];
                if (!k_nxt) { kw[0] = cur.h; kw[1] = ktile(cur, k_kk); }
                else if (has_next) {
                    if (k_kk >= nxt.nk) return fail("K fetch beyond the next item", k_kk, nxt.nk);
                    kw[0] = nxt.h; kw[1] = ktile(nxt, k_kk);
                } else { kw[0] = kw[1] = -1; }
                if (!v_nxt) { vw[0] = cur.h; vw[1] = vtile(cur, v_kk); }
                else if (has_next) {
                    if (v_kk >= nxt.nk) return fail("V fetch beyond the next item", v_kk, nxt.nk);
                    vw[0] = nxt.h; vw[1] = vtile(nxt, v_kk);
                } else { vw[0] = vw[1] = -1; }
                stream_tiles_total++;
            }
            kb = (kb + cur.nk) % 3;
            vb = (vb + cur.nk) & 1;
            cur = nxt;
        }
    }
    std::printf("stream tiles %ld\n", stream_tiles_total);

    // plain longest-first over the same XCD groups, for comparison
    std::vector<std::vector<long>> xc(8);
    for (int s = 0; s < S; s++)
        for (int k = P.sched_start[s]; k < P.sched_start[s + 1]; k++) {
            const int32_t* d = &P.sched_desc[(size_t)k * 8];
            xc[s % 8].push_back(10 * awa::stream_tiles(d[5], P.ntt) + 25);
        }
    long lpt = 0, total = 0;
    for (int x = 0; x < 8; x++) {
        std::sort(xc[x].rbegin(), xc[x].rend());
        std::vector<long> l(S / 8, 0);
        for (long c : xc[x]) {
            *std::min_element(l.begin(), l.end()) += c;
            total += c;
        }
        lpt = std::max(lpt, *std::max_element(l.begin(), l.end()));
    }
    const long mk = *std::max_element(load.begin(), load.end());
    std::printf("windows %d items %d slots %d makespan %ld lpt %ld mean %.1f\n", nwin, NI * H, S, mk, lpt,
                (double)total / S);
    if (mk > lpt) return fail("makespan above longest-first", mk, lpt);
    std::printf("rc=0\n");
    return 0;
}

// test_plan.cpp — the host planner of the bf16 attention kernel (awa::plan_tiles,
// awa::plan_schedule in seedvr2-2b-ncnn_amd/csrc/awa_capi.cpp) on the CPU.
//
// Usage: test_plan t h w nw_t nw_h nw_w txt shifted n_slots
// Builds the windows with awa_plan_windows (awa_window.cpp:15-78), their
// cumulative sizes, the tiles and the schedule, then checks:
//   - every (head, work item) appears in exactly one slot, once;
//   - every descriptor matches its item (window, query tiles, tile ranges);
//   - all items of one (window, head) sit on slots of one XCD (slot % 8);
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
    if (argc != 10) {
        std::printf("usage: test_plan t h w nw_t nw_h nw_w txt shifted n_slots\nrc=2\n");
        return 2;
    }
    int v[9];
    for (int i = 0; i < 9; i++) v[i] = std::atoi(argv[i + 1]);
    const int32_t nw[3] = {v[3], v[4], v[5]};
    const int txt = v[6], shifted = v[7], n_slots = v[8];
    const int nwin = awa_plan_windows(v[0], v[1], v[2], nw, shifted, nullptr, 0);
    if (nwin <= 0) return fail("window count", nwin, 0);
    std::vector<int32_t> sl((size_t)nwin * 6);
    if (awa_plan_windows(v[0], v[1], v[2], nw, shifted, sl.data(), nwin) != nwin) return fail("windows", nwin, 0);

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
            load[s] += 10 * (d[5] + P.ntt) + 25;
        }
    }
    for (size_t i = 0; i < seen.size(); i++)
        if (seen[i] != 1) return fail("item not scheduled", (long)i, seen[i]);

    // plain longest-first over the same XCD groups, for comparison
    std::vector<std::vector<long>> xc(8);
    for (int s = 0; s < S; s++)
        for (int k = P.sched_start[s]; k < P.sched_start[s + 1]; k++) {
            const int32_t* d = &P.sched_desc[(size_t)k * 8];
            xc[s % 8].push_back(10 * (d[5] + P.ntt) + 25);
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

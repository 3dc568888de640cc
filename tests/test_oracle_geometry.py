"""Pins the oracle's window geometry (awa_window.cpp:15-150, awa_vk.cpp:73-88).

Checks: the reference's own window counts, sequence lengths and frequency
table hashes for every configuration (tests/golden/window_summary.json),
split points, tiling invariants, frequency closed forms, and the host
planner of the C ABI against the oracle over a sweep of shapes.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

SUMMARY = json.load(open(os.path.join(GOLDEN, "window_summary.json")))["cases"]


def fnv1a_words(*arrays):
    h = 0x811C9DC5
    for a in arrays:
        for x in np.ascontiguousarray(a, np.float32).ravel().view(np.uint32).tolist():
            h ^= x
            h = (h * 0x01000193) & 0xFFFFFFFF
    return h


@pytest.mark.parametrize("case", SUMMARY, ids=lambda c: f"{c['name']}-{'sh' if c['shifted'] else 'ns'}")
def test_reference_window_summary(oracle, case):
    g = oracle.Geometry(*case["grid"], case["num_windows"], case["txt_len"], case["shifted"])
    S = g.S
    assert g.nwin == case["nwin"]
    assert (int(S.min()), int(S.max()), int(S.sum())) == (case["S_min"], case["S_max"], case["S_sum"])
    gflop = sum(4 * 128 * 20 * int(s) ** 2 for s in S) / 1e9
    assert abs(gflop - case["sdpa_gflop"]) < 1e-3
    assert fnv1a_words(g.vid_freq, g.txt_freq) == int(case["freq_fnv1a"], 16)
    if "h_splits" in case:
        hs = sorted(set(g.slices[:, 2].tolist()) | set(g.slices[:, 3].tolist()))
        ws = sorted(set(g.slices[:, 4].tolist()) | set(g.slices[:, 5].tolist()))
        assert hs == case["h_splits"] and ws == case["w_splits"]


def check_tiling(g):
    """Every grid token in exactly one window; vidx in window-major C order."""
    counts = np.zeros(g.Lv, np.int64)
    np.add.at(counts, g.vidx, 1)
    assert np.all(counts == 1)
    g_ = 0
    for wi, (st, en, sh, eh, sw, ew) in enumerate(g.slices):
        assert g.cumf[wi] == g_
        tt, hh, ww = np.meshgrid(np.arange(st, en), np.arange(sh, eh), np.arange(sw, ew), indexing="ij")
        tok = ((tt * g.h + hh) * g.w + ww).ravel()
        assert np.array_equal(g.vidx[g_:g_ + tok.size], tok)
        g_ += tok.size
    assert g.cumf[-1] == g.sumf == g.Lv


@pytest.mark.parametrize("shape", [(1, 23, 27), (1, 45, 53), (1, 68, 80), (1, 71, 97), (1, 1, 1),
                                   (3, 5, 7), (2, 9, 64), (40, 2, 3), (1, 120, 7)])
@pytest.mark.parametrize("nw", [(4, 3, 3), (1, 4, 4), (2, 40, 40), (7, 1, 2)])
@pytest.mark.parametrize("shifted", [0, 1])
def test_tiling_invariant(oracle, shape, nw, shifted):
    check_tiling(oracle.Geometry(*shape, nw, 5, shifted))


def test_unshifted_closed_form(oracle):
    """Unshifted windows are the ceil-divided blocks of the 45x80-proxy sizes."""
    import math
    for (t, h, w) in [(1, 68, 80), (1, 23, 27), (5, 33, 17)]:
        nw = (4, 3, 3)
        scale = math.sqrt(3600 / (h * w))
        wh = -(-int(round(h * scale)) // nw[1])
        ww = -(-int(round(w * scale)) // nw[2])
        wt = -(-min(t, 30) // nw[0])
        g = oracle.Geometry(t, h, w, nw, 3, 0)
        assert g.nwin == -(-t // wt) * -(-h // wh) * -(-w // ww)
        assert np.all((g.slices[:, 3] - g.slices[:, 2]) <= wh)
        assert np.all(g.slices[:, 2] % wh == 0) and np.all(g.slices[:, 4] % ww == 0)


def test_shift_is_half_window(oracle):
    """Shifted interior boundaries are int((i - 0.5) * window) (awa_window.cpp:66-76)."""
    g0 = oracle.Geometry(1, 68, 80, (4, 3, 3), 58, 0)
    g1 = oracle.Geometry(1, 68, 80, (4, 3, 3), 58, 1)
    for lo, hi, X in ((2, 3, 68), (4, 5, 80)):
        win = int(g0.slices[0, hi] - g0.slices[0, lo])
        bounds = sorted(set(g1.slices[:, lo].tolist()) | set(g1.slices[:, hi].tolist()))
        interior = [x for x in bounds if 0 < x < X]
        assert interior == [int((i - 0.5) * win) for i in range(1, len(interior) + 1)]


def test_no_shift_when_window_covers_axis(oracle):
    """wX >= X: the shifted variant keeps a single window on that axis."""
    g = oracle.Geometry(1, 4, 4, (1, 1, 1), 3, 1)
    assert g.nwin == 1 and list(g.slices[0]) == [0, 1, 0, 4, 0, 4]


def test_empty_shifted_slices_are_skipped(oracle):
    """(2,3,4) with num_windows (2,40,40): the first t, last h and last w
    shifted slices are empty and dropped."""
    g = oracle.Geometry(2, 3, 4, (2, 40, 40), 3, 1)
    assert g.nwin == 12
    assert set(map(tuple, g.slices[:, 0:2].tolist())) == {(0, 1), (1, 2)}
    check_tiling(g)


def test_freq_closed_form(oracle):
    """vid rows: (TXT + lt, lh, lw) x base, pair-repeated; text rows: ii x base."""
    txt = 7
    g = oracle.Geometry(2, 9, 11, (2, 3, 3), txt, 1)
    base = 1.0 / np.power(10000.0, np.arange(0, 42, 2, dtype=np.float64) / 42)
    row = 0
    for (st, en, sh, eh, sw, ew) in g.slices:
        for lt in range(en - st):
            for lh in range(eh - sh):
                for lw in range(ew - sw):
                    expect = np.concatenate([np.repeat((txt + lt) * base, 2), np.repeat(lh * base, 2),
                                             np.repeat(lw * base, 2)]).astype(np.float32)
                    assert np.array_equal(g.vid_freq[row], expect)
                    row += 1
    tf = g.txt_freq.reshape(g.nwin, txt, 126)
    for ii in range(txt):
        expect = np.tile(np.repeat(ii * base, 2), 3).astype(np.float32)
        assert np.all(tf[:, ii] == expect)


@pytest.mark.parametrize("shifted", [0, 1])
def test_capi_planner_matches_oracle(oracle, awa, shifted):
    """Integer restatement in the C ABI == the reference's double arithmetic."""
    rng = np.random.default_rng(5)
    shapes = [(1, 68, 80), (1, 71, 97), (1, 9, 64), (3, 5, 7)]
    shapes += [tuple(int(x) for x in rng.integers(1, [40, 150, 150])) for _ in range(300)]
    for shp in shapes:
        nw = tuple(int(x) for x in rng.integers(1, 9, 3))
        g = oracle.Geometry(*shp, nw, 2, shifted)
        sl = awa.plan_windows(*shp, nw, shifted)
        assert np.array_equal(sl, g.slices), (shp, nw)


def test_capi_planner_on_random_shapes(oracle, awa):
    """The GPU parity sweep's shapes (random_shapes): the C ABI's window plan
    equals the oracle's before any of them reaches the device."""
    from conftest import random_shapes
    for t, h, w, nw, txt, sh in random_shapes():
        g = oracle.Geometry(t, h, w, nw, txt, sh)
        assert np.array_equal(awa.plan_windows(t, h, w, nw, sh), g.slices), (t, h, w, nw, txt, sh)

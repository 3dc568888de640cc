"""Pins the oracle bit for bit against the reference's own CPU routines.

oracle/_ref/libref_bridge.so is src/verify_dit.cpp compiled unchanged (see
oracle/Makefile); it exists only where the reference sources were present at
build time, so these tests skip elsewhere.  The committed fixtures
tests/golden/awa_ref_*.npz carry the reference's outputs to machines without
it (test_reference_fixtures).
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN, seeded_awa_inputs

pytestmark = []


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def R(oracle):
    if not oracle.ref_available():
        pytest.skip("reference bridge not built (reference sources absent)")
    return oracle.ref()


def test_qk_norm_rope_rmsnorm(oracle, R):
    rng = np.random.default_rng(1)
    for scale in (1.0, 1e-3, 40.0):
        x = (scale * rng.standard_normal(2560)).astype(np.float32)
        w = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
        out = np.empty(2560, np.float32)
        R.ref_qk_norm(x, w, out)
        assert np.array_equal(bits(oracle.qk_norm(x, w)), bits(out))
        R.ref_rmsnorm(x, 2560, None, out)
        assert np.array_equal(bits(oracle.rmsnorm(x)), bits(out))
        wt = np.ascontiguousarray(np.tile(w, 20))
        R.ref_rmsnorm(x, 2560, wt.ctypes.data, out)
        assert np.array_equal(bits(oracle.rmsnorm(x, wt)), bits(out))
    for _ in range(50):
        fr = (rng.standard_normal(126) * 60).astype(np.float32)
        q = rng.standard_normal(128).astype(np.float32)
        out = np.empty(128, np.float32)
        R.ref_apply_rope(fr, q, out)
        assert np.array_equal(bits(oracle.apply_rope(fr, q)), bits(out))


def test_sinusoidal_silu_linear(oracle, R):
    for t in (1000.0, 500.0, 1.0, 0.0):
        e = np.empty(256, np.float32)
        R.ref_sinusoidal(t, 256, e)
        assert np.array_equal(bits(oracle.sinusoidal(t)), bits(e))
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(4096) * 6).astype(np.float32)
    y = x.copy()
    R.ref_silu(y, y.size)
    assert np.array_equal(bits(oracle.silu(x)), bits(y))
    X = rng.standard_normal((5, 333)).astype(np.float32)
    W = rng.standard_normal((77, 333)).astype(np.float32)
    b = rng.standard_normal(77).astype(np.float32)
    y = np.empty((5, 77), np.float32)
    R.ref_linear(X, W, b.ctypes.data, 5, 333, 77, y)
    assert np.array_equal(bits(oracle.linear(X, W, b)), bits(y))
    R.ref_linear(X, W, None, 5, 333, 77, y)
    assert np.array_equal(bits(oracle.linear(X, W)), bits(y))


def test_time_embedding(oracle, R):
    rng = np.random.default_rng(3)
    ws = [(0.02 * rng.standard_normal(s)).astype(np.float32)
          for s in ((2560, 256), (2560,), (2560, 2560), (2560,), (15360, 2560), (15360,))]
    e = np.empty(15360, np.float32)
    R.ref_time_embedding(1000.0, *ws, e)
    assert np.array_equal(bits(oracle.time_embedding(1000.0, *ws)), bits(e))


@pytest.mark.parametrize("case", [((1, 6, 8), (1, 30, 30), 5, 0), ((1, 6, 8), (1, 30, 30), 5, 1),
                                  ((2, 9, 11), (2, 3, 3), 7, 1), ((1, 2, 6), (1, 1, 1), 4, 0)])
def test_awa_bit_exact(oracle, R, case):
    """orc_awa_forward == verify_dit.cpp::awa_forward on the same vqkv."""
    grid, nw, txt, sh = case
    g = oracle.Geometry(*grid, nw, txt, sh)
    rng = np.random.default_rng(4)
    Lv = g.Lv
    vid = rng.standard_normal((Lv, 2560)).astype(np.float32)
    tx = rng.standard_normal((txt, 2560)).astype(np.float32)
    Wv = (0.02 * rng.standard_normal((7680, 2560))).astype(np.float32)
    Wt = (0.02 * rng.standard_normal((7680, 2560))).astype(np.float32)
    gains = [(1 + 0.02 * rng.standard_normal(128)).astype(np.float32) for _ in range(4)]
    vq = np.empty((Lv, 7680), np.float32)
    tq = np.empty((txt, 7680), np.float32)
    va = np.empty((Lv, 2560), np.float32)
    ta = np.empty((txt, 2560), np.float32)
    R.ref_awa_block(vid, Lv, tx, txt, *grid, g.slices, g.nwin, g.vid_freq, g.sumf, g.txt_freq,
                    Wv, Wt, *gains, vq, tq, va, ta)
    oa, ot = oracle.awa_forward(vq, tq, g, *gains, eps=1e-5)
    assert np.array_equal(bits(oa), bits(va))
    assert np.array_equal(bits(ot), bits(ta))


@pytest.mark.slow
def test_awa_bit_exact_360p(oracle, R):
    """Config 0 geometry (1x23x27, TXT 58, four windows) through the reference."""
    g = oracle.Geometry(1, 23, 27, (4, 3, 3), 58, 0)
    rng = np.random.default_rng(0)
    Lv = g.Lv
    vid = rng.standard_normal((Lv, 2560)).astype(np.float32)
    tx = rng.standard_normal((58, 2560)).astype(np.float32)
    Wv = (0.02 * rng.standard_normal((7680, 2560))).astype(np.float32)
    gains = [(1 + 0.02 * rng.standard_normal(128)).astype(np.float32) for _ in range(4)]
    vq = np.empty((Lv, 7680), np.float32)
    tq = np.empty((58, 7680), np.float32)
    va = np.empty((Lv, 2560), np.float32)
    ta = np.empty((58, 2560), np.float32)
    R.ref_awa_block(vid, Lv, tx, 58, 1, 23, 27, g.slices, g.nwin, g.vid_freq, g.sumf, g.txt_freq,
                    Wv, Wv, *gains, vq, tq, va, ta)
    oa, ot = oracle.awa_forward(vq, tq, g, *gains, eps=1e-5)
    assert np.array_equal(bits(oa), bits(va)) and np.array_equal(bits(ot), bits(ta))


def load_fixture(name):
    z = np.load(os.path.join(GOLDEN, f"awa_ref_{name}.npz"))
    return z, json.loads(str(z["meta"]))


def fixture_inputs(meta):
    """Rebuilds the fixture's vqkv/tqkv and gains (see make_awa_golden.py)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("mk", os.path.join(GOLDEN, "make_awa_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    _, perm = mk.qkv_map()
    vid, txt, gains = mk.inputs(tuple(meta["grid"]), meta["txt_len"], meta["seed"])
    return mk.expand(vid, perm), mk.expand(txt, perm), gains


@pytest.mark.parametrize("name", ["t2_unshifted", "t2_shifted"])
def test_reference_fixtures(oracle, name):
    """The oracle reproduces the reference's stored outputs bit for bit."""
    z, meta = load_fixture(name)
    g = oracle.Geometry(*meta["grid"], meta["num_windows"], meta["txt_len"], meta["shifted"])
    assert np.array_equal(g.slices, z["slices"])
    vq, tq, gains = fixture_inputs(meta)
    oa, ot = oracle.awa_forward(vq, tq, g, *gains, eps=meta["eps"])
    assert np.array_equal(bits(oa), bits(z["vattn"]))
    assert np.array_equal(bits(ot), bits(z["tattn"]))

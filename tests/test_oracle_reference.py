"""Pins the oracle bit for bit against the reference's own CPU routines.

oracle/_ref/libref_bridge.so is src/verify_dit.cpp compiled unchanged (see
oracle/Makefile); it exists only where the reference sources were present at
build time, so these tests skip elsewhere.  The committed fixtures
tests/golden/awa_ref_*.npz carry the reference's outputs to machines without
it (test_reference_fixtures).
"""
import json
import os
import tempfile

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


# ---- the whole 32-layer DiT of the reference's verify_dit main() ----

STACK_GRID, STACK_NW, STACK_TXT, STACK_MLP = (2, 4, 6), (2, 30, 30), 8, 128
REPORTED_BLOCKS = (0, 1, 2, 3, 15, 31)


def _fp16_values(a):
    """The fp32 values an fp16 InnerProduct file holds for a (what load_linear decodes)."""
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def _stack_branch(i, flow):
    """Branch of layer i (flow 'v', 't' or 'a'), seeded per branch.  Matrices
    hold fp16 values k 2^-17, k uniform in [-2048, 2048) (|w| < 0.016, exact in
    fp16 and cheap to draw for the 42 branches); qk gains 1 + N(0, 0.02); ada
    vectors and biases N(0, 0.02)."""
    rng = np.random.default_rng([31, i, ord(flow)])
    f = lambda *s: rng.standard_normal(s, dtype=np.float32) * np.float32(0.02)
    h = lambda *s: rng.integers(-2048, 2048, size=s, dtype=np.int16).astype(np.float16) \
        * np.float16(2.0 ** -17)
    br = {"qkv_w": h(7680, 2560), "out_w": h(2560, 2560), "out_b": f(2560),
          "mlp_in_w": h(STACK_MLP, 2560), "mlp_g_w": h(STACK_MLP, 2560),
          "mlp_out_w": h(2560, STACK_MLP), "nq": 1 + f(128), "nk": 1 + f(128)}
    for k in ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
        br[k] = f(2560)
    return br


def _stack_layers():
    out = []
    for i in range(32):
        if i < 10:
            out.append((_stack_branch(i, "v"), _stack_branch(i, "t")))
        else:
            b = _stack_branch(i, "a")
            out.append((b, b))
    return out


@pytest.mark.slow
def test_dit_stack_matches_reference_main(oracle, R):
    """The reference's own verify_dit main() (verify_dit.cpp:350-485, compiled
    unchanged) runs its 32-layer loop over a model directory in its layout and
    compares its hidden state after blocks 0-3, 15 and 31 and its final output
    with files; the files hold the oracle's chained orc_dit_layer outputs (text
    on every layer, t = 500, fp16-decoded weights).  Every comparison must show
    max|diff| == 0, i.e. the oracle's layer composition (ada slots, gates,
    residual order, SwiGLU, even/odd geometry, input and output layers) is the
    reference's bit for bit."""
    # the 2.2 GB model directory lives in memory where /dev/shm exists
    shm = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=shm) as d:
        _run_stack(oracle, R, d)


def _run_stack(oracle, R, top):
    import ctypes as C
    from dit_reference import random_io
    from model_files import write_model, write_raw_f, write_win

    root = os.path.join(top, "models", "m5")
    rng = np.random.default_rng(30)
    io = random_io(rng)
    for k in ("vid_in_w", "txt_in_w", "vid_out_w"):
        io[k] = _fp16_values(io[k])
    tws = [(0.02 * rng.standard_normal(s)).astype(np.float32)
           for s in ((2560, 256), (2560,), (2560, 2560), (2560,), (15360, 2560), (15360,))]
    for k in (0, 2, 4):
        tws[k] = _fp16_values(tws[k])
    layers = _stack_layers()
    write_model(root, io, layers, tws, 10, fp16=True)

    t, h, w = STACK_GRID
    geoms = [oracle.Geometry(t, h, w, STACK_NW, STACK_TXT, s) for s in (0, 1)]
    for g, name in zip(geoms, ("win_nonshifted.bin", "win_shifted.bin")):
        hdr = [t, h, w, *STACK_NW, 0, 0, 0, g.nwin]
        write_win(os.path.join(root, name), hdr, g.slices, g.vid_freq, g.txt_freq)
    Lv = t * h * w
    x_patch = rng.standard_normal((Lv, 132)).astype(np.float32)
    x_txt = rng.standard_normal((STACK_TXT, 5120)).astype(np.float32)
    write_raw_f(os.path.join(root, "x_patch.bin"), x_patch)
    write_raw_f(os.path.join(root, "x_txt.bin"), x_txt)

    # the oracle's chain: input layers, time embedding at t = 500, 32 layers, output layer
    vid = oracle.linear(x_patch, io["vid_in_w"], io["vid_in_b"])
    txt = oracle.linear(x_txt, io["txt_in_w"], io["txt_in_b"])
    emb = oracle.time_embedding(500.0, *tws)
    for i, (vb, tb) in enumerate(layers):
        vid, txt = oracle.dit_layer(vid, txt, emb, vb, tb, geoms[i % 2], txt_vid_only=False)
        if i in REPORTED_BLOCKS:
            write_raw_f(os.path.join(root, f"vid_b{i}.bin"), vid)
    vn = np.stack([oracle.rmsnorm(vid[r], io["out_norm_w"]) for r in range(Lv)])
    vn = vn * (emb[1::6] + io["out_ada_scale"]) + (emb[0::6] + io["out_ada_shift"])
    write_raw_f(os.path.join(root, "ref_vid_out.bin"), oracle.linear(vn, io["vid_out_w"], io["vid_out_b"]))

    cap = 16
    blocks = np.zeros(cap, np.int32)
    cos = np.zeros(cap, np.float64)
    md = np.zeros(cap, np.float64)
    n = C.c_int(0)
    rc = R.ref_verify_dit_main(top.encode(), blocks, cos, md, cap, C.byref(n))
    assert rc == 0, rc
    got = {int(b): (float(c), float(d)) for b, c, d in zip(blocks[: n.value], cos, md)}
    assert sorted(got) == sorted(REPORTED_BLOCKS + (-1,)), got
    for b, (c, d) in got.items():
        assert d == 0.0 and abs(c - 1.0) < 1e-6, (b, c, d)

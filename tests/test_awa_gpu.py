"""GPU parity of the AWA op through the C ABI against the oracle.

Bars (from the op's specification):
  - window and index metadata: bit-exact;
  - fp32 storage: cos >= 0.99999 and max|d| / max|ref| <= 1e-4 against the
    reference C++ attention (the oracle, bit-exact to it);
  - bf16 storage: cos >= 0.9999 against the reference bf16 path, emulated as
    bf16 inputs widened exactly, fp32 attention, outputs rounded to nearest
    even (awa_layer.cpp:338-451).
"""
import json
import os
import sys

import numpy as np
import pytest

from conftest import GOLDEN, metrics, rel_elementwise, seeded_awa_inputs

pytestmark = pytest.mark.gpu

F32_COS, F32_REL, BF16_COS = 0.99999, 1e-4, 0.9999


def f32_check(out, ref, tag=""):
    """The fp32 bar: cos >= 0.99999 and max|d| / max|ref| <= 1e-4 (the
    normalised relative error); the elementwise relative error over the
    elements with |ref| >= 1e-3 max|ref| is reported beside it."""
    cos, rel, _ = metrics(out, ref)
    erel, n = rel_elementwise(out, ref)
    note(f"  {tag}cos={cos:.8f} rel(max-normalised)={rel:.2e} rel(elementwise, |ref| >= 1e-3 max)={erel:.2e} "
         f"over {n} elements")
    assert cos >= F32_COS and rel <= F32_REL, (cos, rel)
    return erel

CONFIGS = {
    # name: grid, num_windows, txt, seed, outlier fraction
    "cfg0_360p": ((1, 23, 27), (4, 3, 3), 58, 0, 0.0),
    "cfg1_720p": ((1, 45, 53), (4, 3, 3), 58, 1, 0.0),
    "cfg2_1080p": ((1, 68, 80), (4, 3, 3), 58, 2, 0.0),
    "cfg4_ragged": ((1, 71, 97), (1, 4, 4), 77, 4, 0.01),
    # several latent frames: temporal RoPE positions and windows across frames
    "cfg5_frames": ((5, 23, 27), (4, 3, 3), 58, 5, 0.0),
    "cfg6_frames": ((9, 8, 10), (2, 2, 3), 30, 6, 0.0),
    # three latent frames at the 720p latent grid (7,155 video rows)
    "cfg7_frames_720p": ((3, 45, 53), (4, 3, 3), 58, 7, 0.0),
}


def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("name", list(CONFIGS) + ["edge"])
@pytest.mark.parametrize("shifted", [0, 1])
def test_geometry_bit_exact(oracle, ctx, name, shifted):
    cases = [CONFIGS[name][:3]] if name != "edge" else [
        ((1, 1, 1), (1, 1, 1), 1), ((2, 3, 4), (2, 40, 40), 3), ((40, 2, 3), (7, 1, 2), 5),
        ((1, 120, 7), (2, 40, 40), 2), ((3, 5, 7), (4, 3, 3), 70)]
    for grid, nw, txt in cases:
        note(f"geometry {grid} {nw} txt={txt} shifted={shifted}")
        g = ctx.build_geometry(*grid, nw, txt, shifted)
        d = g.read()
        o = oracle.Geometry(*grid, nw, txt, shifted)
        info = g.info()
        assert info["nwin"] == o.nwin and info["sumf"] == o.sumf and info["Lv"] == o.Lv
        assert np.array_equal(d["slices"], o.slices)
        assert np.array_equal(d["cumf"], o.cumf)
        assert np.array_equal(d["vidx"], o.vidx)
        assert np.array_equal(d["vid_freq"].view(np.uint32), o.vid_freq.view(np.uint32))
        assert np.array_equal(d["txt_freq"].view(np.uint32), o.txt_freq.view(np.uint32))
        g.close()


def run_gpu(ctx, geom, vqkv, tqkv, gains, dtype, eps=1e-5):
    torch, dev = torch_dev()
    vq = torch.from_numpy(vqkv).to(dev, dtype)
    tq = torch.from_numpy(tqkv).to(dev, dtype)
    g4 = [torch.from_numpy(g).to(dev) for g in gains]
    va, ta = ctx.forward(geom, vq, tq, *g4, eps=eps)
    torch.cuda.synchronize()
    return va.float().cpu().numpy(), ta.float().cpu().numpy()


@pytest.mark.parametrize("name", ["t2_unshifted", "t2_shifted"])
def test_f32_against_reference_fixture(ctx, name):
    """fp32 GPU output vs the reference's own stored output."""
    sys.path.insert(0, os.path.dirname(__file__))
    from test_oracle_reference import fixture_inputs, load_fixture
    z, meta = load_fixture(name)
    vq, tq, gains = fixture_inputs(meta)
    torch, _ = torch_dev()
    geom = ctx.build_geometry(*meta["grid"], meta["num_windows"], meta["txt_len"], meta["shifted"])
    va, ta = run_gpu(ctx, geom, vq, tq, gains, torch.float32, meta["eps"])
    for out, ref in ((va, z["vattn"]), (ta, z["tattn"])):
        f32_check(out, ref)


@pytest.mark.parametrize("shifted", [0, 1])
def test_f32_config0_360p(oracle, ctx, shifted):
    torch, _ = torch_dev()
    grid, nw, txt, seed, _ = CONFIGS["cfg0_360p"]
    note(f"f32 360p shifted={shifted}")
    vq, tq, gains = seeded_awa_inputs(grid[0] * grid[1] * grid[2], txt, seed)
    o = oracle.Geometry(*grid, nw, txt, shifted)
    rv, rt = oracle.awa_forward(vq, tq, o, *gains, eps=1e-5)
    geom = ctx.build_geometry(*grid, nw, txt, shifted)
    va, ta = run_gpu(ctx, geom, vq, tq, gains, torch.float32)
    for out, ref in ((va, rv), (ta, rt)):
        f32_check(out, ref)


@pytest.mark.parametrize("name", ["cfg5_frames", "cfg6_frames"])
@pytest.mark.parametrize("shifted", [0, 1])
def test_f32_multi_frame(oracle, ctx, name, shifted):
    """fp32 path on grids of several latent frames (T > 1)."""
    torch, _ = torch_dev()
    grid, nw, txt, seed, _ = CONFIGS[name]
    note(f"f32 {name} shifted={shifted}")
    vq, tq, gains = seeded_awa_inputs(grid[0] * grid[1] * grid[2], txt, seed)
    o = oracle.Geometry(*grid, nw, txt, shifted)
    assert len(set(o.slices[:, 0].tolist())) > 1  # windows start on more than one frame
    rv, rt = oracle.awa_forward(vq, tq, o, *gains, eps=1e-5)
    geom = ctx.build_geometry(*grid, nw, txt, shifted)
    va, ta = run_gpu(ctx, geom, vq, tq, gains, torch.float32)
    for out, ref in ((va, rv), (ta, rt)):
        f32_check(out, ref)


def bf16_reference(oracle, vq, tq, gains, geom_o):
    """The reference bf16 path: bf16 in, fp32 attention, bf16 out."""
    rv, rt = oracle.awa_forward(oracle.bf16_round(vq), oracle.bf16_round(tq), geom_o, *gains, eps=1e-5)
    return oracle.bf16_round(rv), oracle.bf16_round(rt)


@pytest.mark.parametrize("name", ["cfg1_720p", "cfg2_1080p", "cfg4_ragged", "cfg0_360p", "cfg5_frames", "cfg6_frames",
                                  "cfg7_frames_720p"])
@pytest.mark.parametrize("shifted", [0, 1])
def test_bf16_configs(oracle, ctx, name, shifted):
    torch, _ = torch_dev()
    grid, nw, txt, seed, outl = CONFIGS[name]
    note(f"bf16 {name} shifted={shifted}")
    vq, tq, gains = seeded_awa_inputs(grid[0] * grid[1] * grid[2], txt, seed, outlier_frac=outl)
    o = oracle.Geometry(*grid, nw, txt, shifted)
    rv, rt = bf16_reference(oracle, vq, tq, gains, o)
    geom = ctx.build_geometry(*grid, nw, txt, shifted)
    va, ta = run_gpu(ctx, geom, vq, tq, gains, torch.bfloat16)
    for out, ref in ((va, rv), (ta, rt)):
        cos, rel, md = metrics(out, ref)
        note(f"  cos={cos:.8f} rel={rel:.2e} maxd={md:.3e}")
        assert np.all(np.isfinite(out))
        assert cos >= BF16_COS, cos


@pytest.mark.parametrize("txt", [1, 63, 64, 65, 130])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_text_lengths(oracle, ctx, txt, dtype):
    """Text lengths around the 64-row tile: one row, a tile less one, exactly
    one tile, one row into a second tile, three tiles (the text keys of a
    window then span several key tiles, and the text queries several query
    tiles), shifted 1x12x20 windows (1,2,2)."""
    torch, _ = torch_dev()
    grid, nw = (1, 12, 20), (1, 2, 2)
    note(f"text length {txt} {dtype}")
    vq, tq, gains = seeded_awa_inputs(grid[0] * grid[1] * grid[2], txt, 40 + txt)
    o = oracle.Geometry(*grid, nw, txt, 1)
    geom = ctx.build_geometry(*grid, nw, txt, 1)
    if dtype == "bf16":
        rv, rt = bf16_reference(oracle, vq, tq, gains, o)
        va, ta = run_gpu(ctx, geom, vq, tq, gains, torch.bfloat16)
    else:
        rv, rt = oracle.awa_forward(vq, tq, o, *gains, eps=1e-5)
        va, ta = run_gpu(ctx, geom, vq, tq, gains, torch.float32)
    for out, ref in ((va, rv), (ta, rt)):
        cos, rel, md = metrics(out, ref)
        note(f"  cos={cos:.8f} rel={rel:.2e}")
        assert np.all(np.isfinite(out))
        if dtype == "bf16":
            assert cos >= BF16_COS, cos
        else:
            f32_check(out, ref)


def test_f32_on_bf16_config_shapes(oracle, ctx):
    """The fp32 path at the 1080p shifted shape (25 ragged windows)."""
    torch, _ = torch_dev()
    grid, nw, txt, seed, _ = CONFIGS["cfg2_1080p"]
    vq, tq, gains = seeded_awa_inputs(grid[0] * grid[1] * grid[2], txt, seed)
    o = oracle.Geometry(*grid, nw, txt, 1)
    rv, rt = oracle.awa_forward(vq, tq, o, *gains, eps=1e-5)
    geom = ctx.build_geometry(*grid, nw, txt, 1)
    va, ta = run_gpu(ctx, geom, vq, tq, gains, torch.float32)
    for out, ref in ((va, rv), (ta, rt)):
        f32_check(out, ref)


def test_injected_geometry_matches_built(oracle, ctx):
    """set_window_geometry with the reference's float arrays == device-built."""
    torch, _ = torch_dev()
    grid, nw, txt = (1, 23, 27), (4, 3, 3), 58
    vq, tq, gains = seeded_awa_inputs(grid[1] * grid[2], txt, 7)
    for shifted in (0, 1):
        o = oracle.Geometry(*grid, nw, txt, shifted)
        g_set = ctx.set_geometry(o.vidx.astype(np.float32), o.cumf.astype(np.float32), o.vid_freq,
                                 o.txt_freq, o.nwin, o.Lv, txt)
        g_bld = ctx.build_geometry(*grid, nw, txt, shifted)
        for dt in (torch.float32, torch.bfloat16):
            a = run_gpu(ctx, g_set, vq, tq, gains, dt)
            b = run_gpu(ctx, g_bld, vq, tq, gains, dt)
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_partial_cover_zero_fill(oracle, ctx):
    """Tokens outside every window get zero rows (awa_layer.cpp:386-399)."""
    torch, _ = torch_dev()
    o = oracle.Geometry(1, 6, 8, (1, 30, 30), 5, 0)
    keep = 3  # drop the last windows: their tokens become uncovered
    cumf = o.cumf[: keep + 1]
    vidx = o.vidx[: cumf[-1]]
    vq, tq, gains = seeded_awa_inputs(o.Lv, 5, 8)
    g = ctx.set_geometry(vidx.astype(np.float32), cumf.astype(np.float32), o.vid_freq[: cumf[-1]],
                         o.txt_freq[: keep * 5], keep, o.Lv, 5)
    torch_, dev = torch_dev()
    out = torch_.full((o.Lv, 2560), 7.0, device=dev)
    tout = torch_.empty((5, 2560), device=dev)
    ctx.forward(g, torch_.from_numpy(vq).to(dev), torch_.from_numpy(tq).to(dev),
                *[torch_.from_numpy(x).to(dev) for x in gains], vattn=out, tattn=tout)
    torch_.cuda.synchronize()
    va = out.cpu().numpy()
    covered = np.zeros(o.Lv, bool)
    covered[vidx] = True
    assert np.all(va[~covered] == 0.0)
    # the covered rows equal the oracle run on the same partial geometry
    import types
    og = types.SimpleNamespace(t=1, h=6, w=8, Lv=o.Lv, txt_len=5, slices=np.ascontiguousarray(o.slices[:keep]),
                               nwin=keep, vid_freq=np.ascontiguousarray(o.vid_freq[: cumf[-1]]),
                               txt_freq=np.ascontiguousarray(o.txt_freq[: keep * 5]))
    rv, rt = oracle.awa_forward(vq, tq, og, *gains, eps=1e-5)
    cos, rel, _ = metrics(va[covered], rv[covered])
    assert cos >= F32_COS and rel <= F32_REL
    cos, rel, _ = metrics(tout.cpu().numpy(), rt)
    assert cos >= F32_COS and rel <= F32_REL


def test_single_window_is_plain_attention(oracle, ctx):
    """num_windows (1,1,1) on a small grid: one window, so the op is ordinary
    softmax attention over Lv + TXT rows of normalised, rotated q/k (checked
    in fp64 with torch's SDPA on the CPU)."""
    import torch
    o = oracle.Geometry(1, 5, 7, (1, 1, 1), 6, 0)
    assert o.nwin == 1
    vq, tq, gains = seeded_awa_inputs(o.Lv, 6, 9)
    g = ctx.build_geometry(1, 5, 7, (1, 1, 1), 6, 0)
    va, ta = run_gpu(ctx, g, vq, tq, gains, torch.float32)
    # fp64 reference built from the oracle's per-token ops
    rows = [(vq[tok], gains[0], gains[1], o.vid_freq[r]) for r, tok in enumerate(o.vidx)]
    rows += [(tq[i], gains[2], gains[3], o.txt_freq[i]) for i in range(6)]
    Q, K, V = [], [], []
    for x, gq, gk, fr in rows:
        qn = oracle.qk_norm(x[:2560], gq).reshape(20, 128)
        kn = oracle.qk_norm(x[2560:5120], gk).reshape(20, 128)
        Q.append(np.stack([oracle.apply_rope(fr, qn[h]) for h in range(20)]))
        K.append(np.stack([oracle.apply_rope(fr, kn[h]) for h in range(20)]))
        V.append(x[5120:].reshape(20, 128))
    Q, K, V = (torch.from_numpy(np.stack(a).transpose(1, 0, 2).astype(np.float64)) for a in (Q, K, V))
    O_ = torch.nn.functional.scaled_dot_product_attention(Q, K, V).numpy().transpose(1, 0, 2).reshape(-1, 2560)
    ref_v = np.zeros_like(va)
    ref_v[o.vidx] = O_[: o.Lv]
    for out, ref in ((va, ref_v), (ta, O_[o.Lv:])):
        f32_check(out, ref, "fp64 SDPA: ")


def test_forward_host_matches_device(oracle, ctx):
    """AwaVk-style host-vector entry == the device entry (fp32)."""
    torch, _ = torch_dev()
    vq, tq, gains = seeded_awa_inputs(6 * 8, 5, 10)
    g = ctx.build_geometry(1, 6, 8, (1, 30, 30), 5, 1)
    hv, ht = ctx.forward_host(g, vq, tq, *gains)
    dv, dt = run_gpu(ctx, g, vq, tq, gains, torch.float32)
    assert np.array_equal(hv, dv) and np.array_equal(ht, dt)


def test_deterministic(ctx):
    torch, _ = torch_dev()
    vq, tq, gains = seeded_awa_inputs(68 * 80, 58, 2)
    g = ctx.build_geometry(1, 68, 80, (4, 3, 3), 58, 1)
    a = run_gpu(ctx, g, vq, tq, gains, torch.bfloat16)
    b = run_gpu(ctx, g, vq, tq, gains, torch.bfloat16)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_error_paths(oracle, ctx, awa):
    """Bad shapes and geometry return AWA_EARG with a message; no kernel runs."""
    import torch
    dev = torch.device("cuda:0")
    g = ctx.build_geometry(1, 6, 8, (1, 30, 30), 5, 0)
    vq = torch.zeros((48, 7680), device=dev)
    tq = torch.zeros((5, 7680), device=dev)
    gn = [torch.ones(128, device=dev) for _ in range(4)]
    with pytest.raises(awa.AwaError) as e:
        ctx.forward(g, torch.zeros((47, 7680), device=dev), tq, *gn)
    assert e.value.code == awa.AWA_EARG and "Lv" in str(e.value)
    with pytest.raises(awa.AwaError):
        ctx.forward(g, vq, torch.zeros((4, 7680), device=dev), *gn)
    with pytest.raises(awa.AwaError):
        ctx.forward(g, vq, tq, *gn, eps=0.0)
    with pytest.raises(awa.AwaError):
        ctx.build_geometry(0, 6, 8, (1, 1, 1), 5, 0)
    o = oracle.Geometry(1, 6, 8, (1, 30, 30), 5, 0)
    bad = o.vidx.astype(np.float32).copy()
    bad[1] = bad[0]  # a token in two windows
    with pytest.raises(awa.AwaError):
        ctx.set_geometry(bad, o.cumf.astype(np.float32), o.vid_freq, o.txt_freq, o.nwin, o.Lv, 5)
    bad = o.vidx.astype(np.float32).copy()
    bad[0] = o.Lv  # outside the grid
    with pytest.raises(awa.AwaError):
        ctx.set_geometry(bad, o.cumf.astype(np.float32), o.vid_freq, o.txt_freq, o.nwin, o.Lv, 5)
    vf = o.vid_freq.copy()
    vf[0, 1] += 1.0  # channel pair no longer repeated
    with pytest.raises(awa.AwaError):
        ctx.set_geometry(o.vidx.astype(np.float32), o.cumf.astype(np.float32), vf, o.txt_freq, o.nwin, o.Lv, 5)


def test_cpp_host_mirror():
    """The C++ AwaLayer / AwaVk mirror (csrc/awa_layer.hpp) as a standalone
    executable, like the reference's own test programs."""
    import subprocess
    exe = os.path.join(os.path.dirname(__file__), "cpp", "bin", "test_awa_layer")
    assert os.path.exists(exe), "build it: make -C seedvr2-2b-ncnn_amd tests"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.parametrize("name,shifted", [("cfg2_1080p", 1), ("cfg4_ragged", 0), ("cfg5_frames", 1),
                                          ("cfg0_360p", 0)])
def test_geometry_from_reference_win_file(oracle, ctx, awa, tmp_path, name, shifted):
    """A win_*.bin file in load_win's layout (dit_vk.cpp:74-93), read by
    dit_read_win and bound through awa_geom_from_win (the reference's Win,
    awa_vk.h:40-45), gives the same geometry as awa_geom_build and the same
    output bits."""
    import torch
    from model_files import write_win
    grid, nw, txt, seed, frac = CONFIGS[name]
    og = oracle.Geometry(*grid, nw, txt, shifted)
    path = tmp_path / "win.bin"
    write_win(str(path), [*grid, *nw, 0, 0, 0, og.nwin], og.slices, og.vid_freq, og.txt_freq)
    d = awa.read_win(path, txt)
    gw = ctx.geometry_from_win(*grid, d["slices"], d["vid_freq"], d["txt_freq"], txt)
    gb = ctx.build_geometry(*grid, nw, txt, shifted)
    rw, rb = gw.read(), gb.read()
    for k in ("slices", "cumf", "vidx"):
        assert np.array_equal(rw[k], rb[k]), k
    for k in ("vid_freq", "txt_freq"):
        assert np.array_equal(rw[k].view(np.uint32), rb[k].view(np.uint32)), k
    assert gw.info() == gb.info()
    vqkv, tqkv, gains = seeded_awa_inputs(og.Lv, txt, seed, frac)
    dtypes = [torch.bfloat16] + ([torch.float32] if og.Lv <= 3200 else [])
    for dt in dtypes:
        note(f"win file {name} shifted={shifted} {dt}")
        a = run_gpu(ctx, gw, vqkv, tqkv, gains, dt)
        b = run_gpu(ctx, gb, vqkv, tqkv, gains, dt)
        assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
        assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    gw.close()
    gb.close()


@pytest.mark.parametrize("txt", [58, 77])
def test_window_without_video_rows(oracle, ctx, awa, txt):
    """A win file whose windows include one with no tokens (an empty slice on
    the h axis), as load_win accepts (dit_vk.cpp:74-93).  Its text rows attend
    to the text keys only and still count in the text average (dit_vk.cpp:
    440-444).  With 58 text rows the window's work item has a single key tile
    of its own, which the bf16 kernel's DMA stream pads to two (a regression
    case: the next item on that slot once read the wrong K and V tiles)."""
    import types
    import torch
    grid, nw = (1, 23, 27), (4, 3, 3)
    og = oracle.Geometry(*grid, nw, txt, 0)
    for at in (0, 2, og.nwin):
        sl = np.insert(og.slices, at, [0, 1, 5, 5, 0, 27], axis=0).astype(np.int32)
        nwin = og.nwin + 1
        tf = np.ascontiguousarray(np.concatenate([og.txt_freq[:txt]] * nwin))
        geo = types.SimpleNamespace(t=1, h=23, w=27, Lv=og.Lv, txt_len=txt, slices=sl, nwin=nwin,
                                    vid_freq=og.vid_freq, txt_freq=tf)
        g = ctx.geometry_from_win(*grid, sl, og.vid_freq, tf, txt)
        assert g.info()["nwin"] == nwin
        vq, tq, gains = seeded_awa_inputs(og.Lv, txt, 60 + at)
        note(f"empty window at {at} txt={txt}")
        rv, rt = oracle.awa_forward(oracle.bf16_round(vq), oracle.bf16_round(tq), geo, *gains, eps=1e-5)
        va, ta = run_gpu(ctx, g, vq, tq, gains, torch.bfloat16)
        for out, ref in ((va, oracle.bf16_round(rv)), (ta, oracle.bf16_round(rt))):
            cos, rel, md = metrics(out, ref)
            note(f"  bf16 cos={cos:.8f} rel={rel:.2e}")
            assert np.all(np.isfinite(out)) and cos >= BF16_COS, cos
        rv, rt = oracle.awa_forward(vq, tq, geo, *gains, eps=1e-5)
        va, ta = run_gpu(ctx, g, vq, tq, gains, torch.float32)
        for out, ref in ((va, rv), (ta, rt)):
            f32_check(out, ref, "f32 ")
        g.close()


def test_geometry_from_win_rejects(oracle, ctx, awa):
    """Slices outside the grid and a token in two windows are refused."""
    og = oracle.Geometry(1, 23, 27, (4, 3, 3), 58, 0)
    def vf_for(sl):
        return np.zeros((int(np.prod(sl[:, 1::2] - sl[:, 0::2], axis=1).sum()), 126), np.float32)

    sl = og.slices.copy()
    sl[0, 3] = 24  # h end beyond the grid
    with pytest.raises(awa.AwaError, match="outside"):
        ctx.geometry_from_win(1, 23, 27, sl, vf_for(sl), og.txt_freq, 58)
    sl = og.slices.copy()
    s0 = sl[0]
    sl[1] = [s0[0], s0[0] + 1, s0[2], s0[2] + 1, s0[4], s0[4] + 1]  # window 0's first token again
    with pytest.raises(awa.AwaError, match="two windows"):
        ctx.geometry_from_win(1, 23, 27, sl, vf_for(sl), og.txt_freq, 58)


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 16, (56 << 20) + 48])
def test_stream_copy(ctx, awa, nbytes):
    """awa_stream_copy (the measuring copy) moves every byte, including a
    partial last block, and rejects sizes that are not multiples of 16."""
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(nbytes)
    src = torch.randint(0, 255, (nbytes,), generator=g, device=dev, dtype=torch.uint8)
    dst = torch.zeros_like(src)
    ctx.stream_copy(src, dst)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    with pytest.raises(awa.AwaError):
        ctx.stream_copy(src[:-8], dst[:-8])

"""GPU parity of the DiT block (include/dit_capi.h) against the layer reference.

Bars: the plain GEMM kernel within bf16 output rounding of an fp32 product;
one layer's hidden-state output cos >= 0.9999 (bf16 bar of the op's
specification), checked also on the layer's update x_out - x_in (a stricter
view, since x_in dominates x_out).
"""
import sys

import numpy as np
import pytest

from conftest import metrics, random_shapes
from dit_reference import layer_emulation, random_branch, random_emb, to_device

pytestmark = pytest.mark.gpu

BF16_COS = 0.9999


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("shape", [(5440, 7680, 2560), (58, 7680, 2560), (5498, 2560, 6912),
                                   (1, 256, 64), (300, 512, 128)])
def test_gemm_bf16(ctx, shape):
    import torch
    M, N, K = shape
    note(f"gemm M={M} N={N} K={K}")
    g = torch.Generator(device="cpu").manual_seed(M + N + K)
    A = torch.randn((M, K), generator=g).to("cuda", torch.bfloat16)
    W = (0.05 * torch.randn((N, K), generator=g)).to("cuda", torch.bfloat16)
    C = ctx.gemm(A, W)
    ref = torch.mm(A.float(), W.float().t().contiguous())
    torch.cuda.synchronize()
    cos, rel, _ = metrics(C.float().cpu().numpy(), ref.cpu().numpy())
    note(f"  cos={cos:.8f} rel={rel:.2e}")
    assert cos >= 0.99999 and rel <= 1e-2


def test_gemm_rejects_bad_shapes(ctx, awa):
    import torch
    A = torch.zeros((8, 64), dtype=torch.bfloat16, device="cuda")
    W = torch.zeros((100, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(awa.AwaError):
        ctx.gemm(A, W)
    # N or K above the kernel's 32-bit resource ranges (2^20): rejected
    # before any device work (the shapes are not backed by the buffers)
    import ctypes as C
    for n, k in (((1 << 20) + 256, 64), (256, (1 << 20) + 64)):
        rc = awa.lib().dit_gemm_bf16(ctx.ptr, C.c_void_p(A.data_ptr()), C.c_void_p(W.data_ptr()),
                                     C.c_void_p(A.data_ptr()), 8, n, k, None)
        assert rc != 0, (n, k)
    g = ctx.build_geometry(1, 4, 4, (1, 1, 1), 3, 0)
    with pytest.raises(awa.AwaError):
        ctx.dit_reserve(g, (1 << 19) + 128)
    g.close()


def test_time_embedding(oracle, ctx):
    import torch
    rng = np.random.default_rng(30)
    emb_ref, ws = random_emb(rng, oracle)
    dws = [torch.from_numpy(w).cuda() for w in ws]
    emb = ctx.time_embedding(1000.0, *dws)
    torch.cuda.synchronize()
    cos, rel, _ = metrics(emb.cpu().numpy(), emb_ref)
    assert cos >= 0.999999 and rel <= 1e-5, (cos, rel)


def run_layer(oracle, ctx, grid, nw, TXT, shifted, mlp, kind, seed):
    import torch
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)
    og = oracle.Geometry(*grid, nw, TXT, shifted)
    emb, _ = random_emb(rng, oracle)
    vb = random_branch(rng, mlp, oracle)
    tb = vb if kind == "shared" else random_branch(rng, mlp, oracle)
    x = rng.standard_normal((og.Lv + TXT, 2560)).astype(np.float32)
    last = kind == "last"
    ref = layer_emulation(oracle, x, emb, vb, tb, og, og.Lv, TXT, last=last, bf16=True)
    geom = ctx.build_geometry(*grid, nw, TXT, shifted)
    dvb = to_device(vb, mlp, ctx, dev)
    dtb = dvb if tb is vb else to_device(tb, mlp, ctx, dev)
    dx = torch.from_numpy(x).to(dev)
    demb = torch.from_numpy(emb).to(dev)
    ctx.layer(geom, dvb, dtb, demb, dx, og.Lv, TXT, mlp=mlp, txt_vid_only=last)
    torch.cuda.synchronize()
    out = dx.cpu().numpy()
    return x, out, ref, og.Lv


@pytest.mark.parametrize("kind", ["shared", "dual", "last"])
@pytest.mark.parametrize("shifted", [0, 1])
def test_layer_small(oracle, ctx, kind, shifted):
    note(f"layer small {kind} shifted={shifted}")
    x, out, ref, Lv = run_layer(oracle, ctx, (1, 12, 20), (4, 3, 3), 9, shifted, 256, kind, 40 + shifted)
    for sl in (slice(0, Lv), slice(Lv, None)):
        cos, rel, _ = metrics(out[sl], ref[sl])
        dcos, drel, _ = metrics(out[sl] - x[sl], ref[sl] - x[sl])
        note(f"  cos={cos:.8f} update cos={dcos:.7f} rel={drel:.2e}")
        assert cos >= BF16_COS and dcos >= 0.999, (cos, dcos)


LAYER_SHAPES = random_shapes(6, seed=77, max_rows=700)


@pytest.mark.parametrize("k", range(len(LAYER_SHAPES)))
def test_layer_random_shapes(oracle, ctx, k):
    """Whole layers on seeded random shapes (random_shapes, up to 700 video rows
    and 1-140 text rows), the three kinds in turn: the block's GEMMs see row
    counts M = Lv + TXT (and the branches' Lv and TXT) at many offsets within
    their 224- and 256-row tiles, which their epilogues bound through buffer
    resources."""
    t, h, w, nw, txt, sh = LAYER_SHAPES[k]
    kind = ("shared", "dual", "last")[k % 3]
    note(f"layer random shape {k}: grid ({t},{h},{w}) windows {nw} txt {txt} shifted {sh} {kind}")
    x, out, ref, Lv = run_layer(oracle, ctx, (t, h, w), nw, txt, sh, 256, kind, 70 + k)
    for sl in (slice(0, Lv), slice(Lv, None)):
        cos, rel, _ = metrics(out[sl], ref[sl])
        dcos, drel, _ = metrics(out[sl] - x[sl], ref[sl] - x[sl])
        note(f"  cos={cos:.8f} update cos={dcos:.7f} rel={drel:.2e}")
        assert np.all(np.isfinite(out[sl]))
        assert cos >= BF16_COS and dcos >= 0.999, (cos, dcos)


@pytest.mark.parametrize("kind,mlp", [("shared", 6912), ("dual", 6912), ("shared", 10240)])
def test_layer_1080p(oracle, ctx, kind, mlp):
    """One full-size layer (1x68x80 grid, TXT 58), odd (shifted) geometry, at the
    reference checkpoint's MLP width 6912 (dit_vk.cpp:19) and at 10240, the MLP
    width of the 1080p DiT-step workload's stated shape (timed by bench.py as
    the MLP-10240 step)."""
    note(f"layer 1080p {kind} mlp={mlp}")
    x, out, ref, Lv = run_layer(oracle, ctx, (1, 68, 80), (4, 3, 3), 58, 1, mlp, kind, 50)
    for sl in (slice(0, Lv), slice(Lv, None)):
        cos, rel, _ = metrics(out[sl], ref[sl])
        dcos, drel, _ = metrics(out[sl] - x[sl], ref[sl] - x[sl])
        note(f"  cos={cos:.8f} update cos={dcos:.7f} rel={drel:.2e}")
        assert cos >= BF16_COS and dcos >= 0.999, (cos, dcos)


@pytest.mark.parametrize("key", ["attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"])
def test_last_layer_ignores_text_ada(oracle, ctx, key):
    """dit_layer_forward with txt_vid_only = 1 (forward_latent's last layer,
    dit_vk.cpp:523-620): a different text-branch ada vector leaves every
    output row unchanged, bit for bit; with txt_vid_only = 0 it changes the
    text rows."""
    import torch
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(70)
    grid, nw, TXT, mlp = (1, 12, 20), (4, 3, 3), 9, 256
    og = oracle.Geometry(*grid, nw, TXT, 1)
    emb, _ = random_emb(rng, oracle)
    vb = random_branch(rng, mlp, oracle)
    tb = random_branch(rng, mlp, oracle)
    tb2 = dict(tb)
    tb2[key] = tb[key] + 0.5 + rng.standard_normal(tb[key].shape).astype(np.float32)
    x = rng.standard_normal((og.Lv + TXT, 2560)).astype(np.float32)
    geom = ctx.build_geometry(*grid, nw, TXT, 1)
    dvb = to_device(vb, mlp, ctx, dev)
    demb = torch.from_numpy(emb).to(dev)
    for last in (True, False):
        outs = []
        for t in (tb, tb2):
            dx = torch.from_numpy(x).to(dev)
            ctx.layer(geom, dvb, to_device(t, mlp, ctx, dev), demb, dx, og.Lv, TXT, mlp=mlp, txt_vid_only=last)
            torch.cuda.synchronize()
            outs.append(dx.cpu().numpy())
        if last:
            assert np.array_equal(outs[0], outs[1]), key
        else:
            assert not np.array_equal(outs[0][og.Lv:], outs[1][og.Lv:]), key
    geom.close()


def test_embed_and_final(oracle, ctx):
    """dit_embed / dit_final (input projections and the output layer) against
    their emulation at the block's bf16 rounding points."""
    import torch
    from dit_reference import embed_emulation, final_emulation, io_to_device, random_io
    note("embed / final")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(60)
    T, H, W, TXT = 2, 24, 40, 9
    io = random_io(rng, oracle)
    grid = rng.standard_normal((T, H, W, 33)).astype(np.float32)
    txt = rng.standard_normal((TXT, 5120)).astype(np.float32)
    emb, _ = random_emb(rng, oracle)
    dio = ctx.io_layers(io_to_device(io, dev))
    x = ctx.embed(dio, torch.from_numpy(grid).to(dev), torch.from_numpy(txt).to(dev))
    torch.cuda.synchronize()
    ref = embed_emulation(oracle, grid, txt, io)
    cos, rel, _ = metrics(x.cpu().numpy(), ref)
    note(f"  embed cos={cos:.8f} rel={rel:.2e}")
    assert cos >= 0.99999 and rel <= 1e-3, (cos, rel)
    out = ctx.final(dio, torch.from_numpy(emb).to(dev), x, T, H, W)
    torch.cuda.synchronize()
    Lv = T * (H // 2) * (W // 2)
    ref_out = final_emulation(oracle, x.cpu().numpy()[:Lv], emb, io, T, H, W)
    cos, rel, _ = metrics(out.cpu().numpy(), ref_out)
    note(f"  final cos={cos:.8f} rel={rel:.2e}")
    assert out.shape == (T, H, W, 16)
    assert cos >= BF16_COS, (cos, rel)


def test_embed_rejects_odd_grid(ctx, awa):
    import torch
    from dit_reference import io_to_device, random_io
    rng = np.random.default_rng(61)
    dio = ctx.io_layers(io_to_device(random_io(rng), torch.device("cuda:0")))
    grid = torch.zeros((1, 5, 8, 33), device="cuda:0")
    txt = torch.zeros((4, 5120), device="cuda:0")
    x = torch.empty((2 * 4 + 4, 2560), device="cuda:0")
    with pytest.raises(awa.AwaError):
        ctx.embed(dio, grid, txt, x=x)


def test_forward_grid_two_layers(oracle, ctx):
    """forward_grid (dit_vk.cpp:752-763) with two layers (unshifted, then shifted
    geometry, dual branches on the first): grid in, 16-channel grid out."""
    import torch
    from dit_reference import embed_emulation, final_emulation, io_to_device, random_io
    note("forward_grid 2 layers")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(62)
    T, H, W, TXT, mlp, nw = 1, 24, 40, 9, 256, (4, 3, 3)
    io = random_io(rng, oracle)
    grid = rng.standard_normal((T, H, W, 33)).astype(np.float32)
    txt = rng.standard_normal((TXT, 5120)).astype(np.float32)
    emb, _ = random_emb(rng, oracle)
    b0v, b0t, b1 = (random_branch(rng, mlp, oracle) for _ in range(3))
    g = [oracle.Geometry(T, H // 2, W // 2, nw, TXT, s) for s in (0, 1)]
    Lv = g[0].Lv
    x = embed_emulation(oracle, grid, txt, io)
    x = layer_emulation(oracle, x, emb, b0v, b0t, g[0], Lv, TXT)
    x = layer_emulation(oracle, x, emb, b1, b1, g[1], Lv, TXT)
    ref = final_emulation(oracle, x[:Lv], emb, io, T, H, W)

    dio = ctx.io_layers(io_to_device(io, dev))
    geoms = [ctx.build_geometry(T, H // 2, W // 2, nw, TXT, s) for s in (0, 1)]
    d0v, d0t, d1 = (to_device(b, mlp, ctx, dev) for b in (b0v, b0t, b1))
    demb = torch.from_numpy(emb).to(dev)
    dx = ctx.embed(dio, torch.from_numpy(grid).to(dev), torch.from_numpy(txt).to(dev))
    ctx.layer(geoms[0], d0v, d0t, demb, dx, Lv, TXT, mlp=mlp)
    ctx.layer(geoms[1], d1, d1, demb, dx, Lv, TXT, mlp=mlp)
    out = ctx.final(dio, demb, dx, T, H, W)
    torch.cuda.synchronize()
    cos, rel, _ = metrics(out.cpu().numpy(), ref)
    note(f"  out cos={cos:.8f} rel={rel:.2e}")
    assert cos >= BF16_COS, (cos, rel)


@pytest.mark.parametrize("thw", [(1, 24, 40), (3, 16, 22)])
def test_forward_grid_call(oracle, ctx, thw):
    """dit_forward_grid in one call (embed, timestep MLP, three layers with the
    last one text-free as forward_latent's, final) against the emulation chain,
    on one latent frame and on three."""
    import torch
    from dit_reference import embed_emulation, final_emulation, io_to_device, random_io
    note(f"dit_forward_grid 3 layers {thw}")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(63)
    (T, H, W), TXT, mlp, nw = thw, 9, 256, (4, 3, 3)
    io = random_io(rng, oracle)
    grid = rng.standard_normal((T, H, W, 33)).astype(np.float32)
    txt = rng.standard_normal((TXT, 5120)).astype(np.float32)
    emb, tws = random_emb(rng, oracle)   # time_embedding(1000) of these weights
    br = [random_branch(rng, mlp, oracle) for _ in range(4)]
    layers = [(br[0], br[1]), (br[2], br[2]), (br[3], br[3])]
    g = [oracle.Geometry(T, H // 2, W // 2, nw, TXT, s) for s in (0, 1)]
    Lv = g[0].Lv
    x = embed_emulation(oracle, grid, txt, io)
    for i, (vb, tb) in enumerate(layers):
        x = layer_emulation(oracle, x, emb, vb, tb, g[i % 2], Lv, TXT, last=(i == len(layers) - 1))
    ref = final_emulation(oracle, x[:Lv], emb, io, T, H, W)

    dio = ctx.io_layers(io_to_device(io, dev))
    geoms = [ctx.build_geometry(T, H // 2, W // 2, nw, TXT, s) for s in (0, 1)]
    dbr = [to_device(b, mlp, ctx, dev) for b in br]
    dl = [(dbr[0], dbr[1]), (dbr[2], dbr[2]), (dbr[3], dbr[3])]
    dtw = [torch.from_numpy(w).to(dev) for w in tws]
    out = ctx.forward_grid(dio, dtw, dl, geoms[0], geoms[1], 1000.0, torch.from_numpy(grid).to(dev),
                           torch.from_numpy(txt).to(dev), mlp=mlp, last_txt_vid_only=True)
    torch.cuda.synchronize()
    cos, rel, _ = metrics(out.cpu().numpy(), ref)
    note(f"  out cos={cos:.8f} rel={rel:.2e}")
    assert cos >= BF16_COS, (cos, rel)


SMALL_MODEL = dict(T=1, H=24, W=40, TXT=9, mlp=256, nw=(4, 3, 3), t=500.0)


def _model_reference(oracle, io_d, br_d, emb, grid, txt):
    """The two-layer small model (first layer dual) on the weights as the
    loader holds them, through the layer emulation."""
    from dit_reference import embed_emulation, final_emulation
    T, H, W, _ = grid.shape
    TXT, nw = txt.shape[0], SMALL_MODEL["nw"]
    g = [oracle.Geometry(T, H // 2, W // 2, nw, TXT, s) for s in (0, 1)]
    Lv = g[0].Lv
    x = embed_emulation(oracle, grid, txt, io_d)
    x = layer_emulation(oracle, x, emb, br_d[0], br_d[1], g[0], Lv, TXT)
    x = layer_emulation(oracle, x, emb, br_d[2], br_d[2], g[1], Lv, TXT)
    return final_emulation(oracle, x[:Lv], emb, io_d, T, H, W)


def test_model_directory(oracle, ctx, tmp_path):
    """A model directory in the reference's layout (fp16 InnerProduct weights,
    read_raw_f vectors; two layers, the first dual) through dit_model_load and
    dit_model_forward_grid, against the emulation on the weights as stored."""
    import torch
    from dit_reference import random_io
    from model_files import write_model
    note("model directory")
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(64)
    T, H, W, TXT, mlp, nw, t = (SMALL_MODEL[k] for k in ("T", "H", "W", "TXT", "mlp", "nw", "t"))
    io = random_io(rng)
    br = [random_branch(rng, mlp) for _ in range(3)]
    layers = [(br[0], br[1]), (br[2], br[2])]
    _, tws = random_emb(rng, oracle)
    write_model(str(tmp_path), io, layers, tws, mm_layers=1)
    # the weights as the loader holds them: fp16 on disk, bf16 on the device (the
    # timestep MLP stays fp32)
    h = lambda a: a.astype(np.float16).astype(np.float32)
    hb = lambda a: oracle.bf16_round(h(a))
    io_d = {k: (hb(v) if k in ("vid_in_w", "txt_in_w", "vid_out_w") else v) for k, v in io.items()}
    lin = ("qkv_w", "out_w", "mlp_in_w", "mlp_g_w", "mlp_out_w")
    br_d = [{k: (hb(v) if k in lin else v) for k, v in b.items()} for b in br]
    emb = oracle.time_embedding(t, *[h(w) if w.ndim == 2 else w for w in tws])
    grid = rng.standard_normal((T, H, W, 33)).astype(np.float32)
    txt = rng.standard_normal((TXT, 5120)).astype(np.float32)
    ref = _model_reference(oracle, io_d, br_d, emb, grid, txt)

    model = ctx.load_model(tmp_path, 2, 1)
    assert model.info() == {"n_layers": 2, "mm_layers": 1, "mlp": mlp}
    geoms = [ctx.build_geometry(T, H // 2, W // 2, nw, TXT, s) for s in (0, 1)]
    out = ctx.model_forward_grid(model, geoms[0], geoms[1], t, torch.from_numpy(grid).to(dev),
                                 torch.from_numpy(txt).to(dev))
    torch.cuda.synchronize()
    cos, rel, _ = metrics(out.cpu().numpy(), ref)
    note(f"  out cos={cos:.8f} rel={rel:.2e}")
    assert cos >= BF16_COS, (cos, rel)

    # the same forward captured in a HIP graph, replayed on new inputs: every
    # replay equals the eager forward bit for bit (no kernel here reduces with
    # atomics), with eager work and synchronisations between the replays
    note("model graph")
    s = torch.cuda.Stream()
    d_grid = torch.from_numpy(grid).to(dev)
    d_txt = torch.from_numpy(txt).to(dev)
    Lv = T * (H // 2) * (W // 2)
    x = torch.empty((Lv + TXT, 2560), dtype=torch.float32, device=dev)
    gout = torch.empty((T, H, W, 16), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    graph = ctx.model_graph(model, geoms[0], geoms[1], t, d_grid, d_txt, x, gout, stream=s)
    s.synchronize()
    assert torch.equal(gout, out), "graph creation's eager run differs from the forward"
    for rep in range(3):
        grid2 = rng.standard_normal((T, H, W, 33)).astype(np.float32)
        txt2 = rng.standard_normal((TXT, 5120)).astype(np.float32)
        d_grid.copy_(torch.from_numpy(grid2))
        d_txt.copy_(torch.from_numpy(txt2))
        torch.cuda.synchronize()
        eager = ctx.model_forward_grid(model, geoms[0], geoms[1], t, d_grid, d_txt)
        torch.cuda.synchronize()
        gout.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.launch(stream=s)
        s.synchronize()
        note(f"  replay {rep}: max |graph - eager| = {(gout - eager).abs().max().item():.3e}")
        assert torch.equal(gout, eager), rep
        if rep == 0:
            cos, rel, _ = metrics(gout.cpu().numpy(), _model_reference(oracle, io_d, br_d, emb, grid2, txt2))
            note(f"  replay cos={cos:.8f} rel={rel:.2e}")
            assert cos >= BF16_COS, (cos, rel)
    graph.close()

    # the C++ DitVk mirror (csrc/dit_vk.hpp) on the same directory and inputs:
    # the same device path, so the same bits as the forward driven from here
    # (with the last layer's text rows attending to video only, as
    # forward_latent runs them)
    note("C++ DitVk")
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(__file__), "cpp", "bin", "test_dit_vk")
    assert os.path.exists(exe), f"{exe} missing: build it with make -C seedvr2-2b-ncnn_amd tests"
    grid.tofile(tmp_path / "grid.f32")
    txt.tofile(tmp_path / "txt.f32")
    r = subprocess.run([exe, str(tmp_path), "2", "1", str(tmp_path / "grid.f32"), str(tmp_path / "txt.f32"),
                        str(T), str(H), str(W), str(TXT), repr(float(t)), str(tmp_path / "out.f32")],
                       capture_output=True, text=True, timeout=120)
    note("  " + (r.stdout + r.stderr).strip().replace("\n", "\n  "))
    assert r.returncode == 0, r.stderr
    cpp_out = np.fromfile(tmp_path / "out.f32", np.float32).reshape(T, H, W, 16)
    d_grid.copy_(torch.from_numpy(grid))
    d_txt.copy_(torch.from_numpy(txt))
    py_out = ctx.model_forward_grid(model, geoms[0], geoms[1], t, d_grid, d_txt, last_txt_vid_only=True)
    torch.cuda.synchronize()
    assert np.array_equal(cpp_out, py_out.cpu().numpy())

    # the same weights merged into one graph file (export_dit_graph.py layout),
    # the timestep MLP from the directory: the same device weights, the same output
    note("merged graph file")
    from model_files import write_graph
    write_graph(str(tmp_path), tmp_path / "g.param", tmp_path / "g.bin", 2, 1)
    gmodel = ctx.load_graph_model(tmp_path / "g.param", tmp_path / "g.bin", tmp_path)
    assert gmodel.info() == {"n_layers": 2, "mm_layers": 1, "mlp": mlp}
    d_grid.copy_(torch.from_numpy(grid))
    d_txt.copy_(torch.from_numpy(txt))
    out2 = ctx.model_forward_grid(gmodel, geoms[0], geoms[1], t, d_grid, d_txt)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
    gmodel.close()


def test_model_directory_errors(ctx, awa, tmp_path):
    """A missing or mis-shaped file fails the load with a message, nothing loaded;
    a graph cannot be captured on the null stream."""
    import ctypes as C
    with pytest.raises(awa.AwaError, match="cannot open"):
        ctx.load_model(tmp_path, 1, 0)
    h = C.c_void_p()
    rc = awa.lib().dit_graph_create(ctx.ptr, C.c_void_p(1), None, None, 0, 1e-5, 1000.0, None, 1, 2, 2, None, 1,
                                    None, None, None, C.byref(h))
    assert rc != 0 and h.value is None
    assert "null stream" in awa.lib().awa_last_error(ctx.ptr).decode()

"""The DiT block at the full workload shapes on the GPU, layer by layer.

- 32-layer 1080p stack (1x68x80 latent tokens, 58 text rows, windows (4,3,3),
  MLP 6912; layers 0-9 with separate video/text branches, 10-31 shared; even
  layers unshifted, odd shifted; t = 1000; seed 3).  The hidden state after
  every one of the 32 layers is compared with the layer reference fed the
  GPU's own input to that layer, as the reference dumps and compares after
  every layer (dit_vk.cpp:636-654); four tests of eight layers each (each
  replays the device stack from layer 0 with the same seed), with the
  reference's matrix products computed in fp32 on the device and its
  attention by the oracle on the CPU.  Two levels:
    * the block's own rounding points (bf16 GEMM inputs, qkv, attention and
      SwiGLU outputs; weights as the bf16 values the device holds):
      cos >= 0.9999, update (x_out - x_in) cos >= 0.999;
    * the reference's fp32 forward_latent arithmetic on the fp16 weight values
      of its checkpoint format (no bf16 rounding anywhere): cos >= 0.9999.  The
      device narrows fp16 weights to bf16 (3 mantissa bits fewer) and computes
      the projections from bf16 inputs; this bar measures that choice.
- The ragged stress shape: two layers (unshifted, then shifted) on a 1x71x97
  grid with 77 text rows, windows (1,4,4), hidden-state inputs with 1% of the
  entries scaled by 8, seed 4.
- The drift of a chained 32-layer stack (1x24x40 grid) against the fp32
  chain on fp16 weights, reported after every layer.

Weights are N(0, 0.02) rounded to fp16 (the checkpoint's storage), generated
on the device one layer at a time; host copies are taken only for the layers
compared.
"""
import sys

import numpy as np
import pytest

from conftest import metrics
from dit_reference import layer_emulation

pytestmark = pytest.mark.gpu

BF16_COS = 0.9999
ADA = ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate")


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_branch(ctx, gen, mlp, host):
    """Device branch (bf16 matrices from fp16 values) and, if host, two host
    copies for the layer reference: the fp16 values and the bf16 values."""
    import torch
    bf = torch.bfloat16

    def w16(*s):
        return (0.02 * torch.randn(s, generator=gen, device="cuda")).half()

    def f32(*s):
        return 0.02 * torch.randn(s, generator=gen, device="cuda")

    m = {"qkv_w": w16(7680, 2560), "out_w": w16(2560, 2560), "mlp_in_w": w16(mlp, 2560),
         "mlp_g_w": w16(mlp, 2560), "mlp_out_w": w16(2560, mlp)}
    v = {"out_b": f32(2560), "nq": 1 + f32(128), "nk": 1 + f32(128)}
    for k in ADA:
        v[k] = f32(2560)
    d = {"qkv_w": m["qkv_w"].to(bf), "out_w": m["out_w"].to(bf), "mlp_out_w": m["mlp_out_w"].to(bf)}
    d["mlp_w"] = ctx.pack_mlp(m["mlp_in_w"].to(bf), m["mlp_g_w"].to(bf))
    d.update(v)
    if not host:
        return d, None, None
    vh = {k: t.cpu().numpy() for k, t in v.items()}
    h16 = dict(vh, **{k: t.float().cpu().numpy() for k, t in m.items()})
    hbf = dict(vh, **{k: t.to(bf).float().cpu().numpy() for k, t in m.items()})
    return d, h16, hbf


def stack_layers(ctx, gen, n_layers, n_dual, mlp, keep):
    """Yields (i, video branch, text branch, host copies or None) layer by
    layer, so that only the layer in use is held."""
    for i in range(n_layers):
        vb, v16, vbf = make_branch(ctx, gen, mlp, i in keep)
        if i < n_dual:
            tb, t16, tbf = make_branch(ctx, gen, mlp, i in keep)
        else:
            tb, t16, tbf = vb, v16, vbf
        yield i, vb, tb, (((v16, t16), (vbf, tbf)) if i in keep else None)


def time_weights(gen):
    import torch
    r = lambda *s: 0.02 * torch.randn(s, generator=gen, device="cuda")
    return [r(2560, 256), r(2560), r(2560, 2560), r(2560), r(15360, 2560), r(15360)]


def device_mm():
    """fp32 a @ w.T on the device (torch.mm, full fp32: no reduced-precision
    inputs), for the layer reference at full size."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False

    def mm(a, w):
        ta = torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
        tw = torch.from_numpy(np.ascontiguousarray(w, np.float32)).cuda()
        return torch.mm(ta, tw.t().contiguous()).cpu().numpy()
    return mm


def check_layer(oracle, tag, x_in, out, emb, hosts, og, Lv, TXT, mm=None):
    (v16, t16), (vbf, tbf) = hosts
    kw = {} if mm is None else {"mm": mm}
    ref = layer_emulation(oracle, x_in, emb, vbf, tbf, og, Lv, TXT, bf16=True, **kw)
    ref32 = layer_emulation(oracle, x_in, emb, v16, t16, og, Lv, TXT, bf16=False, **kw)
    for part, sl in (("vid", slice(0, Lv)), ("txt", slice(Lv, None))):
        cos, _, _ = metrics(out[sl], ref[sl])
        dcos, _, _ = metrics(out[sl] - x_in[sl], ref[sl] - x_in[sl])
        cos32, _, _ = metrics(out[sl], ref32[sl])
        dcos32, _, _ = metrics(out[sl] - x_in[sl], ref32[sl] - x_in[sl])
        note(f"  {tag} {part}: cos={cos:.8f} update cos={dcos:.7f} | fp32 on fp16 weights: "
             f"cos={cos32:.8f} update cos={dcos32:.7f}")
        assert cos >= BF16_COS and dcos >= 0.999, (tag, part, cos, dcos)
        assert cos32 >= BF16_COS, (tag, part, cos32)


@pytest.mark.parametrize("chunk", [0, 1, 2, 3])
def test_cfg3_1080p_32_layers_layer_by_layer(oracle, ctx, chunk):
    import torch
    grid, nw, TXT, mlp = (1, 68, 80), (4, 3, 3), 58, 6912
    keep = tuple(range(8 * chunk, 8 * chunk + 8))
    mm = device_mm()
    gen = torch.Generator(device="cuda").manual_seed(3)
    note(f"cfg3: 32 layers (10 dual + 22 shared), branches generated on the device; layers {keep[0]}-{keep[-1]}")
    emb = ctx.time_embedding(1000.0, *time_weights(gen))
    Lv = grid[0] * grid[1] * grid[2]
    x = torch.randn((Lv + TXT, 2560), generator=gen, device="cuda")
    geoms = [ctx.build_geometry(*grid, nw, TXT, s) for s in (0, 1)]
    ogeoms = [oracle.Geometry(*grid, nw, TXT, s) for s in (0, 1)]
    emb_h = emb.cpu().numpy()
    for i, vb, tb, hosts in stack_layers(ctx, gen, keep[-1] + 1, 10, mlp, keep):
        if i in keep:
            torch.cuda.synchronize()
            x_in = x.cpu().numpy()
        ctx.layer(geoms[i % 2], vb, tb, emb, x, Lv, TXT, mlp=mlp)
        if i in keep:
            torch.cuda.synchronize()
            note(f"cfg3 layer {i} ({'dual' if i < 10 else 'shared'}, {'shifted' if i % 2 else 'unshifted'})")
            check_layer(oracle, f"layer {i}", x_in, x.cpu().numpy(), emb_h, hosts, ogeoms[i % 2], Lv, TXT, mm)
    assert bool(torch.isfinite(x).all())
    for g in geoms:
        g.close()


def test_cfg4_ragged_two_layers(oracle, ctx):
    import torch
    grid, nw, TXT, mlp = (1, 71, 97), (1, 4, 4), 77, 6912
    gen = torch.Generator(device="cuda").manual_seed(4)
    note("cfg4: two layers on 1x71x97, 77 text rows, windows (1,4,4)")
    emb = ctx.time_embedding(1000.0, *time_weights(gen))
    Lv = grid[0] * grid[1] * grid[2]
    x = torch.randn((Lv + TXT, 2560), generator=gen, device="cuda")
    outl = torch.rand(x.shape, generator=gen, device="cuda") < 0.01
    x[outl] *= 8.0
    geoms = [ctx.build_geometry(*grid, nw, TXT, s) for s in (0, 1)]
    ogeoms = [oracle.Geometry(*grid, nw, TXT, s) for s in (0, 1)]
    emb_h = emb.cpu().numpy()
    for i, vb, tb, hosts in stack_layers(ctx, gen, 2, 1, mlp, (0, 1)):
        torch.cuda.synchronize()
        x_in = x.cpu().numpy()
        ctx.layer(geoms[i % 2], vb, tb, emb, x, Lv, TXT, mlp=mlp)
        torch.cuda.synchronize()
        note(f"cfg4 layer {i} ({'shifted' if i % 2 else 'unshifted'}, {ogeoms[i % 2].nwin} windows)")
        check_layer(oracle, f"layer {i}", x_in, x.cpu().numpy(), emb_h, hosts, ogeoms[i % 2], Lv, TXT)
    for g in geoms:
        g.close()


def test_chained_drift_32_layers(oracle, ctx):
    """The GPU's 32 chained layers against the fp32 chain on fp16 weights (the
    reference's forward_latent arithmetic), after every layer: 1 - cos of the
    hidden state, and cos of the accumulated update x_i - x_0 (with N(0, 0.02)
    weights the N(0, 1) input dominates the hidden state, so the update shows
    the drift).  The reference reports its own bf16 graph path against its
    fp32 path at cos 0.9999913 after layer 2 and 0.9993-0.9995 after layer 30
    (bench/LAYER_COMPARISON.md:14-17); the bar here is 0.999 for the hidden
    state and for the accumulated update on every layer."""
    import torch
    grid, nw, TXT, mlp = (1, 24, 40), (4, 3, 3), 58, 6912
    gen = torch.Generator(device="cuda").manual_seed(33)
    emb = ctx.time_embedding(1000.0, *time_weights(gen))
    Lv = grid[0] * grid[1] * grid[2]
    x = torch.randn((Lv + TXT, 2560), generator=gen, device="cuda")
    x0 = x.cpu().numpy()
    xr = x0.copy()
    geoms = [ctx.build_geometry(*grid, nw, TXT, s) for s in (0, 1)]
    ogeoms = [oracle.Geometry(*grid, nw, TXT, s) for s in (0, 1)]
    emb_h = emb.cpu().numpy()
    worst = 1.0
    for i, vb, tb, hosts in stack_layers(ctx, gen, 32, 10, mlp, tuple(range(32))):
        ctx.layer(geoms[i % 2], vb, tb, emb, x, Lv, TXT, mlp=mlp)
        (v16, t16), _ = hosts
        xr = layer_emulation(oracle, xr, emb_h, v16, t16, ogeoms[i % 2], Lv, TXT, bf16=False)
        torch.cuda.synchronize()
        out = x.cpu().numpy()
        line = []
        for part, sl in (("vid", slice(0, Lv)), ("txt", slice(Lv, None))):
            c, _, _ = metrics(out[sl], xr[sl])
            cu, _, _ = metrics(out[sl] - x0[sl], xr[sl] - x0[sl])
            line.append(f"{part} 1-cos={1 - c:.2e} update cos={cu:.7f}")
            worst = min(worst, c, cu)
        note(f"  chained layer {i:2d}: " + "  ".join(line))
    assert worst >= 0.999, worst
    for g in geoms:
        g.close()

"""GPU parity on a seeded sweep of random AWA shapes (tests/conftest.py
random_shapes: 1-4 latent frames, thin and square grids up to 2,500 video rows,
1-3 windows in time and 1-6 per spatial axis, 1-140 text rows, both
geometries; inputs N(0, 1) with 1 % of the values x8), through the C ABI against
the oracle (AWA_SWEEP_N / AWA_SWEEP_SEED widen or move the sweep):
  - the device geometry (slices, cumf, vidx, RoPE tables): bit-exact;
  - bf16 storage: cos >= 0.9999 against the reference bf16 path (bf16 inputs
    widened exactly, fp32 attention, outputs rounded to nearest even);
  - fp32 storage: cos >= 0.99999 and max|d| / max|ref| <= 1e-4.
The same shapes pass the planner's CPU checks first (tests/test_plan_cpu.py:
every item scheduled once, every slot's DMA stream replayed)."""
import sys

import numpy as np
import pytest

from conftest import metrics, random_shapes, seeded_awa_inputs

pytestmark = pytest.mark.gpu

SHAPES = random_shapes()


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("k", range(len(SHAPES)))
def test_random_shape(oracle, ctx, k):
    import torch
    dev = torch.device("cuda:0")
    t, h, w, nw, txt, sh = SHAPES[k]
    note(f"random shape {k}: grid ({t},{h},{w}) windows {nw} txt {txt} shifted {sh}")
    g = ctx.build_geometry(t, h, w, nw, txt, sh)
    o = oracle.Geometry(t, h, w, nw, txt, sh)
    d = g.read()
    assert g.info()["nwin"] == o.nwin and g.info()["Lv"] == o.Lv
    assert np.array_equal(d["slices"], o.slices)
    assert np.array_equal(d["cumf"], o.cumf)
    assert np.array_equal(d["vidx"], o.vidx)
    assert np.array_equal(d["vid_freq"].view(np.uint32), o.vid_freq.view(np.uint32))
    assert np.array_equal(d["txt_freq"].view(np.uint32), o.txt_freq.view(np.uint32))
    vq, tq, gains = seeded_awa_inputs(o.Lv, txt, 100 + k, outlier_frac=0.01)
    g4 = [torch.from_numpy(x).to(dev) for x in gains]
    rv, rt = oracle.awa_forward(oracle.bf16_round(vq), oracle.bf16_round(tq), o, *gains, eps=1e-5)
    refs = {"bf16": (oracle.bf16_round(rv), oracle.bf16_round(rt))}
    refs["f32"] = oracle.awa_forward(vq, tq, o, *gains, eps=1e-5)
    for name, dt in (("bf16", torch.bfloat16), ("f32", torch.float32)):
        va, ta = ctx.forward(g, torch.from_numpy(vq).to(dev, dt), torch.from_numpy(tq).to(dev, dt), *g4, eps=1e-5)
        torch.cuda.synchronize()
        for out, ref in ((va.float().cpu().numpy(), refs[name][0]), (ta.float().cpu().numpy(), refs[name][1])):
            cos, rel, _ = metrics(out, ref)
            note(f"  {name}: cos={cos:.8f} rel={rel:.2e}")
            assert np.all(np.isfinite(out))
            if name == "bf16":
                assert cos >= 0.9999, cos
            else:
                assert cos >= 0.99999 and rel <= 1e-4, (cos, rel)
    g.close()

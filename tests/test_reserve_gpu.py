"""awa_reserve / dit_reserve: after the reservation, the op (fp32 storage, whose
scratch the geometry build does not size) and a whole DiT layer are captured
into a HIP graph on a fresh context with no eager call first; three replays,
with eager work between them, equal the eager results bit for bit."""
import numpy as np
import pytest

from conftest import seeded_awa_inputs
from dit_reference import random_branch, random_emb, to_device

pytestmark = pytest.mark.gpu


def test_op_capture_after_reserve(awa):
    import torch
    dev = torch.device("cuda:0")
    c = awa.Context(0)
    try:
        g = c.build_geometry(1, 12, 20, (4, 3, 3), 9, 1)
        Lv = g.info()["Lv"]
        vqkv, tqkv, gains = seeded_awa_inputs(Lv, 9, 31, 0.01)
        vq, tq = torch.from_numpy(vqkv).to(dev), torch.from_numpy(tqkv).to(dev)
        g4 = [torch.from_numpy(x).to(dev) for x in gains]
        va = torch.empty((Lv, 2560), dtype=torch.float32, device=dev)
        ta = torch.empty((9, 2560), dtype=torch.float32, device=dev)
        c.reserve(g, "f32")
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            c.forward(g, vq, tq, *g4, vattn=va, tattn=ta)
        ref_v, ref_t = c.forward(g, vq, tq, *g4)
        torch.cuda.synchronize()
        for _ in range(3):
            va.zero_()
            ta.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(va, ref_v) and torch.equal(ta, ref_t)
            c.forward(g, vq, tq, *g4)  # eager work between replays
            torch.cuda.synchronize()
        del graph
        g.close()
    finally:
        c.close()


def test_layer_capture_after_reserve(awa, oracle):
    import torch
    dev = torch.device("cuda:0")
    c = awa.Context(0)
    try:
        rng = np.random.default_rng(32)
        mlp, TXT = 256, 9
        og = oracle.Geometry(1, 12, 20, (4, 3, 3), TXT, 0)
        emb, _ = random_emb(rng, oracle)
        vb = to_device(random_branch(rng, mlp, oracle), mlp, c, dev)
        tb = to_device(random_branch(rng, mlp, oracle), mlp, c, dev)
        g = c.build_geometry(1, 12, 20, (4, 3, 3), TXT, 0)
        x0 = torch.from_numpy(rng.standard_normal((og.Lv + TXT, 2560)).astype(np.float32)).to(dev)
        demb = torch.from_numpy(emb).to(dev)
        c.dit_reserve(g, mlp)
        dx = x0.clone()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            c.layer(g, vb, tb, demb, dx, og.Lv, TXT, mlp=mlp)
        dy = x0.clone()
        for _ in range(3):  # each replay applies the layer again, as the eager call does
            graph.replay()
            torch.cuda.synchronize()
            c.layer(g, vb, tb, demb, dy, og.Lv, TXT, mlp=mlp)
            torch.cuda.synchronize()
            assert torch.equal(dx, dy)
        del graph
        g.close()
    finally:
        c.close()

"""awa_forward_noalloc (the entry point that allocates nothing) against
awa_forward, through the C ABI: bit-identical outputs on two calls in a row,
the second with a smaller input, and on an fp32 call; no change of the
device's free memory across the calls; geometries whose scratch exceeds the
fixed array are refused with AWA_EARG before any kernel runs."""
import ctypes as C
import sys

import numpy as np
import pytest

from conftest import seeded_awa_inputs

pytestmark = pytest.mark.gpu


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def hip_free_bytes():
    import torch  # noqa: F401  (its HIP runtime is the one the library uses)
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


CASES = [  # grid, num_windows, txt, shifted, dtype name, seed
    ((1, 68, 80), (4, 3, 3), 58, 1, "bf16", 40),
    ((1, 45, 53), (4, 3, 3), 58, 0, "bf16", 41),
    ((1, 23, 27), (4, 3, 3), 58, 0, "f32", 42),
]


def test_noalloc_matches_forward(awa):
    import torch
    dev = torch.device("cuda:0")
    ref_ctx = awa.Context(0)
    na_ctx = awa.Context(0)  # never runs awa_forward
    runs = []
    for grid, nw, txt, sh, dt, seed in CASES:
        dtype = torch.bfloat16 if dt == "bf16" else torch.float32
        g_ref = ref_ctx.build_geometry(*grid, nw, txt, sh)
        g_na = na_ctx.build_geometry(*grid, nw, txt, sh)
        vqkv, tqkv, gains = seeded_awa_inputs(grid[0] * grid[1] * grid[2], txt, seed)
        vq = torch.from_numpy(vqkv).to(dev, dtype)
        tq = torch.from_numpy(tqkv).to(dev, dtype)
        g4 = [torch.from_numpy(x).to(dev) for x in gains]
        note(f"noalloc case {grid} shifted={sh} {dt}: awa_forward")
        va, ta = ref_ctx.forward(g_ref, vq, tq, *g4, eps=1e-5)
        out_v = torch.empty_like(va)
        out_t = torch.empty_like(ta)
        runs.append((grid, dt, g_na, vq, tq, g4, va, ta, out_v, out_t))
    torch.cuda.synchronize()
    # the calls run back to back between the two readings of the free device
    # memory; the comparisons (whose temporaries torch allocates) come after
    free0 = hip_free_bytes()
    for grid, dt, g_na, vq, tq, g4, va, ta, out_v, out_t in runs:
        note(f"noalloc case {grid} {dt}: awa_forward_noalloc")
        na_ctx.forward(g_na, vq, tq, *g4, eps=1e-5, vattn=out_v, tattn=out_t, noalloc=True)
        torch.cuda.synchronize()
    free1 = hip_free_bytes()
    assert free1 == free0, (free0, free1)
    for grid, dt, g_na, vq, tq, g4, va, ta, out_v, out_t in runs:
        bits = torch.int16 if dt == "bf16" else torch.int32
        assert torch.equal(out_v.view(bits), va.view(bits)), (grid, dt)
        assert torch.equal(out_t.view(bits), ta.view(bits)), (grid, dt)
    for r in runs:
        r[2].close()
    ref_ctx.close()
    na_ctx.close()


def test_noalloc_refuses_oversized_geometry(awa):
    """1080p with fp32 storage needs about 200 MiB of scratch, more than the
    fixed array holds: refused before any kernel is enqueued."""
    import torch
    dev = torch.device("cuda:0")
    ctx = awa.Context(0)
    g = ctx.build_geometry(1, 68, 80, (4, 3, 3), 58, 1)
    vq = torch.zeros((5440, 7680), dtype=torch.float32, device=dev)
    tq = torch.zeros((58, 7680), dtype=torch.float32, device=dev)
    gains = [torch.ones(128, device=dev) for _ in range(4)]
    with pytest.raises(awa.AwaError) as e:
        ctx.forward(g, vq, tq, *gains, eps=1e-5, noalloc=True)
    assert e.value.code == awa.AWA_EARG
    assert "at most" in str(e.value)
    g.close()
    ctx.close()

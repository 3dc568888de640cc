import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "seedvr2-2b-ncnn_amd")
for p in (os.path.join(ROOT, "oracle"), PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def awa():
    """The HIP binding; its import fails loudly when the library is missing."""
    import awa_hip
    awa_hip.lib()
    return awa_hip


@pytest.fixture(scope="session")
def ctx(awa):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    c = awa.Context(0)
    yield c
    c.close()


def metrics(out, ref):
    """cos, max|d| / max|ref| (the relative error bar used throughout), max|d|."""
    a = np.asarray(out, np.float64).ravel()
    b = np.asarray(ref, np.float64).ravel()
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
    md = float(np.max(np.abs(a - b))) if a.size else 0.0
    rel = md / (float(np.max(np.abs(b))) + 1e-30)
    return cos, rel, md


def rel_elementwise(out, ref, floor=1e-3):
    """Elementwise relative error max |out - ref| / |ref| over the elements with
    |ref| >= floor * max|ref| (below the floor a relative error measures
    cancellation in the reference, not the result), and the count of such
    elements."""
    a = np.asarray(out, np.float64).ravel()
    b = np.asarray(ref, np.float64).ravel()
    big = np.abs(b) >= floor * np.max(np.abs(b))
    if not big.any():
        return 0.0, 0
    return float(np.max(np.abs(a[big] - b[big]) / np.abs(b[big]))), int(big.sum())


def seeded_awa_inputs(Lv, txt, seed, outlier_frac=0.0, outlier_scale=8.0):
    """q/k/v ~ N(0,1) rows [Lv,7680] / [txt,7680], gains 1 + N(0,0.02)."""
    rng = np.random.default_rng(seed)
    vqkv = rng.standard_normal((Lv, 7680), dtype=np.float32)
    tqkv = rng.standard_normal((txt, 7680), dtype=np.float32)
    if outlier_frac > 0:
        for a in (vqkv, tqkv):
            m = rng.random(a.shape) < outlier_frac
            a[m] *= outlier_scale
    gains = [(1.0 + 0.02 * rng.standard_normal(128)).astype(np.float32) for _ in range(4)]
    return vqkv, tqkv, gains


def random_shapes(n=None, seed=None, max_rows=2500):
    """A seeded list of AWA shapes (t, h, w, num_windows, txt, shifted) with at
    most max_rows video rows: 1-4 frames, thin and square grids, 1-6 windows
    per spatial axis and 1-3 in time, 1-140 text rows (around the 64-row
    tile), both geometries.  The same list drives the planner's CPU stream
    check and the GPU parity sweep; AWA_SWEEP_N and AWA_SWEEP_SEED (default
    24 shapes, seed 1234) widen or move it for a run of both."""
    n = int(os.environ.get("AWA_SWEEP_N", 24)) if n is None else n
    seed = int(os.environ.get("AWA_SWEEP_SEED", 1234)) if seed is None else seed
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        t = int(rng.integers(1, 5))
        h = int(rng.integers(1, 48))
        w = int(rng.integers(1, 48))
        if t * h * w > max_rows or t * h * w < 2:
            continue
        nw = (int(rng.integers(1, 4)), int(rng.integers(1, 7)), int(rng.integers(1, 7)))
        txt = int(rng.choice([1, 2, 31, 58, 63, 64, 65, 77, 128, 140]))
        out.append((t, h, w, nw, txt, len(out) % 2))
    return out

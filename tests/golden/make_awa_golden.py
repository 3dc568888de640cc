"""Writes tests/golden/awa_ref_*.npz from the reference's own CPU attention.

Runs src/verify_dit.cpp::awa_forward (compiled unchanged into
oracle/_ref/libref_bridge.so by oracle/Makefile) on small seeded inputs and
stores its outputs.  The q/k/v projection is an exact map (q = x,
k = x[:, perm], v = 2 * x[:, ::-1], all products with 0, 1 or 2), so the test
can rebuild the same vqkv from the seed without storing it, and the
out-projection is the identity, so the stored rows are the raw attention
outputs.  Run where the reference sources are (the tests only read the
stored fixture):

    python tests/golden/make_awa_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

DIM, QKV = 2560, 7680

CASES = [
    # name, grid (t,h,w), num_windows, txt_len, shifted, seed
    ("t2_unshifted", (2, 3, 4), (2, 40, 40), 3, 0, 11),
    ("t2_shifted", (2, 3, 4), (2, 40, 40), 3, 1, 12),
]


def qkv_map():
    """[7680, 2560] weights of the exact map x -> [x, x[:, perm], 2 x[:, ::-1]]."""
    perm = np.random.default_rng(7).permutation(DIM)
    W = np.zeros((QKV, DIM), np.float32)
    W[np.arange(DIM), np.arange(DIM)] = 1.0
    W[DIM + np.arange(DIM), perm] = 1.0
    W[2 * DIM + np.arange(DIM), DIM - 1 - np.arange(DIM)] = 2.0
    return W, perm


def inputs(grid, txt_len, seed):
    rng = np.random.default_rng(seed)
    Lv = grid[0] * grid[1] * grid[2]
    vid = rng.standard_normal((Lv, DIM)).astype(np.float32)
    txt = rng.standard_normal((txt_len, DIM)).astype(np.float32)
    gains = [(1.0 + 0.02 * rng.standard_normal(128)).astype(np.float32) for _ in range(4)]
    return vid, txt, gains


def expand(x, perm):
    """vqkv rows the exact map produces."""
    return np.concatenate([x, x[:, perm], 2.0 * x[:, ::-1]], axis=1).astype(np.float32)


def main():
    R = O.ref()
    if R is None:
        sys.exit("oracle/_ref/libref_bridge.so is not built (make -C oracle)")
    W, perm = qkv_map()
    for name, grid, nw, txt_len, shifted, seed in CASES:
        geom = O.Geometry(*grid, nw, txt_len, shifted)
        vid, txt, gains = inputs(grid, txt_len, seed)
        Lv = vid.shape[0]
        vq = np.empty((Lv, QKV), np.float32)
        tq = np.empty((txt_len, QKV), np.float32)
        va = np.empty((Lv, DIM), np.float32)
        ta = np.empty((txt_len, DIM), np.float32)
        R.ref_awa_block(vid, Lv, txt, txt_len, *grid, geom.slices, geom.nwin, geom.vid_freq,
                        geom.sumf, geom.txt_freq, W, W, *gains, vq, tq, va, ta)
        assert np.array_equal(vq, expand(vid, perm)) and np.array_equal(tq, expand(txt, perm))
        meta = dict(grid=list(grid), num_windows=list(nw), txt_len=txt_len, shifted=shifted,
                    seed=seed, perm_seed=7, eps=1e-5, nwin=geom.nwin)
        np.savez_compressed(os.path.join(HERE, f"awa_ref_{name}.npz"), vattn=va, tattn=ta,
                            slices=geom.slices, meta=json.dumps(meta))
        print(name, "nwin", geom.nwin, "Lv", Lv)


if __name__ == "__main__":
    main()

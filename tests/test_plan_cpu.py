"""The attention kernel's host planner (awa::plan_tiles and awa::plan_schedule,
seedvr2-2b-ncnn_amd/csrc/awa_capi.cpp) on the CPU, through the driver
tests/cpp/test_plan.cpp (built with hipcc, linked against the built library;
no device call):
every (head, work item) of a geometry scheduled exactly once with matching
descriptors, the items of one (window, head) on one XCD, the makespan no
worse than plain longest-first (on the 1080p unshifted layer, where first fit
decreasing packs the few item sizes better, strictly lower), and the kernel's
DMA stream replayed slot by slot: every key tile an item reads is the one its
fetch two (K) or one (V) tiles earlier put into the ring, including items of
a window without video rows (one text tile of its own, padded to two).
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "seedvr2-2b-ncnn_amd")
LIB = os.path.join(PKG, "lib", "libseedvr2_awa.so")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc) or not os.path.exists(LIB):
        pytest.skip("hipcc or the built library missing")
    exe = str(tmp_path_factory.mktemp("plan") / "test_plan")
    # the shared header holds device helpers too, so the host driver is
    # compiled by hipcc, as the library's own host files are
    cmd = [hipcc, "--offload-arch=gfx950", "-std=c++17", "-O1",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG, "csrc"),
           os.path.join(ROOT, "tests", "cpp", "test_plan.cpp"), "-o", exe,
           "-L", os.path.join(PKG, "lib"), "-lseedvr2_awa", "-Wl,-rpath," + os.path.join(PKG, "lib")]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def run(driver, t, h, w, nw, txt, shifted, slots, empty_at=None):
    extra = [] if empty_at is None else [empty_at]
    r = subprocess.run([driver] + [str(x) for x in (t, h, w, *nw, txt, shifted, slots, *extra)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip().endswith("rc=0"), r.stdout[-2000:] + r.stderr[-2000:]
    m = re.search(r"makespan (\d+) lpt (\d+) mean ([\d.]+)", r.stdout)
    return int(m.group(1)), int(m.group(2)), float(m.group(3))


CASES = [
    (1, 68, 80, (4, 3, 3), 58, 0, 512),   # 1080p layers
    (1, 68, 80, (4, 3, 3), 58, 1, 512),
    (1, 45, 53, (4, 3, 3), 58, 1, 512),   # 720p
    (1, 23, 27, (4, 3, 3), 58, 0, 512),   # 360p
    (1, 71, 97, (1, 4, 4), 77, 1, 512),   # ragged grid
    (5, 23, 27, (4, 3, 3), 58, 1, 512),   # several frames
    (1, 12, 20, (1, 2, 2), 1, 1, 512),    # one text row
    (2, 9, 11, (1, 1, 1), 130, 0, 512),   # three text tiles
    (1, 68, 80, (4, 3, 3), 58, 0, 8),     # one slot per XCD
    (1, 68, 80, (4, 3, 3), 58, 1, 20),    # slot count not a multiple of 8
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}x{c[1]}x{c[2]}-s{c[5]}-n{c[6]}" for c in CASES])
def test_schedule_covers_every_item(driver, case):
    mk, lpt, mean = run(driver, *case)
    assert mk <= lpt and mk >= mean


def test_packing_beats_longest_first_on_1080p(driver):
    mk, lpt, mean = run(driver, 1, 68, 80, (4, 3, 3), 58, 0, 512)
    assert mk < lpt, (mk, lpt)


@pytest.mark.parametrize("txt", [1, 58, 64, 65])
@pytest.mark.parametrize("empty_at", [0, 3, 9])
def test_stream_with_empty_window(driver, txt, empty_at):
    """An injected geometry may hold a window without video rows (awa_geom_set
    with a repeated cumf entry, a win file with an empty slice); with at most
    64 text rows its work item has one key tile of its own."""
    mk, lpt, mean = run(driver, 1, 23, 27, (4, 3, 3), txt, 0, 16, empty_at)
    assert mk <= lpt and mk >= mean


def test_schedule_on_random_shapes(driver):
    """The seeded random shapes of the GPU parity sweep: every item scheduled
    once with matching descriptors and every slot's DMA stream replayed
    (the driver's checks), on the CPU before any of them reaches the device."""
    from conftest import random_shapes
    for t, h, w, nw, txt, sh in random_shapes():
        mk, lpt, mean = run(driver, t, h, w, nw, txt, sh, 512)
        assert mk <= lpt and mk >= mean, (t, h, w, nw, txt, sh)

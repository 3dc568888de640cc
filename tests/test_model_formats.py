"""The reference's on-disk formats through the library's readers (include/dit_model.h).

Host code only (no GPU): files written by tests/model_files.py in the formats the
reference reads (read_raw_f dit_vk.cpp:38-45, load_linear verify_dit.cpp:80-102,
load_win dit_vk.cpp:74-93) are read back through the C ABI.  The fp16 decoding is
pinned against numpy's IEEE binary16 on every one of the 65536 bit patterns.
"""
import numpy as np
import pytest

from model_files import write_linear, write_raw_f, write_win


@pytest.fixture(scope="module")
def hip():
    import sys, os
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", "seedvr2-2b-ncnn_amd"))
    import awa_hip
    awa_hip.lib()
    return awa_hip


def test_fp16_linear_all_bit_patterns(hip, tmp_path):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    w16 = bits.view(np.float16).reshape(256, 256)
    b = np.linspace(-1, 1, 256).astype(np.float32)
    write_linear(str(tmp_path / "lin"), w16, b, fp16=True)
    W, bias = hip.read_linear(tmp_path / "lin", True)
    ref = w16.astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(W), nan)
    assert np.array_equal(W[~nan], ref[~nan])
    assert np.array_equal(np.signbit(W[~nan]), np.signbit(ref[~nan]))   # -0.0 stays -0.0
    assert np.array_equal(bias, b)


def test_fp32_linear_without_bias(hip, tmp_path):
    rng = np.random.default_rng(1)
    w = rng.standard_normal((48, 20)).astype(np.float32)
    write_linear(str(tmp_path / "l32"), w, None, fp16=False)
    W, bias = hip.read_linear(tmp_path / "l32", False)
    assert bias is None and np.array_equal(W, w)


def test_raw_f_round_trip(hip, tmp_path):
    rng = np.random.default_rng(2)
    for shape in ((2560,), (3, 5, 7), (1,), ()):
        a = rng.standard_normal(shape).astype(np.float32)
        write_raw_f(str(tmp_path / "a.bin"), a)
        got = hip.read_raw_f(tmp_path / "a.bin")
        assert got.shape == a.shape and np.array_equal(got, a)


def test_win_file_matches_window_planner(hip, oracle, tmp_path):
    """A window file holding the oracle's geometry and frequency tables reads back
    split at txt_len as load_win splits it."""
    g = oracle.Geometry(1, 23, 27, (4, 3, 3), 58, 0)
    sl = np.asarray(g.slices, np.int64).reshape(-1, 6)
    hdr = [1, 23, 27, 0, 0, 0, 4, 3, 3, sl.shape[0]]
    write_win(str(tmp_path / "w.bin"), hdr, sl, g.vid_freq, g.txt_freq)
    got = hip.read_win(tmp_path / "w.bin", 58)
    assert got["header"] == hdr
    assert np.array_equal(got["slices"], sl)
    assert np.array_equal(got["vid_freq"], np.asarray(g.vid_freq, np.float32).ravel())
    assert np.array_equal(got["txt_freq"], np.asarray(g.txt_freq, np.float32).ravel())


def test_reader_errors(hip, tmp_path):
    with pytest.raises(hip.HostError, match="cannot open"):
        hip.read_raw_f(tmp_path / "missing.bin")
    write_linear(str(tmp_path / "x"), np.zeros((4, 4), np.float32), None, fp16=True)
    with open(tmp_path / "x.bin", "r+b") as f:     # an int8-quantised tag is not a float storage
        f.write(np.uint32(0x000D4B38).tobytes())
    with pytest.raises(hip.HostError, match="tag"):
        hip.read_linear(tmp_path / "x", False)
    write_linear(str(tmp_path / "y"), np.zeros((4, 4), np.float32), np.zeros(4, np.float32))
    with open(tmp_path / "y.bin", "r+b") as f:     # tag, 16 fp16 weights, half the bias
        f.truncate(4 + 32 + 8)
    with pytest.raises(hip.HostError, match="short"):
        hip.read_linear(tmp_path / "y", True)
    (tmp_path / "z.param").write_text("7767517\n1 1\nInput in0 0 1 in0\n")
    (tmp_path / "z.bin").write_bytes(b"\0" * 64)
    with pytest.raises(hip.HostError, match="InnerProduct"):
        hip.read_linear(tmp_path / "z", False)

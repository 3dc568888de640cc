"""The reference's on-disk formats through the library's readers (include/dit_model.h).

Host code only (no GPU): files written by tests/model_files.py in the formats the
reference reads (read_raw_f dit_vk.cpp:38-45, load_linear verify_dit.cpp:80-102,
load_win dit_vk.cpp:74-93) are read back through the C ABI.  The fp16 decoding is
pinned against numpy's IEEE binary16 on every one of the 65536 bit patterns, and the
InnerProduct reader against the reference's own fp16 fixture (models/test_linear.param
/.bin, a Linear 3->2 with the weights and known answer of export/make_test_model.py:
34-62).  The merged whole-model graph (export_dit_graph.py) is written from a model
directory by tests/model_files.write_graph, a restatement of the exporter, and every
weight read from it by its directory name must equal the same weight read from the
directory: the graph index follows the layers' load_model order (ada_compose.cpp,
awa_layer.cpp, ncnn InnerProduct / RMSNorm), the writer the exporter's, so a
misplaced vector or a wrong blob extent in either shows as a mismatch.
"""
import numpy as np
import pytest

import os

from model_files import write_graph, write_linear, write_model, write_raw_f, write_win

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


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


def test_reference_fp16_linear_fixture(hip):
    """models/test_linear.{param,bin} of the reference: tag 0x01306B47, fp16 weights
    [[0.1, 0.2, 0.3], [0.4, 0.5, 0.6]], fp32 bias [0.7, 0.8]; y = W [1, 2, 3] + b is
    [2.1, 4.0] up to the fp16 rounding of the weights (make_test_model.py:57-62).
    The exporter's fp32 -> fp16 conversion rounds toward zero (0.3 is stored as
    0x34CC = 0.2998, not the nearest 0x34CD), so the stored weights are the fp16
    values nearest the fp32 ones on the side of zero."""
    W, b = hip.read_linear(os.path.join(GOLDEN, "ncnn_test_linear"), True)
    x = np.array([[0.1, 0.2, 0.3], [0.4, 0.5, 0.6]], np.float32)
    h = x.astype(np.float16)
    h = np.where(np.abs(h.astype(np.float32)) > np.abs(x), np.nextafter(h, np.float16(0)), h)
    w_ref = h.astype(np.float32)
    assert W.shape == (2, 3) and np.array_equal(W, w_ref), (W, w_ref)
    assert np.array_equal(b, np.array([0.7, 0.8], np.float32))
    y = W @ np.array([1, 2, 3], np.float32) + b
    assert np.allclose(y, [2.1, 4.0], atol=2e-3), y


# a small model: the graph's layout does not depend on the widths, except the
# 128-wide qk-norm vectors of the AWA layer and AdaCompose's dim
SMALL = dict(dim=64, qkv=96, mlp=40, vid_in=35, txt_in=24, vid_out=16)


def _small_model(rng, n_layers, mm_layers):
    d, r = SMALL["dim"], lambda *s: rng.standard_normal(s).astype(np.float32)
    io = {"vid_in_w": r(SMALL["vid_in"] // 5, 5), "vid_in_b": r(SMALL["vid_in"] // 5),   # 7x5: odd fp16 count
          "txt_in_w": r(d, SMALL["txt_in"]), "txt_in_b": r(d), "vid_out_w": r(SMALL["vid_out"], d),
          "vid_out_b": r(SMALL["vid_out"]), "out_norm_w": r(d), "out_ada_shift": r(d), "out_ada_scale": r(d)}

    def branch():
        b = {"qkv_w": r(SMALL["qkv"], d), "out_w": r(d, d), "out_b": r(d), "mlp_in_w": r(SMALL["mlp"], d),
             "mlp_g_w": r(SMALL["mlp"], d), "mlp_out_w": r(d, SMALL["mlp"]), "nq": r(128), "nk": r(128)}
        for k in ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
            b[k] = r(d)
        return b

    layers = []
    for i in range(n_layers):
        vb = branch()
        layers.append((vb, branch() if i < mm_layers else vb))
    tws = [r(d, 8), r(d), r(d, d), r(d), r(6 * d, d), r(6 * d)]
    return io, layers, tws


def _directory_names(n_layers, mm_layers):
    """(name, is_linear, has_bias) of every weight a merged graph holds."""
    names = [("vid_in_proj", True, True), ("txt_in", True, True), ("vid_out_proj", True, True)]
    names += [(n, False, False) for n in ("vid_out_norm_w", "vid_out_ada_shift", "vid_out_ada_scale")]
    for i in range(n_layers):
        for base in ((f"b{i}_vid", f"b{i}_txt") if i < mm_layers else (f"b{i}_all",)):
            names += [(base + "_qkv", True, False), (base + "_out", True, True)]
            names += [(base + k, True, False) for k in ("_mlp_in", "_mlp_g", "_mlp_out")]
            names += [(f"{base}_{k}", False, False) for k in ("nq", "nk", "attn_shift", "attn_scale", "attn_gate",
                                                                "mlp_shift", "mlp_scale", "mlp_gate")]
    return names


ADA = ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate")


@pytest.mark.parametrize("ada_compose", [True, False])
def test_merged_graph_weights_match_directory(hip, tmp_path, ada_compose):
    n_layers, mm = 4, 2
    rng = np.random.default_rng(40 + ada_compose)
    io, layers, tws = _small_model(rng, n_layers, mm)
    d = str(tmp_path / "m")
    write_model(d, io, layers, tws, mm_layers=mm)
    gp, gb = tmp_path / "g.param", tmp_path / "g.bin"
    write_graph(d, gp, gb, n_layers, mm, ada_compose=ada_compose, dim=SMALL["dim"])
    names = _directory_names(n_layers, mm)
    in_graph = [n for n in names if ada_compose or not (n[0].startswith("vid_out_ada") or n[0].endswith(ADA))]
    info = hip.graph_file_info(gp, gb, -1 if ada_compose else mm)
    assert info == (n_layers, mm, len(in_graph)), info
    mm_arg = -1 if ada_compose else mm
    for name, lin, bias in in_graph:
        w, b = hip.read_graph_weight(gp, gb, name, mm_arg)
        if lin:
            W, B = hip.read_linear(os.path.join(d, name), bias)
            assert np.array_equal(w, W), name
            assert (b is None) == (B is None) and (B is None or np.array_equal(b, B)), name
        else:
            assert b is None and np.array_equal(w, hip.read_raw_f(os.path.join(d, name + ".bin")).ravel()), name
    for n in names:
        if n not in in_graph:
            with pytest.raises(hip.HostError, match="not in the graph"):
                hip.read_graph_weight(gp, gb, n[0], mm_arg)
    with pytest.raises(hip.HostError, match="not in the graph"):
        hip.read_graph_weight(gp, gb, "emb_proj_in", mm_arg)   # the host's timestep MLP


def test_merged_graph_errors(hip, tmp_path):
    n_layers, mm = 2, 1
    io, layers, tws = _small_model(np.random.default_rng(5), n_layers, mm)
    d = str(tmp_path / "m")
    write_model(d, io, layers, tws, mm_layers=mm)
    gp, gb = tmp_path / "g.param", tmp_path / "g.bin"
    write_graph(d, gp, gb, n_layers, mm, dim=SMALL["dim"])
    assert hip.graph_file_info(gp, gb)[:2] == (n_layers, mm)
    with pytest.raises(hip.HostError, match="dual-branch"):
        hip.graph_file_info(gp, gb, mm + 1)
    text, data = gp.read_text(), gb.read_bytes()
    bad = tmp_path / "bad.param"
    bad.write_text(text.replace("Input in_vid0 0 1 in_vid0\n", "Input v_cur_0 0 1 v_cur_0\n"))
    with pytest.raises(hip.HostError, match="block"):
        hip.graph_file_info(bad, gb)
    bad.write_text(text.replace("Swish sw_0_v", "Softmax sw_0_v"))
    with pytest.raises(hip.HostError, match="not part of the DiT graph"):
        hip.graph_file_info(bad, gb)
    bad.write_text(text.replace("AdaCompose", "Noop").replace(" 2=1 3=64 4=1", ""))
    with pytest.raises(hip.HostError, match="AdaCompose"):
        hip.graph_file_info(bad, gb)
    short, long_ = tmp_path / "short.bin", tmp_path / "long.bin"
    short.write_bytes(data[:-8])
    with pytest.raises(hip.HostError, match="end inside|read"):
        hip.graph_file_info(gp, short)
    long_.write_bytes(data + b"\0" * 4)
    with pytest.raises(hip.HostError, match="read"):
        hip.graph_file_info(gp, long_)
    with pytest.raises(hip.HostError, match="not an ncnn"):
        hip.graph_file_info(gb, gb)


@pytest.mark.slow
@pytest.mark.parametrize("layout", ["adacompose", "inputs"])
def test_graph_layout_matches_reference_exporter(hip, layout):
    """The reference's own exporter (export/export_dit_graph.py, run by
    tests/golden/make_graph_golden.py) wrote graph_ref_2layer.json from a
    seeded two-layer model directory.  write_graph on the same directory
    reproduces its .param line for line and token for token (the exporter
    pads with runs of spaces, which ncnn's tokenizer ignores) and its .bin
    blob for blob (offset, tag, size, SHA-256); the product's graph readers
    load the reference-written .param and return the directory's weights."""
    import importlib.util
    import json
    import tempfile
    spec = importlib.util.spec_from_file_location("mkg", os.path.join(GOLDEN, "make_graph_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    gold = json.load(open(os.path.join(GOLDEN, "graph_ref_2layer.json")))
    ref = gold["layouts"][layout]
    ada = layout == "adacompose"
    n_layers, mm = gold["n_layers"], 10   # the exporter's MM_LAYERS
    shm = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=shm) as tmp:
        model = os.path.join(tmp, "m5")
        mk.make_model_dir(model)
        gp, gb = os.path.join(tmp, "g.param"), os.path.join(tmp, "g.bin")
        write_graph(model, gp, gb, n_layers, mm, ada_compose=ada)
        text = open(gp).read()
        assert [ln.split() for ln in text.splitlines()] == [ln.split() for ln in ref["param"]]
        man = mk.manifest(text, open(gb, "rb").read())
        for got, want in zip(man["parts"], ref["bin"]["parts"]):
            assert got == want, (got, want)
        assert man == ref["bin"]

        ref_param = os.path.join(tmp, "ref.param")
        with open(ref_param, "w") as f:
            f.write("\n".join(ref["param"]) + "\n")
        mm_arg = -1 if ada else mm   # AdaCompose's 2= carries the exporter's MM_LAYERS (10)
        assert hip.graph_file_info(ref_param, gb, mm_arg)[:2] == (n_layers, mm)
        for name, bias in (("b0_vid_qkv", False), ("b1_txt_out", True), ("b1_vid_mlp_out", False),
                           ("vid_out_proj", True), ("txt_in", True)):
            w, b = hip.read_graph_weight(ref_param, gb, name, mm_arg)
            W, B = hip.read_linear(os.path.join(model, name), bias)
            assert np.array_equal(w, W) and (B is None or np.array_equal(b, B)), name
        for name in ("b1_txt_nk", "vid_out_norm_w") + (("b0_vid_mlp_gate",) if ada else ()):
            w, _ = hip.read_graph_weight(ref_param, gb, name, mm_arg)
            assert np.array_equal(w, hip.read_raw_f(os.path.join(model, name + ".bin")).ravel()), name

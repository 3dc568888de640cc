"""Writes tests/golden/graph_ref_2layer.json from the reference's own exporter.

Runs export/export_dit_graph.py (the reference's merged-graph writer, standard
library only) on a seeded two-layer model directory in the reference's layout
(both layers dual-branch, as its MM_LAYERS = 10 makes them; SwiGLU width 128),
once with AdaCompose (its default) and once without (SEEDVR_ADACOMPOSE=0), and
stores for each layout the .param text it wrote and a manifest of its .bin:
every weight blob in file order with its layer, offset, storage tag, byte
count and SHA-256, plus the size and SHA-256 of the whole file.  The test
(tests/test_model_formats.py) rebuilds the same directory from the seeds, so
only these small records are kept.  Run in the build container, where the
reference is present:

    python tests/golden/make_graph_golden.py
"""
import hashlib
import json
import os
import runpy
import struct
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
from model_files import write_model  # noqa: E402

EXPORTER = "/root/reference/export/export_dit_graph.py"
N_LAYERS, MLP, DIM = 2, 128, 2560
OUT = os.path.join(HERE, "graph_ref_2layer.json")


def make_model_dir(root):
    """The seeded two-layer model: matrices with fp16 values k 2^-17 (k an
    integer in [-2048, 2048)), vectors N(0, 1) float32; shapes of the
    reference checkpoint except the SwiGLU width."""
    rng = np.random.default_rng(77)
    h = lambda *s: rng.integers(-2048, 2048, size=s, dtype=np.int16).astype(np.float32) * np.float32(2.0 ** -17)
    f = lambda *s: rng.standard_normal(s, dtype=np.float32)
    io = {"vid_in_w": h(DIM, 132), "vid_in_b": f(DIM), "txt_in_w": h(DIM, 5120), "txt_in_b": f(DIM),
          "vid_out_w": h(64, DIM), "vid_out_b": f(64), "out_norm_w": f(DIM), "out_ada_shift": f(DIM),
          "out_ada_scale": f(DIM)}

    def branch():
        b = {"qkv_w": h(3 * DIM, DIM), "out_w": h(DIM, DIM), "out_b": f(DIM), "mlp_in_w": h(MLP, DIM),
             "mlp_g_w": h(MLP, DIM), "mlp_out_w": h(DIM, MLP), "nq": f(128), "nk": f(128)}
        for k in ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
            b[k] = f(DIM)
        return b

    layers = [(branch(), branch()) for _ in range(N_LAYERS)]
    tws = [h(DIM, 256), f(DIM), h(DIM, DIM), f(DIM), h(6 * DIM, DIM), f(6 * DIM)]
    write_model(root, io, layers, tws, mm_layers=10, fp16=True)


def manifest(param_text, data):
    """The weight blobs of a merged graph in file order, from its layer lines:
    AdaCompose 6 vectors per (layer, flow) and the output layer's 2, each a
    4-byte tag and DIM floats; InnerProduct a 4-byte tag, the [0=][2=/0=]
    weight (fp16 padded to 4 bytes, or fp32) and 0= bias floats when 1=1; AWA
    four 128-float vectors, each tagged; RMSNorm with 2=1 DIM floats, untagged."""
    parts, off = [], 0

    def take(layer, what, n, tagged):
        nonlocal off
        tag = struct.unpack_from("<I", data, off)[0] if tagged else None
        blob = data[off:off + n]
        parts.append({"layer": layer, "what": what, "offset": off, "tag": tag, "bytes": n,
                      "sha256": hashlib.sha256(blob).hexdigest()})
        off += n

    for line in param_text.splitlines()[2:]:
        tok = line.split()
        kind, name = tok[0], tok[1]
        kv = dict(t.split("=", 1) for t in tok if "=" in t)
        if kind == "AdaCompose":
            n_vec = int(kv["1"]) * 12 + 2 * int(kv["4"])
            for j in range(n_vec):
                take(name, f"vector {j}", 4 + 4 * DIM, True)
        elif kind == "InnerProduct":
            n_out, bias, n_w = int(kv["0"]), int(kv["1"]), int(kv["2"])
            tag = struct.unpack_from("<I", data, off)[0]
            wbytes = 2 * n_w + (-(2 * n_w) % 4) if tag == 0x01306B47 else 4 * n_w
            take(name, "weight", 4 + wbytes, True)
            if bias:
                take(name, "bias", 4 * n_out, False)
        elif kind == "AWA":
            for v in ("nq_v", "nk_v", "nq_t", "nk_t"):
                take(name, v, 4 + 4 * 128, True)
        elif kind == "RMSNorm" and kv.get("2") == "1":
            take(name, "gamma", 4 * DIM, False)
    assert off == len(data), (off, len(data))
    return {"bytes": len(data), "sha256": hashlib.sha256(data).hexdigest(), "parts": parts}


def main():
    if not os.path.exists(EXPORTER):
        sys.exit(f"{EXPORTER} not found: run where the reference is present")
    out = {"n_layers": N_LAYERS, "mlp": MLP, "layouts": {}}
    with tempfile.TemporaryDirectory() as tmp:
        model = os.path.join(tmp, "m5")
        make_model_dir(model)
        for layout, env in (("adacompose", "1"), ("inputs", "0")):
            os.environ["SEEDVR_ADACOMPOSE"] = env
            argv = sys.argv
            sys.argv = [EXPORTER, model, str(N_LAYERS)]
            try:
                runpy.run_path(EXPORTER, run_name="__main__")
            finally:
                sys.argv = argv
            param = open(os.path.join(model + "_graph", "dit_graph.param")).read()
            data = open(os.path.join(model + "_graph", "dit_graph.bin"), "rb").read()
            out["layouts"][layout] = {"param": param.splitlines(), "bin": manifest(param, data)}
    with open(OUT, "w") as fp:
        json.dump(out, fp, indent=1)
    print("wrote", OUT)


if __name__ == "__main__":
    main()

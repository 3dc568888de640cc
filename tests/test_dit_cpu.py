"""CPU checks of the block reference: the numpy layer restatement used by the
GPU tests equals the C oracle's forward_latent layer (itself built from
functions bit-exact to the reference's) in fp32, for shared, dual and last
layers."""
import numpy as np
import pytest

from conftest import metrics
from dit_reference import layer_emulation, random_branch, random_emb


@pytest.mark.parametrize("kind", ["shared", "dual", "last"])
def test_emulation_matches_oracle_layer(oracle, kind):
    rng = np.random.default_rng(21)
    mlp, TXT = 256, 5
    g = oracle.Geometry(1, 6, 8, (1, 30, 30), TXT, 1)
    emb, _ = random_emb(rng, oracle)
    vb = random_branch(rng, mlp)
    tb = vb if kind == "shared" else random_branch(rng, mlp)
    x = rng.standard_normal((g.Lv + TXT, 2560)).astype(np.float32)
    last = kind == "last"
    ref_v, ref_t = oracle.dit_layer(x[: g.Lv], x[g.Lv:], emb, vb, tb, g, txt_vid_only=last)
    emu = layer_emulation(oracle, x, emb, vb, tb, g, g.Lv, TXT, last=last, bf16=False)
    for out, ref, x0 in ((emu[: g.Lv], ref_v, x[: g.Lv]), (emu[g.Lv:], ref_t, x[g.Lv:])):
        cos, rel, _ = metrics(out - x0, ref - x0)
        assert cos >= 0.999999 and rel <= 1e-4, (kind, cos, rel)  # fp32 GEMM order only


def test_last_layer_text_skips_mlp(oracle):
    """vid_only last layer (dit_vk.cpp:523-620): the MLP weights leave the text rows
    untouched and still change the video rows; in a full layer they change both."""
    rng = np.random.default_rng(22)
    mlp, TXT = 128, 4
    g = oracle.Geometry(1, 4, 6, (1, 30, 30), TXT, 0)
    emb, _ = random_emb(rng, oracle)
    vb = random_branch(rng, mlp)
    vb2 = dict(vb)
    vb2["mlp_out_w"] = 2.0 * vb["mlp_out_w"]
    x = rng.standard_normal((g.Lv + TXT, 2560)).astype(np.float32)
    for last in (True, False):
        a = layer_emulation(oracle, x, emb, vb, vb, g, g.Lv, TXT, last=last, bf16=False)
        b = layer_emulation(oracle, x, emb, vb2, vb2, g, g.Lv, TXT, last=last, bf16=False)
        assert not np.array_equal(a[: g.Lv], b[: g.Lv])
        assert np.array_equal(a[g.Lv:], b[g.Lv:]) == last

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


ADA = ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate")


@pytest.mark.parametrize("key", ADA)
def test_last_layer_ignores_text_ada(oracle, key):
    """forward_latent's last layer is vid_only (dit_vk.cpp:523-620): for the
    text rows it skips the ada modulation before attention (:538), the
    attention gate (:560), the MLP norm and ada (:579, :590) and the MLP with
    its gate (:610, :617), so none of the text branch's six ada vectors may
    change any output row; in a full layer each one changes the text rows.
    Checked on the C oracle (orc_dit_layer, txt_vid_only = 1 / 0) with
    separate video and text branches."""
    rng = np.random.default_rng(23)
    mlp, TXT = 128, 4
    g = oracle.Geometry(1, 4, 6, (1, 30, 30), TXT, 1)
    emb, _ = random_emb(rng, oracle)
    vb = random_branch(rng, mlp)
    tb = random_branch(rng, mlp)
    tb2 = dict(tb)
    tb2[key] = tb[key] + 0.5 + rng.standard_normal(tb[key].shape).astype(np.float32)
    x = rng.standard_normal((g.Lv + TXT, 2560)).astype(np.float32)
    for last in (True, False):
        a = oracle.dit_layer(x[: g.Lv], x[g.Lv:], emb, vb, tb, g, txt_vid_only=last)
        b = oracle.dit_layer(x[: g.Lv], x[g.Lv:], emb, vb, tb2, g, txt_vid_only=last)
        if last:
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), key
        else:
            assert not np.array_equal(a[1], b[1]), key


def test_last_layer_text_rows_closed_form(oracle):
    """The text rows of the vid_only last layer are x_t + out_t(attention),
    the attention's text input being the plain RMSNorm of x_t (no ada, no
    gate, no MLP).  A full layer whose text branch modulates by the identity
    (ada vectors that cancel emb's slots to scale 1, shift 0, gate 1) and
    whose text MLP output weights are zero computes the same rows, up to the
    last bits of the cancellations."""
    rng = np.random.default_rng(24)
    mlp, TXT = 128, 5
    g = oracle.Geometry(1, 4, 6, (1, 30, 30), TXT, 0)
    emb, _ = random_emb(rng, oracle)
    vb = random_branch(rng, mlp)
    tb = random_branch(rng, mlp)
    # emb[6d + k] + vector = identity: scale 1 (k = 1), shift 0 (k = 0), gate 1 (k = 2)
    ident = dict(tb)
    ident["attn_shift"] = (-emb[0::6]).astype(np.float32)
    ident["attn_scale"] = (1.0 - emb[1::6]).astype(np.float32)
    ident["attn_gate"] = (1.0 - emb[2::6]).astype(np.float32)
    ident["mlp_out_w"] = np.zeros_like(tb["mlp_out_w"])
    x = rng.standard_normal((g.Lv + TXT, 2560)).astype(np.float32)
    last = oracle.dit_layer(x[: g.Lv], x[g.Lv:], emb, vb, tb, g, txt_vid_only=True)
    full = oracle.dit_layer(x[: g.Lv], x[g.Lv:], emb, vb, ident, g, txt_vid_only=False)
    # the same arithmetic up to the multiplications by exactly 1 and additions of 0,
    # which may differ in the last bit where emb's slots do not cancel exactly
    cos, rel, _ = metrics(full[1] - x[g.Lv:], last[1] - x[g.Lv:])
    assert cos >= 0.9999999 and rel <= 1e-5, (cos, rel)
    cos, rel, _ = metrics(full[0], last[0])
    assert cos >= 0.9999999 and rel <= 1e-5, (cos, rel)


def test_patchify_known_answer():
    """Row (t, hh, ww), column (ph*2 + pw)*33 + c holds grid[t, 2hh+ph, 2ww+pw, c]
    (dit_vk.cpp:717-733), on a grid whose values encode their own indices."""
    from dit_reference import patchify
    T, H, W, Cc = 2, 6, 8, 33
    t, h, w, c = np.meshgrid(np.arange(T), np.arange(H), np.arange(W), np.arange(Cc), indexing="ij")
    grid = (t * 1000000 + h * 10000 + w * 100 + c).astype(np.float32)
    p = patchify(grid)
    assert p.shape == (T * (H // 2) * (W // 2), 132)
    for row in (0, 5, 11, 23):
        tt, rem = divmod(row, (H // 2) * (W // 2))
        hh, ww = divmod(rem, W // 2)
        for j in (0, 32, 33, 65, 66, 100, 131):
            ph, pw, cc = j // 66, (j // 33) % 2, j % 33
            assert p[row, j] == tt * 1000000 + (2 * hh + ph) * 10000 + (2 * ww + pw) * 100 + cc


def test_unpatchify_inverts_patchify():
    """dit_vk.cpp:735-750 writes back exactly the (ph, pw, c) order that
    patchify reads, so the two are inverse on a 16-channel grid."""
    from dit_reference import patchify, unpatchify
    rng = np.random.default_rng(7)
    g = rng.standard_normal((2, 10, 14, 16)).astype(np.float32)
    assert np.array_equal(unpatchify(patchify(g), 2, 10, 14), g)


def test_final_emulation_matches_oracle(oracle):
    """The output layer in fp32 against the oracle's rmsnorm (with weight) and
    linear (dit_vk.cpp:657-675), row by row."""
    from dit_reference import final_emulation, random_emb, random_io, unpatchify
    rng = np.random.default_rng(8)
    io = random_io(rng)
    emb, _ = random_emb(rng, oracle)
    T, H, W = 1, 4, 6
    Lv = T * (H // 2) * (W // 2)
    x = rng.standard_normal((Lv, 2560)).astype(np.float32)
    got = final_emulation(oracle, x, emb, io, T, H, W, bf16=False)
    vn = np.stack([oracle.rmsnorm(x[i], io["out_norm_w"]) for i in range(Lv)])
    vn = vn * (emb[1::6] + io["out_ada_scale"]) + (emb[0::6] + io["out_ada_shift"])
    ref = unpatchify(oracle.linear(vn, io["vid_out_w"], io["vid_out_b"]), T, H, W)
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-5), np.abs(got - ref).max()

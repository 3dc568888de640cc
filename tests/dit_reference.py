"""Reference for one DiT layer at the block's precision (test infrastructure).

layer_emulation() restates DitVk::forward_latent's layer body
(dit_vk.cpp:517-632, swiglu :465-472, awa_forward :312-463) with numpy fp32
GEMMs and the oracle's attention.  With bf16=True it rounds to bf16 (nearest
even) exactly where the MI355X block stores bf16: the projection inputs, the
qkv and attention outputs (AwaLayer's bf16 boundary, awa_layer.cpp:338-451)
and the SwiGLU product; weights are taken as the bf16 values they are stored
as.  With bf16=False it is the fp32 layer, checked against the C oracle's
orc_dit_layer (tests/test_dit_cpu.py).
"""
import numpy as np

DIM = 2560


def rmsnorm_rows(x, eps):
    """dit_vk.cpp:48-52: double-accumulated mean square, float scale."""
    ss = (x.astype(np.float64) ** 2).sum(axis=1) / x.shape[1]
    r = (np.float32(1.0) / np.sqrt(ss.astype(np.float32) + np.float32(eps))).astype(np.float32)
    return x * r[:, None]


def ada_vectors(emb, br):
    """AdaCompose slots (ada_compose.cpp:16): emb[6d + k] + branch vector."""
    return {"a_sc": emb[1::6] + br["attn_scale"], "a_sh": emb[0::6] + br["attn_shift"],
            "a_g": emb[2::6] + br["attn_gate"], "m_sc": emb[4::6] + br["mlp_scale"],
            "m_sh": emb[3::6] + br["mlp_shift"], "m_g": emb[5::6] + br["mlp_gate"]}


def silu(v):
    return v / (np.float32(1.0) + np.exp(-v))


def np_mm(a, w):
    """a @ w.T in fp32 (numpy)."""
    return a @ w.T


def layer_emulation(O, x, emb, vb, tb, geom, Lv, TXT, last=False, eps=1e-5, bf16=True, mm=np_mm):
    """One layer on x [Lv+TXT, 2560] fp32; branches are dicts of fp32 numpy arrays with
    keys qkv_w, out_w, out_b, mlp_in_w, mlp_g_w, mlp_out_w, nq, nk and the six ada vectors.
    mm(a, w) computes the fp32 product a @ w.T (numpy by default; the full-size GPU
    tests pass an fp32 device product to keep the CPU time of 1080p layers short)."""
    rnd = O.bf16_round if bf16 else (lambda a: np.asarray(a, np.float32))
    x = np.array(x, np.float32, copy=True)
    xv, xt = x[:Lv], x[Lv:]
    av, at = ada_vectors(emb, vb), ada_vectors(emb, tb)
    hv = rnd(rmsnorm_rows(xv, eps) * av["a_sc"] + av["a_sh"])
    ht = rmsnorm_rows(xt, eps)
    if not last:
        ht = ht * at["a_sc"] + at["a_sh"]
    ht = rnd(ht)
    qv = rnd(mm(hv, vb["qkv_w"]))
    qt = rnd(mm(ht, tb["qkv_w"]))
    va, ta = O.awa_forward(qv, qt, geom, vb["nq"], vb["nk"], tb["nq"], tb["nk"], eps=eps)
    va, ta = rnd(va), rnd(ta)
    xv += av["a_g"] * (mm(va, vb["out_w"]) + vb["out_b"])
    ot = mm(ta, tb["out_w"]) + tb["out_b"]
    xt += ot if last else at["a_g"] * ot
    hv = rnd(rmsnorm_rows(xv, eps) * av["m_sc"] + av["m_sh"])
    uv = rnd(silu(mm(hv, vb["mlp_g_w"])) * mm(hv, vb["mlp_in_w"]))
    xv += av["m_g"] * mm(uv, vb["mlp_out_w"])
    if not last:
        ht = rnd(rmsnorm_rows(xt, eps) * at["m_sc"] + at["m_sh"])
        ut = rnd(silu(mm(ht, tb["mlp_g_w"])) * mm(ht, tb["mlp_in_w"]))
        xt += at["m_g"] * mm(ut, tb["mlp_out_w"])
    return x


def random_branch(rng, mlp, O=None, scale=0.02):
    """Weights ~ N(0, 0.02) (bf16-representable if O is given), gains 1 + N(0, 0.02)."""
    r = (lambda a: O.bf16_round(a)) if O is not None else (lambda a: a)
    f = lambda *s: (scale * rng.standard_normal(s)).astype(np.float32)
    br = {"qkv_w": r(f(7680, DIM)), "out_w": r(f(DIM, DIM)), "out_b": f(DIM),
          "mlp_in_w": r(f(mlp, DIM)), "mlp_g_w": r(f(mlp, DIM)), "mlp_out_w": r(f(DIM, mlp)),
          "nq": (1 + f(128)).astype(np.float32), "nk": (1 + f(128)).astype(np.float32)}
    for k in ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
        br[k] = f(DIM)
    return br


def random_emb(rng, O, scale=0.02):
    """time_embedding(1000) through random N(0, scale) timestep-MLP weights."""
    ws = [(scale * rng.standard_normal(s)).astype(np.float32)
          for s in ((DIM, 256), (DIM,), (DIM, DIM), (DIM,), (6 * DIM, DIM), (6 * DIM,))]
    return O.time_embedding(1000.0, *ws), ws


def to_device(br, mlp, ctx, dev):
    """Device tensors of a branch in the block's storage formats."""
    import torch
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev, torch.bfloat16)
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev, torch.float32)
    d = {"qkv_w": bf(br["qkv_w"]), "out_w": bf(br["out_w"]), "out_b": f32(br["out_b"]),
         "mlp_out_w": bf(br["mlp_out_w"])}
    d["mlp_w"] = ctx.pack_mlp(bf(br["mlp_in_w"]), bf(br["mlp_g_w"]))
    for k in ("nq", "nk", "attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
        d[k] = f32(br[k])
    return d


# ---- input and output layers (DitVk::forward_grid, dit_vk.cpp:752-763) ----

def patchify(grid):
    """dit_vk.cpp:717-733: (T, H, W, C) -> (T (H/2) (W/2), 4 C), patch order (ph, pw, c)."""
    T, H, W, Cc = grid.shape
    g = grid.reshape(T, H // 2, 2, W // 2, 2, Cc)          # t, hh, ph, ww, pw, c
    return np.ascontiguousarray(g.transpose(0, 1, 3, 2, 4, 5).reshape(-1, 4 * Cc))


def unpatchify(y, T, H, W, Cc=16):
    """dit_vk.cpp:735-750: (T (H/2) (W/2), 4 C) -> (T, H, W, C)."""
    g = y.reshape(T, H // 2, W // 2, 2, 2, Cc)              # t, hh, ww, ph, pw, c
    return np.ascontiguousarray(g.transpose(0, 1, 3, 2, 4, 5).reshape(T, H, W, Cc))


def random_io(rng, O=None, scale=0.02):
    """Input/output layer weights ~ N(0, 0.02) (bf16-representable if O is given)."""
    r = (lambda a: O.bf16_round(a)) if O is not None else (lambda a: a)
    f = lambda *s: (scale * rng.standard_normal(s)).astype(np.float32)
    return {"vid_in_w": r(f(DIM, 132)), "vid_in_b": f(DIM), "txt_in_w": r(f(DIM, 5120)), "txt_in_b": f(DIM),
            "out_norm_w": (1 + f(DIM)).astype(np.float32), "out_ada_shift": f(DIM),
            "out_ada_scale": f(DIM), "vid_out_w": r(f(64, DIM)), "vid_out_b": f(64)}


def io_to_device(io, dev):
    import torch
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev, torch.bfloat16)
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev, torch.float32)
    return {k: (bf(v) if k.endswith("_w") and k != "out_norm_w" else f32(v)) for k, v in io.items()}


def embed_emulation(O, grid, txt, io, bf16=True):
    """forward_latent's input projections (dit_vk.cpp:494-497) on the patchified grid;
    with bf16=True the projection inputs are rounded to bf16 as the block stores them."""
    rnd = O.bf16_round if bf16 else (lambda a: np.asarray(a, np.float32))
    xv = rnd(patchify(grid)) @ io["vid_in_w"].T + io["vid_in_b"]
    xt = rnd(txt) @ io["txt_in_w"].T + io["txt_in_b"]
    return np.concatenate([xv, xt]).astype(np.float32)


def final_emulation(O, x_vid, emb, io, T, H, W, eps=1e-5, bf16=True):
    """forward_latent's output layer (dit_vk.cpp:657-675) and unpatchify (:735-750)."""
    rnd = O.bf16_round if bf16 else (lambda a: np.asarray(a, np.float32))
    vn = rmsnorm_rows(x_vid, eps) * io["out_norm_w"]
    h = rnd(vn * (emb[1::6] + io["out_ada_scale"]) + (emb[0::6] + io["out_ada_shift"]))
    y = h @ io["vid_out_w"].T + io["vid_out_b"]
    return unpatchify(y.astype(np.float32), T, H, W)

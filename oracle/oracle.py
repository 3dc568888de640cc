"""ctypes front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loads ``oracle/liboracle.so`` (the C restatement in ``oracle.c``) and, when it
was built, ``oracle/_ref/libref_bridge.so`` (the reference's own
``src/verify_dit.cpp`` compiled unchanged).  Only tests, ``smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module; the product path
never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_bridge.so")

HEADS, HEAD_D, DIM, QKV, ROPE_ROT, MLP = 20, 128, 2560, 7680, 126, 6912

_lib = None
_ref = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and _ref when the reference sources exist)."""
    target = "all" if ref else "liboracle.so"
    subprocess.run(["make", "-s", "-C", HERE, target], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        L = C.CDLL(LIB_PATH)
        L.orc_make_windows.restype = C.c_int
        L.orc_make_windows.argtypes = [C.c_int, C.c_int, C.c_int, _i32p, C.c_int, C.c_void_p, C.c_int]
        L.orc_build_freqs.restype = C.c_int
        L.orc_build_freqs.argtypes = [_i32p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        L.orc_build_index.restype = C.c_int
        L.orc_build_index.argtypes = [_i32p, C.c_int, C.c_int, C.c_int, _i32p, _i32p]
        L.orc_rmsnorm.argtypes = [_f32p, C.c_int, C.c_void_p, C.c_float, _f32p]
        L.orc_qk_norm.argtypes = [_f32p, _f32p, C.c_float, _f32p]
        L.orc_apply_rope.argtypes = [_f32p, _f32p, _f32p]
        L.orc_awa_forward.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                      _i32p, C.c_int, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                      C.c_float, _f32p, _f32p, C.c_int]
        L.orc_f32_to_bf16.argtypes = [_f32p, _u16p, C.c_int64]
        L.orc_bf16_to_f32.argtypes = [_u16p, _f32p, C.c_int64]
        L.orc_linear.argtypes = [_f32p, _f32p, C.c_void_p, C.c_int, C.c_int, C.c_int, _f32p, C.c_int]
        L.orc_sinusoidal.argtypes = [C.c_float, C.c_int, _f32p]
        L.orc_silu.argtypes = [_f32p, C.c_int64]
        L.orc_time_embedding.argtypes = [C.c_float] + [_f32p] * 7
        L.orc_dit_layer.argtypes = [_f32p, _f32p, C.c_int, C.c_int, _f32p, C.c_void_p, C.c_void_p,
                                    C.c_int, C.c_int, C.c_int, C.c_int, _i32p, C.c_int, _f32p, _f32p,
                                    C.c_float, C.c_int, C.c_int]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own routines (verify_dit.cpp), or None if not built."""
    global _ref
    if _ref is None and ref_available():
        R = C.CDLL(REF_PATH)
        R.ref_rmsnorm.argtypes = [_f32p, C.c_int, C.c_void_p, _f32p]
        R.ref_qk_norm.argtypes = [_f32p, _f32p, _f32p]
        R.ref_apply_rope.argtypes = [_f32p, _f32p, _f32p]
        R.ref_sinusoidal.argtypes = [C.c_float, C.c_int, _f32p]
        R.ref_silu.argtypes = [_f32p, C.c_int]
        R.ref_linear.argtypes = [_f32p, _f32p, C.c_void_p, C.c_int, C.c_int, C.c_int, _f32p]
        R.ref_time_embedding.argtypes = [C.c_float] + [_f32p] * 7
        _f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        R.ref_verify_dit_main.restype = C.c_int
        R.ref_verify_dit_main.argtypes = [C.c_char_p, _i32p, _f64p, _f64p, C.c_int,
                                          C.POINTER(C.c_int)]
        R.ref_awa_block.argtypes = [_f32p, C.c_int, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                    _i32p, C.c_int, _f32p, C.c_int, _f32p, _f32p, _f32p,
                                    _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        _ref = R
    return _ref


def _nthreads(n):
    if n is None:
        n = min(16, os.cpu_count() or 1)
    return int(n)


# ---------------------------------------------------------------- geometry
class Geometry:
    """Window geometry exactly as awa::make_win builds it (awa_window.cpp:133-150)."""

    def __init__(self, t, h, w, num_windows, txt_len, shifted):
        self.t, self.h, self.w = int(t), int(h), int(w)
        self.num_windows = tuple(int(x) for x in num_windows)
        self.txt_len = int(txt_len)
        self.shifted = bool(shifted)
        nw = np.array(self.num_windows, dtype=np.int32)
        n = lib().orc_make_windows(self.t, self.h, self.w, nw, int(self.shifted), None, 0)
        sl = np.zeros((max(n, 1), 6), dtype=np.int32)
        lib().orc_make_windows(self.t, self.h, self.w, nw, int(self.shifted),
                               sl.ctypes.data_as(C.c_void_p), n)
        self.slices = np.ascontiguousarray(sl[:n])
        self.nwin = n
        sizes = (self.slices[:, 1] - self.slices[:, 0]) * (self.slices[:, 3] - self.slices[:, 2]) \
            * (self.slices[:, 5] - self.slices[:, 4])
        self.sumf = int(sizes.sum())
        self.vid_freq = np.zeros((self.sumf, ROPE_ROT), dtype=np.float32)
        self.txt_freq = np.zeros((n * self.txt_len, ROPE_ROT), dtype=np.float32)
        lib().orc_build_freqs(self.slices, n, self.txt_len,
                              self.vid_freq.ctypes.data_as(C.c_void_p),
                              self.txt_freq.ctypes.data_as(C.c_void_p))
        self.cumf = np.zeros(n + 1, dtype=np.int32)
        self.vidx = np.zeros(max(self.sumf, 1), dtype=np.int32)
        lib().orc_build_index(self.slices, n, self.h, self.w, self.cumf, self.vidx)
        self.vidx = self.vidx[: self.sumf]

    @property
    def Lv(self):
        return self.t * self.h * self.w

    @property
    def S(self):
        return np.diff(self.cumf) + self.txt_len


# ---------------------------------------------------------------- ops
def qk_norm(x, w, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(DIM, np.float32)
    lib().orc_qk_norm(x, np.ascontiguousarray(w, np.float32), eps, out)
    return out


def apply_rope(freq, q):
    out = np.empty(HEAD_D, np.float32)
    lib().orc_apply_rope(np.ascontiguousarray(freq, np.float32), np.ascontiguousarray(q, np.float32), out)
    return out


def rmsnorm(x, w=None, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    wp = None if w is None else np.ascontiguousarray(w, np.float32)
    lib().orc_rmsnorm(x, x.size, None if wp is None else wp.ctypes.data_as(C.c_void_p), eps, out)
    return out


def awa_forward(vqkv, tqkv, geom: Geometry, nq_v, nk_v, nq_t, nk_t, eps=1e-5, nthreads=None):
    """fp32 AWA op (dit_vk.cpp:345-462): returns (vattn [Lv,2560], tattn [TXT,2560])."""
    vqkv = np.ascontiguousarray(vqkv, np.float32)
    tqkv = np.ascontiguousarray(tqkv, np.float32)
    Lv = vqkv.shape[0]
    TXT = tqkv.shape[0]
    assert Lv == geom.Lv and TXT == geom.txt_len
    vattn = np.empty((Lv, DIM), np.float32)
    tattn = np.empty((max(TXT, 1), DIM), np.float32)
    g = [np.ascontiguousarray(a, np.float32) for a in (nq_v, nk_v, nq_t, nk_t)]
    lib().orc_awa_forward(vqkv, tqkv if TXT else np.zeros((1, QKV), np.float32), Lv, TXT,
                          geom.t, geom.h, geom.w, geom.slices, geom.nwin, geom.vid_freq,
                          geom.txt_freq if TXT else np.zeros((1, ROPE_ROT), np.float32),
                          *g, float(eps), vattn, tattn, _nthreads(nthreads))
    return vattn, tattn[:TXT]


def f32_to_bf16(x):
    """Round-to-nearest-even bits (cast_f32_bf16.comp:24) as uint16."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(b):
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_bf16_to_f32(b.reshape(-1), out.reshape(-1), b.size)
    return out


def bf16_round(x):
    return bf16_to_f32(f32_to_bf16(x))


def linear(x, W, b=None, nthreads=None):
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    Ln, n_in = x.shape
    n_out = W.shape[0]
    y = np.empty((Ln, n_out), np.float32)
    bp = None if b is None else np.ascontiguousarray(b, np.float32)
    lib().orc_linear(x, W, None if bp is None else bp.ctypes.data_as(C.c_void_p), Ln, n_in, n_out,
                     y, _nthreads(nthreads))
    return y


def sinusoidal(t, dim=256):
    e = np.empty(dim, np.float32)
    lib().orc_sinusoidal(float(t), dim, e)
    return e


def silu(x):
    x = np.array(x, np.float32, copy=True)
    lib().orc_silu(x.reshape(-1), x.size)
    return x


def time_embedding(t, w_in, b_in, w_hid, b_hid, w_out, b_out):
    emb = np.empty(6 * DIM, np.float32)
    args = [np.ascontiguousarray(a, np.float32) for a in (w_in, b_in, w_hid, b_hid, w_out, b_out)]
    lib().orc_time_embedding(float(t), *args, emb)
    return emb


class Branch(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "qkv_w", "out_w", "out_b", "mlp_in_w", "mlp_g_w", "mlp_out_w", "nq", "nk",
        "attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate")]


BRANCH_KEYS = ("qkv_w", "out_w", "out_b", "mlp_in_w", "mlp_g_w", "mlp_out_w", "nq", "nk",
               "attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate")


def _branch(d):
    arrs = {k: np.ascontiguousarray(d[k], np.float32) for k in BRANCH_KEYS}
    b = Branch(**{k: arrs[k].ctypes.data_as(C.c_void_p) for k in BRANCH_KEYS})
    return b, arrs


def dit_layer(vid, txt, emb, vbranch, tbranch, geom: Geometry, eps=1e-5, txt_vid_only=False,
              nthreads=None):
    """One forward_latent layer (dit_vk.cpp:517-632); returns new (vid, txt)."""
    vid = np.array(vid, np.float32, copy=True)
    txt = np.array(txt, np.float32, copy=True)
    vb, keep_v = _branch(vbranch)
    tb, keep_t = _branch(tbranch)
    mlp = int(np.asarray(vbranch["mlp_in_w"]).shape[0])
    lib().orc_dit_layer(vid, txt, vid.shape[0], txt.shape[0], np.ascontiguousarray(emb, np.float32),
                        C.byref(vb), C.byref(tb), mlp, geom.t, geom.h, geom.w, geom.slices,
                        geom.nwin, geom.vid_freq, geom.txt_freq, float(eps), int(txt_vid_only),
                        _nthreads(nthreads))
    del keep_v, keep_t
    return vid, txt

"""Python binding of the C ABI in include/awa_capi.h (ctypes over lib/libseedvr2_awa.so).

This is the binding a Python caller (and the test-suite and bench) uses; the
product is the C ABI itself.  Device buffers are torch tensors on a ROCm
device; the stream is torch's current stream.  There is no fallback: if the
shared library is missing, import fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libseedvr2_awa.so")
HEADER_DIR = os.path.join(os.path.dirname(HERE), "include")

AWA_OK, AWA_EARG, AWA_EHIP = 0, -1, -2
AWA_F32, AWA_BF16 = 0, 1
HEADS, HEAD_D, DIM, QKV, ROPE_ROT = 20, 128, 2560, 7680, 126

_lib = None


class AwaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"AWA error {code}: {msg}")
        self.code = code


BRANCH_FIELDS = ("qkv_w", "out_w", "out_b", "mlp_w", "mlp_out_w", "nq", "nk", "attn_shift",
                 "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate")


class DitBranch(C.Structure):
    """dit_branch of include/dit_capi.h (device pointers)."""
    _fields_ = [(n, C.c_void_p) for n in BRANCH_FIELDS]


IO_FIELDS = ("vid_in_w", "vid_in_b", "txt_in_w", "txt_in_b", "out_norm_w", "out_ada_shift",
             "out_ada_scale", "vid_out_w", "vid_out_b")


class DitIoWeights(C.Structure):
    """dit_io_weights of include/dit_capi.h (device pointers)."""
    _fields_ = [(n, C.c_void_p) for n in IO_FIELDS]


class DitTimeWeights(C.Structure):
    """dit_time_weights of include/dit_capi.h (device pointers)."""
    _fields_ = [(n, C.c_void_p) for n in ("w_in", "b_in", "w_hid", "b_hid", "w_out", "b_out")]


class GeomInfo(C.Structure):
    _fields_ = [(n, C.c_int32) for n in
                ("t", "h", "w", "nwin", "sumf", "Lv", "txt_len", "max_S", "n_tiles", "n_items")]


def build():
    """Compile lib/libseedvr2_awa.so with hipcc for gfx950."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE, f"-j{min(8, os.cpu_count() or 1)}"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it (make -C {HERE}) before use")
        # torch ships its own HIP runtime with the same soname
        # (libamdhip64.so.7).  Load it first so the library binds to that one
        # runtime instead of starting a second one from /opt/rocm in the same
        # process: torch's tensors and streams then belong to our runtime too.
        import torch  # noqa: F401
        L = C.CDLL(LIB_PATH)
        vp, i32p, f32p = C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_float)
        L.awa_create.argtypes = [C.POINTER(vp), C.c_int]
        L.awa_destroy.argtypes = [vp]
        L.awa_destroy.restype = None
        L.awa_last_error.argtypes = [vp]
        L.awa_last_error.restype = C.c_char_p
        L.awa_plan_windows.argtypes = [C.c_int, C.c_int, C.c_int, i32p, C.c_int, i32p, C.c_int]
        L.awa_geom_build.argtypes = [vp, C.c_int, C.c_int, C.c_int, i32p, C.c_int, C.c_int,
                                     C.POINTER(vp), vp]
        L.awa_geom_set.argtypes = [vp, f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int,
                                   C.POINTER(vp), vp]
        L.awa_geom_from_win.argtypes = [vp, C.c_int, C.c_int, C.c_int, C.c_int, i32p, f32p, f32p, C.c_int,
                                        C.POINTER(vp), vp]
        L.awa_geom_query.argtypes = [vp, C.POINTER(GeomInfo)]
        L.awa_geom_read.argtypes = [vp, vp, vp, vp, vp, vp, vp]
        L.awa_geom_destroy.argtypes = [vp]
        L.awa_geom_destroy.restype = None
        L.awa_forward.argtypes = [vp, vp, C.c_int, vp, vp, C.c_int, C.c_int, vp, vp, vp, vp,
                                  C.c_float, vp, vp, vp]
        L.awa_forward_noalloc.argtypes = [vp, vp, C.c_int, vp, vp, C.c_int, C.c_int, vp, vp, vp, vp,
                                          C.c_float, vp, vp, vp]
        L.awa_forward_host.argtypes = [vp, vp, f32p, f32p, C.c_int, C.c_int, f32p, f32p, f32p, f32p,
                                       C.c_float, f32p, f32p]
        L.awa_timing_enable.argtypes = [vp, C.c_int]
        L.awa_timing_read.argtypes = [vp, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                      C.POINTER(C.c_double), C.POINTER(C.c_int)]
        L.dit_pack_mlp_weights.argtypes = [vp, vp, vp, C.c_int, vp, vp]
        L.dit_time_embedding.argtypes = [vp, C.c_float, vp, vp, vp, vp, vp, vp, vp, vp]
        L.dit_layer_forward.argtypes = [vp, vp, C.POINTER(DitBranch), C.POINTER(DitBranch), vp, C.c_int,
                                        C.c_int, C.c_float, vp, C.c_int, C.c_int, vp]
        L.dit_timing_read.argtypes = [vp, C.POINTER(C.c_double), C.POINTER(C.c_double),
                                      C.POINTER(C.c_double), C.POINTER(C.c_int)]
        L.dit_gemm_bf16.argtypes = [vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp]
        L.dit_io_create.argtypes = [vp, C.POINTER(DitIoWeights), C.POINTER(vp), vp]
        L.dit_io_destroy.argtypes = [vp, vp]
        L.dit_io_destroy.restype = None
        L.dit_embed.argtypes = [vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp, vp]
        L.dit_final.argtypes = [vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_float, vp, vp]
        L.dit_host_last_error.restype = C.c_char_p
        L.dit_free_host.argtypes = [vp]
        L.dit_free_host.restype = None
        L.dit_read_raw_f.argtypes = [C.c_char_p, C.POINTER(vp), C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                     C.POINTER(C.c_int)]
        L.dit_read_linear.argtypes = [C.c_char_p, C.c_int, C.POINTER(vp), C.POINTER(vp), C.POINTER(C.c_int),
                                      C.POINTER(C.c_int)]
        L.dit_read_win.argtypes = [C.c_char_p, C.c_int, C.POINTER(C.c_int64), C.POINTER(vp), C.POINTER(vp),
                                   C.POINTER(C.c_int64), C.POINTER(vp), C.POINTER(C.c_int64)]
        L.dit_model_load.argtypes = [vp, C.c_char_p, C.c_int, C.c_int, C.POINTER(vp), vp]
        L.dit_model_load_graph.argtypes = [vp, C.c_char_p, C.c_char_p, C.c_char_p, C.c_int, C.POINTER(vp), vp]
        L.dit_graph_file_info.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                          C.POINTER(C.c_int)]
        L.dit_read_graph_weight.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_char_p, C.POINTER(vp),
                                            C.POINTER(vp), C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.dit_model_info.argtypes = [vp, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.dit_model_forward_grid.argtypes = [vp, vp, vp, vp, C.c_int, C.c_float, C.c_float, vp, C.c_int, C.c_int,
                                             C.c_int, vp, C.c_int, vp, vp, vp]
        L.dit_model_destroy.argtypes = [vp, vp]
        L.dit_model_destroy.restype = None
        L.dit_graph_create.argtypes = [vp, vp, vp, vp, C.c_int, C.c_float, C.c_float, vp, C.c_int, C.c_int,
                                       C.c_int, vp, C.c_int, vp, vp, vp, C.POINTER(vp)]
        L.dit_graph_launch.argtypes = [vp, vp, vp]
        L.dit_graph_destroy.argtypes = [vp]
        L.dit_graph_destroy.restype = None
        L.dit_forward_grid.argtypes = [vp, vp, C.POINTER(DitTimeWeights), C.POINTER(C.POINTER(DitBranch)),
                                       C.POINTER(C.POINTER(DitBranch)), C.c_int, vp, vp, C.c_int, C.c_int,
                                       C.c_float, C.c_float, vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, vp,
                                       vp, vp]
        L.awa_cast_f32_to_bf16.argtypes = [vp, vp, vp, C.c_int64, vp]
        L.awa_cast_bf16_to_f32.argtypes = [vp, vp, vp, C.c_int64, vp]
        L.awa_stream_copy.argtypes = [vp, vp, vp, C.c_int64, vp]
        L.awa_reserve.argtypes = [vp, vp, C.c_int]
        L.dit_reserve.argtypes = [vp, vp, C.c_int]
        L.awa_time_phases.argtypes = [vp, vp, C.c_int, vp, vp, C.c_int, C.c_int, vp, vp, vp, vp,
                                      C.c_float, vp, vp, C.c_int, C.POINTER(C.c_double), vp]
        _lib = L
    return _lib


def _host_array(ptr, n, dtype):
    """Copy n values from a dit_* host buffer, then free it."""
    ct = {np.float32: C.c_float, np.int32: C.c_int32}[dtype]
    a = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ct)), shape=(int(n),)).copy() if n else np.zeros(0, dtype)
    lib().dit_free_host(ptr)
    return a


class HostError(RuntimeError):
    pass


def _host_check(rc, what):
    if rc != 0:
        raise HostError(f"{what}: {lib().dit_host_last_error().decode()}")


def read_raw_f(path):
    """dit_read_raw_f: the array with its stored shape."""
    p, n, nd = C.c_void_p(), C.c_int64(), C.c_int()
    shape = (C.c_int64 * 8)()
    _host_check(lib().dit_read_raw_f(str(path).encode(), C.byref(p), C.byref(n), shape, C.byref(nd)), "dit_read_raw_f")
    return _host_array(p, n.value, np.float32).reshape([shape[i] for i in range(nd.value)])


def read_linear(base, has_bias):
    """dit_read_linear: (W [out][in] float32, bias or None)."""
    w, b, no, ni = C.c_void_p(), C.c_void_p(), C.c_int(), C.c_int()
    _host_check(lib().dit_read_linear(str(base).encode(), int(bool(has_bias)), C.byref(w), C.byref(b),
                                      C.byref(no), C.byref(ni)), "dit_read_linear")
    W = _host_array(w, no.value * ni.value, np.float32).reshape(no.value, ni.value)
    return W, (_host_array(b, no.value, np.float32) if has_bias else None)


def read_win(path, txt_len):
    """dit_read_win: dict with header, slices [nwin][6], vid_freq, txt_freq."""
    hdr = (C.c_int64 * 10)()
    sl, vf, tf = C.c_void_p(), C.c_void_p(), C.c_void_p()
    nv, nt = C.c_int64(), C.c_int64()
    _host_check(lib().dit_read_win(str(path).encode(), int(txt_len), hdr, C.byref(sl), C.byref(vf), C.byref(nv),
                                   C.byref(tf), C.byref(nt)), "dit_read_win")
    nwin = hdr[9]
    return {"header": list(hdr), "slices": _host_array(sl, 6 * nwin, np.int32).reshape(nwin, 6),
            "vid_freq": _host_array(vf, nv.value, np.float32), "txt_freq": _host_array(tf, nt.value, np.float32)}


def graph_file_info(param, bin_path, mm_layers=-1):
    """dit_graph_file_info: (n_layers, mm_layers, distinct weights) of a merged graph."""
    n, mm, nw = C.c_int(), C.c_int(), C.c_int()
    _host_check(lib().dit_graph_file_info(str(param).encode(), str(bin_path).encode(), int(mm_layers), C.byref(n),
                                          C.byref(mm), C.byref(nw)), "dit_graph_file_info")
    return n.value, mm.value, nw.value


def read_graph_weight(param, bin_path, name, mm_layers=-1):
    """dit_read_graph_weight: (W [out][in], bias or None) of a linear weight, or
    (vector, None), by its model-directory name."""
    w, b, no, ni = C.c_void_p(), C.c_void_p(), C.c_int(), C.c_int()
    _host_check(lib().dit_read_graph_weight(str(param).encode(), str(bin_path).encode(), int(mm_layers),
                                            name.encode(), C.byref(w), C.byref(b), C.byref(no), C.byref(ni)),
                "dit_read_graph_weight")
    if ni.value == 0:
        return _host_array(w, no.value, np.float32), None
    W = _host_array(w, no.value * ni.value, np.float32).reshape(no.value, ni.value)
    return W, (_host_array(b, no.value, np.float32) if b.value else None)


def header_symbols():
    """Function names declared in include/*.h."""
    import re
    names = []
    for fn in sorted(os.listdir(HEADER_DIR)):
        if fn.endswith(".h"):
            txt = open(os.path.join(HEADER_DIR, fn)).read()
            txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
            names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s+\**([a-z_][a-z0-9_]*)\s*\(",
                                txt, flags=re.M)
    return names


def _ptr(a):
    return C.cast(a.ctypes.data, C.POINTER(C.c_int32)) if a is not None else None


def plan_windows(t, h, w, num_windows, shifted):
    """Host-only window planner (awa_plan_windows): returns int32 [nwin, 6]."""
    nw = np.ascontiguousarray(num_windows, np.int32)
    n = lib().awa_plan_windows(t, h, w, _ptr(nw), int(bool(shifted)), None, 0)
    if n < 0:
        raise AwaError(n, "awa_plan_windows rejected the sizes")
    out = np.zeros((max(n, 1), 6), np.int32)
    lib().awa_plan_windows(t, h, w, _ptr(nw), int(bool(shifted)), _ptr(out), n)
    return out[:n]


def _stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class Context:
    """awa_ctx: one per device and stream (owns the op's scratch)."""

    def __init__(self, device=0):
        self.ptr = C.c_void_p()
        rc = lib().awa_create(C.byref(self.ptr), int(device))
        if rc != AWA_OK:
            raise AwaError(rc, f"awa_create(device={device}) failed")
        self.device = int(device)

    def error(self):
        return lib().awa_last_error(self.ptr).decode()

    def check(self, rc, what):
        if rc != AWA_OK:
            raise AwaError(rc, f"{what}: {self.error()}")

    def close(self):
        if self.ptr:
            lib().awa_destroy(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- timing
    def timing(self, enable=True):
        self.check(lib().awa_timing_enable(self.ptr, int(bool(enable))), "awa_timing_enable")

    def timing_read(self):
        """Summed per-phase ms since the last read: (pack, attention, text, calls)."""
        a, b, c = C.c_double(), C.c_double(), C.c_double()
        n = C.c_int()
        self.check(lib().awa_timing_read(self.ptr, C.byref(a), C.byref(b), C.byref(c), C.byref(n)),
                   "awa_timing_read")
        return a.value, b.value, c.value, n.value

    # ---- geometry
    def build_geometry(self, t, h, w, num_windows, txt_len, shifted, stream=None):
        g = C.c_void_p()
        nw = np.ascontiguousarray(num_windows, np.int32)
        rc = lib().awa_geom_build(self.ptr, t, h, w, _ptr(nw), txt_len, int(bool(shifted)),
                                  C.byref(g), _stream_ptr(stream))
        self.check(rc, "awa_geom_build")
        return Geometry(self, g)

    def set_geometry(self, vidx, cumf, vfreq, tfreq, nwin, Lv, txt_len, stream=None):
        """AwaLayer::set_window_geometry with the reference's float-encoded arrays."""
        arrs = [np.ascontiguousarray(a, np.float32) for a in (vidx, cumf, vfreq, tfreq)]
        fp = [a.ctypes.data_as(C.POINTER(C.c_float)) for a in arrs]
        g = C.c_void_p()
        rc = lib().awa_geom_set(self.ptr, *fp, int(nwin), int(Lv), int(txt_len), C.byref(g),
                                _stream_ptr(stream))
        self.check(rc, "awa_geom_set")
        return Geometry(self, g)

    def geometry_from_win(self, t, h, w, slices, vid_freq, txt_freq, txt_len, stream=None):
        """awa_geom_from_win: a reference Win (grid, nwin x 6 slices, the two
        frequency tables), e.g. as read_win returns a win_*.bin file."""
        sl = np.ascontiguousarray(slices, np.int32).reshape(-1, 6)
        vf = np.ascontiguousarray(vid_freq, np.float32)
        tf = np.ascontiguousarray(txt_freq, np.float32)
        sizes = np.clip(sl[:, 1::2] - sl[:, 0::2], 0, None).prod(axis=1)
        if vf.size != int(sizes.sum()) * ROPE_ROT or tf.size != sl.shape[0] * int(txt_len) * ROPE_ROT:
            raise ValueError("geometry_from_win: frequency tables do not match the windows")
        g = C.c_void_p()
        rc = lib().awa_geom_from_win(self.ptr, int(t), int(h), int(w), sl.shape[0], _ptr(sl),
                                     vf.ctypes.data_as(C.POINTER(C.c_float)),
                                     tf.ctypes.data_as(C.POINTER(C.c_float)), int(txt_len), C.byref(g),
                                     _stream_ptr(stream))
        self.check(rc, "awa_geom_from_win")
        return Geometry(self, g)

    # ---- the op
    def forward(self, geom, vqkv, tqkv, nq_v, nk_v, nq_t, nk_t, eps=1e-5, vattn=None, tattn=None,
                stream=None, noalloc=False):
        """AwaLayer::forward: torch tensors on the device; returns (vattn, tattn).
        noalloc=True calls awa_forward_noalloc (the library's fixed device
        scratch instead of the context's)."""
        import torch
        if vqkv.dtype == torch.bfloat16:
            dtype = AWA_BF16
        elif vqkv.dtype == torch.float32:
            dtype = AWA_F32
        else:
            raise TypeError(f"unsupported dtype {vqkv.dtype}")
        if tqkv.dtype != vqkv.dtype:
            raise TypeError("vqkv and tqkv must share a dtype")
        for t_ in (vqkv, tqkv):
            if not t_.is_cuda or not t_.is_contiguous():
                raise ValueError("inputs must be contiguous device tensors")
        Lv, TXT = vqkv.shape[0], tqkv.shape[0]
        if vqkv.shape[1] != QKV or tqkv.shape[1] != QKV:
            raise ValueError("rows must have 7680 columns (q|k|v)")
        gains = [g.to(device=vqkv.device, dtype=torch.float32).contiguous() for g in (nq_v, nk_v, nq_t, nk_t)]
        if vattn is None:
            vattn = torch.empty((Lv, DIM), dtype=vqkv.dtype, device=vqkv.device)
        if tattn is None:
            tattn = torch.empty((TXT, DIM), dtype=vqkv.dtype, device=vqkv.device)
        fn = lib().awa_forward_noalloc if noalloc else lib().awa_forward
        rc = fn(self.ptr, geom.ptr, dtype, C.c_void_p(vqkv.data_ptr()),
                               C.c_void_p(tqkv.data_ptr()), Lv, TXT,
                               *[C.c_void_p(g.data_ptr()) for g in gains], float(eps),
                               C.c_void_p(vattn.data_ptr()), C.c_void_p(tattn.data_ptr()),
                               _stream_ptr(stream))
        self.check(rc, "awa_forward_noalloc" if noalloc else "awa_forward")
        self._keep = gains  # alive until the stream consumed them
        return vattn, tattn

    def time_phases(self, geom, vqkv, tqkv, nq_v, nk_v, nq_t, nk_t, reps, eps=1e-5, vattn=None,
                    tattn=None, stream=None):
        """awa_time_phases: the op, then each of its kernels (pack, attention,
        text average) `reps` more times back to back between two events;
        returns the mean ms per launch of each, (pack, attention, text)."""
        import torch
        dtype = AWA_BF16 if vqkv.dtype == torch.bfloat16 else AWA_F32
        Lv, TXT = vqkv.shape[0], tqkv.shape[0]
        gains = [g.to(device=vqkv.device, dtype=torch.float32).contiguous() for g in (nq_v, nk_v, nq_t, nk_t)]
        if vattn is None:
            vattn = torch.empty((Lv, DIM), dtype=vqkv.dtype, device=vqkv.device)
        if tattn is None:
            tattn = torch.empty((TXT, DIM), dtype=vqkv.dtype, device=vqkv.device)
        ms = (C.c_double * 3)()
        rc = lib().awa_time_phases(self.ptr, geom.ptr, dtype, C.c_void_p(vqkv.data_ptr()),
                                   C.c_void_p(tqkv.data_ptr()), Lv, TXT,
                                   *[C.c_void_p(g.data_ptr()) for g in gains], float(eps),
                                   C.c_void_p(vattn.data_ptr()), C.c_void_p(tattn.data_ptr()), int(reps),
                                   ms, _stream_ptr(stream))
        self.check(rc, "awa_time_phases")
        return ms[0], ms[1], ms[2]

    # ---- boundary casts
    def cast_f32_to_bf16(self, src, out, stream=None):
        """awa_cast_f32_to_bf16: fp32 device tensor -> 16-bit device tensor (bf16 bits)."""
        if src.numel() != out.numel() or src.element_size() != 4 or out.element_size() != 2:
            raise ValueError("cast_f32_to_bf16: 4-byte source and 2-byte output of one size")
        rc = lib().awa_cast_f32_to_bf16(self.ptr, C.c_void_p(src.data_ptr()), C.c_void_p(out.data_ptr()),
                                        src.numel(), _stream_ptr(stream))
        self.check(rc, "awa_cast_f32_to_bf16")
        return out

    def cast_bf16_to_f32(self, src, out, stream=None):
        """awa_cast_bf16_to_f32: 16-bit device tensor (bf16 bits) -> fp32 device tensor."""
        if src.numel() != out.numel() or src.element_size() != 2 or out.element_size() != 4:
            raise ValueError("cast_bf16_to_f32: 2-byte source and 4-byte output of one size")
        rc = lib().awa_cast_bf16_to_f32(self.ptr, C.c_void_p(src.data_ptr()), C.c_void_p(out.data_ptr()),
                                        src.numel(), _stream_ptr(stream))
        self.check(rc, "awa_cast_bf16_to_f32")
        return out

    def stream_copy(self, src, out, stream=None):
        """awa_stream_copy: device copy of src's bytes into out (the HBM ceiling's copy kernel)."""
        nb = src.numel() * src.element_size()
        if out.numel() * out.element_size() != nb or not (src.is_contiguous() and out.is_contiguous()):
            raise ValueError("stream_copy: contiguous source and output of one byte size")
        rc = lib().awa_stream_copy(self.ptr, C.c_void_p(out.data_ptr()), C.c_void_p(src.data_ptr()), nb,
                                   _stream_ptr(stream))
        self.check(rc, "awa_stream_copy")
        return out

    # ---- the DiT block (include/dit_capi.h)
    def gemm(self, A, W, out=None, stream=None):
        """C = A W^T, bf16 [M,K] x [N,K] -> [M,N] bf16 (the block's GEMM kernel)."""
        import torch
        M, K = A.shape
        N = W.shape[0]
        if out is None:
            out = torch.empty((M, N), dtype=torch.bfloat16, device=A.device)
        rc = lib().dit_gemm_bf16(self.ptr, C.c_void_p(A.data_ptr()), C.c_void_p(W.data_ptr()),
                                 C.c_void_p(out.data_ptr()), M, N, K, _stream_ptr(stream))
        self.check(rc, "dit_gemm_bf16")
        return out

    def pack_mlp(self, w_in, w_gate, stream=None):
        import torch
        mlp = w_in.shape[0]
        out = torch.empty((2 * mlp, w_in.shape[1]), dtype=torch.bfloat16, device=w_in.device)
        rc = lib().dit_pack_mlp_weights(self.ptr, C.c_void_p(w_in.data_ptr()), C.c_void_p(w_gate.data_ptr()),
                                        mlp, C.c_void_p(out.data_ptr()), _stream_ptr(stream))
        self.check(rc, "dit_pack_mlp_weights")
        return out

    def time_embedding(self, t, w_in, b_in, w_hid, b_hid, w_out, b_out, stream=None):
        import torch
        emb = torch.empty(15360, dtype=torch.float32, device=w_in.device)
        ts = (w_in, b_in, w_hid, b_hid, w_out, b_out)
        rc = lib().dit_time_embedding(self.ptr, float(t), *[C.c_void_p(x.data_ptr()) for x in ts],
                                      C.c_void_p(emb.data_ptr()), _stream_ptr(stream))
        self.check(rc, "dit_time_embedding")
        return emb

    def reserve(self, geom, dtype="bf16"):
        """awa_reserve: size the op's scratch for geom in this storage dtype."""
        self.check(lib().awa_reserve(self.ptr, geom.ptr, AWA_BF16 if dtype == "bf16" else AWA_F32), "awa_reserve")

    def dit_reserve(self, geom, mlp=6912):
        """dit_reserve: size the layer / embed / final workspaces and the op's scratch."""
        self.check(lib().dit_reserve(self.ptr, geom.ptr, int(mlp)), "dit_reserve")

    def layer(self, geom, vbranch, tbranch, emb, x, Lv, TXT, mlp=6912, txt_vid_only=False, eps=1e-5,
              stream=None):
        """dit_layer_forward in place on x (fp32 [Lv+TXT, 2560]).  Branches are dicts of
        device tensors keyed like dit_branch; pass the same dict for shared layers."""
        vb = DitBranch(**{k: vbranch[k].data_ptr() for k in BRANCH_FIELDS})
        tb = vb if tbranch is vbranch else DitBranch(**{k: tbranch[k].data_ptr() for k in BRANCH_FIELDS})
        rc = lib().dit_layer_forward(self.ptr, geom.ptr, C.byref(vb), C.byref(tb),
                                     C.c_void_p(emb.data_ptr()), int(mlp), int(bool(txt_vid_only)),
                                     float(eps), C.c_void_p(x.data_ptr()), int(Lv), int(TXT),
                                     _stream_ptr(stream))
        self.check(rc, "dit_layer_forward")
        return x

    def io_layers(self, weights, stream=None):
        """dit_io_create from a dict of device tensors keyed like dit_io_weights; the
        returned object keeps the tensors alive (the handle borrows some of them)."""
        w = DitIoWeights(**{k: weights[k].data_ptr() for k in IO_FIELDS})
        h = C.c_void_p()
        self.check(lib().dit_io_create(self.ptr, C.byref(w), C.byref(h), _stream_ptr(stream)), "dit_io_create")
        return DitIo(self, h, weights)

    def embed(self, io, grid, txt, x=None, stream=None):
        """dit_embed: grid fp32 (T, H, W, 33), txt fp32 [TXT, 5120] -> x fp32 [Lv+TXT, 2560]."""
        import torch
        T, H, W, _ = grid.shape
        TXT = txt.shape[0]
        Lv = T * (H // 2) * (W // 2)
        if x is None:
            x = torch.empty((Lv + TXT, DIM), dtype=torch.float32, device=grid.device)
        rc = lib().dit_embed(self.ptr, io.ptr, C.c_void_p(grid.data_ptr()), int(T), int(H), int(W),
                             C.c_void_p(txt.data_ptr()), int(TXT), C.c_void_p(x.data_ptr()), _stream_ptr(stream))
        self.check(rc, "dit_embed")
        return x

    def final(self, io, emb, x, T, H, W, eps=1e-5, out=None, stream=None):
        """dit_final: video rows of x -> fp32 (T, H, W, 16)."""
        import torch
        if out is None:
            out = torch.empty((T, H, W, 16), dtype=torch.float32, device=x.device)
        rc = lib().dit_final(self.ptr, io.ptr, C.c_void_p(emb.data_ptr()), C.c_void_p(x.data_ptr()), int(T),
                             int(H), int(W), float(eps), C.c_void_p(out.data_ptr()), _stream_ptr(stream))
        self.check(rc, "dit_final")
        return out

    def forward_grid(self, io, time_w, layers, geom_even, geom_odd, t, grid, txt, mlp=6912,
                     last_txt_vid_only=False, eps=1e-5, x=None, out=None, stream=None):
        """dit_forward_grid.  time_w: 6 device tensors (w_in, b_in, w_hid, b_hid, w_out, b_out);
        layers: list of (video branch dict, text branch dict) of device tensors."""
        import torch
        T, H, W, _ = grid.shape
        TXT = txt.shape[0]
        Lv = T * (H // 2) * (W // 2)
        if x is None:
            x = torch.empty((Lv + TXT, DIM), dtype=torch.float32, device=grid.device)
        if out is None:
            out = torch.empty((T, H, W, 16), dtype=torch.float32, device=grid.device)
        tw = DitTimeWeights(*[w.data_ptr() for w in time_w])
        cache = {}

        def br(d):
            if id(d) not in cache:
                cache[id(d)] = DitBranch(**{k: d[k].data_ptr() for k in BRANCH_FIELDS})
            return cache[id(d)]
        n = len(layers)
        vb = (C.POINTER(DitBranch) * max(n, 1))(*[C.pointer(br(v)) for v, _ in layers])
        tb = (C.POINTER(DitBranch) * max(n, 1))(*[C.pointer(br(t_)) for _, t_ in layers])
        rc = lib().dit_forward_grid(self.ptr, io.ptr, C.byref(tw), vb, tb, n, geom_even.ptr,
                                    geom_odd.ptr if geom_odd is not None else None, int(mlp),
                                    int(bool(last_txt_vid_only)), float(eps), float(t),
                                    C.c_void_p(grid.data_ptr()), int(T), int(H), int(W),
                                    C.c_void_p(txt.data_ptr()), int(TXT), C.c_void_p(x.data_ptr()),
                                    C.c_void_p(out.data_ptr()), _stream_ptr(stream))
        self.check(rc, "dit_forward_grid")
        return out

    def load_model(self, path, n_layers, mm_layers, stream=None):
        """dit_model_load of a model directory in the reference's layout."""
        h = C.c_void_p()
        self.check(lib().dit_model_load(self.ptr, str(path).encode(), int(n_layers), int(mm_layers), C.byref(h),
                                        _stream_ptr(stream)), "dit_model_load")
        return DitModel(self, h)

    def load_graph_model(self, param, bin_path, model_dir=None, mm_layers=-1, stream=None):
        """dit_model_load_graph: a merged whole-model graph (.param/.bin), the
        timestep MLP from model_dir."""
        h = C.c_void_p()
        self.check(lib().dit_model_load_graph(self.ptr, str(param).encode(), str(bin_path).encode(),
                                              str(model_dir).encode() if model_dir is not None else None,
                                              int(mm_layers), C.byref(h), _stream_ptr(stream)),
                   "dit_model_load_graph")
        return DitModel(self, h)

    def model_forward_grid(self, model, geom_even, geom_odd, t, grid, txt, last_txt_vid_only=False, eps=1e-5,
                           x=None, out=None, stream=None):
        import torch
        T, H, W, _ = grid.shape
        TXT = txt.shape[0]
        Lv = T * (H // 2) * (W // 2)
        if x is None:
            x = torch.empty((Lv + TXT, DIM), dtype=torch.float32, device=grid.device)
        if out is None:
            out = torch.empty((T, H, W, 16), dtype=torch.float32, device=grid.device)
        rc = lib().dit_model_forward_grid(self.ptr, model.ptr, geom_even.ptr,
                                          geom_odd.ptr if geom_odd is not None else None,
                                          int(bool(last_txt_vid_only)), float(eps), float(t),
                                          C.c_void_p(grid.data_ptr()), int(T), int(H), int(W),
                                          C.c_void_p(txt.data_ptr()), int(TXT), C.c_void_p(x.data_ptr()),
                                          C.c_void_p(out.data_ptr()), _stream_ptr(stream))
        self.check(rc, "dit_model_forward_grid")
        return out

    def model_graph(self, model, geom_even, geom_odd, t, grid, txt, x, out, last_txt_vid_only=False,
                    eps=1e-5, stream=None):
        """dit_graph_create: model_forward_grid captured for these buffers (run
        once eagerly, so out already holds the result); DitGraph.launch replays it."""
        T, H, W, _ = grid.shape
        h = C.c_void_p()
        rc = lib().dit_graph_create(self.ptr, model.ptr, geom_even.ptr,
                                    geom_odd.ptr if geom_odd is not None else None,
                                    int(bool(last_txt_vid_only)), float(eps), float(t),
                                    C.c_void_p(grid.data_ptr()), int(T), int(H), int(W),
                                    C.c_void_p(txt.data_ptr()), int(txt.shape[0]), C.c_void_p(x.data_ptr()),
                                    C.c_void_p(out.data_ptr()), _stream_ptr(stream), C.byref(h))
        self.check(rc, "dit_graph_create")
        return DitGraph(self, h.value, (model, geom_even, geom_odd, grid, txt, x, out))

    def dit_timing_read(self):
        a, b, c = C.c_double(), C.c_double(), C.c_double()
        n = C.c_int()
        self.check(lib().dit_timing_read(self.ptr, C.byref(a), C.byref(b), C.byref(c), C.byref(n)),
                   "dit_timing_read")
        return a.value, b.value, c.value, n.value

    def forward_host(self, geom, vqkv, tqkv, nq_v, nk_v, nq_t, nk_t, eps=1e-5):
        """AwaVk::forward: numpy fp32 in and out, synchronous."""
        f = lambda a: np.ascontiguousarray(a, np.float32)
        vqkv, tqkv = f(vqkv), f(tqkv)
        g4 = [f(x) for x in (nq_v, nk_v, nq_t, nk_t)]
        Lv, TXT = vqkv.shape[0], tqkv.shape[0]
        vo = np.empty((Lv, DIM), np.float32)
        to = np.empty((TXT, DIM), np.float32)
        P = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
        rc = lib().awa_forward_host(self.ptr, geom.ptr, P(vqkv), P(tqkv), Lv, TXT, *[P(x) for x in g4],
                                    float(eps), P(vo), P(to))
        self.check(rc, "awa_forward_host")
        return vo, to


class Geometry:
    def __init__(self, ctx, ptr):
        self.ctx = ctx
        self.ptr = ptr

    def info(self):
        gi = GeomInfo()
        rc = lib().awa_geom_query(self.ptr, C.byref(gi))
        if rc != AWA_OK:
            raise AwaError(rc, "awa_geom_query")
        return {n: getattr(gi, n) for n, _ in GeomInfo._fields_}

    def read(self):
        i = self.info()
        sl = np.zeros((i["nwin"], 6), np.int32)
        cumf = np.zeros(i["nwin"] + 1, np.int32)
        vidx = np.zeros(i["sumf"], np.int32)
        vf = np.zeros((i["sumf"], ROPE_ROT), np.float32)
        tf = np.zeros((i["nwin"] * i["txt_len"], ROPE_ROT), np.float32)
        rc = lib().awa_geom_read(self.ctx.ptr, self.ptr, *[C.c_void_p(a.ctypes.data) for a in (sl, cumf, vidx, vf, tf)])
        self.ctx.check(rc, "awa_geom_read")
        return {"slices": sl, "cumf": cumf, "vidx": vidx, "vid_freq": vf, "txt_freq": tf}

    def close(self):
        if self.ptr:
            lib().awa_geom_destroy(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DitIo:
    """Handle of dit_io_create; destroyed with the object."""

    def __init__(self, ctx, ptr, weights):
        self.ctx, self.ptr, self._weights = ctx, ptr, weights

    def close(self):
        if self.ptr:
            lib().dit_io_destroy(self.ctx.ptr, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DitGraph:
    """Handle of dit_graph_create; keeps what the graph reads alive."""

    def __init__(self, ctx, ptr, keep):
        self.ctx, self.ptr, self._keep = ctx, ptr, keep

    def launch(self, stream=None):
        self.ctx.check(lib().dit_graph_launch(self.ctx.ptr, self.ptr, _stream_ptr(stream)), "dit_graph_launch")

    def close(self):
        if self.ptr:
            lib().dit_graph_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DitModel:
    """Handle of dit_model_load; destroyed with the object."""

    def __init__(self, ctx, ptr):
        self.ctx, self.ptr = ctx, ptr

    def info(self):
        a, b, c = C.c_int(), C.c_int(), C.c_int()
        lib().dit_model_info(self.ptr, C.byref(a), C.byref(b), C.byref(c))
        return {"n_layers": a.value, "mm_layers": b.value, "mlp": c.value}

    def close(self):
        if self.ptr:
            lib().dit_model_destroy(self.ctx.ptr, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

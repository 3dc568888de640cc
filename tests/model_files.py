"""Writers of the reference's on-disk formats, for the loader tests (test infrastructure).

write_linear: ncnn InnerProduct pair as load_linear reads it (verify_dit.cpp:80-102):
.param with an InnerProduct line carrying 0=num_output 1=bias_term 2=weight_data_size,
.bin = storage tag (0x01306B47 fp16 / 0 fp32), the [out][in] weight, then the fp32 bias.
write_raw_f: read_raw_f's int64 ndim, int64 shape, float32 data (dit_vk.cpp:38-45).
write_win: load_win's 10 int64 header, nwin x 6 int64 slices, vid_freq then txt_freq
float32 (dit_vk.cpp:74-93).
"""
import os

import numpy as np

TAG_FP16 = 0x01306B47


def write_linear(base, w, b=None, fp16=True):
    n_out, n_in = w.shape
    with open(base + ".param", "w") as f:
        f.write("7767517\n2 2\n")
        f.write("Input in0 0 1 in0\n")
        f.write(f"InnerProduct linear 1 1 in0 out0 0={n_out} 1={int(b is not None)} 2={n_out * n_in}\n")
    with open(base + ".bin", "wb") as f:
        f.write(np.uint32(TAG_FP16 if fp16 else 0).tobytes())
        f.write(np.ascontiguousarray(w, np.float16 if fp16 else np.float32).tobytes())
        if b is not None:
            f.write(np.ascontiguousarray(b, np.float32).tobytes())


def write_raw_f(path, a):
    a = np.array(a, np.float32, order="C")   # keeps 0-d arrays 0-d
    with open(path, "wb") as f:
        f.write(np.int64(a.ndim).tobytes())
        f.write(np.asarray(a.shape, np.int64).tobytes())
        f.write(a.tobytes())


def write_win(path, header, slices, vid_freq, txt_freq):
    with open(path, "wb") as f:
        f.write(np.asarray(header, np.int64).tobytes())
        f.write(np.asarray(slices, np.int64).tobytes())
        f.write(np.ascontiguousarray(vid_freq, np.float32).tobytes())
        f.write(np.ascontiguousarray(txt_freq, np.float32).tobytes())


def write_model(root, io, layers, time_ws, mm_layers, fp16=True):
    """A model directory in the reference's layout (verify_dit.cpp:351-384):
    io = dit_reference.random_io dict, layers = [(vid branch, txt branch)] with
    dit_reference.random_branch dicts, time_ws = the six timestep-MLP arrays."""
    os.makedirs(root, exist_ok=True)
    p = lambda n: os.path.join(root, n)
    write_linear(p("vid_in_proj"), io["vid_in_w"], io["vid_in_b"], fp16)
    write_linear(p("txt_in"), io["txt_in_w"], io["txt_in_b"], fp16)
    write_linear(p("vid_out_proj"), io["vid_out_w"], io["vid_out_b"], fp16)
    for n in ("out_norm_w", "out_ada_shift", "out_ada_scale"):
        write_raw_f(p("vid_" + n + ".bin"), io[n])
    for n, (w, b) in zip(("emb_proj_in", "emb_proj_hid", "emb_proj_out"),
                         ((time_ws[0], time_ws[1]), (time_ws[2], time_ws[3]), (time_ws[4], time_ws[5]))):
        write_linear(p(n), w, b, fp16)
    for i, (vb, tb) in enumerate(layers):
        names = [(f"b{i}_vid", vb), (f"b{i}_txt", tb)] if i < mm_layers else [(f"b{i}_all", vb)]
        for base, br in names:
            write_linear(p(base + "_qkv"), br["qkv_w"], None, fp16)
            write_linear(p(base + "_out"), br["out_w"], br["out_b"], fp16)
            write_linear(p(base + "_mlp_in"), br["mlp_in_w"], None, fp16)
            write_linear(p(base + "_mlp_g"), br["mlp_g_w"], None, fp16)
            write_linear(p(base + "_mlp_out"), br["mlp_out_w"], None, fp16)
            for k in ("nq", "nk", "attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
                write_raw_f(p(f"{base}_{k}.bin"), br[k])

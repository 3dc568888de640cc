"""Writers of the reference's on-disk formats, for the loader tests (test infrastructure).

write_linear: ncnn InnerProduct pair as load_linear reads it (verify_dit.cpp:80-102):
.param with an InnerProduct line carrying 0=num_output 1=bias_term 2=weight_data_size,
.bin = storage tag (0x01306B47 fp16 / 0 fp32), the [out][in] weight, then the fp32 bias.
write_raw_f: read_raw_f's int64 ndim, int64 shape, float32 data (dit_vk.cpp:38-45).
write_win: load_win's 10 int64 header, nwin x 6 int64 slices, vid_freq then txt_freq
float32 (dit_vk.cpp:74-93).
write_graph: the merged whole-model graph built from a model directory the way
export_dit_graph.py:47-258 builds it (layer lines, and the .bin as the concatenation
of each layer's weights in layer order).
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
        data = np.ascontiguousarray(w, np.float16 if fp16 else np.float32).tobytes()
        f.write(data + b"\0" * (-len(data) % 4))   # fp16 data is padded to 4 bytes
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


def _ip_line(root, base, bottom, top, name):
    """An InnerProduct line with the .param values of <base>.param, and its .bin bytes."""
    last = open(os.path.join(root, base + ".param")).read().splitlines()[-1]
    kv = dict(t.split("=", 1) for t in last.split() if "=" in t)
    return (f"InnerProduct {name} 1 1 {bottom} {top} 0={kv['0']} 1={kv['1']} 2={kv['2']}",
            open(os.path.join(root, base + ".bin"), "rb").read())


def _raw_data(path):
    """The float32 data of a read_raw_f file (its header dropped)."""
    b = open(path, "rb").read()
    nd = int(np.frombuffer(b[:8], np.int64)[0])
    return b[8 + 8 * nd:]


def write_graph(root, out_param, out_bin, n_layers, mm_layers, ada_compose=True, dim=2560, txt=58):
    """Merge the model directory root into one graph, layer lines and weights in the
    exporter's order: Inputs, AdaCompose (per layer and flow the six ada vectors
    shift/scale/gate of attn then mlp, then the output layer's shift and scale, each
    tagged fp32), the input projections, per layer RMSNorm/BinaryOp/InnerProduct/AWA
    (four tagged 128-vectors nq_v, nk_v, nq_t, nk_t)/Swish lines, then the final
    RMSNorm (raw gamma) and vid_out_proj.  ada_compose=False writes the older
    layout whose ada vectors are graph inputs (no weights)."""
    tag0 = np.uint32(0).tobytes()
    lines, parts = [], []
    P = lambda n: os.path.join(root, n)

    def br(i, f):
        return f"b{i}_{'vid' if f == 'v' else 'txt'}" if i < mm_layers else f"b{i}_all"

    def inp(name):
        lines.append(f"Input {name} 0 1 {name}")

    def ip(base, bottom, top, name):
        line, data = _ip_line(root, base, bottom, top, name)
        lines.append(line)
        parts.append(data)

    inp("in_vid0")
    inp("in_txt0")
    ada = {(i, f): tuple(f"ada_{i}_{f}_{k}" for k in ("a_sc", "a_sh", "a_g", "m_sc", "m_sh", "m_g"))
           for i in range(n_layers) for f in "vt"}
    if ada_compose:
        inp("emb")
        outs = [n for i in range(n_layers) for f in "vt" for n in ada[i, f]] + ["ada_fin_sc", "ada_fin_sh"]
        lines.append(f"AdaCompose ada_compose 1 {len(outs)} emb {' '.join(outs)} "
                     f"0=\"models/m5/\" 1={n_layers} 2={mm_layers} 3={dim} 4=1")
        for i in range(n_layers):
            for f in "vt":
                for k in ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
                    parts.append(tag0 + _raw_data(P(f"{br(i, f)}_{k}.bin")))
        parts.append(tag0 + _raw_data(P("vid_out_ada_shift.bin")))
        parts.append(tag0 + _raw_data(P("vid_out_ada_scale.bin")))
    else:
        for i in range(n_layers):
            for f in "vt":
                for n in ada[i, f]:
                    inp(n)
        inp("ada_fin_sc")
        inp("ada_fin_sh")
    ip("vid_in_proj", "in_vid0", "v_cur_0", "proj_vid_in")
    ip("txt_in", "in_txt0", "t_cur_0", "proj_txt_in")
    for i in range(n_layers):
        for f in "vt":
            sc, sh = ada[i, f][0], ada[i, f][1]
            lines.append(f"RMSNorm rn_a_{i}_{f} 1 1 {f}_cur_{i} {f}_rn_{i} 0={dim} 1=0.00001 2=0")
            lines.append(f"BinaryOp ad_sc_{i}_{f} 2 1 {f}_rn_{i} {sc} {f}_m1_{i} 0=2")
            lines.append(f"BinaryOp ad_sh_{i}_{f} 2 1 {f}_m1_{i} {sh} {f}_m2_{i} 0=0")
            ip(f"{br(i, f)}_qkv", f"{f}_m2_{i}", f"{f}_qkv_{i}", f"qkv_{i}_{f}")
        lines.append(f"AWA awa_{i} 2 2 v_qkv_{i} t_qkv_{i} v_attn_{i} t_attn_{i} 0=\"models/m5/\" "
                     f"1={i % 2} 2=0 3={txt}")
        for f in "vt":
            for k in ("nq", "nk"):
                parts.append(tag0 + _raw_data(P(f"{br(i, f)}_{k}.bin")))
        for f in "vt":
            ip(f"{br(i, f)}_out", f"{f}_attn_{i}", f"{f}_outp_{i}", f"out_{i}_{f}")
        for f in "vt":
            lines.append(f"BinaryOp g_{i}_{f} 2 1 {f}_outp_{i} {ada[i, f][2]} {f}_g_{i} 0=2")
        for f in "vt":
            lines.append(f"BinaryOp res_{i}_{f} 2 1 {f}_g_{i} {f}_cur_{i} {f}_cur_{i}_a 0=0")
        for f in "vt":
            a_g, m_sc, m_sh, m_g = ada[i, f][2:]
            lines.append(f"RMSNorm rn_m_{i}_{f} 1 1 {f}_cur_{i}_a {f}_rn2_{i} 0={dim} 1=0.00001 2=0")
            lines.append(f"BinaryOp ad_msc_{i}_{f} 2 1 {f}_rn2_{i} {m_sc} {f}_m3_{i} 0=2")
            lines.append(f"BinaryOp ad_msh_{i}_{f} 2 1 {f}_m3_{i} {m_sh} {f}_m4_{i} 0=0")
            ip(f"{br(i, f)}_mlp_in", f"{f}_m4_{i}", f"{f}_h_{i}", f"min_{i}_{f}")
            ip(f"{br(i, f)}_mlp_g", f"{f}_m4_{i}", f"{f}_g2_{i}", f"mig_{i}_{f}")
            lines.append(f"Swish sw_{i}_{f} 1 1 {f}_g2_{i} {f}_gs_{i}")
            lines.append(f"BinaryOp mul_{i}_{f} 2 1 {f}_h_{i} {f}_gs_{i} {f}_hs_{i} 0=2")
            ip(f"{br(i, f)}_mlp_out", f"{f}_hs_{i}", f"{f}_o_{i}", f"mout_{i}_{f}")
            lines.append(f"BinaryOp mg_{i}_{f} 2 1 {f}_o_{i} {m_g} {f}_og_{i} 0=2")
            lines.append(f"BinaryOp mres_{i}_{f} 2 1 {f}_og_{i} {f}_cur_{i}_a {f}_cur_{i + 1} 0=0")
    lines.append(f"RMSNorm rn_fin 1 1 v_cur_{n_layers} v_fin 0={dim} 1=0.00001 2=1")
    parts.append(_raw_data(P("vid_out_norm_w.bin")))
    lines.append("BinaryOp fin_sc 2 1 v_fin ada_fin_sc v_f1 0=2")
    lines.append("BinaryOp fin_sh 2 1 v_f1 ada_fin_sh v_f2 0=0")
    ip("vid_out_proj", "v_f2", "out0", "outproj")
    n_blobs = sum(int(ln.split()[3]) for ln in lines)
    with open(out_param, "w") as f:
        f.write("\n".join(["7767517", f"{len(lines)} {n_blobs}"] + lines) + "\n")
    with open(out_bin, "wb") as f:
        for b in parts:
            f.write(b)

"""The host file readers (seedvr2-2b-ncnn_amd/csrc/dit_files.cpp) under
AddressSanitizer and UndefinedBehaviorSanitizer, on valid files and on
truncated and corrupted ones.

The readers parse files a caller hands over (read_raw_f vectors, dit_vk.cpp:
38-45; ncnn InnerProduct .param/.bin pairs, verify_dit.cpp:80-102; window
files, dit_vk.cpp:74-93; the merged graph, export_dit_graph.py:47-258).  The
driver tests/cpp/test_files.cpp is built here with g++ and the sanitizers
(host code only, no GPU) and run on: valid files written by
tests/model_files.py (the reader must succeed and return what was written);
every prefix-truncation at a spread of lengths; header fields set to zero,
negative, huge and random values; and .param lines with corrupted numbers or
removed lines.  A corrupted file must give rc=-1 or a clean success, never a
sanitizer report or a crash.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest

from model_files import write_graph, write_linear, write_model, write_raw_f, write_win

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = [os.path.join(ROOT, "tests", "cpp", "test_files.cpp"),
       os.path.join(ROOT, "seedvr2-2b-ncnn_amd", "csrc", "dit_files.cpp")]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = str(tmp_path_factory.mktemp("asan") / "test_files")
    cmd = [gxx, "-std=c++17", "-g", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROOT, "seedvr2-2b-ncnn_amd", "csrc")] + SRC + ["-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def run(driver, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=24")
    r = subprocess.run([driver] + [str(a) for a in args], capture_output=True, text=True, env=env, timeout=60)
    assert r.returncode == 0 and "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, \
        f"{args}: rc {r.returncode}\n{r.stdout[-1000:]}\n{r.stderr[-3000:]}"
    last = r.stdout.strip().splitlines()[-1]
    assert last.startswith("rc="), r.stdout
    return int(last.split()[0][3:]), r.stdout


def mutants(data, rng, header_words, word_size=8):
    """Truncations at a spread of lengths, and header words overwritten."""
    n = len(data)
    cuts = sorted({0, 1, 3, 4, 7, 8, 9, 15, 16, 17, 24, 40, 79, 80, 81, n // 3, n // 2, n - 5, n - 1})
    for c in cuts:
        if 0 <= c < n:
            yield f"cut{c}", data[:c]
    big = [0, 1, -1, -2 ** 31, 2 ** 31 - 1, 2 ** 40, -2 ** 62, 2 ** 62, 4097, 5000]
    for w in range(header_words):
        for v in big:
            b = bytearray(data)
            if word_size == 8:
                b[8 * w:8 * w + 8] = np.int64(v).tobytes()
            else:
                b[4 * w:4 * w + 4] = np.int64(v).astype(np.int32).tobytes()
            yield f"w{w}={v}", bytes(b)
    for k in range(6):
        b = bytearray(data)
        pos = rng.integers(0, n, size=8)
        for p in pos:
            b[p] = rng.integers(0, 256)
        yield f"rand{k}", bytes(b)


def test_raw_f(driver, tmp_path):
    rng = np.random.default_rng(11)
    a = rng.standard_normal((3, 5, 7)).astype(np.float32)
    p = tmp_path / "v.bin"
    write_raw_f(str(p), a)
    rc, out = run(driver, "raw", p)
    assert rc == 0 and f"n={a.size} ndim=3" in out
    data = p.read_bytes()
    n_bad = 0
    for tag, m in mutants(data, rng, header_words=4):
        q = tmp_path / f"m_{tag}.bin"
        q.write_bytes(m)
        rc, _ = run(driver, "raw", q)
        n_bad += rc != 0
    assert n_bad > 20


def test_linear(driver, tmp_path):
    rng = np.random.default_rng(12)
    w = rng.standard_normal((24, 40)).astype(np.float32)
    b = rng.standard_normal(24).astype(np.float32)
    for fp16 in (True, False):
        base = tmp_path / ("l16" if fp16 else "l32")
        write_linear(str(base), w, b, fp16=fp16)
        rc, out = run(driver, "linear", base, 1)
        assert rc == 0 and "out=24 in=40" in out
        data = (tmp_path / (base.name + ".bin")).read_bytes()
        for tag, m in mutants(data, rng, header_words=1, word_size=4):
            mb = tmp_path / f"m{tag}"
            (tmp_path / f"m{tag}.bin").write_bytes(m)
            shutil.copy(str(base) + ".param", str(mb) + ".param")
            run(driver, "linear", mb, 1)
        ptext = open(str(base) + ".param").read()
        for k, (old, new) in enumerate((("0=24", "0=-24"), ("0=24", "0=0"), ("2=960", "2=-960"),
                                         ("2=960", "2=961"), ("0=24", "0=2147483647"),
                                         ("2=960", "2=9223372036854775807"), ("InnerProduct", "Inner"),
                                         ("0=24", "0=24x"))):
            mb = tmp_path / f"p{k}"
            open(str(mb) + ".param", "w").write(ptext.replace(old, new))
            shutil.copy(str(base) + ".bin", str(mb) + ".bin")
            rc, _ = run(driver, "linear", mb, 1)
            assert rc != 0 or new == "0=24x"


def test_win(driver, tmp_path):
    rng = np.random.default_rng(13)
    sl = np.array([[0, 1, 0, 4, 0, 5], [0, 1, 4, 8, 0, 5]], np.int64)
    vf = rng.standard_normal((40, 126)).astype(np.float32)
    tf = rng.standard_normal((2 * 9, 126)).astype(np.float32)
    p = tmp_path / "w.bin"
    write_win(str(p), [1, 8, 5, 1, 2, 1, 1, 0, 0, 2], sl, vf, tf)
    rc, out = run(driver, "win", p, 9)
    assert rc == 0 and "nwin=2 nv=5040 nt=2268" in out
    data = p.read_bytes()
    for tag, m in mutants(data, rng, header_words=12):
        q = tmp_path / f"m_{tag}.bin"
        q.write_bytes(m)
        run(driver, "win", q, 9)
    for txt in (0, -1, 100000):
        run(driver, "win", p, txt)


def _tiny_model(root, rng, dim=64, mlp=32, n_layers=2, mm=1):
    h = lambda *s: (rng.standard_normal(s) * 0.05).astype(np.float32)
    io = {"vid_in_w": h(dim, 132), "vid_in_b": h(dim), "txt_in_w": h(dim, 48), "txt_in_b": h(dim),
          "vid_out_w": h(64, dim), "vid_out_b": h(64), "out_norm_w": h(dim), "out_ada_shift": h(dim),
          "out_ada_scale": h(dim)}

    def branch():
        b = {"qkv_w": h(3 * dim, dim), "out_w": h(dim, dim), "out_b": h(dim), "mlp_in_w": h(mlp, dim),
             "mlp_g_w": h(mlp, dim), "mlp_out_w": h(dim, mlp), "nq": h(128), "nk": h(128)}
        for k in ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
            b[k] = h(dim)
        return b

    layers = [(branch(), branch()) for _ in range(n_layers)]
    tws = [h(dim, 256), h(dim), h(dim, dim), h(dim), h(6 * dim, dim), h(6 * dim)]
    write_model(root, io, layers, tws, mm_layers=mm, fp16=True)


def test_graph(driver, tmp_path):
    rng = np.random.default_rng(14)
    model = str(tmp_path / "m5")
    _tiny_model(model, rng)
    param, binf = str(tmp_path / "g.param"), str(tmp_path / "g.bin")
    write_graph(model, param, binf, 2, 1, ada_compose=True, dim=64, txt=9)
    rc, out = run(driver, "graph", param, binf, -1, "b1_all_qkv")
    assert rc == 0 and "layers=2 mm=1" in out and "out=192 in=64" in out
    for name in ("b0_txt_mlp_out", "b0_vid_nq", "vid_out_norm_w", "b1_all_attn_gate", "vid_in_proj"):
        rc, _ = run(driver, "graph", param, binf, -1, name)
        assert rc == 0, name
    data = open(binf, "rb").read()
    for tag, m in mutants(data, rng, header_words=3, word_size=4):
        q = tmp_path / f"mb_{tag}.bin"
        q.write_bytes(m)
        run(driver, "graph", param, q, -1, "vid_out_norm_w")
    lines = open(param).read().splitlines()
    cases = []
    for i, ln in enumerate(lines[2:], start=2):
        toks = ln.split()
        for j, t in enumerate(toks):
            if "=" in t and not t.startswith(("0=\"", "0='")):
                k, v = t.split("=", 1)
                for nv in ("-1", "0", "999999999", "-999999999", "x"):
                    cases.append((i, j, f"{k}={nv}"))
    rng.shuffle(cases)
    for n, (i, j, nt) in enumerate(cases[:60]):
        toks = lines[i].split()
        toks[j] = nt
        mod = lines[:i] + [" ".join(toks)] + lines[i + 1:]
        q = tmp_path / f"mp_{n}.param"
        q.write_text("\n".join(mod) + "\n")
        run(driver, "graph", q, binf, -1, "vid_out_norm_w")
        run(driver, "graph", q, binf, -1, "b0_vid_attn_shift")
    # sizes that would move the blob offsets backwards are refused outright
    for old, new in (("0=64 1=0.00001 2=1", "0=-64 1=0.00001 2=1"), (" 3=64 ", " 3=-64 ")):
        assert old in "\n".join(lines), old
        q = tmp_path / "neg.param"
        q.write_text("\n".join(lines).replace(old, new) + "\n")
        rc, out = run(driver, "graph", q, binf, -1, "vid_out_norm_w")
        assert rc == -1
    # value counts near 2^62 (tagged_bytes' 2 n + 3 and 4 n would overflow,
    # a vector of that size would throw): refused before any arithmetic
    text = "\n".join(lines)
    for k, key in enumerate(("2=", "0=")):
        ip = next(ln for ln in lines if ln.startswith("InnerProduct"))
        tok = next(t for t in ip.split() if t.startswith(key))
        for huge in ("4611686018427387904", "2305843009213693952", "9223372036854775807"):
            q = tmp_path / f"huge_{k}_{huge[:4]}.param"
            q.write_text(text.replace(ip, ip.replace(" " + tok, f" {key}{huge}"), 1) + "\n")
            rc, out = run(driver, "graph", q, binf, -1, "vid_out_norm_w")
            assert rc == -1, (key, huge)
    rn = next(ln for ln in lines if ln.startswith("RMSNorm") and " 2=1" in ln)
    tok = next(t for t in rn.split() if t.startswith("0="))
    q = tmp_path / "huge_rms.param"
    q.write_text(text.replace(rn, rn.replace(" " + tok, " 0=4611686018427387904"), 1) + "\n")
    rc, out = run(driver, "graph", q, binf, -1, "vid_out_norm_w")
    assert rc == -1
    for drop in (1, 2, 5, len(lines) // 2, len(lines) - 1):
        q = tmp_path / f"md_{drop}.param"
        q.write_text("\n".join(lines[:drop] + lines[drop + 1:]) + "\n")
        run(driver, "graph", q, binf, -1, "vid_out_norm_w")

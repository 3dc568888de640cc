"""No kernel of the library uses scratch (private) memory.

Each HIP source of seedvr2-2b-ncnn_amd/csrc is compiled to AMD assembly with
the library's own flags (as the Makefile expands them) and every kernel's
private segment size must be 0: a register spill or an array the compiler
could not keep in registers goes to scratch memory, which costs the hot loops
memory round trips (the fp32 attention kernel once kept its K/V staging array
there and ran 40 % slower).  The check is made on the CPU.
"""
import glob
import os
import re
import shlex
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "seedvr2-2b-ncnn_amd")
HIPCC = "/opt/rocm/bin/hipcc"
SOURCES = sorted(os.path.basename(p) for p in glob.glob(os.path.join(PKG, "csrc", "*.hip")))


def compile_flags(obj):
    r = subprocess.run(["make", "-n", "-B", "-C", PKG, "_build/" + obj], capture_output=True, text=True, timeout=60)
    line = next(l for l in r.stdout.split("\n") if "hipcc" in l and " -c " in l)
    toks = shlex.split(line.split(" -c ")[0])
    return [t for t in toks[1:] if t != "-fPIC"]


@pytest.mark.parametrize("src", SOURCES)
def test_no_scratch(src, tmp_path):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not present")
    out = tmp_path / (src + ".s")
    cmd = [HIPCC] + compile_flags(src.replace(".hip", ".o")) + ["--cuda-device-only", "-S",
                                                                os.path.join(PKG, "csrc", src), "-o", str(out)]
    r = subprocess.run(cmd, cwd=PKG, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    sizes = re.findall(r"\.set (\S+)\.private_seg_size, (\d+)", out.read_text())
    if src != "awa_noalloc.hip":  # that file holds the allocation-free entry's device array, no kernel
        assert sizes, "no kernels found"
    using = [(k, int(v)) for k, v in sizes if int(v) != 0]
    assert not using, using

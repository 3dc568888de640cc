"""Static check of the attention kernel's hand-placed fragment loads.

sdpa_bf16_kernel (seedvr2-2b-ncnn_amd/csrc/awa_sdpa.hip) loads the next work
item's query fragments with inline-asm `global_load_dwordx4 a[..]` straight
into accumulation registers while the current item finishes, and waits for
them with the item start's `s_waitcnt vmcnt(0)`; it reads the next
unit's K fragments with inline-asm `ds_read_b128 a[..]` a phase early and
waits for them with `s_waitcnt lgkmcnt(0)`.  The compiler does not see those
loads as loads: if it ever placed a copy or any other use of those registers
between a load and its wait (a phi copy on a loop edge, a move under register
pressure), the use would read stale data without any error.  This test
compiles the kernel to AMD assembly with the library's own flags (Makefile)
and proves on its control-flow graph that on every path from such a load no
instruction touches the loaded registers before a wait that covers it
(`vmcnt(N)` with at least N vector memory instructions issued after the load
on every path, `lgkmcnt(0)` for LDS reads).  The
analysis is checked on planted mistakes first.  A second
check: the kernel's LDS DMA takes its destination from M0, written by the
kernel's asm once per four DMA instructions, so no compiler-generated
instruction may write M0 anywhere in the kernel.  A third: the compiler puts
no wait states before an inline-asm statement, so asm that reads MFMA (or
transcendental) results must be fenced by the kernel itself; every such read
in the library's MFMA kernels is checked for its wait states on every path.
"""
import os
import re
import shlex
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "seedvr2-2b-ncnn_amd")
KERNEL = "_ZN3awa12_GLOBAL__N_116sdpa_bf16_kernelENS_8SdpaArgsE"
HIPCC = "/opt/rocm/bin/hipcc"

AREG = re.compile(r"\ba\[(\d+):(\d+)\]|\ba(\d+)\b")
LABEL = re.compile(r"^(\.LBB\d+_\d+):")
VMEM_LOAD = re.compile(r"^(global|buffer|flat)_load_")
LDS_LOAD = re.compile(r"^ds_read")
VMEM_ANY = re.compile(r"^(global|buffer|flat|scratch)_")


def makefile_flags():
    """The library's compile flags for awa_sdpa.hip, as make expands them."""
    r = subprocess.run(["make", "-n", "-B", "-C", PKG, "_build/awa_sdpa.o"], capture_output=True, text=True,
                       timeout=60)
    line = next(l for l in r.stdout.split("\n") if "awa_sdpa.hip" in l and "hipcc" in l)
    toks = shlex.split(line.split(" -c ")[0])
    return [t for t in toks[1:] if t != "-fPIC"]


def regs(operands):
    out = set()
    for m in AREG.finditer(operands):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def parse(asm_text):
    """The kernel's instructions as (label or None, opcode, operands) in order."""
    lines = asm_text.split("\n")
    start = next(i for i, l in enumerate(lines) if l.startswith(KERNEL + ":"))
    out = []
    for l in lines[start + 1:]:
        if l.startswith(".Lfunc_end"):
            break
        m = LABEL.match(l)
        if m:
            out.append((m.group(1), None, ""))
            continue
        s = l.split(";")[0].strip()
        if not s or s.startswith("."):
            continue
        op, _, rest = s.partition(" ")
        out.append((None, op, rest.strip()))
    return out


def check(insts, load=VMEM_LOAD, wait=r"vmcnt\(0\)"):
    """Returns the violations: (block, instruction, registers) where a
    register loaded by an AGPR-destination load (vector memory, or with
    load=LDS_LOAD an LDS read) is touched before an s_waitcnt covering it
    (wait) on some path, and the number of such loads."""
    # basic blocks
    blocks, order = {}, []
    cur = "entry"
    blocks[cur] = []
    order.append(cur)
    anon = 0
    for lab, op, rest in insts:
        if lab is not None:
            cur = lab
            blocks[cur] = []
            order.append(cur)
            continue
        blocks[cur].append((op, rest))
        if op.startswith("s_branch") or op.startswith("s_cbranch") or op == "s_endpgm":
            anon += 1
            cur = f"anon{anon}"
            blocks[cur] = []
            order.append(cur)
    succ = {}
    for i, b in enumerate(order):
        nxt = order[i + 1] if i + 1 < len(order) else None
        body = blocks[b]
        last = body[-1] if body else None
        s = []
        if last and last[0] == "s_endpgm":
            pass
        elif last and last[0].startswith("s_branch"):
            s.append(last[1].split()[0])
        else:
            if last and last[0].startswith("s_cbranch"):
                s.append(last[1].split()[0])
            if nxt is not None:
                s.append(nxt)
        succ[b] = [x for x in s if x in blocks]
    n_loads = sum(1 for b in order for op, rest in blocks[b] if load.match(op) and rest.startswith("a"))
    # pending: loaded register -> vector memory instructions issued since its
    # load (the fewest over the paths that reach here).  Vector memory
    # operations complete in issue order, so `s_waitcnt vmcnt(N)` covers a
    # load with at least N such instructions after it; for LDS reads (whose
    # counter SMEM shares, out of order) only a full wait counts.
    counted = load is VMEM_LOAD
    pend_in = {b: {} for b in order}
    violations = []

    def run(b, pending, record):
        pending = dict(pending)
        for op, rest in blocks[b]:
            if op == "s_waitcnt":
                if re.search(wait, rest):
                    pending.clear()
                    continue
                m = re.search(r"vmcnt\((\d+)\)", rest)
                if counted and m:
                    n = int(m.group(1))
                    pending = {r: c for r, c in pending.items() if c < n}
                continue
            r = regs(rest)
            if load.match(op) and rest.startswith("a"):
                for x in r:
                    pending[x] = 0
                continue
            hit = r & set(pending)
            if hit and record:
                violations.append((b, f"{op} {rest}", sorted(hit)))
            if counted and VMEM_ANY.match(op):
                pending = {x: c + 1 for x, c in pending.items()}
        return pending

    def merge(into, new):
        out = dict(into)
        for x, c in new.items():
            out[x] = min(c, out[x]) if x in out else c
        return out

    changed = True
    while changed:
        changed = False
        for b in order:
            out = run(b, pend_in[b], False)
            for s in succ[b]:
                m = merge(pend_in[s], out)
                if m != pend_in[s]:
                    pend_in[s] = m
                    changed = True
    for b in order:
        run(b, pend_in[b], True)
    return violations, n_loads


@pytest.fixture(scope="module")
def sdpa_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not present")
    out = tmp_path_factory.mktemp("asm") / "awa_sdpa.s"
    cmd = [HIPCC] + makefile_flags() + ["--cuda-device-only", "-S",
                                        os.path.join(PKG, "csrc", "awa_sdpa.hip"), "-o", str(out)]
    r = subprocess.run(cmd, cwd=PKG, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    return open(out).read()


def test_analysis_finds_planted_uses(sdpa_asm):
    insts = parse(sdpa_asm)
    k = next(i for i, (lab, op, rest) in enumerate(insts)
             if op and VMEM_LOAD.match(op) and rest.startswith("a"))
    reg = min(regs(insts[k][2]))
    # a copy of a loaded register right after the load: found
    planted = insts[:k + 1] + [(None, "v_accvgpr_read_b32", f"v0, a{reg}")] + insts[k + 1:]
    v, _ = check(planted)
    assert any(reg in hit for _, _, hit in v)
    # the same copy behind a wait: clean
    waited = insts[:k + 1] + [(None, "s_waitcnt", "vmcnt(0)"), (None, "v_accvgpr_read_b32", f"v0, a{reg}")] + \
        insts[k + 1:]
    v2, _ = check(waited)
    assert not any("v0, a%d" % reg in ins for _, ins, _ in v2)
    # a use reached only through a branch (the load's block jumps past the
    # next wait in text order): found through the control-flow graph
    lab = "_planted"
    branchy = insts[:k + 1] + [(None, "s_branch", lab), (None, "s_waitcnt", "vmcnt(0)"), (lab, None, ""),
                               (None, "v_mov_b32", f"v1, a{reg}")] + insts[k + 1:]
    v3, _ = check(branchy)
    assert any("v1, a%d" % reg in ins for _, ins, _ in v3)
    # a count-based wait covers the load only with that many vector memory
    # instructions issued after it
    short = insts[:k + 1] + [(None, "global_store_dwordx4", "v0, v[0:3], off"),
                             (None, "s_waitcnt", "vmcnt(2)"), (None, "v_accvgpr_read_b32", f"v0, a{reg}")] + insts[k + 1:]
    v4, _ = check(short)
    assert any("v0, a%d" % reg in ins for _, ins, _ in v4)
    enough = insts[:k + 1] + [(None, "global_store_dwordx4", "v0, v[0:3], off"),
                              (None, "global_store_dwordx4", "v0, v[0:3], off offset:16"),
                              (None, "s_waitcnt", "vmcnt(2)"), (None, "v_accvgpr_read_b32", f"v0, a{reg}")] + \
        insts[k + 1:]
    v5, _ = check(enough)
    assert not any("v0, a%d" % reg in ins for _, ins, _ in v5)


def test_query_fragment_loads_are_waited_for(sdpa_asm):
    violations, n_loads = check(parse(sdpa_asm))
    assert n_loads >= 16, "no asm query-fragment loads found: the check would be vacuous"
    assert not violations, violations[:5]


def test_k_fragment_reads_are_waited_for(sdpa_asm):
    insts = parse(sdpa_asm)
    violations, n_loads = check(insts, LDS_LOAD, r"lgkmcnt\(0\)")
    assert n_loads >= 16, "no asm K-fragment reads found: the check would be vacuous"
    assert not violations, violations[:5]
    # a planted use right after such a read is found
    k = next(i for i, (lab, op, rest) in enumerate(insts) if op and LDS_LOAD.match(op) and rest.startswith("a"))
    reg = min(regs(insts[k][2]))
    planted = insts[:k + 1] + [(None, "v_accvgpr_read_b32", f"v0, a{reg}")] + insts[k + 1:]
    v, _ = check(planted, LDS_LOAD, r"lgkmcnt\(0\)")
    assert any(reg in hit for _, _, hit in v)


M0_WRITE = re.compile(r"^\s*s_\w+\s+m0\b")


def m0_writes(asm_text):
    """Instructions of the kernel that write M0, split into those inside the
    kernel's own inline asm (between ;;#ASMSTART and ;;#ASMEND) and the rest."""
    lines = asm_text.split("\n")
    start = next(i for i, l in enumerate(lines) if l.startswith(KERNEL + ":"))
    inside, outside, in_asm = [], [], False
    for l in lines[start + 1:]:
        if l.startswith(".Lfunc_end"):
            break
        if ";;#ASMSTART" in l:
            in_asm = True
            continue
        if ";;#ASMEND" in l:
            in_asm = False
            continue
        s = l.split(";")[0]
        if M0_WRITE.match(s):
            (inside if in_asm else outside).append(s.strip())
    return inside, outside


def test_m0_written_only_by_the_kernels_asm(sdpa_asm):
    """The kernel's LDS DMA instructions take their LDS address from M0, which
    its own asm sets once per four instructions, the instructions issued one by
    one between score MFMAs.  A compiler-generated M0 write anywhere in the
    kernel could land between such a write and its instructions and send the
    DMA elsewhere in LDS, so there must be none."""
    inside, outside = m0_writes(sdpa_asm)
    assert len(inside) >= 8, "no asm M0 writes found: the check would be vacuous"
    assert not outside, outside[:5]
    # a planted compiler-style write outside the asm is found
    planted = sdpa_asm.replace(";;#ASMSTART", "\ts_mov_b32 m0, -1\n\t;;#ASMSTART", 1)
    _, outside2 = m0_writes(planted)
    assert outside2 == ["s_mov_b32 m0, -1"]


# Wait states a read needs after the write of its register (gfx950), as the
# compiler inserts them for its own instructions: a VALU, memory or MFMA
# source read of a v_mfma_f32_32x32x16_bf16 result 12 (s_nop 11), of a
# v_mfma_f32_16x16x32_bf16 result 8, of a v_mfma_f32_32x32x2_f32 result 18;
# a read of a transcendental result one.
MFMA_READ_WAIT = {"v_mfma_f32_32x32x16_bf16": 12, "v_mfma_f32_16x16x32_bf16": 8, "v_mfma_f32_32x32x2_f32": 18,
                  "v_mfma_f32_16x16x4_f32": 10}
TRANS_READ_WAIT = 1
VREG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
TRANS = re.compile(r"^v_(exp|log|rcp|rsq|sqrt|sin|cos)_f32")


def vregs(operands):
    out = set()
    for m in VREG.finditer(operands):
        if m.group(1):
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


def wait_state_violations(insts):
    """Reads of MFMA or transcendental results with fewer wait states between
    write and read than the hardware needs, on any control-flow path.  The
    compiler inserts these waits for its own instructions but not before an
    inline-asm statement, so asm that reads such results must be preceded by an
    explicit fence.  An MFMA's accumulator operand (src2) is exempt: a chain of
    MFMAs on one accumulator is interlocked."""
    blocks, order, cur, anon = {"entry": []}, ["entry"], "entry", 0
    for lab, op, rest in insts:
        if lab is not None:
            cur = lab
            blocks[cur] = []
            order.append(cur)
            continue
        blocks[cur].append((op, rest))
        if op.startswith("s_branch") or op.startswith("s_cbranch") or op == "s_endpgm":
            anon += 1
            cur = f"anon{anon}"
            blocks[cur] = []
            order.append(cur)
    succ = {}
    for i, b in enumerate(order):
        body, nxt = blocks[b], (order[i + 1] if i + 1 < len(order) else None)
        last = body[-1] if body else None
        s = []
        if last and last[0] == "s_endpgm":
            pass
        elif last and last[0].startswith("s_branch"):
            s.append(last[1].split()[0])
        else:
            if last and last[0].startswith("s_cbranch"):
                s.append(last[1].split()[0])
            if nxt is not None:
                s.append(nxt)
        succ[b] = [x for x in s if x in blocks]

    def step(b, state, record, out):
        state = dict(state)
        for op, rest in blocks[b]:
            ops = [o.strip() for o in rest.split(",")] if rest else []
            if op.startswith("v_") or op.startswith("ds_") or op.startswith("buffer_") or op.startswith("global_"):
                if op.startswith("v_mfma"):
                    srcs = ops[1:3]
                elif op.startswith("ds_write") or op.startswith("buffer_store") or op.startswith("global_store"):
                    srcs = ops
                elif op.startswith("v_"):
                    srcs = ops[1:]
                else:
                    srcs = ops[1:]
                rd = set()
                for o in srcs:
                    rd |= vregs(o)
                hit = {r for r in rd if state.get(r, 0) > 0}
                if hit and record:
                    out.append((b, f"{op} {rest}", sorted(hit)[:4]))
            n = 1
            if op == "s_nop":
                n = int(rest.split()[0], 0) + 1
            state = {r: w - n for r, w in state.items() if w - n > 0}
            # a register another instruction writes no longer holds the result
            if ops and not op.startswith("v_mfma") and (op.startswith("v_") or op.startswith("ds_read")
                                                         or op.startswith("global_load")
                                                         or (op.startswith("buffer_load") and "lds" not in rest)):
                for r in vregs(ops[0]):
                    state.pop(r, None)
            if op.startswith("v_mfma") and ops:
                for r in vregs(ops[0]):
                    state[r] = MFMA_READ_WAIT.get(op, 18)
            elif TRANS.match(op) and ops:
                for r in vregs(ops[0]):
                    state[r] = max(state.get(r, 0), TRANS_READ_WAIT)
        return state

    st_in = {b: {} for b in order}
    changed = True
    while changed:
        changed = False
        for b in order:
            o = step(b, st_in[b], False, None)
            for s in succ[b]:
                m = dict(st_in[s])
                for r, w in o.items():
                    if w > m.get(r, 0):
                        m[r] = w
                if m != st_in[s]:
                    st_in[s] = m
                    changed = True
    out = []
    for b in order:
        step(b, st_in[b], True, out)
    return out


def test_mfma_results_read_after_enough_wait_states(sdpa_asm):
    """Phase B's asm reads the score MFMAs' results (row maxima) and the
    exponentials (row sums); the compiler puts no wait states before asm, so
    the kernel fences them itself.  Every read of an MFMA or transcendental
    result in the kernel, compiler-generated or asm, must have its wait
    states on every path."""
    insts = parse(sdpa_asm)
    assert sum(1 for _, op, _ in insts if op and op.startswith("v_mfma")) >= 64
    v = wait_state_violations(insts)
    assert not v, v[:5]
    # a planted asm-style read right after an MFMA is found, and one behind
    # s_nop 11 is not
    k = next(i for i, (lab, op, rest) in enumerate(insts) if op and op.startswith("v_mfma") and rest.startswith("v["))
    dst = insts[k][2].split(",")[0].strip()
    first = dst[2:].split(":")[0]
    planted = insts[:k + 1] + [(None, "v_max3_f32", f"v255, v255, v{first}, v{first}")] + insts[k + 1:]
    assert any(("v", int(first)) in hit for _, _, hit in wait_state_violations(planted))
    fenced = insts[:k + 1] + [(None, "s_nop", "11"), (None, "v_max3_f32", f"v255, v255, v{first}, v{first}")] + \
        insts[k + 1:]
    assert not any("v255, v255" in ins for _, ins, _ in wait_state_violations(fenced))


@pytest.mark.parametrize("src", ["awa_sdpa_f32", "dit_gemm"])
def test_other_mfma_kernels_wait_states(tmp_path, src):
    """The same wait-state check over the library's other MFMA kernels (the
    fp32 attention kernel and every GEMM instantiation), whose epilogues read
    accumulators after asm fences."""
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not present")
    r = subprocess.run(["make", "-n", "-B", "-C", PKG, f"_build/{src}.o"], capture_output=True, text=True, timeout=60)
    line = next(l for l in r.stdout.split("\n") if f"{src}.hip" in l and "hipcc" in l)
    flags = [t for t in shlex.split(line.split(" -c ")[0])[1:] if t != "-fPIC"]
    out = tmp_path / f"{src}.s"
    r = subprocess.run([HIPCC] + flags + ["--cuda-device-only", "-S", os.path.join(PKG, "csrc", f"{src}.hip"), "-o",
                                          str(out)], cwd=PKG, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    text = open(out).read()
    kernels = re.findall(r"^(_Z\S+):", text, re.M)
    assert kernels
    global KERNEL
    saved, n_mfma = KERNEL, 0
    try:
        for k in kernels:
            KERNEL = k
            insts = parse(text)
            n_mfma += sum(1 for _, op, _ in insts if op and op.startswith("v_mfma"))
            v = wait_state_violations(insts)
            assert not v, (k, v[:5])
    finally:
        KERNEL = saved
    assert n_mfma >= 64

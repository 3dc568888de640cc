#!/usr/bin/env python3
"""Benchmark: the SeedVR2 AWA layer at the 1080p shape, bf16, one MI355X.

A step is one AWA layer forward (qk-norm + RoPE + window partition, window
attention, cross-window text average) on resident inputs: vqkv [5440, 7680]
and tqkv [58, 7680] bf16 for the 1x68x80 token grid, 20 heads x 128, 58 text
tokens, num_windows (4,3,3).  Steps alternate the unshifted (16 windows) and
shifted (25 windows) geometry, as even and odd DiT layers do; geometry is
built once per resolution before timing, as the reference caches it.

Prints one JSON line.  `value` is ms per AWA layer (wall clock over the
timed steps, captured as one HIP graph of that many layers as the DiT
forward captures its layers, bracketed by device synchronisation; the
eager and graph-per-layer figures are reported beside it).  `roofline` covers the
dominant kernel (window attention): HIP events on its stream around
back-to-back launches of it on the same inputs, per geometry, mixed as in the
timed steps (the per-phase events of the timed steps, which add a launch gap
to every phase, give `frac_by_phase_events`).  `cpu_baseline` times the oracle's single-threaded
restatement of the reference CPU attention (dit_vk.cpp:345-462) on one full
unshifted 1080p layer.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "seedvr2-2b-ncnn_amd"))

METRIC = "1080p bf16 AWA-layer ms & MFMA util; 32-layer DiT step sec; 1 GPU"
GRID, NUM_WINDOWS, TXT, SEED = (1, 68, 80), (4, 3, 3), 58, 2
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
# HBM bytes per launch measured with rocprofv3 PMC counters (FETCH_SIZE, WRITE_SIZE,
# calibrated against a plain copy); the counters need a profiler run of their own.
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic.json")


def measured_traffic():
    try:
        with open(TRAFFIC_JSON) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA
# The other workloads of the op, timed beside the headline one:
#   name: grid, num_windows, txt, shifted, storage, seed, outlier fraction
CONFIGS = {
    "cfg0_360p_fp32": ((1, 23, 27), (4, 3, 3), 58, 0, "f32", 0, 0.0),
    "cfg1_720p_bf16": ((1, 45, 53), (4, 3, 3), 58, 1, "bf16", 1, 0.0),
    "cfg4_ragged_bf16": ((1, 71, 97), (1, 4, 4), 77, 1, "bf16", 4, 0.01),
}


def sdpa_flops(S_list):
    # QK^T + PV over each window's S = f + TXT rows, 20 heads x 128
    return sum(4.0 * 128 * 20 * s * s for s in S_list)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(vq_bf16_f32, tq_bf16_f32, gains):
    """Single-threaded oracle (bit-exact restatement of the reference CPU AWA)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    g = O.Geometry(*GRID, NUM_WINDOWS, TXT, 0)
    t0 = time.perf_counter()
    O.awa_forward(vq_bf16_f32, tq_bf16_f32, g, *gains, eps=1e-5, nthreads=1)
    dt = time.perf_counter() - t0
    # the same restatement parallel over (window, head) on the host cores
    # (at most 16 threads: the host cores a single GPU's job gets)
    nt = max(1, min(16, os.cpu_count() or 1))
    t0 = time.perf_counter()
    O.awa_forward(vq_bf16_f32, tq_bf16_f32, g, *gains, eps=1e-5, nthreads=nt)
    dt_omp = time.perf_counter() - t0
    return {"value": round(dt * 1e3, 1), "unit": "ms per AWA layer", "cores": 1, "kind": "port",
            "sample": "one full 1080p unshifted AWA layer (16 windows, fp32 CPU attention of "
                      "dit_vk.cpp:345-462 via the bit-exact oracle), single thread",
            "cpu": cpu_model(), "nproc": os.cpu_count(),
            "omp_all_cores": {"value": round(dt_omp * 1e3, 1), "unit": "ms per AWA layer", "threads": nt,
                              "note": "same layer, OpenMP over (window, head)"},
            "dit_step_extrapolated": cpu_step_extrapolated(O, vq_bf16_f32, tq_bf16_f32, gains, nt)}


def config_runs(ctx, torch, steps, cpu=True):
    """Each extra workload: ms per AWA layer (eager launches, wall clock), the
    attention kernel's MFMA fraction (fp32 peak for fp32 storage), the pack
    and text-average passes against HBM, and the oracle's CPU attention on
    the same layer (1 thread and all host cores, up to 16)."""
    import numpy as np
    res = {}
    dev = torch.device("cuda:0")
    for name, (grid, nw, txt, sh, store, seed, frac) in CONFIGS.items():
        rng = np.random.default_rng(seed)
        Lv = grid[0] * grid[1] * grid[2]
        vqn = rng.standard_normal((Lv, 7680), dtype=np.float32)
        tqn = rng.standard_normal((txt, 7680), dtype=np.float32)
        if frac > 0:
            for a in (vqn, tqn):
                a[rng.random(a.shape) < frac] *= 8.0
        gains_np = [(1.0 + 0.02 * rng.standard_normal(128)).astype(np.float32) for _ in range(4)]
        dt = torch.float32 if store == "f32" else torch.bfloat16
        vq = torch.from_numpy(vqn).to(dev, dt)
        tq = torch.from_numpy(tqn).to(dev, dt)
        gains = [torch.from_numpy(g).to(dev) for g in gains_np]
        va = torch.empty((Lv, 2560), dtype=dt, device=dev)
        ta = torch.empty((txt, 2560), dtype=dt, device=dev)
        g = ctx.build_geometry(*grid, nw, txt, sh)
        d = g.read()
        S = [int(c1 - c0) + txt for c0, c1 in zip(d["cumf"][:-1], d["cumf"][1:])]
        fl = sdpa_flops(S)
        for _ in range(3):
            ctx.forward(g, vq, tq, *gains, eps=1e-5, vattn=va, tattn=ta)
        torch.cuda.synchronize()
        # wall clock with per-phase events off, then the phases in a pass of
        # their own (the events add work to every call)
        t0 = time.perf_counter()
        for _ in range(steps):
            ctx.forward(g, vq, tq, *gains, eps=1e-5, vattn=va, tattn=ta)
        torch.cuda.synchronize()
        layer_ms = (time.perf_counter() - t0) * 1e3 / steps
        ctx.timing(True)
        ctx.timing_read()
        for _ in range(steps):
            ctx.forward(g, vq, tq, *gains, eps=1e-5, vattn=va, tattn=ta)
        torch.cuda.synchronize()
        mp, ma, mt, c = ctx.timing_read()
        ctx.timing(False)
        es = 4 if store == "f32" else 2
        peak = PEAK_FP32_TFLOPS if store == "f32" else PEAK_BF16_TFLOPS
        attn_s = ma * 1e-3 / c
        # the kernels' own times: back-to-back launches between two events
        pk_k, attn_k, tx_k = (x * 1e-3 for x in ctx.time_phases(g, vq, tq, *gains, reps=max(4, steps), eps=1e-5,
                                                                  vattn=va, tattn=ta))
        tfl = fl / attn_k / 1e12
        qk_bytes = 2 * (Lv + txt) * 2 * 2560 * es
        co_bytes = (g.info()["nwin"] + 1) * txt * 2560 * 4
        r = {"grid": list(grid), "num_windows": list(nw), "txt_len": txt, "shifted": bool(sh),
             "storage": store, "nwin": g.info()["nwin"], "ms_per_layer": round(layer_ms, 4),
             "phases_us": {"pack": round(pk_k * 1e6, 2), "attention": round(attn_k * 1e6, 2),
                           "text_average": round(tx_k * 1e6, 2)},
             "phases_us_by_events": {"pack": round(mp * 1e3 / c, 2), "attention": round(attn_s * 1e6, 2),
                                     "text_average": round(mt * 1e3 / c, 2)},
             "attention_roofline": {"bound": "mfma", "achieved": round(tfl, 1), "peak": peak,
                                    "unit": "TFLOP/s", "frac": round(tfl / peak, 4),
                                    "avg_launch_us": round(attn_k * 1e6, 2),
                                    "frac_by_phase_events": round(fl / attn_s / 1e12 / peak, 4),
                                    "gflop_per_launch": round(fl / 1e9, 3)},
             "hbm_qknorm_rope_frac": round(qk_bytes / pk_k / 1e9 / PEAK_HBM_GBS, 4),
             "hbm_text_average_frac": round(co_bytes / tx_k / 1e9 / PEAK_HBM_GBS, 4)}
        if cpu:
            sys.path.insert(0, os.path.join(ROOT, "oracle"))
            import oracle as O
            og = O.Geometry(*grid, nw, txt, sh)
            vqf, tqf = vq.float().cpu().numpy(), tq.float().cpu().numpy()
            nt = max(1, min(16, os.cpu_count() or 1))
            t0 = time.perf_counter()
            O.awa_forward(vqf, tqf, og, *gains_np, eps=1e-5, nthreads=1)
            t1 = time.perf_counter()
            O.awa_forward(vqf, tqf, og, *gains_np, eps=1e-5, nthreads=nt)
            t2 = time.perf_counter()
            r["cpu_baseline"] = {"value": round((t1 - t0) * 1e3, 1), "unit": "ms per AWA layer",
                                 "cores": 1, "kind": "port",
                                 "omp_all_cores": {"value": round((t2 - t1) * 1e3, 1), "threads": nt}}
        g.close()
        res[name] = r
    return res


def cpu_step_extrapolated(O, vq, tq, gains, nt, rows=256, mlp=6912):
    """CPU 32-layer step, extrapolated: the oracle's fp32 GEMMs of one layer
    (qkv 2560->7680, out 2560->2560, MLP in and gate 2560->6912, MLP out
    6912->2560) timed on `rows` token rows and scaled to Lv + TXT rows (GEMM
    time is linear in the rows), plus the oracle AWA of an even (unshifted) and
    an odd (shifted) layer in full, on nt threads; x16 layer pairs.  The
    reference's own CPU step used ncnn GEMMs, which are not available here."""
    import numpy as np
    rng = np.random.default_rng(3)
    x = rng.standard_normal((rows, 2560), dtype=np.float32)
    h = rng.standard_normal((rows, mlp), dtype=np.float32)
    shapes = [(7680, 2560, x), (2560, 2560, x), (mlp, 2560, x), (mlp, 2560, x), (2560, mlp, h)]
    t_gemm = 0.0
    for n_out, n_in, a in shapes:
        W = (0.02 * rng.standard_normal((n_out, n_in), dtype=np.float32))
        t0 = time.perf_counter()
        O.linear(a, W, nthreads=nt)
        t_gemm += time.perf_counter() - t0
    M = GRID[0] * GRID[1] * GRID[2] + TXT
    t_gemm_layer = t_gemm * M / rows
    t_awa = 0.0
    for sh in (0, 1):
        g = O.Geometry(*GRID, NUM_WINDOWS, TXT, sh)
        t0 = time.perf_counter()
        O.awa_forward(vq, tq, g, *gains, eps=1e-5, nthreads=nt)
        t_awa += time.perf_counter() - t0
    step = 16 * (2 * t_gemm_layer + t_awa)
    return {"value": round(step, 1), "unit": "s per 32-layer DiT step (extrapolated)", "threads": nt,
            "sample": f"GEMMs of one layer on {rows} of {M} rows scaled by rows, AWA of one even and one "
                      "odd layer in full, x16; elementwise work not counted",
            "reference_published_cpu_dit_s": 358.96}


def dit_step(ctx, awa_hip, torch, steps, warmup, mlp=6912, graph=True):
    """32-layer DiT step at 1080p: time embedding (t=1000) + 32 layers, layers
    0-9 with separate video/text branches, 10-31 shared, even layers unshifted,
    odd shifted; weights N(0, 0.02) bf16 resident in HBM (42 branches)."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    Lv = GRID[0] * GRID[1] * GRID[2]

    def rnd(*shape, dtype=torch.bfloat16, scale=0.02):
        return (scale * torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)).to(dtype)

    def branch():
        b = {"qkv_w": rnd(7680, 2560), "out_w": rnd(2560, 2560), "out_b": rnd(2560, dtype=torch.float32),
             "mlp_out_w": rnd(2560, mlp)}
        b["mlp_w"] = ctx.pack_mlp(rnd(mlp, 2560), rnd(mlp, 2560))
        b["nq"] = 1 + rnd(128, dtype=torch.float32)
        b["nk"] = 1 + rnd(128, dtype=torch.float32)
        for k in ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate"):
            b[k] = rnd(2560, dtype=torch.float32)
        return b

    layers = []
    for i in range(32):
        vb = branch()
        layers.append((vb, branch() if i < 10 else vb))
    temb = [rnd(2560, 256, dtype=torch.float32), rnd(2560, dtype=torch.float32),
            rnd(2560, 2560, dtype=torch.float32), rnd(2560, dtype=torch.float32),
            rnd(15360, 2560, dtype=torch.float32), rnd(15360, dtype=torch.float32)]
    geoms = [ctx.build_geometry(*GRID, NUM_WINDOWS, TXT, sh) for sh in (0, 1)]
    x0 = torch.randn((Lv + TXT, 2560), generator=gen, device=dev, dtype=torch.float32)
    x = torch.empty_like(x0)

    def one_step():
        x.copy_(x0)
        emb = ctx.time_embedding(1000.0, *temb)
        for i, (vb, tb) in enumerate(layers):
            ctx.layer(geoms[i % 2], vb, tb, emb, x, Lv, TXT, mlp=mlp, txt_vid_only=False)

    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize()
    # wall clock with the per-phase events off, then the phase breakdown in a
    # pass of its own (the events add work to every phase)
    t0 = time.perf_counter()
    for _ in range(steps):
        one_step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    assert bool(torch.isfinite(x).all()), "non-finite hidden state"
    step_s = (t1 - t0) / steps
    ctx.timing(True)
    ctx.dit_timing_read()
    ctx.timing_read()
    t2 = time.perf_counter()
    for _ in range(steps):
        one_step()
    torch.cuda.synchronize()
    step_s_events = (time.perf_counter() - t2) / steps
    ms_gemm, ms_awa, ms_elt, nl = ctx.dit_timing_read()
    ctx.timing_read()
    ctx.timing(False)

    M = Lv + TXT
    gemm_flops = 32 * 2 * M * 2560 * (7680 + 2560 + 3 * mlp)
    res = {"value": round(step_s, 5), "unit": "s per 32-layer DiT step", "steps": steps,
           "timing": "eager launches, wall clock with the per-phase events off; per_step_ms from a "
                     "second pass with the events on (value_with_events)",
           "value_with_events": round(step_s_events, 5),
           "awa_ms_per_layer_in_step": round(ms_awa / steps / 32, 4),
           "warmup": warmup, "mlp": mlp,
           "txt_semantics": "text rows processed on every layer (merged-graph order)",
           "per_step_ms": {"gemm": round(ms_gemm / steps, 3), "awa": round(ms_awa / steps, 3),
                           "norm_ada_eltwise": round(ms_elt / steps, 3)},
           "gemm_tflops": round(gemm_flops / (ms_gemm / steps * 1e-3) / 1e12, 1),
           "gemm_frac_of_bf16_peak": round(gemm_flops / (ms_gemm / steps * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
           "layers_timed": nl}
    if not graph:
        for g in geoms:
            g.close()
        return res

    # the same step captured as one HIP graph (the launches above, recorded on a
    # side stream) and replayed; each step starts from x0, so a replay must equal
    # the eager result bit for bit
    x_eager = x.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        one_step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g_step = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_step, stream=side):
        one_step()
    x.zero_()
    torch.cuda.synchronize()
    g_step.replay()
    torch.cuda.synchronize()
    assert torch.equal(x, x_eager), "graph replay differs from the eager step"
    t0 = time.perf_counter()
    for _ in range(steps):
        g_step.replay()
    torch.cuda.synchronize()
    graph_s = (time.perf_counter() - t0) / steps
    del g_step
    for g in geoms:
        g.close()
    res["graph_replay_s"] = round(graph_s, 5)
    return res


def copy_ceiling(ctx, torch, nbytes, reps=20):
    """The HBM rate a device copy reaches on the same byte count as a
    memory-bound pass (read nbytes, write nbytes; the source re-read each
    time, as the layer's inputs are): the library's streaming copy and
    torch's copy_ (its vectorised elementwise kernel), HIP events around reps
    back-to-back launches each; the faster one is the ceiling."""
    n = nbytes // 16 * 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    us_ours = timed(lambda: ctx.stream_copy(src, dst))
    us_torch = timed(lambda: dst.copy_(src))
    us = min(us_ours, us_torch)
    gbs = 2 * n * 4 / (us * 1e-6) / 1e9
    return {"bytes_read_plus_write": 2 * n * 4, "us": round(us, 2), "GBs": round(gbs, 1),
            "frac": round(gbs / PEAK_HBM_GBS, 4),
            "kernel": "stream_copy_kernel" if us_ours <= us_torch else "torch copy_",
            "stream_copy_us": round(us_ours, 2), "torch_copy_us": round(us_torch, 2),
            "timing": "HIP events, back to back; the faster of the two copies"}


def gemm_shapes(awa_hip, torch, steps, warmup):
    """The block's GEMM kernel (plain bf16 store) against hipBLASLt (torch.mm)
    on the projection shapes of a 1080p layer: M = 5440 + 58 rows; QKV, out,
    MLP in + gate (fused width 2 x 6912) and MLP out."""
    ctx = awa_hip.Context(0)
    dev = torch.device("cuda:0")
    M = GRID[0] * GRID[1] * GRID[2] + TXT
    res = {}
    for name, N, K in (("qkv", 7680, 2560), ("out", 2560, 2560), ("mlp_in", 13824, 2560),
                       ("mlp_out", 2560, 6912)):
        g = torch.Generator(device=dev).manual_seed(N + K)
        A = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
        W = (0.02 * torch.randn((N, K), generator=g, device=dev)).to(torch.bfloat16)
        C = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
        entry = {"M": M, "N": N, "K": K}
        fns = (("ours", lambda: ctx.gemm(A, W, out=C)), ("hipblaslt", lambda: torch.mm(A, W.t(), out=C)))
        best = {who: float("inf") for who, _ in fns}
        for _, fn in fns:
            for _ in range(warmup):
                fn()
        # alternating rounds, best round each: neither side pays the clock ramp
        for _ in range(3):
            for who, fn in fns:
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(steps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                best[who] = min(best[who], e0.elapsed_time(e1) * 1e3 / steps)
        for who, us in best.items():
            entry[who] = {"us": round(us, 1), "tflops": round(2.0 * M * N * K / us / 1e6, 1)}
        res[name] = entry
    ctx.close()
    return {"gemm_shapes": res, "unit": "us per GEMM (HIP events, back-to-back launches, best of 3 alternating rounds)"}


def torch_attention(awa_hip, torch, steps, warmup):
    """PyTorch's fused attention (its flash and memory-efficient backends; the
    math backend is never used) on exactly the windows of the 1080p layers:
    every window's S = f + TXT rows attend among themselves, 20 heads of 128,
    bf16, windows of equal S batched into one call; the same flops as the
    attention kernel, which is timed beside it (awa_time_phases, back to back)."""
    import numpy as np
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    ctx = awa_hip.Context(0)
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(SEED)
    Lv = GRID[0] * GRID[1] * GRID[2]
    vq = torch.from_numpy(rng.standard_normal((Lv, 7680), dtype=np.float32)).to(dev, torch.bfloat16)
    tq = torch.from_numpy(rng.standard_normal((TXT, 7680), dtype=np.float32)).to(dev, torch.bfloat16)
    gains = [torch.from_numpy((1.0 + 0.02 * rng.standard_normal(128)).astype(np.float32)).to(dev)
             for _ in range(4)]
    res = {}
    for sh in (0, 1):
        g = ctx.build_geometry(*GRID, NUM_WINDOWS, TXT, sh)
        d = g.read()
        S = [int(c1 - c0) + TXT for c0, c1 in zip(d["cumf"][:-1], d["cumf"][1:])]
        fl = sdpa_flops(S)
        groups = {}
        for s in S:
            groups[s] = groups.get(s, 0) + 1
        gen = torch.Generator(device=dev).manual_seed(sh)
        ops = [[torch.randn((cnt, 20, s, 128), generator=gen, device=dev).to(torch.bfloat16) for _ in range(3)]
               for s, cnt in sorted(groups.items())]
        entry = {"windows": len(S), "window_rows": sorted(groups.items()), "gflop": round(fl / 1e9, 3)}
        _, attn_ms, _ = ctx.time_phases(g, vq, tq, *gains, reps=steps, eps=1e-5)
        entry["ours"] = {"us": round(attn_ms * 1e3, 2), "tflops": round(fl / (attn_ms * 1e-3) / 1e12, 1)}
        for name, be in (("torch_flash", SDPBackend.FLASH_ATTENTION),
                         ("torch_efficient", SDPBackend.EFFICIENT_ATTENTION)):
            try:
                with sdpa_kernel([be]):
                    def run():
                        for q, k, v in ops:
                            F.scaled_dot_product_attention(q, k, v)
                    for _ in range(warmup):
                        run()
                    best = float("inf")
                    for _ in range(3):
                        torch.cuda.synchronize()
                        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        e0.record()
                        for _ in range(steps):
                            run()
                        e1.record()
                        torch.cuda.synchronize()
                        best = min(best, e0.elapsed_time(e1) * 1e3 / steps)
                entry[name] = {"us": round(best, 2), "tflops": round(fl / (best * 1e-6) / 1e12, 1)}
            except RuntimeError as ex:  # backend not built for this device
                entry[name] = {"unavailable": str(ex)[:160]}
        res["shifted" if sh else "unshifted"] = entry
        g.close()
    # the same backends on uniform batches (batch, 20 heads, S rows, 128)
    uni = {}
    for B, S in ((16, 398), (25, 264), (4, 2048)):
        gen = torch.Generator(device=dev).manual_seed(S)
        q, k, v = (torch.randn((B, 20, S, 128), generator=gen, device=dev).to(torch.bfloat16) for _ in range(3))
        fl = 4.0 * B * 20 * S * S * 128
        for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
            try:
                with sdpa_kernel([be]):
                    for _ in range(warmup):
                        F.scaled_dot_product_attention(q, k, v)
                    torch.cuda.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(steps):
                        F.scaled_dot_product_attention(q, k, v)
                    e1.record()
                    torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / steps
                uni[f"B{B}_S{S}_{name}"] = {"us": round(us, 1), "tflops": round(fl / (us * 1e-6) / 1e12, 1)}
            except RuntimeError as ex:
                uni[f"B{B}_S{S}_{name}"] = {"unavailable": str(ex)[:160]}
    res["uniform_batches"] = uni
    ctx.close()
    return {"torch_attention": res,
            "unit": "us per layer's attention (all windows, 20 heads), HIP events over back-to-back launches, "
                    "torch: best of 3 rounds, one call per group of equal-length windows"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dit", action="store_true", help="skip the 32-layer DiT step")
    ap.add_argument("--dit-steps", type=int, default=5)
    ap.add_argument("--no-configs", action="store_true", help="skip the 360p fp32, 720p and ragged workloads")
    ap.add_argument("--no-mlp10240", action="store_true", help="skip the MLP-10240 DiT step variant")
    ap.add_argument("--gemm-shapes", action="store_true",
                    help="only time the DiT block's GEMM kernel and hipBLASLt (torch.mm) on the four "
                         "1080p projection shapes (bf16 in and out), print one JSON line and exit")
    ap.add_argument("--torch-attention", action="store_true",
                    help="only time PyTorch's fused attention (flash / memory-efficient backends) on the "
                         "1080p layers' windows beside the attention kernel, print one JSON line and exit")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                    help="only run the library's streaming device copy of MB MiB (14 times) to "
                         "calibrate the FETCH_SIZE/WRITE_SIZE counters, then exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the AWA path is single-GPU here (no sharding, no "
              "collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import awa_hip

    if args.calibrate_copy:
        ctx = awa_hip.Context(0)
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(4):
            ctx.stream_copy(src, dst)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(10):
            ctx.stream_copy(src, dst)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / 10
        ctx.close()
        print(json.dumps({"calibration_copy_bytes": n * 4, "launches": 14, "kernel": "stream_copy_kernel",
                          "copy_GBs_read_plus_write": round(2 * n * 4 / dt / 1e9, 1)}))
        return

    if args.gemm_shapes:
        print(json.dumps(gemm_shapes(awa_hip, torch, args.steps, args.warmup)))
        return

    if args.torch_attention:
        print(json.dumps(torch_attention(awa_hip, torch, args.steps, args.warmup)))
        return

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(SEED)
    Lv = GRID[0] * GRID[1] * GRID[2]
    vq = torch.from_numpy(rng.standard_normal((Lv, 7680), dtype=np.float32)).to(dev, torch.bfloat16)
    tq = torch.from_numpy(rng.standard_normal((TXT, 7680), dtype=np.float32)).to(dev, torch.bfloat16)
    gains_np = [(1.0 + 0.02 * rng.standard_normal(128)).astype(np.float32) for _ in range(4)]
    gains = [torch.from_numpy(g).to(dev) for g in gains_np]
    vattn = torch.empty((Lv, 2560), dtype=torch.bfloat16, device=dev)
    tattn = torch.empty((TXT, 2560), dtype=torch.bfloat16, device=dev)

    ctx = awa_hip.Context(0)
    geom_ms = []
    geoms = []
    for sh in (0, 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        geoms.append(ctx.build_geometry(*GRID, NUM_WINDOWS, TXT, sh))
        torch.cuda.synchronize()
        geom_ms.append((time.perf_counter() - t0) * 1e3)
    infos = [g.info() for g in geoms]
    S_lists = []
    for g in geoms:
        d = g.read()
        S_lists.append([int(c1 - c0) + TXT for c0, c1 in zip(d["cumf"][:-1], d["cumf"][1:])])
    flops = [sdpa_flops(S) for S in S_lists]

    def step(k):
        ctx.forward(geoms[k % 2], vq, tq, *gains, eps=1e-5, vattn=vattn, tattn=tattn)

    for k in range(args.warmup):
        step(k)
    torch.cuda.synchronize()
    # eager wall clock with the per-phase events off, then the per-phase
    # events in a pass of their own (the events add work to every phase)
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(k)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_eager = (t1 - t0) * 1e3 / args.steps
    ctx.timing(True)
    ctx.timing_read()  # clear
    torch.cuda.synchronize()
    for k in range(args.steps):
        step(k)
    torch.cuda.synchronize()
    ms_pack, ms_attn, ms_text, calls = ctx.timing_read()
    ctx.timing(False)
    assert calls == args.steps

    # The same layers replayed from HIP graphs (one per geometry, replayed
    # alternately), as they run inside the captured DiT forward: no launch
    # gaps between the kernels.  The replays must reproduce the eager outputs
    # bit for bit.
    outs_eager = []
    for k in range(2):
        step(k)
        torch.cuda.synchronize()
        outs_eager.append((vattn.clone(), tattn.clone()))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(0)
        step(1)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graphs = []
    for k in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            step(k)
        graphs.append(g)
    for k in range(2):
        vattn.zero_()
        tattn.zero_()
        torch.cuda.synchronize()
        graphs[k].replay()
        torch.cuda.synchronize()
        assert torch.equal(vattn, outs_eager[k][0]) and torch.equal(tattn, outs_eager[k][1]), \
            "graph replay differs from eager"
    for k in range(args.warmup):
        graphs[k % 2].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        graphs[k % 2].replay()
    torch.cuda.synchronize()
    ms_step_1 = (time.perf_counter() - t0) * 1e3 / args.steps
    del graphs
    # The timed steps as one graph of `steps` layers (geometries alternating), the
    # form the layers take inside the captured DiT forward: one graph launch for
    # the stack, where a graph per layer adds the launch gap between replays
    # (about 8 us, measured in the kernel trace) to every layer.  Its first replay
    # must reproduce the eager outputs of the last step bit for bit.
    g_stack = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_stack, stream=side):
        for k in range(args.steps):
            step(k)
    vattn.zero_()
    tattn.zero_()
    torch.cuda.synchronize()
    g_stack.replay()
    torch.cuda.synchronize()
    last = (args.steps - 1) % 2
    assert torch.equal(vattn, outs_eager[last][0]) and torch.equal(tattn, outs_eager[last][1]), \
        "stacked graph replay differs from eager"
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g_stack.replay()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    del g_stack

    # per-variant breakdown (separate short runs, events only)
    per_variant = {}
    for sh, name in ((0, "unshifted"), (1, "shifted")):
        ctx.timing(True)
        ctx.timing_read()
        n = max(4, args.steps // 2)
        torch.cuda.synchronize()
        a = time.perf_counter()
        for _ in range(n):
            ctx.forward(geoms[sh], vq, tq, *gains, eps=1e-5, vattn=vattn, tattn=tattn)
        torch.cuda.synchronize()
        b = time.perf_counter()
        p, s_, t_, c = ctx.timing_read()
        ctx.timing(False)
        per_variant[name] = {"layer_ms": round((b - a) * 1e3 / n, 4), "pack_us": round(p / c * 1e3, 2),
                             "attn_us": round(s_ / c * 1e3, 2), "text_avg_us": round(t_ / c * 1e3, 2),
                             "attn_tflops": round(flops[sh] / (s_ / c * 1e-3) / 1e12, 1),
                             "nwin": infos[sh]["nwin"]}

    # roofline of the dominant kernel (window attention) over the timed steps
    n_unsh = (args.steps + 1) // 2
    n_sh = args.steps // 2
    flops_timed = n_unsh * flops[0] + n_sh * flops[1]
    attn_evt_s = ms_attn * 1e-3 / calls  # per-phase events: the launch gap after each event included
    # the kernels' own times: HIP events around `steps` back-to-back launches of
    # each kernel per geometry on its stream (awa_time_phases), the timed mix of
    # the two geometries
    reps = max(4, args.steps)
    t_ph = [ctx.time_phases(geoms[k], vq, tq, *gains, reps=reps, eps=1e-5, vattn=vattn, tattn=tattn)
            for k in range(2)]
    mix = lambda i: (n_unsh * t_ph[0][i] + n_sh * t_ph[1][i]) * 1e-3 / args.steps
    attn_avg_s = mix(1)
    achieved = flops_timed / calls / attn_avg_s / 1e12
    # memory-bound pass: qk-norm + RoPE, algorithmic bytes = read + write q and k
    qk_bytes = 2 * (Lv + TXT) * 2 * 2560 * 2
    pack_avg_s = mix(0)
    traffic = measured_traffic()
    sdpa_bytes = traffic.get("sdpa_bf16_kernel", {}).get("total_bytes")
    pack_bytes = traffic.get("pack_bf16_kernel", {}).get("total_bytes")

    out = {
        "metric": METRIC,
        "value": round(ms_step, 4),
        "unit": "ms per AWA layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (q/k/v ~ N(0,1), gains 1+N(0,0.02), seed 2)",
        "timing": "the timed steps captured as one HIP graph of `steps` layers, the two geometries "
                  "alternating (the form the layers take inside the captured DiT forward), replayed "
                  "once; one graph per layer replayed alternately: graph_per_layer_ms (adds the "
                  "launch gap between graph replays to each layer); eager launches (per-phase events "
                  "off): eager_ms_per_layer",
        "graph_per_layer_ms": round(ms_step_1, 4),
        "eager_ms_per_layer": round(ms_eager, 4),
        "geometry_build_ms": {"unshifted": round(geom_ms[0], 3), "shifted": round(geom_ms[1], 3),
                              "note": "once per resolution (host planner + geom_build_kernel), "
                                      "not in value: layers reuse it"},
        "config": {"workload": "awa_layer_1080p_bf16", "grid": list(GRID), "txt_len": TXT,
                   "heads": 20, "head_dim": 128, "num_windows": list(NUM_WINDOWS),
                   "steps_alternate": "unshifted (16 windows) / shifted (25 windows)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": sdpa_bytes, "traffic_unit": "bytes per launch (rocprofv3 PMC)",
                     "kernel": "sdpa_bf16_kernel",
                     "avg_launch_us": round(attn_avg_s * 1e6, 2),
                     "timing": "HIP events around back-to-back launches of the attention kernel on its "
                               "stream, per geometry, mixed as in the timed steps (awa_time_phases)",
                     "frac_by_phase_events": round(flops_timed / calls / attn_evt_s / 1e12 / PEAK_BF16_TFLOPS, 4),
                     "algorithmic_gflop_per_launch": round(flops_timed / calls / 1e9, 3)},
        "phases_us": {"pack_qknorm_rope": round(pack_avg_s * 1e6, 2),
                      "attention": round(attn_avg_s * 1e6, 2),
                      "text_average": round(mix(2) * 1e6, 2),
                      "timing": "each kernel back to back between two events (awa_time_phases)"},
        "phases_us_by_events": {"pack_qknorm_rope": round(ms_pack * 1e3 / calls, 2),
                                "attention": round(attn_evt_s * 1e6, 2),
                                "text_average": round(ms_text * 1e3 / calls, 2),
                                "timing": "per-phase events of the timed eager steps (launch gaps included)"},
        "hbm_qknorm_rope": {"algorithmic_bytes": qk_bytes,
                            "achieved_GBs": round(qk_bytes / pack_avg_s / 1e9, 1),
                            "frac": round(qk_bytes / pack_avg_s / 1e9 / PEAK_HBM_GBS, 4),
                            "measured_bytes": pack_bytes,
                            "measured_GBs": round(pack_bytes / pack_avg_s / 1e9, 1) if pack_bytes else None},
        "per_variant": per_variant,
    }
    # the ceiling: a hand-written streaming copy of the same bytes as the pass
    ceil = copy_ceiling(ctx, torch, qk_bytes // 2)
    out["hbm_qknorm_rope"]["copy_ceiling"] = ceil
    out["hbm_qknorm_rope"]["frac_of_copy"] = round(qk_bytes / pack_avg_s / 1e9 / ceil["GBs"], 4)
    # the text average against HBM: (nwin + 1) TXT 2560 fp32 bytes per launch
    co_bytes = [(infos[k]["nwin"] + 1) * TXT * 2560 * 4 for k in range(2)]
    text_avg_s = mix(2)
    co_mix = (n_unsh * co_bytes[0] + n_sh * co_bytes[1]) / calls
    out["hbm_text_average"] = {"algorithmic_bytes": round(co_mix),
                               "achieved_GBs": round(co_mix / text_avg_s / 1e9, 1),
                               "frac": round(co_mix / text_avg_s / 1e9 / PEAK_HBM_GBS, 4),
                               "note": "back-to-back repeats re-read the partials from the L2 caches (an upper "
                                       "bound); inside the layer they come from the attention kernel's writes",
                               "frac_by_phase_events": round(co_mix / (ms_text * 1e-3 / calls) / 1e9
                                                             / PEAK_HBM_GBS, 4)}
    if not args.no_configs:
        out["configs"] = config_runs(ctx, torch, max(4, args.steps // 2), cpu=not args.no_cpu_baseline)
    if not args.no_dit:
        out["dit_step"] = dit_step(ctx, awa_hip, torch, args.dit_steps, 1)
        # the AWA layer inside the step: inputs written by the QKV GEMM just before,
        # outputs read by the out projection (the headline value replays one layer on
        # resident inputs, whose ~225 MB working set stays in the 256 MB Infinity Cache)
        out["awa_ms_per_layer_in_dit_step"] = out["dit_step"]["awa_ms_per_layer_in_step"]
        if not args.no_mlp10240:
            out["dit_step_mlp10240"] = dit_step(ctx, awa_hip, torch, max(2, args.dit_steps // 2), 1, mlp=10240,
                                                graph=False)
            out["dit_step_mlp10240"]["label"] = ("the DiT-step workload with the MLP written as 2560->10240->2560; "
                                                 "the reference checkpoint's width is 6912 (dit_step)")
    if not args.no_cpu_baseline:
        vqf = vq.float().cpu().numpy()
        tqf = tq.float().cpu().numpy()
        out["cpu_baseline"] = cpu_baseline(vqf, tqf, gains_np)
    for g in geoms:
        g.close()
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()

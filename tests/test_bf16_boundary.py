"""The bf16 boundary: round to nearest even down (cast_f32_bf16.comp:23-24),
exact widening up (cast_bf16_f32.comp:18-19).

CPU: the oracle's rounding against a hand-checked table and against torch's
float32 -> bfloat16 cast (round to nearest even) on every finite float32
pattern; widening on all 65536 bf16 patterns.  GPU: the C-ABI casts
(awa_cast_f32_to_bf16 / awa_cast_bf16_to_f32) against the same, and the bf16
stores of the AWA op itself on inputs whose exact result is a bf16 value.

NaN patterns are left out of the comparisons: the reference's integer formula
can carry a NaN with only low mantissa bits into infinity (0x7F800001 ->
0x7F80), where torch keeps a quiet NaN; no finite input reaches that path.
"""
import numpy as np
import pytest

from conftest import seeded_awa_inputs

# (float32 bits, bf16 bits), each worked out by hand from the rounding rule:
# keep the upper 16 bits, add one ulp when the dropped 16 bits exceed 0x8000,
# or equal 0x8000 and the kept lsb is 1.
RNE_TABLE = [
    (0x3F800000, 0x3F80),  # 1.0 exact
    (0x3F807FFF, 0x3F80),  # below the tie: down
    (0x3F808000, 0x3F80),  # tie, kept lsb 0: stays (even)
    (0x3F808001, 0x3F81),  # above the tie: up
    (0x3F818000, 0x3F82),  # tie, kept lsb 1: up to even
    (0x3F81FFFF, 0x3F82),  # just below the next value: up
    (0x3FFF8000, 0x4000),  # tie with lsb 1 at the top of the mantissa: carries into the exponent (2.0)
    (0x3FFF7FFF, 0x3FFF),  # same, below the tie: no carry
    (0xBF808000, 0xBF80),  # negative tie, lsb 0: magnitude stays
    (0xBF818000, 0xBF82),  # negative tie, lsb 1: magnitude up
    (0x00000000, 0x0000),  # +0
    (0x80000000, 0x8000),  # -0 keeps its sign
    (0x00008000, 0x0000),  # subnormal tie, lsb 0
    (0x00018000, 0x0002),  # subnormal tie, lsb 1
    (0x007FFFFF, 0x0080),  # largest subnormal rounds up to the smallest normal
    (0x7F7F7FFF, 0x7F7F),  # largest finite bf16 region, below the tie
    (0x7F7FFFFF, 0x7F80),  # max float32 overflows to +inf
    (0xFF7FFFFF, 0xFF80),  # and its negative to -inf
    (0x7F800000, 0x7F80),  # +inf
    (0xFF800000, 0xFF80),  # -inf
]


def _finite_chunk(k, size):
    u = np.arange(k * size, (k + 1) * size, dtype=np.uint64).astype(np.uint32)
    e = (u >> 23) & 0xFF
    return u[e != 0xFF]  # drops inf and NaN: the table covers the infinities


def test_rne_table(oracle):
    src = np.array([a for a, _ in RNE_TABLE], np.uint32)
    want = np.array([b for _, b in RNE_TABLE], np.uint16)
    got = oracle.f32_to_bf16(src.view(np.float32))
    assert np.array_equal(got, want), [(hex(a), hex(b), hex(int(g)))
                                       for (a, b), g in zip(RNE_TABLE, got) if b != g]


def test_widening_all_patterns(oracle):
    import torch
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.bf16_to_f32(b).view(np.uint32)
    assert np.array_equal(got, b.astype(np.uint32) << 16)
    t = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).float().numpy().view(np.uint32)
    nan = ((b >> 7) & 0xFF) == 0xFF
    nan &= (b & 0x7F) != 0
    assert np.array_equal(got[~nan], t[~nan])


@pytest.mark.slow
def test_rne_every_finite_pattern_matches_torch(oracle):
    """2^32 - 2^24 finite patterns in 256 chunks: oracle == torch's RNE cast."""
    import torch
    size = 1 << 24
    for k in range(256):
        u = _finite_chunk(k, size)
        f = u.view(np.float32)
        want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        got = oracle.f32_to_bf16(f)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, (k, hex(int(u[bad[0]])), hex(int(got[bad[0]])), hex(int(want[bad[0]])))


@pytest.mark.gpu
def test_gpu_casts_every_finite_pattern(oracle, ctx):
    """awa_cast_f32_to_bf16 on every finite float32 pattern (2^26 per launch)
    against torch's RNE cast on the device, a strided sample of 2^24 of them
    against the oracle, and awa_cast_bf16_to_f32 on all 65536 patterns."""
    import torch
    dev = torch.device("cuda:0")
    size = 1 << 26
    for k in range(64):
        start = k * size - (1 << 32 if k * size >= 1 << 31 else 0)  # signed view of the patterns
        u = torch.arange(start, start + size, dtype=torch.int32, device=dev)
        e = (u >> 23) & 0xFF
        u = u[e != 0xFF]
        f = u.view(torch.float32)
        out = torch.empty(f.numel(), dtype=torch.int16, device=dev)
        ctx.cast_f32_to_bf16(f, out)
        want = f.to(torch.bfloat16).view(torch.int16)
        nbad = int((out != want).sum())
        assert nbad == 0, (k, nbad)
        if k % 4 == 0:
            idx = torch.arange(0, f.numel(), 16, device=dev)
            fs = f[idx].cpu().numpy()
            assert np.array_equal(out[idx].cpu().numpy().view(np.uint16), oracle.f32_to_bf16(fs))
    b = torch.arange(65536, dtype=torch.int32, device=dev).to(torch.int16)
    w = torch.empty(65536, dtype=torch.float32, device=dev)
    ctx.cast_bf16_to_f32(b, w)
    got = w.cpu().numpy().view(np.uint32)
    bn = b.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, oracle.bf16_to_f32(bn).view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("shifted", [0, 1])
def test_gpu_op_bf16_stores_round_to_nearest_even(oracle, ctx, shifted):
    """With every value row of a head equal to one bf16 vector c, softmax
    weights summing to one make the exact output of every video and text row
    c itself; the GPU's fp32 result is c (1 + e) with |e| ~ 1e-6, which round
    to nearest even maps back to c bit for bit (truncation would give the
    next smaller magnitude whenever e < 0).  1080p geometry."""
    import torch
    dev = torch.device("cuda:0")
    grid, nw, txt = (1, 68, 80), (4, 3, 3), 58
    g = ctx.build_geometry(*grid, nw, txt, shifted)
    vqkv, tqkv, gains = seeded_awa_inputs(grid[0] * grid[1] * grid[2], txt, 12 + shifted)
    c = oracle.bf16_round(np.random.default_rng(5).standard_normal(2560).astype(np.float32))
    vqkv[:, 5120:] = c
    tqkv[:, 5120:] = c
    vq = torch.from_numpy(vqkv).to(dev, torch.bfloat16)
    tq = torch.from_numpy(tqkv).to(dev, torch.bfloat16)
    g4 = [torch.from_numpy(x).to(dev) for x in gains]
    va, ta = ctx.forward(g, vq, tq, *g4, eps=1e-5)
    torch.cuda.synchronize()
    want = oracle.f32_to_bf16(c)
    for out in (va, ta):
        bits = out.view(torch.int16).cpu().numpy().view(np.uint16)
        bad = np.flatnonzero(bits != want[None, :])
        assert bad.size == 0, (bad.size, bits.size)
    g.close()

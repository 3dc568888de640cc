// dit_gemm.hip — bf16 MFMA GEMMs of the DiT block with fused epilogues.
//
// D = A W^T with A [M][K] (activations, bf16) and W [N][K] (nn.Linear /
// ncnn InnerProduct layout, bf16); both operands are K-contiguous.  The
// kernel forms the transposed product per 16x16 block, D^T[n][m] =
// sum_k W[n][k] A[m][k], with v_mfma_f32_16x16x32_bf16 so that each lane
// ends with four consecutive output features of one activation row, which
// the epilogues store as 8- or 16-byte pieces of row-major outputs.  The
// 16x16x32 form does the work of the 32x32x16 one in twice the instructions
// but draws less power per flop: with all 256 CUs issuing back-to-back MFMAs
// on random bf16 data the part holds 1.86 GHz with it against 1.65 GHz with
// 32x32x16 (measured), and a full GEMM here runs at the power limit.
//
// Workgroup tile 256 (n) x 256 (m) or 256 x 224 (whichever fills the CUs in
// fewer rounds per row of tile; launch_gemm), K step 64, four wave64 in a 2x2
// grid of 128 x 128 (or 128 x 112) wave tiles, 64 (or 56) accumulators of
// 16x16 per wave.  Operand k-slices
// reach LDS by direct buffer->LDS DMA (buffer_load_dwordx4 ... lds) into two
// 64 KiB stages: while one stage is computed the next one lands.  LDS rows
// are 128 bytes (64 k of one operand row), so every DMA instruction reads
// whole 128-byte segments of global memory: with 64-byte rows (K step 32) the
// same bytes took twice the L2 requests and measurably longer to arrive.  A
// 16-byte-chunk XOR swizzle, chunk ^ ((row >> 1) & 7), keeps the fragment
// reads conflict-free.  The loop waits on the DMA counter with explicit
// s_waitcnt and a bare s_barrier (a __syncthreads would drain every
// outstanding load).  Each k32 sub-step issues its 64 MFMAs with the next
// sub-step's 16 fragment reads and (in the sub-step that refills the freed
// stage) 16 DMA pieces interleaved in its first half.
// Tiles are walked in groups of four m-tiles and assigned to XCDs in
// contiguous ranges, so the workgroups resident on one XCD share A and W
// k-slices through its L2.
//
// Epilogues (the elementwise tail of each projection in dit_vk.cpp:517-632):
//   EPI_STORE     C = bf16(acc)                               (qkv)
//   EPI_RESID     X += gate[n] * (acc + bias[n]), X fp32      (out proj, MLP out)
//   EPI_SWIGLU    U = bf16(silu(g) * h), W rows interleaved   (proj_in + proj_in_gate)
#include <atomic>
#include <type_traits>

#include "dit_internal.hpp"

namespace awa {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) void* lptr_t;

constexpr int BN = 256, BM = 256, BK = 64;
constexpr int NSTAGE = 2;                 // two 64 KiB stages: one computed while the next lands
constexpr int ROW_E = BK;                 // bf16 per LDS row (128 B, 8 chunks)
constexpr int STAGE_E = (BN + BM) * ROW_E;

// LDS has 64 four-byte banks (a 256-byte window); a 128-byte row is half of
// it, so chunk ^ ((row >> 1) & 7) gives the 16 rows read by a quarter-wave
// 16 distinct 16-byte bank groups.
__device__ inline int swz(int row, int chunk) { return row * ROW_E + ((chunk ^ ((row >> 1) & 7)) << 3); }


// A buffer resource over `bytes` from p with wave-uniform fields
// (readfirstlane returns int: each half of the address is taken back to
// uint32_t before widening, or a low word with bit 31 set would sign-extend
// into the high word; a resource the compiler cannot prove uniform makes it
// loop over the lanes at every access).  Loads past `bytes` read zeros and
// stores past it are dropped.
__device__ inline __amdgpu_buffer_rsrc_t uniform_rsrc(const void* p, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0,
                                             __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000);
}

// Epilogues go through LDS so that global memory sees whole rows: stores of
// 8- or 16-byte pieces of 32 rows per instruction (the accumulator layout)
// cost the memory system several times what whole 128-byte lines do.  Each
// wave stages its 128 x 128 block in its own 32 KiB of LDS as rows of the
// output (16-byte chunk c of staged row r at chunk c ^ (r & 15) for rows of
// 16 chunks, c ^ ((r >> 1) & 7) for rows of 8, two of which share a 256-byte
// bank window: conflict-free for both the accumulator-order writes and the
// row reads) and reads it back row by row, 16 (or 8) lanes per row.
//
// Accumulator layout: acc[i][j] is the 16x16 block of output features
// n_base + 16 i + .. and rows m_base + 16 j + ..; lane (col = lane % 16,
// q = lane / 16) holds row 16 j + col, features 16 i + 4 q + t in register t.
template <int EPI, int MJ>
__device__ inline void epilogue(const GemmProblem& p, const f32x4 (&acc)[8][MJ], int n_base,
                                int m_base, int lane, uint16_t* stg) {
    const int q = lane >> 4, col = lane & 15;
    if constexpr (EPI == EPI_STORE) {
        // staged rows: 128 features bf16 = 256 bytes, 16 chunks of 8
#pragma unroll
        for (int j = 0; j < MJ; j++) {
            const int r = 16 * j + col;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const f32x4& a = acc[i][j];
                const uint2 u = make_uint2(bf16x2_rne(a[0], a[1]), bf16x2_rne(a[2], a[3]));
                const int c = 2 * i + (q >> 1);
                *reinterpret_cast<uint2*>(stg + r * 128 + ((c ^ (r & 15)) << 3) + 4 * (q & 1)) = u;
            }
        }
        // read back MJ staged rows per lane at a time, then store them
        // through a resource that ends at row M (no branch per row, so the
        // reads are not each waited for before their store)
        const int c = lane & 15;
        const __amdgpu_buffer_rsrc_t cres = uniform_rsrc(
            reinterpret_cast<uint16_t*>(p.C) + (size_t)m_base * p.ldc,
            (uint32_t)min(max(p.M - m_base, 0), 16 * MJ) * p.ldc * 2);
        const uint32_t ofs0 = 2u * ((uint32_t)(lane >> 4) * p.ldc + n_base + c * 8);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            u32x4 v[MJ];
#pragma unroll
            for (int k = 0; k < MJ; k++) {
                const int r = 4 * (g * MJ + k) + (lane >> 4);
                v[k] = *reinterpret_cast<const u32x4*>(stg + r * 128 + ((c ^ (r & 15)) << 3));
            }
#pragma unroll
            for (int k = 0; k < MJ; k++)
                __builtin_amdgcn_raw_buffer_store_b128(v[k], cres, ofs0 + (g * MJ + k) * 8u * p.ldc, 0, 0);
        }
    } else if constexpr (EPI == EPI_SWIGLU) {
        // W rows alternate 32 in / 32 gate: blocks (4h + e, 4h + 2 + e) are
        // (in, gate) of output features 32 h + 16 e + ..; staged rows: 64
        // features bf16 = 128 bytes, 8 chunks of 8
#pragma unroll
        for (int j = 0; j < MJ; j++) {
            const int r = 16 * j + col;
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    uint32_t packed[2];
#pragma unroll
                    for (int t2 = 0; t2 < 4; t2 += 2) {
                        float o[2];
#pragma unroll
                        for (int t = 0; t < 2; t++) {
                            const float hv = acc[4 * h + e][j][t2 + t];
                            const float gt = acc[4 * h + 2 + e][j][t2 + t];
                            o[t] = gt / (1.f + __expf(-gt)) * hv;
                        }
                        packed[t2 >> 1] = bf16x2_rne(o[0], o[1]);
                    }
                    const int c = 4 * h + 2 * e + (q >> 1);
                    *reinterpret_cast<uint2*>(stg + r * 64 + ((c ^ ((r >> 1) & 7)) << 3) + 4 * (q & 1)) =
                        make_uint2(packed[0], packed[1]);
                }
        }
        // read back MJ staged rows per lane at a time, then store them
        // through a resource that ends at row M (as in EPI_STORE)
        const int c = lane & 7;
        const __amdgpu_buffer_rsrc_t cres = uniform_rsrc(
            reinterpret_cast<uint16_t*>(p.C) + (size_t)m_base * p.ldc,
            (uint32_t)min(max(p.M - m_base, 0), 16 * MJ) * p.ldc * 2);
        const uint32_t ofs0 = 2u * ((uint32_t)(lane >> 3) * p.ldc + (n_base >> 1) + c * 8);
#pragma unroll
        for (int g = 0; g < 2; g++) {
            u32x4 v[MJ];
#pragma unroll
            for (int k = 0; k < MJ; k++) {
                const int r = 8 * (g * MJ + k) + (lane >> 3);
                v[k] = *reinterpret_cast<const u32x4*>(stg + r * 64 + ((c ^ ((r >> 1) & 7)) << 3));
            }
#pragma unroll
            for (int k = 0; k < MJ; k++)
                __builtin_amdgcn_raw_buffer_store_b128(v[k], cres, ofs0 + (g * MJ + k) * 16u * p.ldc, 0, 0);
        }
    } else {  // EPI_RESID, in two halves of 64 features (staged fp32 rows: 256 bytes)
        float* sf = reinterpret_cast<float*>(stg);
        const int c = lane & 15;
        // The residual rows of this wave's block through a buffer resource
        // that ends at row M: rows past it read zeros and their stores are
        // dropped, so there is no branch per row.  Rows go in chunks of 2 MJ
        // (a quarter of the block's rows and features per lane), each
        // chunk's loads issued before the chunk ahead of it is updated and
        // stored: vector memory operations complete in order, so a wait for
        // a chunk never waits for the stores issued after its loads.
        // (Written as load, update, store per row, the compiler cannot tell
        // a row's store from the next row's load apart, and every row waited
        // a full memory round trip behind the one before, from HBM inside
        // the DiT step.)
        const __amdgpu_buffer_rsrc_t xres = uniform_rsrc(reinterpret_cast<float*>(p.C) + (size_t)m_base * p.ldc,
                                                        (uint32_t)min(max(p.M - m_base, 0), 16 * MJ) * p.ldc * 4);
        constexpr int CH = 2 * MJ;  // rows per lane and chunk; chunks (half, part): 4 MJ rows a half
        const uint32_t ofs_it = 16u * p.ldc;
        auto ofs0 = [&](int half) __attribute__((always_inline)) {  // bytes, row 4 it + lane / 16
            return 4u * ((uint32_t)(lane >> 4) * p.ldc + n_base + 64 * half + 4 * c);
        };
        auto load_chunk = [&](float4 (&xr)[CH], int half, int part) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const u32x4 raw =
                    __builtin_amdgcn_raw_buffer_load_b128(xres, ofs0(half) + (part * CH + i) * ofs_it, 0, 0);
                xr[i] = make_float4(__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                                    __uint_as_float(raw[3]));
            }
        };
        auto stage = [&](int half) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < MJ; j++) {
                const int r = 16 * j + col;
#pragma unroll
                for (int i2 = 0; i2 < 4; i2++) {
                    const f32x4& a = acc[4 * half + i2][j];
                    const int ch = 4 * i2 + q;
                    *reinterpret_cast<float4*>(sf + r * 64 + ((ch ^ (r & 15)) << 2)) =
                        make_float4(a[0], a[1], a[2], a[3]);
                }
            }
        };
        // bias and gates of both halves, loaded first and without branches:
        // a null vector gets an empty resource (its loads read zeros) and
        // the value is chosen after the load (bias 0, gates 1)
        auto vec_rsrc = [&](const float* v) __attribute__((always_inline)) {
            return uniform_rsrc(v, v ? p.N * 4 : 0);
        };
        auto vec_load = [&](__amdgpu_buffer_rsrc_t r, int n) __attribute__((always_inline)) {
            const u32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(r, 4u * n, 0, 0);
            return make_float4(__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                               __uint_as_float(raw[3]));
        };
        const __amdgpu_buffer_rsrc_t bres = vec_rsrc(p.bias), g0res = vec_rsrc(p.gate0), g1res = vec_rsrc(p.gate1);
        const float4 one = make_float4(1.f, 1.f, 1.f, 1.f);
        float4 bv[2], g0v[2], g1v[2];
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int n = n_base + 64 * half + 4 * c;
            bv[half] = vec_load(bres, n);
            const float4 l0 = vec_load(g0res, n), l1 = vec_load(g1res, n);
            g0v[half] = p.gate0 ? l0 : one;
            g1v[half] = p.gate1 ? l1 : one;
        }
        auto update = [&](const float4 (&xr)[CH], int half, int part) __attribute__((always_inline)) {
            const float4 b = bv[half], g0 = g0v[half], g1 = g1v[half];
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const int it = part * CH + i;
                const int r = 4 * it + (lane >> 4), m = m_base + r;
                const float4 v = *reinterpret_cast<const float4*>(sf + r * 64 + ((c ^ (r & 15)) << 2));
                const float4 gt = m < p.split ? g0 : g1;
                float4 x = xr[i];
                // gate * (proj + bias), then the residual add (dit_vk.cpp:558-575)
                x.x = gt.x * (v.x + b.x) + x.x;
                x.y = gt.y * (v.y + b.y) + x.y;
                x.z = gt.z * (v.z + b.z) + x.z;
                x.w = gt.w * (v.w + b.w) + x.w;
                const u32x4 w = {__float_as_uint(x.x), __float_as_uint(x.y), __float_as_uint(x.z),
                                 __float_as_uint(x.w)};
                __builtin_amdgcn_raw_buffer_store_b128(w, xres, ofs0(half) + it * ofs_it, 0, 0);
            }
        };
        float4 xa[CH], xc[CH];
        load_chunk(xa, 0, 0);
        stage(0);
        load_chunk(xc, 0, 1);
        update(xa, 0, 0);
        load_chunk(xa, 1, 0);
        update(xc, 0, 1);
        stage(1);  // after the last reads of half 0's staged rows (same wave, LDS in order)
        load_chunk(xc, 1, 1);
        update(xa, 1, 0);
        update(xc, 1, 1);
    }
}

template <int EPI, int MJ>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmBatch b) {
    constexpr int BMT = 32 * MJ;  // rows of A per tile (LDS is laid out for BM)
    __shared__ __align__(16) uint16_t lds[NSTAGE * STAGE_E];
    const int lid = xcd_remap(b.total_tiles);
    if (lid >= b.total_tiles) return;
    const int pi = lid < b.tiles0 ? 0 : 1;
    const GemmProblem& p = b.p[pi];
    int local = lid - (pi ? b.tiles0 : 0);
    // grouped order: four m-tiles per group, n advancing across the group
    constexpr int GM = 4;
    const int group = local / (GM * p.n_tiles);
    const int first_m = group * GM;
    const int gm = min(p.m_tiles - first_m, GM);
    const int in_group = local % (GM * p.n_tiles);
    const int mt = first_m + in_group % gm;
    const int nt = in_group / gm;
    const int n0 = nt * BN, m0 = mt * BMT;

    // wave is uniform: read into a scalar so that the LDS-DMA destinations
    // (M0) are formed by scalar instructions, without v_readfirstlane
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wn = wave >> 1, wm = wave & 1;
    const int q = lane >> 4, r16 = lane & 15;

    // Operand tiles go straight from global memory into LDS
    // (buffer_load_dwordx4 ... lds: lane i of a wave writes 16 bytes at
    // M0 + 16 i).  One wave instruction fills 1 KiB = 8 swizzled rows; lane l
    // lands in row r0 + l/8, physical chunk l%8, so it fetches the logical
    // chunk that the swizzle maps there.  Each wave issues 8 + 8 per stage.
    const int lrow = lane >> 3;
    const uint16_t* Wp = p.W + (size_t)n0 * p.ldw;
    // Buffer loads (SGPR resource + 32-bit lane offset + SGPR k offset) issue
    // measurably faster than global loads with 64-bit lane addresses.  Rows
    // of A past M repeat the last row; the resource range bounds every read.
    const uint16_t* Ap = p.A + (size_t)m0 * p.lda;
    const int arows = min(BMT, p.M - m0);  // LDS rows past BMT are fetched (clamped) but unused
    int woff[8], aoff[8];   // byte offsets of this lane's 16 bytes at k = 0
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int row = (wave * 8 + i) * 8 + lrow;
        const int lch = (lane & 7) ^ ((row >> 1) & 7);
        woff[i] = (row * p.ldw + lch * 8) * 2;
        aoff[i] = (min(row, arows - 1) * p.lda + lch * 8) * 2;
    }
    // raw buffer, 32-bit dword format (word 3 of the resource)
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc((void*)Wp, 0, BN * p.ldw * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc((void*)Ap, 0, arows * p.lda * 2, 0x00020000);
    // piece g (0..15) of stage kt into ring slot `slot`: W block g/2 (even g)
    // or A block g/2 (odd g), 8 rows of 128 bytes
    auto load_piece = [&](int kt, int slot, int g) __attribute__((always_inline)) {
        uint16_t* dst = lds + slot * STAGE_E + ((g & 1) ? BN * ROW_E : 0) + (wave * 8 + (g >> 1)) * 512;
        if (g & 1) __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (lptr_t)dst, 16, aoff[g >> 1], kt * BK * 2, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, (lptr_t)dst, 16, woff[g >> 1], kt * BK * 2, 0, 0);
    };
    auto load = [&](int kt, int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < 16; g++) load_piece(kt, slot, g);
    };

    // no zero fill: the first sub-step's MFMAs take a zero accumulator operand
    f32x4 acc[8][MJ];

    const int nk = p.K / BK;
    int wrow[8], arow[MJ];
#pragma unroll
    for (int i = 0; i < 8; i++) wrow[i] = wn * 128 + 16 * i + r16;
#pragma unroll
    for (int j = 0; j < MJ; j++) arow[j] = wm * 16 * MJ + 16 * j + r16;
    // fragments of one k32 sub-step: eight 16-row blocks of W and of A (lane:
    // row r16 of the block, k 8 q .. 8 q + 7 of the sub-step)
    bf16x8 wf[2][8], af[2][MJ];
    // slot `slot`, k32 sub-step s, fragment buffer buf
    auto read_frags = [&](int slot, int s, int buf) __attribute__((always_inline)) {
        const uint16_t* ws = lds + slot * STAGE_E;
        const uint16_t* as = ws + BN * ROW_E;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            wf[buf][i] = *reinterpret_cast<const bf16x8*>(ws + swz(wrow[i], 4 * s + q));
            if (i < MJ) af[buf][i] = *reinterpret_cast<const bf16x8*>(as + swz(arow[i], 4 * s + q));
        }
    };
    // One k32 sub-step: the 64 MFMAs on fragment buffer `buf`; in the first
    // half, after each even one a fragment read of the next sub-step (slot
    // rslot, sub-step rs, into buffer buf ^ 1) and, when `dma`, after each odd
    // one a DMA piece of stage dma_kt.  sched_barrier pins this order: every
    // read is in flight half a sub-step before its use, the wait for the
    // previous sub-step's reads comes before the first new read (the compiler
    // waits on the LDS counter with lgkmcnt(0)), and the DMA pieces go out
    // early, which leaves them a sub-step and a half to land.
    auto substep = [&](int buf, int rslot, int rs, bool do_read, bool dma, int dma_kt, int dma_slot, bool zc)
        __attribute__((always_inline)) {
        const uint16_t* ws = lds + rslot * STAGE_E;
        const uint16_t* as = ws + BN * ROW_E;
#pragma unroll
        for (int g = 0; g < 8 * MJ; g++) {
            const int i = g / MJ, j = g % MJ;
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                wf[buf][i], af[buf][j], zc ? (f32x4){0.f, 0.f, 0.f, 0.f} : acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (g < 32) {
                if (dma && (g & 1)) load_piece(dma_kt, dma_slot, g >> 1);
                if (do_read && !(g & 1)) {
                    const int r = g >> 2;
                    if (g & 2) {
                        if (r < MJ) af[buf ^ 1][r] = *reinterpret_cast<const bf16x8*>(as + swz(arow[r], 4 * rs + q));
                    }
                    else
                        wf[buf ^ 1][r] = *reinterpret_cast<const bf16x8*>(ws + swz(wrow[r], 4 * rs + q));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Software pipeline over k32 sub-steps, two per stage, two stages: while
    // stage kt is computed from slot kt & 1, stage kt + 1 lands in the other
    // slot.  Sub-step 0 of stage kt reads sub-step 1's fragments from the same
    // slot; then every wave waits for its own DMA of stage kt + 1 and for its
    // LDS reads, and the barrier makes stage kt + 1 visible and slot kt & 1
    // free: sub-step 1 reads stage kt + 1's first fragments and refills slot
    // kt & 1 with stage kt + 2 (past the last stage it repeats the last stage
    // into the free slot, so the loop body stays branch-free and the DMA count
    // it waits on stays fixed).
    const int last = nk - 1;
    load(0, 0);
    load(min(1, last), 1);
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    read_frags(0, 0, 0);
    int slot = 0;
    if (last == 0) {  // one K stage
        substep(0, 0, 1, true, false, 0, 0, true);
        substep(1, 0, 0, false, false, 0, 0, false);
    } else {
        // stage 0 peeled: its first sub-step starts the accumulators
        substep(0, 0, 1, true, false, 0, 0, true);
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        substep(1, 1, 0, true, true, min(2, last), 0, false);
        slot = 1;
        for (int kt = 1; kt < last; kt++) {
            substep(0, slot, 1, true, false, 0, 0, false);
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            substep(1, slot ^ 1, 0, true, true, min(kt + 2, last), slot, false);
            slot ^= 1;
        }
        substep(0, slot, 1, true, false, 0, 0, false);
        substep(1, slot, 0, false, false, 0, 0, false);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the redundant last refill
    // every wave is done with the operand tiles: LDS becomes the staging area
    __syncthreads();
    epilogue<EPI, MJ>(p, acc, n0 + wn * 128, m0 + wm * 16 * MJ, lane, lds + wave * (128 * 128));
}

}  // namespace

// Tiles of 256 x 256 or 256 x 224 (rows of A), whichever needs fewer
// workgroup rounds times rows per tile on the device's CUs: with 5498 rows,
// 2560 output features give 220 tiles of 256 rows (1 round, 36 CUs idle) or
// 250 of 224 (1 round, 12 % less work per tile).
hipError_t launch_gemm(int epi, GemmBatch& b, hipStream_t s) {
    // CU count per device, looked up once (threads may race to store the same value)
    static std::atomic<int> n_cu[64];
    int dev = 0, cus = 256;
    (void)hipGetDevice(&dev);
    if (dev >= 0 && dev < 64) {
        int c = n_cu[dev].load(std::memory_order_relaxed);
        if (c == 0 && hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
            n_cu[dev].store(c, std::memory_order_relaxed);
        if (c > 0) cus = c;
    }
    auto tiles_for = [&](int bm) {
        long t = 0;
        for (int i = 0; i < b.nprob; i++) t += (long)(b.p[i].N / BN) * ((b.p[i].M + bm - 1) / bm);
        return t;
    };
    const long t8 = tiles_for(256), t7 = tiles_for(224);
    const int mj = ((t7 + cus - 1) / cus) * 7 < ((t8 + cus - 1) / cus) * 8 ? 7 : 8;
    const int bm = 32 * mj;
    b.total_tiles = 0;
    for (int i = 0; i < b.nprob; i++) {
        GemmProblem& p = b.p[i];
        p.n_tiles = p.N / BN;
        p.m_tiles = (p.M + bm - 1) / bm;
        if (i == 0) b.tiles0 = p.n_tiles * p.m_tiles;
        b.total_tiles += p.n_tiles * p.m_tiles;
    }
    if (b.nprob == 1) b.p[1] = b.p[0];
    if (b.total_tiles == 0) return hipSuccess;
    const int grid = ((b.total_tiles + 7) >> 3) << 3;
#define GEMM_LAUNCH(E)                                                                  \
    do {                                                                                \
        if (mj == 7) hipLaunchKernelGGL((gemm_kernel<E, 7>), dim3(grid), dim3(256), 0, s, b); \
        else hipLaunchKernelGGL((gemm_kernel<E, 8>), dim3(grid), dim3(256), 0, s, b);         \
    } while (0)
    switch (epi) {
        case EPI_STORE: GEMM_LAUNCH(EPI_STORE); break;
        case EPI_RESID: GEMM_LAUNCH(EPI_RESID); break;
        case EPI_SWIGLU: GEMM_LAUNCH(EPI_SWIGLU); break;
        default: return hipErrorInvalidValue;
    }
#undef GEMM_LAUNCH
    return hipGetLastError();
}

}  // namespace awa

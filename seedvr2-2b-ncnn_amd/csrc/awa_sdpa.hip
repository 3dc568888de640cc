// awa_sdpa.hip — varlen window attention on CDNA4 matrix cores.
//
// Replaces the per-(window, head) softmax(Q K^T / sqrt(128)) V of
// dit_vk.cpp:406-439 / awa.comp:79-171 for all windows at once.  Window w's
// sequence is its f_w video rows followed by the TXT text rows (dit_vk.cpp:
// 391-405), non-causal.
//
// One workgroup (4 wave64) per (work item, head).  A work item is one window
// and up to two of its 64-row query tiles; each wave owns 32 queries.  The
// window's key/value tiles stream through LDS (double buffered).  Scores are
// formed transposed, S^T = K Q^T, so that a lane owns one query column: the
// online softmax (exp2, log2(e) folded into the scale) then needs only one
// cross-lane exchange (lane ^ 32), and the probabilities leave the MFMA
// accumulator already in the B-operand layout of O^T = V^T P^T.  The bf16
// kernel takes V straight from vqkv / tqkv (no packed copy): its rows are
// gathered into LDS by DMA and the A operand V^T is read back transposed with
// ds_read_b64_tr_b16; the fp32 kernel reads a V^T tile packed per window.
//
// bf16 storage -> v_mfma_f32_32x32x16_bf16 (fp32 accumulation); fp32
// storage -> v_mfma_f32_32x32x2f32 in awa_sdpa_f32.hip (a file of its own:
// this one is compiled with the MFMA accumulators in VGPRs, which the bf16
// kernel's softmax wants and which made the fp32 kernel spill).
//
// Video query rows are scattered back to token order (dit_vk.cpp:445-455);
// text query rows go to per-window fp32 partials that the coalesce kernel
// averages in window order (dit_vk.cpp:440-444).
#include <type_traits>

#include "awa_internal.hpp"

namespace awa {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Two floats -> two bf16 (round to nearest even) in one word, low half
// first: one v_cvt_pk_bf16_f32.
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}


// Writes the normalised O^T accumulators of one wave (lane: query n, register
// r of d-tile dt: channel 32dt + 8(r/4) + 4(lane/32) + r%4).
template <bool kBf16Out>
__device__ inline void store_rows(const f32x16 (&oacc)[4], float inv, int hb, void* dst_row) {
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 32 * dt + 8 * g + 4 * hb;
            const float o0 = oacc[dt][4 * g] * inv, o1 = oacc[dt][4 * g + 1] * inv;
            const float o2 = oacc[dt][4 * g + 2] * inv, o3 = oacc[dt][4 * g + 3] * inv;
            if constexpr (kBf16Out) {
                uint2 u;
                u.x = pack_bf16x2(o0, o1);
                u.y = pack_bf16x2(o2, o3);
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(dst_row) + d0) = u;
            } else {
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(dst_row) + d0) =
                    make_float4(o0, o1, o2, o3);
            }
        }
}

// ----------------------------------------------------------------- bf16
// Persistent kernel: one workgroup of two wave64 per resident slot (two per
// CU, one wave per SIMD), each processing the list of work items the host
// planned for it (GeomPlan::sched_*): a work item is one head, one window and
// one or two of its 64-row query tiles (one per wave).  A wave holds its query
// tile as two 32-query column blocks (qb), so each K or V^T fragment read from
// LDS feeds two MFMAs: with 32 queries per wave the fragment reads alone would
// keep LDS (128 B/clk/CU) as busy as the matrix cores.  K and V^T tiles reach
// LDS by DMA (buffer_load_dwordx4 ... lds: lane i of a wave writes 16 bytes at
// M0 + 16 i), K in a ring of three tile slots and V^T in a ring of two (80 KiB
// per workgroup).  The tiles a slot fetches form one stream across its
// items: each tile fetches the K tile two ahead and the V^T tile one ahead,
// so an item's last two tiles fetch the next item's first tiles, and after
// its last unit the next query tile is loaded: an item starts without memory
// round trips.
//
// The window's keys are processed in 32-key units u (two per tile).  With a
// single wave per SIMD nothing hides latency but the wave's own instruction
// stream, so each unit runs as two phases in which the matrix core and the
// VALU work side by side:
//
//   A(u)  MFMA  S(u+1) = K(u+1) Q^T - m         (2 x 9 MFMAs: a bias k-step
//                                               adds -m, m a bf16 value)
//         VALU  P(u) = exp2(S(u))               (32 exponentials)
//         LDS   V^T(u) fragments                (16 transposed reads)
//   B(u)  MFMA  O^T += V^T(u) P^T(u)            (16 MFMAs)
//         VALU  row maximum of S(u+1), row sums of P(u)
//         LDS   K(u+2) fragments                (8 reads, one per MFMA)
//
// With one wave per SIMD the LDS answers a wave's reads with a latency of a
// few hundred cycles (its read rate grows with the reads in flight: about
// 90 B/clk/CU from four waves, 170-190 from sixteen, measured), so each
// fragment is read a phase before its MFMAs: the K fragments of unit u + 2
// during phase B of unit u, from asm (the compiler does not track them; the
// next phase A starts with an explicit wait naming their registers), and the
// V^T fragments early in phase A, pinned there by a scheduling group.
// Phase A is written with the compiler's MFMA and exp2 builtins, ordered two
// exponentials then one MFMA by sched_group_barrier, and the scores live in
// two register sets that alternate between units (unit u exponentiates set
// u & 1 in place while its MFMAs fill the other): with asm statements naming
// single score registers the compiler copied all 32 of them at every unit
// boundary.  Phase B issues each MFMA and its share of VALU work from one asm
// statement.  The output accumulators O^T (128 AGPRs) and the query fragments
// (64 AGPRs, the B operand of the score MFMAs) are pinned to the accumulation
// registers by asm constraints; the scores live in VGPRs.  The running
// maximum m stays stale until a unit's
// maximum exceeds it by more than 2^8 (the output is divided by the matching
// sum at the end, so the result is unchanged); then O^T, the running sum and
// the pending scores are rescaled.  The upper 32-key half of a short last tile
// is fully masked (P = 0).
//
// Hazards the compiler cannot see through asm: every asm statement issues its
// VALU work before its MFMA, which supplies the two wait states an MFMA needs
// after a VALU write of its operands; explicit waits of sixteen or more cover
// VALU reads of the results of asm MFMAs (eleven are required after an 8-pass
// MFMA).  Around the builtins the compiler places the waits itself.
typedef __attribute__((address_space(1))) void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;
typedef __attribute__((address_space(3))) char lchar_t;
typedef __attribute__((address_space(3))) bf16x4 lbf16x4_t;

// LDS DMA of one wave's half of a K or V tile: eight 16-byte-per-lane loads
// (lane i writes 16 bytes at M0 + offset + 16 i), instruction j filling the
// 1 KiB at LDS byte address m + 1024 j.  The instruction offset moves the
// global address and the LDS destination alike, so four instructions share
// one M0 write with offsets 0, 1024, 2048, 3072, and each lane's global
// offset for instruction j is passed with 1024 (j % 4) already subtracted.
// Issued from asm because for the builtin the compiler tracks the pending LDS
// writes itself: it then drains vmcnt before any LDS store and, since it
// counts them with the LDS operations, turns every later LDS wait into
// lgkmcnt(0), so the fragment reads of the score loop and the epilogue's
// staging round trips could no longer overlap.  The kernel waits for these
// loads itself (vmcnt(0) and a barrier) before any wave reads the tiles they
// fill.  M0 written by an SALU instruction needs one wait state before the
// DMA reads it.
// K: four instructions from buffer r (one tile) at SGPR offset so with lane
// offsets vo[0..3].
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void dma4_k(__amdgpu_buffer_rsrc_t r, uint32_t so, const uint32_t (&vo)[4], uint32_t m) {
    asm volatile(
        "s_mov_b32 m0, %[m]\n\ts_nop 0\n\t"
        "buffer_load_dwordx4 %[v0], %[r], %[so] offen lds\n\t"
        "buffer_load_dwordx4 %[v1], %[r], %[so] offen offset:1024 lds\n\t"
        "buffer_load_dwordx4 %[v2], %[r], %[so] offen offset:2048 lds\n\t"
        "buffer_load_dwordx4 %[v3], %[r], %[so] offen offset:3072 lds"
        :
        : [v0] "v"(vo[0]), [v1] "v"(vo[1]), [v2] "v"(vo[2]), [v3] "v"(vo[3]), [r] "s"(r), [so] "s"(so),
          [m] "s"(m)
        : "memory", "m0");
}
// Single DMA instructions, for spreading a tile's DMA over the MFMA stream
// one instruction at a time: byte offset 1024 o of buffer r (plus SGPR offset
// so for K), into LDS address M0 + 1024 o.  M0 is set by m0_set, once per
// four instructions, and nothing else in the kernel writes M0 (the compiler
// has no use for it in this code: a test checks its assembly for that); the
// asm statements are volatile, so they keep their order.
__device__ __attribute__((always_inline)) inline void m0_set(uint32_t m) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0" : : "s"(m) : "m0");
}
__device__ __attribute__((always_inline)) inline void dma1_k(int o, __amdgpu_buffer_rsrc_t r, uint32_t so, uint32_t vo) {
#define DMA1K(O)                                                                          \
    asm volatile("buffer_load_dwordx4 %[v], %[r], %[so] offen offset:" #O " lds"          \
                 :                                                                        \
                 : [v] "v"(vo), [r] "s"(r), [so] "s"(so)                                  \
                 : "memory")
    switch (o) {
        case 0: DMA1K(0); break;
        case 1: DMA1K(1024); break;
        case 2: DMA1K(2048); break;
        default: DMA1K(3072); break;
    }
#undef DMA1K
}
__device__ __attribute__((always_inline)) inline void dma1_v(int o, __amdgpu_buffer_rsrc_t r, uint32_t vo) {
#define DMA1V(O)                                                                                  \
    asm volatile("buffer_load_dwordx4 %[v], %[r], 0 offen offset:" #O " lds"                      \
                 :                                                                                \
                 : [v] "v"(vo), [r] "s"(r)                                                        \
                 : "memory")
    switch (o) {
        case 0: DMA1V(0); break;
        case 1: DMA1V(1024); break;
        case 2: DMA1V(2048); break;
        default: DMA1V(3072); break;
    }
#undef DMA1V
}
// The eight instructions of a wave's K half tile (the second four 16 rows on).
__device__ inline void dma_k8(__amdgpu_buffer_rsrc_t r, const uint32_t (&vo)[4], uint32_t m) {
    dma4_k(r, 0, vo, m);
    dma4_k(r, 4096, vo, m + 4096);
}
// V rows: four instructions from buffer r (a head's V columns of vqkv or
// tqkv, based 3 KiB early so that the compensated offsets stay positive; an
// offset outside the buffer reads zeros) with lane offsets o_j.
__device__ inline void dma4_vrow(__amdgpu_buffer_rsrc_t r, uint32_t o0, uint32_t o1, uint32_t o2,
                                 uint32_t o3, uint32_t m) {
    asm volatile(
        "s_mov_b32 m0, %[m]\n\ts_nop 0\n\t"
        "buffer_load_dwordx4 %[v0], %[r], 0 offen lds\n\t"
        "buffer_load_dwordx4 %[v1], %[r], 0 offen offset:1024 lds\n\t"
        "buffer_load_dwordx4 %[v2], %[r], 0 offen offset:2048 lds\n\t"
        "buffer_load_dwordx4 %[v3], %[r], 0 offen offset:3072 lds"
        :
        : [v0] "v"(o0), [v1] "v"(o1), [v2] "v"(o2), [v3] "v"(o3), [r] "s"(r), [m] "s"(m)
        : "memory", "m0");
}
#pragma clang diagnostic pop

constexpr int KT_E = TILE * HEAD_D;         // bf16 elements of a K (or V^T) tile
constexpr float RESCALE_LOG2 = 8.f;

// Maximum and sum over lanes l and l ^ 32 (v_permlane32_swap: no LDS trip).
__device__ inline float max_pair(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float sum_pair(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Unit 0's score MFMAs: s += k q^T.
__device__ inline void qk_only(f32x16& s, const bf16x8& k, const bf16x8& q) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(s) : "v"(k), "a"(q));
}
// First MFMA of a chain without exponentials: s = k q^T.
__device__ inline void qk_zero(f32x16& s, const bf16x8& k, const bf16x8& q) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(s) : "v"(k), "a"(q));
}
// Phase B slot: mx = max(mx, y0, y1), ps += x0 + x1, then o += v p^T.
__device__ inline void max_sum_pv(f32x16& o, const bf16x8& v, const bf16x8& p, float& mx, float y0,
                                  float y1, float& ps, float x0, float x1) {
    asm volatile(
        "v_max3_f32 %1, %1, %5, %6\n\tv_add_f32 %2, %2, %7\n\tv_add_f32 %2, %2, %8\n\t"
        "v_mfma_f32_32x32x16_bf16 %0, %3, %4, %0"
        : "+a"(o), "+v"(mx), "+v"(ps)
        : "v"(v), "v"(p), "v"(y0), "v"(y1), "v"(x0), "v"(x1));
}
// Phase B of an item's last unit (no next unit): ps += x0 + x1, o += v p^T.
__device__ inline void sum_pv(f32x16& o, const bf16x8& v, const bf16x8& p, float& ps, float x0, float x1) {
    asm volatile(
        "v_add_f32 %1, %1, %4\n\tv_add_f32 %1, %1, %5\n\ts_nop 0\n\t"
        "v_mfma_f32_32x32x16_bf16 %0, %2, %3, %0"
        : "+a"(o), "+v"(ps)
        : "v"(v), "v"(p), "v"(x0), "v"(x1));
}
// K fragment read issued from asm (the compiler neither counts it nor waits
// for it; the next phase A's start waits for it explicitly, naming the
// registers).
__device__ inline void ds_read_kf(bf16x8& d, uint32_t addr) {
    asm volatile("ds_read_b128 %0, %1" : "=a"(d) : "v"(addr));
}
// bf16 value nearest to x (round to nearest even), as a float.
__device__ inline float bf16_round(float x) { return __uint_as_float(bf16_rne(x) << 16); }
// B-operand fragment of the bias k-step: element 0 of lanes 0-31 holds -m of
// query column n (a bf16 value, so exact), element 1 holds -2^24, everything
// else 0.  Paired with the A fragment of mask_frag (key column 0 = 1, key
// column 1 = 1 for masked keys), the MFMA adds -m to every score and -2^24
// more to the masked ones, whose exponentials are then 0: no separate
// masking pass and no branch in the unit loop.
__device__ inline bf16x8 bias_frag(float m, int hb) {
    bf16x8 b;
#pragma unroll
    for (int i = 0; i < 8; i++) b[i] = (__bf16)0.f;
    if (hb == 0) {
        b[0] = (__bf16)(-m);
        b[1] = (__bf16)(-16777216.f);
    }
    return b;
}
// A-operand fragment of the bias k-step of a unit with kv valid keys (key
// row n of the unit is masked when n >= kv; kv <= 0 masks all).
__device__ inline bf16x8 mask_frag(int kv, int n, int hb) {
    const uint32_t w0 = hb == 0 ? (0x3f80u | (n >= kv ? 0x3f800000u : 0u)) : 0u;
    const u32x4 w = {w0, 0u, 0u, 0u};
    return __builtin_bit_cast(bf16x8, w);
}
// Waits after MFMA writes before anything else touches the results (ties the
// registers so that nothing is scheduled across).
__device__ inline void mfma_fence_v(f32x16 (&s)[2]) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(s[0]), "+v"(s[1]));
}
// The compiler places no wait states before an asm statement for what the
// instructions before it wrote, so the asm of phase B, which reads the results
// of the score MFMAs (builtins: a VALU read needs twelve wait states after
// v_mfma_f32_32x32x16_bf16) and of the exponentials (v_exp_f32: one), comes
// after this fence: it ties both register sets and waits sixteen.  Without it
// the scheduler may end phase A with the MFMA whose scores phase B's first
// maximum reads, which then sees the registers' previous contents.
__device__ inline void score_fence(f32x16 (&s)[2], f32x16 (&p)[2]) {
    asm volatile("s_nop 7\n\ts_nop 7" : "+v"(s[0]), "+v"(s[1]), "+v"(p[0]), "+v"(p[1]));
}
// The same after the exponentials of an item's last unit (no MFMA results).
__device__ inline void exp_fence(f32x16 (&p)[2]) {
    asm volatile("s_nop 1" : "+v"(p[0]), "+v"(p[1]));
}
__device__ inline void acc_fence(f32x16 (&o)[2][4]) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                 : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]),
                   "+a"(o[1][0]), "+a"(o[1][1]), "+a"(o[1][2]), "+a"(o[1][3]));
}
// acc *= alpha, register by register inside asm (the caller fences around).
__device__ inline void acc_scale(f32x16& acc, float alpha) {
#pragma unroll
    for (int r = 0; r < 16; r += 4) {
        float t;
        asm volatile(
            "v_accvgpr_read_b32 %4, %0\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %0, %4\n\t"
            "v_accvgpr_read_b32 %4, %1\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %1, %4\n\t"
            "v_accvgpr_read_b32 %4, %2\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %2, %4\n\t"
            "v_accvgpr_read_b32 %4, %3\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %3, %4"
            : "+a"(acc[r]), "+a"(acc[r + 1]), "+a"(acc[r + 2]), "+a"(acc[r + 3]), "=&v"(t)
            : "v"(alpha));
    }
}
// acc = 0 inside asm: eight MFMAs with zero operands and a zero accumulator
// (one issue slot each, where 128 v_accvgpr_write stall the item start).  The
// leading s_nop covers the wait states between a VALU write of the zero
// operand and its read by the MFMA.  The first readers of these registers are
// unit 1's P.V MFMAs and, after unit 0's score MFMAs and their explicit waits,
// the VALU (rescale, epilogue), so the 8-pass latency needs no wait of its own.
__device__ inline void acc_zero(f32x16 (&o)[2][4]) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    asm volatile(
        "s_nop 4\n\t"
        "v_mfma_f32_32x32x16_bf16 %0, %8, %8, 0\n\tv_mfma_f32_32x32x16_bf16 %1, %8, %8, 0\n\t"
        "v_mfma_f32_32x32x16_bf16 %2, %8, %8, 0\n\tv_mfma_f32_32x32x16_bf16 %3, %8, %8, 0\n\t"
        "v_mfma_f32_32x32x16_bf16 %4, %8, %8, 0\n\tv_mfma_f32_32x32x16_bf16 %5, %8, %8, 0\n\t"
        "v_mfma_f32_32x32x16_bf16 %6, %8, %8, 0\n\tv_mfma_f32_32x32x16_bf16 %7, %8, %8, 0"
        : "=a"(o[0][0]), "=a"(o[0][1]), "=a"(o[0][2]), "=a"(o[0][3]), "=a"(o[1][0]), "=a"(o[1][1]),
          "=a"(o[1][2]), "=a"(o[1][3])
        : "v"(z));
}

// Keys of a 32-key unit at or beyond kvalid get -inf.  Register r holds key
// 8 (r / 4) + 4 hb + r % 4; groups of four registers valid for every lane are
// skipped by a uniform test.
__device__ inline void mask_unit(f32x16 (&s)[2], int kvalid, int hb) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
        if (8 * g + 8 <= kvalid) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool ok = 8 * g + 4 * hb + j < kvalid;
#pragma unroll
            for (int qb = 0; qb < 2; qb++) s[qb][4 * g + j] = ok ? s[qb][4 * g + j] : -INFINITY;
        }
    }
}

// A work item as planned on the host (two int4 per item, in slot order):
// {h | w << 8, first query tile, second query tile (-1: none), cumf[w]},
// {first video tile of w, video tiles of w, first text tile, f_w}.
struct Work {
    int h, w, q0, q1, g0, vbase, nvt, tbase, f;
};
// The descriptors are read through the constant address space, so that the
// uniform loads become scalar loads, waited on by lgkmcnt rather than by the
// vector-memory counter that also counts the output stores.
typedef __attribute__((address_space(4))) const int32_t cint32;
__device__ inline Work load_work(cint32* d, int i) {
    cint32* e = d + 8 * i;
    return Work{e[0] & 255, e[0] >> 8, e[1], e[2], e[3], e[4], e[5], e[6], e[7]};
}

__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(1, 1)))
void sdpa_bf16_kernel(SdpaArgs a) {
    __shared__ __align__(16) uint16_t lds[5 * KT_E];  // K ring (3 tile slots), V^T ring (2 slots)
    const int wi0 = a.sched_start[blockIdx.x], wi1 = a.sched_start[blockIdx.x + 1];
    if (wi0 >= wi1) return;
    cint32* desc = (cint32*)(a.sched_desc);

    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = lane & 31, hb = lane >> 5;
    const size_t head_stride = (size_t)a.n_tiles * KT_E;

    // DMA lane offsets.  K: instruction i of a wave fills the 1 KiB of rows
    // 32 wave + 4 i .. +3; the lane at physical chunk lane % 16 of row
    // 32 wave + 4 i + lane / 16 fetches logical chunk (lane % 16) ^ (row & 15).
    // row & 15 = 4 (i & 3) + lane / 16, so instruction i + 4 is instruction i
    // shifted by 16 rows.  koff[i]: the lane's byte offset within the tile
    // less the instruction offset 1024 i that dma4_k adds.
    uint32_t koff[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = 32 * wave + 4 * i + (lane >> 4);
        koff[i] = 2 * (row * HEAD_D + (((lane & 15) ^ (row & 15)) << 3)) - 1024 * i;  // >= 0: row >= 4 i
    }
    // V tiles in LDS: 64 key rows of 256 bytes, the 16-byte chunk c of row r
    // at physical chunk c ^ vsw(r & 3), vsw = 0, 6, 10, 12.  Instruction j of
    // wave w fills rows 32 w + 4 j .. +3 (row & 3 = lane / 16), so a lane
    // always fetches logical chunk (lane % 16) ^ vsw(lane / 16) of its row;
    // the row's byte offset in the source comes from the geometry's row table
    // (awa_geom::d_vrow), eight per lane and tile.  With this swizzle each group
    // of 16 (and of 32) lanes of a transposed read below touches distinct banks.
    auto vsw = [](int r) __attribute__((always_inline)) { return ((r & 1) ? 6 : 0) ^ ((r & 2) ? 10 : 0); };
    const uint32_t vlane = 16u * (uint32_t)((lane & 15) ^ vsw(lane >> 4));
    // Transposed reads (ds_read_b64_tr_b16): within each 16-lane group G,
    // output lane 16 G + 4 a + b receives as element i element b of the 8 bytes
    // addressed by lane 16 G + 4 i + a.  Read r of fragment (c2, d-tile dt)
    // of a unit must give lane (n, hb) element i = V[key 16 c2 + 8 r + 4 hb +
    // i][d 32 dt + n] (the key order of the P^T operand), so lane 16 G + 4 i + a
    // addresses key row 16 c2 + 8 r + 4 (G >> 1) + i, channels 32 dt +
    // 16 (G & 1) + 4 a .. +3.  vtr[dt]: that address within a tile for
    // c2 = r = 0 (byte offset; the unit, c2 and r add multiples of 256).
    int vtr[4];
    {
        const int G = lane >> 4, i = (lane >> 2) & 3, aa = lane & 3;
        const int x = 2 * (G & 1) + (aa >> 1);
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
            vtr[dt] = 256 * (4 * (G >> 1) + i) + 16 * ((4 * dt + x) ^ vsw(i)) + 8 * (aa & 1);
    }
    const uint32_t lds_base = (uint32_t)(uintptr_t)(lptr_t)lds;
    // tile index of key tile kk of work item W (packed K)
    auto tile_of = [&](const Work& W, int kk) __attribute__((always_inline)) {
        return stream_tile(kk, W.nvt, W.vbase, W.tbase, a.ntt);
    };
    // The DMA stream of a slot is the key tiles of its items in order: tile kk
    // of an item fetches K tile kk + 2 and V^T tile kk + 1 of the stream, which
    // past the item's end are the next item's first tiles (stream_fetch; an
    // item has at least two key tiles, stream_tiles).  Past the slot's last item a
    // tile fetches its own tile again into the free slot, so that every tile
    // issues the same instructions (the kernel waits for these before it
    // ends; those fetches get empty buffers, whose loads write zeros without
    // touching memory).  A tile's fetch: K tile buffer dk_r into LDS byte
    // address dk_m, V^T rows (offsets vo) of buffer dv_r into dv_m.
    __amdgpu_buffer_rsrc_t dk_r, dv_r;
    uint32_t dk_m = 0, dv_m = 0;
    auto set_k = [&](int h, int tile, int slot, bool real) __attribute__((always_inline)) {
        dk_r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(a.Kp) + h * head_stride + (size_t)tile * KT_E), 0,
            real ? 2 * KT_E : 0, 0x00020000);
        dk_m = lds_base + 2 * (slot * KT_E + wave * (KT_E / 2));
    };
    // V^T of head h from the video or the text rows (the buffer starts 3 KiB
    // early, so that the lane offsets of prep_v stay positive)
    auto set_v = [&](int h, bool txt, int slot, bool real) __attribute__((always_inline)) {
        const uint32_t col = 2 * (2 * DIM + h * HEAD_D) - 3072;
        dv_r = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(static_cast<const char*>(txt ? a.tsrc : a.vsrc)) + col,
                                                 0, real ? (txt ? a.tsrc_bytes : a.vsrc_bytes) - col : 0, 0x00020000);
        dv_m = lds_base + 2 * ((3 + slot) * KT_E + wave * (KT_E / 2));
    };
    // Row offsets of the next V tile to fetch (vt0: instructions 0-3, vt1:
    // 4-7), loaded one tile ahead with ordinary loads, so that the compiler
    // waits for them before any use.  prep_v turns them into this tile's DMA
    // offsets at the start of a tile, before the tile issues any DMA of its
    // own, so that this wait never waits for those.
    u32x4 vt0, vt1;
    uint32_t vo[8];
    auto vtile_of = [&](const Work& W, int kk) __attribute__((always_inline)) {
        return stream_tile(kk, W.nvt, W.vbase, a.n_vid_tiles, a.ntt);
    };
    auto load_vt = [&](int vtile) __attribute__((always_inline)) {
        const u32x4* p = reinterpret_cast<const u32x4*>(a.vrow + (size_t)vtile * TILE + wave * 32 + (lane >> 4) * 8);
        vt0 = p[0];
        vt1 = p[1];
    };
    auto prep_v = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            vo[j] = (vt0[j] << 1) + vlane + (3072u - 1024u * j);
            vo[4 + j] = (vt1[j] << 1) + vlane + (3072u - 1024u * j);
        }
        asm volatile("" : "+v"(vo[0]), "+v"(vo[1]), "+v"(vo[2]), "+v"(vo[3]), "+v"(vo[4]), "+v"(vo[5]),
                          "+v"(vo[6]), "+v"(vo[7]));
    };
    auto wait_vmem = [&]() __attribute__((always_inline)) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
    // instruction i (0-7) of the K and of the V^T fetch
    // instruction i (0-7) of the K fetch, then of the V^T fetch, with the M0
    // write each fourth one needs issued after the one before
    auto dma_k_i = [&](int i) __attribute__((always_inline)) {
        dma1_k(i & 3, dk_r, i < 4 ? 0u : 4096u, koff[i & 3]);
        if (i == 3) m0_set(dk_m + 4096);
        if (i == 7) m0_set(dv_m);
    };
    auto dma_v_i = [&](int i) __attribute__((always_inline)) {
        dma1_v(i & 3, dv_r, vo[i]);
        if (i == 3) m0_set(dv_m + 4096);
    };
    auto dma_k_all = [&]() __attribute__((always_inline)) {
        dma_k8(dk_r, koff, dk_m);
    };
    auto dma_v_all = [&]() __attribute__((always_inline)) {
        dma4_vrow(dv_r, vo[0], vo[1], vo[2], vo[3], dv_m);
        dma4_vrow(dv_r, vo[4], vo[5], vo[6], vo[7], dv_m + 4096);
    };
    // B operand of S^T = K Q^T for column block qb, k-step s:
    // Q[slot 32 qb + n][16 s + 8 hb .. +8]
    bf16x8 qf[2][8];
    // Output rows of this wave's two query columns, fetched with the query tile
    // so that the epilogue has no dependent loads: a video row goes to token
    // vidx[...] of vattn, a text row to the window's partial sums; -1: padding.
    int orow[2] = {-1, -1};
    // The fragments are loaded on every path (an idle wave loads its
    // partner's tile and leaves orow at -1), so that the new fragments can
    // take the registers of the dead ones: a conditional load keeps the old
    // values alive, and the register copies that follows wait for the load.
    auto load_q = [&](const Work& W) __attribute__((always_inline)) {
        const int kq = wave == 0 ? W.q0 : W.q1;
        const int kql = kq < 0 ? W.q0 : kq;
        const int nvq = kq < 0 ? 0
                      : kq < W.nvt ? min(TILE, W.f - TILE * kq) : min(TILE, a.txt_len - TILE * (kq - W.nvt));
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            const int slot = 32 * qb + n;
            orow[qb] = -1;
            if (slot < nvq) orow[qb] = kq < W.nvt ? a.vidx[W.g0 + TILE * kq + slot] : TILE * (kq - W.nvt) + slot;
        }
        const uint16_t* qt = reinterpret_cast<const uint16_t*>(a.Qp) + W.h * head_stride +
                             (size_t)tile_of(W, kql) * KT_E + 8 * hb;
        // Loaded by asm straight into the fragment registers: the compiler
        // neither waits for these loads where it would copy them (it sees
        // no load) nor may it move them; the wait for them is the item
        // start's s_waitcnt vmcnt(0).
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            const uint16_t* row = qt + (32 * qb + n) * HEAD_D;
#pragma unroll
            for (int s = 0; s < 8; s++)
                asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=a"(qf[qb][s]) : "v"(row), "n"(32 * s));
        }
    };

    // LDS fragment addresses.  K fragment (k-step s) of a unit: row n of the
    // unit, chunk 2 s + hb (rows 32 apart share the swizzle).
    int kadr[8];
#pragma unroll
    for (int s = 0; s < 8; s++) kadr[s] = n * HEAD_D + (((2 * s + hb) ^ (n & 15)) << 3);

    Work cur = load_work(desc, wi0);
    int kb = 0, vb = 0;  // ring slots of the current item's key tile 0
    // the stream's first K tiles and V^T tile, then the row offsets of the
    // V^T tile that tile 0 fetches
    load_vt(vtile_of(cur, 0));
    prep_v();
    set_k(cur.h, tile_of(cur, 0), 0, true);
    dma_k_all();
    set_k(cur.h, tile_of(cur, 1), 1, true);
    dma_k_all();
    set_v(cur.h, 0 >= cur.nvt, 0, true);
    dma_v_all();
    load_vt(vtile_of(cur, 1));
    load_q(cur);

    for (int wi = wi0; wi < wi1; wi++) {
        const bool has_next = wi + 1 < wi1;
        const Work nxt = load_work(desc, has_next ? wi + 1 : wi);
        const int orow_cur[2] = {orow[0], orow[1]};
        const int nk = stream_tiles(cur.nvt, a.ntt);
        const int kq = wave == 0 ? cur.q0 : cur.q1;
        const bool active = kq >= 0;
        auto nvalid = [&](int kk) __attribute__((always_inline)) {
            return kk < cur.nvt ? min(TILE, cur.f - TILE * kk) : min(TILE, a.txt_len - TILE * (kk - cur.nvt));
        };
        auto k_ofs = [&](int u) __attribute__((always_inline)) {  // K rows of unit u
            return ((kb + (u >> 1)) % 3) * KT_E + (u & 1) * 32 * HEAD_D;
        };
        auto unit_kv = [&](int u) __attribute__((always_inline)) {  // valid keys, <= 0: none
            return nvalid(u >> 1) - 32 * (u & 1);
        };

        f32x16 oacc[2][4];
        // scores relative to m of the current unit (later its exponentials) and
        // of the next one: unit u reads sc[u & 1] and writes sc[(u + 1) & 1]
        f32x16 sc[2][2];
        bf16x8 bfr[2];      // bias fragments (-m)
        float m_i[2] = {0.f, 0.f}, l_i[2] = {0.f, 0.f}, mtc[2] = {0.f, 0.f};
        acc_zero(oacc);

        // the query fragments arrive by asm loads: the wait names them, so
        // nothing reads them before it
        asm volatile("s_waitcnt vmcnt(0)"
                     : "+a"(qf[0][0]), "+a"(qf[0][1]), "+a"(qf[0][2]), "+a"(qf[0][3]),
                       "+a"(qf[0][4]), "+a"(qf[0][5]), "+a"(qf[0][6]), "+a"(qf[0][7]), "+a"(qf[1][0]),
                       "+a"(qf[1][1]), "+a"(qf[1][2]), "+a"(qf[1][3]), "+a"(qf[1][4]), "+a"(qf[1][5]),
                       "+a"(qf[1][6]), "+a"(qf[1][7])
                     :
                     : "memory");
        __syncthreads();

        // K fragments of the next unit's score MFMAs, read a phase ahead
        bf16x8 kfn[8];
        // Unit 0: raw scores, m = their row maximum (rounded to bf16), scores
        // relative to m.
        if (active) {
            f32x16 s0[2];
            bf16x8 kf[8];
            const int ko = k_ofs(0), ko1 = k_ofs(1);
#pragma unroll
            for (int st = 0; st < 8; st++) kf[st] = *reinterpret_cast<const bf16x8*>(lds + ko + kadr[st]);
#pragma unroll
            for (int st = 0; st < 8; st++) ds_read_kf(kfn[st], lds_base + 2 * (ko1 + kadr[st]));
#pragma unroll
            for (int st = 0; st < 8; st++)
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    if (st == 0) qk_zero(s0[qb], kf[0], qf[qb][0]);
                    else qk_only(s0[qb], kf[st], qf[qb][st]);
                }
            mfma_fence_v(s0);
            const int kv0 = unit_kv(0);
            if (kv0 < 32) mask_unit(s0, kv0, hb);
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                float mx = fmaxf(s0[qb][0], s0[qb][1]);
#pragma unroll
                for (int r = 2; r < 16; r++) mx = fmaxf(mx, s0[qb][r]);
                m_i[qb] = bf16_round(max_pair(mx));  // finite: unit 0 has a valid key
                bfr[qb] = bias_frag(m_i[qb], hb);
#pragma unroll
                for (int r = 0; r < 16; r++) sc[0][qb][r] = s0[qb][r] - m_i[qb];
            }
        }

        int nv_tile = 0;  // V^T tile whose row offsets the current tile loads
        // One unit: phases A and B as described above.
        // dma: the unit also issues its tile's fetch, one DMA instruction per
        // score MFMA from the third on (K, then V^T, then the next row
        // offsets): a 1 KiB instruction occupies the CU's address unit for 16
        // cycles, so issued back to back they would stall the wave, while one
        // per 32-cycle MFMA goes through without a stall.
        auto unit = [&](int u, bool has_succ, bool dma, bool pf) __attribute__((always_inline)) {
            // ---- stale-maximum rule for this unit's scores (mtc: their row max relative to m)
            if (__any(mtc[0] > RESCALE_LOG2 || mtc[1] > RESCALE_LOG2)) {
                float alpha[2];
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    // new m: a bf16 value at or above the unit maximum
                    const float mn = mtc[qb] > 0.f ? bf16_round(m_i[qb] + mtc[qb]) : m_i[qb];
                    const float up = mn - m_i[qb];
                    alpha[qb] = __builtin_amdgcn_exp2f(-up);
                    m_i[qb] = mn;
                    bfr[qb] = bias_frag(mn, hb);
                    l_i[qb] *= alpha[qb];
#pragma unroll
                    for (int r = 0; r < 16; r++) sc[u & 1][qb][r] -= up;
                }
                acc_fence(oacc);
#pragma unroll
                for (int qb = 0; qb < 2; qb++)
#pragma unroll
                    for (int dt = 0; dt < 4; dt++) acc_scale(oacc[qb][dt], alpha[qb]);
                acc_fence(oacc);
            }
            // V^T fragments of this unit (loaded once half of the K fragments
            // are dead): two transposed reads each, keys 32 (u & 1) + 16 c2 + 8 r.
            lchar_t* vslot = (lchar_t*)lds + 2 * (3 + ((vb + (u >> 1)) & 1)) * KT_E;
            bf16x8 vf[2][4];
            auto load_vf = [&]() __attribute__((always_inline)) {
#pragma unroll
                for (int dt = 0; dt < 4; dt++) {
                    lchar_t* pv = vslot + vtr[dt];
#pragma unroll
                    for (int c2 = 0; c2 < 2; c2++) {
                        const int row = 32 * (u & 1) + 16 * c2;
                        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                            (lbf16x4_t*)(pv + 256 * row));
                        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                            (lbf16x4_t*)(pv + 256 * (row + 8)));
                        vf[c2][dt] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                    }
                }
            };
            f32x16 (&p)[2] = sc[u & 1];  // exponentials in place
            f32x16 (&snx)[2] = sc[(u + 1) & 1];
            float ps[2] = {0.f, 0.f};
            if (has_succ) {
                // ---- phase A: S(u+1) MFMAs with the exponentials of this unit
                const bf16x8 onesm = mask_frag(unit_kv(u + 1), n, hb);
                if (dma) m0_set(dk_m);
                bf16x8 (&kf)[8] = kfn;  // read in the previous phase B (or at the item start)
                asm volatile("s_waitcnt lgkmcnt(0)"
                             : "+a"(kfn[0]), "+a"(kfn[1]), "+a"(kfn[2]), "+a"(kfn[3]), "+a"(kfn[4]),
                               "+a"(kfn[5]), "+a"(kfn[6]), "+a"(kfn[7])
                             :
                             : "memory");
                // 18 slots: slot 0 / 1 are the bias k-steps of blocks 0 / 1, slot
                // j >= 2 k-step (j - 2) / 2 of block j & 1; exponentials two per
                // slot, block 0 in slots 0-7, block 1 in slots 8-15.
#pragma unroll
                for (int j = 0; j < 18; j++) {
                    const int qb = j & 1, st = (j - 2) >> 1;
                    const int eq = j >> 3, er = 2 * (j & 7);
                    if (j < 16) {
                        p[eq][er] = __builtin_amdgcn_exp2f(p[eq][er]);
                        p[eq][er + 1] = __builtin_amdgcn_exp2f(p[eq][er + 1]);
                    }
                    if (j < 2)
                        snx[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(onesm, bfr[qb], f32x16{}, 0, 0, 0);
                    else
                        snx[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[st], qf[qb][st], snx[qb], 0, 0, 0);
                    if (j < 16) __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (j == 3) {
                        load_vf();
                        __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // the V^T reads here
                    }
                    if (dma && j >= 2 && j < 10) dma_k_i(j - 2);
                    if (dma && j >= 10) dma_v_i(j - 10);
                    if (dma && j == 17) load_vt(nv_tile);
                    // the DMA asm belongs to no scheduling group, so the
                    // scheduler would gather the sixteen instructions into a
                    // burst; a full scheduling barrier keeps each at its slot
                    if (dma && j >= 2) __builtin_amdgcn_sched_barrier(0);
                }
                score_fence(snx, p);
            } else {
                load_vf();
#pragma unroll
                for (int qb = 0; qb < 2; qb++)
#pragma unroll
                    for (int r = 0; r < 16; r++) p[qb][r] = __builtin_amdgcn_exp2f(p[qb][r]);
                exp_fence(p);
            }
            // P^T in the B-operand order of O^T += V^T P^T: element i of
            // pb[qb][c2] is register 8 c2 + i of S^T[qb]
            bf16x8 pb[2][2];
#pragma unroll
            for (int qb = 0; qb < 2; qb++)
#pragma unroll
                for (int c2 = 0; c2 < 2; c2++)
#pragma unroll
                    for (int i = 0; i < 8; i++) pb[qb][c2][i] = (__bf16)p[qb][8 * c2 + i];
            // the K fragments of unit u + 2 (the next phase A): one read after
            // each of phase B's first eight MFMAs
            const uint32_t kpf = lds_base + 2 * k_ofs(u + 2);
            auto prefetch_k = [&](int j) __attribute__((always_inline)) {
                if (pf && j < 8) ds_read_kf(kfn[j], kpf + 2 * kadr[j]);
            };
            if (has_succ) {
                // ---- phase B: P.V MFMAs with the row maxima of S(u+1) and the row sums of P(u)
                float mx[2] = {-INFINITY, -INFINITY};
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const int qb = j & 1, dt = (j >> 1) & 3, c2 = j >> 3;  // MFMA
                    const int eq = j >> 3, er = 2 * (j & 7);                // max / sum items
                    max_sum_pv(oacc[qb][dt], vf[c2][dt], pb[qb][c2], mx[eq], snx[eq][er], snx[eq][er + 1],
                               ps[eq], p[eq][er], p[eq][er + 1]);
                    prefetch_k(j);
                }
                mtc[0] = max_pair(mx[0]);
                mtc[1] = max_pair(mx[1]);

            } else {
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const int qb = j & 1, dt = (j >> 1) & 3, c2 = j >> 3;
                    const int eq = j >> 3, er = 2 * (j & 7);
                    sum_pv(oacc[qb][dt], vf[c2][dt], pb[qb][c2], ps[eq], p[eq][er], p[eq][er + 1]);
                    prefetch_k(j);
                }
            }
            l_i[0] += ps[0];
            l_i[1] += ps[1];
        };

        // Tile kk issues the DMA of K(kk+2) and V(kk+1) (the last tile: the
        // next item's first tiles); its second unit ends with the wait for
        // that DMA and a barrier.  The loop body holds one tile (two units, so
        // the current and next score registers alternate without copies); the
        // last tile is peeled because its second unit has no successor.
        auto tile = [&](int kk, bool last) __attribute__((always_inline)) {
            // this tile's fetch (K tile kk + 2 and V^T tile kk + 1 of the
            // stream) and the V^T tile of the next tile's fetch
            // (values, not a choice between the two items' fields: a
            // conditional lvalue keeps both items in scratch memory)
            int k_kk, k_nxt, v_kk, v_nxt;
            stream_fetch(kk, nk, &k_kk, &k_nxt, &v_kk, &v_nxt);
            int kh = cur.h, kt = tile_of(cur, kk), vh = cur.h;
            bool vtxt = kk >= cur.nvt;
            nv_tile = vtile_of(cur, min(kk + 1, nk - 1));
            if (!k_nxt) {
                kt = tile_of(cur, k_kk);
                nv_tile = vtile_of(cur, k_kk);
            } else if (has_next) {
                kh = nxt.h;
                kt = tile_of(nxt, k_kk);
                nv_tile = vtile_of(nxt, k_kk);
            }
            if (!v_nxt) {
                vtxt = v_kk >= cur.nvt;
            } else if (has_next) {
                vh = nxt.h;
                vtxt = v_kk >= nxt.nvt;
            }
            set_k(kh, kt, (kb + kk + 2) % 3, !k_nxt || has_next);
            set_v(vh, vtxt, (vb + kk + 1) & 1, !v_nxt || has_next);
            prep_v();
            if (active) {
                unit(2 * kk, true, true, !last);
            } else {  // an idle wave still fills its half of the tiles
                dma_k_all();
                dma_v_all();
                load_vt(nv_tile);
            }
            // the item's last unit computes no scores: Q is dead, so the
            // next item's query tile loads during it (after the slot's last
            // item: the same tile again, unused)
            if (last) load_q(nxt);
            if (active) unit(2 * kk + 1, !last, false, !last);
            if (!last) {
                wait_vmem();
                __syncthreads();
            }
        };
        for (int kk = 0; kk + 1 < nk; kk++) tile(kk, false);
        tile(nk - 1, true);

        // Item epilogue.  Text rows (fp32 partials) are stored straight from
        // the accumulators.  Video rows go through LDS: once both waves are
        // done with the last tile, its K slot (wave 0) and V slot (wave 1)
        // are free, so each wave writes its normalised bf16 tile there
        // (16-byte chunk c of row r at chunk c ^ (r & 15)) and reads it back
        // as whole 256-byte rows, four rows per store instruction.  Stores of
        // 16-byte pieces of 32 rows each cost the memory system far more than
        // the same bytes in whole lines.  The next item's start (wait and
        // barrier) keeps its DMA out of these slots until both waves have
        // read them back.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (active) {
            acc_fence(oacc);
            float inv[2];
#pragma unroll
            for (int qb = 0; qb < 2; qb++) inv[qb] = 1.f / sum_pair(l_i[qb]);
            if (kq >= cur.nvt) {
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    if (orow_cur[qb] < 0) continue;
                    store_rows<false>(oacc[qb], inv[qb], hb,
                                      a.tpart + ((size_t)cur.w * a.txt_len + orow_cur[qb]) * DIM +
                                          (size_t)cur.h * HEAD_D);
                }
            } else {
                // all token lookups (first, so that their round trips through
                // LDS overlap the staging), then all row reads, then all stores:
                // each group waits once.  Padding rows (token -1) get an offset
                // past the buffer's end, which the buffer store drops, so no
                // lane branches around its store.
                const __amdgpu_buffer_rsrc_t ores =
                    __builtin_amdgcn_make_buffer_rsrc(a.vattn, 0, a.vattn_bytes, 0x00020000);
                const uint32_t col = 2 * ((uint32_t)cur.h * HEAD_D + (lane & 15) * 8);
                uint32_t ofs[16];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int tok = __shfl(orow_cur[i >> 3], (4 * i + (lane >> 4)) & 31);
                    ofs[i] = tok >= 0 ? (uint32_t)tok * (2 * DIM) + col : 0x80000000u;
                }
                uint16_t* stg = lds + (wave == 0 ? (kb + nk - 1) % 3 : 3 + ((vb + nk - 1) & 1)) * KT_E;
                // the lane's swizzle terms, formed here (an opaque copy keeps
                // the compiler from computing the twenty staging addresses
                // once and holding them in registers across the item loop)
                int nn = n, ln = lane;
                asm volatile("" : "+v"(nn), "+v"(ln));
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    const int row = 32 * qb + nn;
#pragma unroll
                    for (int dt = 0; dt < 4; dt++)
#pragma unroll
                        for (int g = 0; g < 4; g++) {
                            const f32x16& o = oacc[qb][dt];
                            const float iv = inv[qb];
                            uint2 u;
                            u.x = pack_bf16x2(o[4 * g] * iv, o[4 * g + 1] * iv);
                            u.y = pack_bf16x2(o[4 * g + 2] * iv, o[4 * g + 3] * iv);
                            const int c = 4 * dt + g;
                            *reinterpret_cast<uint2*>(stg + row * HEAD_D + ((c ^ (row & 15)) << 3) + 4 * hb) = u;
                        }
                }
                u32x4 v[16];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int row = 4 * i + (ln >> 4), c = ln & 15;
                    v[i] = *reinterpret_cast<const u32x4*>(stg + row * HEAD_D + ((c ^ (row & 15)) << 3));
                }
#pragma unroll
                for (int i = 0; i < 16; i++) __builtin_amdgcn_raw_buffer_store_b128(v[i], ores, ofs[i], 0, 0);
            }
        }
        kb = (kb + nk) % 3;
        vb = (vb + nk) & 1;
        cur = nxt;
    }
    wait_vmem();  // the last tiles' fetches and query loads land before the workgroup's LDS is released
}

}  // namespace

hipError_t launch_sdpa(int dtype, const SdpaArgs& a, hipStream_t s) {
    if (dtype != AWA_BF16) return launch_sdpa_f32(a, s);
    hipLaunchKernelGGL(sdpa_bf16_kernel, dim3(a.n_slots), dim3(128), 0, s, a);
    return hipGetLastError();
}

}  // namespace awa

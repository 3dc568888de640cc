// awa_coalesce.hip — cross-window text average and boundary casts.
//
// tattn[i][c] = (sum over windows w, in window order, of tpart[w][i][c]) / nwin
// (dit_vk.cpp:440-444, awa_coalesce.comp:19-29): fp32 sums in the same order
// as the reference, then one division, then the output store (fp32, or bf16
// rounded to nearest even as cast_f32_bf16.comp:24).  HBM-bound.
#include "awa_internal.hpp"

namespace awa {

namespace {

constexpr int CO_BLOCK = 64;  // one wave per workgroup: the loads spread over every CU

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// two floats -> two bf16, round to nearest even (v_cvt_pk_bf16_f32)
__device__ inline uint32_t pk_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// One float4 of [TXT x 2560] per thread.  The loads of up to kBatch windows
// are issued together (window indices past the last clamped to it, so every
// load is unconditional and all are in flight at once: one memory round trip
// for up to kBatch windows, where loads behind a branch each would wait for
// the ones before); the adds then run in window order.  The launch picks the
// smallest batch that holds every window (8, 16 or 32).
template <bool kBf16Out, int kBatch>
__global__ __launch_bounds__(CO_BLOCK) void coalesce_kernel(const float* __restrict__ tpart,
                                                            void* __restrict__ out, int nwin, int n4) {
    const int i = blockIdx.x * CO_BLOCK + threadIdx.x;
    if (i >= n4) return;
    const float4* src = reinterpret_cast<const float4*>(tpart) + i;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int w = 0; w < nwin; w += kBatch) {
        float4 v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; j++) v[j] = src[(size_t)min(w + j, nwin - 1) * n4];
#pragma unroll
        for (int j = 0; j < kBatch; j++) {
            if (w + j < nwin) {  // uniform
                s.x += v[j].x; s.y += v[j].y; s.z += v[j].z; s.w += v[j].w;
            }
        }
    }
    const float fn = (float)nwin;
    s.x /= fn; s.y /= fn; s.z /= fn; s.w /= fn;
    if constexpr (kBf16Out) {
        uint2 u;
        u.x = pk_bf16(s.x, s.y);
        u.y = pk_bf16(s.z, s.w);
        reinterpret_cast<uint2*>(out)[i] = u;
    } else {
        reinterpret_cast<float4*>(out)[i] = s;
    }
}

__global__ __launch_bounds__(256) void cast_f32_bf16_kernel(const float* __restrict__ in,
                                                            uint16_t* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t j = i; j < n; j += stride) out[j] = (uint16_t)bf16x2_rne(in[j], 0.f);
}

__global__ __launch_bounds__(256) void cast_bf16_f32_kernel(const uint16_t* __restrict__ in,
                                                            float* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t j = i; j < n; j += stride) out[j] = __uint_as_float((uint32_t)in[j] << 16);
}

// A fill kernel rather than hipMemsetAsync, so the op stays graph-capturable.
__global__ __launch_bounds__(256) void zero_kernel(uint4* __restrict__ p, size_t n16) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t j = i; j < n16; j += stride) p[j] = make_uint4(0, 0, 0, 0);
}

// Streaming device copy: CP_U 16-byte loads per thread in flight, then CP_U
// nontemporal stores; it sets the HBM ceiling that the memory-bound passes
// are compared with.  Whole blocks take a path with no bounds test, so the
// loads are issued together and waited for once (with a test per load the
// compiler waited for each load before the next); only the last block tests.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int CP_U = 4;
__global__ __launch_bounds__(256) void stream_copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                          size_t n16) {
    const size_t block0 = (size_t)blockIdx.x * CP_U * 256;
    const size_t base = block0 + threadIdx.x;
    u32x4 v[CP_U];
    if (block0 + CP_U * 256 <= n16) {
#pragma unroll
        for (int u = 0; u < CP_U; u++) v[u] = src[base + (size_t)u * 256];
#pragma unroll
        for (int u = 0; u < CP_U; u++) __builtin_nontemporal_store(v[u], dst + base + (size_t)u * 256);
        return;
    }
#pragma unroll
    for (int u = 0; u < CP_U; u++) {
        const size_t i = base + (size_t)u * 256;
        if (i < n16) v[u] = src[i];
    }
#pragma unroll
    for (int u = 0; u < CP_U; u++) {
        const size_t i = base + (size_t)u * 256;
        if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
    }
}

inline unsigned grid_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b < 1) b = 1;
    if (b > 65535) b = 65535;
    return (unsigned)b;
}

template <bool kBf16Out>
void launch_coalesce_t(const float* tpart, void* tattn, int nwin, int n4, unsigned blocks, hipStream_t s) {
    if (nwin <= 8)
        hipLaunchKernelGGL((coalesce_kernel<kBf16Out, 8>), dim3(blocks), dim3(CO_BLOCK), 0, s, tpart, tattn, nwin, n4);
    else if (nwin <= 16)
        hipLaunchKernelGGL((coalesce_kernel<kBf16Out, 16>), dim3(blocks), dim3(CO_BLOCK), 0, s, tpart, tattn, nwin, n4);
    else
        hipLaunchKernelGGL((coalesce_kernel<kBf16Out, 32>), dim3(blocks), dim3(CO_BLOCK), 0, s, tpart, tattn, nwin, n4);
}

}  // namespace

hipError_t launch_coalesce(int dtype, const float* tpart, void* tattn, int nwin, int txt_len,
                           hipStream_t s) {
    const int n4 = txt_len * DIM / 4;
    const unsigned blocks = (unsigned)((n4 + CO_BLOCK - 1) / CO_BLOCK);
    if (blocks == 0 || nwin <= 0) return hipSuccess;
    if (dtype == AWA_BF16) launch_coalesce_t<true>(tpart, tattn, nwin, n4, blocks, s);
    else launch_coalesce_t<false>(tpart, tattn, nwin, n4, blocks, s);
    return hipGetLastError();
}

hipError_t launch_cast_f32_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(cast_f32_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, out, n);
    return hipGetLastError();
}

hipError_t launch_cast_bf16_f32(const uint16_t* in, float* out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(cast_bf16_f32_kernel, dim3(grid_for(n)), dim3(256), 0, s, in, out, n);
    return hipGetLastError();
}

hipError_t launch_stream_copy(void* dst, const void* src, size_t bytes, hipStream_t s) {
    const size_t n16 = bytes / 16;  // callers pass multiples of 16 bytes
    if (n16 == 0) return hipSuccess;
    const size_t blocks = (n16 + CP_U * 256 - 1) / (CP_U * 256);
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, s, reinterpret_cast<u32x4*>(dst),
                       reinterpret_cast<const u32x4*>(src), n16);
    return hipGetLastError();
}

hipError_t launch_zero(void* p, size_t bytes, hipStream_t s) {
    const size_t n16 = bytes / 16;  // callers pass multiples of 16 bytes
    if (n16 == 0) return hipSuccess;
    hipLaunchKernelGGL(zero_kernel, dim3(grid_for((int64_t)n16)), dim3(256), 0, s,
                       reinterpret_cast<uint4*>(p), n16);
    return hipGetLastError();
}

}  // namespace awa

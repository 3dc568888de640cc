// awa_noalloc.hip — the AWA op without any device allocation.
//
// awa_forward_noalloc runs the same kernels as awa_forward (pack, window
// attention, text average), but its scratch (packed q/k/v tiles and the
// per-window text partials) is the file-scope device array `scratch` below,
// of a fixed size, instead of the context's buffer that awa_forward grows
// with hipMalloc.  It is for callers that cannot allocate: code under HIP
// graph capture, tight serving loops, harnesses that forbid allocation.
//
// Every device that loads this library holds its own copy of the array until
// the process ends.  Host code never passes the array's name to a kernel (on
// the host that name is only a stand-in, not a device address): awa_create
// looks up the current device's address once with hipGetSymbolAddress, and
// that pointer is what the kernels receive.  The kernels overwrite every byte
// they later read (padding rows of the packed tiles are written as zeros,
// every window writes all of its text partial rows), so nothing needs
// clearing between calls.  All calls on one device share the array: calls
// that overlap in time on one device, on any streams or contexts, race.
#include <mutex>

#include "awa_internal.hpp"

constexpr size_t kScratchBytes = (size_t)AWA_NOALLOC_SCRATCH_MIB << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_mu;

}  // namespace

namespace awa {

hipError_t noalloc_resolve(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_scratch_ptr[device]) return hipSuccess;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) g_scratch_ptr[device] = p;
    return e;
}

void* noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    return g_scratch_ptr[device];
}

}  // namespace awa

using namespace awa;

extern "C" int awa_forward_noalloc(awa_ctx* ctx, const awa_geom* g, int dtype, const void* d_vqkv,
                                   const void* d_tqkv, int Lv, int TXT, const float* d_nq_v,
                                   const float* d_nk_v, const float* d_nq_t, const float* d_nk_t,
                                   float eps, void* d_vattn, void* d_tattn, awa_stream_t stream) {
    const int rc = check_forward_args("awa_forward_noalloc", ctx, g, dtype, d_vqkv, d_tqkv, Lv, TXT,
                                      d_nq_v, d_nk_v, d_nq_t, d_nk_t, eps, d_vattn, d_tattn);
    if (rc != AWA_OK) return rc;
    const size_t need = op_scratch_bytes(g->plan, dtype);
    if (need > kScratchBytes) {
        set_err(ctx,
                "awa_forward_noalloc: this geometry needs %zu bytes of scratch (%s storage); the "
                "allocation-free entry holds at most %zu (use awa_forward)",
                need, dtype == AWA_BF16 ? "bf16" : "fp32", kScratchBytes);
        return AWA_EARG;
    }
    if (ctx->noalloc_status != hipSuccess) {
        set_err(ctx, "awa_forward_noalloc: scratch lookup failed at awa_create: %s",
                hipGetErrorString(ctx->noalloc_status));
        return AWA_EHIP;
    }
    void* p = noalloc_scratch(ctx->device);
    if (!p) {
        set_err(ctx, "awa_forward_noalloc: no scratch address for device %d", ctx->device);
        return AWA_EHIP;
    }
    DeviceGuard dg(ctx->device);
    return forward_impl(ctx, g, dtype, d_vqkv, d_tqkv, d_nq_v, d_nk_v, d_nq_t, d_nk_t, eps, d_vattn,
                        d_tattn, reinterpret_cast<hipStream_t>(stream), p);
}

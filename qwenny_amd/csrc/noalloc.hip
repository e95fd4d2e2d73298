// The allocation-free product entry point (qh_gemm_noalloc): qh_gemm with its launch scratch in a file-scope device
// array instead of the context's allocations, for callers that cannot allocate device memory around a product (code
// under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The array holds, in this order, the argmax table (ARGMAX_SCRATCH_BYTES), the prefill's
// stream-K partials and item counters (PF_SK_SCRATCH_BYTES) and the f16 activations of prefill launches with f16
// operands (X16_SCRATCH_BYTES): the same scratch qh_open allocates per context, so both
// entry points make the same launch plans and the same results. Every GPU the library runs on holds its own copy
// until the process ends. In host code `scratch` names a host-side stand-in, not device memory: its device address on
// each GPU is resolved once per device by noalloc_init (called by qh_open with the device current) and only that
// address is ever passed to kernels or memory operations.
//
// Every launch leaves the counters and the table at zero, so consecutive calls start clean; calls that overlap on one
// GPU (two streams, two threads, two contexts on the same device) share the array and race.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "gemm.h"
#include "internal.h"

namespace qh {

constexpr size_t NOALLOC_ARGMAX_OFF = 0;
constexpr size_t NOALLOC_SK_OFF = (ARGMAX_SCRATCH_BYTES + 255) & ~(size_t)255;
constexpr size_t NOALLOC_X16_OFF = NOALLOC_SK_OFF + PF_SK_SCRATCH_BYTES;
constexpr size_t NOALLOC_BYTES = NOALLOC_X16_OFF + X16_SCRATCH_BYTES;  // 160 MiB + 48.25 KiB

static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

constexpr int MAX_DEVICES = 64;
// device address of `scratch` on each device, null until set up: stored (release) under scratch_mu once the array is
// cleared, read (acquire) without the lock by every call
static std::atomic<void*> scratch_ptr[MAX_DEVICES];
static std::mutex scratch_mu;

int noalloc_init(int device) {
    if (device < 0 || device >= MAX_DEVICES) return fail(QH_EINVAL, "no-alloc scratch: device %d", device);
    std::lock_guard<std::mutex> g(scratch_mu);
    if (scratch_ptr[device].load(std::memory_order_acquire)) return QH_OK;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(QH_EHIP, "no-alloc scratch on device %d: hipGetSymbolAddress: %s", device, hipGetErrorString(e));
    // the table and every counter start at zero (launches leave them so): clear the counters, not the 128 MiB of
    // partials, which are written before they are read
    e = hipMemset((uint8_t*)ptr + NOALLOC_ARGMAX_OFF, 0, ARGMAX_SCRATCH_BYTES);
    if (e == hipSuccess)
        e = hipMemset((uint8_t*)ptr + NOALLOC_SK_OFF + PF_SK_PART_BYTES, 0, PF_SK_SCRATCH_BYTES - PF_SK_PART_BYTES);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(QH_EHIP, "no-alloc scratch on device %d: clear: %s", device, hipGetErrorString(e));
    scratch_ptr[device].store(ptr, std::memory_order_release);
    return QH_OK;
}

}  // namespace qh

using namespace qh;

extern "C" int qh_gemm_noalloc(qh_ctx* ctx, void* stream, const qh_mat* w, const void* x, size_t ldx, size_t n,
                               const int32_t* out_rows, size_t n_out, void* y, int epi, uint64_t* keys, int whole) {
    if (!ctx) return fail(QH_EINVAL, "gemm (no-alloc): null");
    const int device = ctx_device(ctx);
    void* ptr = device >= 0 && device < MAX_DEVICES ? scratch_ptr[device].load(std::memory_order_acquire) : nullptr;
    if (!ptr) return fail(QH_EINVAL, "gemm (no-alloc): scratch of device %d not set up (qh_open)", device);
    return gemm_with_scratch(ctx, stream, w, x, ldx, n, out_rows, n_out, y, epi, keys, whole,
                             Scratch{(uint8_t*)ptr + NOALLOC_ARGMAX_OFF, (uint8_t*)ptr + NOALLOC_SK_OFF,
                                     (uint8_t*)ptr + NOALLOC_X16_OFF});
}

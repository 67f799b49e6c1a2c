// noalloc.hip -- mi_gemm_f32_noalloc: mi_gemm_f32 for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  The scratch mi_gemm_f32's kernels use
// (split-K partial tiles, stream-K partial tiles, packed operand copies: the
// caller's workspace) is here a file-scope device array of fixed size
// instead, so a call allocates nothing.
//
// The array's name is a host-side stand-in, not a device address: its
// address on the current device comes from hipGetSymbolAddress, looked up
// once per device (with that device current) on the first call there and
// kept; only that pointer is ever handed to kernels.  Each device holds its
// own copy of the array for the life of the process.
//
// Every call on one device shares that device's array and leaves the last
// call's partials in it: calls that overlap on one device (different
// streams, or host threads, without ordering between them) race.  Nothing in
// it needs to start at zero -- every split writes each of its partial tiles
// whole before the fixed-order reduction reads them.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "../../include/mi355_gemm.h"

// 64 MiB: the BASELINE large-K product (256 x 256, K = 2^20) takes 256 splits
// of a 256 KiB partial, exactly this much.
static constexpr size_t kScratchBytes = MI_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "whole 256-byte lines");

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];  // device address of `scratch`, per device
std::mutex g_lookup;

// Device address of this device's copy of `scratch` (looked up on first use).
int scratch_on_current_device(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MI_ERR_NO_DEVICE;
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_lookup);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return (int)e;
            if (p == nullptr) return MI_ERR_NO_DEVICE;
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return MI_OK;
}

}  // namespace

extern "C" {

int mi_gemm_f32_noalloc(const mi_gemm_args* args, void* stream) {
    if (!args) return MI_ERR_NULL_POINTER;
    mi_gemm_args a = *args;
    a.workspace = nullptr;
    a.workspace_bytes = 0;
    // The plan mi_gemm_f32 uses with a workspace of mi_gemm_workspace_bytes:
    // the same kernels, split and reduction order, so the same result bit
    // for bit.  (0 for an invalid problem: mi_gemm_f32 reports it below.)
    const size_t need = mi_gemm_workspace_bytes(&a);
    void* ws = nullptr;
    int rc = scratch_on_current_device(&ws);
    if (rc != MI_OK) return rc;
    if (need <= kScratchBytes) {
        a.workspace = need ? ws : nullptr;
        a.workspace_bytes = need;
        return mi_gemm_f32(&a, stream);
    }
    // The preferred plan wants more scratch than the array holds: plan with
    // the array as the workspace limit instead.  The planner then picks among
    // the plans that fit (fewer splits, stream-K, no packed copies, ...; an
    // unsplit plan needing none always exists), so the result may differ from
    // mi_gemm_f32's with its preferred workspace in the last bits.  Only a
    // plan_override that forces a plan needing more is refused, before any
    // launch.
    a.workspace = ws;
    a.workspace_bytes = kScratchBytes;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return MI_ERR_NO_DEVICE;
    mi_plan p{};
    rc = mi_gemm_plan(&a, cus, &p);
    if (rc != MI_OK) return rc;
    if (p.workspace_bytes > kScratchBytes) return MI_ERR_SCRATCH_LIMIT;
    return mi_gemm_f32(&a, stream);
}

}  // extern "C"

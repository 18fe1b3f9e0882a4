// mpattn_fwd_noalloc: the forward for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). It has no counterpart in the reference. It runs the
// kernels of mpattn_fwd with the workspace in a static device array instead
// of a caller buffer, and calls no allocating routine.
#include <stdio.h>

#include <mutex>

#include "mpattn_common.h"

namespace mpattn {
int api_validate_fwd(const mpattn_fwd_params* p);
int api_launch_fwd(const mpattn_fwd_params& p, void* stream);
void api_clear_error();
int api_fail(int code, const char* msg);
int64_t fwd_workspace_bytes(int B, int H, int L, int D, int dtype, int rope);
}  // namespace mpattn

namespace {

// The forward's workspace for mpattn_fwd_noalloc. Each GPU the library runs
// on holds its own copy for the life of the process. On the host the array's
// name only stands in for the symbol and is never passed to a kernel: the
// device address comes from hipGetSymbolAddress, looked up once per device
// with that device current, and is kept in g_scratch.
constexpr int64_t kScratchBytes = MPATTN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

int failf(int code, const char* fmt, long long a, long long b, const char* s) {
    char msg[384];
    snprintf(msg, sizeof(msg), fmt, a, b, s);
    return mpattn::api_fail(code, msg);
}

// Device address of `scratch` on the device that runs `stream`.
int scratch_ptr(hipStream_t stream, void** out) {
    int dev = 0;
    hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess)
        return failf(MPATTN_ERR_LAUNCH, "scratch: no device for the stream (%lld, %lld): %s", 0, 0,
                     hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return failf(MPATTN_ERR_UNSUPPORTED, "scratch: device %lld outside 0..%lld%s", dev, kMaxDevices - 1, "");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        int cur = 0;
        if ((e = hipGetDevice(&cur)) != hipSuccess)
            return failf(MPATTN_ERR_LAUNCH, "scratch: hipGetDevice (%lld, %lld): %s", 0, 0, hipGetErrorString(e));
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
            return failf(MPATTN_ERR_LAUNCH, "scratch: hipSetDevice(%lld) (%lld): %s", dev, 0, hipGetErrorString(e));
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || !ptr)
            return failf(MPATTN_ERR_LAUNCH, "scratch: hipGetSymbolAddress on device %lld (%lld): %s", dev, 0,
                         hipGetErrorString(e));
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return MPATTN_OK;
}

}  // namespace

extern "C" int mpattn_fwd_noalloc(const mpattn_fwd_params* p, void* stream) {
    mpattn::api_clear_error();
    int rc = mpattn::api_validate_fwd(p);
    if (rc) return rc;
    const int64_t need = mpattn::fwd_workspace_bytes(p->B, p->H, p->L, p->D, p->dtype, p->rope);
    if (need > kScratchBytes)
        return failf(MPATTN_ERR_UNSUPPORTED,
                     "mpattn_fwd_noalloc: this shape needs %lld bytes of scratch, more than the "
                     "%lld-byte static scratch (MPATTN_NOALLOC_SCRATCH_BYTES)%s; use mpattn_fwd",
                     (long long)need, (long long)kScratchBytes, "");
    void* ws = nullptr;
    if ((rc = scratch_ptr((hipStream_t)stream, &ws))) return rc;
    // Every workspace entry the kernels read is written earlier in the same
    // call (by the prep kernel), so the previous call's contents need no
    // clearing. Calls that overlap on one GPU share the array and race.
    mpattn_fwd_params q = *p;
    q.workspace = ws;
    q.workspace_bytes = kScratchBytes;
    return mpattn::api_launch_fwd(q, stream);
}

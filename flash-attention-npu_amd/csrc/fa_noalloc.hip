// fa_noalloc.hip -- fa_mha_fwd_kvcache_noalloc: the kvcache forward for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc). It has no counterpart in
// the reference.
//
// The kernels' scratch (the split plan, the split-KV partial rows and, for
// decode with rotary, the rotated q) lives in `scratch`, a file-scope device
// array of FA_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds
// until the process ends. Host code never passes the array's name to a kernel
// (on the host that name is only a stand-in, not a device address): the first
// call on a device looks up that device's copy with hipGetSymbolAddress, with
// the device current, and keeps the address per device.
//
// Every call on a GPU shares that GPU's array, so calls that overlap on one
// GPU (other streams, other threads) race; serialise them. No byte of the
// scratch needs to start at zero: every byte a kernel reads was written
// earlier in the same call (the plan by the attention kernel's first
// workgroup, each partial row by the worker that owns it), so the previous
// call's contents are never read.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "../../include/fa_mi355x.h"

namespace fa {
fa_status_t forward_kvcache_on(const fa_fwd_params* p, void* stream, void* scratch, size_t bytes);
fa_status_t report_error(fa_status_t st, const char* msg);
}  // namespace fa

static __device__ __align__(256) unsigned char scratch[FA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {nullptr};
}  // namespace

extern "C" fa_status_t fa_mha_fwd_kvcache_noalloc(const fa_fwd_params* p, void* stream) {
    size_t need = 0;
    fa_status_t st = fa_fwd_workspace_size(p, FA_KIND_KVCACHE, &need);
    if (st != FA_OK) return st;
    if (need > (size_t)FA_NOALLOC_SCRATCH_BYTES) {
        char msg[256];
        snprintf(msg, sizeof(msg),
                 "fa_mha_fwd_kvcache_noalloc: this call needs %zu bytes of scratch, more than the %zu the library "
                 "holds; call fa_mha_fwd_kvcache with a workspace instead",
                 need, (size_t)FA_NOALLOC_SCRATCH_BYTES);
        return fa::report_error(FA_EWORKSPACE, msg);
    }
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fa::report_error(FA_EHIP, "fa_mha_fwd_kvcache_noalloc: no usable current device");
    void* ptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_ptr[dev]) {
            void* addr = nullptr;
            e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !addr) {
                char msg[256];
                snprintf(msg, sizeof(msg), "fa_mha_fwd_kvcache_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                         hipGetErrorString(e));
                return fa::report_error(FA_EHIP, msg);
            }
            g_ptr[dev] = addr;
        }
        ptr = g_ptr[dev];
    }
    return fa::forward_kvcache_on(p, stream, ptr, (size_t)FA_NOALLOC_SCRATCH_BYTES);
}

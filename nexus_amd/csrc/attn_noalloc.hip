// nexus_amd/csrc/attn_noalloc.hip -- nexus_hip_attn_decode_noalloc: split-KV decode for
// callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).  It runs the kernels of nexus_hip_attn_decode_gated
// with the split partials in a fixed device array instead of a caller workspace.
//
// The array lives for the whole process on every GPU the library runs on (8 MiB each).  Its
// device address is looked up once per device, at the first call on that device, with that
// device current; host code only ever passes that address, never the array's own name (a
// host-side stand-in).  Nothing in it must start at zero: every split writes its whole
// partial before the combine reads it.  All calls on one GPU share the array, so calls that
// overlap on one GPU (two streams at once) race on it; one call in flight per GPU at a time.
#include <hip/hip_runtime.h>

#include <mutex>

#include "attn_kernels.h"
#include "capi_status.h"
#include "nexus_hip_attn.h"

// The split partials of one call (head_dim + 2 floats per row and split).
constexpr size_t kScratchBytes = NEXUS_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};          // device address of `scratch`, per device

// Device address of this device's `scratch`, looked up once per device.
int scratch_ptr(float** out)
{
    int dev = 0;
    const hipError_t ge = hipGetDevice(&dev);
    if (ge != hipSuccess) return nxa::capi_fail(NEXUS_E_LAUNCH, "hipGetDevice: %s", hipGetErrorString(ge));
    if (dev < 0 || dev >= kMaxDevices)
        return nxa::capi_fail(NEXUS_E_UNSUPPORTED, "device %d beyond the %d devices served", dev, kMaxDevices);
    std::lock_guard<std::mutex> l(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return nxa::capi_fail(NEXUS_E_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                                  hipGetErrorString(e));
        g_scratch[dev] = (float*)p;
    }
    *out = g_scratch[dev];
    return NEXUS_OK;
}

}  // namespace

extern "C" int nexus_hip_attn_decode_noalloc(const nexus_attn_desc* desc, const void* q, const uint16_t* k,
                                             const uint16_t* v, const float* gate, void* out, int n_splits,
                                             nexus_stream_t stream)
{
    float* ws = nullptr;
    const int rc = scratch_ptr(&ws);
    if (rc != NEXUS_OK) return rc;
    return nxa::decode_into(desc, q, k, v, gate, out, ws, kScratchBytes, n_splits, (hipStream_t)stream);
}

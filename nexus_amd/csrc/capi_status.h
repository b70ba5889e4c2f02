// nexus_amd/csrc/capi_status.h -- the per-thread "last error" shared by every C-ABI source
// (read back through nexus_hip_attn_last_error()).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "nexus_hip_attn.h"

namespace nxa {

// Record a printf-style message and return `code` (a negative nexus_status).
int capi_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clear the message and return NEXUS_OK.
int capi_ok();

// One split-KV decode with its partials in `ws` (ws_cap bytes): the whole call is validated
// first and declined with nothing launched if it does not fit.  n_splits <= 0 takes the
// library's default split count, lowered until the partials fit in ws_cap.  Shared by
// nexus_hip_attn_decode_gated and the allocation-free nexus_hip_attn_decode_noalloc.
int decode_into(const nexus_attn_desc* desc, const void* q, const uint16_t* k, const uint16_t* v,
                const float* gate, void* out, float* ws, size_t ws_cap, int n_splits, hipStream_t stream);

}  // namespace nxa

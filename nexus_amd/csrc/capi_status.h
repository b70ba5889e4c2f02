// nexus_amd/csrc/capi_status.h -- the per-thread "last error" shared by every C-ABI source
// (read back through nexus_hip_attn_last_error()).
#pragma once

namespace nxa {

// Record a printf-style message and return `code` (a negative nexus_status).
int capi_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clear the message and return NEXUS_OK.
int capi_ok();

}  // namespace nxa

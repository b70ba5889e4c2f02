// tests/cpp/backend_shim.cpp -- TEST INFRASTRUCTURE: C entry points over
// nexus::hip::HipAttnBackend so the pytest suite can call the engine-side backend with
// host arrays.  Built with plain g++ (no HIP headers), the way an engine translation unit
// that includes hip_attn_backend.h is built, and linked against libnexus_hip_attn.so.
#include "hip_attn_backend.h"

using nexus::hip::backend;

extern "C" {

int shim_ready(void) { return backend().ready() ? 1 : 0; }

int shim_attention_gpu(const float* q, float* out, int n_heads, int n_kv_heads, int head_dim, int layer,
                       int n_ctx, const void* k, const void* v, size_t kv_bytes)
{
    return backend().attention_gpu(q, out, n_heads, n_kv_heads, head_dim, layer, n_ctx, k, v, kv_bytes) ? 1 : 0;
}

int shim_attention_batch_gpu(const float* q, float* out, int hq, int hkv, int hd, int n_ctx, int nq, int base,
                             int sw, float scale, float softcap, const void* k, const void* v, size_t kv_bytes)
{
    return backend().attention_batch_gpu(q, out, hq, hkv, hd, n_ctx, nq, base, sw, scale, softcap, k, v, kv_bytes)
               ? 1 : 0;
}

int shim_attention_stream_gpu(const float* q, float* out, int hq, int hkv, int hd, int n_ctx, int nq, int base,
                              float scale, float softcap, const void* k, const void* v, int chunk_tokens)
{
    return backend().attention_stream_gpu(q, out, hq, hkv, hd, n_ctx, nq, base, scale, softcap, k, v, chunk_tokens)
               ? 1 : 0;
}

int shim_attention_flash_gpu(const float* q, float* out, int hq, int hkv, int hd, int n_ctx, int nq, int base,
                             int sw, float scale, float softcap, const void* k, const void* v)
{
    return backend().attention_flash_gpu(q, out, hq, hkv, hd, n_ctx, nq, base, sw, scale, softcap, k, v) ? 1 : 0;
}

long long shim_calls_run(void) { return backend().calls_run(); }
long long shim_calls_declined(void) { return backend().calls_declined(); }
const char* shim_last_decline(void) { return backend().last_decline(); }

}  // extern "C"

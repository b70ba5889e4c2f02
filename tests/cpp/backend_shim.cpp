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

// q35_attention with the host cache as one array [n_kv][host_cap][hd] (per-head pointers
// built here) and device pointers for qg / k_raw / v_raw / out.
// async_kv_slot >= 0: the chained form (kv_out unused; the K/V land in that chain slot).
int shim_q35_attention_slot(const void* owner, int layer, int n_heads, int n_kv, int hd, int rot, int pos, float eps,
                            float scale, int has_gate, int interleaved, const float* q_norm, const float* k_norm,
                            int q_zc, int k_zc, const float* tab, const uint16_t* k_host, const uint16_t* v_host,
                            long long host_cap, int host_tokens, int host_synced, const float* qg, const float* k_raw,
                            const float* v_raw, float* out, float* kv_out, unsigned* mirror_valid, void* stream,
                            int async_kv_slot)
{
    if (n_kv <= 0 || n_kv > 64) return 0;
    const uint16_t* kp[64];
    const uint16_t* vp[64];
    for (int h = 0; h < n_kv; ++h) {
        kp[h] = k_host + (size_t)h * (size_t)host_cap * (size_t)hd;
        vp[h] = v_host + (size_t)h * (size_t)host_cap * (size_t)hd;
    }
    nexus::hip::HipAttnBackend::KvLayerDesc d;
    d.owner = owner;
    d.layer = layer;
    d.n_heads = (uint32_t)n_heads;
    d.n_kv = (uint32_t)n_kv;
    d.hd = (uint32_t)hd;
    d.rot = (uint32_t)rot;
    d.pos = (uint32_t)pos;
    d.norm_eps = eps;
    d.scale = scale;
    d.has_gate = has_gate != 0;
    d.rope_interleaved = interleaved != 0;
    d.q_norm = q_norm;
    d.k_norm = k_norm;
    d.q_zc = q_zc != 0;
    d.k_zc = k_zc != 0;
    d.rope_tab = tab;
    d.k_host = kp;
    d.v_host = vp;
    d.host_tokens = (uint32_t)host_tokens;
    d.host_synced = (uint32_t)host_synced;
    return backend().q35_attention(d, qg, k_raw, v_raw, out, kv_out, mirror_valid, (nexus_stream_t)stream,
                                   async_kv_slot)
               ? 1
               : 0;
}

int shim_q35_attention(const void* owner, int layer, int n_heads, int n_kv, int hd, int rot, int pos, float eps,
                       float scale, int has_gate, int interleaved, const float* q_norm, const float* k_norm, int q_zc,
                       int k_zc, const float* tab, const uint16_t* k_host, const uint16_t* v_host,
                       long long host_cap, int host_tokens, int host_synced, const float* qg, const float* k_raw,
                       const float* v_raw, float* out, float* kv_out, unsigned* mirror_valid, void* stream)
{
    return shim_q35_attention_slot(owner, layer, n_heads, n_kv, hd, rot, pos, eps, scale, has_gate, interleaved,
                                   q_norm, k_norm, q_zc, k_zc, tab, k_host, v_host, host_cap, host_tokens, host_synced,
                                   qg, k_raw, v_raw, out, kv_out, mirror_valid, stream, -1);
}

int shim_chain_end(void) { return backend().chain_end() ? 1 : 0; }
int shim_chain_is_open(void) { return backend().chain_is_open() ? 1 : 0; }
// copies n floats of chain slot `slot` into dst; 0 when the slot has no memory
int shim_chain_kv(int slot, float* dst, int n)
{
    const float* p = backend().chain_kv_ptr(slot);
    if (!p) return 0;
    for (int i = 0; i < n; ++i) dst[i] = p[i];
    return 1;
}

void shim_q35_kv_drop(const void* owner, int layer) { backend().q35_kv_drop(owner, layer); }
void shim_set_gpu_kv_mb(int mb) { backend().set_gpu_kv_mb(mb); }
size_t shim_kv_mirror_used(void) { return backend().kv_mirror_used(); }
void shim_set_mirror_store_rne(int on) { backend().set_mirror_store_rne(on != 0); }

int shim_kv_mirror_info(const void* owner, int layer, size_t* cap, size_t* valid)
{
    return backend().kv_mirror_info(owner, layer, cap, valid) ? 1 : 0;
}

int shim_kv_mirror_read(const void* owner, int layer, int kv_head, int pos0, int n, uint16_t* k_out, uint16_t* v_out)
{
    return backend().kv_mirror_read(owner, layer, kv_head, pos0, n, k_out, v_out) ? 1 : 0;
}

// device-resident forms: device pointers, the caller's stream (a hipStream_t as void*)
int shim_prefill_device(const nexus_attn_desc* d, const void* q, const void* k, const void* v, void* out,
                        void* stream)
{
    return backend().prefill_device(*d, q, (const uint16_t*)k, (const uint16_t*)v, out, (nexus_stream_t)stream) ? 1
                                                                                                                 : 0;
}
int shim_decode_device(const nexus_attn_desc* d, const void* q, const void* k, const void* v, void* out,
                       int n_splits, void* stream)
{
    return backend().decode_device(*d, q, (const uint16_t*)k, (const uint16_t*)v, out, n_splits,
                                   (nexus_stream_t)stream)
               ? 1
               : 0;
}

long long shim_calls_run(void) { return backend().calls_run(); }
long long shim_calls_declined(void) { return backend().calls_declined(); }
const char* shim_last_decline(void) { return backend().last_decline(); }

}  // extern "C"

// nexus_amd/host/hip_attn_backend.cpp -- HipAttnBackend: the reference's attention member
// functions over the HIP kernels of include/nexus_hip_attn.h.
#include "hip_attn_backend.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <set>
#include <string>

namespace nexus {
namespace hip {

namespace {

// Once per distinct reason, like nx_decline (src/gpu/vulkan_backend.h:187-192).
void log_decline_once(const char* why)
{
    static std::mutex m;
    static std::set<std::string> seen;
    std::lock_guard<std::mutex> l(m);
    if (seen.size() < 64 && seen.insert(why).second) {
        fprintf(stderr, "[nexus_hip_attn] GPU attention declined: %s\n", why);
        fflush(stderr);
    }
}

nexus_attn_desc host_desc(int hq, int hkv, int hd, int n_ctx, int n_query, int q_base, int sw,
                          float scale, float softcap)
{
    nexus_attn_desc d{};
    d.n_q_heads = hq;
    d.n_kv_heads = hkv;
    d.head_dim = hd;
    d.n_query = n_query;
    d.q_base_pos = q_base;
    d.n_ctx = n_ctx;
    d.kv_row_stride = n_ctx;            // packed [Hkv][n_ctx][hd]
    d.sliding_window = sw;
    d.scale = scale;
    d.softcap = softcap;
    d.q_dtype = NEXUS_DT_F32;
    d.o_dtype = NEXUS_DT_F32;
    return d;
}

}  // namespace

HipAttnBackend::~HipAttnBackend()
{
    if (!ready_) return;
    (void)hipSetDevice(device_);
    for (DevBuf* b : {&q_, &k_, &v_, &o_, &ws_})
        if (b->ptr) (void)hipFree(b->ptr);
    if (stream_) (void)hipStreamDestroy((hipStream_t)stream_);
}

bool HipAttnBackend::init(int device)
{
    std::lock_guard<std::mutex> l(mu_);
    if (ready_) return device == device_;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) {
        (void)hipGetLastError();
        return false;
    }
    if (hipSetDevice(device) != hipSuccess) return false;
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return false;
    stream_ = s;
    device_ = device;
    ready_ = true;
    return true;
}

bool HipAttnBackend::decline(const char* why)
{
    last_decline_ = why;
    ++calls_declined_;
    log_decline_once(why);
    return false;
}

bool HipAttnBackend::ensure(DevBuf& b, size_t bytes, bool zero)
{
    if (bytes == 0) bytes = 256;
    if (b.ptr && b.bytes >= bytes) return true;
    if (b.ptr) {
        // the stream may still read the old buffer
        if (hipStreamSynchronize((hipStream_t)stream_) != hipSuccess) return false;
        (void)hipFree(b.ptr);
        b = DevBuf{};
    }
    const size_t rounded = (bytes + (2u << 20) - 1) & ~(size_t)((2u << 20) - 1);
    void* p = nullptr;
    if (hipMalloc(&p, rounded) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (zero && hipMemset(p, 0, rounded) != hipSuccess) {
        (void)hipFree(p);
        return false;
    }
    b.ptr = p;
    b.bytes = rounded;
    return true;
}

bool HipAttnBackend::run_device(const nexus_attn_desc& d, const void* q, const uint16_t* k,
                                const uint16_t* v, void* out, int n_splits, bool decode, void* stream)
{
    // the sizing query validates the whole descriptor without launching anything
    const size_t ws_bytes = decode ? nexus_hip_attn_decode_ws_bytes(&d, n_splits)
                                   : nexus_hip_attn_prefill_ws_bytes(&d);
    if (decode && ws_bytes == 0) return decline(nexus_hip_attn_last_error());
    if (!ensure(ws_, ws_bytes, /*zero=*/true)) return decline("workspace allocation failed");
    const int rc = decode
        ? nexus_hip_attn_decode(&d, q, k, v, out, (float*)ws_.ptr, n_splits, (nexus_stream_t)stream)
        : nexus_hip_attn_prefill(&d, q, k, v, out, ws_.ptr, ws_.bytes, (nexus_stream_t)stream);
    if (rc != NEXUS_OK) return decline(nexus_hip_attn_last_error());
    ++calls_run_;
    return true;
}

bool HipAttnBackend::run_host(const nexus_attn_desc& d, const float* q, const void* k_flat,
                              const void* v_flat, float* out, bool decode)
{
    if (!ready_) return decline("no HIP device (HipAttnBackend::init not called or failed)");
    if (!q || !out || !k_flat || !v_flat) return decline("null pointer");
    // validate before staging anything
    if (nexus_hip_attn_decode_ws_bytes(&d, 0) == 0) return decline(nexus_hip_attn_last_error());
    if (hipSetDevice(device_) != hipSuccess) return decline("hipSetDevice failed");
    const size_t qo_bytes = (size_t)d.n_query * d.n_q_heads * d.head_dim * sizeof(float);
    const size_t kv_bytes = (size_t)d.n_kv_heads * (size_t)d.n_ctx * d.head_dim * sizeof(uint16_t);
    if (!ensure(q_, qo_bytes, false) || !ensure(o_, qo_bytes, false) || !ensure(k_, kv_bytes, false) ||
        !ensure(v_, kv_bytes, false))
        return decline("device staging allocation failed");
    hipStream_t s = (hipStream_t)stream_;
    if (hipMemcpyAsync(q_.ptr, q, qo_bytes, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(k_.ptr, k_flat, kv_bytes, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(v_.ptr, v_flat, kv_bytes, hipMemcpyHostToDevice, s) != hipSuccess)
        return decline("host-to-device copy failed");
    if (!run_device(d, q_.ptr, (const uint16_t*)k_.ptr, (const uint16_t*)v_.ptr, o_.ptr, 0, decode, stream_))
        return false;
    --calls_run_;   // counted once below, after the copy back
    if (hipMemcpyAsync(out, o_.ptr, qo_bytes, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return decline("device-to-host copy failed");
    ++calls_run_;
    return true;
}

bool HipAttnBackend::attention_gpu(const float* q, float* out, int n_heads, int n_kv_heads, int head_dim,
                                   int /*layer*/, int n_ctx, const void* k_flat, const void* v_flat,
                                   size_t kv_bytes)
{
    std::lock_guard<std::mutex> l(mu_);
    if (n_ctx <= 0 || head_dim <= 0 || n_kv_heads <= 0) return decline("attention_gpu: empty shape");
    if (kv_bytes < (size_t)n_kv_heads * (size_t)n_ctx * head_dim * sizeof(uint16_t))
        return decline("attention_gpu: kv_bytes smaller than n_kv_heads * n_ctx * head_dim f16");
    nexus_attn_desc d = host_desc(n_heads, n_kv_heads, head_dim, n_ctx, 1, n_ctx - 1, 0,
                                  1.0f / std::sqrt((float)head_dim), 0.f);
    return run_host(d, q, k_flat, v_flat, out, /*decode=*/true);
}

bool HipAttnBackend::attention_batch_gpu(const float* q_batch, float* out_batch, int n_q_heads, int n_kv_heads,
                                         int head_dim, int n_ctx, int n_query, int q_base_pos,
                                         int sliding_window, float scale, float softcap, const void* k_flat,
                                         const void* v_flat, size_t kv_bytes)
{
    std::lock_guard<std::mutex> l(mu_);
    if (n_ctx <= 0 || head_dim <= 0 || n_kv_heads <= 0) return decline("attention_batch_gpu: empty shape");
    if (kv_bytes < (size_t)n_kv_heads * (size_t)n_ctx * head_dim * sizeof(uint16_t))
        return decline("attention_batch_gpu: kv_bytes smaller than n_kv_heads * n_ctx * head_dim f16");
    nexus_attn_desc d = host_desc(n_q_heads, n_kv_heads, head_dim, n_ctx, n_query, q_base_pos, sliding_window,
                                  scale, softcap);
    return run_host(d, q_batch, k_flat, v_flat, out_batch, /*decode=*/false);
}

bool HipAttnBackend::attention_stream_gpu(const float* q_batch, float* out_batch, int n_q_heads,
                                          int n_kv_heads, int head_dim, int n_ctx, int n_query,
                                          int q_base_pos, float scale, float softcap, const void* k_flat,
                                          const void* v_flat, int chunk_tokens)
{
    std::lock_guard<std::mutex> l(mu_);
    if (n_ctx <= 0) return decline("attention_stream_gpu: n_ctx <= 0");
    if (chunk_tokens < 0) return decline("attention_stream_gpu: chunk_tokens < 0");
    nexus_attn_desc d = host_desc(n_q_heads, n_kv_heads, head_dim, n_ctx, n_query, q_base_pos, 0, scale,
                                  softcap);
    return run_host(d, q_batch, k_flat, v_flat, out_batch, /*decode=*/false);
}

bool HipAttnBackend::attention_flash_gpu(const float* q_batch, float* out_batch, int n_q_heads, int n_kv_heads,
                                         int head_dim, int n_ctx, int n_query, int q_base_pos,
                                         int sliding_window, float scale, float softcap, const void* k_flat,
                                         const void* v_flat)
{
    std::lock_guard<std::mutex> l(mu_);
    static const bool disabled = std::getenv("NEXUS_ATTN_NOFLASH") != nullptr;
    if (disabled) return decline("attention_flash_gpu: NEXUS_ATTN_NOFLASH is set");
    if (head_dim <= 0 || head_dim > 256 || head_dim % 64 != 0)
        return decline("attention_flash_gpu: head_dim must be a multiple of 64 up to 256");
    if (n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads != 0)
        return decline("attention_flash_gpu: n_q_heads must be a multiple of n_kv_heads");
    if (n_ctx <= 0 || n_query <= 0) return decline("attention_flash_gpu: empty shape");
    if (const char* e = std::getenv("NEXUS_FLASH_KV_MB")) {
        const long mb = std::atol(e);
        const size_t kvb = (size_t)n_kv_heads * (size_t)n_ctx * head_dim * sizeof(uint16_t);
        if (mb > 0 && 2 * kvb > (size_t)mb * 1024 * 1024)
            return decline("attention_flash_gpu: K+V above NEXUS_FLASH_KV_MB");
    }
    nexus_attn_desc d = host_desc(n_q_heads, n_kv_heads, head_dim, n_ctx, n_query, q_base_pos, sliding_window,
                                  scale, softcap);
    return run_host(d, q_batch, k_flat, v_flat, out_batch, /*decode=*/false);
}

bool HipAttnBackend::prefill_device(const nexus_attn_desc& d, const void* q, const uint16_t* k,
                                    const uint16_t* v, void* out, nexus_stream_t stream)
{
    std::lock_guard<std::mutex> l(mu_);
    if (!ready_) return decline("no HIP device (HipAttnBackend::init not called or failed)");
    return run_device(d, q, k, v, out, 0, /*decode=*/false, (void*)stream);
}

bool HipAttnBackend::decode_device(const nexus_attn_desc& d, const void* q, const uint16_t* k,
                                   const uint16_t* v, void* out, int n_splits, nexus_stream_t stream)
{
    std::lock_guard<std::mutex> l(mu_);
    if (!ready_) return decline("no HIP device (HipAttnBackend::init not called or failed)");
    return run_device(d, q, k, v, out, n_splits, /*decode=*/true, (void*)stream);
}

HipAttnBackend& backend()
{
    static HipAttnBackend b;
    static std::once_flag once;
    std::call_once(once, [] { (void)b.init(0); });
    return b;
}

}  // namespace hip
}  // namespace nexus

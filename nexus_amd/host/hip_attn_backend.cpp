// nexus_amd/host/hip_attn_backend.cpp -- HipAttnBackend: the reference's attention member
// functions over the HIP kernels of include/nexus_hip_attn.h.
#include "hip_attn_backend.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
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
    (void)hipDeviceSynchronize();
    for (DevBuf* b : {&q_, &k_, &v_, &o_, &ws_, &prep_kv_, &prep_par_})
        if (b->ptr) (void)hipFree(b->ptr);
    for (auto& m : mirrors_) {
        if (m.second.k.ptr) (void)hipFree(m.second.k.ptr);
        if (m.second.v.ptr) (void)hipFree(m.second.v.ptr);
    }
    if (chain_ring_) (void)hipHostFree(chain_ring_);
    if (ws_done_) (void)hipEventDestroy((hipEvent_t)ws_done_);
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
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
        (void)hipStreamDestroy(s);
        return false;
    }
    stream_ = s;
    ws_done_ = ev;
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
        // work in flight on any stream (the caller's too) may still read the old buffer
        if (hipDeviceSynchronize() != hipSuccess) return false;
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

bool HipAttnBackend::ws_acquire(void* stream)
{
    // the event is recorded after every launch that used ws_, on the stream it ran on; an
    // event never recorded is complete, so the first wait is free
    return hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)ws_done_, 0) == hipSuccess;
}

void HipAttnBackend::ws_release(void* stream)
{
    if (hipEventRecord((hipEvent_t)ws_done_, (hipStream_t)stream) != hipSuccess) {
        // without the event the next user cannot be ordered after this one: wait here
        (void)hipGetLastError();
        (void)hipStreamSynchronize((hipStream_t)stream);
    }
}

bool HipAttnBackend::run_device(const nexus_attn_desc& d, const void* q, const uint16_t* k,
                                const uint16_t* v, void* out, int n_splits, bool decode, void* stream)
{
    // the sizing query validates the whole descriptor without launching anything
    const size_t ws_bytes = decode ? nexus_hip_attn_decode_ws_bytes(&d, n_splits)
                                   : nexus_hip_attn_prefill_ws_bytes(&d);
    if (decode && ws_bytes == 0) return decline(nexus_hip_attn_last_error());
    if (!ensure(ws_, ws_bytes, /*zero=*/true)) return decline("workspace allocation failed");
    if (!ws_acquire(stream)) return decline("hipStreamWaitEvent failed");
    const int rc = decode
        ? nexus_hip_attn_decode(&d, q, k, v, out, (float*)ws_.ptr, n_splits, (nexus_stream_t)stream)
        : nexus_hip_attn_prefill(&d, q, k, v, out, ws_.ptr, ws_.bytes, (nexus_stream_t)stream);
    ws_release(stream);
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

// ------------------------------------------------------------------ device KV mirror

bool HipAttnBackend::alloc_exact(DevBuf& b, size_t bytes)
{
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    b.ptr = p;
    b.bytes = bytes;
    return true;
}

void HipAttnBackend::free_buf(DevBuf& b)
{
    if (b.ptr) (void)hipFree(b.ptr);
    b = DevBuf{};
}

void HipAttnBackend::drop_locked(const void* owner, int layer)
{
    bool synced = false;
    for (auto it = mirrors_.begin(); it != mirrors_.end();) {
        if (it->first.first == owner && (layer < 0 || it->first.second == layer)) {
            if (!synced) {                               // kernels in flight may still read it
                (void)hipDeviceSynchronize();
                synced = true;
            }
            kv_mirror_used_ -= std::min(kv_mirror_used_, it->second.bytes);
            free_buf(it->second.k);
            free_buf(it->second.v);
            it = mirrors_.erase(it);
        } else {
            ++it;
        }
    }
}

void HipAttnBackend::q35_kv_drop(const void* owner, int layer)
{
    std::lock_guard<std::mutex> l(mu_);
    if (!ready_) return;
    (void)hipSetDevice(device_);
    drop_locked(owner, layer);
}

void HipAttnBackend::set_gpu_kv_mb(int mb)
{
    std::lock_guard<std::mutex> l(mu_);
    gpu_kv_mb_ = mb < 0 ? -1 : mb;
}

int HipAttnBackend::gpu_kv_mb()
{
    if (gpu_kv_mb_ == -2) {                              // vulkan_backend.h:5277-5284
        gpu_kv_mb_ = -1;
        if (const char* e = std::getenv("NEXUS_GPU_KV")) {
            if (!std::strcmp(e, "off") || !std::strcmp(e, "0")) gpu_kv_mb_ = 0;
            else if (std::strcmp(e, "auto") && *e) {
                const int v = std::atoi(e);
                gpu_kv_mb_ = v > 0 ? v : -1;
            }
        }
    }
    return gpu_kv_mb_;
}

size_t HipAttnBackend::kv_mirror_cap_bytes()
{
    const int mb = gpu_kv_mb();
    if (mb == 0 || !ready_) return 0;
    if (mb > 0) return (size_t)mb << 20;
    // auto (vulkan_backend.h:5192-5205, with the runtime's free-memory figure in place of
    // the reference's weight bookkeeping): what is free now plus the mirrors' own bytes.
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    const size_t avail = free_b + kv_mirror_used_;
    const size_t margin = std::max<size_t>(768ull << 20, total_b / 5) + (64ull << 20);
    return avail > margin ? avail - margin : 0;
}

bool HipAttnBackend::kv_mirror_info(const void* owner, int layer, size_t* cap, size_t* valid)
{
    std::lock_guard<std::mutex> l(mu_);
    auto it = mirrors_.find({owner, layer});
    if (it == mirrors_.end() || it->second.cap == 0) return false;
    if (cap) *cap = it->second.cap;
    if (valid) *valid = it->second.valid;
    return true;
}

bool HipAttnBackend::kv_mirror_read(const void* owner, int layer, int kv_head, int pos0, int n, uint16_t* k_out,
                                    uint16_t* v_out)
{
    std::lock_guard<std::mutex> l(mu_);
    auto it = mirrors_.find({owner, layer});
    if (it == mirrors_.end() || it->second.cap == 0 || !k_out || !v_out) return false;
    const KvMirror& m = it->second;
    if (kv_head < 0 || (uint32_t)kv_head >= m.n_kv || pos0 < 0 || n < 0 || (size_t)pos0 + (size_t)n > m.cap)
        return false;
    (void)hipSetDevice(device_);
    const size_t row = (size_t)m.hd * sizeof(uint16_t);
    const size_t off = ((size_t)kv_head * m.cap + (size_t)pos0) * row;
    hipStream_t s = (hipStream_t)stream_;
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpyAsync(k_out, (const char*)m.k.ptr + off, (size_t)n * row, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipMemcpyAsync(v_out, (const char*)m.v.ptr + off, (size_t)n * row, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return false;
    return true;
}

bool HipAttnBackend::chain_end()
{
    std::lock_guard<std::mutex> l(mu_);
    if (!chain_open_) return true;
    chain_open_ = false;
    return hipStreamSynchronize((hipStream_t)chain_stream_) == hipSuccess;
}

const float* HipAttnBackend::chain_kv_ptr(int slot) const
{
    if (slot < 0 || slot >= kChainKvSlots || !chain_ring_) return nullptr;
    return chain_ring_ + (size_t)slot * kChainSlotFloats;
}

bool HipAttnBackend::q35_attention(const KvLayerDesc& d, const float* qg, const float* k_raw, const float* v_raw,
                                   float* attn_out, float* kv_out_host, uint32_t* mirror_valid_out,
                                   nexus_stream_t stream, int async_kv_slot)
{
    std::lock_guard<std::mutex> l(mu_);
    if (!ready_) return decline("no HIP device (HipAttnBackend::init not called or failed)");
    const bool chained = async_kv_slot >= 0;
    if (!qg || !k_raw || !v_raw || !attn_out || (!chained && !kv_out_host))
        return decline("q35_attention: null pointer");
    if (async_kv_slot >= kChainKvSlots) return decline("q35_attention: async_kv_slot >= kChainKvSlots");
    const uint32_t nh = d.n_heads, nkv = d.n_kv, hd = d.hd;
    if (chained && (size_t)2 * nkv * hd > kChainSlotFloats)
        return decline("q35_attention: K/V row larger than a chain slot (n_kv * hd > 8192)");
    if (nh == 0 || nkv == 0 || nh % nkv != 0) return decline("q35_attention: n_heads must be a multiple of n_kv");
    if (d.rot > hd || (d.rot & 1) || (d.rot > 0 && !d.rope_tab))
        return decline("q35_attention: rot must be even, <= hd, with a table");
    if (d.has_gate && (!d.q_norm || !d.k_norm)) return decline("q35_attention: gated layer without q/k norm");
    if (!d.k_host || !d.v_host || d.host_tokens < d.pos) return decline("q35_attention: host cache missing or short");
    if (d.pos >= (uint32_t)INT32_MAX - 1) return decline("q35_attention: pos beyond the 31-bit range");
    for (uint32_t h = 0; h < nkv; ++h)
        if (d.pos > 0 && (!d.k_host[h] || !d.v_host[h])) return decline("q35_attention: null host head");
    const uint32_t need = d.pos + 1;

    // attention over the mirror: validated before anything is allocated or copied
    nexus_attn_desc ad{};
    ad.n_q_heads = (int)nh;
    ad.n_kv_heads = (int)nkv;
    ad.head_dim = (int)hd;
    ad.n_query = 1;
    ad.q_base_pos = (int)d.pos;
    ad.n_ctx = (int)need;
    ad.kv_row_stride = need;                             // the real stride (cap >= need) is set below
    ad.scale = d.scale;
    ad.q_dtype = NEXUS_DT_F32;
    ad.o_dtype = NEXUS_DT_F32;
    const int splits = nexus_hip_attn_decode_default_splits(&ad);
    const size_t ws_bytes = splits > 0 ? nexus_hip_attn_decode_ws_bytes(&ad, splits) : 0;
    if (ws_bytes == 0) return decline(nexus_hip_attn_last_error());

    const size_t cap_bytes = kv_mirror_cap_bytes();
    if (cap_bytes == 0) return decline("q35_attention: GPU KV mirror is off (NEXUS_GPU_KV / set_gpu_kv_mb)");
    if (hipSetDevice(device_) != hipSuccess) return decline("hipSetDevice failed");
    hipStream_t s = stream ? (hipStream_t)stream : (hipStream_t)stream_;
    if (chained) {
        if (chain_open_ && chain_stream_ != (void*)s) return decline("q35_attention: chained calls on two streams");
        if (!chain_ring_ && hipHostMalloc((void**)&chain_ring_, kChainKvSlots * kChainSlotFloats * sizeof(float),
                                          hipHostMallocDefault) != hipSuccess) {
            chain_ring_ = nullptr;
            (void)hipGetLastError();
            return decline("q35_attention: pinned allocation of the chain ring failed");
        }
    }

    // ---- find / grow (vulkan_backend.h:5349-5391)
    const std::pair<const void*, int> key{d.owner, d.layer};
    auto it = mirrors_.find(key);
    if (it != mirrors_.end() && it->second.cap && (it->second.n_kv != nkv || it->second.hd != hd)) {
        drop_locked(d.owner, d.layer);
        it = mirrors_.end();
    }
    if (it == mirrors_.end()) it = mirrors_.emplace(key, KvMirror{}).first;
    KvMirror& mm = it->second;
    size_t eff_valid = std::min<size_t>(mm.valid, d.host_synced);
    if (mm.cap < need) {
        if (mm.refused_need && need < mm.refused_need)
            return decline("q35_attention: the mirror was refused for a larger context recently");
        const size_t per_tok = (size_t)nkv * hd * 2 * sizeof(uint16_t);     // K + V
        size_t newcap = std::max<size_t>(((size_t)need * 5 / 4 + 255) & ~(size_t)255, 2048);
        const size_t others = kv_mirror_used_ - std::min(kv_mirror_used_, mm.bytes);
        if (others + newcap * per_tok > cap_bytes) newcap = ((size_t)need + 255) & ~(size_t)255;
        if (others + newcap * per_tok > cap_bytes) {
            if (mm.cap) drop_locked(d.owner, d.layer);
            mirrors_[key].refused_need = need + 1024;
            return decline("q35_attention: the mirror would exceed the GPU KV budget");
        }
        const size_t half = newcap * (size_t)nkv * hd * sizeof(uint16_t);
        KvMirror nm;
        bool ok = alloc_exact(nm.k, half) && alloc_exact(nm.v, half);
        if (!ok && mm.cap) {                             // no room for both: give the old one up first
            free_buf(nm.k);
            free_buf(nm.v);
            drop_locked(d.owner, d.layer);
            it = mirrors_.emplace(key, KvMirror{}).first;
            eff_valid = 0;
            ok = alloc_exact(nm.k, half) && alloc_exact(nm.v, half);
        }
        KvMirror& cur = it->second;
        if (!ok) {
            free_buf(nm.k);
            free_buf(nm.v);
            cur.refused_need = need + 1024;
            return decline("q35_attention: device allocation of the mirror failed");
        }
        if (cur.cap && eff_valid > 0) {
            // keep the rows still in sync: one strided device copy per cache instead of a
            // refill over PCIe (the reference reallocates and refills from the host)
            const size_t row = (size_t)hd * sizeof(uint16_t);
            if (hipMemcpy2DAsync(nm.k.ptr, newcap * row, cur.k.ptr, cur.cap * row, eff_valid * row, nkv,
                                 hipMemcpyDeviceToDevice, s) != hipSuccess ||
                hipMemcpy2DAsync(nm.v.ptr, newcap * row, cur.v.ptr, cur.cap * row, eff_valid * row, nkv,
                                 hipMemcpyDeviceToDevice, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess) {
                (void)hipGetLastError();
                eff_valid = 0;
            }
        } else {
            eff_valid = 0;
        }
        if (cur.cap) (void)hipDeviceSynchronize();
        kv_mirror_used_ -= std::min(kv_mirror_used_, cur.bytes);
        free_buf(cur.k);
        free_buf(cur.v);
        nm.cap = newcap;
        nm.bytes = newcap * per_tok;
        nm.n_kv = nkv;
        nm.hd = hd;
        nm.valid = eff_valid;
        kv_mirror_used_ += nm.bytes;
        cur = nm;
    }
    KvMirror& m = it->second;

    // ---- per-call device buffers (grown, never shrunk)
    const size_t kv_bytes = 2 * (size_t)nkv * hd * sizeof(float);
    const size_t par_floats = (size_t)d.rot + 2 * (size_t)hd;
    if (!ensure(prep_kv_, kv_bytes, false) || !ensure(prep_par_, par_floats * sizeof(float), false) ||
        !ensure(ws_, ws_bytes, true))
        return decline("q35_attention: device scratch allocation failed");

    // ---- fill rows [eff_valid, pos) from the host (vulkan_backend.h:5392-5418)
    const size_t row = (size_t)hd * sizeof(uint16_t);
    if (eff_valid < d.pos) {
        const size_t n = d.pos - eff_valid;
        for (uint32_t h = 0; h < nkv; ++h) {
            const size_t off = ((size_t)h * m.cap + eff_valid) * row;
            if (hipMemcpyAsync((char*)m.k.ptr + off, d.k_host[h] + eff_valid * hd, n * row, hipMemcpyHostToDevice, s) !=
                    hipSuccess ||
                hipMemcpyAsync((char*)m.v.ptr + off, d.v_host[h] + eff_valid * hd, n * row, hipMemcpyHostToDevice, s) !=
                    hipSuccess) {
                m.valid = std::min(m.valid, eff_valid);
                return decline("q35_attention: host-to-device fill failed");
            }
        }
    }
    m.valid = d.pos;

    // ---- norm weights and the RoPE table: one small upload
    float* par = (float*)prep_par_.ptr;
    const float* tab_d = par;
    const float* qnw_d = par + d.rot;
    const float* knw_d = par + d.rot + hd;
    const size_t fb = sizeof(float);
    if ((d.rot && hipMemcpyAsync(par, d.rope_tab, d.rot * fb, hipMemcpyHostToDevice, s) != hipSuccess) ||
        (d.q_norm && hipMemcpyAsync(par + d.rot, d.q_norm, hd * fb, hipMemcpyHostToDevice, s) != hipSuccess) ||
        (d.k_norm && hipMemcpyAsync(par + d.rot + hd, d.k_norm, hd * fb, hipMemcpyHostToDevice, s) != hipSuccess))
        return decline("q35_attention: parameter upload failed");

    // ---- prep + split-KV attention + gated combine (vulkan_backend.h:5446-5482) in two
    // launches: the head norms, RoPE and the store of row `pos` run inside the split-KV kernel
    nexus_attn_prep_desc pd{};
    pd.n_heads = (int)nh;
    pd.n_kv_heads = (int)nkv;
    pd.head_dim = (int)hd;
    pd.rot_dims = (int)d.rot;
    pd.pos = (int)d.pos;
    pd.cap = (int64_t)m.cap;
    pd.eps = d.norm_eps;
    pd.flags = (d.q_zc ? NEXUS_PREP_Q_NORM_ADD_ONE : 0) | (d.k_zc ? NEXUS_PREP_K_NORM_ADD_ONE : 0) |
               (d.has_gate ? 0 : NEXUS_PREP_NO_GATE) | (d.q_norm ? 0 : NEXUS_PREP_NO_Q_NORM) |
               (d.k_norm ? 0 : NEXUS_PREP_NO_K_NORM) | (d.rope_interleaved ? NEXUS_PREP_ROPE_INTERLEAVED : 0) |
               (mirror_rne_ ? 0 : NEXUS_PREP_TRUNC_STORE);
    float* kv_d = (float*)prep_kv_.ptr;
    if (!ws_acquire(s)) return decline("hipStreamWaitEvent failed");
    const int rc = nexus_hip_attn_decode_layer(&pd, d.scale, qg, k_raw, v_raw, d.q_norm ? qnw_d : nullptr,
                                               d.k_norm ? knw_d : nullptr, d.rot ? tab_d : nullptr,
                                               (uint16_t*)m.k.ptr, (uint16_t*)m.v.ptr, kv_d, attn_out,
                                               (float*)ws_.ptr, splits, (nexus_stream_t)s);
    ws_release(s);
    if (rc != NEXUS_OK) {
        m.valid = std::min<size_t>(m.valid, d.pos);
        return decline(nexus_hip_attn_last_error());
    }
    if (chained) {
        // K/V into the ring slot; joined by chain_end()
        if (hipMemcpyAsync(chain_ring_ + (size_t)async_kv_slot * kChainSlotFloats, kv_d, kv_bytes,
                           hipMemcpyDeviceToHost, s) != hipSuccess)
            return decline("q35_attention: device-to-host copy of K/V failed");
        chain_open_ = true;
        chain_stream_ = (void*)s;
    } else if (hipMemcpyAsync(kv_out_host, kv_d, kv_bytes, hipMemcpyDeviceToHost, s) != hipSuccess ||
               hipStreamSynchronize(s) != hipSuccess) {
        return decline("q35_attention: device-to-host copy of K/V failed");
    }
    m.valid = need;
    if (mirror_valid_out) *mirror_valid_out = need;
    ++calls_run_;
    return true;
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

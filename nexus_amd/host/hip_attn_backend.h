// nexus_amd/host/hip_attn_backend.h -- the engine-side attention backend for one MI355X.
//
// HipAttnBackend keeps the attention member functions of the reference's GPU backend
// with their exact signatures and meaning, so the engine's call sites switch by changing
// the object they call:
//   attention_gpu         src/gpu/vulkan_backend.h:576-580  (impl :3731-3817)
//   attention_batch_gpu   src/gpu/vulkan_backend.h:584-588  (impl :3819-3934)
//   attention_stream_gpu  src/gpu/vulkan_backend.h:594-599  (impl :4085-4257)
//   attention_flash_gpu   src/gpu/vulkan_backend.h:604-608  (impl :4260-4408)
// and the callers in src/model/transformer.h:8478-8494 (prefill) and :11052 (decode).
//
// Contract carried over from the reference:
//  * host pointers in and out: Q f32 [n_query][Hq][hd], K/V f16 [Hkv][n_ctx][hd] (the
//    layout KVCache::pack_k/pack_v writes, src/model/kvcache.h:655-672), out f32;
//  * synchronous: the call returns after the output is in host memory;
//  * `return false` BEFORE any side effect when the call cannot run (unsupported shape,
//    no device, allocation failure, disabled by NEXUS_ATTN_NOFLASH / NEXUS_FLASH_KV_MB),
//    each distinct reason printed once to stderr like nx_decline (vulkan_backend.h:187-192);
//    the caller then runs its CPU attention.
// What changes: the kernels are the HIP ones behind include/nexus_hip_attn.h, the staging
// buffers are device memory owned by the backend (grown, never shrunk), and the
// device-resident entry points below skip the host round trip entirely.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <utility>

#include "nexus_hip_attn.h"

namespace nexus {
namespace hip {

class HipAttnBackend {
public:
    HipAttnBackend() = default;
    ~HipAttnBackend();
    HipAttnBackend(const HipAttnBackend&) = delete;
    HipAttnBackend& operator=(const HipAttnBackend&) = delete;

    // Bind to a HIP device and create the backend's stream (default priority).  Returns
    // false when no device is usable; every entry point then declines.
    bool init(int device = 0);
    bool ready() const { return ready_; }
    int device() const { return device_; }

    // ---- the reference's member functions (host pointers, synchronous) ----

    // Decode of one token that sees all n_ctx keys; scale 1/sqrt(head_dim) as the
    // reference's push constants set it (vulkan_backend.h:3785-3789).  `layer` is unused,
    // as in the reference.  kv_bytes = bytes of one of K/V.
    bool attention_gpu(const float* q, float* out,
                       int n_heads, int n_kv_heads, int head_dim,
                       int layer, int n_ctx,
                       const void* k_flat, const void* v_flat,
                       size_t kv_bytes);

    // Batched prefill: query i at absolute position q_base_pos + i, causal, optional
    // sliding window and softcap; scale 0 means 1/sqrt(head_dim).
    bool attention_batch_gpu(const float* q_batch, float* out_batch,
                             int n_q_heads, int n_kv_heads, int head_dim,
                             int n_ctx, int n_query, int q_base_pos, int sliding_window,
                             float scale, float softcap,
                             const void* k_flat, const void* v_flat, size_t kv_bytes);

    // Same results as attention_batch_gpu with no sliding window.  The reference streams
    // K/V through a small device buffer in chunk_tokens pieces because its cards are short
    // of memory; one MI355X holds any cache this entry point can be handed, so the whole
    // K/V is staged once and chunk_tokens (>= 0) is accepted and not needed.
    bool attention_stream_gpu(const float* q_batch, float* out_batch,
                              int n_q_heads, int n_kv_heads, int head_dim,
                              int n_ctx, int n_query, int q_base_pos,
                              float scale, float softcap,
                              const void* k_flat, const void* v_flat,
                              int chunk_tokens);

    // Tiled causal prompt attention (the engine's first choice for prefill).  Declines
    // like the reference: NEXUS_ATTN_NOFLASH set, head_dim % 64 != 0 or > 256,
    // Hq % Hkv != 0, null pointers, or 2 * K bytes above NEXUS_FLASH_KV_MB when that
    // variable is set (unset: no limit, the cache lives in 288 GB of HBM).
    bool attention_flash_gpu(const float* q_batch, float* out_batch,
                             int n_q_heads, int n_kv_heads, int head_dim,
                             int n_ctx, int n_query, int q_base_pos, int sliding_window,
                             float scale, float softcap,
                             const void* k_flat, const void* v_flat);

    // ---- device-resident forms (device pointers, stream-ordered, no host copies) ----
    // The split workspace is the backend's own: every launch that uses it first waits (on
    // its stream) for the previous user, whichever stream that ran on, so calls on
    // different streams take turns on it instead of overwriting partials still being read.
    bool prefill_device(const nexus_attn_desc& d, const void* q, const uint16_t* k,
                        const uint16_t* v, void* out, nexus_stream_t stream);
    bool decode_device(const nexus_attn_desc& d, const void* q, const uint16_t* k,
                       const uint16_t* v, void* out, int n_splits, nexus_stream_t stream);

    // ---- device-resident KV cache (the attention half of q35_full_layer) ----
    //
    // One decode token of a full-attention layer over a KV cache kept in HBM, replacing
    // the attention part of VulkanBackend::q35_full_layer (src/gpu/vulkan_backend.h:
    // 5272-5483): the per-(owner, layer) mirror is found or grown, tokens the host changed
    // or the mirror never had are copied from the host cache (which stays the source of
    // truth), then nexus_hip_attn_decode_layer runs over the mirror: head norms, RoPE and the
    // store of row `pos` inside the split-KV kernel, then the gated combine (two launches).  The projections before and the output
    // projection after stay with the caller: qg / k_raw / v_raw and attn_out are device
    // f32 buffers the engine's own matvecs produce and consume.
    struct KvLayerDesc {                                 // vulkan_backend.h:491-515, attention fields
        const void* owner = nullptr;
        int layer = 0;
        uint32_t n_heads = 0, n_kv = 0, hd = 0, rot = 0, pos = 0;
        float norm_eps = 1e-6f, scale = 0.f;             // scale 0: 1/sqrt(hd)
        bool has_gate = true;                            // qg holds [q | gate] per head
        bool rope_interleaved = false;
        const float* q_norm = nullptr;                   // host [hd] or nullptr (no q head norm)
        const float* k_norm = nullptr;
        bool q_zc = false, k_zc = false;                 // (1 + w) norms
        const float* rope_tab = nullptr;                 // host [rot]: cos then sin for `pos`
        const uint16_t* const* k_host = nullptr;         // [n_kv] -> host f16 [tokens][hd]
        const uint16_t* const* v_host = nullptr;
        uint32_t host_tokens = 0;                        // tokens on the host (>= pos)
        uint32_t host_synced = 0;                        // host rows [0, host_synced) unchanged since the last sync
    };
    // Synchronous like the reference's call: returns once kv_out_host ([2][n_kv][hd] f32,
    // K then V of token `pos` as stored, for KVCache::store) is written; attn_out is
    // ready on `stream` (nullptr: the backend's stream).  *mirror_valid_out = pos + 1,
    // the value for KVCache::set_mirror_valid.  Declines (false, nothing touched) on an
    // unsupported shape, null pointers, host_tokens < pos, or when the mirror would
    // exceed the budget (then it also remembers the refused size, as the reference does).
    //
    // Chained form (the async_kv_slot of q35_full_layer, vulkan_backend.h:5275, joined by
    // Transformer::q35_chain_flush, transformer.h:10083-10100): with async_kv_slot in
    // [0, kChainKvSlots) the call returns once its work is queued; K then V of token `pos` land in
    // slot async_kv_slot of a pinned host ring instead of kv_out_host (which may be null), and
    // are read with chain_kv_ptr() after chain_end().  The device work of a call is the two
    // launches of nexus_hip_attn_decode_layer plus the copies, so a chain of layers runs back to
    // back on the stream; all chained calls use one stream.
    bool q35_attention(const KvLayerDesc& d, const float* qg, const float* k_raw, const float* v_raw,
                       float* attn_out, float* kv_out_host, uint32_t* mirror_valid_out,
                       nexus_stream_t stream = nullptr, int async_kv_slot = -1);
    static constexpr int kChainKvSlots = 16;
    bool chain_is_open() const { return chain_open_; }
    // Waits for every chained call (their attn_out and K/V slots are then complete); false when
    // the stream reports an error.
    bool chain_end();
    // K/V of the chained call that used `slot` ([2][n_kv][hd] f32), valid after chain_end().
    const float* chain_kv_ptr(int slot) const;
    // Free the mirrors of `owner`: one layer, or all of them when layer < 0
    // (vulkan_backend.h:5207-5217).
    void q35_kv_drop(const void* owner, int layer);
    // Mirror budget in MiB: -1 auto (free HBM now plus the mirrors' own bytes, less a
    // margin of max(768 MiB, 1/5 of HBM) and 64 MiB of scratch), 0 off, N at most N MiB.
    // The NEXUS_GPU_KV environment variable ("off", "auto", or MiB) sets the start value.
    void set_gpu_kv_mb(int mb);
    int gpu_kv_mb();
    size_t kv_mirror_used() const { return kv_mirror_used_; }
    size_t kv_mirror_cap_bytes();
    // Row store of the mirror: truncating (default, bit-identical to the host cache that
    // stores the returned K/V with KVCache::store) or round-to-nearest-even (the shader's
    // packHalf2x16).
    void set_mirror_store_rne(bool rne) { mirror_rne_ = rne; }
    // Introspection for tests and logs.
    bool kv_mirror_info(const void* owner, int layer, size_t* cap, size_t* valid);
    bool kv_mirror_read(const void* owner, int layer, int kv_head, int pos0, int n, uint16_t* k_out,
                        uint16_t* v_out);

    // Counters for tests and logs.
    long long calls_run() const { return calls_run_; }
    long long calls_declined() const { return calls_declined_; }
    const char* last_decline() const { return last_decline_; }

private:
    struct DevBuf {
        void* ptr = nullptr;
        size_t bytes = 0;
    };
    bool decline(const char* why);
    bool ensure(DevBuf& b, size_t bytes, bool zero);
    // Shared body of the host-pointer entry points: stage, run, copy back, wait.
    bool run_host(const nexus_attn_desc& d, const float* q, const void* k_flat,
                  const void* v_flat, float* out, bool decode);
    bool run_device(const nexus_attn_desc& d, const void* q, const uint16_t* k,
                    const uint16_t* v, void* out, int n_splits, bool decode, void* stream);

    struct KvMirror {                                    // vulkan_backend.h:823
        DevBuf k, v;
        size_t cap = 0, valid = 0, bytes = 0, refused_need = 0;
        uint32_t n_kv = 0, hd = 0;
    };
    bool alloc_exact(DevBuf& b, size_t bytes);
    void free_buf(DevBuf& b);
    void drop_locked(const void* owner, int layer);

    std::mutex mu_;
    std::map<std::pair<const void*, int>, KvMirror> mirrors_;
    size_t kv_mirror_used_ = 0;
    int gpu_kv_mb_ = -2;                                 // -2: not read from the environment yet
    bool mirror_rne_ = false;
    DevBuf prep_kv_, prep_par_;
    // chained q35_attention: pinned K/V ring, kChainKvSlots slots of kChainSlotFloats
    static constexpr size_t kChainSlotFloats = 2 * 16 * 512;   // 2 x n_kv <= 16 x hd <= 512
    float* chain_ring_ = nullptr;
    bool chain_open_ = false;
    void* chain_stream_ = nullptr;
    bool ready_ = false;
    int device_ = -1;
    void* stream_ = nullptr;                 // hipStream_t
    DevBuf q_, k_, v_, o_, ws_;
    void* ws_done_ = nullptr;                // hipEvent_t recorded after the last launch using ws_
    // Order a launch that uses ws_ on `stream` after the previous one, and record it.
    bool ws_acquire(void* stream);
    void ws_release(void* stream);
    long long calls_run_ = 0, calls_declined_ = 0;
    const char* last_decline_ = "";
};

// Process-wide backend bound to device 0 on first use (the reference's gpu::gpu()
// singleton, vulkan_backend.h:6079-6082).
HipAttnBackend& backend();

}  // namespace hip
}  // namespace nexus

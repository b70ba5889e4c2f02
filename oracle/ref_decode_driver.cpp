// oracle/ref_decode_driver.cpp -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// Thin C entry points around the reference's OWN CPU code, compiled from the
// reference sources where they lie (oracle/Makefile target `ref`, output only in
// oracle/_ref/).  Nothing from the reference is copied here; this file only calls:
//   nexus::model::AttentionLayer::forward_cached_scores   model/attention.h:1201-1259
//   nexus::model::KVCache::{init, store, write_raw, read_raw, set_n_tokens, pack_k, pack_v}
//                                                          model/kvcache.h:69-78,148-178,214-241,655-672
//   nexus::model::KVCache::f32_to_f16_rne                  model/kvcache.h:256-274
//   nexus::quant::f16_to_f32                               gguf/quant.h:128-161
//   nexus::cpu::rms_norm                                   cpu/matmul.h:1860-1880
//   nexus::model::rope_apply                               model/attention.h:491-608
// Transformer::attn_batch_cpu (model/transformer.h:8653-8685) is NOT built: its header
// pulls in the Vulkan backend and the prebuilt SPIR-V blob headers, so it is restated
// in attn_oracle.c and pinned against forward_cached_scores row by row instead.
#include "model/attention.h"

#include <cstdint>
#include <cstring>
#include <vector>

using nexus::model::AttentionConfig;
using nexus::model::AttentionLayer;
using nexus::model::KVCache;

extern "C" {

// Decode of one token at `pos` over keys [0, pos] of a single-layer cache whose
// kv head h holds K[h][0..pos] (row stride kv_stride tokens).  Returns 0 on success.
int ref_forward_cached_scores(const float* q, float* out, const uint16_t* K, const uint16_t* V,
                              long kv_stride, int n_q_heads, int n_kv_heads, int head_dim,
                              int pos, float scale, float softcap, int n_threads)
{
    KVCache kv;
    kv.init(1, n_kv_heads, head_dim);
    for (int h = 0; h < n_kv_heads; ++h) {
        const size_t off = (size_t)h * (size_t)kv_stride * head_dim;
        if (!kv.write_raw(0, h, 0, pos + 1, K + off, V + off)) return -1;
    }
    kv.set_n_tokens(pos + 1);
    AttentionConfig cfg;
    cfg.n_heads = n_q_heads;
    cfg.n_kv_heads = n_kv_heads;
    cfg.head_dim = head_dim;
    cfg.scale = scale;
    cfg.n_threads = n_threads;
    cfg.attn_softcap = softcap;
    cfg.sliding_window = 0;
    AttentionLayer layer;
    layer.forward_cached_scores(q, out, kv, 0, pos, cfg);
    return 0;
}

// KVCache::store of `n_tok` tokens (f32 [n_tok][n_kv_heads*head_dim] each for K and V)
// followed by pack_k/pack_v of [0, n_tok): writes the packed f16 [n_kv][n_tok][hd] bits.
int ref_kv_store_pack(const float* k, const float* v, int n_tok, int n_kv_heads, int head_dim,
                      uint16_t* k_packed, uint16_t* v_packed)
{
    KVCache kv;
    kv.init(1, n_kv_heads, head_dim);
    const int kv_dim = n_kv_heads * head_dim;
    for (int p = 0; p < n_tok; ++p)
        kv.store(0, p, k + (size_t)p * kv_dim, v + (size_t)p * kv_dim, kv_dim);
    kv.pack_k(0, n_tok, k_packed);
    kv.pack_v(0, n_tok, v_packed);
    return kv.n_tokens() == n_tok ? 0 : -1;
}

// Slot capacity the reference's growth policy reaches after storing positions 0..n_tok-1.
long ref_kv_capacity_after(int n_tok, int head_dim)
{
    KVCache kv;
    kv.init(1, 1, head_dim);
    std::vector<float> z((size_t)head_dim, 0.f);
    for (int p = 0; p < n_tok; ++p) kv.store(0, p, z.data(), z.data(), head_dim);
    return (long)kv.slot_capacity(0, 0);
}

uint16_t ref_f32_to_f16_rne(float f) { return KVCache::f32_to_f16_rne(f); }

float ref_f16_to_f32(uint16_t h) { return nexus::quant::f16_to_f32(h); }

void ref_rms_norm(const float* x, const float* w, float* y, long n, float eps)
{
    nexus::cpu::rms_norm(x, w, y, (size_t)n, eps);
}

// Standard RoPE (type 0) of one head in place; layout 0 = interleaved, 1 = rotate_half.
void ref_rope_apply(float* x, int pos, int head_dim, float freq_base, int layout)
{
    nexus::model::RoPEConfig cfg;
    cfg.freq_base = freq_base;
    cfg.layout = layout;
    nexus::model::rope_apply(x, pos, head_dim, cfg);
}

}  // extern "C"

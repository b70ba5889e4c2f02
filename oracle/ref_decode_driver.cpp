// oracle/ref_decode_driver.cpp -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// Thin C entry points around the reference's OWN CPU code, compiled from the
// reference sources where they lie (oracle/Makefile target `ref`, output only in
// oracle/_ref/).  Nothing from the reference is copied here; this file only calls:
//   nexus::model::AttentionLayer::forward_cached_scores   model/attention.h:1201-1259
//   nexus::model::KVCache::{init, store, write_raw, read_raw, set_n_tokens, pack_k, pack_v}
//                                                          model/kvcache.h:69-78,148-178,214-241,655-672
//   nexus::model::KVCache::f32_to_f16_rne                  model/kvcache.h:256-274
//   nexus::model::KVCache::{init_per_layer, save, save_to_buffer, save_layer_to_buffer,
//                           load_from_buffer, load_layer_from_buffer}
//                                                          model/kvcache.h:88-109,352-551
//   nexus::quant::f16_to_f32                               gguf/quant.h:128-161
//   nexus::cpu::rms_norm                                   cpu/matmul.h:1860-1880
//   nexus::model::rope_apply                               model/attention.h:491-608
// Transformer::attn_batch_cpu (model/transformer.h:8653-8685) is NOT built: its header
// pulls in the Vulkan backend and the prebuilt SPIR-V blob headers, so it is restated
// in attn_oracle.c and pinned against forward_cached_scores row by row instead.
#include <chrono>
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

// Seconds per call of forward_cached_scores (the CPU baseline of the decode configs): the cache
// is filled once, untimed, then `reps` calls are timed back to back with the reference's own
// threading (n_threads: heads in parallel on its shared pool, attention.h:1255-1257).  Returns
// -1 when the cache cannot be filled.
double ref_time_cached_scores(const float* q, float* out, const uint16_t* K, const uint16_t* V,
                              long kv_stride, int n_q_heads, int n_kv_heads, int head_dim,
                              int pos, float scale, float softcap, int n_threads, int reps)
{
    KVCache kv;
    kv.init(1, n_kv_heads, head_dim);
    for (int h = 0; h < n_kv_heads; ++h) {
        const size_t off = (size_t)h * (size_t)kv_stride * head_dim;
        if (!kv.write_raw(0, h, 0, pos + 1, K + off, V + off)) return -1.0;
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
    layer.forward_cached_scores(q, out, kv, 0, pos, cfg);          // warm: pool threads, pages
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < reps; ++i) layer.forward_cached_scores(q, out, kv, 0, pos, cfg);
    const auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double>(t1 - t0).count() / (reps > 0 ? reps : 1);
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

// ---- KV session formats through the reference's own KVCache (kvcache.h:352-551).
// Geometry: layer l has nh[l] kv heads of dim hd[l] (per_layer != 0: init_per_layer, else
// init with nh[0]/hd[0] for every layer).  Rows of layer l, head h live at
// K[l] + h * stride * hd[l] (and V[l]); a layer with K[l] == NULL stays empty.

namespace {
void ref_kv_build(KVCache& kv, int n_layers, const int* nh, const int* hd, int per_layer)
{
    if (per_layer) kv.init_per_layer(std::vector<int>(nh, nh + n_layers), std::vector<int>(hd, hd + n_layers));
    else kv.init(n_layers, nh[0], hd[0]);
}

int ref_kv_fill(KVCache& kv, int n_layers, const int* nh, const int* hd, const uint16_t* const* K,
                const uint16_t* const* V, long stride, int n_tok)
{
    for (int l = 0; l < n_layers; ++l) {
        if (!K[l] || n_tok == 0) continue;
        for (int h = 0; h < nh[l]; ++h) {
            const size_t off = (size_t)h * (size_t)stride * (size_t)hd[l];
            if (!kv.write_raw(l, h, 0, n_tok, K[l] + off, V[l] + off)) return -1;
        }
    }
    kv.set_n_tokens(n_tok);
    return 0;
}

long ref_kv_out(const std::vector<uint8_t>& buf, uint8_t* out, long cap)
{
    if ((long)buf.size() <= cap && !buf.empty()) std::memcpy(out, buf.data(), buf.size());
    return (long)buf.size();
}

int ref_kv_read(KVCache& kv, int n_layers, const int* nh, uint16_t* const* K, uint16_t* const* V, long stride,
                const int* hd, int n_tok)
{
    for (int l = 0; l < n_layers; ++l) {
        if (!K[l] || n_tok == 0) continue;
        for (int h = 0; h < nh[l]; ++h) {
            const size_t off = (size_t)h * (size_t)stride * (size_t)hd[l];
            if (!kv.read_raw(l, h, 0, n_tok, K[l] + off, V[l] + off)) return -1;
        }
    }
    return 0;
}
}  // namespace

// save_to_buffer (NXKVCACH): returns the image size (copied to out when it fits).
long ref_kv_save_cache(int n_layers, const int* nh, const int* hd, int per_layer, const uint16_t* const* K,
                       const uint16_t* const* V, long stride, int n_tok, uint8_t* out, long cap)
{
    KVCache kv;
    ref_kv_build(kv, n_layers, nh, hd, per_layer);
    if (ref_kv_fill(kv, n_layers, nh, hd, K, V, stride, n_tok) != 0) return -1;
    return ref_kv_out(kv.save_to_buffer(), out, cap);
}

// save(path) (NXKVCACH file): 0 on success.
int ref_kv_save_file(const char* path, int n_layers, const int* nh, const int* hd, int per_layer,
                     const uint16_t* const* K, const uint16_t* const* V, long stride, int n_tok)
{
    KVCache kv;
    ref_kv_build(kv, n_layers, nh, hd, per_layer);
    if (ref_kv_fill(kv, n_layers, nh, hd, K, V, stride, n_tok) != 0) return -1;
    return kv.save(path) ? 0 : -1;
}

// save_layer_to_buffer (NXKVLYR1) of `layer`.
long ref_kv_save_layer(int n_layers, const int* nh, const int* hd, int per_layer, const uint16_t* const* K,
                       const uint16_t* const* V, long stride, int n_tok, int layer, uint8_t* out, long cap)
{
    KVCache kv;
    ref_kv_build(kv, n_layers, nh, hd, per_layer);
    if (ref_kv_fill(kv, n_layers, nh, hd, K, V, stride, n_tok) != 0) return -1;
    return ref_kv_out(kv.save_layer_to_buffer(layer), out, cap);
}

// load_from_buffer (NXKVCACH) into a fresh cache, rows read back with read_raw: returns the
// token count, or -1 when the reference refuses the image.
int ref_kv_load_cache(int n_layers, const int* nh, const int* hd, int per_layer, const uint8_t* data, long size,
                      uint16_t* const* K, uint16_t* const* V, long stride)
{
    KVCache kv;
    ref_kv_build(kv, n_layers, nh, hd, per_layer);
    if (!kv.load_from_buffer(data, (size_t)size)) return -1;
    const int n_tok = kv.n_tokens();
    if (n_tok > stride || ref_kv_read(kv, n_layers, nh, K, V, stride, hd, n_tok) != 0) return -1;
    return n_tok;
}

// load_layer_from_buffer (NXKVLYR1) into a fresh cache: returns the token count afterwards.
int ref_kv_load_layer(int n_layers, const int* nh, const int* hd, int per_layer, const uint8_t* data, long size,
                      uint16_t* const* K, uint16_t* const* V, long stride)
{
    KVCache kv;
    ref_kv_build(kv, n_layers, nh, hd, per_layer);
    if (!kv.load_layer_from_buffer(data, (size_t)size)) return -1;
    const int n_tok = kv.n_tokens();
    if (n_tok > stride || ref_kv_read(kv, n_layers, nh, K, V, stride, hd, n_tok) != 0) return -1;
    return n_tok;
}

}  // extern "C"

/*
 * nexus_hip_kv.h -- KV session formats straight to and from device-resident KV caches.
 *
 * The reference saves and restores its KV cache (src/model/kvcache.h) in two formats:
 *   NXKVCACH  the whole cache, KVCache::save / save_to_buffer / load / load_from_buffer
 *             (kvcache.h:352-372, 427-449, 476-551): magic "NXKVCACH", int32
 *             {n_layers, n_kv_heads, head_dim, n_tokens}, then for every layer and every
 *             kv head of that layer: K [n_tokens][hd_l] f16, then V [n_tokens][hd_l] f16.
 *             n_kv_heads / head_dim in the header are the largest over the layers (the
 *             per-layer geometry of KVCache::init_per_layer, kvcache.h:88-109); layers
 *             without KV take no bytes.  A "legacy" file, written when every layer had the
 *             header geometry (zero blocks for layers without KV), is recognised by its
 *             size and read with those blocks skipped (kvcache.h:452-474).
 *   NXKVLYR1  one layer, KVCache::save_layer_to_buffer / load_layer_from_buffer
 *             (kvcache.h:383-426): magic "NXKVLYR1", int32 {layer, n_kv_heads, head_dim,
 *             n_tokens}, then per kv head K then V as above.
 * Byte order is the host's (little-endian), as the reference writes it.
 *
 * Here the cache lives in HBM as one pair of f16 arrays per layer, K and V
 * [n_kv_heads][row_stride][head_dim] (the device mirror layout the attention entry points
 * read, kv_row_stride = row_stride), described by nexus_kv_layer_view.  Rows [0, n_tokens)
 * of every head move between device memory and the file/buffer with DMA copies; no host
 * copy of the cache is built.  The file forms stream through two pinned staging buffers
 * so disk and PCIe transfers overlap.
 *
 * All calls are synchronous (they return once the data has arrived) and validate the whole
 * request -- header, geometry, sizes, capacity -- before the first copy: a call that
 * returns an error has not touched device memory or the output buffer (the reference
 * can stop part-way through a truncated buffer; this library does not) -- except a read
 * that fails part-way through a file (NEXUS_E_IO), which can leave rows of the device
 * cache partly overwritten.  Errors are the
 * nexus_status codes of nexus_hip_attn.h, with the message in nexus_hip_attn_last_error().
 */
#ifndef NEXUS_HIP_KV_H
#define NEXUS_HIP_KV_H

#include <stddef.h>
#include <stdint.h>

#include "nexus_hip_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One layer's device cache. */
typedef struct nexus_kv_layer_view {
    uint16_t* k;             /* device f16 [n_kv_heads][row_stride][head_dim]               */
    uint16_t* v;             /* NULL on save: the layer is written as zeros (no data yet)   */
    int32_t n_kv_heads;      /* 0: a layer without KV (e.g. linear attention)               */
    int32_t head_dim;        /* > 0 when n_kv_heads > 0                                     */
    int64_t row_stride;      /* rows per head, >= the tokens saved or loaded                */
} nexus_kv_layer_view;

/* Bytes of an NXKVLYR1 record / an NXKVCACH image holding n_tokens tokens (0 when the
 * layer has no KV, as save_layer_to_buffer returns an empty buffer; 0 on bad arguments). */
size_t nexus_hip_kv_layer_bytes(const nexus_kv_layer_view* view, int n_tokens);
size_t nexus_hip_kv_cache_bytes(const nexus_kv_layer_view* views, int n_layers, int n_tokens);

/* NXKVLYR1: write layer `layer`'s rows [0, n_tokens) into buf (buf_bytes >=
 * nexus_hip_kv_layer_bytes).  Replaces KVCache::save_layer_to_buffer. */
int nexus_hip_kv_layer_save(int layer, const nexus_kv_layer_view* view, int n_tokens,
                            void* buf, size_t buf_bytes, nexus_stream_t stream);
/* NXKVLYR1: apply one record to views[record's layer] (n_layers views, one per layer);
 * *layer_out and *n_tokens_out receive the record's layer and token count.  Replaces
 * KVCache::load_layer_from_buffer. */
int nexus_hip_kv_layer_load(const void* buf, size_t buf_bytes,
                            const nexus_kv_layer_view* views, int n_layers,
                            int* layer_out, int* n_tokens_out, nexus_stream_t stream);

/* NXKVCACH in memory.  Replace KVCache::save_to_buffer / load_from_buffer. */
int nexus_hip_kv_cache_save(const nexus_kv_layer_view* views, int n_layers, int n_tokens,
                            void* buf, size_t buf_bytes, nexus_stream_t stream);
int nexus_hip_kv_cache_load(const void* buf, size_t buf_bytes,
                            const nexus_kv_layer_view* views, int n_layers,
                            int* n_tokens_out, nexus_stream_t stream);

/* NXKVCACH files.  Replace KVCache::save / load (kvcache.h:352-372, 509-551). */
int nexus_hip_kv_cache_save_file(const char* path, const nexus_kv_layer_view* views,
                                 int n_layers, int n_tokens, nexus_stream_t stream);
int nexus_hip_kv_cache_load_file(const char* path, const nexus_kv_layer_view* views,
                                 int n_layers, int* n_tokens_out, nexus_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* NEXUS_HIP_KV_H */

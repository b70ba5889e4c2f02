/*
 * oracle/attn_oracle.h -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * CPU restatement of sjnettifee/Nexus's own CPU attention, used only as the
 * parity checker for the HIP kernels and as the timed CPU baseline ("port").
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product library never links it and never falls back to it.
 *
 * Layouts (identical to the reference):
 *   Q   f32  [n_query][n_q_heads][head_dim]
 *   K,V f16  [n_kv_heads][kv_stride][head_dim]   (kv_stride = n_ctx when packed,
 *                                                 = slot capacity for KVCache slots)
 *   Out f32  [n_query][n_q_heads][head_dim]
 *   GQA map: kv head = h * n_kv_heads / n_q_heads   (transformer.h:8667)
 */
#ifndef NEXUS_ATTN_ORACLE_H
#define NEXUS_ATTN_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 -> binary32, subnormals/inf/nan included (quant.h:140-161). */
float    nx_f16_bits_to_f32(uint16_t h);
/* KVCache::store conversion: truncating, f16 subnormals flushed to signed zero,
 * overflow to +-inf (kvcache.h:903-911). */
uint16_t nx_f32_to_f16_trunc(float f);
/* KVCache::f32_to_f16_rne (kvcache.h:256-274). */
uint16_t nx_f32_to_f16_rne(float f);
void     nx_f32_to_f16_trunc_n(const float* in, uint16_t* out, size_t n);
void     nx_f32_to_f16_rne_n(const float* in, uint16_t* out, size_t n);
void     nx_f16_to_f32_n(const uint16_t* in, float* out, size_t n);

/* Transformer::attn_batch_cpu (transformer.h:8653-8685): per (query, head) online
 * softmax with m=-1e30, l=0, f16->f32 decode of every K/V element, tanh softcap,
 * causal window [start, min(q_base+qi, n_ctx-1)].  kv_stride generalises the packed
 * layout (the reference passes n_ctx).  n_threads > 1 parallelises over (query, head)
 * rows for the all-cores baseline; n_threads == 1 is the reference's threading. */
void oracle_attn_batch(const float* Q, const uint16_t* K, const uint16_t* V, float* Out,
                       int n_q_heads, int n_kv_heads, int head_dim,
                       int n_ctx, long kv_stride, int n_query, int q_base_pos,
                       int sliding_window, float scale, float softcap, int n_threads);

/* Same as oracle_attn_batch but only for the (query, head) rows listed in rows[]
 * (row index = qi * n_q_heads + h); used for bounded CPU-baseline samples. */
void oracle_attn_batch_rows(const float* Q, const uint16_t* K, const uint16_t* V, float* Out,
                            int n_q_heads, int n_kv_heads, int head_dim,
                            int n_ctx, long kv_stride, int n_query, int q_base_pos,
                            int sliding_window, float scale, float softcap,
                            const int* rows, int n_rows, int n_threads);

/* AttentionLayer::forward_cached_scores (attention.h:1201-1259): decode of one token at
 * position pos over keys [0, pos]; two-pass softmax (max, expf, divide by the sum),
 * Pade tanh softcap (attention.h:232-252), weights below 1e-9 skipped in the V sum.
 * Parallel over heads when n_threads > 1 (the reference's ThreadPool). scale 0 = 1/sqrt(hd). */
void oracle_cached_scores(const float* q, float* out, const uint16_t* K, const uint16_t* V,
                          long kv_stride, int n_q_heads, int n_kv_heads, int head_dim,
                          int pos, float scale, float softcap, int n_threads);

/* Split-K decode semantics (qwen35_attn_part.comp:1-108): for every (q head, chunk of
 * `chunk` keys) write acc[hd] = sum exp(s-m_c) v, m_c, l_c to part[h][c][hd+2].
 * n_query > 1 rows use the causal rule of attn_batch_cpu (row = qi*Hq + h). */
void oracle_split_partials(const float* Q, const uint16_t* K, const uint16_t* V, float* part,
                           int n_q_heads, int n_kv_heads, int head_dim,
                           int n_ctx, long kv_stride, int n_query, int q_base_pos,
                           float scale, int n_chunks, int chunk);
/* qwen35_attn_comb.comp:1-41 without the gate: out = sum_c acc_c e^{m_c-M} / sum_c l_c e^{m_c-M}. */
void oracle_split_combine(const float* part, float* out, int n_rows, int head_dim, int n_chunks);

void oracle_gate_mul(float* out, const float* gate, size_t n);

void oracle_decode_prep(int n_heads, int n_kv, int hd, int rot, int flags, float eps, int pos, long cap,
                        const float* qg, const float* kraw, const float* vraw,
                        const float* qnw, const float* knw, const float* tab,
                        float* q_out, float* gate_out, uint16_t* kc, uint16_t* vc, float* kv_out, int rne);

/* Independent checker: float64 naive softmax attention with the same mask rules. */
void oracle_naive_f64(const float* Q, const uint16_t* K, const uint16_t* V, double* Out,
                      int n_q_heads, int n_kv_heads, int head_dim,
                      int n_ctx, long kv_stride, int n_query, int q_base_pos,
                      int sliding_window, double scale, double softcap);

/* KV session formats (model/kvcache.h:352-551).  Layer l: nh[l] heads of dim hd[l], rows of
 * head h at K[l] + h * stride * hd[l].  Savers return the image size (written when <= cap);
 * legacy != 0 writes every layer at the header geometry (zero blocks for nh[l] == 0).
 * Loaders return the token count, or -1 where the reference refuses the image. */
long oracle_kv_cache_save(int n_layers, const int* nh, const int* hd, const uint16_t* const* K,
                          const uint16_t* const* V, long stride, int n_tok, uint8_t* out, long cap, int legacy);
long oracle_kv_layer_save(int layer, int nh, int hd, const uint16_t* K, const uint16_t* V, long stride, int n_tok,
                          uint8_t* out, long cap);
int oracle_kv_cache_load(int n_layers, const int* nh, const int* hd, const uint8_t* data, long size,
                         uint16_t* const* K, uint16_t* const* V, long stride);
int oracle_kv_layer_load(int n_layers, const int* nh, const int* hd, const uint8_t* data, long size,
                         uint16_t* const* K, uint16_t* const* V, long stride, int* layer_out);

#ifdef __cplusplus
}
#endif
#endif

/*
 * oracle/attn_oracle.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * Clean-room CPU restatement of sjnettifee/Nexus's CPU attention.  It is the parity
 * checker for the HIP kernels and the CPU baseline that bench.py times ("port").
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Function -> reference code it follows (paths relative to the reference's src/):
 *   nx_f16_bits_to_f32    gguf/quant.h:140-161, model/transformer.h:8659-8665
 *   nx_f32_to_f16_trunc   model/kvcache.h:903-911   (KVCache::store conversion)
 *   nx_f32_to_f16_rne     model/kvcache.h:256-274   (KVCache::f32_to_f16_rne)
 *   oracle_attn_batch     model/transformer.h:8653-8685 (Transformer::attn_batch_cpu)
 *   oracle_cached_scores  model/attention.h:1201-1259 (AttentionLayer::forward_cached_scores),
 *                         softcap via fast_tanh/attn_softcap attention.h:232-245
 *   oracle_split_partials gpu/shaders/qwen35_attn_part.comp:1-108 (partial (acc, m, l))
 *   oracle_split_combine  gpu/shaders/qwen35_attn_comb.comp:1-41 (LSE merge, no gate)
 *   oracle_gate_mul       model/transformer.h:8505-8512 (post-gate of the batched prefill;
 *                         the same clamped sigmoid as qwen35_attn_comb.comp:34-38)
 *   oracle_decode_prep    gpu/shaders/qwen35_attn_prep.comp:1-101 for one token: per-head
 *                         RMSNorm as cpu::rms_norm (cpu/matmul.h:1860-1880) or
 *                         nx_rms_norm_add_one (model/transformer.h:504-520), selected as
 *                         nx_apply_projection_norm_inplace does (transformer.h:580-618);
 *                         RoPE as rope_apply (model/attention.h:491-608) with the angle table
 *                         supplied; K/V store with kvcache.h:903-911 or :256-274 conversion
 *   oracle_kv_*           NXKVCACH / NXKVLYR1 images (model/kvcache.h:352-551): the
 *                         save_to_buffer / save_layer_to_buffer byte layout, the legacy
 *                         layout load_from_buffer still accepts, and both loaders
 *   oracle_naive_f64      independent float64 brute force (checker only)
 *
 * How each function is pinned (tests/test_oracle.py):
 *   f16 decode     exhaustively against numpy's float16 over all 2^16 codes;
 *   trunc store    against the definition "nearest f16 toward zero" (numpy nextafter),
 *                  plus flush/overflow special cases;
 *   rne store      against numpy's float16 cast (a library RNE) on 2M random patterns;
 *   cached_scores  against the reference's own forward_cached_scores compiled from its
 *                  sources (oracle/_ref) and against committed fixtures it wrote;
 *   attn_batch     every row against the reference's forward_cached_scores at that
 *                  query's position, against float64 brute force, and against closed
 *                  forms (one key, zero query, one-hot key, window of one);
 *   split/combine  split-vs-unsplit identity (LSE associativity) for many chunkings;
 *   gate_mul       against scipy's expit inside (-80, 80) and the clamp values outside;
 *   kv session     byte-for-byte against the reference's own KVCache writers and loaders
 *                  (oracle/_ref) and against fixtures they wrote (tests/golden);
 *   decode_prep    norm against the reference's own cpu::rms_norm (oracle/_ref), the (1+w)
 *                  form against it with 1+w weights; RoPE against the reference's own
 *                  rope_apply with the same angles, identity/composition/norm-preserving
 *                  invariants and the neox<->interleaved permutation; stores as above.
 */
#include "attn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- f16 <-> f32 */

float nx_f16_bits_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1fu) {
        bits = sign | 0x7f800000u | (m << 13);            /* inf / nan, payload kept */
    } else if (e != 0u) {
        bits = sign | ((e + 112u) << 23) | (m << 13);     /* normal: rebias 15 -> 127 */
    } else {
        /* zero or subnormal: the value is m * 2^-24, exact in binary32 */
        const float f = (float)m * 5.9604644775390625e-8f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t nx_f32_to_f16_trunc(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const int e16 = (int)((x >> 23) & 0xffu) - 112;      /* exponent rebias 127 -> 15 */
    if (e16 <= 0) return sign;                            /* f16 subnormal range: flush */
    if (e16 >= 31) return (uint16_t)(sign | 0x7c00u);     /* overflow, inf and nan -> inf */
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | ((x >> 13) & 0x3ffu));
}

uint16_t nx_f32_to_f16_rne(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);   /* nan -> quiet nan */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {
        /* result is an f16 subnormal (or zero / min normal after rounding):
         * round |f| * 2^24 to an integer, ties to even (exact scaling by 2^24). */
        float a;
        memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint16_t)nearbyintf(a * 16777216.0f));
    }
    /* normal: round half to even at mantissa bit 13, then rebias the exponent */
    const uint32_t r = ax + 0x0fffu + ((ax >> 13) & 1u);
    return (uint16_t)(sign | (uint16_t)((r - 0x38000000u) >> 13));
}

void nx_f32_to_f16_trunc_n(const float* in, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = nx_f32_to_f16_trunc(in[i]);
}

void nx_f32_to_f16_rne_n(const float* in, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = nx_f32_to_f16_rne(in[i]);
}

void nx_f16_to_f32_n(const uint16_t* in, float* out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = nx_f16_bits_to_f32(in[i]);
}

/* ------------------------------------------------------- attn_batch_cpu restatement */

/* One (query, head) row of Transformer::attn_batch_cpu.  acc is caller scratch [hd]. */
static void batch_row(const float* Q, const uint16_t* K, const uint16_t* V, float* Out,
                      int Hq, int Hkv, int hd, int n_ctx, long kv_stride, int q_base,
                      int sw, float scale, float softcap, int qi, int h, float* acc)
{
    const int kv = h * Hkv / Hq;
    const int qpos = q_base + qi;
    const int start = (sw > 0 && qpos + 1 > sw) ? qpos + 1 - sw : 0;
    const int last = qpos < n_ctx - 1 ? qpos : n_ctx - 1;
    const float* qh = Q + ((size_t)qi * Hq + h) * hd;
    const uint16_t* Kh = K + (size_t)kv * (size_t)kv_stride * hd;
    const uint16_t* Vh = V + (size_t)kv * (size_t)kv_stride * hd;
    float* oh = Out + ((size_t)qi * Hq + h) * hd;

    for (int e = 0; e < hd; ++e) acc[e] = 0.f;
    float m = -1e30f, l = 0.f;
    for (int p = start; p <= last; ++p) {
        const uint16_t* kr = Kh + (size_t)p * hd;
        const uint16_t* vr = Vh + (size_t)p * hd;
        float d = 0.f;
        for (int e = 0; e < hd; ++e) d += qh[e] * nx_f16_bits_to_f32(kr[e]);
        float s = d * scale;
        if (softcap > 0.f) s = softcap * tanhf(s / softcap);
        const float mn = (m < s) ? s : m;
        const float cr = expf(m - mn);
        const float w = expf(s - mn);
        for (int e = 0; e < hd; ++e) acc[e] = acc[e] * cr + w * nx_f16_bits_to_f32(vr[e]);
        l = l * cr + w;
        m = mn;
    }
    const float inv = (l > 0.f) ? 1.f / l : 0.f;
    for (int e = 0; e < hd; ++e) oh[e] = acc[e] * inv;
}

void oracle_attn_batch(const float* Q, const uint16_t* K, const uint16_t* V, float* Out,
                       int n_q_heads, int n_kv_heads, int head_dim,
                       int n_ctx, long kv_stride, int n_query, int q_base_pos,
                       int sliding_window, float scale, float softcap, int n_threads)
{
    const long n_rows = (long)n_query * n_q_heads;
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads) if (n_threads > 1)
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)head_dim);
#pragma omp for schedule(dynamic, 4)
        for (long r = 0; r < n_rows; ++r)
            batch_row(Q, K, V, Out, n_q_heads, n_kv_heads, head_dim, n_ctx, kv_stride,
                      q_base_pos, sliding_window, scale, softcap,
                      (int)(r / n_q_heads), (int)(r % n_q_heads), acc);
        free(acc);
    }
}

void oracle_attn_batch_rows(const float* Q, const uint16_t* K, const uint16_t* V, float* Out,
                            int n_q_heads, int n_kv_heads, int head_dim,
                            int n_ctx, long kv_stride, int n_query, int q_base_pos,
                            int sliding_window, float scale, float softcap,
                            const int* rows, int n_rows, int n_threads)
{
    (void)n_query;
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads) if (n_threads > 1)
    {
        float* acc = (float*)malloc(sizeof(float) * (size_t)head_dim);
#pragma omp for schedule(dynamic, 1)
        for (int i = 0; i < n_rows; ++i)
            batch_row(Q, K, V, Out, n_q_heads, n_kv_heads, head_dim, n_ctx, kv_stride,
                      q_base_pos, sliding_window, scale, softcap,
                      rows[i] / n_q_heads, rows[i] % n_q_heads, acc);
        free(acc);
    }
}

/* ------------------------------------------------ forward_cached_scores restatement */

/* Pade [5/4] tanh with clamp beyond |x| > 4.5 (attention.h:232-238). */
static float pade_tanh(float x)
{
    if (x > 4.5f) return 1.0f;
    if (x < -4.5f) return -1.0f;
    const float x2 = x * x;
    return x * (945.0f + x2 * (105.0f + x2)) / (945.0f + x2 * (420.0f + x2 * 15.0f));
}

static float pade_softcap(float x, float cap)
{
    if (cap <= 0.0f) return x;
    return pade_tanh(x * (1.0f / cap)) * cap;
}

static void cached_head(const float* q, float* out, const uint16_t* K, const uint16_t* V,
                        long kv_stride, int Hq, int Hkv, int hd, int pos, float sc,
                        float softcap, int h, float* s)
{
    const int nctx = pos + 1;
    const int kvh = h / (Hq / Hkv);
    const float* qh = q + (size_t)h * hd;
    const uint16_t* Kh = K + (size_t)kvh * (size_t)kv_stride * hd;
    const uint16_t* Vh = V + (size_t)kvh * (size_t)kv_stride * hd;
    for (int t = 0; t < nctx; ++t) {
        const uint16_t* kr = Kh + (size_t)t * hd;
        float d = 0.f;
        for (int e = 0; e < hd; ++e) d += qh[e] * nx_f16_bits_to_f32(kr[e]);
        s[t] = pade_softcap(d * sc, softcap);
    }
    float mx = s[0];
    for (int t = 1; t < nctx; ++t) if (s[t] > mx) mx = s[t];
    float sum = 0.f;
    for (int t = 0; t < nctx; ++t) { s[t] = expf(s[t] - mx); sum += s[t]; }
    if (sum > 0.f) for (int t = 0; t < nctx; ++t) s[t] /= sum;
    float* oh = out + (size_t)h * hd;
    for (int e = 0; e < hd; ++e) oh[e] = 0.f;
    for (int t = 0; t < nctx; ++t) {
        const float w = s[t];
        if (w < 1e-9f) continue;                          /* attention.h:1242 */
        const uint16_t* vr = Vh + (size_t)t * hd;
        for (int e = 0; e < hd; ++e) oh[e] += w * nx_f16_bits_to_f32(vr[e]);
    }
}

void oracle_cached_scores(const float* q, float* out, const uint16_t* K, const uint16_t* V,
                          long kv_stride, int n_q_heads, int n_kv_heads, int head_dim,
                          int pos, float scale, float softcap, int n_threads)
{
    const float sc = scale != 0.f ? scale : 1.f / sqrtf((float)head_dim);
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads) if (n_threads > 1)
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)(pos + 1));
#pragma omp for schedule(dynamic, 1)
        for (int h = 0; h < n_q_heads; ++h)
            cached_head(q, out, K, V, kv_stride, n_q_heads, n_kv_heads, head_dim, pos, sc,
                        softcap, h, s);
        free(s);
    }
}

/* ------------------------------------------------------------ split-K semantics */

void oracle_split_partials(const float* Q, const uint16_t* K, const uint16_t* V, float* part,
                           int n_q_heads, int n_kv_heads, int head_dim,
                           int n_ctx, long kv_stride, int n_query, int q_base_pos,
                           float scale, int n_chunks, int chunk)
{
    const int hd = head_dim;
    const size_t stride = (size_t)hd + 2;
    float* sc = (float*)malloc(sizeof(float) * (size_t)chunk);
    for (int qi = 0; qi < n_query; ++qi) {
        const int last = q_base_pos + qi < n_ctx - 1 ? q_base_pos + qi : n_ctx - 1;
        for (int h = 0; h < n_q_heads; ++h) {
            const int kv = h * n_kv_heads / n_q_heads;
            const float* qh = Q + ((size_t)qi * n_q_heads + h) * hd;
            const uint16_t* Kh = K + (size_t)kv * (size_t)kv_stride * hd;
            const uint16_t* Vh = V + (size_t)kv * (size_t)kv_stride * hd;
            const size_t row = (size_t)qi * n_q_heads + h;
            for (int c = 0; c < n_chunks; ++c) {
                float* pr = part + (row * (size_t)n_chunks + (size_t)c) * stride;
                const int k0 = c * chunk;
                int k1 = k0 + chunk - 1;
                if (k1 > last) k1 = last;
                float m = -1e30f;
                for (int k = k0; k <= k1; ++k) {
                    float d = 0.f;
                    for (int e = 0; e < hd; ++e) d += qh[e] * nx_f16_bits_to_f32(Kh[(size_t)k * hd + e]);
                    sc[k - k0] = d * scale;
                    if (sc[k - k0] > m) m = sc[k - k0];
                }
                float l = 0.f;
                for (int e = 0; e < hd; ++e) pr[e] = 0.f;
                for (int k = k0; k <= k1; ++k) {
                    const float p = expf(sc[k - k0] - m);
                    l += p;
                    for (int e = 0; e < hd; ++e) pr[e] += p * nx_f16_bits_to_f32(Vh[(size_t)k * hd + e]);
                }
                pr[hd] = m;
                pr[hd + 1] = l;
            }
        }
    }
    free(sc);
}

void oracle_split_combine(const float* part, float* out, int n_rows, int head_dim, int n_chunks)
{
    const size_t stride = (size_t)head_dim + 2;
    for (int r = 0; r < n_rows; ++r) {
        const float* pr = part + (size_t)r * n_chunks * stride;
        float M = -3.0e38f;
        for (int c = 0; c < n_chunks; ++c) if (pr[c * stride + head_dim] > M) M = pr[c * stride + head_dim];
        float L = 0.f;
        for (int c = 0; c < n_chunks; ++c) L += expf(pr[c * stride + head_dim] - M) * pr[c * stride + head_dim + 1];
        for (int d = 0; d < head_dim; ++d) {
            float a = 0.f;
            for (int c = 0; c < n_chunks; ++c) a += pr[c * stride + d] * expf(pr[c * stride + head_dim] - M);
            out[(size_t)r * head_dim + d] = L > 0.f ? a / L : 0.f;
        }
    }
}

/* -------------------------------------------------------------------- output gate */

/* out[i] *= sigmoid(gate[i]) with the clamp of model/transformer.h:8508-8510. */
void oracle_gate_mul(float* out, const float* gate, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        const float z = gate[i];
        const float s = (z > 80.0f) ? 1.0f : (z < -80.0f) ? 0.0f : 1.0f / (1.0f + expf(-z));
        out[i] *= s;
    }
}

/* ------------------------------------------------------------------- decode prep */

/* RMSNorm of one head row in place.  zc = 0: (x * w) * inv as cpu::rms_norm
 * (cpu/matmul.h:1876-1880); zc = 1: x * inv * (1 + w) as nx_rms_norm_add_one
 * (model/transformer.h:511-520).  inv = 1 / sqrtf(sum x^2 / n + eps). */
static void head_rms_norm(float* x, const float* w, int n, float eps, int zc)
{
    float ss = 0.0f;
    for (int i = 0; i < n; ++i) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; ++i) x[i] = zc ? x[i] * inv * (1.0f + w[i]) : (x[i] * w[i]) * inv;
}

/* RoPE of the first `rot` dims of one head row in place, angles from tab (cos at tab[i],
 * sin at tab[rot/2 + i]); interleaved pairs (2i, 2i+1) or rotate_half pairs (i, i + rot/2),
 * the two layouts of rope_apply (model/attention.h:593-608). */
static void head_rope(float* x, int rot, const float* tab, int interleaved)
{
    const int half = rot / 2;
    for (int i = 0; i < half; ++i) {
        const float c = tab[i], s = tab[half + i];
        if (interleaved) {
            const float x0 = x[2 * i], x1 = x[2 * i + 1];
            x[2 * i] = x0 * c - x1 * s;
            x[2 * i + 1] = x0 * s + x1 * c;
        } else {
            const float x0 = x[i], x1 = x[i + half];
            x[i] = x0 * c - x1 * s;
            x[i + half] = x1 * c + x0 * s;
        }
    }
}

/* One token of qwen35_attn_prep.comp.  qg: per head [q(hd) | gate(hd)] (flags & 4: plain q
 * [n_heads][hd]); kraw/vraw [n_kv][hd]; qnw/knw [hd] (unused when the norm is off);
 * tab [rot].  Writes q_out [n_heads][hd], gate_out [n_heads][hd] (gated layers), the f16
 * bits of K and V into kc/vc [n_kv][cap][hd] at row `pos`, and kv_out [2][n_kv][hd] (f32
 * K then V as stored).  flags: 1 q norm (1+w), 2 k norm (1+w), 4 no gate, 8 no q norm,
 * 16 no k norm, 32 interleaved RoPE.  rne = 0: truncating store (kvcache.h:903-911). */
void oracle_decode_prep(int n_heads, int n_kv, int hd, int rot, int flags, float eps, int pos, long cap,
                        const float* qg, const float* kraw, const float* vraw,
                        const float* qnw, const float* knw, const float* tab,
                        float* q_out, float* gate_out, uint16_t* kc, uint16_t* vc, float* kv_out, int rne)
{
    const int gated = (flags & 4) == 0, inter = (flags & 32) != 0;
    float* row = (float*)malloc((size_t)hd * sizeof(float));
    for (int h = 0; h < n_heads; ++h) {
        const float* src = gated ? qg + (size_t)h * 2 * hd : qg + (size_t)h * hd;
        memcpy(row, src, (size_t)hd * sizeof(float));
        if (gated) memcpy(gate_out + (size_t)h * hd, src + hd, (size_t)hd * sizeof(float));
        if (!(flags & 8)) head_rms_norm(row, qnw, hd, eps, flags & 1);
        head_rope(row, rot, tab, inter);
        memcpy(q_out + (size_t)h * hd, row, (size_t)hd * sizeof(float));
    }
    for (int which = 0; which < 2; ++which) {
        for (int h = 0; h < n_kv; ++h) {
            memcpy(row, (which ? vraw : kraw) + (size_t)h * hd, (size_t)hd * sizeof(float));
            if (which == 0) {
                if (!(flags & 16)) head_rms_norm(row, knw, hd, eps, flags & 2);
                head_rope(row, rot, tab, inter);
            }
            uint16_t* dst = (which ? vc : kc) + ((size_t)h * cap + pos) * hd;
            for (int d = 0; d < hd; ++d) dst[d] = rne ? nx_f32_to_f16_rne(row[d]) : nx_f32_to_f16_trunc(row[d]);
            memcpy(kv_out + ((size_t)which * n_kv + h) * hd, row, (size_t)hd * sizeof(float));
        }
    }
    free(row);
}

/* ------------------------------------------------------------ KV session formats */

/* Header geometry: the largest head count / head dim over the layers (KVCache::init_per_layer,
 * kvcache.h:88-109). */
static void kv_header_geometry(int n_layers, const int* nh, const int* hd, int32_t* mh, int32_t* md)
{
    *mh = 0;
    *md = 0;
    for (int l = 0; l < n_layers; ++l) {
        if (nh[l] > *mh) *mh = nh[l];
        if (hd[l] > *md) *md = hd[l];
    }
}

static uint8_t* kv_put_header(uint8_t* p, const char* magic, int32_t a, int32_t b, int32_t c, int32_t d)
{
    const int32_t hdr[4] = {a, b, c, d};
    memcpy(p, magic, 8);
    memcpy(p + 8, hdr, sizeof(hdr));
    return p + 24;
}

/* K then V of every head of one layer, rows [0, n_tok); K == NULL writes zeros. */
static uint8_t* kv_put_layer(uint8_t* p, int nh, int hd, const uint16_t* K, const uint16_t* V, long stride, int n_tok)
{
    const size_t blk = (size_t)n_tok * (size_t)hd * 2;
    for (int h = 0; h < nh; ++h) {
        const size_t off = (size_t)h * (size_t)stride * (size_t)hd;
        if (K) memcpy(p, K + off, blk); else memset(p, 0, blk);
        p += blk;
        if (V) memcpy(p, V + off, blk); else memset(p, 0, blk);
        p += blk;
    }
    return p;
}

long oracle_kv_cache_save(int n_layers, const int* nh, const int* hd, const uint16_t* const* K,
                          const uint16_t* const* V, long stride, int n_tok, uint8_t* out, long cap, int legacy)
{
    int32_t mh, md;
    kv_header_geometry(n_layers, nh, hd, &mh, &md);
    size_t total = 24;
    for (int l = 0; l < n_layers; ++l) {
        const int h = legacy ? mh : nh[l], d = legacy ? md : hd[l];
        total += (size_t)h * (size_t)n_tok * (size_t)d * 4;
    }
    if ((long)total > cap) return (long)total;
    uint8_t* p = kv_put_header(out, "NXKVCACH", n_layers, mh, md, n_tok);
    for (int l = 0; l < n_layers; ++l) {
        if (legacy && nh[l] == 0) p = kv_put_layer(p, mh, md, NULL, NULL, 0, n_tok);
        else p = kv_put_layer(p, nh[l], hd[l], K[l], V[l], stride, n_tok);
    }
    return (long)total;
}

long oracle_kv_layer_save(int layer, int nh, int hd, const uint16_t* K, const uint16_t* V, long stride, int n_tok,
                          uint8_t* out, long cap)
{
    if (nh == 0) return 0;
    const size_t total = 24 + (size_t)nh * (size_t)n_tok * (size_t)hd * 4;
    if ((long)total > cap) return (long)total;
    kv_put_layer(kv_put_header(out, "NXKVLYR1", layer, nh, hd, n_tok), nh, hd, K, V, stride, n_tok);
    return (long)total;
}

static const uint8_t* kv_get_layer(const uint8_t* p, int nh, int hd, uint16_t* K, uint16_t* V, long stride, int n_tok)
{
    const size_t blk = (size_t)n_tok * (size_t)hd * 2;
    for (int h = 0; h < nh; ++h) {
        const size_t off = (size_t)h * (size_t)stride * (size_t)hd;
        memcpy(K + off, p, blk);
        p += blk;
        memcpy(V + off, p, blk);
        p += blk;
    }
    return p;
}

int oracle_kv_cache_load(int n_layers, const int* nh, const int* hd, const uint8_t* data, long size,
                         uint16_t* const* K, uint16_t* const* V, long stride)
{
    int32_t mh, md, hdr[4];
    if (size < 24 || memcmp(data, "NXKVCACH", 8) != 0) return -1;
    memcpy(hdr, data + 8, sizeof(hdr));
    kv_header_geometry(n_layers, nh, hd, &mh, &md);
    if (hdr[0] != n_layers || hdr[1] != mh || hdr[2] != md || hdr[3] < 0 || hdr[3] > stride) return -1;
    const int n_tok = hdr[3];
    size_t cur = 24, old = 24;
    for (int l = 0; l < n_layers; ++l) {
        cur += (size_t)nh[l] * (size_t)n_tok * (size_t)hd[l] * 4;
        old += (size_t)mh * (size_t)n_tok * (size_t)md * 4;
    }
    const int legacy = old != cur && (size_t)size == old;
    if (!legacy && (size_t)size < cur) return -1;
    const uint8_t* p = data + 24;
    for (int l = 0; l < n_layers; ++l) {
        if (legacy && nh[l] == 0) { p += (size_t)mh * (size_t)n_tok * (size_t)md * 4; continue; }
        if (p + (size_t)nh[l] * (size_t)n_tok * (size_t)hd[l] * 4 > data + size) return -1;
        p = kv_get_layer(p, nh[l], hd[l], K[l], V[l], stride, n_tok);
    }
    return n_tok;
}

int oracle_kv_layer_load(int n_layers, const int* nh, const int* hd, const uint8_t* data, long size,
                         uint16_t* const* K, uint16_t* const* V, long stride, int* layer_out)
{
    int32_t hdr[4];
    if (size < 24 || memcmp(data, "NXKVLYR1", 8) != 0) return -1;
    memcpy(hdr, data + 8, sizeof(hdr));
    const int l = hdr[0];
    if (l < 0 || l >= n_layers || hdr[1] != nh[l] || hdr[2] != hd[l] || hdr[3] < 0 || hdr[3] > stride) return -1;
    if (24 + (size_t)nh[l] * (size_t)hdr[3] * (size_t)hd[l] * 4 > (size_t)size) return -1;
    kv_get_layer(data + 24, nh[l], hd[l], K[l], V[l], stride, hdr[3]);
    *layer_out = l;
    return hdr[3];
}

/* ------------------------------------------------------------ float64 brute force */

void oracle_naive_f64(const float* Q, const uint16_t* K, const uint16_t* V, double* Out,
                      int n_q_heads, int n_kv_heads, int head_dim,
                      int n_ctx, long kv_stride, int n_query, int q_base_pos,
                      int sliding_window, double scale, double softcap)
{
    const int hd = head_dim;
    double* s = (double*)malloc(sizeof(double) * (size_t)(n_ctx > 0 ? n_ctx : 1));
    for (int qi = 0; qi < n_query; ++qi) {
        const int qpos = q_base_pos + qi;
        for (int h = 0; h < n_q_heads; ++h) {
            const int kv = h * n_kv_heads / n_q_heads;
            const float* qh = Q + ((size_t)qi * n_q_heads + h) * hd;
            const uint16_t* Kh = K + (size_t)kv * (size_t)kv_stride * hd;
            const uint16_t* Vh = V + (size_t)kv * (size_t)kv_stride * hd;
            double* oh = Out + ((size_t)qi * n_q_heads + h) * hd;
            for (int e = 0; e < hd; ++e) oh[e] = 0.0;
            double mx = -INFINITY;
            int any = 0;
            for (int p = 0; p < n_ctx; ++p) {
                const int visible = p <= qpos && !(sliding_window > 0 && p < qpos + 1 - sliding_window);
                if (!visible) { s[p] = -INFINITY; continue; }
                double d = 0.0;
                for (int e = 0; e < hd; ++e) d += (double)qh[e] * (double)nx_f16_bits_to_f32(Kh[(size_t)p * hd + e]);
                d *= scale;
                if (softcap > 0.0) d = softcap * tanh(d / softcap);
                s[p] = d;
                if (d > mx) mx = d;
                any = 1;
            }
            if (!any) continue;
            double sum = 0.0;
            for (int p = 0; p < n_ctx; ++p) {
                if (s[p] == -INFINITY) continue;
                const double w = exp(s[p] - mx);
                sum += w;
                for (int e = 0; e < hd; ++e) oh[e] += w * (double)nx_f16_bits_to_f32(Vh[(size_t)p * hd + e]);
            }
            for (int e = 0; e < hd; ++e) oh[e] /= sum;
        }
    }
    free(s);
}

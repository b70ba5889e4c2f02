// tests/cpp/engine_prefill.cpp -- TEST INFRASTRUCTURE: a one-layer, Engine-shaped prompt
// attention driver over nexus::hip::HipAttnBackend, so the tests can run the exact sequence
// the reference's engine runs around its GPU attention call, tile by tile:
//
//   Transformer::layer_batch_tiled (src/model/transformer.h:8551-8651): a prompt of n tokens
//   is cut into n_tiles = ceil(n / T) even tiles (T = NEXUS_PREFILL_TILE, default 1024), the
//   last one never a lone token; each tile is one call of
//   Transformer::forward_full_attn_prefill_layer_batch, whose attention section
//   (transformer.h:8443-8515) does:
//     1. KVCache::store of every token of the tile, serially, with the cache's truncating
//        f32 -> f16 conversion (kvcache.h:148-178, 903-911);
//     2. KVCache::pack_k / pack_v of rows [0, n_ctx) into [n_kv][n_ctx][hd] (kvcache.h:655-672);
//     3. attention_flash_gpu; on decline attention_batch_gpu (NEXUS_ATTN_PATH=batch) or
//        attention_stream_gpu; on decline attn_batch_cpu -- the GPU only for tiles of 16 or
//        more tokens (transformer.h:8342);
//     4. the post-gate: out *= sigmoid(gate), 1 above 80, 0 below -80 (transformer.h:8502-8515).
//
// The host cache keeps the KVCache slot layout: per kv head f16 [capacity][hd], capacity
// 512 tokens at first, doubled up to 8192, then grown by 4096 (kvcache.h:715-730, 856-873).
// The engine's CPU attention (step 3's last resort) is the test oracle's restatement of
// attn_batch_cpu: this driver stands in for the engine, it is not the product.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "attn_oracle.h"
#include "hip_attn_backend.h"

using nexus::hip::backend;

namespace {

struct HostKvCache {                        // one layer of KVCache
    int n_kv = 0, hd = 0;
    size_t cap = 0;
    std::vector<std::vector<uint16_t>> k, v;   // [n_kv] -> [cap][hd]

    void ensure(size_t need)
    {
        if (need <= cap) return;
        size_t nc = cap == 0 ? 512 : (cap < 8192 ? cap * 2 : cap + 4096);
        while (nc < need) nc += nc < 8192 ? nc : 4096;
        for (int h = 0; h < n_kv; ++h) {
            k[h].resize(nc * hd, 0);
            v[h].resize(nc * hd, 0);
        }
        cap = nc;
    }
    void store(int pos, const float* krow, const float* vrow)    // krow: [n_kv * hd]
    {
        ensure((size_t)pos + 1);
        for (int h = 0; h < n_kv; ++h)
            for (int d = 0; d < hd; ++d) {
                k[h][(size_t)pos * hd + d] = nx_f32_to_f16_trunc(krow[h * hd + d]);
                v[h][(size_t)pos * hd + d] = nx_f32_to_f16_trunc(vrow[h * hd + d]);
            }
    }
    void pack(int n_ctx, uint16_t* kout, uint16_t* vout) const
    {
        for (int h = 0; h < n_kv; ++h) {
            memcpy(kout + (size_t)h * n_ctx * hd, k[h].data(), (size_t)n_ctx * hd * sizeof(uint16_t));
            memcpy(vout + (size_t)h * n_ctx * hd, v[h].data(), (size_t)n_ctx * hd * sizeof(uint16_t));
        }
    }
};

constexpr uint32_t kSentinel = 0x7fc0dead;   // a NaN no attention output can produce

bool untouched(const float* p, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        uint32_t b;
        memcpy(&b, p + i, 4);
        if (b != kSentinel) return false;
    }
    return true;
}

void fill_sentinel(float* p, size_t n)
{
    for (size_t i = 0; i < n; ++i) memcpy(p + i, &kSentinel, 4);
}

}  // namespace

extern "C" {

enum {
    EH_GATED = 1,            // the layer has the Qwen3.5 output gate
    EH_NO_GPU_FALLBACK = 2,  // a declined flash call goes to the CPU attention directly
    EH_BATCHED = 4,          // NEXUS_ATTN_PATH=batch: attention_batch_gpu as the GPU fallback
};

struct eh_layer {
    int n_heads, n_kv, head_dim;
    float scale, softcap;    // scale 0: 1/sqrt(head_dim)
    int tile;                // NEXUS_PREFILL_TILE; <= 0: the whole prompt in one call
    int flags;
    int cpu_threads;
};

void* eh_cache_new(int n_kv, int head_dim)
{
    HostKvCache* c = new HostKvCache;
    c->n_kv = n_kv;
    c->hd = head_dim;
    c->k.resize(n_kv);
    c->v.resize(n_kv);
    return c;
}

void eh_cache_free(void* c) { delete (HostKvCache*)c; }

long eh_cache_capacity(void* c) { return (long)((HostKvCache*)c)->cap; }

// Rows [pos0, pos0 + n) of kv head h as stored (f16 bits); 0 when out of range.
int eh_cache_read(void* cv, int h, int pos0, int n, uint16_t* k_out, uint16_t* v_out)
{
    const HostKvCache* c = (const HostKvCache*)cv;
    if (h < 0 || h >= c->n_kv || pos0 < 0 || n < 0 || (size_t)pos0 + n > c->cap) return 0;
    memcpy(k_out, c->k[h].data() + (size_t)pos0 * c->hd, (size_t)n * c->hd * sizeof(uint16_t));
    memcpy(v_out, c->v[h].data() + (size_t)pos0 * c->hd, (size_t)n * c->hd * sizeof(uint16_t));
    return 1;
}

// The prompt tokens [start_pos, start_pos + n_tokens) of one layer.  Q and gate:
// [n_tokens][n_heads * hd]; K and V (after RoPE, before the store): [n_tokens][n_kv * hd];
// out: [n_tokens][n_heads * hd].  path[i] = 0 flash, 1 batch/stream on the GPU, 2 CPU for
// tile i; *clean = 1 when every declined GPU call left its tile's output untouched.  Returns
// the number of tiles (at most max_tiles are recorded).
int eh_prefill_layer(const eh_layer* L, void* cache, int start_pos, int n_tokens, const float* Q, const float* K,
                     const float* V, const float* gate, float* out, int* path, int max_tiles, int* clean)
{
    HostKvCache& kv = *(HostKvCache*)cache;
    const int hd = L->head_dim, q_dim = L->n_heads * hd, kv_dim = L->n_kv * hd;
    const float scale = L->scale != 0.f ? L->scale : 1.0f / std::sqrt((float)hd);
    std::vector<uint16_t> kflat, vflat;
    *clean = 1;

    // one call of the batched layer over tokens [t0, t0 + cnt) of the prompt
    auto layer_call = [&](int t0, int cnt) -> int {
        const int pos0 = start_pos + t0;
        for (int t = 0; t < cnt; ++t)                          // the KV store stays serial
            kv.store(pos0 + t, K + (size_t)(t0 + t) * kv_dim, V + (size_t)(t0 + t) * kv_dim);
        const int n_ctx = pos0 + cnt;
        kflat.resize((size_t)L->n_kv * n_ctx * hd);
        vflat.resize(kflat.size());
        kv.pack(n_ctx, kflat.data(), vflat.data());
        const float* q = Q + (size_t)t0 * q_dim;
        float* ao = out + (size_t)t0 * q_dim;
        const size_t n_out = (size_t)cnt * q_dim;
        const bool on_card = cnt >= 16;
        int used = 2;
        fill_sentinel(ao, n_out);
        if (on_card && backend().attention_flash_gpu(q, ao, L->n_heads, L->n_kv, hd, n_ctx, cnt, pos0, 0, scale,
                                                     L->softcap, kflat.data(), vflat.data())) {
            used = 0;
        } else {
            if (!untouched(ao, n_out)) *clean = 0;
            bool ok = false;
            if (on_card && !(L->flags & EH_NO_GPU_FALLBACK)) {
                ok = (L->flags & EH_BATCHED)
                         ? backend().attention_batch_gpu(q, ao, L->n_heads, L->n_kv, hd, n_ctx, cnt, pos0, 0, scale,
                                                         L->softcap, kflat.data(), vflat.data(),
                                                         kflat.size() * sizeof(uint16_t))
                         : backend().attention_stream_gpu(q, ao, L->n_heads, L->n_kv, hd, n_ctx, cnt, pos0, scale,
                                                          L->softcap, kflat.data(), vflat.data(), 0);
                if (ok) used = 1;
                else if (!untouched(ao, n_out)) *clean = 0;
            }
            if (!ok)
                oracle_attn_batch(q, kflat.data(), vflat.data(), ao, L->n_heads, L->n_kv, hd, n_ctx, n_ctx, cnt, pos0,
                                  0, scale, L->softcap, L->cpu_threads > 0 ? L->cpu_threads : 1);
        }
        if (L->flags & EH_GATED) {                             // post-gate
            const float* gt = gate + (size_t)t0 * q_dim;
            for (size_t i = 0; i < n_out; ++i) {
                const float z = gt[i];
                const float s = (z > 80.0f) ? 1.0f : (z < -80.0f) ? 0.0f : 1.0f / (1.0f + std::exp(-z));
                ao[i] *= s;
            }
        }
        return used;
    };

    int n_tiles = 0;
    auto record = [&](int used) {
        if (n_tiles < max_tiles) path[n_tiles] = used;
        ++n_tiles;
    };
    const int T = L->tile;
    if (T <= 0 || n_tokens <= T) {
        record(layer_call(0, n_tokens));
        return n_tiles;
    }
    const int tiles = (n_tokens + T - 1) / T;
    const int tile = (n_tokens + tiles - 1) / tiles;           // even split
    for (int t0 = 0; t0 < n_tokens;) {
        int cnt = tile < n_tokens - t0 ? tile : n_tokens - t0;
        if (n_tokens - t0 - cnt == 1) ++cnt;                   // never a lone last token
        record(layer_call(t0, cnt));
        t0 += cnt;
    }
    return n_tiles;
}

}  // extern "C"

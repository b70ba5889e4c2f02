/*
 * nexus_hip_attn.h -- C ABI of the MI355X (gfx950) attention kernels.
 *
 * This is the drop-in boundary for Nexus's attention operator.  The reference engine
 * calls its GPU attention through VulkanBackend member functions that take host
 * pointers and return `false` (before any side effect) when they cannot run:
 *   attention_flash_gpu   src/gpu/vulkan_backend.h:604-608 (impl :4260-4408)
 *   attention_batch_gpu   src/gpu/vulkan_backend.h:584-588 (impl :3819-3934)
 *   attention_stream_gpu  src/gpu/vulkan_backend.h:594-599 (impl :4085-4257)
 *   attention_gpu         src/gpu/vulkan_backend.h:576-580 (impl :3731-3817)
 *   q35_full_layer's attention core (split-K part + comb over the device KV mirror)
 *                         src/gpu/vulkan_backend.h:5272-5483,
 *                         src/gpu/shaders/qwen35_attn_part.comp, qwen35_attn_comb.comp
 * The C++ backend in nexus_amd/host/hip_attn_backend.h keeps those member signatures and
 * calls the two entry points below with device pointers.  All calls are asynchronous
 * on the given stream; the library allocates nothing on these paths.
 *
 * Layouts (identical to the reference):
 *   Q    [n_query][n_q_heads][head_dim]           f32 or f16 (q_dtype)
 *   K, V [n_kv_heads][kv_row_stride][head_dim]    f16 bit patterns (uint16)
 *        kv_row_stride = n_ctx for the packed layout of KVCache::pack_k/pack_v
 *        (src/model/kvcache.h:655-672), = slot capacity for the device mirror
 *        [kv_head][cap][hd] (src/gpu/vulkan_backend.h:488, 5411)
 *   Out  [n_query][n_q_heads][head_dim]           f32 or f16 (o_dtype)
 *   GQA: q head h reads kv head h * n_kv_heads / n_q_heads (attn_flash.comp:55)
 *   Mask: query i sits at absolute position q_base_pos + i and sees keys
 *         [start, min(q_base_pos + i, n_ctx - 1)], start = q_pos + 1 - sliding_window
 *         when sliding_window > 0 (transformer.h:8666-8670); a query that sees no key
 *         writes zeros (transformer.h:8682).
 *   Scores: s = (q.k) * scale, then softcap * tanh(s / softcap) when softcap > 0.
 *
 * Errors: every entry point validates its arguments first and returns a negative
 * code WITHOUT launching anything or touching any output when it declines; the C++
 * wrapper maps that to the reference's `return false` (caller uses the CPU path).
 */
#ifndef NEXUS_HIP_ATTN_H
#define NEXUS_HIP_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers (it is `struct ihipStream_t*`). */
typedef struct ihipStream_t* nexus_stream_t;

enum nexus_dtype {
    NEXUS_DT_F32 = 0,
    NEXUS_DT_F16 = 1
};

enum nexus_status {
    NEXUS_OK              = 0,
    NEXUS_E_UNSUPPORTED   = -1,   /* shape the kernels do not cover (declined, like nx_decline) */
    NEXUS_E_INVALID       = -2,   /* null pointer or inconsistent argument */
    NEXUS_E_WORKSPACE     = -3,   /* workspace missing or too small for the requested split */
    NEXUS_E_LAUNCH        = -4,   /* the HIP runtime refused the launch or a copy */
    NEXUS_E_IO            = -5    /* a file could not be opened, read or written (nexus_hip_kv.h) */
};

/* One attention call.  Mirrors the push constants of attn_flash.comp:18-31
 * {Hq, Hkv, hd, n_ctx, n_query, q_base_pos, sliding_window, scale, softcap}
 * plus the row stride of the cache and the Q/O element types. */
typedef struct nexus_attn_desc {
    int32_t n_q_heads;       /* Hq  (> 0, multiple of n_kv_heads)                    */
    int32_t n_kv_heads;      /* Hkv (> 0)                                            */
    int32_t head_dim;        /* 64, 128, 192 or 256 (reference: hd % 64 == 0, <= 256) */
    int32_t n_query;         /* queries in this call (> 0)                           */
    int32_t q_base_pos;      /* absolute position of query 0 (>= 0)                  */
    int32_t n_ctx;           /* keys [0, n_ctx) are valid in K/V (> 0)               */
    int64_t kv_row_stride;   /* tokens between kv heads in K/V (>= n_ctx)            */
    int32_t sliding_window;  /* 0 = off                                              */
    float   scale;           /* 0 = 1/sqrt(head_dim)                                 */
    float   softcap;         /* 0 = off                                              */
    int32_t q_dtype;         /* enum nexus_dtype                                     */
    int32_t o_dtype;         /* enum nexus_dtype                                     */
} nexus_attn_desc;

/* Causal GQA flash-attention prefill over an f16 cache: cold prompts (q_base_pos = 0)
 * and prompt chunks appended after q_base_pos cached tokens.  Replaces
 * attention_flash_gpu / attention_batch_gpu / attention_stream_gpu
 * (src/gpu/vulkan_backend.h:584-608).  The workspace lets the library split a long key
 * range over several workgroups (its size comes from nexus_hip_attn_prefill_ws_bytes();
 * NULL/0, or a smaller one, runs unsplit); split partials are merged by a second launch
 * on the same stream.  Short chunks (n_query * G <= 32, e.g. speculative verify, and a few
 * more queries behind long caches) run through the split-KV decode kernels when the
 * workspace allows.  The workspace holds f32 partials only and carries no state between
 * calls (no zeroing needed); calls in flight at once must not share it. */
int nexus_hip_attn_prefill(const nexus_attn_desc* desc,
                           const void* q, const uint16_t* k, const uint16_t* v, void* out,
                           void* workspace, size_t workspace_bytes,
                           nexus_stream_t stream);
size_t nexus_hip_attn_prefill_ws_bytes(const nexus_attn_desc* desc);

/* The launch plan nexus_hip_attn_prefill(_gated) follows for `desc` when given
 * nexus_hip_attn_prefill_ws_bytes() bytes of workspace, on the current device (256 compute
 * units when no device is visible).  No counterpart in the reference: a diagnostic that lets
 * tests and tuning check a shape's route without timing it.  Returns NEXUS_OK, or the shape
 * error nexus_hip_attn_prefill would return for `desc`. */
enum { NEXUS_PLAN_PREFILL = 0, NEXUS_PLAN_DECODE = 1 };
typedef struct nexus_attn_prefill_plan {
    int32_t kernel;      /* NEXUS_PLAN_PREFILL: pipelined prefill kernel; NEXUS_PLAN_DECODE: split-KV decode kernel */
    int32_t block_rows;  /* rows per workgroup: 64 or 128 (prefill), 16 or 32 (decode)       */
    int32_t splits;      /* key splits; above 1 a combine launch follows                     */
    int32_t packed;      /* 1: prefill blocks over the (query, head-in-group) rows of a kv head */
    int32_t workgroups;  /* workgroups of the attention launch                               */
} nexus_attn_prefill_plan;
int nexus_hip_attn_prefill_plan(const nexus_attn_desc* desc, nexus_attn_prefill_plan* plan);

/* Split-KV decode over the cache: n_query >= 1 tokens at positions q_base_pos + i
 * (n_query = 1 is ordinary decode, n_query > 1 is speculative/MTP verify with the
 * causal mask among the drafts).  Replaces attention_gpu (vulkan_backend.h:576-580)
 * and the attention core of q35_full_layer (part + comb, vulkan_backend.h:5462-5482).
 * Two launches on `stream`, like the reference's part + comb: every split writes its
 * partial, then the combine merges them (one split writes `out` directly).  partial_ws
 * must hold nexus_hip_attn_decode_ws_bytes() bytes: f32 partials holding, per row
 * (n_query * n_q_heads of them) and split, (sum_k e^{s_k - m} v_k, m, l) exactly as
 * qwen35_attn_part.comp:3 defines them, stored as acc [n_splits][rows][head_dim] followed
 * by (m, l) [n_splits][rows][2] (16-byte stores, a split's rows contiguous).  It
 * carries no state between calls; calls in flight at once must not share it.
 * n_splits <= 0 lets the library choose. */
int nexus_hip_attn_decode(const nexus_attn_desc* desc,
                          const void* q, const uint16_t* k, const uint16_t* v, void* out,
                          float* partial_ws, int n_splits,
                          nexus_stream_t stream);
size_t nexus_hip_attn_decode_ws_bytes(const nexus_attn_desc* desc, int n_splits);
/* The split count nexus_hip_attn_decode uses when called with n_splits <= 0. */
int nexus_hip_attn_decode_default_splits(const nexus_attn_desc* desc);

/* The two calls above with the output gate of the gated attention layers fused into the
 * epilogue: out = attention * sigmoid(gate), with sigmoid clamped to 1 above 80 and to 0
 * below -80.  Replaces the gate of qwen35_attn_comb.comp:34-38 (decode, inside the
 * combine) and the post-gate of the batched prefill (src/model/transformer.h:8502-8515).
 * gate: f32 [n_query][n_q_heads][head_dim] on the device, 16-byte aligned; NULL = no gate
 * (the plain entries above). */
int nexus_hip_attn_prefill_gated(const nexus_attn_desc* desc,
                                 const void* q, const uint16_t* k, const uint16_t* v,
                                 const float* gate, void* out,
                                 void* workspace, size_t workspace_bytes,
                                 nexus_stream_t stream);
int nexus_hip_attn_decode_gated(const nexus_attn_desc* desc,
                                const void* q, const uint16_t* k, const uint16_t* v,
                                const float* gate, void* out,
                                float* partial_ws, int n_splits,
                                nexus_stream_t stream);

/* Allocation-free decode.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  nexus_hip_attn_decode_gated with the split partials in a fixed
 * device array of NEXUS_DECODE_NOALLOC_SCRATCH_BYTES that the library keeps on every GPU
 * it runs on until the process ends, instead of a caller workspace; it calls no hipMalloc,
 * hipFree or allocating library routine.  n_splits <= 0: the default split count, lowered
 * until the partials fit; an explicit n_splits whose partials exceed the array returns
 * NEXUS_E_WORKSPACE with nothing launched.  All calls on one GPU share the array: calls
 * that overlap on one GPU (several streams at once) race on it, so keep one in flight per
 * GPU.  The first call on a device looks up that device's array address. */
#define NEXUS_DECODE_NOALLOC_SCRATCH_BYTES (8u << 20)
int nexus_hip_attn_decode_noalloc(const nexus_attn_desc* desc,
                                  const void* q, const uint16_t* k, const uint16_t* v,
                                  const float* gate, void* out, int n_splits,
                                  nexus_stream_t stream);

/* Decode prep for one token, the step before the decode call in the gated (and plain)
 * full-attention layers: per-head RMSNorm of q and k, RoPE over the first rot_dims dims
 * from a host cos/sin table, the f16 store of K and V into row `pos` of the device cache,
 * and an f32 echo of the stored K/V for the host cache.  Replaces
 * qwen35_attn_prep.comp:1-101 as dispatched by q35_full_layer
 * (src/gpu/vulkan_backend.h:5446-5460); the descriptor carries that shader's push
 * constants {n_heads, n_kv, hd, rot, pos, cap, flags, eps}.
 * Layouts (device, f32 unless noted):
 *   qg        [n_heads][2*head_dim] per head q | gate; [n_heads][head_dim] with NO_GATE
 *   k_raw, v_raw [n_kv_heads][head_dim]
 *   q_norm_w, k_norm_w [head_dim] (read only when that norm is on)
 *   rope_tab  [rot_dims]: cos(theta_i) for i < rot_dims/2, then sin(theta_i)
 *   q_out     [n_heads][head_dim] normed + roped q;  gate_out [n_heads][head_dim] raw gate
 *   k_cache, v_cache [n_kv_heads][cap][head_dim] f16 bits: row `pos` written
 *   kv_out    [2][n_kv_heads][head_dim]: K then V as stored (before the f16 rounding)
 * Norm: x * inv * (1 + w) with the ADD_ONE flag (nx_rms_norm_add_one,
 * src/model/transformer.h:504-520), else (x * w) * inv (cpu::rms_norm,
 * src/cpu/matmul.h:1860-1880), inv = 1/sqrt(mean(x^2) + eps).  RoPE pairs (i, i + rot/2),
 * or (2i, 2i+1) with ROPE_INTERLEAVED (rope_apply, src/model/attention.h:593-608).
 * f16 store: round to nearest even like the shader's packHalf2x16, or, with TRUNC_STORE,
 * the host cache's own truncating conversion (KVCache::store, src/model/kvcache.h:903-911)
 * so a device mirror stays bit-identical to the host cache. */
enum nexus_prep_flags {
    NEXUS_PREP_Q_NORM_ADD_ONE   = 1,
    NEXUS_PREP_K_NORM_ADD_ONE   = 2,
    NEXUS_PREP_NO_GATE          = 4,
    NEXUS_PREP_NO_Q_NORM        = 8,
    NEXUS_PREP_NO_K_NORM        = 16,
    NEXUS_PREP_ROPE_INTERLEAVED = 32,
    NEXUS_PREP_TRUNC_STORE      = 64    /* no counterpart in the shader (see above) */
};

typedef struct nexus_attn_prep_desc {
    int32_t n_heads;         /* q heads (> 0)                                  */
    int32_t n_kv_heads;      /* k/v heads (> 0)                                */
    int32_t head_dim;        /* 1..512 (the shader's limit)                    */
    int32_t rot_dims;        /* even, 0..head_dim                              */
    int32_t pos;             /* cache row written, 0 <= pos < cap              */
    int32_t flags;           /* enum nexus_prep_flags                          */
    int64_t cap;             /* rows per kv head in k_cache / v_cache          */
    float   eps;             /* RMSNorm epsilon (>= 0)                         */
    int32_t reserved;        /* 0                                              */
} nexus_attn_prep_desc;

int nexus_hip_attn_decode_prep(const nexus_attn_prep_desc* desc,
                               const float* qg, const float* k_raw, const float* v_raw,
                               const float* q_norm_w, const float* k_norm_w, const float* rope_tab,
                               float* q_out, float* gate_out,
                               uint16_t* k_cache, uint16_t* v_cache, float* kv_out,
                               nexus_stream_t stream);

/* The attention of one decode token of a full-attention layer, prep included: what
 * nexus_hip_attn_decode_prep followed by nexus_hip_attn_decode_gated computes over
 * k_cache / v_cache rows [0, pos] (row pos being the new token), in two launches instead of
 * three.  Replaces the prep + part + comb dispatches of q35_full_layer
 * (src/gpu/vulkan_backend.h:5446-5482).  The split-KV kernel normalises and rotates q in its
 * prologue; the workgroups of the split that holds key `pos` prepare the new K/V row
 * themselves, attend it, and store it into row `pos` of the caches and into kv_out, so no
 * workgroup reads a row written in the same launch; the combine applies the gate, read from
 * qg.  Arguments as for nexus_hip_attn_decode_prep (q_out / gate_out are not produced),
 * plus the attention scale (0: 1/sqrt(head_dim)) and:
 *   out        [n_heads][head_dim] f32: the gated attention output
 *   partial_ws nexus_hip_attn_decode_layer_ws_bytes(desc, n_splits) bytes (split partials)
 *   n_splits   <= 0 lets the library choose, as nexus_hip_attn_decode does.
 * head_dim 64, 128, 192 or 256; the caches hold at least pos + 1 rows (cap > pos). */
int nexus_hip_attn_decode_layer(const nexus_attn_prep_desc* desc, float scale,
                                const float* qg, const float* k_raw, const float* v_raw,
                                const float* q_norm_w, const float* k_norm_w, const float* rope_tab,
                                uint16_t* k_cache, uint16_t* v_cache, float* kv_out, float* out,
                                float* partial_ws, int n_splits, nexus_stream_t stream);
size_t nexus_hip_attn_decode_layer_ws_bytes(const nexus_attn_prep_desc* desc, int n_splits);
/* The split count nexus_hip_attn_decode_layer uses when called with n_splits <= 0. */
int nexus_hip_attn_decode_layer_default_splits(const nexus_attn_prep_desc* desc);

/* Message for the last non-zero status on the calling thread ("" if none). */
const char* nexus_hip_attn_last_error(void);
/* Library version, e.g. "nexus_hip_attn 0.1.0 gfx950". */
const char* nexus_hip_attn_version(void);

#ifdef __cplusplus
}
#endif
#endif /* NEXUS_HIP_ATTN_H */

// nexus_amd/csrc/attn_capi.cpp -- the C ABI declared in include/nexus_hip_attn.h.
//
// Every entry point validates the whole call before it launches anything, so a
// declined call (negative status) leaves every output untouched -- the contract of the
// reference's GPU attention ops, which `return false` before any side effect
// (src/gpu/vulkan_backend.h:4267-4277 for attention_flash_gpu, :5290-5308 for the
// decode split-K; nx_decline :187-192).
#include "nexus_hip_attn.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "attn_kernels.h"
#include "capi_status.h"

namespace {
thread_local char g_last_error[512] = "";
}  // namespace

int nxa::capi_fail(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int nxa::capi_ok()
{
    g_last_error[0] = '\0';
    return NEXUS_OK;
}

namespace {

using nxa::capi_fail;
int ok() { return nxa::capi_ok(); }

constexpr int kMaxDevices = 64;
using nxa::kMaxSplits;

// Compute units of the current device (cached); 256 (MI355X) when no device is visible,
// so workspace sizing is still defined on a host without a GPU.
int device_cus()
{
    static int cache[kMaxDevices] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return 256;
    }
    if (cache[dev] > 0) return cache[dev];
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
        (void)hipGetLastError();
        return 256;
    }
    cache[dev] = cus;
    return cus;
}

bool supported_head_dim(int hd) { return hd == 64 || hd == 128 || hd == 192 || hd == 256; }

// Shape checks shared by both entry points (pointer checks are separate so that the
// sizing helpers can reuse this).  Mirrors the reference's declines: head_dim % 64 != 0
// or > 256, Hq % Hkv != 0, non-positive sizes (vulkan_backend.h:4270-4273).
int check_desc(const nexus_attn_desc* d)
{
    if (!d) return capi_fail(NEXUS_E_INVALID, "desc is NULL");
    if (d->n_q_heads <= 0 || d->n_kv_heads <= 0 || d->n_q_heads % d->n_kv_heads != 0)
        return capi_fail(NEXUS_E_UNSUPPORTED, "n_q_heads=%d must be a positive multiple of n_kv_heads=%d",
                    d->n_q_heads, d->n_kv_heads);
    if (!supported_head_dim(d->head_dim))
        return capi_fail(NEXUS_E_UNSUPPORTED, "head_dim=%d not in {64,128,192,256}", d->head_dim);
    if (d->n_query <= 0 || d->n_ctx <= 0 || d->q_base_pos < 0)
        return capi_fail(NEXUS_E_INVALID, "n_query=%d n_ctx=%d q_base_pos=%d", d->n_query, d->n_ctx, d->q_base_pos);
    if ((long long)d->q_base_pos + d->n_query > INT_MAX - 4096 || d->n_ctx > INT_MAX - 4096)
        return capi_fail(NEXUS_E_UNSUPPORTED, "positions exceed the 31-bit range");
    if ((long long)d->n_ctx * d->head_dim * 2 >= (1LL << 31))
        return capi_fail(NEXUS_E_UNSUPPORTED, "n_ctx * head_dim exceeds the 2 GiB per-kv-head buffer range");
    if ((long long)d->n_query * d->n_q_heads * d->head_dim * 4 >= (1LL << 31))
        return capi_fail(NEXUS_E_UNSUPPORTED, "n_query * n_q_heads * head_dim exceeds the 2 GiB query buffer range");
    if (d->kv_row_stride < d->n_ctx)
        return capi_fail(NEXUS_E_INVALID, "kv_row_stride=%lld < n_ctx=%d", (long long)d->kv_row_stride, d->n_ctx);
    if (d->sliding_window < 0) return capi_fail(NEXUS_E_INVALID, "sliding_window=%d", d->sliding_window);
    if (!(d->scale >= 0.f) || !std::isfinite(d->scale)) return capi_fail(NEXUS_E_INVALID, "scale=%g", (double)d->scale);
    if (!(d->softcap >= 0.f) || !std::isfinite(d->softcap)) return capi_fail(NEXUS_E_INVALID, "softcap=%g", (double)d->softcap);
    if ((d->q_dtype != NEXUS_DT_F32 && d->q_dtype != NEXUS_DT_F16) ||
        (d->o_dtype != NEXUS_DT_F32 && d->o_dtype != NEXUS_DT_F16))
        return capi_fail(NEXUS_E_UNSUPPORTED, "q_dtype=%d o_dtype=%d", d->q_dtype, d->o_dtype);
    return NEXUS_OK;
}

float eff_scale(const nexus_attn_desc* d)
{
    return d->scale > 0.f ? d->scale : 1.0f / std::sqrt((float)d->head_dim);
}

bool is_ext(const nexus_attn_desc* d) { return d->sliding_window > 0 || d->softcap > 0.f; }

// Key range any query of the call can see: [k_begin, k_end).
void key_range(const nexus_attn_desc* d, int* k_begin, int* k_end)
{
    const long long last = std::min<long long>((long long)d->q_base_pos + d->n_query - 1, (long long)d->n_ctx - 1);
    long long b = 0;
    if (d->sliding_window > 0 && (long long)d->q_base_pos + 1 > d->sliding_window)
        b = (long long)d->q_base_pos + 1 - d->sliding_window;
    const long long e = last + 1;
    if (b > e) b = e;
    *k_begin = (int)b;
    *k_end = (int)e;
}

long long decode_rows(const nexus_attn_desc* d)
{
    return (long long)d->n_query * (d->n_q_heads / d->n_kv_heads);
}

// 16-row tiles per workgroup: two when the rows need more than one tile, so a 32-row verify
// batch (4 drafts x 8 heads) shares every K/V byte the workgroup stages.
int decode_row_tiles(const nexus_attn_desc* d)
{
    return decode_rows(d) > nxa::kDecodeRowTile ? nxa::kDecodeMaxRowTiles : 1;
}

int decode_rowgroups(const nexus_attn_desc* d)
{
    const long long per = (long long)nxa::kDecodeRowTile * decode_row_tiles(d);
    return (int)((decode_rows(d) + per - 1) / per);
}

// Keys per split at least: two 32-key stages of the ring.
constexpr long long kDecodeMinSplitKeys = 64;

int default_decode_splits(const nexus_attn_desc* d)
{
    int kb, ke;
    key_range(d, &kb, &ke);
    const long long kv_len = ke - kb;
    const long long base = (long long)d->n_kv_heads * decode_rowgroups(d);
    // as many workgroups as are resident at once (one wave of the grid): a second wave would
    // pay the per-workgroup start (Q load, ring prologue) and the partial again
    const long long target = (long long)nxa::decode_wg_per_cu(d->head_dim) * device_cus();
    long long s = target / base;
    if (s < 1) s = 1;
    const long long by_len = (kv_len + kDecodeMinSplitKeys - 1) / kDecodeMinSplitKeys;
    if (s > by_len) s = by_len;
    if (s < 1) s = 1;
    if (s > kMaxSplits) s = kMaxSplits;
    return (int)s;
}

size_t decode_ws_bytes(const nexus_attn_desc* d, int n_splits)
{
    return nxa::ws_partial_bytes((long long)d->n_query * d->n_q_heads, n_splits, d->head_dim);
}

size_t prefill_split_ws_bytes(const nexus_attn_desc* d, int splits)
{
    return nxa::ws_partial_bytes((long long)d->n_query * d->n_q_heads, splits, d->head_dim);
}

// Split count of a prefill grid of `base` query-block workgroups.  Splitting costs a partial
// write + read per row and split plus a combine launch, so a grid of at least one workgroup per
// CU stays whole (320 pipelined workgroups of 64 queries x 40 heads in 2 splits took 96 us
// against 62 unsplit).  Below that the key range is split so the grid reaches about one
// workgroup per CU, or two at head dims <= 128 (two resident per CU; a workgroup alone on its CU
// runs one wave per SIMD) while each split keeps >= 12 key tiles of 64; always >= 4 tiles per
// split and at most 64 splits.  Measured on MI355X: 40q/8kv hd 128, 200/256 queries over 32k
// keys in 160 workgroups 432/427 us, split three ways 192/204 us; 32q/8kv, 256 over 16k (128
// workgroups) 187 -> 90 us; 32/48/64 queries over 32k at one workgroup per CU 61/75/89 us, at two
// 48/54/62 us, 64 over 12k (16 tiles per split at two) 36 -> 33 us; 24 over 9k (4 tiles per split
// at two) 18 -> 24 us, 64 over 9k (12 tiles) 27.3 -> 27.7 us; 16q/2kv hd 256
// behind 32k keys, 32/48 queries at most 16 splits 76/80 us, 64 splits 43/52 us; 24q/4kv hd 192,
// 32 queries 93 -> 49 us; 4-head MHA, 64 queries 34 -> 21 us.
int prefill_splits(const nexus_attn_desc* d, long long base)
{
    const long long cus = device_cus();
    if (base >= cus) return 1;
    int kb, ke;
    key_range(d, &kb, &ke);
    const long long tiles = (ke - kb + 63) / 64;
    long long s = cus / base;                                  // about one workgroup per CU
    if (nxa::decode_wg_per_cu(d->head_dim) == 2 && tiles * base >= 12LL * 2 * cus)
        s = 2 * cus / base;                                    // two, while splits keep >= 12 tiles
    if (s > tiles / 4) s = tiles / 4;
    if (s > 64) s = 64;
    return s < 1 ? 1 : (int)s;
}

// Prefill grid of the pipelined kernel (every supported head dim, softcap and sliding window
// included): 128-row blocks (KS = 1), or 64-row blocks with the key range split over two waves
// of the workgroup (KS = 2) when 128-row blocks give at most one workgroup per CU (one wave per
// SIMD), or fewer than two per CU for a chunk longer than the cache before it, where causal
// blocks range up to about twice the mean length and smaller blocks balance better (measured on
// MI355X with the CU pairing of pair_rotate, 40 q heads: 1024 queries cold 29.7 -> 25.4 us,
// 36q/4kv 27.6 -> 21.4 us; from a cache as long as the chunk on, 128-row blocks are faster: 40
// q heads, 1024 after 1024 51.1 vs 53.3 us, 48 q heads 52.3 vs 56.4, head dim 64 31.0 vs 36.6;
// 1024 after 2048/3072/4096/7168 without the pairing 76/100/124/195 vs 80/107/136/223 us).
// Head dims 192 and 256 have the 128-row form only: the two-key-group form does not fit one wave
// per SIMD's registers.  Either grid splits the key range over workgroups by the rule above.
// Packed rows: a chunk of at most 512 queries with several q heads per kv head can have its
// blocks over the (query, head-in-group) pairs of each kv head instead of one padded block per q
// head, so the group's heads share every K/V tile (read once per block, not once per q head) and
// only the last block of a kv head is partly filled.  It pays behind long caches, where the
// unpacked grid's G-fold K/V reads dominate: taken behind >= 8k keys at head dims >= 128 (>= 16k
// at 64) when it has fewer blocks than the unpacked grid and its grid keeps at least 3/4 of the
// workgroups of the unpacked one or of the CUs.  Measured on MI355X: 40q/8kv hd 128, 32/48/96
// queries over 32k keys 90/92/160 -> 63/76/128 us, 24 over 9k 25.7 -> 18.1 us; 64q/8kv, 20
// queries over 12k 39.3 -> 23.5 us, 40 over 32k (240 packed workgroups against 256) 129 -> 93
// us; 24q/4kv hd 192, 48 queries over 12k 42.7 -> 34.7 us; 129-512 queries, 16q/2kv hd 256, 160
// over 32k 157 -> 114 us, 64q/8kv, 160 over 16k 130 -> 102 us, 40q/8kv, 200 over 32k 178 -> 153
// us (packing was first limited to 128 queries); as many blocks either way (40q/8kv, 64
// queries) or head dim 64 behind 9k keys: 1-7% slower packed; behind 4-6k keys within +-10%
// either way; 16q/2kv hd 256, 32 queries over 8k packed into 64 workgroups instead of 256: 14%
// slower.
struct PrefillPlan {
    int ks;
    int splits;
    bool pack;
};

// Blocks of `rows` rows of a prefill grid (per q head, or per kv head when packed).
long long query_blocks(const nexus_attn_desc* d, long long rows, bool pack)
{
    const long long units = pack ? d->n_kv_heads : d->n_q_heads;
    const long long n = pack ? (long long)d->n_query * (d->n_q_heads / d->n_kv_heads) : d->n_query;
    return units * ((n + rows - 1) / rows);
}

PrefillPlan prefill_plan_for(const nexus_attn_desc* d, bool pack)
{
    PrefillPlan p{1, 1, pack};
    const long long b1 = query_blocks(d, nxa::prefill_wide_rows(1), pack), cus = device_cus();
    const bool ks2 = b1 <= cus || (b1 < 2 * cus && d->q_base_pos < d->n_query);
    p.ks = ks2 && d->head_dim <= 128 ? 2 : 1;
    const long long b = query_blocks(d, nxa::prefill_wide_rows(p.ks), pack);
    p.splits = prefill_splits(d, b);
    // Behind a cache of >= 8k keys at least as long as the chunk, 128-row blocks (K/V tiles shared
    // by four row waves) in key splits beat 64-row ones when they pad no more rows, their split
    // grid is as large and each split keeps >= 16 key tiles (40q/8kv hd 128: 512 queries over 16k
    // 215 -> 180 us, 200-384 queries over 16-32k 7% faster; with more padding, 160 queries, or a
    // smaller grid, 512 queries over 8k with 64 q heads, 10-12% slower).
    if (p.ks == 2 && d->q_base_pos >= d->n_query && d->q_base_pos >= 8192 && b == 2 * b1) {
        const int s1 = prefill_splits(d, b1);
        int kb, ke;
        key_range(d, &kb, &ke);
        if ((long long)s1 * b1 >= (long long)p.splits * b && 16LL * 64 * s1 <= ke - kb) {
            p.ks = 1;
            p.splits = s1;
        }
    }
    return p;
}

long long prefill_plan_wgs(const nexus_attn_desc* d, const PrefillPlan& p)
{
    return query_blocks(d, nxa::prefill_wide_rows(p.ks), p.pack) * p.splits;
}

PrefillPlan prefill_plan(const nexus_attn_desc* d)
{
    const PrefillPlan plain = prefill_plan_for(d, false);
    if (d->n_query > 512 || d->n_q_heads == d->n_kv_heads || d->n_ctx < (d->head_dim >= 128 ? 8192 : 16384))
        return plain;
    const PrefillPlan packed = prefill_plan_for(d, true);
    // packing must save K/V reads (fewer blocks) and keep the grid at 3/4 of the plain one or of the CUs
    if (query_blocks(d, nxa::prefill_wide_rows(packed.ks), true) >= query_blocks(d, nxa::prefill_wide_rows(plain.ks), false))
        return plain;
    return 4 * prefill_plan_wgs(d, packed) >= 3 * std::min<long long>(prefill_plan_wgs(d, plain), device_cus()) ? packed : plain;
}

// Chunks short enough for the split-KV decode kernel.  It streams a kv head's K/V once per group
// of 32 (query, head-in-group) rows (R groups), where the unpacked prefill kernel reads it once
// per q head (G times) into 128-query blocks such a chunk barely fills, and the packed one once
// per 64 or 128 rows.  Measured on MI355X (8-64 queries): the decode kernel wins for one group at
// any length, and against the unpacked prefill kernel while 2R <= G behind 8k-16k keys (16q/2kv
// hd 256, 16 queries over 8k: 22.8 vs 27.7 us; 64q/8kv hd 128, 8 queries over 12k: 20.9 vs 37.2)
// or R < G behind >= 16k (16q/2kv hd 256, 12-16 queries over 17k: 24-28 vs 44-46 us).  Packed rows
// beat it wherever they fill the grid (R = 2: 40q/8kv hd 128, 12 queries over 17k/32k 27/44 ->
// 23/37 us, 32q/8kv hd 64, 16 over 32k 31 -> 21 us, 40q/8kv, 8 over 64k 77 -> 59 us; R >= 3:
// 64q/8kv, 12/16 queries over 12k 28/31 -> 20/21 us, 24 over 17k/32k 52/94 -> 34/64 us; 16q/2kv hd
// 256, 24 queries 39/63 -> 33/40 us; 24q/4kv hd 192, 16/24 over 32k 51/80 -> 35/48 us), so the
// decode kernel keeps the chunks that do not pack.  Otherwise the prefill kernel's lower fixed
// costs win (40q/8kv hd 128, 12 queries over 4k: 14.6 vs 16.2 us).
bool small_query_path(const nexus_attn_desc* d)
{
    const long long per = (long long)nxa::kDecodeRowTile * nxa::kDecodeMaxRowTiles;
    const long long groups = (decode_rows(d) + per - 1) / per;
    const long long g = d->n_q_heads / d->n_kv_heads;
    if (groups <= 1) return true;
    const bool fewer = d->n_ctx >= 16384 ? groups < g : (d->n_ctx >= 8192 && 2 * groups <= g);
    return fewer && !prefill_plan(d).pack;
}

int launch_combine_for(const nexus_attn_desc* d, float* ws, void* out, const float* gate, int n_splits,
                       hipStream_t stream)
{
    nxa::CombineArgs c{};
    c.part = ws;
    c.out = out;
    c.gate = gate;
    c.gate_stride = d->head_dim;
    c.n_rows = d->n_query * d->n_q_heads;
    c.n_splits = n_splits;
    const hipError_t e = nxa::launch_combine(c, d->head_dim, d->o_dtype == NEXUS_DT_F32, stream);
    if (e != hipSuccess) return capi_fail(NEXUS_E_LAUNCH, "combine launch: %s", hipGetErrorString(e));
    return NEXUS_OK;
}

int run_decode(const nexus_attn_desc* d, const void* q, const uint16_t* k, const uint16_t* v, void* out,
               const float* gate, float* ws, int n_splits, hipStream_t stream)
{
    int kb, ke;
    key_range(d, &kb, &ke);
    const long long kv_len = ke - kb;
    long long chunk = (kv_len + n_splits - 1) / n_splits;
    chunk = (chunk + nxa::kDecodeKeys - 1) / nxa::kDecodeKeys * nxa::kDecodeKeys;
    if (chunk < nxa::kDecodeKeys) chunk = nxa::kDecodeKeys;

    nxa::DecodeArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.gate = gate;
    a.gate_stride = d->head_dim;
    a.part = ws;
    a.kv_stride = d->kv_row_stride;
    a.n_q_heads = d->n_q_heads;
    a.n_kv_heads = d->n_kv_heads;
    a.group = d->n_q_heads / d->n_kv_heads;
    a.n_query = d->n_query;
    a.q_base = d->q_base_pos;
    a.n_ctx = d->n_ctx;
    a.sliding_window = d->sliding_window;
    a.scale = eff_scale(d);
    a.scale_log2 = a.scale * 1.4426950408889634f;
    a.softcap = d->softcap;
    a.n_splits = n_splits;
    a.chunk = (int)chunk;
    a.k_begin = kb;
    a.k_end = ke;
    a.n_rows = (int)decode_rows(d);
    a.row_tiles = decode_row_tiles(d);
    hipError_t e = nxa::launch_decode(a, d->head_dim, d->q_dtype == NEXUS_DT_F32, d->o_dtype == NEXUS_DT_F32,
                                      is_ext(d), decode_rowgroups(d), stream);
    if (e != hipSuccess) return capi_fail(NEXUS_E_LAUNCH, "decode launch: %s", hipGetErrorString(e));
    if (n_splits > 1) {
        const int rc = launch_combine_for(d, ws, out, gate, n_splits, stream);
        if (rc != NEXUS_OK) return rc;
    }
    return ok();
}

}  // namespace

int nxa::decode_into(const nexus_attn_desc* desc, const void* q, const uint16_t* k, const uint16_t* v,
                     const float* gate, void* out, float* ws, size_t ws_cap, int n_splits, hipStream_t stream)
{
    const int rc = check_desc(desc);
    if (rc != NEXUS_OK) return rc;
    if (!q || !k || !v || !out) return capi_fail(NEXUS_E_INVALID, "null q/k/v/out pointer");
    if (gate && ((uintptr_t)gate & 15u)) return capi_fail(NEXUS_E_INVALID, "gate is not 16-byte aligned");
    if (n_splits > kMaxSplits) return capi_fail(NEXUS_E_UNSUPPORTED, "n_splits=%d > %d", n_splits, kMaxSplits);
    if (n_splits <= 0) {
        n_splits = default_decode_splits(desc);
        const size_t per_split = decode_ws_bytes(desc, 1);
        if (n_splits > 1 && decode_ws_bytes(desc, n_splits) > ws_cap)
            n_splits = per_split > 0 ? (int)std::max<size_t>(1, ws_cap / per_split) : 1;
    }
    // one split writes `out` directly and touches no partials
    if (n_splits > 1 && (!ws || decode_ws_bytes(desc, n_splits) > ws_cap))
        return capi_fail(NEXUS_E_WORKSPACE, "n_splits=%d needs %zu bytes of partials, the workspace holds %zu",
                         n_splits, decode_ws_bytes(desc, n_splits), ws_cap);
    return run_decode(desc, q, k, v, out, gate, ws, n_splits, stream);
}

extern "C" {

size_t nexus_hip_attn_decode_ws_bytes(const nexus_attn_desc* desc, int n_splits)
{
    if (check_desc(desc) != NEXUS_OK) return 0;
    if (n_splits <= 0) n_splits = default_decode_splits(desc);
    if (n_splits > kMaxSplits) return 0;
    return decode_ws_bytes(desc, n_splits);
}

int nexus_hip_attn_decode_default_splits(const nexus_attn_desc* desc)
{
    if (check_desc(desc) != NEXUS_OK) return 0;
    return default_decode_splits(desc);
}

int nexus_hip_attn_decode_gated(const nexus_attn_desc* desc, const void* q, const uint16_t* k,
                                const uint16_t* v, const float* gate, void* out, float* partial_ws,
                                int n_splits, nexus_stream_t stream)
{
    const int rc = check_desc(desc);
    if (rc != NEXUS_OK) return rc;
    if (!partial_ws) return capi_fail(NEXUS_E_WORKSPACE, "partial_ws is NULL");
    // the caller sized partial_ws for this split count (nexus_hip_attn_decode_ws_bytes)
    const int s = n_splits <= 0 ? default_decode_splits(desc) : n_splits;
    return nxa::decode_into(desc, q, k, v, gate, out, partial_ws, s <= kMaxSplits ? decode_ws_bytes(desc, s) : 0,
                            s, (hipStream_t)stream);
}

int nexus_hip_attn_decode(const nexus_attn_desc* desc, const void* q, const uint16_t* k,
                          const uint16_t* v, void* out, float* partial_ws, int n_splits,
                          nexus_stream_t stream)
{
    return nexus_hip_attn_decode_gated(desc, q, k, v, nullptr, out, partial_ws, n_splits, stream);
}

static_assert(NEXUS_PREP_Q_NORM_ADD_ONE == nxa::kPrepQZeroCentred && NEXUS_PREP_K_NORM_ADD_ONE == nxa::kPrepKZeroCentred &&
                  NEXUS_PREP_NO_GATE == nxa::kPrepNoGate && NEXUS_PREP_NO_Q_NORM == nxa::kPrepNoQNorm &&
                  NEXUS_PREP_NO_K_NORM == nxa::kPrepNoKNorm && NEXUS_PREP_ROPE_INTERLEAVED == nxa::kPrepInterleaved &&
                  NEXUS_PREP_TRUNC_STORE == nxa::kPrepTruncStore,
              "prep flag bits of the C ABI and the kernel differ");

}  // extern "C"

namespace {

// Descriptor and input checks shared by the prep and the fused decode layer.
int check_prep(const nexus_attn_prep_desc* d, const float* qg, const float* k_raw, const float* v_raw,
               const float* q_norm_w, const float* k_norm_w, const float* rope_tab, const uint16_t* k_cache,
               const uint16_t* v_cache, const float* kv_out)
{
    if (!d) return capi_fail(NEXUS_E_INVALID, "desc is NULL");
    if (d->n_heads <= 0 || d->n_kv_heads <= 0 || d->n_heads > 65536 || d->n_kv_heads > 65536)
        return capi_fail(NEXUS_E_INVALID, "n_heads=%d n_kv_heads=%d", d->n_heads, d->n_kv_heads);
    if (d->head_dim <= 0 || d->head_dim > nxa::kPrepMaxHeadDim)
        return capi_fail(NEXUS_E_UNSUPPORTED, "head_dim=%d not in [1, %d]", d->head_dim, nxa::kPrepMaxHeadDim);
    if (d->rot_dims < 0 || d->rot_dims > d->head_dim || (d->rot_dims & 1))
        return capi_fail(NEXUS_E_INVALID, "rot_dims=%d must be even and in [0, head_dim=%d]", d->rot_dims, d->head_dim);
    if (d->cap <= 0 || d->pos < 0 || d->pos >= d->cap)
        return capi_fail(NEXUS_E_INVALID, "pos=%d outside the cache rows [0, cap=%lld)", d->pos, (long long)d->cap);
    if (d->flags & ~127) return capi_fail(NEXUS_E_INVALID, "unknown flag bits 0x%x", d->flags & ~127);
    if (!(d->eps >= 0.f) || !std::isfinite(d->eps)) return capi_fail(NEXUS_E_INVALID, "eps=%g", (double)d->eps);
    if (d->reserved != 0) return capi_fail(NEXUS_E_INVALID, "reserved=%d must be 0", d->reserved);
    if (!qg || !k_raw || !v_raw || !k_cache || !v_cache || !kv_out)
        return capi_fail(NEXUS_E_INVALID, "null qg/k_raw/v_raw/k_cache/v_cache/kv_out pointer");
    if (!(d->flags & NEXUS_PREP_NO_Q_NORM) && !q_norm_w) return capi_fail(NEXUS_E_INVALID, "q_norm_w is NULL");
    if (!(d->flags & NEXUS_PREP_NO_K_NORM) && !k_norm_w) return capi_fail(NEXUS_E_INVALID, "k_norm_w is NULL");
    if (d->rot_dims > 0 && !rope_tab) return capi_fail(NEXUS_E_INVALID, "rope_tab is NULL");
    return NEXUS_OK;
}

// The attention descriptor of the fused decode layer: one token at pos over rows [0, pos]
// of [n_kv][cap][hd] caches, f32 q and out.
nexus_attn_desc layer_attn_desc(const nexus_attn_prep_desc* d, float scale)
{
    nexus_attn_desc a{};
    a.n_q_heads = d->n_heads;
    a.n_kv_heads = d->n_kv_heads;
    a.head_dim = d->head_dim;
    a.n_query = 1;
    a.q_base_pos = d->pos;
    a.n_ctx = d->pos + 1;
    a.kv_row_stride = d->cap;
    a.scale = scale;
    a.q_dtype = NEXUS_DT_F32;
    a.o_dtype = NEXUS_DT_F32;
    return a;
}

// Shape checks of the fused layer beyond check_prep (decode head dims, a GQA group).
int check_layer_shape(const nexus_attn_prep_desc* d, float scale)
{
    if (d->n_heads % d->n_kv_heads != 0)
        return capi_fail(NEXUS_E_UNSUPPORTED, "n_heads=%d must be a multiple of n_kv_heads=%d", d->n_heads,
                         d->n_kv_heads);
    if (!supported_head_dim(d->head_dim))
        return capi_fail(NEXUS_E_UNSUPPORTED, "head_dim=%d not in {64,128,192,256}", d->head_dim);
    const nexus_attn_desc a = layer_attn_desc(d, scale);
    return check_desc(&a);
}

}  // namespace

extern "C" {

int nexus_hip_attn_decode_prep(const nexus_attn_prep_desc* d, const float* qg, const float* k_raw,
                               const float* v_raw, const float* q_norm_w, const float* k_norm_w,
                               const float* rope_tab, float* q_out, float* gate_out, uint16_t* k_cache,
                               uint16_t* v_cache, float* kv_out, nexus_stream_t stream)
{
    const int rc = check_prep(d, qg, k_raw, v_raw, q_norm_w, k_norm_w, rope_tab, k_cache, v_cache, kv_out);
    if (rc != NEXUS_OK) return rc;
    if (!q_out) return capi_fail(NEXUS_E_INVALID, "q_out is NULL");
    const bool gated = (d->flags & NEXUS_PREP_NO_GATE) == 0;
    if (gated && !gate_out) return capi_fail(NEXUS_E_INVALID, "gate_out is NULL for a gated layer");

    nxa::PrepArgs a{};
    a.qg = qg;
    a.kraw = k_raw;
    a.vraw = v_raw;
    a.qnw = q_norm_w;
    a.knw = k_norm_w;
    a.tab = rope_tab;
    a.q_out = q_out;
    a.gate_out = gate_out;
    a.kc = k_cache;
    a.vc = v_cache;
    a.kv_out = kv_out;
    a.cap = d->cap;
    a.n_heads = d->n_heads;
    a.n_kv = d->n_kv_heads;
    a.hd = d->head_dim;
    a.rot = d->rot_dims;
    a.pos = d->pos;
    a.flags = d->flags;
    a.eps = d->eps;
    const hipError_t e = nxa::launch_decode_prep(a, (hipStream_t)stream);
    if (e != hipSuccess) return capi_fail(NEXUS_E_LAUNCH, "decode prep launch: %s", hipGetErrorString(e));
    return ok();
}

size_t nexus_hip_attn_decode_layer_ws_bytes(const nexus_attn_prep_desc* desc, int n_splits)
{
    if (!desc || check_layer_shape(desc, 0.f) != NEXUS_OK) return 0;
    const nexus_attn_desc a = layer_attn_desc(desc, 0.f);
    if (n_splits <= 0) n_splits = default_decode_splits(&a);
    if (n_splits > kMaxSplits) return 0;
    return decode_ws_bytes(&a, n_splits);
}

int nexus_hip_attn_decode_layer_default_splits(const nexus_attn_prep_desc* desc)
{
    if (!desc || check_layer_shape(desc, 0.f) != NEXUS_OK) return 0;
    const nexus_attn_desc a = layer_attn_desc(desc, 0.f);
    return default_decode_splits(&a);
}

int nexus_hip_attn_decode_layer(const nexus_attn_prep_desc* d, float scale, const float* qg, const float* k_raw,
                                const float* v_raw, const float* q_norm_w, const float* k_norm_w,
                                const float* rope_tab, uint16_t* k_cache, uint16_t* v_cache, float* kv_out,
                                float* out, float* partial_ws, int n_splits, nexus_stream_t stream)
{
    int rc = check_prep(d, qg, k_raw, v_raw, q_norm_w, k_norm_w, rope_tab, k_cache, v_cache, kv_out);
    if (rc != NEXUS_OK) return rc;
    rc = check_layer_shape(d, scale);
    if (rc != NEXUS_OK) return rc;
    if (!out) return capi_fail(NEXUS_E_INVALID, "out is NULL");
    const nexus_attn_desc ad = layer_attn_desc(d, scale);
    if (n_splits > kMaxSplits) return capi_fail(NEXUS_E_UNSUPPORTED, "n_splits=%d > %d", n_splits, kMaxSplits);
    if (n_splits <= 0) n_splits = default_decode_splits(&ad);
    if (n_splits > 1 && !partial_ws) return capi_fail(NEXUS_E_WORKSPACE, "partial_ws is NULL");

    int kb, ke;
    key_range(&ad, &kb, &ke);
    long long chunk = (ke - kb + n_splits - 1) / n_splits;
    chunk = (chunk + nxa::kDecodeKeys - 1) / nxa::kDecodeKeys * nxa::kDecodeKeys;
    if (chunk < nxa::kDecodeKeys) chunk = nxa::kDecodeKeys;
    const bool gated = (d->flags & NEXUS_PREP_NO_GATE) == 0;
    const int hd = d->head_dim;

    nxa::DecodeArgs a{};
    a.k = k_cache;
    a.v = v_cache;
    a.out = out;
    a.gate = gated ? qg + hd : nullptr;
    a.gate_stride = 2 * (long long)hd;
    a.part = partial_ws;
    a.kv_stride = d->cap;
    a.n_q_heads = d->n_heads;
    a.n_kv_heads = d->n_kv_heads;
    a.group = d->n_heads / d->n_kv_heads;
    a.n_query = 1;
    a.q_base = d->pos;
    a.n_ctx = d->pos + 1;
    a.scale = eff_scale(&ad);
    a.scale_log2 = a.scale * 1.4426950408889634f;
    a.n_splits = n_splits;
    a.chunk = (int)chunk;
    a.k_begin = kb;
    a.k_end = ke;
    a.n_rows = (int)decode_rows(&ad);
    a.row_tiles = decode_row_tiles(&ad);
    a.qg = qg;
    a.kraw = k_raw;
    a.vraw = v_raw;
    a.qnw = q_norm_w;
    a.knw = k_norm_w;
    a.tab = rope_tab;
    a.kc = k_cache;
    a.vc = v_cache;
    a.kv_out = kv_out;
    a.rot = d->rot_dims;
    a.prep_flags = d->flags;
    a.pos_split = (int)((d->pos - kb) / chunk);
    a.eps = d->eps;
    const hipError_t e = nxa::launch_decode_layer(a, hd, decode_rowgroups(&ad), (hipStream_t)stream);
    if (e != hipSuccess) return capi_fail(NEXUS_E_LAUNCH, "decode layer launch: %s", hipGetErrorString(e));
    if (n_splits > 1) {
        nxa::CombineArgs c{};
        c.part = partial_ws;
        c.out = out;
        c.gate = gated ? qg + hd : nullptr;
        c.gate_stride = 2 * (long long)hd;
        c.n_rows = d->n_heads;
        c.n_splits = n_splits;
        const hipError_t e2 = nxa::launch_combine(c, hd, true, (hipStream_t)stream);
        if (e2 != hipSuccess) return capi_fail(NEXUS_E_LAUNCH, "combine launch: %s", hipGetErrorString(e2));
    }
    return ok();
}

size_t nexus_hip_attn_prefill_ws_bytes(const nexus_attn_desc* desc)
{
    if (check_desc(desc) != NEXUS_OK) return 0;
    if (small_query_path(desc)) return decode_ws_bytes(desc, default_decode_splits(desc));
    const int s = prefill_plan(desc).splits;
    if (s <= 1) return 0;
    return prefill_split_ws_bytes(desc, s);
}

int nexus_hip_attn_prefill_plan(const nexus_attn_desc* desc, nexus_attn_prefill_plan* plan)
{
    const int rc = check_desc(desc);
    if (rc != NEXUS_OK) return rc;
    if (!plan) return capi_fail(NEXUS_E_INVALID, "null plan pointer");
    if (small_query_path(desc)) {
        const int splits = default_decode_splits(desc);
        plan->kernel = NEXUS_PLAN_DECODE;
        plan->block_rows = nxa::kDecodeRowTile * decode_row_tiles(desc);
        plan->splits = splits;
        plan->packed = 0;
        plan->workgroups = splits * desc->n_kv_heads * decode_rowgroups(desc);
        return ok();
    }
    const PrefillPlan p = prefill_plan(desc);
    plan->kernel = NEXUS_PLAN_PREFILL;
    plan->block_rows = nxa::prefill_wide_rows(p.ks);
    plan->splits = p.splits;
    plan->packed = p.pack ? 1 : 0;
    const long long wgs = prefill_plan_wgs(desc, p);
    plan->workgroups = wgs > INT_MAX ? INT_MAX : (int)wgs;
    return ok();
}

int nexus_hip_attn_prefill_gated(const nexus_attn_desc* desc, const void* q, const uint16_t* k,
                                 const uint16_t* v, const float* gate, void* out, void* workspace,
                                 size_t workspace_bytes, nexus_stream_t stream)
{
    const int rc = check_desc(desc);
    if (rc != NEXUS_OK) return rc;
    if (!q || !k || !v || !out) return capi_fail(NEXUS_E_INVALID, "null q/k/v/out pointer");
    if (gate && ((uintptr_t)gate & 15u)) return capi_fail(NEXUS_E_INVALID, "gate is not 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;

    // A handful of queries (speculative verify, tiny prompts): the split-KV kernel fills
    // the GPU where 128-query blocks could not.
    if (small_query_path(desc) && workspace) {
        const int splits = default_decode_splits(desc);
        if (workspace_bytes >= decode_ws_bytes(desc, splits))
            return run_decode(desc, q, k, v, out, gate, (float*)workspace, splits, s);
    }

    const PrefillPlan plan = prefill_plan(desc);
    int splits = plan.splits;
    if (splits > 1 && (!workspace || workspace_bytes < prefill_split_ws_bytes(desc, splits))) splits = 1;

    nxa::PrefillArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.gate = gate;
    a.part = (float*)workspace;
    a.kv_stride = desc->kv_row_stride;
    a.n_q_heads = desc->n_q_heads;
    a.n_kv_heads = desc->n_kv_heads;
    a.group = desc->n_q_heads / desc->n_kv_heads;
    a.n_query = desc->n_query;
    a.q_base = desc->q_base_pos;
    a.n_ctx = desc->n_ctx;
    a.sliding_window = desc->sliding_window;
    a.scale = eff_scale(desc);
    a.scale_log2 = a.scale * 1.4426950408889634f;
    a.softcap = desc->softcap;
    const long long rows = nxa::prefill_wide_rows(plan.ks);
    const long long row_space = plan.pack ? (long long)desc->n_query * a.group : desc->n_query;
    a.pack = plan.pack ? 1 : 0;
    a.n_qblocks = (int)((row_space + rows - 1) / rows);
    a.n_splits = splits;
    const long long items = (long long)(plan.pack ? desc->n_kv_heads : desc->n_q_heads) * a.n_qblocks * splits;
    if (items > INT_MAX) return capi_fail(NEXUS_E_UNSUPPORTED, "grid too large");
    a.n_items = (int)items;
    // a grid between one and two workgroups per CU at two per CU: the CUs that hold two run the
    // lightest blocks (pair_rotate)
    const long long cus = device_cus();
    if (nxa::decode_wg_per_cu(desc->head_dim) == 2 && cus % 8 == 0 && items > cus && items < 2 * cus &&
        (items - cus) % 8 == 0) {
        a.pair_rot = (int)((items - cus) / 8);
        a.pair_span = (int)(cus / 8);
    }
    const bool q32 = desc->q_dtype == NEXUS_DT_F32, o32 = desc->o_dtype == NEXUS_DT_F32;
    // the softcap form (EXT) only when there is a softcap: a sliding window is masking, which the
    // plain form does too
    const hipError_t e = nxa::launch_prefill_wide(a, desc->head_dim, plan.ks, q32, o32, desc->softcap > 0.f, s);
    if (e != hipSuccess) return capi_fail(NEXUS_E_LAUNCH, "prefill launch: %s", hipGetErrorString(e));
    if (splits > 1) {
        const int rc2 = launch_combine_for(desc, (float*)workspace, out, gate, splits, s);
        if (rc2 != NEXUS_OK) return rc2;
    }
    return ok();
}

int nexus_hip_attn_prefill(const nexus_attn_desc* desc, const void* q, const uint16_t* k,
                           const uint16_t* v, void* out, void* workspace, size_t workspace_bytes,
                           nexus_stream_t stream)
{
    return nexus_hip_attn_prefill_gated(desc, q, k, v, nullptr, out, workspace, workspace_bytes, stream);
}

const char* nexus_hip_attn_last_error(void) { return g_last_error; }

const char* nexus_hip_attn_version(void) { return "nexus_hip_attn 0.1.0 gfx950"; }

}  // extern "C"

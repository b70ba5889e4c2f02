// nexus_amd/csrc/attn_kernels.h -- kernel argument blocks, workspace layout and launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nxa {

// Prefill workgroup size (attn_prefill_wide.hip): 4 waves.
constexpr int kPrefillThreads = 256;
// Pipelined prefill (attn_prefill_wide.hip): 32 query rows per wave, 4 waves per workgroup
// as 4 row waves (KS = 1, 128 rows) or 2 row waves x 2 key groups (KS = 2, 64 rows).
constexpr int kWideRowsPerWave = 32;
// Split-KV decode (attn_decode.hip): 4 waves per (split, kv head, row group) sharing an LDS
// ring of 32-key stages, 16 query rows (n_query * G) per row tile and one or two row tiles
// per row group.
constexpr int kDecodeThreads = 256;
// Decode workgroups resident per CU: two with a 64 KB ring up to head dim 128, one with a
// 120-128 KB ring above.
constexpr int decode_wg_per_cu(int head_dim) { return head_dim <= 128 ? 2 : 1; }
constexpr int kDecodeKeys = 32;
constexpr int kDecodeRowTile = 16;
constexpr int kDecodeMaxRowTiles = 2;
constexpr int kMaxSplits = 1024;

struct PrefillArgs {
    const void* q;
    const uint16_t* k;
    const uint16_t* v;
    void* out;
    const float* gate;              // [n_query][Hq][hd] f32 or null: out *= sigmoid(gate)
    float* part;                    // split partials of n_query*Hq rows (n_splits > 1), part_acc / part_ml
    long long kv_stride;            // tokens between kv heads
    int n_q_heads, n_kv_heads, group;
    int n_query, q_base, n_ctx;
    int sliding_window;
    float scale;                    // natural-log scale applied to q.k
    float scale_log2;               // scale * log2(e)
    float softcap;
    int n_qblocks, n_splits, n_items;
    int pack;                       // non-zero: a block's rows are (query, head-in-group) pairs of
                                    // its kv head (row p: query p / group, head kv * group + p % group)
    int pair_rot, pair_span;        // pair_rotate() of the dispatch position (0, 0: none)
};

struct DecodeArgs {
    const void* q;
    const uint16_t* k;
    const uint16_t* v;
    void* out;                      // [n_query][Hq][hd]
    const float* gate;              // f32 gate of row qi*Hq + h at gate + row * gate_stride, or null
                                    // (applied here with one split, by the combine otherwise)
    long long gate_stride;          // floats between rows of the gate (hd, or 2 hd inside [q | gate])
    float* part;                    // split partials of n_query*Hq rows (n_splits > 1), part_acc / part_ml
    long long kv_stride;
    int n_q_heads, n_kv_heads, group;
    int n_query, q_base, n_ctx;
    int sliding_window;
    float scale, scale_log2, softcap;
    int n_splits;
    int chunk;                      // keys per split, a positive multiple of kDecodeKeys
    int k_begin;                    // first key any row can see
    int k_end;                      // one past the last key any row can see
    int n_rows;                     // n_query * group
    int row_tiles;                  // 16-row tiles per row group (1 or 2)
    // Fused decode prep (the decode-layer kernel only; n_query = 1, f32 q and out): q is
    // normalised and rotated from qg in the prologue, and the workgroups of the split holding
    // key `pos` compute the new K/V row from kraw/vraw, attend it, and (row group 0) store it
    // into kc/vc row `pos` and kv_out, as decode_prep_kernel does.
    const float* qg;                // [Hq][2 hd] (q | gate) or [Hq][hd] with kPrepNoGate
    const float* kraw;              // [Hkv][hd]
    const float* vraw;
    const float* qnw;               // [hd] or null (no q norm)
    const float* knw;
    const float* tab;               // [rot]: cos then sin
    uint16_t* kc;                   // the cache a.k / a.v point into, written at row pos
    uint16_t* vc;
    float* kv_out;                  // [2][Hkv][hd]
    int rot, prep_flags, pos_split;
    float eps;
};

struct CombineArgs {
    const float* part;              // split partials of n_rows rows, part_acc / part_ml
    void* out;                      // [n_rows][hd], row = qi*Hq + h
    const float* gate;              // f32 gate of row r at gate + r * gate_stride, or null:
                                    // out *= sigmoid(gate)
    long long gate_stride;
    int n_rows, n_splits;
};

// Decode prep (attn_prep.hip): flag bits of qwen35_attn_prep.comp:7-8, plus a truncating
// store that matches the host cache's own conversion (KVCache::store, kvcache.h:903-911).
constexpr int kPrepMaxHeadDim = 512;
constexpr int kPrepQZeroCentred = 1;
constexpr int kPrepKZeroCentred = 2;
constexpr int kPrepNoGate = 4;
constexpr int kPrepNoQNorm = 8;
constexpr int kPrepNoKNorm = 16;
constexpr int kPrepInterleaved = 32;
constexpr int kPrepTruncStore = 64;

struct PrepArgs {
    const float* qg;                // [n_heads][2*hd] (q | gate) or [n_heads][hd] without gate
    const float* kraw;              // [n_kv][hd]
    const float* vraw;              // [n_kv][hd]
    const float* qnw;               // [hd] q norm weight (read only when the q norm is on)
    const float* knw;               // [hd]
    const float* tab;               // [rot]: cos[rot/2] then sin[rot/2]
    float* q_out;                   // [n_heads][hd]
    float* gate_out;                // [n_heads][hd] (gated layers)
    uint16_t* kc;                   // [n_kv][cap][hd] f16
    uint16_t* vc;
    float* kv_out;                  // [2][n_kv][hd]: K then V as stored
    long long cap;
    int n_heads, n_kv, hd, rot, pos, flags;
    float eps;
};

// Workspace = f32 split partials with the meaning of the reference's split-K partials
// (qwen35_attn_part.comp:3: per row and split, acc[hd] = sum_k e^{s_k - m} v_k, m, l), laid
// out for 16-byte stores: acc as [split][row][hd], then (m, l) pairs as [split][row][2].  A
// workgroup's rows of one split are contiguous, so its stores fill whole cache lines.  It
// carries no state between calls.
inline size_t ws_partial_bytes(long long rows, int splits, int head_dim)
{
    return (size_t)rows * (size_t)splits * (size_t)(head_dim + 2) * sizeof(float);
}
// Offsets (in floats) of a partial's acc vector and of its (m, l) pair.
__host__ __device__ inline size_t part_acc(int split, long long row, long long n_rows, int head_dim)
{
    return ((size_t)split * (size_t)n_rows + (size_t)row) * (size_t)head_dim;
}
__host__ __device__ inline size_t part_ml(int split, long long row, long long n_rows, int n_splits, int head_dim)
{
    return (size_t)n_splits * (size_t)n_rows * (size_t)head_dim + ((size_t)split * (size_t)n_rows + (size_t)row) * 2;
}

// Each launcher returns hipSuccess or the launch error; shapes are validated by the caller.
// Pipelined prefill: causal shapes at head dims 64, 128, 192, 256 (KS = 2 at 64 and 128 only),
// sliding window in either form, softcap when `ext`; n_qblocks counts prefill_wide_rows(ks)-row
// blocks.
int prefill_wide_rows(int ks);
hipError_t launch_prefill_wide(const PrefillArgs& a, int head_dim, int ks, bool q_f32, bool o_f32, bool ext,
                               hipStream_t stream);
hipError_t launch_decode(const DecodeArgs& a, int head_dim, bool q_f32, bool o_f32, bool ext,
                         int n_rowgroups, hipStream_t stream);
// The decode-layer form (prep fused, f32 q and out, n_query = 1): DecodeArgs with the prep
// fields set.
hipError_t launch_decode_layer(const DecodeArgs& a, int head_dim, int n_rowgroups, hipStream_t stream);
hipError_t launch_combine(const CombineArgs& a, int head_dim, bool o_f32, hipStream_t stream);
// Which combine kernel runs: one wave per row for many rows with few splits (split prefill),
// one workgroup per row otherwise (decode: tens of rows, up to 256 splits).
constexpr bool combine_by_rows(int n_rows, int n_splits) { return n_rows >= 256 && n_splits <= 16; }
// One workgroup (one wave) per q, k and v head: n_heads + 2 * n_kv workgroups.
hipError_t launch_decode_prep(const PrepArgs& a, hipStream_t stream);

}  // namespace nxa

// nexus_amd/csrc/attn_kernels.h -- kernel argument blocks, workspace layout and launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nxa {

// Prefill: 128 queries x one q head per workgroup (4 waves x 32 rows), 64-key tiles.
constexpr int kPrefillBM = 128;
constexpr int kPrefillBN = 64;
constexpr int kPrefillThreads = 256;
// Split-KV decode: 4 waves per (split, kv head, row group), 32 keys per wave step,
// up to 32 query rows (n_query * G) per row group.
constexpr int kDecodeThreads = 256;
constexpr int kDecodeKeys = 32;
constexpr int kDecodeRows = 32;
constexpr int kMaxSplits = 1024;

struct PrefillArgs {
    const void* q;
    const uint16_t* k;
    const uint16_t* v;
    void* out;
    float* part;                    // [n_query*Hq][n_splits][hd+2] partials (n_splits > 1)
    unsigned int* counters;         // [n_qblocks * Hq] arrival counters (n_splits > 1)
    long long kv_stride;            // tokens between kv heads
    int n_q_heads, n_kv_heads, group;
    int n_query, q_base, n_ctx;
    int sliding_window;
    float scale;                    // natural-log scale applied to q.k
    float scale_log2;               // scale * log2(e)
    float softcap;
    int n_qblocks, n_splits, n_items;
};

struct DecodeArgs {
    const void* q;
    const uint16_t* k;
    const uint16_t* v;
    void* out;                      // [n_query][Hq][hd]
    float* part;                    // [n_query*Hq][n_splits][hd+2]
    unsigned int* counters;         // [Hkv * n_rowgroups] arrival counters (fused merge)
    long long kv_stride;
    int n_q_heads, n_kv_heads, group;
    int n_query, q_base, n_ctx;
    int sliding_window;
    float scale, scale_log2, softcap;
    int n_splits;
    int chunk;                      // keys per split, multiple of kDecodeKeys
    int k_begin;                    // first key any row can see
    int k_end;                      // one past the last key any row can see
    int n_rows;                     // n_query * group
    int fused_merge;                // 1: last split merges; 0: combine kernel follows
};

struct CombineArgs {
    const float* part;              // [n_rows][n_splits][hd+2]
    void* out;                      // [n_rows][hd], row = qi*Hq + h
    int n_rows, n_splits;
};

// Workspace = f32 partials [rows][splits][hd+2] (the reference's split-K partial format,
// qwen35_attn_part.comp:3) followed, 256-byte aligned, by one 4-byte counter per merge
// group (8 bytes reserved per group).  Counters start at zero and are left at zero.
inline size_t ws_partial_bytes(long long rows, int splits, int head_dim)
{
    return (size_t)rows * (size_t)splits * (size_t)(head_dim + 2) * sizeof(float);
}
inline size_t ws_counter_offset(long long rows, int splits, int head_dim)
{
    return (ws_partial_bytes(rows, splits, head_dim) + 255) & ~(size_t)255;
}
inline size_t ws_total_bytes(long long rows, int splits, int head_dim, long long n_counters)
{
    return ws_counter_offset(rows, splits, head_dim) + (size_t)n_counters * 8;
}

// Each launcher returns hipSuccess or the launch error; shapes are validated by the caller.
hipError_t launch_prefill(const PrefillArgs& a, int head_dim, bool q_f32, bool o_f32, bool ext,
                          hipStream_t stream);
hipError_t launch_decode(const DecodeArgs& a, int head_dim, bool q_f32, bool o_f32, bool ext,
                         int n_rowgroups, hipStream_t stream);
hipError_t launch_combine(const CombineArgs& a, int head_dim, bool o_f32, hipStream_t stream);

// Largest partial volume (bytes) one merging workgroup folds in the fused merge; beyond it
// a separate combine kernel spreads the merge over (row, dim-chunk) workgroups.
constexpr size_t kFusedMergeBytes = 256u << 10;

}  // namespace nxa

// nexus_amd/csrc/attn_kernels.h -- kernel argument blocks and launchers (host side).
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

struct PrefillArgs {
    const void* q;
    const uint16_t* k;
    const uint16_t* v;
    void* out;             // final output (n_splits == 1)
    float* part;           // [n_query*Hq][n_splits][hd+2] partials (n_splits > 1)
    long long kv_stride;   // tokens between kv heads
    int n_q_heads, n_kv_heads, group;
    int n_query, q_base, n_ctx;
    int sliding_window;
    float scale;           // natural-log scale applied to q.k
    float scale_log2;      // scale * log2(e)
    float softcap;
    int n_qblocks, n_splits, n_items;
};

struct DecodeArgs {
    const void* q;
    const uint16_t* k;
    const uint16_t* v;
    float* part;           // [n_query*Hq][n_splits][hd+2]
    long long kv_stride;
    int n_q_heads, n_kv_heads, group;
    int n_query, q_base, n_ctx;
    int sliding_window;
    float scale, scale_log2, softcap;
    int n_splits;
    int chunk;             // keys per split, multiple of kDecodeKeys
    int k_begin;           // first key any row can see
    int k_end;             // one past the last key any row can see
    int n_rows;            // n_query * group
};

struct CombineArgs {
    const float* part;     // [n_rows][n_splits][hd+2]
    void* out;             // [n_rows][hd], row = qi*Hq + h
    int n_rows, n_splits;
};

// Each launcher returns hipSuccess or the launch error; shapes are validated by the caller.
hipError_t launch_prefill(const PrefillArgs& a, int head_dim, bool q_f32, bool o_f32, bool ext,
                          hipStream_t stream);
hipError_t launch_decode(const DecodeArgs& a, int head_dim, bool q_f32, bool ext,
                         int n_rowgroups, hipStream_t stream);
hipError_t launch_combine(const CombineArgs& a, int head_dim, bool o_f32, hipStream_t stream);

// Dynamic LDS bytes each kernel needs (host side, for validation and attributes).
size_t prefill_lds_bytes(int head_dim);
size_t decode_lds_bytes(int head_dim);

}  // namespace nxa

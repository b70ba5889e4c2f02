// nexus_amd/csrc/attn_prefill_wide.hip -- software-pipelined causal GQA flash-attention
// prefill for gfx950.
//
// Semantics are those of Transformer::attn_batch_cpu (src/model/transformer.h:8653-8685) and
// attn_flash.comp (src/gpu/shaders/attn_flash.comp:66-72, 121-159): query i sits at absolute
// position q_base + i and sees keys [start, min(q_base + i, n_ctx - 1)], start = q_base + i +
// 1 - window with a sliding window, scores softcapped when softcap > 0 (the EXT
// instantiation).  Head dims 64, 128, 192 and 256.  A key split across workgroups writes the
// reference's split-K partials for the combine kernel.
//
// Design:
//  * A wave owns 32 query rows; two waves per SIMD (one at head dims 192 and 256, with O and
//    Q^T in AGPRs and the MFMAs as inline asm).  Workgroup = 4 waves.  KS = 1: four row
//    waves (128 query rows) share every K/V tile.  KS = 2: two row waves x two key groups
//    (64 rows); key group g takes the tiles t = g (mod 2) and the groups' (O, m, l) merge
//    through LDS at the end -- for short chunks, where 128-row blocks leave CUs idle.
//  * Software pipeline over key tiles.  While the MFMAs of S(t+1) = K(t+1) Q^T run, the VALU
//    turns S(t) into P(t) (exp2, f16 pack, row sums); while the MFMAs of O^T += V(t)^T P(t)^T
//    run, the VALU takes the row max of S(t+1).  A wave issues in order, so its VALU work
//    only overlaps its own MFMAs when the two alternate in program order: each MFMA slot is
//    written with its share of VALU work and LDS reads and fenced with sched_barrier.  The
//    two S^T tiles swap roles from step to step (loop unrolled by two, no copies).
//  * Every wave of a workgroup runs the same steps: no per-wave branch in the loop body, so
//    O, Q^T and both S^T tiles keep fixed registers (the last step is peeled).
//  * K runs one tile ahead of V in an LDS ring of two tiles per operand: step s reads K(s+1)
//    and V(s) while K(s+2) and V(s+1) load (buffer-load-to-LDS of XOR-swizzled 16-byte chunks,
//    each lane choosing the global chunk for its LDS slot); one barrier per step.  With the loop unrolled by two
//    the slot parity is static, so every LDS address is a per-lane register plus an immediate.
//  * S^T = K Q^T with Q as given -- f16 queries exactly, f32 queries as an f16 high part
//    (registers) plus the f16 residual (LDS, a second MFMA per k-step), so scores carry ~22
//    mantissa bits like the reference's f32 dot products -- and the accumulator seeded with
//    -m (raw units), so a probability is exp2(scale * log2(e) * S): the scale is applied in
//    f32, never folded into an f16 operand.  The running max moves lazily (only past a 2^8
//    margin), the row max is v_max3 + v_permlane32_swap, row sums are fp32 adds of the
//    probabilities.  EXT (softcap): accumulators seeded with 0, and the VALU turns each raw
//    score into softcap * tanh(x scale / softcap) * log2(e) - m before the row max.  A sliding
//    window is masking only, in both forms.
#include "attn_common.h"
#include "attn_kernels.h"

namespace nxa {

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8;

template <int HD, int KS>
struct WideLayout {
    // keys per tile: 32 at head dim 128 keeps two S^T tiles, O and Q^T of a 32-row wave in
    // the 256 registers of two waves per SIMD
    static constexpr int BN = HD >= 128 ? 32 : 64;
    static constexpr int SB = BN / 32;                          // 32-key S^T blocks per tile
    static constexpr int NB = kWideRowsPerWave / 32;            // 32-row blocks per wave
    static constexpr int RWAVES = 4 / KS;                       // row waves per workgroup
    static constexpr int BM = RWAVES * kWideRowsPerWave;        // query rows per workgroup
    static constexpr int ROW = HD * 2;                          // bytes per K/V row
    static constexpr int CPR = HD / 8;                          // 16-byte chunks per row
    static constexpr int TILE = BN * ROW;
    // K and V each hold two tiles per key group: the step being computed and the next one
    // (loading); with the loop unrolled by two, every LDS address is an immediate offset
    static constexpr int DEPTH = 2;
    static constexpr int SLOTS = DEPTH * KS;                    // ring slots per operand
    static constexpr int VBASE = SLOTS * TILE;
    static constexpr int RING_BYTES = 2 * SLOTS * TILE;
    // KS = 2: per row wave, O of both row blocks (16 registers x 64 lanes per 32-dim block)
    // and (m, l) per row block
    static constexpr int MERGE_FLOATS = NB * (HD / 32) * 16 * 64 + NB * 2 * 64;
    static constexpr int MERGE_BYTES = KS > 1 ? RWAVES * MERGE_FLOATS * 4 : 0;
    static constexpr int LDS_BYTES = RING_BYTES > MERGE_BYTES ? RING_BYTES : MERGE_BYTES;
    // f32 queries: the f16 residual of each row wave's Q^T operands, [row wave][row block]
    // [k-step][lane] x 16 bytes, after the ring (the merge reuses the ring once it is done)
    static constexpr int QLO_WAVE = NB * (HD / 16) * 64 * 16;
    static constexpr int QLO_BYTES = RWAVES * QLO_WAVE;
    static constexpr int LDS_BYTES_QF32 = RING_BYTES + QLO_BYTES > MERGE_BYTES ? RING_BYTES + QLO_BYTES : MERGE_BYTES;
    static constexpr int LOADS = TILE / (kPrefillThreads * 16); // 16-byte loads per thread per tile
    static constexpr int SWZ = (CPR % 16 == 0) ? 15 : 7;
    static_assert(LOADS >= 1 && TILE % (kPrefillThreads * 16) == 0, "tile staging");
    static_assert(LDS_BYTES_QF32 <= 160 * 1024, "LDS");
};

// Slot of global chunk c of K row r and of V row r (XOR swizzles that keep the operand reads
// free of bank conflicts: a K operand read spreads its 32 rows over 16 slots; a transposing V
// read puts its 4 rows x 64 bytes per 32 lanes on disjoint banks).
template <int HD>
__device__ __forceinline__ int wk_slot(int r, int c) { return c ^ (r & WideLayout<HD, 1>::SWZ); }
template <int HD>
__device__ __forceinline__ int wv_slot(int r, int c)
{
    return c ^ ((WideLayout<HD, 1>::ROW % 256 == 0) ? 4 * (r & 3) : 4 * ((r >> 1) & 1));
}

// ds_read_b64_tr_b16 as inline asm: the builtin makes the compiler drain every in-flight
// buffer-load-to-LDS first (it cannot tell the ring slots apart).  The reads are waited for
// explicitly (wait_lgkm); LDS operations of a wave complete in order.
template <int OFF>
__device__ __forceinline__ u32x2 ds_read_tr16(const lds_u8* p)
{
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(p), "i"(OFF) : "memory");
    return r;
}
// ds_read_b128 as inline asm, for the same reason (K operands); waited for with wait_lgkm
template <int OFF>
__device__ __forceinline__ u32x4 ds_read_b128(const lds_u8* p)
{
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(p), "i"(OFF) : "memory");
    return r;
}
// s_waitcnt lgkmcnt(N), ordered before every use of the registers
template <int N>
__device__ __forceinline__ void wait_lgkm(u32x2& a, u32x2& b)
{
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}
template <int N>
__device__ __forceinline__ void wait_lgkm(u32x4& a)
{
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "i"(N));
}
template <int N>
__device__ __forceinline__ void wait_lgkm(u32x4& a, u32x4& b)
{
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}
// ds_write_b128 as inline asm (a plain LDS store makes the compiler drain the ring's loads)
__device__ __forceinline__ void ds_write_b128(lds_u8* p, u32x4 v)
{
    asm volatile("ds_write_b128 %0, %1" : : "v"(p), "v"(v) : "memory");
}

// f(std::integral_constant<int, I>) for I = B .. E-1, unrolled at compile time
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// operand read-ahead: V^T operand groups in flight ahead of the PV MFMAs, K operands ahead of
// the S MFMAs
constexpr int kWideVAhead = 2;
constexpr int kWideKAhead = 4;

// Head dim 256: a 32-row wave's O (128 registers) and Q^T operands (64) do not fit two waves
// per SIMD, so the kernel runs one wave per SIMD with both held in AGPRs -- MFMAs take C/D and
// A/B from AGPRs, the VALU does not -- which is the only allocation in which the compiler does
// not shuttle accumulators between the two register files.  Those MFMAs are inline asm with
// AGPR operand constraints, and the hazard waits the compiler would insert for them are
// written here (gfx950): two wait states before each MFMA (for a VALU or AGPR write of one of
// its operands just before it), and 20 (> 18 for a 16-pass 32x32 MFMA) between the last MFMA
// writing a result and the first VALU access to it, tied to every register of the result.
template <int HD>
constexpr bool wide_agpr() { return HD > 128; }
//   O^T += A B, accumulator in AGPRs
__device__ __forceinline__ void mfma_acc(f32x16& acc, f16x8 a, f16x8 b)
{
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
//   S^T = A B + C, B (Q^T) in AGPRs, S in VGPRs
template <bool FIRST>
__device__ __forceinline__ void mfma_s(f32x16& d, f16x8 a, const f16x8& b, const f32x16& c0)
{
    if constexpr (FIRST)
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %3" : "=&v"(d) : "v"(a), "a"(b), "v"(c0));
    else
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
}
//   S^T = A B (no bias), B in AGPRs
__device__ __forceinline__ void mfma_s_zero(f32x16& d, f16x8 a, const f16x8& b)
{
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "a"(b));
}
//   S^T += A B, B (the f16 residual of f32 queries) in VGPRs
__device__ __forceinline__ void mfma_s_lo(f32x16& d, f16x8 a, f16x8 b)
{
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
template <int N1, int N2>
__device__ __forceinline__ void acc_settle(f32x16 (&x)[N1][N2])
{
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+a"(x[0][0]));
#pragma unroll
    for (int i = 0; i < N1; ++i)
#pragma unroll
        for (int j = 0; j < N2; ++j) asm volatile("" : "+a"(x[i][j]));
}
template <int N1, int N2>
__device__ __forceinline__ void s_settle(f32x16 (&x)[N1][N2])
{
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(x[0][0]));
#pragma unroll
    for (int i = 0; i < N1; ++i)
#pragma unroll
        for (int j = 0; j < N2; ++j) asm volatile("" : "+v"(x[i][j]));
}

// The bias (SrcC) of the first S MFMA of a tile is read by the MFMA over its passes: its
// registers must not be rewritten (a VALU result, an LDS read landing) until the MFMA is done.
// A use after the settle keeps them allocated until then.
template <int N>
__device__ __forceinline__ void keep_bias(const f32x16 (&x)[N])
{
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) asm volatile("" ::"v"(x[i][v]));   // per element: the host pass has no 64-byte "v" operand
}

// s_waitcnt vmcnt(n) (expcnt and lgkmcnt left at their maxima)
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0f70; }

}  // namespace

template <int HD, int KS, bool Q_F32, bool O_F32, bool EXT>
__global__ void __launch_bounds__(kPrefillThreads, kWideRowsPerWave == 32 && !wide_agpr<HD>() ? 2 : 1)
prefill_wide_kernel(PrefillArgs a)
{
    using L = WideLayout<HD, KS>;
    constexpr int BN = L::BN, SB = L::SB, NB = L::NB, BM = L::BM;
    constexpr int KSTEPS = HD / 16, DBLK = HD / 32;
    constexpr int RPW = kWideRowsPerWave;
    constexpr bool kAgpr = wide_agpr<HD>();               // O and Q^T in AGPRs (asm MFMAs)
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    lds_u8* lds3 = (lds_u8*)lds;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, hh = lane >> 5;
    const int rw = wave % L::RWAVES, kg = wave / L::RWAVES;

    // ---- work item: (kv head, query block [heaviest first], q head in group, key split).
    // Packed (short chunks): a block's rows are the (query, head-in-group) pairs p of its kv head
    // -- query p / group, head kv * group + p % group -- so the group's heads share every K/V tile
    // and no block is padded to its row count; the item then has no head index.
    const int heads_per_item = a.pack ? 1 : a.group;
    const int per_kv = heads_per_item * a.n_qblocks * a.n_splits;
    const int item = xcd_remap_kv(pair_rotate(blockIdx.x, a.pair_rot, a.pair_span), a.n_items, a.n_kv_heads, per_kv, a.n_splits);
    const int kvh = item / per_kv;
    int r = item - kvh * per_kv;
    const int qb = a.n_qblocks - 1 - r / (heads_per_item * a.n_splits);
    r %= heads_per_item * a.n_splits;
    const int g = r / a.n_splits;
    const int split = r - g * a.n_splits;
    const int h = kvh * a.group + g;                      // the block's q head (not packed)
    const int n_rows = a.pack ? a.n_query * a.group : a.n_query;   // rows of the block row space
    auto row_query = [&](int p) { return a.pack ? p / a.group : p; };
    auto row_head = [&](int p) { return a.pack ? kvh * a.group + p % a.group : h; };

    // ---- key tiles of this workgroup: [t0, t1) of the block's tiles t_lo .. k_hi / BN, split
    // evenly over n_splits workgroups; keys from kmax on belong to later splits (or past the
    // cache end) and are masked.  A sliding window starts the range at the tile of the first
    // row's first key (later rows' earlier keys are masked).
    const int q0 = qb * BM;                               // first row of the block
    const int qa = row_query(q0), qz = row_query(min(q0 + BM, n_rows) - 1);   // its first and last query
    const int k_hi = min(a.q_base + qz, a.n_ctx - 1);
    const int n_tiles = k_hi / BN + 1;
    const bool swa = a.sliding_window > 0;
    const int t_lo = swa ? min(max(0, a.q_base + qa + 1 - a.sliding_window) / BN, n_tiles) : 0;
    const int tps = (n_tiles - t_lo + a.n_splits - 1) / a.n_splits;
    const int t0 = min(t_lo + split * tps, n_tiles), t1 = min(t0 + tps, n_tiles);
    const int kmax = min(a.n_ctx, t1 * BN);
    const int n_steps = (t1 - t0 + KS - 1) / KS;         // 0 for an empty split

    // ---- this wave's rows.  Every wave runs all n_steps steps of the workgroup (same trip
    // count, no per-wave branches in the loop): tiles past a wave's diagonal are fully masked
    // for it, and key group 1 of an odd tile count takes one tile past t1 (loaded like any
    // other, zero past the cache end, fully masked).
    const int w_first = q0 + RPW * rw;                    // first row of this wave
    const bool wave_active = w_first < n_rows;
    const int wq_first = row_query(w_first), wq_last = row_query(w_first + RPW - 1);   // the wave's queries
    int qpos[NB];
#pragma unroll
    for (int rb = 0; rb < NB; ++rb) qpos[rb] = a.q_base + row_query(w_first + 32 * rb + n);

    // ---- K/V staging: thread tid, load j fills LDS bytes 16 * (256 j + tid) of a tile
    const uint32_t kv_bytes = (uint32_t)a.n_ctx * HD * 2;
    const rsrc_t krs = make_rsrc_uniform(a.k + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    const rsrc_t vrs = make_rsrc_uniform(a.v + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    // The K swizzle depends on the row modulo 16 and the V swizzle on the row modulo 4 (or
    // 2), and load j + 1 lands 4096 bytes after load j: 16 or more rows at head dim <= 128,
    // so one per-lane offset serves every load (load j adds 4096 j); 8 rows at head dim 256,
    // where loads of odd j take the K offset of the row 8 further on.  At head dim 192 (rows
    // of 384 bytes) a load covers 10 2/3 rows: each load has its own offsets.
    constexpr bool kRowAligned = 4096 % L::ROW == 0;
    constexpr int RPL = kRowAligned ? kPrefillThreads * 16 / L::ROW : 0;   // rows per load
    static_assert(!kRowAligned || RPL % 16 == 0 || RPL == 8, "swizzle period");
    constexpr int NKOFF = kRowAligned ? 2 : L::LOADS, NVOFF = kRowAligned ? 1 : L::LOADS;
    int koff[NKOFF], voff[NVOFF];                          // minus 4096 j, added back per load
    if constexpr (kRowAligned) {
        const int b = 16 * tid;
        const int row = b / L::ROW, slot = (b % L::ROW) / 16;
        koff[0] = row * L::ROW + 16 * wk_slot<HD>(row, slot);
        koff[1] = row * L::ROW + 16 * wk_slot<HD>(row + RPL, slot);
        voff[0] = row * L::ROW + 16 * wv_slot<HD>(row, slot);
    } else {
#pragma unroll
        for (int j = 0; j < L::LOADS; ++j) {
            const int b = 16 * tid + 4096 * j;
            const int row = b / L::ROW, slot = (b % L::ROW) / 16;
            koff[j] = row * L::ROW + 16 * wk_slot<HD>(row, slot) - 4096 * j;
            voff[j] = row * L::ROW + 16 * wv_slot<HD>(row, slot) - 4096 * j;
        }
    }
    // tiles of step `st`: tile st * KS + i goes to slot (st % 2) * KS + i.  Loads past the cache
    // end are issued too (the descriptor returns zeros): every step issues the same number of
    // loads, so a fixed vmcnt tells when a step's tiles have landed.
    constexpr int D = L::DEPTH;
    constexpr int LPS = 2 * L::LOADS * KS;                 // loads per thread per step (K + V)
    static_assert((D - 1) * LPS <= 63, "vmcnt range");
    auto issue_tiles = [&](int st, bool k_side) {
        const int slot0 = (st & 1) * KS;
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            const int base = (t0 + st * KS + i) * BN * L::ROW;
            lds_u8* dst = lds3 + (k_side ? 0 : L::VBASE) + (slot0 + i) * L::TILE + 1024 * wave;
#pragma unroll
            for (int j = 0; j < L::LOADS; ++j) {
                // the whole offset in the vector operand: the descriptor's range check
                // (zeros past the cache end) covers it.  (Computed before the builtin: with the
                // array selection inside its argument list the host pass drops the kernel.)
                const int goff = (k_side ? koff[kRowAligned ? (RPL == 8 ? (j & 1) : 0) : j]
                                         : voff[kRowAligned ? 0 : j]) + base + 4096 * j;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    k_side ? krs : vrs, (void __attribute__((address_space(3)))*)(dst + 4096 * j), 16, goff, 0, 0, 0);
            }
        }
    };
    // group st: what step st consumes, K(st + 1) and V(st)
    auto issue_group = [&](int st) {
        issue_tiles(st + 1, true);
        issue_tiles(st, false);
    };

    // ---- Q^T operands of both row blocks, pre-scaled by scale * log2(e): lane (row n, k-group
    // hh) holds dims 16 ks + 8 hh .. +7.  The raw loads go out first, then the ring prologue,
    // then the conversion (which waits for the Q loads only).
    constexpr uint32_t QE = Q_F32 ? 4u : 2u;
    constexpr int QV = Q_F32 ? 2 : 1;                      // 16-byte loads per k-step
    u32x4 qraw[NB][KSTEPS][QV];
    {
        const size_t row_bytes = (size_t)a.n_q_heads * HD * QE;
        const rsrc_t qr = make_rsrc_uniform((const char*)a.q + (size_t)qa * row_bytes, (uint32_t)((qz - qa + 1) * row_bytes));
#pragma unroll
        for (int rb = 0; rb < NB; ++rb) {
            // rows past the row space point past the descriptor and read as zero
            const int p = q0 + RPW * rw + 32 * rb + n;
            const uint32_t qoff = p < n_rows ? (uint32_t)((size_t)(row_query(p) - qa) * row_bytes +
                                                          ((size_t)row_head(p) * HD + 8 * hh) * QE)
                                             : 0x7fffff00u;
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
                for (int u = 0; u < QV; ++u) qraw[rb][ks][u] = buf_load16(qr, qoff + 16 * QE * ks + 16 * u);
        }
    }

    // ring prologue: K(0), then the groups of steps 0 .. D - 2 (kept behind the Q loads, so
    // converting Q waits for Q only)
    __builtin_amdgcn_sched_barrier(0);
    if (n_steps > 0) {
        issue_tiles(0, true);
#pragma unroll
        for (int st = 0; st < D - 1; ++st) issue_group(st);
    }
    __builtin_amdgcn_sched_barrier(0);

    static_assert(NB == 1 || !Q_F32, "the residual Q^T reads in the pipelined S phase assume one row block");
    f16x8 qt[NB][KSTEPS];
    // this lane's 16 bytes of the row wave's residual Q^T operands (f32 queries)
    const int qlo_lane = L::RING_BYTES + rw * L::QLO_WAVE + 16 * lane;
#pragma unroll
    for (int rb = 0; rb < NB; ++rb)
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            float x[8];
            if constexpr (Q_F32) {
                const f32x4 x0 = __builtin_bit_cast(f32x4, qraw[rb][ks][0]);
                const f32x4 x1 = __builtin_bit_cast(f32x4, qraw[rb][ks][QV - 1]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[i] = x0[i];
                    x[4 + i] = x1[i];
                }
            } else {
                const f16x8 hq = as_f16x8(qraw[rb][ks][0]);
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = (float)hq[i];
            }
            // the query as given: the scale goes onto the scores in f32
            qt[rb][ks] = cvt_f16x8(x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]);
            if constexpr (Q_F32) {
                // the f16 residual, one copy per row wave (key group 0 writes it); read by the
                // second MFMA of each k-step
                const f16x8 hq = qt[rb][ks];
                const f16x8 lo = cvt_f16x8(x[0] - (float)hq[0], x[1] - (float)hq[1], x[2] - (float)hq[2],
                                           x[3] - (float)hq[3], x[4] - (float)hq[4], x[5] - (float)hq[5],
                                           x[6] - (float)hq[6], x[7] - (float)hq[7]);
                if (kg == 0) ds_write_b128(lds3 + qlo_lane + (rb * KSTEPS + ks) * 1024, as_u32x4(lo));
            }
            if constexpr (kAgpr) asm volatile("" : "+a"(qt[rb][ks]));    // its home: AGPRs
        }
    if constexpr (Q_F32) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // before the prologue barrier

    // ---- per-lane LDS read offsets within a tile
    // K operand of block sb, k-step ks: row 32 sb + n, chunk 2 ks + hh
    int ka_off[KSTEPS];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) ka_off[ks] = kg * L::TILE + n * L::ROW + 16 * wk_slot<HD>(n, 2 * ks + hh);
    // V^T transposing reads: source lane i = lane & 15 of each 16-lane group addresses
    // V[kb + i/4][d0 + 4 (i%4)], kb = 32 sb + 16 j + 4 hh (+8 for the second read),
    // d0 = 32 db + 16 ((lane >> 4) & 1); within a 16-lane group the read hands lane j the four
    // keys kb .. kb+3 of dim d0 + j
    int vt_off[DBLK];
    {
        const int i = lane & 15;
        const int rr = 4 * hh + (i >> 2);
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
            const int dim = 32 * db + 16 * ((lane >> 4) & 1) + 4 * (i & 3);
            vt_off[db] = L::VBASE + kg * L::TILE + rr * L::ROW + 16 * wv_slot<HD>(rr, dim >> 3) + 8 * ((dim >> 2) & 1);
        }
    }

    // ---- online-softmax state per row block: running max m_used (units of the raw score
    // q.k; log2 units with EXT), its negated splat (seed of every S^T accumulator), `seen`
    // (the row has had a visible key) and this lane's share of the row sum.  cs turns a
    // seeded accumulator into log2 units (applied where the row max is taken, so the tile is
    // in log2 units from then on: p = exp2(S)); inv_cs turns a log2 step back into raw units.
    const float cs = EXT ? 1.f : a.scale_log2;
    const float inv_cs = EXT ? 1.f : 1.f / a.scale_log2;
    f32x16 o[NB][DBLK];
    f32x16 negm[NB];
    float m_used[NB], l_part[NB];
    bool seen[NB];
#pragma unroll
    for (int rb = 0; rb < NB; ++rb) {
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[rb][db][v] = 0.f;
        if constexpr (kAgpr)
#pragma unroll
            for (int db = 0; db < DBLK; ++db) asm volatile("" : "+a"(o[rb][db]));
#pragma unroll
        for (int v = 0; v < 16; ++v) negm[rb][v] = 0.f;
        m_used[rb] = 0.f;
        l_part[rb] = 0.f;
        seen[rb] = false;
    }

    // S^T tiles, double buffered: the step that exponentiates one computes the next tile's
    // into the other (the two swap roles from step to step, so no copies)
    typedef f32x16 STile[NB][SB];
    STile sA, sB;
    constexpr bool kSCopy = NB > 1;

    // byte offset of ring slot parity `par` (key group 0) for K or V; the key group's slot
    // offset is folded into ka_off / vt_off
    constexpr int SLOT_PAR = KS * L::TILE;

    // S^T of one tile, not interleaved (prologue)
    auto s_tile = [&](STile& sn) {
        static_for<0, KSTEPS * SB>([&](auto I) {
            constexpr int i = decltype(I)::value, ks = i / SB, sb = i % SB;
            u32x4 ka = ds_read_b128<32 * sb * L::ROW>(lds3 + ka_off[ks]);
            u32x4 ql[NB];
            if constexpr (Q_F32)
#pragma unroll
                for (int rb = 0; rb < NB; ++rb) ql[rb] = ds_read_b128<0>(lds3 + qlo_lane + (rb * KSTEPS + ks) * 1024);
            wait_lgkm<0>(ka);
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) {
                if constexpr (Q_F32) wait_lgkm<0>(ql[rb]);
                if constexpr (kAgpr && ks == 0)
                    mfma_s_zero(sn[rb][sb], __builtin_bit_cast(f16x8, ka), qt[rb][ks]);   // m = 0 here
                else if constexpr (kAgpr)
                    mfma_s<false>(sn[rb][sb], __builtin_bit_cast(f16x8, ka), qt[rb][ks], negm[rb]);
                else
                    sn[rb][sb] = mfma32x32x16(__builtin_bit_cast(f16x8, ka), qt[rb][ks], ks == 0 ? negm[rb] : sn[rb][sb]);
                if constexpr (Q_F32) {
                    if constexpr (kAgpr)
                        mfma_s_lo(sn[rb][sb], __builtin_bit_cast(f16x8, ka), __builtin_bit_cast(f16x8, ql[rb]));
                    else
                        sn[rb][sb] = mfma32x32x16(__builtin_bit_cast(f16x8, ka), __builtin_bit_cast(f16x8, ql[rb]), sn[rb][sb]);
                }
            }
        });
    };
    // causal / cache-end / window mask of tile t; wave-uniform test (diagonal and last tiles,
    // and tiles with keys before the window of the wave's last row)
    auto tile_needs_mask = [&](int t) {
        return t * BN + BN - 1 > a.q_base + wq_first || t * BN + BN > kmax ||
               (swa && t * BN < a.q_base + wq_last + 1 - a.sliding_window);
    };
    auto mask_tile = [&](STile& sv, int t) {
        const int key0 = t * BN;
#pragma unroll
        for (int rb = 0; rb < NB; ++rb)
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = key0 + 32 * sb + 8 * (v >> 2) + 4 * hh + (v & 3);
                    bool vis = key <= qpos[rb] && key < kmax;
                    if (swa) vis = vis && key >= qpos[rb] + 1 - a.sliding_window;
                    sv[rb][sb][v] = vis ? sv[rb][sb][v] : -INFINITY;
                }
    };
    auto row_max = [&](const STile& sv, int rb) {
        float m = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int v = 0; v < 16; v += 2) m = __builtin_fmaxf(m, __builtin_fmaxf(sv[rb][sb][v], sv[rb][sb][v + 1]));
        return max_xor32(m);
    };
    // lazy rescale: a row moves its max when it first sees a key, or when its scores exceed
    // the current max by more than 2^8
    auto rescale = [&](STile& sv, const float (&mx)[NB]) {
        bool need[NB];
        bool any_need = false;
#pragma unroll
        for (int rb = 0; rb < NB; ++rb) {
            need[rb] = seen[rb] ? (mx[rb] > kRescaleThresh) : (mx[rb] > -INFINITY);
            any_need = any_need || need[rb];
        }
        if (__any(any_need)) {
            if constexpr (kAgpr) acc_settle(o);
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) {
                const float d = need[rb] ? mx[rb] : 0.f;      // log2 units
                const float corr = fast_exp2(-d);
                m_used[rb] += d * inv_cs;
                seen[rb] = seen[rb] || need[rb];
                l_part[rb] *= corr;
#pragma unroll
                for (int db = 0; db < DBLK; ++db) {
                    o[rb][db] *= corr;
                    if constexpr (kAgpr) asm volatile("" : "+a"(o[rb][db]));
                }
#pragma unroll
                for (int sb = 0; sb < SB; ++sb) sv[rb][sb] -= d;
                if constexpr (!EXT)
#pragma unroll
                    for (int v = 0; v < 16; ++v) negm[rb][v] = -m_used[rb];
            }
        }
    };
    // EXT: the MFMAs leave raw scores x = q.k (accumulators seeded with 0); the VALU turns each
    // into softcap * tanh(x scale / softcap) * log2(e) - m = (c2 - m) - 2 c2 / (2^(x c1) + 1)
    // with c1 = 2 log2(e) scale / softcap and c2 = softcap log2(e) (tanh(y) = 1 - 2 / (e^(2y) + 1),
    // as softcap_log2): a multiply, v_exp_f32, an add, v_rcp_f32 and one fma per score
    const bool capped = EXT && a.softcap > 0.f;
    const float cap_c1 = capped ? 2.f * kLog2e * a.scale / a.softcap : a.scale * kLog2e;
    const float cap_c2 = a.softcap * kLog2e;
    auto ext_score = [&](float x, int rb) {
        if (!capped) return x * cap_c1 - m_used[rb];
        return __builtin_fmaf(-2.f * cap_c2, __builtin_amdgcn_rcpf(fast_exp2(x * cap_c1) + 1.f), cap_c2 - m_used[rb]);
    };
    // finish tile t's scores: mask if needed, row max, rescale
    auto finish_scores = [&](STile& sv, int t, float (&mx)[NB]) {
        if (tile_needs_mask(t)) {
            mask_tile(sv, t);
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) mx[rb] = row_max(sv, rb);
        }
        rescale(sv, mx);
    };
    // P(t) in packed f16 pairs: pw[rb][sb][j][w] holds the B-operand dword w of keys
    // 8 j + 2 w .. +1 of S^T block sb (register v = 8 j + 2 w of the accumulator)
    typedef uint32_t PTile[NB][SB][2][4];
    // probabilities of flattened score elements e, e + 1 (e = (rb * SB + sb) * 16 + v): exp2,
    // f16 pack, fp32 row sum.  (The sum uses fp32 adds, not v_dot2 on the packed pair: on
    // gfx950 v_dot2 does not issue alongside the MFMAs, the adds do.)
    auto p_pair = [&](const STile& sc, PTile& pw, int e) {
        const int rb = e / (SB * 16), sb = (e / 16) % SB, v = e % 16;
        const f32x2 x = {fast_exp2(sc[rb][sb][v]), fast_exp2(sc[rb][sb][v + 1])};
        const f16x2 h2 = __builtin_convertvector(x, f16x2);
        pw[rb][sb][v / 8][(v % 8) / 2] = __builtin_bit_cast(uint32_t, h2);
        l_part[rb] += x[0] + x[1];
    };
    auto p_operand = [&](const PTile& pw, int rb, int sb, int j) {
        return __builtin_bit_cast(f16x8, u32x4{pw[rb][sb][j][0], pw[rb][sb][j][1], pw[rb][sb][j][2], pw[rb][sb][j][3]});
    };
    constexpr int KITER = KSTEPS * SB;                   // K operand reads per tile
    constexpr int PELEMS = NB * SB * 16;                 // score elements per lane per tile
    // the P work (score pairs) is spread over the K MFMA slots and the row-max work over the
    // PV groups: slot i of n takes pairs [i * PAIRS / n, (i + 1) * PAIRS / n)
    constexpr int PAIRS = PELEMS / 2;

    // Phase A of a step: S^T(next) = K Q^T - m on the MFMAs, with P(t) on the VALU.  The
    // program order below is the issue order (sched_barrier between slices): K reads run
    // four operands ahead (explicit lgkmcnt waits: the only LDS operations in flight are
    // these reads), each MFMA slot carries 1/KITER of the P work.
    auto phase_a = [&](auto KPAR, const STile& sc, STile& sn, PTile& pw) {
        constexpr int kbase = decltype(KPAR)::value * SLOT_PAR;
        // f32 queries read the residual operand beside each K operand (two reads per slot,
        // fewer slots ahead to stay within two waves' registers)
        constexpr int KAH = Q_F32 ? 2 : kWideKAhead;
        constexpr int AHEAD = KITER < KAH ? KITER : KAH;
        constexpr int RPS = Q_F32 ? 2 : 1;               // LDS reads per slot
        u32x4 ka[KITER], qlr[KITER];
        auto rd = [&](auto I) {
            constexpr int i = decltype(I)::value, ks = i / SB, sb = i % SB;
            ka[i] = ds_read_b128<kbase + 32 * sb * L::ROW>(lds3 + ka_off[ks]);
            if constexpr (Q_F32) qlr[i] = ds_read_b128<ks * 1024>(lds3 + qlo_lane);
        };
        static_for<0, AHEAD>(rd);
        static_for<0, KITER>([&](auto I) {
            constexpr int i = decltype(I)::value, ks = i / SB, sb = i % SB;
            if constexpr (i + AHEAD < KITER) rd(std::integral_constant<int, i + AHEAD>{});
            // reads issued after read i: i + 1 .. min(i + AHEAD, KITER - 1)
            constexpr int LATER = (KITER - 1 - i) < AHEAD ? (KITER - 1 - i) : AHEAD;
            if constexpr (Q_F32)
                wait_lgkm<RPS * LATER>(ka[i], qlr[i]);
            else
                wait_lgkm<LATER>(ka[i]);
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) {
                if constexpr (kAgpr && EXT && ks == 0)
                    mfma_s_zero(sn[rb][sb], __builtin_bit_cast(f16x8, ka[i]), qt[rb][ks]);   // raw scores
                else if constexpr (kAgpr)
                    mfma_s<ks == 0>(sn[rb][sb], __builtin_bit_cast(f16x8, ka[i]), qt[rb][ks], negm[rb]);
                else
                    sn[rb][sb] = mfma32x32x16(__builtin_bit_cast(f16x8, ka[i]), qt[rb][ks], ks == 0 ? negm[rb] : sn[rb][sb]);
                if constexpr (Q_F32) {
                    if constexpr (kAgpr)
                        mfma_s_lo(sn[rb][sb], __builtin_bit_cast(f16x8, ka[i]), __builtin_bit_cast(f16x8, qlr[i]));
                    else
                        sn[rb][sb] = mfma32x32x16(__builtin_bit_cast(f16x8, ka[i]), __builtin_bit_cast(f16x8, qlr[i]), sn[rb][sb]);
                }
            }
#pragma unroll
            for (int pr = i * PAIRS / KITER; pr < (i + 1) * PAIRS / KITER; ++pr) p_pair(sc, pw, 2 * pr);
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // O^T += V^T P^T over one tile, operand group gv = (sb, j, db); two groups of V^T reads in
    // flight ahead of the MFMAs; between(gv) is VALU work issued behind group gv's MFMAs
    constexpr int VGROUPS = SB * 2 * DBLK;
    auto pv_tile = [&](auto VPAR, const PTile& pw, auto between) {
        constexpr int vbase = decltype(VPAR)::value * SLOT_PAR;
        constexpr int VAH = kWideVAhead < VGROUPS ? kWideVAhead : VGROUPS;   // groups in flight
        u32x2 vr[VGROUPS][2];
        auto rd = [&](auto GV) {
            constexpr int gv = decltype(GV)::value;
            constexpr int sb = gv / (2 * DBLK), j = (gv / DBLK) % 2, db = gv % DBLK;
            vr[gv][0] = ds_read_tr16<vbase + (32 * sb + 16 * j) * L::ROW>(lds3 + vt_off[db]);
            vr[gv][1] = ds_read_tr16<vbase + (32 * sb + 16 * j + 8) * L::ROW>(lds3 + vt_off[db]);
        };
        static_for<0, VAH>(rd);
        static_for<0, VGROUPS>([&](auto GV) {
            constexpr int gv = decltype(GV)::value;
            constexpr int sb = gv / (2 * DBLK), j = (gv / DBLK) % 2, db = gv % DBLK;
            if constexpr (gv + VAH < VGROUPS) rd(std::integral_constant<int, gv + VAH>{});
            // reads issued after group gv's: groups gv + 1 .. min(gv + VAH, VGROUPS - 1)
            constexpr int LATER = (VGROUPS - 1 - gv) < VAH ? (VGROUPS - 1 - gv) : VAH;
            wait_lgkm<2 * LATER>(vr[gv][0], vr[gv][1]);
            const f16x8 va = __builtin_bit_cast(f16x8, u32x4{vr[gv][0][0], vr[gv][0][1], vr[gv][1][0], vr[gv][1][1]});
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) {
                if constexpr (kAgpr)
                    mfma_acc(o[rb][db], va, p_operand(pw, rb, sb, j));
                else
                    o[rb][db] = mfma32x32x16(va, p_operand(pw, rb, sb, j), o[rb][db]);
            }
            between(GV);
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // sync point of step s: this step's tiles landed, older slots free; the next loads go out
    // The ring needs no memory fence: the loads land in LDS, each thread waits for its own
    // (vmcnt) and every LDS read of the previous step has returned (lgkmcnt) before the
    // barrier.  (A workgroup fence here makes the compiler drain every in-flight load.)
    // Wave priorities (s_setprio): 0 through the sync and the score finish, 1 through phase A,
    // 2 through phase B.  When the two waves of a SIMD drift out of step, the arbiter then
    // favours the one feeding the matrix core, and within the MFMA phases the one nearer the
    // end of its step; measured on MI355X: cfg2 73.4 -> 65.3 us, cfg3 743 -> 710 us, against
    // 66-70 us / 718-727 us for a single raised level or for raising phase A only.
    auto step_sync = [&](int s) {
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_s_waitcnt(wait_vm((D - 2) * LPS));  // this thread's group s landed
        __builtin_amdgcn_s_barrier();                        // ... every thread's; step s-1 done
        issue_group(s + D - 1);                              // into the slots step s-1 freed
        __builtin_amdgcn_s_setprio(1);
    };
    // one full step: P(t) from sc, O += V(t)^T P(t)^T; S(t + KS) into sn, t = s KS + kg
    // sc: S(t) (VALU side); sn: where the MFMAs put S(tn).  kSCopy: sn is a separate MFMA
    // accumulator whose values are copied into sc during phase B (then sc holds S(tn) for the
    // next step); otherwise sc and sn swap roles from step to step.
    auto step_full = [&](int s, auto PAR, STile& sc, STile& sn) {
        constexpr int par = decltype(PAR)::value;                 // s % 2
        step_sync(s);
        const int tn = t0 + (s + 1) * KS + kg;
        PTile pw;
        // phase A: S(tn) MFMAs, P(t) on the VALU
        phase_a(std::integral_constant<int, par ^ 1>{}, sc, sn, pw);
        if constexpr (kAgpr) {
            s_settle(sn);                                  // S(tn) is read by the VALU below
            if constexpr (!EXT) keep_bias(negm);
        }
        __builtin_amdgcn_s_setprio(2);
        // phase B: PV(t) MFMAs, row max of S(tn) on the VALU (running max3 over element pairs)
        STile& sx = kSCopy ? sc : sn;
        float mrun[NB];
#pragma unroll
        for (int rb = 0; rb < NB; ++rb) mrun[rb] = -INFINITY;
        pv_tile(PAR, pw, [&](auto GV) {
            constexpr int gv = decltype(GV)::value;
#pragma unroll
            for (int pr = gv * PAIRS / VGROUPS; pr < (gv + 1) * PAIRS / VGROUPS; ++pr) {
                const int e = 2 * pr;
                const int rb = e / (SB * 16), sb = (e / 16) % SB, v = e % 16;
                if constexpr (kSCopy) {
                    sc[rb][sb][v] = sn[rb][sb][v];
                    sc[rb][sb][v + 1] = sn[rb][sb][v + 1];
                }
                if constexpr (EXT) {
                    sx[rb][sb][v] = ext_score(sx[rb][sb][v], rb);
                    sx[rb][sb][v + 1] = ext_score(sx[rb][sb][v + 1], rb);
                } else {
                    sx[rb][sb][v] *= cs;                          // raw units -> log2 units
                    sx[rb][sb][v + 1] *= cs;
                }
                mrun[rb] = __builtin_fmaxf(mrun[rb], __builtin_fmaxf(sx[rb][sb][v], sx[rb][sb][v + 1]));
            }
        });
        float mx[NB];
#pragma unroll
        for (int rb = 0; rb < NB; ++rb) mx[rb] = max_xor32(mrun[rb]);
        __builtin_amdgcn_s_setprio(0);
        finish_scores(sx, tn, mx);
    };
    // the last step: P(t) and O += V(t)^T P(t)^T only
    auto step_last = [&](int s, auto PAR, STile& sc) {
        step_sync(s);
        PTile pw;
#pragma unroll
        for (int e = 0; e < PELEMS; e += 2) p_pair(sc, pw, e);
        pv_tile(PAR, pw, [](auto) {});
        // the paths into the epilogue join here: the compiler's register copies that join
        // them come after this wait
        if constexpr (kAgpr) acc_settle(o);
    };

    if (n_steps > 0) {                                     // workgroup-uniform: empty split
        // ---- prologue: K(0) resident, S of this wave's first tile
        __builtin_amdgcn_s_waitcnt(wait_vm((D - 1) * LPS));
        __builtin_amdgcn_s_barrier();
        {
            if constexpr (kSCopy) {
                s_tile(sB);
                if constexpr (kAgpr) s_settle(sB);
#pragma unroll
                for (int rb = 0; rb < NB; ++rb)
#pragma unroll
                    for (int sb = 0; sb < SB; ++sb) sA[rb][sb] = sB[rb][sb];
            } else {
                s_tile(sA);
                if constexpr (kAgpr) s_settle(sA);
            }
#pragma unroll
            for (int rb = 0; rb < NB; ++rb)
#pragma unroll
                for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) sA[rb][sb][v] = EXT ? ext_score(sA[rb][sb][v], rb) : sA[rb][sb][v] * cs;
            float mx[NB];
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) mx[rb] = row_max(sA, rb);
            finish_scores(sA, t0 + kg, mx);
        }
        // ---- key loop: n_steps - 1 full steps, two per iteration (S buffers swap roles), then
        // the last step
        int s = 0;
        if constexpr (kSCopy) {
            for (; s + 2 < n_steps; s += 2) {
                step_full(s, std::integral_constant<int, 0>{}, sA, sB);
                step_full(s + 1, std::integral_constant<int, 1>{}, sA, sB);
            }
            if (s + 1 < n_steps) {
                step_full(s, std::integral_constant<int, 0>{}, sA, sB);
                step_last(s + 1, std::integral_constant<int, 1>{}, sA);
            } else {
                step_last(s, std::integral_constant<int, 0>{}, sA);
            }
        } else {
            for (; s + 2 < n_steps; s += 2) {
                step_full(s, std::integral_constant<int, 0>{}, sA, sB);
                step_full(s + 1, std::integral_constant<int, 1>{}, sB, sA);
            }
            if (s + 1 < n_steps) {
                step_full(s, std::integral_constant<int, 0>{}, sA, sB);
                step_last(s + 1, std::integral_constant<int, 1>{}, sB);
            } else {
                step_last(s, std::integral_constant<int, 0>{}, sA);
            }
        }
    }

    // the loads past the end are still in flight: none may land in LDS after this point
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_waitcnt(wait_vm(0));
    if constexpr (kAgpr) acc_settle(o);

    // ---- epilogue
    float l_tot[NB], m_out[NB];
#pragma unroll
    for (int rb = 0; rb < NB; ++rb) {
        l_tot[rb] = sum_xor32(l_part[rb]);
        m_out[rb] = seen[rb] ? m_used[rb] * cs : -INFINITY;              // log2 units
    }

    if constexpr (KS > 1) {
        // key group 1 hands (O, m, l) to key group 0 through LDS; lane-major, conflict free
        __syncthreads();                                     // ring reads done
        float* mrg = (float*)lds + rw * L::MERGE_FLOATS;
        if (kg == 1) {
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) {
#pragma unroll
                for (int db = 0; db < DBLK; ++db)
#pragma unroll
                    for (int v = 0; v < 16; ++v) mrg[((rb * DBLK + db) * 16 + v) * 64 + lane] = o[rb][db][v];
                mrg[NB * DBLK * 16 * 64 + (2 * rb) * 64 + lane] = m_out[rb];
                mrg[NB * DBLK * 16 * 64 + (2 * rb + 1) * 64 + lane] = l_tot[rb];
            }
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int rb = 0; rb < NB; ++rb) {
                const float m1 = mrg[NB * DBLK * 16 * 64 + (2 * rb) * 64 + lane];
                const float l1 = mrg[NB * DBLK * 16 * 64 + (2 * rb + 1) * 64 + lane];
                const float m0 = m_out[rb];
                const float mn = fmaxf(m0, m1);
                const float c0 = mn == -INFINITY ? 0.f : fast_exp2(m0 - mn);
                const float c1 = mn == -INFINITY ? 0.f : fast_exp2(m1 - mn);
                l_tot[rb] = l_tot[rb] * c0 + l1 * c1;
                m_out[rb] = mn;
#pragma unroll
                for (int db = 0; db < DBLK; ++db)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        o[rb][db][v] = o[rb][db][v] * c0 + mrg[((rb * DBLK + db) * 16 + v) * 64 + lane] * c1;
            }
        }
    }
    if (kg != 0 || !wave_active) return;

    if (a.n_splits > 1) {
        // split-KV partial in the reference's format (qwen35_attn_part.comp:3): unnormalised
        // O, then (m, l) with m in natural-log units; a row with no visible key in this split
        // carries the reference's initial max and l = 0.  The combine kernel merges.
#pragma unroll
        for (int rb = 0; rb < NB; ++rb) {
            const int p = w_first + 32 * rb + n;
            if (p >= n_rows) continue;
            const long long prow = (long long)row_query(p) * a.n_q_heads + row_head(p);
            const long long n_all = (long long)a.n_query * a.n_q_heads;
            float* pr = a.part + part_acc(split, prow, n_all, HD);
#pragma unroll
            for (int db = 0; db < DBLK; ++db)
#pragma unroll
                for (int a4 = 0; a4 < 4; ++a4)
                    *(f32x4*)(pr + 32 * db + 8 * a4 + 4 * hh) =
                        f32x4{o[rb][db][4 * a4], o[rb][db][4 * a4 + 1], o[rb][db][4 * a4 + 2], o[rb][db][4 * a4 + 3]};
            if (hh == 0)
                *(f32x2*)(a.part + part_ml(split, prow, n_all, a.n_splits, HD)) =
                    f32x2{m_out[rb] > -INFINITY ? m_out[rb] * kLn2 : kNegBig, l_tot[rb]};
        }
        return;
    }

    // lane (row n, hh) holds dims 32 db + 8 a4 + 4 hh + (0..3) of its row
#pragma unroll
    for (int rb = 0; rb < NB; ++rb) {
        const int p = w_first + 32 * rb + n;
        if (p >= n_rows) continue;
        const float inv = l_tot[rb] > 0.f ? 1.f / l_tot[rb] : 0.f;
        const size_t obase = ((size_t)row_query(p) * a.n_q_heads + row_head(p)) * HD;
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const int dim = 32 * db + 8 * a4 + 4 * hh;
                const f32x4 gt = gate4(a.gate, obase + dim);
                const float v0 = o[rb][db][4 * a4] * inv * gt[0], v1 = o[rb][db][4 * a4 + 1] * inv * gt[1];
                const float v2 = o[rb][db][4 * a4 + 2] * inv * gt[2], v3 = o[rb][db][4 * a4 + 3] * inv * gt[3];
                if constexpr (O_F32) {
                    *(f32x4*)((float*)a.out + obase + dim) = f32x4{v0, v1, v2, v3};
                } else {
                    f32x2 p0 = {v0, v1}, p1 = {v2, v3};
                    f16x2 h0 = __builtin_convertvector(p0, f16x2);
                    f16x2 h1 = __builtin_convertvector(p1, f16x2);
                    *(u32x2*)((uint16_t*)a.out + obase + dim) =
                        u32x2{__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
                }
            }
    }
}

// ---- launchers

int prefill_wide_rows(int ks) { return (4 / ks) * kWideRowsPerWave; }

template <int HD, int KS, bool QF, bool OF, bool EXT>
static hipError_t launch_wide_t(const PrefillArgs& a, hipStream_t stream)
{
    constexpr int lds_bytes = QF ? WideLayout<HD, KS>::LDS_BYTES_QF32 : WideLayout<HD, KS>::LDS_BYTES;
    static std::atomic<uint64_t> lds_set{0};          // devices whose LDS limit is raised
    const hipError_t e = ensure_dyn_lds((const void*)prefill_wide_kernel<HD, KS, QF, OF, EXT>, lds_bytes, lds_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((prefill_wide_kernel<HD, KS, QF, OF, EXT>), dim3(a.n_items), dim3(kPrefillThreads),
                       lds_bytes, stream, a);
    return hipGetLastError();
}

template <int HD, int KS, bool EXT>
static hipError_t launch_wide_qo(const PrefillArgs& a, bool q_f32, bool o_f32, hipStream_t s)
{
    if (q_f32) return o_f32 ? launch_wide_t<HD, KS, true, true, EXT>(a, s) : launch_wide_t<HD, KS, true, false, EXT>(a, s);
    return o_f32 ? launch_wide_t<HD, KS, false, true, EXT>(a, s) : launch_wide_t<HD, KS, false, false, EXT>(a, s);
}

template <int HD, int KS>
static hipError_t launch_wide_ks(const PrefillArgs& a, bool q_f32, bool o_f32, bool ext, hipStream_t s)
{
    return ext ? launch_wide_qo<HD, KS, true>(a, q_f32, o_f32, s) : launch_wide_qo<HD, KS, false>(a, q_f32, o_f32, s);
}

hipError_t launch_prefill_wide(const PrefillArgs& a, int head_dim, int ks, bool q_f32, bool o_f32, bool ext,
                               hipStream_t stream)
{
    if (ks != 1 && ks != 2) return hipErrorInvalidValue;
    switch (head_dim) {
    case 64: return ks == 1 ? launch_wide_ks<64, 1>(a, q_f32, o_f32, ext, stream) : launch_wide_ks<64, 2>(a, q_f32, o_f32, ext, stream);
    case 128: return ks == 1 ? launch_wide_ks<128, 1>(a, q_f32, o_f32, ext, stream) : launch_wide_ks<128, 2>(a, q_f32, o_f32, ext, stream);
    // head dim 256: 128-row blocks only.  Two key groups per workgroup need more registers
    // than one wave per SIMD has (the merge and the second group's state); the compiler then
    // moves accumulator blocks between register files right beside the inline-asm MFMAs.
    case 192: return ks == 1 ? launch_wide_ks<192, 1>(a, q_f32, o_f32, ext, stream) : hipErrorInvalidValue;
    case 256: return ks == 1 ? launch_wide_ks<256, 1>(a, q_f32, o_f32, ext, stream) : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

}  // namespace nxa

// nexus_amd/csrc/attn_prefill.hip -- causal GQA flash-attention prefill for gfx950.
//
// Semantics follow Transformer::attn_batch_cpu (src/model/transformer.h:8653-8685) and
// attn_flash.comp (src/gpu/shaders/attn_flash.comp:66-72, 121-159): query i sits at
// absolute position q_base + i and sees keys [start, min(q_base + i, n_ctx - 1)].
//
// Built for head dim 192 (the pipelined kernel in attn_prefill_wide.hip covers 64, 128 and
// 256).  Design (one workgroup = 128 queries of one q head, 4 waves x 32 queries, 2 per CU):
//  * K/V tiles (BN keys) go from HBM straight into LDS with buffer-load-to-LDS (16 bytes
//    per lane, no VGPR staging, no transpose work) through a ring of STAGES buffers: the
//    next STAGES - 1 tiles are in flight while the current one is consumed, one barrier
//    per tile.  Each lane picks the
//    global chunk whose LDS slot it writes, which XOR-swizzles the 16-byte chunks of every
//    row so the operand reads below are free of bank conflicts.  Rows past the cache end
//    read as zero through the buffer descriptor.
//  * S^T = K Q^T on v_mfma_f32_32x32x16_f16: A = K rows from LDS, B = Q^T in registers for
//    the whole key loop.  Q is pre-multiplied by scale * log2(e), and the accumulator
//    starts at -m (the row's running max, a register splat), so the MFMA result is already
//    s * scale * log2(e) - m and a probability is one exp2.
//  * Online softmax in fp32, lazily rescaled: the running max only moves when a row's new
//    scores exceed it by more than 2^8 (P stays <= 256, safe in f16), which is rare after
//    the first tile; a per-row flag marks rows that have seen a visible key.  Row max: one
//    v_max3 per two scores plus one v_permlane32_swap.  Row sums: v_dot2_f32_f16 on
//    the packed f16 P, i.e. exactly the values the PV MFMA consumes.
//  * O^T += V^T P^T on the same MFMA: B = P^T straight from the S^T registers (the D layout
//    leaves lane (query n, half hh) with keys 8j + 4hh + (0..3)), A = V^T read from the
//    row-major V tile with ds_read_b64_tr_b16: within 16 lanes the transposing read hands
//    lane j four consecutive keys of dim d0 + j, two reads make an 8-key operand.
//  * Work items are remapped so each XCD owns whole KV heads (L2 reuse of K/V); within a KV
//    head the heaviest (latest) query blocks start first.
//  * Optional split of the key range over n_splits workgroups (short chunks over a long
//    cache).  Each split writes fp32 partials (acc, m, l) in the reference's split-K format;
//    the decode path's combine kernel merges them with the LSE rule of
//    qwen35_attn_comb.comp:16-40.
#include "attn_common.h"
#include "attn_kernels.h"

namespace nxa {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Key tile and ring depth: the tiles in flight must cover the K/V load latency (a few us
// from the MALL) while two workgroups share a CU's LDS.
constexpr int prefill_bn(int hd) { return hd <= 128 ? 64 : 32; }
constexpr int prefill_stages(int hd) { return 2 + 0 * hd; }

template <int HD>
struct PrefillLayout {
    static constexpr int BN = prefill_bn(HD);
    static constexpr int SB = BN / 32;                        // 32-key S^T blocks per tile
    static constexpr int ROW = HD * 2;                        // bytes per K/V row
    static constexpr int CPR = HD / 8;                        // 16-byte chunks per row
    static constexpr int TILE = BN * ROW;                     // K (or V) tile bytes
    static constexpr int BUF = 2 * TILE;                      // K + V
    static constexpr int STAGES = prefill_stages(HD);
    static constexpr int LDS_BYTES = STAGES * BUF;            // ring of STAGES tiles
    static constexpr int LOADS = TILE / (kPrefillThreads * 16);   // 16-byte loads per thread per tile
    // chunk swizzles stay inside aligned groups of 16 (or 8) chunks of a row
    static constexpr int SWZ = (CPR % 16 == 0) ? 15 : 7;
    static_assert(LOADS >= 1 && TILE % (kPrefillThreads * 16) == 0, "tile staging");
};

// Slot of global chunk c of K row r, and of V row r.  K: the 32 rows an A-operand read
// touches (same chunk) spread over 16 slots.  V: a transposing read touches 4 consecutive
// rows x 64 bytes per 32 lanes; XOR-ing the chunk with 4 * (row % 4) (rows a multiple of
// 256 bytes apart, which share banks) or 4 * ((row / 2) % 2) (128- or 384-byte rows) puts
// those segments on disjoint banks.
template <int HD>
__device__ __forceinline__ int k_slot(int r, int c) { return c ^ (r & PrefillLayout<HD>::SWZ); }
template <int HD>
__device__ __forceinline__ int v_slot(int r, int c)
{
    return c ^ ((PrefillLayout<HD>::ROW % 256 == 0) ? 4 * (r & 3) : 4 * ((r >> 1) & 1));
}

// Two waves per SIMD (two workgroups per CU) up to head_dim 128; larger head dims need one.
constexpr int prefill_waves_per_simd(int hd) { return hd <= 128 ? 2 : 1; }

// ds_read_b64_tr_b16 issued as inline asm.  The compiler does not see these reads as LDS
// accesses that may alias the in-flight buffer-load-to-LDS of the next tile (the builtin
// makes it drain all of them first, serialising the K/V load latency into every tile).
// The caller waits for them with wait_lgkm0() on the result registers; LDS operations
// complete in order, so untracked reads only ever make the compiler's own lgkmcnt waits
// stronger.
template <int OFF>
__device__ __forceinline__ u32x2 ds_read_tr16_b64(const lds_u8* p)
{
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(p), "i"(OFF) : "memory");
    return r;
}

// s_waitcnt lgkmcnt(0) that the compiler must order before every use of the four values.
__device__ __forceinline__ void wait_lgkm0(u32x2& a, u32x2& b, u32x2& c, u32x2& d)
{
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}

template <int HD, bool Q_F32, bool O_F32, bool EXT>
__global__ void __launch_bounds__(kPrefillThreads, prefill_waves_per_simd(HD))
prefill_kernel(PrefillArgs a)
{
    using L = PrefillLayout<HD>;
    constexpr int BM = kPrefillBM, BN = L::BN, SB = L::SB;
    constexpr int KSTEPS = HD / 16, DBLK = HD / 32;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    lds_u8* lds3 = (lds_u8*)lds;

    // the wave index is uniform across the wave: readfirstlane lets the compiler keep
    // per-wave bounds and branches scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, hh = lane >> 5;

    // ---- work item: (kv head, query block [heaviest first], q head in group, key split)
    const int item = xcd_remap(blockIdx.x, a.n_items);
    const int per_kv = a.group * a.n_qblocks * a.n_splits;
    const int kvh = item / per_kv;
    int r = item - kvh * per_kv;
    const int qb = a.n_qblocks - 1 - r / (a.group * a.n_splits);
    r %= a.group * a.n_splits;
    const int g = r / a.n_splits;
    const int split = r - g * a.n_splits;
    const int h = kvh * a.group + g;

    const int q0 = qb * BM;
    const int q_last_wg = min(q0 + BM, a.n_query) - 1;
    const int k_hi = min(a.q_base + q_last_wg, a.n_ctx - 1);
    int k_lo = 0;
    if (EXT && a.sliding_window > 0 && a.q_base + q0 + 1 > a.sliding_window)
        k_lo = a.q_base + q0 + 1 - a.sliding_window;
    const int tile_first = k_lo / BN;
    const int n_tiles = (k_hi >= k_lo) ? k_hi / BN - tile_first + 1 : 0;
    const int tps = (n_tiles + a.n_splits - 1) / a.n_splits;
    const int t_begin = tile_first + min(split * tps, n_tiles);
    const int t_end = tile_first + min((split + 1) * tps, n_tiles);

    // ---- this lane's query column and this wave's key bounds
    const int qrow = q0 + 32 * wave + n;
    const bool row_ok = qrow < a.n_query;
    const int qpos = a.q_base + qrow;
    const int w_first = q0 + 32 * wave;
    const bool wave_active = w_first < a.n_query;
    const int w_last = min(w_first + 31, a.n_query - 1);
    const int w_khi = min(a.q_base + w_last, a.n_ctx - 1);
    int w_klo = 0;
    if (EXT && a.sliding_window > 0 && a.q_base + w_first + 1 > a.sliding_window)
        w_klo = a.q_base + w_first + 1 - a.sliding_window;

    // ---- K/V tile staging: thread tid, load j fills LDS bytes 16 * (256 j + tid) of a tile
    const uint32_t kv_bytes = (uint32_t)a.n_ctx * HD * 2;
    const rsrc_t krs = make_rsrc_uniform(a.k + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    const rsrc_t vrs = make_rsrc_uniform(a.v + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    uint32_t koff[L::LOADS], voff[L::LOADS];              // byte offsets within a tile's rows
#pragma unroll
    for (int j = 0; j < L::LOADS; ++j) {
        const int b = 16 * (kPrefillThreads * j + tid);
        const int row = b / L::ROW, slot = (b % L::ROW) / 16;
        koff[j] = (uint32_t)(row * L::ROW + 16 * k_slot<HD>(row, slot));
        voff[j] = (uint32_t)(row * L::ROW + 16 * v_slot<HD>(row, slot));
    }
    auto issue_tile = [&](int t, int buf) {
        const uint32_t base = (uint32_t)(t * BN) * L::ROW;
        lds_u8* kl = lds3 + buf * L::BUF + 1024 * wave;
        lds_u8* vl = kl + L::TILE;
#pragma unroll
        for (int j = 0; j < L::LOADS; ++j) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (void __attribute__((address_space(3)))*)(kl + 4096 * j), 16,
                                                     (int)(base + koff[j]), 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (void __attribute__((address_space(3)))*)(vl + 4096 * j), 16,
                                                     (int)(base + voff[j]), 0, 0, 0);
        }
    };
    // ring prologue: tiles t_begin .. t_begin + STAGES - 2 in flight
#pragma unroll
    for (int st = 0; st + 1 < L::STAGES; ++st)
        if (t_begin + st < t_end) issue_tile(t_begin + st, st);

    // ---- Q^T operands, pre-scaled: lane (query n, k-group hh) holds dims 16*ks + 8*hh .. +7
    const float qscale = EXT ? a.scale : a.scale_log2;
    const float cap_c1 = a.softcap > 0.f ? 2.f * kLog2e / a.softcap : 0.f, cap_c2 = a.softcap * kLog2e;
    constexpr uint32_t QE = Q_F32 ? 4u : 2u;
    f16x8 qt[KSTEPS];
    {
        const size_t row_bytes = (size_t)a.n_q_heads * HD * QE;
        const int blk_rows = min(BM, a.n_query - q0);
        const rsrc_t qr = make_rsrc_uniform((const char*)a.q + (size_t)q0 * row_bytes, (uint32_t)(blk_rows * row_bytes));
        const uint32_t qoff = (uint32_t)((32 * wave + n) * row_bytes + ((size_t)h * HD + 8 * hh) * QE);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            float x[8];
            if constexpr (Q_F32) {
                const f32x4 x0 = __builtin_bit_cast(f32x4, buf_load16(qr, qoff + 64 * ks));
                const f32x4 x1 = __builtin_bit_cast(f32x4, buf_load16(qr, qoff + 64 * ks + 16));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[i] = x0[i];
                    x[4 + i] = x1[i];
                }
            } else {
                const f16x8 hq = as_f16x8(buf_load16(qr, qoff + 32 * ks));
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = (float)hq[i];
            }
            qt[ks] = cvt_f16x8(x[0] * qscale, x[1] * qscale, x[2] * qscale, x[3] * qscale, x[4] * qscale,
                               x[5] * qscale, x[6] * qscale, x[7] * qscale);
        }
    }

    // ---- per-lane LDS read offsets (bytes within a tile)
    // K A operand, block sb, k-step ks: row 32 sb + n, chunk 2 ks + hh
    int ka_off[KSTEPS];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) ka_off[ks] = n * L::ROW + 16 * k_slot<HD>(n, 2 * ks + hh);
    // V^T transposing reads: source lane i = lane & 15 of each 16-lane group addresses
    // V[kb + i/4][d0 + 4 (i%4)], kb = 32 sb + 16 j + 4 hh (+8 for the second half),
    // d0 = 32 db + 16 ((lane >> 4) & 1); the swizzle depends on the row only through
    // (4 hh + i/4) mod 4, which is the same for every (sb, j, half).
    int vt_off[DBLK];
    {
        const int i = lane & 15;
        const int rr = 4 * hh + (i >> 2);                 // row within a 16-key group (mod 16)
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
            const int dim = 32 * db + 16 * ((lane >> 4) & 1) + 4 * (i & 3);
            vt_off[db] = rr * L::ROW + 16 * v_slot<HD>(rr, dim >> 3) + 8 * ((dim >> 2) & 1);
        }
    }

    f32x16 o[DBLK];
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
    // running max m_used (log2 units of the pre-scaled score) and its negated splat, which
    // seeds every S^T accumulator; `seen` marks a row that has had a visible key
    float m_used = 0.f;
    bool seen = false;
    f32x16 negm;
#pragma unroll
    for (int v = 0; v < 16; ++v) negm[v] = 0.f;
    float l_part = 0.f;                                   // this lane's share of the row sum
    const f16x2 ones = {(_Float16)1.f, (_Float16)1.f};

    constexpr int LOADS_PER_TILE = 2 * L::LOADS;
    // s_waitcnt immediate for vmcnt(n) (expcnt and lgkmcnt left at their maxima)
    constexpr int kWaitLater = ((L::STAGES - 2) * LOADS_PER_TILE & 15) |
                               (((L::STAGES - 2) * LOADS_PER_TILE >> 4) << 14) | 0x0f70;
    static_assert((L::STAGES - 2) * LOADS_PER_TILE < 64, "vmcnt range");
    for (int t = t_begin; t < t_end; ++t) {
        const int buf = (t - t_begin) % L::STAGES;
        // this thread's tile-t loads have landed once at most the later tiles' loads remain
        if (t + L::STAGES - 2 < t_end) __builtin_amdgcn_s_waitcnt(kWaitLater);
        else __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();                                  // ... everyone's; the oldest buffer is free
        if (t + L::STAGES - 1 < t_end) issue_tile(t + L::STAGES - 1, (buf + L::STAGES - 1) % L::STAGES);
        const int key0 = t * BN;
        if (!(wave_active && key0 <= w_khi && key0 + BN - 1 >= w_klo)) continue;
        const lds_u8* kl = lds3 + buf * L::BUF;
        const lds_u8* vl = kl + L::TILE;

        // S^T = K Q^T (+ -m seed).  All K operands of the tile are read first, then the
        // MFMAs run with the independent accumulators interleaved; the scheduling barriers
        // keep the compiler from pairing every read with its MFMA (a serial chain of LDS
        // and MFMA latencies).
        f16x8 ka[SB][KSTEPS];
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
                ka[sb][ks] = *(const f16x8 __attribute__((address_space(3)))*)(kl + 32 * sb * L::ROW + ka_off[ks]);
        __builtin_amdgcn_sched_barrier(0);
        f32x16 s[SB];
#pragma unroll
        for (int sb = 0; sb < SB; ++sb) s[sb] = EXT ? f32x16{} : negm;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
            for (int sb = 0; sb < SB; ++sb) s[sb] = mfma32x32x16(ka[sb][ks], qt[ks], s[sb]);
        // V^T operands of the first 32-key block, read while the S MFMAs execute
        u32x2 vr[SB][DBLK][2][2];
        auto read_vt = [&](auto SBc) {
            constexpr int sb = decltype(SBc)::value;
#pragma unroll
            for (int db = 0; db < DBLK; ++db) {
                const lds_u8* vb = vl + vt_off[db];
                vr[sb][db][0][0] = ds_read_tr16_b64<(32 * sb + 0) * L::ROW>(vb);
                vr[sb][db][0][1] = ds_read_tr16_b64<(32 * sb + 8) * L::ROW>(vb);
                vr[sb][db][1][0] = ds_read_tr16_b64<(32 * sb + 16) * L::ROW>(vb);
                vr[sb][db][1][1] = ds_read_tr16_b64<(32 * sb + 24) * L::ROW>(vb);
            }
        };
        // wait for this block's reads; the "+v" operands order the wait before every use
        auto wait_vt = [&](auto SBc) {
            constexpr int sb = decltype(SBc)::value;
#pragma unroll
            for (int db = 0; db < DBLK; ++db)
                wait_lgkm0(vr[sb][db][0][0], vr[sb][db][0][1], vr[sb][db][1][0], vr[sb][db][1][1]);
        };
        read_vt(std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        // scores -> log2 domain relative to m_used, masked
        const bool need_mask = (key0 + BN - 1 > a.q_base + w_first) || (key0 + BN > a.n_ctx) ||
                               (EXT && a.sliding_window > 0 && key0 < a.q_base + w_last + 1 - a.sliding_window);
        if constexpr (EXT) {
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float x = s[sb][v];
                    s[sb][v] = (a.softcap > 0.f ? softcap_log2(x, cap_c1, cap_c2) : x * kLog2e) - m_used;
                }
        }
        if (need_mask) {                                  // wave-uniform: diagonal / boundary tiles
#pragma unroll
            for (int sb = 0; sb < SB; ++sb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = key0 + 32 * sb + 8 * (v >> 2) + 4 * hh + (v & 3);
                    bool vis = key <= qpos && key < a.n_ctx;
                    if (EXT && a.sliding_window > 0) vis = vis && key >= qpos + 1 - a.sliding_window;
                    s[sb][v] = vis ? s[sb][v] : -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int v = 0; v < 16; v += 2) mx = __builtin_fmaxf(mx, __builtin_fmaxf(s[sb][v], s[sb][v + 1]));
        mx = max_xor32(mx);
        // lazy rescale: a row moves its max when it first sees a key, or when its scores
        // exceed the current max by more than 2^8
        const bool need = seen ? (mx > kRescaleThresh) : (mx > -INFINITY);
        if (__any(need)) {
            const float d = need ? mx : 0.f;
            const float corr = fast_exp2(-d);
            m_used += d;
            seen = seen || need;
            l_part *= corr;
#pragma unroll
            for (int db = 0; db < DBLK; ++db) o[db] *= corr;
#pragma unroll
            for (int sb = 0; sb < SB; ++sb) s[sb] -= d;
#pragma unroll
            for (int v = 0; v < 16; ++v) negm[v] = -m_used;
        }
        // P = exp2(S), packed to f16 for the PV MFMA; row sums from the packed values
        f16x8 pb[SB][2];
#pragma unroll
        for (int sb = 0; sb < SB; ++sb)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float p[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) p[i] = fast_exp2(s[sb][8 * j + i]);
                const f16x8 ph = cvt_f16x8(p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);
                pb[sb][j] = ph;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f16x2 pp = {ph[2 * i], ph[2 * i + 1]};
                    l_part = __builtin_amdgcn_fdot2(pp, ones, l_part, false);
                }
            }
        // O^T += V^T P^T, the DBLK independent accumulators interleaved; the next block's V^T
        // operands are read while the current block's MFMAs execute
        auto pv = [&](auto SBc) {
            constexpr int sb = decltype(SBc)::value;
            wait_vt(SBc);
            if constexpr (sb + 1 < SB) read_vt(std::integral_constant<int, sb + 1>{});
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int db = 0; db < DBLK; ++db) {
                    const f16x8 va = __builtin_bit_cast(
                        f16x8, u32x4{vr[sb][db][j][0][0], vr[sb][db][j][0][1], vr[sb][db][j][1][0], vr[sb][db][j][1][1]});
                    o[db] = mfma32x32x16(va, pb[sb][j], o[db]);
                }
        };
        pv(std::integral_constant<int, 0>{});
        if constexpr (SB > 1) pv(std::integral_constant<int, 1>{});
    }

    // ---- epilogue: lane (query n, hh) holds dims 32*db + 8*a4 + 4*hh + (0..3)
    float l_tot = sum_xor32(l_part);
    auto store_out = [&](float inv) {
        const size_t obase = ((size_t)qrow * a.n_q_heads + h) * HD;
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const int dim = 32 * db + 8 * a4 + 4 * hh;
                const f32x4 gt = gate4(a.gate, obase + dim);
                const float v0 = o[db][4 * a4] * inv * gt[0], v1 = o[db][4 * a4 + 1] * inv * gt[1];
                const float v2 = o[db][4 * a4 + 2] * inv * gt[2], v3 = o[db][4 * a4 + 3] * inv * gt[3];
                if constexpr (O_F32) {
                    f32x4 x = {v0, v1, v2, v3};
                    *(f32x4*)((float*)a.out + obase + dim) = x;
                } else {
                    f32x2 p0 = {v0, v1}, p1 = {v2, v3};
                    f16x2 h0 = __builtin_convertvector(p0, f16x2);
                    f16x2 h1 = __builtin_convertvector(p1, f16x2);
                    u32x2 x = {__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
                    *(u32x2*)((uint16_t*)a.out + obase + dim) = x;
                }
            }
    };
    if (a.n_splits == 1) {
        if (row_ok) store_out(l_tot > 0.f ? 1.f / l_tot : 0.f);
        return;
    }

    // ---- split-KV: publish this split's partial; the combine kernel merges the splits
    const size_t prow = (size_t)qrow * a.n_q_heads + h;
    if (row_ok) {
        float* pr = a.part + (prow * a.n_splits + split) * (HD + 2);
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const int dim = 32 * db + 8 * a4 + 4 * hh;
                *(f32x2*)(pr + dim) = f32x2{o[db][4 * a4], o[db][4 * a4 + 1]};
                *(f32x2*)(pr + dim + 2) = f32x2{o[db][4 * a4 + 2], o[db][4 * a4 + 3]};
            }
        // m in natural-log units; a row with no visible key in this split carries the
        // reference's initial max and l = 0
        if (hh == 0) *(f32x2*)(pr + HD) = f32x2{seen ? m_used * kLn2 : kNegBig, l_tot};
    }
}

// ---- launchers

template <int HD, bool QF, bool OF, bool EXT>
static hipError_t launch_prefill_t(const PrefillArgs& a, hipStream_t stream)
{
    constexpr int lds_bytes = PrefillLayout<HD>::LDS_BYTES;
    static std::atomic<uint64_t> lds_set{0};          // devices whose LDS limit is raised
    const hipError_t e = ensure_dyn_lds((const void*)prefill_kernel<HD, QF, OF, EXT>, lds_bytes, lds_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((prefill_kernel<HD, QF, OF, EXT>), dim3(a.n_items), dim3(kPrefillThreads),
                       lds_bytes, stream, a);
    return hipGetLastError();
}

template <int HD>
static hipError_t launch_prefill_hd(const PrefillArgs& a, bool q_f32, bool o_f32, bool ext, hipStream_t s)
{
    if (ext) {
        if (q_f32) return o_f32 ? launch_prefill_t<HD, true, true, true>(a, s) : launch_prefill_t<HD, true, false, true>(a, s);
        return o_f32 ? launch_prefill_t<HD, false, true, true>(a, s) : launch_prefill_t<HD, false, false, true>(a, s);
    }
    if (q_f32) return o_f32 ? launch_prefill_t<HD, true, true, false>(a, s) : launch_prefill_t<HD, true, false, false>(a, s);
    return o_f32 ? launch_prefill_t<HD, false, true, false>(a, s) : launch_prefill_t<HD, false, false, false>(a, s);
}

hipError_t launch_prefill(const PrefillArgs& a, int head_dim, bool q_f32, bool o_f32, bool ext,
                          hipStream_t stream)
{
    // head dims 64, 128 and 256 run on the pipelined kernel (attn_prefill_wide.hip)
    switch (head_dim) {
    case 192: return launch_prefill_hd<192>(a, q_f32, o_f32, ext, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace nxa

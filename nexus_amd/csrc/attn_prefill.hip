// nexus_amd/csrc/attn_prefill.hip -- causal GQA flash-attention prefill for gfx950.
//
// Semantics follow Transformer::attn_batch_cpu (src/model/transformer.h:8653-8685) and
// attn_flash.comp (src/gpu/shaders/attn_flash.comp:66-72, 121-159): query i sits at
// absolute position q_base + i and sees keys [start, min(q_base + i, n_ctx - 1)].
//
// Design (one workgroup = 128 queries of one q head, 4 waves x 32 queries):
//  * S^T = K Q^T on v_mfma_f32_32x32x16_f16.  A = K tile rows (keys) straight from LDS,
//    B = Q^T held in registers for the whole key loop.  The D layout leaves each lane
//    with one query column and 16 keys of a 32-key block, so the row max needs one
//    cross-lane exchange (lane ^ 32) and P^T feeds the next MFMA without a shuffle.
//  * O^T += V^T P^T on the same MFMA: A = V^T read from LDS, B = P^T from registers.
//    V is transposed while it is staged into LDS (4 keys x 8 dims per thread, v_perm),
//    and the keys of every 16-key group are stored in the order [0-3, 8-11, 4-7, 12-15]
//    so that the 8 keys a lane contributes to P^T are one contiguous 16-byte LDS read.
//  * Online softmax in fp32 registers, exp2 with log2(e) folded into the scale, lazy
//    rescaling of O (only when a row max grows by more than 2^8).
//  * K/V tiles (64 keys) are double-buffered in LDS; the next tile's global loads are
//    issued before the current tile's MFMAs, one barrier per tile.
//  * Blocks are remapped so each XCD owns whole KV heads (L2 reuse of K/V), and within a
//    KV head the heaviest (latest) query blocks start first.
//  * K/V/Q come in through raw buffer loads whose descriptor ends at the cache end (or
//    the last query), so rows past it read as zero with no branch in the loop.
//  * Optional split of the key range over n_splits workgroups (short chunks over a long
//    cache, e.g. 512 queries after 4096 cached tokens).  Each split writes fp32 partials
//    (acc, m, l) in the reference's split-K format; the decode path's combine kernel merges
//    them with the LSE rule of qwen35_attn_comb.comp:16-40.
#include "attn_common.h"
#include "attn_kernels.h"

namespace nxa {

template <int HD>
struct PrefillLayout {
    static constexpr int BN = kPrefillBN;
    static constexpr int CPR = HD / 8;                        // 16-byte chunks per K row
    static constexpr int K_BYTES = BN * HD * 2;               // K tile, row-major, swizzled
    static constexpr int V_ROW = BN * 2;                      // V^T row (one dim, 64 keys)
    static constexpr int V_BYTES = HD * V_ROW;
    static constexpr int BUF_BYTES = K_BYTES + V_BYTES;
    static constexpr int LDS_BYTES = 2 * BUF_BYTES;
    // XOR mask that keeps a chunk inside its 8- or 16-chunk aligned group of the row
    static constexpr int K_SWZ = (CPR % 16 == 0) ? 15 : 7;
    static constexpr int K_LOADS = BN * CPR / kPrefillThreads;
    static constexpr int V_BLOCKS = 16 * CPR;                 // (4-key quad, 8-dim chunk)
    static constexpr int V_LOADS = (V_BLOCKS + kPrefillThreads - 1) / kPrefillThreads;
    static_assert(K_LOADS >= 1, "K staging");
};

// LDS byte offset of K tile row `key`, 16-byte chunk `c` (XOR swizzle against bank conflicts).
template <int HD>
__device__ __forceinline__ int k_off(int key, int c)
{
    using L = PrefillLayout<HD>;
    return key * (HD * 2) + 16 * (c ^ (key & L::K_SWZ));
}

// LDS byte offset of V^T row `d`, 16-byte chunk `c` (8 key slots).
__device__ __forceinline__ int vt_off(int d, int c)
{
    return d * (kPrefillBN * 2) + 16 * (c ^ ((d >> 1) & 7));
}

template <int HD, bool Q_F32, bool O_F32, bool EXT>
__global__ void __launch_bounds__(kPrefillThreads, HD <= 128 ? 2 : 1)
prefill_kernel(PrefillArgs a)
{
    using L = PrefillLayout<HD>;
    constexpr int BM = kPrefillBM, BN = kPrefillBN;
    constexpr int KSTEPS = HD / 16, DBLK = HD / 32;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

    // ---- Q^T operands: lane (query n, k-group hh) holds dims 16*ks + 8*hh .. +7
    constexpr uint32_t QE = Q_F32 ? 4u : 2u;
    f16x8 qt[KSTEPS];
    {
        const size_t row_bytes = (size_t)a.n_q_heads * HD * QE;
        const int blk_rows = min(BM, a.n_query - q0);
        const rsrc_t qr = make_rsrc((const char*)a.q + (size_t)q0 * row_bytes, (uint32_t)(blk_rows * row_bytes));
        const uint32_t qoff = (uint32_t)((32 * wave + n) * row_bytes + ((size_t)h * HD + 8 * hh) * QE);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            if constexpr (Q_F32) {
                const f32x4 x0 = __builtin_bit_cast(f32x4, buf_load16(qr, qoff + 64 * ks));
                const f32x4 x1 = __builtin_bit_cast(f32x4, buf_load16(qr, qoff + 64 * ks + 16));
                qt[ks] = cvt_f16x8(x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]);
            } else {
                qt[ks] = as_f16x8(buf_load16(qr, qoff + 32 * ks));
            }
        }
    }

    // K/V of this kv head; the descriptors end at row n_ctx
    const uint32_t kv_bytes = (uint32_t)a.n_ctx * HD * 2;
    const rsrc_t krs = make_rsrc(a.k + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    const rsrc_t vrs = make_rsrc(a.v + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    u32x4 kreg[L::K_LOADS];
    u32x4 vreg[L::V_LOADS][4];

    // global -> registers for tile t
    auto load_tile = [&](int t) {
        const uint32_t key0 = (uint32_t)(t * BN);
#pragma unroll
        for (int i = 0; i < L::K_LOADS; ++i) {
            const int idx = tid + kPrefillThreads * i;
            const int key = idx / L::CPR, c = idx % L::CPR;
            kreg[i] = buf_load16(krs, ((key0 + key) * HD + 8 * c) * 2);
        }
#pragma unroll
        for (int j = 0; j < L::V_LOADS; ++j) {
            const int blk = tid + kPrefillThreads * j;
            if (L::V_BLOCKS % kPrefillThreads == 0 || blk < L::V_BLOCKS) {
                const int kq = blk & 15, cc = blk >> 4;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    vreg[j][i] = buf_load16(vrs, ((key0 + 4 * kq + i) * HD + 8 * cc) * 2);
            }
        }
    };
    // registers -> LDS buffer `buf` (K as is, V transposed + key-permuted)
    auto store_tile = [&](int buf) {
        uint8_t* kl = lds + buf * L::BUF_BYTES;
        uint8_t* vl = kl + L::K_BYTES;
#pragma unroll
        for (int i = 0; i < L::K_LOADS; ++i) {
            const int idx = tid + kPrefillThreads * i;
            const int key = idx / L::CPR, c = idx % L::CPR;
            *(u32x4*)(kl + k_off<HD>(key, c)) = kreg[i];
        }
#pragma unroll
        for (int j = 0; j < L::V_LOADS; ++j) {
            const int blk = tid + kPrefillThreads * j;
            if (L::V_BLOCKS % kPrefillThreads == 0 || blk < L::V_BLOCKS) {
                const int kq = blk & 15, cc = blk >> 4;
                const int q4 = kq & 3;
                const int pos = ((q4 & 1) << 1) | (q4 >> 1);      // slot quad within the 16-key group
                const int c = 2 * (kq >> 2) + (pos >> 1);
                const int half = (pos & 1) * 8;
#pragma unroll
                for (int dd = 0; dd < 8; ++dd) {
                    const int d = 8 * cc + dd;
                    const int wj = dd >> 1;
                    const uint32_t sel = (dd & 1) ? kSelHi : kSelLo;
                    u32x2 val;
                    val[0] = perm_b32(vreg[j][1][wj], vreg[j][0][wj], sel);
                    val[1] = perm_b32(vreg[j][3][wj], vreg[j][2][wj], sel);
                    *(u32x2*)(vl + vt_off(d, c) + half) = val;
                }
            }
        }
    };

    f32x16 o[DBLK];
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
    float m_used = kNegBig;     // log2 units
    float l_part = 0.f;         // this lane's share of the row sum (its 16 keys per block)
    const float fc = EXT ? 1.f : a.scale_log2;

    if (t_begin < t_end) {
        load_tile(t_begin);
        store_tile(0);
    }
    __syncthreads();

    for (int t = t_begin; t < t_end; ++t) {
        const int buf = (t - t_begin) & 1;
        const bool has_next = t + 1 < t_end;
        if (has_next) load_tile(t + 1);
        const int key0 = t * BN;
        if (wave_active && key0 <= w_khi && key0 + BN - 1 >= w_klo) {
            const uint8_t* kl = lds + buf * L::BUF_BYTES;
            const uint8_t* vl = kl + L::K_BYTES;
            f32x16 s[2];
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
                for (int v = 0; v < 16; ++v) s[sb][v] = 0.f;
                const int kr = 32 * sb + n;
#pragma unroll
                for (int ks = 0; ks < KSTEPS; ++ks) {
                    const f16x8 ka = *(const f16x8*)(kl + k_off<HD>(kr, 2 * ks + hh));
                    s[sb] = mfma32x32x16(ka, qt[ks], s[sb]);
                }
            }
            const bool need_mask = (key0 + BN - 1 > a.q_base + w_first) || (key0 + BN > a.n_ctx) ||
                                   (EXT && a.sliding_window > 0 &&
                                    key0 < a.q_base + w_last + 1 - a.sliding_window);
            float mx = -INFINITY;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    float x = s[sb][v];
                    if constexpr (EXT) {
                        x *= a.scale;
                        if (a.softcap > 0.f) x = a.softcap * tanhf(x / a.softcap);
                        x *= kLog2e;
                    }
                    if (need_mask) {
                        const int key = key0 + 32 * sb + 8 * (v >> 2) + 4 * hh + (v & 3);
                        bool vis = key <= qpos && key < a.n_ctx;
                        if (EXT && a.sliding_window > 0) vis = vis && key >= qpos + 1 - a.sliding_window;
                        if (!vis) x = -INFINITY;
                    }
                    s[sb][v] = x;
                    mx = fmaxf(mx, x);
                }
            }
            mx = fmaxf(mx, xor32(mx));
            const float mt = mx * fc;
            const bool need = mt > m_used + kRescaleThresh;
            if (__any(need)) {
                const float m_new = need ? mt : m_used;
                const float corr = fast_exp2(m_used - m_new);
                l_part *= corr;
#pragma unroll
                for (int db = 0; db < DBLK; ++db)
#pragma unroll
                    for (int v = 0; v < 16; ++v) o[db][v] *= corr;
                m_used = m_new;
            }
            f16x8 pb[2][2];
            float lsum = 0.f;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                float p[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    p[v] = fast_exp2(fmaf(s[sb][v], fc, -m_used));
                    lsum += p[v];
                }
                pb[sb][0] = cvt_f16x8(p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);
                pb[sb][1] = cvt_f16x8(p[8], p[9], p[10], p[11], p[12], p[13], p[14], p[15]);
            }
            l_part += lsum;
#pragma unroll
            for (int db = 0; db < DBLK; ++db) {
                const int d = 32 * db + n;
#pragma unroll
                for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const f16x8 va = *(const f16x8*)(vl + vt_off(d, 2 * (2 * sb + j) + hh));
                        o[db] = mfma32x32x16(va, pb[sb][j], o[db]);
                    }
            }
        }
        if (has_next) store_tile(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: lane (query n, hh) holds dims 32*db + 8*a4 + 4*hh + (0..3)
    float l_tot = l_part + xor32(l_part);
    auto store_out = [&](float inv) {
        const size_t obase = ((size_t)qrow * a.n_q_heads + h) * HD;
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const int dim = 32 * db + 8 * a4 + 4 * hh;
                const float v0 = o[db][4 * a4] * inv, v1 = o[db][4 * a4 + 1] * inv;
                const float v2 = o[db][4 * a4 + 2] * inv, v3 = o[db][4 * a4 + 3] * inv;
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
        if (hh == 0) *(f32x2*)(pr + HD) = f32x2{m_used * kLn2, l_tot};   // m in natural-log units
    }
}

// ---- launchers

template <int HD, bool QF, bool OF, bool EXT>
static hipError_t launch_prefill_t(const PrefillArgs& a, hipStream_t stream)
{
    constexpr int lds_bytes = PrefillLayout<HD>::LDS_BYTES;
    static bool attr_done = false;        // set once per instantiation (benign race: idempotent)
    if (!attr_done) {
        hipError_t e = hipFuncSetAttribute((const void*)prefill_kernel<HD, QF, OF, EXT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
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
    switch (head_dim) {
    case 64: return launch_prefill_hd<64>(a, q_f32, o_f32, ext, stream);
    case 128: return launch_prefill_hd<128>(a, q_f32, o_f32, ext, stream);
    case 192: return launch_prefill_hd<192>(a, q_f32, o_f32, ext, stream);
    case 256: return launch_prefill_hd<256>(a, q_f32, o_f32, ext, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace nxa

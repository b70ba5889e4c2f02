// nexus_amd/csrc/attn_decode.hip -- split-KV ("flash decoding") attention for gfx950.
//
// Pass 1 of the reference's decode split-K (src/gpu/shaders/qwen35_attn_part.comp:1-108):
// one workgroup per (split, kv head, group of <= 32 query rows) writes, for every query
// row, acc[hd] = sum_k e^{s_k - m} v_k, m (the split's max score) and l = sum_k e^{s_k - m}
// to part[row][split][hd + 2] -- the reference's partial format.  The last workgroup of
// a (kv head, row group) to finish merges all splits with the LSE rule of pass 2
// (qwen35_attn_comb.comp:16-40, without the gate) and writes the output: one launch.
//
// Rows are (draft i, q head g of the GQA group) pairs, so every K/V byte a workgroup
// reads is shared by all G heads of the group and all drafts of a speculative verify
// (the reference's part kernel shares K/V rows across the G heads the same way).
//
// Per wave and 32-key step:
//  * K rows go straight from HBM into MFMA A-operand registers (16-byte loads,
//    lane = (key, half of a 16-dim slice)): no LDS round trip for K.
//  * S^T = K Q^T on v_mfma_f32_32x32x16_f16.  f32 queries are split into an f16 high
//    part and an f16 residual (two MFMAs), so scores carry ~22 mantissa bits like the
//    reference's f32 dot products.  Causal mask among drafts (key <= q_base + i).
//  * Exact online softmax (row max via one lane ^ 32 exchange), exp2 with log2(e) folded.
//  * V is staged into a wave-private LDS region transposed (v_perm) and key-permuted so
//    that P^T from the S^T registers feeds O^T += V^T P^T without shuffles.
//  * The 4 waves of a workgroup take interleaved 32-key steps of the split and merge
//    their (m, l, O) in LDS at the end.
#include "attn_common.h"
#include "attn_kernels.h"

namespace nxa {

template <int HD>
struct DecodeLayout {
    static constexpr int KEYS = kDecodeKeys;                  // 32 keys per wave step
    static constexpr int CPR = HD / 8;
    static constexpr int KSTEPS = HD / 16;
    static constexpr int DBLK = HD / 32;
    static constexpr int V_ROW = KEYS * 2;                    // bytes per V^T row
    static constexpr int V_WAVE = HD * V_ROW;                 // per-wave V^T region
    static constexpr int V_BLOCKS = (KEYS / 4) * CPR;         // (4-key quad, 8-dim chunk) per wave
    static constexpr int V_LOADS = V_BLOCKS / 64;
    static constexpr int MERGE_SLOT = (DBLK * 16 * 64 + 2 * 64) * 4;
    static constexpr int LDS_BYTES = (4 * V_WAVE > 2 * MERGE_SLOT) ? 4 * V_WAVE : 2 * MERGE_SLOT;
    static_assert(V_LOADS >= 1, "V staging");
};

__device__ __forceinline__ int dvt_off(int d, int c)
{
    // 64-byte V^T rows; XOR the chunk with (d >> 2) so 16 consecutive rows hit distinct banks.
    return d * (kDecodeKeys * 2) + 16 * (c ^ ((d >> 2) & 3));
}

template <int HD, bool Q_F32, bool O_F32, bool EXT>
__global__ void __launch_bounds__(kDecodeThreads, HD <= 128 ? 2 : 1)
decode_kernel(DecodeArgs a)
{
    using L = DecodeLayout<HD>;
    constexpr int KSTEPS = L::KSTEPS, DBLK = L::DBLK;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 31, hh = lane >> 5;
    const int split = blockIdx.x, kvh = blockIdx.y, rg = blockIdx.z;

    // ---- query row of this lane's column: R = draft * G + head-in-group
    const int R = rg * kDecodeRows + n;
    const bool row_ok = R < a.n_rows;
    const int qi = row_ok ? R / a.group : 0;
    const int h = kvh * a.group + (row_ok ? R - qi * a.group : 0);
    const int qpos = a.q_base + qi;
    int row_klo = 0;
    if (EXT && a.sliding_window > 0 && qpos + 1 > a.sliding_window) row_klo = qpos + 1 - a.sliding_window;
    const int row_khi = min(qpos, a.n_ctx - 1);

    // ---- Q^T operands (f16 high part + f16 residual for f32 queries)
    constexpr uint32_t QE = Q_F32 ? 4u : 2u;
    f16x8 qhi[KSTEPS];
    f16x8 qlo[Q_F32 ? KSTEPS : 1];
    {
        const rsrc_t qr = make_rsrc(a.q, (uint32_t)((size_t)a.n_query * a.n_q_heads * HD * QE));
        // rows past n_rows point past the descriptor and read as zero
        const uint32_t qoff = row_ok ? (uint32_t)((((size_t)qi * a.n_q_heads + h) * HD + 8 * hh) * QE) : 0x7fffff00u;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            if constexpr (Q_F32) {
                const f32x4 x0 = __builtin_bit_cast(f32x4, buf_load16(qr, qoff + 64 * ks));
                const f32x4 x1 = __builtin_bit_cast(f32x4, buf_load16(qr, qoff + 64 * ks + 16));
                const f16x8 hi = cvt_f16x8(x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]);
                qhi[ks] = hi;
                qlo[ks] = cvt_f16x8(x0[0] - (float)hi[0], x0[1] - (float)hi[1], x0[2] - (float)hi[2],
                                    x0[3] - (float)hi[3], x1[0] - (float)hi[4], x1[1] - (float)hi[5],
                                    x1[2] - (float)hi[6], x1[3] - (float)hi[7]);
            } else {
                qhi[ks] = as_f16x8(buf_load16(qr, qoff + 32 * ks));
            }
        }
    }

    const int s_begin = a.k_begin + split * a.chunk;
    const int s_end = min(s_begin + a.chunk, a.k_end);
    const int n_sub = s_begin < s_end ? (s_end - s_begin + L::KEYS - 1) / L::KEYS : 0;

    // K/V of this kv head; the descriptors end at this split's last key
    const uint32_t kv_bytes = (uint32_t)max(s_end, 0) * HD * 2;
    const rsrc_t krs = make_rsrc(a.k + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    const rsrc_t vrs = make_rsrc(a.v + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    uint8_t* vw = lds + wave * L::V_WAVE;
    const float fc = EXT ? 1.f : a.scale_log2;

    f32x16 o[DBLK];
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
    float m = kNegBig, l = 0.f;

    for (int j = wave; j < n_sub; j += 4) {
        const int key0 = s_begin + L::KEYS * j;
        // K rows -> A operands: lane (key n, k-group hh)
        f16x8 ka[KSTEPS];
        {
            const uint32_t koff = ((uint32_t)(key0 + n) * HD + 8 * hh) * 2;
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) ka[ks] = as_f16x8(buf_load16(krs, koff + 32 * ks));
        }
        // V rows -> registers: 4 consecutive keys x 8 dims per block
        u32x4 vr[L::V_LOADS][4];
#pragma unroll
        for (int i = 0; i < L::V_LOADS; ++i) {
            const int blk = lane + 64 * i;
            const int kq = blk & 7, cc = blk >> 3;
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                vr[i][r4] = buf_load16(vrs, ((uint32_t)(key0 + 4 * kq + r4) * HD + 8 * cc) * 2);
        }
        // S^T = K Q^T
        f32x16 s;
#pragma unroll
        for (int v = 0; v < 16; ++v) s[v] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            s = mfma32x32x16(ka[ks], qhi[ks], s);
            if constexpr (Q_F32) s = mfma32x32x16(ka[ks], qlo[ks], s);
        }
        // V^T -> LDS (keys of each 16-key group in slot order [0-3, 8-11, 4-7, 12-15])
#pragma unroll
        for (int i = 0; i < L::V_LOADS; ++i) {
            const int blk = lane + 64 * i;
            const int kq = blk & 7, cc = blk >> 3;
            const int q4 = kq & 3;
            const int pos = ((q4 & 1) << 1) | (q4 >> 1);
            const int c = 2 * (kq >> 2) + (pos >> 1);
            const int half = (pos & 1) * 8;
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) {
                const int d = 8 * cc + dd;
                const int wj = dd >> 1;
                const uint32_t sel = (dd & 1) ? kSelHi : kSelLo;
                u32x2 val;
                val[0] = perm_b32(vr[i][1][wj], vr[i][0][wj], sel);
                val[1] = perm_b32(vr[i][3][wj], vr[i][2][wj], sel);
                *(u32x2*)(vw + dvt_off(d, c) + half) = val;
            }
        }
        wave_lds_sync();
        // mask, softmax update
        float mx = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int key = key0 + 8 * (v >> 2) + 4 * hh + (v & 3);
            float x = s[v];
            if constexpr (EXT) {
                x *= a.scale;
                if (a.softcap > 0.f) x = a.softcap * tanhf(x / a.softcap);
                x *= kLog2e;
            }
            const bool vis = row_ok && key < s_end && key <= row_khi && key >= row_klo;
            if (!vis) x = -INFINITY;
            s[v] = x;
            mx = fmaxf(mx, x);
        }
        mx = fmaxf(mx, xor32(mx));
        const float m_new = fmaxf(m, mx * fc);
        const float corr = fast_exp2(m - m_new);
        float p[16];
        float lsum = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            p[v] = fast_exp2(fmaf(s[v], fc, -m_new));
            lsum += p[v];
        }
        l = l * corr + lsum;
        m = m_new;
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[db][v] *= corr;
        const f16x8 pb0 = cvt_f16x8(p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);
        const f16x8 pb1 = cvt_f16x8(p[8], p[9], p[10], p[11], p[12], p[13], p[14], p[15]);
        // O^T += V^T P^T
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
            const int d = 32 * db + n;
            const f16x8 va0 = *(const f16x8*)(vw + dvt_off(d, hh));
            const f16x8 va1 = *(const f16x8*)(vw + dvt_off(d, 2 + hh));
            o[db] = mfma32x32x16(va0, pb0, o[db]);
            o[db] = mfma32x32x16(va1, pb1, o[db]);
        }
        wave_lds_sync();
    }

    // ---- merge the 4 waves' (m, l, O) in LDS (log2 units)
    float l_tot = l + xor32(l);
    __syncthreads();                                       // V^T regions are reused below
    float* slot0 = (float*)lds;
    float* slot1 = (float*)(lds + L::MERGE_SLOT);
    auto put = [&](float* sl) {
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) sl[(db * 16 + v) * 64 + lane] = o[db][v];
        sl[DBLK * 16 * 64 + lane] = m;
        sl[DBLK * 16 * 64 + 64 + lane] = l_tot;
    };
    auto take = [&](const float* sl) {
        const float m2 = sl[DBLK * 16 * 64 + lane];
        const float l2 = sl[DBLK * 16 * 64 + 64 + lane];
        const float M = fmaxf(m, m2);
        const float c1 = fast_exp2(m - M), c2 = fast_exp2(m2 - M);
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[db][v] = o[db][v] * c1 + sl[(db * 16 + v) * 64 + lane] * c2;
        l_tot = l_tot * c1 + l2 * c2;
        m = M;
    };
    auto merge_waves = [&]() {                             // result in wave 0
        if (wave >= 2) put(wave == 2 ? slot0 : slot1);
        __syncthreads();
        if (wave < 2) take(wave == 0 ? slot0 : slot1);
        __syncthreads();
        if (wave == 1) put(slot0);
        __syncthreads();
        if (wave == 0) take(slot0);
    };
    auto store_out = [&]() {                               // wave 0: normalised output row
        const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
        const size_t obase = ((size_t)qi * a.n_q_heads + h) * HD;
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
    merge_waves();
    if (a.n_splits == 1) {
        if (wave == 0 && row_ok) store_out();
        return;
    }

    // ---- publish this split's partial; the last split to arrive merges all of them
    const size_t prow = (size_t)qi * a.n_q_heads + h;
    if (wave == 0 && row_ok) {
        float* pr = a.part + (prow * a.n_splits + split) * (HD + 2);
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const int dim = 32 * db + 8 * a4 + 4 * hh;
                f32x2 x0 = {o[db][4 * a4], o[db][4 * a4 + 1]};
                f32x2 x1 = {o[db][4 * a4 + 2], o[db][4 * a4 + 3]};
                *(f32x2*)(pr + dim) = x0;
                *(f32x2*)(pr + dim + 2) = x1;
            }
        if (hh == 0) {
            pr[HD] = m * kLn2;               // natural-log units, as qwen35_attn_part.comp stores m
            pr[HD + 1] = l_tot;
        }
    }
    release_agent();
    __shared__ int s_last;
    __syncthreads();
    if (!a.fused_merge) return;                            // a combine kernel follows
    unsigned int* cnt = a.counters + (size_t)kvh * gridDim.z + rg;
    if (tid == 0) s_last = arrive_is_last(cnt, (unsigned int)a.n_splits);
    __syncthreads();
    if (!s_last) return;
    acquire_agent();
    // wave w folds splits w, w + 4, ... of its rows, then the 4 waves merge in LDS
    m = kNegBig;
    l_tot = 0.f;
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
    if (row_ok) {
        for (int s2 = wave; s2 < a.n_splits; s2 += 4) {
            const float* pr = a.part + (prow * a.n_splits + s2) * (HD + 2);
            const float m2 = pr[HD] * kLog2e, l2 = pr[HD + 1];
            const float M = fmaxf(m, m2);
            const float c1 = fast_exp2(m - M), c2 = fast_exp2(m2 - M);
#pragma unroll
            for (int db = 0; db < DBLK; ++db)
#pragma unroll
                for (int a4 = 0; a4 < 4; ++a4) {
                    const int dim = 32 * db + 8 * a4 + 4 * hh;
                    const f32x2 x0 = *(const f32x2*)(pr + dim);
                    const f32x2 x1 = *(const f32x2*)(pr + dim + 2);
                    o[db][4 * a4] = o[db][4 * a4] * c1 + x0[0] * c2;
                    o[db][4 * a4 + 1] = o[db][4 * a4 + 1] * c1 + x0[1] * c2;
                    o[db][4 * a4 + 2] = o[db][4 * a4 + 2] * c1 + x1[0] * c2;
                    o[db][4 * a4 + 3] = o[db][4 * a4 + 3] * c1 + x1[1] * c2;
                }
            l_tot = l_tot * c1 + l2 * c2;
            m = M;
        }
    }
    __syncthreads();
    merge_waves();
    if (wave == 0 && row_ok) store_out();
    if (tid == 0) counter_reset(cnt);
}

// ---- LSE combine for large fan-in (qwen35_attn_comb.comp:16-40 without the gate):
// out[row][d] = sum_c acc_c[d] e^{m_c - M} / sum_c l_c e^{m_c - M}, zeros for a row that
// saw no key.  One wave per (row, 64-dim chunk); split weights are computed once per wave.
constexpr int kCombineThreads = 64;

template <int HD, bool O_F32>
__global__ void __launch_bounds__(kCombineThreads)
combine_kernel(CombineArgs a)
{
    __shared__ float wgt[kMaxSplits];
    const int row = blockIdx.x, lane = threadIdx.x;
    const int d = blockIdx.y * kCombineThreads + lane;
    const float* pr = a.part + (size_t)row * a.n_splits * (HD + 2);
    float mx = -3.0e38f;
    for (int c = lane; c < a.n_splits; c += kCombineThreads) mx = fmaxf(mx, pr[(size_t)c * (HD + 2) + HD]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float lsum = 0.f;
    for (int c = lane; c < a.n_splits; c += kCombineThreads) {
        const float w = fast_exp2((pr[(size_t)c * (HD + 2) + HD] - mx) * kLog2e);
        wgt[c] = w;
        lsum += w * pr[(size_t)c * (HD + 2) + HD + 1];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off);
    __syncthreads();
    if (d >= HD) return;
    float acc = 0.f;
    for (int c = 0; c < a.n_splits; ++c) acc += pr[(size_t)c * (HD + 2) + d] * wgt[c];
    const float y = lsum > 0.f ? acc / lsum : 0.f;
    if constexpr (O_F32) ((float*)a.out)[(size_t)row * HD + d] = y;
    else ((_Float16*)a.out)[(size_t)row * HD + d] = (_Float16)y;
}

template <int HD, bool OF>
static hipError_t launch_combine_t(const CombineArgs& a, hipStream_t stream)
{
    hipLaunchKernelGGL((combine_kernel<HD, OF>), dim3(a.n_rows, (HD + kCombineThreads - 1) / kCombineThreads),
                       dim3(kCombineThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs& a, int head_dim, bool o_f32, hipStream_t stream)
{
    if (a.n_splits < 1 || a.n_splits > kMaxSplits) return hipErrorInvalidValue;
    switch (head_dim) {
    case 64: return o_f32 ? launch_combine_t<64, true>(a, stream) : launch_combine_t<64, false>(a, stream);
    case 128: return o_f32 ? launch_combine_t<128, true>(a, stream) : launch_combine_t<128, false>(a, stream);
    case 192: return o_f32 ? launch_combine_t<192, true>(a, stream) : launch_combine_t<192, false>(a, stream);
    case 256: return o_f32 ? launch_combine_t<256, true>(a, stream) : launch_combine_t<256, false>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int HD, bool QF, bool OF, bool EXT>
static hipError_t launch_decode_t(const DecodeArgs& a, int n_rowgroups, hipStream_t stream)
{
    constexpr int lds_bytes = DecodeLayout<HD>::LDS_BYTES;
    static bool attr_done = false;        // set once per instantiation (idempotent)
    if (!attr_done) {
        hipError_t e = hipFuncSetAttribute((const void*)decode_kernel<HD, QF, OF, EXT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    hipLaunchKernelGGL((decode_kernel<HD, QF, OF, EXT>), dim3(a.n_splits, a.n_kv_heads, n_rowgroups),
                       dim3(kDecodeThreads), lds_bytes, stream, a);
    return hipGetLastError();
}

template <int HD, bool QF>
static hipError_t launch_decode_q(const DecodeArgs& a, bool o_f32, bool ext, int nrg, hipStream_t s)
{
    if (ext) return o_f32 ? launch_decode_t<HD, QF, true, true>(a, nrg, s) : launch_decode_t<HD, QF, false, true>(a, nrg, s);
    return o_f32 ? launch_decode_t<HD, QF, true, false>(a, nrg, s) : launch_decode_t<HD, QF, false, false>(a, nrg, s);
}

template <int HD>
static hipError_t launch_decode_hd(const DecodeArgs& a, bool q_f32, bool o_f32, bool ext, int nrg, hipStream_t s)
{
    return q_f32 ? launch_decode_q<HD, true>(a, o_f32, ext, nrg, s) : launch_decode_q<HD, false>(a, o_f32, ext, nrg, s);
}

hipError_t launch_decode(const DecodeArgs& a, int head_dim, bool q_f32, bool o_f32, bool ext,
                         int n_rowgroups, hipStream_t stream)
{
    switch (head_dim) {
    case 64: return launch_decode_hd<64>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 128: return launch_decode_hd<128>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 192: return launch_decode_hd<192>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 256: return launch_decode_hd<256>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace nxa

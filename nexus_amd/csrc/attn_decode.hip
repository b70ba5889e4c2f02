// nexus_amd/csrc/attn_decode.hip -- split-KV ("flash decoding") attention for gfx950.
//
// Two passes, as the reference's decode split-K (src/gpu/shaders/qwen35_attn_part.comp and
// qwen35_attn_comb.comp, dispatched back to back at src/gpu/vulkan_backend.h:5462-5482):
//  * decode_part_kernel: one workgroup per (split, kv head, row group) streams its slice of
//    the cache once and writes, for every query row, acc[hd] = sum_k e^{s_k - m} v_k,
//    m (the split's max scaled score) and l = sum_k e^{s_k - m} to
//    part[row][split][hd + 2] -- the reference's partial format (qwen35_attn_part.comp:3).
//    With one split it writes the normalised output directly.
//  * combine_kernel: out = sum_c acc_c e^{m_c - M} / sum_c l_c e^{m_c - M}, M = max_c m_c
//    (qwen35_attn_comb.comp:16-40, without the output gate).
// The kernel boundary makes the partials visible to the combine; an in-kernel
// "last workgroup merges" scheme needs an agent-scope release per workgroup, which
// writes back the XCD's L2 each time and measured slower than the second launch.
//
// Rows are (draft i, q head g of the GQA group) pairs, row = i * G + g, so every K/V byte a
// workgroup reads feeds all G heads of the group and all drafts of a speculative verify.
//
// Per wave and 32-key step (4 waves take interleaved steps of the split):
//  * K rows go from HBM straight into MFMA A-operand registers (non-temporal 16-byte
//    buffer loads, 64 contiguous bytes per key per instruction).  S^T = K Q^T on
//    v_mfma_f32_16x16x32_f16, 16 query rows per row tile (RT tiles per wave).  f32
//    queries are split into an f16 high part and an f16 residual (two MFMAs), so scores
//    carry ~22 mantissa bits like the reference's f32 dot products.
//  * The 32 keys of a step form two 16-key S^T tiles whose rows are the keys
//    8*(r/4) + 4*t + (r%4) (tile t, row r).  The D layout then leaves lane (row n, group g)
//    holding keys 8g..8g+7 of row n -- exactly the B operand of O^T += V^T P^T, so P
//    needs no shuffle.  Row max/sum: v_permlane16_swap + v_permlane32_swap on the VALU.
//  * V rows are transposed into a wave-private LDS region (v_perm, 8-byte writes) and read
//    back as V^T A operands (16 bytes = 8 keys of one dim).
//  * Software pipeline over register double buffers: K and V of step s + 2 are issued as
//    soon as step s has consumed its K and V registers, so two steps (32 KB at hd 128) stay
//    in flight per wave (one step from hd x rows > 128, with two waves per SIMD).  The Q^T
//    operands (f16 high/low parts) sit in LDS, one copy per workgroup, which keeps the
//    register budget at two waves per SIMD for hd 128.
//  * The waves merge their (m, l, O) through LDS before the partial is written: a tree at
//    four waves, and at eight a flat merge (all hand over at once, each wave then folds the
//    eight slots for its share of the dims and writes those dims).
#include "attn_common.h"
#include "attn_kernels.h"

namespace nxa {

// Register budget per (head_dim x row tiles): two waves per SIMD up to 256 (two steps of K/V
// in flight up to 128, one step above); one wave per SIMD beyond, which the host avoids for
// head dims above 128 by using one row tile and more row groups (at one wave per SIMD the
// compiler moves the accumulators through AGPRs on every step).
constexpr int decode_waves_per_simd(int hd, int rt) { return hd * rt <= 256 ? 2 : 1; }
constexpr int decode_depth(int hd, int rt) { return hd * rt <= 128 ? 2 : (hd * rt <= 256 ? 1 : (hd * rt <= 384 ? 2 : 1)); }

template <int HD, int RT>
struct DecodeLayout {
    static constexpr int NW = decode_waves(HD, RT);               // waves per workgroup
    static constexpr int KEYS = kDecodeKeys;                  // 32 keys per wave step
    static constexpr int KS = HD / 32;                        // 32-dim k-steps of S^T
    static constexpr int DT = HD / 16;                        // 16-dim tiles of O^T
    static constexpr int VB = (KEYS / 4) * (HD / 8) / 64;     // (4-key, 8-dim) V blocks per lane
    static constexpr int VT_WAVE = HD * KEYS * 2;             // V^T bytes per wave
    static constexpr int DEPTH = decode_depth(HD, RT);        // steps of K/V in flight
    static constexpr int Q_BYTES = RT * KS * 2 * 64 * 16;     // Q^T operands (hi, lo) per workgroup
    static constexpr int OREGS = RT * DT * 4;                 // f32 O^T values per lane
    static constexpr int MERGE_SLOT = (OREGS + 2 * RT) * 64 * 4;
    // merge: a tree through NW / 2 slots at four waves; at eight, every wave's slot at once
    // (one barrier, then each wave folds all eight for its share of the dims)
    static constexpr bool FLAT_MERGE = NW == 8;
    static constexpr int MERGE_BYTES = (FLAT_MERGE ? NW : NW / 2) * MERGE_SLOT;
    static constexpr int MAIN_BYTES = NW * VT_WAVE > MERGE_BYTES ? NW * VT_WAVE : MERGE_BYTES;
    static constexpr int LDS_BYTES = MAIN_BYTES + Q_BYTES;
    static_assert(VB >= 1 && (KEYS / 4) * (HD / 8) % 64 == 0, "V staging");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

// V^T byte offset: dim row d (64-byte rows of 32 keys), 8-key chunk c, 4-key half h.  The
// chunk is XOR-swizzled with bits 1-2 of the row, so the 16 rows an operand read touches
// (16*dt + 0..15, same chunk) fall on distinct banks within every 8 lanes.
__device__ __forceinline__ int vt_off(int d, int c, int h)
{
    return d * (kDecodeKeys * 2) + 16 * (c ^ ((d >> 1) & 3)) + 8 * h;
}

constexpr int kAuxNT = 2;   // buffer-load cache policy: non-temporal (streaming K/V)

__device__ __forceinline__ u32x4 buf_load16_nt(rsrc_t r, uint32_t byte_off)
{
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, kAuxNT));
}

template <int HD, int RT, bool Q_F32, bool O_F32, bool EXT>
__global__ void __launch_bounds__(64 * decode_waves(HD, RT), decode_waves_per_simd(HD, RT))
decode_part_kernel(DecodeArgs a)
{
    using L = DecodeLayout<HD, RT>;
    constexpr int NW = L::NW;
    constexpr int KS = L::KS, DT = L::DT, VB = L::VB;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    // the wave index is uniform across the wave: readfirstlane lets the compiler keep
    // per-wave bounds and branches scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, kvh = blockIdx.y, rg = blockIdx.z;

    // ---- query rows of this lane's columns: R = draft * G + head-in-group
    int R[RT], qi[RT], h[RT], khi[RT], klo[RT];
    bool rok[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        R[rt] = rg * (16 * RT) + 16 * rt + n;
        rok[rt] = R[rt] < a.n_rows;
        qi[rt] = rok[rt] ? R[rt] / a.group : 0;
        h[rt] = kvh * a.group + (rok[rt] ? R[rt] - qi[rt] * a.group : 0);
        const int qpos = a.q_base + qi[rt];
        khi[rt] = min(qpos, a.n_ctx - 1);
        klo[rt] = (EXT && a.sliding_window > 0 && qpos + 1 > a.sliding_window) ? qpos + 1 - a.sliding_window : 0;
    }

    // ---- Q^T B operands in LDS: lane (row n, group g) holds dims 32*ks + 8*g .. +7, as an
    // f16 high part and (f32 queries) the f16 residual.  Wave 0 issues the Q loads before
    // the K/V prologue and converts them once those loads are in flight, so the two
    // latencies overlap.
    constexpr uint32_t QE = Q_F32 ? 4u : 2u;
    constexpr int QV = Q_F32 ? 2 : 1;                           // 16-byte loads per operand
    uint8_t* qlds = lds + L::MAIN_BYTES;
    auto qslot = [&](int rt, int ks, int hl) { return qlds + (((rt * KS + ks) * 2 + hl) * 64 + lane) * 16; };
    u32x4 qraw[RT][KS][QV];
    if (wave == 0) {
        const rsrc_t qr = make_rsrc_uniform(a.q, (uint32_t)((size_t)a.n_query * a.n_q_heads * HD * QE));
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            // rows past n_rows point past the descriptor and read as zero
            const uint32_t qoff = rok[rt] ? (uint32_t)((((size_t)qi[rt] * a.n_q_heads + h[rt]) * HD + 8 * g) * QE)
                                          : 0x7fffff00u;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int j = 0; j < QV; ++j) qraw[rt][ks][j] = buf_load16(qr, qoff + 32 * QE * ks + 16 * j);
        }
    }
    auto store_q = [&]() {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if constexpr (Q_F32) {
                    const f32x4 x0 = __builtin_bit_cast(f32x4, qraw[rt][ks][0]);
                    const f32x4 x1 = __builtin_bit_cast(f32x4, qraw[rt][ks][QV - 1]);
                    const f16x8 hi = cvt_f16x8(x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]);
                    *(f16x8*)qslot(rt, ks, 0) = hi;
                    *(f16x8*)qslot(rt, ks, 1) =
                        cvt_f16x8(x0[0] - (float)hi[0], x0[1] - (float)hi[1], x0[2] - (float)hi[2],
                                  x0[3] - (float)hi[3], x1[0] - (float)hi[4], x1[1] - (float)hi[5],
                                  x1[2] - (float)hi[6], x1[3] - (float)hi[7]);
                } else {
                    *(f16x8*)qslot(rt, ks, 0) = as_f16x8(qraw[rt][ks][0]);
                }
            }
    };

    const int s_begin = a.k_begin + split * a.chunk;
    const int s_end = min(s_begin + a.chunk, a.k_end);
    const int n_sub = s_begin < s_end ? (s_end - s_begin + L::KEYS - 1) / L::KEYS : 0;
    const int n_my = n_sub > wave ? (n_sub - wave + NW - 1) / NW : 0;   // steps wave, wave+NW, ...

    // K/V of this kv head; the descriptors end at this split's last key
    const uint32_t kv_bytes = (uint32_t)max(s_end, 0) * HD * 2;
    const rsrc_t krs = make_rsrc_uniform(a.k + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    const rsrc_t vrs = make_rsrc_uniform(a.v + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    uint8_t* vw = lds + wave * L::VT_WAVE;
    const float fc = EXT ? 1.f : a.scale_log2;
    const float cap_c1 = a.softcap > 0.f ? 2.f * kLog2e / a.softcap : 0.f, cap_c2 = a.softcap * kLog2e;

    // per-lane K rows of the two 16-key tiles: tile t, row n -> key 8*(n/4) + 4t + n%4
    const uint32_t krow0 = 8 * (n >> 2) + (n & 3);
    // V^T write bases of this lane (block i adds 4096*i: its dim chunk is 8 further)
    int vt_wbase[4];
    {
        const int kq = lane & 7, cc0 = lane >> 3;
#pragma unroll
        for (int k2 = 0; k2 < 4; ++k2) vt_wbase[k2] = 512 * cc0 + 16 * ((kq >> 1) ^ k2) + 8 * (kq & 1);
    }

    constexpr int DEPTH = L::DEPTH;
    u32x4 kb[DEPTH][2 * KS];
    u32x4 vb[DEPTH][VB][4];
    auto key0_of = [&](int s) { return s_begin + L::KEYS * (wave + NW * s); };
    // K and V of step s into register buffer B (loads past the split read as zero)
    auto issue = [&](auto B, int s) {
        constexpr int b = DEPTH == 2 ? decltype(B)::value : 0;
        const uint32_t key0 = (uint32_t)key0_of(s);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                kb[b][t * KS + ks] = buf_load16_nt(krs, ((key0 + krow0 + 4 * t) * HD + 32 * ks + 8 * g) * 2);
#pragma unroll
        for (int i = 0; i < VB; ++i) {
            const int blk = lane + 64 * i;
            const int kq = blk & 7, cc = blk >> 3;
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                vb[b][i][r4] = buf_load16_nt(vrs, ((key0 + 4 * kq + r4) * HD + 8 * cc) * 2);
        }
    };

    f32x4 o[RT][DT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m[RT], l[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        m[rt] = kNegBig;
        l[rt] = 0.f;
    }

    // step s consumes register buffer B = s & 1 (buffer 0 at depth 1), then refills it with
    // step s + DEPTH
    auto step = [&](auto B, int s) {
        constexpr int b = DEPTH == 2 ? decltype(B)::value : 0;
        const int key0 = key0_of(s);
        // S^T = K Q^T for the two 16-key tiles
        f32x4 sc[2][RT];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) sc[t][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const f16x8 qh = *(const f16x8*)qslot(rt, ks, 0);
                f16x8 ql;
                if constexpr (Q_F32) ql = *(const f16x8*)qslot(rt, ks, 1);
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const f16x8 ka = as_f16x8(kb[b][t * KS + ks]);
                    sc[t][rt] = mfma16x16x32(ka, qh, sc[t][rt]);
                    if constexpr (Q_F32) sc[t][rt] = mfma16x16x32(ka, ql, sc[t][rt]);
                }
            }
        // V^T of this step -> LDS: block (key quad kq, dim chunk cc) becomes 8 rows of 4 keys.
        // Row 8*cc + dd, chunk kq/2 lands at vt_off = 512*cc + 64*dd + 16*((kq/2) ^ (dd/2)) +
        // 8*(kq%2): four lane-dependent bases (one per dd/2) plus immediates.
#pragma unroll
        for (int i = 0; i < VB; ++i) {
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) {
                const int wj = dd >> 1;
                const uint32_t sel = (dd & 1) ? kSelHi : kSelLo;
                u32x2 val;
                val[0] = perm_b32(vb[b][i][1][wj], vb[b][i][0][wj], sel);
                val[1] = perm_b32(vb[b][i][3][wj], vb[b][i][2][wj], sel);
                *(u32x2*)(vw + vt_wbase[dd >> 1] + 4096 * i + 64 * dd) = val;
            }
        }
        // both register halves of this step are consumed: refill them with step s + DEPTH.  The
        // loads are unconditional (steps past the split read as zero through the descriptor
        // and touch no memory), so every iteration issues the same loads in the same order
        // and the compiler's wait counts keep two steps in flight.
        __builtin_amdgcn_sched_barrier(0);
        issue(B, s + DEPTH);
        __builtin_amdgcn_sched_barrier(0);
        wave_lds_sync();
        // mask, online softmax (log2 units)
        f16x8 pb[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = key0 + 8 * g + 4 * t + i;
                    float x = sc[t][rt][i];
                    if constexpr (EXT) {
                        x *= a.scale;
                        x = a.softcap > 0.f ? softcap_log2(x, cap_c1, cap_c2) : x * kLog2e;
                    }
                    const bool vis = rok[rt] && key < s_end && key <= khi[rt] && key >= klo[rt];
                    x = vis ? x : -INFINITY;
                    sc[t][rt][i] = x;
                    mx = fmaxf(mx, x);
                }
            mx = max_xor32(max_xor16(mx));
            const float m_new = fmaxf(m[rt], mx * fc);
            if (__any(m_new != m[rt])) {
                const float corr = fast_exp2(m[rt] - m_new);
                l[rt] *= corr;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o[rt][dt] *= corr;
                m[rt] = m_new;
            }
            float p[8];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) p[4 * t + i] = fast_exp2(fmaf(sc[t][rt][i], fc, -m[rt]));
            l[rt] += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            pb[rt] = cvt_f16x8(p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);
        }
        // O^T += V^T P^T
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const f16x8 va = *(const f16x8*)(vw + vt_off(16 * dt + n, g, 0));
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) o[rt][dt] = mfma16x16x32(va, pb[rt], o[rt][dt]);
        }
        wave_lds_sync();
    };

    // Steps run in pairs (static buffer indices); an odd count gets one fully masked step.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // The prologue issues in the same order as the loop (K then V, step by step), so the
    // wait counts at the loop header stay those of the steady state.
    __builtin_amdgcn_sched_barrier(0);
    issue(I0{}, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DEPTH == 2) issue(I1{}, 1);
    __builtin_amdgcn_sched_barrier(0);
    if (wave == 0) store_q();
    __syncthreads();
    for (int s = 0; s < n_my; s += 2) {
        step(I0{}, s);
        step(I1{}, s + 1);
    }

    // ---- row sums across the four lanes of a row, then merge the NW waves in LDS (four
    // waves: a tree, the upper half handing its (O, m, l) to the lower half, log2 NW times;
    // eight: the flat merge below)
    float lt[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        lt[rt] = sum_xor32(sum_xor16(l[rt]));
    }
    __syncthreads();                                       // V^T regions are reused below
    auto put = [&](float* sl) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) sl[((rt * DT + dt) * 4 + i) * 64 + lane] = o[rt][dt][i];
            sl[(L::OREGS + 2 * rt) * 64 + lane] = m[rt];
            sl[(L::OREGS + 2 * rt + 1) * 64 + lane] = lt[rt];
        }
    };
    auto take = [&](const float* sl) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float m2 = sl[(L::OREGS + 2 * rt) * 64 + lane];
            const float l2 = sl[(L::OREGS + 2 * rt + 1) * 64 + lane];
            const float M = fmaxf(m[rt], m2);
            const float c1 = fast_exp2(m[rt] - M), c2 = fast_exp2(m2 - M);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[rt][dt][i] = o[rt][dt][i] * c1 + sl[((rt * DT + dt) * 4 + i) * 64 + lane] * c2;
            lt[rt] = lt[rt] * c1 + l2 * c2;
            m[rt] = M;
        }
    };
    if constexpr (L::FLAT_MERGE) {
        // every wave hands its (O, m, l) over at once; wave w then folds the eight slots for
        // the dim tiles dt = w, w + NW, ... (into o[rt][dt], with lt and m the merged row
        // values) and writes those dims
        put((float*)(lds + wave * L::MERGE_SLOT));
        __syncthreads();
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float ms[NW], M = -INFINITY;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                ms[w] = ((const float*)(lds + w * L::MERGE_SLOT))[(L::OREGS + 2 * rt) * 64 + lane];
                M = fmaxf(M, ms[w]);
            }
            float Lt = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float* sl = (const float*)(lds + w * L::MERGE_SLOT);
                ms[w] = fast_exp2(ms[w] - M);                // the slot's weight
                Lt += sl[(L::OREGS + 2 * rt + 1) * 64 + lane] * ms[w];
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                if (dt % NW != wave) continue;               // wave-uniform
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    const float* sl = (const float*)(lds + w * L::MERGE_SLOT);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] += sl[((rt * DT + dt) * 4 + i) * 64 + lane] * ms[w];
                }
                o[rt][dt] = acc;
            }
            lt[rt] = Lt;
            m[rt] = M;
        }
    } else {
#pragma unroll
        for (int half = NW / 2; half >= 1; half /= 2) {
            if (wave >= half && wave < 2 * half) put((float*)(lds + (wave - half) * L::MERGE_SLOT));
            __syncthreads();
            if (wave < half) take((const float*)(lds + wave * L::MERGE_SLOT));
            if (half > 1) __syncthreads();                 // slots are rewritten next level
        }
        if (wave != 0) return;
    }
    // dim tiles this wave writes: all (tree merge: wave 0), or dt = wave, wave + NW, ... (flat)
    auto mine = [&](int dt) { return !L::FLAT_MERGE || dt % NW == wave; };

    // ---- lane (row n, group g) holds dims 16*dt + 4*g + (0..3) of its rows
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        if (!rok[rt]) continue;
        const size_t prow = (size_t)qi[rt] * a.n_q_heads + h[rt];
        if (a.n_splits == 1) {
            const float inv = lt[rt] > 0.f ? 1.f / lt[rt] : 0.f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                if (!mine(dt)) continue;
                const int dim = 16 * dt + 4 * g;
                const f32x4 y = o[rt][dt] * inv * gate4(a.gate, prow * HD + dim);
                if constexpr (O_F32) {
                    *(f32x4*)((float*)a.out + prow * HD + dim) = y;
                } else {
                    f32x2 p0 = {y[0], y[1]}, p1 = {y[2], y[3]};
                    f16x2 h0 = __builtin_convertvector(p0, f16x2);
                    f16x2 h1 = __builtin_convertvector(p1, f16x2);
                    u32x2 x = {__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
                    *(u32x2*)((uint16_t*)a.out + prow * HD + dim) = x;
                }
            }
        } else {
            float* pr = a.part + (prow * a.n_splits + split) * (HD + 2);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                if (!mine(dt)) continue;
                const int dim = 16 * dt + 4 * g;
                *(f32x2*)(pr + dim) = f32x2{o[rt][dt][0], o[rt][dt][1]};
                *(f32x2*)(pr + dim + 2) = f32x2{o[rt][dt][2], o[rt][dt][3]};
            }
            if (g == 0 && wave == 0) *(f32x2*)(pr + HD) = f32x2{m[rt] * kLn2, lt[rt]};   // m in natural-log units
        }
    }
}

// ---- LSE combine (qwen35_attn_comb.comp:16-40 without the gate):
// out[row][d] = sum_c acc_c[d] e^{m_c - M} / sum_c l_c e^{m_c - M}, zeros for a row that
// saw no key.  One workgroup per row: thread (split group sg, dim pair dp) folds splits
// sg, sg + G, ... of dims 2dp, 2dp+1.  All of a thread's loads (its acc pairs and the
// (m, l) pair every lane of a wave shares) are independent, so a batch of 16 splits is one
// memory round trip; the G groups then merge through LDS.
template <int HD>
struct CombineLayout {
    static constexpr int DP = HD / 2;                          // dim pairs per row
    static constexpr int G = DP >= 256 ? 1 : 256 / DP;         // split groups
    static constexpr int THREADS = DP * G;
    static constexpr int BATCH = 16;                           // splits in flight per thread
};

template <int HD, bool O_F32>
__global__ void __launch_bounds__(CombineLayout<HD>::THREADS)
combine_kernel(CombineArgs a)
{
    using C = CombineLayout<HD>;
    __shared__ float sm_m[C::G], sm_l[C::G];
    __shared__ f32x2 sm_acc[C::G][C::DP];
    const int row = blockIdx.x;
    const int dp = threadIdx.x % C::DP, sg = threadIdx.x / C::DP;
    const float* pr = a.part + (size_t)row * a.n_splits * (HD + 2);

    float M = kNegBig * 4.f, L = 0.f;               // below any partial's m (kNegBig)
    f32x2 acc = {0.f, 0.f};
    for (int c0 = sg; c0 < a.n_splits; c0 += C::G * C::BATCH) {
        f32x2 x[C::BATCH], ml[C::BATCH];
#pragma unroll
        for (int j = 0; j < C::BATCH; ++j) {
            const int c = c0 + j * C::G;
            const bool ok = c < a.n_splits;
            const float* ps = pr + (size_t)(ok ? c : 0) * (HD + 2);
            x[j] = *(const f32x2*)(ps + 2 * dp);
            ml[j] = *(const f32x2*)(ps + HD);
            if (!ok) {
                x[j] = f32x2{0.f, 0.f};
                ml[j] = f32x2{kNegBig * 4.f, 0.f};
            }
        }
        float Mb = M;
#pragma unroll
        for (int j = 0; j < C::BATCH; ++j) Mb = fmaxf(Mb, ml[j][0]);
        const float cr = fast_exp2((M - Mb) * kLog2e);
        acc *= cr;
        L *= cr;
#pragma unroll
        for (int j = 0; j < C::BATCH; ++j) {
            const float w = fast_exp2((ml[j][0] - Mb) * kLog2e);
            acc += x[j] * w;
            L += ml[j][1] * w;
        }
        M = Mb;
    }
    if constexpr (C::G > 1) {
        if (dp == 0) {
            sm_m[sg] = M;
            sm_l[sg] = L;
        }
        sm_acc[sg][dp] = acc;
        __syncthreads();
        if (sg != 0) return;
        float Mt = sm_m[0];
#pragma unroll
        for (int j = 1; j < C::G; ++j) Mt = fmaxf(Mt, sm_m[j]);
        acc = f32x2{0.f, 0.f};
        L = 0.f;
#pragma unroll
        for (int j = 0; j < C::G; ++j) {
            const float w = fast_exp2((sm_m[j] - Mt) * kLog2e);
            acc += sm_acc[j][dp] * w;
            L += sm_l[j] * w;
        }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const f32x2 y = acc * inv * gate2(a.gate, (size_t)row * HD + 2 * dp);
    if constexpr (O_F32) {
        *(f32x2*)((float*)a.out + (size_t)row * HD + 2 * dp) = y;
    } else {
        const f16x2 hy = __builtin_convertvector(y, f16x2);
        *(f16x2*)((_Float16*)a.out + (size_t)row * HD + 2 * dp) = hy;
    }
}

// The same merge for many rows with few splits (split prefill): one wave per row, four rows
// per workgroup, lane l folding every split of dim pairs l, l + 64, ...; a batch of 8 splits
// is one memory round trip.  The one-workgroup-per-row kernel above spends its time on
// workgroup dispatch there (20480 rows x 2 splits: 37.8 us).
constexpr int kCombineRowsWaves = 4;

template <int HD, bool O_F32>
__global__ void __launch_bounds__(64 * kCombineRowsWaves)
combine_rows_kernel(CombineArgs a)
{
    constexpr int DP = HD / 2, PPL = (DP + 63) / 64, BATCH = 8;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kCombineRowsWaves + (int)(threadIdx.x >> 6);
    if (row >= a.n_rows) return;
    const float* pr = a.part + (size_t)row * a.n_splits * (HD + 2);

    float M = kNegBig * 4.f, L = 0.f;               // below any partial's m (kNegBig)
    f32x2 acc[PPL];
#pragma unroll
    for (int p = 0; p < PPL; ++p) acc[p] = f32x2{0.f, 0.f};
    for (int c0 = 0; c0 < a.n_splits; c0 += BATCH) {
        f32x2 x[BATCH][PPL], ml[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const int c = c0 + j;
            const bool ok = c < a.n_splits;
            const float* ps = pr + (size_t)(ok ? c : 0) * (HD + 2);
#pragma unroll
            for (int p = 0; p < PPL; ++p) {
                const int d = lane + 64 * p;
                x[j][p] = (ok && d < DP) ? *(const f32x2*)(ps + 2 * d) : f32x2{0.f, 0.f};
            }
            ml[j] = ok ? *(const f32x2*)(ps + HD) : f32x2{kNegBig * 4.f, 0.f};
        }
        float Mb = M;
#pragma unroll
        for (int j = 0; j < BATCH; ++j) Mb = fmaxf(Mb, ml[j][0]);
        const float cr = fast_exp2((M - Mb) * kLog2e);
        L *= cr;
#pragma unroll
        for (int p = 0; p < PPL; ++p) acc[p] *= cr;
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const float w = fast_exp2((ml[j][0] - Mb) * kLog2e);
            L += ml[j][1] * w;
#pragma unroll
            for (int p = 0; p < PPL; ++p) acc[p] += x[j][p] * w;
        }
        M = Mb;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
    for (int p = 0; p < PPL; ++p) {
        const int d = lane + 64 * p;
        if (d >= DP) continue;
        const f32x2 y = acc[p] * inv * gate2(a.gate, (size_t)row * HD + 2 * d);
        if constexpr (O_F32) {
            *(f32x2*)((float*)a.out + (size_t)row * HD + 2 * d) = y;
        } else {
            const f16x2 hy = __builtin_convertvector(y, f16x2);
            *(f16x2*)((_Float16*)a.out + (size_t)row * HD + 2 * d) = hy;
        }
    }
}

template <int HD, bool OF>
static hipError_t launch_combine_t(const CombineArgs& a, hipStream_t stream)
{
    if (combine_by_rows(a.n_rows, a.n_splits)) {
        const int wgs = (a.n_rows + kCombineRowsWaves - 1) / kCombineRowsWaves;
        hipLaunchKernelGGL((combine_rows_kernel<HD, OF>), dim3(wgs), dim3(64 * kCombineRowsWaves), 0, stream, a);
    } else {
        hipLaunchKernelGGL((combine_kernel<HD, OF>), dim3(a.n_rows), dim3(CombineLayout<HD>::THREADS), 0, stream, a);
    }
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

template <int HD, int RT, bool QF, bool OF, bool EXT>
static hipError_t launch_decode_t(const DecodeArgs& a, int n_rowgroups, hipStream_t stream)
{
    constexpr int lds_bytes = DecodeLayout<HD, RT>::LDS_BYTES;
    static std::atomic<uint64_t> lds_set{0};          // devices whose LDS limit is raised
    const hipError_t e = ensure_dyn_lds((const void*)decode_part_kernel<HD, RT, QF, OF, EXT>, lds_bytes, lds_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((decode_part_kernel<HD, RT, QF, OF, EXT>), dim3(a.n_splits, a.n_kv_heads, n_rowgroups),
                       dim3(64 * DecodeLayout<HD, RT>::NW), lds_bytes, stream, a);
    return hipGetLastError();
}

template <int HD, int RT>
static hipError_t launch_decode_rt(const DecodeArgs& a, bool q_f32, bool o_f32, bool ext, int nrg, hipStream_t s)
{
    if (ext) {
        if (q_f32) return o_f32 ? launch_decode_t<HD, RT, true, true, true>(a, nrg, s)
                                : launch_decode_t<HD, RT, true, false, true>(a, nrg, s);
        return o_f32 ? launch_decode_t<HD, RT, false, true, true>(a, nrg, s)
                     : launch_decode_t<HD, RT, false, false, true>(a, nrg, s);
    }
    if (q_f32) return o_f32 ? launch_decode_t<HD, RT, true, true, false>(a, nrg, s)
                            : launch_decode_t<HD, RT, true, false, false>(a, nrg, s);
    return o_f32 ? launch_decode_t<HD, RT, false, true, false>(a, nrg, s)
                 : launch_decode_t<HD, RT, false, false, false>(a, nrg, s);
}

template <int HD>
static hipError_t launch_decode_hd(const DecodeArgs& a, bool q_f32, bool o_f32, bool ext, int nrg, hipStream_t s)
{
    return a.row_tiles == 1 ? launch_decode_rt<HD, 1>(a, q_f32, o_f32, ext, nrg, s)
                            : launch_decode_rt<HD, 2>(a, q_f32, o_f32, ext, nrg, s);
}

hipError_t launch_decode(const DecodeArgs& a, int head_dim, bool q_f32, bool o_f32, bool ext,
                         int n_rowgroups, hipStream_t stream)
{
    if (a.row_tiles != 1 && a.row_tiles != 2) return hipErrorInvalidValue;
    switch (head_dim) {
    case 64: return launch_decode_hd<64>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 128: return launch_decode_hd<128>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 192: return launch_decode_hd<192>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 256: return launch_decode_hd<256>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace nxa

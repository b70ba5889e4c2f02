// nexus_amd/csrc/attn_decode.hip -- split-KV ("flash decoding") attention for gfx950.
//
// Two passes, as the reference's decode split-K (src/gpu/shaders/qwen35_attn_part.comp and
// qwen35_attn_comb.comp, dispatched back to back at src/gpu/vulkan_backend.h:5462-5482):
//  * decode_ring_kernel: one workgroup per (split, kv head, row group) streams its slice of
//    the cache once and writes, for every query row, acc[hd] = sum_k e^{s_k - m} v_k,
//    m (the split's max scaled score) and l = sum_k e^{s_k - m} -- the reference's partial
//    (qwen35_attn_part.comp:3), stored as acc [split][row][hd] and (m, l) [split][row].
//    With one split it writes the normalised output directly.
//  * combine_slices_kernel: out = sum_c acc_c e^{m_c - M} / sum_c l_c e^{m_c - M},
//    M = max_c m_c (qwen35_attn_comb.comp:16-40), output gate included.
//
// Rows are (draft i, q head g of the GQA group) pairs, row = i * G + g, so every K/V byte a
// workgroup reads feeds all G heads of the group and all drafts of a speculative verify (up
// to 32 rows per workgroup; more rows take more row groups).
//
// The ring kernel:
//  * K and V go HBM -> LDS with buffer-load-to-LDS into a ring of NSTAGE stages of 32 keys
//    (48-96 KB per workgroup): no register holds data in flight, so a workgroup keeps
//    NSTAGE - 1 stages (32-64 KB) of loads outstanding.  Every thread loads its share of each
//    stage; per stage: wait for the own loads (vmcnt), one s_barrier, refill the slot the
//    previous stage used, compute.  16-byte chunks are XOR-swizzled per row, each lane picking
//    the global chunk for its LDS slot, so both operand reads below are free of bank conflicts.
//  * Waves split the work, not the keys: wave w takes row tile w / DG (16 query rows) and the
//    dims [w % DG * HD / DG, ...) of the output, DG = 4 / row tiles.  The DG waves of a row tile
//    split the score reduction S^T = K Q^T over head dims (k-steps dg, dg + DG, ... of 32 dims
//    each, on v_mfma_f32_16x16x32_f16), exchange the partial scores through LDS and add them
//    in one fixed order, so all DG waves hold bit-identical scores, m and l; each then does
//    O^T += V^T P^T for its own dims.  The waves never merge (m, l, O) with each other: each
//    writes its own dims.  f32 queries are split into an f16 high part and an f16 residual
//    (two MFMAs), so scores carry ~22 mantissa bits like the reference's f32 dot products;
//    f16 queries are used as given.
//  * Rows past n_rows (a 16-row tile with fewer real rows) compute with zero queries and are
//    never written; masks apply only to stages that hold an invisible key for some row.
//  * The two 16-key S^T tiles of a stage hold the keys 8*(r/4) + 4*t + (r%4) (tile t, row r),
//    so the MFMA result leaves lane (query row n, group g) with keys 8g .. 8g+7 of row n --
//    exactly the B operand of O^T += V^T P^T: P needs no shuffle.  V^T operands come from LDS
//    with ds_read_b64_tr_b16 (two transposing reads = 8 keys of one dim).
#include <climits>

#include "attn_common.h"
#include "attn_kernels.h"

namespace nxa {

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8;

template <int HD>
struct RingLayout {
    static constexpr int ROW = HD * 2;                          // bytes per K/V row
    static constexpr int SK = kDecodeKeys;                      // keys per stage
    static constexpr int STAGE = SK * ROW;                      // bytes per stage per operand
    static constexpr int NL = STAGE / (kDecodeThreads * 16);    // 16-byte loads per thread per operand
    // ring depth: two or three stages in flight while one is computed (measured on MI355X: a
    // fourth stage at head dims 128 and 256 makes the calls 1-3% slower); 48-64 KB per workgroup
    // at two workgroups per CU (head dims <= 128), 96 KB at one per CU above
    static constexpr int NSTAGE = HD <= 64 ? 8 : (HD <= 128 ? 3 : (HD <= 192 ? 4 : 3));
    static constexpr int WG_PER_CU = decode_wg_per_cu(HD);
    static constexpr int VBASE = NSTAGE * STAGE;
    static constexpr int XBASE = 2 * NSTAGE * STAGE;            // partial scores: [wave][tile][lane] f32x4
    static constexpr int LDS_BYTES = XBASE + 4 * 2 * 64 * 16;
    static constexpr int KS = HD / 32;                          // 32-dim k-steps of S^T
    static constexpr int CPR = HD / 8;                          // 16-byte chunks per row
    static constexpr int KSWZ = CPR % 16 == 0 ? 15 : 7;         // K chunk swizzle mask
    static constexpr int LPS = 2 * NL;                          // loads per thread per stage
    static_assert(STAGE % (kDecodeThreads * 16) == 0 && NL >= 1, "stage staging");
    static_assert(LDS_BYTES * WG_PER_CU <= 160 * 1024, "LDS budget");
    static_assert((NSTAGE - 2) * LPS <= 63, "vmcnt range");
};

// Swizzled slot of K chunk c of row r: rows 8*(n/4) + 4t + (n%4) of a score tile (n = 0..15)
// get slot c ^ n, so the 16 lanes of an operand read hit 16 different 16-byte slots.
template <int HD>
__device__ __forceinline__ int rk_slot(int r, int c)
{
    return c ^ (((r & 3) | (((r >> 3) & 3) << 2)) & RingLayout<HD>::KSWZ);
}
// Swizzled slot of V chunk c of row r: the four rows of a transposing read (r % 4 = 0..3) land
// 32 bytes apart within one 128-byte span.
__device__ __forceinline__ int rv_slot(int r, int c) { return c ^ (2 * (r & 3)); }

constexpr int kAuxNT = 2;   // buffer-load cache policy: non-temporal (streaming K/V)

// LDS reads as inline asm: the compiler cannot tell the ring slots apart from the slots the
// buffer-load-to-LDS writes are filling, and would wait for all of them before a plain LDS
// load.  Each read is waited for explicitly (lgkm_wait); a wave's LDS operations complete in
// order.
__device__ __forceinline__ u32x4 lds_b128(const lds_u8* p)
{
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(p) : "memory");
    return r;
}
template <int OFF>
__device__ __forceinline__ u32x2 lds_tr16(const lds_u8* p)
{
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(p), "i"(OFF) : "memory");
    return r;
}
template <int N>
__device__ __forceinline__ void lgkm_wait(u32x4& a)
{
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "i"(N));
}
template <int N>
__device__ __forceinline__ void lgkm_wait(u32x2& a, u32x2& b)
{
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}
// Scalar LDS accesses of the fused prep prologue, as inline asm for the same reason (the ring's
// loads are in flight); waited for with lgkm_wait_all.
__device__ __forceinline__ void lds_st32(lds_u8* p, float v)
{
    asm volatile("ds_write_b32 %0, %1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_st16(lds_u8* p, uint32_t v)
{
    asm volatile("ds_write_b16 %0, %1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_st128(lds_u8* p, u32x4 v)
{
    asm volatile("ds_write_b128 %0, %1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ float lds_ld32(const lds_u8* p)
{
    float r;
    asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(p) : "memory");
    return r;
}
__device__ __forceinline__ void lgkm_wait_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// after lgkm_wait_all: the value is only used from here on
__device__ __forceinline__ void after_wait(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void after_wait(u32x4& x) { asm volatile("" : "+v"(x)); }

// s_waitcnt vmcnt(n) (expcnt and lgkmcnt left at their maxima)
template <int N>
__device__ __forceinline__ void vm_wait()
{
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

}  // namespace

template <int HD, int RT, bool Q_F32, bool O_F32, bool EXT, bool PREP>
__global__ void __launch_bounds__(kDecodeThreads, decode_wg_per_cu(HD))
decode_ring_kernel(DecodeArgs a)
{
    static_assert(!PREP || (Q_F32 && O_F32 && !EXT), "the fused prep runs with f32 q and out, no softcap or window");
    using L = RingLayout<HD>;
    constexpr int KS = L::KS, ROW = L::ROW, NSTAGE = L::NSTAGE;
    constexpr int DG = 4 / RT;                                  // dim groups per row tile
    constexpr int DTW = HD / DG / 16;                           // 16-dim output tiles per wave
    constexpr int KSW = (KS + DG - 1) / DG;                     // score k-steps per wave (at most)
    static_assert(DTW >= 1 && HD % (16 * DG) == 0, "dims per wave");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    lds_u8* lds3 = (lds_u8*)lds;

    // the wave index is uniform across the wave: readfirstlane keeps per-wave values scalar
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int rt = wave / DG, dg = wave % DG;
    const int split = blockIdx.x, kvh = blockIdx.y, rg = blockIdx.z;

    // ---- this lane's query row (as an MFMA column): R = draft * G + head-in-group.  A row
    // past n_rows computes with a zero query, is never written, and is not masked.
    const int R = rg * (16 * RT) + 16 * rt + n;
    const bool rok = R < a.n_rows;
    const int qi = rok ? R / a.group : 0;
    const int h = kvh * a.group + (rok ? R - qi * a.group : 0);
    const int qpos = a.q_base + qi;
    const int khi = rok ? min(qpos, a.n_ctx - 1) : INT_MAX;
    const int klo = (EXT && rok && a.sliding_window > 0 && qpos + 1 > a.sliding_window) ? qpos + 1 - a.sliding_window : 0;

    // ---- keys of this workgroup
    const int s_begin = a.k_begin + split * a.chunk;
    const int s_end = min(s_begin + a.chunk, a.k_end);
    const int n_st = s_begin < s_end ? (s_end - s_begin + L::SK - 1) / L::SK : 0;

    // ---- Q^T B operands of this wave's k-steps ks = dg + DG * i, loaded first: lane (row n,
    // group g) holds dims 32 ks + 8 g .. +7
    constexpr uint32_t QE = Q_F32 ? 4u : 2u;
    constexpr int QV = Q_F32 ? 2 : 1;
    u32x4 qraw[KSW][QV];
    // PREP: the raw inputs of the prep go out before the ring, so converting them waits for
    // them only.  Wave w prepares the q rows w, w + 4, ... of the workgroup (one head each,
    // lane l owning elements l, l + 64, ... as decode_prep_kernel); in the workgroups of the
    // split holding key pos, waves 0 and 1 also prepare the new K and V row.
    constexpr int PER = HD / 64;
    constexpr int PRW = PREP ? 4 * RT : 1;                      // q rows prepared per wave
    float xq[PRW][PER], wq[PER], wk[PER], rc[PER], rs[PER], xn[PER];
    const bool pos_wg = PREP && split == a.pos_split;           // workgroup-uniform
    const bool gated = PREP && (a.prep_flags & kPrepNoGate) == 0;
    const bool inter = (a.prep_flags & kPrepInterleaved) != 0;
    if constexpr (PREP) {
        const long long qstride = gated ? 2 * HD : HD;
#pragma unroll
        for (int i = 0; i < PRW; ++i) {
            const int r = rg * (16 * RT) + wave + 4 * i;      // n_query = 1: row = head in group
#pragma unroll
            for (int j = 0; j < PER; ++j)
                xq[i][j] = r < a.n_rows ? a.qg[(size_t)(kvh * a.group + r) * qstride + lane + 64 * j] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int d = lane + 64 * j;
            wq[j] = (a.prep_flags & kPrepNoQNorm) ? 0.f : a.qnw[d];
            const int ci = prep_rope_cos_index(d, a.rot, inter);
            rc[j] = d < a.rot ? a.tab[ci] : 0.f;
            rs[j] = d < a.rot ? a.tab[(a.rot >> 1) + ci] : 0.f;
            wk[j] = pos_wg && wave == 0 && !(a.prep_flags & kPrepNoKNorm) ? a.knw[d] : 0.f;
            xn[j] = pos_wg && wave < 2 ? (wave == 0 ? a.kraw : a.vraw)[(size_t)kvh * HD + d] : 0.f;
        }
    } else {
        const rsrc_t qr = make_rsrc_uniform(a.q, (uint32_t)((size_t)a.n_query * a.n_q_heads * HD * QE));
        // rows past n_rows point past the descriptor and read as zero
        const uint32_t qoff = rok ? (uint32_t)((((size_t)qi * a.n_q_heads + h) * HD + 8 * g) * QE) : 0x7fffff00u;
#pragma unroll
        for (int i = 0; i < KSW; ++i) {
            const int ks = dg + DG * i;                         // past KS: reads beyond the row, unused
#pragma unroll
            for (int j = 0; j < QV; ++j) qraw[i][j] = buf_load16(qr, qoff + 32 * QE * ks + 16 * j);
        }
    }

    // ---- ring loads: thread tid, load j fills bytes 4096 j + 16 tid of a stage's K (or V)
    // slot; the descriptors end at this split's last key, so later rows read as zero
    const uint32_t kv_bytes = (uint32_t)max(s_end, 0) * ROW;
    const rsrc_t krs = make_rsrc_uniform(a.k + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    const rsrc_t vrs = make_rsrc_uniform(a.v + (size_t)kvh * (size_t)a.kv_stride * HD, kv_bytes);
    int koff[L::NL], voff[L::NL];
#pragma unroll
    for (int j = 0; j < L::NL; ++j) {
        const int b = 4096 * j + 16 * tid;
        const int row = b / ROW, slot = (b % ROW) / 16;
        koff[j] = row * ROW + 16 * rk_slot<HD>(row, slot);
        voff[j] = row * ROW + 16 * rv_slot(row, slot);
    }
    // stage st into ring slot st % NSTAGE.  Stages past the split are issued too (they read
    // zeros and touch no memory): every thread issues the same loads in the same order, so a
    // fixed vmcnt tells when a stage has landed.
    auto issue = [&](int st) {
        const int sl = st % NSTAGE;
        const int key0 = s_begin + L::SK * st;
        lds_u8* kd = lds3 + sl * L::STAGE + 1024 * wave;
        lds_u8* vd = lds3 + L::VBASE + sl * L::STAGE + 1024 * wave;
#pragma unroll
        for (int j = 0; j < L::NL; ++j) {
            const int go = key0 * ROW + koff[j];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (void __attribute__((address_space(3)))*)(kd + 4096 * j), 16,
                                                     go, 0, 0, kAuxNT);
        }
#pragma unroll
        for (int j = 0; j < L::NL; ++j) {
            const int go = key0 * ROW + voff[j];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (void __attribute__((address_space(3)))*)(vd + 4096 * j), 16,
                                                     go, 0, 0, kAuxNT);
        }
    };
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < NSTAGE - 1; ++st) issue(st);
    __builtin_amdgcn_sched_barrier(0);

    // ---- Q conversion (waits for the Q loads only: they were issued before the ring)
    vm_wait<(NSTAGE - 1) * L::LPS>();
    u32x4 kvchunk = {0u, 0u, 0u, 0u};    // PREP: wave 0 lane t holds 16 bytes of the new K|V row
    if constexpr (PREP) {
        // q rows go to the free ring slot NSTAGE - 1 (f32, rows 0-15 in its K half, 16-31 in its
        // V half, 16-byte chunks XOR-swizzled by row); per-wave scratch for the RoPE partners
        // and the new f16 K|V row go to the score-exchange area, unused until the first stage
        auto qrow = [&](int r) {
            return lds3 + (r < 16 ? 0 : L::VBASE) + (NSTAGE - 1) * L::STAGE + (r & 15) * (HD * 4);
        };
        auto qaddr = [&](int r, int d) { return qrow(r) + 16 * ((d >> 2) ^ (r & 15)) + 4 * (d & 3); };
        lds_u8* scratch = lds3 + L::XBASE + wave * (HD * 4);
        lds_u8* newrow = lds3 + L::XBASE + 4 * (HD * 4);       // [K | V] f16
        // head norm (optional) and RoPE of one row held as x[j] = element lane + 64 j
        auto prep_head = [&](float (&x)[PER], bool norm, bool add_one, const float (&w)[PER]) {
            if (norm) {
                float ss = 0.f;
#pragma unroll
                for (int j = 0; j < PER; ++j) ss += x[j] * x[j];
                const float inv = prep_norm_inv(prep_wave_sum(ss), HD, a.eps);
#pragma unroll
                for (int j = 0; j < PER; ++j) x[j] = prep_norm_apply(x[j], inv, w[j], add_one);
            }
            if (a.rot > 0) {
                float pr[PER];
                if (!prep_rope_partners(x, pr, lane, a.rot, inter)) {      // other rotations: via LDS
#pragma unroll
                    for (int j = 0; j < PER; ++j)
                        if (lane + 64 * j < a.rot) lds_st32(scratch + 4 * (lane + 64 * j), x[j]);
                    lgkm_wait_all();
#pragma unroll
                    for (int j = 0; j < PER; ++j) {
                        const int d = lane + 64 * j;
                        pr[j] = lds_ld32(scratch + 4 * (d < a.rot ? prep_rope_partner(d, a.rot, inter) : 0));
                    }
                    lgkm_wait_all();
#pragma unroll
                    for (int j = 0; j < PER; ++j) after_wait(pr[j]);
                }
#pragma unroll
                for (int j = 0; j < PER; ++j) {
                    const int d = lane + 64 * j;
                    if (d < a.rot) x[j] = prep_rope(d, x[j], pr[j], rc[j], rs[j], a.rot, inter);
                }
            }
        };
        const bool qnorm = (a.prep_flags & kPrepNoQNorm) == 0, qzc = (a.prep_flags & kPrepQZeroCentred) != 0;
#pragma unroll
        for (int i = 0; i < PRW; ++i) {
            const int r = wave + 4 * i;
            if (rg * (16 * RT) + r >= a.n_rows) continue;      // wave-uniform
            prep_head(xq[i], qnorm, qzc, wq);
#pragma unroll
            for (int j = 0; j < PER; ++j) lds_st32(qaddr(r, lane + 64 * j), xq[i][j]);
        }
        if (pos_wg && wave < 2) {
            // the new row: K normed and rotated, V as given, in the cache's f16 conversion (its
            // global stores wait for the end of the kernel: issued here, they would hold up this
            // workgroup's first wait on its ring loads)
            if (wave == 0) prep_head(xn, (a.prep_flags & kPrepNoKNorm) == 0, (a.prep_flags & kPrepKZeroCentred) != 0, wk);
            const bool trunc = (a.prep_flags & kPrepTruncStore) != 0;
#pragma unroll
            for (int j = 0; j < PER; ++j)
                lds_st16(newrow + 2 * (wave * HD + lane + 64 * j), trunc ? f16_trunc_bits(xn[j]) : f16_rne_bits(xn[j]));
        }
        lgkm_wait_all();
        __builtin_amdgcn_s_barrier();
        // Q^T operands from the prepared rows (rows past n_rows compute with zeros)
        const int rl = 16 * rt + n;
#pragma unroll
        for (int i = 0; i < KSW; ++i) {
            const int ks = dg + DG * i;
            if (ks < KS) {                                      // wave-uniform
                qraw[i][0] = lds_b128(qaddr(rl, 32 * ks + 8 * g));
                qraw[i][1] = lds_b128(qaddr(rl, 32 * ks + 8 * g + 4));
            }
        }
        if (pos_wg && wave == 0 && lane < 2 * L::CPR) kvchunk = lds_b128(newrow + 16 * lane);
        lgkm_wait_all();
#pragma unroll
        for (int i = 0; i < KSW; ++i) {
            after_wait(qraw[i][0]);
            after_wait(qraw[i][1]);
            if (!rok || dg + DG * i >= KS) qraw[i][0] = qraw[i][1] = u32x4{0u, 0u, 0u, 0u};
        }
        after_wait(kvchunk);
    }
    f16x8 qh[KSW], ql[KSW];
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
        if constexpr (Q_F32) {
            const f32x4 x0 = __builtin_bit_cast(f32x4, qraw[i][0]);
            const f32x4 x1 = __builtin_bit_cast(f32x4, qraw[i][QV - 1]);
            qh[i] = cvt_f16x8(x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]);
            ql[i] = cvt_f16x8(x0[0] - (float)qh[i][0], x0[1] - (float)qh[i][1], x0[2] - (float)qh[i][2],
                              x0[3] - (float)qh[i][3], x1[0] - (float)qh[i][4], x1[1] - (float)qh[i][5],
                              x1[2] - (float)qh[i][6], x1[3] - (float)qh[i][7]);
        } else {
            qh[i] = as_f16x8(qraw[i][0]);
        }
    }

    // ---- per-lane LDS read offsets within a stage slot
    // K operand of score tile t, k-step ks: row 8*(n/4) + 4t + n%4, chunk 4 ks + g
    int ka_off[KSW][2];
#pragma unroll
    for (int i = 0; i < KSW; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t)
            ka_off[i][t] = (8 * (n >> 2) + 4 * t + (n & 3)) * ROW + 16 * rk_slot<HD>(8 * (n >> 2) + (n & 3),
                                                                                      4 * (dg + DG * i) + g);
    // V^T of output tile dt: lane i = n of 16-lane group g addresses row 8g + i/4 (and 4 rows
    // on), dims 16 dt + 4 (i%4) .. +3; the read hands lane n the keys of dim 16 dt + n
    int vt_off[DTW];
    {
        const int vr = 8 * g + (n >> 2);
#pragma unroll
        for (int w = 0; w < DTW; ++w) {
            const int dt = dg * DTW + w;
            vt_off[w] = L::VBASE + vr * ROW + 16 * rv_slot(vr, 2 * dt + ((n & 3) >> 1)) + 8 * (n & 1);
        }
    }
    // partial scores: this wave's slot, and those of its row tile's DG waves in order
    lds_u8* xw = lds3 + L::XBASE + (wave * 2 * 64 + lane) * 16;
    const lds_u8* xr = lds3 + L::XBASE + (rt * DG * 2 * 64 + lane) * 16;

    f32x4 o[DTW];
#pragma unroll
    for (int w = 0; w < DTW; ++w) o[w] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = kNegBig, l = 0.f;
    const float fc = EXT ? 1.f : a.scale_log2;
    const float cap_c1 = a.softcap > 0.f ? 2.f * kLog2e / a.softcap : 0.f, cap_c2 = a.softcap * kLog2e;
    constexpr int VR = DTW < 4 ? DTW : 4;                       // V^T tiles read ahead of the PV MFMAs

    for (int s = 0; s < n_st; ++s) {
        // stage s has landed in every thread's share once each thread's own loads have
        // (NSTAGE - 2 later stages may still be in flight) and every wave passed the barrier
        vm_wait<(NSTAGE - 2) * L::LPS>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // every wave has finished stage s - 1: its slot takes stage s + NSTAGE - 1
        issue(s + NSTAGE - 1);
        __builtin_amdgcn_sched_barrier(0);
        const lds_u8* kb = lds3 + (s % NSTAGE) * L::STAGE;
        const int key0 = s_begin + L::SK * s;
        if (PREP && pos_wg && a.q_base - key0 < L::SK) {        // workgroup-uniform: the stage of key pos
            // the ring loaded row pos from the cache before this launch wrote it: replace it with
            // the row prepared above (chunk c of K or V to the slot the ring loads put it in)
            if (wave == 0 && lane < 2 * L::CPR) {
                const int pr = a.q_base - key0, c = lane % L::CPR;
                lds_u8* dst = lane < L::CPR ? lds3 + (s % NSTAGE) * L::STAGE + pr * ROW + 16 * rk_slot<HD>(pr, c)
                                            : lds3 + L::VBASE + (s % NSTAGE) * L::STAGE + pr * ROW + 16 * rv_slot(pr, c);
                lds_st128(dst, kvchunk);
            }
            lgkm_wait_all();
            __builtin_amdgcn_s_barrier();
        }

        // this wave's share of S^T = K Q^T for the two 16-key tiles: k-steps dg, dg + DG, ...
        // (high and residual parts of f32 queries in separate accumulators: four chains)
        f32x4 sh[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
        f32x4 sl2[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
        u32x4 kr[KSW][2];
        static_for<0, KSW>([&](auto I) {
            constexpr int i = decltype(I)::value;
            if (dg + DG * i < KS) {                             // wave-uniform
                kr[i][0] = lds_b128(kb + ka_off[i][0]);
                kr[i][1] = lds_b128(kb + ka_off[i][1]);
            }
        });
        static_for<0, KSW>([&](auto I) {
            constexpr int i = decltype(I)::value;
            if (dg + DG * i < KS) {
                lgkm_wait<0>(kr[i][0]);
                lgkm_wait<0>(kr[i][1]);
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const f16x8 ka = as_f16x8(kr[i][t]);
                    sh[t] = mfma16x16x32(ka, qh[i], sh[t]);
                    if constexpr (Q_F32) sl2[t] = mfma16x16x32(ka, ql[i], sl2[t]);
                }
            }
        });
        f32x4 sp[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) sp[t] = Q_F32 ? sh[t] + sl2[t] : sh[t];
        // hand the partial over, then read the row tile's partials once every wave wrote its own
        *(__attribute__((address_space(3))) f32x4*)(xw) = sp[0];
        *(__attribute__((address_space(3))) f32x4*)(xw + 1024) = sp[1];
        // V^T operand reads of this wave's dims (they land during the exchange and softmax)
        const lds_u8* vb = lds3 + (s % NSTAGE) * L::STAGE;
        u32x2 va[VR][2];
        static_for<0, VR>([&](auto W) {
            constexpr int w = decltype(W)::value;
            va[w][0] = lds_tr16<0>(vb + vt_off[w]);
            va[w][1] = lds_tr16<4 * ROW>(vb + vt_off[w]);
        });
        asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(2 * VR) : "memory");   // own partial written
        __builtin_amdgcn_s_barrier();
        // every partial of the row tile (the wave's own one too: all DG waves then add the same
        // values in the same order, d = 0, 1, ..., and hold bit-identical scores)
        u32x4 xp[DG][2];
#pragma unroll
        for (int d = 0; d < DG; ++d)
#pragma unroll
            for (int t = 0; t < 2; ++t) xp[d][t] = lds_b128(xr + (d * 2 + t) * 1024);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        f32x4 sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            asm volatile("" : "+v"(xp[0][t]));                  // the wait above precedes every use
            sc[t] = __builtin_bit_cast(f32x4, xp[0][t]);
#pragma unroll
            for (int d = 1; d < DG; ++d) {
                asm volatile("" : "+v"(xp[d][t]));
                sc[t] += __builtin_bit_cast(f32x4, xp[d][t]);
            }
        }

        // mask (only stages with a key some row must not see), online softmax (log2 units)
        const bool full = __all(key0 + L::SK - 1 <= khi && key0 >= klo) && key0 + L::SK <= s_end;
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = sc[t][i];
                if constexpr (EXT) {
                    x *= a.scale;
                    x = a.softcap > 0.f ? softcap_log2(x, cap_c1, cap_c2) : x * kLog2e;
                }
                if (!full) {
                    const int key = key0 + 8 * g + 4 * t + i;
                    x = (key < s_end && key <= khi && key >= klo) ? x : -INFINITY;
                }
                sc[t][i] = x;
                mx = fmaxf(mx, x);
            }
        mx = max_xor32(max_xor16(mx));
        const float m_new = fmaxf(m, mx * fc);
        if (__any(m_new != m)) {
            const float corr = fast_exp2(m - m_new);
            l *= corr;
#pragma unroll
            for (int w = 0; w < DTW; ++w) o[w] *= corr;
            m = m_new;
        }
        float p[8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) p[4 * t + i] = fast_exp2(fmaf(sc[t][i], fc, -m));
        l += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
        const f16x8 pb = cvt_f16x8(p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);

        // O^T += V^T P^T for this wave's dims, VR tiles read ahead
        static_for<0, DTW>([&](auto W) {
            constexpr int w = decltype(W)::value;
            constexpr int left = DTW - 1 - w < VR - 1 ? DTW - 1 - w : VR - 1;   // reads issued after w
            lgkm_wait<2 * left>(va[w % VR][0], va[w % VR][1]);
            const u32x4 vv = {va[w % VR][0][0], va[w % VR][0][1], va[w % VR][1][0], va[w % VR][1][1]};
            o[w] = mfma16x16x32(as_f16x8(vv), pb, o[w]);
            if constexpr (w + VR < DTW) {
                va[w % VR][0] = lds_tr16<0>(vb + vt_off[w + VR]);
                va[w % VR][1] = lds_tr16<4 * ROW>(vb + vt_off[w + VR]);
            }
        });
    }
    // stages issued past the split are still landing in LDS: drain them before the
    // workgroup's LDS can be handed to another workgroup
    vm_wait<0>();
    if (PREP && pos_wg && wave < 2 && rg == 0) {       // one row group stores the new row
        const bool trunc = (a.prep_flags & kPrepTruncStore) != 0;
        uint16_t* dst = (wave == 0 ? a.kc : a.vc) + ((size_t)kvh * a.kv_stride + a.q_base) * HD;
        float* echo = a.kv_out + ((size_t)wave * a.n_kv_heads + kvh) * HD;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int d = lane + 64 * j;
            dst[d] = trunc ? f16_trunc_bits(xn[j]) : f16_rne_bits(xn[j]);
            echo[d] = xn[j];
        }
    }

    // ---- row sums across the four lanes of a row; lane (row n, group g) holds dims
    // 16 dt + 4 g + (0..3) of row n
    const float lt = sum_xor32(sum_xor16(l));
    if (!rok) return;
    const size_t prow = (size_t)qi * a.n_q_heads + h;
    if (a.n_splits == 1) {
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
        for (int w = 0; w < DTW; ++w) {
            const int dim = 16 * (dg * DTW + w) + 4 * g;
            const f32x4 y = o[w] * inv * gate4(a.gate, prow * a.gate_stride + dim);
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
        // 16-byte stores; the rows of this workgroup's split are contiguous in the workspace.
        // With two row tiles (32 rows, up to 32 KB of partials per workgroup at hd 256) they
        // are non-temporal: measured on MI355X, 4-draft verify at 32k keys, hd 256: 22.3 ->
        // 21.5 us; with one row tile (a few KB per workgroup) plain stores are faster (decode
        // at 61k keys, hd 128: 44.6 vs 45.4 us; hd-256 decode layer 18.7 vs 19.1 us).
        const long long n_all = (long long)a.n_query * a.n_q_heads;
        float* pr = a.part + part_acc(split, (long long)prow, n_all, HD);
#pragma unroll
        for (int w = 0; w < DTW; ++w) {
            f32x4* dst = (f32x4*)(pr + 16 * (dg * DTW + w) + 4 * g);
            if constexpr (RT == 2) __builtin_nontemporal_store(o[w], dst);
            else *dst = o[w];
        }
        if (g == 0 && dg == 0)                                              // m in natural-log units
            *(f32x2*)(a.part + part_ml(split, (long long)prow, n_all, a.n_splits, HD)) = f32x2{m * kLn2, lt};
    }
}

// ---- LSE combine (qwen35_attn_comb.comp:16-40, with the output gate of :34-38):
// out[row][d] = sum_c acc_c[d] e^{m_c - M} / sum_c l_c e^{m_c - M}, zeros for a row that
// saw no key.  One workgroup per (row, 64 dims): thread (split group sg, dim quad dq) folds
// splits sg, sg + 16, ... of dims 4 dq .. 4 dq + 3 of the slice, eight splits per memory
// round trip (one round trip up to 128 splits); the 16 split groups merge through LDS.  The
// partials are read once, with non-temporal loads (measured on MI355X: 4-draft verify at 32k
// keys, hd 256, 21.5 -> 19.9 us per call; one-token decodes unchanged or slightly faster).
constexpr int kCombineSliceDims = 64;
constexpr int kCombineSplitGroups = 16;

template <int HD, bool O_F32>
__global__ void __launch_bounds__(256)
combine_slices_kernel(CombineArgs a)
{
    constexpr int SG = kCombineSplitGroups, BATCH = 8;
    __shared__ float sm_m[SG][16], sm_l[SG][16];
    __shared__ f32x4 sm_acc[SG][16];
    const int row = blockIdx.x;
    const int dq = threadIdx.x & 15, sg = threadIdx.x >> 4;
    const int dim = kCombineSliceDims * blockIdx.y + 4 * dq;

    float M = kNegBig * 4.f, L = 0.f;               // below any partial's m (kNegBig)
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = sg; c0 < a.n_splits; c0 += SG * BATCH) {
        f32x4 x[BATCH];
        f32x2 ml[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const int c = c0 + j * SG;
            const bool ok = c < a.n_splits;
            const int cs = ok ? c : 0;
            x[j] = __builtin_nontemporal_load((const f32x4*)(a.part + part_acc(cs, row, a.n_rows, HD) + dim));
            ml[j] = *(const f32x2*)(a.part + part_ml(cs, row, a.n_rows, a.n_splits, HD));
            if (!ok) ml[j] = f32x2{kNegBig * 4.f, 0.f};
        }
        float Mb = M;
#pragma unroll
        for (int j = 0; j < BATCH; ++j) Mb = fmaxf(Mb, ml[j][0]);
        const float cr = fast_exp2((M - Mb) * kLog2e);
        acc *= cr;
        L *= cr;
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const float w = c0 + j * SG < a.n_splits ? fast_exp2((ml[j][0] - Mb) * kLog2e) : 0.f;
            acc += x[j] * w;
            L += ml[j][1] * w;
        }
        M = Mb;
    }
    sm_m[sg][dq] = M;
    sm_l[sg][dq] = L;
    sm_acc[sg][dq] = acc;
    __syncthreads();
    if (sg != 0) return;
    float Mt = sm_m[0][dq];
#pragma unroll
    for (int j = 1; j < SG; ++j) Mt = fmaxf(Mt, sm_m[j][dq]);
    acc = f32x4{0.f, 0.f, 0.f, 0.f};
    L = 0.f;
#pragma unroll
    for (int j = 0; j < SG; ++j) {
        const float w = fast_exp2((sm_m[j][dq] - Mt) * kLog2e);
        acc += sm_acc[j][dq] * w;
        L += sm_l[j][dq] * w;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const f32x4 y = acc * inv * gate4(a.gate, (size_t)row * a.gate_stride + dim);
    if constexpr (O_F32) {
        *(f32x4*)((float*)a.out + (size_t)row * HD + dim) = y;
    } else {
        f32x2 p0 = {y[0], y[1]}, p1 = {y[2], y[3]};
        f16x2 h0 = __builtin_convertvector(p0, f16x2);
        f16x2 h1 = __builtin_convertvector(p1, f16x2);
        *(u32x2*)((uint16_t*)a.out + (size_t)row * HD + dim) =
            u32x2{__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
    }
}

// The same merge for many rows with few splits (split prefill): one wave per row, four rows
// per workgroup, lane l folding every split of dim pairs l, l + 64, ...; a batch of 8 splits
// is one memory round trip.
constexpr int kCombineRowsWaves = 4;

template <int HD, bool O_F32>
__global__ void __launch_bounds__(64 * kCombineRowsWaves)
combine_rows_kernel(CombineArgs a)
{
    constexpr int DP = HD / 2, PPL = (DP + 63) / 64, BATCH = 8;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kCombineRowsWaves + (int)(threadIdx.x >> 6);
    if (row >= a.n_rows) return;

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
            const float* ps = a.part + part_acc(ok ? c : 0, row, a.n_rows, HD);
#pragma unroll
            for (int p = 0; p < PPL; ++p) {
                const int d = lane + 64 * p;
                x[j][p] = (ok && d < DP) ? *(const f32x2*)(ps + 2 * d) : f32x2{0.f, 0.f};
            }
            ml[j] = ok ? *(const f32x2*)(a.part + part_ml(c, row, a.n_rows, a.n_splits, HD)) : f32x2{kNegBig * 4.f, 0.f};
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
        const f32x2 y = acc[p] * inv * gate2(a.gate, (size_t)row * a.gate_stride + 2 * d);
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
        static_assert(HD % kCombineSliceDims == 0, "combine slices");
        hipLaunchKernelGGL((combine_slices_kernel<HD, OF>), dim3(a.n_rows, HD / kCombineSliceDims), dim3(256), 0,
                           stream, a);
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

template <int HD, int RT, bool QF, bool OF, bool EXT, bool PREP = false>
static hipError_t launch_decode_t(const DecodeArgs& a, int n_rowgroups, hipStream_t stream)
{
    constexpr int lds_bytes = RingLayout<HD>::LDS_BYTES;
    static std::atomic<uint64_t> lds_set{0};          // devices whose LDS limit is raised
    const hipError_t e =
        ensure_dyn_lds((const void*)decode_ring_kernel<HD, RT, QF, OF, EXT, PREP>, lds_bytes, lds_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((decode_ring_kernel<HD, RT, QF, OF, EXT, PREP>), dim3(a.n_splits, a.n_kv_heads, n_rowgroups),
                       dim3(kDecodeThreads), lds_bytes, stream, a);
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

template <int HD>
static hipError_t launch_decode_layer_hd(const DecodeArgs& a, int nrg, hipStream_t s)
{
    return a.row_tiles == 1 ? launch_decode_t<HD, 1, true, true, false, true>(a, nrg, s)
                            : launch_decode_t<HD, 2, true, true, false, true>(a, nrg, s);
}

hipError_t launch_decode_layer(const DecodeArgs& a, int head_dim, int n_rowgroups, hipStream_t stream)
{
    if (a.row_tiles != 1 && a.row_tiles != 2) return hipErrorInvalidValue;
    if (a.chunk % kDecodeKeys != 0 || a.chunk <= 0 || a.n_query != 1) return hipErrorInvalidValue;
    switch (head_dim) {
    case 64: return launch_decode_layer_hd<64>(a, n_rowgroups, stream);
    case 128: return launch_decode_layer_hd<128>(a, n_rowgroups, stream);
    case 192: return launch_decode_layer_hd<192>(a, n_rowgroups, stream);
    case 256: return launch_decode_layer_hd<256>(a, n_rowgroups, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_decode(const DecodeArgs& a, int head_dim, bool q_f32, bool o_f32, bool ext,
                         int n_rowgroups, hipStream_t stream)
{
    if (a.row_tiles != 1 && a.row_tiles != 2) return hipErrorInvalidValue;
    if (a.chunk % kDecodeKeys != 0 || a.chunk <= 0) return hipErrorInvalidValue;
    switch (head_dim) {
    case 64: return launch_decode_hd<64>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 128: return launch_decode_hd<128>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 192: return launch_decode_hd<192>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    case 256: return launch_decode_hd<256>(a, q_f32, o_f32, ext, n_rowgroups, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace nxa

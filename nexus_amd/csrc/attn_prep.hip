// Decode prep for one token: per-head RMSNorm of q and k, RoPE over the first `rot` dims
// from a host cos/sin table, the f16 store of K and V into the device cache row `pos`, and
// an f32 echo of the stored K/V for the host cache.
//
// Follows qwen35_attn_prep.comp:1-101 (flag bits, buffer layouts, workgroup -> head map):
//   workgroups [0, n_heads) are q heads, [n_heads, n_heads + n_kv) k heads, then v heads.
// The norm and RoPE follow the host code (prep_norm_apply / prep_rope in attn_common.h), so
// the f32 results agree with the CPU path to rounding.
//
// MI355X shape: the whole op moves a few hundred KB, so it is launch-latency bound; one
// 64-lane wave per head keeps every reduction inside the wave (DPP and permlane steps on the
// VALU, no LDS) and lets all heads run at once on separate CUs; RoPE partners come from
// registers for the usual rotations and through LDS (one barrier) for the others.  Lane l owns
// elements l, l + 64, ... (coalesced 256-byte rows).
#include "attn_common.h"
#include "attn_kernels.h"

namespace nxa {

namespace {

constexpr int kPrepPer = kPrepMaxHeadDim / 64;

__global__ __launch_bounds__(64) void decode_prep_kernel(PrepArgs a)
{
    __shared__ float row[kPrepMaxHeadDim];
    const int g = blockIdx.x, lane = threadIdx.x, hd = a.hd;
    const bool isq = g < a.n_heads;
    const bool isk = !isq && g < a.n_heads + a.n_kv;
    const int head = isq ? g : (isk ? g - a.n_heads : g - a.n_heads - a.n_kv);
    const bool gated = (a.flags & kPrepNoGate) == 0;

    const float* src = isq ? a.qg + (size_t)head * (gated ? 2 : 1) * hd
                           : (isk ? a.kraw : a.vraw) + (size_t)head * hd;
    float x[kPrepPer];
#pragma unroll
    for (int j = 0; j < kPrepPer; ++j) {
        const int d = lane + 64 * j;
        x[j] = d < hd ? src[d] : 0.f;
    }
    if (isq && gated) {
#pragma unroll
        for (int j = 0; j < kPrepPer; ++j) {
            const int d = lane + 64 * j;
            if (d < hd) a.gate_out[(size_t)head * hd + d] = src[hd + d];
        }
    }

    if (isq || isk) {
        const bool norm = (a.flags & (isq ? kPrepNoQNorm : kPrepNoKNorm)) == 0;
        if (norm) {                                       // uniform over the workgroup
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < kPrepPer; ++j) ss += x[j] * x[j];
            const float inv = prep_norm_inv(prep_wave_sum(ss), hd, a.eps);
            const bool zc = (a.flags & (isq ? kPrepQZeroCentred : kPrepKZeroCentred)) != 0;
            const float* w = isq ? a.qnw : a.knw;
#pragma unroll
            for (int j = 0; j < kPrepPer; ++j) {
                const int d = lane + 64 * j;
                if (d < hd) x[j] = prep_norm_apply(x[j], inv, w[d], zc);
            }
        }
        const int rot = a.rot;
        if (rot > 0) {
            const bool inter = (a.flags & kPrepInterleaved) != 0;
            float pr[kPrepPer];
            if (!prep_rope_partners(x, pr, lane, rot, inter)) {   // other rotations: via LDS
#pragma unroll
                for (int j = 0; j < kPrepPer; ++j) {
                    const int d = lane + 64 * j;
                    if (d < rot) row[d] = x[j];
                }
                __syncthreads();
#pragma unroll
                for (int j = 0; j < kPrepPer; ++j) {
                    const int d = lane + 64 * j;
                    pr[j] = d < rot ? row[prep_rope_partner(d, rot, inter)] : 0.f;
                }
            }
#pragma unroll
            for (int j = 0; j < kPrepPer; ++j) {
                const int d = lane + 64 * j;
                if (d >= rot) continue;
                const int ci = prep_rope_cos_index(d, rot, inter);
                x[j] = prep_rope(d, x[j], pr[j], a.tab[ci], a.tab[(rot >> 1) + ci], rot, inter);
            }
        }
    }

    if (isq) {
#pragma unroll
        for (int j = 0; j < kPrepPer; ++j) {
            const int d = lane + 64 * j;
            if (d < hd) a.q_out[(size_t)head * hd + d] = x[j];
        }
        return;
    }
    uint16_t* dst = (isk ? a.kc : a.vc) + ((size_t)head * a.cap + a.pos) * hd;
    float* echo = a.kv_out + (isk ? 0 : (size_t)a.n_kv * hd) + (size_t)head * hd;
    const bool trunc = (a.flags & kPrepTruncStore) != 0;
#pragma unroll
    for (int j = 0; j < kPrepPer; ++j) {
        const int d = lane + 64 * j;
        if (d < hd) {
            dst[d] = trunc ? f16_trunc_bits(x[j]) : f16_rne_bits(x[j]);
            echo[d] = x[j];
        }
    }
}

}  // namespace

hipError_t launch_decode_prep(const PrepArgs& a, hipStream_t stream)
{
    hipLaunchKernelGGL(decode_prep_kernel, dim3(a.n_heads + 2 * a.n_kv), dim3(64), 0, stream, a);
    return hipGetLastError();
}

}  // namespace nxa

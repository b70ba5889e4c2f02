// Decode prep for one token: per-head RMSNorm of q and k, RoPE over the first `rot` dims
// from a host cos/sin table, the f16 store of K and V into the device cache row `pos`, and
// an f32 echo of the stored K/V for the host cache.
//
// Follows qwen35_attn_prep.comp:1-101 (flag bits, buffer layouts, workgroup -> head map):
//   workgroups [0, n_heads) are q heads, [n_heads, n_heads + n_kv) k heads, then v heads.
// The norm is written as the host does it, so the f32 results agree with the CPU path to
// rounding: cpu::rms_norm (src/cpu/matmul.h:1860-1880) computes (x * w) * inv,
// nx_rms_norm_add_one (src/model/transformer.h:504-520) computes x * inv * (1 + w), with
// inv = 1 / sqrt(mean(x^2) + eps).  RoPE pairs are (i, i + rot/2) (rotate_half) or
// (2i, 2i + 1) (interleaved), the two layouts of rope_apply (src/model/attention.h:593-608),
// with cos at tab[i] and sin at tab[rot/2 + i].
//
// MI355X shape: the whole op moves a few hundred KB, so it is launch-latency bound; one
// 64-lane wave per head keeps every reduction inside the wave (no LDS tree, no barriers
// beyond the one before the RoPE partner reads) and lets all heads run at once on
// separate CUs.  Lane l owns elements l, l + 64, ... (coalesced 256-byte rows).
#include "attn_common.h"
#include "attn_kernels.h"

namespace nxa {

namespace {

constexpr int kPrepPer = kPrepMaxHeadDim / 64;

__device__ __forceinline__ float wave_sum(float x)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// f32 -> f16 bits, round to nearest even: the hardware conversion, which matches
// KVCache::f32_to_f16_rne (src/model/kvcache.h:256-274) on every non-NaN input
// (f16 subnormals are kept, overflow goes to inf); NaN becomes the quiet NaN that
// function returns.
__device__ __forceinline__ uint16_t f16_rne_bits(float f)
{
    if (f != f) return (uint16_t)(((__float_as_uint(f) >> 16) & 0x8000u) | 0x7e00u);
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// f32 -> f16 bits as KVCache::store converts (src/model/kvcache.h:903-911): mantissa
// truncated, results below the f16 normal range flushed to signed zero, exponent
// overflow (inf and NaN included) to signed inf.
__device__ __forceinline__ uint16_t f16_trunc_bits(float f)
{
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int e = (int)((x >> 23) & 0xffu) - 112;
    if (e <= 0) return (uint16_t)sign;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | ((x >> 13) & 0x3ffu));
}

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
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
            const bool zc = (a.flags & (isq ? kPrepQZeroCentred : kPrepKZeroCentred)) != 0;
            const float* w = isq ? a.qnw : a.knw;
#pragma unroll
            for (int j = 0; j < kPrepPer; ++j) {
                const int d = lane + 64 * j;
                if (d < hd) x[j] = zc ? x[j] * inv * (1.0f + w[d]) : (x[j] * w[d]) * inv;
            }
        }
        const int rot = a.rot, half = rot >> 1;
        if (rot > 0) {
#pragma unroll
            for (int j = 0; j < kPrepPer; ++j) {
                const int d = lane + 64 * j;
                if (d < rot) row[d] = x[j];
            }
            __syncthreads();
            const bool inter = (a.flags & kPrepInterleaved) != 0;
#pragma unroll
            for (int j = 0; j < kPrepPer; ++j) {
                const int d = lane + 64 * j;
                if (d >= rot) continue;
                if (inter) {
                    const int i = d >> 1;
                    const float c = a.tab[i], s = a.tab[half + i];
                    x[j] = (d & 1) == 0 ? row[d] * c - row[d + 1] * s : row[d - 1] * s + row[d] * c;
                } else if (d < half) {
                    x[j] = row[d] * a.tab[d] - row[d + half] * a.tab[half + d];
                } else {
                    const int i = d - half;
                    x[j] = row[d] * a.tab[i] + row[i] * a.tab[half + i];
                }
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

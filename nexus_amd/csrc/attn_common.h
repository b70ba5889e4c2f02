// nexus_amd/csrc/attn_common.h -- device-side types and helpers shared by the gfx950
// attention kernels (prefill MFMA kernel, split-KV decode kernel, LSE combine).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

namespace nxa {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Initial running max of the online softmax (transformer.h:8675 uses -1e30 too): finite,
// so exp2(m_old - m_new) never evaluates (-inf) - (-inf).
constexpr float kNegBig = -1e30f;
// Lazy rescale threshold in log2 units: the prefill kernel keeps a stale row max until
// the true max exceeds it by more than this, so probabilities stay <= 2^8 (safe in f16).
constexpr float kRescaleThresh = 8.0f;

// D = A(32x16) * B(16x32) + C, f16 inputs, f32 accumulate (v_mfma_f32_32x32x16_f16).
// Lane l supplies A row (l & 31) and B column (l & 31), each with the 8 k-values of
// k-group (l >> 5).  D: lane l holds column (l & 31), rows 8*(i/4) + 4*(l>>5) + (i&3).
__device__ __forceinline__ f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// D = A(16x32) * B(32x16) + C, f16 inputs, f32 accumulate (v_mfma_f32_16x16x32_f16).
// Lane l supplies A row (l & 15) and B column (l & 15), each with 8 k-values of k-group
// (l >> 4); A and B assign k-values to register slots the same way, so any consistent
// mapping of real indices to (group, slot) yields the full dot product.
// D: lane l holds column (l & 15), rows 4*(l >> 4) + (0..3).
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f16x8 as_f16x8(u32x4 x) { return __builtin_bit_cast(f16x8, x); }
__device__ __forceinline__ u32x4 as_u32x4(f16x8 x) { return __builtin_bit_cast(u32x4, x); }

// Round-to-nearest-even f32 -> f16 of 8 values (v_cvt_pk_f16_f32 on gfx950).
__device__ __forceinline__ f16x8 cvt_f16x8(float a0, float a1, float a2, float a3,
                                           float a4, float a5, float a6, float a7)
{
    f32x2 p0 = {a0, a1}, p1 = {a2, a3}, p2 = {a4, a5}, p3 = {a6, a7};
    f16x2 h0 = __builtin_convertvector(p0, f16x2);
    f16x2 h1 = __builtin_convertvector(p1, f16x2);
    f16x2 h2 = __builtin_convertvector(p2, f16x2);
    f16x2 h3 = __builtin_convertvector(p3, f16x2);
    f16x8 r = {h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
    return r;
}

// Value of the same register in lane (l ^ 32): pairs the two k-groups of a 32x32 tile.
__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32); }

// Cross-lane reductions on the VALU (v_permlane{16,32}_swap, no LDS round trip).  The
// instruction swaps the upper half (lanes 32-63, or the odd 16-lane rows) of its first
// operand with the lower half (lanes 0-31, or the even rows) of its second; with both
// starting as x, the pair then holds x[l] and x[l ^ 32] (or x[l ^ 16]) in every lane, so
// max/sum of the pair is the reduction over the two lanes.  Issued as inline asm so the two
// results are two registers (s_nop 1: two wait states after the VALU writes of x).
__device__ __forceinline__ void swap_halves32(float& a, float& b)
{
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap_rows16(float& a, float& b)
{
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float max_xor32(float x)
{
    float a = x, b = x;
    swap_halves32(a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor32(float x)
{
    float a = x, b = x;
    swap_halves32(a, b);
    return a + b;
}
__device__ __forceinline__ float max_xor16(float x)
{
    float a = x, b = x;
    swap_rows16(a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor16(float x)
{
    float a = x, b = x;
    swap_rows16(a, b);
    return a + b;
}

// Byte permute of two dwords (v_perm_b32): selector bytes 0-3 pick from lo, 4-7 from hi.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel)
{
    return __builtin_amdgcn_perm(hi, lo, sel);
}
// Pack the low (or high) f16 halves of two dwords: {a.half, b.half}.
constexpr uint32_t kSelLo = 0x05040100u;
constexpr uint32_t kSelHi = 0x07060302u;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Softcapped score in log2 units, softcap * tanh(x / softcap) * log2(e), with
// tanh(y) = 1 - 2 / (e^(2y) + 1) on v_exp_f32 and v_rcp_f32: five VALU operations instead of
// a division and a library tanh; absolute error of tanh ~1e-7, the +-1 limits exact (e^(2y)
// overflows to inf or underflows to 0).  c1 = 2 log2(e) / softcap, c2 = softcap log2(e).
__device__ __forceinline__ float softcap_log2(float x, float c1, float c2)
{
    return c2 - 2.f * c2 * __builtin_amdgcn_rcpf(fast_exp2(x * c1) + 1.f);
}

// Output gate of the gated attention layers: sigmoid(z), clamped to 1 above z = 80 and to 0
// below -80 (qwen35_attn_comb.comp:34-38; the CPU path, transformer.h:8508-8511).
__device__ __forceinline__ float gate_sigmoid(float z)
{
    return z > 80.f ? 1.f : (z < -80.f ? 0.f : 1.f / (1.f + fast_exp2(-z * kLog2e)));
}
// Gate factors of 4 (or 2) consecutive output elements starting at `off` (16- or 8-byte
// aligned); all 1 when the call has no gate.
__device__ __forceinline__ f32x4 gate4(const float* gate, size_t off)
{
    if (!gate) return f32x4{1.f, 1.f, 1.f, 1.f};
    const f32x4 z = *(const f32x4*)(gate + off);
    return f32x4{gate_sigmoid(z[0]), gate_sigmoid(z[1]), gate_sigmoid(z[2]), gate_sigmoid(z[3])};
}
__device__ __forceinline__ f32x2 gate2(const float* gate, size_t off)
{
    if (!gate) return f32x2{1.f, 1.f};
    const f32x2 z = *(const f32x2*)(gate + off);
    return f32x2{gate_sigmoid(z[0]), gate_sigmoid(z[1])};
}

// ---- decode prep math (one head on one 64-lane wave, lane l owning elements l, l + 64, ...),
// shared by the prep kernel and the fused decode-layer kernel so both compute the same f32
// values.  The norm is written as the host does it: cpu::rms_norm (src/cpu/matmul.h:1860-1880)
// computes (x * w) * inv, nx_rms_norm_add_one (src/model/transformer.h:504-520) computes
// x * inv * (1 + w), inv = 1 / sqrt(mean(x^2) + eps).  RoPE pairs are (i, i + rot/2)
// (rotate_half) or (2i, 2i + 1) (interleaved), the two layouts of rope_apply
// (src/model/attention.h:593-608), cos at tab[i] and sin at tab[rot/2 + i].
// x of the lane a DPP control selects (gfx9 controls; every lane is a valid source)
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;          // quad_perm [1, 0, 3, 2]: lane l ^ 1
constexpr int kDppXor2 = 0x4E;          // quad_perm [2, 3, 0, 1]: lane l ^ 2
constexpr int kDppHalfMirror = 0x141;   // row_half_mirror: lane 7 - i within 8 lanes
constexpr int kDppMirror = 0x140;       // row_mirror: lane 15 - i within 16 lanes
// x of lane l ^ 32 (v_permlane32_swap leaves x[l ^ 32] in the second register of lanes 0-31
// and in the first of lanes 32-63)
__device__ __forceinline__ float lane_xor32(float x, int lane)
{
    float a = x, b = x;
    swap_halves32(a, b);
    return lane < 32 ? b : a;
}
__device__ __forceinline__ float lane_xor16(float x, int lane)
{
    float a = x, b = x;
    swap_rows16(a, b);
    return (lane & 16) == 0 ? b : a;
}
// Sum over the 64 lanes, the same value in every lane, on the VALU: lanes l ^ 1 and l ^ 2 (quad
// permutes), then the mirrors within 8- and 16-lane rows (each quad, then each half row, holds
// one value by then, so a mirror adds the neighbouring one), then the other 16-lane row and the
// other half of the wave (permlane swaps).  Both lanes of every pair add the same two operands.
__device__ __forceinline__ float prep_wave_sum(float x)
{
    x += dpp_mov<kDppXor1>(x);
    x += dpp_mov<kDppXor2>(x);
    x += dpp_mov<kDppHalfMirror>(x);
    x += dpp_mov<kDppMirror>(x);
    x = sum_xor16(x);
    return sum_xor32(x);
}
__device__ __forceinline__ float prep_norm_inv(float sum_sq, int hd, float eps)
{
    return 1.0f / sqrtf(sum_sq / (float)hd + eps);
}
__device__ __forceinline__ float prep_norm_apply(float x, float inv, float w, bool add_one)
{
    return add_one ? x * inv * (1.0f + w) : (x * w) * inv;
}
// Rotated value of element d (< rot) from its own pre-rotation value x, its partner p
// (prep_rope_partner) and the table entries c = tab[ci], s = tab[rot/2 + ci] with
// ci = prep_rope_cos_index(d).
__device__ __forceinline__ int prep_rope_partner(int d, int rot, bool interleaved)
{
    return interleaved ? (d ^ 1) : (d < (rot >> 1) ? d + (rot >> 1) : d - (rot >> 1));
}
__device__ __forceinline__ int prep_rope_cos_index(int d, int rot, bool interleaved)
{
    return interleaved ? (d >> 1) : (d < (rot >> 1) ? d : d - (rot >> 1));
}
__device__ __forceinline__ float prep_rope(int d, float x, float p, float c, float s, int rot, bool interleaved)
{
    if (interleaved) return (d & 1) == 0 ? x * c - p * s : p * s + x * c;
    return d < (rot >> 1) ? x * c - p * s : x * c + p * s;
}
// RoPE partners p[j] of the elements x[j] = element lane + 64 j below rot, taken from registers
// where the pairing allows it: interleaved pairs are lanes l, l ^ 1; rotate_half pairs d, d + rot/2
// are lanes l, l ^ 16 (rot 32) or l ^ 32 (rot 64), or elements j, j ^ 1 (rot 128) or j ^ 2 (rot 256)
// of one lane.  False for other rotations (the caller exchanges through LDS).  Wave-uniform.
template <int PER>
__device__ __forceinline__ bool prep_rope_partners(const float (&x)[PER], float (&p)[PER], int lane, int rot,
                                                   bool interleaved)
{
    if (interleaved) {
#pragma unroll
        for (int j = 0; j < PER; ++j) p[j] = dpp_mov<kDppXor1>(x[j]);
        return true;
    }
    switch (rot) {
    case 32:
        p[0] = lane_xor16(x[0], lane);
        return true;
    case 64:
        p[0] = lane_xor32(x[0], lane);
        return true;
    case 128:
        if constexpr (PER >= 2) {
            p[0] = x[1];
            p[1] = x[0];
            return true;
        }
        return false;
    case 256:
        if constexpr (PER >= 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = x[j ^ 2];
            return true;
        }
        return false;
    default:
        return false;
    }
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

// Order this wave's LDS writes before its later LDS reads (wave-private LDS regions).
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Dispatch position of the workgroup whose item block b runs, for grids of cus < n < 2 cus
// workgroups at two per CU (cus, n multiples of 8).  The hardware deals block b to XCD b % 8
// and places the first cus blocks one per CU; block cus + j then lands on the CU of block j
// (measured on MI355X, every launch alike).  Items are ordered heaviest first per XCD (position
// t = b / 8 within it), so without this the shared CUs would pair the heaviest blocks with the
// lightest.  Within each XCD the first-round positions rotate by rot = (n - cus) / 8: positions
// t < rot (beside an overflow block) take ranks span - rot .. span - 1, the lightest of the first
// round, and positions rot .. span - 1 (alone on their CU) ranks 0 .. span - rot - 1; overflow
// positions (t >= span = cus / 8) keep theirs.  A bijection on positions; rot = 0 is identity.
__device__ __forceinline__ int pair_rotate(int b, int rot, int span)
{
    const int x = b & 7, t = b >> 3;
    if (rot <= 0 || t >= span) return b;
    return x + 8 * (t < rot ? t + span - rot : t - rot);
}

// Map a linear block index to a work item so that each XCD (blocks are dealt round-robin
// over the 8 XCDs) receives one contiguous range of items: items that share a KV head
// then share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int b, int n_items)
{
    const int per = n_items >> 3, rem = n_items & 7;
    const int x = b & 7, t = b >> 3;
    return x * per + (x < rem ? x : rem) + t;
}

// The same for causal query blocks ordered (kv head, heaviest first) in runs of per_kv per kv
// head, one work item per block (no key splits).  Contiguous ranges would hand one XCD a kv
// head's heaviest blocks and another its lightest whenever a kv head spans several XCDs or an
// XCD boundary cuts through one (blocks differ in length up to n_qblocks-fold).  Instead the 8
// XCDs form g = gcd(n_kv, 8) groups of 8 / g, each serving n_kv / g kv heads whose blocks it
// deals round robin over its XCDs: every XCD gets the same mix of heavy and light blocks,
// heaviest first within each kv head, and reads only its group's K/V.  With n_kv a multiple of
// 8 this is the contiguous mapping (whole kv heads per XCD).  Measured on MI355X, 16q/2kv hd
// 256, 8192 tokens cold: 970 -> 612 us.  Key-split items are near equal in length and keep the
// contiguous ranges (512 queries over 32k keys in 4 splits: 305 vs 309 us).
__device__ __forceinline__ int xcd_remap_kv(int b, int n_items, int n_kv, int per_kv, int n_splits)
{
    if (n_splits == 1) {
        const int g = min(n_kv & -n_kv, 8);                   // gcd(n_kv, 8)
        const int c = 8 / g;                                  // XCDs per group
        if (per_kv % c == 0) {                                // n_items = 8 * (n_kv / g) * per_kv / c
            const int x = b & 7, t = b >> 3;
            return (x / c) * (n_kv / g) * per_kv + t * c + x % c;
        }
    }
    return xcd_remap(b, n_items);
}

// ---- raw buffer loads: the descriptor's byte range makes out-of-range loads return 0,
// so K/V rows past the cache end (or Q rows past n_query) need no branch.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;     // raw 32-bit dword buffer, gfx9 family

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
// Same, for a base and size that are uniform across the wave: readfirstlane keeps the
// descriptor in scalar registers (a descriptor the compiler places in vector registers
// turns every buffer access into a waterfall loop).
__device__ __forceinline__ rsrc_t make_rsrc_uniform(const void* base, uint32_t bytes)
{
    const uint64_t p = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    return make_rsrc((const void*)(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t byte_off)
{
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}

// Host side: raise a kernel's dynamic LDS limit (hipFuncAttributeMaxDynamicSharedMemorySize)
// once per device.  The attribute belongs to the device current at the call, so a process
// that drives several GPUs sets it on each; `done` is the kernel's bitmask of devices already
// set (device ids below 64; others set it on every launch).
inline hipError_t ensure_dyn_lds(const void* kernel, int bytes, std::atomic<uint64_t>& done)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
    if (bit && (done.load(std::memory_order_relaxed) & bit)) return hipSuccess;
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_relaxed);
    return e;
}

}  // namespace nxa

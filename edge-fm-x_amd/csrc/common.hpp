// Shared device helpers for the gfx950 kernels of the EdgeFM hot path.
//
// Activations and weights are stored as raw bf16 bit patterns (uint16_t) and all
// arithmetic is fp32. Every fp32 -> bf16 rounding goes through the helpers below
// (round-to-nearest-even, quiet NaN), so the rule is identical in every kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "edgefm_hip.h"

namespace efm {

constexpr int kWave = 64;
// Split-KV decode partials that the o_proj GEMV's merge prologue holds (one register
// slot per split and input float4): query widths up to 2048 (two float4 per thread) with
// up to 12 splits (a variant with 8 slots takes up to 8: fewer instructions ahead of the
// weight stream), or up to 1024 (one float4) with up to 24.
constexpr int kMergeMaxSplits = 12;
constexpr int kMergeShortSplits = 8;
constexpr int kMergeMaxWidth = 2048;
constexpr int kMergeNarrowMaxSplits = 24;
constexpr int kMergeNarrowMaxWidth = 1024;

// Splits the o_proj merge prologue takes for a query width (0: none).
__host__ __device__ constexpr int merge_max_splits(int64_t q_width) {
    return q_width <= kMergeNarrowMaxWidth ? kMergeNarrowMaxSplits : (q_width <= kMergeMaxWidth ? kMergeMaxSplits : 0);
}

// Split plan of the decode partials (efm_decode_attention_partials) that every consumer of
// them reads back: keys per split, splits, and whether the one-wave tile kernel writes
// them (else the 4- / 8-wave kernels).
struct DecodePartialsPlan {
    int keys_per_split, split_cap;
    bool tile;
};

typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 with round-to-nearest-even (NaN -> quiet NaN), using the gfx950
// conversion instruction v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)f);
}

__device__ __forceinline__ float round_bf16(float f) {
    return bf16_to_f32(f32_to_bf16(f));
}

// silu(g) = g / (1 + e^-g), the activation's own formula, in about a third of the
// instructions of expf and an IEEE division: e^-g = 2^(-g log2 e) on v_exp_f32, then
// q = g * rcp(d) and one residual step q + (g - d q) rcp(d), which rounds like the
// division. The residual is formed as -(d q - g) so that g = -0 keeps its sign. Where the
// step is not finite (g = +inf, -inf, NaN, or e^-g overflowing for g < -88.7) q is the
// quotient: +inf, NaN, NaN, -0, as g / (1 + e^-g) gives. For g in (-88.7, -87.3) the
// reciprocal is below the normal range and the result, under 1e-36 in magnitude, may
// differ from the division's. Every SwiGLU epilogue uses this one form, so the decode
// GEMVs, the prefill GEMMs and the standalone activation agree bit for bit.
__device__ __forceinline__ float silu_f32(float g) {
    const float d = 1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    const float r = __builtin_amdgcn_rcpf(d);
    const float q = g * r;
    const float s = __builtin_fmaf(-__builtin_fmaf(d, q, -g), r, q);
    return __builtin_isfinite(s) ? s : q;
}

// Low and high bf16 halves of a packed 32-bit word, as fp32.
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// Unpack 8 bf16 (one 16-byte vector) into fp32.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
    f[0] = lo_f32(v.x); f[1] = hi_f32(v.x);
    f[2] = lo_f32(v.y); f[3] = hi_f32(v.y);
    f[4] = lo_f32(v.z); f[5] = hi_f32(v.z);
    f[6] = lo_f32(v.w); f[7] = hi_f32(v.w);
}

__device__ __forceinline__ uint4 pack8(const float* f) {
    uint4 v;
    v.x = pack_bf16x2(f[0], f[1]);
    v.y = pack_bf16x2(f[2], f[3]);
    v.z = pack_bf16x2(f[4], f[5]);
    v.w = pack_bf16x2(f[6], f[7]);
    return v;
}

// 8-wide bf16 dot product accumulated in fp32.
// acc + a . b over 8 bf16 pairs in fp32, as four v_dot2c_f32_bf16 (each adds two exact
// bf16 x bf16 products to the accumulator); no unpacking, a quarter of the VALU work of
// scalar FMAs. Every GEMV shares this helper, so fused and unfused kernels agree bit for
// bit.
__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.x), __builtin_bit_cast(bf16x2_t, b.x), acc,
                                          false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.y), __builtin_bit_cast(bf16x2_t, b.y), acc,
                                          false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.z), __builtin_bit_cast(bf16x2_t, b.z), acc,
                                          false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.w), __builtin_bit_cast(bf16x2_t, b.w), acc,
                                          false);
    return acc;
}

// Streaming 16-byte load for data read exactly once per step (weights, KV):
// marked non-temporal so it does not evict the small activation working set.
__device__ __forceinline__ uint4 load_stream16(const void* p) {
    const uint4* q = reinterpret_cast<const uint4*>(p);
    uint4 v;
    v.x = __builtin_nontemporal_load(&q->x);
    v.y = __builtin_nontemporal_load(&q->y);
    v.z = __builtin_nontemporal_load(&q->z);
    v.w = __builtin_nontemporal_load(&q->w);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        v += __shfl_xor(v, off, kWave);
    }
    return v;
}

// DPP move of a float across lanes (CTRL: quad_perm 0x00-0xff, row_mirror 0x140,
// row_half_mirror 0x141, ...; every source lane valid).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes of a wave, returned uniform: four 16-lane DPP steps (xor 1, xor 2,
// half-row mirror, row mirror), then row broadcasts (lane 15 into rows 1 and 3, lane 31
// into rows 2 and 3) leave the total in lane 63, which is read out. No LDS-crossbar round
// trips: every decode GEMV reduces its dot products with this.
__device__ __forceinline__ float wave_total(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));   // row_bcast:15
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));   // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Max over the 64 lanes of a wave, returned uniform (as wave_total; rows outside a
// broadcast's row mask keep -inf).
__device__ __forceinline__ float wave_max_uniform(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    const int ninf = __float_as_int(-INFINITY);
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x142, 0xA, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x143, 0xC, 0xF, false)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over a 1-D block of `nthreads` (multiple of 64), valid in every thread: DPP wave
// totals, one LDS word per wave (`red`, nthreads / 64 floats, not read before in the
// launch), one barrier.
template <int nthreads>
__device__ __forceinline__ float block_total(float v, float* red) {
    v = wave_total(v);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < nthreads / kWave; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        v = fmaxf(v, __shfl_xor(v, off, kWave));
    }
    return v;
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = width / 2; off >= 1; off >>= 1) {
        v += __shfl_xor(v, off, kWave);
    }
    return v;
}

// (value, index) argmax with ties resolved to the lowest index
// (src/layers/sampler.cu:21-26, src/layers/linear.cu:155-160).
struct ArgMax {
    float v;
    int32_t i;
};

__device__ __forceinline__ ArgMax argmax_pick(ArgMax a, ArgMax b) {
    if (a.v > b.v) return a;
    if (b.v > a.v) return b;
    return (a.i <= b.i) ? a : b;
}

__device__ __forceinline__ ArgMax wave_argmax(ArgMax a) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        ArgMax o;
        o.v = __shfl_xor(a.v, off, kWave);
        o.i = __shfl_xor(a.i, off, kWave);
        a = argmax_pick(a, o);
    }
    return a;
}

// Block-wide fp32 sum for a 1-D block of `nthreads` (multiple of 64) threads.
// `scratch` must hold nthreads/64 floats. Result is valid in every thread.
template <int nthreads>
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    constexpr int nw = nthreads / kWave;
    v = wave_sum(v);
    const int w = threadIdx.x / kWave;
    const int l = threadIdx.x % kWave;
    __syncthreads();
    if (l == 0) scratch[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < nw; ++i) t += scratch[i];
    return t;
}

// RoPE inverse frequencies, computed on the host once per launch and passed in the
// kernel arguments: inv_freq[d] = fp32((1/rope_scale) / theta^(2d/head_dim)), evaluated
// in double and rounded once. The rotation angle is fp32(pos) * inv_freq[d] in fp32.
// (src/operators/attention_op.cu:363-364, src/layers/attention.cu:57-60)
constexpr int kMaxHalfDim = 64;
struct RopeTable {
    float inv_freq[kMaxHalfDim];
};

static inline void rope_table_fill(RopeTable* t, int head_dim, float theta, float rope_scale) {
    for (int d = 0; d < kMaxHalfDim; ++d) {
        const double e = (2.0 * (double)d) / (double)head_dim;
        t->inv_freq[d] = (d < head_dim / 2) ? (float)(exp(-e * log((double)theta)) / (double)rope_scale) : 0.f;
    }
}

// sin/cos of an fp32 angle (radians, |a| < 2^22): Cody-Waite reduction by 2*pi split
// into an fp32 head and tail, then the hardware sin/cos on the reduced argument in
// revolutions (|r| <= 0.5).
__device__ __forceinline__ void sincos_reduced(float a, float* s, float* c) {
    const float k = rintf(a * 0.15915494309189535f);
    float r = fmaf(-k, 6.28318548202514648f, a);
    r = fmaf(-k, -1.7484555314695172e-07f, r);
    const float rev = r * 0.15915494309189535f;
    *s = __builtin_amdgcn_sinf(rev);
    *c = __builtin_amdgcn_cosf(rev);
}

// ---- tagged-word exchange between workgroups of one launch ----
// Tag of the current launch: epoch % 65535 + 1, never 0 (zeroed words never match) and
// different from the previous launch's, whose words are the stale ones a poll can see.
__device__ __forceinline__ uint32_t launch_tag(const uint32_t* epoch) {
    const uint32_t e = __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return e % 65535u + 1u;
}

// One tagged word (16-bit payload | tag << 16), written with an agent-scope atomic
// exchange: performed where the atomics of every XCD meet, so a poll from another XCD
// sees it without a cache flush on either side.
__device__ __forceinline__ void tagged_publish(uint32_t* p, uint32_t tag, uint32_t bits16) {
    (void)__hip_atomic_exchange(p, (tag << 16) | (bits16 & 0xffffu), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace efm

// Error reporting shared by every entry point of the C ABI.
namespace efm {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Kernel-path override set through efm_testing_set_kernel_path (EFM_KNOB_*); 0 = the
// library's own choice.
int kernel_knob(int knob);
}  // namespace efm

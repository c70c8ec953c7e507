// Batch-1 decode GEMV family for gfx950: device code shared by the GEMV kernels
// (gemv.hip) and the fused QKV projection + decode attention kernel
// (decode_qkv_attention.hip).
//
// y[n] = x . W[n, :] with W row-major [rows, K] bf16 (the reference's cuBLASLt layout,
// TRANSA=T on [out, in], src/layers/linear.cu:740). The kernel is HBM-bound: every
// weight byte is read exactly once per decode step, so the design goal is to keep
// enough 16-byte loads in flight on all 256 CUs and to do nothing else on the
// critical path.
//
//  * 256-thread workgroups (4 wave64s). A "row group" of R logical rows is owned by
//    KS waves that split the K dimension; a workgroup owns 4/KS row groups.
//  * Each lane loads 16 B (8 bf16) per row per step with non-temporal loads; a wave
//    covers 1 KiB contiguous of a row per load instruction (fully coalesced).
//  * All weight loads of a row block are issued first; the input-vector prologue
//    (plain copy, RMSNorm, or residual add + RMSNorm) runs while they are in flight and
//    leaves x in LDS as bf16, exactly as the unfused reference would have written it.
//  * Workgroups walk row blocks grid-stride; the next block's loads are issued before
//    the current block's cross-lane reductions and epilogue.
//  * Epilogues: bf16 store (+bias), fp32 store, QKV split with K/V written straight
//    into the KV-cache slot (optionally also published as tagged words, or with q and k
//    rotated: the rows d and d + hd/2 of a head are the two parts of one logical row),
//    SwiGLU over paired up/gate rows, and greedy top-1 with a last-workgroup grid
//    reduction (no second launch, self-resetting counter).
#pragma once

#include "common.hpp"

namespace efm {

enum { PRO_PLAIN = 0, PRO_NORM = 1, PRO_ADD_NORM = 2, PRO_ATTN_MERGE = 3, PRO_ATTN_MERGE_N = 4, PRO_ATTN_MERGE_W = 5 };
enum { EPI_BF16 = 0, EPI_F32 = 1, EPI_QKV = 2, EPI_SWIGLU = 3, EPI_TOP1 = 4, EPI_QKV_TAG = 5, EPI_QKV_ROPE = 6 };

// Weight-stream load of the GEMV main loop: a non-temporal 16-byte buffer load (weights
// are read once per decode step and must not evict the activation working set). Offsets
// at or past the resource's num_records read as zero without a memory access, so tails
// (rows past N, chunks past K, unused load slots) need no branch: every wave issues the
// same straight-line loads, and the compiler counts them exactly when it waits for the
// prologue's loads issued before them.
__device__ __forceinline__ uint4 gemv_wload(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 2 /* nt */);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
constexpr uint32_t kWloadSkip = 0x80000000u;   // past every num_records the GEMV builds

constexpr int kGemvThreads = 256;
constexpr int kNJMax = 6;
constexpr int kTop1MaxGridDev = 2048;  // top-1 workspace slots (its first 8 bytes hold the best key)
constexpr int kProMax = 4;       // max prologue chunks per thread (K <= 8192)

struct GemvArgs {
    int K;                      // input features
    int N;                      // logical output rows
    const bf16_t* W;            // [physical rows, K]
    const bf16_t* x;            // input vector (PLAIN) or h (NORM / ADD_NORM)
    const bf16_t* r_in;         // ADD_NORM residual input
    bf16_t* r_out;              // NORM / ADD_NORM residual output (written by block 0)
    const bf16_t* norm_w;       // RMSNorm weight
    float eps;
    const bf16_t* bias;         // optional, per logical row
    void* y;                    // output
    int q_dim, kv_dim;          // QKV split
    bf16_t* k_cache;
    bf16_t* v_cache;
    const uint32_t* d_kv_len;
    ArgMax* partials;           // TOP1: one per workgroup
    uint32_t* counter;          // TOP1: arrival counter (zero between launches)
    int32_t* token_out;
    // ATTN_MERGE: decode-attention split partials (efm_decode_attention_partials)
    const float* o_part;        // [Hkv][split_cap][G][hd]
    const float* ml_part;       // [Hkv][split_cap][G][2]
    int split_cap, keys_per_split, head_dim, group;
    const uint32_t* attn_len;   // *attn_len = attended rows (clamped to attn_max_len)
    uint32_t attn_max_len;
    // QKV_TAG: every output row n is also published as the tagged word tag_words[n]
    // (bf16 bits | launch tag << 16) for the attention workgroups of the same launch
    uint32_t* tag_words;
    const uint32_t* epoch;      // launch counter the tag derives from (launch_tag)
    // QKV_ROPE: logical row n = (head n / rope_half, pair d = n % rope_half) computes the
    // rows d and d + rope_half of that head; q and k heads are rotated at position
    // *d_kv_len - 1 (+ q_pos_off / k_pos_off) by inv_freq[d]
    int rope_half, q_pos_off, k_pos_off;
    RopeTable rope;
};


constexpr int kPlainPre = 4;   // PLAIN input chunks per thread loaded ahead of the weights
constexpr int kNormPre = 2;    // NORM / ADD_NORM chunks per thread loaded ahead (K <= 4096)

// Attention-merge prologues: ATTN_MERGE takes up to kMergeShortSplits splits of inputs up
// to 2048 wide (two float4 of every split per thread), ATTN_MERGE_W up to kMergeMaxSplits
// of them, ATTN_MERGE_N up to kMergeNarrowMaxSplits splits of inputs up to 1024 wide (one
// float4 per split: the same registers hold twice the splits).
constexpr bool pro_merge(int PRO) { return PRO == PRO_ATTN_MERGE || PRO == PRO_ATTN_MERGE_N || PRO == PRO_ATTN_MERGE_W; }
template <int PRO>
struct MergeShape {
    static constexpr int MS = (PRO == PRO_ATTN_MERGE_N) ? kMergeNarrowMaxSplits
                            : (PRO == PRO_ATTN_MERGE_W ? kMergeMaxSplits : (PRO == PRO_ATTN_MERGE ? kMergeShortSplits : 1));
    static constexpr int NQ = (PRO == PRO_ATTN_MERGE || PRO == PRO_ATTN_MERGE_W) ? 2 : 1;   // float4 of the input per thread
    // (m, l) loads per wave and input slice: lanes cover (head, split) pairs, 64 / heads
    // per slice splits per load (at least 16: head_dim 64 puts 4 heads in a wave's slice)
    static constexpr int ML = (MS + 15) / 16;
};
static_assert(MergeShape<PRO_ATTN_MERGE_N>::NQ * 4 * kGemvThreads == kMergeNarrowMaxWidth &&
              MergeShape<PRO_ATTN_MERGE>::NQ * 4 * kGemvThreads == kMergeMaxWidth, "merge widths");
static_assert(MergeShape<PRO_ATTN_MERGE>::MS % 4 == 0 && MergeShape<PRO_ATTN_MERGE_N>::MS % 4 == 0 &&
              MergeShape<PRO_ATTN_MERGE_W>::MS % 4 == 0,
              "merge weights are read four splits at a time");

// The prologue's own loads (input vector, residual, norm weight), issued before the first
// weight loads of the workgroup: loads return in issue order, so issued after the weight
// stream they would wait for all of it, and the norm's reduction would start only then.
template <int PRO>
struct ProLoads {
    static constexpr int N = (PRO == PRO_PLAIN) ? kPlainPre : (pro_merge(PRO) ? 0 : kNormPre);
    static constexpr int MS = MergeShape<PRO>::MS, NQ = MergeShape<PRO>::NQ;
    uint4 x[N > 0 ? N : 1], r[PRO == PRO_ADD_NORM ? N : 1], w[(PRO == PRO_NORM || PRO == PRO_ADD_NORM) ? N : 1];
    float2 ml[NQ][MergeShape<PRO>::ML];   // ATTN_MERGE*: (m, l) of this lane's (head, split) pairs
    float4 op[NQ][MS];   // ATTN_MERGE*: this thread's NQ x 4 input elements of every split
    uint32_t len;        // ATTN_MERGE*: attended rows
};

// The one-round-trip attention merge (prologue of merge + o_proj) covers these shapes.
template <int PRO>
__device__ __forceinline__ bool merge_fast(const GemvArgs& a) {
    return a.K <= MergeShape<PRO>::NQ * 4 * kGemvThreads && a.split_cap <= MergeShape<PRO>::MS;
}

// Max / sum over each aligned group of 16 lanes (or 32 with wide), the result in every lane
// of the group: four DPP steps within a row (xor 1, xor 2, half-row mirror, row mirror),
// plus one swizzle (xor 16) across the row pair for 32 lanes. No LDS round trips.
__device__ __forceinline__ float lane_group_max(float v, bool wide) {
    v = fmaxf(v, dpp_f32<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f32<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dpp_f32<0x140>(v));   // row_mirror
    if (wide) v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
    return v;
}
__device__ __forceinline__ float lane_group_sum(float v, bool wide) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    if (wide) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
    return v;
}

// Branch-free like the weight loads (chunks past K read as zero), so that the compiler
// waits for each of them by its exact position in the wave's load sequence.
template <int PRO>
__device__ __forceinline__ void gemv_prologue_load(const GemvArgs& a, ProLoads<PRO>& p) {
    if constexpr (pro_merge(PRO)) {
        // The split slots of this thread's elements: the head offset is computed once, slot
        // j adds j splits (one add per load); the merge never uses the slots past
        // split_cap, since the live split count is at most split_cap. The split
        // statistics come once per
        // wave: the slice's hpw = 256 / head_dim heads take 64 / hpw lanes each, lane l
        // holding (head l / (64 / hpw), split l % (64 / hpw) + i * 64 / hpw). Threads past
        // the elements and shapes outside merge_fast read zeros.
        typedef float f32x2_t __attribute__((ext_vector_type(2)));
        typedef float f32x4_t __attribute__((ext_vector_type(4)));
        constexpr int MS = MergeShape<PRO>::MS, NQ = MergeShape<PRO>::NQ, ML = MergeShape<PRO>::ML;
        const bool fast = merge_fast<PRO>(a);
        p.len = fast ? min(a.attn_len[0], a.attn_max_len) : 0u;
        const int hd = a.head_dim, G = a.group, cap = a.split_cap;
        const int Hq = a.K / hd, Hkv = Hq / G;
        const int hd_shift = __builtin_ctz((unsigned)hd);   // head_dim 64 or 128
        const int hpw_shift = 8 - hd_shift;                 // log2(256 / head_dim)
        const uint32_t ml_split = (uint32_t)(G * 8), op_split = (uint32_t)(G * hd * 4);
        const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.ml_part), (short)0, fast ? (int)((uint32_t)Hkv * cap * ml_split) : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t rop = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.o_part), (short)0, fast ? (int)((uint32_t)Hkv * cap * op_split) : 0, 0x00020000);
        const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
        uint32_t vml[NQ], vop[NQ];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int c = threadIdx.x + q * kGemvThreads;
            const int n0 = c * 4, h = n0 >> hd_shift, d0 = n0 & (hd - 1);
            const int kvh = h / G, g = h - kvh * G;
            vop[q] = (c < (a.K >> 2)) ? ((uint32_t)(kvh * cap * G + g) * (uint32_t)hd + (uint32_t)d0) * 4u : kWloadSkip;
            const int hs = (((wave + q * (kGemvThreads / kWave)) * kWave * 4) >> hd_shift) + (lane >> (6 - hpw_shift));
            const int kvs = hs / G, gs = hs - kvs * G;
            vml[q] = (hs < Hq) ? (uint32_t)(kvs * cap * G + gs) * 8u : kWloadSkip;
        }
        const int jl = lane & ((kWave >> hpw_shift) - 1);
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int i = 0; i < ML; ++i) {
                const int js = jl + (i << (6 - hpw_shift));
                const uint32_t off = (js < cap) ? vml[q] + (uint32_t)js * ml_split : kWloadSkip;
                const f32x2_t m = __builtin_amdgcn_raw_buffer_load_b64(rml, off, 0, 0);
                p.ml[q][i] = make_float2(m[0], m[1]);
            }
        // With more than kMergeShortSplits slots, groups of four slots wholly past
        // split_cap issue no load (one uniform branch per group: a load costs the address
        // unit the same whether its data is used or not); the 8-slot variant loads every
        // slot (its few dead loads cost less than the branches). Slots past split_cap that
        // do load read entries of the next KV head, or zeros past the last.
#pragma unroll
        for (int j0 = 0; j0 < MS; j0 += 4) {
            if (MS <= kMergeShortSplits || j0 < cap) {
#pragma unroll
                for (int j = j0; j < j0 + 4; ++j)
#pragma unroll
                    for (int q = 0; q < NQ; ++q) {
                        const f32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rop, vop[q] + j * op_split, 0, 0);
                        p.op[q][j] = make_float4(v[0], v[1], v[2], v[3]);
                    }
            } else {
#pragma unroll
                for (int j = j0; j < j0 + 4; ++j)
#pragma unroll
                    for (int q = 0; q < NQ; ++q) p.op[q][j] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    }
    if constexpr (!pro_merge(PRO)) {
        const int nbytes = a.K * 2;
        auto rsrc = [&](const bf16_t* v) {
            return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(v), (short)0, nbytes, 0x00020000);
        };
        auto ld = [&](__amdgpu_buffer_rsrc_t rs, uint32_t off) {
            typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
            return make_uint4(v[0], v[1], v[2], v[3]);
        };
        const __amdgpu_buffer_rsrc_t rx = rsrc(a.x);
#pragma unroll
        for (int i = 0; i < ProLoads<PRO>::N; ++i) {
            const uint32_t off = (uint32_t)(threadIdx.x + i * kGemvThreads) * 16u;
            p.x[i] = ld(rx, off);
            if constexpr (PRO == PRO_ADD_NORM) p.r[i] = ld(rsrc(a.r_in), off);
            if constexpr (PRO == PRO_NORM || PRO == PRO_ADD_NORM) p.w[i] = ld(rsrc(a.norm_w), off);
        }
    }
}

template <int PRO>
__device__ __forceinline__ void gemv_prologue(const GemvArgs& a, const ProLoads<PRO>& pl, bf16_t* xs, float* red,
                                              int blk) {
    const int C = a.K >> 3;
    const uint4* x4 = reinterpret_cast<const uint4*>(a.x);
    uint4* xs4 = reinterpret_cast<uint4*>(xs);
    if constexpr (PRO == PRO_PLAIN) {
#pragma unroll
        for (int i = 0; i < kPlainPre; ++i) {
            const int c = threadIdx.x + i * kGemvThreads;
            if (c < C) xs4[c] = pl.x[i];
        }
        for (int c = threadIdx.x + kPlainPre * kGemvThreads; c < C; c += kGemvThreads) xs4[c] = x4[c];
        return;
    }
    if constexpr (!pro_merge(PRO)) {
        // Chunks past K hold zeros: they add nothing to the sum of squares. Chunks beyond the
        // preloaded ones (K > 4096) are loaded here, behind the weights, and read again for
        // the normalisation instead of being kept in registers.
        auto pre_sum = [&](int i, float (&v)[8]) {
            unpack8(pl.x[i], v);
            if (PRO == PRO_ADD_NORM) {
                float r[8];
                unpack8(pl.r[i], r);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += r[e];
            }
        };
        auto late_sum = [&](int c, float (&v)[8]) {
            unpack8(reinterpret_cast<const uint4*>(a.x)[c], v);
            if (PRO == PRO_ADD_NORM) {
                float r[8];
                unpack8(reinterpret_cast<const uint4*>(a.r_in)[c], r);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += r[e];
            }
        };
        float s[kNormPre][8];
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kNormPre; ++i) {
            pre_sum(i, s[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(s[i][e], s[i][e], ss);
        }
        // the residual stream's new value, once (after every use of the preloaded chunks: a
        // store in a branch would blur the compiler's count of the loads in flight)
        const bool store_r = blk == 0 && a.r_out != nullptr;
        if (store_r) {
#pragma unroll
            for (int i = 0; i < kNormPre; ++i) {
                const int c = threadIdx.x + i * kGemvThreads;
                if (c < C) reinterpret_cast<uint4*>(a.r_out)[c] = pack8(s[i]);
            }
        }
        for (int c = threadIdx.x + kNormPre * kGemvThreads; c < C; c += kGemvThreads) {
            float v[8];
            late_sum(c, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
            if (store_r) reinterpret_cast<uint4*>(a.r_out)[c] = pack8(v);
        }
        const float tot = block_total<kGemvThreads>(ss, red);
        const float inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
#pragma unroll
        for (int i = 0; i < kNormPre; ++i) {
            const int c = threadIdx.x + i * kGemvThreads;
            if (c < C) {
                float w[8], o[8];
                unpack8(pl.w[i], w);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = (s[i][e] * inv) * w[e];
                xs4[c] = pack8(o);
            }
        }
        for (int c = threadIdx.x + kNormPre * kGemvThreads; c < C; c += kGemvThreads) {
            float v[8], w[8], o[8];
            late_sum(c, v);
            unpack8(reinterpret_cast<const uint4*>(a.norm_w)[c], w);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (v[e] * inv) * w[e];
            xs4[c] = pack8(o);
        }
        return;
    }
    if constexpr (pro_merge(PRO)) {
    constexpr int MS = MergeShape<PRO>::MS, NQ = MergeShape<PRO>::NQ;
    {
        // x[h*hd + d] = bf16( sum_s w[h][s] * o_part[kvh][s][g][d] ), w[h][s] = exp2(m_s - M)
        // / sum_s exp2(m_s - M) l_s (log-sum-exp merge of the splits), with every load
        // issued up front, ahead of the weight stream (gemv_prologue_load): one memory
        // round trip, under the weights' instead of after them. The host admits only shapes
        // within merge_fast (outside it the loads read zeros and so does the projection's
        // input). Each wave merges its own input slice: the lanes holding a head's split
        // statistics reduce its max and denominator across lanes, write the head's split
        // weights to the wave's own LDS rows, and every lane applies its head's weights to
        // its partial outputs. Slots past the live split count take no part.
        constexpr int ML = MergeShape<PRO>::ML;
        __shared__ __align__(16) float swl[kGemvThreads / kWave][NQ][4 * MS];   // [wave][slice][head][split]
        const uint32_t L = pl.len;
        const int kps = a.keys_per_split;
        const int nsplit = (L == 0) ? 1 : (int)((L + kps - 1) / kps);
        const int hd_shift = __builtin_ctz((unsigned)a.head_dim);
        const int hpw_shift = 8 - hd_shift;
        const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
        const int hl = lane >> (6 - hpw_shift), jl = lane & ((kWave >> hpw_shift) - 1);
        const bool wide_group = hd_shift == 7;   // 32 lanes per head (head_dim 128), else 16
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            float M = -INFINITY;
#pragma unroll
            for (int i = 0; i < ML; ++i) {
                const int js = jl + (i << (6 - hpw_shift));
                if (js < nsplit) M = fmaxf(M, pl.ml[q][i].x);
            }
            M = lane_group_max(M, wide_group);
            float e[ML], den = 0.f;
#pragma unroll
            for (int i = 0; i < ML; ++i) {
                const int js = jl + (i << (6 - hpw_shift));
                const float m = pl.ml[q][i].x;
                e[i] = (js < nsplit && m != -INFINITY) ? exp2f(m - M) : 0.f;
                den = fmaf(e[i], pl.ml[q][i].y, den);
            }
            den = lane_group_sum(den, wide_group);
            const float inv = (den > 0.f) ? 1.f / den : 0.f;
#pragma unroll
            for (int i = 0; i < ML; ++i) {
                const int js = jl + (i << (6 - hpw_shift));
                if (js < MS) swl[wave][q][hl * MS + js] = e[i] * inv;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int he = (lane * 4) >> hd_shift;   // head of this lane's elements in the slice
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int c = threadIdx.x + q * kGemvThreads;
            const float* w = &swl[wave][q][he * MS];
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < MS; j += 4) {
                if (j < nsplit) {
                    const float4 w4 = *reinterpret_cast<const float4*>(w + j);
                    const float wj[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if (j + t < nsplit) {
                            const float4 o = pl.op[q][j + t];
                            acc[0] = fmaf(wj[t], o.x, acc[0]);
                            acc[1] = fmaf(wj[t], o.y, acc[1]);
                            acc[2] = fmaf(wj[t], o.z, acc[2]);
                            acc[3] = fmaf(wj[t], o.w, acc[3]);
                        }
                    }
                }
            }
            if (c < (a.K >> 2)) {
                uint2 pk;
                pk.x = pack_bf16x2(acc[0], acc[1]);
                pk.y = pack_bf16x2(acc[2], acc[3]);
                reinterpret_cast<uint2*>(xs)[c] = pk;
            }
        }
        return;
    }
    }
}

// 64-bit key of a top-1 candidate whose unsigned order is the argmax order: the value's
// bits mapped to an order-preserving unsigned word (-0 as +0; NaN lowest, so it never
// wins) in the high half, the inverted index in the low half (equal values -> lowest
// index wins). 0 is below every key.
__device__ __forceinline__ unsigned long long top1_key(ArgMax c) {
    uint32_t bits = __float_as_uint(c.v == 0.f ? 0.f : c.v);
    if (c.v != c.v) bits = 0u;
    else bits = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    return ((unsigned long long)bits << 32) | (unsigned long long)(~(uint32_t)c.i);
}

// Physical weight row of logical row n, part p (SwiGLU: p=0 up row n, p=1 gate row N+n;
// QKV_ROPE: rows d and d + half of head n / half, d = n % half).
template <int EPI>
__device__ __forceinline__ int phys_row(int n, int p, int N, int half) {
    if (EPI == EPI_QKV_ROPE) return (n / half) * 2 * half + p * half + n % half;
    return (EPI == EPI_SWIGLU && p == 1) ? (N + n) : n;
}

// QKV_ROPE: cos / sin of logical row n (the pair d = n % half of its head) at position
// L - 1 + the q or k offset. The row is the same for every lane of a wave (one row per
// wave group), so the frequency comes through a scalar load, not a per-lane load of the
// kernel-argument table.
__device__ __forceinline__ float2 qkv_rope_cs(const GemvArgs& a, int n, uint32_t L) {
    n = __builtin_amdgcn_readfirstlane(n);
    const int half = a.rope_half, d = n % half;
    const int n0 = (n / half) * 2 * half + d;
    const int pos = (int)L - 1 + (n0 < a.q_dim ? a.q_pos_off : a.k_pos_off);
    float sn, cs;
    sincos_reduced((float)pos * a.rope.inv_freq[d], &sn, &cs);
    return make_float2(cs, sn);
}

// Body of the GEMV kernel for workgroup `blk` of `nblk` (grid-stride over row blocks),
// shared by gemv_kernel and the fused QKV + attention kernel.
template <int R, int KS, int PRO, int EPI, int NJM = kNJMax>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, int nj, int nseg, int blk, int nblk) {
    constexpr int P = (EPI == EPI_SWIGLU || EPI == EPI_QKV_ROPE) ? 2 : 1;
    constexpr int G = 4 / KS;          // row groups per block
    constexpr int RB = G * R;          // logical rows per block
    extern __shared__ __align__(16) unsigned char smem_raw[];
    bf16_t* xs = reinterpret_cast<bf16_t*>(smem_raw);
    __shared__ float red[kGemvThreads / kWave];
    __shared__ float part[G][KS][R * P];
    __shared__ ArgMax amx[G];

    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int grp = wave / KS;
    const int kw = wave % KS;
    const int C = a.K >> 3;
    const int segC = nj * kWave * KS;
    const int nrb = (a.N + RB - 1) / RB;

    ArgMax best;
    best.v = -INFINITY;
    best.i = 0x7fffffff;

    // Weight loads of row block rb, segment seg: one buffer resource per block and part
    // (uniform across the workgroup) covering the block's rows below N.
    // NJM: load slots per lane and row (nj <= NJM live; launches take the fewest slots that
    // hold their rows, so no slot past a row is issued: an unused slot costs the address
    // unit as much as a used one)
    uint4 wr[R][P][NJM];
    const int grpu = __builtin_amdgcn_readfirstlane(grp);
    const int kwu = __builtin_amdgcn_readfirstlane(kw);
    auto issue = [&](int rb, int seg) {
        const int row0 = rb * RB;
        const int rows = max(0, min(RB, a.N - row0));
        const int nrec = __builtin_amdgcn_readfirstlane(rows * a.K * 2);
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const bf16_t* base = a.W + (size_t)phys_row<EPI>(row0, p, a.N, a.rope_half) * (size_t)a.K;
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, nrec, 0x00020000);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t roff = (uint32_t)((grpu * R + r) * a.K) * 2u;
#pragma unroll
                for (int j = 0; j < NJM; ++j) {
                    const int c = seg * segC + kwu * kWave + lane + j * kWave * KS;
                    const uint32_t off = (j < nj && c < C) ? roff + (uint32_t)c * 16u : kWloadSkip;
                    wr[r][p][j] = gemv_wload(rs, off);
                }
            }
        }
    };

    const uint32_t tag = (EPI == EPI_QKV_TAG) ? launch_tag(a.epoch) : 0u;
    // QKV_ROPE: the cache length is read first, so that its round trip runs under the
    // prologue's and the weights' instead of after them
    uint32_t rope_len = 0;
    if constexpr (EPI == EPI_QKV_ROPE) rope_len = a.d_kv_len[0];
    ProLoads<PRO> pl;
    gemv_prologue_load<PRO>(a, pl);
    int rb = blk;
    issue(rb, 0);   // unconditional (a block past the end reads zeros): see gemv_wload
    __builtin_amdgcn_sched_barrier(0);   // every load goes out before the prologue's first wait
    gemv_prologue<PRO>(a, pl, xs, red, blk);
    // QKV_ROPE: the first row block's cos / sin while the weights stream (the epilogue
    // recomputes them for any later block of a grid-stride walk)
    float2 rcs[R];
    if constexpr (EPI == EPI_QKV_ROPE) {
#pragma unroll
        for (int r = 0; r < R; ++r) rcs[r] = qkv_rope_cs(a, blk * RB + grp * R + r, rope_len);
    }
    __syncthreads();
    const uint4* xs4 = reinterpret_cast<const uint4*>(xs);

    while (rb < nrb) {
        float acc[R][P];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int p = 0; p < P; ++p) acc[r][p] = 0.f;

        for (int seg = 0; seg < nseg; ++seg) {
            if (seg > 0) issue(rb, seg);
#pragma unroll
            for (int j = 0; j < NJM; ++j) {
                const int c = seg * segC + kw * kWave + lane + j * kWave * KS;
                if (j < nj && c < C) {
                    const uint4 xv = xs4[c];
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int p = 0; p < P; ++p) acc[r][p] = dot8(wr[r][p][j], xv, acc[r][p]);
                }
            }
        }
        const int next = rb + nblk;
        if (next < nrb) issue(next, 0);

#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int p = 0; p < P; ++p) acc[r][p] = wave_total(acc[r][p]);
        if (KS > 1) {
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int p = 0; p < P; ++p) part[grp][kw][r * P + p] = acc[r][p];
            }
            __syncthreads();
            if (kw == 0 && lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int p = 0; p < P; ++p) {
                        float t = 0.f;
#pragma unroll
                        for (int k = 0; k < KS; ++k) t += part[grp][k][r * P + p];
                        acc[r][p] = t;
                    }
            }
            __syncthreads();
        }

        if (kw == 0 && lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int n = rb * RB + grp * R + r;
                if (n >= a.N) continue;
                if (EPI == EPI_QKV_ROPE) {
                    // bf16(x . W + b) for rows d and d + half of the head, then q and k
                    // rotated as the reference rotates them on read; K / V into the slot
                    const int half = a.rope_half;
                    const int d = n % half;
                    const int n0 = (n / half) * 2 * half + d, n1 = n0 + half;
                    float v0 = acc[r][0], v1 = acc[r][P - 1];
                    if (a.bias != nullptr) {
                        v0 += bf16_to_f32(a.bias[n0]);
                        v1 += bf16_to_f32(a.bias[n1]);
                    }
                    float x0 = round_bf16(v0), x1 = round_bf16(v1);
                    const uint32_t L = rope_len;
                    if (n0 < a.q_dim + a.kv_dim) {
                        const float2 c2 = (rb == blk) ? rcs[r] : qkv_rope_cs(a, n, L);
                        const float cs = c2.x, sn = c2.y;
                        const float y0 = x0 * cs - x1 * sn, y1 = x1 * cs + x0 * sn;
                        x0 = y0;
                        x1 = y1;
                    }
                    const bf16_t b0 = (bf16_t)f32_to_bf16(x0), b1 = (bf16_t)f32_to_bf16(x1);
                    if (n0 < a.q_dim) {
                        reinterpret_cast<bf16_t*>(a.y)[n0] = b0;
                        reinterpret_cast<bf16_t*>(a.y)[n1] = b1;
                    } else if (L > 0) {
                        const size_t slot = (size_t)(L - 1) * (size_t)a.kv_dim;
                        const int m0 = n0 - a.q_dim;
                        bf16_t* dst = (m0 < a.kv_dim) ? a.k_cache + slot + m0 : a.v_cache + slot + (m0 - a.kv_dim);
                        dst[0] = b0;
                        dst[half] = b1;
                    }
                    continue;
                }
                float v = acc[r][0];
                if (a.bias != nullptr) v += bf16_to_f32(a.bias[n]);
                if (EPI == EPI_BF16) {
                    reinterpret_cast<bf16_t*>(a.y)[n] = (bf16_t)f32_to_bf16(v);
                } else if (EPI == EPI_F32) {
                    reinterpret_cast<float*>(a.y)[n] = v;
                } else if (EPI == EPI_QKV || EPI == EPI_QKV_TAG) {
                    // QKV_TAG: q and the K / V row go to the attention workgroups as tagged
                    // words (K / V only when there is a slot); the K row reaches the cache
                    // from the attention split that rotates it, the V row is stored here
                    const bf16_t bv = (bf16_t)f32_to_bf16(v);
                    if (n < a.q_dim) {
                        if (EPI == EPI_QKV) reinterpret_cast<bf16_t*>(a.y)[n] = bv;
                        else tagged_publish(a.tag_words + n, tag, (uint32_t)bv);
                    } else {
                        const uint32_t L = a.d_kv_len[0];
                        if (L > 0) {
                            const size_t slot = (size_t)(L - 1) * (size_t)a.kv_dim;
                            const int m = n - a.q_dim;
                            if (EPI == EPI_QKV_TAG) tagged_publish(a.tag_words + n, tag, (uint32_t)bv);
                            if (m < a.kv_dim) {
                                if (EPI == EPI_QKV) a.k_cache[slot + m] = bv;
                            } else {
                                a.v_cache[slot + (m - a.kv_dim)] = bv;
                            }
                        }
                    }
                } else if (EPI == EPI_SWIGLU) {
                    const float u = round_bf16(acc[r][0]);
                    const float g = round_bf16(acc[r][P - 1]);
                    const float sg = silu_f32(g);
                    reinterpret_cast<bf16_t*>(a.y)[n] = (bf16_t)f32_to_bf16(sg * u);
                } else if (EPI == EPI_TOP1) {
                    ArgMax c;
                    c.v = v;
                    c.i = n;
                    best = argmax_pick(best, c);
                }
            }
        }
        rb = next;
    }

    if (EPI == EPI_TOP1) {
        if (kw == 0 && lane == 0) amx[grp] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            ArgMax b = amx[0];
#pragma unroll
            for (int g = 1; g < G; ++g) b = argmax_pick(b, amx[g]);
            // Grid reduction without fences: every workgroup max-combines one 64-bit key
            // (top1_key) at the point where the atomics of every XCD meet, waits for that
            // atomic to return, then counts itself in; the last to arrive reads the winner
            // and clears both words for the next launch.
            unsigned long long* best_key = reinterpret_cast<unsigned long long*>(a.partials);
            const unsigned long long old =
                __hip_atomic_fetch_max(best_key, top1_key(b), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" : : "v"(old) : "memory");
            const uint32_t prev = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (prev == (uint32_t)nblk - 1u) {
                const unsigned long long k = __hip_atomic_load(best_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                a.token_out[0] = (int32_t)~(uint32_t)k;
                __hip_atomic_store(best_key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// Host: launch geometry of a GEMV over K inputs and N logical rows of P physical rows
// (R rows per wave group, KS-way K split, nj chunks per lane per segment, nseg segments,
// grid workgroups over nrb row blocks).
struct GemvCfg {
    int R, KS, nj, nseg, grid, nrb;
};
GemvCfg gemv_pick_config(int K, int N, int P, int max_grid, bool tall, bool single_row);

}  // namespace efm

// Single-query GQA decode attention over the fixed-prefix KV cache, on the gfx950
// matrix cores.
//
// Semantics (FlashInfer single_decode_with_kv_cache, ROPE_LLAMA, as called from
// src/operators/attention_op.cu:1428-1466): for each query head h with KV head
// g = h / (Hq / Hkv),
//     o_h = sum_j softmax_j( RoPE(q_h, L-1) . RoPE(k_gj, j) / sqrt(hd) ) v_gj,  j < L,
// with RoPE the rotate-half rotation of pairs (d, d + hd/2). The cache holds
// un-rotated K, so keys are rotated on read.
//
// Kernel design (grid = splits x Hkv, 4 wave64s per workgroup):
//  * The G query heads of a KV head are the N dimension of v_mfma_f32_32x32x16_bf16:
//    scores are computed transposed, S^T = K . Q^T (K tile = A operand straight from
//    global memory, the pre-rotated, pre-scaled queries = B operand held in registers),
//    so each lane owns one head column and 16 keys; the online softmax is in-lane plus
//    one cross-half exchange. O^T = V^T . P^T reuses P from the score registers; V^T is
//    staged per wave in LDS with the same key permutation as the accumulator rows.
//  * Keys are either rotated on read (cache of un-rotated K, the reference's layout) by
//    angle addition: cos/sin(k * f_d) for the 32 key offsets of a tile are tabulated
//    once per workgroup, cos/sin(base * f_d) once per tile (one sincos per thread); or
//    the cache already holds rotated keys and only this step's newest row is rotated
//    (and stored back) by the two lanes that hold it. The tables use sincos_reduced
//    (Cody-Waite reduction + the hardware sin/cos, ~1e-6 absolute), as the reference's
//    decode kernel uses the fast sin/cos intrinsics.
//  * Latency first: the query, the first tile of every wave and the RoPE frequencies
//    are requested before *d_kv_len is read. Split b always covers keys
//    [b * kps, (b + 1) * kps) (kps fixed per launch from max_kv_len), so those loads do
//    not wait for the length; rows past it are masked afterwards.
//  * Each wave walks 32-key tiles of the workgroup's split; the next tile's K/V loads
//    are issued before the current tile's matrix work. Waves merge their (m, l, O)
//    through LDS.
//  * One launch geometry (sized by max_kv_len) serves every step of a captured HIP
//    graph. A single split writes the output itself; otherwise every split writes fp32
//    (o, m, l) partials that a second kernel (one workgroup per query head) merges, or
//    that the o_proj GEMV merges in its prologue (efm_decode_attention_merge_o_proj).
#include "decode_attn_impl.hpp"

#include <mutex>

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace efm {



// MERGE = true: a single split (split_cap == 1) writes the normalised output directly.
// MERGE = false: every split writes its (o, m, l) partial; a consumer merges them
// (decode_merge_kernel, or the o_proj GEMV prologue of efm_decode_attention_merge_o_proj).
// ROTK = true: every key is rotated on read (the cache holds un-rotated K). ROTK = false:
// the cache holds rotated K; with a.fix_last its newest row L - 1 is still un-rotated
// (written by the QKV projection of this step): the two lanes holding it rotate it,
// use it and store it back rotated, so the cache is fully rotated after the call.
template <int HD, int G, bool MERGE, bool ROTK>
// ROTK = false fits 2 workgroups per CU (<= 256 VGPRs); rotate-on-read keeps 1.
__global__ __launch_bounds__(kAttnThreads, ROTK ? 1 : 2) void decode_attn_kernel(DecodeArgs a) {
    constexpr int HALF = HD / 2;
    constexpr int KS = HD / 16;        // MFMA k-steps over head_dim
    constexpr int DT = HD / 32;        // d tiles of O^T
    constexpr int VP = kTileKeys + 8;  // V^T row pitch (bf16)
    static_assert(G <= 32, "group too large");

    __shared__ float2 cs_qk[2][HALF];                                 // cos/sin at q's / key L-1's position
    __shared__ float sfreq[ROTK ? HALF : 1];
    __shared__ float2 cs_off[ROTK ? kTileKeys : 1][HALF + 1];         // cos/sin(k * f_d), k < 32
    __shared__ float2 cs_base[ROTK ? kAttnWaves : 1][HALF];           // cos/sin(tile base * f_d)
    __shared__ __align__(16) bf16_t Vt[kAttnWaves][HD * VP];
    __shared__ float om[kAttnWaves][32], ol[kAttnWaves][32];
    __shared__ float ob[kAttnWaves][G][HD];

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int ql = lane % 32, hh = lane / 32;
    const int kvh = blockIdx.y;
    const int b = blockIdx.x;
    const int kps = a.keys_per_split;   // a multiple of 32 keys (>= 128), fixed per launch
    const int start = b * kps;

    const bf16_t* kbase = a.k + (size_t)kvh * a.k_sh;
    const bf16_t* vbase = a.v + (size_t)kvh * a.v_sh;

    // ---- 1. every load that does not depend on L goes out first: the query, each
    //         wave's first tile (rows below the allocation bound; rows >= L are masked
    //         once L is known) and the RoPE frequencies
    uint4 qraw[KS];
    {
        const bool qv = ql < G;
        const bf16_t* qp = a.q + (size_t)(kvh * G + (qv ? ql : 0)) * a.q_sh + hh * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qraw[ks] = qv ? *reinterpret_cast<const uint4*>(qp + ks * 16) : make_uint4(0, 0, 0, 0);
    }
    uint4 kr[KS], vr[KS];
    auto load_tile = [&](int t, int lim) {
        const int j = start + t * kTileKeys + ql;
        const bool ok = j < lim;
        const bf16_t* kp = kbase + (size_t)(ok ? j : 0) * a.k_sn + hh * 8;
        const bf16_t* vp = vbase + (size_t)(ok ? j : 0) * a.v_sn + hh * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            kr[ks] = ok ? load_stream16(kp + ks * 16) : make_uint4(0, 0, 0, 0);
            vr[ks] = ok ? load_stream16(vp + ks * 16) : make_uint4(0, 0, 0, 0);
        }
    };
    load_tile(wave, min(a.row_bound, start + kps));
    const float freq = (a.rope_q && tid < 2 * HALF) ? a.rope.inv_freq[tid % HALF] : 0.f;

    // ---- 2. the context length and this split's key range [start, end)
    uint32_t L = a.kv_len;
    if (a.d_kv_len != nullptr) L = min(a.d_kv_len[0], a.max_kv_len);
    const int nsplit = (L == 0) ? 1 : (int)((L + kps - 1) / kps);
    if (b >= nsplit) return;
    const int end = min((int)L, start + kps);
    const int ntiles = (end > start) ? (end - start + kTileKeys - 1) / kTileKeys : 0;
    const int rounds = (ntiles + kAttnWaves - 1) / kAttnWaves;

    // ---- 3. RoPE: cos/sin at the query position (threads < HALF) and at the newest
    //         key's position (threads HALF .. 2 HALF - 1), one sincos per thread
    if (a.rope_q && tid < 2 * HALF) {
        const int pos = (int)L - 1 + (tid < HALF ? a.q_pos_off : a.k_pos_off);
        float sn, cs;
        sincos_reduced((float)pos * freq, &sn, &cs);
        cs_qk[tid / HALF][tid % HALF] = make_float2(cs, sn);
        if (ROTK && tid < HALF) sfreq[tid] = freq;
    }
    if (ROTK) {
        __syncthreads();
        for (int i = tid; i < kTileKeys * HALF; i += kAttnThreads) {
            const int kk = i / HALF, d = i % HALF;
            float sn, cs;
            sincos_reduced((float)kk * sfreq[d], &sn, &cs);
            cs_off[kk][d] = make_float2(cs, sn);
        }
    }
    __syncthreads();

    // ---- queries: B operand, lane = head column ql (zero for ql >= G), d = ks*16 + hh*8 + e
    BfPack qf[KS];
    {
        float x[KS][8];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) unpack8(qraw[ks], x[ks]);
        if (a.rope_q) {
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float2 c2 = cs_qk[0][ks * 16 + hh * 8 + e];
                    const float cs = c2.x, sn = c2.y;
                    const float x0 = x[ks][e], x1 = x[ks + KS / 2][e];
                    x[ks][e] = x0 * cs - x1 * sn;
                    x[ks + KS / 2][e] = x1 * cs + x0 * sn;
                }
        }
        const float qscale = kLog2e / sqrtf((float)HD);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[ks][e] *= qscale;
            qf[ks].u = pack8(x[ks]);
        }
    }

    f32x16_t oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[t][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    bf16_t* vt = Vt[wave];
    const int fix_row = (!ROTK && a.rope_q && a.fix_last && L > 0) ? (int)L - 1 : -1;

    for (int r = 0; r < rounds; ++r) {
        const int t = r * kAttnWaves + wave;
        const bool active = t < ntiles;
        const int t0 = start + t * kTileKeys;
        if (ROTK && tid < kAttnWaves * HALF) {
            // base-angle table for the 4 tiles of this round: one sincos per thread
            const int w = tid / HALF, d = tid % HALF;
            const int base = start + (r * kAttnWaves + w) * kTileKeys + a.k_pos_off;
            float sn, cs;
            sincos_reduced((float)base * sfreq[d], &sn, &cs);
            cs_base[w][d] = make_float2(cs, sn);
        }
        // the first tile was loaded before L was known: rows >= end carry P = 0 but
        // may hold any bits (NaN / Inf), so their V is zeroed
        if (r == 0 && t0 + ql >= end) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) vr[ks] = make_uint4(0, 0, 0, 0);
        }
        // V^T into this wave's LDS tile: Vt[d][key]
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint32_t w4[4] = {vr[ks].x, vr[ks].y, vr[ks].z, vr[ks].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d = ks * 16 + hh * 8 + 2 * e;
                vt[d * VP + ql] = (bf16_t)(w4[e] & 0xffffu);
                vt[(d + 1) * VP + ql] = (bf16_t)(w4[e] >> 16);
            }
        }
        __syncthreads();

        // the A operand: keys rotated in registers (angle addition), or as stored
        BfPack kp[KS];
        if (ROTK) {
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks) {
                float x0[8], x1[8];
                unpack8(kr[ks], x0);
                unpack8(kr[ks + KS / 2], x1);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = ks * 16 + hh * 8 + e;
                    const float2 cb = cs_base[wave][d];
                    const float2 co = cs_off[ql][d];
                    const float c = cb.x * co.x - cb.y * co.y;
                    const float sn = cb.y * co.x + cb.x * co.y;
                    const float y0 = x0[e] * c - x1[e] * sn;
                    const float y1 = x1[e] * c + x0[e] * sn;
                    x0[e] = y0;
                    x1[e] = y1;
                }
                kp[ks].u = pack8(x0);
                kp[ks + KS / 2].u = pack8(x1);
            }
        } else {
            // only the split that owns row L - 1 touches it: with kps not a multiple of
            // 4 x 32 keys the idle tiles of a split's last round lie in the next split
            if (active && t0 + ql == fix_row && fix_row < end) {
                // the newest key: rotate at its position and store it back rotated
                bf16_t* kw = const_cast<bf16_t*>(kbase) + (size_t)fix_row * a.k_sn + hh * 8;
#pragma unroll
                for (int ks = 0; ks < KS / 2; ++ks) {
                    float x0[8], x1[8];
                    unpack8(kr[ks], x0);
                    unpack8(kr[ks + KS / 2], x1);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float2 c2 = cs_qk[1][ks * 16 + hh * 8 + e];
                        const float y0 = x0[e] * c2.x - x1[e] * c2.y;
                        const float y1 = x1[e] * c2.x + x0[e] * c2.y;
                        x0[e] = y0;
                        x1[e] = y1;
                    }
                    kr[ks] = pack8(x0);
                    kr[ks + KS / 2] = pack8(x1);
                    *reinterpret_cast<uint4*>(kw + ks * 16) = kr[ks];
                    *reinterpret_cast<uint4*>(kw + (ks + KS / 2) * 16) = kr[ks + KS / 2];
                }
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) kp[ks].u = kr[ks];
        }
        // prefetch the next round's tile while this one is multiplied
        load_tile(t + kAttnWaves, end);

        if (active) {
            f32x16_t s;
#pragma unroll
            for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kp[ks].v, qf[ks].v, s, 0, 0, 0);
            // element e: key = t0 + (e/4)*8 + hh*4 + e%4, head = ql
            float mloc = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int j = t0 + (e / 4) * 8 + hh * 4 + (e % 4);
                s[e] = (j < end) ? s[e] : -INFINITY;
                mloc = fmaxf(mloc, s[e]);
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
            const float m_new = fmaxf(m_run, mloc);  // finite: the tile holds a valid key
            float p[16], psum = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                p[e] = exp2f(s[e] - m_new);
                psum += p[e];
            }
            psum += __shfl_xor(psum, 32, kWave);
            if (r == 0) {
                l_run = psum;   // first tile: nothing accumulated yet to rescale
            } else {
                const float alpha = exp2f(m_run - m_new);
                l_run = l_run * alpha + psum;
#pragma unroll
                for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                    for (int e = 0; e < 16; ++e) oacc[tt][e] *= alpha;
            }
            m_run = m_new;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                BfPack pb;
                pb.u = pack8(&p[8 * kb]);
                const int kcol = kb * 16 + hh * 4;
#pragma unroll
                for (int tt = 0; tt < DT; ++tt) {
                    const bf16_t* vrow = &vt[(tt * 32 + ql) * VP + kcol];
                    BfPack va;
                    const uint2 v0 = *reinterpret_cast<const uint2*>(vrow);
                    const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + 8);
                    va.w[0] = v0.x;
                    va.w[1] = v0.y;
                    va.w[2] = v1.x;
                    va.w[3] = v1.y;
                    oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va.v, pb.v, oacc[tt], 0, 0, 0);
                }
            }
        }
        __syncthreads();  // cs_base / Vt are rewritten next round
    }

    // ---- merge the 4 waves through LDS
    if (hh == 0) {
        om[wave][ql] = m_run;
        ol[wave][ql] = l_run;
    }
    if (ql < G) {
#pragma unroll
        for (int tt = 0; tt < DT; ++tt)
#pragma unroll
            for (int e = 0; e < 16; ++e) ob[wave][ql][tt * 32 + (e / 4) * 8 + hh * 4 + (e % 4)] = oacc[tt][e];
    }
    __syncthreads();
    float* o_part = a.o_part + ((size_t)kvh * a.split_cap + b) * G * HD;
    float* ml_part = a.ml_part + ((size_t)kvh * a.split_cap + b) * G * 2;
    for (int i = tid; i < G * HD; i += kAttnThreads) {
        const int g = i / HD, d = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, om[w][g]);
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float sc = (om[w][g] == -INFINITY) ? 0.f : exp2f(om[w][g] - M);
            num = fmaf(sc, ob[w][g][d], num);
            den = fmaf(sc, ol[w][g], den);
        }
        if (MERGE && nsplit == 1) {
            a.o[(size_t)(kvh * G + g) * HD + d] = (bf16_t)f32_to_bf16(den > 0.f ? num / den : 0.f);
        } else {
            o_part[i] = num;
            if (d == 0) {
                ml_part[g * 2 + 0] = M;
                ml_part[g * 2 + 1] = den;
            }
        }
    }
}

// LDS-staged kernels (head_dim 128, rotated cache); bodies in decode_attn_impl.hpp.
template <int G, bool MERGE>
__global__ __launch_bounds__(kAttnThreads, 2) void decode_attn_lds_kernel(DecodeArgs a) {
    decode_attn_lds_body<G, MERGE, false>(a, blockIdx.x, blockIdx.y, FusedAttnArgs{});
}

template <int G, bool MERGE>
__global__ __launch_bounds__(kWideThreads, 1) void decode_attn_wide_kernel(DecodeArgs a) {
    decode_attn_wide_body<G, MERGE>(a, blockIdx.x, blockIdx.y);
}

// Split merge of efm_attention_decode: kMergeSlices workgroups per query head (blockIdx.y
// takes a quarter of the head's columns, so a workgroup reads a quarter of the partials),
// 256 threads = NCOL float4 columns x NPART split lanes. The partial loads of the first
// chunk are issued before the (m, l) pairs are reduced into the normalised split weights
// w_s = exp2(m_s - M) / sum_s exp2(m_s - M) l_s; each lane accumulates its splits in
// order and the lanes are summed in a fixed order.
constexpr int kMergeSlices = 4;

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void decode_merge_kernel(DecodeArgs a, int G) {
    constexpr int NCOL = HD / 4 / kMergeSlices;
    constexpr int NPART = kAttnThreads / NCOL;
    constexpr int CH = 128 / NPART;  // loads in flight per thread: up to 128 splits in one round trip
    __shared__ float sw[kMaxSplits];
    __shared__ float4 red[NPART][NCOL];
    const int tid = threadIdx.x;
    const int h = blockIdx.x, kvh = h / G, g = h % G;
    const int col = blockIdx.y * NCOL + tid % NCOL, part = tid / NCOL;
    uint32_t L = a.kv_len;
    if (a.d_kv_len != nullptr) L = min(a.d_kv_len[0], a.max_kv_len);
    const int kps = a.keys_per_split;
    const int nsplit = (L == 0) ? 1 : (int)((L + kps - 1) / kps);
    const size_t row0 = (size_t)kvh * a.split_cap * G + g;   // (kvh, split 0, g) in units of rows
    const float* op = a.o_part + row0 * HD + col * 4;
    float4 v[CH];
    auto load_chunk = [&](int s0) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int sp = s0 + k * NPART;
            v[k] = (sp < nsplit) ? *reinterpret_cast<const float4*>(op + (size_t)sp * G * HD)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    load_chunk(part);
    if (tid < kWave) {
        constexpr int kPerLane = kMaxSplits / kWave;
        float ms[kPerLane], ls[kPerLane];
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < kPerLane; ++k) {
            const int sp = tid + k * kWave;
            ms[k] = -INFINITY;
            ls[k] = 0.f;
            if (sp < nsplit) {
                const float2 ml = *reinterpret_cast<const float2*>(a.ml_part + (row0 + (size_t)sp * G) * 2);
                ms[k] = ml.x;
                ls[k] = ml.y;
            }
            M = fmaxf(M, ms[k]);
        }
        M = wave_max(M);
        float den = 0.f;
#pragma unroll
        for (int k = 0; k < kPerLane; ++k) den += (ms[k] == -INFINITY) ? 0.f : exp2f(ms[k] - M) * ls[k];
        den = wave_sum(den);
        const float inv = (den > 0.f) ? 1.f / den : 0.f;
#pragma unroll
        for (int k = 0; k < kPerLane; ++k) {
            const int sp = tid + k * kWave;
            if (sp < nsplit) sw[sp] = (ms[k] == -INFINITY) ? 0.f : exp2f(ms[k] - M) * inv;
        }
    }
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = part; s0 < nsplit; s0 += CH * NPART) {
        if (s0 != part) load_chunk(s0);
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int sp = s0 + k * NPART;
            if (sp < nsplit) {
                const float wk = sw[sp];
                acc.x = fmaf(wk, v[k].x, acc.x);
                acc.y = fmaf(wk, v[k].y, acc.y);
                acc.z = fmaf(wk, v[k].z, acc.z);
                acc.w = fmaf(wk, v[k].w, acc.w);
            }
        }
    }
    const int lc = tid % NCOL;
    red[part][lc] = acc;
    __syncthreads();
    if (part == 0) {
        float4 t = red[0][lc];
#pragma unroll
        for (int p = 1; p < NPART; ++p) {
            t.x += red[p][lc].x;
            t.y += red[p][lc].y;
            t.z += red[p][lc].z;
            t.w += red[p][lc].w;
        }
        bf16_t* o = a.o + (size_t)h * HD + col * 4;
        o[0] = (bf16_t)f32_to_bf16(t.x);
        o[1] = (bf16_t)f32_to_bf16(t.y);
        o[2] = (bf16_t)f32_to_bf16(t.z);
        o[3] = (bf16_t)f32_to_bf16(t.w);
    }
}

// Split geometry: 128 keys (one 32-key tile per wave, one LDS round) per workgroup, so
// that every K/V load of a workgroup is in flight at once, while the grid stays within
// 512 workgroups (two per CU). Longer contexts take splits of up to kWideMaxTiles tiles
// for the 8-wave kernel, one workgroup per CU (kChipCUs on MI355X) and every tile in
// flight at once: at 16k keys and 4 KV heads, 58 splits of 288 keys instead of 65 of 256
// loaded in two serial 128-key rounds (64 splits of 258 keys, every CU busy, measured
// 12.5 us against 12.0). Past that, splits grow in whole 128-key rounds.
// Split b covers keys [b * kps, (b + 1) * kps) whatever the current length, so its first
// loads need not wait for *d_kv_len. Every launch that shares split partials (attention,
// merge, merge + o_proj, the fused front half) takes its plan from here.
constexpr int kKeysPerSplit = 128;
constexpr int kChipCUs = 256;

int decode_keys_per_split(int num_kv_heads, uint32_t max_kv_len) {
    const uint32_t bound = std::max<uint32_t>(max_kv_len, 1u);
    const uint32_t heads = (uint32_t)std::max(1, num_kv_heads);
    const uint32_t by_chip = std::max<uint32_t>(1u, (uint32_t)kMaxSplits / heads);
    if ((bound + kKeysPerSplit - 1) / kKeysPerSplit <= by_chip) return kKeysPerSplit;
    const uint32_t per_cu = std::max<uint32_t>(1u, (uint32_t)kChipCUs / heads);
    const uint32_t wide = kTileKeys * ((bound + kTileKeys * per_cu - 1) / (kTileKeys * per_cu));
    if (wide <= (uint32_t)(kWideMaxTiles * kTileKeys)) return (int)wide;
    const uint32_t rounds = (bound + kKeysPerSplit * by_chip - 1) / (kKeysPerSplit * by_chip);
    return (int)(rounds * kKeysPerSplit);
}

// The LDS-staged kernels load K / V rows with buffer loads: 32-bit byte offsets from the
// head's first row.
static bool decode_lds_offsets_fit(const DecodeArgs& a) {
    return (int64_t)a.row_bound * a.k_sn * 2 < 0x7fffffffLL && (int64_t)a.row_bound * a.v_sn * 2 < 0x7fffffffLL;
}

// The 8-wave kernel takes splits of more than 4 and at most kWideMaxTiles tiles.
static bool decode_wide_fits(const DecodeArgs& a) {
    return a.keys_per_split > kKeysPerSplit && a.keys_per_split <= kWideMaxTiles * kTileKeys;
}

int decode_split_cap(int num_kv_heads, uint32_t max_kv_len) {
    const uint32_t bound = std::max<uint32_t>(max_kv_len, 1u);
    const int kps = decode_keys_per_split(num_kv_heads, bound);
    return (int)((bound + kps - 1) / kps);
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct DecodeWs {
    size_t o_bytes, ml_bytes, cnt_bytes;
    size_t total() const { return o_bytes + ml_bytes + cnt_bytes; }
};

static DecodeWs decode_ws(const efm_attention_ctx* c, uint32_t max_kv_len) {
    const int G = c->num_qo_heads / c->num_kv_heads;
    const int cap = decode_split_cap(c->num_kv_heads, max_kv_len);
    DecodeWs w;
    w.o_bytes = align256((size_t)c->num_kv_heads * cap * G * c->head_dim * sizeof(float));
    w.ml_bytes = align256((size_t)c->num_kv_heads * cap * G * 2 * sizeof(float));
    w.cnt_bytes = align256((size_t)c->num_kv_heads * sizeof(uint32_t));
    return w;
}

int validate_attention_ctx(const efm_attention_ctx* c, const char* who) {
    if (c == nullptr) return set_error(EFM_ERR_INVALID_ARGUMENT, "%s: null context", who);
    if (c->dtype != EFM_DTYPE_BF16)
        return set_error(EFM_ERR_UNSUPPORTED, "%s: only bf16 is supported (dtype %d)", who, c->dtype);
    if (c->head_dim != 64 && c->head_dim != 128)
        return set_error(EFM_ERR_UNSUPPORTED, "%s: head_dim %u not supported (64, 128)", who, c->head_dim);
    if (c->num_kv_heads == 0 || c->num_qo_heads % c->num_kv_heads != 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "%s: num_qo_heads %u not a multiple of num_kv_heads %u", who,
                         c->num_qo_heads, c->num_kv_heads);
    const uint32_t G = c->num_qo_heads / c->num_kv_heads;
    if (!(G == 1 || G == 2 || G == 3 || G == 4 || G == 6 || G == 7 || G == 8))
        return set_error(EFM_ERR_UNSUPPORTED, "%s: GQA group size %u not supported", who, G);
    if (c->pos_encoding != EFM_POS_NONE && c->pos_encoding != EFM_POS_ROPE_LLAMA)
        return set_error(EFM_ERR_UNSUPPORTED, "%s: pos_encoding %d", who, c->pos_encoding);
    if (c->k_already_prerotated < 0 || c->k_already_prerotated > EFM_K_PREROTATED_EXCEPT_NEWEST)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "%s: k_already_prerotated %d", who, c->k_already_prerotated);
    if (c->pos_encoding == EFM_POS_ROPE_LLAMA && (c->rope_theta <= 0.f || c->rope_scale <= 0.f))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "%s: rope_theta/rope_scale must be positive", who);
    const uint32_t strides[6] = {c->q_stride_n, c->q_stride_h, c->k_stride_n, c->k_stride_h, c->kv_stride_n,
                                 c->kv_stride_h};
    for (uint32_t s : strides)
        if (s % 8 != 0) return set_error(EFM_ERR_UNSUPPORTED, "%s: strides must be multiples of 8 elements", who);
    return EFM_OK;
}

size_t decode_workspace_bytes(const efm_attention_ctx* ctx, uint32_t max_kv_len) {
    if (validate_attention_ctx(ctx, "attention_decode_workspace_bytes") != EFM_OK) return 0;
    return decode_ws(ctx, max_kv_len).total();
}

// Offset of the (m, l) partials inside the workspace (after the o partials).
size_t decode_ml_offset(const efm_attention_ctx* ctx, uint32_t max_kv_len) {
    return decode_ws(ctx, max_kv_len).o_bytes;
}


static int decode_launch(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v, void* o,
                         uint32_t kv_len, const uint32_t* d_kv_len, uint32_t max_kv_len, void* workspace,
                         size_t workspace_bytes, bool merge, hipStream_t stream) {
    int rc = validate_attention_ctx(ctx, "attention_decode");
    if (rc) return rc;
    if (q == nullptr || k == nullptr || v == nullptr || (merge && o == nullptr))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "attention_decode: null tensor pointer");
    const uint32_t bound = (d_kv_len != nullptr) ? max_kv_len : kv_len;
    if (d_kv_len != nullptr && max_kv_len == 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "attention_decode: max_kv_len must be > 0 with d_kv_len");
    const DecodeWs ws = decode_ws(ctx, std::max<uint32_t>(bound, 1u));
    if (workspace == nullptr || workspace_bytes < ws.total())
        return set_error(EFM_ERR_WORKSPACE, "attention_decode: workspace of %zu bytes required", ws.total());

    const int hd = (int)ctx->head_dim;
    const int G = (int)(ctx->num_qo_heads / ctx->num_kv_heads);
    DecodeArgs a;
    a.q = static_cast<const bf16_t*>(q);
    a.k = static_cast<const bf16_t*>(k);
    a.v = static_cast<const bf16_t*>(v);
    a.o = static_cast<bf16_t*>(o);
    a.kv_len = kv_len;
    a.d_kv_len = d_kv_len;
    a.max_kv_len = max_kv_len;
    a.num_kv_heads = (int)ctx->num_kv_heads;
    a.q_sn = ctx->q_stride_n ? (int)ctx->q_stride_n : (int)(ctx->num_qo_heads * hd);
    a.q_sh = ctx->q_stride_h ? (int)ctx->q_stride_h : hd;
    a.k_sn = ctx->k_stride_n ? (int)ctx->k_stride_n : (int)(ctx->num_kv_heads * hd);
    a.k_sh = ctx->k_stride_h ? (int)ctx->k_stride_h : hd;
    a.v_sn = ctx->kv_stride_n ? (int)ctx->kv_stride_n : (int)(ctx->num_kv_heads * hd);
    a.v_sh = ctx->kv_stride_h ? (int)ctx->kv_stride_h : hd;
    rope_table_fill(&a.rope, hd, ctx->rope_theta, ctx->rope_scale);
    a.q_pos_off = (int)ctx->q_rope_pos_offset;
    a.k_pos_off = (int)ctx->k_rope_pos_offset;
    a.rope_q = ctx->pos_encoding == EFM_POS_ROPE_LLAMA;
    const bool rotk = a.rope_q && ctx->k_already_prerotated == 0;
    a.fix_last = a.rope_q && ctx->k_already_prerotated == EFM_K_PREROTATED_EXCEPT_NEWEST;
    a.row_bound = (int)std::max<uint32_t>(bound, 1u);
    a.split_cap = decode_split_cap((int)ctx->num_kv_heads, bound);
    a.keys_per_split = decode_keys_per_split((int)ctx->num_kv_heads, bound);
    char* wsb = static_cast<char*>(workspace);
    a.o_part = reinterpret_cast<float*>(wsb);
    a.ml_part = reinterpret_cast<float*>(wsb + ws.o_bytes);
    a.counter = reinterpret_cast<uint32_t*>(wsb + ws.o_bytes + ws.ml_bytes);

    dim3 grid(a.split_cap, ctx->num_kv_heads), block(kAttnThreads);
    // one split: that workgroup writes the output; more: partials, then the merge kernel
    const bool direct = merge && a.split_cap == 1;
    if (hd == 128 && !rotk && decode_lds_offsets_fit(a) && kernel_knob(EFM_KNOB_DECODE_REGISTER) == 0) {
        const bool wide = decode_wide_fits(a);
        const dim3 wblock(kWideThreads);
#define EFM_DEC_LDS_CASE(GV)                                                                                   \
        if (G == GV) {                                                                                         \
            if (wide && direct) hipLaunchKernelGGL((decode_attn_wide_kernel<GV, true>), grid, wblock, 0, stream, a); \
            else if (wide) hipLaunchKernelGGL((decode_attn_wide_kernel<GV, false>), grid, wblock, 0, stream, a);  \
            else if (direct) hipLaunchKernelGGL((decode_attn_lds_kernel<GV, true>), grid, block, 0, stream, a); \
            else hipLaunchKernelGGL((decode_attn_lds_kernel<GV, false>), grid, block, 0, stream, a);           \
            if (merge && !direct)                                                                              \
                hipLaunchKernelGGL((decode_merge_kernel<128>), dim3(ctx->num_qo_heads, kMergeSlices), block, 0, stream, a, G); \
            return check_launch("attention_decode");                                                           \
        }
        EFM_DEC_LDS_CASE(1) EFM_DEC_LDS_CASE(2) EFM_DEC_LDS_CASE(3) EFM_DEC_LDS_CASE(4)
        EFM_DEC_LDS_CASE(6) EFM_DEC_LDS_CASE(7) EFM_DEC_LDS_CASE(8)
#undef EFM_DEC_LDS_CASE
    }
#define EFM_DEC_CASE(HDV, GV)                                                                                  \
    if (hd == HDV && G == GV) {                                                                                \
        if (direct && rotk) hipLaunchKernelGGL((decode_attn_kernel<HDV, GV, true, true>), grid, block, 0, stream, a); \
        else if (direct) hipLaunchKernelGGL((decode_attn_kernel<HDV, GV, true, false>), grid, block, 0, stream, a);   \
        else if (rotk) hipLaunchKernelGGL((decode_attn_kernel<HDV, GV, false, true>), grid, block, 0, stream, a);     \
        else hipLaunchKernelGGL((decode_attn_kernel<HDV, GV, false, false>), grid, block, 0, stream, a);              \
        if (merge && !direct)                                                                                  \
            hipLaunchKernelGGL((decode_merge_kernel<HDV>), dim3(ctx->num_qo_heads, kMergeSlices), block, 0, stream, a, G);    \
        return check_launch("attention_decode");                                                               \
    }
    EFM_DEC_CASE(128, 1) EFM_DEC_CASE(128, 2) EFM_DEC_CASE(128, 3) EFM_DEC_CASE(128, 4)
    EFM_DEC_CASE(128, 6) EFM_DEC_CASE(128, 7) EFM_DEC_CASE(128, 8)
    EFM_DEC_CASE(64, 1) EFM_DEC_CASE(64, 2) EFM_DEC_CASE(64, 3) EFM_DEC_CASE(64, 4)
    EFM_DEC_CASE(64, 6) EFM_DEC_CASE(64, 7) EFM_DEC_CASE(64, 8)
#undef EFM_DEC_CASE
    return set_error(EFM_ERR_UNSUPPORTED, "attention_decode: hd=%d G=%d", hd, G);
}

// ---- no-allocation variant (efm_attention_decode_noalloc) ----
// The split partials live in `scratch`, a file-scope device array that every GPU the
// library runs on holds until the process ends. In host code `scratch` names a host-side
// stand-in, never the device memory: the device address comes from hipGetSymbolAddress,
// fetched once per device (with that device current) on the entry point's first call
// there, and only that address is passed to kernels. Nothing in the partials needs to
// start at zero: every split writes its own slots before the merge reads them.
constexpr size_t kNoAllocScratchBytes = EFM_ATTENTION_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kNoAllocMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kNoAllocMaxDevices];

static int noalloc_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(EFM_ERR_DEVICE, "attention_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kNoAllocMaxDevices)
        return set_error(EFM_ERR_UNSUPPORTED, "attention_decode_noalloc: device %d beyond %d", dev, kNoAllocMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return set_error(EFM_ERR_DEVICE, "attention_decode_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return EFM_OK;
}

static int decode_noalloc(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v, void* o,
                          uint32_t kv_len, const uint32_t* d_kv_len, uint32_t max_kv_len, hipStream_t stream) {
    int rc = validate_attention_ctx(ctx, "attention_decode_noalloc");
    if (rc) return rc;
    const uint32_t bound = (d_kv_len != nullptr) ? max_kv_len : kv_len;
    const size_t need = decode_ws(ctx, std::max<uint32_t>(bound, 1u)).total();
    if (need > kNoAllocScratchBytes)
        return set_error(EFM_ERR_UNSUPPORTED,
                         "attention_decode_noalloc: this shape needs %zu bytes of split scratch; the library holds %zu "
                         "(use efm_attention_decode with a workspace)", need, kNoAllocScratchBytes);
    void* ptr = nullptr;
    rc = noalloc_scratch(&ptr);
    if (rc) return rc;
    return decode_launch(ctx, q, k, v, o, kv_len, d_kv_len, max_kv_len, ptr, kNoAllocScratchBytes, true, stream);
}

}  // namespace efm

extern "C" int efm_attention_decode_noalloc(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v,
                                            void* o, uint32_t kv_len, const uint32_t* d_kv_len, uint32_t max_kv_len,
                                            hipStream_t stream) {
    return efm::decode_noalloc(ctx, q, k, v, o, kv_len, d_kv_len, max_kv_len, stream);
}

extern "C" size_t efm_attention_decode_workspace_bytes(const efm_attention_ctx* ctx, uint32_t max_kv_len) {
    return efm::decode_workspace_bytes(ctx, max_kv_len);
}

extern "C" int efm_attention_decode(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v,
                                    void* o, uint32_t kv_len, const uint32_t* d_kv_len, uint32_t max_kv_len,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return efm::decode_launch(ctx, q, k, v, o, kv_len, d_kv_len, max_kv_len, workspace, workspace_bytes, true,
                              stream);
}

extern "C" int efm_decode_attention_partials(const efm_attention_ctx* ctx, const void* q, const void* k,
                                             const void* v, const uint32_t* d_kv_len, uint32_t max_kv_len,
                                             void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (d_kv_len == nullptr) return efm::set_error(EFM_ERR_INVALID_ARGUMENT, "attention_partials: d_kv_len is required");
    return efm::decode_launch(ctx, q, k, v, nullptr, 0, d_kv_len, max_kv_len, workspace, workspace_bytes, false,
                              stream);
}

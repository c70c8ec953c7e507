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
    const int kps = a.keys_per_split;   // >= 128 keys, fixed per launch
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

template <int G, bool MERGE, bool ROTK>
__global__ __launch_bounds__(kWideThreads, 1) void decode_attn_wide_kernel(DecodeArgs a) {
    decode_attn_wide_body<G, MERGE, ROTK>(a, blockIdx.x, blockIdx.y);
}

// ---- one-wave splits (short and mid contexts) ----
// A launch of few workgroups is bound by what each workgroup loads and by its serial
// chain, not by the chip's bandwidth: an MI355X graph node costs 1.6 us with nothing in
// it, 1.8 us when each workgroup loads 8 KB of cold memory, 2.2 us at 16 KB and 3.0 us at
// 64 KB. So short contexts take one wave64 per workgroup and one split of T (1 or 2)
// 32-key tiles: every K / V byte of the split is requested up front (buffer loads straight
// into LDS), the wave computes S^T = K . Q^T and O^T = V^T . P^T on the matrix cores with
// an online softmax over its tiles, and writes one partial (or, with one split, the
// output). No barrier and no wave merge: the splits meet in decode_merge_kernel.
//
// LDS rows are 16-byte chunks, swizzled so that the K-operand reads (ds_read_b128, rows
// of 16 lanes at one chunk) and the V^T reads (ds_read_b64_tr_b16, 4 rows x 32 columns
// per 32 lanes) hit distinct banks of gfx950's 64: head_dim 128 (256-byte rows) uses the
// attn_pipe layouts; head_dim 64 (128-byte rows) puts chunk c of K row r at
// c ^ ((r >> 1) & 7) and of V row r at c ^ (((r >> 1) & 1) << 2).
constexpr int kTileMaxT = 2;       // tiles per split
constexpr int kTileMaxWG = 256;    // workgroups of a launch (one per CU)

template <int HD>
struct TileLayout {
    static constexpr int ROW = HD * 2;            // bytes per K / V row
    static constexpr int CPR = ROW / 16;          // 16-byte chunks per row
    static constexpr int TB = kTileKeys * ROW;    // bytes of K (or V) per tile
    static constexpr int RPL = 1024 / ROW;        // rows per 1 KB wave load
    static constexpr int LPK = TB / 1024;         // wave loads per K (or V) tile
    __device__ static int kswz(int r) { return HD == 128 ? (r & 15) : ((r >> 1) & 7); }
    __device__ static int vswz(int r) { return HD == 128 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2); }
    __device__ static uint32_t k_off(int r, int c) { return (uint32_t)(r * ROW + ((c ^ kswz(r)) << 4)); }
    __device__ static uint32_t v_off(int r, int c) { return (uint32_t)(r * ROW + ((c ^ vswz(r)) << 4)); }
    // V^T operand of d tile tt: lane j = 4 e + q of 16-lane group g reads key 4 (g / 2) + e,
    // d = 32 tt + 16 (g % 2) + 4 q (attn_pipe.hpp describes the transposing read)
    __device__ static uint32_t v_tr_lane_off(int lane, int tt) {
        const int g = lane >> 4, j = lane & 15;
        const int r = (g >> 1) * 4 + (j >> 2);
        const int d = tt * 32 + 16 * (g & 1) + 4 * (j & 3);
        return v_off(r, d >> 3) + (uint32_t)((d & 7) << 1);
    }
};

// ROTK = true: every key is rotated on read at its position (the reference's un-rotated
// cache); its cos / sin are computed while the tiles load. ROTK = false: keys are used as
// stored (rotated cache, or no RoPE), and with a.fix_last row L - 1 is rotated, used and
// stored back by the lane that holds it.
template <int HD, int G, int T, bool ROTK>
__global__ __launch_bounds__(kWave) void decode_attn_tile_kernel(DecodeArgs a) {
    using Lay = TileLayout<HD>;
    constexpr int HALF = HD / 2, KS = HD / 16, DT = HD / 32;
    constexpr int TB = Lay::TB, LPK = Lay::LPK;
    static_assert(G <= 32 && T >= 1 && T <= kTileMaxT, "tile kernel shape");
    __shared__ __align__(1024) unsigned char smem[T * 2 * TB];   // per tile: K | V
    __shared__ __align__(16) float2 cs_qk[2][HALF];              // cos/sin at q's / key L-1's position
    __shared__ float sfreq[ROTK ? HALF : 1];

    const int lane = threadIdx.x, ql = lane % 32, hh = lane / 32;
    const int kvh = blockIdx.y, b = blockIdx.x;
    const int kps = a.keys_per_split;   // T * 32 (host plan)
    const int start = b * kps;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);

    // ---- 1. loads that do not depend on L: the query fragments (B operand: lane = head
    //         column ql, d = 16 ks + 8 hh + e), the RoPE frequency, every tile of the split
    // (lanes past the group read head G - 1 and zero it below: a load under a lane
    // condition becomes a branch, after which the compiler waits for it before the tiles)
    uint4 qraw[KS];
    {
        const bf16_t* qp = a.q + (size_t)(kvh * G + min(ql, G - 1)) * a.q_sh + hh * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qraw[ks] = *reinterpret_cast<const uint4*>(qp + ks * 16);
    }
    const float freq = (a.rope_q && lane < HALF) ? a.rope.inv_freq[lane] : 0.f;
    const int q_pos_off = __builtin_amdgcn_readfirstlane(a.q_pos_off);
    const int k_pos_off = __builtin_amdgcn_readfirstlane(a.k_pos_off);
    {
        const int k_sn = __builtin_amdgcn_readfirstlane(a.k_sn), v_sn = __builtin_amdgcn_readfirstlane(a.v_sn);
        const int lim = min(a.row_bound, start + kps) - 1;   // last row this split may read
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<bf16_t*>(a.k + (size_t)kvh * a.k_sh), (short)0,
            __builtin_amdgcn_readfirstlane(a.row_bound * k_sn * 2), 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<bf16_t*>(a.v + (size_t)kvh * a.v_sh), (short)0,
            __builtin_amdgcn_readfirstlane(a.row_bound * v_sn * 2), 0x00020000);
        const int rin = lane / Lay::CPR, slot = lane % Lay::CPR;
#pragma unroll
        for (int t = 0; t < T; ++t) {
#pragma unroll
            for (int q = 0; q < 2 * LPK; ++q) {
                const bool isv = q >= LPK;
                const int row = (q % LPK) * Lay::RPL + rin;   // row of the tile
                const int key = start + t * kTileKeys + row;
                const int c = slot ^ (isv ? Lay::vswz(row) : Lay::kswz(row));
                // rows past the split's last readable row read nothing (zeros)
                const uint32_t off = (key <= lim) ? (uint32_t)(key * (isv ? v_sn : k_sn) + c * 8) * 2u : kWloadSkipAttn;
                wide_lds_load(isv ? rv : rk, lds0 + (uint32_t)(t * 2 * TB + q * 1024), off);
            }
        }
    }

    // ---- 2. the context length and this split's key range [start, end)
    const uint32_t L = decode_len(a);
    const int nsplit = (L == 0) ? 1 : (int)((L + kps - 1) / kps);
    if (b >= nsplit) {
        attn_pipe::vm_wait<0>();   // no LDS write may outlive the workgroup
        return;
    }
    const int end = min((int)L, start + kps);

    // ---- 3. RoPE at the query position and at the newest key's position; the queries
    //         rotated in registers (pair d, d + HD/2 sits in chunks ks, ks + KS/2 of the
    //         same lane) and scaled by log2(e) / sqrt(hd) into the MFMA operand
    if (a.rope_q) {
#pragma unroll
        for (int i = lane; i < 2 * HALF; i += kWave) {
            const float f = __shfl(freq, i % HALF, kWave);
            const int pos = (int)L - 1 + (i < HALF ? q_pos_off : k_pos_off);
            float sn, cs;
            sincos_reduced((float)pos * f, &sn, &cs);
            cs_qk[i / HALF][i % HALF] = make_float2(cs, sn);
        }
        if (ROTK && lane < HALF) sfreq[lane] = freq;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // one wave: LDS order is issue order
    }
    bf16x8_t qf[KS];
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
                    const float x0 = x[ks][e], x1 = x[ks + KS / 2][e];
                    x[ks][e] = x0 * c2.x - x1 * c2.y;
                    x[ks + KS / 2][e] = x1 * c2.x + x0 * c2.y;
                }
        }
        const float qscale = kLog2e / sqrtf((float)HD);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[ks][e] *= qscale;
            BfPack pk;
            pk.u = pack8(x[ks]);
            if (ql >= G) pk.u = make_uint4(0, 0, 0, 0);   // head columns past the group
            qf[ks] = pk.v;
        }
    }
    const int fix_row = (!ROTK && a.rope_q && a.fix_last && L > 0) ? (int)L - 1 : -1;
    const bf16_t* kbase = a.k + (size_t)kvh * a.k_sh;

    f32x16_t oacc[DT];
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[tt][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    typedef short s4_t __attribute__((ext_vector_type(4)));

#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int t0 = start + t * kTileKeys;
        // ROTK: cos / sin of this lane's key (t0 + ql) for its d = 16 ks + 8 hh + e, ks <
        // KS / 2, computed before the wait so that they overlap the tile loads
        float2 ck[ROTK ? KS / 2 : 1][8];
        if (ROTK) {
            const float pos = (float)(t0 + ql + k_pos_off);
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float sn, cs;
                    sincos_reduced(pos * sfreq[ks * 16 + hh * 8 + e], &sn, &cs);
                    ck[ks][e] = make_float2(cs, sn);
                }
        }
        if (t == 0 && T > 1) attn_pipe::vm_wait<(T - 1) * 2 * LPK>();   // tile 0 landed
        else attn_pipe::vm_wait<0>();
        asm volatile("" ::: "memory");
        if (t0 >= end) continue;
        unsigned char* tile = smem + t * 2 * TB;
        const uint32_t sb = lds0 + (uint32_t)(t * 2 * TB);
        if (t0 + kTileKeys > end) {
            // zero the V rows past the length (P is 0 there, but the rows may hold NaN)
            for (int x = lane; x < (t0 + kTileKeys - end) * Lay::CPR; x += kWave) {
                const int row = end - t0 + x / Lay::CPR;
                *reinterpret_cast<uint4*>(tile + TB + row * Lay::ROW + (x % Lay::CPR) * 16) = make_uint4(0, 0, 0, 0);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        bf16x8_t kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) attn_pipe::read_b128<0>(kf[ks], sb + Lay::k_off(ql, ks * 2 + hh));
        s4_t vf[2][DT][2];
        auto read_v = [&](auto kbc) {
            constexpr int kb = decltype(kbc)::value;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) {
                const uint32_t va = sb + (uint32_t)TB + Lay::v_tr_lane_off(lane, tt);
                attn_pipe::read_tr16<(kb * 16) * Lay::ROW>(vf[kb][tt][0], va);
                attn_pipe::read_tr16<(kb * 16 + 8) * Lay::ROW>(vf[kb][tt][1], va);
            }
        };
        read_v(std::integral_constant<int, 0>{});
        asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(2 * DT) : "memory");   // the K reads (issued first) are done
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kf[ks]));
        if (ROTK || (t0 + ql == fix_row && fix_row < end)) {
            // rotate this lane's key: every key (ROTK) or the newest one, which is then
            // stored back rotated
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks) {
                BfPack u0, u1;
                u0.v = kf[ks];
                u1.v = kf[ks + KS / 2];
                float x0[8], x1[8];
                unpack8(u0.u, x0);
                unpack8(u1.u, x1);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float2 c2 = ROTK ? ck[ks][e] : cs_qk[1][ks * 16 + hh * 8 + e];
                    const float y0 = x0[e] * c2.x - x1[e] * c2.y;
                    const float y1 = x1[e] * c2.x + x0[e] * c2.y;
                    x0[e] = y0;
                    x1[e] = y1;
                }
                u0.u = pack8(x0);
                u1.u = pack8(x1);
                kf[ks] = u0.v;
                kf[ks + KS / 2] = u1.v;
                if (!ROTK) {
                    bf16_t* kw = const_cast<bf16_t*>(kbase) + (size_t)fix_row * a.k_sn + hh * 8;
                    *reinterpret_cast<uint4*>(kw + ks * 16) = u0.u;
                    *reinterpret_cast<uint4*>(kw + (ks + KS / 2) * 16) = u1.u;
                }
            }
        }
        f32x16_t s = {};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], s, 0, 0, 0);
        read_v(std::integral_constant<int, 1>{});
        // element e: key = t0 + (e/4)*8 + hh*4 + e%4, head = ql
        if (t0 + kTileKeys > end) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int j = t0 + (e / 4) * 8 + hh * 4 + (e % 4);
                s[e] = (j < end) ? s[e] : -INFINITY;
            }
        }
        float mloc = fmaxf(s[0], s[1]);
#pragma unroll
        for (int e = 2; e < 16; ++e) mloc = fmaxf(mloc, s[e]);
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc), __float_as_uint(mloc), false, false);
            mloc = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        const float m_new = fmaxf(m_run, mloc);   // finite: the tile holds a valid key
        float p[16], psum = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            p[e] = __builtin_amdgcn_exp2f(s[e] - m_new);
            psum += p[e];
        }
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(psum), __float_as_uint(psum), false, false);
            psum = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        if (t == 0) {
            l_run = psum;
        } else {
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run = l_run * alpha + psum;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[tt][e] *= alpha;
        }
        m_run = m_new;
        BfPack pb[2];
        pb[0].u = pack8(&p[0]);
        pb[1].u = pack8(&p[8]);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) {
                if (tt == 0) {
                    if (kb == 0) asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(2 * DT) : "memory");
                    else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                }
                asm volatile("" : "+v"(vf[kb][tt][0]), "+v"(vf[kb][tt][1]));
                union {
                    s4_t h[2];
                    bf16x8_t v;
                } vv;
                vv.h[0] = vf[kb][tt][0];   // A slots 0-3: keys 16 kb + 4 hh + 0..3
                vv.h[1] = vf[kb][tt][1];   // A slots 4-7: keys 16 kb + 8 + 4 hh + 0..3
                oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vv.v, pb[kb].v, oacc[tt], 0, 0, 0);
            }
    }

    // ---- 4. the split's partial (o unnormalised, m, l), or with one split the output;
    //         lane (ql, hh) holds d = 32 tt + 8 eb + 4 hh + 0..3 of head ql
    if (ql < G) {
        if (a.split_cap == 1 && a.o != nullptr) {
            const float inv = (l_run > 0.f) ? 1.f / l_run : 0.f;
            bf16_t* o = a.o + (size_t)(kvh * G + ql) * HD;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                for (int eb = 0; eb < 4; ++eb) {
                    uint2 pk;
                    pk.x = pack_bf16x2(oacc[tt][eb * 4 + 0] * inv, oacc[tt][eb * 4 + 1] * inv);
                    pk.y = pack_bf16x2(oacc[tt][eb * 4 + 2] * inv, oacc[tt][eb * 4 + 3] * inv);
                    *reinterpret_cast<uint2*>(o + tt * 32 + eb * 8 + hh * 4) = pk;
                }
        } else {
            float* op = a.o_part + (((size_t)kvh * a.split_cap + b) * G + ql) * HD;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                for (int eb = 0; eb < 4; ++eb)
                    *reinterpret_cast<float4*>(op + tt * 32 + eb * 8 + hh * 4) =
                        make_float4(oacc[tt][eb * 4 + 0], oacc[tt][eb * 4 + 1], oacc[tt][eb * 4 + 2],
                                    oacc[tt][eb * 4 + 3]);
            if (hh == 0)
                *reinterpret_cast<float2*>(a.ml_part + (((size_t)kvh * a.split_cap + b) * G + ql) * 2) =
                    make_float2(m_run, l_run);
        }
    }
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
        M = wave_max_uniform(M);
        float den = 0.f;
#pragma unroll
        for (int k = 0; k < kPerLane; ++k) den += (ms[k] == -INFINITY) ? 0.f : exp2f(ms[k] - M) * ls[k];
        den = wave_total(den);
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
    // one 8-wave workgroup per CU in whole 32-key tiles: a tile's 16 load requests take
    // the address unit's time whether or not its rows exist, so whole tiles on fewer CUs
    // beat partial ones on every CU (16512 rows x 4 KV heads: 58 splits of 288 rows
    // 11.0 us; 60 of 276 11.4; 64 of 260 11.6)
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

// One-wave split plan of efm_attention_decode (decode_attn_tile_kernel): splits of T
// tiles, the fewest T <= kTileMaxT that keeps the launch within kTileMaxWG workgroups over
// all KV heads; 0 when none does (the 4- and 8-wave plans above take those lengths). The
// partials entry points keep the 4-wave plan: their consumers (the o_proj merge, the
// fused front half) merge at most a few 128-key splits.
static int tile_keys_per_split(int num_kv_heads, uint32_t max_kv_len) {
    const uint32_t tiles = (std::max<uint32_t>(max_kv_len, 1u) + kTileKeys - 1) / kTileKeys;
    const uint32_t heads = (uint32_t)std::max(1, num_kv_heads);
    for (int t = 1; t <= kTileMaxT; ++t)
        if ((tiles + t - 1) / t * heads <= (uint32_t)kTileMaxWG) return t * kTileKeys;
    return 0;
}

// Partials plan (efm_decode_attention_partials, read back by
// efm_decode_attention_merge_o_proj): one-wave splits of 1 or 2 tiles (the fewest tiles
// that keep the splits within what the o_proj merge prologue holds for this query width)
// where they fit: more workgroups than the 4-wave plan and no merge across waves
// (head_dim 64, 14 / 2 heads: partials + merge + o_proj 7.1-8.8 us against 9.4-10.6 up to
// 1.5k rows); longer caches take the plan above.
DecodePartialsPlan decode_partials_plan(const efm_attention_ctx* c, uint32_t max_kv_len) {
    const uint32_t bound = std::max<uint32_t>(max_kv_len, 1u);
    const int Hkv = std::max(1, (int)c->num_kv_heads), hd = (int)c->head_dim;
    DecodePartialsPlan p;
    p.keys_per_split = decode_keys_per_split(Hkv, bound);
    p.split_cap = (int)((bound + p.keys_per_split - 1) / p.keys_per_split);
    p.tile = false;
    const int64_t k_sn = c->k_stride_n ? (int64_t)c->k_stride_n : (int64_t)Hkv * hd;
    const int64_t v_sn = c->kv_stride_n ? (int64_t)c->kv_stride_n : (int64_t)Hkv * hd;
    const bool offsets_fit = (int64_t)bound * k_sn * 2 < 0x7fffffffLL && (int64_t)bound * v_sn * 2 < 0x7fffffffLL;
    const int ms = merge_max_splits((int64_t)c->num_qo_heads * hd);
    if (ms == 0 || !offsets_fit || kernel_knob(EFM_KNOB_DECODE_TILE) != 0) return p;
    // head_dim 128 takes one-tile splits only, at most kMergeMaxSplits of them: two-tile
    // splits load 32 KB through one wave and were measured slower than the 4-wave plan
    // (12 / 2 heads at 768 rows: 10.4 against 9.5 us for partials + merge + o_proj)
    const uint32_t tiles = (bound + kTileKeys - 1) / kTileKeys;
    const int max_t = (hd == 64) ? kTileMaxT : 1;
    const int max_cap = (hd == 64) ? ms : std::min(ms, kMergeMaxSplits);
    for (int t = 1; t <= max_t; ++t) {
        const uint32_t cap = (tiles + t - 1) / t;
        if (cap <= (uint32_t)max_cap && cap * (uint32_t)Hkv <= (uint32_t)kTileMaxWG) {
            p.keys_per_split = t * kTileKeys;
            p.split_cap = (int)cap;
            p.tile = true;
            return p;
        }
    }
    return p;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct DecodeWs {
    size_t o_bytes, ml_bytes, cnt_bytes;
    size_t total() const { return o_bytes + ml_bytes + cnt_bytes; }
};

static DecodeWs decode_ws(const efm_attention_ctx* c, uint32_t max_kv_len) {
    const int G = c->num_qo_heads / c->num_kv_heads;
    const uint32_t bound = std::max<uint32_t>(max_kv_len, 1u);
    int cap = decode_split_cap(c->num_kv_heads, bound);
    if (const int tk = tile_keys_per_split((int)c->num_kv_heads, bound))
        cap = std::max(cap, (int)((bound + tk - 1) / tk));
    cap = std::max(cap, decode_partials_plan(c, bound).split_cap);
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

    // Merged calls on short and mid contexts: one-wave splits, then the merge kernel (or,
    // with one split, the output written by that wave). Partials calls take them where
    // their plan says so, and end with the partials.
    const DecodePartialsPlan pp = merge ? DecodePartialsPlan{0, 0, false} : decode_partials_plan(ctx, bound);
    const int tile_kps = merge ? tile_keys_per_split((int)ctx->num_kv_heads, a.row_bound) : (pp.tile ? pp.keys_per_split : 0);
    if (tile_kps > 0 && decode_lds_offsets_fit(a) && kernel_knob(EFM_KNOB_DECODE_TILE) == 0) {
        a.keys_per_split = tile_kps;
        a.split_cap = (a.row_bound + tile_kps - 1) / tile_kps;
        const dim3 tgrid(a.split_cap, ctx->num_kv_heads), tblock(kWave);
        const int T = tile_kps / kTileKeys;
#define EFM_DEC_TILE_CASE(HDV, GV)                                                                             \
        if (hd == HDV && G == GV) {                                                                            \
            if (rotk && T == 1) hipLaunchKernelGGL((decode_attn_tile_kernel<HDV, GV, 1, true>), tgrid, tblock, 0, stream, a);  \
            else if (rotk) hipLaunchKernelGGL((decode_attn_tile_kernel<HDV, GV, 2, true>), tgrid, tblock, 0, stream, a);      \
            else if (T == 1) hipLaunchKernelGGL((decode_attn_tile_kernel<HDV, GV, 1, false>), tgrid, tblock, 0, stream, a);  \
            else hipLaunchKernelGGL((decode_attn_tile_kernel<HDV, GV, 2, false>), tgrid, tblock, 0, stream, a);              \
            if (merge && a.split_cap > 1)                                                                      \
                hipLaunchKernelGGL((decode_merge_kernel<HDV>), dim3(ctx->num_qo_heads, kMergeSlices), dim3(kAttnThreads), 0, \
                                   stream, a, G);                                                              \
            return check_launch("attention_decode");                                                           \
        }
        EFM_DEC_TILE_CASE(128, 1) EFM_DEC_TILE_CASE(128, 2) EFM_DEC_TILE_CASE(128, 3) EFM_DEC_TILE_CASE(128, 4)
        EFM_DEC_TILE_CASE(128, 6) EFM_DEC_TILE_CASE(128, 7) EFM_DEC_TILE_CASE(128, 8)
        EFM_DEC_TILE_CASE(64, 1) EFM_DEC_TILE_CASE(64, 2) EFM_DEC_TILE_CASE(64, 3) EFM_DEC_TILE_CASE(64, 4)
        EFM_DEC_TILE_CASE(64, 6) EFM_DEC_TILE_CASE(64, 7) EFM_DEC_TILE_CASE(64, 8)
#undef EFM_DEC_TILE_CASE
        return set_error(EFM_ERR_UNSUPPORTED, "attention_decode: hd=%d G=%d", hd, G);
    }

    dim3 grid(a.split_cap, ctx->num_kv_heads), block(kAttnThreads);
    // one split: that workgroup writes the output; more: partials, then the merge kernel
    const bool direct = merge && a.split_cap == 1;
    // The reference's un-rotated cache (rotk) takes the 8-wave kernel where its splits fit
    // it, else the register-staged kernel; the 4-wave LDS kernel reads rotated keys only.
    const bool wide = decode_wide_fits(a);
    if (hd == 128 && (!rotk || wide) && decode_lds_offsets_fit(a) && kernel_knob(EFM_KNOB_DECODE_REGISTER) == 0) {
        const dim3 wblock(kWideThreads);
#define EFM_DEC_LDS_CASE(GV)                                                                                   \
        if (G == GV) {                                                                                         \
            if (wide && direct && rotk) hipLaunchKernelGGL((decode_attn_wide_kernel<GV, true, true>), grid, wblock, 0, stream, a); \
            else if (wide && rotk) hipLaunchKernelGGL((decode_attn_wide_kernel<GV, false, true>), grid, wblock, 0, stream, a); \
            else if (wide && direct) hipLaunchKernelGGL((decode_attn_wide_kernel<GV, true, false>), grid, wblock, 0, stream, a); \
            else if (wide) hipLaunchKernelGGL((decode_attn_wide_kernel<GV, false, false>), grid, wblock, 0, stream, a); \
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
// fetched once per device (with that device current) by efm_init, or by the entry point's
// first call on that device when it is not being captured into a graph, and only that
// address is passed to kernels. Nothing in the partials needs to start at zero: every
// split writes its own slots before the merge reads them.
constexpr size_t kNoAllocScratchBytes = EFM_ATTENTION_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kNoAllocMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kNoAllocMaxDevices];

// capture_stream: the call's stream; a first lookup while that stream is being captured
// is refused (the runtime call may load code objects), so capture needs efm_init first.
static int noalloc_scratch(void** out, hipStream_t capture_stream, bool check_capture) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(EFM_ERR_DEVICE, "attention_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kNoAllocMaxDevices)
        return set_error(EFM_ERR_UNSUPPORTED, "attention_decode_noalloc: device %d beyond %d", dev, kNoAllocMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_dev[dev] == nullptr) {
        if (check_capture) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(capture_stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
                return set_error(EFM_ERR_INVALID_ARGUMENT,
                                 "attention_decode_noalloc: first call on device %d inside a graph capture; call "
                                 "efm_init on this device before capturing", dev);
        }
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
    rc = noalloc_scratch(&ptr, stream, true);
    if (rc) return rc;
    return decode_launch(ctx, q, k, v, o, kv_len, d_kv_len, max_kv_len, ptr, kNoAllocScratchBytes, true, stream);
}

}  // namespace efm

extern "C" int efm_init(void) {
    void* ptr = nullptr;
    return efm::noalloc_scratch(&ptr, nullptr, false);
}

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

// Batch-1 decode GEMV family for gfx950.
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
//    into the KV-cache slot, SwiGLU over paired up/gate rows, and greedy top-1 with a
//    last-workgroup grid reduction (no second launch, self-resetting counter).
#include "common.hpp"

#include <algorithm>

namespace efm {

enum { PRO_PLAIN = 0, PRO_NORM = 1, PRO_ADD_NORM = 2, PRO_ATTN_MERGE = 3 };
enum { EPI_BF16 = 0, EPI_F32 = 1, EPI_QKV = 2, EPI_SWIGLU = 3, EPI_TOP1 = 4 };

// Weight-stream load used by the GEMV main loop (non-temporal: weights are read once
// per decode step and must not evict the activation working set).
#ifndef EFM_WEIGHT_LOAD
#define EFM_WEIGHT_LOAD load_stream16
#endif

constexpr int kGemvThreads = 256;
constexpr int kNJMax = 6;
constexpr int kTop1MaxGridDev = 2048;  // max workgroups of a top-1 launch (partials slots)        // max 16-byte chunks per lane per row per segment
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
};

constexpr int kMergeMaxSplits = 8;
constexpr int kMergeMaxHeads = 64;

template <int PRO>
__device__ __forceinline__ void gemv_prologue(const GemvArgs& a, bf16_t* xs, float* red) {
    const int C = a.K >> 3;
    const uint4* x4 = reinterpret_cast<const uint4*>(a.x);
    uint4* xs4 = reinterpret_cast<uint4*>(xs);
    if (PRO == PRO_PLAIN) {
        for (int c = threadIdx.x; c < C; c += kGemvThreads) xs4[c] = x4[c];
        return;
    }
    if (PRO == PRO_ATTN_MERGE && a.K <= 2 * 4 * kGemvThreads && a.split_cap <= kMergeMaxSplits) {
        // Same merge as below with every load issued up front (the cache length, each head's
        // split statistics and this thread's partial outputs for every split slot; slots
        // beyond the live split count get weight 0): one memory round trip instead of two.
        __shared__ float swf[kMergeMaxHeads * kMergeMaxSplits];
        const int hd = a.head_dim, G = a.group, cap = a.split_cap;
        const int Hq = a.K / hd;
        const uint32_t L = min(a.attn_len[0], a.attn_max_len);
        float2 ml[kMergeMaxSplits];
        if ((int)threadIdx.x < Hq) {
            const int h = threadIdx.x;
#pragma unroll
            for (int j = 0; j < kMergeMaxSplits; ++j) {
                const size_t idx = ((size_t)(h / G) * cap + j) * G + (h % G);
                ml[j] = (j < cap) ? *reinterpret_cast<const float2*>(a.ml_part + idx * 2) : make_float2(0.f, 0.f);
            }
        }
        float4 op[2][kMergeMaxSplits];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int c = threadIdx.x + q * kGemvThreads;
            if (c < (a.K >> 2)) {
                const int n0 = c * 4, h = n0 / hd, d0 = n0 % hd;
                const float* base = a.o_part + ((size_t)(h / G) * cap * G + (h % G)) * hd + d0;
#pragma unroll
                for (int j = 0; j < kMergeMaxSplits; ++j)
                    op[q][j] = (j < cap) ? *reinterpret_cast<const float4*>(base + (size_t)j * G * hd)
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        const int kps = a.keys_per_split;
        const int nsplit = (L == 0) ? 1 : (int)((L + kps - 1) / kps);
        if ((int)threadIdx.x < Hq) {
            const int h = threadIdx.x;
            float M = -INFINITY;
#pragma unroll
            for (int j = 0; j < kMergeMaxSplits; ++j)
                if (j < nsplit) M = fmaxf(M, ml[j].x);
            float den = 0.f, w[kMergeMaxSplits];
#pragma unroll
            for (int j = 0; j < kMergeMaxSplits; ++j) {
                if (j < nsplit) {
                    w[j] = (ml[j].x == -INFINITY) ? 0.f : exp2f(ml[j].x - M);
                    den = fmaf(w[j], ml[j].y, den);
                }
            }
            const float inv = (den > 0.f) ? 1.f / den : 0.f;
#pragma unroll
            for (int j = 0; j < kMergeMaxSplits; ++j)
                if (j < nsplit) swf[h * nsplit + j] = w[j] * inv;
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int c = threadIdx.x + q * kGemvThreads;
            if (c < (a.K >> 2)) {
                const int h = (c * 4) / hd;
                float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < kMergeMaxSplits; ++j) {
                    if (j < nsplit) {
                        const float wj = swf[h * nsplit + j];
                        acc[0] = fmaf(wj, op[q][j].x, acc[0]);
                        acc[1] = fmaf(wj, op[q][j].y, acc[1]);
                        acc[2] = fmaf(wj, op[q][j].z, acc[2]);
                        acc[3] = fmaf(wj, op[q][j].w, acc[3]);
                    }
                }
                uint2 pk;
                pk.x = pack_bf16x2(acc[0], acc[1]);
                pk.y = pack_bf16x2(acc[2], acc[3]);
                reinterpret_cast<uint2*>(xs)[c] = pk;
            }
        }
        return;
    }
    if (PRO == PRO_ATTN_MERGE) {
        // x[h*hd + d] = bf16( sum_s w[h][s] * o_part[kvh][s][g][d] ),
        // w[h][s] = exp2(m_s - M) / sum_s exp2(m_s - M) l_s  (log-sum-exp merge of the splits)
        __shared__ float sw[kMergeMaxHeads * kMergeMaxSplits];
        const uint32_t L = min(a.attn_len[0], a.attn_max_len);
        const int kps = a.keys_per_split;
        const int nsplit = (L == 0) ? 1 : (int)((L + kps - 1) / kps);
        const int hd = a.head_dim, G = a.group;
        const int Hq = a.K / hd;
        for (int i = threadIdx.x; i < Hq * nsplit; i += kGemvThreads) {
            const int h = i / nsplit, sidx = i % nsplit;
            const size_t idx = ((size_t)(h / G) * a.split_cap + sidx) * G + (h % G);
            sw[i] = a.ml_part[idx * 2];
        }
        __syncthreads();
        if (threadIdx.x < Hq) {
            const int h = threadIdx.x;
            float M = -INFINITY;
            for (int j = 0; j < nsplit; ++j) M = fmaxf(M, sw[h * nsplit + j]);
            float den = 0.f, w[kMergeMaxSplits];
            for (int j = 0; j < nsplit; ++j) {
                const size_t idx = ((size_t)(h / G) * a.split_cap + j) * G + (h % G);
                const float m = sw[h * nsplit + j];
                w[j] = (m == -INFINITY) ? 0.f : exp2f(m - M);
                den = fmaf(w[j], a.ml_part[idx * 2 + 1], den);
            }
            const float inv = (den > 0.f) ? 1.f / den : 0.f;
            for (int j = 0; j < nsplit; ++j) sw[h * nsplit + j] = w[j] * inv;
        }
        __syncthreads();
        for (int c = threadIdx.x; c < (a.K >> 2); c += kGemvThreads) {
            const int n0 = c * 4, h = n0 / hd, d0 = n0 % hd;
            const float* op = a.o_part + ((size_t)(h / G) * a.split_cap * G + (h % G)) * hd + d0;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int j = 0; j < nsplit; ++j) {
                const float4 v = *reinterpret_cast<const float4*>(op + (size_t)j * G * hd);
                const float wj = sw[h * nsplit + j];
                acc[0] = fmaf(wj, v.x, acc[0]);
                acc[1] = fmaf(wj, v.y, acc[1]);
                acc[2] = fmaf(wj, v.z, acc[2]);
                acc[3] = fmaf(wj, v.w, acc[3]);
            }
            uint2 pk;
            pk.x = pack_bf16x2(acc[0], acc[1]);
            pk.y = pack_bf16x2(acc[2], acc[3]);
            reinterpret_cast<uint2*>(xs)[c] = pk;
        }
        return;
    }
    float s[kProMax][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kProMax; ++i) {
        const int c = threadIdx.x + i * kGemvThreads;
        if (c < C) {
            uint4 hv = x4[c];
            unpack8(hv, s[i]);
            if (PRO == PRO_ADD_NORM) {
                float r[8];
                unpack8(reinterpret_cast<const uint4*>(a.r_in)[c], r);
#pragma unroll
                for (int e = 0; e < 8; ++e) s[i][e] += r[e];
            }
            if (blockIdx.x == 0 && a.r_out != nullptr) {
                reinterpret_cast<uint4*>(a.r_out)[c] = (PRO == PRO_ADD_NORM) ? pack8(s[i]) : hv;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(s[i][e], s[i][e], ss);
        }
    }
    const float tot = block_sum<kGemvThreads>(ss, red);
    const float inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
    const uint4* w4 = reinterpret_cast<const uint4*>(a.norm_w);
#pragma unroll
    for (int i = 0; i < kProMax; ++i) {
        const int c = threadIdx.x + i * kGemvThreads;
        if (c < C) {
            float w[8], o[8];
            unpack8(w4[c], w);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (s[i][e] * inv) * w[e];
            xs4[c] = pack8(o);
        }
    }
}

// Physical weight row of logical row n, part p (SwiGLU: p=0 up row n, p=1 gate row N+n).
template <int EPI>
__device__ __forceinline__ int phys_row(int n, int p, int N) {
    return (EPI == EPI_SWIGLU && p == 1) ? (N + n) : n;
}

template <int R, int KS, int PRO, int EPI>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a, int nj, int nseg) {
    constexpr int P = (EPI == EPI_SWIGLU) ? 2 : 1;
    constexpr int G = 4 / KS;          // row groups per block
    constexpr int RB = G * R;          // logical rows per block
    extern __shared__ __align__(16) unsigned char smem_raw[];
    bf16_t* xs = reinterpret_cast<bf16_t*>(smem_raw);
    __shared__ float red[kGemvThreads / kWave];
    __shared__ float part[G][KS][R * P];
    __shared__ ArgMax amx[G];
    __shared__ ArgMax fin[kGemvThreads / kWave];
    __shared__ bool is_last;

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

    uint4 wr[R][P][kNJMax];
    auto issue = [&](int rb, int seg) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = rb * RB + grp * R + r;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const bf16_t* row = a.W + (size_t)phys_row<EPI>(n, p, a.N) * (size_t)a.K;
#pragma unroll
                for (int j = 0; j < kNJMax; ++j) {
                    const int c = seg * segC + kw * kWave + lane + j * kWave * KS;
                    if (j < nj && n < a.N && c < C) {
                        wr[r][p][j] = EFM_WEIGHT_LOAD(row + (size_t)c * 8);
                    } else {
                        wr[r][p][j] = make_uint4(0u, 0u, 0u, 0u);
                    }
                }
            }
        }
    };

    int rb = blockIdx.x;
    if (rb < nrb) issue(rb, 0);
    gemv_prologue<PRO>(a, xs, red);
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
            for (int j = 0; j < kNJMax; ++j) {
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
        const int next = rb + gridDim.x;
        if (next < nrb) issue(next, 0);

#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int p = 0; p < P; ++p) acc[r][p] = wave_sum(acc[r][p]);
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
                float v = acc[r][0];
                if (a.bias != nullptr) v += bf16_to_f32(a.bias[n]);
                if (EPI == EPI_BF16) {
                    reinterpret_cast<bf16_t*>(a.y)[n] = (bf16_t)f32_to_bf16(v);
                } else if (EPI == EPI_F32) {
                    reinterpret_cast<float*>(a.y)[n] = v;
                } else if (EPI == EPI_QKV) {
                    const bf16_t bv = (bf16_t)f32_to_bf16(v);
                    if (n < a.q_dim) {
                        reinterpret_cast<bf16_t*>(a.y)[n] = bv;
                    } else {
                        const uint32_t L = a.d_kv_len[0];
                        if (L > 0) {
                            const size_t slot = (size_t)(L - 1) * (size_t)a.kv_dim;
                            const int m = n - a.q_dim;
                            if (m < a.kv_dim) a.k_cache[slot + m] = bv;
                            else a.v_cache[slot + (m - a.kv_dim)] = bv;
                        }
                    }
                } else if (EPI == EPI_SWIGLU) {
                    const float u = round_bf16(acc[r][0]);
                    const float g = round_bf16(acc[r][P - 1]);
                    const float sg = g / (1.0f + expf(-g));
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
            a.partials[blockIdx.x] = b;
            __threadfence();
            const uint32_t prev = atomicAdd(a.counter, 1u);
            is_last = (prev == gridDim.x - 1);
        }
        __syncthreads();
        if (is_last) {
            __threadfence();
            // The partials were written by other workgroups; load them all before
            // reducing (independent loads, not a dependent chain).
            constexpr int kPer = kTop1MaxGridDev / kGemvThreads;
            ArgMax pv[kPer];
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int i = threadIdx.x + k * kGemvThreads;
                if (i < (int)gridDim.x) {
                    pv[k].v = __builtin_nontemporal_load(&a.partials[i].v);
                    pv[k].i = __builtin_nontemporal_load(&a.partials[i].i);
                } else {
                    pv[k].v = -INFINITY;
                    pv[k].i = 0x7fffffff;
                }
            }
            ArgMax b = pv[0];
#pragma unroll
            for (int k = 1; k < kPer; ++k) b = argmax_pick(b, pv[k]);
            b = wave_argmax(b);
            if (lane == 0) fin[wave] = b;
            __syncthreads();
            if (threadIdx.x == 0) {
                ArgMax f = fin[0];
#pragma unroll
                for (int w = 1; w < kGemvThreads / kWave; ++w) f = argmax_pick(f, fin[w]);
                a.token_out[0] = f.i;
                a.counter[0] = 0u;
            }
        }
    }
}

}  // namespace efm

// ----------------------------------------------------------------------------------
// Host-side dispatch.
// ----------------------------------------------------------------------------------
namespace efm {

struct GemvCfg {
    int R, KS, nj, nseg, grid, nrb;
};

// Launch geometry for K inputs and N logical rows (P physical rows each), chosen from
// a sweep on MI355X: one row per wave (R = 1) except for very tall matrices (the LM
// head, R = 4); the K split KS keeps each lane at <= 6 16-byte chunks per row;
// about 4 workgroups per CU (2 for the top-1 reduction) walking row blocks grid-stride
// amortise the per-workgroup prologue (the RMSNorm of the input vector).
static GemvCfg gemv_pick(int K, int N, int P, int max_grid, bool tall) {
    GemvCfg g;
    const int C = K / 8;
    g.KS = (C <= 256) ? 1 : (C <= 512 ? 2 : 4);
    const int per = kWave * g.KS;
    const int need = (C + per - 1) / per;
    g.nseg = (need + kNJMax - 1) / kNJMax;
    g.nj = (need + g.nseg - 1) / g.nseg;
    const int groups = 4 / g.KS;
    g.R = 1;
    if (tall && (int64_t)N >= 65536) g.R = 4;
    else if (P == 1 && g.KS == 4 && (int64_t)N * K >= (64 << 20)) g.R = 2;  // very large K x N (7B down)
    // two-wave K split (7B q/o rows): six workgroups per CU measured 4-7 % faster
    if (P == 1 && g.KS == 2 && !tall) max_grid = std::max(max_grid, 1536);
    g.nrb = (N + groups * g.R - 1) / (groups * g.R);
    g.grid = std::min(g.nrb, max_grid);
    return g;
}

template <int PRO, int EPI>
static int gemv_launch(const GemvCfg& g, const GemvArgs& a, hipStream_t stream) {
    const size_t smem = (size_t)a.K * sizeof(bf16_t);
    dim3 grid(g.grid), block(kGemvThreads);
#define EFM_GEMV_CASE(RR, KK)                                                                  \
    if (g.R == RR && g.KS == KK) {                                                             \
        hipLaunchKernelGGL((gemv_kernel<RR, KK, PRO, EPI>), grid, block, smem, stream, a, g.nj, \
                           g.nseg);                                                            \
        return check_launch("gemv");                                                           \
    }
    EFM_GEMV_CASE(1, 1) EFM_GEMV_CASE(2, 1) EFM_GEMV_CASE(4, 1)
    EFM_GEMV_CASE(1, 2) EFM_GEMV_CASE(2, 2) EFM_GEMV_CASE(4, 2)
    EFM_GEMV_CASE(1, 4) EFM_GEMV_CASE(2, 4) EFM_GEMV_CASE(4, 4)
#undef EFM_GEMV_CASE
    return set_error(EFM_ERR_UNSUPPORTED, "gemv: no kernel for R=%d KS=%d", g.R, g.KS);
}

static GemvArgs gemv_args(int K, int N, const void* W, const void* x) {
    GemvArgs a = {};
    a.K = K;
    a.N = N;
    a.W = static_cast<const bf16_t*>(W);
    a.x = static_cast<const bf16_t*>(x);
    return a;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int gemv_check(int64_t K, int64_t N, const void* W, const void* x, const void* y, bool prologue) {
    if (W == nullptr || x == nullptr || y == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "gemv: null pointer");
    if (K <= 0 || N <= 0 || K % 8 != 0)
        return set_error(EFM_ERR_UNSUPPORTED, "gemv: in_features must be a positive multiple of 8 (got %lld)",
                         (long long)K);
    if (K > 65536 || N > (int64_t)0x7fffffff / 2)
        return set_error(EFM_ERR_UNSUPPORTED, "gemv: shape too large (K=%lld N=%lld)", (long long)K, (long long)N);
    if (prologue && K > 8 * kGemvThreads * kProMax)
        return set_error(EFM_ERR_UNSUPPORTED, "gemv: fused RMSNorm supports hidden <= %d", 8 * kGemvThreads * kProMax);
    if (!aligned16(W) || !aligned16(x))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "gemv: weight and input must be 16-byte aligned");
    return EFM_OK;
}

constexpr int kTop1MaxGrid = kTop1MaxGridDev;
constexpr size_t kTop1CounterOffset = kTop1MaxGrid * sizeof(ArgMax);

int gemv_plain(int64_t K, int64_t N, const void* x, const void* W, const void* bias, void* y, int32_t out_dtype,
               hipStream_t stream) {
    int rc = gemv_check(K, N, W, x, y, false);
    if (rc) return rc;
    GemvArgs a = gemv_args((int)K, (int)N, W, x);
    a.bias = static_cast<const bf16_t*>(bias);
    a.y = y;
    if (out_dtype == EFM_DTYPE_BF16) {
        return gemv_launch<PRO_PLAIN, EPI_BF16>(gemv_pick((int)K, (int)N, 1, 1024, false), a, stream);
    }
    if (out_dtype == EFM_DTYPE_F32) {
        return gemv_launch<PRO_PLAIN, EPI_F32>(gemv_pick((int)K, (int)N, 1, 512, true), a, stream);
    }
    return set_error(EFM_ERR_UNSUPPORTED, "linear: output dtype %d not supported", out_dtype);
}

int gemv_swiglu(int64_t K, int64_t inter, const void* x, const void* W, void* y, hipStream_t stream) {
    int rc = gemv_check(K, inter, W, x, y, false);
    if (rc) return rc;
    GemvArgs a = gemv_args((int)K, (int)inter, W, x);
    a.y = y;
    return gemv_launch<PRO_PLAIN, EPI_SWIGLU>(gemv_pick((int)K, (int)inter, 2, 1024, false), a, stream);
}

}  // namespace efm

using namespace efm;

extern "C" size_t efm_lm_head_top1_workspace_bytes(int64_t vocab) {
    (void)vocab;
    return kTop1CounterOffset + 256;
}

extern "C" int efm_lm_head_top1(int64_t hidden, int64_t vocab, const void* x, const void* w, int32_t* token_out,
                                void* workspace, size_t workspace_bytes, hipStream_t stream) {
    int rc = gemv_check(hidden, vocab, w, x, token_out, false);
    if (rc) return rc;
    if (workspace == nullptr || workspace_bytes < efm_lm_head_top1_workspace_bytes(vocab))
        return set_error(EFM_ERR_WORKSPACE, "lm_head_top1: workspace of %zu bytes required",
                         efm_lm_head_top1_workspace_bytes(vocab));
    GemvArgs a = gemv_args((int)hidden, (int)vocab, w, x);
    a.partials = static_cast<ArgMax*>(workspace);
    a.counter = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + kTop1CounterOffset);
    a.token_out = token_out;
    return gemv_launch<PRO_PLAIN, EPI_TOP1>(gemv_pick((int)hidden, (int)vocab, 1, 512, true), a, stream);
}

extern "C" int efm_decode_norm_qkv(int32_t hidden, int32_t q_dim, int32_t kv_dim, float eps, const void* h,
                                   const void* residual_in, void* residual_out, const void* norm_w,
                                   const void* w_qkv, const void* b_qkv, void* q_out, void* k_cache,
                                   void* v_cache, const uint32_t* d_kv_len, hipStream_t stream) {
    const int N = q_dim + 2 * kv_dim;
    int rc = gemv_check(hidden, N, w_qkv, h, q_out, true);
    if (rc) return rc;
    if (norm_w == nullptr || residual_out == nullptr || k_cache == nullptr || v_cache == nullptr ||
        d_kv_len == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv: null pointer");
    if (residual_out == h || (residual_in != nullptr && residual_out == residual_in))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv: residual_out must not alias its inputs");
    GemvArgs a = gemv_args(hidden, N, w_qkv, h);
    a.r_in = static_cast<const bf16_t*>(residual_in);
    a.r_out = static_cast<bf16_t*>(residual_out);
    a.norm_w = static_cast<const bf16_t*>(norm_w);
    a.eps = eps;
    a.bias = static_cast<const bf16_t*>(b_qkv);
    a.y = q_out;
    a.q_dim = q_dim;
    a.kv_dim = kv_dim;
    a.k_cache = static_cast<bf16_t*>(k_cache);
    a.v_cache = static_cast<bf16_t*>(v_cache);
    a.d_kv_len = d_kv_len;
    const GemvCfg g = gemv_pick(hidden, N, 1, 1024, false);
    if (residual_in == nullptr) return gemv_launch<PRO_NORM, EPI_QKV>(g, a, stream);
    return gemv_launch<PRO_ADD_NORM, EPI_QKV>(g, a, stream);
}

extern "C" int efm_decode_norm_gate_up_swiglu(int32_t hidden, int32_t inter, float eps, const void* a_in,
                                              const void* residual_in, void* residual_out, const void* norm_w,
                                              const void* w_up_gate, void* out, hipStream_t stream) {
    int rc = gemv_check(hidden, inter, w_up_gate, a_in, out, true);
    if (rc) return rc;
    if (residual_in == nullptr || residual_out == nullptr || norm_w == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_gate_up_swiglu: null pointer");
    if (residual_out == a_in || residual_out == residual_in)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_gate_up_swiglu: residual_out must not alias");
    GemvArgs a = gemv_args(hidden, inter, w_up_gate, a_in);
    a.r_in = static_cast<const bf16_t*>(residual_in);
    a.r_out = static_cast<bf16_t*>(residual_out);
    a.norm_w = static_cast<const bf16_t*>(norm_w);
    a.eps = eps;
    a.y = out;
    return gemv_launch<PRO_ADD_NORM, EPI_SWIGLU>(gemv_pick(hidden, inter, 2, 1024, false), a, stream);
}

namespace efm {
int decode_split_cap(int num_kv_heads, uint32_t max_kv_len);
int decode_keys_per_split(int num_kv_heads, uint32_t max_kv_len);
size_t decode_workspace_bytes(const efm_attention_ctx* ctx, uint32_t max_kv_len);
size_t decode_ml_offset(const efm_attention_ctx* ctx, uint32_t max_kv_len);
int validate_attention_ctx(const efm_attention_ctx* c, const char* who);
}  // namespace efm

extern "C" int efm_decode_attention_merge_o_proj(const efm_attention_ctx* ctx, const uint32_t* d_kv_len,
                                                 uint32_t max_kv_len, const void* workspace,
                                                 size_t workspace_bytes, const void* w_o, int32_t hidden, void* out,
                                                 hipStream_t stream) {
    int rc = validate_attention_ctx(ctx, "attention_merge_o_proj");
    if (rc) return rc;
    if (d_kv_len == nullptr || workspace == nullptr || w_o == nullptr || out == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "attention_merge_o_proj: null pointer");
    const int q_dim = (int)(ctx->num_qo_heads * ctx->head_dim);
    rc = gemv_check(q_dim, hidden, w_o, workspace, out, false);
    if (rc) return rc;
    const int cap = decode_split_cap((int)ctx->num_kv_heads, max_kv_len);
    if ((int64_t)cap > kMergeMaxSplits || (int)ctx->num_qo_heads > kMergeMaxHeads)
        return set_error(EFM_ERR_UNSUPPORTED, "attention_merge_o_proj: %d splits / %u heads exceed the fused merge",
                         cap, ctx->num_qo_heads);
    if (workspace_bytes < decode_workspace_bytes(ctx, max_kv_len))
        return set_error(EFM_ERR_WORKSPACE, "attention_merge_o_proj: workspace too small");
    GemvArgs a = gemv_args(q_dim, hidden, w_o, workspace);
    a.y = out;
    a.o_part = static_cast<const float*>(workspace);
    a.ml_part = reinterpret_cast<const float*>(static_cast<const char*>(workspace) + decode_ml_offset(ctx, max_kv_len));
    a.split_cap = cap;
    a.keys_per_split = decode_keys_per_split((int)ctx->num_kv_heads, max_kv_len);
    a.head_dim = (int)ctx->head_dim;
    a.group = (int)(ctx->num_qo_heads / ctx->num_kv_heads);
    a.attn_len = d_kv_len;
    a.attn_max_len = max_kv_len;
    return gemv_launch<PRO_ATTN_MERGE, EPI_BF16>(gemv_pick(q_dim, hidden, 1, 1024, false), a, stream);
}

extern "C" int efm_decode_norm_lm_head_top1(int32_t hidden, int64_t vocab, float eps, const void* h,
                                            const void* residual_in, const void* norm_w, const void* w_lm,
                                            int32_t* token_out, void* workspace, size_t workspace_bytes,
                                            hipStream_t stream) {
    int rc = gemv_check(hidden, vocab, w_lm, h, token_out, true);
    if (rc) return rc;
    if (residual_in == nullptr || norm_w == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_lm_head_top1: null pointer");
    if (workspace == nullptr || workspace_bytes < efm_lm_head_top1_workspace_bytes(vocab))
        return set_error(EFM_ERR_WORKSPACE, "decode_norm_lm_head_top1: workspace of %zu bytes required",
                         efm_lm_head_top1_workspace_bytes(vocab));
    GemvArgs a = gemv_args(hidden, (int)vocab, w_lm, h);
    a.r_in = static_cast<const bf16_t*>(residual_in);
    a.r_out = nullptr;
    a.norm_w = static_cast<const bf16_t*>(norm_w);
    a.eps = eps;
    a.partials = static_cast<ArgMax*>(workspace);
    a.counter = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + kTop1CounterOffset);
    a.token_out = token_out;
    return gemv_launch<PRO_ADD_NORM, EPI_TOP1>(gemv_pick(hidden, (int)vocab, 1, 512, true), a, stream);
}

// Post-attention decode chain of one transformer layer in a single persistent launch.
//
// For decode layer l it computes, in one kernel, what the unfused path does in four:
//   a     = bf16(merge(attention split partials)) . W_o^T          (o_proj, merge folded in)
//   r'    = bf16(a + r_l);  x2 = RMSNorm(r') * post_norm
//   mid   = bf16(silu(bf16(x2 . W_gate^T)) * bf16(x2 . W_up^T))    (fused gate/up + SwiGLU)
//   h     = bf16(mid . W_down^T)
//   r_l+1 = bf16(h + r');   x = RMSNorm(r_l+1) * in_norm_{l+1}
//   qkv   = bf16(x . W_qkv_{l+1}^T + b_qkv_{l+1}) -> q, and K / V into cache slot L-1
// i.e. the operator sequence of the Qwen2.5 decode layer from the o_proj through the next
// layer's fused QKV projection (src/models/qwen2_5/qwen2_5.cpp:600-929). On the last layer
// the chain stops after h and hands (h, r') to the final norm + LM head.
//
// Design for MI355X (one workgroup per CU; 8 worker waves + 1 control wave):
//  * At launch every worker wave issues all of its weight loads for the layer: its o_proj
//    row and its gate/up rows into registers, and its share of the workgroup's down_proj
//    rows straight into LDS (global_load_lds). HBM streams the whole layer from the first
//    cycle; each phase below only waits for its activation input.
//  * Workgroups exchange the three all-to-all vectors (o_proj output, SwiGLU output,
//    down_proj output) as tagged 32-bit words, bf16 payload | 16-bit tag of this launch,
//    written and polled with agent-scope atomic stores / loads (coherent across the
//    per-XCD L2 caches). A word is valid when its tag matches: no fence, no counter and
//    no grid barrier. The tag comes from a launch counter in the workspace that
//    workgroup 0 advances after it has received every workgroup's last output.
//  * The control wave merges the attention splits, does the residual adds and RMSNorms,
//    publishes results and polls for inputs; waves meet at workgroup barriers, which do
//    not drain the workers' outstanding weight loads.
//  * Every reduction replicates the order of the standalone kernels (the gemv family's
//    lane/chunk layout and K split, the 256-thread block sum of its RMSNorm prologue, the
//    log-sum-exp merge of the o_proj prologue), so the results are bit-identical to the
//    unfused sequence.
//  * Polls are bounded: a word that does not arrive within the spin limit (for example
//    when not every workgroup could be resident) raises the workspace's abort flag, and
//    every later poll gives up at once, so the launch always drains.
#include "common.hpp"

#include <algorithm>

namespace efm {

constexpr int kChainWorkers = 8;
constexpr int kChainThreads = (kChainWorkers + 1) * kWave;  // 576
constexpr int kChainNJ = 3;              // 16-byte chunks per lane of a row with K <= 1536
constexpr int kChainMaxK = 1536;         // hidden size and q_dim limit (gemv K split 1)
constexpr int kChainMaxRows = 8;         // o_proj / down_proj / qkv rows per workgroup
constexpr int kChainMaxOut = 5;          // gate/up outputs per worker wave
constexpr int kChainPreOut = 3;          // of which issued at launch (the rest when the phase starts)
constexpr int kChainStageBytes = 112 * 1024;
constexpr int kChainMaxInter = 10240;
constexpr int kChainDownNJ = 6;          // chunks per lane of a down_proj row part
constexpr int kChainMaxSplit = 8;
constexpr int kChainMaxHeads = 64;
constexpr uint32_t kChainSpin = 1u << 20;
#ifndef EFM_CHAIN_POLL_SLEEP
#define EFM_CHAIN_POLL_SLEEP 2   // back-off between poll rounds, in units of 64 cycles
#endif

// Phase timestamps for tuning builds (-DEFM_CHAIN_TRACE): 16 wall-clock stamps per
// workgroup after the workspace's control words. Compiled out otherwise.
#ifdef EFM_CHAIN_TRACE
#define CHAIN_STAMP(ev)                                                              \
    do {                                                                             \
        if (lane == 0) a.trace[(size_t)blockIdx.x * 16 + (ev)] = wall_clock64();      \
    } while (0)
#else
#define CHAIN_STAMP(ev) \
    do {                \
    } while (0)
#endif

struct ChainArgs {
    int H, QD, KVD, I, HD, G, Hq;
    float eps;
    const bf16_t* w_o;
    const bf16_t* post_norm;
    const bf16_t* w_gu;        // [2I, H], rows [up; gate]
    const bf16_t* w_down;      // [H, I]
    const bf16_t* in_norm_next;
    const bf16_t* w_qkv_next;  // [QD + 2 KVD, H]
    const bf16_t* b_qkv_next;
    bf16_t* q_next;
    bf16_t* k_cache_next;
    bf16_t* v_cache_next;
    const float* o_part;       // [Hkv][split_cap][G][HD]
    const float* ml_part;      // [Hkv][split_cap][G][2]
    int split_cap, keys_per_split;
    const uint32_t* d_kv_len;
    uint32_t max_kv_len;
    const bf16_t* r_in;
    bf16_t* r_out;
    bf16_t* h_out;
    uint32_t* xa;
    uint32_t* xh;
    uint32_t* xmid;
    uint32_t* epoch;
    uint32_t* abort_flag;
    uint64_t* trace;
    int last;
};

// Publishes one tagged word. An agent-scope atomic exchange (performed where atomics of
// every XCD meet) rather than a plain store, so the word is visible to the other XCDs'
// polls as soon as it is performed.
__device__ __forceinline__ void tagged_store(uint32_t* p, uint32_t tag, uint32_t bits16) {
    (void)__hip_atomic_exchange(p, (tag << 16) | (bits16 & 0xffffu), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t coherent_load(uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Orders LDS accesses of different lanes of one wave (control-wave hand-offs).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Copies the payloads of n tagged words src[0..n) into dst (LDS) once each word carries
// `tag`. Participating threads have indices idx in [0, nthr). Every round issues the
// loads of all words still pending before checking any, so a round costs one memory
// round trip however many words are late.
template <int MAXW>
__device__ uint32_t poll_tagged(uint32_t* src, int n, uint32_t tag, bf16_t* dst, int idx, int nthr,
                                uint32_t* abort_flag) {
    uint32_t pending = 0u;
#pragma unroll
    for (int k = 0; k < MAXW; ++k)
        if (idx + k * nthr < n) pending |= 1u << k;
    uint32_t spins = 0;
    while (true) {
        uint32_t w[MAXW];
#pragma unroll
        for (int k = 0; k < MAXW; ++k) w[k] = (pending >> k & 1u) ? coherent_load(src + idx + k * nthr) : 0u;
#pragma unroll
        for (int k = 0; k < MAXW; ++k) {
            if ((pending >> k & 1u) && (w[k] >> 16) == tag) {
                dst[idx + k * nthr] = (bf16_t)(w[k] & 0xffffu);
                pending &= ~(1u << k);
            }
        }
        if (pending == 0u) break;
        if (++spins > kChainSpin || coherent_load(abort_flag) != 0u) {
            __hip_atomic_store(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(EFM_CHAIN_POLL_SLEEP);
    }
    return spins;
}

__global__ __launch_bounds__(kChainThreads, 1) void decode_chain_kernel(ChainArgs a) {
    __shared__ __align__(16) unsigned char stage[kChainStageBytes];  // this workgroup's down_proj rows
    __shared__ __align__(16) bf16_t xin[kChainMaxK];                 // hidden-size input vector
    __shared__ __align__(16) bf16_t xbig[kChainMaxInter];            // SwiGLU output (down_proj input)
    __shared__ __align__(16) bf16_t rres[kChainMaxK];                // residual stream
    __shared__ __align__(16) bf16_t nw_post[kChainMaxK];
    __shared__ __align__(16) bf16_t nw_in[kChainMaxK];
    __shared__ float sbias[kChainWorkers];
    __shared__ float sw[kChainMaxHeads * kChainMaxSplit];
    __shared__ float red[4];
    __shared__ uint32_t s_epoch;
    __shared__ int s_nsplit;

    const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
    const bool ctrl = (wave == kChainWorkers);
    const int NB = gridDim.x, b = blockIdx.x;
    const int H = a.H, QD = a.QD, I = a.I;
    // Row ownership is interleaved: workgroup b owns rows b, b + NB, b + 2 NB, ... of every
    // matrix, so at any moment the whole chip streams one contiguous band of each weight.
    const int NQ = QD + 2 * a.KVD;
    const int nro = (H - b + NB - 1) / NB;  // o_proj / down_proj rows of this workgroup
    const int nrq = (NQ - b + NB - 1) / NB; // qkv rows
    const int Co = QD >> 3, Ch = H >> 3, Cd = I >> 3;
    const int KSd = (Cd <= 256) ? 1 : (Cd <= 512 ? 2 : 4);
    const int njd = (Cd + kWave * KSd - 1) / (kWave * KSd);
    const int hd = a.HD, G = a.G;
    const uint4* xin4 = reinterpret_cast<const uint4*>(xin);
    const uint4* xbig4 = reinterpret_cast<const uint4*>(xbig);

    // Residual add + RMSNorm by worker waves 0-3, one 8-element chunk per lane in the
    // order of the 256-thread gemv prologue: rres = bf16(v + rres), v = bf16(s * inv * w).
    auto add_norm = [&](const bf16_t* nw) {
        float sv[8];
        const int c = wave * kWave + lane;
        const bool act = wave < 4 && c < Ch;
        float ss = 0.f;
        if (act) {
            float r[8];
            unpack8(xin4[c], sv);
            unpack8(reinterpret_cast<const uint4*>(rres)[c], r);
#pragma unroll
            for (int e = 0; e < 8; ++e) sv[e] += r[e];
            reinterpret_cast<uint4*>(rres)[c] = pack8(sv);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(sv[e], sv[e], ss);
        }
        if (wave < 4) {
            ss = wave_sum(ss);
            if (lane == 0) red[wave] = ss;
        }
        __syncthreads();
        if (act) {
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < 4; ++w) tot += red[w];
            const float inv = 1.0f / sqrtf(tot / (float)H + a.eps);
            float w8[8], o[8];
            unpack8(reinterpret_cast<const uint4*>(nw)[c], w8);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (sv[e] * inv) * w8[e];
            reinterpret_cast<uint4*>(xin)[c] = pack8(o);
        }
    };

    // ---- launch: small operands first (merge inputs, residual, norm weights, bias), then
    // the o_proj row. Workers read every split slot (stale slots get weight 0), so the
    // loads do not wait for the cache length.
    float4 opart[kChainMaxSplit];
    uint4 wo[kChainNJ];
    const int gi = tid;  // merge group of a worker thread: 4 consecutive outputs
    if (!ctrl) {
        if (gi < (QD >> 2)) {
            const int n0 = gi * 4, h = n0 / hd, d0 = n0 % hd;
            const float* op = a.o_part + ((size_t)(h / G) * a.split_cap * G + (h % G)) * hd + d0;
#pragma unroll
            for (int j = 0; j < kChainMaxSplit; ++j)
                opart[j] = (j < a.split_cap) ? *reinterpret_cast<const float4*>(op + (size_t)j * G * hd)
                                             : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const int row = b + wave * NB;
#pragma unroll
        for (int j = 0; j < kChainNJ; ++j) {
            const int c = lane + j * kWave;
            wo[j] = (wave < nro && c < Co) ? load_stream16(a.w_o + (size_t)row * QD + (size_t)c * 8)
                                           : make_uint4(0u, 0u, 0u, 0u);
        }
    } else {
        CHAIN_STAMP(9);
        if (lane == 0) s_epoch = coherent_load(a.epoch);
        const uint32_t L = min(a.d_kv_len[0], a.max_kv_len);
        const int kps = a.keys_per_split;
        const int nsplit = (L == 0) ? 1 : (int)((L + kps - 1) / kps);
        uint4 rv[4], pv[4], iv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int c = lane + k * kWave;
            rv[k] = (c < Ch) ? reinterpret_cast<const uint4*>(a.r_in)[c] : make_uint4(0u, 0u, 0u, 0u);
            pv[k] = (c < Ch) ? reinterpret_cast<const uint4*>(a.post_norm)[c] : make_uint4(0u, 0u, 0u, 0u);
            iv[k] = (c < Ch && !a.last) ? reinterpret_cast<const uint4*>(a.in_norm_next)[c] : make_uint4(0u, 0u, 0u, 0u);
        }
        float bias = 0.f;
        if (!a.last && lane < nrq) bias = bf16_to_f32(a.b_qkv_next[b + lane * NB]);
        float m[kChainMaxSplit], l[kChainMaxSplit];
        if (lane < a.Hq) {
            const int h = lane;
#pragma unroll
            for (int j = 0; j < kChainMaxSplit; ++j) {
                if (j < nsplit) {
                    const size_t idx = ((size_t)(h / G) * a.split_cap + j) * G + (h % G);
                    m[j] = a.ml_part[idx * 2];
                    l[j] = a.ml_part[idx * 2 + 1];
                }
            }
            float M = -INFINITY;
#pragma unroll
            for (int j = 0; j < kChainMaxSplit; ++j)
                if (j < nsplit) M = fmaxf(M, m[j]);
            float den = 0.f, w[kChainMaxSplit];
#pragma unroll
            for (int j = 0; j < kChainMaxSplit; ++j) {
                if (j < nsplit) {
                    w[j] = (m[j] == -INFINITY) ? 0.f : exp2f(m[j] - M);
                    den = fmaf(w[j], l[j], den);
                }
            }
            const float inv = (den > 0.f) ? 1.f / den : 0.f;
#pragma unroll
            for (int j = 0; j < kChainMaxSplit; ++j)
                if (j < nsplit) sw[h * nsplit + j] = w[j] * inv;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int c = lane + k * kWave;
            if (c < Ch) {
                reinterpret_cast<uint4*>(rres)[c] = rv[k];
                reinterpret_cast<uint4*>(nw_post)[c] = pv[k];
                reinterpret_cast<uint4*>(nw_in)[c] = iv[k];
            }
        }
        if (lane < kChainWorkers) sbias[lane] = bias;
        if (lane == 0) s_nsplit = nsplit;
        CHAIN_STAMP(0);
    }
    __syncthreads();
    if (wave == 0) CHAIN_STAMP(10);
    const uint32_t tag = (s_epoch % 65535u) + 1u;

    // ---- merged attention output -> xbig[0, QD) (the o_proj input)
    if (!ctrl && gi < (QD >> 2)) {
        const int nsplit = s_nsplit;
        const int h = (gi * 4) / hd;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < kChainMaxSplit; ++j) {
            if (j < nsplit) {
                const float wj = sw[h * nsplit + j];
                acc[0] = fmaf(wj, opart[j].x, acc[0]);
                acc[1] = fmaf(wj, opart[j].y, acc[1]);
                acc[2] = fmaf(wj, opart[j].z, acc[2]);
                acc[3] = fmaf(wj, opart[j].w, acc[3]);
            }
        }
        uint2 pk;
        pk.x = pack_bf16x2(acc[0], acc[1]);
        pk.y = pack_bf16x2(acc[2], acc[3]);
        reinterpret_cast<uint2*>(xbig)[gi] = pk;
    }
    if (wave == 0) CHAIN_STAMP(11);
    __syncthreads();
    if (wave == 0) CHAIN_STAMP(12);

    // ---- o_proj (one row per worker wave), publish, then issue the gate/up rows
    uint4 wg[kChainPreOut][2][kChainNJ];
    uint4 wg2[kChainMaxOut - kChainPreOut][2][kChainNJ];
    auto load_gu = [&](uint4 (*dst)[2][kChainNJ], int k0, int nk) {
#pragma unroll
        for (int k = 0; k < kChainMaxOut; ++k) {
            if (k >= nk) break;
            const int n = b + (wave + (k0 + k) * kChainWorkers) * NB;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const bf16_t* rowp = a.w_gu + (size_t)(p ? I + n : n) * (size_t)H;
#pragma unroll
                for (int j = 0; j < kChainNJ; ++j) {
                    const int c = lane + j * kWave;
                    dst[k][p][j] = (n < I && c < Ch) ? load_stream16(rowp + (size_t)c * 8) : make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
    };
    if (!ctrl) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < kChainNJ; ++j) {
            const int c = lane + j * kWave;
            if (c < Co) acc = dot8(wo[j], xbig4[c], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0 && wave < nro) tagged_store(a.xa + b + wave * NB, tag, f32_to_bf16(acc));
        load_gu(wg, 0, kChainPreOut);
        load_gu(wg2, kChainPreOut, kChainMaxOut - kChainPreOut);
        if (wave == 0) CHAIN_STAMP(1);
#ifdef EFM_CHAIN_TRACE_LANDED
        __builtin_amdgcn_s_waitcnt(0);
        if (wave == 0) CHAIN_STAMP(11);
#endif
    } else {
        poll_tagged<kChainMaxK / kWave>(a.xa, H, tag, xin, lane, kWave, a.abort_flag);
        CHAIN_STAMP(2);
    }
    __syncthreads();
    add_norm(nw_post);  // r' = bf16(a + r_l); xin = RMSNorm(r') * post_norm
    __syncthreads();
    if (ctrl) CHAIN_STAMP(3);

    // ---- gate/up + SwiGLU, publish, then issue the down_proj rows into LDS
    if (!ctrl) {
        auto gu_out = [&](const uint4 (*w)[kChainNJ], int k) {
            const int n = b + (wave + k * kChainWorkers) * NB;
            float au = 0.f, ag = 0.f;
#pragma unroll
            for (int j = 0; j < kChainNJ; ++j) {
                const int c = lane + j * kWave;
                if (c < Ch) {
                    const uint4 xv = xin4[c];
                    au = dot8(w[0][j], xv, au);
                    ag = dot8(w[1][j], xv, ag);
                }
            }
            au = wave_sum(au);
            ag = wave_sum(ag);
            if (lane == 0 && n < I) {
                const float u = round_bf16(au);
                const float g = round_bf16(ag);
                const float sg = g / (1.0f + expf(-g));
                tagged_store(a.xmid + n, tag, f32_to_bf16(sg * u));
            }
        };
#pragma unroll
        for (int k = 0; k < kChainPreOut; ++k) gu_out(wg[k], k);
#pragma unroll
        for (int k = 0; k < kChainMaxOut - kChainPreOut; ++k) gu_out(wg2[k], kChainPreOut + k);
        if (wave == 0) CHAIN_STAMP(4);
        // row i of this workgroup (global row b + i NB) lands at stage + i * I * 2
        const int rbytes = I * 2;
        const int nsl = (rbytes + 1023) / 1024;
        for (int t = wave; t < nro * nsl; t += kChainWorkers) {
            const int i = t / nsl, s = t % nsl;
            const int off = s * 1024 + lane * 16;
            if (off < rbytes)
                __builtin_amdgcn_global_load_lds(
                    static_cast<const void*>(reinterpret_cast<const char*>(a.w_down + (size_t)(b + i * NB) * I) +
                                             off),
                    (__attribute__((address_space(3))) void*)(stage + (size_t)i * rbytes + (size_t)s * 1024), 16,
                    0, 0);
        }
    }
    poll_tagged<(kChainMaxInter + kChainThreads - 1) / kChainThreads>(a.xmid, I, tag, xbig, tid, kChainThreads,
                                                                     a.abort_flag);
    __syncthreads();
    if (ctrl) CHAIN_STAMP(5);

    // ---- down_proj from LDS: one row per worker wave, its K parts summed in the gemv
    // K-split order; publish, then issue the next layer's QKV row
    uint4 wq[kChainNJ];
    if (!ctrl) {
        if (wave < nro) {
            const uint4* wrow = reinterpret_cast<const uint4*>(stage + (size_t)wave * I * 2);
            float t = 0.f;
#pragma unroll
            for (int kw = 0; kw < 4; ++kw) {
                if (kw < KSd) {
                    float acc = 0.f;
#pragma unroll
                    for (int j = 0; j < kChainDownNJ; ++j) {
                        const int c = kw * kWave + lane + j * kWave * KSd;
                        if (j < njd && c < Cd) acc = dot8(wrow[c], xbig4[c], acc);
                    }
                    acc = wave_sum(acc);
                    t = (KSd > 1) ? (t + acc) : acc;
                }
            }
            if (lane == 0) tagged_store(a.xh + b + wave * NB, tag, f32_to_bf16(t));
        }
        if (!a.last) {
            const int row = b + wave * NB;
#pragma unroll
            for (int j = 0; j < kChainNJ; ++j) {
                const int c = lane + j * kWave;
                wq[j] = (wave < nrq && c < Ch) ? load_stream16(a.w_qkv_next + (size_t)row * H + (size_t)c * 8)
                                               : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        if (wave == 0) CHAIN_STAMP(6);
    }
    const uint32_t rounds_h = poll_tagged<(kChainMaxK + kChainThreads - 1) / kChainThreads>(
        a.xh, H, tag, xin, tid, kChainThreads, a.abort_flag);
#ifdef EFM_CHAIN_TRACE
    if (wave == 0) CHAIN_STAMP(13);
    if (ctrl) CHAIN_STAMP(14);
    if (ctrl && lane == 0) a.trace[(size_t)blockIdx.x * 16 + 15] = rounds_h;
#else
    (void)rounds_h;
#endif
    __syncthreads();
    if (ctrl) CHAIN_STAMP(7);

    if (a.last) {
        if (ctrl && b == 0) {
            for (int c = lane; c < Ch; c += kWave) {
                reinterpret_cast<uint4*>(a.h_out)[c] = xin4[c];
                reinterpret_cast<uint4*>(a.r_out)[c] = reinterpret_cast<const uint4*>(rres)[c];
            }
        }
    } else {
        add_norm(nw_in);  // r_{l+1} = bf16(h + r'); xin = RMSNorm(r_{l+1}) * in_norm_next
        if (b == 0 && !ctrl && wave < 4) {
            const int c = wave * kWave + lane;
            if (c < Ch) reinterpret_cast<uint4*>(a.r_out)[c] = reinterpret_cast<const uint4*>(rres)[c];
        }
        __syncthreads();
        if (!ctrl) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < kChainNJ; ++j) {
                const int c = lane + j * kWave;
                if (c < Ch) acc = dot8(wq[j], xin4[c], acc);
            }
            acc = wave_sum(acc);
            const int n = b + wave * NB;
            if (lane == 0 && wave < nrq) {
                const bf16_t bv = (bf16_t)f32_to_bf16(acc + sbias[wave]);
                if (n < QD) {
                    a.q_next[n] = bv;
                } else {
                    const uint32_t L = a.d_kv_len[0];
                    if (L > 0) {
                        const size_t slot = (size_t)(L - 1) * (size_t)a.KVD;
                        const int m = n - QD;
                        if (m < a.KVD) a.k_cache_next[slot + m] = bv;
                        else a.v_cache_next[slot + (m - a.KVD)] = bv;
                    }
                }
            }
        }
    }
    if (ctrl) CHAIN_STAMP(8);
    // workgroup 0 has received every workgroup's down_proj output, so every workgroup
    // has read this launch's counter: advance it for the next launch
    if (ctrl && b == 0 && lane == 0)
        __hip_atomic_store(a.epoch, s_epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace efm

// ----------------------------------------------------------------------------------
// Host side
// ----------------------------------------------------------------------------------
namespace efm {

int decode_split_cap(int num_kv_heads, uint32_t max_kv_len);
int decode_keys_per_split(int num_kv_heads, uint32_t max_kv_len);
size_t decode_workspace_bytes(const efm_attention_ctx* ctx, uint32_t max_kv_len);
size_t decode_ml_offset(const efm_attention_ctx* ctx, uint32_t max_kv_len);
int validate_attention_ctx(const efm_attention_ctx* c, const char* who);

static size_t chain_align(size_t x) { return (x + 255) & ~(size_t)255; }

struct ChainWs {
    size_t xa, xh, xmid, epoch, abort_flag, total;
};

static ChainWs chain_ws(int hidden, int inter) {
    ChainWs w;
    w.xa = 0;
    w.xh = chain_align((size_t)hidden * 4);
    w.xmid = w.xh + chain_align((size_t)hidden * 4);
    w.epoch = w.xmid + chain_align((size_t)inter * 4);
    w.abort_flag = w.epoch + 256;
    w.total = w.abort_flag + 256;
#ifdef EFM_CHAIN_TRACE
    w.total += 1024 * 16 * sizeof(uint64_t);
#endif
    return w;
}

static int chain_grid(int* grid) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(EFM_ERR_DEVICE, "decode_chain: hipGetDevice failed");
    static int cached[64] = {0};
    if (dev < 0 || dev >= 64) return set_error(EFM_ERR_UNSUPPORTED, "decode_chain: device index %d", dev);
    if (cached[dev] == 0) {
        int cus = 0, occ = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            return set_error(EFM_ERR_DEVICE, "decode_chain: cannot read the CU count");
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, decode_chain_kernel, kChainThreads, 0) != hipSuccess ||
            occ < 1)
            return set_error(EFM_ERR_UNSUPPORTED, "decode_chain: kernel does not fit on a CU");
        cached[dev] = cus;
    }
    *grid = cached[dev];
    return EFM_OK;
}

static int chain_check(const efm_attention_ctx* ctx, int hidden, int inter, uint32_t max_kv_len, int grid) {
    int rc = validate_attention_ctx(ctx, "decode_chain");
    if (rc) return rc;
    const int hd = (int)ctx->head_dim, Hq = (int)ctx->num_qo_heads, Hkv = (int)ctx->num_kv_heads;
    const int QD = Hq * hd, KVD = Hkv * hd;
    auto cdiv = [](int x, int y) { return (x + y - 1) / y; };
    if (hidden <= 0 || inter <= 0 || hidden % 8 || inter % 8)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_chain: hidden %d / inter %d must be positive multiples of 8",
                         hidden, inter);
    if (hidden > kChainMaxK || QD > kChainMaxK || inter > kChainMaxInter || Hq > kChainMaxHeads)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_chain: hidden %d, q_dim %d, inter %d or %d heads too large",
                         hidden, QD, inter, Hq);
    if (cdiv(hidden, grid) > kChainWorkers || cdiv(QD + 2 * KVD, grid) > kChainWorkers ||
        cdiv(inter, grid) > kChainWorkers * kChainMaxOut ||
        (size_t)cdiv(hidden, grid) * (size_t)inter * 2 > (size_t)kChainStageBytes)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_chain: layer too large for %d workgroups", grid);
    if (decode_split_cap(Hkv, std::max<uint32_t>(max_kv_len, 1u)) > kChainMaxSplit)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_chain: max_kv_len %u needs more than %d attention splits",
                         max_kv_len, kChainMaxSplit);
    return EFM_OK;
}

}  // namespace efm

using namespace efm;

extern "C" size_t efm_decode_chain_workspace_bytes(int32_t hidden, int32_t inter) {
    if (hidden <= 0 || inter <= 0) return 0;
    return chain_ws(hidden, inter).total;
}

extern "C" int efm_decode_chain_supported(const efm_attention_ctx* ctx, int32_t hidden, int32_t inter,
                                          uint32_t max_kv_len) {
    int grid = 0;
    int rc = chain_grid(&grid);
    if (rc) return rc;
    return chain_check(ctx, hidden, inter, max_kv_len, grid);
}

extern "C" int efm_decode_layer_chain(const efm_attention_ctx* ctx, int32_t hidden, int32_t inter, float eps,
                                      const efm_decode_chain_layer* layer, const uint32_t* d_kv_len,
                                      uint32_t max_kv_len, const void* attn_workspace, size_t attn_workspace_bytes,
                                      const void* residual_in, void* residual_out, void* hidden_out,
                                      void* chain_workspace, size_t chain_workspace_bytes, hipStream_t stream) {
    int grid = 0;
    int rc = chain_grid(&grid);
    if (rc) return rc;
    rc = chain_check(ctx, hidden, inter, max_kv_len, grid);
    if (rc) return rc;
    if (layer == nullptr || d_kv_len == nullptr || attn_workspace == nullptr || residual_in == nullptr ||
        residual_out == nullptr || chain_workspace == nullptr || layer->w_o == nullptr ||
        layer->post_norm == nullptr || layer->w_up_gate == nullptr || layer->w_down == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_chain: null pointer");
    if (max_kv_len == 0) return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_chain: max_kv_len must be > 0");
    const bool last = layer->in_norm_next == nullptr;
    if (last && hidden_out == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_chain: the last layer needs hidden_out");
    if (!last && (layer->w_qkv_next == nullptr || layer->b_qkv_next == nullptr || layer->q_next == nullptr ||
                  layer->k_cache_next == nullptr || layer->v_cache_next == nullptr))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_chain: next-layer pointers missing");
    if (residual_in == residual_out)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_chain: residual_in and residual_out must differ");
    if (attn_workspace_bytes < decode_workspace_bytes(ctx, max_kv_len))
        return set_error(EFM_ERR_WORKSPACE, "decode_chain: attention workspace too small");
    const ChainWs ws = chain_ws(hidden, inter);
    if (chain_workspace_bytes < ws.total)
        return set_error(EFM_ERR_WORKSPACE, "decode_chain: chain workspace of %zu bytes required", ws.total);
    const uintptr_t align_or = reinterpret_cast<uintptr_t>(residual_in) | reinterpret_cast<uintptr_t>(residual_out) |
                               reinterpret_cast<uintptr_t>(hidden_out) | reinterpret_cast<uintptr_t>(layer->w_o) |
                               reinterpret_cast<uintptr_t>(layer->w_up_gate) |
                               reinterpret_cast<uintptr_t>(layer->w_down) |
                               reinterpret_cast<uintptr_t>(layer->post_norm) |
                               reinterpret_cast<uintptr_t>(layer->in_norm_next) |
                               reinterpret_cast<uintptr_t>(layer->w_qkv_next);
    if (align_or & 15u) return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_chain: pointers must be 16-byte aligned");

    const int hd = (int)ctx->head_dim, Hq = (int)ctx->num_qo_heads, Hkv = (int)ctx->num_kv_heads;
    ChainArgs a;
    a.H = hidden;
    a.QD = Hq * hd;
    a.KVD = Hkv * hd;
    a.I = inter;
    a.HD = hd;
    a.G = Hq / Hkv;
    a.Hq = Hq;
    a.eps = eps;
    a.w_o = static_cast<const bf16_t*>(layer->w_o);
    a.post_norm = static_cast<const bf16_t*>(layer->post_norm);
    a.w_gu = static_cast<const bf16_t*>(layer->w_up_gate);
    a.w_down = static_cast<const bf16_t*>(layer->w_down);
    a.in_norm_next = static_cast<const bf16_t*>(layer->in_norm_next);
    a.w_qkv_next = static_cast<const bf16_t*>(layer->w_qkv_next);
    a.b_qkv_next = static_cast<const bf16_t*>(layer->b_qkv_next);
    a.q_next = static_cast<bf16_t*>(layer->q_next);
    a.k_cache_next = static_cast<bf16_t*>(layer->k_cache_next);
    a.v_cache_next = static_cast<bf16_t*>(layer->v_cache_next);
    a.o_part = static_cast<const float*>(attn_workspace);
    a.ml_part = reinterpret_cast<const float*>(static_cast<const char*>(attn_workspace) +
                                               decode_ml_offset(ctx, max_kv_len));
    a.split_cap = decode_split_cap(Hkv, max_kv_len);
    a.keys_per_split = decode_keys_per_split(Hkv, max_kv_len);
    a.d_kv_len = d_kv_len;
    a.max_kv_len = max_kv_len;
    a.r_in = static_cast<const bf16_t*>(residual_in);
    a.r_out = static_cast<bf16_t*>(residual_out);
    a.h_out = static_cast<bf16_t*>(hidden_out);
    char* w = static_cast<char*>(chain_workspace);
    a.xa = reinterpret_cast<uint32_t*>(w + ws.xa);
    a.xh = reinterpret_cast<uint32_t*>(w + ws.xh);
    a.xmid = reinterpret_cast<uint32_t*>(w + ws.xmid);
    a.epoch = reinterpret_cast<uint32_t*>(w + ws.epoch);
    a.abort_flag = reinterpret_cast<uint32_t*>(w + ws.abort_flag);
    a.trace = reinterpret_cast<uint64_t*>(w + ws.abort_flag + 256);
    a.last = last ? 1 : 0;
    hipLaunchKernelGGL(decode_chain_kernel, dim3(grid), dim3(kChainThreads), 0, stream, a);
    return check_launch("decode_chain");
}

extern "C" int efm_decode_chain_status(void* chain_workspace, int32_t hidden, int32_t inter, hipStream_t stream) {
    if (chain_workspace == nullptr || hidden <= 0 || inter <= 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_chain_status: bad arguments");
    const ChainWs ws = chain_ws(hidden, inter);
    uint32_t flag = 0;
    char* p = static_cast<char*>(chain_workspace) + ws.abort_flag;
    if (hipMemcpyAsync(&flag, p, 4, hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return set_error(EFM_ERR_DEVICE, "decode_chain_status: cannot read the abort flag");
    if (flag == 0u) return EFM_OK;
    const uint32_t zero = 0;
    (void)hipMemcpyAsync(p, &zero, 4, hipMemcpyHostToDevice, stream);
    (void)hipStreamSynchronize(stream);
    return set_error(EFM_ERR_DEVICE,
                     "decode_chain: a workgroup did not receive its inputs in time (not every workgroup was "
                     "resident?); results of the affected steps are invalid");
}

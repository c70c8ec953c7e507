// Device code of the LDS-staged decode attention (head_dim 128, rotated K cache), shared
// by efm_attention_decode / efm_decode_attention_partials (attention_decode.hip) and the
// fused QKV projection + attention kernel (decode_qkv_attention.hip).
#pragma once

#include "attn_pipe.hpp"
#include "common.hpp"

#include <type_traits>

namespace efm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kTileKeys = 32;
constexpr int kMaxSplits = 512;  // split_cap <= 512 / num_kv_heads (two workgroups per CU)
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeArgs {
    const bf16_t* q;
    const bf16_t* k;
    const bf16_t* v;
    bf16_t* o;
    uint32_t kv_len;
    const uint32_t* d_kv_len;
    uint32_t max_kv_len;
    int num_kv_heads;
    int q_sn, q_sh, k_sn, k_sh, v_sn, v_sh;   // element strides
    int q_pos_off, k_pos_off;
    int rope_q;                               // rotate q (and, by ROTK / fix_last, keys)
    int fix_last;                             // rotate + store back row L - 1 (ROTK = false)
    int row_bound;                            // rows that may be read (allocation bound)
    int split_cap;                            // gridDim.x
    int keys_per_split;                       // keys of split b: [b * kps, (b + 1) * kps)
    float* o_part;                            // [Hkv][split_cap][G][HD]
    float* ml_part;                           // [Hkv][split_cap][G][2]
    uint32_t* counter;                        // [Hkv] (reserved in the workspace, unused)
    RopeTable rope;
};

union BfPack {
    bf16x8_t v;
    uint4 u;
    uint32_t w[4];
};

// Tagged-word exchange of the fused QKV + attention kernel. The GEMV workgroups publish
// every projected row n as words[n] = bf16 bits | tag << 16 (agent-scope atomic exchange,
// visible across XCDs without cache flushes); the attention workgroups poll the words they
// need. sync = {epoch, done, abort}: the tag of a launch is epoch % 65535 + 1 (never 0,
// and different from the previous launch, whose words a poll may still see); the last
// attention workgroup to finish polling advances the epoch and clears `done`. Polls are
// bounded: on time-out they raise `abort` (reported by efm_decode_qkv_attention_status)
// and go on with zeros for the words that did not arrive, so the launch always drains
// (its outputs are then wrong, and the status call says so).
struct FusedAttnArgs {
    const uint32_t* words;   // [q_dim + 2 kv_dim]
    uint32_t* sync;          // [0] epoch, [1] done, [2] abort
    int q_dim, kv_dim;
    uint32_t n_attn;         // attention workgroups of the launch
    uint32_t spin_limit;     // polls before a wait gives up (kFusedSpin)
    uint32_t tag_or;         // OR-ed into the awaited tag: 0, or 1 << 16 (test hook: no word matches)
};

constexpr uint32_t kFusedSpin = 1u << 20;
constexpr uint32_t kWloadSkipAttn = 0x80000000u;   // past every buffer resource the attention builds
constexpr uint32_t kFusedTestSpin = 64u;   // spin limit of the forced time-out (test hook)

// Polls words addr(k) for every k set in `pending` until each carries `tag`; every round
// issues the loads of all words still pending before checking any.
template <int NW, class Addr>
__device__ __forceinline__ void fused_poll(uint32_t (&w)[NW], uint32_t pending, uint32_t tag, Addr addr,
                                           uint32_t* sync, uint32_t spin_limit) {
#pragma unroll
    for (int k = 0; k < NW; ++k) w[k] = 0u;
    uint32_t spins = 0;
    while (pending != 0u) {
        uint32_t v[NW];
#pragma unroll
        for (int k = 0; k < NW; ++k)
            v[k] = (pending >> k & 1u) ? __hip_atomic_load(addr(k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
#pragma unroll
        for (int k = 0; k < NW; ++k)
            if ((pending >> k & 1u) && (v[k] >> 16) == tag) {
                w[k] = v[k];
                pending &= ~(1u << k);
            }
        if (pending == 0u) break;
        if (++spins > spin_limit) {
            __hip_atomic_store(sync + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// One thread per attention workgroup, once it needs no more words.
__device__ __forceinline__ void fused_attn_done(const FusedAttnArgs& f) {
    const uint32_t prev = __hip_atomic_fetch_add(f.sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == f.n_attn - 1u) {
        __hip_atomic_store(f.sync + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        (void)__hip_atomic_fetch_add(f.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Context length for the decode kernels, read through the scalar cache after the first
// tile loads have gone out: a plain load there would be a vector load (the tile loads may
// write memory, as far as the compiler knows), and its wait would cover every tile.
__device__ __forceinline__ uint32_t decode_len(const DecodeArgs& a) {
    if (a.d_kv_len == nullptr) return a.kv_len;
    uint32_t v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(a.d_kv_len) : "memory");
    return min(v, a.max_kv_len);
}

// Workgroup barrier for LDS data only: __syncthreads() also waits for every outstanding
// global load (its fence counts the K / V tiles still streaming into LDS).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// LDS-staged variant for head_dim 128 with a rotated cache (ROTK = false): each round
// stages 128 keys of K and V with buffer loads straight into LDS (1 KB wave loads: 4 rows x
// 256 bytes, so every load instruction reads whole 256-byte row pieces), in the layouts of
// attn_pipe.hpp. Wave w then takes the keys [32 w, 32 w + 32) of the round: the K operand
// of S^T = K . Q^T comes from ds_read_b128, the V^T operand of O^T = V^T . P^T from
// ds_read_b64_tr_b16 (no transpose through registers). Rows past the length are masked
// in the scores and their V rows are zeroed in LDS (stale cache rows may hold NaN).
//
// FUSED = true: the body runs inside the fused QKV + attention kernel, whose GEMV
// workgroups produce this step's query and newest K/V row while the split's K/V tiles
// load. The query and the newest row are then taken from the GEMV's tagged words (see
// FusedAttnArgs); the owning split stores the rotated newest key into the cache.
template <int G, bool MERGE, bool FUSED>
__device__ __forceinline__ void decode_attn_lds_body(const DecodeArgs& a, int b, int kvh, const FusedAttnArgs& f) {
    constexpr int HD = 128, HALF = 64, KS = 8, DT = 4;
    constexpr int RK = kAttnWaves * kTileKeys;                // keys per round
    constexpr int TILE = RK * attn_pipe::kRow;                 // bytes of K (or V) per round
    constexpr int LPW = 2 * TILE / 1024 / kAttnWaves;          // 1 KB wave loads per wave per round
    static_assert(G <= 32, "group too large");
    static_assert((kAttnWaves * G * (HD + 8) + 2 * kAttnWaves * 32) * 4 <= 2 * TILE,
                  "merge buffers must fit the tiles");
    __shared__ __align__(1024) unsigned char smem[2 * TILE];   // K | V of one round; then the wave merge
    __shared__ float2 cs_qk[2][HALF];
    __shared__ __align__(16) bf16_t qs[G * HD];   // the group's queries as read
    __shared__ __align__(16) bf16_t qr[G * HD];   // rotated and scaled: the MFMA operand

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int ql = lane % 32, hh = lane / 32;
    const int kps = a.keys_per_split;
    const int start = b * kps;
    const bf16_t* kbase = a.k + (size_t)kvh * a.k_sh;
    const bf16_t* vbase = a.v + (size_t)kvh * a.v_sh;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);

    // ---- 1. loads that do not depend on L: the query, the first round of K / V (rows
    //         below the allocation bound), the RoPE frequencies
    const uint32_t tag = FUSED ? (launch_tag(f.sync) | f.tag_or) : 0u;
    // the group's G x 128 queries, 16 bytes per thread (staged in LDS below)
    uint4 qld = make_uint4(0, 0, 0, 0);
    if (!FUSED && tid < G * (HD / 8))
        qld = *reinterpret_cast<const uint4*>(a.q + (size_t)(kvh * G + tid / (HD / 8)) * a.q_sh + (tid % (HD / 8)) * 8);
    const int lim = min(a.row_bound, start + kps) - 1;   // last row this split may read
    // uniform copies read before the first tile loads: read after them, a kernel argument
    // or the length would come through a vector load that waits for every tile load
    const int k_sn = __builtin_amdgcn_readfirstlane(a.k_sn), v_sn = __builtin_amdgcn_readfirstlane(a.v_sn);
    // Tile loads are buffer loads straight into LDS (byte offsets below 2 GB: host-checked),
    // which the compiler counts exactly, so the prologue's waits for its own loads (issued
    // first) do not wait for the tiles.
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t*>(kbase), (short)0, __builtin_amdgcn_readfirstlane(a.row_bound * k_sn * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16_t*>(vbase), (short)0, __builtin_amdgcn_readfirstlane(a.row_bound * v_sn * 2), 0x00020000);
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    auto issue = [&](int r) {
        const int k0 = start + r * RK;
        const int pr = lane >> 4, pc = lane & 15;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int q = wu + i * kAttnWaves;                 // wave-load index: K 0..31, V 32..63
            constexpr int HL = TILE / 1024 / kAttnWaves;          // loads per wave per operand
            const bool isv = i >= HL;                              // = q >= TILE / 1024 (wu < 4)
            const int row = (wu + (i % HL) * kAttnWaves) * 4 + pr;
            const int c = isv ? (pc ^ ((row & 3) << 2)) : (pc ^ (row & 15));
            const int j = min(k0 + row, lim);
            const uint32_t off = (uint32_t)(j * (isv ? v_sn : k_sn) + c * 8) * 2u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(isv ? rv : rk,
                                                     (__attribute__((address_space(3))) void*)(smem + q * 1024), 16,
                                                     off, 0, 0, 0);
        }
    };
    const float freq = (a.rope_q && tid < 2 * HALF) ? a.rope.inv_freq[tid % HALF] : 0.f;
    const int q_pos_off = __builtin_amdgcn_readfirstlane(a.q_pos_off);
    const int k_pos_off = __builtin_amdgcn_readfirstlane(a.k_pos_off);
    issue(0);

    // ---- 2. the context length and this split's key range [start, end)
    const uint32_t L = decode_len(a);
    const int nsplit = (L == 0) ? 1 : (int)((L + kps - 1) / kps);
    if (b >= nsplit) {
        attn_pipe::vm_wait<0>();   // no LDS write may outlive the workgroup
        if (FUSED && tid == 0) fused_attn_done(f);
        return;
    }
    const int end = min((int)L, start + kps);
    const int rounds = (end > start) ? (end - start + RK - 1) / RK : 0;

    // ---- 3. RoPE at the query position and at the newest key's position
    if (a.rope_q && tid < 2 * HALF) {
        const int pos = (int)L - 1 + (tid < HALF ? q_pos_off : k_pos_off);
        float sn, cs;
        sincos_reduced((float)pos * freq, &sn, &cs);
        cs_qk[tid / HALF][tid % HALF] = make_float2(cs, sn);
    }
    if (!FUSED && tid < G * (HD / 8)) *reinterpret_cast<uint4*>(&qs[tid * 8]) = qld;
    lds_barrier();
    // FUSED: wait for this step's query words (and, in the split that owns row L - 1,
    // the newest K / V row: thread t < 128 takes K[t], t >= 128 takes V[t - 128])
    const bool owner = FUSED && L > 0 && (int)L - 1 >= start && (int)L - 1 < end;
    uint32_t newest = 0u;
    if (FUSED) {
        constexpr int NQW = (G * HD + kAttnThreads - 1) / kAttnThreads;
        uint32_t w[NQW + 1];
        uint32_t pending = 0u;
#pragma unroll
        for (int k = 0; k < NQW; ++k)
            if (tid + k * kAttnThreads < G * HD) pending |= 1u << k;
        const uint32_t* qw = f.words + (size_t)kvh * G * HD;
        const uint32_t* nw = f.words + f.q_dim + (tid < HD ? 0 : f.kv_dim) + kvh * HD + (tid % HD);
        if (owner) pending |= 1u << NQW;
        fused_poll<NQW + 1>(w, pending, tag, [&](int k) { return k < NQW ? qw + tid + k * kAttnThreads : nw; },
                            f.sync, f.spin_limit);
#pragma unroll
        for (int k = 0; k < NQW; ++k)
            if (tid + k * kAttnThreads < G * HD) qs[tid + k * kAttnThreads] = (bf16_t)(w[k] & 0xffffu);
        newest = w[NQW] & 0xffffu;
        lds_barrier();
    }
    // rotate (pairs d, d + 64 at the query position) and scale by log2(e) / sqrt(hd), one
    // element per thread and step (independent LDS reads, no serial chain), then every
    // lane reads its MFMA operand fragments
    {
        const float qscale = kLog2e / sqrtf((float)HD);
#pragma unroll
        for (int k = 0; k < (G * HD + kAttnThreads - 1) / kAttnThreads; ++k) {
            const int i = tid + k * kAttnThreads;
            if (i < G * HD) {
                const int d = i % HD;
                const float x = bf16_to_f32(qs[i]);
                float r = x;
                if (a.rope_q) {
                    const float y = bf16_to_f32(qs[i ^ HALF]);   // the pair partner d +- 64
                    const float2 c2 = cs_qk[0][d % HALF];
                    r = (d < HALF) ? x * c2.x - y * c2.y : x * c2.x + y * c2.y;
                }
                qr[i] = (bf16_t)f32_to_bf16(r * qscale);
            }
        }
    }
    lds_barrier();
    bf16x8_t qf[KS];
    {
        const bool qv = ql < G;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            BfPack pk;
            pk.u = qv ? *reinterpret_cast<const uint4*>(&qr[ql * HD + ks * 16 + hh * 8]) : make_uint4(0, 0, 0, 0);
            qf[ks] = pk.v;
        }
    }
    const int fix_row = (a.rope_q && a.fix_last && L > 0) ? (int)L - 1 : -1;

    f32x16_t oacc[DT];
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[tt][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    uint32_t koff[KS], voff[DT];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) koff[ks] = lds0 + attn_pipe::k_off(wave * 32 + ql, ks * 2 + hh);
#pragma unroll
    for (int tt = 0; tt < DT; ++tt) voff[tt] = lds0 + (uint32_t)TILE + (uint32_t)(wave * 32 * attn_pipe::kRow) +
                                               attn_pipe::v_tr_lane_off(lane, tt);
    typedef short s4_t __attribute__((ext_vector_type(4)));

    for (int r = 0; r < rounds; ++r) {
        const int k0 = start + r * RK;
        if (r > 0) {
            __syncthreads();   // every wave is done with the previous round's tiles
            issue(r);
        }
        attn_pipe::vm_wait<0>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (FUSED && owner) {
            // the newest row, as published this step, over its stale prefetched copy
            const int rr = (int)L - 1 - k0, d = tid % HD, c = d >> 3;
            const int slot = (tid < HD) ? rr * attn_pipe::kRow + ((c ^ (rr & 15)) << 4)
                                        : TILE + rr * attn_pipe::kRow + ((c ^ ((rr & 3) << 2)) << 4);
            *reinterpret_cast<bf16_t*>(smem + slot + (d & 7) * 2) = (bf16_t)newest;
            __syncthreads();
        }
        if (end < k0 + RK) {
            // zero the V rows past the length (P is 0 there, but the rows may hold NaN)
            for (int i = tid; i < (k0 + RK - end) * 16; i += kAttnThreads) {
                const int row = end - k0 + i / 16;
                *reinterpret_cast<uint4*>(smem + TILE + row * attn_pipe::kRow + (i % 16) * 16) = make_uint4(0, 0, 0, 0);
            }
            __syncthreads();
        }
        const int t0 = k0 + wave * 32;
        if (t0 >= end) continue;
        bf16x8_t kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) attn_pipe::read_b128<0>(kf[ks], koff[ks]);
        s4_t vf[2][DT][2];
        auto read_v = [&](auto kbc) {
            constexpr int kb = decltype(kbc)::value;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) {
                attn_pipe::read_tr16<(kb * 16) * attn_pipe::kRow>(vf[kb][tt][0], voff[tt]);
                attn_pipe::read_tr16<(kb * 16 + 8) * attn_pipe::kRow>(vf[kb][tt][1], voff[tt]);
            }
        };
        read_v(std::integral_constant<int, 0>{});
        asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");   // the K reads (issued first) are done
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kf[ks]));
        if (t0 + ql == fix_row && fix_row < end) {
            // the newest key: rotate at its position, use it and store it back rotated
            bf16_t* kw = const_cast<bf16_t*>(kbase) + (size_t)fix_row * a.k_sn + hh * 8;
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
                    const float2 c2 = cs_qk[1][ks * 16 + hh * 8 + e];
                    const float y0 = x0[e] * c2.x - x1[e] * c2.y;
                    const float y1 = x1[e] * c2.x + x0[e] * c2.y;
                    x0[e] = y0;
                    x1[e] = y1;
                }
                u0.u = pack8(x0);
                u1.u = pack8(x1);
                kf[ks] = u0.v;
                kf[ks + KS / 2] = u1.v;
                *reinterpret_cast<uint4*>(kw + ks * 16) = u0.u;
                *reinterpret_cast<uint4*>(kw + (ks + KS / 2) * 16) = u1.u;
            }
        }
        f32x16_t s = {};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], s, 0, 0, 0);
        read_v(std::integral_constant<int, 1>{});
        // element e: key = t0 + (e/4)*8 + hh*4 + e%4, head = ql
        if (t0 + 32 > end) {
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
        if (r == 0) {
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
                    if (kb == 0) asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
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

    // ---- merge the 4 waves through LDS (the tile buffers are free now): every output is
    //      the fixed-order sum of sc_w o_w with the wave weights sc_w = exp2(m_w - M) of
    //      its head (M the running max over the waves) and den = sum sc_w l_w. A wave's 64
    //      outputs of one pass all belong to one head, so each wave derives that head's
    //      weights itself from the (m, l) words (no second barrier). Rows of o_w are padded
    //      to HD + 8 floats: the 16-byte writes of lanes (ql, hh) then fall in distinct banks.
    constexpr int OBS = HD + 8;
    __syncthreads();
    float* om = reinterpret_cast<float*>(smem);                  // [4][32]
    float* ol = om + kAttnWaves * 32;                            // [4][32]
    float* ob = ol + kAttnWaves * 32;                            // [4][G][OBS]
    if (hh == 0) {
        om[wave * 32 + ql] = m_run;
        ol[wave * 32 + ql] = l_run;
    }
    if (ql < G) {
#pragma unroll
        for (int tt = 0; tt < DT; ++tt)
#pragma unroll
            for (int eb = 0; eb < 4; ++eb)
                *reinterpret_cast<float4*>(&ob[(wave * G + ql) * OBS + tt * 32 + eb * 8 + hh * 4]) =
                    make_float4(oacc[tt][eb * 4 + 0], oacc[tt][eb * 4 + 1], oacc[tt][eb * 4 + 2], oacc[tt][eb * 4 + 3]);
    }
    __syncthreads();
    float* o_part = a.o_part + ((size_t)kvh * a.split_cap + b) * G * HD;
    float* ml_part = a.ml_part + ((size_t)kvh * a.split_cap + b) * G * 2;
    constexpr int NO = (G * HD + kAttnThreads - 1) / kAttnThreads;
    static_assert(HD % kWave == 0 && kAttnWaves == 4, "a wave's outputs of one pass share a head; quads hold the waves");
#pragma unroll
    for (int k = 0; k < NO; ++k) {
        const int i = tid + k * kAttnThreads;
        if (i >= G * HD) break;
        const int g = i / HD, d = i % HD;
        // lane w of every quad takes wave w's (m, l): one exp for the four weights, the
        // max over the quad through DPP, the weights handed to the wave by readlane
        const int wl = lane & (kAttnWaves - 1);
        const float mw = om[wl * 32 + g], lw = ol[wl * 32 + g];
        float M = fmaxf(mw, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mw), 0xB1, 0xf, 0xf, false)));
        M = fmaxf(M, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(M), 0x4E, 0xf, 0xf, false)));
        const float scl = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float sc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scl), w));
            den = fmaf(sc, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lw), w)), den);
            num = fmaf(sc, ob[(w * G + g) * OBS + d], num);
        }
        if (MERGE) {
            a.o[(size_t)(kvh * G + g) * HD + d] = (bf16_t)f32_to_bf16(den > 0.f ? num / den : 0.f);
        } else {
            o_part[i] = num;
            if (d == 0) *reinterpret_cast<float2*>(&ml_part[g * 2]) = make_float2(M, den);
        }
    }
    // FUSED: counted in only now (the returning atomic stays off the critical path); every
    // word this workgroup needed arrived long before
    if (FUSED && tid == 0) fused_attn_done(f);
}

// Wide variant for long contexts (head_dim 128, unfused launches): one
// 8-wave workgroup per CU holds every 32-key tile of its split in LDS (up to
// kWideMaxTiles: 288 keys, 144 KB), all requested at the start; wave w computes the tiles
// w and w + 8 (a split need not be whole tiles: rows past its end read as zeros and are
// masked). Eight waves per CU keep more K/V loads in flight than the 4-wave kernel's
// two workgroups, whose 256-key splits at 16k keys had to load their second 128-key
// round after the first. The loads are buffer loads straight into LDS, issued before the
// length is known; rows past the split's last readable row read past the resource (no
// memory access) and land as zeros.
// ROTK = true: every key is rotated on read at its position (the reference's un-rotated
// cache); each wave computes its tile's cos / sin before waiting for the tile, under the
// load phase. ROTK = false: keys are used as stored, and with a.fix_last row L - 1 is
// rotated, used and stored back by the lane that holds it.
constexpr int kWideWaves = 8;
constexpr int kWideThreads = kWideWaves * kWave;
constexpr int kWideMaxTiles = 9;
constexpr int kWideTileBytes = 2 * kTileKeys * attn_pipe::kRow;   // K and V of one tile

__device__ __forceinline__ void wide_lds_load(__amdgpu_buffer_rsrc_t rs, uint32_t lds_addr, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(uintptr_t)lds_addr, 16, off,
                                             0, 0, 0);
}

template <int G, bool MERGE, bool ROTK>
__device__ __forceinline__ void decode_attn_wide_body(const DecodeArgs& a, int b, int kvh) {
    constexpr int HD = 128, HALF = 64, KS = 8, DT = 4, W = kWideWaves, NT = kWideThreads;
    constexpr int KB = kTileKeys * attn_pipe::kRow;            // bytes of K (or V) of a tile
    constexpr int LPT = 2 * KB / 1024;                         // 1 KB wave loads per tile
    static_assert((W * G * (HD + 8) + 2 * W * 32) * 4 <= kWideMaxTiles * kWideTileBytes,
                  "merge buffers must fit the tiles");
    __shared__ __align__(1024) unsigned char smem[kWideMaxTiles * kWideTileBytes];   // tiles; then the merge
    __shared__ float2 cs_qk[2][HALF];
    __shared__ float sfreq[ROTK ? HALF : 1];
    // ROTK: (cos, sin) as fp16 pairs for the keys of tile W (wave 0's second tile), row =
    // key, 16-byte chunks XOR-swizzled by the row; built by every thread during set-up
    __shared__ __align__(16) uint32_t cs9[ROTK ? kTileKeys * HALF : 1];
    __shared__ __align__(16) bf16_t qs[G * HD];
    __shared__ __align__(16) bf16_t qr[G * HD];

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int ql = lane % 32, hh = lane / 32;
    const int kps = a.keys_per_split;
    const int start = b * kps;
    const int ntiles = (kps + kTileKeys - 1) / kTileKeys;      // <= kWideMaxTiles (host-checked)
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);

    // ---- 1. the query and the RoPE frequencies, then every tile of the split (rows below
    //         the allocation bound; the length is not known yet)
    uint4 qld = make_uint4(0, 0, 0, 0);
    if (tid < G * (HD / 8))
        qld = *reinterpret_cast<const uint4*>(a.q + (size_t)(kvh * G + tid / (HD / 8)) * a.q_sh + (tid % (HD / 8)) * 8);
    const float freq = (a.rope_q && tid < 2 * HALF) ? a.rope.inv_freq[tid % HALF] : 0.f;
    const int q_pos_off = __builtin_amdgcn_readfirstlane(a.q_pos_off);
    const int k_pos_off = __builtin_amdgcn_readfirstlane(a.k_pos_off);
    // ROTK: cos / sin of this lane's key in its first tile (t0 + ql) for its d = 16 ks + 8 hh
    // + e, ks < KS / 2. The tile loads are bound by the address unit, which takes the
    // workgroup's requests in turn: waves W/2.. compute theirs before issuing their loads
    // (while the unit works through the first half's requests), waves ..W/2-1 after
    // issuing theirs (while it works through the second half's).
    float2 ck[ROTK ? KS / 2 : 1][8];
    const bool ck_early = ROTK && __builtin_amdgcn_readfirstlane(wave) >= W / 2;
    if (ck_early) {
        const float pos = (float)(start + wave * kTileKeys + ql + k_pos_off);
#pragma unroll
        for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // both candidates as uniform (scalar) loads, then a per-lane select
                const float flo = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(a.rope.inv_freq[ks * 16 + e])));
                const float fhi = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(a.rope.inv_freq[ks * 16 + 8 + e])));
                const float f = hh ? fhi : flo;
                float sn, cs;
                sincos_reduced(pos * f, &sn, &cs);
                ck[ks][e] = make_float2(cs, sn);
            }
    }
    {
        const int lim = min(a.row_bound, start + kps) - 1;   // last row this split may read
        const int nrec = __builtin_amdgcn_readfirstlane(a.row_bound * a.k_sn * 2);
        const int nrecv = __builtin_amdgcn_readfirstlane(a.row_bound * a.v_sn * 2);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<bf16_t*>(a.k + (size_t)kvh * a.k_sh), (short)0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<bf16_t*>(a.v + (size_t)kvh * a.v_sh), (short)0, nrecv, 0x00020000);
        const int pr = lane >> 4, pc = lane & 15;
        const int wu = __builtin_amdgcn_readfirstlane(wave);
        // Only wave 0 can have a second tile (ntiles <= W + 1); the other waves issue no
        // loads for it (load requests that read nothing still take address-unit time: with
        // seven waves issuing a skipped tile the 16k call took 1 us longer).
        const uint32_t smem_a = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int t = wu + i * W;
            if (i == 1 && t >= ntiles) break;
            const uint32_t slot = smem_a + (uint32_t)(t * kWideTileBytes);
            const int k0 = start + t * kTileKeys;
#pragma unroll
            for (int q = 0; q < LPT; ++q) {
                const bool isv = q >= KB / 1024;                 // loads 0..7: K rows, 8..15: V rows
                const int row = (q % (KB / 1024)) * 4 + pr;       // row of the tile
                const int c = isv ? (pc ^ ((row & 3) << 2)) : (pc ^ (row & 15));
                // rows past the split's last readable row read nothing (zeros)
                const uint32_t rowm = k0 + row <= lim ? ~0u : 0u;
                const uint32_t off = ((uint32_t)((k0 + row) * (isv ? a.v_sn : a.k_sn) + c * 8) * 2u & rowm) |
                                     (kWloadSkipAttn & ~rowm);
                wide_lds_load(isv ? rv : rk, slot + (uint32_t)q * 1024u, off);
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
    //         rotated and scaled by log2(e) / sqrt(hd) into the MFMA operand
    if (a.rope_q && tid < 2 * HALF) {
        const int pos = (int)L - 1 + (tid < HALF ? q_pos_off : k_pos_off);
        float sn, cs;
        sincos_reduced((float)pos * freq, &sn, &cs);
        cs_qk[tid / HALF][tid % HALF] = make_float2(cs, sn);
        if (ROTK && tid < HALF) sfreq[tid] = freq;
    }
    if (tid < G * (HD / 8)) *reinterpret_cast<uint4*>(&qs[tid * 8]) = qld;
    lds_barrier();
    {
        const float qscale = kLog2e / sqrtf((float)HD);
#pragma unroll
        for (int k = 0; k < (G * HD + NT - 1) / NT; ++k) {
            const int i = tid + k * NT;
            if (i < G * HD) {
                const int d = i % HD;
                const float x = bf16_to_f32(qs[i]);
                float r = x;
                if (a.rope_q) {
                    const float y = bf16_to_f32(qs[i ^ HALF]);
                    const float2 c2 = cs_qk[0][d % HALF];
                    r = (d < HALF) ? x * c2.x - y * c2.y : x * c2.x + y * c2.y;
                }
                qr[i] = (bf16_t)f32_to_bf16(r * qscale);
            }
        }
    }
    if (ROTK && ntiles > W && start + W * kTileKeys < end) {
        // the (cos, sin) table of tile W: 32 keys x 64 frequencies, 4 entries per thread
#pragma unroll
        for (int k = 0; k < kTileKeys * HALF / NT; ++k) {
            const int e = tid + k * NT, j = e / HALF, d = e % HALF;
            float sn, cs;
            sincos_reduced((float)(start + W * kTileKeys + j + k_pos_off) * sfreq[d], &sn, &cs);
            typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
            const h2_t h = {(_Float16)cs, (_Float16)sn};
            cs9[j * HALF + (((d >> 2) ^ (j & 15)) << 2) + (d & 3)] = __builtin_bit_cast(uint32_t, h);
        }
    }
    lds_barrier();
    bf16x8_t qf[KS];
    {
        const bool qv = ql < G;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            BfPack pk;
            pk.u = qv ? *reinterpret_cast<const uint4*>(&qr[ql * HD + ks * 16 + hh * 8]) : make_uint4(0, 0, 0, 0);
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
    for (int i = 0; i < 2; ++i) {
        const int t = wave + i * W;
        const int t0 = start + t * kTileKeys;
        // ROTK: the first tile's cos / sin (waves below W/2: now, before the wait); the
        // second tile, wave 0's ninth, reads them from the set-up table
        if (ROTK && i == 0 && !ck_early && t < ntiles && t0 < end) {
            const float pos = (float)(t0 + ql + k_pos_off);
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float sn, cs;
                    sincos_reduced(pos * sfreq[ks * 16 + hh * 8 + e], &sn, &cs);
                    ck[ks][e] = make_float2(cs, sn);
                }
        } else if (ROTK && i == 1 && t < ntiles && t0 < end) {
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int d0 = ks * 16 + hh * 8 + c * 4;   // 4 entries = one 16-byte chunk
                    const uint4 w = *reinterpret_cast<const uint4*>(
                        &cs9[ql * HALF + (((d0 >> 2) ^ (ql & 15)) << 2)]);
                    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
                        const h2_t h = __builtin_bit_cast(h2_t, wv[e]);
                        ck[ks][c * 4 + e] = make_float2((float)h.x, (float)h.y);
                    }
                }
        }
        if (i == 0 && wave + W < ntiles) attn_pipe::vm_wait<LPT>();   // tile 0 landed (the second may fly)
        else attn_pipe::vm_wait<0>();
        asm volatile("" ::: "memory");
        if (t >= ntiles || t0 >= end) continue;
        unsigned char* tile = smem + t * kWideTileBytes;
        const uint32_t sb = lds0 + (uint32_t)(t * kWideTileBytes);
        if (t0 + kTileKeys > end) {
            // zero the V rows past the length (P is 0 there, but the rows may hold NaN)
            for (int x = lane; x < (t0 + kTileKeys - end) * 16; x += kWave) {
                const int row = end - t0 + x / 16;
                *reinterpret_cast<uint4*>(tile + KB + row * attn_pipe::kRow + (x % 16) * 16) = make_uint4(0, 0, 0, 0);
            }
        }
        bf16x8_t kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) attn_pipe::read_b128<0>(kf[ks], sb + attn_pipe::k_off(ql, ks * 2 + hh));
        s4_t vf[2][DT][2];
        auto read_v = [&](auto kbc) {
            constexpr int kb = decltype(kbc)::value;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) {
                const uint32_t va = sb + (uint32_t)KB + attn_pipe::v_tr_lane_off(lane, tt);
                attn_pipe::read_tr16<(kb * 16) * attn_pipe::kRow>(vf[kb][tt][0], va);
                attn_pipe::read_tr16<(kb * 16 + 8) * attn_pipe::kRow>(vf[kb][tt][1], va);
            }
        };
        read_v(std::integral_constant<int, 0>{});
        asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");   // the K reads (issued first) are done
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kf[ks]));
        if (ROTK || (t0 + ql == fix_row && fix_row < end)) {
            // rotate this lane's key: every key (ROTK) or the newest one, which is then
            // stored back rotated
            bf16_t* kw = const_cast<bf16_t*>(kbase) + (size_t)max(fix_row, 0) * a.k_sn + hh * 8;
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
        if (i == 0) {
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
                    if (kb == 0) asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
                    else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                }
                asm volatile("" : "+v"(vf[kb][tt][0]), "+v"(vf[kb][tt][1]));
                union {
                    s4_t h[2];
                    bf16x8_t v;
                } vv;
                vv.h[0] = vf[kb][tt][0];
                vv.h[1] = vf[kb][tt][1];
                oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vv.v, pb[kb].v, oacc[tt], 0, 0, 0);
            }
    }

    // ---- merge the 8 waves through LDS (every tile load has landed: the waits above), as
    //      the 4-wave kernel's merge: rows of o_w padded to HD + 8 floats (distinct banks for
    //      the lanes' 16-byte writes), each wave deriving its head's wave weights itself
    //      (lane w of every octet takes wave w's (m, l): one exp, a DPP max over the octet,
    //      the weights handed to the wave by readlane), the fixed-order sum of sc_w o_w
    constexpr int OBS = HD + 8;
    __syncthreads();
    float* om = reinterpret_cast<float*>(smem);                  // [W][32]
    float* ol = om + W * 32;                                     // [W][32]
    float* ob = ol + W * 32;                                     // [W][G][OBS]
    if (hh == 0) {
        om[wave * 32 + ql] = m_run;
        ol[wave * 32 + ql] = l_run;
    }
    if (ql < G) {
#pragma unroll
        for (int tt = 0; tt < DT; ++tt)
#pragma unroll
            for (int eb = 0; eb < 4; ++eb)
                *reinterpret_cast<float4*>(&ob[(wave * G + ql) * OBS + tt * 32 + eb * 8 + hh * 4]) =
                    make_float4(oacc[tt][eb * 4 + 0], oacc[tt][eb * 4 + 1], oacc[tt][eb * 4 + 2], oacc[tt][eb * 4 + 3]);
    }
    __syncthreads();
    float* o_part = a.o_part + ((size_t)kvh * a.split_cap + b) * G * HD;
    float* ml_part = a.ml_part + ((size_t)kvh * a.split_cap + b) * G * 2;
    constexpr int NO = (G * HD + NT - 1) / NT;
    static_assert(HD % kWave == 0 && W == 8, "a wave's outputs of one pass share a head; octets hold the waves");
#pragma unroll
    for (int k = 0; k < NO; ++k) {
        const int i = tid + k * NT;
        if (i >= G * HD) break;
        const int g = i / HD, d = i % HD;
        const int wl = lane & (W - 1);
        const float mw = om[wl * 32 + g], lw = ol[wl * 32 + g];
        float M = fmaxf(mw, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(mw), 0xB1, 0xf, 0xf, false)));
        M = fmaxf(M, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(M), 0x4E, 0xf, 0xf, false)));
        M = fmaxf(M, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(M), 0x141, 0xf, 0xf, false)));
        const float scl = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float sc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scl), w));
            den = fmaf(sc, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lw), w)), den);
            num = fmaf(sc, ob[(w * G + g) * OBS + d], num);
        }
        if (MERGE) {
            a.o[(size_t)(kvh * G + g) * HD + d] = (bf16_t)f32_to_bf16(den > 0.f ? num / den : 0.f);
        } else {
            o_part[i] = num;
            if (d == 0) *reinterpret_cast<float2*>(&ml_part[g * 2]) = make_float2(M, den);
        }
    }
}

}  // namespace efm

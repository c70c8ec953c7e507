// Causal GQA prefill attention on the gfx950 matrix cores (bf16 in, fp32 softmax).
//
// Semantics (FlashInfer SinglePrefillWithKVCache with ROPE_LLAMA as called from
// src/operators/attention_op.cu:1345-1426): query row i (position i + q_rope_pos_offset)
// of head h attends keys j <= i + (L - S) of KV head h / (Hq/Hkv); with RoPE-Llama both
// q and k (at position j + k_rope_pos_offset) are rotated in the kernel.
//
// Kernel design (one workgroup = 4 wave64s = 128 query rows of one head):
//  * Scores are computed transposed, S^T = K . Q^T, with v_mfma_f32_32x32x16_bf16: the
//    K tile is the A operand (read from LDS), the wave's 32 query rows are the B operand
//    held in registers for the whole kernel. Each lane then owns one query row and 16
//    of the 32 keys of a sub-tile, so the online-softmax max / sum are in-lane plus one
//    cross-half exchange.
//  * The output is accumulated transposed as well, O^T = V^T . P^T: P stays in the
//    lanes that produced it (packed to bf16), V^T comes from LDS. The 16-key blocks of
//    P are in the MFMA accumulator's row order; V^T is read with the same key
//    permutation so the contraction is unchanged.
//  * RoPE is applied while staging: q pairs (d, d+hd/2) sit in the same lane, K pairs
//    are loaded together by one thread before the LDS store.
//  * Causal tiles past the diagonal are skipped; late query tiles are scheduled first.
#include "attn_pipe.hpp"
#include "common.hpp"

#include <algorithm>
#include <type_traits>
#include <cstdlib>

namespace efm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kPfThreads = 256;
constexpr int kPfQ = 128;   // query rows per workgroup (32 per wave)
constexpr int kPfKV = 64;   // keys per LDS tile

struct PrefillArgs {
    const bf16_t* q;
    const bf16_t* k;
    const bf16_t* v;
    bf16_t* o;
    int S, L, Hq, Hkv;
    int q_sn, q_sh, k_sn, k_sh, v_sn, v_sh;
    int o_sn, o_sh;
    int causal;
    int rope_q, rope_k;
    int q_pos_off, k_pos_off;
    float sm_scale_log2;
    RopeTable rope;
};

union Pack8 {
    bf16x8_t v;
    uint4 u;
    uint32_t w[4];
};

template <int HD>
__global__ __launch_bounds__(kPfThreads) void prefill_attn_kernel(PrefillArgs a) {
    constexpr int HALF = HD / 2;
    constexpr int KS = HD / 16;         // MFMA k-steps over head_dim
    constexpr int DT = HD / 32;         // 32-row d tiles of O^T
    constexpr int KP = HD + 8;          // LDS pitch of the K tile (bf16)
    constexpr int VP = kPfKV + 8;       // LDS pitch of the V^T tile (bf16)
    __shared__ __align__(16) bf16_t Ks[kPfKV * KP];
    __shared__ __align__(16) bf16_t Vt[HD * VP];
    __shared__ float sfreq[HALF];

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int ql = lane % 32, hh = lane / 32;
    const int nqt = (a.S + kPfQ - 1) / kPfQ;
    const int qt = nqt - 1 - (int)blockIdx.x;  // heavy (late) tiles first
    const int head = blockIdx.y;
    const int kvh = head / (a.Hq / a.Hkv);
    const int q0 = qt * kPfQ + wave * 32;
    const int qi = q0 + ql;                     // this lane's query row
    const int diag = a.L - a.S;                 // key j visible to row i iff j <= i + diag
    if (tid < HALF) sfreq[tid] = a.rope.inv_freq[tid];
    __syncthreads();

    // ---- Q (B operand) for this lane's row: d = ks*16 + hh*8 + e, kept in registers.
    Pack8 qf[KS];
    {
        float x[KS][8];
        const bool qv = qi < a.S;
        const bf16_t* qp = a.q + (size_t)(qv ? qi : 0) * a.q_sn + (size_t)head * a.q_sh;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint4 u = qv ? *reinterpret_cast<const uint4*>(qp + ks * 16 + hh * 8) : make_uint4(0, 0, 0, 0);
            unpack8(u, x[ks]);
        }
        if (a.rope_q) {
            const float pos = (float)(qi + a.q_pos_off);
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = ks * 16 + hh * 8 + e;  // < HALF; partner at ks + KS/2
                    float sn, cs;
                    sincosf(pos * sfreq[d], &sn, &cs);
                    const float x0 = x[ks][e], x1 = x[ks + KS / 2][e];
                    x[ks][e] = x0 * cs - x1 * sn;
                    x[ks + KS / 2][e] = x1 * cs + x0 * sn;
                }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[ks].u = pack8(x[ks]);
    }

    f32x16_t oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[t][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    const int q_last = min(a.S - 1, qt * kPfQ + kPfQ - 1);
    const int kv_end = a.causal ? min(a.L, q_last + diag + 1) : a.L;
    const int ntiles = (kv_end + kPfKV - 1) / kPfKV;

    const bf16_t* kbase = a.k + (size_t)kvh * a.k_sh;
    const bf16_t* vbase = a.v + (size_t)kvh * a.v_sh;
    // K staging: thread -> (key, 8 rotation pairs starting at kd0); kd0 is fixed per
    // thread because the thread count is a multiple of the pair-chunks per key.
    constexpr int KCH = HALF / 8;
    static_assert(kPfThreads % KCH == 0, "K staging assumes a fixed pair chunk per thread");
    const int kd0 = (tid % KCH) * 8;
    float kif[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) kif[e] = sfreq[kd0 + e];

    for (int t = 0; t < ntiles; ++t) {
        const int k0 = t * kPfKV;
        __syncthreads();
        // ---- stage K (rotated)
        for (int c = tid; c < kPfKV * KCH; c += kPfThreads) {
            const int kr = c / KCH, d0 = kd0;
            const int j = k0 + kr;
            uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
            if (j < kv_end) {
                const bf16_t* kp = kbase + (size_t)j * a.k_sn;
                lo = *reinterpret_cast<const uint4*>(kp + d0);
                hi = *reinterpret_cast<const uint4*>(kp + d0 + HALF);
                if (a.rope_k) {
                    float x0[8], x1[8];
                    unpack8(lo, x0);
                    unpack8(hi, x1);
                    const float pos = (float)(j + a.k_pos_off);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        float sn, cs;
                        sincos_reduced(pos * kif[e], &sn, &cs);
                        const float y0 = x0[e] * cs - x1[e] * sn;
                        const float y1 = x1[e] * cs + x0[e] * sn;
                        x0[e] = y0;
                        x1[e] = y1;
                    }
                    lo = pack8(x0);
                    hi = pack8(x1);
                }
            }
            *reinterpret_cast<uint4*>(&Ks[kr * KP + d0]) = lo;
            *reinterpret_cast<uint4*>(&Ks[kr * KP + d0 + HALF]) = hi;
        }
        // ---- stage V transposed: Vt[d][key]
        constexpr int VCH = HD / 8;
        for (int c = tid; c < kPfKV * VCH; c += kPfThreads) {
            const int kr = c / VCH, d0 = (c % VCH) * 8;
            const int j = k0 + kr;
            uint4 u = (j < kv_end) ? *reinterpret_cast<const uint4*>(vbase + (size_t)j * a.v_sn + d0)
                                   : make_uint4(0, 0, 0, 0);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                Vt[(d0 + 2 * e) * VP + kr] = (bf16_t)(w[e] & 0xffffu);
                Vt[(d0 + 2 * e + 1) * VP + kr] = (bf16_t)(w[e] >> 16);
            }
        }
        __syncthreads();

        if (q0 >= a.S) continue;  // wave past the end of the sequence (still joins barriers)
#pragma unroll
        for (int sub = 0; sub < kPfKV / 32; ++sub) {
            const int kb0 = k0 + sub * 32;
            if (a.causal && kb0 > q0 + 31 + diag) break;   // whole sub-tile above the diagonal
            if (kb0 >= kv_end) break;
            f32x16_t s;
#pragma unroll
            for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const bf16x8_t ka =
                    *reinterpret_cast<const bf16x8_t*>(&Ks[(sub * 32 + ql) * KP + ks * 16 + hh * 8]);
                s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[ks].v, s, 0, 0, 0);
            }
            // element e: key = kb0 + (e/4)*8 + hh*4 + e%4, query = qi
            float mloc = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int j = kb0 + (e / 4) * 8 + hh * 4 + (e % 4);
                const bool ok = (j < kv_end) && (!a.causal || j <= qi + diag);
                s[e] = ok ? s[e] * a.sm_scale_log2 : -INFINITY;
                mloc = fmaxf(mloc, s[e]);
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
            const float m_new = fmaxf(m_run, mloc);
            const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
            float psum = 0.f;
            float p[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                p[e] = (m_new == -INFINITY) ? 0.f : exp2f(s[e] - m_new);
                psum += p[e];
            }
            psum += __shfl_xor(psum, 32, kWave);
            l_run = l_run * alpha + psum;
            m_run = m_new;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[tt][e] *= alpha;
            // P^T operand per 16-key block kb: slots i<8 -> elements e = 8*kb + i.
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                Pack8 pb;
                pb.u = pack8(&p[8 * kb]);
                const int kcol = sub * 32 + kb * 16 + hh * 4;
#pragma unroll
                for (int tt = 0; tt < DT; ++tt) {
                    const bf16_t* vr = &Vt[(tt * 32 + ql) * VP + kcol];
                    Pack8 va;
                    const uint2 v0 = *reinterpret_cast<const uint2*>(vr);
                    const uint2 v1 = *reinterpret_cast<const uint2*>(vr + 8);
                    va.w[0] = v0.x;
                    va.w[1] = v0.y;
                    va.w[2] = v1.x;
                    va.w[3] = v1.y;
                    oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va.v, pb.v, oacc[tt], 0, 0, 0);
                }
            }
        }
    }

    if (qi >= a.S) return;
    // O^T tile tt: element e -> d = tt*32 + (e/4)*8 + hh*4 + e%4, query = qi.
    const float inv = (l_run > 0.f) ? 1.f / l_run : 0.f;
    bf16_t* op = a.o + (size_t)qi * a.o_sn + (size_t)head * a.o_sh;
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = tt * 32 + g * 8 + hh * 4;
            uint2 w;
            w.x = pack_bf16x2(oacc[tt][g * 4 + 0] * inv, oacc[tt][g * 4 + 1] * inv);
            w.y = pack_bf16x2(oacc[tt][g * 4 + 2] * inv, oacc[tt][g * 4 + 3] * inv);
            *reinterpret_cast<uint2*>(op + d) = w;
        }
}

// ---------------------------------------------------------------------------------
// Pipelined variant (head_dim 128, keys already rotated): one workgroup = 4 or 8 wave64s
// = 128 or 256 query rows of one head, 32 per wave. 64-key K and V tiles stream global ->
// LDS with global_load_lds into an S-deep ring (no staging registers), so S - 1 tiles are
// in flight while the matrix cores work on one; the tile layouts and operand reads are
// described in attn_pipe.hpp (K read with ds_read_b128, the V^T operand of
// O^T = V^T . P^T with ds_read_b64_tr_b16 from the row-major V tile).
//
// The matrix cores take the arithmetic; the vector ALU work per tile is kept to what the
// softmax needs (one exp2 per score, a max, a bf16 pack and a row sum), because the
// vector ALU, not the MFMA pipe, bounded the first version of this kernel:
//  * Q is multiplied by log2(e) / sqrt(head_dim) before its bf16 rounding, so scores
//    come out of the MFMAs in log2 units;
//  * the running max m is folded into the MFMA accumulator start (C = -m), so
//    p = exp2(s) needs no subtraction; m is raised only when a row's tile max exceeds it
//    by more than 2^8 (p <= 256 otherwise), which is rare after the first tile;
//  * row sums add the bf16-rounded p that the PV MFMAs use (v_dot2c_f32_bf16 against
//    (1, 1)), so the normalisation matches the weights exactly;
//  * the DMA addresses are a per-lane offset fixed for the whole loop plus a
//    workgroup-uniform tile base (the last, partial tile clamps its rows).
// Tiles that neither cross the diagonal nor the end are not masked.
// ---------------------------------------------------------------------------------
constexpr int kP2KV = 64;          // keys per tile
constexpr int kP2HD = 128;
constexpr int kP2Row = kP2HD * 2;  // bytes per K / V row in LDS
constexpr int kP2Tile = kP2KV * kP2Row;
constexpr int kP2Stage = 2 * kP2Tile;
constexpr float kP2Lazy = 8.0f;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Sum of the two bf16 halves of `w` added to acc (fp32).
__device__ __forceinline__ float add_bf16_pair(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w),
                                           __builtin_bit_cast(bf16x2_t, 0x3f803f80u), acc, false);
}

// Waves per SIMD the register allocation aims for: 8 / WAVES, but never more than the
// LDS ring lets reside (S stages of kP2Stage bytes out of 160 KB per CU, four SIMDs).
constexpr int pipe_waves_per_eu(int waves, int stages) {
    const int by_lds = (160 * 1024 / (stages * kP2Stage)) * waves / 4;
    const int want = 8 / waves;
    return by_lds < 1 ? 1 : (by_lds < want ? by_lds : want);
}

template <int WAVES, int S>
__global__ __launch_bounds__(WAVES * 64, pipe_waves_per_eu(WAVES, S)) void prefill_attn_pipe_kernel(PrefillArgs a,
                                                                                                   int nqt) {
    constexpr int THREADS = WAVES * 64;
    constexpr int QR = WAVES * 32;                         // query rows per workgroup
    constexpr int LPW = kP2Stage / 1024 / WAVES;           // 1 KB wave loads per wave per tile
    constexpr int KS = kP2HD / 16;     // 8 k-steps
    constexpr int DT = kP2HD / 32;     // 4 d tiles
    static_assert(LPW * WAVES * 1024 == kP2Stage && S >= 2 && S <= 4, "bad pipeline shape");
    __shared__ __align__(1024) unsigned char smem[S * kP2Stage];

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int ql = lane % 32, hh = lane / 32;
    const int t = (int)blockIdx.x;
    const int qt = nqt - 1 - t / a.Hq;       // heavy (late) query tiles first
    const int head = t % a.Hq;
    const int kvh = head / (a.Hq / a.Hkv);
    const int q0 = qt * QR + wave * 32;
    const int qi = q0 + ql;
    const int diag = a.L - a.S;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);

    const int q_last = min(a.S - 1, qt * QR + QR - 1);
    const int kv_end = a.causal ? min(a.L, q_last + diag + 1) : a.L;
    const int ntiles = (kv_end + kP2KV - 1) / kP2KV;
    const char* kbase = reinterpret_cast<const char*>(a.k + (size_t)kvh * a.k_sh);
    const char* vbase = reinterpret_cast<const char*>(a.v + (size_t)kvh * a.v_sh);

    // wave load i of a tile: 4 rows x 16 chunks; lane -> (row l / 16, physical chunk l % 16).
    // Load i is a K load for i < LPW / 2 and a V load after (q = wave + i * WAVES < 16).
    const int pr = lane >> 4, pc = lane & 15;
    uint32_t loff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
        const int q = wave + i * WAVES;
        const bool isv = i >= LPW / 2;
        const int row = (q % (kP2Tile / 1024)) * 4 + pr;
        const int c = isv ? (pc ^ ((row & 3) << 2)) : (pc ^ (row & 15));
        loff[i] = (uint32_t)((row * (isv ? a.v_sn : a.k_sn) + c * 8) * 2);
    }
    const uint32_t dst0 = __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(wave * 1024));
    auto issue = [&](int tile, int slot) {
        const int k0 = tile * kP2KV;
        const char* kt0 = kbase + (size_t)k0 * a.k_sn * 2;
        const char* vt0 = vbase + (size_t)k0 * a.v_sn * 2;
        const uint32_t dst = dst0 + (uint32_t)(slot * kP2Stage);
        auto load = [&](int i, uint32_t off) {
            const char* src = (i >= LPW / 2 ? vt0 : kt0) + off;
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src),
                (__attribute__((address_space(3))) void*)(uintptr_t)(dst + (uint32_t)(i * WAVES * 1024)), 16, 0, 0);
        };
        if (k0 + kP2KV <= a.L) {
#pragma unroll
            for (int i = 0; i < LPW; ++i) load(i, loff[i]);
        } else {   // the last, partial tile: rows past the end read the last row
#pragma unroll
            for (int i = 0; i < LPW; ++i) {
                const bool isv = i >= LPW / 2;
                const int q = wave + i * WAVES;
                const int row = (q % (kP2Tile / 1024)) * 4 + pr;
                const int c = isv ? (pc ^ ((row & 3) << 2)) : (pc ^ (row & 15));
                load(i, (uint32_t)((min(row, a.L - 1 - k0) * (isv ? a.v_sn : a.k_sn) + c * 8) * 2));
            }
        }
    };
    // ---- Q (B operand) of this lane's row, d = ks*16 + hh*8 + e; requested before the
    //      first tiles so that its wait does not include them
    uint4 qraw[KS];
    {
        const bool qv = qi < a.S;
        const bf16_t* qp = a.q + (size_t)(qv ? qi : 0) * a.q_sn + (size_t)head * a.q_sh;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            qraw[ks] = qv ? *reinterpret_cast<const uint4*>(qp + ks * 16 + hh * 8) : make_uint4(0, 0, 0, 0);
    }
    // With a 4-slot ring the tiles go in pairs: one barrier per two tiles (after this wave's
    // loads of both have landed), then the next pair is loaded into the slots of the
    // previous pair, which every wave has finished. Smaller rings keep one barrier per tile,
    // with S - 1 tiles in flight.
    constexpr bool PAIR = (S == 4);
    const int pre = PAIR ? min(2, ntiles) : min(S - 1, ntiles);
    for (int p = 0; p < pre; ++p) issue(p, p);
    const float scale = a.sm_scale_log2;
    bf16x8_t qf[KS];
    {
        float x[KS][8];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) unpack8(qraw[ks], x[ks]);
        if (a.rope_q) {
            const float pos = (float)(qi + a.q_pos_off);
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = ks * 16 + hh * 8 + e;
                    float sn, cs;
                    sincosf(pos * a.rope.inv_freq[d], &sn, &cs);
                    const float x0 = x[ks][e], x1 = x[ks + KS / 2][e];
                    x[ks][e] = x0 * cs - x1 * sn;
                    x[ks + KS / 2][e] = x1 * cs + x0 * sn;
                }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[ks][e] *= scale;
            Pack8 pk;
            pk.u = pack8(x[ks]);
            qf[ks] = pk.v;
        }
    }

    f32x16_t oacc[DT];
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[tt][e] = 0.f;
    // m_run: running row max (log2 units), -inf before the first tile; sinit = -m_run
    // (0 before the first tile) starts every score accumulator
    float m_run = -INFINITY, l_run = 0.f;
    f32x16_t sinit;
#pragma unroll
    for (int e = 0; e < 16; ++e) sinit[e] = 0.f;
    const int wave_last_key = q0 + 31 + diag;   // causal: last key any row of this wave sees

    // lane parts of the operand addresses inside a stage (rows of the tile and the
    // (kb, c) parts of the V reads are immediates)
    uint32_t koff[KS], voff[DT];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) koff[ks] = attn_pipe::k_off(ql, ks * 2 + hh);
#pragma unroll
    for (int tt = 0; tt < DT; ++tt) voff[tt] = (uint32_t)kP2Tile + attn_pipe::v_tr_lane_off(lane, tt);
    typedef short s4_t __attribute__((ext_vector_type(4)));

    for (int kt = 0; kt < ntiles; ++kt) {
        if constexpr (PAIR) {
            if (kt % 2 == 0) {
                attn_pipe::vm_wait<0>();
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                if (kt + 2 < ntiles) issue(kt + 2, (kt + 2) % S);
                if (kt + 3 < ntiles) issue(kt + 3, (kt + 3) % S);
            }
        } else {
            attn_pipe::vm_wait_tiles<LPW>(min(S - 2, ntiles - 1 - kt));
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (kt + S - 1 < ntiles) issue(kt + S - 1, (kt + S - 1) % S);
        }
        if (q0 >= a.S) continue;                      // rows past the end: barriers only
        const int kb0 = kt * kP2KV;
        if (a.causal && kb0 > wave_last_key) continue;   // the whole tile is above this wave's rows
        const bool two = kb0 + 32 < kv_end && !(a.causal && kb0 + 32 > wave_last_key);   // keys 32..63 needed
        const uint32_t stage = lds0 + (uint32_t)((kt % S) * kP2Stage);
        uint32_t ka[KS], va[DT];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) ka[ks] = stage + koff[ks];
#pragma unroll
        for (int tt = 0; tt < DT; ++tt) va[tt] = stage + voff[tt];

        // ---- S^T - m for keys 0..31 (s0) and 32..63 (s1) of the tile
        bf16x8_t kf0[KS], kf1[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) attn_pipe::read_b128<0>(kf0[ks], ka[ks]);
        if (two) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) attn_pipe::read_b128<32 * attn_pipe::kRow>(kf1[ks], ka[ks]);
            asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
        } else {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kf0[ks]));
        // keys 32..63 are all masked when !two (the edge masking below sets them to -inf)
        f32x16_t s0 = sinit, s1 = sinit;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf0[ks], qf[ks], s0, 0, 0, 0);
        if (two) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kf1[ks]));
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf1[ks], qf[ks], s1, 0, 0, 0);
        }
        // ---- V^T operand reads for key blocks 0 and 1 go out under the softmax
        s4_t vf[4][DT][2];
        auto read_v = [&](auto kbc) {
            constexpr int kb = decltype(kbc)::value;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) {
                attn_pipe::read_tr16<(kb * 16) * attn_pipe::kRow>(vf[kb][tt][0], va[tt]);
                attn_pipe::read_tr16<(kb * 16 + 8) * attn_pipe::kRow>(vf[kb][tt][1], va[tt]);
            }
        };
        read_v(std::integral_constant<int, 0>{});
        read_v(std::integral_constant<int, 1>{});

        // ---- online softmax over the 64 keys (element e of s0 / s1: key kb0 + 32 * half
        //      + (e/4)*8 + hh*4 + e%4, query qi)
        if (kb0 + kP2KV > kv_end || (a.causal && kb0 + kP2KV - 1 > q0 + diag)) {
            const int lim = a.causal ? min(kv_end, qi + diag + 1) : kv_end;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int j = kb0 + (e / 4) * 8 + hh * 4 + (e % 4);
                s0[e] = (j < lim) ? s0[e] : -INFINITY;
                s1[e] = (j + 32 < lim) ? s1[e] : -INFINITY;
            }
        }
        float mloc = fmaxf(s0[0], s1[0]);
#pragma unroll
        for (int e = 1; e < 16; ++e) mloc = fmaxf(fmaxf(mloc, s0[e]), s1[e]);
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc), __float_as_uint(mloc), false, false);
            mloc = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));   // tile max - m_run (or raw before)
        }
        // raise m when some row's tile max exceeds it by more than 2^8 (always on the
        // first tile, where m_run = -inf); a real (wave-uniform) branch
        if (__any(m_run == -INFINITY || mloc > kP2Lazy)) {
            asm volatile("" ::: "memory");
            const float base = (m_run == -INFINITY) ? 0.f : m_run;   // what the accumulators started from
            const float m_new = fmaxf(m_run, base + mloc);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // 0 on the first tile
            const float shift = m_new - base;
            l_run *= alpha;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[tt][e] *= alpha;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                s0[e] -= shift;
                s1[e] -= shift;
                sinit[e] = -m_new;
            }
            m_run = m_new;
        }
        Pack8 pb[4];
        {
            float p0[16], p1[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                p0[e] = __builtin_amdgcn_exp2f(s0[e]);
                p1[e] = __builtin_amdgcn_exp2f(s1[e]);
            }
            pb[0].u = pack8(&p0[0]);
            pb[1].u = pack8(&p0[8]);
            pb[2].u = pack8(&p1[0]);
            pb[3].u = pack8(&p1[8]);
        }
        float psum = 0.f;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            psum = add_bf16_pair(pb[b].u.x, psum);
            psum = add_bf16_pair(pb[b].u.y, psum);
            psum = add_bf16_pair(pb[b].u.z, psum);
            psum = add_bf16_pair(pb[b].u.w, psum);
        }
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(psum), __float_as_uint(psum), false, false);
            l_run += __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }

        // ---- O^T += V^T . P^T, key block by key block (the reads of block kb + 2 are
        //      issued once block kb has landed, so at most 16 are outstanding)
        auto pv = [&](int kb) {
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) {
                asm volatile("" : "+v"(vf[kb][tt][0]), "+v"(vf[kb][tt][1]));
                union {
                    s4_t h[2];
                    bf16x8_t v;
                } vv;
                vv.h[0] = vf[kb][tt][0];   // A slots 0-3: keys 16 kb + 4 hh + 0..3
                vv.h[1] = vf[kb][tt][1];   // A slots 4-7: keys 16 kb + 8 + 4 hh + 0..3
                oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vv.v, pb[kb].v, oacc[tt], 0, 0, 0);
            }
        };
        asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
        pv(0);
        if (two) {
            read_v(std::integral_constant<int, 2>{});
            asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
            pv(1);
            read_v(std::integral_constant<int, 3>{});
            asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
            pv(2);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            pv(3);
        } else {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            pv(1);
        }
    }

    if (qi >= a.S) return;
    const float inv = (l_run > 0.f) ? 1.f / l_run : 0.f;
    bf16_t* op = a.o + (size_t)qi * a.o_sn + (size_t)head * a.o_sh;
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = tt * 32 + g * 8 + hh * 4;
            uint2 w;
            w.x = pack_bf16x2(oacc[tt][g * 4 + 0] * inv, oacc[tt][g * 4 + 1] * inv);
            w.y = pack_bf16x2(oacc[tt][g * 4 + 2] * inv, oacc[tt][g * 4 + 3] * inv);
            *reinterpret_cast<uint2*>(op + d) = w;
        }
}

int validate_attention_ctx(const efm_attention_ctx* c, const char* who);

// EFM_KNOB_PREFILL_REGISTER selects the register-staged kernel (kept as the reference
// path of the pipelined one in the tests).
static bool prefill_pipe_enabled() { return kernel_knob(EFM_KNOB_PREFILL_REGISTER) == 0; }

int prefill_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace efm

using namespace efm;

extern "C" int efm_attention_prefill(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v,
                                     void* o, uint32_t qo_len, uint32_t kv_len, int32_t causal, hipStream_t stream) {
    int rc = validate_attention_ctx(ctx, "attention_prefill");
    if (rc) return rc;
    if (ctx->k_already_prerotated == EFM_K_PREROTATED_EXCEPT_NEWEST)
        return set_error(EFM_ERR_UNSUPPORTED, "attention_prefill: k_already_prerotated = 2 is a decode-only mode");
    if (!q || !k || !v || !o) return set_error(EFM_ERR_INVALID_ARGUMENT, "attention_prefill: null tensor pointer");
    if (kv_len < qo_len)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "attention_prefill: kv_len %u < qo_len %u", kv_len, qo_len);
    if (qo_len == 0) return EFM_OK;
    if (qo_len > (1u << 20) || kv_len > (1u << 24))
        return set_error(EFM_ERR_UNSUPPORTED, "attention_prefill: sequence too long");
    const int hd = (int)ctx->head_dim;
    PrefillArgs a;
    a.q = static_cast<const bf16_t*>(q);
    a.k = static_cast<const bf16_t*>(k);
    a.v = static_cast<const bf16_t*>(v);
    a.o = static_cast<bf16_t*>(o);
    a.S = (int)qo_len;
    a.L = (int)kv_len;
    a.Hq = (int)ctx->num_qo_heads;
    a.Hkv = (int)ctx->num_kv_heads;
    a.q_sn = ctx->q_stride_n ? (int)ctx->q_stride_n : a.Hq * hd;
    a.q_sh = ctx->q_stride_h ? (int)ctx->q_stride_h : hd;
    a.k_sn = ctx->k_stride_n ? (int)ctx->k_stride_n : a.Hkv * hd;
    a.k_sh = ctx->k_stride_h ? (int)ctx->k_stride_h : hd;
    a.v_sn = ctx->kv_stride_n ? (int)ctx->kv_stride_n : a.Hkv * hd;
    a.v_sh = ctx->kv_stride_h ? (int)ctx->kv_stride_h : hd;
    a.o_sn = a.Hq * hd;
    a.o_sh = hd;
    a.causal = causal != 0;
    a.rope_q = ctx->pos_encoding == EFM_POS_ROPE_LLAMA;
    a.rope_k = a.rope_q && !ctx->k_already_prerotated;
    a.q_pos_off = (int)ctx->q_rope_pos_offset;
    a.k_pos_off = (int)ctx->k_rope_pos_offset;
    rope_table_fill(&a.rope, hd, ctx->rope_theta, ctx->rope_scale);
    a.sm_scale_log2 = 1.4426950408889634f / sqrtf((float)hd);
    if (hd == kP2HD && !a.rope_k && prefill_pipe_enabled()) {
        // 8 waves (256 rows, 4-deep ring, one workgroup per CU) when those workgroups fill
        // the chip; fewer rows: 4 waves (128 rows) over a 2-deep ring, two workgroups per
        // CU (twice the workgroups). Measured (causal, no prefix): 12/2 heads S 256 / 512 /
        // 2048: 10.7 / 15.9 / 46.0 us with 4 waves against 11.4 / 18.2 / 62.8 with the
        // 2-wave (64-row) kernel and 12.5 / 19.2 / 58.7 with 8 waves; 16/2 S 1344: 31.2
        // against 42.9 / 38.7; 28/4 S 4096: 151.4 against 237.4 / 146.2. The 2-wave kernel
        // stays for EFM_KNOB_PREFILL_SHAPE = 2 (2 / 4 / 8 force a shape).
        const int knob = kernel_knob(EFM_KNOB_PREFILL_SHAPE);
        const int cus = prefill_cus();
        const int shape = knob != 0 ? knob : (int)((qo_len + 255) / 256) * a.Hq >= cus ? 8 : 4;
        if (shape == 2) {
            const int nqt = (int)((qo_len + 63) / 64);
            hipLaunchKernelGGL((prefill_attn_pipe_kernel<2, 2>), dim3(nqt * a.Hq), dim3(128), 0, stream, a, nqt);
        } else if (shape == 4) {
            const int nqt = (int)((qo_len + 127) / 128);
            hipLaunchKernelGGL((prefill_attn_pipe_kernel<4, 2>), dim3(nqt * a.Hq), dim3(256), 0, stream, a, nqt);
        } else {
            const int nqt = (int)((qo_len + 255) / 256);
            hipLaunchKernelGGL((prefill_attn_pipe_kernel<8, 4>), dim3(nqt * a.Hq), dim3(512), 0, stream, a, nqt);
        }
        return check_launch("attention_prefill");
    }
    dim3 grid((qo_len + kPfQ - 1) / kPfQ, a.Hq), block(kPfThreads);
    if (hd == 128) hipLaunchKernelGGL(prefill_attn_kernel<128>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(prefill_attn_kernel<64>, grid, block, 0, stream, a);
    return check_launch("attention_prefill");
}

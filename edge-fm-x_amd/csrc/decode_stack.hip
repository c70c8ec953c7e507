// One decode step of a Qwen2.5 text decoder (every layer) in a single persistent launch:
// efm_decode_stack. It computes what the per-layer launch sequence does
// (src/models/qwen2_5/qwen2_5.cpp:534-930): embedding of the previous token, then per
// layer RMSNorm (+ residual add) -> fused QKV + bias -> KV-cache write -> GQA attention
// (RoPE-Llama at L-1 on a rotated cache, split over 128-key ranges) -> split merge ->
// o_proj -> add + RMSNorm -> gate/up + SwiGLU -> down_proj; it leaves the last layer's
// h and residual for the final norm + LM head.
//
// Why one launch: at batch 1 every layer is five all-to-all dependencies (each projection
// needs the whole previous vector). Between launches each hand-off costs a kernel
// boundary (about 4 us on MI355X) and the next matrix only starts streaming after it.
// Here the weight stream never stops: every workgroup knows which rows it will multiply
// for the rest of the step and streams them into LDS ahead of time, across phases and
// layers, while the hand-offs travel between workgroups.
//
// Layout of the grid (one 512-thread workgroup per CU, all co-resident):
//  * workgroups [0, n_attn): attention, one (KV head, 128-key split) each. They prefetch
//    their K / V tile of the next layer as soon as the current one is consumed, wait for
//    this step's query and newest K / V row, run the MFMA split attention and publish the
//    split's (max, sum, unnormalised output); then each merges the splits of its query
//    heads (head h -> workgroup h % n_attn) and publishes the merged bf16 head.
//  * workgroups [n_attn, grid): GEMV. Each owns a fixed slice of rows of every matrix
//    (QKV, o_proj, [up; gate], down). Six compute waves stream row pieces (<= 4 KB) of
//    that slice through private LDS rings with global_load_lds, in the order they are
//    needed, and take dot products against the phase's input vector in LDS; two control
//    waves poll the inputs, do the residual adds and RMSNorms, apply the epilogues (bias,
//    bf16 rounding, SwiGLU, V-cache write) and publish the workgroup's outputs.
//
// Hand-offs between workgroups are 16-byte records {tag, 3 payload words} written and
// read with sc1 (device-coherent) buffer accesses: a record is valid when it carries the
// tag of this launch and layer, so no fence, counter or flag is needed and a reader can
// never use stale data. A record is written and read whole (one 16-byte access). Every
// poll is bounded: a time-out (for example when not every workgroup could be resident)
// raises the workspace's abort word, later polls give up at once, and the launch always
// drains; efm_decode_stack_status reports it.
#include "attn_pipe.hpp"
#include "common.hpp"

#include <algorithm>
#include <mutex>

namespace efm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kStkThreads = 512;
constexpr int kStkCompute = 6;         // waves 0-5: weight stream + dot products
constexpr int kStkCtrlWave = 6;        // waves 6-7: control
constexpr int kStkCtrl = 128;          // control threads
constexpr int kStkPiece = 2048;        // elements per row piece (4 KB)
constexpr int kStkMaxRing = 15;        // 1 KB ring blocks per compute wave (vmcnt range)
constexpr int kStkKeys = 128;          // keys per attention split
constexpr int kStkMaxCap = 16;         // splits per KV head
constexpr int kStkMaxAttn = 64;        // attention workgroups
constexpr int kStkOutSlots = 2048;     // fp32 piece sums of one phase
constexpr int kStkMaxHidden = 4096;
constexpr int kStkMaxInter = 20480;
constexpr int kStkMaxPoll = 32;        // records per control thread per poll
constexpr int kPartRec = 44;           // records of one split's head: 128 o + max + sum
constexpr int kHeadRec = 22;           // records of one merged head (128 bf16)
constexpr int kStkLds = 160 * 1024;
constexpr uint32_t kStkSpin = 1u << 18;
constexpr float kStkLog2e = 1.4426950408889634f;

struct StackLayer {
    const bf16_t* in_norm;
    const bf16_t* w_qkv;
    const bf16_t* b_qkv;
    const bf16_t* w_o;
    const bf16_t* post_norm;
    const bf16_t* w_gu;
    const bf16_t* w_down;
    bf16_t* k_cache;
    bf16_t* v_cache;
};
static_assert(sizeof(StackLayer) == sizeof(efm_decode_stack_layer), "layer table layout");

struct StackArgs {
    int H, QD, KVD, I, Hq, Hkv, layers;
    int64_t vocab;
    float eps;
    const StackLayer* layer;
    const bf16_t* embed;
    const int32_t* token;
    const uint32_t* d_kv_len;
    uint32_t max_kv_len;
    int n_attn, cap, ng, ring;     // attention workgroups, splits per KV head, GEMV workgroups, ring blocks
    int x_off, r_off, out_off, misc_off;   // LDS carve-up of a GEMV workgroup (bytes)
    int tab_off;                   // LDS copy of the layers' matrix / cache pointers (both roles)
    RopeTable rope;
    int q_pos_off, k_pos_off;
    uint32_t* ctl;                 // [0] epoch, [1] abort
    uint4* rec_h;                  // down_proj output, ceil(H / 6) records
    uint4* rec_qkv;                // ceil((QD + 2 KVD) / 6)
    uint4* rec_part;               // Hkv * cap * G * 44
    uint4* rec_head;               // Hq * 22
    uint4* rec_a;                  // o_proj output, ceil(H / 6)
    uint4* rec_mid;                // SwiGLU output, ceil(I / 6)
    bf16_t* h_out;
    bf16_t* r_out;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t stk_rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 0x7fffffff, 0x00020000);
}

// One record, written whole with a device-coherent (sc1) 16-byte store.
__device__ __forceinline__ void rec_store(uint4* base, int k, uint32_t tag, uint32_t w0, uint32_t w1, uint32_t w2) {
    u32x4_t v = {tag, w0, w1, w2};
    __builtin_amdgcn_raw_buffer_store_b128(v, stk_rsrc(base), k * 16, 0, 16);
}

__device__ __forceinline__ u32x4_t rec_load(const uint4* base, int k) {
    return __builtin_amdgcn_raw_buffer_load_b128(stk_rsrc(base), k * 16, 0, 16);
}

__device__ __forceinline__ uint32_t stk_tag(uint32_t epoch, int layer) {
    return ((epoch % 0xffffffu + 1u) << 8) | (uint32_t)layer;
}

// Polls records base[index(k)], k in [0, nrec) (thread t of `nthr` takes t, t + nthr, ...)
// until each carries `tag`, handing every valid record to sink(k, v). Loads of all
// still-pending records are issued before any is checked. Returns false after a time-out
// or when another workgroup has aborted.
template <class Index, class Sink>
__device__ __forceinline__ bool stk_poll(const uint4* base, int nrec, uint32_t tag, int t, int nthr, uint32_t* ctl, int* lds_abort,
                         Index index, Sink sink) {
    if (*reinterpret_cast<volatile int*>(lds_abort)) return false;
    const int mine = (t < nrec) ? (nrec - t + nthr - 1) / nthr : 0;
    uint32_t pending = (mine >= 32) ? ~0u : ((1u << mine) - 1u);
    uint32_t spins = 0;
    while (true) {
        u32x4_t v[8];
#pragma unroll 1
        for (int j0 = 0; j0 < kStkMaxPoll; j0 += 8) {
            if ((pending >> j0 & 0xffu) == 0u) continue;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (pending >> (j0 + j) & 1u) v[j] = rec_load(base, index(t + (j0 + j) * nthr));
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if ((pending >> (j0 + j) & 1u) && v[j][0] == tag) {
                    sink(t + (j0 + j) * nthr, v[j]);
                    pending &= ~(1u << (j0 + j));
                }
        }
        if (!__any(pending != 0u)) return true;
        if (((++spins) & 255u) == 0u) {
            const uint32_t ab = __hip_atomic_load(ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (ab != 0u || spins > kStkSpin) {
                if (ab == 0u) __hip_atomic_store(ctl + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *reinterpret_cast<volatile int*>(lds_abort) = 1;
                return false;
            }
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Workgroup barrier that leaves outstanding global loads (the weight stream) in flight:
// only this wave's LDS accesses are waited for.
__device__ __forceinline__ void stk_bar() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void vm_wait_dyn(int n) {
    switch (n) {
        case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
        case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
        case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
        case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
        case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
        case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
        case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
        case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
        case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
        case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
        case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
        case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
        default: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    }
}

// The two control waves meet (LDS counter; `gen` advances by 2 per call).
__device__ __forceinline__ void ctrl_sync(uint32_t* cnt, uint32_t& gen) {
    gen += 2u;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < gen) __builtin_amdgcn_s_sleep(1);
    asm volatile("" ::: "memory");
}

// Element range [e0, e1) of an n-element vector owned by GEMV workgroup j of ng: whole
// records [nrec j / ng, nrec (j + 1) / ng).
__device__ __forceinline__ void own_range(int n, int j, int ng, int& r0, int& r1, int& e0, int& e1) {
    const int nrec = (n + 5) / 6;
    r0 = (int)((long)nrec * j / ng);
    r1 = (int)((long)nrec * (j + 1) / ng);
    e0 = 6 * r0;
    e1 = min(6 * r1, n);
}

// ---------------------------------------------------------------------------------
// GEMV workgroup
// ---------------------------------------------------------------------------------
struct PieceMap {
    int H, QD, I, npH, npQ, npI;
    int q0, nq, o0, no, g0, ngu, c0, c1, c2, c4, T;   // row starts / counts, segment piece counts
};

// Matrix pointers of one layer as the compute waves read them (from LDS: a global read
// would be a vector-memory operation and break the vmcnt accounting of the weight ring).
struct LayerPtrs {
    uint64_t m[6];   // w_qkv, w_o, w_gu, w_down, k_cache, v_cache
};

__device__ __forceinline__ const bf16_t* lds_ptr(const LayerPtrs* tab, int layer, int which) {
    const uint64_t v = tab[layer].m[which];
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const bf16_t*>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ void stk_gemv(const StackArgs& a, int j, unsigned char* smem, uint32_t epoch) {
    // wave index in a scalar register: everything derived from it (piece descriptors,
    // layer-table reads) stays scalar, so the only vector-memory operations a compute wave
    // issues are its weight loads, which the vmcnt waits below count
    const int tid = threadIdx.x, lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int H = a.H, QD = a.QD, KVD = a.KVD, I = a.I, NQKV = QD + 2 * KVD;
    bf16_t* x = reinterpret_cast<bf16_t*>(smem + a.x_off);
    bf16_t* r = reinterpret_cast<bf16_t*>(smem + a.r_off);
    float* out = reinterpret_cast<float*>(smem + a.out_off);
    uint32_t* misc = reinterpret_cast<uint32_t*>(smem + a.misc_off);   // [0] ctrl counter, [1] abort, [2..3] sums
    const LayerPtrs* tab = reinterpret_cast<const LayerPtrs*>(smem + a.tab_off);
    PieceMap m;
    m.H = H; m.QD = QD; m.I = I;
    m.npH = (H + kStkPiece - 1) / kStkPiece;
    m.npQ = (QD + kStkPiece - 1) / kStkPiece;
    m.npI = (I + kStkPiece - 1) / kStkPiece;
    int qr0, qr1, qe0, qe1, hr0, hr1, he0, he1, gr0, gr1, ge0, ge1;
    own_range(NQKV, j, a.ng, qr0, qr1, qe0, qe1);
    own_range(H, j, a.ng, hr0, hr1, he0, he1);
    own_range(I, j, a.ng, gr0, gr1, ge0, ge1);
    m.q0 = qe0; m.nq = qe1 - qe0;
    m.o0 = he0; m.no = he1 - he0;
    m.g0 = ge0; m.ngu = ge1 - ge0;
    m.c0 = m.nq * m.npH;
    m.c1 = m.no * m.npQ;
    m.c2 = m.ngu * m.npH;
    m.c4 = m.no * m.npI;
    m.T = m.c0 + m.c1 + 2 * m.c2 + m.c4;
    const uint32_t L = min(a.d_kv_len[0], a.max_kv_len);

    if (wave < kStkCompute) {
        // ---- compute wave. Per layer the workgroup's pieces are the segments QKV rows,
        // o_proj rows, up rows, gate rows, down rows, each row cut into pieces of <= 2048
        // elements; wave w takes pieces w, w + 6, ... of every layer. Two iterators walk
        // that sequence: `iss` issues the pieces' loads into the wave's ring as far ahead
        // as the ring allows (across phases and layers), `cmp` consumes them. No
        // division in the loop: the segment constants sit in scalar registers and the
        // row / piece split uses a 16-bit reciprocal (row counts are small).
        auto uni = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
        const int RB = uni(a.ring);
        const uint32_t ring0 = (uint32_t)(wave * RB * 1024);
        const int c0 = uni(m.c0), c1 = uni(m.c1), c2 = uni(m.c2), c4 = uni(m.c4);
        const int npH = uni(m.npH), npQ = uni(m.npQ), npI = uni(m.npI);
        const int mulH = uni((65536 + npH - 1) / npH), mulQ = uni((65536 + npQ - 1) / npQ),
                  mulI = uni((65536 + npI - 1) / npI);
        const int q0 = uni(m.q0), o0 = uni(m.o0), g0 = uni(m.g0);
        struct It {
            int layer, seg, ts;
        };
        const int nlayers = uni(a.layers);
        // carry ts over segment ends (explicit branches: no table of the segment sizes)
        auto settle = [=](It it) {
            while (it.layer < nlayers) {
                if (it.seg == 0) { if (it.ts < c0) return it; it.ts -= c0; it.seg = 1; }
                if (it.seg == 1) { if (it.ts < c1) return it; it.ts -= c1; it.seg = 2; }
                if (it.seg == 2) { if (it.ts < c2) return it; it.ts -= c2; it.seg = 3; }
                if (it.seg == 3) { if (it.ts < c2) return it; it.ts -= c2; it.seg = 4; }
                if (it.ts < c4) return it;
                ++it.layer;
                it.seg = 0;
                it.ts = wave;
            }
            return it;
        };
        struct Geo {
            int K, row, pc;
        };
        // piece geometry: K, row within the matrix, piece index within the row
        auto geom = [=](It it) {
            int K = H, np = npH, mul = mulH, rb = q0;
            if (it.seg == 1) { K = QD; np = npQ; mul = mulQ; rb = o0; }
            else if (it.seg == 2) { rb = g0; }
            else if (it.seg == 3) { rb = I + g0; }
            else if (it.seg == 4) { K = I; np = npI; mul = mulI; rb = o0; }
            const int rr = (np == 1) ? it.ts : ((it.ts * mul) >> 16);
            Geo g;
            g.K = K;
            g.pc = it.ts - rr * np;
            g.row = rb + rr;
            return g;
        };
        It iss = settle(It{0, 0, wave});
        It cmp = iss;
        int head = 0, tail = 0, hslot = 0, tslot = 0, cur_l = -1;
        const bf16_t *bq = nullptr, *bo = nullptr, *bg = nullptr, *bd = nullptr;
        auto issue_more = [&]() {
            while (iss.layer < nlayers) {
                const Geo g = geom(iss);
                const int K = g.K, row = g.row, pc = g.pc;
                const int nel = min(kStkPiece, K - pc * kStkPiece);
                const int nbytes = nel * 2, nb = (nbytes + 1023) >> 10;
                if (head + nb - tail > RB) break;
                if (iss.layer != cur_l) {
                    cur_l = iss.layer;
                    bq = lds_ptr(tab, cur_l, 0);
                    bo = lds_ptr(tab, cur_l, 1);
                    bg = lds_ptr(tab, cur_l, 2);
                    bd = lds_ptr(tab, cur_l, 3);
                }
                const bf16_t* base = iss.seg == 0 ? bq : iss.seg == 1 ? bo : iss.seg == 4 ? bd : bg;
                const unsigned char* src =
                    reinterpret_cast<const unsigned char*>(base + (size_t)row * K + (size_t)pc * kStkPiece);
                for (int i = 0; i < nb; ++i) {
                    int off = i * 1024 + lane * 16;
                    if (off >= nbytes) off = nbytes - 16;
                    __builtin_amdgcn_global_load_lds(
                        static_cast<const void*>(src + off),
                        (__attribute__((address_space(3))) void*)(smem + ring0 + hslot * 1024), 16, 0, 0);
                    if (++hslot == RB) hslot = 0;
                }
                head += nb;
                iss.ts += kStkCompute;
                iss = settle(iss);
            }
        };
        issue_more();
        for (int l = 0; l < a.layers; ++l) {
            for (int ph = 0; ph < 4; ++ph) {
                stk_bar();   // the phase's input vector is in x
                while (cmp.layer == l && (cmp.seg == 4 ? 3 : cmp.seg == 3 ? 2 : cmp.seg) == ph) {
                    const Geo g = geom(cmp);
                    const int elem0 = g.pc * kStkPiece;
                    const int nel = min(kStkPiece, g.K - elem0);
                    const int nb = (nel * 2 + 1023) >> 10;
                    const int slot = (cmp.seg == 3 ? c2 : 0) + cmp.ts;
                    vm_wait_dyn(head - tail - nb);
                    float acc = 0.f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int c = i * kWave + lane;
                        if (i < nb && c * 8 < nel) {
                            int rs = tslot + i;
                            if (rs >= RB) rs -= RB;
                            const uint4 wv = *reinterpret_cast<const uint4*>(smem + ring0 + rs * 1024 + lane * 16);
                            const uint4 xv = *reinterpret_cast<const uint4*>(x + elem0 + c * 8);
                            acc = dot8(wv, xv, acc);
                        }
                    }
                    acc = wave_sum(acc);
                    if (lane == 0) out[slot] = acc;
                    tail += nb;
                    tslot += nb;
                    if (tslot >= RB) tslot -= RB;
                    cmp.ts += kStkCompute;
                    cmp = settle(cmp);
                    issue_more();
                }
                stk_bar();   // the phase's piece sums are in out
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    // ---- control waves
    const int ct = tid - kStkCtrlWave * kWave;   // 0..127
    uint32_t gen = 0;
    int* lds_abort = reinterpret_cast<int*>(misc + 1);
    float* sums = reinterpret_cast<float*>(misc + 2);
    constexpr int kMaxE = kStkMaxHidden / kStkCtrl;   // norm elements per control thread
    // the residual stream r and the normalised input x (RMSNorm of s = in + r with
    // weight w; the first layer's input is the embedding row and r = that row)
    auto add_norm = [&](const float (&w)[kMaxE], bool add) {
        float sv[kMaxE];
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kMaxE; ++i) {
            const int e = ct + i * kStkCtrl;
            sv[i] = 0.f;
            if (e < H) {
                float s = bf16_to_f32(x[e]);
                if (add) s += bf16_to_f32(r[e]);
                r[e] = (bf16_t)f32_to_bf16(s);
                sv[i] = s;
                ss = fmaf(s, s, ss);
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) sums[wave - kStkCtrlWave] = ss;
        ctrl_sync(misc, gen);
        const float tot = sums[0] + sums[1];
        const float inv = 1.0f / sqrtf(tot / (float)H + a.eps);
#pragma unroll
        for (int i = 0; i < kMaxE; ++i) {
            const int e = ct + i * kStkCtrl;
            if (e < H) x[e] = (bf16_t)f32_to_bf16((sv[i] * inv) * w[i]);
        }
        ctrl_sync(misc, gen);   // sums may be reused after both waves read them
    };
    auto poll_vec = [&](const uint4* rec, int n, uint32_t tag) {
        const int nrec = (n + 5) / 6;
        stk_poll(rec, nrec, tag, ct, kStkCtrl, a.ctl, lds_abort, [](int k) { return k; }, [&](int k, const u32x4_t& v) {
            uint32_t* dst = reinterpret_cast<uint32_t*>(x) + 3 * k;
            const int e = 6 * k;
            if (e + 6 <= n) {
                dst[0] = v[1]; dst[1] = v[2]; dst[2] = v[3];
            } else {
#pragma unroll
                for (int i = 0; i < 6; ++i)
                    if (e + i < n) x[e + i] = (bf16_t)((v[1 + i / 2] >> (16 * (i & 1))) & 0xffffu);
            }
        });
        ctrl_sync(misc, gen);
    };
    auto sum_slots = [&](int slot0, int np) {
        float s = 0.f;
        for (int p = 0; p < np; ++p) s += out[slot0 + p];
        return s;
    };

    for (int l = 0; l < a.layers; ++l) {
        const StackLayer& Ly = a.layer[l];
        const uint32_t tag = stk_tag(epoch, l);
        // this layer's norm weights and QKV bias, requested before any wait so that they
        // arrive while the inputs are polled
        float w_in[kMaxE], w_post[kMaxE], bias[12];
#pragma unroll
        for (int i = 0; i < kMaxE; ++i) {
            const int e = ct + i * kStkCtrl;
            w_in[i] = (e < H) ? bf16_to_f32(Ly.in_norm[e]) : 0.f;
            w_post[i] = (e < H) ? bf16_to_f32(Ly.post_norm[e]) : 0.f;
        }
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            const int e = 6 * (qr0 + ct + (i / 6) * kStkCtrl) + i % 6;
            bias[i] = (Ly.b_qkv != nullptr && qr0 + ct + (i / 6) * kStkCtrl < qr1 && e < NQKV)
                          ? bf16_to_f32(Ly.b_qkv[e]) : 0.f;
        }
        // ---- QKV input: h of the previous layer (or the embedding row) + residual, RMSNorm
        if (l == 0) {
            const int32_t tok = a.token[0];
            const bool ok = tok >= 0 && (int64_t)tok < a.vocab;
            for (int e = ct; e < H; e += kStkCtrl) x[e] = ok ? a.embed[(size_t)tok * H + e] : (bf16_t)0;
            ctrl_sync(misc, gen);
            add_norm(w_in, false);
        } else {
            poll_vec(a.rec_h, H, stk_tag(epoch, l - 1));
            add_norm(w_in, true);
        }
        stk_bar();
        stk_bar();
        // ---- publish q / k / v (+ bias), V row into the cache slot L - 1
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int k = qr0 + ct + kk * kStkCtrl;
            if (k >= qr1) continue;
            uint32_t wv[3] = {0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                const int e = 6 * k + i;
                if (e >= NQKV) continue;
                float v = sum_slots((e - qe0) * m.npH, m.npH) + bias[kk * 6 + i];
                const uint32_t b = f32_to_bf16(v);
                wv[i / 2] |= b << (16 * (i & 1));
                if (e >= QD + KVD && L > 0) Ly.v_cache[(size_t)(L - 1) * KVD + (e - QD - KVD)] = (bf16_t)b;
            }
            rec_store(a.rec_qkv, k, tag, wv[0], wv[1], wv[2]);
        }
        // ---- O input: the merged attention heads
        {
            const int nrec = a.Hq * kHeadRec;
            stk_poll(a.rec_head, nrec, tag, ct, kStkCtrl, a.ctl, lds_abort, [](int k) { return k; },
                     [&](int k, const u32x4_t& v) {
                const int h = k / kHeadRec, jj = k % kHeadRec;
#pragma unroll
                for (int i = 0; i < 6; ++i)
                    if (6 * jj + i < 128) x[h * 128 + 6 * jj + i] = (bf16_t)((v[1 + i / 2] >> (16 * (i & 1))) & 0xffffu);
            });
            ctrl_sync(misc, gen);
        }
        stk_bar();
        stk_bar();
        // ---- publish a = o_proj output
        for (int k = hr0 + ct; k < hr1; k += kStkCtrl) {
            uint32_t wv[3] = {0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                const int e = 6 * k + i;
                if (e < H) wv[i / 2] |= f32_to_bf16(sum_slots((e - he0) * m.npQ, m.npQ)) << (16 * (i & 1));
            }
            rec_store(a.rec_a, k, tag, wv[0], wv[1], wv[2]);
        }
        // ---- GU input: a + residual, RMSNorm
        poll_vec(a.rec_a, H, tag);
        add_norm(w_post, true);
        stk_bar();
        stk_bar();
        // ---- publish mid = SwiGLU(up, gate)
        for (int k = gr0 + ct; k < gr1; k += kStkCtrl) {
            uint32_t wv[3] = {0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                if (6 * k + i >= I) continue;
                const int n = 6 * k + i - ge0;
                const float u = round_bf16(sum_slots(n * m.npH, m.npH));
                const float g = round_bf16(sum_slots(m.c2 + n * m.npH, m.npH));
                const float sg = silu_f32(g);
                wv[i / 2] |= f32_to_bf16(sg * u) << (16 * (i & 1));
            }
            rec_store(a.rec_mid, k, tag, wv[0], wv[1], wv[2]);
        }
        // ---- DOWN input: mid
        poll_vec(a.rec_mid, I, tag);
        stk_bar();
        stk_bar();
        // ---- publish h = down_proj output
        for (int k = hr0 + ct; k < hr1; k += kStkCtrl) {
            uint32_t wv[3] = {0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                const int e = 6 * k + i;
                if (e < H) wv[i / 2] |= f32_to_bf16(sum_slots((e - he0) * m.npI, m.npI)) << (16 * (i & 1));
            }
            rec_store(a.rec_h, k, tag, wv[0], wv[1], wv[2]);
        }
    }
    // ---- the first GEMV workgroup hands (h, residual) of the last layer to the LM head
    if (j == 0) {
        poll_vec(a.rec_h, H, stk_tag(epoch, a.layers - 1));
        for (int e = ct; e < H; e += kStkCtrl) {
            a.h_out[e] = x[e];
            a.r_out[e] = r[e];
        }
        if (ct == 0) a.ctl[0] = epoch + 1u;   // read by the next launch only
    }
}

// ---------------------------------------------------------------------------------
// Attention workgroup (waves 0-3; head_dim 128, K cache rotated except row L - 1)
// ---------------------------------------------------------------------------------
template <int G>
__device__ __forceinline__ void stk_attention(const StackArgs& a, int b, unsigned char* smem, uint32_t epoch) {
    constexpr int HD = 128, HALF = 64, KS = 8, DT = 4, NW = 4, NT = 256;
    constexpr int TILE = kStkKeys * attn_pipe::kRow;   // 32 KB of K (or V)
    constexpr int LPW = 2 * TILE / 1024 / NW;         // 16 wave loads per wave
    // All eight waves stay to the end and meet at every barrier; waves 0-3 do the MFMA
    // work, all eight poll.
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave, ql = lane % 32, hh = lane / 32;
    const bool mma = wave < NW;
    const int kvh = b / a.cap, s = b % a.cap;
    const int start = s * kStkKeys;
    const int QD = a.QD, KVD = a.KVD;
    float2* cs_qk = reinterpret_cast<float2*>(smem + 2 * TILE);             // [2][64]
    bf16_t* qs = reinterpret_cast<bf16_t*>(smem + 2 * TILE + 1024);          // [G][128]
    bf16_t* qr = qs + 8 * HD;                                                // [G][128]
    bf16_t* newest = qr + 8 * HD;                                            // K row | V row
    float* pst = reinterpret_cast<float*>(newest + 2 * HD);                  // [cap][130]
    bf16_t* headbuf = reinterpret_cast<bf16_t*>(pst + kStkMaxCap * 130);     // merged head, 132 slots
    int* lds_abort = reinterpret_cast<int*>(headbuf + 136);
    const uint32_t lds0 =
        (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);

    const uint32_t L = min(a.d_kv_len[0], a.max_kv_len);
    const int nsplit = (L == 0) ? 1 : (int)((L + kStkKeys - 1) / kStkKeys);
    const bool active = s < nsplit;
    const int end = min((int)L, start + kStkKeys);
    const bool owner = L > 0 && (int)L - 1 >= start && (int)L - 1 < end;
    const int lim = min((int)a.max_kv_len, start + kStkKeys) - 1;

    const LayerPtrs* tab = reinterpret_cast<const LayerPtrs*>(smem + a.tab_off);
    auto issue = [&](int l) {
        const bf16_t* kbase = lds_ptr(tab, l, 4) + (size_t)kvh * HD;
        const bf16_t* vbase = lds_ptr(tab, l, 5) + (size_t)kvh * HD;
        const int pr = lane >> 4, pc = lane & 15;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int q = wave + i * NW;              // K 0..31, V 32..63
            const bool isv = q >= TILE / 1024;
            const int row = (q % (TILE / 1024)) * 4 + pr;
            const int c = isv ? (pc ^ ((row & 3) << 2)) : (pc ^ (row & 15));
            const int jrow = min(start + row, lim);
            const bf16_t* src = (isv ? vbase : kbase) + (size_t)jrow * KVD + c * 8;
            __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                             (__attribute__((address_space(3))) void*)(smem + q * 1024), 16, 0, 0);
        }
    };
    if (tid == 0) *lds_abort = 0;
    if (active && mma) issue(0);
    // RoPE at position L - 1 for the query and the newest key
    if (tid < 2 * HALF) {
        const float freq = a.rope.inv_freq[tid % HALF];
        float sn, cs;
        sincos_reduced((float)((int)L - 1 + (tid < HALF ? a.q_pos_off : a.k_pos_off)) * freq, &sn, &cs);
        cs_qk[tid] = make_float2(cs, sn);
    }
    stk_bar();   // the first tile's loads stay in flight

    const float qscale = kStkLog2e / sqrtf((float)HD);
    for (int l = 0; l < a.layers; ++l) {
        const uint32_t tag = stk_tag(epoch, l);
        if (active) {
            // ---- this step's query (the group's G heads) and, for the owner, the newest K / V row
            const int qa = kvh * G * HD, qb = qa + G * HD;
            const int r0 = qa / 6, nq = (qb - 1) / 6 - r0 + 1;
            const int ka = QD + kvh * HD, va = QD + KVD + kvh * HD;
            const int kr0 = ka / 6, nkr = (ka + HD - 1) / 6 - kr0 + 1;
            const int vr0 = va / 6, nvr = (va + HD - 1) / 6 - vr0 + 1;
            const int ntot = nq + (owner ? nkr + nvr : 0);
            auto rec_of = [&](int k) { return k < nq ? r0 + k : (k < nq + nkr ? kr0 + (k - nq) : vr0 + (k - nq - nkr)); };
            stk_poll(a.rec_qkv, ntot, tag, tid, kStkThreads, a.ctl, lds_abort, rec_of, [&](int k, const u32x4_t& v) {
                int rec, lo, hi;
                bf16_t* dst;
                if (k < nq) { rec = r0 + k; lo = qa; hi = qb; dst = qs - qa; }
                else if (k < nq + nkr) { rec = kr0 + (k - nq); lo = ka; hi = ka + HD; dst = newest - ka; }
                else { rec = vr0 + (k - nq - nkr); lo = va; hi = va + HD; dst = newest + HD - va; }
#pragma unroll
                for (int i = 0; i < 6; ++i) {
                    const int e = 6 * rec + i;
                    if (e >= lo && e < hi) dst[e] = (bf16_t)((v[1 + i / 2] >> (16 * (i & 1))) & 0xffffu);
                }
            });
            attn_pipe::vm_wait<0>();   // the K / V tile has landed
            __syncthreads();
            if (owner && tid < 2 * HD) {
                // the newest row, as published this step, over its stale prefetched copy
                const int rr = (int)L - 1 - start, d = tid % HD, c = d >> 3;
                const int off = (tid < HD) ? rr * attn_pipe::kRow + ((c ^ (rr & 15)) << 4)
                                           : TILE + rr * attn_pipe::kRow + ((c ^ ((rr & 3) << 2)) << 4);
                *reinterpret_cast<bf16_t*>(smem + off + (d & 7) * 2) = newest[tid];
            }
            if (end < start + kStkKeys) {
                // zero the V rows past the length (P is 0 there, but the rows may hold NaN)
                for (int i = tid; i < (start + kStkKeys - end) * 16; i += kStkThreads) {
                    const int row = end - start + i / 16;
                    *reinterpret_cast<uint4*>(smem + TILE + row * attn_pipe::kRow + (i % 16) * 16) =
                        make_uint4(0, 0, 0, 0);
                }
            }
            // rotate q (pairs d, d + 64 at L - 1) and scale by log2(e) / sqrt(hd)
#pragma unroll
            for (int k = 0; k < (G * HD + NT - 1) / NT; ++k) {
                const int i = tid + k * NT;
                if (mma && i < G * HD) {
                    const int d = i % HD;
                    const float xq = bf16_to_f32(qs[i]);
                    const float yq = bf16_to_f32(qs[i ^ HALF]);
                    const float2 c2 = cs_qk[d % HALF];
                    const float rq = (d < HALF) ? xq * c2.x - yq * c2.y : xq * c2.x + yq * c2.y;
                    qr[i] = (bf16_t)f32_to_bf16(rq * qscale);
                }
            }
            __syncthreads();
            bf16x8_t qf[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                union {
                    uint4 u;
                    bf16x8_t v;
                } pk;
                pk.u = (ql < G) ? *reinterpret_cast<const uint4*>(&qr[ql * HD + ks * 16 + hh * 8]) : make_uint4(0, 0, 0, 0);
                qf[ks] = pk.v;
            }
            f32x16_t oacc[DT];
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[tt][e] = 0.f;
            float m_run = -INFINITY, l_run = 0.f;
            const int t0 = start + wave * 32;
            typedef short s4_t __attribute__((ext_vector_type(4)));
            if (mma && t0 < end) {
                bf16x8_t kf[KS];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    attn_pipe::read_b128<0>(kf[ks], lds0 + attn_pipe::k_off(wave * 32 + ql, ks * 2 + hh));
                s4_t vf[2][DT][2];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int tt = 0; tt < DT; ++tt) {
                        const uint32_t vo = lds0 + (uint32_t)TILE + (uint32_t)(wave * 32 * attn_pipe::kRow) +
                                            attn_pipe::v_tr_lane_off(lane, tt) + (uint32_t)(kb * 16 * attn_pipe::kRow);
                        attn_pipe::read_tr16<0>(vf[kb][tt][0], vo);
                        attn_pipe::read_tr16<8 * attn_pipe::kRow>(vf[kb][tt][1], vo);
                    }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(kf[ks]));
                if (owner && t0 + ql == (int)L - 1) {
                    // the newest key: rotate at L - 1, use it and store it back rotated
                    bf16_t* kw = const_cast<bf16_t*>(lds_ptr(tab, l, 4)) + (size_t)((int)L - 1) * KVD + (size_t)kvh * HD + hh * 8;
#pragma unroll
                    for (int ks = 0; ks < KS / 2; ++ks) {
                        union {
                            uint4 u;
                            bf16x8_t v;
                        } u0, u1;
                        u0.v = kf[ks];
                        u1.v = kf[ks + KS / 2];
                        float x0[8], x1[8];
                        unpack8(u0.u, x0);
                        unpack8(u1.u, x1);
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const float2 c2 = cs_qk[HALF + ks * 16 + hh * 8 + e];
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
                f32x16_t sc = {};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], sc, 0, 0, 0);
                // element e: key t0 + (e / 4) * 8 + hh * 4 + e % 4, head ql
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int jk = t0 + (e / 4) * 8 + hh * 4 + (e % 4);
                    sc[e] = (jk < end) ? sc[e] : -INFINITY;
                }
                float mloc = sc[0];
#pragma unroll
                for (int e = 1; e < 16; ++e) mloc = fmaxf(mloc, sc[e]);
                {
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc), __float_as_uint(mloc), false, false);
                    mloc = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
                }
                m_run = mloc;   // finite: the tile holds a valid key
                float p[16], psum = 0.f;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    p[e] = __builtin_amdgcn_exp2f(sc[e] - m_run);
                    psum += p[e];
                }
                {
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(psum), __float_as_uint(psum), false, false);
                    psum = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
                }
                l_run = psum;
                union {
                    uint4 u;
                    bf16x8_t v;
                } pb[2];
                pb[0].u = pack8(&p[0]);
                pb[1].u = pack8(&p[8]);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int tt = 0; tt < DT; ++tt) {
                        union {
                            s4_t h[2];
                            bf16x8_t v;
                        } vv;
                        vv.h[0] = vf[kb][tt][0];
                        vv.h[1] = vf[kb][tt][1];
                        oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vv.v, pb[kb].v, oacc[tt], 0, 0, 0);
                    }
            }
            // ---- merge the 4 waves (tile buffers are free now): per head M, wave weights
            //      exp2(m_w - M), den = sum of weighted l_w; o = fixed-order weighted sum
            __syncthreads();
            float* om = reinterpret_cast<float*>(smem);
            float* ol = om + NW * 32;
            float* ob = ol + NW * 32;
            float* sw = ob + NW * G * HD;
            float* md = sw + NW * G;
            if (mma && hh == 0) {
                om[wave * 32 + ql] = m_run;
                ol[wave * 32 + ql] = l_run;
            }
            if (mma && ql < G) {
#pragma unroll
                for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                    for (int eb = 0; eb < 4; ++eb)
                        *reinterpret_cast<float4*>(&ob[(wave * G + ql) * HD + tt * 32 + eb * 8 + hh * 4]) =
                            make_float4(oacc[tt][eb * 4 + 0], oacc[tt][eb * 4 + 1], oacc[tt][eb * 4 + 2],
                                        oacc[tt][eb * 4 + 3]);
            }
            __syncthreads();
            if (tid < G) {
                float M = -INFINITY;
#pragma unroll
                for (int w = 0; w < NW; ++w) M = fmaxf(M, om[w * 32 + tid]);
                float den = 0.f;
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    const float mw = om[w * 32 + tid];
                    const float scw = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
                    sw[w * G + tid] = scw;
                    den = fmaf(scw, ol[w * 32 + tid], den);
                }
                md[tid * 2 + 0] = M;
                md[tid * 2 + 1] = den;
            }
            __syncthreads();
            // ---- publish the split: per head 130 floats (128 o, max, sum) as 44 records
            for (int k = tid; k < G * kPartRec; k += kStkThreads) {
                const int g = k / kPartRec, jj = k % kPartRec;
                uint32_t wv[3];
#pragma unroll
                for (int i = 0; i < 3; ++i) {
                    const int d = 3 * jj + i;
                    float v = 0.f;
                    if (d < HD) {
#pragma unroll
                        for (int w = 0; w < NW; ++w) v = fmaf(sw[w * G + g], ob[(w * G + g) * HD + d], v);
                    } else if (d < HD + 2) {
                        v = md[g * 2 + (d - HD)];
                    }
                    wv[i] = __float_as_uint(v);
                }
                rec_store(a.rec_part, ((kvh * a.cap + s) * G + g) * kPartRec + jj, tag, wv[0], wv[1], wv[2]);
            }
            stk_bar();   // the tile region is free (the record stores need not complete here)
            if (l + 1 < a.layers && mma) issue(l + 1);
        }
        // ---- merger of query heads h = b, b + n_attn, ...: log-sum-exp over the splits
        for (int h = b; h < a.Hq; h += a.n_attn) {
            const int kv2 = h / G, g2 = h % G;
            const int nrec = nsplit * kPartRec;
            auto part_of = [&](int k) { return ((kv2 * a.cap + k / kPartRec) * G + g2) * kPartRec + k % kPartRec; };
            stk_poll(a.rec_part, nrec, tag, tid, kStkThreads, a.ctl, lds_abort, part_of, [&](int k, const u32x4_t& v) {
                const int s2 = k / kPartRec, jj = k % kPartRec;
#pragma unroll
                for (int i = 0; i < 3; ++i)
                    if (3 * jj + i < 130) pst[s2 * 130 + 3 * jj + i] = __uint_as_float(v[1 + i]);
            });
            stk_bar();
            // weights w_s = exp2(m_s - M) / sum_s exp2(m_s - M) l_s (every thread, nsplit <= 16),
            // then one output element per thread as the fixed-order sum over the splits
            float M = -INFINITY;
            for (int s2 = 0; s2 < nsplit; ++s2) M = fmaxf(M, pst[s2 * 130 + HD]);
            float den = 0.f;
            for (int s2 = 0; s2 < nsplit; ++s2) {
                const float ms = pst[s2 * 130 + HD];
                den = fmaf((ms == -INFINITY) ? 0.f : exp2f(ms - M), pst[s2 * 130 + HD + 1], den);
            }
            const float inv = (den > 0.f) ? 1.f / den : 0.f;
            if (tid < HD) {
                float acc = 0.f;
                for (int s2 = 0; s2 < nsplit; ++s2) {
                    const float ms = pst[s2 * 130 + HD];
                    const float ws = ((ms == -INFINITY) ? 0.f : exp2f(ms - M)) * inv;
                    acc = fmaf(ws, pst[s2 * 130 + tid], acc);
                }
                headbuf[tid] = (bf16_t)f32_to_bf16(acc);
            }
            stk_bar();
            if (tid < kHeadRec) {
                const uint32_t* hb = reinterpret_cast<const uint32_t*>(headbuf) + 3 * tid;
                rec_store(a.rec_head, h * kHeadRec + tid, tag, hb[0], hb[1], tid == kHeadRec - 1 ? 0u : hb[2]);
            }
            stk_bar();   // pst is reused by the next head (the next tile's loads stay in flight)
        }
    }
    attn_pipe::vm_wait<0>();
}

template <int G>
__global__ __launch_bounds__(kStkThreads, 1) void decode_stack_kernel(StackArgs a) {
    extern __shared__ __align__(1024) unsigned char stk_smem[];
    const uint32_t epoch = a.ctl[0];
    LayerPtrs* tab = reinterpret_cast<LayerPtrs*>(stk_smem + a.tab_off);
    for (int i = threadIdx.x; i < a.layers * 6; i += kStkThreads) {
        const StackLayer& Ly = a.layer[i / 6];
        const int w = i % 6;
        const void* ptr = w == 0 ? (const void*)Ly.w_qkv : w == 1 ? (const void*)Ly.w_o : w == 2 ? (const void*)Ly.w_gu
                        : w == 3 ? (const void*)Ly.w_down : w == 4 ? (const void*)Ly.k_cache : (const void*)Ly.v_cache;
        tab[i / 6].m[w] = reinterpret_cast<uint64_t>(ptr);
    }
    if ((int)blockIdx.x >= a.n_attn && threadIdx.x < 4)
        reinterpret_cast<uint32_t*>(stk_smem + a.misc_off)[threadIdx.x] = 0u;
    __syncthreads();
    if ((int)blockIdx.x < a.n_attn) stk_attention<G>(a, (int)blockIdx.x, stk_smem, epoch);
    else stk_gemv(a, (int)blockIdx.x - a.n_attn, stk_smem, epoch);
}

// ---------------------------------------------------------------------------------
// Host: plan, workspace, launch
// ---------------------------------------------------------------------------------
int validate_attention_ctx(const efm_attention_ctx* c, const char* who);

struct StackPlan {
    int G, cap, n_attn, ng, grid, ring;
    int x_off, r_off, out_off, misc_off, tab_off, lds;
    size_t off_h, off_qkv, off_part, off_head, off_a, off_mid, total;
};

static size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }
static int a16(int x) { return (x + 15) & ~15; }

static int stack_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
        cached[dev] = n;
    }
    return cached[dev];
}

static int stack_plan(const efm_attention_ctx* ctx, int H, int I, int layers, uint32_t max_kv_len, bool need_device,
                      StackPlan* p) {
    int rc = validate_attention_ctx(ctx, "decode_stack");
    if (rc) return rc;
    const int hd = (int)ctx->head_dim, Hq = (int)ctx->num_qo_heads, Hkv = (int)ctx->num_kv_heads;
    if (hd != 128 || ctx->pos_encoding != EFM_POS_ROPE_LLAMA || ctx->k_already_prerotated != EFM_K_PREROTATED_EXCEPT_NEWEST)
        return set_error(EFM_ERR_UNSUPPORTED,
                         "decode_stack: needs head_dim 128, RoPE-Llama and a rotated cache whose newest row is "
                         "written by the call (k_already_prerotated = 2)");
    const uint32_t kvd = (uint32_t)(Hkv * hd);
    if ((ctx->q_stride_n != 0 && ctx->q_stride_n != (uint32_t)(Hq * hd)) || (ctx->q_stride_h != 0 && ctx->q_stride_h != (uint32_t)hd) ||
        (ctx->k_stride_n != 0 && ctx->k_stride_n != kvd) || (ctx->kv_stride_n != 0 && ctx->kv_stride_n != kvd) ||
        (ctx->k_stride_h != 0 && ctx->k_stride_h != (uint32_t)hd) || (ctx->kv_stride_h != 0 && ctx->kv_stride_h != (uint32_t)hd))
        return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: q and the K / V caches must be contiguous rows");
    if (H <= 0 || H % 8 != 0 || H > kStkMaxHidden || I <= 0 || I % 8 != 0 || I > kStkMaxInter)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: hidden %d / intermediate %d (multiples of 8, <= %d / %d)", H,
                         I, kStkMaxHidden, kStkMaxInter);
    if (layers <= 0 || layers > 128) return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: %d layers (1..128)", layers);
    if (max_kv_len == 0) return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_stack: max_kv_len is 0");
    const int G = Hq / Hkv;
    const int cap = (int)((max_kv_len + kStkKeys - 1) / kStkKeys);
    if (cap > kStkMaxCap || Hkv * cap > kStkMaxAttn)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: %d KV heads x %d splits of %d keys (needs <= %d splits, <= %d "
                         "attention workgroups)", Hkv, cap, kStkKeys, kStkMaxCap, kStkMaxAttn);
    if (Hq * kHeadRec > kStkMaxPoll * kStkCtrl || (I + 5) / 6 > kStkMaxPoll * kStkCtrl)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: too many query heads or too large an intermediate size");
    p->G = G;
    p->cap = cap;
    p->n_attn = Hkv * cap;
    int cus = 256;
    if (need_device) {
        cus = stack_cus();
        if (cus <= 0) return set_error(EFM_ERR_DEVICE, "decode_stack: cannot query the CU count");
    }
    p->grid = cus;
    p->ng = cus - p->n_attn;
    if (p->ng < 32) return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: too few GEMV workgroups (%d)", p->ng);
    const int QD = Hq * hd, NQKV = QD + 2 * (int)kvd;
    // piece slots of one phase of the busiest workgroup
    auto max_rows = [&](int n) { return 6 * (((n + 5) / 6 + p->ng - 1) / p->ng); };
    const int npH = (H + kStkPiece - 1) / kStkPiece, npQ = (QD + kStkPiece - 1) / kStkPiece,
              npI = (I + kStkPiece - 1) / kStkPiece;
    const int slots = std::max({max_rows(NQKV) * npH, max_rows(H) * npQ, 2 * max_rows(I) * npH, max_rows(H) * npI});
    if (slots > kStkOutSlots) return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: %d piece slots per phase", slots);
    if (((NQKV + 5) / 6 + p->ng - 1) / p->ng > 2 * kStkCtrl)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: too many QKV rows per workgroup");
    // LDS of a GEMV workgroup: rings | x | r | out | misc; of an attention workgroup: a
    // 64 KB K / V tile, RoPE table, queries, newest row, split staging
    const int xb = a16(2 * std::max({H, QD, I})), rb = a16(2 * H), ob = kStkOutSlots * 4, mb = 64;
    const int fixed = xb + rb + ob + mb + 16 + layers * 48;
    int ring = (kStkLds - fixed) / (kStkCompute * 1024);
    ring = std::min(ring, kStkMaxRing);
    if (ring < 4) return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: activations leave no room for the weight rings");
    p->ring = ring;
    p->x_off = kStkCompute * ring * 1024;
    p->r_off = p->x_off + xb;
    p->out_off = p->r_off + rb;
    p->misc_off = p->out_off + ob;
    const int gemv_end = p->misc_off + mb;
    const int attn_end = 2 * kStkKeys * 256 + 1024 + 3 * 8 * 128 * 2 + kStkMaxCap * 130 * 4 + 136 * 2 + 16;
    p->tab_off = a16(std::max(gemv_end, attn_end));
    p->lds = p->tab_off + layers * 48;
    if (p->lds > kStkLds) return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: %d bytes of LDS needed", p->lds);
    p->off_h = 256;
    p->off_qkv = p->off_h + a256((size_t)(H + 5) / 6 * 16);
    p->off_part = p->off_qkv + a256((size_t)(NQKV + 5) / 6 * 16);
    p->off_head = p->off_part + a256((size_t)Hkv * cap * G * kPartRec * 16);
    p->off_a = p->off_head + a256((size_t)Hq * kHeadRec * 16);
    p->off_mid = p->off_a + a256((size_t)(H + 5) / 6 * 16);
    p->total = p->off_mid + a256((size_t)(I + 5) / 6 * 16);
    return EFM_OK;
}

template <int G>
static int stack_launch(const StackArgs& a, const StackPlan& p, hipStream_t stream) {
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_stack_kernel<G>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, kStkLds);
    });
    if (attr != hipSuccess)
        return set_error(EFM_ERR_DEVICE, "decode_stack: cannot raise the LDS limit: %s", hipGetErrorString(attr));
    hipLaunchKernelGGL((decode_stack_kernel<G>), dim3(p.grid), dim3(kStkThreads), p.lds, stream, a);
    return check_launch("decode_stack");
}

}  // namespace efm

using namespace efm;

extern "C" size_t efm_decode_stack_workspace_bytes(const efm_attention_ctx* ctx, int32_t hidden, int32_t inter,
                                                   int32_t layers, uint32_t max_kv_len) {
    StackPlan p;
    if (stack_plan(ctx, hidden, inter, layers, max_kv_len, false, &p) != EFM_OK) return 0;
    return p.total;
}

extern "C" int efm_decode_stack_supported(const efm_attention_ctx* ctx, int32_t hidden, int32_t inter, int32_t layers,
                                          uint32_t max_kv_len) {
    StackPlan p;
    return stack_plan(ctx, hidden, inter, layers, max_kv_len, true, &p);
}

extern "C" int efm_decode_stack(const efm_attention_ctx* ctx, int32_t hidden, int32_t inter, int32_t layers, float eps,
                                const efm_decode_stack_layer* layer_table, const void* embed, int64_t vocab,
                                const int32_t* token, const uint32_t* d_kv_len, uint32_t max_kv_len, void* h_out,
                                void* residual_out, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    StackPlan p;
    int rc = stack_plan(ctx, hidden, inter, layers, max_kv_len, true, &p);
    if (rc) return rc;
    if (layer_table == nullptr || embed == nullptr || token == nullptr || d_kv_len == nullptr || h_out == nullptr ||
        residual_out == nullptr || vocab <= 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_stack: null pointer or empty vocabulary");
    if (workspace == nullptr || workspace_bytes < p.total || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return set_error(EFM_ERR_WORKSPACE, "decode_stack: a 256-byte aligned workspace of %zu bytes is required", p.total);
    StackArgs a;
    a.H = hidden;
    a.QD = (int)(ctx->num_qo_heads * ctx->head_dim);
    a.KVD = (int)(ctx->num_kv_heads * ctx->head_dim);
    a.I = inter;
    a.Hq = (int)ctx->num_qo_heads;
    a.Hkv = (int)ctx->num_kv_heads;
    a.layers = layers;
    a.vocab = vocab;
    a.eps = eps;
    a.layer = reinterpret_cast<const StackLayer*>(layer_table);
    a.embed = static_cast<const bf16_t*>(embed);
    a.token = token;
    a.d_kv_len = d_kv_len;
    a.max_kv_len = max_kv_len;
    a.n_attn = p.n_attn;
    a.cap = p.cap;
    a.ng = p.ng;
    a.ring = p.ring;
    a.x_off = p.x_off;
    a.r_off = p.r_off;
    a.out_off = p.out_off;
    a.misc_off = p.misc_off;
    a.tab_off = p.tab_off;
    rope_table_fill(&a.rope, (int)ctx->head_dim, ctx->rope_theta, ctx->rope_scale);
    a.q_pos_off = (int)ctx->q_rope_pos_offset;
    a.k_pos_off = (int)ctx->k_rope_pos_offset;
    char* w = static_cast<char*>(workspace);
    a.ctl = reinterpret_cast<uint32_t*>(w);
    a.rec_h = reinterpret_cast<uint4*>(w + p.off_h);
    a.rec_qkv = reinterpret_cast<uint4*>(w + p.off_qkv);
    a.rec_part = reinterpret_cast<uint4*>(w + p.off_part);
    a.rec_head = reinterpret_cast<uint4*>(w + p.off_head);
    a.rec_a = reinterpret_cast<uint4*>(w + p.off_a);
    a.rec_mid = reinterpret_cast<uint4*>(w + p.off_mid);
    a.h_out = static_cast<bf16_t*>(h_out);
    a.r_out = static_cast<bf16_t*>(residual_out);
    switch (p.G) {
        case 1: return stack_launch<1>(a, p, stream);
        case 2: return stack_launch<2>(a, p, stream);
        case 3: return stack_launch<3>(a, p, stream);
        case 4: return stack_launch<4>(a, p, stream);
        case 6: return stack_launch<6>(a, p, stream);
        case 7: return stack_launch<7>(a, p, stream);
        case 8: return stack_launch<8>(a, p, stream);
        default: return set_error(EFM_ERR_UNSUPPORTED, "decode_stack: group %d", p.G);
    }
}

extern "C" int efm_decode_stack_status(void* workspace, hipStream_t stream) {
    if (workspace == nullptr) return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_stack_status: null workspace");
    uint32_t ab = 0;
    hipError_t e = hipMemcpyAsync(&ab, static_cast<uint32_t*>(workspace) + 1, 4, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return set_error(EFM_ERR_DEVICE, "decode_stack_status: %s", hipGetErrorString(e));
    if (ab == 0u) return EFM_OK;
    const uint32_t zero = 0u;
    e = hipMemcpyAsync(static_cast<uint32_t*>(workspace) + 1, &zero, 4, hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    return set_error(EFM_ERR_DEVICE,
                     "decode_stack: a hand-off between workgroups timed out (not every workgroup was resident); the "
                     "step's outputs are invalid");
}

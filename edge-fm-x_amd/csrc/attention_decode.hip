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
//  * RoPE on read by angle addition: cos/sin(k * f_d) for the 32 key offsets of a tile
//    are tabulated once per workgroup, cos/sin(base * f_d) once per tile (one sincos
//    per thread), so rotating a key pair costs FMAs, not transcendentals. The tables
//    use sincos_reduced (Cody-Waite reduction + the hardware sin/cos, ~1e-6 absolute),
//    as the reference's decode kernel uses the fast sin/cos intrinsics.
//  * Each wave walks 32-key tiles of the workgroup's chunk; the next tile's K/V loads
//    are issued before the current tile's matrix work. Waves merge their (m, l, O)
//    through LDS.
//  * The split count is derived on the device from L = *d_kv_len and a host-chosen
//    keys-per-split target, so one launch geometry (sized by max_kv_len) serves every
//    step of a captured HIP graph. Short contexts run one workgroup per KV head (no
//    merge); long ones write fp32 (o, m, l) partials and the last workgroup of a KV head
//    (device-scope fence + atomic counter) merges them and resets the counter.
#include "common.hpp"

#include <algorithm>

namespace efm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kTileKeys = 32;
constexpr int kMaxSplits = 256;  // split_cap <= 256 / num_kv_heads
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
    int rope_q, rope_k;                       // apply rotation to q / to k
    int split_cap;                            // gridDim.x
    int keys_per_split;                       // target chunk length
    float* o_part;                            // [Hkv][split_cap][G][HD]
    float* ml_part;                           // [Hkv][split_cap][G][2]
    uint32_t* counter;                        // [Hkv]
    RopeTable rope;
};

union BfPack {
    bf16x8_t v;
    uint4 u;
    uint32_t w[4];
};

// MERGE = true: self-contained operator (the last workgroup of a KV head merges the
// splits). MERGE = false: every split only writes its (o, m, l) partial; the consumer
// (the o_proj GEMV prologue, efm_decode_attention_merge_o_proj) merges them.
template <int HD, int G, bool MERGE>
__global__ __launch_bounds__(kAttnThreads, 1) void decode_attn_kernel(DecodeArgs a) {
    constexpr int HALF = HD / 2;
    constexpr int KS = HD / 16;        // MFMA k-steps over head_dim
    constexpr int DT = HD / 32;        // d tiles of O^T
    constexpr int VP = kTileKeys + 8;  // V^T row pitch (bf16)
    static_assert(G <= 32, "group too large");

    __shared__ float sfreq[HALF];
    __shared__ float2 cs_off[kTileKeys][HALF + 1];      // cos/sin(k * f_d), k < 32 (padded rows)
    __shared__ float2 cs_q[HALF];                       // cos/sin(qpos * f_d)
    __shared__ float2 cs_base[kAttnWaves][HALF];        // cos/sin(base * f_d) of each wave's tile
    __shared__ __align__(16) bf16_t Vt[kAttnWaves][HD * VP];
    __shared__ float om[kAttnWaves][32], ol[kAttnWaves][32];
    __shared__ float ob[kAttnWaves][G][HD];
    __shared__ float sml[kMaxSplits * G];
    __shared__ float sll[kMaxSplits * G];
    __shared__ bool is_last;

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int ql = lane % 32, hh = lane / 32;
    const int kvh = blockIdx.y;
    const int b = blockIdx.x;

    uint32_t L = a.kv_len;
    if (a.d_kv_len != nullptr) L = min(a.d_kv_len[0], a.max_kv_len);
    const int kps = max(a.keys_per_split, kTileKeys);
    const int nsplit = (L == 0) ? 1 : (int)min((uint32_t)a.split_cap, (L + kps - 1) / kps);
    if (b >= nsplit) return;
    const int chunk = (L == 0) ? 0 : (int)((L + nsplit - 1) / nsplit);
    const int start = b * chunk;
    const int end = min((int)L, start + chunk);
    const int ntiles = (end > start) ? (end - start + kTileKeys - 1) / kTileKeys : 0;
    const int rounds = (ntiles + kAttnWaves - 1) / kAttnWaves;

    const bf16_t* kbase = a.k + (size_t)kvh * a.k_sh;
    const bf16_t* vbase = a.v + (size_t)kvh * a.v_sh;

    // ---- issue the first tile's K / V loads before anything else
    uint4 kr[KS], vr[KS];
    auto load_tile = [&](int t) {
        const int j = start + t * kTileKeys + ql;
        const bool ok = (t < ntiles) && (j < end);
        const bf16_t* kp = kbase + (size_t)(ok ? j : 0) * a.k_sn + hh * 8;
        const bf16_t* vp = vbase + (size_t)(ok ? j : 0) * a.v_sn + hh * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            kr[ks] = ok ? load_stream16(kp + ks * 16) : make_uint4(0, 0, 0, 0);
            vr[ks] = ok ? load_stream16(vp + ks * 16) : make_uint4(0, 0, 0, 0);
        }
    };
    load_tile(wave);

    // ---- RoPE tables
    if (tid < HALF) sfreq[tid] = a.rope.inv_freq[tid];
    __syncthreads();
    if (a.rope_q && tid < HALF) {
        float sn, cs;
        sincos_reduced((float)((int)L - 1 + a.q_pos_off) * sfreq[tid], &sn, &cs);
        cs_q[tid] = make_float2(cs, sn);
    }
    if (a.rope_k) {
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
        const bool qv = ql < G;
        const bf16_t* qp = a.q + (size_t)(kvh * G + (qv ? ql : 0)) * a.q_sh + hh * 8;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint4 u = qv ? *reinterpret_cast<const uint4*>(qp + ks * 16) : make_uint4(0, 0, 0, 0);
            unpack8(u, x[ks]);
        }
        if (a.rope_q) {
#pragma unroll
            for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float2 c2 = cs_q[ks * 16 + hh * 8 + e];
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

    for (int r = 0; r < rounds; ++r) {
        const int t = r * kAttnWaves + wave;
        const bool active = t < ntiles;
        const int t0 = start + t * kTileKeys;
        // base-angle table for the 4 tiles of this round: one sincos per thread
        if (a.rope_k && tid < kAttnWaves * HALF) {
            const int w = tid / HALF, d = tid % HALF;
            const int base = start + (r * kAttnWaves + w) * kTileKeys + a.k_pos_off;
            float sn, cs;
            sincos_reduced((float)base * sfreq[d], &sn, &cs);
            cs_base[w][d] = make_float2(cs, sn);
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

        // rotate K in registers (angle addition) and pack the A operand
        BfPack kp[KS];
        if (a.rope_k) {
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
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) kp[ks].u = kr[ks];
        }
        // prefetch the next round's tile while this one is multiplied
        load_tile(t + kAttnWaves);

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
            const float alpha = exp2f(m_run - m_new);
            float p[16], psum = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                p[e] = exp2f(s[e] - m_new);
                psum += p[e];
            }
            psum += __shfl_xor(psum, 32, kWave);
            l_run = l_run * alpha + psum;
            m_run = m_new;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[tt][e] *= alpha;
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
    if (!MERGE || nsplit == 1) return;

    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&a.counter[kvh], 1u);
        is_last = (prev == (uint32_t)nsplit - 1);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();

    // Merge: stage every split's (m, l) in LDS with parallel loads, turn them into
    // normalised weights w_s = exp2(m_s - M) / sum_s exp2(m_s - M) l_s (one wave per query
    // head), then accumulate the partial outputs with independent, unrolled loads.
    const size_t head_base = (size_t)kvh * a.split_cap * G;
    for (int i = tid; i < nsplit * G; i += kAttnThreads) {
        sml[i] = a.ml_part[(head_base + i) * 2];
        sll[i] = a.ml_part[(head_base + i) * 2 + 1];
    }
    __syncthreads();
    for (int g = wave; g < G; g += kAttnWaves) {
        float M = -INFINITY;
        for (int s = lane; s < nsplit; s += kWave) M = fmaxf(M, sml[s * G + g]);
        M = wave_max(M);
        float den = 0.f;
        for (int s = lane; s < nsplit; s += kWave) {
            const float m = sml[s * G + g];
            den += (m == -INFINITY) ? 0.f : exp2f(m - M) * sll[s * G + g];
        }
        den = wave_sum(den);
        const float inv = (den > 0.f) ? 1.f / den : 0.f;
        for (int s = lane; s < nsplit; s += kWave) {
            const float m = sml[s * G + g];
            sml[s * G + g] = (m == -INFINITY) ? 0.f : exp2f(m - M) * inv;
        }
    }
    __syncthreads();
    for (int t = tid; t < G * HD; t += kAttnThreads) {
        const int g = t / HD, d = t % HD;
        const float* op = a.o_part + (head_base + g) * HD + d;
        float num = 0.f;
#pragma unroll 8
        for (int s = 0; s < nsplit; ++s) num = fmaf(sml[s * G + g], op[(size_t)s * G * HD], num);
        a.o[(size_t)(kvh * G + g) * HD + d] = (bf16_t)f32_to_bf16(num);
    }
    if (tid == 0) a.counter[kvh] = 0u;
}

// Keys per split: one 32-key tile per wave (128 keys per workgroup) so that every K/V
// load of a workgroup is in flight at once; the split count is capped at 256 workgroups.
constexpr int kKeysPerSplit = 128;

int decode_split_cap(int num_kv_heads, uint32_t max_kv_len) {
    const int by_len = (int)std::max<uint32_t>(1u, (max_kv_len + kKeysPerSplit - 1) / kKeysPerSplit);
    const int by_chip = std::max(1, kMaxSplits / std::max(1, num_kv_heads));
    return std::min(by_len, by_chip);
}

int decode_keys_per_split() { return kKeysPerSplit; }

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
    a.rope_k = a.rope_q && !ctx->k_already_prerotated;
    a.split_cap = decode_split_cap((int)ctx->num_kv_heads, std::max<uint32_t>(bound, 1u));
    a.keys_per_split = kKeysPerSplit;
    char* wsb = static_cast<char*>(workspace);
    a.o_part = reinterpret_cast<float*>(wsb);
    a.ml_part = reinterpret_cast<float*>(wsb + ws.o_bytes);
    a.counter = reinterpret_cast<uint32_t*>(wsb + ws.o_bytes + ws.ml_bytes);

    dim3 grid(a.split_cap, ctx->num_kv_heads), block(kAttnThreads);
#define EFM_DEC_CASE(HDV, GV)                                                                             \
    if (hd == HDV && G == GV) {                                                                           \
        if (merge) hipLaunchKernelGGL((decode_attn_kernel<HDV, GV, true>), grid, block, 0, stream, a);    \
        else hipLaunchKernelGGL((decode_attn_kernel<HDV, GV, false>), grid, block, 0, stream, a);         \
        return check_launch("attention_decode");                                                          \
    }
    EFM_DEC_CASE(128, 1) EFM_DEC_CASE(128, 2) EFM_DEC_CASE(128, 3) EFM_DEC_CASE(128, 4)
    EFM_DEC_CASE(128, 6) EFM_DEC_CASE(128, 7) EFM_DEC_CASE(128, 8)
    EFM_DEC_CASE(64, 1) EFM_DEC_CASE(64, 2) EFM_DEC_CASE(64, 3) EFM_DEC_CASE(64, 4)
    EFM_DEC_CASE(64, 6) EFM_DEC_CASE(64, 7) EFM_DEC_CASE(64, 8)
#undef EFM_DEC_CASE
    return set_error(EFM_ERR_UNSUPPORTED, "attention_decode: hd=%d G=%d", hd, G);
}

}  // namespace efm

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

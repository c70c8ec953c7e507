// Single-query GQA decode attention over the fixed-prefix KV cache (gfx950).
//
// Semantics (FlashInfer single_decode_with_kv_cache, ROPE_LLAMA, as called from
// src/operators/attention_op.cu:1428-1466): for each query head h with KV head
// g = h / (Hq / Hkv),
//     o_h = sum_j softmax_j( RoPE(q_h, L-1) . RoPE(k_gj, j) / sqrt(hd) ) v_gj,  j < L,
// with RoPE the rotate-half rotation of pairs (d, d + hd/2). The cache holds
// un-rotated K, so keys are rotated on read.
//
// Kernel design:
//  * grid (splits, Hkv), 256 threads. All G = Hq/Hkv query heads of a KV head share
//    every K/V byte a workgroup loads, so KV traffic is read once per step.
//  * The split count and chunk length are derived on the device from L = *d_kv_len,
//    so one launch geometry (sized by max_kv_len) stays valid for every decode step
//    of a captured HIP graph.
//  * QK: hd/16 lanes per key; each lane holds 8 rotation pairs (16-byte loads of
//    both halves), rotates them in registers and dot-products with the pre-rotated,
//    pre-scaled q held in registers; partial dots are reduced across those lanes.
//  * Online softmax in base 2 (log2(e)/sqrt(hd) folded into q); PV with 16-byte V
//    loads per lane; K and V for a pass are loaded together so one memory round trip
//    covers both.
//  * Splits write fp32 (o, m, l) partials; the last workgroup of a KV head to arrive
//    (device-scope fence + atomic counter) merges them with the log-sum-exp rule and
//    resets the counter, so there is no second launch and no host-side state.
#include "common.hpp"

#include <algorithm>

namespace efm {

constexpr int kAttnThreads = 256;
constexpr int kMaxSplits = 512;  // split_cap <= 512 / num_kv_heads
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
    float* o_part;                            // [Hkv][split_cap][G][HD]
    float* ml_part;                           // [Hkv][split_cap][G][2]
    uint32_t* counter;                        // [Hkv]
    RopeTable rope;
};

template <int HD, int G>
__global__ __launch_bounds__(kAttnThreads) void decode_attn_kernel(DecodeArgs a) {
    constexpr int HALF = HD / 2;
    constexpr int TPK = HALF / 8;              // lanes per key in QK
    constexpr int KP = kAttnThreads / TPK;     // keys per pass
    constexpr int DCH = HD / 8;                // 16-byte chunks per V row
    constexpr int KG = kAttnThreads / DCH;     // key groups in PV
    constexpr int VPT = KP / KG;               // V rows per lane per pass
    static_assert(VPT >= 1 && KP % KG == 0, "bad decode tiling");

    __shared__ float qs[G][HD];
    __shared__ float sfreq[HALF];
    __shared__ float sc[G][KP];
    __shared__ float ored[kAttnThreads / kWave][G][HD];
    __shared__ float sml[kMaxSplits * G];
    __shared__ float sll[kMaxSplits * G];
    __shared__ bool is_last;

    const int tid = threadIdx.x;
    const int lane = tid % kWave;
    const int wave = tid / kWave;
    const int kvh = blockIdx.y;
    const int b = blockIdx.x;

    uint32_t L = a.kv_len;
    if (a.d_kv_len != nullptr) L = min(a.d_kv_len[0], a.max_kv_len);
    const int nsplit = (L == 0) ? 1 : (int)min((uint32_t)a.split_cap, (L + KP - 1) / KP);
    if (b >= nsplit) return;
    const int chunk = (L == 0) ? 0 : (int)((L + nsplit - 1) / nsplit);
    const int start = b * chunk;
    const int end = min((int)L, start + chunk);

    if (tid < HALF) sfreq[tid] = a.rope.inv_freq[tid];
    __syncthreads();
    // Rotated, scaled queries -> LDS.
    const float qscale = kLog2e / sqrtf((float)HD);
    for (int t = tid; t < G * HALF; t += kAttnThreads) {
        const int g = t / HALF, d = t % HALF;
        const bf16_t* qp = a.q + (size_t)(kvh * G + g) * a.q_sh;
        const float x0 = bf16_to_f32(qp[d]);
        const float x1 = bf16_to_f32(qp[d + HALF]);
        float y0 = x0, y1 = x1;
        if (a.rope_q) {
            const float ang = (float)((int)L - 1 + a.q_pos_off) * sfreq[d];
            float sn, cs;
            sincosf(ang, &sn, &cs);
            y0 = x0 * cs - x1 * sn;
            y1 = x1 * cs + x0 * sn;
        }
        qs[g][d] = y0 * qscale;
        qs[g][d + HALF] = y1 * qscale;
    }
    __syncthreads();

    // QK role.
    const int kk = tid / TPK;
    const int d0 = (tid % TPK) * 8;
    float qlo[G][8], qhi[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            qlo[g][e] = qs[g][d0 + e];
            qhi[g][e] = qs[g][d0 + HALF + e];
        }
    float ifreq[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) ifreq[e] = sfreq[d0 + e];

    // PV role.
    const int dch = tid % DCH;
    const int kg = tid / DCH;
    float acc[G][8];
    float m_run[G], l_run[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    }

    const bf16_t* kbase = a.k + (size_t)kvh * a.k_sh;
    const bf16_t* vbase = a.v + (size_t)kvh * a.v_sh;

    for (int base = start; base < end; base += KP) {
        const int j = base + kk;
        const bool kvalid = j < end;
        uint4 klo = make_uint4(0, 0, 0, 0), khi = make_uint4(0, 0, 0, 0);
        if (kvalid) {
            const bf16_t* kr = kbase + (size_t)j * a.k_sn;
            klo = load_stream16(kr + d0);
            khi = load_stream16(kr + d0 + HALF);
        }
        uint4 vv[VPT];
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int jv = base + kg + KG * i;
            vv[i] = (jv < end) ? load_stream16(vbase + (size_t)jv * a.v_sn + dch * 8) : make_uint4(0, 0, 0, 0);
        }

        float k0[8], k1[8];
        unpack8(klo, k0);
        unpack8(khi, k1);
        if (a.rope_k) {
            const float pos = (float)(j + a.k_pos_off);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float sn, cs;
                sincos_reduced(pos * ifreq[e], &sn, &cs);
                const float x0 = k0[e], x1 = k1[e];
                k0[e] = x0 * cs - x1 * sn;
                k1[e] = x1 * cs + x0 * sn;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                s = fmaf(qlo[g][e], k0[e], s);
                s = fmaf(qhi[g][e], k1[e], s);
            }
            s = group_sum<TPK>(s);
            if ((tid % TPK) == 0) sc[g][kk] = kvalid ? s : -INFINITY;
        }
        __syncthreads();

#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float sl = (lane < KP) ? sc[g][lane % KP] : -INFINITY;
            const float tmax = wave_max(sl);
            const float m_new = fmaxf(m_run[g], tmax);
            // m_new is finite: every pass holds at least one valid key.
            const float alpha = exp2f(m_run[g] - m_new);
            const float tsum = wave_sum((lane < KP) ? exp2f(sl - m_new) : 0.f);
            l_run[g] = l_run[g] * alpha + tsum;
            m_run[g] = m_new;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
#pragma unroll
            for (int i = 0; i < VPT; ++i) {
                const float p = exp2f(sc[g][kg + KG * i] - m_new);
                float vf[8];
                unpack8(vv[i], vf);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p, vf[e], acc[g][e]);
            }
        }
        __syncthreads();
    }

    // Reduce acc over key groups: lanes sharing dch inside a wave, then across waves.
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = acc[g][e];
#pragma unroll
            for (int off = DCH; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
            acc[g][e] = v;
        }
    if (lane < DCH) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) ored[wave][g][dch * 8 + e] = acc[g][e];
    }
    __syncthreads();

    const size_t part_base = ((size_t)kvh * a.split_cap + b) * G;
    for (int t = tid; t < G * HD; t += kAttnThreads) {
        const int g = t / HD, d = t % HD;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnThreads / kWave; ++w) s += ored[w][g][d];
        a.o_part[(part_base + g) * HD + d] = s;
    }
    if (tid < G) {
        // m_run / l_run are wave-uniform and identical in every thread.
        float mv = 0.f, lv = 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g)
            if (g == tid) { mv = m_run[g]; lv = l_run[g]; }
        a.ml_part[(part_base + tid) * 2 + 0] = mv;
        a.ml_part[(part_base + tid) * 2 + 1] = lv;
    }

    if (nsplit == 1) {
        // Single split: normalise directly, no merge needed.
        __syncthreads();
        for (int t = tid; t < G * HD; t += kAttnThreads) {
            const int g = t / HD, d = t % HD;
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < kAttnThreads / kWave; ++w) s += ored[w][g][d];
            float lv = 0.f;
#pragma unroll
            for (int gg = 0; gg < G; ++gg)
                if (gg == g) lv = l_run[gg];
            const float outv = (lv > 0.f) ? s / lv : 0.f;
            a.o[(size_t)(kvh * G + g) * HD + d] = (bf16_t)f32_to_bf16(outv);
        }
        return;
    }

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
    for (int g = wave; g < G; g += kAttnThreads / kWave) {
        float M = -INFINITY;
        for (int s = lane; s < nsplit; s += kWave) M = fmaxf(M, sml[s * G + g]);
        M = wave_max(M);
        float den = 0.f;
        for (int s = lane; s < nsplit; s += kWave) den += exp2f(sml[s * G + g] - M) * sll[s * G + g];
        den = wave_sum(den);
        const float inv = (den > 0.f) ? 1.f / den : 0.f;
        for (int s = lane; s < nsplit; s += kWave) sml[s * G + g] = exp2f(sml[s * G + g] - M) * inv;
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

static int decode_keys_per_pass(int hd) { return kAttnThreads / (hd / 16); }

static int decode_split_cap(int num_kv_heads, int hd, uint32_t max_kv_len) {
    const int kp = decode_keys_per_pass(hd);
    const int by_len = (int)std::max<uint32_t>(1u, (max_kv_len + kp - 1) / kp);
    const int by_chip = std::max(1, 512 / std::max(1, num_kv_heads));
    return std::min(by_len, by_chip);
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct DecodeWs {
    size_t o_bytes, ml_bytes, cnt_bytes;
    size_t total() const { return o_bytes + ml_bytes + cnt_bytes; }
};

static DecodeWs decode_ws(const efm_attention_ctx* c, uint32_t max_kv_len) {
    const int G = c->num_qo_heads / c->num_kv_heads;
    const int cap = decode_split_cap(c->num_kv_heads, c->head_dim, max_kv_len);
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

}  // namespace efm

using namespace efm;

extern "C" size_t efm_attention_decode_workspace_bytes(const efm_attention_ctx* ctx, uint32_t max_kv_len) {
    if (validate_attention_ctx(ctx, "attention_decode_workspace_bytes") != EFM_OK) return 0;
    return decode_ws(ctx, max_kv_len).total();
}

extern "C" int efm_attention_decode(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v,
                                    void* o, uint32_t kv_len, const uint32_t* d_kv_len, uint32_t max_kv_len,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
    int rc = validate_attention_ctx(ctx, "attention_decode");
    if (rc) return rc;
    if (q == nullptr || k == nullptr || v == nullptr || o == nullptr)
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
    a.split_cap = decode_split_cap((int)ctx->num_kv_heads, hd, std::max<uint32_t>(bound, 1u));
    char* wsb = static_cast<char*>(workspace);
    a.o_part = reinterpret_cast<float*>(wsb);
    a.ml_part = reinterpret_cast<float*>(wsb + ws.o_bytes);
    a.counter = reinterpret_cast<uint32_t*>(wsb + ws.o_bytes + ws.ml_bytes);

    dim3 grid(a.split_cap, ctx->num_kv_heads), block(kAttnThreads);
#define EFM_DEC_CASE(HDV, GV)                                                             \
    if (hd == HDV && G == GV) {                                                           \
        hipLaunchKernelGGL((decode_attn_kernel<HDV, GV>), grid, block, 0, stream, a);     \
        return check_launch("attention_decode");                                          \
    }
    EFM_DEC_CASE(128, 1) EFM_DEC_CASE(128, 2) EFM_DEC_CASE(128, 3) EFM_DEC_CASE(128, 4)
    EFM_DEC_CASE(128, 6) EFM_DEC_CASE(128, 7) EFM_DEC_CASE(128, 8)
    EFM_DEC_CASE(64, 1) EFM_DEC_CASE(64, 2) EFM_DEC_CASE(64, 3) EFM_DEC_CASE(64, 4)
    EFM_DEC_CASE(64, 6) EFM_DEC_CASE(64, 7) EFM_DEC_CASE(64, 8)
#undef EFM_DEC_CASE
    return set_error(EFM_ERR_UNSUPPORTED, "attention_decode: hd=%d G=%d", hd, G);
}

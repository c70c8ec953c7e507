// Row-wise and element-wise kernels of the hot path: RMSNorm, fused add + RMSNorm,
// SiLU-and-mul, embedding gather, decode runtime scalars, KV-slot copies and the
// greedy sampler. All are bandwidth/latency-bound; rows are processed with 16-byte
// vectors by one 256-thread workgroup per row.
#include "common.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>

namespace efm {

constexpr int kRowThreads = 256;
constexpr int kRowMaxChunks = 8;  // hidden <= 8 * 256 * 8 = 16384

// RMSNorm of one row (src/operators/norm_op.cu:20-106): fp32 sum of squares,
// out = bf16((x * rsqrt(mean + eps)) * w). FUSED: s = x + residual, residual <- bf16(s),
// and the normalisation uses the fp32 sum (FlashInfer FusedAddRMSNorm).
template <bool FUSED>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_kernel(const bf16_t* in, bf16_t* residual, const bf16_t* w,
                                                              bf16_t* out, int hidden, float eps) {
    __shared__ float red[kRowThreads / kWave];
    const int C = hidden >> 3;
    const size_t row = blockIdx.x;
    const uint4* x4 = reinterpret_cast<const uint4*>(in + row * hidden);
    uint4* r4 = FUSED ? reinterpret_cast<uint4*>(residual + row * hidden) : nullptr;
    float s[kRowMaxChunks][8];
    float ss = 0.f;
    // the norm weight's chunks go out with the row's (not after the reduction)
    const uint4* w4 = reinterpret_cast<const uint4*>(w);
    uint4 wv[kRowMaxChunks];
#pragma unroll
    for (int i = 0; i < kRowMaxChunks; ++i) {
        const int c = threadIdx.x + i * kRowThreads;
        wv[i] = (c < C) ? w4[c] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kRowMaxChunks; ++i) {
        const int c = threadIdx.x + i * kRowThreads;
        if (c < C) {
            unpack8(x4[c], s[i]);
            if (FUSED) {
                float r[8];
                unpack8(r4[c], r);
#pragma unroll
                for (int e = 0; e < 8; ++e) s[i][e] += r[e];
                r4[c] = pack8(s[i]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(s[i][e], s[i][e], ss);
        }
    }
    const float tot = block_total<kRowThreads>(ss, red);
    const float inv = 1.0f / sqrtf(tot / (float)hidden + eps);
    uint4* o4 = reinterpret_cast<uint4*>(out + row * hidden);
#pragma unroll
    for (int i = 0; i < kRowMaxChunks; ++i) {
        const int c = threadIdx.x + i * kRowThreads;
        if (c < C) {
            float wf[8], o[8];
            unpack8(wv[i], wf);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (s[i][e] * inv) * wf[e];
            o4[c] = pack8(o);
        }
    }
}

// out[b, i] = bf16(silu(gate) * up); input row = [gate | up] or [up | gate]
// (src/operators/activation_op.cu:36-76).
__global__ __launch_bounds__(kRowThreads) void act_and_mul_kernel(const bf16_t* in, bf16_t* out, int64_t hidden,
                                                                  int up_first) {
    const int64_t row = blockIdx.y;
    const bf16_t* base = in + row * 2 * hidden;
    const uint4* up4 = reinterpret_cast<const uint4*>(base + (up_first ? 0 : hidden));
    const uint4* gate4 = reinterpret_cast<const uint4*>(base + (up_first ? hidden : 0));
    uint4* o4 = reinterpret_cast<uint4*>(out + row * hidden);
    const int64_t C = hidden >> 3;
    for (int64_t c = (int64_t)blockIdx.x * kRowThreads + threadIdx.x; c < C; c += (int64_t)gridDim.x * kRowThreads) {
        float u[8], g[8], o[8];
        unpack8(up4[c], u);
        unpack8(gate4[c], g);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = silu_f32(g[e]) * u[e];
        o4[c] = pack8(o);
    }
}

// One workgroup per token row (src/layers/embed_head.cu:63-132).
__global__ __launch_bounds__(kRowThreads) void embedding_kernel(const int32_t* ids, const bf16_t* table,
                                                                const bf16_t* custom, int64_t n_custom,
                                                                int32_t embed_token_id, int64_t vocab,
                                                                int64_t hidden, bf16_t* out) {
    const int64_t t = blockIdx.x;
    const int32_t id = ids[t];
    const bf16_t* src = nullptr;
    if (custom != nullptr && embed_token_id >= 0 && (int64_t)id >= embed_token_id &&
        (int64_t)id < (int64_t)embed_token_id + n_custom) {
        src = custom + (int64_t)(id - embed_token_id) * hidden;
    } else if (id >= 0 && (int64_t)id < vocab) {
        src = table + (int64_t)id * hidden;
    }
    uint4* o4 = reinterpret_cast<uint4*>(out + t * hidden);
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    for (int64_t c = threadIdx.x; c < (hidden >> 3); c += kRowThreads) {
        o4[c] = (src != nullptr) ? s4[c] : make_uint4(0, 0, 0, 0);
    }
}

// Decode KV-slot copy (decode_runtime_kernels.cu:101-150): row -> slot (*d_kv_len - 1).
__global__ void copy_kv_slots_kernel(const bf16_t* k_src, const bf16_t* v_src, bf16_t* k_cache, bf16_t* v_cache,
                                     int k_elems, int v_elems, const uint32_t* d_kv_len) {
    const uint32_t L = d_kv_len[0];
    if (L == 0) return;
    const size_t slot = L - 1;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < k_elems + v_elems; i += gridDim.x * blockDim.x) {
        if (i < k_elems) k_cache[slot * k_elems + i] = k_src[i];
        else v_cache[slot * v_elems + (i - k_elems)] = v_src[i - k_elems];
    }
}

__global__ void finalize_token_kernel(const int32_t* sampled, int32_t* response, uint32_t* d_kv_len) {
    if (threadIdx.x == 0) {
        if (sampled != nullptr && response != nullptr) response[0] = sampled[0];
        if (d_kv_len != nullptr) d_kv_len[0] += 1u;
    }
}

__global__ void increment_triplet_kernel(int32_t* v) {
    if (threadIdx.x < 3) v[threadIdx.x] += 1;
}

// Greedy argmax over fp32 logits rows, two stages (src/layers/sampler.cu:39-105):
// stage 1: grid (parts, rows) -> partial (value, index); stage 2: one workgroup per row.
constexpr int kArgmaxParts = 64;

__global__ __launch_bounds__(kRowThreads) void argmax_stage1(const float* logits, int64_t vocab, ArgMax* part) {
    __shared__ ArgMax wbest[kRowThreads / kWave];
    const int64_t row = blockIdx.y;
    const float* x = logits + row * vocab;
    const int64_t per = (vocab + gridDim.x - 1) / gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * per;
    const int64_t hi = lo + per < vocab ? lo + per : vocab;
    ArgMax b;
    b.v = -INFINITY;
    b.i = 0x7fffffff;
    for (int64_t i = lo + threadIdx.x; i < hi; i += kRowThreads) {
        ArgMax c;
        c.v = x[i];
        c.i = (int32_t)i;
        b = argmax_pick(b, c);
    }
    b = wave_argmax(b);
    if (threadIdx.x % kWave == 0) wbest[threadIdx.x / kWave] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        ArgMax f = wbest[0];
        for (int w = 1; w < kRowThreads / kWave; ++w) f = argmax_pick(f, wbest[w]);
        part[row * gridDim.x + blockIdx.x] = f;
    }
}

__global__ __launch_bounds__(kWave) void argmax_stage2(const ArgMax* part, int parts, int32_t* out) {
    const int64_t row = blockIdx.x;
    ArgMax b;
    b.v = -INFINITY;
    b.i = 0x7fffffff;
    for (int i = threadIdx.x; i < parts; i += kWave) b = argmax_pick(b, part[row * parts + i]);
    b = wave_argmax(b);
    if (threadIdx.x == 0) out[row] = (b.i == 0x7fffffff) ? 0 : b.i;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace efm

using namespace efm;

extern "C" int efm_rms_norm(uint32_t batch, uint32_t hidden, float eps, const void* input, const void* weight,
                            void* output, hipStream_t stream) {
    if (input == nullptr || weight == nullptr || output == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "rms_norm: null pointer");
    if (hidden == 0 || hidden % 8 != 0 || hidden > 8u * kRowThreads * kRowMaxChunks)
        return set_error(EFM_ERR_UNSUPPORTED, "rms_norm: hidden %u must be a multiple of 8 and <= %d", hidden,
                         8 * kRowThreads * kRowMaxChunks);
    if (!aligned16(input) || !aligned16(weight) || !aligned16(output))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "rms_norm: pointers must be 16-byte aligned");
    if (batch == 0) return EFM_OK;
    hipLaunchKernelGGL((rmsnorm_kernel<false>), dim3(batch), dim3(kRowThreads), 0, stream,
                       static_cast<const bf16_t*>(input), (bf16_t*)nullptr, static_cast<const bf16_t*>(weight),
                       static_cast<bf16_t*>(output), (int)hidden, eps);
    return check_launch("rms_norm");
}

extern "C" int efm_fused_add_rms_norm(uint32_t batch, uint32_t hidden, float eps, void* inout, void* residual,
                                      const void* weight, hipStream_t stream) {
    if (inout == nullptr || residual == nullptr || weight == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "fused_add_rms_norm: null pointer");
    if (hidden == 0 || hidden % 8 != 0 || hidden > 8u * kRowThreads * kRowMaxChunks)
        return set_error(EFM_ERR_UNSUPPORTED, "fused_add_rms_norm: hidden %u unsupported", hidden);
    if (!aligned16(inout) || !aligned16(residual) || !aligned16(weight))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "fused_add_rms_norm: pointers must be 16-byte aligned");
    if (batch == 0) return EFM_OK;
    hipLaunchKernelGGL((rmsnorm_kernel<true>), dim3(batch), dim3(kRowThreads), 0, stream,
                       static_cast<const bf16_t*>(inout), static_cast<bf16_t*>(residual),
                       static_cast<const bf16_t*>(weight), static_cast<bf16_t*>(inout), (int)hidden, eps);
    return check_launch("fused_add_rms_norm");
}

extern "C" int efm_act_and_mul(int64_t batch, int64_t hidden, int32_t layout, const void* input, void* output,
                               hipStream_t stream) {
    if (input == nullptr || output == nullptr) return set_error(EFM_ERR_INVALID_ARGUMENT, "act_and_mul: null pointer");
    if (hidden <= 0 || hidden % 8 != 0) return set_error(EFM_ERR_UNSUPPORTED, "act_and_mul: hidden %% 8 != 0");
    if (layout != EFM_LAYOUT_GATE_UP && layout != EFM_LAYOUT_UP_GATE)
        return set_error(EFM_ERR_UNSUPPORTED, "act_and_mul: layout %d", layout);
    if (!aligned16(input) || !aligned16(output))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "act_and_mul: pointers must be 16-byte aligned");
    if (batch <= 0) return EFM_OK;
    if (batch > 65535) return set_error(EFM_ERR_UNSUPPORTED, "act_and_mul: batch > 65535");
    const int64_t C = hidden / 8;
    const int gx = (int)std::min<int64_t>((C + kRowThreads - 1) / kRowThreads, 64);
    hipLaunchKernelGGL(act_and_mul_kernel, dim3(gx, (unsigned)batch), dim3(kRowThreads), 0, stream,
                       static_cast<const bf16_t*>(input), static_cast<bf16_t*>(output), hidden,
                       layout == EFM_LAYOUT_UP_GATE ? 1 : 0);
    return check_launch("act_and_mul");
}

extern "C" int efm_embedding_lookup(int64_t n_tokens, int64_t hidden, int64_t vocab, const int32_t* ids,
                                    const void* table, const void* custom_embeddings, int64_t n_custom,
                                    int32_t embed_token_id, void* out, hipStream_t stream) {
    if (ids == nullptr || table == nullptr || out == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "embedding_lookup: null pointer");
    if (hidden <= 0 || hidden % 8 != 0) return set_error(EFM_ERR_UNSUPPORTED, "embedding_lookup: hidden %% 8 != 0");
    if (n_tokens < 0 || n_tokens > 0x7fffffff) return set_error(EFM_ERR_INVALID_ARGUMENT, "embedding_lookup: n_tokens");
    if (n_tokens == 0) return EFM_OK;
    hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)n_tokens), dim3(kRowThreads), 0, stream, ids,
                       static_cast<const bf16_t*>(table), static_cast<const bf16_t*>(custom_embeddings), n_custom,
                       embed_token_id, vocab, hidden, static_cast<bf16_t*>(out));
    return check_launch("embedding_lookup");
}

extern "C" int efm_copy_decode_kv_cache_slots(const void* k_src, const void* v_src, void* k_cache, void* v_cache,
                                              int32_t k_elems, int32_t v_elems, const uint32_t* d_kv_len,
                                              hipStream_t stream) {
    if (!k_src || !v_src || !k_cache || !v_cache || !d_kv_len)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "copy_decode_kv_cache_slots: null pointer");
    if (k_elems <= 0 || v_elems <= 0) return set_error(EFM_ERR_INVALID_ARGUMENT, "copy_decode_kv_cache_slots: sizes");
    const int n = k_elems + v_elems;
    hipLaunchKernelGGL(copy_kv_slots_kernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                       static_cast<const bf16_t*>(k_src), static_cast<const bf16_t*>(v_src),
                       static_cast<bf16_t*>(k_cache), static_cast<bf16_t*>(v_cache), k_elems, v_elems, d_kv_len);
    return check_launch("copy_decode_kv_cache_slots");
}

extern "C" int efm_finalize_decode_token(const int32_t* sampled_token, int32_t* response_token, uint32_t* d_kv_len,
                                         hipStream_t stream) {
    hipLaunchKernelGGL(finalize_token_kernel, dim3(1), dim3(kWave), 0, stream, sampled_token, response_token, d_kv_len);
    return check_launch("finalize_decode_token");
}

extern "C" int efm_increment_int32_triplet(int32_t* values, hipStream_t stream) {
    if (values == nullptr) return set_error(EFM_ERR_INVALID_ARGUMENT, "increment_int32_triplet: null pointer");
    hipLaunchKernelGGL(increment_triplet_kernel, dim3(1), dim3(kWave), 0, stream, values);
    return check_launch("increment_int32_triplet");
}

extern "C" size_t efm_sampler_greedy_workspace_bytes(int64_t rows, int64_t vocab) {
    (void)vocab;
    return (size_t)std::max<int64_t>(rows, 1) * kArgmaxParts * sizeof(ArgMax);
}

extern "C" int efm_sampler_greedy(int64_t rows, int64_t vocab, const float* logits, int32_t* out, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
    if (logits == nullptr || out == nullptr) return set_error(EFM_ERR_INVALID_ARGUMENT, "sampler_greedy: null pointer");
    if (vocab <= 0 || vocab > 0x7fffffff) return set_error(EFM_ERR_INVALID_ARGUMENT, "sampler_greedy: vocab");
    if (rows <= 0) return EFM_OK;
    if (rows > 65535) return set_error(EFM_ERR_UNSUPPORTED, "sampler_greedy: rows > 65535");
    if (workspace == nullptr || workspace_bytes < efm_sampler_greedy_workspace_bytes(rows, vocab))
        return set_error(EFM_ERR_WORKSPACE, "sampler_greedy: workspace of %zu bytes required",
                         efm_sampler_greedy_workspace_bytes(rows, vocab));
    ArgMax* part = static_cast<ArgMax*>(workspace);
    hipLaunchKernelGGL(argmax_stage1, dim3(kArgmaxParts, (unsigned)rows), dim3(kRowThreads), 0, stream, logits, vocab,
                       part);
    int rc = check_launch("sampler_greedy stage1");
    if (rc) return rc;
    hipLaunchKernelGGL(argmax_stage2, dim3((unsigned)rows), dim3(kWave), 0, stream, (const ArgMax*)part, kArgmaxParts,
                       out);
    return check_launch("sampler_greedy stage2");
}

// ----------------------------------------------------------------------------------
// M-RoPE (src/layers/attention.cu:17-118): rotation pair d of a head uses the position
// row of its section (cumulative mrope_section boundaries; both halves of a pair share
// the section of d). Rotated values are written back as bf16.
// ----------------------------------------------------------------------------------
namespace efm {

struct MropeArgs {
    bf16_t* q;
    bf16_t* k;
    const int32_t* pos;   // [3, pos_stride]; NULL: every section uses pos_offset + token
    int pos_stride;       // tokens per position row
    int pos_offset;
    int S, Hq, Hkv, hd;
    int q_sn, k_sn;       // token strides (elements); heads are contiguous hd apart
    int cum0, cum1;
    RopeTable rope;
};

__device__ __forceinline__ void mrope_pair(bf16_t* row, int d, int half, int p, float inv) {
    float sn, cs;
    sincosf((float)p * inv, &sn, &cs);
    const float x0 = bf16_to_f32(row[d]);
    const float x1 = bf16_to_f32(row[d + half]);
    row[d] = (bf16_t)f32_to_bf16(x0 * cs - x1 * sn);
    row[d + half] = (bf16_t)f32_to_bf16(x1 * cs + x0 * sn);
}

// grid (S, Hq + Hkv), block >= hd/2 threads.
__global__ void mrope_kernel(MropeArgs a) {
    const int t = blockIdx.x;
    const int h = blockIdx.y;
    const int half = a.hd / 2;
    const int d = threadIdx.x;
    if (d >= half) return;
    const int sec = (d < a.cum0) ? 0 : (d < a.cum1 ? 1 : 2);
    const int p = (a.pos != nullptr) ? a.pos[sec * a.pos_stride + t] : a.pos_offset + t;
    const float inv = a.rope.inv_freq[d];
    bf16_t* row = (h < a.Hq) ? a.q + (size_t)t * a.q_sn + (size_t)h * a.hd
                             : a.k + (size_t)t * a.k_sn + (size_t)(h - a.Hq) * a.hd;
    mrope_pair(row, d, half, p, inv);
}

// Decode: rotate q (src -> dst) and k, write rotated k and raw v to cache slot
// (*d_kv_len - 1) (decode_runtime_kernels.cu:152-225). grid (1, Hq + 2*Hkv).
__global__ void decode_mrope_write_kv_kernel(const bf16_t* q_src, const bf16_t* k_src, const bf16_t* v_src,
                                             bf16_t* q_dst, bf16_t* k_cache, bf16_t* v_cache, int Hq, int Hkv,
                                             int hd, const int32_t* pos, int cum0, int cum1, RopeTable rope,
                                             const uint32_t* d_kv_len) {
    const int h = blockIdx.y;
    const int half = hd / 2;
    const int d = threadIdx.x;
    if (d >= half) return;
    const uint32_t L = d_kv_len[0];
    const size_t slot = (L > 0) ? (size_t)(L - 1) : 0;
    const int kvd = Hkv * hd;
    if (h >= Hq + Hkv) {  // V rows: plain copy
        if (L == 0) return;
        const int hv = h - Hq - Hkv;
        v_cache[slot * kvd + hv * hd + d] = v_src[hv * hd + d];
        v_cache[slot * kvd + hv * hd + d + half] = v_src[hv * hd + d + half];
        return;
    }
    const int sec = (d < cum0) ? 0 : (d < cum1 ? 1 : 2);
    const float inv = rope.inv_freq[d];
    float sn, cs;
    sincosf((float)pos[sec] * inv, &sn, &cs);
    const bf16_t* src = (h < Hq) ? q_src + (size_t)h * hd : k_src + (size_t)(h - Hq) * hd;
    const float x0 = bf16_to_f32(src[d]);
    const float x1 = bf16_to_f32(src[d + half]);
    const bf16_t y0 = (bf16_t)f32_to_bf16(x0 * cs - x1 * sn);
    const bf16_t y1 = (bf16_t)f32_to_bf16(x1 * cs + x0 * sn);
    if (h < Hq) {
        q_dst[(size_t)h * hd + d] = y0;
        q_dst[(size_t)h * hd + d + half] = y1;
    } else if (L > 0) {
        const int hk = h - Hq;
        k_cache[slot * kvd + hk * hd + d] = y0;
        k_cache[slot * kvd + hk * hd + d + half] = y1;
    }
}

// Prefill: rotate the S new tokens' queries in place in the fused QKV buffer, rotate their
// keys into the K cache rows and copy their values into the V cache rows, in one pass.
// One workgroup per token: the cos / sin of the token's hd/2 angles are computed once
// (sincosf, as mrope_kernel) into LDS and shared by every head; each thread then rotates
// 4 consecutive pairs (d .. d+3 with d+half .. d+half+3) of one head with 8-byte loads.
struct RopeWriteArgs {
    bf16_t* qkv;            // [S, qkv_sn]: q at 0, k at Hq*hd, v at (Hq+Hkv)*hd
    bf16_t* k_dst;          // [S, kv_sn] cache rows of this prefill
    bf16_t* v_dst;
    const int32_t* pos;     // [3, pos_stride] M-RoPE, or NULL: pos_offset + token
    int pos_stride, pos_offset;
    int S, Hq, Hkv, hd, qkv_sn, kv_sn, cum0, cum1;
    RopeTable rope;
};

__global__ __launch_bounds__(256) void rope_write_kv_kernel(RopeWriteArgs a) {
    __shared__ float2 cs[kMaxHalfDim];
    const int t = blockIdx.x;
    const int half = a.hd / 2;
    for (int d = threadIdx.x; d < half; d += blockDim.x) {
        const int sec = (d < a.cum0) ? 0 : (d < a.cum1 ? 1 : 2);
        const int p = (a.pos != nullptr) ? a.pos[sec * a.pos_stride + t] : a.pos_offset + t;
        float sn, c;
        sincosf((float)p * a.rope.inv_freq[d], &sn, &c);
        cs[d] = make_float2(c, sn);
    }
    __syncthreads();
    bf16_t* row = a.qkv + (size_t)t * a.qkv_sn;
    const int qd = a.Hq * a.hd, kvd = a.Hkv * a.hd;
    const int quads = half / 4;   // 4-pair groups per head
    // rotated heads: q (in place) and k (into the cache)
    for (int i = threadIdx.x; i < (a.Hq + a.Hkv) * quads; i += blockDim.x) {
        const int h = i / quads, d = (i % quads) * 4;
        const bf16_t* src = row + h * a.hd;   // k heads follow the q heads in the row
        bf16_t* dst = (h < a.Hq) ? row + h * a.hd : a.k_dst + (size_t)t * a.kv_sn + (h - a.Hq) * a.hd;
        const uint2 lo = *reinterpret_cast<const uint2*>(src + d);
        const uint2 hi = *reinterpret_cast<const uint2*>(src + d + half);
        const uint32_t lw[2] = {lo.x, lo.y}, hw[2] = {hi.x, hi.y};
        uint32_t ol[2], oh[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float2 c0 = cs[d + 2 * e], c1 = cs[d + 2 * e + 1];
            const float x0a = bf16_to_f32(lw[e] & 0xffffu), x0b = bf16_to_f32(lw[e] >> 16);
            const float x1a = bf16_to_f32(hw[e] & 0xffffu), x1b = bf16_to_f32(hw[e] >> 16);
            ol[e] = f32_to_bf16(x0a * c0.x - x1a * c0.y) | (f32_to_bf16(x0b * c1.x - x1b * c1.y) << 16);
            oh[e] = f32_to_bf16(x1a * c0.x + x0a * c0.y) | (f32_to_bf16(x1b * c1.x + x0b * c1.y) << 16);
        }
        *reinterpret_cast<uint2*>(dst + d) = make_uint2(ol[0], ol[1]);
        *reinterpret_cast<uint2*>(dst + d + half) = make_uint2(oh[0], oh[1]);
    }
    // values: plain copy into the cache, 16 bytes per thread
    const uint4* vs = reinterpret_cast<const uint4*>(row + qd + kvd);
    uint4* vd = reinterpret_cast<uint4*>(a.v_dst + (size_t)t * a.kv_sn);
    for (int i = threadIdx.x; i < kvd / 8; i += blockDim.x) vd[i] = vs[i];
}

static int mrope_check_sections(int hd, int s0, int s1, int s2) {
    if (s0 < 0 || s1 < 0 || s2 < 0 || s0 + s1 + s2 != hd / 2)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "mrope: sections %d+%d+%d must sum to head_dim/2 = %d", s0, s1, s2,
                         hd / 2);
    return EFM_OK;
}

}  // namespace efm

extern "C" int efm_mrope(void* q, void* k, const int32_t* position_ids, int32_t position_stride, int32_t seq_len,
                         int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t q_stride_n,
                         int32_t k_stride_n, int32_t section0, int32_t section1, int32_t section2, float rope_theta,
                         float rope_scale, hipStream_t stream) {
    if (!q || !k || !position_ids) return set_error(EFM_ERR_INVALID_ARGUMENT, "mrope: null pointer");
    if (head_dim <= 0 || head_dim % 2 || head_dim > 2 * kMaxHalfDim) return set_error(EFM_ERR_UNSUPPORTED, "mrope: head_dim");
    int rc = mrope_check_sections(head_dim, section0, section1, section2);
    if (rc) return rc;
    if (seq_len < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || position_stride < seq_len)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "mrope: bad sizes");
    if (seq_len == 0) return EFM_OK;
    MropeArgs a;
    a.q = static_cast<bf16_t*>(q);
    a.k = static_cast<bf16_t*>(k);
    a.pos = position_ids;
    a.pos_stride = position_stride;
    a.pos_offset = 0;
    a.S = seq_len;
    a.Hq = num_qo_heads;
    a.Hkv = num_kv_heads;
    a.hd = head_dim;
    a.q_sn = q_stride_n ? q_stride_n : num_qo_heads * head_dim;
    a.k_sn = k_stride_n ? k_stride_n : num_kv_heads * head_dim;
    a.cum0 = section0;
    a.cum1 = section0 + section1;
    rope_table_fill(&a.rope, head_dim, rope_theta, rope_scale);
    hipLaunchKernelGGL(mrope_kernel, dim3(seq_len, num_qo_heads + num_kv_heads), dim3(((head_dim / 2) + 63) / 64 * 64),
                       0, stream, a);
    return check_launch("mrope");
}

extern "C" int efm_rope_llama_inplace(void* q, void* k, int32_t seq_len, int32_t num_qo_heads, int32_t num_kv_heads,
                                      int32_t head_dim, int32_t q_stride_n, int32_t k_stride_n, int32_t pos_offset,
                                      float rope_theta, float rope_scale, hipStream_t stream) {
    if (!q || !k) return set_error(EFM_ERR_INVALID_ARGUMENT, "rope_llama_inplace: null pointer");
    if (head_dim <= 0 || head_dim % 2 || head_dim > 2 * kMaxHalfDim)
        return set_error(EFM_ERR_UNSUPPORTED, "rope_llama_inplace: head_dim");
    if (seq_len < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || pos_offset < 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "rope_llama_inplace: bad sizes");
    if (seq_len == 0) return EFM_OK;
    MropeArgs a;
    a.q = static_cast<bf16_t*>(q);
    a.k = static_cast<bf16_t*>(k);
    a.pos = nullptr;
    a.pos_stride = 0;
    a.pos_offset = pos_offset;
    a.S = seq_len;
    a.Hq = num_qo_heads;
    a.Hkv = num_kv_heads;
    a.hd = head_dim;
    a.q_sn = q_stride_n ? q_stride_n : num_qo_heads * head_dim;
    a.k_sn = k_stride_n ? k_stride_n : num_kv_heads * head_dim;
    a.cum0 = head_dim / 2;
    a.cum1 = head_dim / 2;
    rope_table_fill(&a.rope, head_dim, rope_theta, rope_scale);
    hipLaunchKernelGGL(mrope_kernel, dim3(seq_len, num_qo_heads + num_kv_heads), dim3(((head_dim / 2) + 63) / 64 * 64),
                       0, stream, a);
    return check_launch("rope_llama_inplace");
}

extern "C" int efm_prefill_rope_write_kv(void* qkv, int32_t qkv_stride_n, void* k_dst, void* v_dst,
                                         int32_t kv_stride_n, int32_t seq_len, int32_t num_qo_heads,
                                         int32_t num_kv_heads, int32_t head_dim, const int32_t* position_ids,
                                         int32_t position_stride, int32_t pos_offset, int32_t section0,
                                         int32_t section1, int32_t section2, float rope_theta, float rope_scale,
                                         hipStream_t stream) {
    if (!qkv || !k_dst || !v_dst) return set_error(EFM_ERR_INVALID_ARGUMENT, "prefill_rope_write_kv: null pointer");
    if (head_dim <= 0 || head_dim % 8 || head_dim > 2 * kMaxHalfDim)
        return set_error(EFM_ERR_UNSUPPORTED, "prefill_rope_write_kv: head_dim %d (multiple of 8, <= %d)", head_dim,
                         2 * kMaxHalfDim);
    if (seq_len < 0 || num_qo_heads <= 0 || num_kv_heads <= 0 || pos_offset < 0)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "prefill_rope_write_kv: bad sizes");
    const int kvd = num_kv_heads * head_dim, tot = num_qo_heads * head_dim + 2 * kvd;
    const int qsn = qkv_stride_n ? qkv_stride_n : tot, ksn = kv_stride_n ? kv_stride_n : kvd;
    if (qsn < tot || ksn < kvd || qsn % 8 || ksn % 8 ||
        ((reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(k_dst) | reinterpret_cast<uintptr_t>(v_dst)) &
         15u))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "prefill_rope_write_kv: strides / alignment");
    if (position_ids != nullptr) {
        int rc = mrope_check_sections(head_dim, section0, section1, section2);
        if (rc) return rc;
        if (position_stride < seq_len)
            return set_error(EFM_ERR_INVALID_ARGUMENT, "prefill_rope_write_kv: position_stride < seq_len");
    }
    if (seq_len == 0) return EFM_OK;
    RopeWriteArgs a;
    a.qkv = static_cast<bf16_t*>(qkv);
    a.k_dst = static_cast<bf16_t*>(k_dst);
    a.v_dst = static_cast<bf16_t*>(v_dst);
    a.pos = position_ids;
    a.pos_stride = position_stride;
    a.pos_offset = pos_offset;
    a.S = seq_len;
    a.Hq = num_qo_heads;
    a.Hkv = num_kv_heads;
    a.hd = head_dim;
    a.qkv_sn = qsn;
    a.kv_sn = ksn;
    a.cum0 = position_ids ? section0 : head_dim / 2;
    a.cum1 = position_ids ? section0 + section1 : head_dim / 2;
    rope_table_fill(&a.rope, head_dim, rope_theta, rope_scale);
    hipLaunchKernelGGL(rope_write_kv_kernel, dim3(seq_len), dim3(256), 0, stream, a);
    return check_launch("prefill_rope_write_kv");
}

extern "C" int efm_decode_mrope_write_kv(const void* q_src, const void* k_src, const void* v_src, void* q_dst,
                                         void* k_cache, void* v_cache, int32_t num_qo_heads, int32_t num_kv_heads,
                                         int32_t head_dim, const int32_t* position_ids, int32_t section0,
                                         int32_t section1, int32_t section2, float rope_theta, float rope_scale,
                                         const uint32_t* d_kv_len, hipStream_t stream) {
    if (!q_src || !k_src || !v_src || !q_dst || !k_cache || !v_cache || !position_ids || !d_kv_len)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_mrope_write_kv: null pointer");
    if (head_dim <= 0 || head_dim % 2 || head_dim > 2 * kMaxHalfDim)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_mrope_write_kv: head_dim");
    int rc = mrope_check_sections(head_dim, section0, section1, section2);
    if (rc) return rc;
    RopeTable rope;
    rope_table_fill(&rope, head_dim, rope_theta, rope_scale);
    hipLaunchKernelGGL(decode_mrope_write_kv_kernel, dim3(1, num_qo_heads + 2 * num_kv_heads),
                       dim3(((head_dim / 2) + 63) / 64 * 64), 0, stream, static_cast<const bf16_t*>(q_src),
                       static_cast<const bf16_t*>(k_src), static_cast<const bf16_t*>(v_src),
                       static_cast<bf16_t*>(q_dst), static_cast<bf16_t*>(k_cache), static_cast<bf16_t*>(v_cache),
                       num_qo_heads, num_kv_heads, head_dim, position_ids, section0, section0 + section1, rope,
                       d_kv_len);
    return check_launch("decode_mrope_write_kv");
}

// Device-side response write for graph-replayed decode: response[*step] = sampled[0],
// *step += 1, *d_kv_len += 1 (replaces finalize_decode_token_kernel plus the per-step
// retargeting of the response pointer in the captured graph, standard_engine.h:33-65).
__global__ void finalize_indexed_kernel(const int32_t* sampled, int32_t* response, uint32_t* step,
                                        uint32_t* d_kv_len, uint32_t capacity) {
    if (threadIdx.x == 0) {
        const uint32_t s = step[0];
        if (s < capacity) response[s] = sampled[0];
        step[0] = s + 1u;
        if (d_kv_len != nullptr) d_kv_len[0] += 1u;
    }
}

extern "C" int efm_finalize_decode_token_indexed(const int32_t* sampled_token, int32_t* response_base,
                                                 uint32_t* d_step, uint32_t* d_kv_len, uint32_t capacity,
                                                 hipStream_t stream) {
    if (!sampled_token || !response_base || !d_step)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "finalize_decode_token_indexed: null pointer");
    hipLaunchKernelGGL(finalize_indexed_kernel, dim3(1), dim3(kWave), 0, stream, sampled_token, response_base, d_step,
                       d_kv_len, capacity);
    return check_launch("finalize_decode_token_indexed");
}

// dst[*d_index] <- src (row_bytes bytes) when *d_index < max_rows: a per-step copy whose
// destination row is read on the device, so one captured decode graph stores every step.
__global__ __launch_bounds__(256) void store_row_indexed_kernel(const uint4* src, uint4* dst, int64_t n16,
                                                                const uint32_t* d_index, uint32_t max_rows) {
    const uint32_t r = d_index[0];
    if (r >= max_rows) return;
    uint4* d = dst + (size_t)r * (size_t)n16;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256ll) d[i] = src[i];
}

extern "C" int efm_store_row_indexed(const void* src, void* dst, int64_t row_bytes, const uint32_t* d_index,
                                     uint32_t max_rows, hipStream_t stream) {
    if (!src || !dst || !d_index) return set_error(EFM_ERR_INVALID_ARGUMENT, "store_row_indexed: null pointer");
    if (row_bytes <= 0 || row_bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "store_row_indexed: rows must be 16-byte multiples, 16-byte aligned");
    const int64_t n16 = row_bytes / 16;
    const int grid = (int)std::min<int64_t>(1024, (n16 + 255) / 256);
    hipLaunchKernelGGL(store_row_indexed_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const uint4*>(src),
                       static_cast<uint4*>(dst), n16, d_index, max_rows);
    return check_launch("store_row_indexed");
}

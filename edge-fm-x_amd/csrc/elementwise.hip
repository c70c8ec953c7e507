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
    const float tot = block_sum<kRowThreads>(ss, red);
    const float inv = 1.0f / sqrtf(tot / (float)hidden + eps);
    const uint4* w4 = reinterpret_cast<const uint4*>(w);
    uint4* o4 = reinterpret_cast<uint4*>(out + row * hidden);
#pragma unroll
    for (int i = 0; i < kRowMaxChunks; ++i) {
        const int c = threadIdx.x + i * kRowThreads;
        if (c < C) {
            float wf[8], o[8];
            unpack8(w4[c], wf);
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
        for (int e = 0; e < 8; ++e) o[e] = (g[e] / (1.0f + expf(-g[e]))) * u[e];
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

/*
 * edgefm_hip.h — C ABI of the MI355X (gfx950) kernels behind EdgeFM's operator layer.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t, launches
 * asynchronously on that stream, never synchronises, never allocates device memory
 * (scratch comes in through explicit workspace arguments) and is therefore safe to
 * record into a HIP graph. Activations and weights are bf16 (raw 16-bit patterns),
 * accumulation is fp32. Return value: EFM_OK or an EFM_ERR_* code; the message of the
 * most recent failure on the calling thread is available from efm_last_error().
 *
 * Each declaration names the reference interface it replaces (file:line in the
 * EdgeFM sources). The C++ operator adapters in edge-fm-x_amd/host map the status
 * codes onto EdgeFM's exception types (ConfigurationError, InvalidRequestError,
 * DeviceError).
 */
#ifndef EDGEFM_HIP_H_
#define EDGEFM_HIP_H_

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define EFM_OK 0
#define EFM_ERR_INVALID_ARGUMENT 1 /* bad shape/pointer -> InvalidRequestError      */
#define EFM_ERR_UNSUPPORTED 2      /* config outside the kernel -> ConfigurationError */
#define EFM_ERR_DEVICE 3           /* HIP runtime failure -> DeviceError              */
#define EFM_ERR_WORKSPACE 4        /* workspace missing or too small                 */

/* DType ordinals, identical to edge_fm::DType (include/edge-fm/core.h:17-25). */
#define EFM_DTYPE_F32 0
#define EFM_DTYPE_F16 1
#define EFM_DTYPE_BF16 2
#define EFM_DTYPE_I32 3

/* Positional encoding applied inside attention (src/operators/attention_op.h:15-18). */
#define EFM_POS_NONE 0
#define EFM_POS_ROPE_LLAMA 1

/* Activation input layouts (src/operators/activation_op.h:18-21). */
#define EFM_LAYOUT_GATE_UP 0
#define EFM_LAYOUT_UP_GATE 1

/* Message of the last failed call on this thread ("" if none). */
const char* efm_last_error(void);

/* Library version string. */
const char* efm_version(void);

/* Per-device set-up of the current device (no counterpart in the reference, which sets
 * its buffers up inside its engine): looks up the device address of the library-held
 * array that efm_attention_decode_noalloc uses. Call it once per device, with that device
 * current, before capturing efm_attention_decode_noalloc into a graph; outside capture
 * the entry point's first call does the same by itself. Allocates nothing. */
int efm_init(void);

/* Test hook (no counterpart in the reference): process-wide choice between kernels that
 * compute the same operator, so that tests can compare a fast kernel with the simpler
 * one it replaces on the same inputs. value 0 restores the library's own choice.
 *   EFM_KNOB_DECODE_REGISTER   1: decode attention (head_dim 128, rotated cache) runs the
 *                              register-staged kernel instead of the LDS-staged one
 *   EFM_KNOB_PREFILL_REGISTER  1: prefill and Sage attention (head_dim 128) run the
 *                              register-staged kernels instead of the pipelined ones
 *   EFM_KNOB_PREFILL_SHAPE     4 or 8: the pipelined prefill / Sage kernels run with
 *                              4-wave (128-row) or 8-wave (256-row) workgroups; 2: the
 *                              prefill kernel runs 2-wave (64-row) workgroups (the Sage
 *                              kernel treats 2 as 4)
 *   EFM_KNOB_GEMM_TILE         prefill GEMM kernel (K % 64 == 0): 1 the two-workgroup-
 *                              per-CU 128 x 128 / 128 x 64 / 64 x 64 kernel, 2 the
 *                              one-workgroup-per-CU 256 x 256 kernel, 3 the same kernel
 *                              with 192 x 256 tiles
 *   EFM_KNOB_FRONT_WAIT_TIMEOUT 1: efm_decode_norm_qkv_attention launches whose attention
 *                              workgroups wait for a tag that no projected word carries,
 *                              with a 64-poll limit: every wait gives up, the launch
 *                              drains with wrong outputs and the time-out is reported by
 *                              efm_decode_qkv_attention_status (tests of that path)
 *   EFM_KNOB_DECODE_TILE       1: efm_attention_decode leaves the one-wave split kernel
 *                              of short and mid contexts aside and runs the 4-wave /
 *                              8-wave / register kernels those lengths had before it
 * Unknown knobs or values: EFM_ERR_INVALID_ARGUMENT. Not for production callers. */
#define EFM_KNOB_DECODE_REGISTER 0
#define EFM_KNOB_PREFILL_REGISTER 1
#define EFM_KNOB_PREFILL_SHAPE 2
#define EFM_KNOB_GEMM_TILE 3
#define EFM_KNOB_FRONT_WAIT_TIMEOUT 4
#define EFM_KNOB_DECODE_TILE 5
#define EFM_KNOB_COUNT 6
int efm_testing_set_kernel_path(int32_t knob, int32_t value);

/* ------------------------------------------------------------------------------------
 * Attention.  Mirrors edge_fm::AttentionOpContext (src/operators/attention_op.h:20-39).
 * Strides are in elements; 0 means contiguous ([n, heads, head_dim] NHD layout).
 * ---------------------------------------------------------------------------------- */
typedef struct efm_attention_ctx {
    uint32_t num_qo_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t q_stride_n;
    uint32_t q_stride_h;
    uint32_t k_stride_n;
    uint32_t k_stride_h;
    uint32_t kv_stride_n; /* V strides (the reference's kv_stride_*) */
    uint32_t kv_stride_h;
    float rope_scale;
    float rope_theta;
    uint32_t q_rope_pos_offset;
    uint32_t k_rope_pos_offset;
    int32_t dtype;        /* EFM_DTYPE_BF16 only */
    int32_t pos_encoding; /* EFM_POS_NONE | EFM_POS_ROPE_LLAMA */
    int32_t k_already_prerotated; /* 0, 1, or EFM_K_PREROTATED_EXCEPT_NEWEST (decode only) */
} efm_attention_ctx;

/* k_already_prerotated value for the decode entry points (no counterpart in the
 * reference, which rotates every key on read): cache rows [0, L-1) hold keys already
 * rotated at their positions; row L-1 (this step's key, written un-rotated by the QKV
 * projection) is rotated by the call at L-1 + k_rope_pos_offset, used, and stored back
 * rotated. Running the same call twice on one cache state is therefore not idempotent. */
#define EFM_K_PREROTATED_EXCEPT_NEWEST 2

/* Bytes of workspace efm_attention_decode needs for caches of up to max_kv_len rows. */
size_t efm_attention_decode_workspace_bytes(const efm_attention_ctx* ctx, uint32_t max_kv_len);

/* Single-query GQA decode attention, split-KV with an in-kernel log-sum-exp merge.
 * q [1, Hq, hd]; k, v [>= kv rows, Hkv, hd]; o [1, Hq, hd].
 * The number of attended rows is *d_kv_len when d_kv_len != NULL (device-resident,
 * graph-stable; then max_kv_len bounds it and k, v must hold max_kv_len rows, which the
 * kernel may read before *d_kv_len is known), else kv_len. With EFM_POS_ROPE_LLAMA, q is
 * rotated at position (L - 1 + q_rope_pos_offset) and key j at (j + k_rope_pos_offset)
 * on read; the cache holds un-rotated K. sm_scale = 1/sqrt(hd).
 * Replaces AttentionOp::forward_decode (src/operators/attention_op.h:53-61,
 * FlashInferAttentionOp::forward_decode, src/operators/attention_op.cu:1565-1604). */
int efm_attention_decode(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v,
                         void* o, uint32_t kv_len, const uint32_t* d_kv_len, uint32_t max_kv_len,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

/* efm_attention_decode without a workspace argument. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments, semantics and kernels
 * as efm_attention_decode, and the same results bit for bit. The split partials live in
 * a device array the library holds on every GPU it runs on until the process ends, of
 * EFM_ATTENTION_DECODE_NOALLOC_SCRATCH_BYTES; that covers every shape whose
 * efm_attention_decode_workspace_bytes fits in it (all head_dim <= 128, group <= 8 shapes
 * with up to 512 KV heads, any length). Larger needs: EFM_ERR_UNSUPPORTED, nothing
 * launched. The call allocates nothing. The array's device address is looked up once per
 * device, by efm_init or by the first call there; a first call made while its stream is
 * being captured into a graph is refused (EFM_ERR_INVALID_ARGUMENT: call efm_init before
 * capturing). Every call on one GPU shares the array: calls that overlap on one GPU (on
 * different streams, or from several threads without stream order) race. */
#define EFM_ATTENTION_DECODE_NOALLOC_SCRATCH_BYTES 2359296
int efm_attention_decode_noalloc(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v,
                                 void* o, uint32_t kv_len, const uint32_t* d_kv_len, uint32_t max_kv_len,
                                 hipStream_t stream);

/* Decode attention split partials only (no in-kernel merge): every split writes its
 * unnormalised fp32 output and (max, sum) of exp2-domain scores into `workspace`
 * (efm_attention_decode_workspace_bytes(ctx, max_kv_len) bytes); the partials are
 * consumed by efm_decode_attention_merge_o_proj. Same semantics and length handling
 * as efm_attention_decode with d_kv_len (required). Part of the split of
 * AttentionOp::forward_decode + the o_proj LinearImpl::forward
 * (src/models/qwen2_5/qwen2_5.cpp:831-847) into two launches with the merge folded
 * into the projection. */
int efm_decode_attention_partials(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v,
                                  const uint32_t* d_kv_len, uint32_t max_kv_len, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream);

/* o_proj over the merged attention output: out[hidden] = bf16(merge(partials)) . W_o^T,
 * where merge is the log-sum-exp combination of the splits written by
 * efm_decode_attention_partials with the same ctx, d_kv_len, max_kv_len and workspace;
 * the merged vector is rounded to bf16 before the projection, as the unfused
 * attention output would be. Supports the split plans that
 * efm_decode_attention_merge_o_proj_supported accepts: up to 24 splits for query widths
 * up to 1024 and up to 12 for widths up to 2048 (splits of 32 or 64 keys where those fit,
 * else of 128: e.g. head_dim 128 caches up to 1536 rows). Replaces the o_proj
 * LinearImpl::forward (role attention_output, src/layers/linear.cu:41-58). */
int efm_decode_attention_merge_o_proj(const efm_attention_ctx* ctx, const uint32_t* d_kv_len, uint32_t max_kv_len,
                                      const void* workspace, size_t workspace_bytes, const void* w_o, int32_t hidden,
                                      void* out, hipStream_t stream);

/* EFM_OK when efm_decode_attention_merge_o_proj takes the partials that
 * efm_decode_attention_partials writes for (ctx, max_kv_len); otherwise the error code it
 * would return (callers then use efm_attention_decode and efm_linear). Host-side only.
 * Part of the same split of the reference's attention + o_proj pair
 * (src/models/qwen2_5/qwen2_5.cpp:831-847). */
int efm_decode_attention_merge_o_proj_supported(const efm_attention_ctx* ctx, uint32_t max_kv_len);

/* Causal / non-causal GQA prefill attention on the matrix cores. q [qo_len, Hq, hd]
 * (q_stride_* may point into a fused QKV buffer), k, v [kv_len, Hkv, hd] with
 * kv_len >= qo_len; o [qo_len, Hq * hd] contiguous. Query i has RoPE position
 * i + q_rope_pos_offset and, when causal, sees keys j <= i + (kv_len - qo_len); key j is
 * rotated at j + k_rope_pos_offset unless k_already_prerotated. fp32 online softmax,
 * P rounded to bf16 for the PV product, sm_scale = 1/sqrt(hd).
 * Replaces AttentionOp::forward_prefill (src/operators/attention_op.h:45-52,
 * forward_prefill_impl, src/operators/attention_op.cu:1345-1426). */
int efm_attention_prefill(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v, void* o,
                          uint32_t qo_len, uint32_t kv_len, int32_t causal, hipStream_t stream);

/* SageAttention-style prefill attention (named but not implemented by
 * the reference, README.md:23). K is smoothed by its per-(KV head, channel) mean over
 * tokens (float64 sum, rounded to fp32); Q and the smoothed K are quantised to int8 per
 * (128-token block, head) with scale = max|x| / 127 (1 for an all-zero block) and
 * round-half-even; QK^T runs on the int8 matrix cores with exact int32 accumulation,
 * score_log2 = float(acc) * ((sq * sk) * (log2(e) / sqrt(hd))); fp32 online softmax;
 * P (bf16) . V with fp32 accumulation. Layouts as efm_attention_prefill; pos_encoding
 * must be EFM_POS_NONE (rotate before quantising). workspace: see the size query. */
size_t efm_attention_prefill_sage_int8_workspace_bytes(const efm_attention_ctx* ctx, uint32_t qo_len,
                                                       uint32_t kv_len);
int efm_attention_prefill_sage_int8(const efm_attention_ctx* ctx, const void* q, const void* k, const void* v,
                                    void* o, uint32_t qo_len, uint32_t kv_len, int32_t causal, void* workspace,
                                    size_t workspace_bytes, hipStream_t stream);
/* The quantisation step alone (exposed so the integer path can be checked bit-exactly):
 * q8 [qo_len, Hq, hd] int8, q_scales [ceil(qo_len/128), Hq], k8 [kv_len, Hkv, hd] int8,
 * k_scales [ceil(kv_len/128), Hkv], k_mean [Hkv, hd]. */
int efm_sage_quantize(const efm_attention_ctx* ctx, const void* q, const void* k, uint32_t qo_len, uint32_t kv_len,
                      int8_t* q8, float* q_scales, int8_t* k8, float* k_scales, float* k_mean, hipStream_t stream);

/* M-RoPE in place (src/layers/attention.cu:17-118, AttentionLayer::apply_mrope).
 * q [seq_len, Hq, hd] and k [seq_len, Hkv, hd] with token strides q_stride_n /
 * k_stride_n (0 = contiguous); position_ids [3, position_stride] int32 (rows t, h, w);
 * sections (e.g. 16, 24, 24) sum to hd/2. Pair d uses the position row of its section. */
int efm_mrope(void* q, void* k, const int32_t* position_ids, int32_t position_stride, int32_t seq_len,
              int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim, int32_t q_stride_n, int32_t k_stride_n,
              int32_t section0, int32_t section1, int32_t section2, float rope_theta, float rope_scale,
              hipStream_t stream);

/* Rotate-half RoPE in place (the ROPE_LLAMA rotation that the reference applies inside
 * attention, src/operators/attention_op.cu:1345-1426, moved to the cache write so that
 * the cache holds rotated keys): token t of q [seq_len, Hq, hd] and k [seq_len, Hkv, hd]
 * (token strides q_stride_n / k_stride_n, 0 = contiguous) is rotated at position
 * pos_offset + t; pair (d, d + hd/2) by angle pos * theta^(-2d/hd) / rope_scale. */
int efm_rope_llama_inplace(void* q, void* k, int32_t seq_len, int32_t num_qo_heads, int32_t num_kv_heads,
                           int32_t head_dim, int32_t q_stride_n, int32_t k_stride_n, int32_t pos_offset,
                           float rope_theta, float rope_scale, hipStream_t stream);

/* ------------------------------------------------------------------------------------
 * RMSNorm (src/operators/norm_op.h:14-55, FlashInfer norm::RMSNorm / FusedAddRMSNorm
 * called at src/operators/norm_op.cu:33-90).
 * ---------------------------------------------------------------------------------- */
/* out[b,:] = bf16(in * rsqrt(mean(in^2) + eps) * w). */
int efm_rms_norm(uint32_t batch, uint32_t hidden, float eps, const void* input, const void* weight,
                 void* output, hipStream_t stream);

/* s = inout + residual (fp32); residual <- bf16(s); inout <- bf16(s * rsqrt(mean(s^2)+eps) * w). */
int efm_fused_add_rms_norm(uint32_t batch, uint32_t hidden, float eps, void* inout, void* residual,
                           const void* weight, hipStream_t stream);

/* ------------------------------------------------------------------------------------
 * SiLU-and-mul (src/operators/activation_op.h:23-42, act_and_mul_kernel_layout at
 * src/operators/activation_op.cu:36-76). input [batch, 2*hidden] in the given layout,
 * out[b, i] = bf16(silu(gate) * up), silu(x) = x / (1 + exp(-x)).
 * ---------------------------------------------------------------------------------- */
int efm_act_and_mul(int64_t batch, int64_t hidden, int32_t layout, const void* input, void* output,
                    hipStream_t stream);

/* ------------------------------------------------------------------------------------
 * Linear: y[m, out] = x[m, in] . W[out, in]^T (+ bias[out]), fp32 accumulate,
 * output bf16 (EFM_DTYPE_BF16) or fp32 (EFM_DTYPE_F32, the LM-head logits).
 * m == 1 runs the bandwidth-bound GEMV; m > 1 this library's bf16 MFMA GEMM kernels.
 * Replaces LinearLayer::LinearImpl::forward (src/layers/linear.h:131-153) backed by
 * LinearCublasLtImpl (src/operators/linear_impl.cu:315-480).
 * ---------------------------------------------------------------------------------- */
int efm_linear(int64_t m, int64_t in_features, int64_t out_features, const void* x, const void* w,
               const void* bias, void* y, int32_t out_dtype, hipStream_t stream);

/* efm_linear with a caller workspace (the scratch the reference's linear impls take from
 * StaticBufferManager, src/utils/memory.h:31-109). Shapes whose output tiles are too few
 * to fill the chip and whose K is long (prefill down_proj at a few hundred to a few
 * thousand tokens) split K into slices that write fp32 partial sums into the workspace,
 * then reduce them in slice order. efm_linear_workspace_bytes returns the bytes the
 * shape uses (0: none); the split runs only when workspace_bytes >= that figure, and
 * with less workspace the call runs as efm_linear does. The plan depends on the shape
 * alone, so a shape given its figure always runs the same kernels. The split sums K in
 * a different order than efm_linear, so the two agree to fp32 rounding, not bit for
 * bit; each is deterministic. */
size_t efm_linear_workspace_bytes(int64_t m, int64_t in_features, int64_t out_features);
int efm_linear_ws(int64_t m, int64_t in_features, int64_t out_features, const void* x, const void* w,
                  const void* bias, void* y, int32_t out_dtype, void* workspace, size_t workspace_bytes,
                  hipStream_t stream);

/* Fused gate/up projection + SwiGLU: W is the fused [up; gate] matrix [2*inter, hidden]
 * (src/layers/linear.cu:1923-1943); out[m, i] = bf16(silu(bf16(g_i)) * bf16(u_i)).
 * Replaces FusedGateUpActivationOp::run / TrtLlmDecodeSwigluOp
 * (src/operators/fused_gate_up_activation_op.h:14-61, .cu:675-782) and the two-stage
 * gate_up GEMM + act_and_mul fallback (src/layers/gated_mlp.cu:19-67). */
int efm_fused_gate_up_swiglu(int64_t m, int64_t hidden, int64_t inter, const void* x,
                             const void* w_up_gate, void* out, hipStream_t stream);

/* The same with a caller workspace (efm_fused_gate_up_swiglu_workspace_bytes; 0 means
 * none is used). The SwiGLU is the epilogue of the MFMA kernel, so no shape needs a
 * workspace today and the call is efm_fused_gate_up_swiglu; the entry point keeps the
 * signature of the reference's workspace-taking fused op (fused_gate_up_activation_op.h:
 * 14-61) for callers that pass one. */
size_t efm_fused_gate_up_swiglu_workspace_bytes(int64_t m, int64_t hidden, int64_t inter);
int efm_fused_gate_up_swiglu_ws(int64_t m, int64_t hidden, int64_t inter, const void* x,
                                const void* w_up_gate, void* out, void* workspace, size_t workspace_bytes,
                                hipStream_t stream);

/* ------------------------------------------------------------------------------------
 * LM head with fused greedy top-1 (src/layers/linear.cu:140-276, 2288-2369):
 * token_out[0] = argmax_v (x . W[v,:]) with ties to the lowest id (a NaN score never
 * wins). workspace: efm_lm_head_top1_workspace_bytes(vocab) bytes, zero-filled before its
 * first use; every launch leaves it zeroed again, so it is reused as is (launches that
 * share it must be stream-ordered).
 * ---------------------------------------------------------------------------------- */
size_t efm_lm_head_top1_workspace_bytes(int64_t vocab);
int efm_lm_head_top1(int64_t hidden, int64_t vocab, const void* x, const void* w, int32_t* token_out,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------------------
 * Greedy sampler (src/layers/sampler.cu:146-249): out[r] = argmax(logits[r, :]),
 * ties to the lowest index. logits fp32 [rows, vocab].
 * ---------------------------------------------------------------------------------- */
size_t efm_sampler_greedy_workspace_bytes(int64_t rows, int64_t vocab);
int efm_sampler_greedy(int64_t rows, int64_t vocab, const float* logits, int32_t* out, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);


/* ------------------------------------------------------------------------------------
 * Temperature / top-p sampler of one fp32 logits row (the non-greedy branch of
 * SamplerLayer::forward_sampling, src/layers/sampler.cu:251-298, which samples
 * softmax(logits / T) by inverse CDF; top-p is an addition). Exact integer-mass
 * definition: e_i = expf((l_i - max l) / T), w_i = rint(e_i * 2^44); nucleus = all ids
 * when top_p >= 1, else the ids with e_i >= tau, tau the largest value whose upper set
 * holds >= ceil(top_p * sum w) of the mass; the 24-bit draw x = Philox4x32-10(counter =
 * offset (+ *d_offset when d_offset is not NULL), key = seed).x >> 8 picks the smallest
 * nucleus id whose prefix mass exceeds floor(N * x / 2^24).
 * temperature >= 1e-6 (smaller means greedy: use efm_sampler_greedy), top_p > 0,
 * 1 <= vocab < 2^20. workspace: efm_sampler_top_p_workspace_bytes(vocab) bytes of
 * device memory, no initial contents required; calls that share a workspace must be
 * ordered on one stream. 3 launches when top_p >= 1, 6 otherwise.
 * ---------------------------------------------------------------------------------- */
size_t efm_sampler_top_p_workspace_bytes(int64_t vocab);
int efm_sampler_top_p(int64_t vocab, const float* logits, float temperature, float top_p, uint64_t seed,
                      uint64_t offset, const int32_t* d_offset, int32_t* token_out, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------------------
 * Embedding lookup (src/layers/embed_head.cu:23-164). out[t,:] = table[ids[t],:];
 * ids in [embed_token_id, embed_token_id + n_custom) take custom_embeddings rows when
 * custom_embeddings != NULL and embed_token_id >= 0; ids outside the vocabulary give
 * zero rows.
 * ---------------------------------------------------------------------------------- */
int efm_embedding_lookup(int64_t n_tokens, int64_t hidden, int64_t vocab, const int32_t* ids,
                         const void* table, const void* custom_embeddings, int64_t n_custom,
                         int32_t embed_token_id, void* out, hipStream_t stream);

/* ------------------------------------------------------------------------------------
 * Decode runtime kernels (src/engine/tasks/token_generation/cuda/kernels/
 * decode_runtime_kernels.h:9-56).
 * ---------------------------------------------------------------------------------- */
/* Copy one K row and one V row into cache slot (*d_kv_len - 1); no-op when *d_kv_len == 0. */
int efm_copy_decode_kv_cache_slots(const void* k_src, const void* v_src, void* k_cache, void* v_cache,
                                   int32_t k_elems, int32_t v_elems, const uint32_t* d_kv_len,
                                   hipStream_t stream);
/* response_token[0] = sampled_token[0] (if both non-NULL); *d_kv_len += 1 (if non-NULL). */
int efm_finalize_decode_token(const int32_t* sampled_token, int32_t* response_token, uint32_t* d_kv_len,
                              hipStream_t stream);
/* values[0..2] += 1 (decode M-RoPE positions). */
int efm_increment_int32_triplet(int32_t* values, hipStream_t stream);
/* Prefill position encoding + KV write in one pass: rotate the S new tokens' queries in
 * place in the fused QKV buffer ([S, qkv_stride_n], q at column 0, k at Hq*hd, v at
 * (Hq+Hkv)*hd), write their rotated keys into k_dst rows and copy their values into
 * v_dst rows ([S, kv_stride_n], the cache rows [base, base + S)). position_ids NULL:
 * RoPE-Llama at position pos_offset + t (attention_op.cu:327-371, applied at the cache
 * write instead of inside attention); else M-RoPE with position rows [3, position_stride]
 * and sections (attention.cu:17-118). Replaces the two cudaMemcpy2DAsync of
 * qwen2_5.cpp:743-746 and the rotation of the prefill attention. head_dim % 8 == 0. */
int efm_prefill_rope_write_kv(void* qkv, int32_t qkv_stride_n, void* k_dst, void* v_dst, int32_t kv_stride_n,
                              int32_t seq_len, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                              const int32_t* position_ids, int32_t position_stride, int32_t pos_offset,
                              int32_t section0, int32_t section1, int32_t section2, float rope_theta,
                              float rope_scale, hipStream_t stream);

/* Decode M-RoPE on q (q_src -> q_dst) and k, then rotated K and raw V rows into cache slot
 * (*d_kv_len - 1); position_ids is the device [3] decode position
 * (launch_decode_mrope_apply_q_write_kv, decode_runtime_kernels.cu:152-225, 406-472). */
int efm_decode_mrope_write_kv(const void* q_src, const void* k_src, const void* v_src, void* q_dst, void* k_cache,
                              void* v_cache, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                              const int32_t* position_ids, int32_t section0, int32_t section1, int32_t section2,
                              float rope_theta, float rope_scale, const uint32_t* d_kv_len, hipStream_t stream);
/* response_base[*d_step] = sampled_token[0] (if *d_step < capacity); *d_step += 1;
 * *d_kv_len += 1. The device-side step index keeps one captured decode graph valid for
 * every step; it replaces finalize_decode_token_kernel plus the per-replay retargeting
 * of the response pointer (decode_runtime_kernels.cu:54-65, standard_engine.h:33-65). */
int efm_finalize_decode_token_indexed(const int32_t* sampled_token, int32_t* response_base, uint32_t* d_step,
                                      uint32_t* d_kv_len, uint32_t capacity, hipStream_t stream);

/* dst[*d_index * row_bytes ...] <- src[0 .. row_bytes) when *d_index < max_rows, else
 * nothing (device-side row index, so a captured decode graph stores each step's row).
 * row_bytes a multiple of 16, src / dst 16-byte aligned. The engine's per-step logits
 * record (runtime.debug_logits) uses it, in the role of the reference's debug bindings
 * that hand intermediate tensors to its tests (src/python/pybind_debug.cpp:486-1580). */
int efm_store_row_indexed(const void* src, void* dst, int64_t row_bytes, const uint32_t* d_index, uint32_t max_rows,
                          hipStream_t stream);

/* ------------------------------------------------------------------------------------
 * Fused decode-step kernels. Each one replaces a short sequence of the reference's
 * per-token operator calls inside Qwen2_5::forward_impl (src/models/qwen2_5/
 * qwen2_5.cpp:552-930) with a single launch; their results equal the unfused
 * sequence under the same rounding points.
 * ---------------------------------------------------------------------------------- */

/* Input norm + QKV projection + bias + KV-slot write (qwen2_5.cpp:564-597, 624-638).
 * If residual_in == NULL (layer 0): s = h; else s = h + residual_in (fp32).
 * residual_out <- bf16(s); x = bf16(s * rsqrt(mean(s^2)+eps) * norm_w);
 * qkv = x . W_qkv^T + b (W_qkv = [Q; K; V] rows [q_dim + 2*kv_dim, hidden]);
 * q_out <- bf16(qkv[0:q_dim]); K/V rows -> cache slot (*d_kv_len - 1), un-rotated.
 * residual_out must not alias h or residual_in. */
int efm_decode_norm_qkv(int32_t hidden, int32_t q_dim, int32_t kv_dim, float eps, const void* h,
                        const void* residual_in, void* residual_out, const void* norm_w,
                        const void* w_qkv, const void* b_qkv, void* q_out, void* k_cache,
                        void* v_cache, const uint32_t* d_kv_len, hipStream_t stream);

/* efm_decode_norm_qkv with RoPE-Llama applied in the projection's epilogue, for caches
 * that hold rotated keys: with L = *d_kv_len, q_out <- bf16(rot(bf16(q), L - 1 +
 * q_rope_pos_offset)) and the cache slot L - 1 receives bf16(rot(bf16(k), L - 1 +
 * k_rope_pos_offset)) and V; rot turns the pair (d, d + hd/2) by pos * inv_freq[d]
 * (inv_freq as in efm_rope_llama_inplace, cos / sin in fp32). The head geometry and the
 * RoPE parameters come from ctx (pos_encoding EFM_POS_ROPE_LLAMA, contiguous q and cache
 * rows). A following efm_attention_decode with pos_encoding EFM_POS_NONE on that cache
 * computes the reference's RoPE-on-read attention (qwen2_5.cpp:600-790 with
 * attention.cu:135-139): q . k_j after both rotations. Replaces the FusedQKVLinearLayer
 * projection of the decode step plus the RoPE that FlashInferAttentionOp::forward_decode
 * (attention_op.cu:1565-1604) applies to q and to the newest key. */
int efm_decode_norm_qkv_rope(const efm_attention_ctx* ctx, int32_t hidden, float eps, const void* h,
                             const void* residual_in, void* residual_out, const void* norm_w,
                             const void* w_qkv, const void* b_qkv, void* q_out, void* k_cache,
                             void* v_cache, const uint32_t* d_kv_len, hipStream_t stream);

/* Fused front half of a decode layer: efm_decode_norm_qkv followed by
 * efm_decode_attention_partials, in one launch, with bit-identical results. Replaces the
 * input_layernorm -> fused_qkv -> AttentionLayer::forward_decode sequence of
 * qwen2_5.cpp:600-790 (RMSNormLayer, FusedQKVLinearLayer::forward_fp16_bf16
 * linear.cu:1387-1461, FlashInferAttentionOp::forward_decode attention_op.cu:1565-1604)
 * for the engine's rotated cache: ctx needs head_dim 128, RoPE and
 * k_already_prerotated = EFM_K_PREROTATED_EXCEPT_NEWEST. The query never reaches memory:
 * the projection hands it (and the newest K / V row) to the attention splits of the same
 * launch, which write their (o, m, l) partials into attn_workspace for
 * efm_decode_attention_merge_o_proj. Cache slot *d_kv_len - 1 receives V and the rotated
 * K; *d_kv_len >= 1. sync_workspace: efm_decode_qkv_attention_sync_bytes(q_dim, kv_dim)
 * bytes, zero-filled once and then reused by every launch (launches sharing it must be
 * stream-ordered). The attention splits wait for GEMV workgroups of the same grid, which
 * never wait themselves; with at most 128 splits every GEMV workgroup finds a slot as
 * soon as any other workgroup on the GPU ends, so the waits end. They are bounded all the
 * same (2^20 polls): a split that does not receive its inputs in time goes on with zeros
 * and flags the workspace, and efm_decode_qkv_attention_status reports EFM_ERR_DEVICE and
 * clears the flag (it synchronises the stream); launches after it compute correctly.
 * efm_decode_norm_qkv_attention_supported tells whether a shape qualifies (hidden <= 4096,
 * at most 128 attention splits of 128 keys, a cache length whose partials plan is not the
 * one-wave one, contiguous cache rows); otherwise call the two unfused entry points. */
size_t efm_decode_qkv_attention_sync_bytes(int32_t q_dim, int32_t kv_dim);
int efm_decode_norm_qkv_attention_supported(const efm_attention_ctx* ctx, int32_t hidden, uint32_t max_kv_len);
int efm_decode_norm_qkv_attention(const efm_attention_ctx* ctx, int32_t hidden, float eps, const void* h,
                                  const void* residual_in, void* residual_out, const void* norm_w,
                                  const void* w_qkv, const void* b_qkv, void* k_cache, void* v_cache,
                                  const uint32_t* d_kv_len, uint32_t max_kv_len, void* attn_workspace,
                                  size_t attn_workspace_bytes, void* sync_workspace, size_t sync_workspace_bytes,
                                  hipStream_t stream);
int efm_decode_qkv_attention_status(void* sync_workspace, hipStream_t stream);

/* Post-attention fused add-norm + gate/up projection + SwiGLU (qwen2_5.cpp:849-875):
 * s = a + residual_in; residual_out <- bf16(s); x = bf16(s * rsqrt(...) * norm_w);
 * out[i] = bf16(silu(bf16(x.W_gate[i])) * bf16(x.W_up[i])) with W = [up; gate]. */
int efm_decode_norm_gate_up_swiglu(int32_t hidden, int32_t inter, float eps, const void* a,
                                   const void* residual_in, void* residual_out, const void* norm_w,
                                   const void* w_up_gate, void* out, hipStream_t stream);

/* Final fused add-norm + LM head + greedy top-1 (qwen2_5.cpp:883-922). */
int efm_decode_norm_lm_head_top1(int32_t hidden, int64_t vocab, float eps, const void* h,
                                 const void* residual_in, const void* norm_w, const void* w_lm,
                                 int32_t* token_out, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* EDGEFM_HIP_H_ */

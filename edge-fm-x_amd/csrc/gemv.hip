// Batch-1 decode GEMV entry points for gfx950 (kernel body in gemv_impl.hpp): linear,
// fused SwiGLU, fused RMSNorm (+ residual) prologues, QKV split into the KV cache,
// attention-split merge + o_proj, and the LM head with a greedy top-1 epilogue.
#include "gemv_impl.hpp"

#include <algorithm>

namespace efm {

template <int R, int KS, int PRO, int EPI, int NJM>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvArgs a, int nj, int nseg) {
    gemv_body<R, KS, PRO, EPI, NJM>(a, nj, nseg, blockIdx.x, gridDim.x);
}

}  // namespace efm

// ----------------------------------------------------------------------------------
// Host-side dispatch.
// ----------------------------------------------------------------------------------
namespace efm {

// Launch geometry for K inputs and N logical rows (P physical rows each), from a sweep of
// the Qwen2.5 1.5B and 7B decode shapes on MI355X (graph replays over 28 weight copies):
//  * the K split KS keeps each lane at <= 6 16-byte chunks per row and segment;
//  * rows per wave group R: 4 for very tall matrices (the LM head), 2 with one wave per
//    single row (1.5B q/k/v 4.52 -> 3.97 us), else 1 (single_row: always 1);
//  * grid: 768 workgroups for single rows split over 2 or 4 waves (7B q/k/v 8.92 -> 8.27,
//    o_proj 6.72 -> 6.27, down 24.15 -> 23.67; 1.5B down 7.39 -> 7.01 us); paired up /
//    gate rows: 512 with one wave per row pair (1.5B 10.84 -> 10.43 us), 4096 with two (7B
//    41.95 -> 41.04 us); otherwise the caller's cap (about 4 workgroups per CU, 2 for the
//    top-1 reduction). Workgroups walk row blocks grid-stride.
static GemvCfg gemv_pick(int K, int N, int P, int max_grid, bool tall, bool single_row = false) {
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
    else if (!tall && !single_row && P == 1 && g.KS == 1) g.R = 2;
    if (!tall) {
        if (P == 1 && g.KS >= 2) max_grid = 768;
        else if (P == 2) max_grid = (g.KS == 1) ? 512 : 4096;
    }
    g.nrb = (N + groups * g.R - 1) / (groups * g.R);
    g.grid = std::min(g.nrb, max_grid);
    return g;
}

GemvCfg gemv_pick_config(int K, int N, int P, int max_grid, bool tall, bool single_row) {
    return gemv_pick(K, N, P, max_grid, tall, single_row);
}

// Launch with the fewest load slots per lane and row that hold a row's chunks (an unused
// slot costs the address unit as much as a used one): 2-4 with one wave per row, 3-4 with
// two, 3-6 with four.
template <int RR, int KK, int PRO, int EPI>
static void gemv_launch_slots(const GemvCfg& g, dim3 grid, dim3 block, size_t smem, const GemvArgs& a,
                              hipStream_t stream) {
#define EFM_GEMV_SLOTS(NJV)                                                                    \
    if (g.nj <= NJV) {                                                                         \
        hipLaunchKernelGGL((gemv_kernel<RR, KK, PRO, EPI, NJV>), grid, block, smem, stream, a, g.nj, g.nseg); \
        return;                                                                                \
    }
    if constexpr (KK == 1) {
        EFM_GEMV_SLOTS(2) EFM_GEMV_SLOTS(3) EFM_GEMV_SLOTS(4)
    } else if constexpr (KK == 2) {
        EFM_GEMV_SLOTS(3) EFM_GEMV_SLOTS(4)
    } else {
        EFM_GEMV_SLOTS(3) EFM_GEMV_SLOTS(4) EFM_GEMV_SLOTS(5)
    }
#undef EFM_GEMV_SLOTS
    hipLaunchKernelGGL((gemv_kernel<RR, KK, PRO, EPI, kNJMax>), grid, block, smem, stream, a, g.nj, g.nseg);
}

template <int PRO, int EPI>
static int gemv_launch(const GemvCfg& g, const GemvArgs& a, hipStream_t stream) {
    const size_t smem = (size_t)a.K * sizeof(bf16_t);
    dim3 grid(g.grid), block(kGemvThreads);
#define EFM_GEMV_CASE(RR, KK)                                                                  \
    if (g.R == RR && g.KS == KK) {                                                             \
        gemv_launch_slots<RR, KK, PRO, EPI>(g, grid, block, smem, a, stream);                  \
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

namespace efm {
int validate_attention_ctx(const efm_attention_ctx* c, const char* who);
}

extern "C" int efm_decode_norm_qkv_rope(const efm_attention_ctx* ctx, int32_t hidden, float eps, const void* h,
                                        const void* residual_in, void* residual_out, const void* norm_w,
                                        const void* w_qkv, const void* b_qkv, void* q_out, void* k_cache,
                                        void* v_cache, const uint32_t* d_kv_len, hipStream_t stream) {
    int rc = validate_attention_ctx(ctx, "decode_norm_qkv_rope");
    if (rc) return rc;
    const int hd = (int)ctx->head_dim, Hq = (int)ctx->num_qo_heads, Hkv = (int)ctx->num_kv_heads;
    const int q_dim = Hq * hd, kv_dim = Hkv * hd, N = q_dim + 2 * kv_dim;
    if (ctx->pos_encoding != EFM_POS_ROPE_LLAMA)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv_rope: ctx must name EFM_POS_ROPE_LLAMA");
    if ((ctx->q_stride_n != 0 && ctx->q_stride_n != (uint32_t)q_dim) ||
        (ctx->q_stride_h != 0 && ctx->q_stride_h != (uint32_t)hd) ||
        (ctx->k_stride_n != 0 && ctx->k_stride_n != (uint32_t)kv_dim) ||
        (ctx->k_stride_h != 0 && ctx->k_stride_h != (uint32_t)hd) ||
        (ctx->kv_stride_n != 0 && ctx->kv_stride_n != (uint32_t)kv_dim) ||
        (ctx->kv_stride_h != 0 && ctx->kv_stride_h != (uint32_t)hd))
        return set_error(EFM_ERR_UNSUPPORTED, "decode_norm_qkv_rope: q and the K / V cache rows must be contiguous");
    rc = gemv_check(hidden, N, w_qkv, h, q_out, true);
    if (rc) return rc;
    if (norm_w == nullptr || residual_out == nullptr || k_cache == nullptr || v_cache == nullptr ||
        d_kv_len == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv_rope: null pointer");
    if (residual_out == h || (residual_in != nullptr && residual_out == residual_in))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv_rope: residual_out must not alias its inputs");
    GemvArgs a = gemv_args(hidden, N / 2, w_qkv, h);
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
    a.rope_half = hd / 2;
    a.q_pos_off = (int)ctx->q_rope_pos_offset;
    a.k_pos_off = (int)ctx->k_rope_pos_offset;
    rope_table_fill(&a.rope, hd, ctx->rope_theta, ctx->rope_scale);
    // one logical row = the pair (d, d + hd/2) of a head: a row block (4 / KS logical rows)
    // must not straddle two heads
    const GemvCfg g = gemv_pick(hidden, N / 2, 2, 1024, false);
    if ((hd / 2) % (4 / g.KS * g.R) != 0)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_norm_qkv_rope: head_dim %d with hidden %d", hd, hidden);
    if (residual_in == nullptr) return gemv_launch<PRO_NORM, EPI_QKV_ROPE>(g, a, stream);
    return gemv_launch<PRO_ADD_NORM, EPI_QKV_ROPE>(g, a, stream);
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
size_t decode_workspace_bytes(const efm_attention_ctx* ctx, uint32_t max_kv_len);
size_t decode_ml_offset(const efm_attention_ctx* ctx, uint32_t max_kv_len);
DecodePartialsPlan decode_partials_plan(const efm_attention_ctx* c, uint32_t max_kv_len);
int validate_attention_ctx(const efm_attention_ctx* c, const char* who);

// The partials plan's splits fit the merge prologue of this query width: up to 24 splits
// for widths up to 1024, 12 up to 2048.
static int merge_o_proj_supported(const efm_attention_ctx* ctx, uint32_t max_kv_len, DecodePartialsPlan* plan) {
    int rc = validate_attention_ctx(ctx, "attention_merge_o_proj");
    if (rc) return rc;
    if (max_kv_len == 0) return set_error(EFM_ERR_INVALID_ARGUMENT, "attention_merge_o_proj: max_kv_len is 0");
    const DecodePartialsPlan p = decode_partials_plan(ctx, max_kv_len);
    if (plan != nullptr) *plan = p;
    const int64_t width = (int64_t)ctx->num_qo_heads * ctx->head_dim;
    if (p.split_cap > merge_max_splits(width))
        return set_error(EFM_ERR_UNSUPPORTED,
                         "attention_merge_o_proj: %d splits of a %lld-wide query exceed the fused merge (%d)",
                         p.split_cap, (long long)width, merge_max_splits(width));
    return EFM_OK;
}
}  // namespace efm

extern "C" int efm_decode_attention_merge_o_proj_supported(const efm_attention_ctx* ctx, uint32_t max_kv_len) {
    return merge_o_proj_supported(ctx, max_kv_len, nullptr);
}

extern "C" int efm_decode_attention_merge_o_proj(const efm_attention_ctx* ctx, const uint32_t* d_kv_len,
                                                 uint32_t max_kv_len, const void* workspace,
                                                 size_t workspace_bytes, const void* w_o, int32_t hidden, void* out,
                                                 hipStream_t stream) {
    DecodePartialsPlan plan;
    int rc = merge_o_proj_supported(ctx, max_kv_len, &plan);
    if (rc) return rc;
    if (d_kv_len == nullptr || workspace == nullptr || w_o == nullptr || out == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "attention_merge_o_proj: null pointer");
    const int q_dim = (int)(ctx->num_qo_heads * ctx->head_dim);
    rc = gemv_check(q_dim, hidden, w_o, workspace, out, false);
    if (rc) return rc;
    if (workspace_bytes < decode_workspace_bytes(ctx, max_kv_len))
        return set_error(EFM_ERR_WORKSPACE, "attention_merge_o_proj: workspace too small");
    GemvArgs a = gemv_args(q_dim, hidden, w_o, workspace);
    a.y = out;
    a.o_part = static_cast<const float*>(workspace);
    a.ml_part = reinterpret_cast<const float*>(static_cast<const char*>(workspace) + decode_ml_offset(ctx, max_kv_len));
    a.split_cap = plan.split_cap;
    a.keys_per_split = plan.keys_per_split;
    a.head_dim = (int)ctx->head_dim;
    a.group = (int)(ctx->num_qo_heads / ctx->num_kv_heads);
    a.attn_len = d_kv_len;
    a.attn_max_len = max_kv_len;
    // every workgroup repeats the split merge: two rows per wave group (gemv_pick's choice
    // with one wave per row) halve the workgroups and the repeats
    const GemvCfg g = gemv_pick(q_dim, hidden, 1, 1024, false);
    if (q_dim <= kMergeNarrowMaxWidth) return gemv_launch<PRO_ATTN_MERGE_N, EPI_BF16>(g, a, stream);
    if (plan.split_cap <= kMergeShortSplits) return gemv_launch<PRO_ATTN_MERGE, EPI_BF16>(g, a, stream);
    return gemv_launch<PRO_ATTN_MERGE_W, EPI_BF16>(g, a, stream);
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

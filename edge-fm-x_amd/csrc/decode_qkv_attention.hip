// Fused decode step front half: RMSNorm (+ residual add) -> QKV projection -> GQA decode
// attention split partials, in one launch (efm_decode_norm_qkv_attention).
//
// The unfused sequence (efm_decode_norm_qkv, then efm_decode_attention_partials) pays a
// kernel boundary between the projection and the attention, and the attention then waits
// for its K / V tiles. Here the grid holds both kinds of workgroup:
//  * workgroups [0, n_attn): one attention split each (decode_attn_lds_body, FUSED).
//    They start first, stage their K / V tiles from HBM while the projection runs, then
//    take this step's query and newest K / V row from the projection's tagged words;
//  * workgroups [n_attn, grid): the QKV GEMV (gemv_body with the QKV_TAG epilogue), which
//    publishes every projected value as a tagged word and stores the V row into the cache.
// Only the attention workgroups wait, and only for GEMV workgroups, which never wait: with
// n_attn far below the chip's workgroup slots every GEMV workgroup can always be placed,
// so the launch cannot deadlock (polls are bounded all the same). The split that owns row
// L - 1 rotates the newest key and stores it into the cache, as the unfused attention
// does. Results are bit-identical to the unfused pair: same GEMV reduction order, same
// bf16 roundings, same attention arithmetic.
#include "decode_attn_impl.hpp"
#include "gemv_impl.hpp"

#include <algorithm>

namespace efm {

int decode_split_cap(int num_kv_heads, uint32_t max_kv_len);
int decode_keys_per_split(int num_kv_heads, uint32_t max_kv_len);
size_t decode_workspace_bytes(const efm_attention_ctx* ctx, uint32_t max_kv_len);
size_t decode_ml_offset(const efm_attention_ctx* ctx, uint32_t max_kv_len);
DecodePartialsPlan decode_partials_plan(const efm_attention_ctx* c, uint32_t max_kv_len);
int validate_attention_ctx(const efm_attention_ctx* c, const char* who);

constexpr int kFusedMaxAttn = 128;       // attention workgroups (a quarter of the slots)
constexpr int kFusedMaxHidden = 4096;    // GEMV K split <= 2
constexpr size_t kFusedSyncHeader = 256;

template <int KS, int PRO, int G>
__global__ __launch_bounds__(kGemvThreads, 2) void decode_qkv_attn_kernel(GemvArgs ga, DecodeArgs da,
                                                                         FusedAttnArgs f, int nj, int nseg) {
    const int blk = blockIdx.x;
    const int n_attn = (int)f.n_attn;
    if (blk < n_attn) {
        decode_attn_lds_body<G, false, true>(da, blk % da.split_cap, blk / da.split_cap, f);
    } else {
        gemv_body<1, KS, PRO, EPI_QKV_TAG>(ga, nj, nseg, blk - n_attn, (int)gridDim.x - n_attn);
    }
}

static size_t sync_bytes(int q_dim, int kv_dim) {
    return kFusedSyncHeader + (((size_t)(q_dim + 2 * kv_dim) * sizeof(uint32_t) + 255) & ~(size_t)255);
}

static int num_cus() {
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

static int fused_supported(const efm_attention_ctx* ctx, int32_t hidden, uint32_t max_kv_len) {
    int rc = validate_attention_ctx(ctx, "decode_norm_qkv_attention");
    if (rc) return rc;
    const int hd = (int)ctx->head_dim, Hkv = (int)ctx->num_kv_heads;
    const int G = (int)(ctx->num_qo_heads / ctx->num_kv_heads);
    if (hd != 128 || ctx->pos_encoding != EFM_POS_ROPE_LLAMA ||
        ctx->k_already_prerotated != EFM_K_PREROTATED_EXCEPT_NEWEST)
        return set_error(EFM_ERR_UNSUPPORTED,
                         "decode_norm_qkv_attention: needs head_dim 128, RoPE and a rotated cache whose newest "
                         "row is written by this call (k_already_prerotated = 2)");
    const uint32_t kvd = (uint32_t)(Hkv * hd);
    if ((ctx->k_stride_n != 0 && ctx->k_stride_n != kvd) || (ctx->kv_stride_n != 0 && ctx->kv_stride_n != kvd) ||
        (ctx->k_stride_h != 0 && ctx->k_stride_h != (uint32_t)hd) ||
        (ctx->kv_stride_h != 0 && ctx->kv_stride_h != (uint32_t)hd))
        return set_error(EFM_ERR_UNSUPPORTED, "decode_norm_qkv_attention: K / V caches must be contiguous rows");
    if (hidden <= 0 || hidden % 8 != 0 || hidden > kFusedMaxHidden)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_norm_qkv_attention: hidden %d (multiple of 8, <= %d)", hidden,
                         kFusedMaxHidden);
    if (max_kv_len == 0) return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv_attention: max_kv_len is 0");
    if ((int64_t)max_kv_len * kvd * 2 >= 0x7fffffffLL)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_norm_qkv_attention: K / V caches past 2 GB per layer");
    const int kps = decode_keys_per_split(Hkv, max_kv_len);
    const int n_attn = Hkv * decode_split_cap(Hkv, max_kv_len);
    // the partials this launch writes are the plan efm_decode_attention_merge_o_proj reads
    if (decode_partials_plan(ctx, max_kv_len).tile)
        return set_error(EFM_ERR_UNSUPPORTED,
                         "decode_norm_qkv_attention: this cache length takes one-wave splits in the partials plan");
    if (kps != kAttnWaves * kTileKeys || n_attn > kFusedMaxAttn)
        return set_error(EFM_ERR_UNSUPPORTED,
                         "decode_norm_qkv_attention: %d attention workgroups of %d keys (needs <= %d of %d)", n_attn,
                         kps, kFusedMaxAttn, kAttnWaves * kTileKeys);
    if (!(G == 1 || G == 2 || G == 3 || G == 4 || G == 6 || G == 7 || G == 8))
        return set_error(EFM_ERR_UNSUPPORTED, "decode_norm_qkv_attention: group %d", G);
    return EFM_OK;
}

}  // namespace efm

using namespace efm;

extern "C" size_t efm_decode_qkv_attention_sync_bytes(int32_t q_dim, int32_t kv_dim) {
    if (q_dim <= 0 || kv_dim <= 0) return 0;
    return sync_bytes(q_dim, kv_dim);
}

extern "C" int efm_decode_norm_qkv_attention_supported(const efm_attention_ctx* ctx, int32_t hidden,
                                                       uint32_t max_kv_len) {
    return fused_supported(ctx, hidden, max_kv_len);
}

extern "C" int efm_decode_norm_qkv_attention(const efm_attention_ctx* ctx, int32_t hidden, float eps, const void* h,
                                             const void* residual_in, void* residual_out, const void* norm_w,
                                             const void* w_qkv, const void* b_qkv, void* k_cache, void* v_cache,
                                             const uint32_t* d_kv_len, uint32_t max_kv_len, void* attn_workspace,
                                             size_t attn_workspace_bytes, void* sync_workspace,
                                             size_t sync_workspace_bytes, hipStream_t stream) {
    int rc = fused_supported(ctx, hidden, max_kv_len);
    if (rc) return rc;
    const int hd = (int)ctx->head_dim, Hkv = (int)ctx->num_kv_heads, Hq = (int)ctx->num_qo_heads;
    const int G = Hq / Hkv, q_dim = Hq * hd, kv_dim = Hkv * hd, N = q_dim + 2 * kv_dim;
    if (h == nullptr || residual_out == nullptr || norm_w == nullptr || w_qkv == nullptr || k_cache == nullptr ||
        v_cache == nullptr || d_kv_len == nullptr || attn_workspace == nullptr || sync_workspace == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv_attention: null pointer");
    if (residual_out == h || (residual_in != nullptr && residual_out == residual_in))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv_attention: residual_out must not alias its inputs");
    if (((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(w_qkv) | reinterpret_cast<uintptr_t>(norm_w) |
          reinterpret_cast<uintptr_t>(residual_out) | reinterpret_cast<uintptr_t>(k_cache) |
          reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(sync_workspace)) & 15u) != 0 ||
        (residual_in != nullptr && (reinterpret_cast<uintptr_t>(residual_in) & 15u) != 0))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_norm_qkv_attention: pointers must be 16-byte aligned");
    if (attn_workspace_bytes < decode_workspace_bytes(ctx, max_kv_len))
        return set_error(EFM_ERR_WORKSPACE, "decode_norm_qkv_attention: attention workspace of %zu bytes required",
                         decode_workspace_bytes(ctx, max_kv_len));
    if (sync_workspace_bytes < sync_bytes(q_dim, kv_dim))
        return set_error(EFM_ERR_WORKSPACE, "decode_norm_qkv_attention: sync workspace of %zu bytes required",
                         sync_bytes(q_dim, kv_dim));

    // GEMV half: the geometry of efm_decode_norm_qkv, with as many workgroups as fit
    // beside the attention splits (two per CU) and at least one row block each, so every
    // GEMV workgroup publishes words
    const int cap = decode_split_cap(Hkv, max_kv_len);
    const int n_attn = Hkv * cap;
    const GemvCfg g = gemv_pick_config(hidden, N, 1, 1024, false, true);
    if (g.R != 1 || g.KS > 2)
        return set_error(EFM_ERR_UNSUPPORTED, "decode_norm_qkv_attention: GEMV shape R=%d KS=%d", g.R, g.KS);
    const int n_gemv = std::max(1, std::min(g.nrb, 2 * num_cus() - n_attn));
    uint32_t* sync = static_cast<uint32_t*>(sync_workspace);
    uint32_t* words = reinterpret_cast<uint32_t*>(static_cast<char*>(sync_workspace) + kFusedSyncHeader);

    GemvArgs ga = {};
    ga.K = hidden;
    ga.N = N;
    ga.W = static_cast<const bf16_t*>(w_qkv);
    ga.x = static_cast<const bf16_t*>(h);
    ga.r_in = static_cast<const bf16_t*>(residual_in);
    ga.r_out = static_cast<bf16_t*>(residual_out);
    ga.norm_w = static_cast<const bf16_t*>(norm_w);
    ga.eps = eps;
    ga.bias = static_cast<const bf16_t*>(b_qkv);
    ga.q_dim = q_dim;
    ga.kv_dim = kv_dim;
    ga.k_cache = static_cast<bf16_t*>(k_cache);
    ga.v_cache = static_cast<bf16_t*>(v_cache);
    ga.d_kv_len = d_kv_len;
    ga.tag_words = words;
    ga.epoch = sync;

    DecodeArgs da = {};
    da.q = nullptr;
    da.k = static_cast<const bf16_t*>(k_cache);
    da.v = static_cast<const bf16_t*>(v_cache);
    da.o = nullptr;
    da.kv_len = 0;
    da.d_kv_len = d_kv_len;
    da.max_kv_len = max_kv_len;
    da.num_kv_heads = Hkv;
    da.q_sn = q_dim;
    da.q_sh = hd;
    da.k_sn = kv_dim;
    da.k_sh = hd;
    da.v_sn = kv_dim;
    da.v_sh = hd;
    da.q_pos_off = (int)ctx->q_rope_pos_offset;
    da.k_pos_off = (int)ctx->k_rope_pos_offset;
    da.rope_q = 1;
    da.fix_last = 1;
    da.row_bound = (int)max_kv_len;
    da.split_cap = cap;
    da.keys_per_split = decode_keys_per_split(Hkv, max_kv_len);
    char* wsb = static_cast<char*>(attn_workspace);
    da.o_part = reinterpret_cast<float*>(wsb);
    da.ml_part = reinterpret_cast<float*>(wsb + decode_ml_offset(ctx, max_kv_len));
    da.counter = nullptr;
    rope_table_fill(&da.rope, hd, ctx->rope_theta, ctx->rope_scale);

    FusedAttnArgs f;
    f.words = words;
    f.sync = sync;
    f.q_dim = q_dim;
    f.kv_dim = kv_dim;
    f.n_attn = (uint32_t)n_attn;
    const bool force_timeout = kernel_knob(EFM_KNOB_FRONT_WAIT_TIMEOUT) != 0;
    f.spin_limit = force_timeout ? kFusedTestSpin : kFusedSpin;
    f.tag_or = force_timeout ? (1u << 16) : 0u;   // tags are 16 bits: no word matches

    const dim3 grid(n_attn + n_gemv), block(kGemvThreads);
    const size_t smem = (size_t)hidden * sizeof(bf16_t);
#define EFM_QKVA_CASE(KSV, GV)                                                                                   \
    if (g.KS == KSV && G == GV) {                                                                               \
        if (residual_in == nullptr)                                                                             \
            hipLaunchKernelGGL((decode_qkv_attn_kernel<KSV, PRO_NORM, GV>), grid, block, smem, stream, ga, da, f, \
                               g.nj, g.nseg);                                                                   \
        else                                                                                                    \
            hipLaunchKernelGGL((decode_qkv_attn_kernel<KSV, PRO_ADD_NORM, GV>), grid, block, smem, stream, ga, da, \
                               f, g.nj, g.nseg);                                                                \
        return check_launch("decode_norm_qkv_attention");                                                       \
    }
    EFM_QKVA_CASE(1, 1) EFM_QKVA_CASE(1, 2) EFM_QKVA_CASE(1, 3) EFM_QKVA_CASE(1, 4)
    EFM_QKVA_CASE(1, 6) EFM_QKVA_CASE(1, 7) EFM_QKVA_CASE(1, 8)
    EFM_QKVA_CASE(2, 1) EFM_QKVA_CASE(2, 2) EFM_QKVA_CASE(2, 3) EFM_QKVA_CASE(2, 4)
    EFM_QKVA_CASE(2, 6) EFM_QKVA_CASE(2, 7) EFM_QKVA_CASE(2, 8)
#undef EFM_QKVA_CASE
    return set_error(EFM_ERR_UNSUPPORTED, "decode_norm_qkv_attention: KS=%d G=%d", g.KS, G);
}

extern "C" int efm_decode_qkv_attention_status(void* sync_workspace, hipStream_t stream) {
    if (sync_workspace == nullptr) return set_error(EFM_ERR_INVALID_ARGUMENT, "decode_qkv_attention_status: null");
    uint32_t flag = 0;
    uint32_t* abort_word = static_cast<uint32_t*>(sync_workspace) + 2;
    if (hipMemcpyAsync(&flag, abort_word, sizeof(flag), hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return set_error(EFM_ERR_DEVICE, "decode_qkv_attention_status: copy failed");
    if (flag != 0) {
        // Clear the report and step the epoch once more. After a time-out the epoch can
        // advance while a GEMV workgroup of the same launch has not read it yet; that
        // workgroup then tags its words with the next launch's tag, and the next launch
        // could take those stale words for its own. One more step makes the next tag
        // one that no word written so far carries.
        uint32_t head[3] = {0, 0, 0};
        if (hipMemcpyAsync(head, sync_workspace, sizeof(head), hipMemcpyDeviceToHost, stream) != hipSuccess ||
            hipStreamSynchronize(stream) != hipSuccess)
            return set_error(EFM_ERR_DEVICE, "decode_qkv_attention_status: copy failed");
        head[0] += 1u;
        head[2] = 0u;
        if (hipMemcpyAsync(sync_workspace, head, sizeof(head), hipMemcpyHostToDevice, stream) != hipSuccess ||
            hipStreamSynchronize(stream) != hipSuccess)
            return set_error(EFM_ERR_DEVICE, "decode_qkv_attention_status: reset failed");
        return set_error(EFM_ERR_DEVICE, "decode_norm_qkv_attention: an attention split's wait for its inputs timed out; the outputs of "
                         "the launches since the last status call are invalid");
    }
    return EFM_OK;
}

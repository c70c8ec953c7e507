// SageAttention-style prefill attention for gfx950: K smoothing, per-128-token-block
// symmetric int8 quantisation of Q and K, QK^T on the int8 matrix cores
// (v_mfma_i32_32x32x32_i8) with exact int32 accumulation, fp32 online softmax, and
// P.V on the bf16 matrix cores with fp32 accumulation (the EdgeFM
// reference names the feature, README.md:23, but has no implementation).
//
// Definition (Zhang et al., SageAttention, 2024, with the choices fixed here):
//   kmean[h][d] = fp32( sum_j K[j][h][d] (float64) / L )       (softmax-invariant shift)
//   per (128-token block b, head h): scale = max|x| / 127 (1 for an all-zero block),
//   x8 = clamp(round_half_even(x / scale), -127, 127), with x = Q or K - kmean
//   score_log2(i, j) = float(int32(Q8_i . K8_j)) * ((sq * sk) * (log2(e) / sqrt(hd)))
//   causal: query i sees keys j <= i + (L - S); P rounded to bf16 for the PV product.
//
// Three launches: K column sums (float64; the attention entry point: per KV head and row
// slice, coalesced rows; efm_sage_quantize: per KV head and 8 channels), block
// quantisation of Q and K (one workgroup per block x head), attention (one workgroup =
// 128 query rows of one head, 64-key tiles staged in LDS as int8 K and transposed V).
#include "attn_pipe.hpp"
#include "common.hpp"

#include <algorithm>
#include <type_traits>
#include <cstdlib>

namespace efm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int int32x4_t __attribute__((ext_vector_type(4)));
typedef int int32x16_t __attribute__((ext_vector_type(16)));

constexpr int kSageBlock = 128;
constexpr int kSageThreads = 256;
constexpr int kSageQ = 128;   // query rows per attention workgroup
constexpr int kSageKV = 64;   // keys per LDS tile

// ---- K mean over tokens: grid (Hkv, hd / 8), 1024 threads --------------------------
// Workgroup (h, c) owns channels [8c, 8c + 8) of KV head h; thread t adds rows
// j = t (mod 1024) with 16-byte loads (four rows in flight per step: one round trip up to
// 4096 rows), then butterfly sums over each wave and a sum over the 16 waves. Sums of bf16
// values in float64 are exact while their binary range fits the 53-bit significand, as
// it does for cache contents, so the result matches any summation order.
constexpr int kKmeanThreads = 1024;
__global__ __launch_bounds__(kKmeanThreads) void sage_kmean_kernel(const bf16_t* k, int L, int k_sn, int k_sh, int hd,
                                                                   float* kmean) {
    __shared__ double part[kKmeanThreads / kWave][8];
    const int h = blockIdx.x, d0 = blockIdx.y * 8, t = threadIdx.x;
    const bf16_t* base = k + (size_t)h * k_sh + d0;
    double s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = 0.0;
    int j = t;
    for (; j + 3 * kKmeanThreads < L; j += 4 * kKmeanThreads) {
        uint4 u[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) u[r] = *reinterpret_cast<const uint4*>(base + (size_t)(j + r * kKmeanThreads) * k_sn);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float x[8];
            unpack8(u[r], x);
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] += (double)x[e];
        }
    }
    for (; j < L; j += kKmeanThreads) {
        float x[8];
        unpack8(*reinterpret_cast<const uint4*>(base + (size_t)j * k_sn), x);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] += (double)x[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int off = kWave / 2; off >= 1; off >>= 1) s[e] += __shfl_xor(s[e], off, kWave);
    if (t % kWave == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) part[t / kWave][e] = s[e];
    }
    __syncthreads();
    if (t < 8) {
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < kKmeanThreads / kWave; ++w) sum += part[w][t];
        kmean[h * hd + d0 + t] = (float)(sum / (double)L);
    }
}

// ---- K column sums in row slices: grid (Hkv, kKSlices), 256 threads -------------
// The attention entry point's K mean: workgroup (h, sl) sums rows [sl * per, (sl + 1) *
// per) of KV head h over every channel, 16 lanes (hd 128) per row, so a wave's 16-byte
// loads cover four whole 256-byte rows; the quantisation kernel adds the slices (float64:
// exact, so the mean equals sage_kmean_kernel's bit for bit).
constexpr int kKSlices = 16;
__global__ __launch_bounds__(kSageThreads) void sage_kpart_kernel(const bf16_t* k, int L, int k_sn, int k_sh, int hd,
                                                                  double* part) {
    __shared__ double red[kSageThreads][8];
    const int h = blockIdx.x, sl = blockIdx.y, t = threadIdx.x;
    const int cpr = hd / 8, c = t % cpr, r0 = t / cpr, rstep = kSageThreads / cpr;
    const int per = (L + kKSlices - 1) / kKSlices;
    const int j0 = sl * per, j1 = min(L, j0 + per);
    const bf16_t* base = k + (size_t)h * k_sh + c * 8;
    double s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = 0.0;
    int j = j0 + r0;
    for (; j + 3 * rstep < j1; j += 4 * rstep) {
        uint4 u[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) u[r] = *reinterpret_cast<const uint4*>(base + (size_t)(j + r * rstep) * k_sn);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float x[8];
            unpack8(u[r], x);
#pragma unroll
            for (int e = 0; e < 8; ++e) s[e] += (double)x[e];
        }
    }
    for (; j < j1; j += rstep) {
        float x[8];
        unpack8(*reinterpret_cast<const uint4*>(base + (size_t)j * k_sn), x);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] += (double)x[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) red[t][e] = s[e];
    __syncthreads();
    if (t < hd) {
        const int cc = t / 8, e = t % 8;
        double sum = 0.0;
        for (int r = 0; r < rstep; ++r) sum += red[r * cpr + cc][e];
        part[((size_t)sl * gridDim.x + h) * hd + t] = sum;
    }
}

// ---- block quantisation: grid (blocks, H), 256 threads --------------------------
// dst [T][H][hd] int8 (contiguous), scales [blocks][H]. KM = 0: Q (no shift); 1: K with
// its mean from kmean (sage_kmean_kernel); 2: K with its mean added up here from the
// kKSlices row-slice sums in kpart (sage_kpart_kernel; block 0 stores it in kmean_out).
// Every load is issued up front and branch-free (rows past the block's end are buffer
// loads past the resource: zeros, no memory access), so one round trip covers them all.
template <int KM>
__global__ __launch_bounds__(kSageThreads) void sage_quant_kernel(const bf16_t* src, int T, int H, int sn, int sh,
                                                                  int hd, const float* kmean, const double* kpart,
                                                                  float* kmean_out, int8_t* dst, float* scales) {
    __shared__ float red[kSageThreads / kWave];
    __shared__ float kms[KM == 2 ? 128 : 1];
    const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int t0 = b * kSageBlock;
    const int rows = min(kSageBlock, T - t0);
    const int cpr = hd / 8;  // 16-byte chunks per row
    const int nch = rows * cpr;
    constexpr int kMaxPer = kSageBlock * 128 / 8 / kSageThreads;  // 8
    // every chunk of a thread covers the same 8 channels (the thread count is a multiple
    // of the chunks per row), so their K means are loaded once, beside the data
    const int d0 = (tid % cpr) * 8;
    float4 k0 = make_float4(0.f, 0.f, 0.f, 0.f), k1 = k0;
    if constexpr (KM == 1) {
        k0 = *reinterpret_cast<const float4*>(kmean + h * hd + d0);
        k1 = *reinterpret_cast<const float4*>(kmean + h * hd + d0 + 4);
    }
    uint4 raw[kMaxPer];
    {
        typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<bf16_t*>(src + (size_t)t0 * sn + (size_t)h * sh), (short)0, rows * sn * 2, 0x00020000);
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) {
            const int c = tid + i * kSageThreads;
            const uint32_t off = (c < nch) ? (uint32_t)(((c / cpr) * sn + d0) * 2) : 0x80000000u;
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
            raw[i] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    }
    double kv[KM == 2 ? kKSlices : 1];
    if constexpr (KM == 2) {
#pragma unroll
        for (int sl = 0; sl < kKSlices; ++sl) kv[sl] = kpart[((size_t)sl * H + h) * hd + tid % hd];
    }
    float km[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    if constexpr (KM == 2) {
        double sum = 0.0;
#pragma unroll
        for (int sl = 0; sl < kKSlices; ++sl) sum += kv[sl];
        const float mean = (float)(sum / (double)T);
        if (tid < hd) {
            kms[tid] = mean;
            if (b == 0) kmean_out[h * hd + tid] = mean;
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < 8; ++e) km[e] = kms[d0 + e];
    }
    float x[kMaxPer][8];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int c = tid + i * kSageThreads;
        unpack8(raw[i], x[i]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // x - kmean in fp32 (subtracting 0 for Q leaves it unchanged)
            x[i][e] = (c < nch) ? x[i][e] - km[e] : 0.f;
            amax = fmaxf(amax, fabsf(x[i][e]));
        }
    }
    amax = wave_max(amax);
    if (tid % kWave == 0) red[tid / kWave] = amax;
    __syncthreads();
    float m = 0.f;
#pragma unroll
    for (int w = 0; w < kSageThreads / kWave; ++w) m = fmaxf(m, red[w]);
    const float scale = (m > 0.f) ? m / 127.0f : 1.0f;
    if (tid == 0) scales[b * H + h] = scale;
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int c = tid + i * kSageThreads;
        if (c < nch) {
            const int r = c / cpr;
            uint32_t w[2] = {0u, 0u};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float qv = rintf(x[i][e] / scale);
                qv = fminf(fmaxf(qv, -127.f), 127.f);
                w[e / 4] |= ((uint32_t)((int)qv & 0xff)) << (8 * (e % 4));
            }
            *reinterpret_cast<uint2*>(dst + ((size_t)(t0 + r) * H + h) * hd + d0) = make_uint2(w[0], w[1]);
        }
    }
}

// ---- attention -----------------------------------------------------------------
struct SageArgs {
    const bf16_t* q;     // bf16 queries (quantised inside the pipelined kernel)
    int q_sn, q_sh;
    const int8_t* q8;    // [S][Hq][hd]
    const int8_t* k8;    // [L][Hkv][hd]
    const float* sq;     // [ceil(S/128)][Hq]
    const float* sk;     // [ceil(L/128)][Hkv]
    const bf16_t* v;
    bf16_t* o;
    int S, L, Hq, Hkv;
    int v_sn, v_sh;
    int causal;
    float scale_log2;
};

union Pack8 {
    bf16x8_t v;
    uint4 u;
    uint32_t w[4];
};

template <int HD>
__global__ __launch_bounds__(kSageThreads) void sage_attn_kernel(SageArgs a) {
    constexpr int KS8 = HD / 32;       // int8 MFMA k-steps
    constexpr int DT = HD / 32;        // d tiles of O^T
    constexpr int KP = HD + 16;        // LDS pitch of the int8 K tile (bytes)
    constexpr int VP = kSageKV + 8;    // LDS pitch of the V^T tile (bf16)
    __shared__ __align__(16) int8_t Ks[kSageKV * KP];
    __shared__ __align__(16) bf16_t Vt[HD * VP];

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int ql = lane % 32, hh = lane / 32;
    const int nqt = (a.S + kSageQ - 1) / kSageQ;
    const int qt = nqt - 1 - (int)blockIdx.x;  // heavy (late) tiles first
    const int head = blockIdx.y;
    const int kvh = head / (a.Hq / a.Hkv);
    const int q0 = qt * kSageQ + wave * 32;
    const int qi = q0 + ql;
    const int diag = a.L - a.S;

    // Q8 B operand: lane row qi, k = ks*32 + hh*16 + byte
    int32x4_t qf[KS8];
    {
        const bool qv = qi < a.S;
        const int8_t* qp = a.q8 + ((size_t)(qv ? qi : 0) * a.Hq + head) * HD + hh * 16;
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) {
            const uint4 u = qv ? *reinterpret_cast<const uint4*>(qp + ks * 32) : make_uint4(0, 0, 0, 0);
            qf[ks] = int32x4_t{(int)u.x, (int)u.y, (int)u.z, (int)u.w};
        }
    }
    const float qscale = (qi < a.S) ? a.sq[(qi / kSageBlock) * a.Hq + head] * 1.0f : 0.f;

    f32x16_t oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[t][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    const int q_last = min(a.S - 1, qt * kSageQ + kSageQ - 1);
    const int kv_end = a.causal ? min(a.L, q_last + diag + 1) : a.L;
    const int ntiles = (kv_end + kSageKV - 1) / kSageKV;

    for (int t = 0; t < ntiles; ++t) {
        const int k0 = t * kSageKV;
        __syncthreads();
        constexpr int KCH = HD / 16;  // 16-byte chunks per int8 K row
        for (int c = tid; c < kSageKV * KCH; c += kSageThreads) {
            const int kr = c / KCH, off = (c % KCH) * 16;
            const int j = k0 + kr;
            const uint4 u = (j < kv_end) ? *reinterpret_cast<const uint4*>(a.k8 + ((size_t)j * a.Hkv + kvh) * HD + off)
                                         : make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4*>(&Ks[kr * KP + off]) = u;
        }
        constexpr int VCH = HD / 8;
        for (int c = tid; c < kSageKV * VCH; c += kSageThreads) {
            const int kr = c / VCH, d0 = (c % VCH) * 8;
            const int j = k0 + kr;
            const uint4 u = (j < kv_end)
                                ? *reinterpret_cast<const uint4*>(a.v + (size_t)j * a.v_sn + (size_t)kvh * a.v_sh + d0)
                                : make_uint4(0, 0, 0, 0);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                Vt[(d0 + 2 * e) * VP + kr] = (bf16_t)(w[e] & 0xffffu);
                Vt[(d0 + 2 * e + 1) * VP + kr] = (bf16_t)(w[e] >> 16);
            }
        }
        __syncthreads();
        if (q0 >= a.S) continue;
        // sk is per 128-key block; a 64-key tile lies inside one block
        const float coef_k = a.sk[(k0 / kSageBlock) * a.Hkv + kvh];
        const float coef = (qscale * coef_k) * a.scale_log2;
#pragma unroll
        for (int sub = 0; sub < kSageKV / 32; ++sub) {
            const int kb0 = k0 + sub * 32;
            if (a.causal && kb0 > q0 + 31 + diag) break;
            if (kb0 >= kv_end) break;
            int32x16_t acc;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
            for (int ks = 0; ks < KS8; ++ks) {
                const uint4 u = *reinterpret_cast<const uint4*>(&Ks[(sub * 32 + ql) * KP + ks * 32 + hh * 16]);
                const int32x4_t ka = int32x4_t{(int)u.x, (int)u.y, (int)u.z, (int)u.w};
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka, qf[ks], acc, 0, 0, 0);
            }
            float s[16];
            float mloc = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int j = kb0 + (e / 4) * 8 + hh * 4 + (e % 4);
                const bool ok = (j < kv_end) && (!a.causal || j <= qi + diag);
                s[e] = ok ? (float)acc[e] * coef : -INFINITY;
                mloc = fmaxf(mloc, s[e]);
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
            const float m_new = fmaxf(m_run, mloc);
            const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
            float p[16], psum = 0.f;
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
    const float inv = (l_run > 0.f) ? 1.f / l_run : 0.f;
    bf16_t* op = a.o + ((size_t)qi * a.Hq + head) * HD;
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
// Pipelined variant (head_dim 128): 4 or 8 wave64s = 128 or 256 query rows of one head
// per workgroup; 64-key int8 K tiles (8 KB) and bf16 V tiles (16 KB) stream global ->
// LDS with global_load_lds into an S-deep ring, laid out and read as described in
// attn_pipe.hpp (int8 K operand via ds_read_b128, V^T via ds_read_b64_tr_b16). The
// running max is only raised when a row's tile max exceeds it by more than 2^8.
//
// Vector ALU work per score is one FMA, one exp2 and a share of the max, the bf16 pack
// and the row sum (the vector ALU, not the matrix cores, bounded the first version):
//  * the int32 score accumulators start at 1.5 * 2^23 (C operand of the first MFMA), so
//    their bits read as a float are exactly 1.5 * 2^23 + score (|score| <= 127^2 * 128 <
//    2^22): no int -> float conversion; one FMA applies the dequantisation scale, the
//    offset and the running max: s = t * coef - (1.5 * 2^23 * coef + m);
//  * row sums add the bf16-rounded p that the PV MFMAs use (v_dot2c_f32_bf16);
//  * DMA addresses are a per-lane offset fixed for the whole loop plus a
//    workgroup-uniform tile base (the last, partial tile clamps its rows).
// ---------------------------------------------------------------------------------
constexpr int kSPKV = 64;
constexpr int kSPHD = 128;
constexpr int kSPKTile = kSPKV * kSPHD;          // int8 bytes
constexpr int kSPVTile = kSPKV * kSPHD * 2;      // bf16 bytes
constexpr int kSPStage = kSPKTile + kSPVTile;
constexpr float kSPLazy = 8.0f;
constexpr float kMagic = 12582912.0f;   // 1.5 * 2^23: its float ulp is 1

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Sum of the two bf16 halves of `w` added to acc (fp32).
__device__ __forceinline__ float add_bf16_pair(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w),
                                           __builtin_bit_cast(bf16x2_t, 0x3f803f80u), acc, false);
}

template <int WAVES, int S>
__global__ __launch_bounds__(WAVES * 64, 8 / WAVES) void sage_attn_pipe_kernel(SageArgs a, int nqt) {
    constexpr int QR = WAVES * 32;                          // query rows per workgroup
    constexpr int LPW = kSPStage / 1024 / WAVES;            // 1 KB wave loads per wave per tile
    constexpr int KS8 = kSPHD / 32;    // int8 k-steps
    constexpr int DT = kSPHD / 32;
    static_assert(LPW * WAVES * 1024 == kSPStage && S >= 2 && S <= 4, "bad pipeline shape");
    __shared__ __align__(1024) unsigned char smem[S * kSPStage];

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int ql = lane % 32, hh = lane / 32;
    const int t = (int)blockIdx.x;
    const int qt = nqt - 1 - t / a.Hq;
    const int head = t % a.Hq;
    const int kvh = head / (a.Hq / a.Hkv);
    const int q0 = qt * QR + wave * 32;
    const int qi = q0 + ql;
    const int diag = a.L - a.S;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);

    const int q_last = min(a.S - 1, qt * QR + QR - 1);
    const int kv_end = a.causal ? min(a.L, q_last + diag + 1) : a.L;
    const int ntiles = (kv_end + kSPKV - 1) / kSPKV;

    // Q: bf16 row qi at d = ks*32 + hh*16 + 0..15 (the int8 B-operand layout), requested
    // first and quantised here with the scale of its 128-row block (max |q| over the
    // block, scale = max / 127 or 1, q8 = clamp(rint(q / scale), -127, 127): the
    // per-block definition of sage_quant_kernel, computed by the block's 4 waves)
    float xq[KS8][16];
    {
        const bool qv = qi < a.S;
        const bf16_t* qp = a.q + (size_t)(qv ? qi : 0) * a.q_sn + (size_t)head * a.q_sh + hh * 16;
        uint4 u[KS8][2];
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) {
            u[ks][0] = qv ? *reinterpret_cast<const uint4*>(qp + ks * 32) : make_uint4(0, 0, 0, 0);
            u[ks][1] = qv ? *reinterpret_cast<const uint4*>(qp + ks * 32 + 8) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) {
            unpack8(u[ks][0], &xq[ks][0]);
            unpack8(u[ks][1], &xq[ks][8]);
        }
    }
    // wave load i of a stage: K8 loads (8 rows x 8 chunks) first, then V (4 rows x 16);
    // q = wave + i * WAVES, so whether load i is a K load is known at compile time
    constexpr int KL = kSPKTile / 1024;   // K wave loads per stage
    const char* kbase = reinterpret_cast<const char*>(a.k8) + (size_t)kvh * kSPHD;
    const char* vbase = reinterpret_cast<const char*>(a.v + (size_t)kvh * a.v_sh);
    auto load_geo = [&](int i, int& row, int& c) {
        const int q = wave + i * WAVES;
        if (i * WAVES < KL) {
            row = q * 8 + (lane >> 3);
            c = (lane & 7) ^ ((row >> 1) & 7);   // attn_pipe::k8_off
        } else {
            row = (q - KL) * 4 + (lane >> 4);
            c = (lane & 15) ^ ((row & 3) << 2);   // attn_pipe::v_off
        }
    };
    auto load_off = [&](int i, int row, int c) {
        return (i * WAVES < KL) ? (uint32_t)(row * a.Hkv * kSPHD + c * 16) : (uint32_t)((row * a.v_sn + c * 8) * 2);
    };
    uint32_t loff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
        int row, c;
        load_geo(i, row, c);
        loff[i] = load_off(i, row, c);
    }
    const uint32_t dst0 = __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(wave * 1024));
    auto issue = [&](int tile, int slot) {
        const int k0 = tile * kSPKV;
        const char* kt0 = kbase + (size_t)k0 * a.Hkv * kSPHD;
        const char* vt0 = vbase + (size_t)k0 * a.v_sn * 2;
        const uint32_t dst = dst0 + (uint32_t)(slot * kSPStage);
        auto load = [&](int i, uint32_t off) {
            const char* src = (i * WAVES < KL ? kt0 : vt0) + off;
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src),
                (__attribute__((address_space(3))) void*)(uintptr_t)(dst + (uint32_t)(i * WAVES * 1024)), 16, 0, 0);
        };
        if (k0 + kSPKV <= a.L) {
#pragma unroll
            for (int i = 0; i < LPW; ++i) load(i, loff[i]);
        } else {   // the last, partial tile: rows past the end read the last row
#pragma unroll
            for (int i = 0; i < LPW; ++i) {
                int row, c;
                load_geo(i, row, c);
                load(i, load_off(i, min(row, a.L - 1 - k0), c));
            }
        }
    };
    // With a 4-slot ring the tiles go in pairs: one barrier per two tiles (after this wave's
    // loads of both have landed), then the next pair is loaded into the slots of the
    // previous pair, which every wave has finished. Smaller rings keep one barrier per tile,
    // with S - 1 tiles in flight.
    constexpr bool PAIR = (S == 4);
    const int pre = PAIR ? min(2, ntiles) : min(S - 1, ntiles);
    for (int p = 0; p < pre; ++p) issue(p, p);

    __shared__ float s_qmax[WAVES];
    int32x4_t qf[KS8];
    float qscale;
    {
        float amax = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks)
#pragma unroll
            for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(xq[ks][e]));
        amax = wave_max(amax);
        if (lane == 0) s_qmax[wave] = amax;
        __syncthreads();
        const int w0 = (wave / 4) * 4;   // the 4 waves of this 128-row block
        const float m = fmaxf(fmaxf(s_qmax[w0], s_qmax[w0 + 1]), fmaxf(s_qmax[w0 + 2], s_qmax[w0 + 3]));
        const float scale = (m > 0.f) ? m / 127.0f : 1.0f;
        qscale = (qi < a.S) ? scale : 0.f;
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                float qv = rintf(xq[ks][e] / scale);
                qv = fminf(fmaxf(qv, -127.f), 127.f);
                w[e / 4] |= ((uint32_t)((int)qv & 0xff)) << (8 * (e % 4));
            }
            qf[ks] = int32x4_t{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        }
    }

    f32x16_t oacc[DT];
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[tt][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    int32x16_t magic;
#pragma unroll
    for (int e = 0; e < 16; ++e) magic[e] = __float_as_int(kMagic);
    const int wave_last_key = q0 + 31 + diag;
    uint32_t koff[KS8], voff[DT];
#pragma unroll
    for (int ks = 0; ks < KS8; ++ks) koff[ks] = attn_pipe::k8_off(ql, ks * 2 + hh);
#pragma unroll
    for (int tt = 0; tt < DT; ++tt) voff[tt] = (uint32_t)kSPKTile + attn_pipe::v_tr_lane_off(lane, tt);
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
        if (q0 >= a.S) continue;
        const int kb0 = kt * kSPKV;
        if (a.causal && kb0 > wave_last_key) continue;   // the whole tile is above this wave's rows
        const bool two = kb0 + 32 < kv_end && !(a.causal && kb0 + 32 > wave_last_key);   // keys 32..63 needed
        const uint32_t stage = lds0 + (uint32_t)((kt % S) * kSPStage);
        uint32_t ka[KS8], va[DT];
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) ka[ks] = stage + koff[ks];
#pragma unroll
        for (int tt = 0; tt < DT; ++tt) va[tt] = stage + voff[tt];
        // sk is per 128-key block; a 64-key tile lies inside one block
        const float coef = (qscale * a.sk[(kb0 / kSageBlock) * a.Hkv + kvh]) * a.scale_log2;
        const float m_acc = (m_run == -INFINITY) ? 0.f : m_run;
        const float bias = fmaf(kMagic, coef, m_acc);

        // ---- int32 S^T (+ 1.5 * 2^23) for keys 0..31 (acc0) and 32..63 (acc1) of the tile
        int32x4_t kf0[KS8], kf1[KS8];
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) attn_pipe::read_b128<0>(kf0[ks], ka[ks]);
        if (two) {
#pragma unroll
            for (int ks = 0; ks < KS8; ++ks) attn_pipe::read_b128<32 * 128>(kf1[ks], ka[ks]);
            asm volatile("s_waitcnt lgkmcnt(4)" ::: "memory");
        } else {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) asm volatile("" : "+v"(kf0[ks]));
        int32x16_t acc0 = magic, acc1 = magic;
#pragma unroll
        for (int ks = 0; ks < KS8; ++ks) acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf0[ks], qf[ks], acc0, 0, 0, 0);
        if (two) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int ks = 0; ks < KS8; ++ks) asm volatile("" : "+v"(kf1[ks]));
#pragma unroll
            for (int ks = 0; ks < KS8; ++ks) acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf1[ks], qf[ks], acc1, 0, 0, 0);
        }
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

        // s = score * coef - m_acc, in log2 units
        float s0[16], s1[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            s0[e] = fmaf(__int_as_float(acc0[e]), coef, -bias);
            s1[e] = fmaf(__int_as_float(acc1[e]), coef, -bias);   // all masked below when !two
        }
        if (kb0 + kSPKV > kv_end || (a.causal && kb0 + kSPKV - 1 > q0 + diag)) {
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
            mloc = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));   // tile max - m_acc
        }
        // raise m when some row's tile max exceeds it by more than 2^8 (always on the
        // first tile, where m_run = -inf); a real (wave-uniform) branch
        if (__any(m_run == -INFINITY || mloc > kSPLazy)) {
            asm volatile("" ::: "memory");
            const float m_new = fmaxf(m_run, m_acc + mloc);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // 0 on the first tile
            const float shift = m_new - m_acc;
            l_run *= alpha;
#pragma unroll
            for (int tt = 0; tt < DT; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[tt][e] *= alpha;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                s0[e] -= shift;
                s1[e] -= shift;
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
        auto pv = [&](int kb) {
#pragma unroll
            for (int tt = 0; tt < DT; ++tt) {
                asm volatile("" : "+v"(vf[kb][tt][0]), "+v"(vf[kb][tt][1]));
                union {
                    s4_t h[2];
                    bf16x8_t v;
                } vv;
                vv.h[0] = vf[kb][tt][0];
                vv.h[1] = vf[kb][tt][1];
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
    bf16_t* op = a.o + ((size_t)qi * a.Hq + head) * kSPHD;
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

int prefill_cus();
int validate_attention_ctx(const efm_attention_ctx* c, const char* who);

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

struct SageWs {
    size_t q8, k8, sq, sk, km, kp;
    size_t total() const { return q8 + k8 + sq + sk + km + kp; }
};

static SageWs sage_ws(const efm_attention_ctx* c, uint32_t S, uint32_t L) {
    SageWs w;
    const size_t hd = c->head_dim;
    w.q8 = al256((size_t)S * c->num_qo_heads * hd);
    w.k8 = al256((size_t)L * c->num_kv_heads * hd);
    w.sq = al256((size_t)((S + kSageBlock - 1) / kSageBlock) * c->num_qo_heads * 4);
    w.sk = al256((size_t)((L + kSageBlock - 1) / kSageBlock) * c->num_kv_heads * 4);
    w.km = al256((size_t)c->num_kv_heads * hd * 4);
    w.kp = al256((size_t)kKSlices * c->num_kv_heads * hd * 8);
    return w;
}

// kpart == nullptr (efm_sage_quantize): the K mean from one workgroup per (KV head, 8
// channels); else (the attention entry point, whose workspace holds kpart) from row-slice
// sums added up by the quantisation kernel, which also stores the mean in kmean.
static int sage_quantize_impl(const efm_attention_ctx* c, const void* q, const void* k, uint32_t S, uint32_t L,
                              int8_t* q8, float* sq, int8_t* k8, float* sk, float* kmean, hipStream_t stream,
                              bool quant_q = true, double* kpart = nullptr) {
    const int hd = (int)c->head_dim;
    const int q_sn = c->q_stride_n ? (int)c->q_stride_n : (int)(c->num_qo_heads * hd);
    const int q_sh = c->q_stride_h ? (int)c->q_stride_h : hd;
    const int k_sn = c->k_stride_n ? (int)c->k_stride_n : (int)(c->num_kv_heads * hd);
    const int k_sh = c->k_stride_h ? (int)c->k_stride_h : hd;
    if (kpart != nullptr) {
        hipLaunchKernelGGL(sage_kpart_kernel, dim3(c->num_kv_heads, kKSlices), dim3(kSageThreads), 0, stream,
                           static_cast<const bf16_t*>(k), (int)L, k_sn, k_sh, hd, kpart);
    } else {
        hipLaunchKernelGGL(sage_kmean_kernel, dim3(c->num_kv_heads, hd / 8), dim3(kKmeanThreads), 0, stream,
                           static_cast<const bf16_t*>(k), (int)L, k_sn, k_sh, hd, kmean);
    }
    int rc = check_launch("sage kmean");
    if (rc) return rc;
    if (quant_q) {
        hipLaunchKernelGGL(sage_quant_kernel<0>, dim3((S + kSageBlock - 1) / kSageBlock, c->num_qo_heads),
                           dim3(kSageThreads), 0, stream, static_cast<const bf16_t*>(q), (int)S,
                           (int)c->num_qo_heads, q_sn, q_sh, hd, (const float*)nullptr, (const double*)nullptr,
                           (float*)nullptr, q8, sq);
        rc = check_launch("sage quant q");
        if (rc) return rc;
    }
    const dim3 kgrid((L + kSageBlock - 1) / kSageBlock, c->num_kv_heads);
    if (kpart != nullptr)
        hipLaunchKernelGGL(sage_quant_kernel<2>, kgrid, dim3(kSageThreads), 0, stream, static_cast<const bf16_t*>(k),
                           (int)L, (int)c->num_kv_heads, k_sn, k_sh, hd, (const float*)nullptr, (const double*)kpart,
                           kmean, k8, sk);
    else
        hipLaunchKernelGGL(sage_quant_kernel<1>, kgrid, dim3(kSageThreads), 0, stream, static_cast<const bf16_t*>(k),
                           (int)L, (int)c->num_kv_heads, k_sn, k_sh, hd, (const float*)kmean, (const double*)nullptr,
                           (float*)nullptr, k8, sk);
    return check_launch("sage quant k");
}

static int sage_validate(const efm_attention_ctx* c, uint32_t S, uint32_t L) {
    int rc = validate_attention_ctx(c, "sage_attention");
    if (rc) return rc;
    if (c->pos_encoding != EFM_POS_NONE)
        return set_error(EFM_ERR_UNSUPPORTED,
                         "sage_attention: rotate q/k before quantisation (pos_encoding must be NONE)");
    if (L < S) return set_error(EFM_ERR_INVALID_ARGUMENT, "sage_attention: kv_len %u < qo_len %u", L, S);
    if (L == 0 || S > (1u << 20) || L > (1u << 24))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "sage_attention: bad sequence lengths");
    return EFM_OK;
}

}  // namespace efm

using namespace efm;

extern "C" size_t efm_attention_prefill_sage_int8_workspace_bytes(const efm_attention_ctx* ctx, uint32_t qo_len,
                                                                   uint32_t kv_len) {
    if (validate_attention_ctx(ctx, "sage_attention") != EFM_OK) return 0;
    return sage_ws(ctx, qo_len, kv_len).total();
}

extern "C" int efm_sage_quantize(const efm_attention_ctx* ctx, const void* q, const void* k, uint32_t qo_len,
                                 uint32_t kv_len, int8_t* q8, float* q_scales, int8_t* k8, float* k_scales,
                                 float* k_mean, hipStream_t stream) {
    int rc = sage_validate(ctx, qo_len, kv_len);
    if (rc) return rc;
    if (!q || !k || !q8 || !q_scales || !k8 || !k_scales || !k_mean)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "sage_quantize: null pointer");
    if (qo_len == 0) return EFM_OK;
    return sage_quantize_impl(ctx, q, k, qo_len, kv_len, q8, q_scales, k8, k_scales, k_mean, stream);
}

extern "C" int efm_attention_prefill_sage_int8(const efm_attention_ctx* ctx, const void* q, const void* k,
                                               const void* v, void* o, uint32_t qo_len, uint32_t kv_len,
                                               int32_t causal, void* workspace, size_t workspace_bytes,
                                               hipStream_t stream) {
    int rc = sage_validate(ctx, qo_len, kv_len);
    if (rc) return rc;
    if (!q || !k || !v || !o) return set_error(EFM_ERR_INVALID_ARGUMENT, "sage_attention: null tensor pointer");
    if (qo_len == 0) return EFM_OK;
    const SageWs w = sage_ws(ctx, qo_len, kv_len);
    if (workspace == nullptr || workspace_bytes < w.total())
        return set_error(EFM_ERR_WORKSPACE, "sage_attention: workspace of %zu bytes required", w.total());
    char* p = static_cast<char*>(workspace);
    int8_t* q8 = reinterpret_cast<int8_t*>(p);
    int8_t* k8 = reinterpret_cast<int8_t*>(p + w.q8);
    float* sq = reinterpret_cast<float*>(p + w.q8 + w.k8);
    float* sk = reinterpret_cast<float*>(p + w.q8 + w.k8 + w.sq);
    float* km = reinterpret_cast<float*>(p + w.q8 + w.k8 + w.sq + w.sk);
    double* kp = reinterpret_cast<double*>(p + w.q8 + w.k8 + w.sq + w.sk + w.km);
    const int hd = (int)ctx->head_dim;
    const bool pipe = hd == kSPHD && kernel_knob(EFM_KNOB_PREFILL_REGISTER) == 0;
    // the pipelined kernel quantises Q itself (one 128-row block per 4 waves)
    rc = sage_quantize_impl(ctx, q, k, qo_len, kv_len, q8, sq, k8, sk, km, stream, !pipe, kp);
    if (rc) return rc;
    SageArgs a;
    a.q = static_cast<const bf16_t*>(q);
    a.q_sn = ctx->q_stride_n ? (int)ctx->q_stride_n : (int)(ctx->num_qo_heads * hd);
    a.q_sh = ctx->q_stride_h ? (int)ctx->q_stride_h : hd;
    a.q8 = q8;
    a.k8 = k8;
    a.sq = sq;
    a.sk = sk;
    a.v = static_cast<const bf16_t*>(v);
    a.o = static_cast<bf16_t*>(o);
    a.S = (int)qo_len;
    a.L = (int)kv_len;
    a.Hq = (int)ctx->num_qo_heads;
    a.Hkv = (int)ctx->num_kv_heads;
    a.v_sn = ctx->kv_stride_n ? (int)ctx->kv_stride_n : a.Hkv * hd;
    a.v_sh = ctx->kv_stride_h ? (int)ctx->kv_stride_h : hd;
    a.causal = causal != 0;
    a.scale_log2 = (float)(1.4426950408889634 / sqrt((double)hd));
    if (pipe) {
        // as the bf16 kernel: 8 waves over a 4-deep ring when those workgroups fill the
        // chip, else 4 waves / two workgroups per CU (a 3-deep ring of 24 KB stages fits twice)
        const int shape = kernel_knob(EFM_KNOB_PREFILL_SHAPE);
        const bool small = shape != 0 ? shape <= 4 : (int)((qo_len + 255) / 256) * a.Hq < prefill_cus();
        if (small) {
            const int nqt = (int)((qo_len + 127) / 128);
            hipLaunchKernelGGL((sage_attn_pipe_kernel<4, 3>), dim3(nqt * a.Hq), dim3(256), 0, stream, a, nqt);
        } else {
            const int nqt = (int)((qo_len + 255) / 256);
            hipLaunchKernelGGL((sage_attn_pipe_kernel<8, 4>), dim3(nqt * a.Hq), dim3(512), 0, stream, a, nqt);
        }
        return check_launch("sage_attention");
    }
    dim3 grid((qo_len + kSageQ - 1) / kSageQ, a.Hq), block(kSageThreads);
    if (hd == 128) hipLaunchKernelGGL(sage_attn_kernel<128>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(sage_attn_kernel<64>, grid, block, 0, stream, a);
    return check_launch("sage_attention");
}

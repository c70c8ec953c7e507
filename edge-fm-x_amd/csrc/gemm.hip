// Prefill projections on the gfx950 matrix cores: C[M, N] = A[M, K] . B[N, K]^T in
// bf16 with fp32 accumulation (v_mfma_f32_32x32x16_bf16). A holds activations (one
// row per token) and B the weights in their [out, in] layout, so both operands are
// K-contiguous and feed the MFMA lanes with plain 16-byte loads.
//
//  * Workgroup tile BM x BN x 32, 256 threads as a 2 x 2 grid of wave64s; each wave
//    owns a (BM/2) x (BN/2) block of 32 x 32 MFMA tiles.
//  * Global -> register prefetch of the next K slab overlaps the MFMAs of the current
//    one; slabs are double-buffered in LDS with a padded row pitch (40 bf16) so the
//    32 rows read by one MFMA operand fetch spread over the LDS banks.
//  * Epilogues: bf16 (+bias, the cuBLASLt BIAS epilogue), fp32, and SwiGLU, where the
//    B tile interleaves 32-row blocks of up and gate weights so that each lane holds u
//    and g of the same output element: out = bf16(silu(bf16(g)) * bf16(u)).
#include "common.hpp"

#include <algorithm>

namespace efm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

enum { GEPI_BF16 = 0, GEPI_F32 = 1, GEPI_SWIGLU = 2 };

constexpr int kGemmThreads = 256;
constexpr int kBK = 32;
constexpr int kPitch = kBK + 8;  // LDS row pitch in bf16

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(kGemmThreads) void gemm_bf16_kernel(const bf16_t* __restrict__ A,
                                                                 const bf16_t* __restrict__ B,
                                                                 const bf16_t* __restrict__ bias, void* __restrict__ Cout,
                                                                 int M, int N, int K, int ldc) {
    constexpr int WM = BM / 2, WN = BN / 2;        // wave tile
    constexpr int TM = WM / 32, TN = WN / 32;      // MFMA tiles per wave
    constexpr int ACH = BM * kBK / 8;              // 16-byte chunks per A slab
    constexpr int BCH = BN * kBK / 8;
    constexpr int AL = (ACH + kGemmThreads - 1) / kGemmThreads;
    constexpr int BL = (BCH + kGemmThreads - 1) / kGemmThreads;
    static_assert(TM >= 1 && TN >= 1, "tile too small");
    static_assert(EPI != GEPI_SWIGLU || TN % 2 == 0, "SwiGLU needs paired N tiles");

    __shared__ __align__(16) bf16_t As[2][BM * kPitch];
    __shared__ __align__(16) bf16_t Bs[2][BN * kPitch];

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int wm = wave / 2, wn = wave % 2;
    const int m0 = blockIdx.x * BM;
    // For SwiGLU the output tile is BN/2 columns wide; B rows interleave 32-row blocks
    // of up (even blocks) and gate (odd blocks) weights.
    const int n0 = (EPI == GEPI_SWIGLU) ? blockIdx.y * (BN / 2) : blockIdx.y * BN;

    auto b_row = [&](int r) -> int {
        if (EPI == GEPI_SWIGLU) {
            const int blk = r / 32;
            const int col = n0 + (blk / 2) * 32 + (r % 32);
            return (col < N) ? ((blk % 2 == 0) ? col : N + col) : -1;
        }
        const int n = n0 + r;
        return (n < N) ? n : -1;
    };

    uint4 ra[AL], rb[BL];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int c = tid + i * kGemmThreads;
            const int r = c / (kBK / 8), kc = c % (kBK / 8);
            ra[i] = (c < ACH && m0 + r < M) ? *reinterpret_cast<const uint4*>(A + (size_t)(m0 + r) * K + k0 + kc * 8)
                                            : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const int c = tid + i * kGemmThreads;
            const int r = c / (kBK / 8), kc = c % (kBK / 8);
            const int br = (c < BCH) ? b_row(r) : -1;
            rb[i] = (br >= 0) ? load_stream16(B + (size_t)br * K + k0 + kc * 8) : make_uint4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; ++i) {
            const int c = tid + i * kGemmThreads;
            if (c < ACH) {
                const int r = c / (kBK / 8), kc = c % (kBK / 8);
                *reinterpret_cast<uint4*>(&As[buf][r * kPitch + kc * 8]) = ra[i];
            }
        }
#pragma unroll
        for (int i = 0; i < BL; ++i) {
            const int c = tid + i * kGemmThreads;
            if (c < BCH) {
                const int r = c / (kBK / 8), kc = c % (kBK / 8);
                *reinterpret_cast<uint4*>(&Bs[buf][r * kPitch + kc * 8]) = rb[i];
            }
        }
    };

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int nk = K / kBK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
            bf16x8_t af[TM], bfr[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int r = wm * WM + i * 32 + (lane % 32);
                af[i] = *reinterpret_cast<const bf16x8_t*>(&As[buf][r * kPitch + ks * 16 + (lane / 32) * 8]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int r = wn * WN + j * 32 + (lane % 32);
                bfr[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[buf][r * kPitch + ks * 16 + (lane / 32) * 8]);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) {
            lstore(buf ^ 1);
        }
        __syncthreads();
    }

    // Epilogue. Accumulator element e of tile (i, j): row = (e/4)*8 + (lane/32)*4 + e%4,
    // column = lane % 32 within the 32 x 32 tile.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int row = m0 + wm * WM + i * 32 + (e / 4) * 8 + (lane / 32) * 4 + (e % 4);
            if (row >= M) continue;
            if (EPI == GEPI_SWIGLU) {
#pragma unroll
                for (int j = 0; j < TN; j += 2) {
                    const int col = n0 + ((wn * WN + j * 32) / 64) * 32 + (lane % 32);
                    if (col < N) {
                        const float u = round_bf16(acc[i][j][e]);
                        const float g = round_bf16(acc[i][j + 1][e]);
                        const float o = (g / (1.0f + expf(-g))) * u;
                        reinterpret_cast<bf16_t*>(Cout)[(size_t)row * ldc + col] = (bf16_t)f32_to_bf16(o);
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int col = n0 + wn * WN + j * 32 + (lane % 32);
                    if (col >= N) continue;
                    float v = acc[i][j][e];
                    if (bias != nullptr) v += bf16_to_f32(bias[col]);
                    if (EPI == GEPI_F32) reinterpret_cast<float*>(Cout)[(size_t)row * ldc + col] = v;
                    else reinterpret_cast<bf16_t*>(Cout)[(size_t)row * ldc + col] = (bf16_t)f32_to_bf16(v);
                }
            }
        }
    }
}

template <int EPI>
static int gemm_dispatch(int M, int N, int K, const bf16_t* A, const bf16_t* B, const bf16_t* bias, void* C, int ldc,
                         hipStream_t stream) {
    // Output columns per tile: BN (SwiGLU: BN / 2).
    auto tiles = [&](int bm, int bn) {
        const int ocols = (EPI == GEPI_SWIGLU) ? bn / 2 : bn;
        return (long)((M + bm - 1) / bm) * ((N + ocols - 1) / ocols);
    };
    const dim3 block(kGemmThreads);
    if (tiles(128, 128) >= 256) {
        const int oc = (EPI == GEPI_SWIGLU) ? 64 : 128;
        dim3 grid((M + 127) / 128, (N + oc - 1) / oc);
        hipLaunchKernelGGL((gemm_bf16_kernel<128, 128, EPI>), grid, block, 0, stream, A, B, bias, C, M, N, K, ldc);
    } else {
        if constexpr (EPI == GEPI_SWIGLU) {
            dim3 grid((M + 63) / 64, (N + 63) / 64);
            hipLaunchKernelGGL((gemm_bf16_kernel<64, 128, EPI>), grid, block, 0, stream, A, B, bias, C, M, N, K, ldc);
        } else {
            dim3 grid((M + 63) / 64, (N + 63) / 64);
            hipLaunchKernelGGL((gemm_bf16_kernel<64, 64, EPI>), grid, block, 0, stream, A, B, bias, C, M, N, K, ldc);
        }
    }
    return check_launch("gemm_bf16");
}

static int gemm_check(int64_t M, int64_t N, int64_t K, const void* A, const void* B, const void* C) {
    if (A == nullptr || B == nullptr || C == nullptr) return set_error(EFM_ERR_INVALID_ARGUMENT, "gemm: null pointer");
    if (K <= 0 || K % kBK != 0)
        return set_error(EFM_ERR_UNSUPPORTED, "gemm: in_features must be a positive multiple of %d (got %lld)", kBK,
                         (long long)K);
    if (M > 0x7fffffff / 2 || N > 0x7fffffff / 2 || K > 0x7fffffff / 2)
        return set_error(EFM_ERR_UNSUPPORTED, "gemm: shape too large");
    if ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15u)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "gemm: operands must be 16-byte aligned");
    return EFM_OK;
}

int gemm_bf16(int64_t M, int64_t N, int64_t K, const void* A, const void* B, const void* bias, void* C,
              int32_t out_dtype, hipStream_t stream) {
    int rc = gemm_check(M, N, K, A, B, C);
    if (rc) return rc;
    if (M == 0 || N == 0) return EFM_OK;
    const bf16_t* a = static_cast<const bf16_t*>(A);
    const bf16_t* b = static_cast<const bf16_t*>(B);
    const bf16_t* bi = static_cast<const bf16_t*>(bias);
    if (out_dtype == EFM_DTYPE_BF16) return gemm_dispatch<GEPI_BF16>((int)M, (int)N, (int)K, a, b, bi, C, (int)N, stream);
    if (out_dtype == EFM_DTYPE_F32) return gemm_dispatch<GEPI_F32>((int)M, (int)N, (int)K, a, b, bi, C, (int)N, stream);
    return set_error(EFM_ERR_UNSUPPORTED, "linear: output dtype %d not supported", out_dtype);
}

int gemm_swiglu(int64_t M, int64_t inter, int64_t K, const void* A, const void* W, void* out, hipStream_t stream) {
    int rc = gemm_check(M, inter, K, A, W, out);
    if (rc) return rc;
    if (M == 0) return EFM_OK;
    return gemm_dispatch<GEPI_SWIGLU>((int)M, (int)inter, (int)K, static_cast<const bf16_t*>(A),
                                      static_cast<const bf16_t*>(W), nullptr, out, (int)inter, stream);
}

}  // namespace efm

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
#include <type_traits>
#include <cstdlib>

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

// ---------------------------------------------------------------------------------
// Pipelined variant for K % 64 == 0: K slabs of 64 stream global -> LDS with
// global_load_lds (no staging registers) into an S-deep ring, so S - 1 slabs are in
// flight while the matrix cores work on one. Each wave's 1 KB DMA load covers 8 rows x 128
// bytes; lane l fetches chunk (l % 8) ^ (row % 8) of its row, so the ring holds an
// XOR-swizzled layout and the 32-row MFMA operand reads spread over the LDS banks. The
// operand reads are issued as ds_read_b128 with explicit waits: each wave waits for its
// own DMA loads of the slab (vmcnt, counted exactly: every wave issues LPW loads per slab)
// and a workgroup barrier makes all waves' loads visible. Tiles are assigned XCD by XCD
// (dispatch is round-robin over the 8 XCDs), so workgroups that share weight columns
// share an L2.
// ---------------------------------------------------------------------------------
constexpr int kPBK = 64;            // K per slab
constexpr int kPRow = kPBK * 2;     // bytes per operand row in LDS

template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int LPW>
__device__ __forceinline__ void vm_wait_slabs(int slabs) {
    switch (slabs) {
        case 0: vm_wait<0>(); break;
        case 1: vm_wait<1 * LPW>(); break;
        case 2: vm_wait<2 * LPW>(); break;
        case 3: vm_wait<3 * LPW>(); break;
        case 4: vm_wait<4 * LPW>(); break;
        case 5: vm_wait<5 * LPW>(); break;
        default: vm_wait<6 * LPW>(); break;
    }
}

template <int BM, int BN, int S, int EPI>
__global__ __launch_bounds__(kGemmThreads) void gemm_pipe_kernel(const bf16_t* __restrict__ A,
                                                                 const bf16_t* __restrict__ B,
                                                                 const bf16_t* __restrict__ bias,
                                                                 void* __restrict__ Cout, int M, int N, int K, int ldc,
                                                                 int mt, int nt) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int STAGE = (BM + BN) * kPRow;
    constexpr int QA = BM / 8, QB = BN / 8;  // 1 KB wave loads per operand per slab
    constexpr int LPW = (QA + QB) / 4;       // wave loads per wave per slab
    static_assert((QA + QB) % 4 == 0 && S >= 2 && S <= 8 && (S - 2) * LPW <= 63, "bad pipeline shape");
    static_assert(EPI != GEPI_SWIGLU || TN % 2 == 0, "SwiGLU needs paired N tiles");
    __shared__ __align__(1024) unsigned char smem[S * STAGE];

    const int T = mt * nt;
    const int per = (T + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (t >= T) return;
    const int tm = t % mt, tn = t / mt;
    const int m0 = tm * BM;
    const int n0 = (EPI == GEPI_SWIGLU) ? tn * (BN / 2) : tn * BN;

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int wm = wave / 2, wn = wave % 2;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);

    auto b_row = [&](int r) -> int {
        if (EPI == GEPI_SWIGLU) {
            const int blk = r / 32;
            const int col = n0 + (blk / 2) * 32 + (r % 32);
            return (col < N) ? ((blk % 2 == 0) ? col : N + col) : -1;
        }
        const int n = n0 + r;
        return (n < N) ? n : -1;
    };

    auto issue = [&](int kk, int slot) {
        const int k0 = kk * kPBK;
        const int rr = lane >> 3, cs = lane & 7;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int q = wave + i * 4;
            const bf16_t* src;
            if (q < QA) {
                const int row = min(m0 + q * 8 + rr, M - 1);
                src = A + (size_t)row * K + k0 + ((cs ^ rr) << 3);
            } else {
                int br = b_row((q - QA) * 8 + rr);
                if (br < 0) br = 0;
                src = B + (size_t)br * K + k0 + ((cs ^ rr) << 3);
            }
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src),
                (__attribute__((address_space(3))) void*)(smem + slot * STAGE + q * 1024), 16, 0, 0);
        }
    };

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    auto compute = [&](int slot) {
        const uint32_t base = lds0 + (uint32_t)(slot * STAGE);
        constexpr int KSN = kPBK / 16;
        bf16x8_t af[KSN][TM], bfr[KSN][TN];
        // all operand reads of the slab first (one LDS latency per slab), then the MFMAs
#pragma unroll
        for (int ks = 0; ks < KSN; ++ks) {
            const int c = ks * 2 + (lane >> 5);
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int r = wm * WM + i * 32 + (lane & 31);
                const uint32_t addr = base + (uint32_t)(r * kPRow + ((c ^ (r & 7)) << 4));
                asm volatile("ds_read_b128 %0, %1" : "=v"(af[ks][i]) : "v"(addr) : "memory");
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int r = wn * WN + j * 32 + (lane & 31);
                const uint32_t addr = base + (uint32_t)(BM * kPRow + r * kPRow + ((c ^ (r & 7)) << 4));
                asm volatile("ds_read_b128 %0, %1" : "=v"(bfr[ks][j]) : "v"(addr) : "memory");
            }
        }
        // The fragments come from inline-asm reads the compiler cannot track: wait for
        // them, then pass every fragment through an asm "write" so that no MFMA can be
        // scheduled above the wait.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int ks = 0; ks < KSN; ++ks) {
#pragma unroll
            for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[ks][i]));
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bfr[ks][j]));
        }
#pragma unroll
        for (int ks = 0; ks < KSN; ++ks)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][i], bfr[ks][j], acc[i][j], 0, 0, 0);
    };

    const int nk = K / kPBK;
    const int pre = min(S - 1, nk);
    for (int p = 0; p < pre; ++p) issue(p, p);
    for (int kt = 0; kt < nk; ++kt) {
        // Own DMA loads of slab kt have landed in LDS; the bare barrier (no fence, which
        // would drain every slab in flight) then orders them before all waves' reads, and
        // all waves' reads of slot (kt - 1) % S before it is refilled below.
        vm_wait_slabs<LPW>(min(S - 2, nk - 1 - kt));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
        compute(kt % S);
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

template <int BM, int BN, int S, int EPI>
static void gemm_pipe_launch(int M, int N, int K, const bf16_t* A, const bf16_t* B, const bf16_t* bias, void* C,
                             int ldc, hipStream_t stream) {
    const int ocols = (EPI == GEPI_SWIGLU) ? BN / 2 : BN;
    const int mt = (M + BM - 1) / BM, nt = (N + ocols - 1) / ocols;
    const int grid = 8 * ((mt * nt + 7) / 8);
    hipLaunchKernelGGL((gemm_pipe_kernel<BM, BN, S, EPI>), dim3(grid), dim3(kGemmThreads), 0, stream, A, B, bias, C,
                       M, N, K, ldc, mt, nt);
}

// ---------------------------------------------------------------------------------
// Large-tile variant: 256 x 256 output tile per workgroup, 4 waves in a 2 x 2 grid and
// 128 x 128 (4 x 4 MFMA tiles, 256 accumulator registers) per wave, so that each 16-key
// MFMA step issues 16 MFMAs for 8 ds_read_b128 operand reads (the 128 x 128 tile issues
// one read per MFMA and is bound by LDS bandwidth). K slabs of 32 stream global -> LDS
// with global_load_lds into a 4-deep ring (32 KB per slab); each wave load covers 16 rows
// x 64 bytes and lane l fetches chunk (l % 4) ^ ((row >> 2) & 3) of its row, so the 16
// rows read by one operand fetch phase hit distinct LDS banks.
// ---------------------------------------------------------------------------------
constexpr int kBBK = 32;            // K per slab
constexpr int kBRow = kBBK * 2;     // bytes per operand row in LDS

template <int LPW>
__device__ __forceinline__ void vm_wait_big(int slabs) {
    switch (slabs) {
        case 0: vm_wait<0>(); break;
        case 1: vm_wait<1 * LPW>(); break;
        default: vm_wait<2 * LPW>(); break;
    }
}

template <int S, int EPI>
__global__ __launch_bounds__(kGemmThreads) void gemm_big_kernel(const bf16_t* __restrict__ A,
                                                                const bf16_t* __restrict__ B,
                                                                const bf16_t* __restrict__ bias,
                                                                void* __restrict__ Cout, int M, int N, int K, int ldc,
                                                                int mt, int nt) {
    constexpr int BM = 256, BN = 256;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int STAGE = (BM + BN) * kBRow;
    constexpr int QA = BM / 16, QB = BN / 16;   // 1 KB wave loads per operand per slab
    constexpr int LPW = (QA + QB) / 4;
    static_assert(S >= 2 && S <= 4 && (S - 2) * LPW <= 63, "bad pipeline shape");
    __shared__ __align__(1024) unsigned char smem[S * STAGE];

    const int T = mt * nt;
    const int per = (T + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (t >= T) return;
    const int tm = t % mt, tn = t / mt;
    const int m0 = tm * BM;
    const int n0 = (EPI == GEPI_SWIGLU) ? tn * (BN / 2) : tn * BN;

    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int wm = wave / 2, wn = wave % 2;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);

    auto b_row = [&](int r) -> int {
        if (EPI == GEPI_SWIGLU) {
            const int blk = r / 32;
            const int col = n0 + (blk / 2) * 32 + (r % 32);
            return (col < N) ? ((blk % 2 == 0) ? col : N + col) : -1;
        }
        const int n = n0 + r;
        return (n < N) ? n : -1;
    };

    // Per-lane source offsets (elements) of the wave loads are fixed for the whole kernel.
    const int rr = lane >> 2, cs = lane & 3;
    uint32_t srcoff[LPW];
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
        const int q = wave + i * 4;
        if (q < QA) {
            const int row = q * 16 + rr;
            srcoff[i] = (uint32_t)min(m0 + row, M - 1) * (uint32_t)K + ((cs ^ ((row >> 2) & 3)) << 3);
        } else {
            const int row = (q - QA) * 16 + rr;
            int br = b_row(row);
            if (br < 0) br = 0;
            srcoff[i] = (uint32_t)br * (uint32_t)K + ((cs ^ ((row >> 2) & 3)) << 3);
        }
    }
    auto issue = [&](int kk, int slot) {
        const int k0 = kk * kBBK;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int q = wave + i * 4;
            const bf16_t* src = (q < QA ? A : B) + srcoff[i] + k0;
            __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                             (__attribute__((address_space(3))) void*)(smem + slot * STAGE + q * 1024),
                                             16, 0, 0);
        }
    };

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    // lane parts of the operand addresses: row (lane & 31) of the first 32-row tile, chunk
    // 2 ks + (lane >> 5) swizzled by ((row >> 2) & 3); the other tiles are 32 rows
    // (2048 bytes) further and share the swizzle, so their offsets are immediates
    uint32_t aoff[2], boff[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int c = ks * 2 + (lane >> 5);
        const int ra = wm * WM + (lane & 31), rb = wn * WN + (lane & 31);
        aoff[ks] = (uint32_t)(ra * kBRow + ((c ^ ((ra >> 2) & 3)) << 4));
        boff[ks] = (uint32_t)(BM * kBRow + rb * kBRow + ((c ^ ((rb >> 2) & 3)) << 4));
    }

    auto compute = [&](int slot) {
        const uint32_t base = lds0 + (uint32_t)(slot * STAGE);
        bf16x8_t af[2][TM], bfr[2][TN];
        auto rd = [&](auto ic, bf16x8_t& dst, uint32_t addr) {
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "n"(decltype(ic)::value * 32 * kBRow)
                         : "memory");
        };
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const uint32_t a0 = base + aoff[ks], b0 = base + boff[ks];
            rd(std::integral_constant<int, 0>{}, af[ks][0], a0);
            rd(std::integral_constant<int, 1>{}, af[ks][1], a0);
            rd(std::integral_constant<int, 2>{}, af[ks][2], a0);
            rd(std::integral_constant<int, 3>{}, af[ks][3], a0);
            rd(std::integral_constant<int, 0>{}, bfr[ks][0], b0);
            rd(std::integral_constant<int, 1>{}, bfr[ks][1], b0);
            rd(std::integral_constant<int, 2>{}, bfr[ks][2], b0);
            rd(std::integral_constant<int, 3>{}, bfr[ks][3], b0);
        }
        // k-step 0's 8 reads were issued first: wait for them, then the second 8
        asm volatile("s_waitcnt lgkmcnt(8)" ::: "memory");
#pragma unroll
        for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[0][i]));
#pragma unroll
        for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bfr[0][j]));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0][i], bfr[0][j], acc[i][j], 0, 0, 0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[1][i]));
#pragma unroll
        for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bfr[1][j]));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[1][i], bfr[1][j], acc[i][j], 0, 0, 0);
    };

    const int nk = K / kBBK;
    const int pre = min(S - 1, nk);
    for (int p = 0; p < pre; ++p) issue(p, p);
    for (int kt = 0; kt < nk; ++kt) {
        vm_wait_big<LPW>(min(S - 2, nk - 1 - kt));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kt + S - 1 < nk) issue(kt + S - 1, (kt + S - 1) % S);
        compute(kt % S);
    }

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
static void gemm_big_launch(int M, int N, int K, const bf16_t* A, const bf16_t* B, const bf16_t* bias, void* C,
                            int ldc, hipStream_t stream) {
    const int ocols = (EPI == GEPI_SWIGLU) ? 128 : 256;
    const int mt = (M + 255) / 256, nt = (N + ocols - 1) / ocols;
    const int grid = 8 * ((mt * nt + 7) / 8);
    hipLaunchKernelGGL((gemm_big_kernel<4, EPI>), dim3(grid), dim3(kGemmThreads), 0, stream, A, B, bias, C, M, N, K,
                       ldc, mt, nt);
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
    const char* big_env = getenv("EFM_GEMM_BIG");
    const bool big_ok = big_env == nullptr || big_env[0] != '0';
    if (K % kPBK == 0) {
        // Tile choice from a sweep of the prefill shapes on MI355X: the 256 x 256 tile
        // once there are >= 3 tiles per CU; else 128 x 128 double-buffered (two workgroups
        // per CU), which needs >= 1.5 tiles per CU (>= 1 for SwiGLU); else 128 x 64
        // double-buffered; else 64 x 64 (or 64 x 128 for SwiGLU) with shallow pipelines.
        // Every tile shape sums each output over K in the same order: results are
        // bit-identical whichever is chosen.
        if (big_ok && tiles(256, 256) >= 768) {
            gemm_big_launch<EPI>(M, N, K, A, B, bias, C, ldc, stream);
        } else if (tiles(128, 128) >= ((EPI == GEPI_SWIGLU) ? 256 : 384)) {
            gemm_pipe_launch<128, 128, 2, EPI>(M, N, K, A, B, bias, C, ldc, stream);
        } else if constexpr (EPI == GEPI_SWIGLU) {
            gemm_pipe_launch<64, 128, 3, EPI>(M, N, K, A, B, bias, C, ldc, stream);
        } else {
            if (tiles(128, 64) >= 256) gemm_pipe_launch<128, 64, 2, EPI>(M, N, K, A, B, bias, C, ldc, stream);
            else gemm_pipe_launch<64, 64, 4, EPI>(M, N, K, A, B, bias, C, ldc, stream);
        }
        return check_launch("gemm_bf16");
    }
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

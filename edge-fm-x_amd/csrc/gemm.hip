// Prefill projections on the gfx950 matrix cores: C[M, N] = A[M, K] . B[N, K]^T in
// bf16 with fp32 accumulation (v_mfma_f32_32x32x16_bf16). A holds activations (one
// row per token) and B the weights in their [out, in] layout, so both operands are
// K-contiguous and feed the MFMA lanes with 16-byte loads.
//
//  * K % 64 == 0 (every Qwen2.5 projection), two kernels fed by global_load_lds DMA into
//    XOR-swizzled LDS rings, operand reads software-pipelined against the MFMAs and a
//    grouped tile order per XCD:
//      - the wide kernel: 256 x 256 tiles, one 8-wave workgroup per CU (large M);
//      - the pipelined kernel: 128 x 128 (128 x 64, 64 x 64) tiles, two 4-wave
//        workgroups per CU (few tiles), plus its split-K form.
//    A cost model (rounds of resident workgroups) picks between them.
//  * Other K: a register-staged kernel with a padded LDS row pitch (40 bf16).
//  * Epilogues: bf16 (+bias, the cuBLASLt BIAS epilogue), fp32, and SwiGLU, where the
//    B tile interleaves 32-row blocks of up and gate weights so that each lane holds u
//    and g of the same output element: out = bf16(silu(bf16(g)) * bf16(u)).
//  * Every kernel sums each output's keys 16 at a time in increasing order, so results
//    are bit-identical across kernels and tile shapes (split-K aside).
#include "common.hpp"

#include <algorithm>
#include <type_traits>
#include <utility>
#include <cstdlib>

namespace efm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

enum { GEPI_BF16 = 0, GEPI_F32 = 1, GEPI_SWIGLU = 2, GEPI_PARTIAL = 3 };

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
                        const float o = silu_f32(g) * u;
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
// bytes; lane l fetches chunk (l % 8) ^ pipe_swz(row) of its row, so the ring holds an
// XOR-swizzled layout and the 32-row MFMA operand reads spread over the LDS banks. The
// operand reads are issued as ds_read_b128 with explicit waits: each wave waits for its
// own DMA loads of the slab (vmcnt, counted exactly: every wave issues LPW loads per slab)
// and a workgroup barrier makes all waves' loads visible. Tiles are assigned XCD by XCD
// (dispatch is round-robin over the 8 XCDs), so workgroups that share weight columns
// share an L2.
// ---------------------------------------------------------------------------------
// Tile order within one XCD's contiguous range of tile indices: groups of kGroupM row
// tiles are walked column by column, so the workgroups resident on an XCD at one time
// cover a kGroupM x (resident / kGroupM) block of output tiles and share its A and B
// slabs in that XCD's L2 (walking M first, as a plain index split does, re-reads a fresh
// A slab for every tile once M spans many tiles).
constexpr int kGroupM = 8;
__device__ __forceinline__ void tile_of(int t, int mt, int nt, int& tm, int& tn) {
    const int in_group = kGroupM * nt;
    const int first = (t / in_group) * kGroupM;
    const int gm = min(mt - first, kGroupM);
    const int r = t % in_group;
    tm = first + r % gm;
    tn = r / gm;
}

// LDS swizzles. gfx950's LDS has 64 four-byte banks and serves a ds_read_b128 sixteen
// lanes at a time: the 16 rows an MFMA operand read touches at once must land in 16
// distinct 16-byte bank groups. With 128-byte rows (8 chunks) two rows fill the 256-byte
// bank period, so rows of equal parity need distinct chunks: (row / 2) % 8, with the
// parity folded into bit 2 so that any 8 consecutive rows also differ. With 64-byte rows
// (4 chunks) four rows fill the period: rows equal mod 4 need distinct chunks.
__device__ __forceinline__ int pipe_swz(int row) { return ((row >> 1) ^ ((row & 1) << 2)) & 7; }
__device__ __forceinline__ int wide_swz(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }

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
                                                                 int mt, int nt, int ksplit, int kt_per) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int STAGE = (BM + BN) * kPRow;
    constexpr int QA = BM / 8, QB = BN / 8;  // 1 KB wave loads per operand per slab
    constexpr int LPW = (QA + QB) / 4;       // wave loads per wave per slab
    static_assert((QA + QB) % 4 == 0 && S >= 2 && S <= 8 && (S - 2) * LPW <= 63, "bad pipeline shape");
    static_assert(EPI != GEPI_SWIGLU || TN % 2 == 0, "SwiGLU needs paired N tiles");
    __shared__ __align__(1024) unsigned char smem[S * STAGE];

    // split-K (GEPI_PARTIAL): work unit t covers K slice t / (mt * nt), slabs
    // [slice * kt_per, (slice + 1) * kt_per), and writes fp32 partial sums
    const int T = mt * nt * ksplit;
    const int per = (T + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (t >= T) return;
    const int slice = t / (mt * nt);
    int tm, tn;
    tile_of(t % (mt * nt), mt, nt, tm, tn);
    const int kt0 = slice * kt_per;
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
        const int k0 = (kt0 + kk) * kPBK;
        const int rr = lane >> 3, cs = lane & 7;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            const int q = wave + i * 4;
            const bf16_t* src;
            if (q < QA) {
                const int row = min(m0 + q * 8 + rr, M - 1);
                src = A + (size_t)row * K + k0 + ((cs ^ pipe_swz(q * 8 + rr)) << 3);
            } else {
                int br = b_row((q - QA) * 8 + rr);
                if (br < 0) br = 0;
                src = B + (size_t)br * K + k0 + ((cs ^ pipe_swz(q * 8 + rr)) << 3);
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

    // Operand reads of one 16-key step: TM A fragments and TN B fragments (ds_read_b128).
    auto read_step = [&](uint32_t base, int ks, bf16x8_t (&af)[TM], bf16x8_t (&bfr)[TN]) {
        const int c = ks * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int r = wm * WM + i * 32 + (lane & 31);
            const uint32_t addr = base + (uint32_t)(r * kPRow + ((c ^ pipe_swz(r)) << 4));
            asm volatile("ds_read_b128 %0, %1" : "=v"(af[i]) : "v"(addr) : "memory");
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int r = wn * WN + j * 32 + (lane & 31);
            const uint32_t addr = base + (uint32_t)(BM * kPRow + r * kPRow + ((c ^ pipe_swz(r)) << 4));
            asm volatile("ds_read_b128 %0, %1" : "=v"(bfr[j]) : "v"(addr) : "memory");
        }
    };
    // Software pipeline over the slab's four 16-key steps: the reads of step ks + 2 are
    // issued behind the MFMAs of step ks, so LDS latency hides behind matrix work within
    // the wave. The fragments come from inline-asm reads the compiler cannot track: each
    // step waits for its own reads (lgkmcnt = the reads issued after them), then passes
    // its fragments through an asm "write" so that no MFMA is scheduled above the wait.
    auto compute = [&](int slot) {
        const uint32_t base = lds0 + (uint32_t)(slot * STAGE);
        constexpr int KSN = kPBK / 16;
        constexpr int RPS = TM + TN;   // reads per step
        static_assert(RPS <= 15, "lgkmcnt holds at most 15 outstanding reads");
        bf16x8_t af[KSN][TM], bfr[KSN][TN];
        read_step(base, 0, af[0], bfr[0]);
        read_step(base, 1, af[1], bfr[1]);
#pragma unroll
        for (int ks = 0; ks < KSN; ++ks) {
            if (ks + 1 < KSN) asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(RPS) : "memory");
            else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(af[ks][i]));
#pragma unroll
            for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(bfr[ks][j]));
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks][i], bfr[ks][j], acc[i][j], 0, 0, 0);
            if (ks + 2 < KSN) read_step(base, ks + 2, af[ks + 2], bfr[ks + 2]);
        }
    };

    const int nk = min(K / kPBK, kt0 + kt_per) - kt0;
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
                        const float o = silu_f32(g) * u;
                        reinterpret_cast<bf16_t*>(Cout)[(size_t)row * ldc + col] = (bf16_t)f32_to_bf16(o);
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int col = n0 + wn * WN + j * 32 + (lane % 32);
                    if (col >= N) continue;
                    float v = acc[i][j][e];
                    if (EPI == GEPI_PARTIAL) {
                        reinterpret_cast<float*>(Cout)[((size_t)slice * M + row) * N + col] = v;
                        continue;
                    }
                    if (bias != nullptr) v += bf16_to_f32(bias[col]);
                    if (EPI == GEPI_F32) reinterpret_cast<float*>(Cout)[(size_t)row * ldc + col] = v;
                    else reinterpret_cast<bf16_t*>(Cout)[(size_t)row * ldc + col] = (bf16_t)f32_to_bf16(v);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------
// Wide-tile kernel: BM x BN workgroup tiles (256 x 256 in use), one workgroup per CU, its
// WGM x WGN waves (2 x 4 in use: two per SIMD) each owning a (BM/WGM) x (BN/WGN) block of
// 32 x 32 MFMA tiles. Relative to 128 x 128 tiles each MFMA needs half the bytes from L2
// and, with 128 x 64 wave blocks, three quarters of the LDS reads; the second wave on
// each SIMD issues MFMAs while the first waits on its memory instructions. (Measured on
// the 7B gate/up shape: 4 waves with 128 x 128 blocks and 256 AGPR accumulators reach
// 1.08 PF/s, the 2 x 4 layout 1.16 PF/s; the per-stage DMA is the largest cost beyond
// the MFMAs themselves, about a quarter of the time, whether or not its loads hit L2.)
//  * 32-key stages in an S-deep LDS ring filled by global_load_lds (16 bytes per lane,
//    one 1 KB wave load covers 16 rows x 64 bytes). Lane i of a wave load lands at byte
//    16 i of its 1 KB block, so the lane fetches the chunk that belongs there: row i / 4,
//    logical chunk (i % 4) ^ wide_swz(row).
//  * Per stage and wave: two 16-key steps. Step 0's MFMAs run with step 1's operand reads
//    and the DMA of stage s + S - 1 interleaved, one memory instruction per MFMA; step 1's
//    MFMAs run with the reads of stage s + 1's step 0, behind a bare barrier that follows
//    this wave's own vmcnt wait for stage s + 1. That barrier also orders every wave's
//    reads of stage s - 1 before its slot is refilled in the next stage.
// ---------------------------------------------------------------------------------
constexpr int kWBK = 32;            // keys per stage
constexpr int kWRow = kWBK * 2;     // bytes per operand row per stage

template <int OFF>
__device__ __forceinline__ bf16x8_t ds_read16(uint32_t addr) {
    bf16x8_t d;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "n"(OFF) : "memory");
    return d;
}

// One key step's operand fragments: A rows at a + 2048 i, B rows at b + 2048 j.
template <int TM, int TN>
struct WideFrags {
    bf16x8_t a[TM], b[TN];
};

template <int I, int TM, int TN>
__device__ __forceinline__ void wide_read_one(WideFrags<TM, TN>& f, uint32_t a, uint32_t b) {
    if constexpr (I < TM) f.a[I] = ds_read16<I * 32 * kWRow>(a);
    else f.b[I - TM] = ds_read16<(I - TM) * 32 * kWRow>(b);
}

template <int TM, int TN, int... I>
__device__ __forceinline__ void wide_read_all(WideFrags<TM, TN>& f, uint32_t a, uint32_t b,
                                              std::integer_sequence<int, I...>) {
    (wide_read_one<I>(f, a, b), ...);
}

template <int N>
__device__ __forceinline__ void lgkm_wait() {
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}

// DMA of one stage's operand rows: per-lane byte offsets (row, swizzled chunk) of each
// of the wave's loads from the operand base; the stage's base pointers and LDS slot are
// uniform values computed once per stage. EXACT: both operands' 1 KB blocks divide evenly
// over the waves, so load i of every wave reads A for i < LA and lands i * NW blocks past
// the wave's first. Otherwise (192-row tiles: 12 A + 16 B blocks over 8 waves) each load
// carries a wave-uniform operand choice and LDS offset.
template <int LPW, int LA, int NW, bool EXACT>
struct WideDma {
    uint32_t voff[LPW];
    uint32_t dst[EXACT ? 1 : LPW];
    bool from_a[EXACT ? 1 : LPW];
    __device__ __forceinline__ void issue(int i, const unsigned char* sa, const unsigned char* sb,
                                          unsigned char* slot_wave) const {
        const unsigned char* base;
        unsigned char* d;
        if constexpr (EXACT) {
            base = i < LA ? sa : sb;
            d = slot_wave + i * NW * 1024;
        } else {
            base = from_a[i] ? sa : sb;
            d = slot_wave + dst[i];
        }
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(base + voff[i]),
                                         (__attribute__((address_space(3))) void*)d, 16, 0, 0);
    }
};

// MFMA I of a key step (tile I / TN, I % TN) on f, then (READS) operand read I of the next
// step into g and (DMA) this wave's load I of the stage at sa / sb into slot_wave. Each
// group is a scheduling barrier: the memory instructions go out one per MFMA, early in
// the step (measured: issuing the loads evenly over the step is slower).
template <int I, int TM, int TN, int LPW, bool READS, bool DMA, class Dma>
__device__ __forceinline__ void wide_slot(f32x16_t (&acc)[TM][TN], const WideFrags<TM, TN>& f,
                                          WideFrags<TM, TN>& g, uint32_t ga, uint32_t gb, const Dma& dma,
                                          const unsigned char* sa, const unsigned char* sb,
                                          unsigned char* slot_wave) {
    constexpr int i = I / TN, j = I % TN;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
    if constexpr (READS && I < TM + TN) wide_read_one<I>(g, ga, gb);
    if constexpr (DMA && I < LPW) dma.issue(I, sa, sb, slot_wave);
    __builtin_amdgcn_sched_barrier(0);
}

template <int TM, int TN, int LPW, bool READS, bool DMA, class Dma, int... I>
__device__ __forceinline__ void wide_mma_step(f32x16_t (&acc)[TM][TN], const WideFrags<TM, TN>& f,
                                              WideFrags<TM, TN>& g, uint32_t ga, uint32_t gb, const Dma& dma,
                                              const unsigned char* sa, const unsigned char* sb,
                                              unsigned char* slot_wave, std::integer_sequence<int, I...>) {
    (wide_slot<I, TM, TN, LPW, READS, DMA>(acc, f, g, ga, gb, dma, sa, sb, slot_wave), ...);
}

template <int BM, int BN, int WGM, int WGN, int S, int EPI>
__global__ __launch_bounds__(WGM * WGN * kWave, 1) void gemm_wide_kernel(const bf16_t* __restrict__ A,
                                                                    const bf16_t* __restrict__ B,
                                                                    const bf16_t* __restrict__ bias,
                                                                    void* __restrict__ Cout, int M, int N, int K,
                                                                    int ldc, int mt, int nt) {
    constexpr int NW = WGM * WGN;                // waves: a WGM x WGN grid over the tile
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int STAGE = (BM + BN) * kWRow;
    constexpr int QA = BM / 16, QB = BN / 16;   // 1 KB wave loads per operand per stage
    constexpr int Q = QA + QB;
    constexpr bool kExact = QA % NW == 0 && QB % NW == 0;
    constexpr int LA = QA / NW, LPW = (Q + NW - 1) / NW;
    constexpr int NR = TM + TN;                 // operand reads per key step
    static_assert(QA >= NW && S >= 2 && (S - 2) * LPW <= 63, "bad wide GEMM shape");
    static_assert(LPW <= TM * TN && NR <= TM * TN && NR <= 15, "interleave slots");
    static_assert(EPI != GEPI_SWIGLU || TN % 2 == 0, "SwiGLU needs paired N tiles");
    static_assert(EPI != GEPI_PARTIAL, "no split-K in the wide kernel");
    __shared__ __align__(1024) unsigned char smem[S * STAGE];

    const int T = mt * nt;
    const int per = (T + 7) / 8;
    const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (t >= T) return;
    int tm, tn;
    tile_of(t, mt, nt, tm, tn);
    const int m0 = tm * BM;
    const int n0 = (EPI == GEPI_SWIGLU) ? tn * (BN / 2) : tn * BN;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int wm = wave / WGN, wn = wave % WGN;

    auto b_row = [&](int r) -> int {
        if (EPI == GEPI_SWIGLU) {
            const int blk = r / 32;
            const int col = n0 + (blk / 2) * 32 + (r % 32);
            return (col < N) ? ((blk % 2 == 0) ? col : N + col) : -1;
        }
        const int n = n0 + r;
        return (n < N) ? n : -1;
    };

    // DMA sources (the host keeps both operands under 2 GB: 32-bit byte offsets)
    WideDma<LPW, LA, NW, kExact> dma;
    const unsigned char* pa = reinterpret_cast<const unsigned char*>(A);
    const unsigned char* pb = reinterpret_cast<const unsigned char*>(B);
    auto issue_stage = [&](int stage) {
        const unsigned char* sa = pa + stage * kWRow;
        const unsigned char* sb = pb + stage * kWRow;
        unsigned char* sw = smem + (stage % S) * STAGE + wave * 1024;
#pragma unroll
        for (int i = 0; i < LPW; ++i) dma.issue(i, sa, sb, sw);
    };
    {
        const int rr = lane >> 2, cs = lane & 3;
#pragma unroll
        for (int i = 0; i < LPW; ++i) {
            // Block q of the stage; past the last block (Q % NW != 0), a repeat of the
            // wave's first load (same source, same LDS bytes), so that every wave issues
            // LPW loads per stage and the vmcnt waits below count alike in all waves.
            int q = wave + NW * i;
            if (q >= Q) q = wave;
            if constexpr (!kExact) {
                dma.from_a[i] = q < QA;
                dma.dst[i] = (uint32_t)((q - wave) * 1024);
            }
            if (q < QA) {
                const int row = q * 16 + rr;
                const int grow = min(m0 + row, M - 1);
                dma.voff[i] = (uint32_t)((grow * K + ((cs ^ wide_swz(row)) << 3)) * 2);
            } else {
                const int row = (q - QA) * 16 + rr;
                int br = b_row(row);
                if (br < 0) br = 0;
                dma.voff[i] = (uint32_t)((br * K + ((cs ^ wide_swz(row)) << 3)) * 2);
            }
        }
    }

    // Operand read addresses: row (lane % 32) of each 32-row tile, chunk ks * 2 + lane / 32
    // under the stage's swizzle.
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) unsigned char*)smem);
    const int r32 = lane & 31, sw = wide_swz(r32);
    const uint32_t x0 = (uint32_t)(((lane >> 5) ^ sw) << 4), x1 = (uint32_t)(((2 + (lane >> 5)) ^ sw) << 4);
    const uint32_t rowA = (uint32_t)((wm * WM + r32) * kWRow), rowB = (uint32_t)(BM * kWRow + (wn * WN + r32) * kWRow);

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    WideFrags<TM, TN> f0, f1;
    auto tie = [&](WideFrags<TM, TN>& f) {
#pragma unroll
        for (int i = 0; i < TM; ++i) asm volatile("" : "+v"(f.a[i]));
#pragma unroll
        for (int j = 0; j < TN; ++j) asm volatile("" : "+v"(f.b[j]));
    };

    const int nk = K / kWBK;
    const int pre = min(S - 1, nk);
    for (int p = 0; p < pre; ++p) issue_stage(p);
    vm_wait_slabs<LPW>(min(S - 2, nk - 1));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    wide_read_all(f0, lds0 + rowA + x0, lds0 + rowB + x0, std::make_integer_sequence<int, NR>{});

    // Stage s: key step 0 on f0 with step 1's reads and, while stages remain, this wave's
    // loads of stage s + S - 1 (into the slot of stage s - 1, which every wave finished
    // reading before the previous barrier); then key step 1 on f1 with the reads of stage
    // s + 1, behind this wave's vmcnt wait for stage s + 1 and the barrier.
    auto run_stage = [&](int s, auto dma_on, auto next_on) {
        constexpr bool kDma = decltype(dma_on)::value, kNext = decltype(next_on)::value;
        const uint32_t cur = lds0 + (uint32_t)((s % S) * STAGE);
        const int ds = s + S - 1;
        lgkm_wait<0>();
        tie(f0);
        wide_mma_step<TM, TN, LPW, true, kDma>(acc, f0, f1, cur + rowA + x1, cur + rowB + x1, dma, pa + ds * kWRow,
                                               pb + ds * kWRow, smem + (ds % S) * STAGE + wave * 1024,
                                               std::make_integer_sequence<int, TM * TN>{});
        lgkm_wait<0>();
        tie(f1);
        if constexpr (kNext) {
            if constexpr (kDma) vm_wait<(S - 2) * LPW>();
            else vm_wait_slabs<LPW>(min(S - 2, nk - 2 - s));
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
        const uint32_t nxt = lds0 + (uint32_t)(((s + 1) % S) * STAGE);
        wide_mma_step<TM, TN, LPW, kNext, false>(acc, f1, f0, nxt + rowA + x0, nxt + rowB + x0, dma, pa, pb, smem,
                                                 std::make_integer_sequence<int, TM * TN>{});
    };
    int s = 0;
    for (; s < nk - (S - 1); ++s) run_stage(s, std::true_type{}, std::true_type{});
    for (; s < nk - 1; ++s) run_stage(s, std::false_type{}, std::true_type{});
    run_stage(nk - 1, std::false_type{}, std::false_type{});

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
                        const float o = silu_f32(g) * u;
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

// Split-K reduction: out[r, c] = sum over slices s = 0, 1, ... (in that order) of
// part[s, r, c], + bias[c], as bf16 or fp32. Four columns per thread (N % 4 == 0).
template <bool F32OUT>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* __restrict__ part, int ksplit, int M,
                                                                 int N, const bf16_t* __restrict__ bias,
                                                                 void* __restrict__ Cout) {
    const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;   // float4 index
    const size_t plane = (size_t)M * N;
    if (q * 4 >= plane) return;
    float4 acc = *reinterpret_cast<const float4*>(part + q * 4);
    for (int sl = 1; sl < ksplit; ++sl) {
        const float4 v = *reinterpret_cast<const float4*>(part + (size_t)sl * plane + q * 4);
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    }
    const int col = (int)((q * 4) % (size_t)N);
    if (bias != nullptr) {
        acc.x += bf16_to_f32(bias[col + 0]);
        acc.y += bf16_to_f32(bias[col + 1]);
        acc.z += bf16_to_f32(bias[col + 2]);
        acc.w += bf16_to_f32(bias[col + 3]);
    }
    if (F32OUT) {
        reinterpret_cast<float4*>(Cout)[q] = acc;
    } else {
        uint2 pk;
        pk.x = pack_bf16x2(acc.x, acc.y);
        pk.y = pack_bf16x2(acc.z, acc.w);
        reinterpret_cast<uint2*>(Cout)[q] = pk;
    }
}

template <int BM, int BN, int S, int EPI>
static void gemm_pipe_launch(int M, int N, int K, const bf16_t* A, const bf16_t* B, const bf16_t* bias, void* C,
                             int ldc, hipStream_t stream) {
    const int ocols = (EPI == GEPI_SWIGLU) ? BN / 2 : BN;
    const int mt = (M + BM - 1) / BM, nt = (N + ocols - 1) / ocols;
    const int grid = 8 * ((mt * nt + 7) / 8);
    hipLaunchKernelGGL((gemm_pipe_kernel<BM, BN, S, EPI>), dim3(grid), dim3(kGemmThreads), 0, stream, A, B, bias, C,
                       M, N, K, ldc, mt, nt, 1, K / kPBK);
}

template <int BM, int BN, int WGM, int WGN, int S, int EPI>
static void gemm_wide_launch(int M, int N, int K, const bf16_t* A, const bf16_t* B, const bf16_t* bias, void* C,
                             int ldc, hipStream_t stream) {
    const int ocols = (EPI == GEPI_SWIGLU) ? BN / 2 : BN;
    const int mt = (M + BM - 1) / BM, nt = (N + ocols - 1) / ocols;
    const int grid = 8 * ((mt * nt + 7) / 8);
    hipLaunchKernelGGL((gemm_wide_kernel<BM, BN, WGM, WGN, S, EPI>), dim3(grid), dim3(WGM * WGN * kWave), 0, stream, A,
                       B, bias, C, M, N, K, ldc, mt, nt);
}

int prefill_cus();

// Split-K plan for a plain (non-SwiGLU) projection with K % 64 == 0 and K >= 4096 whose
// 128 x 128 tiles leave the chip's workgroup slots empty; ksplit 0 = no split. Each slice
// covers at least 16 slabs (1024 keys). Measured on MI355X (us):
//  * tiles for at most a third of the CUs: as many slices as fill every CU once (at most
//    8), one workgroup per CU over a 4-deep ring: 512 x 8960 -> 1536 33.6 -> 28.3 (5
//    slices, against 8 slices over 2-deep rings, two workgroups per CU), 512 x 11008 ->
//    2048 47.7 -> 39.1 (4 against 6), 768 x 8960 -> 1536 40.9 -> 39.7 (3 against 6);
//  * up to 128 tiles: about 384 workgroups over 2-deep rings, two per CU (two slices over
//    4-deep rings: 1024 x 8960 -> 1536 46.1 -> 50.9, 512 x 18944 -> 3584 101.2 -> 102.9).
struct SplitK {
    int ksplit = 0, kt_per = 0;
    bool deep = false;  // 4-deep ring, one workgroup per CU (else 2-deep, two per CU)
};
static SplitK splitk_plan(int M, int N, int K) {
    SplitK p;
    if (K % kPBK != 0 || N % 4 != 0) return p;
    const long tiles = (long)((M + 127) / 128) * ((N + 127) / 128);
    const int nk = K / kPBK;
    if (tiles > 128 || nk < 64) return p;
    const int fill = (int)std::min<long>({8L, prefill_cus() / tiles, (long)(nk / 16)});
    int ks;
    if (fill >= 3) {
        ks = fill;
        p.deep = true;
    } else {
        ks = (int)std::min<long>(8, (384 + tiles - 1) / tiles);
        ks = std::min(ks, nk / 16);
    }
    if (ks < 2) return p;
    p.kt_per = (nk + ks - 1) / ks;
    p.ksplit = (nk + p.kt_per - 1) / p.kt_per;
    return p;
}
static size_t splitk_bytes(int M, int N, int K) {
    const SplitK p = splitk_plan(M, N, K);
    return p.ksplit == 0 ? 0 : (size_t)p.ksplit * M * N * sizeof(float);
}

// C = A . B^T (+ bias) through ksplit fp32 partial planes in `part`, then the ordered
// reduction.
static void gemm_splitk_launch(int M, int N, int K, const bf16_t* A, const bf16_t* B, const bf16_t* bias, void* C,
                               bool f32out, float* part, const SplitK& p, hipStream_t stream) {
    const int mt = (M + 127) / 128, nt = (N + 127) / 128;
    const int grid = 8 * ((mt * nt * p.ksplit + 7) / 8);
    if (p.deep)
        hipLaunchKernelGGL((gemm_pipe_kernel<128, 128, 4, GEPI_PARTIAL>), dim3(grid), dim3(kGemmThreads), 0, stream, A,
                           B, nullptr, part, M, N, K, N, mt, nt, p.ksplit, p.kt_per);
    else
        hipLaunchKernelGGL((gemm_pipe_kernel<128, 128, 2, GEPI_PARTIAL>), dim3(grid), dim3(kGemmThreads), 0, stream, A,
                           B, nullptr, part, M, N, K, N, mt, nt, p.ksplit, p.kt_per);
    const size_t quads = (size_t)M * N / 4;
    const dim3 rgrid((unsigned)((quads + 255) / 256));
    if (f32out) hipLaunchKernelGGL((gemm_splitk_reduce_kernel<true>), rgrid, dim3(256), 0, stream, part, p.ksplit, M, N, bias, C);
    else hipLaunchKernelGGL((gemm_splitk_reduce_kernel<false>), rgrid, dim3(256), 0, stream, part, p.ksplit, M, N, bias, C);
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
    // 256 x 256 tiles (one 8-wave workgroup per CU, 32-bit operand offsets) against the
    // 128 x 128 kernel (two workgroups per CU): rounds of resident workgroups times the
    // work of one round, each at its measured rate on MI355X (about 1.15 and 0.95 PF/s on
    // the 7B prefill projections), so the wide tile wins once it wastes no more than a
    // partial round: 512 x 1536 -> 2 x 8960 (SwiGLU) runs wide, 1344 x 2048 -> 2 x 11008
    // does not (3 wide rounds, the last nearly empty, against 3.7 narrow ones).
    const int tile_knob = kernel_knob(EFM_KNOB_GEMM_TILE);
    const long b_rows = (EPI == GEPI_SWIGLU) ? 2L * N : (long)N;
    const bool wide_ok = K % kPBK == 0 && (long)M * K * 2 < 0x7fffffffL && b_rows * K * 2 < 0x7fffffffL;
    if (wide_ok && tile_knob != 1) {
        const long r_wide = (tiles(256, 256) + 255) / 256, r_pipe = (tiles(128, 128) + 511) / 512;
        // 192 x 256 tiles (six MFMA tiles per wave instead of eight) take 0.9 of a 256 x
        // 256 round (measured, SwiGLU: 512 x 1536 -> 2 x 8960 48.3 -> 43.3 us in one round
        // of 210 tiles against 140; 512 x 3584 -> 2 x 18944 198.2 -> 177.3 in two rounds,
        // against 196.5 for the 128 x 128 kernel); the fewest weighted rounds wins.
        const long r_192 = (tiles(192, 256) + 255) / 256;
        if (tile_knob == 3 || (tile_knob == 0 && 171 * r_192 < std::min(190 * r_wide, 115 * r_pipe))) {
            gemm_wide_launch<192, 256, 2, 4, 4, EPI>(M, N, K, A, B, bias, C, ldc, stream);
            return check_launch("gemm_bf16");
        }
        if (tile_knob == 2 || 190 * r_wide < 115 * r_pipe) {
            gemm_wide_launch<256, 256, 2, 4, 4, EPI>(M, N, K, A, B, bias, C, ldc, stream);
            return check_launch("gemm_bf16");
        }
    }
    if (K % kPBK == 0) {
        // Tile choice from sweeps of the prefill shapes on MI355X: 128 x 128 double-
        // buffered (two workgroups per CU) once there are >= 1.5 tiles per CU (>= 1 for
        // SwiGLU); K >= 4096 with 129 to one-per-CU 128 x 128 tiles: those tiles over a
        // 4-deep ring, one workgroup per CU (1344 x 11008 -> 2048 129.2 -> 106.6 us,
        // 1024 x 18944 -> 3584 237.6 -> 182.8; at 132 tiles, 1344 x 8960 -> 1536, 80.2 ->
        // 86.1); else 128 x 64 over a 3-deep ring (two per CU; 1024 x 1536 -> 2048 20.2 ->
        // 18.3 against the 2-deep ring, no shape slower); else 64 x 64 (64 x 128 for
        // SwiGLU) with shallow pipelines. Every tile shape sums each output over K in the
        // same order: results are bit-identical whichever is chosen.
        if constexpr (EPI != GEPI_SWIGLU) {
            const long t = tiles(128, 128);
            if (K / kPBK >= 64 && t > 128 && t < 384 && t <= prefill_cus()) {
                gemm_pipe_launch<128, 128, 4, EPI>(M, N, K, A, B, bias, C, ldc, stream);
                return check_launch("gemm_bf16");
            }
        }
        if (tiles(128, 128) >= ((EPI == GEPI_SWIGLU) ? 256 : 384)) {
            gemm_pipe_launch<128, 128, 2, EPI>(M, N, K, A, B, bias, C, ldc, stream);
        } else if constexpr (EPI == GEPI_SWIGLU) {
            gemm_pipe_launch<64, 128, 3, EPI>(M, N, K, A, B, bias, C, ldc, stream);
        } else {
            if (tiles(128, 64) >= 256) gemm_pipe_launch<128, 64, 3, EPI>(M, N, K, A, B, bias, C, ldc, stream);
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

size_t gemm_bf16_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 1 || M > 0x7fffffff / 2 || N > 0x7fffffff / 2 || K > 0x7fffffff / 2) return 0;
    return splitk_bytes((int)M, (int)N, (int)K);
}

int gemm_bf16_ws(int64_t M, int64_t N, int64_t K, const void* A, const void* B, const void* bias, void* C,
                 int32_t out_dtype, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    int rc = gemm_check(M, N, K, A, B, C);
    if (rc) return rc;
    if (M == 0 || N == 0) return EFM_OK;
    if (out_dtype != EFM_DTYPE_BF16 && out_dtype != EFM_DTYPE_F32)
        return set_error(EFM_ERR_UNSUPPORTED, "linear: output dtype %d not supported", out_dtype);
    const SplitK p = splitk_plan((int)M, (int)N, (int)K);
    const size_t need = (p.ksplit == 0) ? 0 : (size_t)p.ksplit * M * N * sizeof(float);
    if (p.ksplit == 0 || workspace == nullptr || workspace_bytes < need ||
        (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
        return gemm_bf16(M, N, K, A, B, bias, C, out_dtype, stream);
    gemm_splitk_launch((int)M, (int)N, (int)K, static_cast<const bf16_t*>(A), static_cast<const bf16_t*>(B),
                       static_cast<const bf16_t*>(bias), C, out_dtype == EFM_DTYPE_F32, static_cast<float*>(workspace),
                       p, stream);
    return check_launch("gemm_bf16 split-K");
}

int gemm_swiglu(int64_t M, int64_t inter, int64_t K, const void* A, const void* W, void* out, hipStream_t stream) {
    int rc = gemm_check(M, inter, K, A, W, out);
    if (rc) return rc;
    if (M == 0) return EFM_OK;
    return gemm_dispatch<GEPI_SWIGLU>((int)M, (int)inter, (int)K, static_cast<const bf16_t*>(A),
                                      static_cast<const bf16_t*>(W), nullptr, out, (int)inter, stream);
}

// Gate/up + SwiGLU with a workspace: the SwiGLU is the MFMA kernel's epilogue, so no
// shape uses the workspace.
size_t gemm_swiglu_workspace_bytes(int64_t, int64_t, int64_t) { return 0; }

int gemm_swiglu_ws(int64_t M, int64_t inter, int64_t K, const void* A, const void* W, void* out, void*, size_t,
                   hipStream_t stream) {
    return gemm_swiglu(M, inter, K, A, W, out, stream);
}

}  // namespace efm

// Temperature / top-p sampling of one fp32 logits row (the non-greedy branch of
// SamplerLayer::forward_sampling, src/layers/sampler.cu:251-298, widened with top-p).
//
// Definition (exact; every mass is an integer so the result is reproducible bit for bit):
//   m    = max_i l_i;  e_i = expf((l_i - m) / T);  w_i = rint(e_i * 2^44)  (uint64)
//   W    = sum_i w_i
//   nucleus = every i when top_p >= 1, else { i : e_i >= tau } where tau is the largest
//          fp32 value with sum_{e_j >= tau} w_j >= max(1, ceil(top_p * W)) (in double)
//   x    = Philox4x32-10(counter = (off_lo, off_hi, 0, 0), key = (seed_lo, seed_hi)).x
//   r    = floor(N * (x >> 8) / 2^24), N = nucleus mass
//   token = the smallest nucleus index i whose inclusive nucleus prefix mass exceeds r.
// e_i <= 1, so w_i <= 2^44 and every sum fits in 64 bits for V < 2^20.
//
// The row is split into blocks of 1024 logits, one 256-thread workgroup each, and the
// passes are separate launches (the launch boundary is the grid-wide barrier):
//   1. block maxima (workgroup 0 also clears the workspace accumulators)
//   2. m from the block maxima; total mass W and the histogram of the top exponent
//      byte of e (device-scope integer atomics: exact and order independent)
//   3-5. each workgroup replays the digit choice of the previous passes from the
//      histograms (positive fp32 values order like their bit patterns), then
//      histograms the next byte of the e_i that share the chosen prefix
//   6. tau is fixed; every block writes its nucleus mass, and the last block to finish
//      scans the block masses, finds the block holding r and scans its elements.
// With top_p >= 1 passes 3-5 are skipped (tau = 0).
#include "common.hpp"

namespace efm {

constexpr int kSampleThreads = 256;
constexpr int kSamplePer = 4;                                  // logits per thread
constexpr int kSampleBlock = kSampleThreads * kSamplePer;      // logits per workgroup
constexpr int kSampleMaxVocab = 1 << 20;
constexpr int kSampleMaxBlocks = kSampleMaxVocab / kSampleBlock;

// Device workspace of one sampler call (efm_sampler_top_p_workspace_bytes).
struct SampleWs {
    float bmax[kSampleMaxBlocks];
    unsigned long long bmass[kSampleMaxBlocks];
    unsigned long long hist[4][256];
    unsigned long long W;
    uint32_t counter;
};

struct SampleArgs {
    const float* logits;
    int V;
    float temperature;
    float top_p;
    uint64_t seed;
    uint64_t offset;
    const int32_t* d_offset;   // optional device-resident addend to `offset`
    int32_t* token_out;
    SampleWs* ws;
    int nblocks;
};

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
// 1, 2, 3", SC'11): ten rounds of two 32x32->64 multiplies with a Weyl key schedule.
__device__ __forceinline__ uint32_t philox_x0(uint64_t counter, uint64_t key) {
    uint32_t c0 = (uint32_t)counter, c1 = (uint32_t)(counter >> 32), c2 = 0u, c3 = 0u;
    uint32_t k0 = (uint32_t)key, k1 = (uint32_t)(key >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

__device__ __forceinline__ float sample_e(float l, float m, float T) { return expf((l - m) / T); }

__device__ __forceinline__ uint64_t sample_w(float e) {
    return (uint64_t)__builtin_rint((double)e * 17592186044416.0);   // 2^44
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ uint64_t wave_scan_u64(uint64_t v, int lane) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const uint64_t o = __shfl_up(v, off, kWave);
        if (lane >= off) v += o;
    }
    return v;
}

// Block-wide reductions of a 256-thread workgroup (4 waves) through LDS.
__device__ __forceinline__ float block_max_f(float v, float* red) {
    v = wave_max(v);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kSampleThreads / kWave; ++w) m = fmaxf(m, red[w]);
    return m;
}

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, unsigned long long* red) {
    v = wave_sum_u64(v);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    uint64_t s = 0;
#pragma unroll
    for (int w = 0; w < kSampleThreads / kWave; ++w) s += red[w];
    return s;
}

// Exclusive prefix (in thread order) and total of a per-thread value.
__device__ __forceinline__ uint64_t block_scan_u64(uint64_t v, unsigned long long* red, uint64_t* total) {
    const int lane = threadIdx.x % kWave, wid = threadIdx.x / kWave;
    const uint64_t incl = wave_scan_u64(v, lane);
    if (lane == kWave - 1) red[wid] = incl;
    __syncthreads();
    uint64_t before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kSampleThreads / kWave; ++w) {
        const uint64_t t = red[w];
        if (w < wid) before += t;
        tot += t;
    }
    *total = tot;
    return before + incl - v;
}

// The logits of this workgroup: element k of thread t is index base + t + 256 k.
__device__ __forceinline__ void load_block(const SampleArgs& a, float (&l)[kSamplePer], bool (&ok)[kSamplePer]) {
    const int base = blockIdx.x * kSampleBlock + threadIdx.x;
#pragma unroll
    for (int k = 0; k < kSamplePer; ++k) {
        const int i = base + k * kSampleThreads;
        ok[k] = i < a.V;
        l[k] = ok[k] ? a.logits[i] : -INFINITY;
    }
}

// Global maximum from the block maxima (identical in every workgroup).
__device__ __forceinline__ float global_max(const SampleArgs& a, float* red) {
    float m = -INFINITY;
    for (int b = threadIdx.x; b < a.nblocks; b += kSampleThreads) m = fmaxf(m, a.ws->bmax[b]);
    return block_max_f(m, red);
}

// Replays the radix choices of passes [0, npass): returns the chosen key prefix and
// the mass still needed inside it. Every workgroup computes the same values.
__device__ uint32_t select_prefix(const SampleArgs& a, int npass, unsigned long long* s_sel) {
    const int lane = threadIdx.x % kWave;
    if (threadIdx.x < kWave) {
        const uint64_t W = a.ws->W;
        uint64_t need = (uint64_t)ceil((double)a.top_p * (double)W);
        if (need < 1) need = 1;
        if (need > W) need = W;
        uint64_t rem = need;
        uint32_t prefix = 0u;
        for (int p = 0; p < npass; ++p) {
            const int shift = 24 - 8 * p;
            // lane j owns digits 255-4j .. 252-4j (descending)
            uint64_t h[4], own = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                h[k] = a.ws->hist[p][255 - 4 * lane - k];
                own += h[k];
            }
            const uint64_t incl = wave_scan_u64(own, lane);
            const uint64_t excl = incl - own;
            // exactly one lane's digit range holds the rem-th unit of mass
            const bool owns = excl < rem && rem <= incl;
            uint32_t digit = 0u;
            uint64_t left = 0ull;
            if (owns) {
                uint64_t acc = excl;
                bool found = false;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (!found && rem <= acc + h[k]) {
                        digit = (uint32_t)(255 - 4 * lane - k);
                        left = rem - acc;
                        found = true;
                    }
                    acc += h[k];
                }
            }
            const int src = __ffsll((unsigned long long)__ballot(owns)) - 1;
            prefix |= (uint32_t)__shfl((int)digit, src, kWave) << shift;
            rem = (uint64_t)__shfl((unsigned long long)left, src, kWave);
        }
        if (lane == 0) s_sel[0] = prefix;
    }
    __syncthreads();
    return (uint32_t)s_sel[0];
}

// pass 1: block maxima; workgroup 0 clears the accumulators the later passes add into
__global__ void __launch_bounds__(kSampleThreads) sample_max_kernel(SampleArgs a) {
    __shared__ float red[kSampleThreads / kWave];
    float l[kSamplePer];
    bool ok[kSamplePer];
    load_block(a, l, ok);
    float m = l[0];
#pragma unroll
    for (int k = 1; k < kSamplePer; ++k) m = fmaxf(m, l[k]);
    m = block_max_f(m, red);
    if (threadIdx.x == 0) a.ws->bmax[blockIdx.x] = m;
    if (blockIdx.x == 0) {
        unsigned long long* h = &a.ws->hist[0][0];
        for (int i = threadIdx.x; i < 4 * 256; i += kSampleThreads) h[i] = 0ull;
        if (threadIdx.x == 0) {
            a.ws->W = 0ull;
            a.ws->counter = 0u;
        }
    }
}

// passes 2-5: pass 2 adds the total mass W; every pass histograms the next byte
// (shift 24 - 8 * npass) of the e_i under the prefix chosen so far.
__global__ void __launch_bounds__(kSampleThreads) sample_hist_kernel(SampleArgs a, int npass, int want_hist) {
    __shared__ float red[kSampleThreads / kWave];
    __shared__ unsigned long long redu[kSampleThreads / kWave];
    __shared__ unsigned long long s_hist[256];
    __shared__ unsigned long long s_sel[1];
    float l[kSamplePer];
    bool ok[kSamplePer];
    load_block(a, l, ok);
    s_hist[threadIdx.x] = 0ull;
    const float m = global_max(a, red);
    const float T = a.temperature;
    uint32_t prefix = 0u;
    if (npass > 0) prefix = select_prefix(a, npass, s_sel);
    const int shift = 24 - 8 * npass;
    const uint32_t mask = (npass == 0) ? 0u : (0xffffffffu << (shift + 8));
    uint64_t tot = 0;
#pragma unroll
    for (int k = 0; k < kSamplePer; ++k) {
        if (!ok[k]) continue;
        const float e = sample_e(l[k], m, T);
        const uint64_t w = sample_w(e);
        tot += w;
        const uint32_t key = __float_as_uint(e);
        if (want_hist && w != 0 && (key & mask) == prefix)
            atomicAdd(&s_hist[(key >> shift) & 255u], (unsigned long long)w);
    }
    if (npass == 0) {
        tot = block_sum_u64(tot, redu);
        if (threadIdx.x == 0) __hip_atomic_fetch_add(&a.ws->W, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (want_hist) {
        __syncthreads();
        const unsigned long long hv = s_hist[threadIdx.x];
        if (hv != 0ull)
            __hip_atomic_fetch_add(&a.ws->hist[npass][threadIdx.x], hv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// pass 6: nucleus mass per block; the last block to finish locates r.
__global__ void __launch_bounds__(kSampleThreads) sample_locate_kernel(SampleArgs a) {
    __shared__ float red[kSampleThreads / kWave];
    __shared__ unsigned long long redu[kSampleThreads / kWave];
    __shared__ unsigned long long s_sel[1];
    __shared__ uint32_t s_last;
    __shared__ int s_block;
    __shared__ unsigned long long s_base;
    float l[kSamplePer];
    bool ok[kSamplePer];
    load_block(a, l, ok);
    const float m = global_max(a, red);
    const float T = a.temperature;
    const uint32_t tau_key = (a.top_p < 1.0f) ? select_prefix(a, 4, s_sel) : 0u;
    uint64_t own = 0;
#pragma unroll
    for (int k = 0; k < kSamplePer; ++k) {
        if (!ok[k]) continue;
        const float e = sample_e(l[k], m, T);
        if (__float_as_uint(e) >= tau_key) own += sample_w(e);
    }
    own = block_sum_u64(own, redu);
    if (threadIdx.x == 0) {
        // publish the block mass, wait for that atomic to return (it is then performed
        // where every XCD's atomics meet), then count in: no cache flush needed, and the
        // last block reads every mass with agent-scope atomic loads
        const uint64_t old =
            __hip_atomic_exchange(&a.ws->bmass[blockIdx.x], own, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" : : "v"(old) : "memory");
        const uint32_t prev = __hip_atomic_fetch_add(&a.ws->counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (uint32_t)a.nblocks - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;

    // last block: N, r, the block that holds r (blocks in index order) ...
    const int per = (a.nblocks + kSampleThreads - 1) / kSampleThreads;   // <= 4
    const int b0 = threadIdx.x * per;
    uint64_t bm[4] = {0ull, 0ull, 0ull, 0ull}, mine = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (k < per && b0 + k < a.nblocks)
            bm[k] = __hip_atomic_load(&a.ws->bmass[b0 + k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mine += bm[k];
    }
    uint64_t N;
    const uint64_t excl = block_scan_u64(mine, redu, &N);
    uint64_t off = a.offset;
    if (a.d_offset != nullptr) off += (uint64_t)(uint32_t)a.d_offset[0];
    const uint64_t bits = philox_x0(off, a.seed) >> 8;
    const uint64_t r = (__umul64hi(N, bits) << 40) | ((N * bits) >> 24);
    if (mine != 0 && excl <= r && r < excl + mine) {
        uint64_t acc = excl;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (acc <= r && r < acc + bm[k]) {
                s_block = b0 + k;
                s_base = acc;
            }
            acc += bm[k];
        }
    }
    __syncthreads();
    // ... then the element: thread t covers indices [4t, 4t + 4) of that block
    const int blk = s_block;
    const int i0 = blk * kSampleBlock + threadIdx.x * kSamplePer;
    uint64_t w4[kSamplePer], tm = 0;
#pragma unroll
    for (int k = 0; k < kSamplePer; ++k) {
        const int i = i0 + k;
        w4[k] = 0;
        if (i < a.V) {
            const float e = sample_e(a.logits[i], m, T);
            if (__float_as_uint(e) >= tau_key) w4[k] = sample_w(e);
        }
        tm += w4[k];
    }
    uint64_t btot;
    const uint64_t ex = s_base + block_scan_u64(tm, redu, &btot);
    if (tm != 0 && ex <= r && r < ex + tm) {
        uint64_t acc = ex;
        int tok = i0 + kSamplePer - 1;
#pragma unroll
        for (int k = 0; k < kSamplePer; ++k) {
            acc += w4[k];
            if (acc > r) {
                tok = i0 + k;
                break;
            }
        }
        a.token_out[0] = tok;
    }
    if (threadIdx.x == 0) a.ws->counter = 0u;
}

}  // namespace efm

using namespace efm;

extern "C" size_t efm_sampler_top_p_workspace_bytes(int64_t vocab) {
    (void)vocab;
    return (sizeof(SampleWs) + 255) & ~(size_t)255;
}

extern "C" int efm_sampler_top_p(int64_t vocab, const float* logits, float temperature, float top_p, uint64_t seed,
                                 uint64_t offset, const int32_t* d_offset, int32_t* token_out, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
    if (logits == nullptr || token_out == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "sampler_top_p: null pointer");
    if (vocab <= 0 || vocab >= kSampleMaxVocab)   // V < 2^20 keeps W = sum w_i < 2^64
        return set_error(EFM_ERR_INVALID_ARGUMENT, "sampler_top_p: vocab %lld outside [1, %d)", (long long)vocab,
                         kSampleMaxVocab);
    if (!(temperature >= 1e-6f) || !(temperature < INFINITY))
        return set_error(EFM_ERR_INVALID_ARGUMENT,
                         "sampler_top_p: temperature must be finite and >= 1e-6 (below that sampling is greedy)");
    if (!(top_p > 0.0f))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "sampler_top_p: top_p must be > 0");
    if (workspace == nullptr || workspace_bytes < sizeof(SampleWs))
        return set_error(EFM_ERR_WORKSPACE, "sampler_top_p: workspace of %zu bytes required", sizeof(SampleWs));
    const int nb = (int)((vocab + kSampleBlock - 1) / kSampleBlock);
    SampleArgs a{logits, (int)vocab, temperature, top_p, seed, offset, d_offset, token_out,
                 static_cast<SampleWs*>(workspace), nb};
    hipLaunchKernelGGL(sample_max_kernel, dim3(nb), dim3(kSampleThreads), 0, stream, a);
    const int passes = (top_p < 1.0f) ? 4 : 1;
    for (int p = 0; p < passes; ++p)
        hipLaunchKernelGGL(sample_hist_kernel, dim3(nb), dim3(kSampleThreads), 0, stream, a, p, top_p < 1.0f ? 1 : 0);
    hipLaunchKernelGGL(sample_locate_kernel, dim3(nb), dim3(kSampleThreads), 0, stream, a);
    return check_launch("sampler_top_p");
}

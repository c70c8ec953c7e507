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
// e_i <= 1, so w_i <= 2^44 and every sum fits in 64 bits for V <= 2^20.
//
// One 1024-thread workgroup does the whole row: the row (<= 4 MiB) stays in L2 across
// its seven passes: max, total mass, four 8-bit radix passes that find tau's bit pattern
// from a mass histogram (positive fp32 values order like their bit patterns), and a
// chunked prefix scan that locates r. Integer LDS atomics make the histograms exact and
// order independent.
#include "common.hpp"

namespace efm {

constexpr int kSampleThreads = 1024;
constexpr int kSampleWaves = kSampleThreads / kWave;
constexpr int kSampleMaxVocab = 1 << 20;

struct SampleArgs {
    const float* logits;
    int V;
    float temperature;
    float top_p;
    uint64_t seed;
    uint64_t offset;
    const int32_t* d_offset;   // optional device-resident addend to `offset`
    int32_t* token_out;
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

__global__ void __launch_bounds__(kSampleThreads) sample_top_p_kernel(SampleArgs a) {
    __shared__ float s_f[kSampleWaves];
    __shared__ unsigned long long s_u[kSampleWaves];
    __shared__ unsigned long long s_hist[256];
    __shared__ unsigned long long s_remaining;
    __shared__ uint32_t s_prefix;

    const int tid = threadIdx.x, lane = tid % kWave, wid = tid / kWave;
    const int V = a.V;
    const float T = a.temperature;
    const float* __restrict__ lg = a.logits;

    // pass 1: max logit
    float m = -INFINITY;
    for (int i = tid; i < V; i += kSampleThreads) m = fmaxf(m, lg[i]);
    m = wave_max(m);
    if (lane == 0) s_f[wid] = m;
    __syncthreads();
    m = s_f[0];
#pragma unroll
    for (int w = 1; w < kSampleWaves; ++w) m = fmaxf(m, s_f[w]);

    // pass 2: total mass W
    uint64_t tot = 0;
    for (int i = tid; i < V; i += kSampleThreads) tot += sample_w(sample_e(lg[i], m, T));
    tot = wave_sum_u64(tot);
    if (lane == 0) s_u[wid] = tot;
    __syncthreads();
    uint64_t W = 0;
#pragma unroll
    for (int w = 0; w < kSampleWaves; ++w) W += s_u[w];

    // passes 3-6: tau by radix selection over fp32 bit patterns, descending
    uint32_t tau_key = 0u;
    if (a.top_p < 1.0f) {
        uint64_t need = (uint64_t)ceil((double)a.top_p * (double)W);
        if (need < 1) need = 1;
        if (need > W) need = W;
        if (tid == 0) {
            s_remaining = need;
            s_prefix = 0u;
        }
        uint32_t mask = 0u;
        for (int shift = 24; shift >= 0; shift -= 8) {
            if (tid < 256) s_hist[tid] = 0ull;
            __syncthreads();
            const uint32_t prefix = s_prefix;
            for (int i = tid; i < V; i += kSampleThreads) {
                const float e = sample_e(lg[i], m, T);
                const uint32_t key = __float_as_uint(e);
                if ((key & mask) == prefix) {
                    const uint64_t w = sample_w(e);
                    if (w) atomicAdd(&s_hist[(key >> shift) & 255u], (unsigned long long)w);
                }
            }
            __syncthreads();
            if (wid == 0) {
                // lane j owns digits 255-4j .. 252-4j (descending)
                uint64_t h[4];
                uint64_t own = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    h[k] = s_hist[255 - 4 * lane - k];
                    own += h[k];
                }
                const uint64_t incl = wave_scan_u64(own, lane);
                const uint64_t excl = incl - own;
                const uint64_t rem = s_remaining;
                if (excl < rem && rem <= incl) {
                    uint64_t acc = excl;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        if (acc < rem && rem <= acc + h[k]) {
                            s_prefix = prefix | ((uint32_t)(255 - 4 * lane - k) << shift);
                            s_remaining = rem - acc;
                        }
                        acc += h[k];
                    }
                }
            }
            mask |= 255u << shift;
            __syncthreads();
        }
        tau_key = s_prefix;
    }

    // pass 7: nucleus mass per contiguous chunk, block scan, locate r
    const int chunk = (V + kSampleThreads - 1) / kSampleThreads;
    const int b = tid * chunk;
    const int e_end = min(V, b + chunk);
    uint64_t own = 0;
    for (int i = b; i < e_end; ++i) {
        const float e = sample_e(lg[i], m, T);
        if (__float_as_uint(e) >= tau_key) own += sample_w(e);
    }
    const uint64_t incl_w = wave_scan_u64(own, lane);
    __syncthreads();
    if (lane == kWave - 1) s_u[wid] = incl_w;
    __syncthreads();
    uint64_t before = 0, N = 0;
#pragma unroll
    for (int w = 0; w < kSampleWaves; ++w) {
        const uint64_t t = s_u[w];
        if (w < wid) before += t;
        N += t;
    }
    const uint64_t excl = before + incl_w - own;
    uint64_t off = a.offset;
    if (a.d_offset != nullptr) off += (uint64_t)(uint32_t)a.d_offset[0];
    const uint64_t bits = philox_x0(off, a.seed) >> 8;
    const uint64_t r = (__umul64hi(N, bits) << 40) | ((N * bits) >> 24);
    if (own != 0 && excl <= r && r < excl + own) {
        uint64_t acc = excl;
        int tok = e_end - 1;
        for (int i = b; i < e_end; ++i) {
            const float e = sample_e(lg[i], m, T);
            if (__float_as_uint(e) >= tau_key) {
                acc += sample_w(e);
                if (acc > r) {
                    tok = i;
                    break;
                }
            }
        }
        a.token_out[0] = tok;
    }
}

}  // namespace efm

using namespace efm;

extern "C" int efm_sampler_top_p(int64_t vocab, const float* logits, float temperature, float top_p, uint64_t seed,
                                 uint64_t offset, const int32_t* d_offset, int32_t* token_out, hipStream_t stream) {
    if (logits == nullptr || token_out == nullptr)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "sampler_top_p: null pointer");
    if (vocab <= 0 || vocab > kSampleMaxVocab)
        return set_error(EFM_ERR_INVALID_ARGUMENT, "sampler_top_p: vocab %lld outside [1, %d]", (long long)vocab,
                         kSampleMaxVocab);
    if (!(temperature >= 1e-6f) || !(temperature < INFINITY))
        return set_error(EFM_ERR_INVALID_ARGUMENT,
                         "sampler_top_p: temperature must be finite and >= 1e-6 (below that sampling is greedy)");
    if (!(top_p > 0.0f))
        return set_error(EFM_ERR_INVALID_ARGUMENT, "sampler_top_p: top_p must be > 0");
    SampleArgs a{logits, (int)vocab, temperature, top_p, seed, offset, d_offset, token_out};
    hipLaunchKernelGGL(sample_top_p_kernel, dim3(1), dim3(kSampleThreads), 0, stream, a);
    return check_launch("sampler_top_p");
}

// Shared pieces of the pipelined prefill attention kernels (bf16 and int8 QK^T):
// the LDS tile layouts, the per-lane operand offsets and the inline-asm LDS reads.
//
// LDS tiles hold rows of 16-byte chunks in row-major order, chunk-swizzled so that the
// operand reads of a wave hit distinct banks:
//  * bf16 K (256-byte rows): chunk c of row r sits at c ^ (r & 15). The S^T = K . Q^T
//    A-operand read (ds_read_b128) takes one chunk of 16 consecutive rows per 256 bytes.
//  * int8 K (128-byte rows, two per 256 bytes): chunk c of row r at c ^ ((r >> 1) & 7).
//  * bf16 V (256-byte rows): chunk c of row r at c ^ ((r & 3) << 2). The V^T operand is
//    read with ds_read_b64_tr_b16: each 32 lanes take 4 chunks of 4 consecutive rows.
// ds_read_b64_tr_b16 (gfx950): within each group of 16 lanes, lane i receives element
// i % 4 of the 8-byte rows addressed by lanes i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4 of
// the group. Lane j = 4 e + q of group g addresses V[key 4 (g / 2) + e][d 16 (g % 2) + 4 q]
// (relative to the 16-key block and the 32-wide d tile), so lane L receives the keys
// 4 (L / 32) + e, e = 0..3, of d column L % 32: the A-operand slots of
// v_mfma_f32_32x32x16_bf16 for those keys.
#pragma once
#include "common.hpp"

namespace efm {
namespace attn_pipe {

constexpr int kRow = 256;   // bytes per bf16 K / V row (head_dim 128)

__device__ __forceinline__ uint32_t k_off(int row, int chunk) {
    return (uint32_t)(row * kRow + ((chunk ^ (row & 15)) << 4));
}
__device__ __forceinline__ uint32_t k8_off(int row, int chunk) {
    return (uint32_t)(row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4));
}
__device__ __forceinline__ uint32_t v_off(int row, int chunk) {
    return (uint32_t)(row * kRow + ((chunk ^ ((row & 3) << 2)) << 4));
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until at most `tiles` tiles of LPW wave loads each are outstanding.
template <int LPW>
__device__ __forceinline__ void vm_wait_tiles(int tiles) {
    switch (tiles) {
        case 0: vm_wait<0>(); break;
        case 1: vm_wait<1 * LPW>(); break;
        default: vm_wait<2 * LPW>(); break;
    }
}

template <int IMM, typename T>
__device__ __forceinline__ void read_b128(T& dst, uint32_t addr) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "n"(IMM) : "memory");
}

template <int IMM, typename T>
__device__ __forceinline__ void read_tr16(T& dst, uint32_t addr) {
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "n"(IMM) : "memory");
}

// Lane part of the V^T operand address for d tile tt (rows of the 16-key block and the
// (kb, c) part are immediates): row 4 (g / 2) + e, d = 32 tt + 16 (g % 2) + 4 q.
__device__ __forceinline__ uint32_t v_tr_lane_off(int lane, int tt) {
    const int g = lane >> 4, j = lane & 15;
    const int row = (g >> 1) * 4 + (j >> 2);
    const int d = tt * 32 + 16 * (g & 1) + 4 * (j & 3);
    return v_off(row, d >> 3) + ((d & 7) << 1);
}

}  // namespace attn_pipe
}  // namespace efm

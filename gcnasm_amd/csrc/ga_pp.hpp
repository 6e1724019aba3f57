// ga_pp.hpp -- pieces shared by the 256x256 eight-wave ("ping-pong") GEMM
// kernels (gemm_mx_pp.hip: MXFP8, gemm_bs_pp.hip: fp32-scaled FP8).
//
// Both keep per K step of 128 two 16 KB half tiles of A and of B in LDS, two
// K-step slots each, and run two groups of four waves one workgroup barrier
// apart (one group's MFMAs overlap the other group's LDS reads and copies).
// Row-major operands sit in LDS as 128-byte rows with 16-byte K chunk c of
// row r at slot c ^ ((r >> 1) & 7): a direct-to-LDS copy instruction (64
// lanes x 16 B) covers 8 whole rows, and the MFMA operand reads (lane
// 16g + r: row r, chunks g and g + 4) hit 64 distinct banks per 16 lanes.
#pragma once

#include "ga_device.hpp"

namespace ga {
namespace pp {

constexpr int kNT = 512;
constexpr int kHalf = 16384; // 128 rows x 128 K of fp8
constexpr int kOpSlot = 2 * kHalf;
constexpr int kARegion = 0;  // A: [slot][half] half tiles
constexpr int kBRegion = 2 * kOpSlot;
constexpr int kOperandBytes = 4 * kOpSlot;

// Uniform byte offset as an SGPR operand, kept opaque so a per-copy address
// is formed at the copy (one VGPR base per operand, no hoisted per-copy VGPRs).
__device__ __forceinline__ uint32_t uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

template <class T>
__device__ __forceinline__ T* uni_ptr(T* p)
{
    const uint64_t u = (uint64_t)(uintptr_t)p;
    const uint64_t lo = uni((uint32_t)u), hi = uni((uint32_t)(u >> 32));
    return (T*)(uintptr_t)((hi << 32) | lo);
}

__device__ __forceinline__ void wait_lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Phase boundary: own copies waited for (N = copies issued after the ones
// the next phase reads), then the workgroup barrier.
template <int N>
__device__ __forceinline__ void phase_sync()
{
    wait_vmcnt<N>();
    wait_lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

// Staged epilogue: a 256x256 bf16 tile goes through LDS as rows of 528 bytes
// (512 + 16: the 16 rows x 2 lanes of one ds_write_b64 half-wave start on
// distinct bank quads), so the global stores write whole 512-byte rows
// instead of 16 rows x 32 bytes per instruction.
constexpr int kStagePitch = 528;
constexpr int kStageBytes = 256 * kStagePitch;

__device__ __forceinline__ void stage_put(char* smem, int row, int col, uint32_t lo, uint32_t hi)
{
    uint2 v;
    v.x = lo;
    v.y = hi;
    *(uint2*)(smem + row * kStagePitch + col * 2) = v;
}

// Wave w stores rows 32w .. 32w+31 of the staged tile, two rows (64 lanes x
// 16 B) per instruction, to dst (the tile's first element, row stride ldd).
// NT: non-temporal stores. A compile-time choice: LLVM merges a store and a
// non-temporal store of the same value under a run-time branch and drops the
// hint.
template <bool NT = false>
__device__ __forceinline__ void stage_store(const char* smem, uint16_t* dst, int ldd, int wave,
                                            int lane)
{
    const int col = (lane & 31) * 8;
#pragma unroll
    for (int it = 0; it < 16; it++) {
        const int row = wave * 32 + it * 2 + (lane >> 5);
        const v4i d = *(const v4i*)(smem + row * kStagePitch + col * 2);
        v4i* o = (v4i*)(dst + (size_t)row * ldd + col);
        if constexpr (NT)
            __builtin_nontemporal_store(d, o);
        else
            *o = d;
    }
}

__device__ __forceinline__ void slot_sync()
{
    __builtin_amdgcn_sched_barrier(0);
    wait_lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ v8i lds_frag(const char* p0, const char* p1)
{
    v4i x0 = *(const v4i*)p0;
    v4i x1 = *(const v4i*)p1;
    return (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
}

// Copy c (0, 1) of a row-major half tile writes LDS bytes c*8192 +
// wave*1024 + lane*16 = row c*64 + wave*8 + lane/8, slot lane%8, which holds
// K chunk slot ^ ((row >> 1) & 7). The chunk does not depend on c or on the
// half (64 and 128 rows keep (row >> 1) & 7). Returns this lane's row (of
// copy 0, half 0) and K chunk.
__device__ __forceinline__ void copy_lane(int wave, int lane, int& row, int& chunk)
{
    row = wave * 8 + (lane >> 3);
    chunk = (lane & 7) ^ ((row >> 1) & 7);
}

// Byte offsets, inside a 16-row block, of the two 16-byte chunks lane
// 16g + r reads for the MFMA (chunks g and g + 4 of row r). Adding multiples
// of 128 keeps bit 6, so the XOR commutes with the block offsets.
__device__ __forceinline__ void operand_lane(int lane, uint32_t& o0, uint32_t& o1)
{
    const uint32_t r = lane & 15, g = lane >> 4;
    o0 = r * 128 + ((g ^ ((r >> 1) & 7)) * 16);
    o1 = o0 ^ 64u;
}

} // namespace pp
} // namespace ga

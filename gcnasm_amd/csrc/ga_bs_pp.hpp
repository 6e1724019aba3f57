// ga_bs_pp.hpp -- pieces of the 256x256 eight-wave fp32-scaled FP8 GEMM
// (gemm_bs_pp.hip: one tile per workgroup; gemm_bs_sk.hip: stream-K) shared
// by both kernels: the LDS plan, the copies of A, B and the scales, the
// operand reads, the scale fold and one quadrant's MFMA slot.
#pragma once

#include "ga_device.hpp"
#include "ga_pp.hpp"

namespace ga {
namespace bspp {

using namespace pp;

enum { PS_GROUP128 = 0, PS_GROUP1 = 1, PS_TENSOR = 2 };

constexpr int kSSlot = 2048; // SFA (1 KB) + SFB (1 KB) of one K group
constexpr int kSRing = 4;    // scale slots: group s in slot s % 4
constexpr int kSBase = kOperandBytes;
constexpr int kLdsBs = kSBase + kSRing * kSSlot;
static_assert(kLdsBs <= 160 * 1024, "LDS budget");
constexpr int kBsGroupM = 4;
// fp32 epilogue staging: 128 rows of 1024 + 16 bytes (the 16 rows of one
// ds_write_b128 quarter-wave start 4 banks apart).
constexpr int kStagePitchF32 = 1040;

struct BsLoad {
    __amdgpu_buffer_rsrc_t ra, rb, rs; // rs: SFA (waves 0-3) or SFB (waves 4-7)
    uint32_t va, vb, vs;               // per-lane offsets (half 0, copy 0, K group 0)
    uint32_t a_hstep, b_hstep;         // bytes between copies 0 and 1 (64 rows)
    uint32_t s_kstep;                  // scale bytes per K group
};

// The copies take their wave-uniform offsets in the SGPR soffset: the
// VALU adds they cost as VGPR offsets sit in a loop whose time is VALU and
// MFMA issue (block scale 8192^3 on the reference driver's data 440.6 ->
// 437.4 us, 4096x2112x7168 77.6 -> 76.6 us on one box; the MXFP8 and MXFP4
// kernel ran slower that way and keeps VGPR offsets).
__device__ __forceinline__ void issue_a(const BsLoad& L, char* smem, int h, int t, int wave)
{
    char* dst = smem + kARegion + (t & 1) * kOpSlot + h * kHalf + wave * 1024;
    const uint32_t o = (uint32_t)h * 2 * L.a_hstep + (uint32_t)t * 128;
    lds_load16(L.ra, (lds_void*)dst, L.va, uni(o));
    lds_load16(L.ra, (lds_void*)(dst + 8192), L.va, uni(o + L.a_hstep));
}

__device__ __forceinline__ void issue_b(const BsLoad& L, char* smem, int h, int t, int wave)
{
    char* dst = smem + kBRegion + (t & 1) * kOpSlot + h * kHalf + wave * 1024;
    const uint32_t o = (uint32_t)h * 2 * L.b_hstep + (uint32_t)t * 128;
    lds_load16(L.rb, (lds_void*)dst, L.vb, uni(o));
    lds_load16(L.rb, (lds_void*)(dst + 8192), L.vb, uni(o + L.b_hstep));
}

// Scales of K group t into ring slot `ring`: one 4-byte copy per lane.
__device__ __forceinline__ void issue_s(const BsLoad& L, char* smem, int t, int ring, int wave)
{
    char* dst = smem + kSBase + ring * kSSlot + wave * 256;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(L.rs, (lds_void*)dst, 4, L.vs,
                                             uni((uint32_t)t * L.s_kstep), 0, 0);
}

struct BsRead {
    const char* a0;
    const char* a1;
    const char* b0;
    const char* b1;
    const char* sa; // this lane's four rows of group grp
    const char* sb; // GROUP_N 1: this lane's four columns of tile 0 (simd block)
};

template <int H>
__device__ __forceinline__ void read_a(const BsRead& rb, int slot, v8i (&a)[4])
{
    const int off = kARegion + slot * kOpSlot + H * kHalf;
#pragma unroll
    for (int i = 0; i < 4; i++)
        a[i] = lds_frag(rb.a0 + off + i * 2048, rb.a1 + off + i * 2048);
}

template <int H>
__device__ __forceinline__ void read_b(const BsRead& rb, int slot, v8i (&b)[2])
{
    const int off = slot * kOpSlot + H * kHalf; // base includes the B region
#pragma unroll
    for (int t = 0; t < 2; t++)
        b[t] = lds_frag(rb.b0 + off + t * 2048, rb.b1 + off + t * 2048);
}

// Scales of quadrant (HM, HN) of the K group in ring slot `ring`: this
// lane's four SFA rows and its SFB value(s).
struct ScaleVals {
    v4f sa;
    v4f sb0, sb1; // GROUP_N 1: columns of tiles 0 and 1; GROUP_N 128: sb0[0]
};

template <int MODE, int HM, int HN>
__device__ __forceinline__ ScaleVals read_scales(const BsRead& rb, int ring)
{
    ScaleVals v;
    if constexpr (MODE != PS_TENSOR) {
        v.sa = *(const v4f*)(rb.sa + ring * kSSlot + HM * 2 * 256);
        if constexpr (MODE == PS_GROUP128) {
            v.sb0[0] = *(const float*)(rb.sb + ring * kSSlot + HN * 4);
        } else {
            const char* sbp = rb.sb + ring * kSSlot + HN * 128 * 4;
            v.sb0 = *(const v4f*)sbp;
            v.sb1 = *(const v4f*)(sbp + 64);
        }
    }
    return v;
}

// acc += p * (SFA * SFB), the product rounded to fp32 first.
template <int MODE>
__device__ __forceinline__ void apply_scales(const ScaleVals& v, v4f (&acc)[4][2],
                                             const v4f (&p)[4][2])
{
    if constexpr (MODE == PS_GROUP128) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float s = v.sa[i] * v.sb0[0];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][t][j] = __builtin_fmaf(p[i][t][j], s, acc[i][t][j]);
        }
    } else if constexpr (MODE == PS_GROUP1) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc[i][0][j] = __builtin_fmaf(p[i][0][j], v.sa[i] * v.sb0[j], acc[i][0][j]);
                acc[i][1][j] = __builtin_fmaf(p[i][1][j], v.sa[i] * v.sb1[j], acc[i][1][j]);
            }
    }
}

// The tiles of a quadrant with t = 1 (GROUP_N 128), folded by the memory
// slot that follows the quadrant's MFMA slot when the fold is split.
template <int MODE>
__device__ __forceinline__ void apply_scales_t1(const ScaleVals& v, v4f (&acc)[4][2],
                                                const v4f (&p)[4][2])
{
    static_assert(MODE == PS_GROUP128, "split fold: one SFB value per quadrant");
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float s = v.sa[i] * v.sb0[0];
#pragma unroll
        for (int j = 0; j < 4; j++)
            acc[i][1][j] = __builtin_fmaf(p[i][1][j], s, acc[i][1][j]);
    }
}

// MFMA slot: the quadrant's 8 MFMAs (4 A tiles x 2 B tiles of one 128-K
// group; unit E8M0 scales). For the block-scale modes each MFMA writes a
// zeroed temporary p[i][t], and just before it the previous quadrant's
// p[i][t] is folded into its accumulator (acc += p * SFA*SFB): the VALU work
// of a tile issues while the MFMA pipe runs the previous tile's MFMA. With
// SPLIT only the t = 0 tiles are folded here; the memory slot before this
// one folded the t = 1 tiles (BS_MEM_SLOT_SPLIT). The B tiles alternate
// direction from one A tile to the next, so consecutive MFMAs differ in one
// operand (fewer operand bits change in the MFMA pipe; every tile's fold
// still comes just before its own MFMA).
template <int MODE, bool APPLY, bool SPLIT = false>
__device__ __forceinline__ void mma_quadrant(v4f (&acc)[4][2], v4f (&p)[4][2], const v8i (&a)[4],
                                             const v8i (&b)[2], v4f (&acc_prev)[4][2],
                                             const ScaleVals& sv)
{
    static_assert(!SPLIT || MODE == PS_GROUP128, "split fold: GROUP_N 128 only");
    __builtin_amdgcn_s_setprio(1);
    static_for<4>([&](auto I) {
        constexpr int i = decltype(I)::value;
        static_for<2>([&](auto T) {
            constexpr int t = (i & 1) ? 1 - decltype(T)::value : decltype(T)::value;
            constexpr bool fold = APPLY && !(SPLIT && t == 1);
            if constexpr (MODE == PS_TENSOR) {
                acc[i][t] = mfma_mx16<0, 0>(b[t], a[i], acc[i][t], 127, 127);
            } else {
                // keep the order fold(tile) -> MFMA(tile), tile by tile
                if constexpr (fold)
                    __builtin_amdgcn_sched_group_barrier(
                        0x2, MODE == PS_GROUP128 ? (t == 0 ? 5 : 4) : 8, 0);
                __builtin_amdgcn_sched_group_barrier(0x8, 1, 0);
                if constexpr (fold) {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float s = MODE == PS_GROUP128 ? sv.sa[i] * sv.sb0[0]
                                                            : sv.sa[i] * (t ? sv.sb1[j] : sv.sb0[j]);
                        acc_prev[i][t][j] = __builtin_fmaf(p[i][t][j], s, acc_prev[i][t][j]);
                    }
                }
                p[i][t] = mfma_mx16<0, 0>(b[t], a[i], (v4f){0.f, 0.f, 0.f, 0.f}, 127, 127);
            }
        });
    });
    __builtin_amdgcn_s_setprio(0);
}

// Memory slot: the copy, the scales of the quadrant the next MFMA slot
// folds in, then the operand read (the MFMA slot's first fold waits only for
// the scale reads, each MFMA only for its own operand), then the phase
// boundary.
#define BS_MEM_SLOT(HMP, HNP, RING, COPIES, READS, WAITN)                                    \
    {                                                                                        \
        COPIES;                                                                              \
        sv = read_scales<MODE, HMP, HNP>(rb, RING);                                          \
        __builtin_amdgcn_sched_barrier(0);                                                   \
        READS;                                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                   \
        phase_sync<WAITN>();                                                                 \
    }

// Memory slot of the split fold (GROUP_N 128): the scales of quadrant (HM,
// HN), which the coming MFMA slot computes, are read one memory slot ahead
// into `svn`; the scales read by the previous memory slot (`sv`) serve this
// slot's fold of the t = 1 tiles of ACCP, the quadrant the previous MFMA
// slot computed, after the operand reads, and the coming MFMA slot's fold of
// its t = 0 tiles. Half of the fold's VALU work so leaves the MFMA slot
// without delaying the operand reads.
#define BS_MEM_SLOT_SPLIT(HM, HN, RING, COPIES, READS, WAITN, ACCP, DOFOLD)                  \
    {                                                                                        \
        sv = svn;                                                                            \
        COPIES;                                                                              \
        svn = read_scales<MODE, HM, HN>(rb, RING);                                           \
        __builtin_amdgcn_sched_barrier(0);                                                   \
        READS;                                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                   \
        if (DOFOLD)                                                                          \
            apply_scales_t1<MODE>(sv, ACCP, p);                                              \
        __builtin_amdgcn_sched_barrier(0);                                                   \
        phase_sync<WAITN>();                                                                 \
    }

} // namespace bspp
} // namespace ga

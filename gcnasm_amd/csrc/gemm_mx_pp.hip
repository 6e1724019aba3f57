// gemm_mx_pp.hip -- 256x256 MXFP8 GEMM tile for large M and N (f4gemm ABI).
//
// Same contract as the 4-wave kernels of gemm_mx.hip (operands, shuffled
// scales, optional preshuffled B, split-K into an fp32 workspace); this file
// holds the high-throughput tile. Design:
//  * 512 threads = 8 waves in two groups. Wave w sits on SIMD w % 4, so each
//    SIMD runs one wave of each group. The groups execute the same program
//    offset by one barrier: while one group issues MFMAs (at raised issue
//    priority), the other does its LDS reads and global->LDS copies, and they
//    swap at every workgroup barrier, so the MFMA pipe of every SIMD is fed
//    by one wave while the other wave's memory work overlaps it.
//  * The 256x256 C tile is four 128x128 quadrants. In each quadrant a wave
//    owns 64 rows (by group) x 32 columns (by SIMD): 4 x 2 MFMA tiles of
//    16x16, 8 MFMAs of 16x16x128 per quadrant per K step, 128 accumulator
//    VGPRs in all.
//  * One K step (128) is two parts per group, two quadrants each: X = 00 +
//    01 (A rows of M half 0 with both B halves), Y = 10 + 11 (A half 1 with
//    the same B fragments). Each part is a memory half (copies, then the LDS
//    reads of the fragments the part multiplies: A0, B0 and B1 before X, A1
//    before Y) and an MFMA half (16 MFMAs); a group's memory half overlaps
//    the other group's MFMA half, so a SIMD's MFMA pipe changes waves twice
//    per K step per group (measured on MI355X, MXFP8 8192^3: 458 -> 403 us
//    against one quadrant per part).
//  * LDS: A and B each hold two K-step slots of two 16 KB half tiles, plus a
//    ring of three 4 KB scale slots: 140 KB. A half tile is refilled with the
//    step two ahead once both groups have read it (A1 one ahead); every
//    half-part ends with the same counted wait, vmcnt(8 + scale copies per
//    step) and lgkmcnt(0), then the workgroup barrier: the copies the next
//    half-part reads have landed in every wave, and every LDS read issued
//    before the barrier is complete before any copy issued after it.
//  * A shuffled scale dword covers 256 K, a pair of K steps, so a ring slot
//    holds one pair (8 A then 8 B 32-row blocks) and each step copies half of
//    the pair two ahead: one 4-byte-per-lane copy per wave per step.
//  * Row-major operands (A, and B without preshuffle) sit in LDS as 128-byte
//    rows, 16-byte K chunk c of row r at slot c ^ ((r >> 1) & 7). Each copy
//    instruction then reads 8 whole 128-byte rows (whole cache lines; a copy
//    touching 16 rows x 64 bytes moves half the bytes per request), and the
//    MFMA operand reads (lane 16g + r: row r, chunks g and g + 4) hit 64
//    distinct banks per 16 lanes.
//  * Preshuffled B keeps its global byte order in LDS: [K/16:8][row:16][16 B]
//    per 16-row group, so a copy is 1 KB contiguous and MFMA operand half h of
//    lane l is the 16 B at h*1024 + l*16.
//  * Addressing is kept out of VGPRs: one VGPR base per operand for the LDS
//    reads (slot and half are compile-time ds_read offsets) and one per
//    operand for the copies (uniform parts added from SGPRs).
#include "ga_device.hpp"
#include "ga_internal.hpp"
#include "ga_pp.hpp"

namespace ga {
namespace {

using namespace pp;

constexpr int kScaleSlot = 16 * 256; // 8 A + 8 B shuffled 32-row scale blocks
constexpr int kScaleBase = kOperandBytes;
constexpr int kLds = kScaleBase + 3 * kScaleSlot;
static_assert(kLds <= 160 * 1024, "LDS budget");
constexpr int kPpGroupM = 4;

struct PpLoad {
    __amdgpu_buffer_rsrc_t ra, rb, rsa, rsb;
    uint32_t va, vb;       // per-lane copy offsets (half 0, copy 0, first K step)
    uint32_t vsa, vsb;     // per-lane offsets of this wave's A / B scale block
    uint32_t a_hstep;      // A bytes between copies 0 and 1 of a half (64 rows)
    uint32_t b_hstep;      // same for B
    uint32_t b_kstep;      // B bytes per 128-K step
};

// Copies (2 per wave) of A half tile h of K step t.
__device__ __forceinline__ void issue_a(const PpLoad& L, char* smem, int h, int t, int wave)
{
    char* dst = smem + kARegion + (t & 1) * kOpSlot + h * kHalf + wave * 1024;
    const uint32_t o = (uint32_t)h * 2 * L.a_hstep + (uint32_t)t * 128;
    lds_load16(L.ra, (lds_void*)dst, L.va + uni(o), 0);
    lds_load16(L.ra, (lds_void*)(dst + 8192), L.va + uni(o + L.a_hstep), 0);
}

__device__ __forceinline__ void issue_b(const PpLoad& L, char* smem, int h, int t, int wave)
{
    char* dst = smem + kBRegion + (t & 1) * kOpSlot + h * kHalf + wave * 1024;
    const uint32_t o = (uint32_t)h * 2 * L.b_hstep + (uint32_t)t * L.b_kstep;
    lds_load16(L.rb, (lds_void*)dst, L.vb + uni(o), 0);
    lds_load16(L.rb, (lds_void*)(dst + 8192), L.vb + uni(o + L.b_hstep), 0);
}

// Half `half` (0: A rows, 1: B rows) of the shuffled scales of 256-K block
// `pair` (an MXFP8 step pair, one MXFP4 step) into ring slot `ring`: wave w
// copies 32-row block w of that operand.
__device__ __forceinline__ void issue_s(const PpLoad& L, char* smem, int pair, int half,
                                        int ring, int wave)
{
    char* dst = smem + kScaleBase + ring * kScaleSlot + half * 2048 + wave * 256;
    const uint32_t q = (uint32_t)pair * 256;
    const __amdgpu_buffer_rsrc_t r = half ? L.rsb : L.rsa;
    const uint32_t v = half ? L.vsb : L.vsa;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 4, v + uni(q), 0, 0, 0);
}

// Per-lane LDS read bases. Swizzled row-major operand: lane 16g + r reads
// row r, chunks g (at o) and g + 4 (at o ^ 64; adding multiples of 128 keeps
// bit 6, so the XOR commutes with the block offsets).
struct ReadBase {
    const char* a0;
    const char* a1;
    const char* b0;
    const char* b1;
    const char* sa;
    const char* sb;
};

// A fragment of slot `slot`, half H: rows H*128 + grp*64 + [0, 64).
template <int H>
__device__ __forceinline__ void read_a(const ReadBase& rb, int slot, v8i (&a)[4])
{
    const int off = kARegion + slot * kOpSlot + H * kHalf;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[i] = lds_frag(rb.a0 + off + i * 2048, rb.a1 + off + i * 2048);
        __builtin_amdgcn_sched_barrier(0); // issue in MFMA order: counted waits
    }
}

// B fragment of slot `slot`, half H: columns H*128 + simd*32 + [0, 32).
template <int H>
__device__ __forceinline__ void read_b(const ReadBase& rb, int slot, v8i (&b)[2])
{
    const int off = slot * kOpSlot + H * kHalf; // base includes the B region
#pragma unroll
    for (int t = 0; t < 2; t++)
        b[t] = lds_frag(rb.b0 + off + t * 2048, rb.b1 + off + t * 2048);
}

// Scales of ring slot `ring`. Byte 2*d4 + d1 of a shuffled dword holds
// 128-K half d4 (the step's parity) of 16-row half d1: a 16-bit read at byte
// offset `hb` = 2 * parity lands this step's two bytes in bits 0-15, straight
// into the MFMA scale operand (no ALU op between the read and the MFMA).
// MXFP4 steps are 256 K: the whole dword (both 128-K halves) is read.
template <int H, bool FP4>
__device__ __forceinline__ void read_sa(const ReadBase& rb, int ring, uint32_t hb,
                                        uint32_t (&s)[2])
{
    const char* p = rb.sa + ring * kScaleSlot + H * 4 * 256 + hb;
    if constexpr (FP4) {
        s[0] = *(const uint32_t*)p;
        s[1] = *(const uint32_t*)(p + 256);
    } else {
        s[0] = *(const uint16_t*)p;
        s[1] = *(const uint16_t*)(p + 256);
    }
}

template <int H, bool FP4>
__device__ __forceinline__ uint32_t read_sb(const ReadBase& rb, int ring, uint32_t hb)
{
    const char* p = rb.sb + ring * kScaleSlot + H * 4 * 256 + hb;
    if constexpr (FP4)
        return *(const uint32_t*)p;
    else
        return *(const uint16_t*)p;
}

// Quadrant MFMAs: 4 A tiles x 2 B tiles; the scale byte is 2*(128-K half) +
// (16-row half inside the 32-row scale block). MXFP8: one MFMA per tile (the
// step's 128 K; its half is in bytes 0-1 of the scale operands). MXFP4: the
// fragment's first 16 bytes per lane are K [0, 128) of the 256-K step and
// its last 16 bytes K [128, 256): two MFMAs per tile, halves 0 and 1.
// The kernel-argument fields a tile uses (names as in ga_f4gemm_kargs), read
// once at kernel entry and made wave-uniform: the compiler fetches this large
// by-value argument with vector loads, and every address derived from a VGPR
// copy would need its own VGPRs and readfirstlanes in the K loop.
struct PpArgs {
    const void* ptr_A;
    const void* ptr_B;
    const void* ptr_ScaleA;
    const void* ptr_ScaleB;
    const void* ptr_C;
    void* ptr_D;
    float alpha, beta;
    uint32_t M, N, K, stride_A0, stride_B0, stride_ScaleA0, stride_ScaleB0, stride_C0;
    int log2_k_split;
};

// One 256x256 output tile (K slice blockIdx.z): prologue, K loop, epilogue.
// On return every LDS read of the tile is complete (the last barrier is
// after the last read); copies of steps past the slice may still be landing,
// each into the LDS bytes its own wave writes first in the next tile.
//
// MXFP4 (FP4): elements are packed two per byte (low nibble first); strides
// and K count elements. A K step is 256 elements = the same 128 bytes per row
// as an MXFP8 step, so copies, LDS layout and fragment reads are shared; a
// step reads one whole shuffled scale dword per 32-row block.
// Two quadrants with shared A fragments: acc0 += A x B0, acc1 += A x B1
// (16 MFMAs at raised issue priority).
// MXFP8 with whole scale dwords: SB = 2 * (128-K half) selects the step's
// bytes in the operand (0 when the step's two bytes were read into 0-15).
// Issue order: A tiles 0-3 in the first quadrant and 3-0 in the second, B
// tiles alternating direction, so consecutive MFMAs differ in one operand
// (the MFMA pipe's power falls with the operand bits that change: MXFP8
// 8192^3 375.3 -> 370.6 us, 4096^3 55.0 -> 54.3 us on one box, best of
// 5 x 100 calls; each accumulator's K order, and so the output, unchanged).
template <bool FP4, int F, int SB = 0>
__device__ __forceinline__ void mma_two(v4f (&acc0)[4][2], v4f (&acc1)[4][2], const v8i (&a)[4],
                                        const v8i (&b0)[2], const v8i (&b1)[2],
                                        const uint32_t (&sa)[2], uint32_t sb0, uint32_t sb1)
{
    __builtin_amdgcn_s_setprio(1);
    auto quadrant = [&](v4f (&acc)[4][2], const v8i (&b)[2], uint32_t sb, auto REV) {
        static_for<4>([&](auto I) {
            constexpr int pos = decltype(I)::value;
            constexpr int i = decltype(REV)::value ? 3 - pos : pos;
            static_for<2>([&](auto T) {
                constexpr int t = (pos & 1) ? 1 - decltype(T)::value : decltype(T)::value;
                if constexpr (FP4) {
                    acc[i][t] = mfma_mx16_fp4<(t & 1), (i & 1)>(b[t], a[i], acc[i][t], (int)sb,
                                                                (int)sa[i >> 1]);
                    acc[i][t] = mfma_mx16_fp4<2 + (t & 1), 2 + (i & 1)>(
                        hi16(b[t]), hi16(a[i]), acc[i][t], (int)sb, (int)sa[i >> 1]);
                } else {
                    acc[i][t] = mfma_mx16<SB + (t & 1), SB + (i & 1), fmt_of_b(F), fmt_of_a(F)>(
                        b[t], a[i], acc[i][t], (int)sb, (int)sa[i >> 1]);
                }
            });
        });
    };
    quadrant(acc0, b0, sb0, std::integral_constant<int, 0>{});
    quadrant(acc1, b1, sb1, std::integral_constant<int, 1>{});
    __builtin_amdgcn_s_setprio(0);
}

// Half-part boundary: own copies older than the last N landed, own LDS reads
// complete, then the workgroup barrier.
template <int N>
__device__ __forceinline__ void part_sync()
{
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<N>();
    wait_lgkmcnt0();
    wait_lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

template <bool BPS, bool FP4, int F>
__device__ __forceinline__ void pp_tile(const PpArgs& args, float* __restrict__ ws,
                                        char* smem, int tile_m, int tile_n)
{
    constexpr int kEPB = FP4 ? 2 : 1;       // elements per byte
    constexpr int kStepK = 128 * kEPB;      // elements per K step
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2, simd = wave & 3;
    const int M = (int)args.M, N = (int)args.N, K = (int)args.K;
    const int m0 = tile_m * 256, n0 = tile_n * 256;

    const int z = blockIdx.z, gdz = gridDim.z;
    int kpt = K;
    if (gdz > 1)
        kpt = ((K >> args.log2_k_split) + 255) / 256 * 256;
    const int kb = z * kpt;
    const int ke = min(K, kb + kpt);
    const int nsteps = (ke - kb) / kStepK;
    const int kbb = kb / kEPB; // byte offset of the slice in a row

    v4f acc[4][4][2];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int t = 0; t < 2; t++)
                acc[q][i][t] = (v4f){0.f, 0.f, 0.f, 0.f};

    if (nsteps > 0) {
        const uint32_t lda = args.stride_A0 / kEPB, ldb = args.stride_B0 / kEPB; // bytes
        const int Kb = K / kEPB;                                                  // bytes
        PpLoad L;
        // Copy c of a row-major half tile writes LDS bytes c*8192 + wave*1024
        // + lane*16 = row c*64 + wave*8 + lane/8, slot lane%8, which holds K
        // chunk slot ^ ((row >> 1) & 7); the chunk does not depend on c or
        // the half (64 and 128 rows keep (row >> 1) & 7).
        int crow, ckc;
        copy_lane(wave, lane, crow, ckc);
        {
            const char* pa = (const char*)args.ptr_A + (size_t)m0 * lda;
            long long abytes = (long long)(M - m0) * lda;
            L.ra = make_rsrc(pa, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
            L.va = (uint32_t)crow * lda + ckc * 16 + (uint32_t)kbb;
            L.a_hstep = 64 * lda;
            if (BPS) {
                // preshuffled B: each 16-row group is Kb*16 contiguous bytes,
                // [Kb/16][16 rows][16 B]; one K step is 2 KB of it. Copy c of
                // half h: groups h*8 + c*4 + wave/2, bytes (wave&1)*1024 + lane*16.
                const char* pb = (const char*)args.ptr_B + (size_t)(n0 / 16) * Kb * 16;
                long long bbytes = (long long)(N - n0) * Kb;
                L.rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
                L.b_kstep = 2048;
                L.b_hstep = 4 * (uint32_t)Kb * 16;
                L.vb = (uint32_t)(wave >> 1) * (uint32_t)Kb * 16 + (wave & 1) * 1024 +
                       lane * 16 + (uint32_t)kbb * 16;
            } else {
                const char* pb = (const char*)args.ptr_B + (size_t)n0 * ldb;
                long long bbytes = (long long)(N - n0) * ldb;
                L.rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
                L.b_kstep = 128;
                L.b_hstep = 64 * ldb;
                L.vb = (uint32_t)crow * ldb + ckc * 16 + (uint32_t)kbb;
            }
            // scales: shuffled layout, 256-byte block per (32 rows, 256 K);
            // wave w copies block w of the tile's 8 A and 8 B blocks
            const uint32_t sna = args.stride_ScaleA0, snb = args.stride_ScaleB0;
            L.rsa = make_rsrc(args.ptr_ScaleA, (uint32_t)((M + 31) / 32 * 32) * sna);
            L.rsb = make_rsrc(args.ptr_ScaleB, (uint32_t)((N + 31) / 32 * 32) * snb);
            L.vsa = ((uint32_t)(m0 / 32 + wave) * (sna / 8) + (uint32_t)(kb / 256)) * 256 +
                    lane * 4;
            L.vsb = ((uint32_t)(n0 / 32 + wave) * (snb / 8) + (uint32_t)(kb / 256)) * 256 +
                    lane * 4;
        }

        ReadBase rb;
        {
            uint32_t o, o64;
            operand_lane(lane, o, o64);
            rb.a0 = smem + grp * 64 * 128 + o;
            rb.a1 = smem + grp * 64 * 128 + o64;
            if (BPS) {
                rb.b0 = smem + kBRegion + simd * 32 * 128 + lane * 16;
                rb.b1 = rb.b0 + 1024;
            } else {
                rb.b0 = smem + kBRegion + simd * 32 * 128 + o;
                rb.b1 = smem + kBRegion + simd * 32 * 128 + o64;
            }
            rb.sa = smem + kScaleBase + grp * 2 * 256 + lane * 4;
            rb.sb = smem + kScaleBase + (8 + simd) * 256 + lane * 4;
        }

        // Operand fragments: rows of one A half, B columns of N half 0 / 1,
        // with their scale dwords.
        v8i fa[4], fb0[2], fb1[2];
        uint32_t sa[2], sb0, sb1;

        // Prologue: the copies a steady pipeline would have issued before
        // step 0, in the same order (Y of steps -2 and -1, X of step -1),
        // MXFP8 preceded by both halves of the scales of pair 0: A0, B0, B1
        // + scales of step 0 (MXFP8: half 0 of pair 1), A1 of step 0, A0,
        // B0, B1 + scales of step 1 (MXFP8: half 1 of pair 1).
        constexpr int kS = FP4 ? 2 : 1; // scale copies per step
        if constexpr (!FP4) {
            issue_s(L, smem, 0, 0, 0, wave);
            issue_s(L, smem, 0, 1, 0, wave);
        }
        issue_a(L, smem, 0, 0, wave);
        issue_b(L, smem, 0, 0, wave);
        issue_b(L, smem, 1, 0, wave);
        if constexpr (FP4) {
            issue_s(L, smem, 0, 0, 0, wave);
            issue_s(L, smem, 0, 1, 0, wave);
        } else {
            issue_s(L, smem, 1, 0, 1, wave);
        }
        issue_a(L, smem, 1, 0, wave);
        issue_a(L, smem, 0, 1, wave);
        issue_b(L, smem, 0, 1, wave);
        issue_b(L, smem, 1, 1, wave);
        if constexpr (FP4) {
            issue_s(L, smem, 1, 0, 1, wave);
            issue_s(L, smem, 1, 1, 1, wave);
        } else {
            issue_s(L, smem, 1, 1, 1, wave);
        }
        // (also retires pending scalar loads: with one in flight the
        // compiler cannot count LDS reads inside the loop)
        part_sync<8 + kS>();
        if (grp == 1)
            slot_sync(); // second group runs one barrier behind

        // Step s of parity P (LDS slot P), per group:
        //   X memory: copy A1(s+1) (2 per wave); read the scales, A0(s),
        //             B0(s), B1(s)
        //   X MFMA:   quadrants 00, 01
        //   Y memory: copy A0(s+2), B0(s+2), B1(s+2) (6) and the scales S;
        //             read A1(s)
        //   Y MFMA:   quadrants 10, 11
        // A copy writes a slot both groups last read at least one barrier
        // earlier (reads complete at every barrier). Every half-part ends
        // with vmcnt(8 + kS): after X memory that retires X(s-1), i.e.
        // A1(s), read in Y; after Y memory, Y(s-1): A0, B0, B1 of step s+1
        // and (copied at least as early) its scales, read in X of step s+1.
        // MXFP8: S is half P of the scales of pair (s >> 1) + 2, into ring
        // slot r2 (that of pair (s >> 1) - 1, last read in step s - 1);
        // MXFP4: both halves of the scales of step s + 2, into ring slot
        // (s + 2) % 3 (that of step s - 1).
        int r0 = 0; // scale ring slot of step s (MXFP8: of pair s >> 1)
        if constexpr (!FP4) {
            // MXFP8, a pair of steps per iteration: the even step reads the
            // pair's whole scale dwords (both 128-K halves; both halves of
            // the pair were copied before step s - 1 ended), the odd step
            // selects its bytes in the same registers (op_sel 2, 3), so
            // scales are read once per pair instead of once per step.
            uint32_t sy[2]; // A scales of M half 1
            auto step = [&](int s, auto PC) {
                constexpr int P = decltype(PC)::value;
                const int r2 = r0 == 0 ? 2 : r0 - 1; // (r0 + 2) % 3
                // X
                issue_a(L, smem, 1, s + 1, wave);
                if constexpr (P == 0) {
                    read_sa<0, true>(rb, r0, 0u, sa);
                    sb0 = read_sb<0, true>(rb, r0, 0u);
                    sb1 = read_sb<1, true>(rb, r0, 0u);
                }
                read_a<0>(rb, P, fa);
                read_b<0>(rb, P, fb0);
                read_b<1>(rb, P, fb1);
                part_sync<8 + kS>();
                mma_two<FP4, F, 2 * P>(acc[0], acc[1], fa, fb0, fb1, sa, sb0, sb1);
                part_sync<8 + kS>();
                // Y
                issue_a(L, smem, 0, s + 2, wave);
                issue_b(L, smem, 0, s + 2, wave);
                issue_b(L, smem, 1, s + 2, wave);
                issue_s(L, smem, (s >> 1) + 2, P, r2, wave);
                if constexpr (P == 0)
                    read_sa<1, true>(rb, r0, 0u, sy);
                read_a<1>(rb, P, fa);
                part_sync<8 + kS>();
                mma_two<FP4, F, 2 * P>(acc[2], acc[3], fa, fb0, fb1, sy, sb0, sb1);
                part_sync<8 + kS>();
                if constexpr (P == 1)
                    r0 = r0 == 2 ? 0 : r0 + 1;
            };
            for (int s = 0; s < nsteps; s += 2) {
                step(s, std::integral_constant<int, 0>{});
                if (s + 1 < nsteps)
                    step(s + 1, std::integral_constant<int, 1>{});
            }
        } else {
            // MXFP4: one ring slot per step; two steps per iteration, so the
            // LDS slot P is a compile-time read offset (no VALU add per read
            // base)
            auto step4 = [&](int s, auto PC) {
                constexpr int P = decltype(PC)::value;
                const int r1 = r0 == 2 ? 0 : r0 + 1; // slot of step s + 1
                const int r2 = r0 == 0 ? 2 : r0 - 1; // (r0 + 2) % 3
                // X
                issue_a(L, smem, 1, s + 1, wave);
                read_sa<0, FP4>(rb, r0, 0u, sa);
                sb0 = read_sb<0, FP4>(rb, r0, 0u);
                sb1 = read_sb<1, FP4>(rb, r0, 0u);
                read_a<0>(rb, P, fa);
                read_b<0>(rb, P, fb0);
                read_b<1>(rb, P, fb1);
                part_sync<8 + kS>();
                mma_two<FP4, F>(acc[0], acc[1], fa, fb0, fb1, sa, sb0, sb1);
                part_sync<8 + kS>();
                // Y
                issue_a(L, smem, 0, s + 2, wave);
                issue_b(L, smem, 0, s + 2, wave);
                issue_b(L, smem, 1, s + 2, wave);
                issue_s(L, smem, s + 2, 0, r2, wave);
                issue_s(L, smem, s + 2, 1, r2, wave);
                read_sa<1, FP4>(rb, r0, 0u, sa);
                read_a<1>(rb, P, fa);
                part_sync<8 + kS>();
                mma_two<FP4, F>(acc[2], acc[3], fa, fb0, fb1, sa, sb0, sb1);
                part_sync<8 + kS>();
                r0 = r1;
            };
            int s = 0;
            for (; s + 1 < nsteps; s += 2) {
                step4(s, std::integral_constant<int, 0>{});
                step4(s + 1, std::integral_constant<int, 1>{});
            }
            if (s < nsteps)
                step4(s, std::integral_constant<int, 0>{});
        }
        if (grp == 0)
            slot_sync(); // matches the second group's extra barrier
    }

    // Epilogue: lane holds C[m][n .. n+3] of each 16x16 tile. The library is
    // built with -ffp-contract=off: alpha*v and + beta*c round separately.
    const int ldd = (int)args.stride_C0;
    const float alpha = args.alpha, beta = args.beta;
    const bool use_c = beta != 0.0f && args.ptr_C != nullptr;
    // Whole interior tiles without C go through LDS (whole-row stores).
    const bool staged = gdz == 1 && !use_c && m0 + 256 <= M && n0 + 256 <= N &&
                        (ldd & 7) == 0 && ((uintptr_t)args.ptr_D & 15) == 0;
    if (staged) {
        static_assert(kStageBytes <= kLds, "staging fits in LDS");
        wait_vmcnt<0>();   // copies of steps past the slice have landed
        wait_lds_barrier(); // ... in every wave, and every operand read is done
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const v4f v = acc[q][i][t];
                    const uint32_t lo = (uint32_t)f32_to_bf16(alpha * v[0]) |
                                        ((uint32_t)f32_to_bf16(alpha * v[1]) << 16);
                    const uint32_t hi = (uint32_t)f32_to_bf16(alpha * v[2]) |
                                        ((uint32_t)f32_to_bf16(alpha * v[3]) << 16);
                    stage_put(smem, (q >> 1) * 128 + grp * 64 + i * 16 + (lane & 15),
                              (q & 1) * 128 + simd * 32 + t * 16 + (lane >> 4) * 4, lo, hi);
                }
        barrier_lds();
        stage_store(smem, (uint16_t*)args.ptr_D + (size_t)m0 * ldd + n0, ldd, wave, lane);
        barrier_lds(); // staged rows read before the LDS takes the next tile's copies
        return;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + (q >> 1) * 128 + grp * 64 + i * 16 + (lane & 15);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int n = n0 + (q & 1) * 128 + simd * 32 + t * 16 + (lane >> 4) * 4;
                if (m >= M || n >= N)
                    continue;
                const v4f v = acc[q][i][t];
                if (gdz > 1) {
                    *(v4f*)(ws + ((size_t)z * M + m) * N + n) = v;
                } else {
                    uint16_t o[4];
                    const uint16_t* cin =
                        use_c ? (const uint16_t*)args.ptr_C + (size_t)m * ldd + n : nullptr;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float x = alpha * v[j];
                        if (use_c)
                            x = x + beta * bf16_to_f32(cin[j]);
                        o[j] = f32_to_bf16(x);
                    }
                    uint2 pk;
                    pk.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
                    pk.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
                    *(uint2*)((uint16_t*)args.ptr_D + (size_t)m * ldd + n) = pk;
                }
            }
        }
    }
}

// Persistent grid: workgroup b computes tiles b, b + gridDim.x, ... of the
// tiles_x x tiles_y tile grid (gridDim.x a multiple of 8, or all tiles in one
// pass, so each workgroup stays on the XCD map_tile assigns its tiles to).
// The epilogue stores of one tile drain while the next tile's first copies
// are in flight, instead of behind a workgroup exit and a new launch.
// F: the operands' 8-bit element formats (fmt_of_a / fmt_of_b; 0 for MXFP4).
template <bool BPS, bool FP4, int F = 0>
__global__ __attribute__((amdgpu_flat_work_group_size(kNT, kNT), amdgpu_waves_per_eu(2, 2)))
void mx_pp_kernel(ga_f4gemm_kargs args, float* __restrict__ ws,
                  const ga_splitk_ws_handle* __restrict__ wsh, int tiles_x, int tiles_y)
{
    __shared__ __attribute__((aligned(1024))) char smem[kLds];
    if (wsh && !(ws = resolve_ws(wsh, gridDim.z, args.M, args.N)))
        return; // workspace slot shorter than the split-K layout: write nothing
    PpArgs a;
    a.ptr_A = uni_ptr(args.ptr_A);
    a.ptr_B = uni_ptr(args.ptr_B);
    a.ptr_ScaleA = uni_ptr(args.ptr_ScaleA);
    a.ptr_ScaleB = uni_ptr(args.ptr_ScaleB);
    a.ptr_C = uni_ptr(args.ptr_C);
    a.ptr_D = uni_ptr(args.ptr_D);
    a.alpha = args.alpha; // epilogue VALU operands: may stay in VGPRs
    a.beta = args.beta;
    a.M = uni(args.M);
    a.N = uni(args.N);
    a.K = uni(args.K);
    a.stride_A0 = uni(args.stride_A0);
    a.stride_B0 = uni(args.stride_B0);
    a.stride_ScaleA0 = uni(args.stride_ScaleA0);
    a.stride_ScaleB0 = uni(args.stride_ScaleB0);
    a.stride_C0 = uni(args.stride_C0);
    a.log2_k_split = (int)uni((uint32_t)args.log2_k_split);
    const int ntiles = tiles_x * tiles_y;
    for (int lin = blockIdx.x; lin < ntiles; lin += gridDim.x) {
        int tile_m, tile_n;
        map_tile_lin(lin, tiles_x, tiles_y, kPpGroupM, tile_m, tile_n);
        pp_tile<BPS, FP4, F>(a, ws, smem, tile_m, tile_n);
    }
    wait_vmcnt<0>(); // copies of steps past the last slice land before exit
}

} // namespace

namespace {

// Workgroups per K slice: one per CU (rounded down to a multiple of 8) when
// the tiles outnumber the CUs, else one per tile.
int pp_grid(int tiles)
{
    int cu = 0;
    if (device_cu_count(&cu) != 0 || cu < 8)
        return tiles;
    const int g = cu / 8 * 8;
    return tiles > g ? g : tiles;
}

} // namespace

void launch_mx_pp_bps(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                      int gdx, int gdy, int gdz, hipStream_t stream)
{
    hipLaunchKernelGGL((mx_pp_kernel<true, false>), dim3(pp_grid(gdx * gdy), 1, gdz), dim3(kNT),
                       0, stream, args, ws, wsh, gdx, gdy);
}

void launch_mx_pp_nobps(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                        int gdx, int gdy, int gdz, hipStream_t stream)
{
    hipLaunchKernelGGL((mx_pp_kernel<false, false>), dim3(pp_grid(gdx * gdy), 1, gdz), dim3(kNT),
                       0, stream, args, ws, wsh, gdx, gdy);
}

void launch_mx4_pp_bps(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                       int gdx, int gdy, int gdz, hipStream_t stream)
{
    hipLaunchKernelGGL((mx_pp_kernel<true, true>), dim3(pp_grid(gdx * gdy), 1, gdz), dim3(kNT),
                       0, stream, args, ws, wsh, gdx, gdy);
}

void launch_mx4_pp_nobps(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                         int gdx, int gdy, int gdz, hipStream_t stream)
{
    hipLaunchKernelGGL((mx_pp_kernel<false, true>), dim3(pp_grid(gdx * gdy), 1, gdz), dim3(kNT),
                       0, stream, args, ws, wsh, gdx, gdy);
}

namespace {

template <bool BPS, int F>
void launch_pp_f(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh, int gdz,
                 hipStream_t stream)
{
    const int gdx = ((int)args.N + 255) / 256, gdy = ((int)args.M + 255) / 256;
    hipLaunchKernelGGL((mx_pp_kernel<BPS, false, F>), dim3(pp_grid(gdx * gdy), 1, gdz), dim3(kNT),
                       0, stream, args, ws, wsh, gdx, gdy);
}

} // namespace

void launch_mx_pp_fmt(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                      int gdz, bool bps, int fmt, hipStream_t stream)
{
    switch (fmt) {
    case 1: bps ? launch_pp_f<true, 1>(args, ws, wsh, gdz, stream)
                : launch_pp_f<false, 1>(args, ws, wsh, gdz, stream); break;
    case 2: bps ? launch_pp_f<true, 2>(args, ws, wsh, gdz, stream)
                : launch_pp_f<false, 2>(args, ws, wsh, gdz, stream); break;
    case 3: bps ? launch_pp_f<true, 3>(args, ws, wsh, gdz, stream)
                : launch_pp_f<false, 3>(args, ws, wsh, gdz, stream); break;
    default: bps ? launch_pp_f<true, 0>(args, ws, wsh, gdz, stream)
                 : launch_pp_f<false, 0>(args, ws, wsh, gdz, stream); break;
    }
}

} // namespace ga

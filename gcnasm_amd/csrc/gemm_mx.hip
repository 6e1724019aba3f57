// gemm_mx.hip -- MXFP8 GEMM for gfx950 behind the f4gemm kernarg ABI.
//
//   D[M, N] bf16 = alpha * A[M, K] * B[N, K]^T (+ beta * C)
//   A, B: OCP E4M3; one E8M0 scale per 1x32 K-block of each row, stored
//   padded + shuffled (f4gemm_ref.hpp:98-130); B optionally preshuffled in
//   16x16-byte subtiles (f4gemm_ref.hpp:78-96).
//
// Kernel design (gfx950, wave64, 256 threads = 4 waves):
//  * block tile BM x BN, K step 128; waves in a WAVES_M x WAVES_N grid, each
//    owning (BM/WAVES_M) x (BN/WAVES_N) of C as 16x16 MFMA tiles.
//  * A and B are staged in LDS with buffer_load ... lds (16 B per lane,
//    out-of-range rows read as zero), 2-4 stages. Row-major operands (A, and
//    B when not preshuffled) sit as 128-byte rows with 16-byte K chunk c of
//    row r at slot c ^ ((r >> 1) & 7): each copy instruction fetches 8 whole
//    rows (full 128-byte lines), and the operand reads are conflict-free.
//    Preshuffled B keeps its own byte order, 2 KB per 16-row x 128-K group
//    ordered [K/16:8][row:16][16 B], so it is a linear copy.
//  * MFMA operand layout of v_mfma_scale_f32_16x16x128_f8f6f4 (fp8): lane
//    l = 16*g + r holds row r; its VGPRs 0-3 carry K [16g, 16g+16) and VGPRs
//    4-7 carry K [64+16g, 64+16g+16): chunks g and g + 4 of row r (for
//    preshuffled B, the 1 KB halves at l*16 and 1024 + l*16).
//    The E8M0 scale in lane 16*b + r applies to row r, K [32b, 32b+32).
//  * v_mfma_scale_f32_16x16x128_f8f6f4 with operands swapped (B rows feed
//    the MFMA's A side) so each lane ends up with 4 consecutive N outputs of
//    one C row -> 8-byte bf16 stores.
//  * The shuffled scale layout puts, for each 32 rows x 256 K, the scales of
//    lane l (row l%16, K-block l/16) in dword l; the byte inside the dword
//    (row half, 128-K half) is picked with the MFMA's op_sel.
//  * Preshuffled-B entries with 32 or 64 rows (32x256, 64x256, 32x512) run a
//    B-streaming tile instead: waves side by side along N, B loaded straight
//    into the MFMA operand registers 4 steps deep, only A and the scales in
//    LDS (mx_bstream_kernel).
//  * Split-K (gdz > 1): each K slice writes fp32 partials to a workspace;
//    the reduce kernel sums the slices in order and applies the epilogue.
//  * Tile order: workgroup ids are dispatched round-robin over the 8 XCDs;
//    they are remapped so each XCD works on a contiguous, M-grouped range of
//    tiles and shares A/B panels in its own L2.
#include "ga_device.hpp"
#include "ga_internal.hpp"
#include "ga_pp.hpp"

#include <atomic>
#include <cstdio>
#include <cstring>
#include <deque>
#include <mutex>
#include <string>
#include <vector>

namespace ga {

template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, bool BPS_, int NS_ = 2, bool FP4_ = false>
struct MxCfg {
    static constexpr int BM = BM_, BN = BN_;
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr bool BPS = BPS_;
    // MXFP4: e2m1 packed two per byte; a step is 256 K = the same 128 bytes
    // per row, so copies and LDS layouts are the MXFP8 ones
    static constexpr bool FP4 = FP4_;
    static constexpr int EPB = FP4 ? 2 : 1;
    static constexpr int NS = NS_; // LDS stages in flight
    static constexpr int NT = 256;
    static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    static constexpr int TM = WTM / 16, TN = WTN / 16;
    static constexpr int SM = TM / 2, SN = TN / 2; // scale dwords: one per 32 rows
    static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
    // E8M0 scales travel with each stage: one 256-byte shuffled block per 32
    // rows of A and of B (all 4 x 16 MFMA lanes' dwords), copied by the waves
    // in turn (padded to a multiple of 4 with repeats of block 0).
    static constexpr int SBLK = BM / 32 + BN / 32;
    static constexpr int S_LOADS = (SBLK + 3) / 4; // per wave per stage
    static constexpr int S_BYTES = 4 * S_LOADS * 256;
    static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
    static constexpr int LDS = NS * STAGE;
    // Two workgroups per CU when two fit in LDS: with more tiles than CUs the
    // second one's copies and MFMAs fill the first one's waits.
    static constexpr int WPE = 2 * LDS <= 160 * 1024 ? 2 : 1;
    static constexpr int A_LOADS = A_BYTES / (NT * 16);
    static constexpr int B_LOADS = B_BYTES / (NT * 16);
    static constexpr int TILE_LOADS = A_LOADS + B_LOADS + S_LOADS; // vmem ops per stage
    static_assert(WAVES_M * WAVES_N == 4, "4 waves");
    // 32-aligned wave tiles: the row half of each 16-row MFMA tile inside a
    // 32-row scale block is (tile index & 1), known at compile time.
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile multiple of 32");
    static_assert(A_BYTES % (NT * 16) == 0 && B_BYTES % (NT * 16) == 0, "tile >= 32 rows");
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(NS >= 2 && TILE_LOADS * (NS - 2) < 64, "vmcnt range");
};

constexpr int kGroupM = 4; // M-tiles per L2 group

template <class C>
struct MxState {
    __amdgpu_buffer_rsrc_t ra, rb, rsa, rsb;
    uint32_t voff_a[C::A_LOADS];
    uint32_t voff_b[C::B_LOADS];
    uint32_t soff[C::S_LOADS]; // scale dword offset of this wave's blocks (first K group)
    bool sfrom_b[C::S_LOADS];  // block is a B block (else A)
    uint32_t b_kstride;        // bytes per K step of 128 in B
};

// Direct-to-LDS copy of step `step` of the slice (byte offset kk inside a
// row, a multiple of 128) into stage `buf`: A and B tiles, then this wave's
// scale blocks. The scale dword covers 256 K: MXFP8 steps use bytes
// 2*d4 + d1 (d4 = step & 1, d1 = 16-row half), an MXFP4 step all four.
template <class C>
__device__ __forceinline__ void issue_stage(const MxState<C>& st, char* smem, int buf, int step,
                                            int kk, int wave)
{
    char* sa = smem + buf * C::STAGE;
    char* sb = sa + C::A_BYTES;
    char* ss = sb + C::B_BYTES;
#pragma unroll
    for (int i = 0; i < C::A_LOADS; i++)
        lds_load16(st.ra, (lds_void*)(sa + (i * 256 + wave * 64) * 16), st.voff_a[i] + kk, 0);
#pragma unroll
    for (int i = 0; i < C::B_LOADS; i++)
        lds_load16(st.rb, (lds_void*)(sb + (i * 256 + wave * 64) * 16),
                   st.voff_b[i] + (uint32_t)(kk / 128) * st.b_kstride, 0);
    const uint32_t q = (uint32_t)(C::FP4 ? step : (step >> 1)) * 256;
#pragma unroll
    for (int i = 0; i < C::S_LOADS; i++) {
        lds_void* dst = (lds_void*)(ss + (wave * C::S_LOADS + i) * 256);
        if (st.sfrom_b[i])
            __builtin_amdgcn_raw_ptr_buffer_load_lds(st.rsb, dst, 4, st.soff[i] + q, 0, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(st.rsa, dst, 4, st.soff[i] + q, 0, 0, 0);
    }
}

// Operand fragments and scale dwords of one K step.
template <class C>
struct MxFrag {
    uint32_t sa[C::SM], sb[C::SN];
    v8i af[C::TM], bf[C::TN];
};

template <class C>
__device__ __forceinline__ void read_stage(const char* smem, int buf, int step, int wm, int wn,
                                           int lane, MxFrag<C>& f)
{
    const char* la = smem + buf * C::STAGE;
    const char* lb = la + C::A_BYTES;
    const char* ls = lb + C::B_BYTES;
    const int lo = lane * 16;
    uint32_t o0, o1; // swizzled row-major operands
    pp::operand_lane(lane, o0, o1);
    const uint32_t b0 = C::BPS ? (uint32_t)lo : o0, b1 = C::BPS ? (uint32_t)lo + 1024 : o1;
    // MXFP8: this step's 128-K half of each scale dword moved to bytes 0-1
    const uint32_t sh = C::FP4 ? 0u : (uint32_t)(step & 1) * 16;
#pragma unroll
    for (int t = 0; t < C::SM; t++)
        f.sa[t] = *(const uint32_t*)(ls + (wm * C::SM + t) * 256 + lane * 4) >> sh;
#pragma unroll
    for (int t = 0; t < C::SN; t++)
        f.sb[t] = *(const uint32_t*)(ls + (C::BM / 32 + wn * C::SN + t) * 256 + lane * 4) >> sh;
#pragma unroll
    for (int t = 0; t < C::TN; t++) {
        const char* g = lb + (wn * C::TN + t) * 2048;
        v4i x0 = *(const v4i*)(g + b0);
        v4i x1 = *(const v4i*)(g + b1);
        f.bf[t] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    }
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        const char* g = la + (wm * C::TM + i) * 2048;
        v4i x0 = *(const v4i*)(g + o0);
        v4i x1 = *(const v4i*)(g + o1);
        f.af[i] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    }
}

template <class C>
__device__ __forceinline__ void mma_stage(const MxFrag<C>& f, v4f (&acc)[C::TM][C::TN])
{
    static_for<C::TM>([&](auto I) {
        constexpr int i = decltype(I)::value;
        static_for<C::TN>([&](auto T) {
            constexpr int t = decltype(T)::value;
            // op_sel picks the 16-row half inside the 32-row scale block; the
            // 128-K half is the dword's low 16 bits (MXFP8: shifted there
            // when read; MXFP4: the first of the step's two MFMAs, the second
            // takes the high 16 bits and the fragments' last 16 bytes)
            if constexpr (C::FP4) {
                acc[i][t] = mfma_mx16_fp4<(t & 1), (i & 1)>(f.bf[t], f.af[i], acc[i][t],
                                                             (int)f.sb[t >> 1], (int)f.sa[i >> 1]);
                acc[i][t] = mfma_mx16_fp4<(t & 1), (i & 1)>(hi16(f.bf[t]), hi16(f.af[i]), acc[i][t],
                                                             (int)(f.sb[t >> 1] >> 16),
                                                             (int)(f.sa[i >> 1] >> 16));
            } else {
                acc[i][t] = mfma_mx16<(t & 1), (i & 1)>(f.bf[t], f.af[i], acc[i][t],
                                                        (int)f.sb[t >> 1], (int)f.sa[i >> 1]);
            }
        });
    });
}

// Epilogue of a wave's TM x TN 16x16 tiles starting at (mb, nb): lane holds
// C[m][n .. n+3] of each tile. Split-K slices write fp32 partials; otherwise
// D = bf16(alpha * acc (+ beta * C)). The library is built with
// -ffp-contract=off: alpha*v and + beta*c round separately.
template <int TM, int TN>
__device__ __forceinline__ void mx_store(const ga_f4gemm_kargs& args, float* ws, int z, int gdz,
                                         int mb, int nb, int lane, const v4f (&acc)[TM][TN])
{
    const int M = (int)args.M, N = (int)args.N;
    const int ldd = (int)args.stride_C0;
    const float alpha = args.alpha, beta = args.beta;
    const bool use_c = beta != 0.0f && args.ptr_C != nullptr;
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int m = mb + i * 16 + (lane & 15);
#pragma unroll
        for (int t = 0; t < TN; t++) {
            const int n = nb + t * 16 + (lane >> 4) * 4;
            if (m >= M || n >= N)
                continue;
            v4f v = acc[i][t];
            if (gdz > 1) {
                *(v4f*)(ws + ((size_t)z * M + m) * N + n) = v;
            } else {
                uint16_t o[4];
                const uint16_t* cin = use_c ? (const uint16_t*)args.ptr_C + (size_t)m * ldd + n
                                            : nullptr;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float r = alpha * v[j];
                    if (use_c)
                        r = r + beta * bf16_to_f32(cin[j]);
                    o[j] = f32_to_bf16(r);
                }
                uint2 pk;
                pk.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
                pk.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
                *(uint2*)((uint16_t*)args.ptr_D + (size_t)m * ldd + n) = pk;
            }
        }
    }
}

template <class C>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(C::WPE, C::WPE)))
void mx_gemm_kernel(ga_f4gemm_kargs args, float* __restrict__ ws,
                    const ga_splitk_ws_handle* __restrict__ wsh)
{
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS];
    if (wsh && !(ws = resolve_ws(wsh, gridDim.z, args.M, args.N)))
        return; // workspace slot shorter than the split-K layout: write nothing

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const int M = (int)args.M, N = (int)args.N, K = (int)args.K;
    int tile_m, tile_n;
    map_tile(blockIdx.x, blockIdx.y, gridDim.x, gridDim.y, kGroupM, tile_m, tile_n);
    const int m0 = tile_m * C::BM, n0 = tile_n * C::BN;

    const int z = blockIdx.z, gdz = gridDim.z;
    int kpt = K;
    if (gdz > 1)
        kpt = ((K >> args.log2_k_split) + 255) / 256 * 256;
    const int kb = z * kpt;
    const int ke = min(K, kb + kpt);
    const int nsteps = (ke - kb) / (128 * C::EPB);
    const int kbb = kb / C::EPB, Kb = K / C::EPB; // bytes

    const uint32_t lda = args.stride_A0 / C::EPB, ldb = args.stride_B0 / C::EPB; // bytes
    const uint32_t sna = args.stride_ScaleA0, snb = args.stride_ScaleB0;

    MxState<C> st;
    {
        const char* pa = (const char*)args.ptr_A + (size_t)m0 * lda;
        long long abytes = (long long)(M - m0) * lda;
        st.ra = make_rsrc(pa, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
        // row-major operands: copy i covers rows 32i .. 32i+31 (wave w: 8
        // whole 128-byte rows) of the swizzled LDS image
        int row0, chunk;
        pp::copy_lane(wave, lane, row0, chunk);
#pragma unroll
        for (int i = 0; i < C::A_LOADS; i++)
            st.voff_a[i] = (uint32_t)(i * 32 + row0) * lda + chunk * 16;
        if (C::BPS) {
            const char* pb = (const char*)args.ptr_B + (size_t)(n0 / 16) * Kb * 16;
            long long bbytes = (long long)(N - n0) * Kb;
            st.rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
            st.b_kstride = 128 * 16;
#pragma unroll
            for (int i = 0; i < C::B_LOADS; i++) {
                int idx = i * 256 + tid;
                int g = idx >> 7, u = idx & 127;
                st.voff_b[i] = (uint32_t)g * (uint32_t)Kb * 16 + (uint32_t)u * 16;
            }
        } else {
            const char* pb = (const char*)args.ptr_B + (size_t)n0 * ldb;
            long long bbytes = (long long)(N - n0) * ldb;
            st.rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
            st.b_kstride = 128;
#pragma unroll
            for (int i = 0; i < C::B_LOADS; i++)
                st.voff_b[i] = (uint32_t)(i * 32 + row0) * ldb + chunk * 16;
        }
        // Scales: shuffled layout, 256-byte block per (32 rows, 256 K).
        const int sma = (M + 31) / 32 * 32, smb = (N + 31) / 32 * 32;
        st.rsa = make_rsrc(args.ptr_ScaleA, (uint32_t)sma * sna);
        st.rsb = make_rsrc(args.ptr_ScaleB, (uint32_t)smb * snb);
        const int q0 = kb / 256;
#pragma unroll
        for (int i = 0; i < C::S_LOADS; i++) {
            int j = wave * C::S_LOADS + i;
            j = j < C::SBLK ? j : 0; // padding slots repeat block 0
            const bool isb = j >= C::BM / 32;
            const int r = isb ? n0 + (j - C::BM / 32) * 32 : m0 + j * 32;
            const uint32_t sn = isb ? snb : sna;
            st.sfrom_b[i] = isb;
            st.soff[i] = ((uint32_t)(r / 32) * (sn / 8) + q0) * 256 + lane * 4;
        }
    }

    v4f acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int t = 0; t < C::TN; t++)
            acc[i][t] = (v4f){0.f, 0.f, 0.f, 0.f};

    // Pipeline: stages 0 .. NS-2 in flight before the loop. Loads past the
    // slice are issued unconditionally (branch-free body): they read in-bounds
    // bytes that are never used, or range-checked zeros past the end of a
    // buffer. Every load of the loop is a direct-to-LDS copy, so the counted
    // vmcnt waits are the only ones.
#pragma unroll
    for (int p = 0; p < C::NS - 1; p++)
        issue_stage<C>(st, smem, p, p, kbb + p * 128, wave);
    if constexpr (C::NS == 2) {
        // Two stages (the tiles that run two workgroups per CU): step s waits
        // for its stage, issues stage s+1 into the buffer step s-1 used (free
        // after the barrier) and computes from stage s.
        for (int s = 0; s < nsteps; s++) {
            wait_vmcnt<0>();
            barrier_lds();
            issue_stage<C>(st, smem, (s + 1) & 1, s + 1, kbb + (s + 1) * 128, wave);
            __builtin_amdgcn_sched_barrier(0);
            MxFrag<C> f;
            read_stage<C>(smem, s & 1, s, wm, wn, lane, f);
            mma_stage<C>(f, acc);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        // Three or more stages (one workgroup per CU, one wave per SIMD): the
        // fragments of step s+1 are read while the MFMAs of step s run. Step s
        // waits for stage s+1 (the barrier also ends every wave's reads of
        // stage s), refills the buffer of step s-1 with stage s+NS-1, reads
        // stage s+1, multiplies the fragments of stage s. Two fragment sets
        // alternate (the loop is unrolled by two).
        MxFrag<C> f0, f1;
        wait_vmcnt<C::TILE_LOADS * (C::NS - 2)>();
        barrier_lds();
        read_stage<C>(smem, 0, 0, wm, wn, lane, f0);
        int buf = 0; // LDS buffer of stage s
        auto step = [&](int s, const MxFrag<C>& cur, MxFrag<C>& nxt) {
            wait_vmcnt<C::TILE_LOADS * (C::NS - 3)>();
            barrier_lds();
            const int prev = buf == 0 ? C::NS - 1 : buf - 1;
            const int next = buf + 1 == C::NS ? 0 : buf + 1;
            issue_stage<C>(st, smem, prev, s + C::NS - 1, kbb + (s + C::NS - 1) * 128, wave);
            __builtin_amdgcn_sched_barrier(0);
            read_stage<C>(smem, next, s + 1, wm, wn, lane, nxt);
            mma_stage<C>(cur, acc);
            __builtin_amdgcn_sched_barrier(0);
            buf = next;
        };
        int s = 0;
        for (; s + 1 < nsteps; s += 2) {
            step(s, f0, f1);
            step(s + 1, f1, f0);
        }
        if (s < nsteps)
            step(s, f0, f1);
    }
    // the copies of steps past the slice land before the workgroup's LDS is freed
    wait_vmcnt<0>();

    mx_store<C::TM, C::TN>(args, ws, z, gdz, m0 + wm * C::WTM, n0 + wn * C::WTN, lane, acc);
}

template <class C>
static void launch_mx(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                      int gdx, int gdy, int gdz, hipStream_t stream)
{
    hipLaunchKernelGGL(mx_gemm_kernel<C>, dim3(gdx, gdy, gdz), dim3(256), 0, stream, args, ws,
                       wsh);
}

// B-streaming tile for preshuffled B and few rows (BM = 32 or 64): the four
// waves sit side by side along N, so no wave shares a B fragment with
// another, and B goes from memory straight into the MFMA operand registers
// (a ring of NS K steps in flight per wave: the preshuffled 2 KB of a 16-row
// group and 128-K step is the operand of 64 lanes as it lies). Only A (BM
// rows, read by all four waves) and the scales pass through LDS, so the
// pipeline depth is bounded by registers, not by LDS: with LDS-staged B the
// 32-row tiles kept one or two steps in flight and waited a memory latency
// per step.
template <int BM_, int BN_, int NS_, bool FP4_>
struct MbCfg {
    static constexpr int BM = BM_, BN = BN_, NS = NS_;
    static constexpr bool FP4 = FP4_;
    static constexpr int EPB = FP4 ? 2 : 1;
    static constexpr int NT = 256;
    static constexpr int WTN = BN / 4;
    static constexpr int TM = BM / 16, TN = WTN / 16;
    static constexpr int SM = TM / 2, SN = TN / 2;
    static constexpr int A_BYTES = BM * 128;
    static constexpr int SBLK = BM / 32 + BN / 32;
    static constexpr int S_LOADS = (SBLK + 3) / 4;
    static constexpr int S_BYTES = 4 * S_LOADS * 256;
    static constexpr int STAGE = A_BYTES + S_BYTES;
    static constexpr int LDS = NS * STAGE;
    static constexpr int A_LOADS = A_BYTES / (NT * 16);
    static constexpr int B_LOADS = 2 * TN; // per wave per step, into registers
    static constexpr int TILE_LOADS = A_LOADS + B_LOADS + S_LOADS;
    static_assert(BM % 32 == 0 && WTN % 32 == 0, "32-row scale blocks");
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(NS >= 2 && TILE_LOADS * (NS - 2) < 64, "vmcnt range");
};

template <class C>
struct MbState {
    __amdgpu_buffer_rsrc_t ra, rb, rsa, rsb;
    uint32_t voff_a[C::A_LOADS];
    uint32_t vb;      // this lane's byte in the wave's first 16-row B group
    uint32_t gstride; // bytes between 16-row B groups (16 * K bytes)
    uint32_t soff[C::S_LOADS];
    bool sfrom_b[C::S_LOADS];
};

// Step `step` (byte offset kk inside a row): A and scales into LDS stage
// `buf`, this wave's B fragments into bq.
template <class C>
__device__ __forceinline__ void mb_issue(const MbState<C>& st, char* smem, int buf, int step,
                                         int kk, int wave, v8i (&bq)[C::TN])
{
    char* sa = smem + buf * C::STAGE;
    char* ss = sa + C::A_BYTES;
#pragma unroll
    for (int i = 0; i < C::A_LOADS; i++)
        lds_load16(st.ra, (lds_void*)(sa + (i * 256 + wave * 64) * 16), st.voff_a[i] + kk, 0);
    const uint32_t q = (uint32_t)(C::FP4 ? step : (step >> 1)) * 256;
#pragma unroll
    for (int i = 0; i < C::S_LOADS; i++) {
        lds_void* dst = (lds_void*)(ss + (wave * C::S_LOADS + i) * 256);
        if (st.sfrom_b[i])
            __builtin_amdgcn_raw_ptr_buffer_load_lds(st.rsb, dst, 4, st.soff[i] + q, 0, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(st.rsa, dst, 4, st.soff[i] + q, 0, 0, 0);
    }
    const uint32_t kq = (uint32_t)(kk / 128) * 2048;
#pragma unroll
    for (int t = 0; t < C::TN; t++) {
        const uint32_t o = st.vb + __builtin_amdgcn_readfirstlane((uint32_t)t * st.gstride + kq);
        v4i x0 = buf_load16(st.rb, o, 0);
        v4i x1 = buf_load16(st.rb, o + 1024, 0);
        bq[t] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    }
}

template <class C>
__device__ __forceinline__ void mb_compute(const char* smem, int buf, int step, int wn, int lane,
                                           const v8i (&bq)[C::TN], v4f (&acc)[C::TM][C::TN])
{
    const char* la = smem + buf * C::STAGE;
    const char* ls = la + C::A_BYTES;
    uint32_t o0, o1;
    pp::operand_lane(lane, o0, o1);
    const uint32_t sh = C::FP4 ? 0u : (uint32_t)(step & 1) * 16;
    uint32_t sa[C::SM], sb[C::SN];
#pragma unroll
    for (int t = 0; t < C::SM; t++)
        sa[t] = *(const uint32_t*)(ls + t * 256 + lane * 4) >> sh;
#pragma unroll
    for (int t = 0; t < C::SN; t++)
        sb[t] = *(const uint32_t*)(ls + (C::BM / 32 + wn * C::SN + t) * 256 + lane * 4) >> sh;
    static_for<C::TM>([&](auto I) {
        constexpr int i = decltype(I)::value;
        const char* g = la + i * 2048;
        v4i x0 = *(const v4i*)(g + o0);
        v4i x1 = *(const v4i*)(g + o1);
        v8i af = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        static_for<C::TN>([&](auto T) {
            constexpr int t = decltype(T)::value;
            if constexpr (C::FP4) {
                acc[i][t] = mfma_mx16_fp4<(t & 1), (i & 1)>(bq[t], af, acc[i][t],
                                                             (int)sb[t >> 1], (int)sa[i >> 1]);
                acc[i][t] = mfma_mx16_fp4<(t & 1), (i & 1)>(hi16(bq[t]), hi16(af), acc[i][t],
                                                             (int)(sb[t >> 1] >> 16),
                                                             (int)(sa[i >> 1] >> 16));
            } else {
                acc[i][t] = mfma_mx16<(t & 1), (i & 1)>(bq[t], af, acc[i][t], (int)sb[t >> 1],
                                                        (int)sa[i >> 1]);
            }
        });
    });
}

template <class C>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void mx_bstream_kernel(ga_f4gemm_kargs args, float* __restrict__ ws,
                       const ga_splitk_ws_handle* __restrict__ wsh)
{
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS];
    if (wsh && !(ws = resolve_ws(wsh, gridDim.z, args.M, args.N)))
        return; // workspace slot shorter than the split-K layout: write nothing
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = (int)args.M, N = (int)args.N, K = (int)args.K;
    int tile_m, tile_n;
    map_tile(blockIdx.x, blockIdx.y, gridDim.x, gridDim.y, kGroupM, tile_m, tile_n);
    const int m0 = tile_m * C::BM, n0 = tile_n * C::BN;
    const int z = blockIdx.z, gdz = gridDim.z;
    int kpt = K;
    if (gdz > 1)
        kpt = ((K >> args.log2_k_split) + 255) / 256 * 256;
    const int kb = z * kpt;
    const int ke = min(K, kb + kpt);
    const int nsteps = (ke - kb) / (128 * C::EPB);
    const int kbb = kb / C::EPB, Kb = K / C::EPB; // bytes
    const uint32_t lda = args.stride_A0 / C::EPB;
    const uint32_t sna = args.stride_ScaleA0, snb = args.stride_ScaleB0;

    MbState<C> st;
    {
        const char* pa = (const char*)args.ptr_A + (size_t)m0 * lda;
        long long abytes = (long long)(M - m0) * lda;
        st.ra = make_rsrc(pa, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
        int row0, chunk;
        pp::copy_lane(wave, lane, row0, chunk);
#pragma unroll
        for (int i = 0; i < C::A_LOADS; i++)
            st.voff_a[i] = (uint32_t)(i * 32 + row0) * lda + chunk * 16;
        // preshuffled B: 16-row group g of the tile holds its K steps as
        // consecutive 2 KB blocks; rows past N read as zero
        const char* pb = (const char*)args.ptr_B + (size_t)(n0 / 16) * Kb * 16;
        long long bbytes = (long long)(N - n0) * Kb;
        st.rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
        st.gstride = (uint32_t)Kb * 16;
        st.vb = (uint32_t)(wave * C::TN) * st.gstride + (uint32_t)lane * 16;
        const int sma = (M + 31) / 32 * 32, smb = (N + 31) / 32 * 32;
        st.rsa = make_rsrc(args.ptr_ScaleA, (uint32_t)sma * sna);
        st.rsb = make_rsrc(args.ptr_ScaleB, (uint32_t)smb * snb);
        const int q0 = kb / 256;
#pragma unroll
        for (int i = 0; i < C::S_LOADS; i++) {
            int j = wave * C::S_LOADS + i;
            j = j < C::SBLK ? j : 0; // padding slots repeat block 0
            const bool isb = j >= C::BM / 32;
            const int r = isb ? n0 + (j - C::BM / 32) * 32 : m0 + j * 32;
            const uint32_t sn = isb ? snb : sna;
            st.sfrom_b[i] = isb;
            st.soff[i] = ((uint32_t)(r / 32) * (sn / 8) + q0) * 256 + lane * 4;
        }
    }

    v4f acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int t = 0; t < C::TN; t++)
            acc[i][t] = (v4f){0.f, 0.f, 0.f, 0.f};

    // Pipeline: steps 0 .. NS-2 in flight before the loop. Step s (ring slot
    // s % NS, a compile-time index: the loop is unrolled NS times) waits for
    // its A and scale copies (counted vmcnt; the compiler adds the waits for
    // the B registers itself), then issues step s+NS-1 into the slot step
    // s-1 used and multiplies.
    v8i bq[C::NS][C::TN];
    static_for<C::NS - 1>([&](auto P) {
        constexpr int p = decltype(P)::value;
        mb_issue<C>(st, smem, p, p, kbb + p * 128, wave, bq[p]);
    });
    for (int s0 = 0; s0 < nsteps; s0 += C::NS) {
        static_for<C::NS>([&](auto P) {
            constexpr int p = decltype(P)::value;
            constexpr int np = (p + C::NS - 1) % C::NS;
            const int s = s0 + p;
            if (s < nsteps) {
                wait_vmcnt<C::TILE_LOADS * (C::NS - 2)>();
                barrier_lds();
                mb_issue<C>(st, smem, np, s + C::NS - 1, kbb + (s + C::NS - 1) * 128, wave,
                            bq[np]);
                __builtin_amdgcn_sched_barrier(0);
                mb_compute<C>(smem, p, s, wave, lane, bq[p], acc);
                __builtin_amdgcn_sched_barrier(0);
            }
        });
    }
    // the loads of steps past the slice land before the workgroup ends
    wait_vmcnt<0>();
    mx_store<C::TM, C::TN>(args, ws, z, gdz, m0, n0 + wave * C::WTN, lane, acc);
}

// Entry tiles BM x BN run as workgroups of C::BN columns (BN a multiple of
// C::BN): the entry's grid fixes the tile a caller sees; a 32x512 workgroup
// would leave half of the CUs idle at M <= 128.
template <class C>
static void launch_mxb(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                       int gdx, int gdy, int gdz, hipStream_t stream)
{
    (void)gdx;
    const int gx = ((int)args.N + C::BN - 1) / C::BN;
    hipLaunchKernelGGL(mx_bstream_kernel<C>, dim3(gx, gdy, gdz), dim3(256), 0, stream, args, ws,
                       wsh);
}

#define GA_MX_ENTRY(BM, BN, WGM, WGN, BPS, NS, SPLIT, SUFFIX)                                  \
    {{BM, BN, SPLIT, BPS,                                                                     \
      "ga_mxfp8_bf16_" GA_BPS_NAME_##BPS "_" #BM "x" #BN SUFFIX,                              \
      "ga_mxfp8_bf16_" GA_BPS_NAME_##BPS "_" #BM "x" #BN SUFFIX ".co"},                       \
     &launch_mx<MxCfg<BM, BN, WGM, WGN, (BPS != 0), NS>>, 64, 8}
// Preshuffled-B entries with 32 or 64 rows run the B-streaming tile (IBN
// columns per workgroup, 4 steps in flight).
#define GA_MXB_ENTRY(BM, BN, IBN, SPLIT, SUFFIX)                                               \
    {{BM, BN, SPLIT, 1, "ga_mxfp8_bf16_BpreShuffle_" #BM "x" #BN SUFFIX,                      \
      "ga_mxfp8_bf16_BpreShuffle_" #BM "x" #BN SUFFIX ".co"},                                 \
     &launch_mxb<MbCfg<BM, IBN, 4, false>>, 64, 8}
#define GA_MX4B_ENTRY(BM, BN, IBN, SPLIT, SUFFIX)                                              \
    {{BM, BN, SPLIT, 1, "ga_mxfp4_bf16_BpreShuffle_" #BM "x" #BN SUFFIX,                      \
      "ga_mxfp4_bf16_BpreShuffle_" #BM "x" #BN SUFFIX ".co"},                                 \
     &launch_mxb<MbCfg<BM, IBN, 4, true>>, 64, 4}
#define GA_BPS_NAME_1 "BpreShuffle"
#define GA_BPS_NAME_0 "noBpreShuffle"

// Manifest order matters: the heuristic breaks ties by it. Entries after
// kManifestCount are found by name (ga_kernel_find) but are not offered to the
// heuristic.
#define GA_MX_PP_ENTRY(BPS, SPLIT, SUFFIX, FN)                                                 \
    {{256, 256, SPLIT, BPS, "ga_mxfp8_bf16_" GA_BPS_NAME_##BPS "_256x256" SUFFIX,               \
      "ga_mxfp8_bf16_" GA_BPS_NAME_##BPS "_256x256" SUFFIX ".co"},                              \
     &FN, 64, 8}
// MXFP4 (the reference's f4gemm_bf16_per1x32Fp4 kernels): e2m1 operands.
#define GA_MX4_ENTRY(BM, BN, WGM, WGN, BPS, NS, SPLIT, SUFFIX)                                 \
    {{BM, BN, SPLIT, BPS,                                                                     \
      "ga_mxfp4_bf16_" GA_BPS_NAME_##BPS "_" #BM "x" #BN SUFFIX,                              \
      "ga_mxfp4_bf16_" GA_BPS_NAME_##BPS "_" #BM "x" #BN SUFFIX ".co"},                       \
     &launch_mx<MxCfg<BM, BN, WGM, WGN, (BPS != 0), NS, true>>, 64, 4}
#define GA_MX4_PP_ENTRY(BPS, SPLIT, SUFFIX, FN)                                                \
    {{256, 256, SPLIT, BPS, "ga_mxfp4_bf16_" GA_BPS_NAME_##BPS "_256x256" SUFFIX,               \
      "ga_mxfp4_bf16_" GA_BPS_NAME_##BPS "_256x256" SUFFIX ".co"},                              \
     &FN, 64, 4}

// Tiles found by name only, as the reference's aiter manifest names them
// (35 tiles, e.g. 96x640 and 128x512): the entry's tile fixes the launch
// contract the caller sees (the grid ceil(N/tN) x ceil(M/tM) x gdz that
// make_launch returns and kernel_launch checks, the split geometry, the
// workspace); the kernel that runs is the one the heuristic picks for the
// shape among this element width's compiled tiles at the same split. Every
// compiled tile computes the same fp32 chain per K slice, so the output does
// not depend on that choice.
template <bool BPS, bool FP4>
static void launch_by_shape(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                            int gdx, int gdy, int gdz, hipStream_t stream);

#define GA_MXV_ENTRY(PREFIX, EB, FP4, BM, BN, SPLIT, SUFFIX)                                  \
    {{BM, BN, SPLIT, 1, PREFIX "_BpreShuffle_" #BM "x" #BN SUFFIX,                            \
      PREFIX "_BpreShuffle_" #BM "x" #BN SUFFIX ".co"},                                       \
     &launch_by_shape<true, FP4>, 64, EB, true}

static const MxKernel g_mx_kernels[] = {
    GA_MX_PP_ENTRY(1, 0, "", launch_mx_pp_bps),
    GA_MX_ENTRY(256, 128, 2, 2, 1, 3, 0, ""),
    GA_MX_ENTRY(128, 256, 2, 2, 1, 3, 0, ""),
    GA_MX_ENTRY(128, 128, 2, 2, 1, 2, 0, ""),
    GA_MXB_ENTRY(64, 256, 256, 0, ""),
    GA_MXB_ENTRY(32, 256, 256, 0, ""),
    GA_MX_PP_ENTRY(1, 1, "_splitK", launch_mx_pp_bps),
    GA_MX_ENTRY(256, 128, 2, 2, 1, 3, 1, "_splitK"),
    GA_MX_ENTRY(128, 256, 2, 2, 1, 3, 1, "_splitK"),
    GA_MX_ENTRY(128, 128, 2, 2, 1, 2, 1, "_splitK"),
    GA_MXB_ENTRY(64, 256, 256, 1, "_splitK"),
    GA_MXB_ENTRY(32, 256, 256, 1, "_splitK"),
    GA_MXB_ENTRY(32, 512, 256, 1, "_splitK"),
    GA_MX_PP_ENTRY(0, 0, "", launch_mx_pp_nobps),
    GA_MX_ENTRY(256, 128, 2, 2, 0, 3, 0, ""),
    GA_MX_ENTRY(128, 128, 2, 2, 0, 2, 1, "_splitK"),
    // tiles of the reference's MXFP4 manifest this one did not have
    GA_MXV_ENTRY("ga_mxfp8_bf16", 8, false, 96, 640, 0, ""),
    GA_MXV_ENTRY("ga_mxfp8_bf16", 8, false, 128, 512, 0, ""),
    GA_MXV_ENTRY("ga_mxfp8_bf16", 8, false, 96, 640, 1, "_splitK"),
    GA_MXV_ENTRY("ga_mxfp8_bf16", 8, false, 128, 512, 1, "_splitK"),
    // not in the manifest: the 4-wave 256x256 tile (two stages)
    GA_MX_ENTRY(256, 256, 2, 2, 1, 2, 0, "_ns2"),
    // the MXFP4 manifest, the MXFP8 one's tiles and order
    GA_MX4_PP_ENTRY(1, 0, "", launch_mx4_pp_bps),
    GA_MX4_ENTRY(256, 128, 2, 2, 1, 3, 0, ""),
    GA_MX4_ENTRY(128, 256, 2, 2, 1, 3, 0, ""),
    GA_MX4_ENTRY(128, 128, 2, 2, 1, 2, 0, ""),
    GA_MX4B_ENTRY(64, 256, 256, 0, ""),
    GA_MX4B_ENTRY(32, 256, 256, 0, ""),
    GA_MX4_PP_ENTRY(1, 1, "_splitK", launch_mx4_pp_bps),
    GA_MX4_ENTRY(256, 128, 2, 2, 1, 3, 1, "_splitK"),
    GA_MX4_ENTRY(128, 256, 2, 2, 1, 3, 1, "_splitK"),
    GA_MX4_ENTRY(128, 128, 2, 2, 1, 2, 1, "_splitK"),
    GA_MX4B_ENTRY(64, 256, 256, 1, "_splitK"),
    GA_MX4B_ENTRY(32, 256, 256, 1, "_splitK"),
    GA_MX4B_ENTRY(32, 512, 256, 1, "_splitK"),
    GA_MX4_PP_ENTRY(0, 0, "", launch_mx4_pp_nobps),
    GA_MX4_ENTRY(256, 128, 2, 2, 0, 3, 0, ""),
    GA_MX4_ENTRY(128, 128, 2, 2, 0, 2, 1, "_splitK"),
    GA_MXV_ENTRY("ga_mxfp4_bf16", 4, true, 96, 640, 0, ""),
    GA_MXV_ENTRY("ga_mxfp4_bf16", 4, true, 128, 512, 0, ""),
    GA_MXV_ENTRY("ga_mxfp4_bf16", 4, true, 96, 640, 1, "_splitK"),
    GA_MXV_ENTRY("ga_mxfp4_bf16", 4, true, 128, 512, 1, "_splitK"),
};
constexpr int kManifestCount = 20;
constexpr int kMx4First = 21;
constexpr int kMx4Count = 20;
constexpr int kStaticCount = (int)(sizeof(g_mx_kernels) / sizeof(g_mx_kernels[0]));
static_assert(kMx4First + kMx4Count == kStaticCount, "registry layout");

// Entries made by ga_kernel_find from a tile name (aiter's
// f4gemm_bf16_per1x32Fp4_[no]BpreShuffle_<tM>x<tN>, or this library's
// ga_mxfp{8,4}_bf16_... with any tile): indices kStaticCount and up. A deque
// keeps earlier entries in place as it grows.
static std::mutex g_named_mu;
static std::deque<MxKernel> g_named;
static std::atomic<int> g_named_count{0};

int mx_registry_count() { return kManifestCount; }
int mx4_registry_first() { return kMx4First; }
int mx4_registry_count() { return kMx4Count; }
int mx_registry_total() { return kStaticCount + g_named_count.load(std::memory_order_acquire); }
const MxKernel* mx_registry_get(int idx)
{
    if (idx < kStaticCount)
        return &g_mx_kernels[idx];
    std::lock_guard<std::mutex> lock(g_named_mu);
    return &g_named[idx - kStaticCount];
}

// The tile a by-name entry runs for a shape, remembered per (B layout,
// element width, M, N, K, log2 split, CU count) in a small direct-mapped
// table, so that repeated launches of one shape do not repeat the selection.
struct ShapePick {
    int key[7];
    int idx;
    bool valid;
};

template <typename F>
static int picked_tile(const int (&key)[7], F select)
{
    static std::mutex mu;
    static ShapePick table[64];
    uint32_t h = 2166136261u;
    for (int v : key)
        h = (h ^ (uint32_t)v) * 16777619u;
    ShapePick& e = table[h % 64];
    {
        std::lock_guard<std::mutex> lock(mu);
        if (e.valid && memcmp(e.key, key, sizeof(e.key)) == 0)
            return e.idx;
    }
    const int idx = select();
    std::lock_guard<std::mutex> lock(mu);
    memcpy(e.key, key, sizeof(e.key));
    e.idx = idx;
    e.valid = true;
    return idx;
}

template <bool BPS, bool FP4>
static int select_by_shape(const ga_f4gemm_kargs& args, int L, int num_cu)
{
    const int first = FP4 ? kMx4First : 0, count = FP4 ? kMx4Count : kManifestCount;
    ga_tile_config table[kManifestCount];
    int map[kManifestCount], n = 0;
    for (int i = first; i < first + count; i++)
        if (!g_mx_kernels[i].by_shape) {
            map[n] = i;
            table[n++] = g_mx_kernels[i].cfg;
        }
    int row = -1, l2 = 0;
    int idx = map[0]; // the 256x256 tile of this width takes any shape
    if (!BPS)
        for (int i = 0; i < n; i++)
            if (!table[i].bpreshuffle && table[i].tile_M == 256 && table[i].tile_N == 256)
                idx = map[i];
    if (ga_select_kernel((int)args.M, (int)args.N, (int)args.K, num_cu, L, BPS ? 1 : 0, table, n,
                         &row, &l2) == GA_OK &&
        row >= 0)
        idx = map[row];
    return idx;
}

template <bool BPS, bool FP4>
static void launch_by_shape(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                            int gdx, int gdy, int gdz, hipStream_t stream)
{
    (void)gdx;
    (void)gdy;
    int num_cu = 0;
    if (device_cu_count(&num_cu) != GA_OK || num_cu <= 0)
        num_cu = 256;
    const int L = gdz > 1 ? args.log2_k_split : 0;
    const int key[7] = {BPS ? 1 : 0, FP4 ? 1 : 0, (int)args.M, (int)args.N, (int)args.K, L, num_cu};
    const int idx = picked_tile(key, [&] { return select_by_shape<BPS, FP4>(args, L, num_cu); });
    const MxKernel& k = g_mx_kernels[idx];
    k.launch(args, ws, wsh, ((int)args.N + k.cfg.tile_N - 1) / k.cfg.tile_N,
             ((int)args.M + k.cfg.tile_M - 1) / k.cfg.tile_M, gdz, stream);
}

// Parses a tile name into a by-shape entry; false when it is not one.
static bool parse_tile_name(const char* name, MxKernel* out)
{
    std::string s(name);
    const bool mangled = s.compare(0, 2, "_Z") == 0;
    if (s.size() > 3 && s.compare(s.size() - 3, 3, ".co") == 0)
        s.resize(s.size() - 3);
    struct Family {
        const char* prefix;
        int elem_bits;
        bool aiter;
    };
    static const Family fams[] = {{"f4gemm_bf16_per1x32Fp4_", 4, true},
                                  {"ga_mxfp4_bf16_", 4, false},
                                  {"ga_mxfp8_bf16_", 8, false}};
    const Family* f = nullptr;
    size_t at = std::string::npos;
    for (const Family& c : fams) {
        at = s.find(c.prefix);
        if (at != std::string::npos && (at == 0 || mangled)) {
            f = &c;
            break;
        }
    }
    if (!f)
        return false;
    std::string rest = s.substr(at + strlen(f->prefix));
    int bps;
    if (rest.compare(0, 12, "BpreShuffle_") == 0) {
        bps = 1;
        rest = rest.substr(12);
    } else if (rest.compare(0, 14, "noBpreShuffle_") == 0) {
        bps = 0;
        rest = rest.substr(14);
    } else {
        return false;
    }
    int tm = 0, tn = 0, used = 0;
    if (sscanf(rest.c_str(), "%dx%d%n", &tm, &tn, &used) != 2)
        return false;
    std::string tail = rest.substr(used);
    int split;
    if (f->aiter) {
        // aiter's names do not mark split-K (its CSV's splitK column does)
        if (!(tail.empty() || (mangled && tail == "E")))
            return false;
        split = 1;
    } else {
        if (tail == "_splitK")
            split = 1;
        else if (tail.empty())
            split = 0;
        else
            return false;
    }
    if (tm < 16 || tn < 16 || tm > 1024 || tn > 1024 || tm % 16 || tn % 16)
        return false;
    if (strlen(name) >= GA_NAME_MAX)
        return false;
    MxKernel k{};
    k.cfg.tile_M = tm;
    k.cfg.tile_N = tn;
    k.cfg.splitK = split;
    k.cfg.bpreshuffle = bps;
    snprintf(k.cfg.knl_name, GA_NAME_MAX, "%s", name);
    if (snprintf(k.cfg.co_name, GA_NAME_MAX, "%s.co", s.c_str()) >= GA_NAME_MAX)
        return false;
    const bool fp4 = f->elem_bits == 4;
    k.launch = fp4 ? (bps ? &launch_by_shape<true, true> : &launch_by_shape<false, true>)
                   : (bps ? &launch_by_shape<true, false> : &launch_by_shape<false, false>);
    k.small_m_stream = 64;
    k.elem_bits = f->elem_bits;
    k.by_shape = true;
    *out = k;
    return true;
}

ga_status default_workspace(size_t bytes, void** ptr)
{
    static std::mutex mu;
    static std::vector<std::pair<void*, size_t>> per_dev;
    std::lock_guard<std::mutex> lock(mu);
    int dev = 0;
    GA_HIP_CHECK(hipGetDevice(&dev));
    if ((int)per_dev.size() <= dev)
        per_dev.resize(dev + 1, {nullptr, 0});
    auto& slot = per_dev[dev];
    if (slot.second < bytes) {
        if (slot.first) {
            GA_HIP_CHECK(hipDeviceSynchronize());
            GA_HIP_CHECK(hipFree(slot.first));
            slot = {nullptr, 0};
        }
        void* p = nullptr;
        GA_HIP_CHECK(hipMalloc(&p, bytes));
        slot = {p, bytes};
    }
    *ptr = slot.first;
    return GA_OK;
}

} // namespace ga

using namespace ga;

extern "C" {

ga_status ga_kernel_find(const char* name, int* idx)
{
    if (!name || !idx)
        return fail(GA_ERR_ARG, "null argument");
    for (int i = 0; i < kStaticCount; i++) {
        const ga_tile_config& c = g_mx_kernels[i].cfg;
        if (!strcmp(c.knl_name, name) || !strcmp(c.co_name, name)) {
            *idx = i;
            return GA_OK;
        }
    }
    MxKernel k;
    const bool parsed = parse_tile_name(name, &k);
    std::lock_guard<std::mutex> lock(g_named_mu);
    for (size_t i = 0; i < g_named.size(); i++) {
        const ga_tile_config& c = g_named[i].cfg;
        if (!strcmp(c.knl_name, name) || !strcmp(c.co_name, name)) {
            *idx = kStaticCount + (int)i;
            return GA_OK;
        }
    }
    if (!parsed) {
        *idx = -1;
        return fail(GA_ERR_NO_KERNEL, "kernel '%s' not in the manifest", name);
    }
    g_named.push_back(k);
    g_named_count.store((int)g_named.size(), std::memory_order_release);
    *idx = kStaticCount + (int)g_named.size() - 1;
    return GA_OK;
}

size_t ga_kernel_workspace_bytes(int idx, const ga_launch_desc* ld, int M, int N)
{
    (void)idx;
    if (!ld || ld->gdz <= 1 || M <= 0 || N <= 0)
        return 0;
    return (size_t)ld->gdz * M * N * sizeof(float);
}

} // extern "C"

namespace ga {

// ga_kernel_launch with the split-K workspace given either as a buffer
// (workspace, workspace_bytes; NULL: the library-owned one) or as a device
// slot read by the kernels at entry (wsh; graph-capture safe), and the
// operand element formats fmt = fmt(A) | fmt(B) << 1 (0 E4M3, 1 E5M2; MXFP8
// kernels only). With fmt != 0 the rows above the decode path run the
// 256x256 kernel whatever the entry's tile: every MXFP8 kernel computes the
// same fp32 chain of 128-K steps per K slice, so the tile is not visible in
// the output.
static ga_status kernel_launch(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy, int gdz,
                               void* workspace, size_t workspace_bytes,
                               const ga_splitk_ws_handle* wsh, void* stream, int fmt = 0)
{
    if (!args || idx < 0 || idx >= mx_registry_total())
        return fail(GA_ERR_ARG, "kernel_launch: bad kernel index %d", idx);
    const MxKernel& k = *mx_registry_get(idx);
    if (fmt < 0 || fmt > 3)
        return fail(GA_ERR_ARG, "kernel_launch: element formats must be 0 (E4M3) or 1 (E5M2)");
    if (fmt != 0 && k.elem_bits != 8)
        return fail(GA_ERR_ARG, "kernel_launch: element formats apply to the MXFP8 kernels "
                                "(kernel %d holds e2m1 operands)", idx);
    const int M = (int)args->M, N = (int)args->N, K = (int)args->K;
    if (M <= 0 || N <= 0 || K <= 0 || !args->ptr_A || !args->ptr_B || !args->ptr_D ||
        !args->ptr_ScaleA || !args->ptr_ScaleB)
        return fail(GA_ERR_ARG, "kernel_launch: null pointer or empty shape");
    // K granule: one K step (128 E4M3 / 256 e2m1 elements: 128 bytes per row),
    // the reference driver's K % 256 for MXFP4 (asm_f4gemm/README.md:43).
    const int kstep = k.elem_bits == 4 ? 256 : 128;
    const uint32_t row_align = k.elem_bits == 4 ? 32 : 16; // 16-byte rows, in elements
    if (K % kstep != 0)
        return fail(GA_ERR_SHAPE, "K must be a multiple of %d (got %d)", kstep, K);
    if (N % 16 != 0)
        return fail(GA_ERR_SHAPE, "N must be a multiple of 16 (got %d)", N);
    if (args->stride_C0 % 4 != 0 || args->stride_C0 < (uint32_t)N)
        return fail(GA_ERR_SHAPE, "stride_C0 must be >= N and a multiple of 4 (got %u)",
                    args->stride_C0);
    if (args->stride_A0 % row_align != 0 || args->stride_A0 < (uint32_t)K ||
        (!k.cfg.bpreshuffle &&
         (args->stride_B0 % row_align != 0 || args->stride_B0 < (uint32_t)K)))
        return fail(GA_ERR_SHAPE, "A/B row strides (elements) must be >= K and multiples of %u",
                    row_align);
    if (args->stride_ScaleA0 < (uint32_t)(K / 32) || args->stride_ScaleA0 % 8 ||
        args->stride_ScaleB0 < (uint32_t)(K / 32) || args->stride_ScaleB0 % 8)
        return fail(GA_ERR_SHAPE, "scale strides must be the padded column count "
                                  "round_up(K/32, 8)");
    {
        // Every kernel reads an operand through a buffer descriptor based at
        // its tile's (or wave's) first row, which addresses 4 GiB: at most
        // 512 rows of A or B, and the whole scale matrices, must fit in it.
        const unsigned long long lim = 0xFFFFFFF0ull;
        const unsigned long long ebits = (unsigned long long)k.elem_bits;
        const unsigned long long lda = args->stride_A0 * ebits / 8;
        const unsigned long long ldb = (k.cfg.bpreshuffle ? (unsigned long long)K
                                                          : args->stride_B0) * ebits / 8;
        const unsigned long long sa = ((unsigned long long)M + 255) / 256 * 256 * args->stride_ScaleA0;
        const unsigned long long sb = ((unsigned long long)N + 255) / 256 * 256 * args->stride_ScaleB0;
        if (512 * lda > lim || 512 * ldb > lim || sa > lim || sb > lim)
            return fail(GA_ERR_SHAPE, "operand rows or scale matrices too large for 32-bit "
                                      "buffer offsets (512 rows of A/B and each scale matrix "
                                      "must fit in 4 GiB)");
    }
    if (gdx != (N + k.cfg.tile_N - 1) / k.cfg.tile_N || gdy != (M + k.cfg.tile_M - 1) / k.cfg.tile_M ||
        gdz < 1)
        return fail(GA_ERR_ARG, "grid (%d,%d,%d) does not match tile %dx%d", gdx, gdy, gdz,
                    k.cfg.tile_M, k.cfg.tile_N);
    if (gdz > 1) {
        int L = args->log2_k_split;
        if (L < 0 || L > 30 || K % (1 << L) != 0)
            return fail(GA_ERR_SPLITK, "bad log2_k_split %d for K=%d", L, K);
        int kpt = ((K >> L) + 255) / 256 * 256;
        if ((K + kpt - 1) / kpt != gdz)
            return fail(GA_ERR_ARG, "gdz=%d does not match log2_k_split=%d", gdz, L);
    }
    hipStream_t s = (hipStream_t)stream;
    // a caller workspace is checked against ga_kernel_workspace_bytes whichever
    // path runs (the in-workgroup decode kernel sums K slices in LDS and needs
    // none)
    if (gdz > 1 && workspace && workspace_bytes < (size_t)gdz * M * N * sizeof(float))
        return fail(GA_ERR_WORKSPACE, "workspace %zu bytes, need %zu", workspace_bytes,
                    (size_t)gdz * M * N * sizeof(float));
    const bool decode = (int)args->M <= k.small_m_stream && mx_decode_applies(*args, gdz);
    int num_cu = 0;
    if (decode) {
        ga_status st = device_cu_count(&num_cu);
        if (st != GA_OK)
            return st;
    }
    int phys = gdz; // workgroups along K of the 17-64-row decode kernels
    const int split_groups = decode ? mx_decode_split_groups(*args, gdz, num_cu, &phys) : 0;
    if (decode && split_groups == 0) {
        // few rows: stream B, K slices summed inside the kernel (no workspace)
        launch_mx_decode(*args, gdz, k.cfg.bpreshuffle != 0, k.elem_bits == 4, fmt, num_cu, s);
        GA_HIP_CHECK(hipGetLastError());
        return GA_OK;
    }
    if (decode && phys == 1) {
        // 17-64 rows, every K slice in one workgroup along K (no workspace)
        launch_mx_decode_split(*args, gdz, 1, split_groups, k.cfg.bpreshuffle != 0,
                               k.elem_bits == 4, fmt, nullptr, nullptr, num_cu, s);
        GA_HIP_CHECK(hipGetLastError());
        return GA_OK;
    }
    float* ws = nullptr;
    if (gdz > 1 && wsh) {
        // the host mirror of a library-made slot catches a missing reserve
        // outside capture; the kernels check the slot itself at every run
        size_t have = 0;
        if (ws_slot_bytes(wsh, &have) && have < (size_t)gdz * M * N * sizeof(float)) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            GA_HIP_CHECK(hipStreamIsCapturing(s, &cs));
            if (cs == hipStreamCaptureStatusNone)
                return fail(GA_ERR_WORKSPACE, "workspace slot holds %zu bytes, need %zu", have,
                            (size_t)gdz * M * N * sizeof(float));
        }
    } else if (gdz > 1) {
        size_t need = (size_t)gdz * M * N * sizeof(float);
        if (workspace) {
            ws = (float*)workspace; // size checked above
        } else {
            // the library-owned buffer may be reallocated by a later call: a
            // captured graph would keep a pointer that is then freed
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            GA_HIP_CHECK(hipStreamIsCapturing(s, &cs));
            if (cs != hipStreamCaptureStatusNone)
                return fail(GA_ERR_WORKSPACE, "split-K launch under stream capture needs a "
                                              "caller workspace");
            void* p = nullptr;
            ga_status st = default_workspace(need, &p);
            if (st != GA_OK)
                return st;
            ws = (float*)p;
        }
    }
    if (split_groups > 0)
        launch_mx_decode_split(*args, gdz, phys, split_groups, k.cfg.bpreshuffle != 0, k.elem_bits == 4,
                               fmt, ws, wsh, num_cu, s);
    else if (fmt != 0)
        launch_mx_pp_fmt(*args, ws, gdz > 1 ? wsh : nullptr, gdz, k.cfg.bpreshuffle != 0, fmt, s);
    else
        k.launch(*args, ws, gdz > 1 ? wsh : nullptr, gdx, gdy, gdz, s);
    GA_HIP_CHECK(hipGetLastError());
    if (gdz > 1) {
        ReduceArgs r;
        r.ws = ws;
        r.wsh = wsh;
        r.out = args->ptr_D;
        r.c_in = (args->beta != 0.0f) ? args->ptr_C : nullptr;
        r.bias = nullptr;
        r.out_dtype = GA_DTYPE_BF16;
        r.bias_dtype = GA_DTYPE_F32;
        r.split_k = gdz;
        r.M = M;
        r.N = N;
        r.batch = 1;
        r.ws_ld = N;
        r.ws_batch = (long long)M * N;
        r.ldc = (int)args->stride_C0;
        r.c_batch_stride = 0;
        r.bias_stride_batch = 0;
        r.alpha = args->alpha;
        r.beta = args->beta;
        return splitk_reduce_launch(r, s);
    }
    return GA_OK;
}

} // namespace ga

extern "C" {

ga_status ga_kernel_launch(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy, int gdz,
                           void* workspace, size_t workspace_bytes, void* stream)
{
    return kernel_launch(idx, args, gdx, gdy, gdz, workspace, workspace_bytes, nullptr, stream);
}

ga_status ga_kernel_launch_ws_handle(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy,
                                     int gdz, const ga_splitk_ws_handle* ws_handle, void* stream)
{
    if (gdz > 1 && !ws_handle)
        return fail(GA_ERR_ARG, "kernel_launch_ws_handle: null workspace slot");
    return kernel_launch(idx, args, gdx, gdy, gdz, nullptr, 0, ws_handle, stream);
}

ga_status ga_kernel_launch_fmt(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy, int gdz,
                               int fmt_a, int fmt_b, void* workspace, size_t workspace_bytes,
                               void* stream)
{
    if (fmt_a < 0 || fmt_a > 1 || fmt_b < 0 || fmt_b > 1)
        return fail(GA_ERR_ARG, "kernel_launch_fmt: formats must be 0 (E4M3) or 1 (E5M2), got "
                                "%d, %d", fmt_a, fmt_b);
    return kernel_launch(idx, args, gdx, gdy, gdz, workspace, workspace_bytes, nullptr, stream,
                         fmt_a | (fmt_b << 1));
}

} // extern "C"

namespace ga {

// Split-K partials of ga_kernel_launch_noalloc: a fixed device array (each
// GPU the library runs on holds its own copy until the process ends). Host
// code never uses the array's name as an address: scratch_address() looks
// the copy of the current device up once with hipGetSymbolAddress.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

static ga_status scratch_address(float** out)
{
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static float* per_device[kMaxDevices] = {};
    int dev = 0;
    GA_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(GA_ERR_ARG, "kernel_launch_noalloc: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(mu);
    if (!per_device[dev]) {
        void* p = nullptr;
        GA_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p)
            return fail(GA_ERR_HIP, "kernel_launch_noalloc: no address for the scratch array");
        per_device[dev] = (float*)p;
    }
    *out = per_device[dev];
    return GA_OK;
}

} // namespace ga

extern "C" {

ga_status ga_kernel_launch_noalloc(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy,
                                   int gdz, void* stream)
{
    if (!args)
        return fail(GA_ERR_ARG, "kernel_launch_noalloc: null args");
    float* ws = nullptr;
    if (gdz > 1) {
        const unsigned long long need =
            (unsigned long long)gdz * args->M * args->N * sizeof(float);
        if (need > kScratchBytes)
            return fail(GA_ERR_WORKSPACE,
                        "kernel_launch_noalloc: split-K partials need %llu bytes, the scratch "
                        "holds %zu (gdz * M * N * 4 must fit)", need, kScratchBytes);
        ga_status st = scratch_address(&ws);
        if (st != GA_OK)
            return st;
    }
    return kernel_launch(idx, args, gdx, gdy, gdz, ws, kScratchBytes, nullptr, stream);
}

ga_status ga_mxfp8_gemm(void* d_D, const void* d_A, const void* d_B, const void* d_ScaleA,
                        const void* d_ScaleB, int M, int N, int K, int stride_D0,
                        int bpreshuffle, int log2_k_split, int num_cu, void* workspace,
                        size_t workspace_bytes, int* chosen, ga_launch_desc* ld_out,
                        void* stream)
{
    if (num_cu <= 0) {
        ga_status st = ga_device_num_cu(&num_cu);
        if (st != GA_OK)
            return st;
    }
    int idx = -1, l2 = 0;
    ga_status st = ga_select_kernel(M, N, K, num_cu, log2_k_split, bpreshuffle, nullptr, 0,
                                    &idx, &l2);
    if (st != GA_OK)
        return st;
    ga_launch_desc ld;
    st = ga_make_launch(&g_mx_kernels[idx].cfg, M, N, K, l2, &ld);
    if (st != GA_OK)
        return st;
    ga_mx_shape sh;
    st = ga_mx_shape_init(M, N, K, 8, &sh);
    if (st != GA_OK)
        return st;
    ga_f4gemm_kargs args;
    ga_fill_args(&args, d_D, nullptr, (void*)d_A, (void*)d_B, (void*)d_ScaleA, (void*)d_ScaleB,
                 M, N, K, stride_D0, sh.scale_cols, sh.scale_cols, 1.0f, 0.0f, ld.log2_k_split);
    if (chosen)
        *chosen = idx;
    if (ld_out)
        *ld_out = ld;
    return ga_kernel_launch(idx, &args, ld.gdx, ld.gdy, ld.gdz, workspace, workspace_bytes,
                            stream);
}

ga_status ga_mxfp4_gemm(void* d_D, const void* d_A, const void* d_B, const void* d_ScaleA,
                        const void* d_ScaleB, int M, int N, int K, int stride_D0,
                        int bpreshuffle, int log2_k_split, int num_cu, void* workspace,
                        size_t workspace_bytes, int* chosen, ga_launch_desc* ld_out,
                        void* stream)
{
    if (num_cu <= 0) {
        ga_status st = ga_device_num_cu(&num_cu);
        if (st != GA_OK)
            return st;
    }
    ga_tile_config table[kMx4Count];
    for (int i = 0; i < kMx4Count; i++)
        table[i] = g_mx_kernels[kMx4First + i].cfg;
    int row = -1, l2 = 0;
    ga_status st = ga_select_kernel(M, N, K, num_cu, log2_k_split, bpreshuffle, table, kMx4Count,
                                    &row, &l2);
    if (st != GA_OK)
        return st;
    const int idx = kMx4First + row;
    ga_launch_desc ld;
    st = ga_make_launch(&g_mx_kernels[idx].cfg, M, N, K, l2, &ld);
    if (st != GA_OK)
        return st;
    ga_mx_shape sh;
    st = ga_mx_shape_init(M, N, K, 4, &sh);
    if (st != GA_OK)
        return st;
    ga_f4gemm_kargs args;
    ga_fill_args(&args, d_D, nullptr, (void*)d_A, (void*)d_B, (void*)d_ScaleA, (void*)d_ScaleB,
                 M, N, K, stride_D0, sh.scale_cols, sh.scale_cols, 1.0f, 0.0f, ld.log2_k_split);
    if (chosen)
        *chosen = idx;
    if (ld_out)
        *ld_out = ld;
    return ga_kernel_launch(idx, &args, ld.gdx, ld.gdy, ld.gdz, workspace, workspace_bytes,
                            stream);
}

} // extern "C"

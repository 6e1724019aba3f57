// gemm_mx_decode.hip -- MXFP8 GEMM for small M (decode), HBM-streaming.
//
// Used by every manifest kernel for M <= 64 rows (measured on MI355X: for
// 33-64 rows the tiles' own grids cover too few CUs, e.g. M = 48, N = 8192,
// K = 28672 on 256x128: 215 us, here 70 us): with so few rows the GEMM
// is a stream over B (N x K bytes), so the design is about keeping HBM busy:
//  * one wave per NG 16-column groups of B and one K slice; B's 2 KB per
//    group and 128-K step (two 1 KB contiguous runs in the preshuffled
//    layout) goes straight from memory into the MFMA operand registers;
//  * a ring of D steps of loads in flight per wave (24 KB of B for M <= 16);
//  * the A rows (<= 64, L2-resident) are loaded the same way, once per step
//    for all NG groups, and multiply B with v_mfma_scale_f32_16x16x128_f8f6f4,
//    one MFMA per 16 rows per group per step;
//  * split-K: the gdz K slices of a column group are separate fp32 chains
//    summed in slice order (slice 0 first), the order the split-K reduce
//    uses, so no workspace is needed. For 1-16 rows one wave runs them in
//    turn, so the split a caller asks for (which fixes the output bits) does
//    not change the stream of loads; for more rows they run in waves of the
//    same workgroup and are summed in LDS;
//  * workgroup = T column tasks x KS slices (T * KS <= 8 waves; KS = 1 for
//    1-16 rows);
//  * MXFP4 (e2m1 packed two per byte): a step is 256 K = the same 128 bytes
//    per row, so the loads are identical; two fp4 MFMAs per group and 16
//    rows (K halves 0 and 1 of the step), one whole scale dword per step.
//  * split variant (XS; 17-64 rows with the caller's gdz > 1, or one slice
//    over N wide enough for five groups per CU): the K slice is blockIdx.y
//    and each wave owns NG (2-8) groups, so a CU reads A once per up to 128
//    columns instead of once per 32 (at 64 rows and NG = 8, A is half the
//    bytes of B rather than twice); waves x slices fill whole rounds of one
//    wave per CU. The slices' fp32 partials go to the split-K workspace and
//    the split-K reduce sums them in slice order, slice 0 first, as above;
//    one slice applies the epilogue in the kernel. Measured on MI355X, M =
//    64, N = 8192, K = 28672: 70 us in-workgroup at any split, 45.9 us here
//    at 4 slices (41.9 us kernel + 4 us reduce); N = 28672, K = 8192, one
//    slice: 65 -> 54.7 us. Each group's next B loads go out right after the
//    MFMAs of the following group, so they never wait on an MFMA still
//    reading their registers and the wave's requests spread over its MFMAs.
#include "ga_device.hpp"
#include "ga_internal.hpp"
#include <algorithm>

namespace ga {
namespace {

// DEEP: up to 4 waves per workgroup, so each may use 512 registers and keep
// more steps in flight (4 of 64 rows, 6 of 32 rows; for long K with one
// column task per CU).
// XS > 0: the cross-workgroup split with XS steps in flight, one wave per
// SIMD (512 registers).
template <int TM, int NG_, bool DEEP = false, int XS = 0>
struct DecCfg {
    static constexpr int NG = NG_; // 16-column groups per wave
    static constexpr int D = XS > 0 ? XS
                           : DEEP ? (TM == 4 ? 4 : 6)
                                  : TM == 1 ? 6 : (TM == 2 ? (NG == 1 ? 6 : 4) : (NG == 1 ? 4 : 3));
    static constexpr int MAX_WAVES = (DEEP || XS > 0) ? 4 : 8;
    // B scale dwords per step: a wave of the split variant with an even NG
    // starts at an even group, so groups 2j and 2j + 1 share the dword of one
    // 32-row block
    static constexpr int NB = (XS > 0 && NG % 2 == 0) ? NG / 2 : NG;
};

// Uniform byte offsets as SGPR operands.
__device__ __forceinline__ uint32_t uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// A K slice's fp32 partials to the split-K workspace, [slice][M][N] (lane
// holds C[m][n .. n+3], m = 16i + lane%16, n = 16cg + 4(lane/16)), for the
// groups [cg0, cg0 + ng_here) and the rows below M.
template <int NG, int TM>
__device__ __forceinline__ void dec_store_partials(float* ws, const v4f (&acc)[NG][TM], int slice,
                                                   int cg0, int ng_here, int M, int N, int lane)
{
#pragma unroll
    for (int c = 0; c < NG; c++) {
        if (c >= ng_here)
            continue;
        const int n = (cg0 + c) * 16 + (lane >> 4) * 4;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int m = i * 16 + (lane & 15);
            if (m < M)
                *(v4f*)(ws + ((size_t)slice * M + m) * N + n) = acc[c][i];
        }
    }
}

// D = alpha * acc (+ beta * C) as bf16, same lane layout and bounds.
template <int NG, int TM>
__device__ __forceinline__ void dec_epilogue(const ga_f4gemm_kargs& args, const v4f (&acc)[NG][TM],
                                             int cg0, int ng_here, int lane)
{
    const int M = (int)args.M;
    const int ldd = (int)args.stride_C0;
    const float alpha = args.alpha, beta = args.beta;
    const bool use_c = beta != 0.0f && args.ptr_C != nullptr;
#pragma unroll
    for (int c = 0; c < NG; c++) {
        if (c >= ng_here)
            continue;
        const int n = (cg0 + c) * 16 + (lane >> 4) * 4;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int m = i * 16 + (lane & 15);
            if (m >= M)
                continue;
            const v4f v = acc[c][i];
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

// F: the operands' 8-bit element formats (fmt_of_a / fmt_of_b; 0 for MXFP4).
// LA (1-16 rows, in-workgroup): the workgroup's A panel, 16 rows x K, is
// copied once into LDS (kLaBytes at most) and every wave reads its A
// fragments from there instead of from L2 at every step.
constexpr int kLaBytes = 128 * 1024;
template <int TM, int NG_, bool BPS, bool FP4, bool DEEP, int XS = 0, int F = 0, bool LA = false>
__global__ __attribute__((amdgpu_flat_work_group_size(64, DecCfg<TM, NG_, DEEP, XS>::MAX_WAVES * 64)))
void mx_decode_kernel(ga_f4gemm_kargs args, int nwg, int ks, float* __restrict__ ws,
                      const ga_splitk_ws_handle* __restrict__ wsh)
{
    using Cfg = DecCfg<TM, NG_, DEEP, XS>;
    static_assert(!LA || (TM == 1 && XS == 0), "LDS-resident A: 1-16 rows, in-workgroup");
    constexpr int kEPB = FP4 ? 2 : 1; // elements per byte
    constexpr int D = Cfg::D, NG = NG_, NB = Cfg::NB;
    // 1-16 rows (in-workgroup variant): one wave runs all ks K slices of its
    // column task, one fp32 chain each, the stream of loads unbroken across
    // them; more rows: one wave per slice, summed through LDS. Split variant:
    // the ks K slices run on gridDim.y workgroups along K, each taking
    // kseq = ceil(ks / gridDim.y) <= 2 consecutive slices (all of them when
    // gridDim.y is 1, for up to 32 rows).
    constexpr bool kSeq = XS == 0 && TM == 1;
    constexpr bool kFoldTot = kSeq || (XS > 0 && TM <= 2); // chains summed in registers
    constexpr int SA = (TM + 1) / 2; // A scale dwords (32-row blocks)
    constexpr int kLoadsA = LA ? 0 : 2 * TM; // A loads per step (LA: LDS reads)
    constexpr int kLoadsPerStep = 2 * NG + kLoadsA + SA + NB;
    static_assert(kLoadsPerStep * (D - 1) < 64, "vmcnt range");
    // MXFP8 in-workgroup: a scale dword covers 256 K = two steps, so only the
    // even ring slots (the even steps: D is even) load scales and the odd
    // step reuses its even neighbour's, kept from that step's MFMAs. The
    // wait before slot J's MFMAs counts the D - 1 other slots' loads, issued
    // after slot J's: D/2 - 1 slots of J's parity and D/2 of the other.
    constexpr bool kPairScales = !FP4 && XS == 0 && D % 2 == 0;
    constexpr int kLoadsOdd = kPairScales ? 2 * NG + kLoadsA : kLoadsPerStep;
    constexpr int kWaitEven =
        kPairScales ? (D / 2 - 1) * kLoadsPerStep + (D / 2) * kLoadsOdd : (D - 1) * kLoadsPerStep;
    constexpr int kWaitOdd =
        kPairScales ? (D / 2) * kLoadsPerStep + (D / 2 - 1) * kLoadsOdd : (D - 1) * kLoadsPerStep;
    // loads of the D prologue steps, issued after the LA copies
    constexpr int kWaitPro = kPairScales ? (D / 2) * (kLoadsPerStep + kLoadsOdd) : D * kLoadsPerStep;
    static_assert(!LA || kWaitPro < 64, "vmcnt range");
    __shared__ __attribute__((aligned(16))) char a_lds[LA ? kLaBytes : 16];
    // in-workgroup K slices are summed through LDS (<= 8 waves; 1-16 rows sum
    // them in registers); the split variant parks the first of its two
    // chains in LDS until both are stored
    __shared__ __attribute__((aligned(16))) float red[(XS > 0 || kSeq) ? 4 : 8 * NG * TM * 256];
    __shared__ __attribute__((aligned(16))) float park[XS > 0 ? NG * TM * 256 : 4];
    if constexpr (XS > 0) {
        if (gridDim.y > 1 && wsh && !(ws = resolve_ws(wsh, ks, args.M, args.N)))
            return; // workspace slot shorter than the split-K layout: write nothing
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kp = (XS > 0 || kSeq) ? 1 : ks; // waves per column task
    const int slice = XS > 0 ? (int)blockIdx.y : wave % kp;
    const int tl = XS > 0 ? wave : wave / kp;
    const int M = (int)args.M, N = (int)args.N, K = (int)args.K;
    // Workgroup b owns 16-column groups [b*G/nwg, (b+1)*G/nwg): equal shares
    // (within one group) for every CU; its waves take NG groups each. In the
    // split variant wave w of workgroup b takes groups from (b*waves + w)*NG.
    const int ngroups = N / 16;
    int g_end, cg0;
    if constexpr (XS > 0) {
        g_end = ngroups;
        cg0 = ((int)blockIdx.x * (int)(blockDim.x >> 6) + tl) * NG;
    } else {
        g_end = (int)(((long long)(blockIdx.x + 1) * ngroups) / nwg);
        cg0 = (int)(((long long)blockIdx.x * ngroups) / nwg) + tl * NG;
    }
    const int ng_here = min(NG, g_end - cg0); // groups past it read as zero
    const bool live = ng_here > 0;

    int kpt = K;
    if (ks > 1)
        kpt = ((K >> args.log2_k_split) + 255) / 256 * 256;
    // the wave's K slices: [z0, z0 + kseq) (kSeq: all of them)
    const int kseq = kSeq ? ks : XS > 0 ? (ks + (int)gridDim.y - 1) / (int)gridDim.y : 1;
    const int z0 = kSeq ? 0 : slice * kseq;
    const int kb = z0 * kpt;
    const int ke = min(K, kb + kseq * kpt);
    const int nsteps = live ? max(0, (ke - kb) / (128 * kEPB)) : 0;
    const int kbb = kb / kEPB, Kb = K / kEPB; // bytes

    v4f acc[NG][TM];
#pragma unroll
    for (int c = 0; c < NG; c++)
#pragma unroll
        for (int i = 0; i < TM; i++)
            acc[c][i] = (v4f){0.f, 0.f, 0.f, 0.f};

    // Sequential slices: each finished chain is added into tot, which starts
    // at -0 (-0 + x == x for every x, signed zeros included), so tot is p0,
    // p0 + p1, ... in slice order, the split-K reduce's order. A fold runs
    // after a chain's last step: fold_at counts the wave's steps (never the
    // final step, whose chain the fold after the loop takes).
    // Split variant over several workgroups: the wave's first chain is
    // parked in LDS at the fold (a store there would count in vmcnt beside
    // the stream's counted loads), both are stored at the end.
    v4f tot[kFoldTot ? NG : 1][kFoldTot ? TM : 1];
    const int sps = kpt / (128 * kEPB); // steps per K slice
    const bool in_regs = XS == 0 || gridDim.y == 1; // chains summed in tot
    int fold_at = ((kSeq || XS > 0) && kseq > 1 && sps < nsteps) ? sps : 0x7FFFFFFF;
    auto fold = [&]() {
        if constexpr (kFoldTot) {
            if (in_regs) {
#pragma unroll
                for (int c = 0; c < NG; c++)
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        tot[c][i] = tot[c][i] + acc[c][i];
                        acc[c][i] = (v4f){0.f, 0.f, 0.f, 0.f};
                    }
            }
        }
        if constexpr (XS > 0) {
            if (!in_regs) {
#pragma unroll
                for (int c = 0; c < NG; c++)
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        *(v4f*)(park + (c * TM + i) * 256 + lane * 4) = acc[c][i];
                        acc[c][i] = (v4f){0.f, 0.f, 0.f, 0.f};
                    }
            }
        }
    };
    if constexpr (kFoldTot) {
#pragma unroll
        for (int c = 0; c < NG; c++)
#pragma unroll
            for (int i = 0; i < TM; i++)
                tot[c][i] = (v4f){-0.f, -0.f, -0.f, -0.f};
    }
    // after the MFMAs of step t (0-based within the wave's range)
    auto fold_after = [&](int t) {
        if constexpr (kSeq || XS > 0) {
            if (t + 1 == fold_at) {
                fold();
                fold_at += sps;
                if (fold_at >= nsteps)
                    fold_at = 0x7FFFFFFF;
            }
        }
    };

    const int r = lane & 15, g = lane >> 4;
    const uint32_t lda = args.stride_A0 / kEPB; // bytes
    const long long abytes = (long long)M * lda;
    const auto ra = make_rsrc(args.ptr_A, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
    // A: lane 16g + r reads row 16i + r, K chunks g and g + 4 of the step
    const uint32_t va = (uint32_t)r * lda + g * 16 + (uint32_t)kbb;
    if constexpr (LA) {
        // The panel holds step s as 16 rows of 128 bytes at LDS byte s * 2048,
        // K chunk c of row r at slot c ^ ((r >> 1) & 7). Copy q = 2s + h
        // writes rows 8h .. 8h + 7 of step s: lane l reads whole 128-byte
        // lines (row 8h + l / 8, slot l % 8; rows past M read as zeros) to LDS
        // byte q * 1024 + l * 16 (copies of 16 rows x 64 bytes per
        // instruction move the same bytes slower). The waves take the copies
        // in turn; a wave without columns waits for its own and meets the
        // others at the barrier the working waves take after their prologue.
        const int nw = (int)(blockDim.x >> 6);
        const int ncopies = 2 * (K / (128 * kEPB));
        const uint32_t crow = (uint32_t)lane >> 3, cslot = lane & 7;
        const uint32_t cva0 = crow * lda + ((cslot ^ ((crow >> 1) & 7)) * 16) + (uint32_t)kbb;
        const uint32_t cva1 = (crow + 8) * lda + ((cslot ^ (((crow + 8) >> 1) & 7)) * 16) +
                              (uint32_t)kbb;
        for (int q = wave; q < ncopies; q += nw)
            lds_load16(ra, (lds_void*)(a_lds + q * 1024),
                       ((q & 1) ? cva1 : cva0) + uni((uint32_t)(q >> 1) * 128), 0);
        __builtin_amdgcn_sched_barrier(0); // the prologue's counted loads follow the copies
        if (nsteps == 0) {
            wait_vmcnt<0>();
            barrier_lds();
        }
    }

    if (nsteps > 0) {
        // B: groups past N read as zero (range-checked buffer)
        __amdgpu_buffer_rsrc_t rbuf;
        uint32_t vb, b_step, b_hi, b_grp;
        if (BPS) {
            // group cg: Kb*16 contiguous bytes, [Kb/16][16 rows][16 B]
            const char* pb = (const char*)args.ptr_B + (size_t)cg0 * Kb * 16;
            rbuf = make_rsrc(pb, (uint32_t)ng_here * (uint32_t)Kb * 16);
            vb = (uint32_t)lane * 16 + (uint32_t)kbb * 16;
            b_step = 2048;
            b_hi = 1024;
            b_grp = (uint32_t)Kb * 16;
        } else {
            const uint32_t ldb = args.stride_B0 / kEPB; // bytes
            const char* pb = (const char*)args.ptr_B + (size_t)cg0 * 16 * ldb;
            rbuf = make_rsrc(pb, (uint32_t)ng_here * 16 * ldb);
            vb = (uint32_t)r * ldb + g * 16 + (uint32_t)kbb;
            b_step = 128;
            b_hi = 64;
            b_grp = 16 * ldb;
        }
        // scales: shuffled dword of lane l covers (row l%16 + 16 h, K block
        // l/16) for 256 K; byte 2*(128-K half) + h (MXFP8: the half is the
        // step parity; MXFP4: both halves in one step)
        const uint32_t sna = args.stride_ScaleA0, snb = args.stride_ScaleB0;
        const auto rsa = make_rsrc(args.ptr_ScaleA, (uint32_t)((M + 31) / 32 * 32) * sna);
        const auto rsb = make_rsrc(args.ptr_ScaleB, (uint32_t)((N + 31) / 32 * 32) * snb);
        const uint32_t vsa = ((uint32_t)(kb / 256)) * 256 + lane * 4;
        // group cg uses byte (cg & 1) of 32-row block cg/2 (one dword per
        // group, or per group pair in the split variant)
        uint32_t vsb[NB];
#pragma unroll
        for (int c = 0; c < NB; c++) {
            const int cg = NB == NG ? cg0 + c : cg0 + 2 * c;
            vsb[c] = ((uint32_t)(cg / 2) * (snb / 8) + (uint32_t)(kb / 256)) * 256 + lane * 4;
        }
        const uint32_t sa_blk = (sna / 8) * 256;

        v8i fb[D][NG];
        v8i fa[D][TM];
        uint32_t fsa[D][SA], fsb[D][NB];

        auto load = [&](int s, auto J) {
            constexpr int j = decltype(J)::value;
            const uint32_t ob = (uint32_t)s * b_step;
#pragma unroll
            for (int c = 0; c < NG; c++) {
                v4i x0 = buf_load16_stream(rbuf, vb + uni(ob + c * b_grp), 0);
                v4i x1 = buf_load16_stream(rbuf, vb + uni(ob + c * b_grp + b_hi), 0);
                fb[j][c] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            }
            if constexpr (!LA) {
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const uint32_t oa = (uint32_t)s * 128 + (uint32_t)i * 16 * lda;
                    v4i y0 = buf_load16(ra, va + uni(oa), 0);
                    v4i y1 = buf_load16(ra, va + uni(oa + 64), 0);
                    fa[j][i] = (v8i){y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
                }
            }
            if constexpr (!kPairScales || j % 2 == 0) {
                const uint32_t q = (uint32_t)(FP4 ? s : (s >> 1)) * 256;
#pragma unroll
                for (int h = 0; h < SA; h++)
                    fsa[j][h] = buf_load4(rsa, vsa + uni(q + h * sa_blk), 0);
#pragma unroll
                for (int c = 0; c < NB; c++)
                    fsb[j][c] = buf_load4(rsb, vsb[c] + uni(q), 0);
            }
        };
        // LA: step s's A fragment from the panel in LDS: lane 16g + r reads
        // row r, chunks g and g + 4 (slots g ^ sw and g ^ sw ^ 4, sw =
        // (r >> 1) & 7: 64 distinct banks per 16 lanes)
        const uint32_t ao = (uint32_t)r * 128 + ((g ^ ((r >> 1) & 7)) * 16);
        auto read_a = [&](int s, auto J) {
            if constexpr (LA) {
                constexpr int j = decltype(J)::value;
                const v4i y0 = *(const v4i*)(a_lds + s * 2048 + ao);
                const v4i y1 = *(const v4i*)(a_lds + s * 2048 + (ao ^ 64u));
                fa[j][0] = (v8i){y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
            }
        };
        // The odd step's scale operands, shifted out of the even slot's
        // registers during the even step: load() refills those registers right
        // after it, so the odd step cannot read them. The empty asm keeps the
        // shifted values from being recomputed (which would keep the even
        // slot's old registers live across the refill).
        uint32_t osa[TM], osb[NG];
        auto mma = [&](int s, auto J) {
            constexpr int j = decltype(J)::value;
            constexpr bool odd = kPairScales && j % 2 == 1;
            const uint32_t sh = FP4 ? 0u : (uint32_t)(s & 1) * 16;
            uint32_t sbv[NG], sav[TM];
#pragma unroll
            for (int c = 0; c < NG; c++)
                sbv[c] = odd ? osb[c] : fsb[j][NB == NG ? c : c / 2] >> (sh + 8 * ((cg0 + c) & 1));
#pragma unroll
            for (int i = 0; i < TM; i++)
                sav[i] = odd ? osa[i] : fsa[j][i >> 1] >> (sh + 8 * (i & 1));
            if constexpr (kPairScales && j % 2 == 0) {
#pragma unroll
                for (int c = 0; c < NG; c++) {
                    osb[c] = fsb[j][NB == NG ? c : c / 2] >> (16 + 8 * ((cg0 + c) & 1));
                    asm volatile("" : "+v"(osb[c]));
                }
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    osa[i] = fsa[j][i >> 1] >> (16 + 8 * (i & 1));
                    asm volatile("" : "+v"(osa[i]));
                }
            }
#pragma unroll
            for (int c = 0; c < NG; c++) {
                const uint32_t sb = sbv[c];
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const uint32_t sa = sav[i];
                    if constexpr (FP4) {
                        acc[c][i] = mfma_mx16_fp4<0, 0>(fb[j][c], fa[j][i], acc[c][i], (int)sb,
                                                        (int)sa);
                        acc[c][i] = mfma_mx16_fp4<0, 0>(hi16(fb[j][c]), hi16(fa[j][i]), acc[c][i],
                                                        (int)(sb >> 16), (int)(sa >> 16));
                    } else {
                        acc[c][i] = mfma_mx16<0, 0, fmt_of_b(F), fmt_of_a(F)>(
                            fb[j][c], fa[j][i], acc[c][i], (int)sb, (int)sa);
                    }
                }
            }
        };

        // Split variant: step s's MFMAs group by group, the B loads of group
        // c - 1 for step sn issued after group c's MFMAs (the MFMAs reading
        // group c - 1's registers are done by then, so the loads do not wait
        // on them): the wave's memory requests spread over the MFMA block
        // instead of following it. Then A and the scales, in load()'s order.
        auto mma_load = [&](int s, int sn, auto J) {
            constexpr int j = decltype(J)::value;
            const uint32_t sh = FP4 ? 0u : (uint32_t)(s & 1) * 16;
            uint32_t sav[SA], sbv[NB];
#pragma unroll
            for (int h = 0; h < SA; h++)
                sav[h] = fsa[j][h];
#pragma unroll
            for (int c = 0; c < NB; c++)
                sbv[c] = fsb[j][c];
            const uint32_t ob = (uint32_t)sn * b_step;
#pragma unroll
            for (int c = 0; c < NG; c++) {
                const uint32_t sb = sbv[NB == NG ? c : c / 2] >> (sh + 8 * ((cg0 + c) & 1));
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const uint32_t sa = sav[i >> 1] >> (sh + 8 * (i & 1));
                    if constexpr (FP4) {
                        acc[c][i] = mfma_mx16_fp4<0, 0>(fb[j][c], fa[j][i], acc[c][i], (int)sb,
                                                        (int)sa);
                        acc[c][i] = mfma_mx16_fp4<0, 0>(hi16(fb[j][c]), hi16(fa[j][i]), acc[c][i],
                                                        (int)(sb >> 16), (int)(sa >> 16));
                    } else {
                        acc[c][i] = mfma_mx16<0, 0, fmt_of_b(F), fmt_of_a(F)>(
                            fb[j][c], fa[j][i], acc[c][i], (int)sb, (int)sa);
                    }
                }
                if (c > 0) {
                    v4i x0 = buf_load16_stream(rbuf, vb + uni(ob + (c - 1) * b_grp), 0);
                    v4i x1 = buf_load16_stream(rbuf, vb + uni(ob + (c - 1) * b_grp + b_hi), 0);
                    fb[j][c - 1] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            {
                v4i x0 = buf_load16_stream(rbuf, vb + uni(ob + (NG - 1) * b_grp), 0);
                v4i x1 = buf_load16_stream(rbuf, vb + uni(ob + (NG - 1) * b_grp + b_hi), 0);
                fb[j][NG - 1] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t oa = (uint32_t)sn * 128 + (uint32_t)i * 16 * lda;
                v4i y0 = buf_load16(ra, va + uni(oa), 0);
                v4i y1 = buf_load16(ra, va + uni(oa + 64), 0);
                fa[j][i] = (v8i){y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
            }
            const uint32_t q = (uint32_t)(FP4 ? sn : (sn >> 1)) * 256;
#pragma unroll
            for (int h = 0; h < SA; h++)
                fsa[j][h] = buf_load4(rsa, vsa + uni(q + h * sa_blk), 0);
#pragma unroll
            for (int c = 0; c < NB; c++)
                fsb[j][c] = buf_load4(rsb, vsb[c] + uni(q), 0);
        };

        // The loads of each step stay in issue order (slot 0 oldest), so the
        // wait before step s+J's MFMAs lets the D-1 younger steps fly.
        static_for<D>([&](auto J) {
            load(min((int)J, nsteps - 1), J);
            __builtin_amdgcn_sched_barrier(0);
        });
        if constexpr (LA) {
            // the panel copies were issued before the prologue's loads: this
            // wave's have landed, and after the barrier every wave's
            wait_vmcnt<kWaitPro>();
            barrier_lds();
            static_for<D>([&](auto J) { read_a(min((int)J, nsteps - 1), J); });
        }
        int s = 0;
        for (; s + D <= nsteps; s += D) {
            static_for<D>([&](auto J) {
                wait_vmcnt<(decltype(J)::value % 2 == 0) ? kWaitEven : kWaitOdd>();
                if constexpr (XS > 0) {
                    mma_load(s + J, min(s + D + (int)J, nsteps - 1), J);
                    fold_after(s + J);
                } else {
                    mma(s + J, J);
                    load(min(s + D + (int)J, nsteps - 1), J);
                    read_a(min(s + D + (int)J, nsteps - 1), J);
                    fold_after(s + J);
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        }
        static_for<D>([&](auto J) {
            if ((int)J < nsteps - s) {
                mma(s + J, J);
                fold_after(s + J);
            }
        });
    }

    // Split variant: this workgroup's K slices' fp32 partials to the
    // workspace (the parked first chain, then the last); one workgroup along
    // K: the epilogue below.
    if constexpr (XS > 0) {
        if (gridDim.y > 1) {
            if (live) {
                int z = z0;
                if (kseq > 1 && ke - kb > kpt) {
                    v4f first[NG][TM];
#pragma unroll
                    for (int c = 0; c < NG; c++)
#pragma unroll
                        for (int i = 0; i < TM; i++)
                            first[c][i] = *(const v4f*)(park + (c * TM + i) * 256 + lane * 4);
                    dec_store_partials<NG, TM>(ws, first, z++, cg0, ng_here, M, N, lane);
                }
                dec_store_partials<NG, TM>(ws, acc, z, cg0, ng_here, M, N, lane);
            }
            return;
        }
    }
    // Sum the K slices of each column group in slice order, then the epilogue.
    if constexpr (kFoldTot) {
        if (ks > 1) {
            fold(); // the last slice
#pragma unroll
            for (int c = 0; c < NG; c++)
#pragma unroll
                for (int i = 0; i < TM; i++)
                    acc[c][i] = tot[c][i];
        }
    } else if (XS == 0 && ks > 1) {
        float* mine = red + ((tl * ks + slice) * NG * TM) * 256;
#pragma unroll
        for (int c = 0; c < NG; c++)
#pragma unroll
            for (int i = 0; i < TM; i++)
                *(v4f*)(mine + (c * TM + i) * 256 + lane * 4) = acc[c][i];
        __syncthreads();
        if (slice != 0)
            return;
#pragma unroll
        for (int c = 0; c < NG; c++)
#pragma unroll
            for (int i = 0; i < TM; i++) {
                v4f t = *(const v4f*)(mine + (c * TM + i) * 256 + lane * 4);
                for (int z = 1; z < ks; z++) {
                    const v4f u =
                        *(const v4f*)(mine + ((z * NG + c) * TM + i) * 256 + lane * 4);
                    t = t + u;
                }
                acc[c][i] = t;
            }
    }
    if (live)
        dec_epilogue<NG, TM>(args, acc, cg0, ng_here, lane);
}

// Shared-A split variant (33-64 rows). A workgroup of W waves (four: one per
// SIMD; eight: two per SIMD) takes K slice blockIdx.y of a contiguous range
// of column groups (nwg equal shares), each wave up to NG of them. Each
// step's A rows (TM x 16 rows x 128 bytes) go into an LDS ring of D steps
// with direct-to-LDS loads, 2 * TM / W one-KB copies per wave, and every wave
// reads the whole step from there: a CU reads A once per step for all its
// columns, and the MFMAs of the 64 rows spread over the four SIMDs. B and the scales stream
// into registers as in the other variants (ring of D steps per wave).
// Step u: wait for the wave's loads of step u, barrier (every wave's copies
// of step u landed, every wave's LDS reads of step u - 1 done), read step u's
// A, copy step u + D - 1's A into the slot step u - 1 used, MFMAs, then step
// u + D's B and scales into the registers step u used. MXFP8 scales as in
// the in-workgroup variant: one dword per pair of steps, loaded on the even
// step, the odd step's operands shifted out during the even step.
// One slice applies the epilogue; more write fp32 partials for the split-K
// reduce (ws, or the slot wsh), as the split variant does.
template <int TM, int NG, bool FP4, int W_ = 4>
struct LaCfg {
    static constexpr int W = W_;                      // waves per workgroup
    static constexpr int SA = (TM + 1) / 2;           // A scale dwords per step
    static constexpr int BPW = 2 * TM / W;            // A copies per wave per step
    static constexpr int LB = 2 * NG;                 // B loads per step
    static constexpr int SS = SA + NG;                // scale loads per (even) step
    // deepest ring whose waits stay within the 63 loads vmcnt counts, at most
    // 6 (measured on MI355X, one-group waves, M = 64, N = 28672, K = 8192,
    // best of 3 x 100 calls: 42.3 us at 6 steps, 42.6 at 4 and 5, 42.8 at 3,
    // 43.8 at 8, 44.0 at 10, 44.5 at 12; 33-48 rows alike)
    static constexpr int depth()
    {
        int d = 2;
        for (int t = 3; t <= 6; t++) {
            const bool pair = !FP4 && t % 2 == 0;
            const int w = LB + (t - 2) * (BPW + LB) + (pair ? SS * t / 2 : SS * (t - 1));
            if (w < 64)
                d = t;
        }
        return d;
    }
    static constexpr int D = depth();
    static constexpr bool kPair = !FP4 && D % 2 == 0;
    // loads issued after the last one step u needs: step u + 1's B and
    // scales, then D - 2 steps of (A copies, B, scales); the scale loads of
    // steps u + 1 .. u + D - 1 (the even ones only with pairs)
    static constexpr int kBase = LB + (D - 2) * (BPW + LB);
    static constexpr int kWaitEven = kBase + (kPair ? SS * (D - 2) / 2 : SS * (D - 1));
    static constexpr int kWaitOdd = kBase + (kPair ? SS * D / 2 : SS * (D - 1));
    static constexpr int kSlot = TM * 2048;           // LDS bytes per step
    static_assert(2 * TM % W == 0, "A copies split evenly over the waves");
    static_assert(kWaitOdd < 64 && kWaitEven < 64, "vmcnt range");
};

// ks: the caller's K slices; with gridDim.y == 1 the waves run them in turn
// (one fp32 chain each, summed in slice order in registers) and apply the
// epilogue, else gridDim.y == ks and each workgroup writes its slice's
// partials.
template <int TM, int NG, bool BPS, bool FP4, int F, int W = 4>
__global__ __launch_bounds__(64 * W) void mx_decode_la_kernel(ga_f4gemm_kargs args, int nwg, int ks,
                                                           float* __restrict__ ws,
                                                           const ga_splitk_ws_handle* __restrict__ wsh)
{
    using Cfg = LaCfg<TM, NG, FP4, W>;
    constexpr int kEPB = FP4 ? 2 : 1;
    constexpr int D = Cfg::D, SA = Cfg::SA, BPW = Cfg::BPW, kSlot = Cfg::kSlot;
    constexpr bool kPair = Cfg::kPair;
    __shared__ __attribute__((aligned(1024))) char smem[D * kSlot];
    if (gridDim.y > 1 && wsh && !(ws = resolve_ws(wsh, gridDim.y, args.M, args.N)))
        return; // workspace slot shorter than the split-K layout: write nothing

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int slice = blockIdx.y;
    const int M = (int)args.M, N = (int)args.N, K = (int)args.K;
    const int ngroups = N / 16;
    const int g_end = (int)(((long long)(blockIdx.x + 1) * ngroups) / nwg);
    const int cg0 = (int)(((long long)blockIdx.x * ngroups) / nwg) + wave * NG;
    const int ng_here = min(NG, g_end - cg0); // this wave's groups (<= 0: none)
    const bool live = ng_here > 0;

    int kpt = K;
    if (ks > 1)
        kpt = ((K >> args.log2_k_split) + 255) / 256 * 256;
    const bool seq = gridDim.y == 1; // every slice in this workgroup
    const int kb = seq ? 0 : slice * kpt;
    const int ke = seq ? K : min(K, kb + kpt);
    // the same for every wave of the workgroup: all of them copy A and meet
    // at every step's barrier, with or without columns of their own
    const int nsteps = max(0, (ke - kb) / (128 * kEPB));
    const int kbb = kb / kEPB, Kb = K / kEPB; // bytes

    v4f acc[NG][TM], tot[NG][TM];
#pragma unroll
    for (int c = 0; c < NG; c++)
#pragma unroll
        for (int i = 0; i < TM; i++) {
            acc[c][i] = (v4f){0.f, 0.f, 0.f, 0.f};
            tot[c][i] = (v4f){-0.f, -0.f, -0.f, -0.f}; // -0 + x == x
        }
    // slices in turn: each finished chain is added into tot, in slice order
    const int sps = kpt / (128 * kEPB);
    int fold_at = (seq && ks > 1 && sps < nsteps) ? sps : 0x7FFFFFFF;
    auto fold = [&]() {
#pragma unroll
        for (int c = 0; c < NG; c++)
#pragma unroll
            for (int i = 0; i < TM; i++) {
                tot[c][i] = tot[c][i] + acc[c][i];
                acc[c][i] = (v4f){0.f, 0.f, 0.f, 0.f};
            }
    };
    auto fold_after = [&](int t) {
        if (t + 1 == fold_at) {
            fold();
            fold_at += sps;
            if (fold_at >= nsteps)
                fold_at = 0x7FFFFFFF;
        }
    };

    if (nsteps > 0) {
        const int r = lane & 15, g = lane >> 4;
        const uint32_t lda = args.stride_A0 / kEPB; // bytes
        const long long abytes = (long long)M * lda;
        const auto ra = make_rsrc(args.ptr_A, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
        // A of a step in LDS: rows 16i .. 16i + 15 as 128-byte rows at byte
        // i * 2048 of the slot, K chunk c of row 16i + t at slot
        // c ^ ((t >> 1) & 7). Copy (i, h) writes rows 16i + 8h .. + 7 from
        // whole 128-byte lines (lane l: row 16i + 8h + l / 8, slot l % 8) to
        // LDS byte (2i + h) * 1024 + l * 16.
        const uint32_t crow = (uint32_t)lane >> 3, cslot = lane & 7;
        const uint32_t cva0 = crow * lda + ((cslot ^ ((crow >> 1) & 7)) * 16) + (uint32_t)kbb;
        const uint32_t cva1 = (crow + 8) * lda + ((cslot ^ (((crow + 8) >> 1) & 7)) * 16) +
                              (uint32_t)kbb;
        __amdgpu_buffer_rsrc_t rbuf;
        uint32_t vb, b_step, b_hi, b_grp;
        const int ngb = live ? ng_here : 0;
        if (BPS) {
            const char* pb = (const char*)args.ptr_B + (size_t)(live ? cg0 : 0) * Kb * 16;
            rbuf = make_rsrc(pb, (uint32_t)ngb * (uint32_t)Kb * 16);
            vb = (uint32_t)lane * 16 + (uint32_t)kbb * 16;
            b_step = 2048;
            b_hi = 1024;
            b_grp = (uint32_t)Kb * 16;
        } else {
            const uint32_t ldb = args.stride_B0 / kEPB; // bytes
            const char* pb = (const char*)args.ptr_B + (size_t)(live ? cg0 : 0) * 16 * ldb;
            rbuf = make_rsrc(pb, (uint32_t)ngb * 16 * ldb);
            vb = (uint32_t)r * ldb + g * 16 + (uint32_t)kbb;
            b_step = 128;
            b_hi = 64;
            b_grp = 16 * ldb;
        }
        const uint32_t sna = args.stride_ScaleA0, snb = args.stride_ScaleB0;
        const auto rsa = make_rsrc(args.ptr_ScaleA, (uint32_t)((M + 31) / 32 * 32) * sna);
        const auto rsb = make_rsrc(args.ptr_ScaleB, (uint32_t)((N + 31) / 32 * 32) * snb);
        const uint32_t vsa = ((uint32_t)(kb / 256)) * 256 + lane * 4;
        uint32_t vsb[NG];
#pragma unroll
        for (int c = 0; c < NG; c++)
            vsb[c] = ((uint32_t)((cg0 + c) / 2) * (snb / 8) + (uint32_t)(kb / 256)) * 256 + lane * 4;
        const uint32_t sa_blk = (sna / 8) * 256;

        v8i fb[D][NG];
        uint32_t fsa[D][SA], fsb[D][NG];
        uint32_t osa[TM], osb[NG];

        auto copy_a = [&](int s, int slot) {
#pragma unroll
            for (int e = 0; e < BPW; e++) {
                const int bi = wave * BPW + e, i = bi >> 1, h = bi & 1;
                lds_load16(ra, (lds_void*)(smem + slot * kSlot + bi * 1024),
                           (h ? cva1 : cva0) + uni((uint32_t)s * 128 + (uint32_t)i * 16 * lda), 0);
            }
        };
        auto load_bs = [&](int s, auto J) {
            constexpr int j = decltype(J)::value;
            const uint32_t ob = (uint32_t)s * b_step;
#pragma unroll
            for (int c = 0; c < NG; c++) {
                v4i x0 = buf_load16_stream(rbuf, vb + uni(ob + c * b_grp), 0);
                v4i x1 = buf_load16_stream(rbuf, vb + uni(ob + c * b_grp + b_hi), 0);
                fb[j][c] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            }
            if constexpr (!kPair || j % 2 == 0) {
                const uint32_t q = (uint32_t)(FP4 ? s : (s >> 1)) * 256;
#pragma unroll
                for (int h = 0; h < SA; h++)
                    fsa[j][h] = buf_load4(rsa, vsa + uni(q + h * sa_blk), 0);
#pragma unroll
                for (int c = 0; c < NG; c++)
                    fsb[j][c] = buf_load4(rsb, vsb[c] + uni(q), 0);
            }
        };
        // step in slot j: A operand of rows 16i .. 16i + 15, lane 16g + r
        // reading row 16i + r, chunks g and g + 4 (64 distinct banks per 16
        // lanes)
        v8i fa[TM];
        const uint32_t ao = (uint32_t)r * 128 + ((g ^ ((r >> 1) & 7)) * 16);
        auto read_a = [&](int j) {
            const char* pa = smem + j * kSlot;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const v4i x0 = *(const v4i*)(pa + i * 2048 + ao);
                const v4i x1 = *(const v4i*)(pa + i * 2048 + (ao ^ 64u));
                fa[i] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            }
        };
        auto mma = [&](int s, auto J) {
            constexpr int j = decltype(J)::value;
            constexpr bool odd = kPair && j % 2 == 1;
            const uint32_t sh = FP4 ? 0u : (uint32_t)(s & 1) * 16;
            uint32_t sbv[NG], sav[TM];
#pragma unroll
            for (int c = 0; c < NG; c++)
                sbv[c] = odd ? osb[c] : fsb[j][c] >> (sh + 8 * ((cg0 + c) & 1));
#pragma unroll
            for (int i = 0; i < TM; i++)
                sav[i] = odd ? osa[i] : fsa[j][i >> 1] >> (sh + 8 * (i & 1));
            if constexpr (kPair && j % 2 == 0) {
#pragma unroll
                for (int c = 0; c < NG; c++) {
                    osb[c] = fsb[j][c] >> (16 + 8 * ((cg0 + c) & 1));
                    asm volatile("" : "+v"(osb[c]));
                }
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    osa[i] = fsa[j][i >> 1] >> (16 + 8 * (i & 1));
                    asm volatile("" : "+v"(osa[i]));
                }
            }
#pragma unroll
            for (int c = 0; c < NG; c++)
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    if constexpr (FP4) {
                        acc[c][i] = mfma_mx16_fp4<0, 0>(fb[j][c], fa[i], acc[c][i], (int)sbv[c],
                                                        (int)sav[i]);
                        acc[c][i] = mfma_mx16_fp4<0, 0>(hi16(fb[j][c]), hi16(fa[i]), acc[c][i],
                                                        (int)(sbv[c] >> 16), (int)(sav[i] >> 16));
                    } else {
                        acc[c][i] = mfma_mx16<0, 0, fmt_of_b(F), fmt_of_a(F)>(
                            fb[j][c], fa[i], acc[c][i], (int)sbv[c], (int)sav[i]);
                    }
                }
        };

        // prologue: A of steps 0 .. D-2, B and scales of steps 0 .. D-1, in
        // step order (steps past the slice repeat its last step: every wave
        // issues the same loads, so the counted waits hold)
        static_for<D>([&](auto J) {
            constexpr int j = decltype(J)::value;
            if constexpr (j < D - 1)
                copy_a(min(j, nsteps - 1), j);
            load_bs(min(j, nsteps - 1), J);
            __builtin_amdgcn_sched_barrier(0);
        });
        int s = 0;
        for (; s + D <= nsteps; s += D) {
            static_for<D>([&](auto J) {
                constexpr int j = decltype(J)::value;
                wait_vmcnt<(j % 2 == 0) ? Cfg::kWaitEven : Cfg::kWaitOdd>();
                barrier_lds();
                __builtin_amdgcn_sched_barrier(0);
                read_a(j);
                // the copies stay ahead of this step's B and scale loads (the
                // waits count them in that order)
                copy_a(min(s + j + D - 1, nsteps - 1), (j + D - 1) % D);
                __builtin_amdgcn_sched_barrier(0);
                mma(s + j, J);
                load_bs(min(s + j + D, nsteps - 1), J);
                fold_after(s + j);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
        wait_vmcnt<0>();
        barrier_lds();
        static_for<D>([&](auto J) {
            if ((int)J < nsteps - s) {
                read_a(J);
                mma(s + J, J);
                fold_after(s + J);
            }
        });
    }

    if (gridDim.y > 1) {
        if (live)
            dec_store_partials<NG, TM>(ws, acc, slice, cg0, ng_here, M, N, lane);
        return;
    }
    if (ks > 1) {
        fold(); // the last slice
#pragma unroll
        for (int c = 0; c < NG; c++)
#pragma unroll
            for (int i = 0; i < TM; i++)
                acc[c][i] = tot[c][i];
    }
    if (live)
        dec_epilogue<NG, TM>(args, acc, cg0, ng_here, lane);
}

// Workgroups: one per CU (more when a CU's share needs over MAX_WAVES
// waves), each with ceil(share / NG) column tasks x kp waves per task: one
// (all ks K slices in turn) for 1-16 rows, else one per slice (ks <=
// MAX_WAVES). Measured on MI355X (1-16 rows, three rotated weight sets, each
// split timed after a discarded first run of the shape): one wave per task is
// as fast as the fastest split -- N = 8192, K = 28672, 16 rows: 37.1 us at
// one slice, 37.1-38.3 with one wave per slice at 2-8 slices.
template <int TM, int NG, bool BPS, bool FP4, bool DEEP = false, int F = 0, bool LA = false>
void launch_dec(const ga_f4gemm_kargs& args, int ks, int num_cu, hipStream_t stream)
{
    const int groups = (int)args.N / 16;
    const int kp = TM == 1 ? 1 : ks;
    const int max_tasks = DecCfg<TM, NG, DEEP>::MAX_WAVES / kp; // tasks per workgroup
    int nwg = std::min(num_cu, (groups + NG - 1) / NG);
    nwg = std::max(nwg, (groups + NG * max_tasks - 1) / (NG * max_tasks));
    const int share = (groups + nwg - 1) / nwg;
    const int tasks = (share + NG - 1) / NG;
    hipLaunchKernelGGL((mx_decode_kernel<TM, NG, BPS, FP4, DEEP, 0, F, LA>), dim3(nwg),
                       dim3(64 * tasks * kp), 0, stream, args, nwg, ks, nullptr, nullptr);
}

// Split variant: one wave of NG groups per workgroup per K slice, grid
// (tasks, gdz); partials to ws (or the slot wsh) for the split-K reduce, or
// with one slice the epilogue in the kernel. Steps in flight: as many as the
// 63 outstanding loads a wave can count allow, at most 4.
template <int TM, int NG, bool FP4>
constexpr int xs_depth()
{
    constexpr int nb = NG % 2 == 0 ? NG / 2 : NG;
    constexpr int loads = 2 * NG + 2 * TM + (TM + 1) / 2 + nb;
    return 1 + 63 / loads > 4 ? 4 : 1 + 63 / loads;
}

template <int TM, int NG, bool BPS, bool FP4, int F>
void launch_dec_xs(const ga_f4gemm_kargs& args, int gdz, int phys, float* ws,
                   const ga_splitk_ws_handle* wsh, hipStream_t stream)
{
    const int groups = (int)args.N / 16;
    const int tasks = (groups + NG - 1) / NG;
    hipLaunchKernelGGL((mx_decode_kernel<TM, NG, BPS, FP4, false, xs_depth<TM, NG, FP4>(), F>),
                       dim3(tasks, phys), dim3(64), 0, stream, args, tasks, gdz, ws, wsh);
}

template <int TM, bool BPS, bool FP4, int F>
void launch_dec_xs_ng(const ga_f4gemm_kargs& args, int gdz, int phys, int ng, float* ws,
                      const ga_splitk_ws_handle* wsh, hipStream_t stream)
{
    if (!BPS || F != 0) // row-major B, and E5M2 operands: the two extremes only
        ng = ng <= 2 ? 2 : 8;
    switch (ng) {
    case 2: launch_dec_xs<TM, 2, BPS, FP4, F>(args, gdz, phys, ws, wsh, stream); break;
    case 4: launch_dec_xs<TM, (F ? 8 : 4), BPS, FP4, F>(args, gdz, phys, ws, wsh, stream); break;
    case 5: launch_dec_xs<TM, (F ? 8 : 5), BPS, FP4, F>(args, gdz, phys, ws, wsh, stream); break;
    case 6: launch_dec_xs<TM, (F ? 8 : 6), BPS, FP4, F>(args, gdz, phys, ws, wsh, stream); break;
    case 7: launch_dec_xs<TM, (F ? 8 : 7), BPS, FP4, F>(args, gdz, phys, ws, wsh, stream); break;
    default: launch_dec_xs<TM, 8, BPS, FP4, F>(args, gdz, phys, ws, wsh, stream); break;
    }
}

// Shared-A split variant: nwg workgroups per slice (phys == gdz), or all
// gdz slices in turn in each workgroup (phys == 1). A share of at most 8
// groups runs eight waves of one group each (some without a group), a
// larger one four waves of up to 4. Measured on MI355X, M = 64, N = 28672,
// K = 8192 (7 groups per workgroup), best of 3 x 100 calls: 44.0 us against
// 45.0 us for four waves of 2, 2, 2 and 1 groups (bit-identical outputs).
template <bool BPS, bool FP4, int F>
void launch_dec_la(const ga_f4gemm_kargs& args, int gdz, int phys, int nwg, float* ws,
                   const ga_splitk_ws_handle* wsh, hipStream_t stream)
{
    const int groups = (int)args.N / 16;
    const int share = (groups + nwg - 1) / nwg;
    const dim3 grid(nwg, phys);
    if (share <= 8)
        hipLaunchKernelGGL((mx_decode_la_kernel<4, 1, BPS, FP4, F, 8>), grid, dim3(512), 0, stream,
                           args, nwg, gdz, ws, wsh);
    else
        hipLaunchKernelGGL((mx_decode_la_kernel<4, 4, BPS, FP4, F>), grid, dim3(256), 0, stream,
                           args, nwg, gdz, ws, wsh);
}

bool la_fits(const ga_f4gemm_kargs& args, bool fp4, int num_cu)
{
    const long long steps = (long long)args.K / (fp4 ? 256 : 128);
    const int groups = (int)args.N / 16;
    const int nwg = std::max(1, std::min(num_cu, groups));
    return steps * 2048 <= kLaBytes && (groups + nwg - 1) / nwg >= 4;
}

template <bool BPS, bool FP4, int F>
void launch_dec_rows(const ga_f4gemm_kargs& args, int gdz, int num_cu, hipStream_t stream)
{
    const int tm = ((int)args.M + 15) / 16;
    // 1-16 rows: A rows past M read as zeros without memory traffic, so up to
    // 8 rows a wave per 16-column group (more waves, A bytes still small)
    // streams fastest; 9-16 rows two groups per wave, which halves A's bytes
    // (measured on MI355X, N = 28672, K = 8192: 1-4 rows 36.9-37.1 us
    // against 39.1-39.4; 8 rows 37.7 against 39.5; 16 rows 43.0 against 40.1)
    // 9-16 rows with the A panel (16 x K bytes) within kLaBytes and at least
    // four groups per CU (waves to share its copies): a wave per group too,
    // A read from LDS (la_fits)
    if (tm == 1 && args.M <= 8)
        launch_dec<1, 1, BPS, FP4, false, F>(args, gdz, num_cu, stream);
    else if (tm == 1 && la_fits(args, FP4, num_cu))
        launch_dec<1, 1, BPS, FP4, false, F, true>(args, gdz, num_cu, stream);
    else if (tm == 1)
        launch_dec<1, 2, BPS, FP4, false, F>(args, gdz, num_cu, stream);
    else if (tm == 2) {
        // 17-32 rows: six steps in flight for one two-group task per CU and
        // long K, as for 64 rows below
        const int groups = (int)args.N / 16;
        const int steps = (int)args.K / (FP4 ? 256 : 128) / gdz;
        if (gdz <= 4 && steps >= 64 && groups > num_cu && (groups + 1) / 2 <= num_cu)
            launch_dec<2, 2, BPS, FP4, true, F>(args, gdz, num_cu, stream);
        else
            launch_dec<2, 2, BPS, FP4, false, F>(args, gdz, num_cu, stream);
    }
    else {
        // 33-64 rows (measured on MI355X, MXFP8 / MXFP4 at M = 33 and 64):
        // with at most one 16-column group per CU a wave per group
        // (N = 4096, K = 4096: 12.1 -> 9.6 us MXFP8 at M = 33); with one
        // two-group task per CU and long K, four steps in flight per wave
        // (N = 8192, K = 28672: 67.9 -> 56.3 us MXFP8 at M = 33, 75.4 ->
        // 69.1 at M = 64)
        const int groups = (int)args.N / 16;
        const int steps = (int)args.K / (FP4 ? 256 : 128) / gdz;
        if (groups <= num_cu)
            launch_dec<4, 1, BPS, FP4, false, F>(args, gdz, num_cu, stream);
        else if (gdz <= 4 && steps >= 64 && (groups + 1) / 2 <= num_cu)
            launch_dec<4, 2, BPS, FP4, true, F>(args, gdz, num_cu, stream);
        else
            launch_dec<4, 2, BPS, FP4, false, F>(args, gdz, num_cu, stream);
    }
}

} // namespace

bool mx_decode_applies(const ga_f4gemm_kargs& args, int gdz)
{
    return args.M >= 1 && args.M <= 64 && gdz <= 8;
}

int mx_decode_split_groups(const ga_f4gemm_kargs& args, int gdz, int num_cu, int* phys)
{
    *phys = gdz;
    if (args.M <= 16 || args.M > 64 || gdz > 8 || num_cu <= 0)
        return 0;
    // Workgroups along K (phys) for the caller's gdz K slices, each running
    // consecutive slices as separate fp32 chains (so the output bits are the
    // split's whatever phys is): one when that gives a wave five or more
    // 16-column groups, else enough for eight groups per wave, with at most
    // two slices per workgroup. Measured on MI355X at 64 rows (best of 100
    // calls, one workgroup per slice): N = 28672, K = 8192: 45.0 us with one
    // workgroup along K (shared-A variant), 48.6 us with two; N = 8192,
    // K = 28672: 46.3 us at four (8 groups per wave), 50.2 at two, 50.9 at
    // eight.
    const long long groups = args.N / 16;
    int p = 1;
    if (groups < 5LL * num_cu)
        p = std::min(gdz, std::max((gdz + 1) / 2, (int)((8LL * num_cu + groups - 1) / groups)));
    // waves (tasks x workgroups along K) in whole rounds of one per CU, as
    // few rounds as eight groups per wave allow, the groups spread evenly
    // over them (N = 28672, one along K: 7 groups, 256 waves; N = 8192, four:
    // 8)
    const long long work = groups * p;
    const long long rounds = (work + 8LL * num_cu - 1) / (8LL * num_cu);
    int ng = (int)((work + rounds * num_cu - 1) / (rounds * num_cu));
    ng = ng < 2 ? 2 : (ng == 3 ? 4 : ng);
    // one slice at fewer than five groups per wave: the in-workgroup kernel
    // (it needs no partials either)
    if (p == 1 && ng < 5)
        return 0;
    *phys = p;
    return ng;
}

namespace {

// Workgroups per slice of the shared-A variant: one per CU over all slices
// (no more than the groups), at most 16 groups (4 per wave of four) each.
int la_workgroups(const ga_f4gemm_kargs& args, int gdz, int num_cu)
{
    const int groups = (int)args.N / 16;
    int nwg = std::max(1, num_cu / gdz);
    nwg = std::min(nwg, groups);
    return std::max(nwg, (groups + 15) / 16);
}

// 33-64 rows at one slice: the shared-A variant (measured on MI355X, M = 64,
// N = 28672, K = 8192: 45.5 us against 50-54 us for the split variant at one
// or two slices; M = 40: 44.2 against 48.1). With more slices the split
// variant stays (M = 64, N = 8192, K = 28672 at 4 slices: 47.6 us, shared-A
// 51.0: the fp32 partials and the reduce cost the same, the shared-A kernel
// streams ~7 % slower there).
// phys == 1 at 33-64 rows: the shared-A variant. The split variant with
// phys == 1 runs at most 32 rows (its 64-row waves have no registers for the
// running sum of the slices).
template <bool BPS, bool FP4, int F>
void launch_split_t(const ga_f4gemm_kargs& args, int gdz, int phys, int ng, float* ws,
                    const ga_splitk_ws_handle* wsh, int num_cu, hipStream_t stream)
{
    if (args.M > 32 && phys == 1 && num_cu > 0)
        launch_dec_la<BPS, FP4, F>(args, gdz, 1, la_workgroups(args, 1, num_cu), ws, wsh, stream);

    else if (args.M > 32)
        launch_dec_xs_ng<4, BPS, FP4, F>(args, gdz, phys, ng, ws, wsh, stream);
    else
        launch_dec_xs_ng<2, BPS, FP4, F>(args, gdz, phys, ng, ws, wsh, stream);
}

template <bool FP4, int F>
void launch_both(const ga_f4gemm_kargs& args, int gdz, int phys, int ng, bool bps, float* ws,
                 const ga_splitk_ws_handle* wsh, int num_cu, hipStream_t stream)
{
    if (ng > 0)
        bps ? launch_split_t<true, FP4, F>(args, gdz, phys, ng, ws, wsh, num_cu, stream)
            : launch_split_t<false, FP4, F>(args, gdz, phys, ng, ws, wsh, num_cu, stream);
    else
        bps ? launch_dec_rows<true, FP4, F>(args, gdz, num_cu, stream)
            : launch_dec_rows<false, FP4, F>(args, gdz, num_cu, stream);
}

// ng > 0: the split variant (ws / wsh when phys > 1), else the in-workgroup
// kernel.
void launch_any(const ga_f4gemm_kargs& args, int gdz, int phys, int ng, bool bps, bool fp4,
                int fmt, float* ws, const ga_splitk_ws_handle* wsh, int num_cu,
                hipStream_t stream)
{
    if (fp4) {
        launch_both<true, 0>(args, gdz, phys, ng, bps, ws, wsh, num_cu, stream);
        return;
    }
    switch (fmt) {
    case 1: launch_both<false, 1>(args, gdz, phys, ng, bps, ws, wsh, num_cu, stream); break;
    case 2: launch_both<false, 2>(args, gdz, phys, ng, bps, ws, wsh, num_cu, stream); break;
    case 3: launch_both<false, 3>(args, gdz, phys, ng, bps, ws, wsh, num_cu, stream); break;
    default: launch_both<false, 0>(args, gdz, phys, ng, bps, ws, wsh, num_cu, stream); break;
    }
}

} // namespace

void launch_mx_decode_split(const ga_f4gemm_kargs& args, int gdz, int phys, int ng, bool bps,
                            bool fp4, int fmt, float* ws, const ga_splitk_ws_handle* wsh,
                            int num_cu, hipStream_t stream)
{
    launch_any(args, gdz, phys, ng, bps, fp4, fmt, ws, wsh, num_cu, stream);
}

void launch_mx_decode(const ga_f4gemm_kargs& args, int gdz, bool bps, bool fp4, int fmt,
                      int num_cu, hipStream_t stream)
{
    launch_any(args, gdz, gdz, 0, bps, fp4, fmt, nullptr, nullptr, num_cu, stream);
}

} // namespace ga

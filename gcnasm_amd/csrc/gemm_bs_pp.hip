// gemm_bs_pp.hip -- 256x256 FP8 GEMM with fp32 scales behind the
// opus_gemm_kargs ABI: DeepSeek block scale (1x128 activations, 128x128 or
// 1x128 weights) and per-tensor scale, fp32 or bf16 C, batched.
//
//   block-scale: C[b,m,n] = sum_g P_g[m,n] * SFA[g, m] * SFB(g, n),
//                acc = fmaf(P_g, SFA*SFB, acc) per 128-K group g in K order
//   per-tensor:  C = (sfa[0] * sfb[0]) * sum_k A*B, one fp32 chain
//
// The structure is the MXFP8 256x256 kernel's (gemm_mx_pp.hip, ga_pp.hpp):
// eight waves in two groups one barrier apart, K step 128 in four phases of
// one 128x128 quadrant, A and B row-major in swizzled LDS rows, two K-step
// slots refilled half tile by half tile. Differences:
//  * the MFMA runs with unit E8M0 scales into a zeroed temporary (8 tiles x
//    4 VGPRs); the fp32 scaling of quadrant k is folded into its accumulator
//    before the next MFMA slot reuses the temporaries: s = SFA[m] * SFB
//    (GROUP_N 1: per column), then four fmaf per tile and lane. GROUP_N 1
//    folds every tile in the next MFMA slot, just before the MFMA that
//    reuses it; GROUP_N 128 splits the fold: the t = 0 tiles there, the
//    t = 1 tiles in the memory slot between the two MFMA slots, after its
//    operand reads (the VALU work of a fold placed in the MFMA slot adds to
//    that slot; half of it in each slot shortens the longer one);
//  * per K group the scales travel with the operands: SFA[g, m0..m0+255]
//    (1 KB, copied by waves 0-3, permuted so a lane's four rows are one
//    16-byte LDS read) and SFB (waves 4-7: the tile's two 128-column blocks,
//    or its 256 columns for GROUP_N 1) into a ring of four 2 KB slots;
//  * per-tensor: the MFMA accumulates across K and the epilogue applies
//    sfa[0] * sfb[0].
#include "ga_bs_pp.hpp"
#include "ga_internal.hpp"

namespace ga {
namespace {

using namespace pp;
using namespace bspp;

template <int MODE, int OUT, bool NT>
__global__ __attribute__((amdgpu_flat_work_group_size(kNT, kNT), amdgpu_waves_per_eu(2, 2)))
void bs_pp_kernel(ga_opus_gemm_kargs ka)
{
    __shared__ __attribute__((aligned(1024))) char smem[kLdsBs];
    constexpr int S = MODE == PS_TENSOR ? 0 : 1; // scale copies per wave per K group

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2, simd = wave & 3;
    const int M = ka.m, N = ka.n, K = ka.k;
    int tile_m, tile_n;
    map_tile(blockIdx.x, blockIdx.y, gridDim.x, gridDim.y, kBsGroupM, tile_m, tile_n);
    const int m0 = tile_m * 256, n0 = tile_n * 256;
    const int b = blockIdx.z;
    const int nsteps = K / 128;

    v4f acc[4][4][2];
    v4f p[4][2]; // MFMA results of the last quadrant, folded before the next MFMA slot reuses them
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int t = 0; t < 2; t++)
                acc[q][i][t] = (v4f){0.f, 0.f, 0.f, 0.f};

    BsLoad L;
    {
        int crow, ckc;
        copy_lane(wave, lane, crow, ckc);
        const char* pa = (const char*)ka.ptr_a + (size_t)b * ka.stride_a_batch +
                         (size_t)m0 * ka.stride_a;
        const char* pb = (const char*)ka.ptr_b + (size_t)b * ka.stride_b_batch +
                         (size_t)n0 * ka.stride_b;
        const long long abytes = (long long)(M - m0) * ka.stride_a;
        const long long bbytes = (long long)(N - n0) * ka.stride_b;
        L.ra = make_rsrc(pa, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
        L.rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
        L.va = (uint32_t)crow * ka.stride_a + ckc * 16;
        L.vb = (uint32_t)crow * ka.stride_b + ckc * 16;
        L.a_hstep = 64 * (uint32_t)ka.stride_a;
        L.b_hstep = 64 * (uint32_t)ka.stride_b;
        L.vs = 0;
        L.s_kstep = 0;
        if constexpr (MODE != PS_TENSOR) {
            const int ngroups = K / 128;
            if (wave < 4) {
                // SFA [K/128, M]: LDS position w*64 + l holds row
                // w*64 + (l%4)*16 + l/4 (rows past M clamp to M-1)
                const float* sfa = (const float*)ka.ptr_sfa + (size_t)b * ka.stride_sfa_batch;
                L.rs = make_rsrc(sfa, (uint32_t)ngroups * ka.stride_sfa * 4);
                const int row = min(m0 + wave * 64 + (lane & 3) * 16 + (lane >> 2), M - 1);
                L.vs = (uint32_t)row * 4;
                L.s_kstep = (uint32_t)ka.stride_sfa * 4;
            } else {
                const float* sfb = (const float*)ka.ptr_sfb + (size_t)b * ka.stride_sfb_batch;
                const int pos = (wave - 4) * 64 + lane;
                if (MODE == PS_GROUP128) {
                    // SFB [ceil(N/128), K/128]: positions 0 and 1 hold the
                    // tile's two 128-column blocks
                    const int nblk = (N + 127) / 128;
                    L.rs = make_rsrc(sfb, (uint32_t)nblk * ka.stride_sfb * 4);
                    const int nb = min(n0 / 128 + (pos & 1), nblk - 1);
                    L.vs = (uint32_t)nb * ka.stride_sfb * 4;
                    L.s_kstep = 4;
                } else {
                    // SFB [K/128, N]: position c holds column n0 + c
                    L.rs = make_rsrc(sfb, (uint32_t)ngroups * ka.stride_sfb * 4);
                    const int col = min(n0 + pos, N - 1);
                    L.vs = (uint32_t)col * 4;
                    L.s_kstep = (uint32_t)ka.stride_sfb * 4;
                }
            }
        }
    }

    BsRead rb;
    {
        uint32_t o, o64;
        operand_lane(lane, o, o64);
        rb.a0 = smem + grp * 64 * 128 + o;
        rb.a1 = smem + grp * 64 * 128 + o64;
        rb.b0 = smem + kBRegion + simd * 32 * 128 + o;
        rb.b1 = smem + kBRegion + simd * 32 * 128 + o64;
        rb.sa = smem + kSBase + grp * 256 + (lane & 15) * 16;
        rb.sb = smem + kSBase + 1024 +
                (MODE == PS_GROUP1 ? (simd * 32 + (lane >> 4) * 4) * 4 : 0);
    }

    v8i fa[4], fb0[2], fb1[2];

    // Prologue: copies in steady-state order (B0+S, A0, B1, A1 of group 0;
    // B0+S, A0, B1 of group 1), then the B0 read of the phase before step 0.
    issue_b(L, smem, 0, 0, wave);
    if (S)
        issue_s(L, smem, 0, 0, wave);
    issue_a(L, smem, 0, 0, wave);
    issue_b(L, smem, 1, 0, wave);
    issue_a(L, smem, 1, 0, wave);
    issue_b(L, smem, 0, 1, wave);
    if (S)
        issue_s(L, smem, 1, 1, wave);
    issue_a(L, smem, 0, 1, wave);
    issue_b(L, smem, 1, 1, wave);
    phase_sync<12 + S>(); // B0 (+ scales) of group 0
    read_b<0>(rb, 0, fb0);
    phase_sync<10 + S>(); // A0 of group 0
    if (grp == 1)
        slot_sync(); // second group runs one barrier behind

    // K group s (LDS slot s & 1, scale ring slot r0). A memory slot issues
    // its copy, reads scales, then its operand read, then waits:
    //   phase  read      copy            quadrant   younger copies
    //   1      A0(s)     A1(s+1)         00         10 + S
    //   2      B1(s)     B0+S(s+2)       01         10 + 2S
    //   3      A1(s)     A0(s+2)         10         10 + S
    //   4      B0(s+1)   B1(s+2)         11         10 + S
    // The loop's first quadrant has nothing to fold in: peel it.
    // Scale ring slot of group s: s % 4. The copy of group s+2 (phase 2 of
    // group s) overwrites group s-2's slot, last read for the fold in phase 1
    // of group s-1 (unsplit fold) or in phase 4 of group s-2 (split).
    ScaleVals sv;
    if constexpr (MODE == PS_GROUP128) {
        // Split fold: each memory slot reads the scales of the quadrant the
        // coming MFMA slot computes and folds the t = 1 tiles of the quadrant
        // the previous MFMA slot computed after its operand reads; the MFMA
        // slot folds the t = 0 tiles between its MFMAs. Phase 1 reads group
        // s's scales, which landed before A0(s) (copied after them), and the
        // last read of a ring slot (phase 4 of its group) precedes its
        // overwrite (phase 2 of the group two later). Same fmaf per tile and
        // group, in the same order, as the unsplit fold.
        ScaleVals svn = {};
        sv = svn;
        // two K groups per iteration: the LDS slot is a compile-time read
        // offset instead of a VALU add per read base
        auto group = [&](int s, auto SLOT) {
            constexpr int slot = decltype(SLOT)::value;
            const int r0 = s & 3, r2 = (s + 2) & 3;
            // phase 1 (folds in quadrant 11 of the previous group)
            BS_MEM_SLOT_SPLIT(0, 0, r0, issue_a(L, smem, 1, s + 1, wave),
                              read_a<0>(rb, slot, fa), 10 + S, acc[3], s > 0);
            if (s > 0)
                mma_quadrant<MODE, true, true>(acc[0], p, fa, fb0, acc[3], sv);
            else
                mma_quadrant<MODE, false, true>(acc[0], p, fa, fb0, acc[3], sv);
            slot_sync();
            // phase 2
            BS_MEM_SLOT_SPLIT(0, 1, r0,
                              issue_b(L, smem, 0, s + 2, wave);
                              issue_s(L, smem, s + 2, r2, wave), read_b<1>(rb, slot, fb1),
                              10 + 2 * S, acc[0], true);
            mma_quadrant<MODE, true, true>(acc[1], p, fa, fb1, acc[0], sv);
            slot_sync();
            // phase 3
            BS_MEM_SLOT_SPLIT(1, 0, r0, issue_a(L, smem, 0, s + 2, wave),
                              read_a<1>(rb, slot, fa), 10 + S, acc[1], true);
            mma_quadrant<MODE, true, true>(acc[2], p, fa, fb0, acc[1], sv);
            slot_sync();
            // phase 4
            BS_MEM_SLOT_SPLIT(1, 1, r0, issue_b(L, smem, 1, s + 2, wave),
                              read_b<0>(rb, slot ^ 1, fb0), 10 + S, acc[2], true);
            mma_quadrant<MODE, true, true>(acc[3], p, fa, fb1, acc[2], sv);
            slot_sync();
        };
        int s = 0;
        for (; s + 1 < nsteps; s += 2) {
            group(s, std::integral_constant<int, 0>{});
            group(s + 1, std::integral_constant<int, 1>{});
        }
        if (s < nsteps)
            group(s, std::integral_constant<int, 0>{});
        if (grp == 0)
            slot_sync(); // matches the second group's extra barrier
        apply_scales<MODE>(svn, acc[3], p);
    } else {
        auto group = [&](int s, auto SLOT) {
            constexpr int slot = decltype(SLOT)::value;
            const int r0 = s & 3, r2 = (s + 2) & 3, rprev = (s - 1) & 3;
            // phase 1 (folds in quadrant 11 of the previous group)
            BS_MEM_SLOT(1, 1, rprev, issue_a(L, smem, 1, s + 1, wave), read_a<0>(rb, slot, fa),
                        10 + S);
            if (s > 0)
                mma_quadrant<MODE, true>(acc[0], p, fa, fb0, acc[3], sv);
            else
                mma_quadrant<MODE, false>(acc[0], p, fa, fb0, acc[3], sv);
            slot_sync();
            // phase 2
            BS_MEM_SLOT(0, 0, r0,
                        issue_b(L, smem, 0, s + 2, wave); if (S) issue_s(L, smem, s + 2, r2, wave),
                        read_b<1>(rb, slot, fb1), 10 + 2 * S);
            mma_quadrant<MODE, true>(acc[1], p, fa, fb1, acc[0], sv);
            slot_sync();
            // phase 3
            BS_MEM_SLOT(0, 1, r0, issue_a(L, smem, 0, s + 2, wave), read_a<1>(rb, slot, fa),
                        10 + S);
            mma_quadrant<MODE, true>(acc[2], p, fa, fb0, acc[1], sv);
            slot_sync();
            // phase 4
            BS_MEM_SLOT(1, 0, r0, issue_b(L, smem, 1, s + 2, wave), read_b<0>(rb, slot ^ 1, fb0),
                        10 + S);
            mma_quadrant<MODE, true>(acc[3], p, fa, fb1, acc[2], sv);
            slot_sync();
        };
        int s = 0;
        for (; s + 1 < nsteps; s += 2) {
            group(s, std::integral_constant<int, 0>{});
            group(s + 1, std::integral_constant<int, 1>{});
        }
        if (s < nsteps)
            group(s, std::integral_constant<int, 0>{});
        if (grp == 0)
            slot_sync(); // matches the second group's extra barrier
        const ScaleVals last = read_scales<MODE, 1, 1>(rb, (nsteps - 1) & 3);
        apply_scales<MODE>(last, acc[3], p);
    }
    wait_vmcnt<0>(); // copies past K land before exit

    // Epilogue: lane holds C[m][n .. n+3] of each 16x16 tile.
    float tscale = 1.0f;
    if constexpr (MODE == PS_TENSOR)
        tscale = ((const float*)ka.ptr_sfa)[0] * ((const float*)ka.ptr_sfb)[0];
    char* pc = (char*)ka.ptr_c + (size_t)b * ka.stride_c_batch * (OUT == GA_DTYPE_F32 ? 4 : 2);
    // Whole interior tiles go through LDS so that the global stores write
    // whole rows (1 KB fp32 or 512 B bf16 per instruction instead of 16 rows
    // x 64 or 32 B): bf16 in one pass, fp32 in two passes of 128 rows.
    const int ldc = ka.stride_c;
    const bool staged = m0 + 256 <= M && n0 + 256 <= N && ((uintptr_t)pc & 15) == 0 &&
                        (ldc & (OUT == GA_DTYPE_F32 ? 3 : 7)) == 0;
    if (staged) {
        barrier_lds(); // every wave's operand and scale reads are done
        if constexpr (OUT == GA_DTYPE_F32) {
            static_assert(128 * kStagePitchF32 <= kLdsBs, "fp32 staging fits in LDS");
#pragma unroll
            for (int h = 0; h < 2; h++) {
                if (h)
                    barrier_lds(); // rows of pass 0 read before pass 1 overwrites them
#pragma unroll
                for (int qq = 0; qq < 2; qq++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int t = 0; t < 2; t++) {
                            const v4f v = acc[2 * h + qq][i][t] * tscale;
                            const int row = grp * 64 + i * 16 + (lane & 15);
                            const int col = qq * 128 + simd * 32 + t * 16 + (lane >> 4) * 4;
                            *(v4f*)(smem + row * kStagePitchF32 + col * 4) = v;
                        }
                barrier_lds();
                float* dst = (float*)pc + (size_t)(m0 + h * 128) * ldc + n0;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = wave * 16 + r;
                    const v4i d = *(const v4i*)(smem + row * kStagePitchF32 + lane * 16);
                    v4i* o = (v4i*)(dst + (size_t)row * ldc + lane * 4);
                    if constexpr (NT)
                        __builtin_nontemporal_store(d, o);
                    else
                        *o = d;
                }
            }
        } else {
            static_assert(kStageBytes <= kLdsBs, "bf16 staging fits in LDS");
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const v4f v = acc[q][i][t] * tscale;
                        const uint32_t lo = (uint32_t)f32_to_bf16(v[0]) |
                                            ((uint32_t)f32_to_bf16(v[1]) << 16);
                        const uint32_t hi = (uint32_t)f32_to_bf16(v[2]) |
                                            ((uint32_t)f32_to_bf16(v[3]) << 16);
                        stage_put(smem, (q >> 1) * 128 + grp * 64 + i * 16 + (lane & 15),
                                  (q & 1) * 128 + simd * 32 + t * 16 + (lane >> 4) * 4, lo, hi);
                    }
            barrier_lds();
            stage_store<NT>(smem, (uint16_t*)pc + (size_t)m0 * ldc + n0, ldc, wave, lane);
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + (q >> 1) * 128 + grp * 64 + i * 16 + (lane & 15);
            if (m >= M)
                continue;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int n = n0 + (q & 1) * 128 + simd * 32 + t * 16 + (lane >> 4) * 4;
                if (n >= N)
                    continue;
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    v[j] = MODE == PS_TENSOR ? acc[q][i][t][j] * tscale : acc[q][i][t][j];
                const size_t off = (size_t)m * ka.stride_c + n;
                const bool full = n + 4 <= N && (ka.stride_c & 3) == 0;
                if constexpr (OUT == GA_DTYPE_F32) {
                    float* o = (float*)pc + off;
                    if (full)
                        *(v4f*)o = (v4f){v[0], v[1], v[2], v[3]};
                    else
                        for (int j = 0; j < 4 && n + j < N; j++)
                            o[j] = v[j];
                } else {
                    uint16_t* o = (uint16_t*)pc + off;
                    if (full) {
                        uint2 pk;
                        pk.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
                        pk.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
                        *(uint2*)o = pk;
                    } else {
                        for (int j = 0; j < 4 && n + j < N; j++)
                            o[j] = f32_to_bf16(v[j]);
                    }
                }
            }
        }
    }
}

// Interior tiles store C with non-temporal stores when C, A and B together
// exceed 320 MiB, more than the 256 MB memory-side cache holds (measured on
// MI355X, block scale GROUP_N 128, best of 3 x 100 calls, plain -> non-
// temporal: fp32 C 16384x16384x2048 672 -> 605 us, 4096x24576x1536 208 ->
// 191, 8192^3 473 -> 465, 4096x16384x4096 273 -> 271; below the limit they
// cost 1-3 %: 8192x8192x2048 158 -> 161, 4096x8192x4096 138 -> 140,
// 4096x7168x2048 73 -> 75, 4096^3 69 -> 71).
bool bs_pp_nontemporal(const ga_opus_gemm_kargs& ka, int out_dtype)
{
    const long long c = (long long)ka.m * ka.n * (out_dtype == GA_DTYPE_F32 ? 4 : 2);
    const long long ab = (long long)(ka.m + ka.n) * ka.k;
    return (c + ab) * ka.batch > (320ll << 20);
}

template <int MODE, int OUT>
void launch_bs_pp_t(const ga_opus_gemm_kargs& ka, hipStream_t stream)
{
    const int tn = (ka.n + 255) / 256, tm = (ka.m + 255) / 256;
    if (bs_pp_nontemporal(ka, OUT))
        hipLaunchKernelGGL((bs_pp_kernel<MODE, OUT, true>), dim3(tn, tm, ka.batch), dim3(kNT), 0,
                           stream, ka);
    else
        hipLaunchKernelGGL((bs_pp_kernel<MODE, OUT, false>), dim3(tn, tm, ka.batch), dim3(kNT), 0,
                           stream, ka);
}

} // namespace

void launch_bs_pp(const ga_opus_gemm_kargs& ka, int mode, int out_dtype, hipStream_t stream)
{
    const bool f32 = out_dtype == GA_DTYPE_F32;
    if (mode == PS_GROUP128)
        f32 ? launch_bs_pp_t<PS_GROUP128, GA_DTYPE_F32>(ka, stream)
            : launch_bs_pp_t<PS_GROUP128, GA_DTYPE_BF16>(ka, stream);
    else if (mode == PS_GROUP1)
        f32 ? launch_bs_pp_t<PS_GROUP1, GA_DTYPE_F32>(ka, stream)
            : launch_bs_pp_t<PS_GROUP1, GA_DTYPE_BF16>(ka, stream);
    else
        f32 ? launch_bs_pp_t<PS_TENSOR, GA_DTYPE_F32>(ka, stream)
            : launch_bs_pp_t<PS_TENSOR, GA_DTYPE_BF16>(ka, stream);
}

} // namespace ga

// gemm_bs_decode.hip -- fp32-scaled FP8 GEMMs (DeepSeek block scale and
// per-tensor, opus_gemm_kargs ABI) for up to 64 rows: an HBM stream over B.
//
// Same results as the tile kernels up to the K split: per 128-K group g the
// MFMA (unit E8M0 scales) gives P_g, folded as acc = fmaf(P_g, SFA*SFB, acc)
// with the scale product rounded first (scale_c_tile, opus_gemm_dist/
// opus_gemm_mem_gemm_a2a/include/opus_gemm_utils.cuh:76-96); per-tensor
// accumulates in the MFMA and scales once. K is cut into `ks` slices of whole
// groups whose chains are summed in slice order.
//
// Design (the MXFP8 decode kernel's, gemm_mx_decode.hip, for row-major B):
//  * one wave per NG 16-column groups of B and one K slice; the wave's B
//    rows and its <= 64 A rows go straight from memory into MFMA operand
//    registers (lane 16g + r: row r, 16-byte K chunks g and g + 4), with a
//    ring of D steps of loads in flight;
//  * the scales of a step travel with it: SFA for the lane's rows, SFB for
//    the group's 128-column block (GROUP_N 128) or its 4 columns (GROUP_N 1);
//  * the K slices of a column group are waves of one workgroup and are summed
//    in LDS in slice order; workgroups take equal shares of the column groups;
//  * columns past N and rows past M read as zero (range-checked buffers),
//    scale indices are clamped, stores are masked.
#include "ga_device.hpp"
#include "ga_internal.hpp"

#include <algorithm>

namespace ga {
namespace {

enum { BD_GROUP128 = 0, BD_GROUP1 = 1, BD_TENSOR = 2 };

// Steps of loads in flight per wave: fewer for more rows (registers), and
// within the 6-bit vmcnt.
template <int TM, int NG, int MODE>
struct BdDepth {
    static constexpr int kLoads = 2 * NG + 2 * TM + (MODE == 2 ? 0 : TM + NG);
    static constexpr int D0 = TM == 1 ? 6 : (TM == 2 ? 4 : 2);
    static constexpr int D = D0 < 63 / kLoads + 1 ? D0 : 63 / kLoads + 1;
};

__device__ __forceinline__ uint32_t bd_uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

template <int TM, int NG, int MODE, int OUT>
__global__ __attribute__((amdgpu_flat_work_group_size(64, 512)))
void bs_decode_kernel(ga_opus_gemm_kargs ka, int nwg, int ks, int gps)
{
    constexpr int D = BdDepth<TM, NG, MODE>::D;
    constexpr int SAL = MODE == BD_TENSOR ? 0 : TM; // SFA loads per step
    constexpr int SBL = MODE == BD_TENSOR ? 0 : NG; // SFB loads per step
    constexpr int kLoadsPerStep = 2 * NG + 2 * TM + SAL + SBL;
    static_assert(kLoadsPerStep * (D - 1) < 64, "vmcnt range");
    __shared__ __attribute__((aligned(16))) float red[8 * NG * TM * 256];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slice = wave % ks, tl = wave / ks;
    const int M = ka.m, N = ka.n, K = ka.k;
    const int b = blockIdx.y;
    const int ngroups = (N + 15) / 16;
    const int g_end = (int)(((long long)(blockIdx.x + 1) * ngroups) / nwg);
    const int cg0 = (int)(((long long)blockIdx.x * ngroups) / nwg) + tl * NG;
    const int ng_here = min(NG, g_end - cg0);
    const bool live = ng_here > 0;
    const int G = K / 128;
    const int gb = slice * gps;
    const int ge = min(G, gb + gps);
    const int nsteps = live ? max(0, ge - gb) : 0;
    const int r = lane & 15, g = lane >> 4;

    v4f acc[NG][TM];
#pragma unroll
    for (int c = 0; c < NG; c++)
#pragma unroll
        for (int i = 0; i < TM; i++)
            acc[c][i] = (v4f){0.f, 0.f, 0.f, 0.f};

    if (nsteps > 0) {
        const uint32_t lda = (uint32_t)ka.stride_a, ldb = (uint32_t)ka.stride_b;
        const char* pa = (const char*)ka.ptr_a + (size_t)b * ka.stride_a_batch;
        const long long abytes = (long long)M * lda;
        const auto ra = make_rsrc(pa, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
        const uint32_t va = (uint32_t)r * lda + g * 16 + (uint32_t)gb * 128;
        const char* pb = (const char*)ka.ptr_b + (size_t)b * ka.stride_b_batch +
                         (size_t)cg0 * 16 * ldb;
        const long long brows = min(ng_here * 16, N - cg0 * 16);
        const auto rb = make_rsrc(pb, (uint32_t)min(brows * ldb, 0xFFFFFFF0ll));
        const uint32_t vb = (uint32_t)r * ldb + g * 16 + (uint32_t)gb * 128;

        // scales (fp32): SFA [K/128, M]; SFB [ceil(N/128), K/128] or [K/128, N]
        __amdgpu_buffer_rsrc_t rsa = ra, rsb = rb;
        uint32_t vsa[TM], vsb[NG], sa_step = 0, sb_step = 0;
        if constexpr (MODE != BD_TENSOR) {
            const float* sfa = (const float*)ka.ptr_sfa + (size_t)b * ka.stride_sfa_batch;
            const float* sfb = (const float*)ka.ptr_sfb + (size_t)b * ka.stride_sfb_batch;
            rsa = make_rsrc(sfa, (uint32_t)G * ka.stride_sfa * 4);
            sa_step = (uint32_t)ka.stride_sfa * 4;
#pragma unroll
            for (int i = 0; i < TM; i++)
                vsa[i] = ((uint32_t)gb * ka.stride_sfa + min(i * 16 + r, M - 1)) * 4;
            if constexpr (MODE == BD_GROUP128) {
                const int nblk = (N + 127) / 128;
                rsb = make_rsrc(sfb, (uint32_t)nblk * ka.stride_sfb * 4);
                sb_step = 4;
#pragma unroll
                for (int c = 0; c < NG; c++)
                    vsb[c] = ((uint32_t)min(((cg0 + c) * 16) / 128, nblk - 1) * ka.stride_sfb +
                              gb) * 4;
            } else {
                rsb = make_rsrc(sfb, (uint32_t)G * ka.stride_sfb * 4);
                sb_step = (uint32_t)ka.stride_sfb * 4;
                // this lane's 4 columns; a group straddling N reads past the
                // row (bytes of the next row or range-checked zeros), and
                // those columns are never stored
#pragma unroll
                for (int c = 0; c < NG; c++)
                    vsb[c] = ((uint32_t)gb * ka.stride_sfb + (cg0 + c) * 16 + g * 4) * 4;
            }
        }

        v8i fb[D][NG];
        v8i fa[D][TM];
        float fsa[D][TM];
        v4f fsb[D][NG];

        auto load = [&](int s, auto J) {
            constexpr int j = decltype(J)::value;
            const uint32_t ok = (uint32_t)s * 128;
#pragma unroll
            for (int c = 0; c < NG; c++) {
                const uint32_t oc = ok + (uint32_t)c * 16 * ldb;
                v4i x0 = buf_load16_stream(rb, vb + bd_uni(oc), 0);
                v4i x1 = buf_load16_stream(rb, vb + bd_uni(oc + 64), 0);
                fb[j][c] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint32_t oa = ok + (uint32_t)i * 16 * lda;
                v4i y0 = buf_load16(ra, va + bd_uni(oa), 0);
                v4i y1 = buf_load16(ra, va + bd_uni(oa + 64), 0);
                fa[j][i] = (v8i){y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
            }
            if constexpr (MODE != BD_TENSOR) {
#pragma unroll
                for (int i = 0; i < TM; i++)
                    fsa[j][i] = __uint_as_float(buf_load4(rsa, vsa[i] + bd_uni((uint32_t)s * sa_step), 0));
#pragma unroll
                for (int c = 0; c < NG; c++) {
                    if constexpr (MODE == BD_GROUP128)
                        fsb[j][c][0] = __uint_as_float(
                            buf_load4(rsb, vsb[c] + bd_uni((uint32_t)s * sb_step), 0));
                    else
                        fsb[j][c] = __builtin_bit_cast(
                            v4f, buf_load16(rsb, vsb[c] + bd_uni((uint32_t)s * sb_step), 0));
                }
            }
        };
        auto mma = [&](auto J) {
            constexpr int j = decltype(J)::value;
#pragma unroll
            for (int c = 0; c < NG; c++)
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    if constexpr (MODE == BD_TENSOR) {
                        acc[c][i] = mfma_mx16<0, 0>(fb[j][c], fa[j][i], acc[c][i], 127, 127);
                    } else {
                        const v4f p =
                            mfma_mx16<0, 0>(fb[j][c], fa[j][i], (v4f){0.f, 0.f, 0.f, 0.f}, 127, 127);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float sc = MODE == BD_GROUP128 ? fsa[j][i] * fsb[j][c][0]
                                                                 : fsa[j][i] * fsb[j][c][e];
                            acc[c][i][e] = __builtin_fmaf(p[e], sc, acc[c][i][e]);
                        }
                    }
                }
        };

        // the loads of each step stay in issue order (slot 0 oldest): the
        // wait before step s+J's MFMAs lets the D-1 younger steps fly
        static_for<D>([&](auto J) {
            load(min((int)J, nsteps - 1), J);
            __builtin_amdgcn_sched_barrier(0);
        });
        int s = 0;
        for (; s + D <= nsteps; s += D) {
            static_for<D>([&](auto J) {
                wait_vmcnt<kLoadsPerStep * (D - 1)>();
                mma(J);
                load(min(s + D + (int)J, nsteps - 1), J);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
        wait_vmcnt<0>();
        static_for<D>([&](auto J) {
            if ((int)J < nsteps - s)
                mma(J);
        });
    }

    // K slices of a column group summed in slice order
    if (ks > 1) {
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
                    const v4f u = *(const v4f*)(mine + ((z * NG + c) * TM + i) * 256 + lane * 4);
                    t = (v4f){t[0] + u[0], t[1] + u[1], t[2] + u[2], t[3] + u[3]};
                }
                acc[c][i] = t;
            }
    }
    if (!live)
        return;

    // lane holds C[m][n .. n+3], m = 16i + lane%16, n = 16cg + 4(lane/16)
    float tscale = 1.0f;
    if constexpr (MODE == BD_TENSOR)
        tscale = ((const float*)ka.ptr_sfa)[0] * ((const float*)ka.ptr_sfb)[0];
    char* pc = (char*)ka.ptr_c + (size_t)b * ka.stride_c_batch * (OUT == GA_DTYPE_F32 ? 4 : 2);
#pragma unroll
    for (int c = 0; c < NG; c++) {
        if (c >= ng_here)
            continue;
        const int n = (cg0 + c) * 16 + g * 4;
        if (n >= N)
            continue;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int m = i * 16 + r;
            if (m >= M)
                continue;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                v[e] = MODE == BD_TENSOR ? acc[c][i][e] * tscale : acc[c][i][e];
            const size_t off = (size_t)m * ka.stride_c + n;
            const bool full = n + 4 <= N && (ka.stride_c & 3) == 0;
            if constexpr (OUT == GA_DTYPE_F32) {
                float* o = (float*)pc + off;
                if (full)
                    *(v4f*)o = (v4f){v[0], v[1], v[2], v[3]};
                else
                    for (int e = 0; e < 4 && n + e < N; e++)
                        o[e] = v[e];
            } else {
                uint16_t* o = (uint16_t*)pc + off;
                if (full) {
                    uint2 pk;
                    pk.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
                    pk.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
                    *(uint2*)o = pk;
                } else {
                    for (int e = 0; e < 4 && n + e < N; e++)
                        o[e] = f32_to_bf16(v[e]);
                }
            }
        }
    }
}

// K slices: double while the waves stay within about four per CU and each
// slice keeps at least two 128-K groups (at most 8 slices); workgroups take
// equal shares of the column groups, at most 8 waves each.
int bsd_ks(int n, int k, int ng, int num_cu)
{
    const int groups = (n + 15) / 16;
    const int G = k / 128;
    const int tasks_total = (groups + ng - 1) / ng;
    int ks = 1;
    while (ks < 8 && (long long)tasks_total * ks * 2 <= 4ll * num_cu && G / (ks * 2) >= 2)
        ks *= 2;
    return ks;
}

// one 16-column group per wave when there are fewer groups than CUs, so the
// grid still reaches every CU; else two (A loads shared by two groups)
int bsd_ng(int n, int num_cu) { return (n + 15) / 16 < num_cu ? 1 : 2; }

template <int TM, int NG, int MODE, int OUT>
ga_status launch_bsd(const ga_opus_gemm_kargs& ka, int num_cu, hipStream_t stream)
{
    const int groups = (ka.n + 15) / 16;
    const int G = ka.k / 128;
    const int tasks_total = (groups + NG - 1) / NG;
    const int ks = bsd_ks(ka.n, ka.k, NG, num_cu);
    const int gps = (G + ks - 1) / ks;
    const int max_tasks = 8 / ks;
    int nwg = std::min(num_cu, tasks_total);
    nwg = std::max(nwg, (groups + NG * max_tasks - 1) / (NG * max_tasks));
    const int share = (groups + nwg - 1) / nwg;
    const int tasks = (share + NG - 1) / NG;
    hipLaunchKernelGGL((bs_decode_kernel<TM, NG, MODE, OUT>), dim3(nwg, ka.batch),
                       dim3(64 * tasks * ks), 0, stream, ka, nwg, ks, gps);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

template <int MODE, int OUT>
ga_status launch_bsd_rows(const ga_opus_gemm_kargs& ka, int num_cu, hipStream_t stream)
{
    const int tm = (ka.m + 15) / 16;
    const bool few = bsd_ng(ka.n, num_cu) == 1;
    if (tm == 1)
        return few ? launch_bsd<1, 1, MODE, OUT>(ka, num_cu, stream)
                   : launch_bsd<1, 2, MODE, OUT>(ka, num_cu, stream);
    if (tm == 2)
        return few ? launch_bsd<2, 1, MODE, OUT>(ka, num_cu, stream)
                   : launch_bsd<2, 2, MODE, OUT>(ka, num_cu, stream);
    return few ? launch_bsd<4, 1, MODE, OUT>(ka, num_cu, stream)
               : launch_bsd<4, 2, MODE, OUT>(ka, num_cu, stream);
}

} // namespace

int bs_decode_groups_per_slice(const ga_opus_gemm_kargs& ka, int num_cu)
{
    const int G = ka.k / 128;
    const int ks = bsd_ks(ka.n, ka.k, bsd_ng(ka.n, num_cu), num_cu);
    return (G + ks - 1) / ks;
}

ga_status launch_bs_decode(const ga_opus_gemm_kargs& ka, int mode, int out_dtype,
                           hipStream_t stream)
{
    int num_cu = 0;
    ga_status st = device_cu_count(&num_cu);
    if (st != GA_OK)
        return st;
    const bool f32 = out_dtype == GA_DTYPE_F32;
    if (mode == BD_GROUP128)
        return f32 ? launch_bsd_rows<BD_GROUP128, GA_DTYPE_F32>(ka, num_cu, stream)
                   : launch_bsd_rows<BD_GROUP128, GA_DTYPE_BF16>(ka, num_cu, stream);
    if (mode == BD_GROUP1)
        return f32 ? launch_bsd_rows<BD_GROUP1, GA_DTYPE_F32>(ka, num_cu, stream)
                   : launch_bsd_rows<BD_GROUP1, GA_DTYPE_BF16>(ka, num_cu, stream);
    return f32 ? launch_bsd_rows<BD_TENSOR, GA_DTYPE_F32>(ka, num_cu, stream)
               : launch_bsd_rows<BD_TENSOR, GA_DTYPE_BF16>(ka, num_cu, stream);
}

} // namespace ga

// gemm_bs.hip -- FP8 GEMMs with fp32 scales behind the opus_gemm_kargs ABI.
//
//   block-scale (DeepSeek):  C[b,m,n] = sum_g P_g[m,n] * SFA[g, m] * SFB(g, n)
//       P_g = sum over the 128-wide K group g of A*B (fp32 from the MFMA)
//       SFB(g, n) = SFB[n/128, g] (GROUP_N 128) or SFB[g, n] (GROUP_N 1)
//       acc = fmaf(P_g, SFA*SFB, acc) per group, in K order
//       (opus_gemm/block_scale_gemm/README.md:7-26, scale_c_tile in
//        opus_gemm_dist/opus_gemm_mem_gemm_a2a/include/opus_gemm_utils.cuh:76-96)
//   per-tensor (fp8_gemm):  C = (sfa[0] * sfb[0]) * sum_k A*B, one fp32 chain
//
// A [batch, M, K] and B [batch, N, K] are row-major E4M3 (B is K-major, not
// preshuffled), K % 128 == 0, M and N arbitrary (rows past M/N load as zero
// through the buffer range check; a partial last N group of 128 is fine).
// C is fp32 (the reference's output type) or bf16.
//
// 33-64 rows with enough columns, or more rows whose 128x128 tiles fit on
// the CUs in one round (this file): 4 waves, 64x256 or 128x128 tile, K step
// 128, three LDS stages, A and B
// staged with buffer_load ... lds (8 whole 128-byte rows per instruction)
// into swizzled LDS rows (chunk c of row r at slot c ^ ((r >> 1) & 7)),
// v_mfma_scale_f32_16x16x128_f8f6f4 with unit E8M0 scales (127) and the
// operands swapped so a lane owns 4 consecutive N of one C row. More rows go
// to the 256x256 eight-wave kernel of gemm_bs_pp.hip, fewer rows (or too
// few 256-column tiles) to the
// B-streaming kernel of gemm_bs_decode.hip.
#include "ga_device.hpp"
#include "ga_internal.hpp"
#include "ga_pp.hpp"

namespace ga {

enum BsMode { BS_GROUP128 = 0, BS_GROUP1 = 1, BS_TENSOR = 2 };

template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int MODE_, int OUT_>
struct BsCfg {
    static constexpr int BM = BM_, BN = BN_;
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int MODE = MODE_, OUT = OUT_;
    static constexpr int NT = 256;
    static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    static constexpr int TM = WTM / 16, TN = WTN / 16;
    static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int NS = 3; // LDS stages: two in flight while one is computed
    static constexpr int LDS = NS * STAGE;
    static constexpr int A_LOADS = A_BYTES / (NT * 16);
    static constexpr int B_LOADS = B_BYTES / (NT * 16);
    static constexpr int SB_PER_TILE = MODE == BS_GROUP1 ? 4 : 1;
    static_assert(WAVES_M * WAVES_N == 4, "4 waves");
    static_assert(A_BYTES % (NT * 16) == 0 && B_BYTES % (NT * 16) == 0, "tile >= 32 rows");
    static_assert(LDS <= 160 * 1024, "LDS budget");
};

constexpr int kBsGroupM = 4;

__device__ __forceinline__ void bs_map_tile(int lin, int gdx, int gdy, int& tm, int& tn)
{
    const int total = gdx * gdy;
    const int full = (total / 8) * 8;
    if (lin < full)
        lin = (lin % 8) * (total / 8) + lin / 8;
    const int per_group = kBsGroupM * gdx;
    const int g = lin / per_group;
    const int first_m = g * kBsGroupM;
    const int gsize = min(gdy - first_m, kBsGroupM);
    const int r = lin - g * per_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

template <class C>
struct BsScales {
    float sa[C::TM];
    float sb[C::TN][C::SB_PER_TILE];
};

template <class C>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void bs_gemm_kernel(ga_opus_gemm_kargs ka, int tiles_n)
{
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    const int M = ka.m, N = ka.n, K = ka.k;
    const int tiles_m = (M + C::BM - 1) / C::BM;
    int tile_m, tile_n;
    bs_map_tile(blockIdx.x, tiles_n, tiles_m, tile_m, tile_n);
    const int m0 = tile_m * C::BM, n0 = tile_n * C::BN;
    const int b = blockIdx.z;

    const char* pa = (const char*)ka.ptr_a + (size_t)b * ka.stride_a_batch + (size_t)m0 * ka.stride_a;
    const char* pb = (const char*)ka.ptr_b + (size_t)b * ka.stride_b_batch + (size_t)n0 * ka.stride_b;
    const long long abytes = (long long)(M - m0) * ka.stride_a;
    const long long bbytes = (long long)(N - n0) * ka.stride_b;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(pa, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
    // copy i covers rows 32i .. 32i+31 (wave w: 8 whole 128-byte rows) of the
    // swizzled LDS image
    uint32_t voff_a[C::A_LOADS], voff_b[C::B_LOADS];
    int row0, chunk;
    pp::copy_lane(wave, lane, row0, chunk);
#pragma unroll
    for (int i = 0; i < C::A_LOADS; i++)
        voff_a[i] = (uint32_t)(i * 32 + row0) * ka.stride_a + chunk * 16;
#pragma unroll
    for (int i = 0; i < C::B_LOADS; i++)
        voff_b[i] = (uint32_t)(i * 32 + row0) * ka.stride_b + chunk * 16;

    // Scale pointers for this lane's C rows / columns.
    const float* sfa = (const float*)ka.ptr_sfa + (size_t)b * ka.stride_sfa_batch;
    const float* sfb = (const float*)ka.ptr_sfb + (size_t)b * ka.stride_sfb_batch;
    int mrow[C::TM], ncol[C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
        mrow[i] = min(m0 + wm * C::WTM + i * 16 + (lane & 15), M - 1);
#pragma unroll
    for (int t = 0; t < C::TN; t++)
        ncol[t] = n0 + wn * C::WTN + t * 16 + (lane >> 4) * 4;

    auto issue = [&](int buf, int kk) {
        char* la = smem + buf * C::STAGE;
        char* lb = la + C::A_BYTES;
#pragma unroll
        for (int i = 0; i < C::A_LOADS; i++)
            lds_load16(ra, (lds_void*)(la + (i * 256 + wave * 64) * 16), voff_a[i] + kk, 0);
#pragma unroll
        for (int i = 0; i < C::B_LOADS; i++)
            lds_load16(rb, (lds_void*)(lb + (i * 256 + wave * 64) * 16), voff_b[i] + kk, 0);
    };
    auto load_scales = [&](int g, BsScales<C>& s) {
        if constexpr (C::MODE != BS_TENSOR) {
#pragma unroll
            for (int i = 0; i < C::TM; i++)
                s.sa[i] = sfa[(size_t)g * ka.stride_sfa + mrow[i]];
#pragma unroll
            for (int t = 0; t < C::TN; t++) {
                if constexpr (C::MODE == BS_GROUP128) {
                    int n = min(ncol[t], N - 1);
                    s.sb[t][0] = sfb[(size_t)(n / 128) * ka.stride_sfb + g];
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        s.sb[t][j] = sfb[(size_t)g * ka.stride_sfb + min(ncol[t] + j, N - 1)];
                }
            }
        }
    };

    v4f acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int t = 0; t < C::TN; t++)
            acc[i][t] = (v4f){0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf, const BsScales<C>& s) {
        const char* la = smem + buf * C::STAGE;
        const char* lb = la + C::A_BYTES;
        uint32_t o0, o1;
        pp::operand_lane(lane, o0, o1);
        v8i bf[C::TN];
#pragma unroll
        for (int t = 0; t < C::TN; t++) {
            const char* g = lb + (wn * C::TN + t) * 2048;
            v4i x0 = *(const v4i*)(g + o0);
            v4i x1 = *(const v4i*)(g + o1);
            bf[t] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        }
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const char* g = la + (wm * C::TM + i) * 2048;
            v4i x0 = *(const v4i*)(g + o0);
            v4i x1 = *(const v4i*)(g + o1);
            v8i af = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
            for (int t = 0; t < C::TN; t++) {
                if constexpr (C::MODE == BS_TENSOR) {
                    acc[i][t] = mfma_mx16<0, 0>(bf[t], af, acc[i][t], 127, 127);
                } else {
                    v4f p = mfma_mx16<0, 0>(bf[t], af, (v4f){0.f, 0.f, 0.f, 0.f}, 127, 127);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float sbv = C::MODE == BS_GROUP128 ? s.sb[t][0] : s.sb[t][j];
                        float sc = s.sa[i] * sbv;
                        acc[i][t][j] = __builtin_fmaf(p[j], sc, acc[i][t][j]);
                    }
                }
            }
        }
    };

    // K loop over three LDS stages. Step s waits for its copies and scales
    // (counted vmcnt: only the copies of step s+1 are younger), then, after
    // the barrier that frees the buffer step s-1 used, loads the scales of
    // step s+1 and copies step s+2 (in that order, so the next wait leaves
    // exactly one step of copies in flight), then computes step s. Two scale
    // sets alternate (the loop is unrolled by two). Copies past the last
    // group read in-bounds bytes that are never used or range-checked zeros;
    // the scale group index is clamped to the last group.
    const int nsteps = K / 128;
    constexpr int TL = C::A_LOADS + C::B_LOADS;
    BsScales<C> sc0, sc1;
    issue(0, 0);
    load_scales(0, sc0);
    __builtin_amdgcn_sched_barrier(0);
    issue(1, 128);
    int buf = 0; // LDS buffer of step s
    auto step = [&](int s, const BsScales<C>& cur, BsScales<C>& nxt) {
        wait_vmcnt<TL>();
        barrier_lds();
        load_scales(min(s + 1, nsteps - 1), nxt);
        __builtin_amdgcn_sched_barrier(0);
        issue(buf == 0 ? 2 : buf - 1, (s + 2) * 128);
        __builtin_amdgcn_sched_barrier(0);
        compute(buf, cur);
        __builtin_amdgcn_sched_barrier(0);
        buf = buf == 2 ? 0 : buf + 1;
    };
    int s = 0;
    for (; s + 1 < nsteps; s += 2) {
        step(s, sc0, sc1);
        step(s + 1, sc1, sc0);
    }
    if (s < nsteps)
        step(s, sc0, sc1);
    wait_vmcnt<0>(); // copies past the last group land before exit

    float tscale = 1.0f;
    if constexpr (C::MODE == BS_TENSOR)
        tscale = ((const float*)ka.ptr_sfa)[0] * ((const float*)ka.ptr_sfb)[0];

    char* pc = (char*)ka.ptr_c + (size_t)b * ka.stride_c_batch * (C::OUT == GA_DTYPE_F32 ? 4 : 2);
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        const int m = m0 + wm * C::WTM + i * 16 + (lane & 15);
        if (m >= M)
            continue;
#pragma unroll
        for (int t = 0; t < C::TN; t++) {
            const int n = ncol[t];
            if (n >= N)
                continue;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                v[j] = C::MODE == BS_TENSOR ? acc[i][t][j] * tscale : acc[i][t][j];
            const size_t off = (size_t)m * ka.stride_c + n;
            const bool full = n + 4 <= N && (ka.stride_c & 3) == 0;
            if constexpr (C::OUT == GA_DTYPE_F32) {
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

template <class C>
static ga_status launch_bs(const ga_opus_gemm_kargs& ka, hipStream_t stream)
{
    const int tn = (ka.n + C::BN - 1) / C::BN, tm = (ka.m + C::BM - 1) / C::BM;
    hipLaunchKernelGGL(bs_gemm_kernel<C>, dim3(tn * tm, 1, ka.batch), dim3(256), 0, stream, ka, tn);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

// Which kernel dispatch_bs runs for these kargs on a device with num_cu CUs.
enum BsPath { BS_PATH_TILE128, BS_PATH_PP, BS_PATH_TILE64, BS_PATH_DECODE };
static BsPath bs_path(const ga_opus_gemm_kargs& ka, int num_cu)
{
    // More than 64 rows: the 256x256 eight-wave kernel (gemm_bs_pp.hip), or
    // this file's 128x128 tile when its tiles fit on the CUs in one round
    // (measured on MI355X, fp32 C: 512x7168x2048 35.4 -> 18.8 us,
    // 512x2112x7168 86.1 -> 43.7 us, 1024x4096x4096 54.9 -> 29.7 us; with a
    // second round, e.g. 768x7168x2048, the eight-wave kernel is faster).
    if (ka.m > 64) {
        const long long t128 =
            (long long)((ka.m + 127) / 128) * ((ka.n + 127) / 128) * ka.batch;
        return t128 <= num_cu ? BS_PATH_TILE128 : BS_PATH_PP;
    }
    // Up to 64 rows: the B-streaming kernel (gemm_bs_decode.hip), unless
    // 33-64 rows leave this file's 64x256 tile enough workgroups (a quarter
    // of the CUs): then its A reuse across 256 columns wins.
    const long long tiles = (long long)((ka.n + 255) / 256) * ka.batch;
    if (ka.m > 32 && tiles * 4 >= num_cu)
        return BS_PATH_TILE64;
    return BS_PATH_DECODE;
}

template <int MODE, int OUT>
static ga_status dispatch_bs(const ga_opus_gemm_kargs& ka, hipStream_t stream)
{
    int num_cu = 0;
    ga_status st = device_cu_count(&num_cu);
    if (st != GA_OK)
        return st;
    switch (bs_path(ka, num_cu)) {
    case BS_PATH_TILE128:
        return launch_bs<BsCfg<128, 128, 2, 2, MODE, OUT>>(ka, stream);
    case BS_PATH_PP:
        launch_bs_pp(ka, MODE, OUT, stream);
        GA_HIP_CHECK(hipGetLastError());
        return GA_OK;
    case BS_PATH_TILE64:
        return launch_bs<BsCfg<64, 256, 1, 4, MODE, OUT>>(ka, stream);
    default:
        return launch_bs_decode(ka, MODE, OUT, stream);
    }
}

static ga_status check_kargs(const ga_opus_gemm_kargs* ka)
{
    if (!ka || !ka->ptr_a || !ka->ptr_b || !ka->ptr_c || !ka->ptr_sfa || !ka->ptr_sfb)
        return fail(GA_ERR_ARG, "opus kargs: null pointer");
    if (ka->m <= 0 || ka->n <= 0 || ka->k <= 0 || ka->batch <= 0)
        return fail(GA_ERR_ARG, "Invalid problem size: M, N, K and batch must be positive.");
    if (ka->k % 128 != 0)
        return fail(GA_ERR_GROUP, "K must be a multiple of GROUP_K (128), got %d", ka->k);
    if (ka->stride_a < ka->k || ka->stride_b < ka->k || ka->stride_a % 16 || ka->stride_b % 16)
        return fail(GA_ERR_SHAPE, "stride_a/stride_b must be >= K and multiples of 16");
    if (ka->stride_c < ka->n)
        return fail(GA_ERR_SHAPE, "stride_c must be >= N");
    if (ka->batch > 65535)
        return fail(GA_ERR_SHAPE, "batch > 65535");
    // operands are read through buffer descriptors based at a tile's first
    // row, which address 4 GiB: 256 rows of A and B must fit in it
    const unsigned long long lim = 0xFFFFFFF0ull;
    if (256ull * (unsigned long long)ka->stride_a > lim ||
        256ull * (unsigned long long)ka->stride_b > lim)
        return fail(GA_ERR_SHAPE, "stride_a/stride_b too large for 32-bit buffer offsets "
                                  "(256 rows must fit in 4 GiB)");
    return GA_OK;
}

// The fp32 scale matrices are read through one descriptor each.
static ga_status check_scales(const ga_opus_gemm_kargs* ka, int group_n)
{
    const unsigned long long lim = 0xFFFFFFF0ull, G = (unsigned long long)ka->k / 128;
    const unsigned long long sfa = G * (unsigned long long)ka->stride_sfa * 4;
    const unsigned long long sfb = (group_n == 128 ? ((unsigned long long)ka->n + 127) / 128 : G) *
                                   (unsigned long long)ka->stride_sfb * 4;
    if (sfa > lim || sfb > lim)
        return fail(GA_ERR_SHAPE, "scale matrices larger than 4 GiB");
    return GA_OK;
}

static ga_status check_blockscale(const ga_opus_gemm_kargs* kargs, int group_n, int out_dtype)
{
    ga_status st = check_kargs(kargs);
    if (st != GA_OK)
        return st;
    if (group_n != 128 && group_n != 1)
        return fail(GA_ERR_ARG, "group_n must be 128 or 1");
    if (out_dtype != GA_DTYPE_F32 && out_dtype != GA_DTYPE_BF16)
        return fail(GA_ERR_ARG, "out_dtype must be GA_DTYPE_F32 or GA_DTYPE_BF16");
    if (group_n == 128 && kargs->stride_sfb < kargs->k / 128)
        return fail(GA_ERR_SHAPE, "stride_sfb must be >= K/128 for GROUP_N 128");
    if (group_n == 1 && kargs->stride_sfb < kargs->n)
        return fail(GA_ERR_SHAPE, "stride_sfb must be >= N for GROUP_N 1");
    if (kargs->stride_sfa < kargs->m)
        return fail(GA_ERR_SHAPE, "stride_sfa must be >= M (SFA is [K/128, M])");
    return check_scales(kargs, group_n);
}

// Workgroups of the stream-K form for these kargs on this device (0: the
// call runs whole tiles).
static ga_status bs_stream_k_plan(const ga_opus_gemm_kargs& ka, int* nwg)
{
    int num_cu = 0;
    ga_status st = device_cu_count(&num_cu);
    if (st != GA_OK)
        return st;
    *nwg = bs_path(ka, num_cu) == BS_PATH_PP ? bs_sk_workgroups(ka, num_cu) : 0;
    return GA_OK;
}

} // namespace ga

using namespace ga;

extern "C" {

ga_status ga_gemm_a8w8_blockscale(const ga_opus_gemm_kargs* kargs, int group_n, int out_dtype,
                                  void* stream)
{
    ga_status st = check_blockscale(kargs, group_n, out_dtype);
    if (st != GA_OK)
        return st;
    hipStream_t s = (hipStream_t)stream;
    if (group_n == 128)
        return out_dtype == GA_DTYPE_F32 ? dispatch_bs<BS_GROUP128, GA_DTYPE_F32>(*kargs, s)
                                         : dispatch_bs<BS_GROUP128, GA_DTYPE_BF16>(*kargs, s);
    return out_dtype == GA_DTYPE_F32 ? dispatch_bs<BS_GROUP1, GA_DTYPE_F32>(*kargs, s)
                                     : dispatch_bs<BS_GROUP1, GA_DTYPE_BF16>(*kargs, s);
}

ga_status ga_blockscale_stream_k(const ga_opus_gemm_kargs* kargs, int* workgroups)
{
    if (!kargs || !workgroups)
        return fail(GA_ERR_ARG, "ga_blockscale_stream_k: null argument");
    if (kargs->m <= 0 || kargs->n <= 0 || kargs->k <= 0 || kargs->batch <= 0 ||
        kargs->k % 128 != 0)
        return fail(GA_ERR_SHAPE, "ga_blockscale_stream_k: M, N, K, batch > 0, K %% 128 == 0");
    return bs_stream_k_plan(*kargs, workgroups);
}

ga_status ga_blockscale_workspace_bytes(const ga_opus_gemm_kargs* kargs, size_t* bytes)
{
    if (!bytes)
        return fail(GA_ERR_ARG, "ga_blockscale_workspace_bytes: null argument");
    int nwg = 0;
    ga_status st = ga_blockscale_stream_k(kargs, &nwg);
    if (st != GA_OK)
        return st;
    *bytes = bs_sk_workspace_bytes(*kargs, nwg);
    return GA_OK;
}

ga_status ga_gemm_a8w8_blockscale_ws(const ga_opus_gemm_kargs* kargs, int group_n, int out_dtype,
                                     void* workspace, size_t workspace_bytes, void* stream)
{
    ga_status st = check_blockscale(kargs, group_n, out_dtype);
    if (st != GA_OK)
        return st;
    int nwg = 0;
    st = bs_stream_k_plan(*kargs, &nwg);
    if (st != GA_OK)
        return st;
    if (nwg > 0 && workspace) {
        const size_t need = bs_sk_workspace_bytes(*kargs, nwg);
        if (workspace_bytes < need)
            return fail(GA_ERR_WORKSPACE, "blockscale workspace holds %zu bytes, need %zu",
                        workspace_bytes, need);
        launch_bs_pp_sk(*kargs, group_n == 128 ? BS_GROUP128 : BS_GROUP1, out_dtype, nwg,
                        workspace, (hipStream_t)stream);
        GA_HIP_CHECK(hipGetLastError());
        return GA_OK;
    }
    return ga_gemm_a8w8_blockscale(kargs, group_n, out_dtype, stream);
}

ga_status ga_blockscale_workspace_check(const ga_opus_gemm_kargs* kargs, void* workspace,
                                       size_t workspace_bytes, void* stream)
{
    if (!kargs)
        return fail(GA_ERR_ARG, "blockscale_workspace_check: null kargs");
    int nwg = 0;
    ga_status st = bs_stream_k_plan(*kargs, &nwg);
    if (st != GA_OK || nwg == 0 || !workspace)
        return st;
    const size_t counters = bs_sk_counter_bytes(*kargs);
    if (workspace_bytes < counters)
        return fail(GA_ERR_WORKSPACE, "blockscale workspace holds %zu bytes, need %zu",
                    workspace_bytes, counters);
    hipStream_t s = (hipStream_t)stream;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    GA_HIP_CHECK(hipStreamIsCapturing(s, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(GA_ERR_ARG, "blockscale_workspace_check synchronises: not under capture");
    const size_t tiles = (size_t)((kargs->n + 255) / 256) * ((kargs->m + 255) / 256);
    unsigned misuse = 0;
    GA_HIP_CHECK(hipStreamSynchronize(s));
    GA_HIP_CHECK(hipMemcpy(&misuse, (const char*)workspace + tiles * 4, 4, hipMemcpyDeviceToHost));
    if (misuse == 0)
        return GA_OK;
    // cleared on the caller's stream and waited for: a hipMemset would queue
    // on the null stream, which does not order against a non-blocking stream
    GA_HIP_CHECK(hipMemsetAsync(workspace, 0, counters, s));
    GA_HIP_CHECK(hipStreamSynchronize(s));
    return fail(GA_ERR_WORKSPACE, "blockscale stream-K workspace was not zero-filled before a "
                                  "call (its tile counters did not start at zero, so some tiles "
                                  "of that call were not summed); counters cleared");
}

ga_status ga_blockscale_k_slices(const ga_opus_gemm_kargs* kargs, int* groups_per_slice)
{
    if (!kargs || !groups_per_slice)
        return fail(GA_ERR_ARG, "ga_blockscale_k_slices: null argument");
    if (kargs->m <= 0 || kargs->n <= 0 || kargs->k <= 0 || kargs->batch <= 0 ||
        kargs->k % 128 != 0)
        return fail(GA_ERR_SHAPE, "ga_blockscale_k_slices: M, N, K, batch > 0, K %% 128 == 0");
    int num_cu = 0;
    ga_status st = device_cu_count(&num_cu);
    if (st != GA_OK)
        return st;
    *groups_per_slice = bs_path(*kargs, num_cu) == BS_PATH_DECODE
                            ? bs_decode_groups_per_slice(*kargs, num_cu)
                            : kargs->k / 128;
    return GA_OK;
}

ga_status ga_fp8_gemm_per_tensor(const ga_opus_gemm_kargs* kargs, int out_dtype, void* stream)
{
    ga_status st = check_kargs(kargs);
    if (st != GA_OK)
        return st;
    if (out_dtype != GA_DTYPE_F32 && out_dtype != GA_DTYPE_BF16)
        return fail(GA_ERR_ARG, "out_dtype must be GA_DTYPE_F32 or GA_DTYPE_BF16");
    hipStream_t s = (hipStream_t)stream;
    return out_dtype == GA_DTYPE_F32 ? dispatch_bs<BS_TENSOR, GA_DTYPE_F32>(*kargs, s)
                                     : dispatch_bs<BS_TENSOR, GA_DTYPE_BF16>(*kargs, s);
}

} // extern "C"

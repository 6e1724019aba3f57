// gemm_a16w16.hip -- bf16 split-K GEMM whose fp32 workspace is found through
// a device-resident handle, the one-call GEMM + reduce, and the management of
// the handle's slot.
//
//   ws[s, b, m, n] = sum over k in slice s of A[b, m, k] * B[b, n, k]   (fp32)
//   C[b, m, n]     = bf16(sum_s ws[s, b, m, n] (+ bias[n]))             (reduce)
//
// Reference: gemm_a16w16_flatmm_splitk_kernel (opus_gemm_dist/
// opus_gemm_mem_gemm_a2a/include/gfx950/opus_gemm_pipeline_a16w16_flatmm_
// splitk_gfx950.cuh:204-563), launched with the reduce by main.cc:299-318;
// kargs and handle opus_gemm_traits_a16w16_gfx950.cuh:588-634.
//
// Kernel design (gfx950, 256 threads = 4 waves in a 2 x 2 grid, tiles from
// 64x64 to 128x256):
//  * K step of 64 bf16 = 128 bytes per row, kept in LDS as the 256x256 FP8
//    kernels keep theirs: 128-byte rows with 16-byte K chunk c of row r at
//    slot c ^ ((r >> 1) & 7), so a direct-to-LDS copy instruction fetches 8
//    whole rows (full 128-byte lines) and the operand reads are free of bank
//    conflicts; rows past M fall outside the buffer range and read as zero.
//  * v_mfma_f32_16x16x32_bf16: lane 16g+r takes row r, K [8g, 8g+8), which is
//    chunk g of the row (K [0, 32)); chunk g + 4 feeds the second MFMA
//    (K [32, 64)).
//  * Operands swapped (B rows on the MFMA's A side), so a lane ends with 4
//    consecutive N outputs of one C row -> 16-byte fp32 stores.
//  * The fragments of K step s+1 are read from LDS while the MFMAs of step s
//    run (two register sets): with one wave per SIMD nothing else would hide
//    the LDS read latency of every step.
//  * Slices follow the reference's partition (pipeline .cuh:234-247): K in
//    128-element iterations, ceil(iters / split_k) per slice, the last slice
//    takes what is left; a slice left empty writes zeros. Chunks at or past
//    the slice end are loaded from an offset outside the buffer (zeros), so
//    a K tail and the prefetches past the slice read nothing.
//  * The workspace pointer and its capacity are read from the handle at
//    kernel entry; a capacity smaller than the layout needs makes the kernel
//    write nothing.
//  * Workgroup ids: XCD round-robin undone (each XCD gets a contiguous range),
//    slice outermost, then M-grouped tiles, so the workgroups of one XCD
//    share A and B panels of the same K range in its L2.
#include "ga_device.hpp"
#include "ga_internal.hpp"
#include "ga_pp.hpp"

#include <mutex>
#include <unordered_map>

namespace ga {

static_assert(sizeof(ga_splitk_ws_handle) == 16, "opus_splitk_ws_handle is 16 bytes");
static_assert(sizeof(ga_flatmm_splitk_kargs) == 96, "flatmm split-K kargs are 96 bytes");

template <int BM_, int BN_, int NS_>
struct A16Cfg {
    static constexpr int BM = BM_, BN = BN_, NS = NS_;
    static constexpr int WTM = BM / 2, WTN = BN / 2;
    static constexpr int TM = WTM / 16, TN = WTN / 16;
    static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int LDS = NS * STAGE;
    static constexpr int A_LOADS = A_BYTES / (256 * 16), B_LOADS = B_BYTES / (256 * 16);
    static constexpr int TILE_LOADS = A_LOADS + B_LOADS;
    static_assert(BM % 32 == 0 && BN % 32 == 0, "tile multiple of 32 rows");
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(NS >= 3 && TILE_LOADS * (NS - 2) < 64, "vmcnt range");
};

struct A16Args {
    ga_flatmm_splitk_kargs ka;
    int tiles_m, tiles_n;
    int kslice; // K elements per slice, a multiple of 128
};

constexpr int kA16GroupM = 4;

// Epilogues: fp32 partials to the workspace (the reference's split-K kernel)
// or, for split_k == 1, bf16 C (+ bias) directly.
enum { EPI_WS = 0, EPI_C = 1 };

template <class C>
struct A16State {
    __amdgpu_buffer_rsrc_t ra, rb;
    uint32_t voff_a[C::A_LOADS];
    uint32_t voff_b[C::B_LOADS];
    int kchunk; // first K element of this lane's 16-byte chunk within a step
};

// Copies K step `step` of the slice into stage `buf`: chunks at or past `ke`
// load from offset 0xFFFFFFF0, outside every buffer range (zeros).
template <class C>
__device__ __forceinline__ void a16_issue(const A16State<C>& st, char* smem, int buf, int step,
                                          int kb, int ke, int wave)
{
    char* sa = smem + buf * C::STAGE;
    char* sb = sa + C::A_BYTES;
    const int kstep = kb + step * 64;
    const bool ok = kstep + st.kchunk < ke;
    const uint32_t kbytes = (uint32_t)kstep * 2;
#pragma unroll
    for (int i = 0; i < C::A_LOADS; i++)
        lds_load16(st.ra, (lds_void*)(sa + (i * 256 + wave * 64) * 16),
                   ok ? st.voff_a[i] + kbytes : 0xFFFFFFF0u, 0);
#pragma unroll
    for (int i = 0; i < C::B_LOADS; i++)
        lds_load16(st.rb, (lds_void*)(sb + (i * 256 + wave * 64) * 16),
                   ok ? st.voff_b[i] + kbytes : 0xFFFFFFF0u, 0);
}

// Operand fragments of one K step: [K half][tile].
template <class C>
struct A16Frag {
    v4i a[2][C::TM], b[2][C::TN];
};

template <class C>
__device__ __forceinline__ void a16_read(const char* smem, int buf, int wm, int wn, int lane,
                                         A16Frag<C>& f)
{
    const char* la = smem + buf * C::STAGE;
    const char* lb = la + C::A_BYTES;
    uint32_t o0, o1;
    pp::operand_lane(lane, o0, o1);
#pragma unroll
    for (int t = 0; t < C::TN; t++) {
        const char* g = lb + (wn * C::TN + t) * 2048;
        f.b[0][t] = *(const v4i*)(g + o0);
        f.b[1][t] = *(const v4i*)(g + o1);
    }
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        const char* g = la + (wm * C::TM + i) * 2048;
        f.a[0][i] = *(const v4i*)(g + o0);
        f.a[1][i] = *(const v4i*)(g + o1);
    }
}

// K [0, 32) over every accumulator, then K [32, 64): no back-to-back
// dependent MFMAs
template <class C>
__device__ __forceinline__ void a16_mma(const A16Frag<C>& f, v4f (&acc)[C::TM][C::TN])
{
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int t = 0; t < C::TN; t++)
                acc[i][t] = mfma_bf16_16x16x32(f.b[h][t], f.a[h][i], acc[i][t]);
}

// Writes acc (+ bias) as bf16 C; lane holds C[m][n .. n+3] of each 16x16 tile.
template <class C>
__device__ __forceinline__ void a16_store_c(const ga_flatmm_splitk_kargs& ka, int b, int m0,
                                            int n0, int wm, int wn, int lane,
                                            const v4f (&acc)[C::TM][C::TN])
{
    uint16_t* cb = (uint16_t*)ka.ptr_c + (size_t)b * (size_t)ka.stride_c_batch;
    const uint16_t* bias = (const uint16_t*)ka.ptr_bias;
    if (bias)
        bias += (size_t)b * (size_t)ka.stride_bias_batch;
    const bool vec = (ka.stride_c & 3) == 0 && (ka.stride_c_batch & 3) == 0 &&
                     ((uintptr_t)ka.ptr_c & 7) == 0;
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        const int m = m0 + wm * C::WTM + i * 16 + (lane & 15);
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int n = n0 + wn * C::WTN + j * 16 + (lane >> 4) * 4;
            if (m >= ka.m || n >= ka.n)
                continue;
            uint16_t* o = cb + (size_t)m * ka.stride_c + n;
            uint16_t q[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float v = acc[i][j][e];
                if (bias && n + e < ka.n)
                    v = v + bf16_to_f32(bias[n + e]);
                q[e] = f32_to_bf16(v);
            }
            if (vec && n + 4 <= ka.n) {
                uint2 pk;
                pk.x = (uint32_t)q[0] | ((uint32_t)q[1] << 16);
                pk.y = (uint32_t)q[2] | ((uint32_t)q[3] << 16);
                *(uint2*)o = pk;
            } else {
                for (int e = 0; e < 4 && n + e < ka.n; e++)
                    o[e] = q[e];
            }
        }
    }
}

// Writes acc as the fp32 partials of slice `split`.
template <class C>
__device__ __forceinline__ void a16_store_ws(const ga_flatmm_splitk_kargs& ka, float* ws, int split,
                                             int b, int m0, int n0, int wm, int wn, int lane,
                                             const v4f (&acc)[C::TM][C::TN])
{
    const size_t split_stride = (size_t)ka.batch * (size_t)ka.stride_ws_batch;
    float* wsb = ws + (size_t)b * (size_t)ka.stride_ws_batch;
    const bool vec = (ka.stride_ws & 3) == 0 && ((uintptr_t)ws & 15) == 0 &&
                     (ka.stride_ws_batch & 3) == 0;
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        const int m = m0 + wm * C::WTM + i * 16 + (lane & 15);
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int n = n0 + wn * C::WTN + j * 16 + (lane >> 4) * 4;
            if (m >= ka.m || n >= ka.n)
                continue;
            float* o = wsb + split * split_stride + (size_t)m * ka.stride_ws + n;
            if (vec && n + 4 <= ka.n) {
                *(v4f*)o = acc[i][j];
            } else {
                for (int e = 0; e < 4 && n + e < ka.n; e++)
                    o[e] = acc[i][j][e];
            }
        }
    }
}

// Workgroup -> (slice, M tile, N tile): XCD round-robin undone (each XCD gets
// a contiguous range), slice outermost, then M-grouped tiles.
__device__ __forceinline__ void a16_map(int tiles_m, int tiles_n, int& split, int& tm, int& tn)
{
    int lin = blockIdx.x;
    const int total = gridDim.x;
    const int full = (total / 8) * 8;
    if (lin < full)
        lin = (lin % 8) * (total / 8) + lin / 8;
    const int tiles = tiles_m * tiles_n;
    split = lin / tiles;
    const int t = lin - split * tiles;
    const int per_group = kA16GroupM * tiles_n;
    const int grp = t / per_group;
    const int first_m = grp * kA16GroupM;
    const int gsize = min(tiles_m - first_m, kA16GroupM);
    const int r = t - grp * per_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

// The workspace of the handle, or null when it is missing or smaller than
// the layout needs (the kernel then writes nothing).
__device__ __forceinline__ float* a16_ws(const ga_flatmm_splitk_kargs& ka)
{
    const ga_splitk_ws_handle* h = ka.ws_handle;
    float* ws = (float*)h->ptr;
    const uint64_t need =
        (uint64_t)ka.split_k * (uint64_t)ka.batch * (uint64_t)ka.stride_ws_batch * 4u;
    return (ws == nullptr || h->bytes < need) ? nullptr : ws;
}

template <class C, int EPI>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256)))
void a16w16_splitk_kernel(A16Args p)
{
    __shared__ __attribute__((aligned(1024))) char smem[C::LDS];
    const ga_flatmm_splitk_kargs& ka = p.ka;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int M = ka.m, N = ka.n, K = ka.k;

    int split, tm, tn;
    a16_map(p.tiles_m, p.tiles_n, split, tm, tn);
    const int m0 = tm * C::BM, n0 = tn * C::BN;
    const int b = blockIdx.z;

    float* ws = nullptr;
    if (EPI != EPI_C) {
        ws = a16_ws(ka);
        if (ws == nullptr)
            return;
    }

    const int kb = split * p.kslice;
    const int ke = min(K, kb + p.kslice);
    const int nsteps = ke > kb ? (ke - kb + 63) / 64 : 0;

    A16State<C> st;
    {
        const uint32_t lda = (uint32_t)ka.stride_a * 2, ldb = (uint32_t)ka.stride_b * 2;
        const char* pa = (const char*)ka.ptr_a +
                         ((size_t)b * (size_t)ka.stride_a_batch + (size_t)m0 * ka.stride_a) * 2;
        const char* pb = (const char*)ka.ptr_b +
                         ((size_t)b * (size_t)ka.stride_b_batch + (size_t)n0 * ka.stride_b) * 2;
        const long long abytes = (long long)(M - m0) * lda;
        const long long bbytes = (long long)(N - n0) * ldb;
        st.ra = make_rsrc(pa, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
        st.rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
        // copy i covers rows 32i .. 32i+31 (wave w: 8 whole rows) of the
        // swizzled LDS image; the lane's K chunk is the same for every i
        int row0, chunk;
        pp::copy_lane(wave, lane, row0, chunk);
        st.kchunk = chunk * 8;
#pragma unroll
        for (int i = 0; i < C::A_LOADS; i++)
            st.voff_a[i] = (uint32_t)(i * 32 + row0) * lda + chunk * 16;
#pragma unroll
        for (int i = 0; i < C::B_LOADS; i++)
            st.voff_b[i] = (uint32_t)(i * 32 + row0) * ldb + chunk * 16;
    }

    v4f acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++)
            acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

    // Pipeline: NS-1 stages in flight, and the operand fragments of step s+1
    // read from LDS while the MFMAs of step s run. Step s waits for stage s+1
    // (counted vmcnt: the loop's only memory reads are direct-to-LDS copies;
    // the barrier also ends every wave's fragment reads of stage s), refills
    // the buffer step s-1 used with stage s+NS-1, reads the fragments of
    // stage s+1, then multiplies the fragments of stage s read one step
    // earlier. Two fragment sets alternate (the loop is unrolled by two).
#pragma unroll
    for (int q = 0; q < C::NS - 1; q++)
        a16_issue<C>(st, smem, q, q, kb, ke, wave);
    A16Frag<C> f0, f1;
    wait_vmcnt<C::TILE_LOADS * (C::NS - 2)>();
    barrier_lds();
    a16_read<C>(smem, 0, wm, wn, lane, f0);
    int buf = 0; // LDS buffer of stage s
    auto step = [&](int s, const A16Frag<C>& cur, A16Frag<C>& nxt) {
        wait_vmcnt<C::TILE_LOADS * (C::NS - 3)>();
        barrier_lds();
        const int prev = buf == 0 ? C::NS - 1 : buf - 1;
        const int next = buf + 1 == C::NS ? 0 : buf + 1;
        a16_issue<C>(st, smem, prev, s + C::NS - 1, kb, ke, wave);
        __builtin_amdgcn_sched_barrier(0);
        a16_read<C>(smem, next, wm, wn, lane, nxt);
        a16_mma<C>(cur, acc);
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
    // drain the prefetches past the slice before the workgroup's LDS is freed
    wait_vmcnt<0>();

    if (EPI == EPI_C) {
        a16_store_c<C>(ka, b, m0, n0, wm, wn, lane, acc);
        return;
    }
    a16_store_ws<C>(ka, ws, split, b, m0, n0, wm, wn, lane, acc);
}

// One configuration over split_k x tiles workgroups (x) and batch (z).
template <class C, int EPI>
static ga_status launch_a16(const ga_flatmm_splitk_kargs& ka, int kslice, hipStream_t stream)
{
    A16Args p;
    p.ka = ka;
    p.tiles_m = (ka.m + C::BM - 1) / C::BM;
    p.tiles_n = (ka.n + C::BN - 1) / C::BN;
    p.kslice = kslice;
    const long long gx = (long long)ka.split_k * p.tiles_m * p.tiles_n;
    if (gx > 0x7FFFFFFFll)
        return fail(GA_ERR_SHAPE, "a16w16 split-K: grid too large");
    hipLaunchKernelGGL((a16w16_splitk_kernel<C, EPI>), dim3((unsigned)gx, 1, ka.batch),
                       dim3(256), 0, stream, p);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

// Tile configurations, largest first. Measured on MI355X (bf16, 2048-8192
// sized problems and the skinny 1024x512x7168): the largest tile whose grid
// still gives every CU a workgroup wins; 128-row tiles are not used for M up
// to 64 (they would compute mostly padding). B loaded straight into
// registers (as the preshuffled MX kernels do) was measured slower here: a
// row-major B fragment load touches 16 rows x 64 bytes per instruction.
typedef A16Cfg<128, 256, 3> A16Huge;
typedef A16Cfg<128, 128, 4> A16Big;
typedef A16Cfg<64, 128, 4> A16Mid;
typedef A16Cfg<64, 64, 6> A16Small;

template <int EPI>
static ga_status dispatch_a16(const ga_flatmm_splitk_kargs& ka, hipStream_t stream)
{
    int num_cu = 0;
    ga_status st = device_cu_count(&num_cu);
    if (st != GA_OK)
        return st;
    const int iters = (ka.k + 127) / 128;
    const int per = (iters + ka.split_k - 1) / ka.split_k;
    const int kslice = per * 128;
    auto wgs = [&](int bm, int bn) {
        return (long long)((ka.m + bm - 1) / bm) * ((ka.n + bn - 1) / bn) * ka.split_k * ka.batch;
    };
    const bool tall = ka.m > 64;
    if (tall && wgs(128, 256) >= num_cu)
        return launch_a16<A16Huge, EPI>(ka, kslice, stream);
    if (tall && wgs(128, 128) >= num_cu)
        return launch_a16<A16Big, EPI>(ka, kslice, stream);
    if (wgs(64, 128) >= num_cu)
        return launch_a16<A16Mid, EPI>(ka, kslice, stream);
    return launch_a16<A16Small, EPI>(ka, kslice, stream);
}

static ga_status check_a16(const ga_flatmm_splitk_kargs* ka)
{
    if (!ka || !ka->ptr_a || !ka->ptr_b)
        return fail(GA_ERR_ARG, "a16w16 split-K: null kargs or operand pointer");
    if (ka->m <= 0 || ka->n <= 0 || ka->k <= 0 || ka->batch <= 0 || ka->split_k <= 0)
        return fail(GA_ERR_ARG, "a16w16 split-K: M, N, K, batch and split_k must be positive");
    if (ka->k % 8 != 0)
        return fail(GA_ERR_SHAPE, "a16w16 split-K: K must be a multiple of 8, got %d", ka->k);
    if (ka->stride_a < ka->k || ka->stride_b < ka->k || ka->stride_a % 8 || ka->stride_b % 8)
        return fail(GA_ERR_SHAPE, "a16w16 split-K: stride_a/stride_b must be >= K and "
                                  "multiples of 8");
    if (ka->stride_a > (1 << 22) || ka->stride_b > (1 << 22))
        return fail(GA_ERR_SHAPE, "a16w16 split-K: row stride above 2^22 elements");
    if (((uintptr_t)ka->ptr_a & 15) || ((uintptr_t)ka->ptr_b & 15))
        return fail(GA_ERR_ARG, "a16w16 split-K: A and B must be 16-byte aligned");
    if (ka->stride_a_batch < 0 || ka->stride_b_batch < 0 || ka->stride_c_batch < 0)
        return fail(GA_ERR_SHAPE, "a16w16 split-K: negative batch stride");
    if (ka->batch > 65535)
        return fail(GA_ERR_SHAPE, "a16w16 split-K: batch > 65535");
    return GA_OK;
}

static ga_status check_ws_layout(const ga_flatmm_splitk_kargs* ka)
{
    if (!ka->ws_handle)
        return fail(GA_ERR_ARG, "a16w16 split-K: null workspace handle");
    if (ka->stride_ws < ka->n || (long long)ka->stride_ws_batch < (long long)ka->m * ka->stride_ws)
        return fail(GA_ERR_SHAPE, "a16w16 split-K: stride_ws must be >= N and "
                                  "stride_ws_batch >= M * stride_ws");
    if ((long double)ka->split_k * ka->batch * ka->stride_ws_batch * 4.0L > 4.0e18L)
        return fail(GA_ERR_SHAPE, "a16w16 split-K: workspace layout too large");
    return GA_OK;
}

// Host mirror of every slot created here: slot -> {buffer, bytes, device}.
struct WsSlot {
    void* ptr;
    size_t bytes;
    int device;
};
static std::mutex g_ws_mu;
static std::unordered_map<const void*, WsSlot>& ws_slots()
{
    static std::unordered_map<const void*, WsSlot> m;
    return m;
}

} // namespace ga

bool ga::ws_slot_bytes(const ga_splitk_ws_handle* slot, size_t* bytes)
{
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = ws_slots().find(slot);
    if (it == ws_slots().end())
        return false;
    *bytes = it->second.bytes;
    return true;
}

namespace ga {

// Runs `f` with `dev` current, restoring the caller's device.
template <class F>
static ga_status on_device(int dev, F&& f)
{
    int cur = 0;
    GA_HIP_CHECK(hipGetDevice(&cur));
    if (cur != dev)
        GA_HIP_CHECK(hipSetDevice(dev));
    ga_status st = f();
    if (cur != dev) {
        hipError_t e = hipSetDevice(cur);
        if (st == GA_OK && e != hipSuccess)
            return hip_fail(e, "hipSetDevice");
    }
    return st;
}

} // namespace ga

using namespace ga;

extern "C" {

// A slot made by ga_ws_handle_create that holds less than the layout needs
// (e.g. never reserved) is refused on the host when the stream is not
// capturing; under capture (and for caller-made slots) the kernels' own
// check applies: they write nothing.
static ga_status check_ws_capacity(const ga_flatmm_splitk_kargs* ka, hipStream_t s)
{
    size_t have = 0;
    const size_t need = ga_a16w16_splitk_workspace_bytes(ka);
    if (!ws_slot_bytes(ka->ws_handle, &have) || have >= need)
        return GA_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    GA_HIP_CHECK(hipStreamIsCapturing(s, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return GA_OK;
    return fail(GA_ERR_WORKSPACE, "a16w16 split-K: workspace slot holds %zu bytes, need %zu",
                have, need);
}

ga_status ga_gemm_a16w16_flatmm_splitk(const ga_flatmm_splitk_kargs* kargs, void* stream)
{
    ga_status st = check_a16(kargs);
    if (st == GA_OK)
        st = check_ws_layout(kargs);
    if (st == GA_OK)
        st = check_ws_capacity(kargs, (hipStream_t)stream);
    if (st != GA_OK)
        return st;
    return dispatch_a16<EPI_WS>(*kargs, (hipStream_t)stream);
}

size_t ga_a16w16_splitk_workspace_bytes(const ga_flatmm_splitk_kargs* kargs)
{
    if (!kargs || kargs->split_k <= 0 || kargs->batch <= 0 || kargs->stride_ws_batch <= 0)
        return 0;
    return (size_t)kargs->split_k * (size_t)kargs->batch * (size_t)kargs->stride_ws_batch *
           sizeof(float);
}

ga_status ga_gemm_a16w16_splitk(const ga_flatmm_splitk_kargs* kargs, void* stream)
{
    ga_status st = check_a16(kargs);
    if (st != GA_OK)
        return st;
    if (!kargs->ptr_c || kargs->stride_c < kargs->n)
        return fail(GA_ERR_ARG, "a16w16 split-K: null C or stride_c < N");
    if (kargs->ptr_bias && kargs->stride_bias_batch < 0)
        return fail(GA_ERR_ARG, "a16w16 split-K: negative stride_bias_batch");
    if ((long long)kargs->batch * kargs->m > 65535ll * 1024)
        return fail(GA_ERR_SHAPE, "a16w16 split-K: batch*M too large");
    hipStream_t s = (hipStream_t)stream;
    if (kargs->split_k == 1)
        return dispatch_a16<EPI_C>(*kargs, s);
    st = check_ws_layout(kargs);
    if (st == GA_OK)
        st = check_ws_capacity(kargs, s);
    if (st != GA_OK)
        return st;
    st = dispatch_a16<EPI_WS>(*kargs, s);
    if (st != GA_OK)
        return st;
    ReduceArgs r;
    r.ws = nullptr;
    r.wsh = kargs->ws_handle;
    r.out = kargs->ptr_c;
    r.c_in = nullptr;
    r.bias = kargs->ptr_bias;
    r.out_dtype = GA_DTYPE_BF16;
    r.bias_dtype = GA_DTYPE_BF16;
    r.split_k = kargs->split_k;
    r.M = kargs->m;
    r.N = kargs->n;
    r.batch = kargs->batch;
    r.ws_ld = kargs->stride_ws;
    r.ws_batch = kargs->stride_ws_batch;
    r.ldc = kargs->stride_c;
    r.c_batch_stride = kargs->stride_c_batch;
    r.bias_stride_batch = kargs->stride_bias_batch;
    r.alpha = 1.0f;
    r.beta = 0.0f;
    return splitk_reduce_launch(r, s);
}

ga_status ga_ws_handle_create(ga_splitk_ws_handle** ws_handle)
{
    if (!ws_handle)
        return fail(GA_ERR_ARG, "ws_handle_create: null argument");
    *ws_handle = nullptr;
    int dev = 0;
    GA_HIP_CHECK(hipGetDevice(&dev));
    void* slot = nullptr;
    GA_HIP_CHECK(hipMalloc(&slot, sizeof(ga_splitk_ws_handle)));
    const ga_splitk_ws_handle init = {nullptr, 0};
    hipError_t e = hipMemcpy(slot, &init, sizeof(init), hipMemcpyHostToDevice);
    if (e == hipSuccess) // the slot is written before any stream reads it
        e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(slot);
        return hip_fail(e, "hipMemcpy(ws slot)");
    }
    std::lock_guard<std::mutex> lock(g_ws_mu);
    ws_slots()[slot] = WsSlot{nullptr, 0, dev};
    *ws_handle = (ga_splitk_ws_handle*)slot;
    return GA_OK;
}

ga_status ga_ws_handle_reserve(ga_splitk_ws_handle* ws_handle, size_t bytes)
{
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = ws_slots().find(ws_handle);
    if (it == ws_slots().end())
        return fail(GA_ERR_ARG, "ws_handle_reserve: not a slot made by ga_ws_handle_create");
    WsSlot& w = it->second;
    if (bytes <= w.bytes)
        return GA_OK;
    return on_device(w.device, [&]() -> ga_status {
        // nothing queued may still use the old buffer once it is freed
        GA_HIP_CHECK(hipDeviceSynchronize());
        void* p = nullptr;
        GA_HIP_CHECK(hipMalloc(&p, bytes));
        const ga_splitk_ws_handle v = {p, (uint64_t)bytes};
        hipError_t e = hipMemcpy(ws_handle, &v, sizeof(v), hipMemcpyHostToDevice);
        if (e == hipSuccess) // the slot is written before any stream reads it
            e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            (void)hipFree(p);
            return hip_fail(e, "hipMemcpy(ws slot)");
        }
        if (w.ptr)
            GA_HIP_CHECK(hipFree(w.ptr));
        w.ptr = p;
        w.bytes = bytes;
        return GA_OK;
    });
}

ga_status ga_ws_handle_query(const ga_splitk_ws_handle* ws_handle, void** ptr, size_t* bytes)
{
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = ws_slots().find(ws_handle);
    if (it == ws_slots().end())
        return fail(GA_ERR_ARG, "ws_handle_query: not a slot made by ga_ws_handle_create");
    if (ptr)
        *ptr = it->second.ptr;
    if (bytes)
        *bytes = it->second.bytes;
    return GA_OK;
}

ga_status ga_ws_handle_destroy(ga_splitk_ws_handle* ws_handle)
{
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = ws_slots().find(ws_handle);
    if (it == ws_slots().end())
        return fail(GA_ERR_ARG, "ws_handle_destroy: not a slot made by ga_ws_handle_create");
    WsSlot w = it->second;
    ws_slots().erase(it);
    return on_device(w.device, [&]() -> ga_status {
        GA_HIP_CHECK(hipDeviceSynchronize());
        if (w.ptr)
            GA_HIP_CHECK(hipFree(w.ptr));
        GA_HIP_CHECK(hipFree(ws_handle));
        return GA_OK;
    });
}

} // extern "C"

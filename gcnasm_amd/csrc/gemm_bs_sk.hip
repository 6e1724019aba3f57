// gemm_bs_sk.hip -- stream-K form of the 256x256 fp32-scaled FP8 GEMM
// (DeepSeek block scale, batch 1), for long-K problems whose 256x256 tiles
// keep few CUs busy (2048 x 2560 x 8192: 80 tiles on 256 CUs).
//
// With T = tiles * G iterations (G = K / 128 groups per tile) and P
// workgroups (one per CU), virtual workgroup v computes iterations
// [v*T/P, (v+1)*T/P): the K groups of consecutive tiles, so every CU does the
// same MFMA work however the tile count falls against the CU count. A tile
// cut between workgroups is a chain of segments in K order; every segment's
// fp32 accumulator goes to a partial slot with device-coherent stores, its
// workgroup counts itself in the tile's counter, and the last to arrive adds
// the segments in K order ((s0 + s1) + s2) and stores the tile, then leaves
// the counter at zero. Nobody waits for anybody (the reference's
// cross-workgroup counter, wmma_opus_rdna4/opus/opus.hpp:1296-1304, spins
// until a count is reached; here the last arrival does the work instead).
// Used when the tiles fill under one round (at most 40 % of the CUs), so a
// workgroup's range touches at most three tiles and the kernel is three
// straight-line segments (a loop around the K loop would cost the registers
// the K loop needs).
#include "ga_bs_pp.hpp"
#include "ga_internal.hpp"

namespace ga {
namespace {

using namespace pp;
using namespace bspp;

struct BsSkArgs {
    ga_opus_gemm_kargs ka;
    int tiles_x, tiles_y; // 256x256 tiles along N and M
    int groups;           // K / 128
    int total;            // tiles * groups
    int nwg;              // workgroups (a multiple of 8)
    unsigned* cnt;        // per-tile arrival counters, zero between calls; then
                          // the misuse word (set when a count ran past its tile's pieces)
    float* part;          // 2 * nwg partial tiles of 65536 floats
};

// The argument block read again where it is used (the segment loop needs
// about 30 scalars of it after each K loop, more than the scalar registers
// the K loop leaves).
__device__ __forceinline__ BsSkArgs sk_args_fresh()
{
    auto p = __builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    const __attribute__((address_space(4))) BsSkArgs* c =
        (const __attribute__((address_space(4))) BsSkArgs*)p;
    BsSkArgs r;
#define GA_SK_FIELD(f) r.ka.f = c->ka.f
    GA_SK_FIELD(ptr_a); GA_SK_FIELD(ptr_b); GA_SK_FIELD(ptr_c);
    GA_SK_FIELD(m); GA_SK_FIELD(n); GA_SK_FIELD(k); GA_SK_FIELD(batch);
    GA_SK_FIELD(stride_a); GA_SK_FIELD(stride_b); GA_SK_FIELD(stride_c);
    GA_SK_FIELD(stride_a_batch); GA_SK_FIELD(stride_b_batch); GA_SK_FIELD(stride_c_batch);
    GA_SK_FIELD(ptr_sfa); GA_SK_FIELD(ptr_sfb); GA_SK_FIELD(stride_sfa); GA_SK_FIELD(stride_sfb);
    GA_SK_FIELD(stride_sfa_batch); GA_SK_FIELD(stride_sfb_batch);
#undef GA_SK_FIELD
    r.tiles_x = c->tiles_x;
    r.tiles_y = c->tiles_y;
    r.groups = c->groups;
    r.total = c->total;
    r.nwg = c->nwg;
    r.cnt = c->cnt;
    r.part = c->part;
    return r;
}

// The lane id formed where it is used, so that nothing derived from it is
// hoisted out of the segment loop and held across the K loop.
__device__ __forceinline__ int fresh_lane()
{
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

__device__ __forceinline__ int sk_begin(int v, int total, int nwg)
{
    return (int)(((long long)v * total) / nwg);
}

// The virtual workgroup whose iterations include `it`.
__device__ __forceinline__ int sk_owner(int it, int total, int nwg)
{
    return (int)((((long long)it + 1) * nwg - 1) / total);
}

// Tile t of the stream in groups of kBsGroupM tile rows, column by column.
__device__ __forceinline__ void sk_tile(int t, int tiles_x, int tiles_y, int& tm, int& tn)
{
    const int per_group = kBsGroupM * tiles_x;
    const int g = t / per_group;
    const int first_m = g * kBsGroupM;
    const int gsize = min(tiles_y - first_m, kBsGroupM);
    const int r = t - g * per_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

// Partial slot of virtual workgroup v for the segment starting at iteration
// `it`: 2v for its first segment, 2v + 1 for its last.
__device__ __forceinline__ int sk_slot(int v, int it, int total, int nwg)
{
    return 2 * v + (it == sk_begin(v, total, nwg) ? 0 : 1);
}

// A segment's K loop: groups [0, nsteps) relative to the copy state's first
// group. One loop body for every group (peeled groups have constant copy
// offsets that the compiler would hoist out of the segment loop into
// registers the K loop needs); group 0's phase 1 folds the zeroed
// temporaries with zeroed scales into the zero accumulator, which leaves it
// zero whatever the scale slot it reads holds.
template <int MODE>
__device__ __forceinline__ void bs_k_loop_flat(int nsteps, const BsLoad& L, const BsRead& rb,
                                               char* smem, int wave, int grp,
                                               v4f (&acc)[4][4][2])
{
    constexpr int S = MODE == PS_TENSOR ? 0 : 1;
    v4f p[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int t = 0; t < 2; t++)
            p[i][t] = (v4f){0.f, 0.f, 0.f, 0.f};
    v8i fa[4], fb0[2], fb1[2];
    ScaleVals sv;
    phase_sync<12 + S>(); // B0 (+ scales) of group 0
    read_b<0>(rb, 0, fb0);
    phase_sync<10 + S>(); // A0 of group 0
    if (grp == 1)
        slot_sync(); // second group runs one barrier behind
    for (int s = 0; s < nsteps; s++) {
        const int slot = s & 1;
        const int r0 = s & 3, r2 = (s + 2) & 3, rprev = (s - 1) & 3;
        // phase 1 (folds in quadrant 11 of the previous group)
        issue_a(L, smem, 1, s + 1, wave);
        sv = read_scales<MODE, 1, 1>(rb, rprev);
        if constexpr (MODE != PS_TENSOR) {
            if (s == 0) {
                sv.sa = (v4f){0.f, 0.f, 0.f, 0.f};
                sv.sb0 = (v4f){0.f, 0.f, 0.f, 0.f};
                sv.sb1 = (v4f){0.f, 0.f, 0.f, 0.f};
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        read_a<0>(rb, slot, fa);
        __builtin_amdgcn_sched_barrier(0);
        phase_sync<10 + S>();
        mma_quadrant<MODE, true>(acc[0], p, fa, fb0, acc[3], sv);
        slot_sync();
        // phase 2
        BS_MEM_SLOT(0, 0, r0,
                    issue_b(L, smem, 0, s + 2, wave); if (S) issue_s(L, smem, s + 2, r2, wave),
                    read_b<1>(rb, slot, fb1), 10 + 2 * S);
        mma_quadrant<MODE, true>(acc[1], p, fa, fb1, acc[0], sv);
        slot_sync();
        // phase 3
        BS_MEM_SLOT(0, 1, r0, issue_a(L, smem, 0, s + 2, wave), read_a<1>(rb, slot, fa), 10 + S);
        mma_quadrant<MODE, true>(acc[2], p, fa, fb0, acc[1], sv);
        slot_sync();
        // phase 4
        BS_MEM_SLOT(1, 0, r0, issue_b(L, smem, 1, s + 2, wave), read_b<0>(rb, slot ^ 1, fb0),
                    10 + S);
        mma_quadrant<MODE, true>(acc[3], p, fa, fb1, acc[2], sv);
        slot_sync();
    }
    if (grp == 0)
        slot_sync(); // matches the second group's extra barrier
    if constexpr (MODE != PS_TENSOR) {
        const ScaleVals last = read_scales<MODE, 1, 1>(rb, (nsteps - 1) & 3);
        apply_scales<MODE>(last, acc[3], p);
    }
}

// Copy state of tile (m0, n0) of batch 0 from K group g0 on.
template <int MODE>
__device__ __forceinline__ BsLoad bs_load_from(const ga_opus_gemm_kargs& ka, int m0, int n0,
                                               int g0, int wave, int lane)
{
    const int M = ka.m, N = ka.n, K = ka.k;
    BsLoad L;
    int crow, ckc;
    copy_lane(wave, lane, crow, ckc);
    const char* pa = (const char*)ka.ptr_a + (size_t)m0 * ka.stride_a;
    const char* pb = (const char*)ka.ptr_b + (size_t)n0 * ka.stride_b;
    const long long abytes = (long long)(M - m0) * ka.stride_a;
    const long long bbytes = (long long)(N - n0) * ka.stride_b;
    L.ra = make_rsrc(pa, (uint32_t)(abytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : abytes));
    L.rb = make_rsrc(pb, (uint32_t)(bbytes > 0xFFFFFFF0ll ? 0xFFFFFFF0ll : bbytes));
    L.va = (uint32_t)crow * ka.stride_a + ckc * 16 + (uint32_t)g0 * 128;
    L.vb = (uint32_t)crow * ka.stride_b + ckc * 16 + (uint32_t)g0 * 128;
    L.a_hstep = 64 * (uint32_t)ka.stride_a;
    L.b_hstep = 64 * (uint32_t)ka.stride_b;
    L.vs = 0;
    L.s_kstep = 0;
    if constexpr (MODE != PS_TENSOR) {
        const int ngroups = K / 128;
        if (wave < 4) {
            const float* sfa = (const float*)ka.ptr_sfa;
            L.rs = make_rsrc(sfa, (uint32_t)ngroups * ka.stride_sfa * 4);
            const int row = min(m0 + wave * 64 + (lane & 3) * 16 + (lane >> 2), M - 1);
            L.s_kstep = (uint32_t)ka.stride_sfa * 4;
            L.vs = (uint32_t)row * 4 + (uint32_t)g0 * L.s_kstep;
        } else {
            const float* sfb = (const float*)ka.ptr_sfb;
            const int pos = (wave - 4) * 64 + lane;
            if (MODE == PS_GROUP128) {
                const int nblk = (N + 127) / 128;
                L.rs = make_rsrc(sfb, (uint32_t)nblk * ka.stride_sfb * 4);
                const int nb = min(n0 / 128 + (pos & 1), nblk - 1);
                L.s_kstep = 4;
                L.vs = (uint32_t)nb * ka.stride_sfb * 4 + (uint32_t)g0 * 4;
            } else {
                L.rs = make_rsrc(sfb, (uint32_t)ngroups * ka.stride_sfb * 4);
                const int col = min(n0 + pos, N - 1);
                L.s_kstep = (uint32_t)ka.stride_sfb * 4;
                L.vs = (uint32_t)col * 4 + (uint32_t)g0 * L.s_kstep;
            }
        }
    }
    return L;
}

template <int MODE>
__device__ __forceinline__ BsRead bs_read_setup(char* smem, int lane, int grp, int simd)
{
    BsRead rb;
    uint32_t o, o64;
    operand_lane(lane, o, o64);
    rb.a0 = smem + grp * 64 * 128 + o;
    rb.a1 = smem + grp * 64 * 128 + o64;
    rb.b0 = smem + kBRegion + simd * 32 * 128 + o;
    rb.b1 = smem + kBRegion + simd * 32 * 128 + o64;
    rb.sa = smem + kSBase + grp * 256 + (lane & 15) * 16;
    rb.sb = smem + kSBase + 1024 + (MODE == PS_GROUP1 ? (simd * 32 + (lane >> 4) * 4) * 4 : 0);
    return rb;
}

// A tile's first copies, in steady-state order: B0+S, A0, B1, A1 of K group
// 0; B0+S, A0, B1 of group 1.
template <int S>
__device__ __forceinline__ void bs_prologue_copies(const BsLoad& L, char* smem, int wave)
{
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
}

constexpr int kSkSlotFloats = 256 * 256;

// A segment's accumulator to its partial slot: chunk (q, i, t) of all 512
// threads is 8 KB of contiguous 16-byte stores, device-coherent (sc1) so
// that a workgroup on another XCD reads them from past its own L2. tid is
// formed by the caller where it is used.
__device__ __forceinline__ void sk_put(float* slot, const v4f (&acc)[4][4][2], int tid)
{
    const __amdgpu_buffer_rsrc_t r = make_rsrc(slot, kSkSlotFloats * 4);
    const uint32_t vo = (uint32_t)tid * 16;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const v4f v = acc[q][i][t];
                const v4i d = {(int)__float_as_uint(v[0]), (int)__float_as_uint(v[1]),
                               (int)__float_as_uint(v[2]), (int)__float_as_uint(v[3])};
                __builtin_amdgcn_raw_buffer_store_b128(d, r, vo, ((q * 4 + i) * 2 + t) * kNT * 16,
                                                       16);
            }
}

// Chunk (q, i, t) of thread tid from a partial slot (device-coherent load).
__device__ __forceinline__ v4f sk_get(__amdgpu_buffer_rsrc_t r, int q, int i, int t, int tid)
{
    const v4i d = __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)tid * 16,
                                                        ((q * 4 + i) * 2 + t) * kNT * 16, 16);
    return (v4f){__uint_as_float((uint32_t)d[0]), __uint_as_float((uint32_t)d[1]),
                 __uint_as_float((uint32_t)d[2]), __uint_as_float((uint32_t)d[3])};
}

// Virtual workgroup of workgroup w: contiguous iteration ranges for the
// workgroups of one XCD (workgroups are dispatched round-robin over the 8).
__device__ __forceinline__ int sk_virtual(int w, int nwg) { return (w % 8) * (nwg / 8) + w / 8; }

// A finished 256x256 tile (acc: lane holds C[m][n .. n+3] of each 16x16
// MFMA tile) into C of batch b at (m0, n0): whole interior tiles through LDS
// as whole rows, the rest lane by lane. Called after the K loop, when no wave
// still needs the operand slots.
template <int MODE, int OUT>
__device__ __forceinline__ void bs_tile_store(const v4f (&acc)[4][4][2],
                                              const ga_opus_gemm_kargs& ka, int b, int m0,
                                              int n0, char* smem, int wave, int grp, int simd,
                                              int lane)
{
    const int M = ka.m, N = ka.n;
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
                    *(v4i*)(dst + (size_t)row * ldc + lane * 4) = d;
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
            stage_store(smem, (uint16_t*)pc + (size_t)m0 * ldc + n0, ldc, wave, lane);
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

// One segment of this workgroup's range, starting at iteration `it` (a
// no-op once the range is done). Everything it needs is formed again from
// the arguments, the workgroup id and the lane id, so that nothing is held
// in registers across the K loops of the segments before it.
template <int MODE, int OUT>
__device__ __forceinline__ void sk_segment(int& it, char* smem, int wave)
{
    // the arrival count goes to the workgroup through the (idle) first LDS
    // word: a second LDS object would leave the compiler unable to tell the
    // operand reads from the in-flight copies, and it would drain them all
    // before every read of the K loops
    unsigned* s_arrived = (unsigned*)smem;
    constexpr int S = MODE == PS_TENSOR ? 0 : 1;
    const int grp = wave >> 2, simd = wave & 3;
    const BsSkArgs a = sk_args_fresh();
    const int nwg = a.nwg, total = a.total, G = a.groups;
    const int v = sk_virtual(blockIdx.x, nwg);
    const int it_end = sk_begin(v + 1, total, nwg);
    if (it >= it_end)
        return;
    const int t = it / G, g0 = it - t * G, g1 = min(G, g0 + (it_end - it));
    int tm, tn;
    sk_tile(t, a.tiles_x, a.tiles_y, tm, tn);
    const int m0 = tm * 256, n0 = tn * 256;
    v4f acc[4][4][2];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int u = 0; u < 2; u++)
                acc[q][i][u] = (v4f){0.f, 0.f, 0.f, 0.f};
    {
        const BsLoad L = bs_load_from<MODE>(a.ka, m0, n0, g0, wave, fresh_lane());
        bs_prologue_copies<S>(L, smem, wave);
        bs_k_loop_flat<MODE>(g1 - g0, L, bs_read_setup<MODE>(smem, threadIdx.x & 63, grp, simd), smem,
                             wave, grp, acc);
    }
    wait_vmcnt<0>(); // copies past the segment have landed
    bool store = g0 == 0 && g1 == G;
    if (!store) {
        float* part = a.part;
        const int lo = sk_owner(t * G, total, nwg), hi = sk_owner(t * G + G - 1, total, nwg);
        // A tile's first K piece is the last segment of its workgroup's
        // range, while the other pieces start theirs, so it usually arrives
        // last: when every other piece is already counted, its workgroup
        // finishes the tile from its registers without writing them out.
        bool regs = false;
        // A count above hi - lo means the counter did not start at zero (the
        // workspace was not left zero-filled): the tile's sum is lost, and the
        // misuse word after the counters says so (ga_blockscale_workspace_check).
        const unsigned* misuse_at = a.cnt + a.tiles_x * a.tiles_y;
        if (v == lo) {
            if (threadIdx.x == 0) {
                const unsigned seen =
                    __hip_atomic_load(a.cnt + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (seen > (unsigned)(hi - lo))
                    __hip_atomic_store((unsigned*)misuse_at, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                *s_arrived = seen;
            }
            barrier_lds();
            regs = __builtin_amdgcn_readfirstlane(*s_arrived) == (unsigned)(hi - lo);
            barrier_lds(); // read in every wave before the word is written again
        }
        if (regs) {
            if (threadIdx.x == 0)
                __hip_atomic_store(a.cnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            store = true;
        } else {
            sk_put(part + (size_t)sk_slot(v, it, total, nwg) * kSkSlotFloats, acc,
                   wave * 64 + fresh_lane());
            wait_vmcnt<0>();    // this thread's partial stores are complete
            wait_lds_barrier(); // ... in every thread, before the count
            if (threadIdx.x == 0) {
                const unsigned old = __hip_atomic_fetch_add(a.cnt + t, 1u, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
                if (old == (unsigned)(hi - lo))
                    __hip_atomic_store(a.cnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else if (old > (unsigned)(hi - lo))
                    __hip_atomic_store((unsigned*)misuse_at, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                *s_arrived = old;
            }
            barrier_lds();
            store = __builtin_amdgcn_readfirstlane(*s_arrived) == (unsigned)(hi - lo);
        }
        if (store) {
            // last in: the tile's pieces summed in K order, piece 0 from the
            // registers (regs) or its slot, the rest from theirs (a piece of
            // this workgroup's own from its slot: the same bits as its
            // registers), two quadrants (16 loads) in flight at a time
            const int tid = wave * 64 + fresh_lane();
            const int slot0 = 2 * lo + (sk_begin(lo, total, nwg) >= t * G ? 0 : 1);
#pragma unroll
            for (int qp = 0; qp < 4; qp += 2) {
                if (!regs) {
                    const __amdgpu_buffer_rsrc_t r0 =
                        make_rsrc(part + (size_t)slot0 * kSkSlotFloats, kSkSlotFloats * 4);
#pragma unroll
                    for (int q = qp; q < qp + 2; q++)
#pragma unroll
                        for (int i = 0; i < 4; i++)
#pragma unroll
                            for (int u = 0; u < 2; u++)
                                acc[q][i][u] = sk_get(r0, q, i, u, tid);
                }
                for (int vj = lo + 1; vj <= hi; vj++) {
                    const __amdgpu_buffer_rsrc_t rj =
                        make_rsrc(part + (size_t)(2 * vj) * kSkSlotFloats, kSkSlotFloats * 4);
                    v4f x[2][4][2];
#pragma unroll
                    for (int q = 0; q < 2; q++)
#pragma unroll
                        for (int i = 0; i < 4; i++)
#pragma unroll
                            for (int u = 0; u < 2; u++)
                                x[q][i][u] = sk_get(rj, qp + q, i, u, tid);
#pragma unroll
                    for (int q = 0; q < 2; q++)
#pragma unroll
                        for (int i = 0; i < 4; i++)
#pragma unroll
                            for (int u = 0; u < 2; u++)
                                acc[qp + q][i][u] = acc[qp + q][i][u] + x[q][i][u];
                }
            }
        }
    }
    if (store)
        bs_tile_store<MODE, OUT>(acc, a.ka, 0, m0, n0, smem, wave, grp, simd, fresh_lane());
    it += g1 - g0;
    barrier_lds(); // every LDS read of this segment is done before the next one's copies
}

template <int MODE, int OUT>
__global__ __attribute__((amdgpu_flat_work_group_size(kNT, kNT), amdgpu_waves_per_eu(2, 2)))
void bs_pp_sk_kernel(BsSkArgs args)
{
    __shared__ __attribute__((aligned(1024))) char smem[kLdsBs];
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    int it = sk_begin(sk_virtual(blockIdx.x, args.nwg), args.total, args.nwg);
    sk_segment<MODE, OUT>(it, smem, wave);
    sk_segment<MODE, OUT>(it, smem, wave);
    sk_segment<MODE, OUT>(it, smem, wave);
}

template <int MODE, int OUT>
void launch_bs_pp_sk_t(const ga_opus_gemm_kargs& ka, int nwg, void* ws, hipStream_t stream)
{
    BsSkArgs a;
    a.ka = ka;
    a.tiles_x = (ka.n + 255) / 256;
    a.tiles_y = (ka.m + 255) / 256;
    a.groups = ka.k / 128;
    a.total = a.tiles_x * a.tiles_y * a.groups;
    a.nwg = nwg;
    a.cnt = (unsigned*)ws;
    a.part = (float*)((char*)ws + bs_sk_counter_bytes(ka));
    hipLaunchKernelGGL((bs_pp_sk_kernel<MODE, OUT>), dim3(nwg), dim3(kNT), 0, stream, a);
}

} // namespace

int bs_sk_workgroups(const ga_opus_gemm_kargs& ka, int num_cu)
{
    const int nwg = num_cu / 8 * 8;
    if (ka.batch != 1 || nwg < 8)
        return 0;
    const long long tiles = (long long)((ka.n + 255) / 256) * ((ka.m + 255) / 256);
    const long long iters = tiles * (ka.k / 128);
    // Worth it only when whole tiles would keep at most 40 % of the CUs busy
    // in their one round, with at least 16 128-K groups per workgroup
    // (measured on MI355X, bf16 C, best of 3 x 100 calls: 80 tiles on 256
    // CUs, K = 8192: 103.1 -> 83.9 us; 99 tiles: 80.0 -> 78.1; 112 tiles:
    // 80.6 -> 81.3; 144 tiles, K = 7168: 94.7 -> 96.9; 448 tiles: 72.3 ->
    // 82.6): the partial tiles' device-coherent traffic and the last
    // arrival's sum cost about as much as a third of the CUs idling.
    if (tiles * 5 > 2ll * nwg || iters < 16ll * nwg)
        return 0;
    return nwg;
}

// One arrival counter per tile, then the misuse word, rounded to 256 bytes.
size_t bs_sk_counter_bytes(const ga_opus_gemm_kargs& ka)
{
    const size_t tiles = (size_t)((ka.n + 255) / 256) * ((ka.m + 255) / 256);
    return ((tiles + 1) * 4 + 255) / 256 * 256;
}

size_t bs_sk_workspace_bytes(const ga_opus_gemm_kargs& ka, int nwg)
{
    return nwg > 0 ? bs_sk_counter_bytes(ka) + (size_t)2 * nwg * kSkSlotFloats * 4 : 0;
}

void launch_bs_pp_sk(const ga_opus_gemm_kargs& ka, int mode, int out_dtype, int nwg, void* ws,
                     hipStream_t stream)
{
    const bool f32 = out_dtype == GA_DTYPE_F32;
    if (mode == PS_GROUP128)
        f32 ? launch_bs_pp_sk_t<PS_GROUP128, GA_DTYPE_F32>(ka, nwg, ws, stream)
            : launch_bs_pp_sk_t<PS_GROUP128, GA_DTYPE_BF16>(ka, nwg, ws, stream);
    else if (mode == PS_GROUP1)
        f32 ? launch_bs_pp_sk_t<PS_GROUP1, GA_DTYPE_F32>(ka, nwg, ws, stream)
            : launch_bs_pp_sk_t<PS_GROUP1, GA_DTYPE_BF16>(ka, nwg, ws, stream);
    else
        f32 ? launch_bs_pp_sk_t<PS_TENSOR, GA_DTYPE_F32>(ka, nwg, ws, stream)
            : launch_bs_pp_sk_t<PS_TENSOR, GA_DTYPE_BF16>(ka, nwg, ws, stream);
}

} // namespace ga

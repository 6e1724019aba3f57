// quant.hip -- FP8 quantisers and device-side layout shuffles (gfx950).
//
// The step before the GEMM: bf16/fp32 activations or weights -> E4M3 codes
// plus scales, in the three scale modes of the library:
//   * MX 1x32:        E8M0 exponent per 32 K-elements (rule selectable)
//   * DeepSeek 1x128: fp32 s = amax/448 per 128 K-elements of a row,
//                     written transposed [K/128, rows] (opus SFA layout)
//   * DeepSeek 128x128: fp32 s per 128x128 tile [ceil(rows/128), K/128]
//   * per-tensor:     one fp32 s = amax/448
// Encoding is the exact integer RNE/saturating E4M3 encode of ga_device.hpp;
// x/s uses IEEE fp32 division (correctly rounded; built without fast-math).
// All kernels are HBM streaming kernels: 16-byte loads per lane (8-byte for
// bf16 rows whose stride does not allow 16), several independent loads in
// flight per lane, cross-lane amax over DPP row exchanges, coalesced stores.
#include "ga_device.hpp"
#include "ga_internal.hpp"

namespace ga {

__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    return a | (b << 8) | (c << 16) | (d << 24);
}

// Up to 8 elements per lane from one 16-byte (f32: 4) or 8/16-byte (bf16: 4/8)
// load; lanes that are out of range read zeros.
template <int IN, int EPL>
__device__ __forceinline__ void load_elems(const void* x, size_t idx, bool ok, float (&v)[EPL])
{
#pragma unroll
    for (int j = 0; j < EPL; j++)
        v[j] = 0.0f;
    if (!ok)
        return;
    if constexpr (IN == GA_IN_F32) {
        static_assert(EPL == 4, "f32: 4 elements per 16-byte load");
        const v4f t = *(const v4f*)((const float*)x + idx);
#pragma unroll
        for (int j = 0; j < 4; j++)
            v[j] = t[j];
    } else if constexpr (EPL == 8) {
        const v4i t = *(const v4i*)((const uint16_t*)x + idx);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[2 * j] = bf16_to_f32((uint16_t)((uint32_t)t[j] & 0xFFFF));
            v[2 * j + 1] = bf16_to_f32((uint16_t)((uint32_t)t[j] >> 16));
        }
    } else {
        const uint2 t = *(const uint2*)((const uint16_t*)x + idx);
        v[0] = bf16_to_f32((uint16_t)(t.x & 0xFFFF));
        v[1] = bf16_to_f32((uint16_t)(t.x >> 16));
        v[2] = bf16_to_f32((uint16_t)(t.y & 0xFFFF));
        v[3] = bf16_to_f32((uint16_t)(t.y >> 16));
    }
}

// Block maxima of |x| are taken on the bit patterns: for x >= 0 the IEEE bit
// order is the value order, and every NaN (quiet or signalling) maps to 0, so
// the maximum ignores NaNs exactly as the CPU reference's `a > amax` scan
// does (a float max would turn a signalling NaN into a NaN result).
__device__ __forceinline__ uint32_t abs_key(float x)
{
    const uint32_t u = __float_as_uint(x) & 0x7FFFFFFFu;
    return u > 0x7F800000u ? 0u : u;
}

template <int EPL>
__device__ __forceinline__ uint32_t amax_n(const float (&v)[EPL])
{
    uint32_t a = abs_key(v[0]);
#pragma unroll
    for (int j = 1; j < EPL; j++)
        a = max(a, abs_key(v[j]));
    return a;
}

// Maximum over aligned groups of W lanes (W = 4, 8, 16, 32). Inside a 16-lane
// row the exchange uses DPP (quad_perm xor 1 and xor 2, then the half- and
// full-row mirrors, which pair each 4- / 8-lane group with its neighbour once
// every lane of a group holds the group's max); across rows one swizzle.
template <int W>
__device__ __forceinline__ uint32_t group_max_dpp(uint32_t a)
{
    auto dpp = [](uint32_t v, auto ctrl) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, decltype(ctrl)::value, 0xF, 0xF,
                                                     false);
    };
    a = max(a, dpp(a, std::integral_constant<int, 0xB1>{})); // quad_perm(1,0,3,2)
    a = max(a, dpp(a, std::integral_constant<int, 0x4E>{})); // quad_perm(2,3,0,1)
    if constexpr (W >= 8)
        a = max(a, dpp(a, std::integral_constant<int, 0x141>{})); // row_half_mirror
    if constexpr (W >= 16)
        a = max(a, dpp(a, std::integral_constant<int, 0x140>{})); // row_mirror
    if constexpr (W >= 32)
        a = max(a, (uint32_t)__shfl_xor((int)a, 16, 64));
    return a;
}

// Maximum of the plain keys bits & 0x7FFFFFFF: one instruction per element
// instead of abs_key's three. A NaN's key is above +inf's, so a maximum above
// 0x7F800000 means the block holds a NaN; only then (rare) is the
// NaN-ignoring maximum taken.
template <int EPL>
__device__ __forceinline__ uint32_t amax_raw(const float (&v)[EPL])
{
    uint32_t a = __float_as_uint(v[0]) & 0x7FFFFFFFu;
#pragma unroll
    for (int j = 1; j < EPL; j++)
        a = max(a, __float_as_uint(v[j]) & 0x7FFFFFFFu);
    return a;
}

// The NaN-ignoring maximum of |x| over aligned groups of W lanes. The
// recomputation is taken by the whole wave when any of its blocks holds a
// NaN (a ballot makes the branch uniform), so the lane exchanges always run
// with every lane active.
template <int W, int EPL>
__device__ __forceinline__ uint32_t block_amax(const float (&v)[EPL])
{
    uint32_t a = group_max_dpp<W>(amax_raw<EPL>(v));
    if (__builtin_amdgcn_ballot_w64(a > 0x7F800000u) != 0)
        a = group_max_dpp<W>(amax_n<EPL>(v));
    return a;
}

// ---- MX 1x32 (E4M3 or packed e2m1 codes) -------------------------------------
// A 1x32 block is LPB = 32/EPL lanes of EPL elements (16-byte loads where the
// layout allows); each lane handles U blocks, BPP = 256/LPB blocks apart, so U
// independent loads are in flight per lane before the first reduction.
// E5: E5M2 elements instead of E4M3 (FP4 false).
template <int IN, int EPL, bool FP4, int U, bool E5 = false>
__global__ __launch_bounds__(256) void quant_mx_kernel(const void* __restrict__ x, int rows,
                                                       int K, int ld_x, uint8_t* __restrict__ q,
                                                       int ld_q, uint8_t* __restrict__ s,
                                                       int ld_s, int rule)
{
    constexpr int LPB = 32 / EPL, BPP = 256 / LPB;
    const int nb = K / 32;
    const long long total = (long long)rows * nb;
    const int sub = threadIdx.x % LPB;
    const long long base = (long long)blockIdx.x * (BPP * U) + threadIdx.x / LPB;
    float v[U][EPL];
    int rr[U], bb[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const long long blk = base + (long long)u * BPP;
        ok[u] = blk < total;
        rr[u] = ok[u] ? (int)(blk / nb) : 0;
        bb[u] = ok[u] ? (int)(blk - (long long)rr[u] * nb) : 0;
        load_elems<IN, EPL>(x, (size_t)rr[u] * ld_x + bb[u] * 32 + sub * EPL, ok[u], v[u]);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        const float amax = __uint_as_float(block_amax<LPB, EPL>(v[u]));
        if (!ok[u])
            continue;
        const int e = FP4 ? mx4_scale_exp(amax, rule)
                          : (E5 ? mx5_scale_exp(amax, rule) : mx_scale_exp(amax, rule));
        uint8_t* qrow = q + (size_t)rr[u] * ld_q;
        if constexpr (FP4) {
            float t[EPL];
#pragma unroll
            for (int j = 0; j < EPL; j++)
                t[j] = ldexpf(v[u][j], -e);
            uint32_t w = e2m1_encode4(t[0], t[1], t[2], t[3]);
            if constexpr (EPL == 8)
                w |= e2m1_encode4(t[4], t[5], t[6], t[7]) << 16;
            if constexpr (EPL == 8)
                *(uint32_t*)(qrow + bb[u] * 16 + sub * 4) = w;
            else
                *(uint16_t*)(qrow + bb[u] * 16 + sub * 2) = (uint16_t)w;
        } else {
            float t[EPL];
#pragma unroll
            for (int j = 0; j < EPL; j++)
                t[j] = ldexpf(v[u][j], -e);
            auto enc4 = [](float p, float q_, float r, float w) {
                return E5 ? e5m2_encode4(p, q_, r, w) : e4m3_encode4(p, q_, r, w);
            };
            if constexpr (EPL == 8) {
                uint2 w;
                w.x = enc4(t[0], t[1], t[2], t[3]);
                w.y = enc4(t[4], t[5], t[6], t[7]);
                *(uint2*)(qrow + bb[u] * 32 + sub * 8) = w;
            } else {
                *(uint32_t*)(qrow + bb[u] * 32 + sub * 4) = enc4(t[0], t[1], t[2], t[3]);
            }
        }
        if (sub == 0)
            s[(size_t)rr[u] * ld_s + bb[u]] = (uint8_t)(e + 127);
    }
}

// ---- DeepSeek 1x128 -----------------------------------------------------------
__device__ __forceinline__ float ds_scale(float amax) { return amax > 0.0f ? amax / 448.0f : 1.0f; }

// x / s for the elements that share one scale s, exact wherever the quotient
// decides an E4M3 code. For finite s >= 2^-64: the reciprocal r = 1/s
// (correctly rounded, once per scale), q0 = x*r, and two corrections
// q <- q + (x - q*s)*r, each residual and product one FMA. With r within
// half an ulp of 1/s and q within one ulp of x/s, the corrected quotient is
// x/s correctly rounded (Markstein's theorem; the first correction brings
// q0, within 1.5 ulp, inside one ulp). The residuals stay normal numbers for
// every x whose quotient is at least 2^-12 (|x| >= 2^-76), the range in which
// the fp32 quotient can change an E4M3 code; smaller quotients come out
// below 2^-11 with x's sign, and such values encode to the signed zero either
// way. The sign is taken from x, so -0 stays -0. tests/scale_div_check.c
// restates this arithmetic on the CPU and compares it with IEEE division
// (every bf16 x and random fp32 x under scales over the whole range; 1.4e9
// quotients without a mismatch). Other scales (subnormal, infinite) divide. Five VALU instructions per element instead
// of the IEEE division's ten; the choice is made once per scale.
struct ScaleDiv {
    float s, r;
    bool fast;
    __device__ __forceinline__ explicit ScaleDiv(float s_)
        : s(s_), r(1.0f / s_), fast(s_ >= 0x1p-64f && s_ <= 3.40282347e38f)
    {
    }
    template <int N>
    __device__ __forceinline__ void div(const float (&v)[N], float (&t)[N]) const
    {
        if (fast) {
#pragma unroll
            for (int j = 0; j < N; j++) {
                const float q0 = v[j] * r;
                const float q1 = fmaf(fmaf(-q0, s, v[j]), r, q0);
                t[j] = copysignf(fmaf(fmaf(-q1, s, v[j]), r, q1), v[j]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < N; j++)
                t[j] = v[j] / s;
        }
    }
};

// A 1x128 group is LPB = 128/EPL lanes; U groups per lane as above.
template <int IN, int EPL, int U>
__global__ __launch_bounds__(256) void quant_1x128_kernel(const void* __restrict__ x, int rows,
                                                          int K, int ld_x, uint8_t* __restrict__ q,
                                                          int ld_q, float* __restrict__ sfa,
                                                          int ld_s)
{
    constexpr int LPB = 128 / EPL, BPP = 256 / LPB;
    const int ng = K / 128;
    const long long total = (long long)rows * ng;
    const int sub = threadIdx.x % LPB;
    const long long base = (long long)blockIdx.x * (BPP * U) + threadIdx.x / LPB;
    float v[U][EPL];
    int rr[U], gg[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const long long blk = base + (long long)u * BPP;
        ok[u] = blk < total;
        rr[u] = ok[u] ? (int)(blk / ng) : 0;
        gg[u] = ok[u] ? (int)(blk - (long long)rr[u] * ng) : 0;
        load_elems<IN, EPL>(x, (size_t)rr[u] * ld_x + gg[u] * 128 + sub * EPL, ok[u], v[u]);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        const float amax = __uint_as_float(block_amax<LPB, EPL>(v[u]));
        if (!ok[u])
            continue;
        const float sc = ds_scale(amax);
        float t[EPL];
        ScaleDiv(sc).div(v[u], t);
        uint8_t* dst = q + (size_t)rr[u] * ld_q + gg[u] * 128 + sub * EPL;
        if constexpr (EPL == 8) {
            uint2 w;
            w.x = e4m3_encode4(t[0], t[1], t[2], t[3]);
            w.y = e4m3_encode4(t[4], t[5], t[6], t[7]);
            *(uint2*)dst = w;
        } else {
            *(uint32_t*)dst = e4m3_encode4(t[0], t[1], t[2], t[3]);
        }
        if (sub == 0)
            sfa[(size_t)gg[u] * ld_s + rr[u]] = sc;
    }
}

// ---- DeepSeek 128x128: one workgroup per tile ----------------------------------
// The tile is read once into registers (32 values per lane with 512 threads:
// 8 / 4 loads in flight for fp32 / bf16), reduced in the workgroup, then
// quantised from registers. Measured on MI355X at 8192x8192 against 256
// threads (fraction of 8 TB/s): fp32 0.72-0.73 -> 0.78, bf16 0.63 -> 0.72.
constexpr int kTileThreads = 512;

template <int IN, int EPL>
__global__ __launch_bounds__(kTileThreads) void quant_128x128_kernel(
    const void* __restrict__ x, int rows, int K, int ld_x, uint8_t* __restrict__ q, int ld_q,
    float* __restrict__ sfb, int ld_s)
{
    constexpr int LPR = 128 / EPL;          // lanes per tile row
    constexpr int RPP = kTileThreads / LPR; // rows per pass
    constexpr int NP = 128 / RPP;           // passes
    __shared__ uint32_t wmax[kTileThreads / 64];
    const int g = blockIdx.x, rb = blockIdx.y;
    const int tid = threadIdx.x;
    const int col = (tid % LPR) * EPL, r_lo = tid / LPR;
    float v[NP][EPL];
    uint32_t amax = 0u;
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int r = rb * 128 + r_lo + i * RPP;
        load_elems<IN, EPL>(x, (size_t)r * ld_x + g * 128 + col, r < rows, v[i]);
    }
    // the tile's maximum over the plain keys; only a tile holding a NaN
    // (the maximum says so, the same in every wave) takes the NaN-ignoring one
    auto tile_max = [&](bool nan_free) {
        uint32_t a = 0u;
#pragma unroll
        for (int i = 0; i < NP; i++)
            a = max(a, nan_free ? amax_n<EPL>(v[i]) : amax_raw<EPL>(v[i]));
        a = group_max_dpp<32>(a);
        a = max(a, (uint32_t)__shfl_xor((int)a, 32, 64));
        if ((tid & 63) == 0)
            wmax[tid >> 6] = a;
        __syncthreads();
        uint32_t m = wmax[0];
#pragma unroll
        for (int w = 1; w < kTileThreads / 64; w++)
            m = max(m, wmax[w]);
        return m;
    };
    amax = tile_max(false);
    if (amax > 0x7F800000u) {
        __syncthreads(); // every wave has read wmax before it is written again
        amax = tile_max(true);
    }
    const float sc = ds_scale(__uint_as_float(amax));
    const ScaleDiv d(sc);
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const int r = rb * 128 + r_lo + i * RPP;
        if (r >= rows)
            continue;
        float t[EPL];
        d.div(v[i], t);
        uint8_t* dst = q + (size_t)r * ld_q + g * 128 + col;
        if constexpr (EPL == 8) {
            uint2 w;
            w.x = e4m3_encode4(t[0], t[1], t[2], t[3]);
            w.y = e4m3_encode4(t[4], t[5], t[6], t[7]);
            *(uint2*)dst = w;
        } else {
            *(uint32_t*)dst = e4m3_encode4(t[0], t[1], t[2], t[3]);
        }
    }
    if (tid == 0)
        sfb[(size_t)rb * ld_s + g] = sc;
}

// ---- per-tensor: zero, amax (atomicMax on the bits of |x|), quantise --------
// Both passes stream x with U loads of 16 bytes (f32) or 8 bytes (bf16) in
// flight per lane; the scalar tail (n % 4) is handled by block 0.
constexpr int kTensorU = 4;

__global__ void zero_u32_kernel(uint32_t* p) { *p = 0u; }

template <int IN>
__global__ __launch_bounds__(256) void amax_kernel(const void* __restrict__ x, size_t n,
                                                   uint32_t* __restrict__ amax_bits)
{
    uint32_t a = 0u;
    const size_t n4 = n / 4;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i0 = (size_t)blockIdx.x * 256 + threadIdx.x; i0 < n4; i0 += stride * kTensorU) {
        float v[kTensorU][4];
#pragma unroll
        for (int u = 0; u < kTensorU; u++) {
            const size_t i = i0 + u * stride;
            load_elems<IN, 4>(x, i * 4, i < n4, v[u]);
        }
#pragma unroll
        for (int u = 0; u < kTensorU; u++)
            a = max(a, amax_n<4>(v[u]));
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        size_t i = n4 * 4 + threadIdx.x;
        float v = IN == GA_IN_F32 ? ((const float*)x)[i] : bf16_to_f32(((const uint16_t*)x)[i]);
        a = max(a, abs_key(v));
    }
    a = group_max_dpp<32>(a);
    a = max(a, (uint32_t)__shfl_xor((int)a, 32, 64));
    if ((threadIdx.x & 63) == 0 && a > 0u)
        atomicMax(amax_bits, a);
}

template <int IN>
__global__ __launch_bounds__(256) void quant_tensor_kernel(const void* __restrict__ x, size_t n,
                                                           const uint32_t* __restrict__ amax_bits,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ scale)
{
    const float sc = ds_scale(__uint_as_float(*amax_bits));
    const ScaleDiv d(sc);
    if (blockIdx.x == 0 && threadIdx.x == 0)
        *scale = sc;
    const size_t n4 = n / 4;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i0 = (size_t)blockIdx.x * 256 + threadIdx.x; i0 < n4; i0 += stride * kTensorU) {
        float v[kTensorU][4];
#pragma unroll
        for (int u = 0; u < kTensorU; u++) {
            const size_t i = i0 + u * stride;
            load_elems<IN, 4>(x, i * 4, i < n4, v[u]);
        }
#pragma unroll
        for (int u = 0; u < kTensorU; u++) {
            const size_t i = i0 + u * stride;
            if (i < n4) {
                float t[4];
                d.div(v[u], t);
                *(uint32_t*)(q + i * 4) = e4m3_encode4(t[0], t[1], t[2], t[3]);
            }
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        size_t i = n4 * 4 + threadIdx.x;
        float v = IN == GA_IN_F32 ? ((const float*)x)[i] : bf16_to_f32(((const uint16_t*)x)[i]);
        const float vv[1] = {v};
        float t[1];
        d.div(vv, t);
        q[i] = (uint8_t)e4m3_encode(t[0]);
    }
}

// ---- device shuffles ----------------------------------------------------------
// One lane per 16-byte destination run of shuffle_weight(layout=(16,16)).
__global__ __launch_bounds__(256) void shuffle_weight_kernel(const uint8_t* __restrict__ src,
                                                             uint8_t* __restrict__ dst, int N,
                                                             int Kp)
{
    const long long run = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long nruns = (long long)N * Kp / 16;
    if (run >= nruns)
        return;
    const int nk = Kp / 32;
    const int n1 = (int)(run & 15);
    const long long t = run >> 4; // ((n0 * nk + k0) * 2 + k1)
    const int k1 = (int)(t & 1);
    const long long t2 = t >> 1;
    const int k0 = (int)(t2 % nk);
    const long long n0 = t2 / nk;
    const v4i v = *(const v4i*)(src + (size_t)(n0 * 16 + n1) * Kp + k0 * 32 + k1 * 16);
    *(v4i*)(dst + (size_t)run * 16) = v;
}

// One lane per destination dword of shuffle_scale: dword (d5, d2) of the
// 256-byte block (d0, d3) holds bytes (d4, d1) = (0,0), (0,1), (1,0), (1,1).
__global__ __launch_bounds__(256) void shuffle_scale_kernel(const uint8_t* __restrict__ src,
                                                            uint8_t* __restrict__ dst, int rows,
                                                            int cols, int sm, int sn)
{
    const long long w = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long nw = (long long)sm * sn / 4;
    if (w >= nw)
        return;
    const int n3 = sn / 8;
    const int in_blk = (int)(w & 63);
    const long long blk = w >> 6; // d0 * n3 + d3
    const int d3 = (int)(blk % n3);
    const int d0 = (int)(blk / n3);
    const int d5 = in_blk >> 4, d2 = in_blk & 15;
    uint32_t out = 0;
#pragma unroll
    for (int d4 = 0; d4 < 2; d4++)
#pragma unroll
        for (int d1 = 0; d1 < 2; d1++) {
            const int r = d0 * 32 + d1 * 16 + d2;
            const int c = d3 * 8 + d4 * 4 + d5;
            const uint32_t v = (r < rows && c < cols) ? src[(size_t)r * cols + c] : 0x7Fu;
            out |= v << (8 * (d4 * 2 + d1));
        }
    *(uint32_t*)(dst + (size_t)w * 4) = out;
}

static inline unsigned grid1d(long long work, int per_block)
{
    return (unsigned)((work + per_block - 1) / per_block);
}

} // namespace ga

using namespace ga;

#define GA_DISPATCH_IN(in_dtype, KERNEL, ...)                                      \
    do {                                                                           \
        if ((in_dtype) == GA_IN_F32)                                               \
            hipLaunchKernelGGL(KERNEL<GA_IN_F32>, __VA_ARGS__);                    \
        else                                                                       \
            hipLaunchKernelGGL(KERNEL<GA_IN_BF16>, __VA_ARGS__);                   \
    } while (0)

// 1x32 / 1x128 blocks per lane: two for fp32 and 8-byte bf16 loads, one for
// 16-byte bf16 loads (16-32 bytes in flight per lane). Measured on MI355X at
// 8192x8192 (fraction of 8 TB/s, 4 blocks -> this): MX E4M3 fp32 0.70 -> 0.73,
// bf16 0.62 -> 0.71; e2m1 bf16 0.55 -> 0.63; 1x128 bf16 0.46 -> 0.51.
constexpr int kQU = 2;
constexpr int kQUWide = 1;

// bf16 inputs use 16-byte loads (8 elements per lane) when the row stride and
// base allow it and the codes' stores stay aligned (store_align: bytes per
// lane store); otherwise 8-byte loads.
static bool bf16_wide(int in_dtype, const void* x, int ld_x, const void* q, int ld_q,
                      int store_align)
{
    return in_dtype == GA_IN_BF16 && ld_x % 8 == 0 && ((uintptr_t)x & 15) == 0 &&
           ld_q % store_align == 0 && ((uintptr_t)q % store_align) == 0;
}

template <bool FP4, bool E5 = false>
static void launch_quant_mx(int in_dtype, bool wide, long long blocks, hipStream_t st,
                            const void* x, int rows, int K, int ld_x, uint8_t* q, int ld_q,
                            uint8_t* s, int ld_s, int rule)
{
    const int epl = in_dtype == GA_IN_F32 ? 4 : (wide ? 8 : 4);
    const int u = (in_dtype != GA_IN_F32 && wide) ? kQUWide : kQU;
    const unsigned grid = grid1d(blocks, (256 / (32 / epl)) * u);
    if (in_dtype == GA_IN_F32)
        hipLaunchKernelGGL((quant_mx_kernel<GA_IN_F32, 4, FP4, kQU, E5>), dim3(grid), dim3(256), 0,
                           st, x, rows, K, ld_x, q, ld_q, s, ld_s, rule);
    else if (wide)
        hipLaunchKernelGGL((quant_mx_kernel<GA_IN_BF16, 8, FP4, kQUWide, E5>), dim3(grid),
                           dim3(256), 0, st, x, rows, K, ld_x, q, ld_q, s, ld_s, rule);
    else
        hipLaunchKernelGGL((quant_mx_kernel<GA_IN_BF16, 4, FP4, kQU, E5>), dim3(grid), dim3(256),
                           0, st, x, rows, K, ld_x, q, ld_q, s, ld_s, rule);
}

static ga_status check_in(int in_dtype)
{
    if (in_dtype != GA_IN_F32 && in_dtype != GA_IN_BF16)
        return fail(GA_ERR_ARG, "input dtype must be GA_IN_F32 or GA_IN_BF16");
    return GA_OK;
}

extern "C" {

ga_status ga_quant_mx8(const void* x, int in_dtype, int rows, int K, int ld_x, void* q, int ld_q,
                       void* scales, int ld_s, int scale_rule, int fmt, void* stream)
{
    if (check_in(in_dtype) != GA_OK)
        return GA_ERR_ARG;
    if (!x || !q || !scales || rows <= 0 || K <= 0 || ld_x < K || ld_q < K || ld_s < K / 32 ||
        scale_rule < 0 || scale_rule > 2 || fmt < 0 || fmt > 1)
        return fail(GA_ERR_ARG, "quant_mx8: bad argument (fmt 0 E4M3 or 1 E5M2)");
    if (K % 32 || ld_x % 4 || ld_q % 4)
        return fail(GA_ERR_SHAPE, "quant_mx8: K %% 32, ld_x %% 4 and ld_q %% 4 must be 0");
    long long blocks = (long long)rows * (K / 32);
    const bool wide = bf16_wide(in_dtype, x, ld_x, q, ld_q, 8);
    if (fmt == 1)
        launch_quant_mx<false, true>(in_dtype, wide, blocks, (hipStream_t)stream, x, rows, K,
                                     ld_x, (uint8_t*)q, ld_q, (uint8_t*)scales, ld_s, scale_rule);
    else
        launch_quant_mx<false>(in_dtype, wide, blocks, (hipStream_t)stream, x, rows, K, ld_x,
                               (uint8_t*)q, ld_q, (uint8_t*)scales, ld_s, scale_rule);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

ga_status ga_quant_mxfp8(const void* x, int in_dtype, int rows, int K, int ld_x, void* q,
                         int ld_q, void* scales, int ld_s, int scale_rule, void* stream)
{
    return ga_quant_mx8(x, in_dtype, rows, K, ld_x, q, ld_q, scales, ld_s, scale_rule, 0, stream);
}

ga_status ga_quant_mxfp4(const void* x, int in_dtype, int rows, int K, int ld_x, void* q,
                         int ld_q, void* scales, int ld_s, int scale_rule, void* stream)
{
    if (check_in(in_dtype) != GA_OK)
        return GA_ERR_ARG;
    if (!x || !q || !scales || rows <= 0 || K <= 0 || ld_x < K || ld_q < K / 2 ||
        ld_s < K / 32 || scale_rule < 0 || scale_rule > 2)
        return fail(GA_ERR_ARG, "quant_mxfp4: bad argument");
    if (K % 32 || ld_x % 4 || ld_q % 2)
        return fail(GA_ERR_SHAPE, "quant_mxfp4: K %% 32, ld_x %% 4 and ld_q %% 2 must be 0");
    long long blocks = (long long)rows * (K / 32);
    launch_quant_mx<true>(in_dtype, bf16_wide(in_dtype, x, ld_x, q, ld_q, 4), blocks,
                          (hipStream_t)stream, x, rows, K, ld_x, (uint8_t*)q, ld_q,
                          (uint8_t*)scales, ld_s, scale_rule);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

ga_status ga_quant_fp8_1x128(const void* x, int in_dtype, int rows, int K, int ld_x, void* q,
                             int ld_q, float* sfa, int ld_s, void* stream)
{
    if (check_in(in_dtype) != GA_OK)
        return GA_ERR_ARG;
    if (!x || !q || !sfa || rows <= 0 || K <= 0 || ld_x < K || ld_q < K || ld_s < rows)
        return fail(GA_ERR_ARG, "quant_fp8_1x128: bad argument");
    if (K % 128 || ld_x % 4 || ld_q % 4)
        return fail(GA_ERR_SHAPE, "quant_fp8_1x128: K %% 128, ld_x %% 4 and ld_q %% 4 must be 0");
    long long blocks = (long long)rows * (K / 128);
    hipStream_t st = (hipStream_t)stream;
    if (in_dtype == GA_IN_F32)
        hipLaunchKernelGGL((quant_1x128_kernel<GA_IN_F32, 4, kQU>), dim3(grid1d(blocks, 8 * kQU)),
                           dim3(256), 0, st, x, rows, K, ld_x, (uint8_t*)q, ld_q, sfa, ld_s);
    else if (bf16_wide(in_dtype, x, ld_x, q, ld_q, 8))
        hipLaunchKernelGGL((quant_1x128_kernel<GA_IN_BF16, 8, kQUWide>),
                           dim3(grid1d(blocks, 16 * kQUWide)), dim3(256), 0, st, x, rows, K, ld_x,
                           (uint8_t*)q, ld_q, sfa, ld_s);
    else
        hipLaunchKernelGGL((quant_1x128_kernel<GA_IN_BF16, 4, kQU>), dim3(grid1d(blocks, 8 * kQU)),
                           dim3(256), 0, st, x, rows, K, ld_x, (uint8_t*)q, ld_q, sfa, ld_s);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

ga_status ga_quant_fp8_128x128(const void* x, int in_dtype, int rows, int K, int ld_x, void* q,
                               int ld_q, float* sfb, int ld_s, void* stream)
{
    if (check_in(in_dtype) != GA_OK)
        return GA_ERR_ARG;
    if (!x || !q || !sfb || rows <= 0 || K <= 0 || ld_x < K || ld_q < K || ld_s < K / 128)
        return fail(GA_ERR_ARG, "quant_fp8_128x128: bad argument");
    if (K % 128 || ld_x % 4 || ld_q % 4)
        return fail(GA_ERR_SHAPE, "quant_fp8_128x128: K %% 128, ld_x %% 4 and ld_q %% 4 must be 0");
    dim3 grid(K / 128, (rows + 127) / 128);
    hipStream_t st = (hipStream_t)stream;
    if (in_dtype == GA_IN_F32)
        hipLaunchKernelGGL((quant_128x128_kernel<GA_IN_F32, 4>), grid, dim3(kTileThreads), 0, st, x, rows,
                           K, ld_x, (uint8_t*)q, ld_q, sfb, ld_s);
    else if (bf16_wide(in_dtype, x, ld_x, q, ld_q, 8))
        hipLaunchKernelGGL((quant_128x128_kernel<GA_IN_BF16, 8>), grid, dim3(kTileThreads), 0, st, x, rows,
                           K, ld_x, (uint8_t*)q, ld_q, sfb, ld_s);
    else
        hipLaunchKernelGGL((quant_128x128_kernel<GA_IN_BF16, 4>), grid, dim3(kTileThreads), 0, st, x, rows,
                           K, ld_x, (uint8_t*)q, ld_q, sfb, ld_s);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

ga_status ga_quant_fp8_per_tensor(const void* x, int in_dtype, size_t n, void* q, float* scale,
                                  void* amax_ws, void* stream)
{
    if (check_in(in_dtype) != GA_OK)
        return GA_ERR_ARG;
    if (!x || !q || !scale || !amax_ws || n == 0)
        return fail(GA_ERR_ARG, "quant_fp8_per_tensor: bad argument");
    hipStream_t s = (hipStream_t)stream;
    const unsigned blocks = (unsigned)std::min<long long>(grid1d((long long)(n / 4) + 1, 256), 2048);
    hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(1), 0, s, (uint32_t*)amax_ws);
    GA_DISPATCH_IN(in_dtype, amax_kernel, dim3(blocks), dim3(256), 0, s, x, n,
                   (uint32_t*)amax_ws);
    GA_DISPATCH_IN(in_dtype, quant_tensor_kernel, dim3(blocks), dim3(256), 0, s, x, n,
                   (const uint32_t*)amax_ws, (uint8_t*)q, scale);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

ga_status ga_shuffle_weight_16x16_device(const void* src, void* dst, int N, int Kp, void* stream)
{
    if (!src || !dst || N <= 0 || Kp <= 0)
        return fail(GA_ERR_ARG, "shuffle_weight_16x16_device: bad argument");
    if (N % 16 || Kp % 32)
        return fail(GA_ERR_SHAPE, "shuffle_weight_16x16 needs N %% 16 == 0 and Kp %% 32 == 0");
    long long runs = (long long)N * Kp / 16;
    hipLaunchKernelGGL(shuffle_weight_kernel, dim3(grid1d(runs, 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint8_t*)src, (uint8_t*)dst, N, Kp);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

ga_status ga_shuffle_scale_device(const void* src, void* dst, int rows, int cols, int sm, int sn,
                                  void* stream)
{
    if (!src || !dst || rows < 0 || cols < 0 || sm <= 0 || sn <= 0)
        return fail(GA_ERR_ARG, "shuffle_scale_device: bad argument");
    if (sm % 32 || sn % 8 || rows > sm || cols > sn)
        return fail(GA_ERR_SHAPE, "shuffle_scale needs sm %% 32 == 0, sn %% 8 == 0, rows <= sm, "
                                  "cols <= sn");
    long long words = (long long)sm * sn / 4;
    hipLaunchKernelGGL(shuffle_scale_kernel, dim3(grid1d(words, 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint8_t*)src, (uint8_t*)dst, rows, cols, sm,
                       sn);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

} // extern "C"

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
// All kernels are HBM streaming kernels: 16-byte (fp32) or 8-byte (bf16)
// loads per lane, cross-lane amax with shuffles, coalesced code stores.
#include "ga_device.hpp"
#include "ga_internal.hpp"

namespace ga {

template <int IN>
__device__ __forceinline__ void load4(const void* x, size_t idx, float (&v)[4])
{
    if (IN == GA_IN_F32) {
        v4f t = *(const v4f*)((const float*)x + idx);
        v[0] = t[0];
        v[1] = t[1];
        v[2] = t[2];
        v[3] = t[3];
    } else {
        uint2 t = *(const uint2*)((const uint16_t*)x + idx);
        v[0] = bf16_to_f32((uint16_t)(t.x & 0xFFFF));
        v[1] = bf16_to_f32((uint16_t)(t.x >> 16));
        v[2] = bf16_to_f32((uint16_t)(t.y & 0xFFFF));
        v[3] = bf16_to_f32((uint16_t)(t.y >> 16));
    }
}

// NaN-ignoring max of |v| (fmaxf returns the non-NaN operand).
__device__ __forceinline__ float amax4(const float (&v)[4])
{
    return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
}

template <int WIDTH>
__device__ __forceinline__ float group_max(float a)
{
#pragma unroll
    for (int o = 1; o < WIDTH; o <<= 1)
        a = fmaxf(a, __shfl_xor(a, o, 64));
    return a;
}

__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    return a | (b << 8) | (c << 16) | (d << 24);
}

// ---- MX 1x32: 8 lanes per block, 4 elements per lane -----------------------
template <int IN>
__global__ __launch_bounds__(256) void quant_mx_kernel(const void* __restrict__ x, int rows,
                                                       int K, int ld_x, uint8_t* __restrict__ q,
                                                       int ld_q, uint8_t* __restrict__ s,
                                                       int ld_s, int rule)
{
    const int nb = K / 32;
    const long long blk = (long long)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int sub = threadIdx.x & 7;
    const bool valid = blk < (long long)rows * nb;
    const int r = valid ? (int)(blk / nb) : 0;
    const int b = valid ? (int)(blk - (long long)r * nb) : 0;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid)
        load4<IN>(x, (size_t)r * ld_x + b * 32 + sub * 4, v);
    const float amax = group_max<8>(amax4(v));
    if (!valid)
        return;
    const int e = mx_scale_exp(amax, rule);
    uint32_t c[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        c[j] = e4m3_encode(ldexpf(v[j], -e));
    *(uint32_t*)(q + (size_t)r * ld_q + b * 32 + sub * 4) = pack4(c[0], c[1], c[2], c[3]);
    if (sub == 0)
        s[(size_t)r * ld_s + b] = (uint8_t)(e + 127);
}

// ---- MXFP4: same blocking, e2m1 codes packed two per byte (low nibble = even
// element), 16 bytes per 1x32 block ------------------------------------------
template <int IN>
__global__ __launch_bounds__(256) void quant_mx4_kernel(const void* __restrict__ x, int rows,
                                                        int K, int ld_x, uint8_t* __restrict__ q,
                                                        int ld_q, uint8_t* __restrict__ s,
                                                        int ld_s, int rule)
{
    const int nb = K / 32;
    const long long blk = (long long)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int sub = threadIdx.x & 7;
    const bool valid = blk < (long long)rows * nb;
    const int r = valid ? (int)(blk / nb) : 0;
    const int b = valid ? (int)(blk - (long long)r * nb) : 0;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid)
        load4<IN>(x, (size_t)r * ld_x + b * 32 + sub * 4, v);
    const float amax = group_max<8>(amax4(v));
    if (!valid)
        return;
    const int e = mx4_scale_exp(amax, rule);
    uint32_t c[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        c[j] = e2m1_encode(ldexpf(v[j], -e));
    *(uint16_t*)(q + (size_t)r * ld_q + b * 16 + sub * 2) =
        (uint16_t)(c[0] | (c[1] << 4) | (c[2] << 8) | (c[3] << 12));
    if (sub == 0)
        s[(size_t)r * ld_s + b] = (uint8_t)(e + 127);
}

// ---- DeepSeek 1x128: 32 lanes per block ------------------------------------
__device__ __forceinline__ float ds_scale(float amax) { return amax > 0.0f ? amax / 448.0f : 1.0f; }

template <int IN>
__global__ __launch_bounds__(256) void quant_1x128_kernel(const void* __restrict__ x, int rows,
                                                          int K, int ld_x, uint8_t* __restrict__ q,
                                                          int ld_q, float* __restrict__ sfa,
                                                          int ld_s)
{
    const int ng = K / 128;
    const long long blk = (long long)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int sub = threadIdx.x & 31;
    const bool valid = blk < (long long)rows * ng;
    const int r = valid ? (int)(blk / ng) : 0;
    const int g = valid ? (int)(blk - (long long)r * ng) : 0;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (valid)
        load4<IN>(x, (size_t)r * ld_x + g * 128 + sub * 4, v);
    const float amax = group_max<32>(amax4(v));
    if (!valid)
        return;
    const float sc = ds_scale(amax);
    uint32_t c[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        c[j] = e4m3_encode(v[j] / sc);
    *(uint32_t*)(q + (size_t)r * ld_q + g * 128 + sub * 4) = pack4(c[0], c[1], c[2], c[3]);
    if (sub == 0)
        sfa[(size_t)g * ld_s + r] = sc;
}

// ---- DeepSeek 128x128: one workgroup per tile -------------------------------
template <int IN>
__global__ __launch_bounds__(256) void quant_128x128_kernel(const void* __restrict__ x, int rows,
                                                            int K, int ld_x,
                                                            uint8_t* __restrict__ q, int ld_q,
                                                            float* __restrict__ sfb, int ld_s)
{
    __shared__ float wmax[4];
    const int g = blockIdx.x, rb = blockIdx.y;
    const int tid = threadIdx.x;
    // 32 lanes span the 128 columns (4 each); 8 row slots, 16 rows per slot.
    const int col = (tid & 31) * 4, r_lo = tid >> 5;
    float amax = 0.0f;
    for (int i = 0; i < 16; i++) {
        const int r = rb * 128 + r_lo + i * 8;
        if (r < rows) {
            float v[4];
            load4<IN>(x, (size_t)r * ld_x + g * 128 + col, v);
            amax = fmaxf(amax, amax4(v));
        }
    }
    amax = group_max<64>(amax);
    if ((tid & 63) == 0)
        wmax[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float sc = ds_scale(amax);
    for (int i = 0; i < 16; i++) {
        const int r = rb * 128 + r_lo + i * 8;
        if (r < rows) {
            float v[4];
            load4<IN>(x, (size_t)r * ld_x + g * 128 + col, v);
            uint32_t c[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                c[j] = e4m3_encode(v[j] / sc);
            *(uint32_t*)(q + (size_t)r * ld_q + g * 128 + col) = pack4(c[0], c[1], c[2], c[3]);
        }
    }
    if (tid == 0)
        sfb[(size_t)rb * ld_s + g] = sc;
}

// ---- per-tensor: zero, amax (atomicMax on the bits of |x|), quantise --------
__global__ void zero_u32_kernel(uint32_t* p) { *p = 0u; }

template <int IN>
__global__ __launch_bounds__(256) void amax_kernel(const void* __restrict__ x, size_t n,
                                                   uint32_t* __restrict__ amax_bits)
{
    float a = 0.0f;
    const size_t n4 = n / 4;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        float v[4];
        load4<IN>(x, i * 4, v);
        a = fmaxf(a, amax4(v));
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        size_t i = n4 * 4 + threadIdx.x;
        float v = IN == GA_IN_F32 ? ((const float*)x)[i] : bf16_to_f32(((const uint16_t*)x)[i]);
        a = fmaxf(a, fabsf(v));
    }
    a = group_max<64>(a);
    if ((threadIdx.x & 63) == 0 && a > 0.0f)
        atomicMax(amax_bits, __float_as_uint(a));
}

template <int IN>
__global__ __launch_bounds__(256) void quant_tensor_kernel(const void* __restrict__ x, size_t n,
                                                           const uint32_t* __restrict__ amax_bits,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ scale)
{
    const float sc = ds_scale(__uint_as_float(*amax_bits));
    if (blockIdx.x == 0 && threadIdx.x == 0)
        *scale = sc;
    const size_t n4 = n / 4;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        float v[4];
        load4<IN>(x, i * 4, v);
        *(uint32_t*)(q + i * 4) = pack4(e4m3_encode(v[0] / sc), e4m3_encode(v[1] / sc),
                                        e4m3_encode(v[2] / sc), e4m3_encode(v[3] / sc));
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        size_t i = n4 * 4 + threadIdx.x;
        float v = IN == GA_IN_F32 ? ((const float*)x)[i] : bf16_to_f32(((const uint16_t*)x)[i]);
        q[i] = (uint8_t)e4m3_encode(v / sc);
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

static ga_status check_in(int in_dtype)
{
    if (in_dtype != GA_IN_F32 && in_dtype != GA_IN_BF16)
        return fail(GA_ERR_ARG, "input dtype must be GA_IN_F32 or GA_IN_BF16");
    return GA_OK;
}

extern "C" {

ga_status ga_quant_mxfp8(const void* x, int in_dtype, int rows, int K, int ld_x, void* q,
                         int ld_q, void* scales, int ld_s, int scale_rule, void* stream)
{
    if (check_in(in_dtype) != GA_OK)
        return GA_ERR_ARG;
    if (!x || !q || !scales || rows <= 0 || K <= 0 || ld_x < K || ld_q < K || ld_s < K / 32 ||
        scale_rule < 0 || scale_rule > 2)
        return fail(GA_ERR_ARG, "quant_mxfp8: bad argument");
    if (K % 32 || ld_x % 4 || ld_q % 4)
        return fail(GA_ERR_SHAPE, "quant_mxfp8: K %% 32, ld_x %% 4 and ld_q %% 4 must be 0");
    long long blocks = (long long)rows * (K / 32);
    GA_DISPATCH_IN(in_dtype, quant_mx_kernel, dim3(grid1d(blocks, 32)), dim3(256), 0,
                   (hipStream_t)stream, x, rows, K, ld_x, (uint8_t*)q, ld_q, (uint8_t*)scales,
                   ld_s, scale_rule);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
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
    GA_DISPATCH_IN(in_dtype, quant_mx4_kernel, dim3(grid1d(blocks, 32)), dim3(256), 0,
                   (hipStream_t)stream, x, rows, K, ld_x, (uint8_t*)q, ld_q, (uint8_t*)scales,
                   ld_s, scale_rule);
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
    GA_DISPATCH_IN(in_dtype, quant_1x128_kernel, dim3(grid1d(blocks, 8)), dim3(256), 0,
                   (hipStream_t)stream, x, rows, K, ld_x, (uint8_t*)q, ld_q, sfa, ld_s);
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
    GA_DISPATCH_IN(in_dtype, quant_128x128_kernel, grid, dim3(256), 0, (hipStream_t)stream, x,
                   rows, K, ld_x, (uint8_t*)q, ld_q, sfb, ld_s);
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

// reduce.hip -- split-K reduce: fp32 workspace -> bf16/fp32 output.
//
// Semantics of splitk_reduce_kernel (opus_gemm_dist/opus_gemm_mem_gemm_a2a/
// include/gfx950/splitk_reduce_gfx950.cuh:68-259): out[b, m, n] is the fp32
// sum over splits s = 0, 1, ... (in that order) of ws[s, b, m, n], plus an
// optional per-N bias, cast to the output type. The MX path folds its
// epilogue (alpha, beta * C) into the same pass.
//
// Layout: one workgroup row per (b, m); 256 threads x 8 consecutive N each,
// loaded as two 16-byte vectors per split; an element loop covers an N tail
// that is not a multiple of 8.
#include "ga_device.hpp"
#include "ga_internal.hpp"

namespace ga {

template <int OUT_DTYPE>
__device__ __forceinline__ void store_out(void* out, size_t idx, float v)
{
    if (OUT_DTYPE == GA_DTYPE_BF16)
        ((uint16_t*)out)[idx] = f32_to_bf16(v);
    else
        ((float*)out)[idx] = v;
}

__device__ __forceinline__ float load_bias(const void* bias, int dtype, size_t idx)
{
    return dtype == GA_DTYPE_BF16 ? bf16_to_f32(((const uint16_t*)bias)[idx])
                                  : ((const float*)bias)[idx];
}

template <int OUT_DTYPE>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceArgs a)
{
    const int bm = blockIdx.y;
    const int b = bm / a.M, m = bm - b * a.M;
    const int n_base = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (n_base >= a.N)
        return;
    const size_t split_stride = (size_t)a.batch * a.padded_M * a.padded_N;
    const size_t row = (size_t)b * a.padded_M * a.padded_N + (size_t)m * a.padded_N;
    const size_t orow = (size_t)b * a.c_batch_stride + (size_t)m * a.ldc;
    const bool vec = (n_base + 8 <= a.N) && ((a.padded_N & 3) == 0);
    float acc[8];
    if (vec) {
        const float* p = a.ws + row + n_base;
        v4f x0 = *(const v4f*)p, x1 = *(const v4f*)(p + 4);
        for (int j = 0; j < 4; j++) {
            acc[j] = x0[j];
            acc[j + 4] = x1[j];
        }
        for (int s = 1; s < a.split_k; s++) {
            p += split_stride;
            x0 = *(const v4f*)p;
            x1 = *(const v4f*)(p + 4);
            for (int j = 0; j < 4; j++) {
                acc[j] = acc[j] + x0[j];
                acc[j + 4] = acc[j + 4] + x1[j];
            }
        }
    } else {
        for (int j = 0; j < 8; j++) {
            if (n_base + j >= a.N)
                break;
            const float* p = a.ws + row + n_base + j;
            float v = p[0];
            for (int s = 1; s < a.split_k; s++)
                v = v + p[s * split_stride];
            acc[j] = v;
        }
    }
    const int nv = min(8, a.N - n_base);
    for (int j = 0; j < nv; j++) {
        float v = a.alpha * acc[j];
        if (a.bias)
            v = v + load_bias(a.bias, a.bias_dtype, (size_t)b * a.bias_stride_batch + n_base + j);
        if (a.c_in)
            v = v + a.beta * bf16_to_f32(((const uint16_t*)a.c_in)[orow + n_base + j]);
        store_out<OUT_DTYPE>(a.out, orow + n_base + j, v);
    }
}

ga_status splitk_reduce_launch(const ReduceArgs& a, hipStream_t stream)
{
    dim3 grid((a.N + 2047) / 2048, a.batch * a.M);
    if (a.out_dtype == GA_DTYPE_BF16)
        hipLaunchKernelGGL(splitk_reduce_kernel<GA_DTYPE_BF16>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(splitk_reduce_kernel<GA_DTYPE_F32>, grid, dim3(256), 0, stream, a);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

} // namespace ga

using namespace ga;

extern "C" ga_status ga_splitk_reduce(const float* ws, void* c_out, int out_dtype, int split_k,
                                      int M, int N, int batch, int padded_M, int padded_N,
                                      const void* bias, int bias_dtype, int bias_stride_batch,
                                      void* stream)
{
    if (!ws || !c_out || split_k < 1 || M <= 0 || N <= 0 || batch <= 0 || padded_M < M ||
        padded_N < N)
        return fail(GA_ERR_ARG, "splitk_reduce: bad argument");
    if ((out_dtype != GA_DTYPE_BF16 && out_dtype != GA_DTYPE_F32) ||
        (bias && bias_dtype != GA_DTYPE_BF16 && bias_dtype != GA_DTYPE_F32))
        return fail(GA_ERR_ARG, "splitk_reduce: bad dtype");
    if (batch * M > 65535 * 1024)
        return fail(GA_ERR_SHAPE, "splitk_reduce: batch*M too large");
    ReduceArgs a;
    a.ws = ws;
    a.out = c_out;
    a.c_in = nullptr;
    a.bias = bias;
    a.out_dtype = out_dtype;
    a.bias_dtype = bias_dtype;
    a.split_k = split_k;
    a.M = M;
    a.N = N;
    a.batch = batch;
    a.padded_M = padded_M;
    a.padded_N = padded_N;
    a.ldc = N;
    a.c_batch_stride = (long long)M * N;
    a.bias_stride_batch = bias_stride_batch;
    a.alpha = 1.0f;
    a.beta = 0.0f;
    return splitk_reduce_launch(a, (hipStream_t)stream);
}

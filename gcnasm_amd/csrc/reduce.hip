// reduce.hip -- split-K reduce: fp32 workspace -> bf16/fp32 output.
//
// Semantics of splitk_reduce_kernel (opus_gemm_dist/opus_gemm_mem_gemm_a2a/
// include/gfx950/splitk_reduce_gfx950.cuh:68-259): out[b, m, n] is the fp32
// sum over splits s = 0, 1, ... (in that order) of ws[s, b, m, n], plus an
// optional per-N bias, cast to the output type. The MX path folds its
// epilogue (alpha, beta * C) into the same pass.
//
// Layout: 256 threads x 8 consecutive N each, loaded as two 16-byte vectors
// per split; a row takes the smallest power of two of threads that covers N
// (at most 256, more workgroups along N beyond that), so short rows share a
// workgroup; an element loop covers an N tail that is not a multiple of 8. The workspace comes as a pointer or, as in the
// reference, through a device slot {ptr, bytes} read at kernel entry.
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
__device__ __forceinline__ void reduce_row(const ReduceArgs& a, const float* ws, int b, int m,
                                           int tpr)
{
    const int n_base = (blockIdx.x * tpr + (threadIdx.x & (tpr - 1))) * 8;
    if (n_base >= a.N)
        return;
    const size_t split_stride = (size_t)a.batch * a.ws_batch;
    const size_t row = (size_t)b * a.ws_batch + (size_t)m * a.ws_ld;
    const size_t orow = (size_t)b * a.c_batch_stride + (size_t)m * a.ldc;
    const bool vec = (n_base + 8 <= a.N) && ((a.ws_ld & 3) == 0) && ((a.ws_batch & 3) == 0) &&
                     (((uintptr_t)ws & 15) == 0);
    float acc[8];
    if (vec) {
        const float* p = ws + row + n_base;
        v4f x0 = *(const v4f*)p, x1 = *(const v4f*)(p + 4);
        for (int j = 0; j < 4; j++) {
            acc[j] = x0[j];
            acc[j + 4] = x1[j];
        }
        // slices added in order; four slices' loads in flight at a time
        int s = 1;
        for (; s + 3 < a.split_k; s += 4) {
            v4f y[4][2];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                y[u][0] = *(const v4f*)(p + (s + u) * split_stride);
                y[u][1] = *(const v4f*)(p + (s + u) * split_stride + 4);
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
                for (int j = 0; j < 4; j++) {
                    acc[j] = acc[j] + y[u][0][j];
                    acc[j + 4] = acc[j + 4] + y[u][1][j];
                }
        }
        for (; s < a.split_k; s++) {
            x0 = *(const v4f*)(p + s * split_stride);
            x1 = *(const v4f*)(p + s * split_stride + 4);
            for (int j = 0; j < 4; j++) {
                acc[j] = acc[j] + x0[j];
                acc[j + 4] = acc[j + 4] + x1[j];
            }
        }
    } else {
        for (int j = 0; j < 8; j++) {
            if (n_base + j >= a.N)
                break;
            const float* p = ws + row + n_base + j;
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

template <int OUT_DTYPE>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(ReduceArgs a)
{
    const float* ws = a.ws;
    if (a.wsh) {
        // the slot is read at entry: a graph captured before the workspace
        // moved still finds it
        ws = (const float*)a.wsh->ptr;
        const uint64_t need =
            (uint64_t)a.split_k * (uint64_t)a.batch * (uint64_t)a.ws_batch * 4u;
        if (ws == nullptr || a.wsh->bytes < need)
            return;
    }
    // rows of 2^tpr_log2 threads, 8 consecutive N per thread; row blocks
    // beyond the grid's y extent are taken in turn
    const int tpr = 1 << a.tpr_log2;
    const int rows = 256 >> a.tpr_log2;
    for (long long rb = blockIdx.y; rb * rows < (long long)a.batch * a.M; rb += gridDim.y) {
        const long long bm = rb * rows + (threadIdx.x >> a.tpr_log2);
        if (bm < (long long)a.batch * a.M)
            reduce_row<OUT_DTYPE>(a, ws, (int)(bm / a.M), (int)(bm % a.M), tpr);
    }
}

ga_status splitk_reduce_launch(const ReduceArgs& args, hipStream_t stream)
{
    // threads per output row: enough 8-wide groups to cover N, up to 256;
    // short rows share a workgroup
    ReduceArgs a = args;
    const int groups = (a.N + 7) / 8;
    a.tpr_log2 = 0;
    while ((1 << a.tpr_log2) < groups && a.tpr_log2 < 8)
        a.tpr_log2++;
    const int tpr = 1 << a.tpr_log2;
    const int rows = 256 / tpr;
    const long long gy = ((long long)a.batch * a.M + rows - 1) / rows;
    dim3 grid((a.N + 8 * tpr - 1) / (8 * tpr), (unsigned)(gy < 65535 ? gy : 65535));
    if (a.out_dtype == GA_DTYPE_BF16)
        hipLaunchKernelGGL(splitk_reduce_kernel<GA_DTYPE_BF16>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(splitk_reduce_kernel<GA_DTYPE_F32>, grid, dim3(256), 0, stream, a);
    GA_HIP_CHECK(hipGetLastError());
    return GA_OK;
}

} // namespace ga

using namespace ga;

static ga_status reduce_entry(const float* ws, const ga_splitk_ws_handle* wsh, void* c_out,
                              int out_dtype, int split_k, int M, int N, int batch, int padded_M,
                              int padded_N, const void* bias, int bias_dtype,
                              int bias_stride_batch, void* stream)
{
    if ((!ws && !wsh) || !c_out || split_k < 1 || M <= 0 || N <= 0 || batch <= 0 ||
        padded_M < M || padded_N < N || bias_stride_batch < 0)
        return fail(GA_ERR_ARG, "splitk_reduce: bad argument");
    if ((out_dtype != GA_DTYPE_BF16 && out_dtype != GA_DTYPE_F32) ||
        (bias && bias_dtype != GA_DTYPE_BF16 && bias_dtype != GA_DTYPE_F32))
        return fail(GA_ERR_ARG, "splitk_reduce: bad dtype");
    if ((long long)batch * M > 65535ll * 1024)
        return fail(GA_ERR_SHAPE, "splitk_reduce: batch*M too large");
    ReduceArgs a;
    a.ws = ws;
    a.wsh = wsh;
    a.out = c_out;
    a.c_in = nullptr;
    a.bias = bias;
    a.out_dtype = out_dtype;
    a.bias_dtype = bias_dtype;
    a.split_k = split_k;
    a.M = M;
    a.N = N;
    a.batch = batch;
    a.ws_ld = padded_N;
    a.ws_batch = (long long)padded_M * padded_N;
    a.ldc = N;
    a.c_batch_stride = (long long)M * N;
    a.bias_stride_batch = bias_stride_batch;
    a.alpha = 1.0f;
    a.beta = 0.0f;
    return splitk_reduce_launch(a, (hipStream_t)stream);
}

extern "C" ga_status ga_splitk_reduce(const float* ws, void* c_out, int out_dtype, int split_k,
                                      int M, int N, int batch, int padded_M, int padded_N,
                                      const void* bias, int bias_dtype, int bias_stride_batch,
                                      void* stream)
{
    if (!ws)
        return fail(GA_ERR_ARG, "splitk_reduce: null workspace");
    return reduce_entry(ws, nullptr, c_out, out_dtype, split_k, M, N, batch, padded_M, padded_N,
                        bias, bias_dtype, bias_stride_batch, stream);
}

extern "C" ga_status ga_splitk_reduce_ws_handle(const ga_splitk_ws_handle* ws_handle, void* c_out,
                                                int out_dtype, int split_k, int M, int N,
                                                int batch, int padded_M, int padded_N,
                                                const void* bias, int bias_dtype,
                                                int bias_stride_batch, void* stream)
{
    if (!ws_handle)
        return fail(GA_ERR_ARG, "splitk_reduce: null workspace handle");
    return reduce_entry(nullptr, ws_handle, c_out, out_dtype, split_k, M, N, batch, padded_M,
                        padded_N, bias, bias_dtype, bias_stride_batch, stream);
}

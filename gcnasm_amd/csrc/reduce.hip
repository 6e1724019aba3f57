// reduce.hip -- split-K reduce: fp32 workspace -> bf16/fp32 output.
//
// Semantics of splitk_reduce_kernel (opus_gemm_dist/opus_gemm_mem_gemm_a2a/
// include/gfx950/splitk_reduce_gfx950.cuh:68-259): out[b, m, n] is the fp32
// sum over splits s = 0, 1, ... (in that order) of ws[s, b, m, n], plus an
// optional per-N bias, cast to the output type. The MX path folds its
// epilogue (alpha, beta * C) into the same pass.
//
// Layout: 256 threads x 8 consecutive N each, loaded as two 16-byte vectors
// per split (for 2, 3, 4 or 8 splits every split's loads before the first
// add), stored as one 16-byte bf16 vector where aligned; a row takes the smallest power of two of threads that covers N
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

// The 8 sums of one thread, slices added in order. S > 0: exactly S slices,
// every load issued before the first add; S = 0: any count, four slices'
// loads in flight at a time.
template <int S>
__device__ __forceinline__ void sum_slices(const float* p, size_t split_stride, int split_k,
                                           float acc[8])
{
    if constexpr (S > 0) {
        v4f y[S][2];
#pragma unroll
        for (int u = 0; u < S; u++) {
            y[u][0] = *(const v4f*)(p + u * split_stride);
            y[u][1] = *(const v4f*)(p + u * split_stride + 4);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc[j] = y[0][0][j];
            acc[j + 4] = y[0][1][j];
        }
#pragma unroll
        for (int u = 1; u < S; u++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc[j] = acc[j] + y[u][0][j];
                acc[j + 4] = acc[j + 4] + y[u][1][j];
            }
    } else {
        v4f x0 = *(const v4f*)p, x1 = *(const v4f*)(p + 4);
        for (int j = 0; j < 4; j++) {
            acc[j] = x0[j];
            acc[j + 4] = x1[j];
        }
        int s = 1;
        for (; s + 3 < split_k; s += 4) {
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
        for (; s < split_k; s++) {
            x0 = *(const v4f*)(p + s * split_stride);
            x1 = *(const v4f*)(p + s * split_stride + 4);
            for (int j = 0; j < 4; j++) {
                acc[j] = acc[j] + x0[j];
                acc[j + 4] = acc[j + 4] + x1[j];
            }
        }
    }
}

template <int OUT_DTYPE, int S>
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
        sum_slices<S>(ws + row + n_base, split_stride, a.split_k, acc);
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
    // eight outputs in one 16-byte (bf16) or two 16-byte (fp32) stores when
    // the row offset and the pointers allow
    // (c_in is bf16 whatever the output: its 16-byte read needs the offset
    // aligned in bf16 elements too)
    const size_t esz = OUT_DTYPE == GA_DTYPE_BF16 ? 2 : 4;
    const bool vout = nv == 8 && ((orow + n_base) * esz) % 16 == 0 &&
                      ((uintptr_t)a.out & 15) == 0 &&
                      (!a.c_in || (((uintptr_t)a.c_in & 15) == 0 &&
                                   ((orow + n_base) * 2) % 16 == 0));
    if (vout) {
        float v[8];
        uint4 cbits = make_uint4(0, 0, 0, 0);
        if (a.c_in)
            cbits = *(const uint4*)((const uint16_t*)a.c_in + orow + n_base);
        const uint32_t cw[4] = {cbits.x, cbits.y, cbits.z, cbits.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            v[j] = a.alpha * acc[j];
            if (a.bias)
                v[j] = v[j] + load_bias(a.bias, a.bias_dtype,
                                        (size_t)b * a.bias_stride_batch + n_base + j);
            if (a.c_in)
                v[j] = v[j] + a.beta * bf16_to_f32((uint16_t)(cw[j >> 1] >> (16 * (j & 1))));
        }
        if (OUT_DTYPE == GA_DTYPE_BF16) {
            uint4 o;
            o.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
            o.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
            o.z = (uint32_t)f32_to_bf16(v[4]) | ((uint32_t)f32_to_bf16(v[5]) << 16);
            o.w = (uint32_t)f32_to_bf16(v[6]) | ((uint32_t)f32_to_bf16(v[7]) << 16);
            *(uint4*)((uint16_t*)a.out + orow + n_base) = o;
        } else {
            float* o = (float*)a.out + orow + n_base;
            *(v4f*)o = (v4f){v[0], v[1], v[2], v[3]};
            *(v4f*)(o + 4) = (v4f){v[4], v[5], v[6], v[7]};
        }
        return;
    }
    for (int j = 0; j < nv; j++) {
        float v = a.alpha * acc[j];
        if (a.bias)
            v = v + load_bias(a.bias, a.bias_dtype, (size_t)b * a.bias_stride_batch + n_base + j);
        if (a.c_in)
            v = v + a.beta * bf16_to_f32(((const uint16_t*)a.c_in)[orow + n_base + j]);
        store_out<OUT_DTYPE>(a.out, orow + n_base + j, v);
    }
}

template <int OUT_DTYPE, int S>
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
            reduce_row<OUT_DTYPE, S>(a, ws, (int)(bm / a.M), (int)(bm % a.M), tpr);
    }
}

template <int OUT_DTYPE>
static void reduce_dispatch(const ReduceArgs& a, dim3 grid, hipStream_t stream)
{
    switch (a.split_k) {
    case 2: hipLaunchKernelGGL((splitk_reduce_kernel<OUT_DTYPE, 2>), grid, dim3(256), 0, stream, a); break;
    case 3: hipLaunchKernelGGL((splitk_reduce_kernel<OUT_DTYPE, 3>), grid, dim3(256), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((splitk_reduce_kernel<OUT_DTYPE, 4>), grid, dim3(256), 0, stream, a); break;
    case 8: hipLaunchKernelGGL((splitk_reduce_kernel<OUT_DTYPE, 8>), grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((splitk_reduce_kernel<OUT_DTYPE, 0>), grid, dim3(256), 0, stream, a); break;
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
        reduce_dispatch<GA_DTYPE_BF16>(a, grid, stream);
    else
        reduce_dispatch<GA_DTYPE_F32>(a, grid, stream);
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

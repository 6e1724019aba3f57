// One v_mfma_scale_f32_16x16x128_f8f6f4 (E4M3 or E5M2 operands) per wave, for recording
// the instruction's outputs as test fixtures (tests/golden/make_mfma_fixture.py).
// Case e: a, b [64 lanes] x 32 bytes, c / d [64 lanes] x 4 floats, scale
// codes sa, sb [64 lanes] (E8M0 in the low byte). Lane l = 16g + r carries
// operand row r, K bytes [16g, 16g+16) and [64+16g, 64+16g+16); the scale of
// lane l applies to row r, K [32g, 32g+32); output lane l holds D[4g+j][r].
#include <hip/hip_runtime.h>

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// FA, FB: the f8f6f4 format codes of the two operands (0 E4M3, 1 E5M2).
template <int FA, int FB>
__global__ __launch_bounds__(64) void mfma_probe_kernel(const v8i* a, const v8i* b, const v4f* c,
                                                        const int* sa, const int* sb, v4f* d,
                                                        int cases)
{
    const int e = blockIdx.x;
    if (e >= cases)
        return;
    const size_t i = (size_t)e * 64 + threadIdx.x;
    d[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[i], b[i], c[i], FA, FB, 0, sa[i], 0,
                                                           sb[i]);
}

#define CHECK(x)                      \
    do {                              \
        hipError_t e_ = (x);          \
        if (e_ != hipSuccess)         \
            return (int)e_;           \
    } while (0)

// Host buffers in, host buffer out; returns a hipError_t code (0 = success).
// fa, fb: operand formats (0 E4M3, 1 E5M2).
extern "C" int mfma_probe_run_fmt(const void* a, const void* b, const void* c, const int* sa,
                                  const int* sb, void* d, int cases, int fa, int fb)
{
    if (cases <= 0 || cases > 65535 || fa < 0 || fa > 1 || fb < 0 || fb > 1)
        return (int)hipErrorInvalidValue;
    const size_t n = (size_t)cases * 64;
    void *da = nullptr, *db = nullptr, *dc = nullptr, *dd = nullptr, *dsa = nullptr,
         *dsb = nullptr;
    CHECK(hipMalloc(&da, n * 32));
    CHECK(hipMalloc(&db, n * 32));
    CHECK(hipMalloc(&dc, n * 16));
    CHECK(hipMalloc(&dd, n * 16));
    CHECK(hipMalloc(&dsa, n * 4));
    CHECK(hipMalloc(&dsb, n * 4));
    CHECK(hipMemcpy(da, a, n * 32, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(db, b, n * 32, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dc, c, n * 16, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dsa, sa, n * 4, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dsb, sb, n * 4, hipMemcpyHostToDevice));
#define PROBE_LAUNCH(FA, FB)                                                                  \
    hipLaunchKernelGGL((mfma_probe_kernel<FA, FB>), dim3(cases), dim3(64), 0, 0, (const v8i*)da, \
                       (const v8i*)db, (const v4f*)dc, (const int*)dsa, (const int*)dsb,          \
                       (v4f*)dd, cases)
    if (fa == 0 && fb == 0)
        PROBE_LAUNCH(0, 0);
    else if (fa == 0)
        PROBE_LAUNCH(0, 1);
    else if (fb == 0)
        PROBE_LAUNCH(1, 0);
    else
        PROBE_LAUNCH(1, 1);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(d, dd, n * 16, hipMemcpyDeviceToHost));
    CHECK(hipFree(da));
    CHECK(hipFree(db));
    CHECK(hipFree(dc));
    CHECK(hipFree(dd));
    CHECK(hipFree(dsa));
    CHECK(hipFree(dsb));
    return 0;
}

extern "C" int mfma_probe_run(const void* a, const void* b, const void* c, const int* sa,
                              const int* sb, void* d, int cases)
{
    return mfma_probe_run_fmt(a, b, c, sa, sb, d, cases, 0, 0);
}

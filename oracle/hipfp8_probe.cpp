// hipfp8_probe.cpp -- exposes ROCm's host-side OCP E4M3 conversion
// (__hip_fp8_e4m3 from <hip/hip_fp8.h>) so the tests can check the oracle's
// encoder against a library implementation. TEST INFRASTRUCTURE ONLY.
#include <hip/hip_fp8.h>
#include <cstdint>
#include <cstring>

extern "C" void hipfp8_encode_e4m3(const float* x, uint8_t* out, long n)
{
    for (long i = 0; i < n; i++) {
        __hip_fp8_e4m3 v(x[i]);
        uint8_t b;
        memcpy(&b, &v, 1);
        out[i] = b;
    }
}

extern "C" void hipfp8_decode_e4m3(const uint8_t* c, float* out, long n)
{
    for (long i = 0; i < n; i++) {
        __hip_fp8_e4m3 v;
        memcpy(&v, &c[i], 1);
        out[i] = (float)v;
    }
}

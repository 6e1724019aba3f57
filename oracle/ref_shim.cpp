// ref_shim.cpp -- extern "C" wrappers around the reference's own header-only
// CPU code, compiled from the headers where they lie in the reference tree
// (asm_f4gemm/f4gemm.hpp and asm_f4gemm/f4gemm_ref.hpp; include path given
// by oracle/Makefile). TEST INFRASTRUCTURE ONLY: the output goes to
// oracle/_ref/ and is used to pin the oracle and as the CPU baseline.
#include "f4gemm.hpp"
#include "f4gemm_ref.hpp"

#include <cstring>
#include <string>
#include <vector>

extern "C" {

void ref_shuffle_weight_16x16(const uint8_t* src, uint8_t* dst, int N, int Kp)
{
    std::vector<uint8_t> s(src, src + (size_t)N * Kp);
    std::vector<uint8_t> d = f4gemm::shuffle_weight_16x16(s, N, Kp);
    memcpy(dst, d.data(), d.size());
}

void ref_shuffle_scale(const uint8_t* src, uint8_t* dst, int rows, int cols, int sm, int sn)
{
    std::vector<uint8_t> s(src, src + (size_t)rows * cols);
    std::vector<uint8_t> d = f4gemm::shuffle_scale(s, rows, cols, sm, sn);
    memcpy(dst, d.data(), d.size());
}

float ref_e8m0_to_f32(uint8_t e) { return f4gemm::e8m0_to_f32(e); }
float ref_bf16_to_f32(uint16_t h) { return f4gemm::bf16_to_f32(h); }
float ref_fp4_lut(int i) { return f4gemm::kFp4Lut[i & 15]; }

void ref_reference_gemm(const float* A, const float* B, int M, int N, int K, float alpha,
                        float* D)
{
    std::vector<float> a(A, A + (size_t)M * K), b(B, B + (size_t)N * K);
    std::vector<float> d = f4gemm::reference_gemm(a, b, M, N, K, alpha, {}, 0.0f);
    memcpy(D, d.data(), d.size() * sizeof(float));
}

static std::vector<f4gemm::Config> mk_cfgs(const int* tm, const int* tn, const int* sk,
                                           const int* bp, int n)
{
    std::vector<f4gemm::Config> v;
    for (int i = 0; i < n; i++) {
        f4gemm::Config c;
        c.tile_M = tm[i];
        c.tile_N = tn[i];
        c.splitK = sk[i];
        c.bpreshuffle = bp[i];
        c.knl_name = "k" + std::to_string(i);
        c.co_name = "k" + std::to_string(i) + ".co";
        v.push_back(c);
    }
    return v;
}

int ref_select_kernel(int M, int N, int K, int num_cu, int log2_k_split, int bpreshuffle,
                      const int* tm, const int* tn, const int* sk, const int* bp, int n,
                      int* log2_out)
{
    auto cfgs = mk_cfgs(tm, tn, sk, bp, n);
    auto r = f4gemm::select_kernel(M, N, K, num_cu, log2_k_split, bpreshuffle, cfgs);
    *log2_out = r.second;
    return r.first;
}

// Only valid inputs: the reference exits the process on K % 2^L != 0.
void ref_make_launch(int tm, int tn, int sk, int bp, int M, int N, int K, int log2_k_split,
                     int* out5)
{
    auto cfgs = mk_cfgs(&tm, &tn, &sk, &bp, 1);
    f4gemm::LaunchDesc d = f4gemm::make_launch(cfgs[0], M, N, K, log2_k_split);
    out5[0] = d.gdx;
    out5[1] = d.gdy;
    out5[2] = d.gdz;
    out5[3] = d.log2_k_split;
    out5[4] = d.zero_out ? 1 : 0;
}

int ref_kernelargs_size(void) { return (int)sizeof(f4gemm::KernelArgs); }

// Threads reference_gemm starts: hardware_concurrency, capped by M (f4gemm_ref.hpp:191-192).
int ref_threads(int M)
{
    unsigned n = std::max(1u, std::thread::hardware_concurrency());
    return (int)std::min<unsigned>(n, (unsigned)M);
}

void ref_fill_args(void* out, void* D, void* C, void* A, void* B, void* SA, void* SB, int M,
                   int N, int K, int stride_D0, int sA0, int sB0, float alpha, float beta,
                   int log2_k_split)
{
    f4gemm::KernelArgs a;
    f4gemm::fill_args(a, D, C, A, B, SA, SB, M, N, K, stride_D0, sA0, sB0, alpha, beta,
                      log2_k_split);
    memcpy(out, &a, sizeof(a));
}

// Only call with a readable, non-empty file: the reference exits otherwise.
int ref_load_configs(const char* path, int* tm, int* tn, int* sk, int* bp, int cap)
{
    auto v = f4gemm::load_configs(path);
    int n = (int)v.size();
    for (int i = 0; i < n && i < cap; i++) {
        tm[i] = v[i].tile_M;
        tn[i] = v[i].tile_N;
        sk[i] = v[i].splitK;
        bp[i] = v[i].bpreshuffle;
    }
    return n;
}

void ref_shape(int M, int N, int K, int* out7)
{
    f4gemm::Shape s{M, N, K};
    out7[0] = s.Kp();
    out7[1] = s.Ks();
    out7[2] = s.scale_cols();
    out7[3] = s.a_rows_pad();
    out7[4] = s.b_rows_pad();
    out7[5] = s.scale_a_rows();
    out7[6] = s.d_rows_pad();
}

void ref_make_operand(int rows, int K, uint32_t seed, uint8_t* packed, uint8_t* scales,
                      float* dequant)
{
    f4gemm::Operand op = f4gemm::make_operand(rows, K, seed);
    memcpy(packed, op.packed.data(), op.packed.size());
    memcpy(scales, op.scales.data(), op.scales.size());
    memcpy(dequant, op.dequant.data(), op.dequant.size() * sizeof(float));
}

} // extern "C"

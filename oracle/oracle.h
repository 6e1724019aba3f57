/*
 * oracle -- CPU restatement of the reference's block-scaled FP8 GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for libgcnasm_amd:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it. No product code path may call into it.
 *
 * Each function names the reference file:line whose algorithm it restates
 * (paths relative to the Fyzyukk/gcnasm tree). How each one is pinned is
 * listed in oracle.c next to the function.
 */
#ifndef GCNASM_ORACLE_H
#define GCNASM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar codecs ------------------------------------------------------ */
uint8_t or_e4m3_encode(float x);      /* OCP E4M3, RNE, saturate to +-448, NaN->0x7F */
void or_e4m3_encode_n(const float* x, uint8_t* out, size_t n);
float or_e4m3_decode(uint8_t c);      /* opus.hpp:858-871 value set (OCP, bias 7)      */
float or_e5m2_decode(uint8_t c);      /* OCP E5M2 (f8f6f4 format 1, opus.hpp:1785)      */
uint8_t or_e5m2_encode(float x);      /* RNE, saturating to +-57344, NaN -> 0x7F         */
void or_e5m2_encode_n(const float* x, uint8_t* out, size_t n);
int or_mx8_scale_exp(float amax, int rule, int fmt); /* MX scale rules, E4M3 / E5M2 max */
float or_e8m0_to_f32(uint8_t e);      /* f4gemm_ref.hpp:29-41                          */
uint16_t or_f32_to_bf16(float x);     /* RNE, opus.hpp:944-950                         */
float or_bf16_to_f32(uint16_t h);     /* f4gemm_ref.hpp:43-49                          */
float or_fp4_decode(uint8_t nibble);  /* kFp4Lut, f4gemm_ref.hpp:24-26                 */
uint8_t or_e2m1_encode(float x);      /* OCP E2M1 RNE, saturate +-6, NaN -> signed 0  */
int or_floor_log2(float a);           /* exact, a > 0 finite (normal or subnormal)     */

/* E8M0 exponent of an MX block from its amax (rule: 0 floor448, 1 ceil448,
 * 2 OCP). Returns the unbiased exponent e; code = e + 127 (clamped). */
int or_mx_scale_exp(float amax, int rule);
/* Same rules for E2M1 elements (max 6): floor/ceil(log2(amax/6)), OCP - 2. */
int or_mx4_scale_exp(float amax, int rule);

/* ---- quantisers --------------------------------------------------------- */
void or_quant_mxfp8(const float* x, int rows, int K, uint8_t* q, uint8_t* scales, int rule);
void or_quant_mx8(const float* x, int rows, int K, uint8_t* q, uint8_t* scales, int rule, int fmt);
/* MXFP4: q [rows, K/2] packed e2m1 (element 2i in the low nibble of byte i,
 * asm_f4gemm/README.md:97-99), scales [rows, K/32]. */
void or_quant_mxfp4(const float* x, int rows, int K, uint8_t* q, uint8_t* scales, int rule);
void or_quant_fp8_1x128(const float* x, int rows, int K, uint8_t* q, float* sfa /*[K/128, rows]*/);
void or_quant_fp8_128x128(const float* x, int rows, int K, uint8_t* q,
                          float* sfb /*[ceil(rows/128), K/128]*/);
void or_quant_fp8_per_tensor(const float* x, size_t n, uint8_t* q, float* scale);

/* ---- layout transforms --------------------------------------------------- */
void or_shuffle_weight_16x16(const uint8_t* src, uint8_t* dst, int N, int Kp);
void or_shuffle_scale(const uint8_t* src, uint8_t* dst, int rows, int cols, int sm, int sn);

/* ---- host launch logic --------------------------------------------------- */
typedef struct or_cfg {
    int tile_M, tile_N, splitK, bpreshuffle;
} or_cfg;
/* f4gemm.hpp:210-267; returns index (-1 none), *log2_out the log2 split. */
int or_select_kernel(int M, int N, int K, int num_cu, int log2_k_split, int bpreshuffle,
                     const or_cfg* cfgs, int n, int* log2_out);
/* f4gemm.hpp:329-349; returns 0, or -1 when K % (1 << log2_k_split) != 0. */
int or_make_launch(const or_cfg* cfg, int M, int N, int K, int log2_k_split, int* gdx,
                   int* gdy, int* gdz, int* zero_out);

/* ---- reference GEMMs ---------------------------------------------------- */
/* f4gemm_ref.hpp:181-222: D = alpha * A * B^T over dequantised f32 operands,
 * f64 accumulation, parallel over M. */
void or_reference_gemm(const float* A, const float* B, int M, int N, int K, float alpha,
                       float* D);

/* MXFP8, exact: f64 sum of every dequantised product (A [M,K] E4M3 row-major,
 * B [N,K] E4M3 row-major (not shuffled), scales [rows, K/32] unshuffled). */
void or_gemm_mxfp8_exact(const uint8_t* A, const uint8_t* B, const uint8_t* sA,
                         const uint8_t* sB, int M, int N, int K, double* D);

/* The two MX GEMMs above/below for either element width: elem_bits 8 (E4M3
 * bytes [rows, K]) or 4 (e2m1 packed [rows, K/2], low nibble first). */
void or_gemm_mx_exact(const uint8_t* A, const uint8_t* B, const uint8_t* sA,
                      const uint8_t* sB, int M, int N, int K, int elem_bits, double* D);
void or_gemm_mx_fp32acc(const uint8_t* A, const uint8_t* B, const uint8_t* sA,
                        const uint8_t* sB, int M, int N, int K, int elem_bits, int log2_k_split,
                        float alpha, float* D);
/* MXFP8 with fp32 accumulation in the order of the GPU kernel: K is cut into
 * gdz slices of k_per_tg = round_up(K / 2^L, 256) (f4gemm.hpp:342-344); in a
 * slice, each 128-wide K step adds its exact product sum to an fp32
 * accumulator with one rounding; slices are summed in fp32 in slice order;
 * out = alpha * acc (fp32). Writes fp32 results. */
void or_gemm_mxfp8_fp32acc(const uint8_t* A, const uint8_t* B, const uint8_t* sA,
                           const uint8_t* sB, int M, int N, int K, int log2_k_split,
                           float alpha, float* D);

/* opus blockscale gemm_ref (opus_gemm/block_scale_gemm/gemm_a8w8_blockscale_host.cc:66-90
 * and block_scale_1x128x1_gemm/..._host.cc:77-101): sum += a*b*(sa*sb) per
 * product in fp32. sfb indexing: group_n == 1 -> sfb[g*stride_sfb + n],
 * else sfb[(n/group_n)*stride_sfb + g]. Requires K % 128 == 0. */
void or_gemm_blockscale_ref(const uint8_t* A, const uint8_t* B, const float* sfa,
                            const float* sfb, float* C, int M, int N, int K, int lda,
                            int ldb, int ldc, int stride_sfa, int stride_sfb, int group_n);

/* Block-scale GEMM in kernel order: per 128-K group g, p = fp32(exact sum),
 * s = fp32(sa*sb), acc = fmaf(p, s, acc). */
void or_gemm_blockscale_fp32acc(const uint8_t* A, const uint8_t* B, const float* sfa,
                                const float* sfb, float* C, int M, int N, int K, int lda,
                                int ldb, int ldc, int stride_sfa, int stride_sfb,
                                int group_n);
/* f64-exact block-scale value: sum_g (exact sum_g) * sa * sb in f64. */
void or_gemm_blockscale_exact(const uint8_t* A, const uint8_t* B, const float* sfa,
                              const float* sfb, double* C, int M, int N, int K,
                              int stride_sfa, int stride_sfb, int group_n);

/* Per-tensor: acc = fp32 chain over 128-K steps (exact step sums),
 * out = fp32(acc * fp32(sa*sb)). */
void or_gemm_per_tensor_fp32acc(const uint8_t* A, const uint8_t* B, float sa, float sb,
                                float* C, int M, int N, int K);

/* ---- the gfx950 FP8 MFMA's K-step sum (measured; see oracle.c) ----------- */
/* One step over n <= 128 K (E4M3 codes a, b; E8M0 scale codes sa, sb per
 * 32-K block, NULL for unit scales): RNE_fp32(c + the truncated group sums). */
/* The same with operand formats fa / fb (0 E4M3, 1 E5M2). */
float or_mfma_f8_step(const uint8_t* a, const uint8_t* b, int n, const uint8_t* sa,
                      const uint8_t* sb, float c, int fa, int fb);
void or_gemm_mx8_mfma(const uint8_t* A, const uint8_t* B, const uint8_t* sA, const uint8_t* sB,
                      int M, int N, int K, int log2_k_split, float alpha, float* D, int fa, int fb);
float or_mfma_fp8_step(const uint8_t* a, const uint8_t* b, int n, const uint8_t* sa,
                       const uint8_t* sb, float c);
/* MXFP8 GEMM with that step sum, in the slice structure of
 * or_gemm_mxfp8_fp32acc. */
void or_gemm_mx_mfma(const uint8_t* A, const uint8_t* B, const uint8_t* sA, const uint8_t* sB,
                     int M, int N, int K, int log2_k_split, float alpha, float* D);
/* Block-scale / per-tensor GEMMs with that step sum; K is cut into slices of
 * gps 128-K groups whose chains are summed in slice order (gps <= 0: one). */
void or_gemm_blockscale_mfma(const uint8_t* A, const uint8_t* B, const float* sfa,
                             const float* sfb, float* C, int M, int N, int K, int lda, int ldb,
                             int ldc, int stride_sfa, int stride_sfb, int group_n, int gps);
void or_gemm_blockscale_mfma_cuts(const uint8_t* A, const uint8_t* B, const float* sfa,
                                  const float* sfb, float* C, int M, int N, int K, int lda,
                                  int ldb, int ldc, int stride_sfa, int stride_sfb, int group_n,
                                  const int* cuts, int ncuts);
void or_gemm_per_tensor_mfma(const uint8_t* A, const uint8_t* B, float sa, float sb, float* C,
                             int M, int N, int K, int gps);

/* splitk_reduce_kernel (splitk_reduce_gfx950.cuh:105-170): fp32 sum over
 * splits in split order (+ bias), output fp32 (cast by caller). */
void or_splitk_reduce(const float* ws, float* out, int split_k, int M, int N, int batch,
                      int padded_M, int padded_N, const float* bias, int bias_stride_batch);

/* bf16 split-K GEMM (opus_gemm_dist/opus_gemm_mem_gemm_a2a, pipeline
 * .cuh:234-247 partition, :204-563 kernel): slice bounds, and the fp32
 * partials ws [split_k, M, N] (per 32-K group: exact sum, one fp32 rounding). */
void or_a16w16_slices(int K, int split_k, int* kb, int* ke);
void or_a16w16_splitk_ws(const uint16_t* A, const uint16_t* B, int M, int N, int K, int lda,
                         int ldb, int split_k, float* ws);

/* ---- synthetic inputs ---------------------------------------------------- */
/* Deterministic stream: splitmix64. Normal samples by Box-Muller on f64. */
void or_randn(float* out, size_t n, uint64_t seed, float mean, float std);
/* MX synthetic operand: x = N(mean, std) * 2^u per 1x32
 * block, u uniform in [-spread, spread]; returns x in `x`. */
void or_gen_mx_input(float* x, int rows, int K, uint64_t seed, float std, int spread);

#ifdef __cplusplus
}
#endif
#endif

/*
 * gcnasm_amd -- block-scaled FP8 GEMM library for MI355X (gfx950).
 *
 * C ABI of the library libgcnasm_amd.so. Plain pointers and sizes only; device
 * pointers are HIP device addresses, streams are hipStream_t passed as void*.
 * Every entry point returns a ga_status (0 = success) instead of exiting the
 * process; ga_last_error() holds a human-readable detail string for the last
 * failure on the calling thread.
 *
 * Reference interfaces replaced (paths relative to the gcnasm tree):
 *   opus_gemm_kargs                 opus_gemm/block_scale_gemm/gemm_a8w8_blockscale_common.h:4-25
 *   gemm_a8w8_blockscale_kernel<<<>>> opus_gemm/block_scale_gemm/gemm_a8w8_blockscale_host.cc:249-257
 *   gemm_a8w8_1x128x1_blockscale_kernel opus_gemm/block_scale_1x128x1_gemm/..._host.cc:223-231
 *   fp8_gemm (per-tensor)           opus_gemm/fp8_gemm/rebuild.sh:3-11 (build line only)
 *   f4gemm::KernelArgs              asm_f4gemm/f4gemm.hpp:55-115
 *   f4gemm::Config / load_configs   asm_f4gemm/f4gemm.hpp:120-200
 *   f4gemm::select_kernel           asm_f4gemm/f4gemm.hpp:210-267
 *   f4gemm::Kernel::load/launch     asm_f4gemm/f4gemm.hpp:272-317
 *   f4gemm::LaunchDesc/make_launch  asm_f4gemm/f4gemm.hpp:322-349
 *   f4gemm::fill_args               asm_f4gemm/f4gemm.hpp:355-392
 *   f4gemm::Shape                   asm_f4gemm/f4gemm_ref.hpp:61-73
 *   f4gemm::shuffle_weight_16x16    asm_f4gemm/f4gemm_ref.hpp:81-96
 *   f4gemm::shuffle_scale           asm_f4gemm/f4gemm_ref.hpp:108-130
 *   splitk_reduce_kernel            opus_gemm_dist/opus_gemm_mem_gemm_a2a/include/gfx950/splitk_reduce_gfx950.cuh:68-259
 *   opus_splitk_ws_handle           opus_gemm_dist/opus_gemm_mem_gemm_a2a/include/gfx950/opus_gemm_traits_a16w16_gfx950.cuh:588-597
 *   opus_gemm_flatmm_splitk_kargs_gfx950  (same file):599-634
 *   gemm_a16w16_flatmm_splitk_kernel opus_gemm_dist/opus_gemm_mem_gemm_a2a/include/gfx950/opus_gemm_pipeline_a16w16_flatmm_splitk_gfx950.cuh:204-563
 */
#ifndef GCNASM_AMD_H
#define GCNASM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------- */
/* Status codes. The reference prints and exit(1)s (f4gemm.hpp:22-35,         */
/* gemm_a8w8_blockscale_host.cc:17-26); every such exit is a status here.     */
/* ------------------------------------------------------------------------- */
typedef int ga_status;
#define GA_OK             0
#define GA_ERR_ARG        1 /* null pointer, negative size, bad enum          */
#define GA_ERR_SHAPE      2 /* K % 128, N % 16, ... (main.cpp:141-150)        */
#define GA_ERR_NO_KERNEL  3 /* heuristic found nothing / unknown kernel name  */
#define GA_ERR_SPLITK     4 /* K % (1 << log2_k_split) != 0 (f4gemm.hpp:336)  */
#define GA_ERR_MANIFEST   5 /* manifest missing or empty (f4gemm.hpp:143-155) */
#define GA_ERR_WORKSPACE  6 /* caller workspace too small                      */
#define GA_ERR_HIP        7 /* HIP runtime reported an error                   */
#define GA_ERR_GROUP      8 /* scale-group divisibility (host.cc:183-187)      */
#define GA_ERR_CAPACITY   9 /* output array too small                          */

const char* ga_status_string(ga_status s);
const char* ga_last_error(void);
const char* ga_version(void);

/* Element / output type codes. */
#define GA_DTYPE_BF16 0
#define GA_DTYPE_F32  1

/* ------------------------------------------------------------------------- */
/* Kernel argument blocks, byte-compatible with the reference.               */
/* ------------------------------------------------------------------------- */

/* opus_gemm_kargs, 96 bytes: ptr_a@0 ptr_b@8 ptr_c@16 m@24 ... ptr_sfa@64
 * ptr_sfb@72 stride_sfa@80 stride_sfb@84 stride_sfa_batch@88
 * stride_sfb_batch@92. Strides are in elements.
 * Replaces opus_gemm/block_scale_gemm/gemm_a8w8_blockscale_common.h:4-25. */
typedef struct ga_opus_gemm_kargs {
    const void* ptr_a;
    const void* ptr_b;
    void* ptr_c;
    int m;
    int n;
    int k;
    int batch;
    int stride_a;
    int stride_b;
    int stride_c;
    int stride_a_batch;
    int stride_b_batch;
    int stride_c_batch;
    const void* ptr_sfa;
    const void* ptr_sfb;
    int stride_sfa;
    int stride_sfb;
    int stride_sfa_batch;
    int stride_sfb_batch;
} ga_opus_gemm_kargs;

/* f4gemm::KernelArgs, 0x174 bytes: one argument per 16-byte slot.
 * Replaces asm_f4gemm/f4gemm.hpp:64-115. The kernels read stride_C0 for both
 * C and D; stride_D0/D1/C1/A1/B1/ScaleA1/ScaleB1 are carried but unread. */
#pragma pack(push, 1)
typedef struct ga_f4gemm_kargs {
    void* ptr_D;              uint32_t _p0[2];
    void* ptr_C;              uint32_t _p1[2];
    void* ptr_A;              uint32_t _p2[2];
    void* ptr_B;              uint32_t _p3[2];
    float alpha;              uint32_t _p4[3];
    float beta;               uint32_t _p5[3];
    uint32_t stride_D0;       uint32_t _p6[3];
    uint32_t stride_D1;       uint32_t _p7[3];
    uint32_t stride_C0;       uint32_t _p8[3];
    uint32_t stride_C1;       uint32_t _p9[3];
    uint32_t stride_A0;       uint32_t _p10[3];
    uint32_t stride_A1;       uint32_t _p11[3];
    uint32_t stride_B0;       uint32_t _p12[3];
    uint32_t stride_B1;       uint32_t _p13[3];
    uint32_t M;               uint32_t _p14[3];
    uint32_t N;               uint32_t _p15[3];
    uint32_t K;               uint32_t _p16[3];
    void* ptr_ScaleA;         uint32_t _p17[2];
    void* ptr_ScaleB;         uint32_t _p18[2];
    uint32_t stride_ScaleA0;  uint32_t _p19[3];
    uint32_t stride_ScaleA1;  uint32_t _p20[3];
    uint32_t stride_ScaleB0;  uint32_t _p21[3];
    uint32_t stride_ScaleB1;  uint32_t _p22[3];
    int log2_k_split;
} ga_f4gemm_kargs;
#pragma pack(pop)

/* opus_splitk_ws_handle, 16 bytes: the device-resident slot through which
 * the split-K kernels find their fp32 workspace. Kernels read it at entry,
 * so a captured HIP graph (which holds the slot's address) still sees a
 * workspace that was grown and moved after capture.
 * Replaces opus_gemm_dist/.../gfx950/opus_gemm_traits_a16w16_gfx950.cuh:588-597. */
typedef struct ga_splitk_ws_handle {
    void* ptr;       /* current workspace; NULL until the first reserve */
    uint64_t bytes;  /* its capacity in bytes                           */
} ga_splitk_ws_handle;

/* opus_gemm_flatmm_splitk_kargs_gfx950, 96 bytes: ptr_a@0 ptr_b@8
 * ws_handle@16 ptr_c@24 ptr_bias@32 m@40 n@44 k@48 batch@52 split_k@56
 * stride_a@60 stride_b@64 stride_ws@68 stride_c@72 stride_a_batch@76
 * stride_b_batch@80 stride_ws_batch@84 stride_c_batch@88
 * stride_bias_batch@92. Strides in elements. The workspace is fp32
 * [split_k, batch, padded_M, padded_N]: stride_ws = padded_N,
 * stride_ws_batch = padded_M * padded_N.
 * Replaces opus_gemm_dist/.../gfx950/opus_gemm_traits_a16w16_gfx950.cuh:599-634. */
typedef struct ga_flatmm_splitk_kargs {
    const void* ptr_a;                    /* bf16 [batch, M, K]            */
    const void* ptr_b;                    /* bf16 [batch, N, K]            */
    const ga_splitk_ws_handle* ws_handle; /* device address of the slot    */
    void* ptr_c;                          /* bf16 [batch, M, N]            */
    const void* ptr_bias;                 /* bf16 [N] or [batch, N]; NULL  */
    int m;
    int n;
    int k;
    int batch;
    int split_k;
    int stride_a;
    int stride_b;
    int stride_ws;
    int stride_c;
    int stride_a_batch;
    int stride_b_batch;
    int stride_ws_batch;
    int stride_c_batch;
    int stride_bias_batch; /* 0: one [N] bias for all batches; N: [batch, N] */
} ga_flatmm_splitk_kargs;

/* ------------------------------------------------------------------------- */
/* Tile manifest (f4gemm::Config, asm_f4gemm/f4gemm.hpp:120-128).            */
/* The library's kernels are compiled in; the manifest is a compiled table   */
/* with the same columns as the reference CSV:                               */
/*   tile_M,tile_N,splitK,bpreshuffle,knl_name,co_name                        */
/* ------------------------------------------------------------------------- */
#define GA_NAME_MAX 96
typedef struct ga_tile_config {
    int tile_M;
    int tile_N;
    int splitK;       /* 1 -> kernel understands log2_k_split / gdz        */
    int bpreshuffle;  /* 1 -> B must be 16x16-tile preshuffled             */
    char knl_name[GA_NAME_MAX];
    char co_name[GA_NAME_MAX];
} ga_tile_config;

/* Number of compiled MXFP8 kernels and row idx of the compiled manifest. */
int ga_manifest_count(void);
ga_status ga_manifest_get(int idx, ga_tile_config* out);
/* Writes the compiled manifest as CSV text (header + one row per kernel).
 * *needed receives the byte count including the terminating NUL. */
ga_status ga_manifest_csv(char* buf, size_t cap, size_t* needed);

/* The MXFP4 manifest: the role of the reference's f4gemm_bf16_per1x32Fp4.csv
 * (asm_f4gemm/README.md:30-40), same columns. Its kernels take OCP e2m1
 * operands packed two per byte (low nibble = even element; A/B strides and
 * K count elements, asm_f4gemm/README.md:86). Select from it by passing
 * its rows to ga_select_kernel, then ga_kernel_find(knl_name). */
int ga_manifest_fp4_count(void);
ga_status ga_manifest_fp4_get(int idx, ga_tile_config* out);
ga_status ga_manifest_fp4_csv(char* buf, size_t cap, size_t* needed);

/* f4gemm::load_configs (f4gemm.hpp:141-200): parse a manifest CSV file. The
 * column order comes from the header row; rows whose column count differs
 * from the header are skipped; rows without knl_name or co_name are dropped.
 * GA_ERR_MANIFEST if the file cannot be opened or is empty. */
ga_status ga_load_configs(const char* csv_path, ga_tile_config* out, int cap, int* count);

/* f4gemm::select_kernel (f4gemm.hpp:210-267). cfgs == NULL selects from the
 * compiled manifest. log2_k_split < 0 lets the heuristic try splitK
 * 2/4/8/16. Writes the chosen index (-1 if none) and the log2 split;
 * returns GA_ERR_NO_KERNEL when nothing fits. */
ga_status ga_select_kernel(int M, int N, int K, int num_cu, int log2_k_split,
                           int bpreshuffle, const ga_tile_config* cfgs, int n_cfgs,
                           int* idx, int* log2_out);

/* f4gemm::LaunchDesc / make_launch (f4gemm.hpp:322-349). */
typedef struct ga_launch_desc {
    int gdx;
    int gdy;
    int gdz;
    int log2_k_split;
    int zero_out;  /* reference semantics: split kernels accumulate into D */
} ga_launch_desc;
ga_status ga_make_launch(const ga_tile_config* cfg, int M, int N, int K,
                         int log2_k_split, ga_launch_desc* out);

/* f4gemm::fill_args (f4gemm.hpp:355-392). */
void ga_fill_args(ga_f4gemm_kargs* args, void* d_D, void* d_C, void* d_A, void* d_B,
                  void* d_ScaleA, void* d_ScaleB, int M, int N, int K,
                  int stride_D0, int stride_ScaleA0, int stride_ScaleB0,
                  float alpha, float beta, int log2_k_split);

/* f4gemm::Shape (f4gemm_ref.hpp:61-73), generalised to the element width:
 * elem_bits = 8 for FP8 (Kp = K bytes), 4 for FP4 (Kp = K/2). */
typedef struct ga_mx_shape {
    int M, N, K;
    int Kp;            /* bytes per A/B row                           */
    int Ks;            /* e8m0 scales per row, K/32                   */
    int scale_cols;    /* round_up(Ks, 8)                             */
    int a_rows_pad;    /* round_up(M, 256)                            */
    int b_rows_pad;    /* round_up(N, 256)                            */
    int scale_a_rows;  /* round_up(M, 256)                            */
    int scale_b_rows;  /* round_up(N, 256)                            */
    int d_rows_pad;    /* round_up(M, 32)                             */
} ga_mx_shape;
ga_status ga_mx_shape_init(int M, int N, int K, int elem_bits, ga_mx_shape* out);

/* ------------------------------------------------------------------------- */
/* Host-side layout transforms (byte-level, dtype-agnostic).                  */
/* ------------------------------------------------------------------------- */
/* shuffle_weight(w, layout=(16,16)) (f4gemm_ref.hpp:81-96):
 *   src[n0*16+n1][k0*32+k1*16+k2] -> dst[(((n0*Kp/32+k0)*2+k1)*16+n1)*16+k2]
 * Needs N % 16 == 0 and Kp % 32 == 0. */
ga_status ga_shuffle_weight_16x16(const uint8_t* src, uint8_t* dst, int N, int Kp);
/* shuffle_scale (f4gemm_ref.hpp:108-130): pad [rows, cols] to [sm, sn] with
 * 0x7F, then padded[d0*32+d1*16+d2][d3*8+d4*4+d5]
 *   -> dst[((((d0*sn/8+d3)*4+d5)*16+d2)*2+d4)*2+d1].
 * Needs sm % 32 == 0, sn % 8 == 0, rows <= sm, cols <= sn. */
ga_status ga_shuffle_scale(const uint8_t* src, uint8_t* dst, int rows, int cols,
                           int sm, int sn);

/* ------------------------------------------------------------------------- */
/* Device-side layout transforms and quantisers (HIP kernels).                */
/* ------------------------------------------------------------------------- */
ga_status ga_shuffle_weight_16x16_device(const void* src, void* dst, int N, int Kp,
                                         void* stream);
ga_status ga_shuffle_scale_device(const void* src, void* dst, int rows, int cols,
                                  int sm, int sn, void* stream);

/* MX scale rules: how the E8M0 exponent of a 1x32 block is derived from its
 * absolute maximum amax (0 for an all-zero block -> code 0x00 ... see
 * ga_quant_mxfp8). */
#define GA_MX_SCALE_FLOOR_448 0 /* e = floor(log2(amax / 448)), literal config rule */
#define GA_MX_SCALE_CEIL_448  1 /* e = ceil(log2(amax / 448)), never saturates     */
#define GA_MX_SCALE_OCP       2 /* e = floor(log2(amax)) - 8, OCP MX v1.0          */
/* For MXFP4 (ga_quant_mxfp4) the same rule numbers use the e2m1 maximum 6:
 * 0: floor(log2(amax / 6)), 1: ceil(log2(amax / 6)), 2: floor(log2(amax)) - 2. */

/* Input element types of the quantisers. */
#define GA_IN_F32  0
#define GA_IN_BF16 1

/* MXFP8 quantiser: x [rows, K] (row stride ld_x elements) -> q [rows, K]
 * E4M3 (row stride ld_q bytes) and scales [rows, K/32] E8M0 (row stride
 * ld_s bytes), unshuffled. K % 32 == 0. */
ga_status ga_quant_mxfp8(const void* x, int in_dtype, int rows, int K, int ld_x,
                         void* q, int ld_q, void* scales, int ld_s, int scale_rule,
                         void* stream);
/* ga_quant_mxfp8 with the element format: fmt 0 = E4M3 (ga_quant_mxfp8), 1 =
 * E5M2 (bf8, for ga_kernel_launch_fmt): round to nearest even, saturate to
 * +-57344, NaN -> 0x7F, scale rules with the E5M2 maximum 57344 = 1.75 * 2^15
 * in place of 448 (rule 2: floor(log2(amax)) - 15). No counterpart in the
 * reference (its quantisers produce E4M3 or e2m1). */
ga_status ga_quant_mx8(const void* x, int in_dtype, int rows, int K, int ld_x, void* q,
                       int ld_q, void* scales, int ld_s, int scale_rule, int fmt, void* stream);
/* MXFP4 quantiser: x [rows, K] -> q [rows, K/2] bytes of OCP e2m1 codes
 * (element 2i in the low nibble of byte i, asm_f4gemm/README.md:99; round to
 * nearest even, saturate to +-6, NaN -> signed zero; row stride ld_q bytes)
 * and scales [rows, K/32] E8M0 (rules above), unshuffled. K % 32 == 0. */
ga_status ga_quant_mxfp4(const void* x, int in_dtype, int rows, int K, int ld_x,
                         void* q, int ld_q, void* scales, int ld_s, int scale_rule,
                         void* stream);
/* DeepSeek activation quantiser: per 1x128 block along K, s = amax/448 (fp32),
 * q = e4m3(x / s). Scales are written transposed, sfa[k/128 * ld_s + row]
 * (opus SFA layout [K/128, M]). K % 128 == 0. */
ga_status ga_quant_fp8_1x128(const void* x, int in_dtype, int rows, int K, int ld_x,
                             void* q, int ld_q, float* sfa, int ld_s, void* stream);
/* DeepSeek weight quantiser: per 128x128 tile, s = amax/448, scales
 * sfb[(row/128) * ld_s + k/128] (opus SFB layout [ceil(N/128), K/128]). */
ga_status ga_quant_fp8_128x128(const void* x, int in_dtype, int rows, int K, int ld_x,
                               void* q, int ld_q, float* sfb, int ld_s, void* stream);
/* Per-tensor quantiser: s = amax/448 over the whole tensor, q = e4m3(x / s).
 * `scale` receives s (one float, device). `amax_ws` is a device scratch of at
 * least 4 bytes. */
ga_status ga_quant_fp8_per_tensor(const void* x, int in_dtype, size_t n, void* q,
                                  float* scale, void* amax_ws, void* stream);

/* ------------------------------------------------------------------------- */
/* GEMM entry points.                                                         */
/* ------------------------------------------------------------------------- */

/* Kernel registry: the compiled analogue of Kernel::load (f4gemm.hpp:277-295).
 * Finds a kernel by knl_name or co_name; GA_ERR_NO_KERNEL if absent. */
ga_status ga_kernel_find(const char* name, int* idx);

/* fp32 workspace needed for a launch (0 when gdz == 1). */
size_t ga_kernel_workspace_bytes(int idx, const ga_launch_desc* ld, int M, int N);

/* Kernel::launch (f4gemm.hpp:297-309): D[M,N] bf16 = alpha*A*B^T (+beta*C).
 * A [M, K] E4M3 row-major (stride_A0 elements), B [N, K] E4M3, preshuffled
 * when the kernel's bpreshuffle is 1, ScaleA/ScaleB E8M0 padded+shuffled
 * (stride_ScaleX0 = padded column count). MXFP4 kernels: A [M, K/2] and
 * B [N, K/2] bytes of packed e2m1 (B preshuffled over Kp = K/2 bytes),
 * strides still in elements, K % 256 == 0. With gdz > 1 the K-slices are
 * summed in fp32 in `workspace` (ga_kernel_workspace_bytes) and a reduce
 * kernel writes bf16 D; D need not be pre-zeroed. workspace == NULL with
 * gdz > 1 uses a library-owned per-device buffer (grown on demand), and is
 * refused with GA_ERR_WORKSPACE while `stream` is capturing a HIP graph.
 * Every such call on a device shares that buffer: split-K launches on
 * different streams that overlap in time race on it, so concurrent callers
 * pass their own workspace. */
ga_status ga_kernel_launch(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy,
                           int gdz, void* workspace, size_t workspace_bytes,
                           void* stream);

/* ga_kernel_launch with the split-K workspace found through a device slot
 * (ga_splitk_ws_handle, as the a16w16 split-K path takes it; no counterpart
 * in asm_f4gemm, whose kernels add K slices with bf16 atomics): the GEMM
 * kernels and the reduce read {ptr, bytes} from the slot when they run, so a
 * captured HIP graph keeps working after ga_ws_handle_reserve grows the
 * buffer. The slot must hold gdz * M * N floats (ga_kernel_workspace_bytes):
 * for a slot made by ga_ws_handle_create this is checked on the host
 * (GA_ERR_WORKSPACE) outside capture; a shorter slot met by the kernels makes
 * them write nothing. gdz == 1 uses no workspace, nor does a split at 1-16
 * rows (the decode kernel sums its K slices in the workgroup). */
ga_status ga_kernel_launch_ws_handle(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy,
                                     int gdz, const ga_splitk_ws_handle* ws_handle,
                                     void* stream);

/* ga_kernel_launch for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc); no
 * counterpart in the reference. Calls no hipMalloc/hipFree: with gdz > 1 the
 * split-K partials [gdz, M, N] fp32 go to a fixed 32 MiB device array of the
 * library (one per GPU it runs on, held until the process ends), so
 * gdz * M * N * 4 must be at most 33554432 bytes (GA_ERR_WORKSPACE
 * otherwise). Nothing in it needs to start at zero: every slice writes its
 * whole partial before the reduce reads it. Every call on a GPU shares that
 * array, so calls that overlap in time on one GPU (other streams, other host
 * threads) race: serialise them. Otherwise as ga_kernel_launch. */
ga_status ga_kernel_launch_noalloc(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy,
                                   int gdz, void* stream);

/* ga_kernel_launch with the 8-bit element format of each MXFP8 operand:
 * fmt_a (A) and fmt_b (B) are f8f6f4 format codes, 0 = E4M3 (fp8, what
 * ga_kernel_launch takes) or 1 = E5M2 (bf8), in any pairing; the E8M0 1x32
 * scales, layouts, preshuffle and split-K are those of ga_kernel_launch (an
 * E5M2 element is one byte too). Replaces the format-code arguments of the
 * reference's scaled-MFMA dispatch (wmma_opus_rdna4/opus/opus.hpp:1785-1786,
 * fmt_a / fmt_b of mfma_scale_f32_16x16x128_f8f6f4) at the GEMM level; the
 * reference's asm_f4gemm kernels have fixed formats. idx must be an MXFP8
 * registry entry (GA_ERR_ARG for MXFP4 kernels and other codes). Rows above
 * the decode path (M > 64) run the 256x256 eight-wave kernel whichever tile
 * idx names (the grid arguments are checked against idx as usual); every
 * MXFP8 kernel computes the same fp32 chain per K slice, so the output does
 * not depend on the tile. fmt_a = fmt_b = 0 is ga_kernel_launch. */
ga_status ga_kernel_launch_fmt(int idx, const ga_f4gemm_kargs* args, int gdx, int gdy, int gdz,
                               int fmt_a, int fmt_b, void* workspace, size_t workspace_bytes,
                               void* stream);

/* One-call MXFP8 GEMM: select_kernel + make_launch + fill_args + launch.
 * log2_k_split as in ga_select_kernel. Writes the chosen kernel index and
 * launch into *chosen / *ld_out when non-NULL. */
ga_status ga_mxfp8_gemm(void* d_D, const void* d_A, const void* d_B,
                        const void* d_ScaleA, const void* d_ScaleB, int M, int N, int K,
                        int stride_D0, int bpreshuffle, int log2_k_split, int num_cu,
                        void* workspace, size_t workspace_bytes, int* chosen,
                        ga_launch_desc* ld_out, void* stream);

/* The same over the MXFP4 manifest (asm_f4gemm/main.cpp's flow for its
 * f4gemm_bf16_per1x32Fp4 kernels): A/B packed e2m1, *chosen is the registry
 * index (ga_kernel_find numbering). */
ga_status ga_mxfp4_gemm(void* d_D, const void* d_A, const void* d_B,
                        const void* d_ScaleA, const void* d_ScaleB, int M, int N, int K,
                        int stride_D0, int bpreshuffle, int log2_k_split, int num_cu,
                        void* workspace, size_t workspace_bytes, int* chosen,
                        ga_launch_desc* ld_out, void* stream);

/* gemm_a8w8_blockscale_kernel (opus_gemm/block_scale_gemm, GROUP 1x128x128)
 * and gemm_a8w8_1x128x1_blockscale_kernel (GROUP 1x1x128):
 *   C[b,m,n] = sum_g (sum_{k in g} A*B) * SFA[g, m] * SFB[...]
 * A [batch, M, K] E4M3, B [batch, N, K] E4M3 (K-major, not preshuffled),
 * SFA [K/128, M] fp32 (stride_sfa = M), SFB [ceil(N/128), K/128] fp32
 * (group_n = 128, stride_sfb = K/128) or [K/128, N] (group_n = 1,
 * stride_sfb = N). C fp32 (reference) or bf16 (out_dtype). K % 128 == 0;
 * M and N are arbitrary (a partial last N-group is allowed). */
ga_status ga_gemm_a8w8_blockscale(const ga_opus_gemm_kargs* kargs, int group_n,
                                  int out_dtype, void* stream);

/* fp8_gemm per-tensor path: C = sfa[0] * sfb[0] * A * B^T. ptr_sfa/ptr_sfb
 * each point at one device fp32. B [N, K] K-major. */
ga_status ga_fp8_gemm_per_tensor(const ga_opus_gemm_kargs* kargs, int out_dtype,
                                 void* stream);

/* Summation order of the two calls above (no counterpart in the reference,
 * whose kernel sums K in one chain): the kernel chosen for these kargs on the
 * current device sums K in slices of *groups_per_slice 128-K groups, each
 * slice in one fp32 chain, and adds the slices in order. K / 128 means one
 * chain. Lets a caller (or a test) reproduce the rounding exactly. */
ga_status ga_blockscale_k_slices(const ga_opus_gemm_kargs* kargs, int* groups_per_slice);

/* ga_gemm_a8w8_blockscale with a caller workspace, which lets long-K
 * problems whose 256x256 tiles would keep few CUs busy (batch 1, more than
 * 64 rows, tiles for at most 40 % of the CUs, at least 16 128-K groups per
 * CU; e.g. 2048x2560x8192: 80 tiles on 256 CUs, 103 -> 84 us on MI355X)
 * run in stream-K form: every CU takes an equal share of the tiles' 128-K
 * groups, and a tile cut between CUs is summed from fp32 partials in K
 * order by the last CU to finish it (the DeepSeek configuration shapes are
 * not among them: their partial traffic costs as much as the balance
 * gains). The reference's kernel has no split, and its cross-workgroup
 * counter (wmma_opus_rdna4/opus/opus.hpp:1296-1304) spins, where here nobody
 * waits. workspace: ga_blockscale_workspace_bytes bytes (up to about 128
 * MiB), zero-filled before its first use (on the call's stream, or waited
 * for before the call: a hipMemset queues on the null stream, which does not
 * order against non-blocking streams) and left zero-filled by every call;
 * calls that overlap in time must not share it. workspace NULL,
 * or a shape the whole-tile kernel suits, runs exactly
 * ga_gemm_a8w8_blockscale; a workspace that is too small is
 * GA_ERR_WORKSPACE. Summation order: ga_blockscale_stream_k. */
ga_status ga_gemm_a8w8_blockscale_ws(const ga_opus_gemm_kargs* kargs, int group_n, int out_dtype,
                                     void* workspace, size_t workspace_bytes, void* stream);

/* Workspace ga_gemm_a8w8_blockscale_ws can use for these kargs on the
 * current device (0: it runs the whole-tile kernel). */
ga_status ga_blockscale_workspace_bytes(const ga_opus_gemm_kargs* kargs, size_t* bytes);

/* No counterpart in the reference (whose cross-workgroup counter has no
 * misuse report). Reports whether a stream-K call of
 * ga_gemm_a8w8_blockscale_ws on this workspace found a tile counter that had
 * not started at zero (a workspace not zero-filled, e.g. reused for other
 * data, or shared by overlapping calls): such a call leaves some of its tiles
 * unsummed, and the kernel records it in a word after the counters. Waits for
 * the stream, then returns GA_OK, or GA_ERR_WORKSPACE after zero-filling the
 * counters and the word again on that stream and waiting for it. GA_OK at once when these kargs take no
 * stream-K plan or workspace is NULL; GA_ERR_ARG under stream capture. */
ga_status ga_blockscale_workspace_check(const ga_opus_gemm_kargs* kargs, void* workspace,
                                        size_t workspace_bytes, void* stream);

/* Stream-K plan of ga_gemm_a8w8_blockscale_ws (given a workspace) on the
 * current device: *workgroups = P, or 0 when that call runs whole tiles.
 * With G = K/128 and T = tiles * G, iteration t*G + g is 128-K group g of
 * tile t, and workgroup v computes iterations [floor(v*T/P),
 * floor((v+1)*T/P)). Tiles are numbered in bands of four tile rows, column
 * by column within a band: with r = t % (4*tiles_n) and h the band's height
 * (4, or fewer in the last band), tile_m = 4*(t / (4*tiles_n)) + r % h and
 * tile_n = r / h. A tile's K is cut where its iterations change workgroup;
 * each piece is one fp32 chain and the pieces are added in K order. */
ga_status ga_blockscale_stream_k(const ga_opus_gemm_kargs* kargs, int* workgroups);

/* splitk_reduce_kernel: C[b, m, n] = sum_s ws[s, b, m, n] (+ bias[n]) in fp32,
 * cast to out_dtype. ws is [split_k, batch, padded_M, padded_N] fp32. bias
 * may be NULL; bias_dtype is GA_DTYPE_BF16/F32; bias_stride_batch 0 means
 * one [N] bias for every batch. */
ga_status ga_splitk_reduce(const float* ws, void* c_out, int out_dtype, int split_k,
                           int M, int N, int batch, int padded_M, int padded_N,
                           const void* bias, int bias_dtype, int bias_stride_batch,
                           void* stream);

/* splitk_reduce_kernel as the reference launches it: the workspace is found
 * through the device slot `ws_handle` at kernel entry (graph-capture safe).
 * Reads that would pass the slot's `bytes` are not made: the kernel then
 * writes nothing. Otherwise as ga_splitk_reduce.
 * Replaces splitk_reduce_gfx950.cuh:68-259 with its handle argument. */
ga_status ga_splitk_reduce_ws_handle(const ga_splitk_ws_handle* ws_handle, void* c_out,
                                     int out_dtype, int split_k, int M, int N, int batch,
                                     int padded_M, int padded_N, const void* bias,
                                     int bias_dtype, int bias_stride_batch, void* stream);

/* gemm_a16w16_flatmm_splitk_kernel (opus_gemm_dist/opus_gemm_mem_gemm_a2a,
 * pipeline .cuh:204-563; launch main.cc:299-318): bf16 A [batch, M, K] times
 * bf16 B [batch, N, K]^T, K split into split_k slices; slice s writes its
 * fp32 partial to workspace[s, b, m, n] (found through kargs->ws_handle).
 * Slices follow the reference's partition: K in 128-element iterations,
 * ceil(iters / split_k) per slice, the last slice takes the remainder; a
 * slice left empty writes zeros (the reference writes nothing there).
 * Requirements: M, N, K, batch, split_k > 0; K % 8 == 0; stride_a and
 * stride_b >= K and multiples of 8; ptr_a / ptr_b 16-byte aligned;
 * stride_ws >= N; stride_ws_batch >= M * stride_ws. The workspace must hold
 * split_k * batch * stride_ws_batch floats (checked in the kernel against
 * the slot's bytes: a slot too small makes it write nothing). ptr_c, ptr_bias
 * are not read here. */
ga_status ga_gemm_a16w16_flatmm_splitk(const ga_flatmm_splitk_kargs* kargs, void* stream);

/* The reference's launch_once pair (main.cc:299-318): the split-K kernel,
 * then the reduce into bf16 C with the optional bf16 bias of kargs (C rows
 * stride_c apart, batches stride_c_batch apart). With split_k == 1 the GEMM
 * writes C (and the bias) directly and the workspace is not touched. */
ga_status ga_gemm_a16w16_splitk(const ga_flatmm_splitk_kargs* kargs, void* stream);

/* fp32 workspace bytes the kargs' layout needs:
 * split_k * batch * stride_ws_batch * 4. */
size_t ga_a16w16_splitk_workspace_bytes(const ga_flatmm_splitk_kargs* kargs);

/* Workspace slot management (the caller-side half of the handle protocol,
 * which the reference leaves to its caller, main.cc:244-264):
 *   create   allocates a device slot {NULL, 0};
 *   reserve  makes the slot's workspace at least `bytes`: when it grows, the
 *            device is synchronised, a new buffer is allocated, the slot is
 *            rewritten and the old buffer is freed. Graphs captured earlier
 *            read the new buffer on their next replay. Not capturable.
 *   query    the slot's current {ptr, bytes} (host-side mirror);
 *   destroy  synchronises and frees the workspace and the slot. */
ga_status ga_ws_handle_create(ga_splitk_ws_handle** ws_handle);
ga_status ga_ws_handle_reserve(ga_splitk_ws_handle* ws_handle, size_t bytes);
ga_status ga_ws_handle_query(const ga_splitk_ws_handle* ws_handle, void** ptr, size_t* bytes);
ga_status ga_ws_handle_destroy(ga_splitk_ws_handle* ws_handle);

/* Device count of compute units of the current device (hipDeviceProp). */
ga_status ga_device_num_cu(int* num_cu);

#ifdef __cplusplus
}
#endif

#endif /* GCNASM_AMD_H */

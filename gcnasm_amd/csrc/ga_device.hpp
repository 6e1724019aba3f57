// ga_device.hpp -- gfx950 device primitives shared by the HIP kernels.
//
// Buffer resources with out-of-range-returns-zero loads, direct-to-LDS
// 16-byte loads, explicit s_waitcnt, the scaled MFMA, and exact codecs
// (E4M3 RNE/saturating encode, bf16 RNE). The primitive set follows what
// the reference's opus.hpp exposes (wmma_opus_rdna4/opus/opus.hpp:1358-1569
// gmem/async-LDS loads, :1726-1733 waitcnt, :1770-1863 scaled MFMA); the
// code is written for gfx950 only.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/gcnasm_amd.h"
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace ga {

// Compile-time loop: f(std::integral_constant<int, 0>{}) ... f(<N-1>).
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>)
{
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f)
{
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer resource: base, size in bytes; loads at offset >= size return 0.
// Word 3 (0x00020000) is the raw-buffer format word for gfx9 parts. Callers
// pass workgroup-uniform values; readfirstlane makes that visible to the
// compiler so the descriptor lives in SGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    const uint64_t p = (uint64_t)(uintptr_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    const uint64_t up = ((uint64_t)hi << 32) | lo;
    return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)up, (short)0,
                                             (int)__builtin_amdgcn_readfirstlane(bytes),
                                             0x00020000);
}

// Split-K workspace found through a device slot {ptr, bytes} at kernel entry
// (graph-capture safe): the slot's buffer when it holds the [gdz, M, N] fp32
// layout, else null (the caller then writes nothing).
__device__ __forceinline__ float* resolve_ws(const ga_splitk_ws_handle* h, uint32_t gdz,
                                             uint32_t M, uint32_t N)
{
    float* ws = (float*)h->ptr;
    const uint64_t need = (uint64_t)gdz * M * N * 4u;
    return (ws == nullptr || h->bytes < need) ? nullptr : ws;
}

// 16 bytes per lane from buffer `r` at byte offset voff+soff into LDS at
// lds_base + lane*16 (lds_base wave-uniform; M0 takes it). The range check
// covers voff + soff (checked on MI355X: lanes whose voff alone is in range
// but voff + soff is not read zeros), so a wave-uniform part of the offset
// can go in soff without a VALU add.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, lds_void* lds_base,
                                           uint32_t voff, uint32_t soff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_base, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ v4i buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

// Streaming variant for data read once: the non-temporal cache policy bit
// (gfx950 "nt") so the stream does not evict reused lines.
__device__ __forceinline__ v4i buf_load16_stream(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                 uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);
}

__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

// s_waitcnt encodings for gfx9: vmcnt[3:0] + vmcnt_hi[15:14], expcnt[6:4],
// lgkmcnt[11:8]. Only vmcnt is waited on here.
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for LDS handoff without a memory-model fence: the fence
// of __syncthreads() also drains every outstanding direct-to-LDS load
// (vmcnt(0)), which would serialise a multi-stage pipeline. Callers wait for
// the loads they need with wait_vmcnt<N>() first; the "memory" clobber keeps
// the compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void barrier_lds()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ void wait_lgkmcnt0()
{
    __builtin_amdgcn_s_waitcnt((0xF) | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));
}

// D = A(16x128) * B(128x16) + C with per-lane E8M0 scales (fp8 operands).
// Lane l = 16*g + r holds row r: VGPRs 0-3 carry K [16g, 16g+16), VGPRs 4-7
// carry K [64+16g, 64+16g+16). The scale byte (chosen by OPSEL) of the scale
// VGPR of lane 16*b + r applies to row r, K [32b, 32b+32). Output: lane l
// holds D[4*(l/16) + j][l%16], j = 0..3.
// FMT_A / FMT_B: the operands' f8f6f4 format codes, 0 E4M3 or 1 E5M2 (one
// byte per element either way, so the lane layout is the same).
template <int OPSEL_A, int OPSEL_B, int FMT_A = 0, int FMT_B = 0>
__device__ __forceinline__ v4f mfma_mx16(v8i a, v8i b, v4f c, int sa, int sb)
{
    static_assert(FMT_A >= 0 && FMT_A <= 1 && FMT_B >= 0 && FMT_B <= 1, "8-bit formats");
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT_A, FMT_B, OPSEL_A, sa,
                                                            OPSEL_B, sb);
}

// A GEMM's operand formats as one template value F = fmt(A) | fmt(B) << 1
// (0 E4M3, 1 E5M2). The kernels put B on the MFMA's first operand, so its
// format is the instruction's first code.
constexpr int fmt_of_a(int F) { return F & 1; }
constexpr int fmt_of_b(int F) { return (F >> 1) & 1; }

// Same with fp4 (e2m1) operands: lane l = 16*g + r holds row r, K
// [32g, 32g+32) in its first 16 bytes (two elements per byte, low nibble
// first); the last 16 bytes of the operand are not read. Scales and output as
// above.
template <int OPSEL_A, int OPSEL_B>
__device__ __forceinline__ v4f mfma_mx16_fp4(v8i a, v8i b, v4f c, int sa, int sb)
{
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 4, OPSEL_A, sa, OPSEL_B,
                                                            sb);
}

// D = A(16x32) * B(32x16) + C with bf16 operands: lane l = 16*g + r holds
// row r, K [8g, 8g+8) (16 bytes). Output as above: lane l holds
// D[4*(l/16) + j][l%16].
typedef __bf16 v8bf16 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ v4f mfma_bf16_16x16x32(v4i a, v4i b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf16, a),
                                                   __builtin_bit_cast(v8bf16, b), c, 0, 0, 0);
}

// The last 16 bytes of a fragment moved to its first 16 (the fp4 operand
// of the second 128-K half).
__device__ __forceinline__ v8i hi16(v8i x)
{
    return (v8i){x[4], x[5], x[6], x[7], 0, 0, 0, 0};
}

// fp32 -> bf16 round to nearest even (quiet NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float x)
{
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u)
        return (uint16_t)((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// OCP E4M3 encode: round to nearest even, saturate to +-448, NaN -> 0x7F.
__device__ __forceinline__ uint32_t e4m3_encode(float x)
{
    uint32_t u = __float_as_uint(x);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t au = u & 0x7FFFFFFFu;
    if (au > 0x7F800000u)
        return 0x7Fu;
    if (au >= 0x43E00000u) // 448.0f
        return sign | 0x7Eu;
    if (au < 0x3C800000u) { // 2^-6: subnormal quantum 2^-9
        float f = __uint_as_float(au) * 512.0f;
        uint32_t i = (uint32_t)f;
        float frac = f - (float)i;
        if (frac > 0.5f || (frac == 0.5f && (i & 1u)))
            i++;
        return sign | i;
    }
    int e = (int)(au >> 23) - 127;
    uint32_t keep = (au >> 20) & 7u, rest = au & 0xFFFFFu;
    if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u)))
        keep++;
    if (keep == 8u) {
        keep = 0;
        e++;
    }
    uint32_t code = ((uint32_t)(e + 7) << 3) | keep;
    return sign | (code > 0x7Eu ? 0x7Eu : code);
}

// Four E4M3 codes packed little-endian, same results as e4m3_encode: the
// hardware converter (v_cvt_pk_fp8_f32: OCP E4M3, round to nearest even) on
// inputs clamped to +-448 (saturation), NaN inputs replaced by 0x7F after.
__device__ __forceinline__ uint32_t e4m3_encode4(float a, float b, float c, float d)
{
    const float x[4] = {a, b, c, d};
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        y[j] = __builtin_fminf(__builtin_fmaxf(x[j], -448.0f), 448.0f);
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], lo, true);
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (x[j] != x[j])
            r = (r & ~(0xFFu << (8 * j))) | (0x7Fu << (8 * j));
    return r;
}

// Four E5M2 (bf8) codes as one dword, same results as the oracle's E5M2
// encode: the hardware converter on inputs clamped to +-57344 (saturation;
// the converter alone would round past the maximum to inf), NaN -> 0x7F.
__device__ __forceinline__ uint32_t e5m2_encode4(float a, float b, float c, float d)
{
    const float x[4] = {a, b, c, d};
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        y[j] = __builtin_fminf(__builtin_fmaxf(x[j], -57344.0f), 57344.0f);
    const int lo = __builtin_amdgcn_cvt_pk_bf8_f32(y[0], y[1], 0, false);
    uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(y[2], y[3], lo, true);
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (x[j] != x[j])
            r = (r & ~(0xFFu << (8 * j))) | (0x7Fu << (8 * j));
    return r;
}

// Four e2m1 codes as 16 bits (element j in bits 4j..4j+3), same results as
// e2m1_encode: the hardware converter (v_cvt_scalef32_pk_fp4_f32, scale 1)
// on inputs clamped to +-6, NaN inputs replaced by a zero of their sign.
__device__ __forceinline__ uint32_t e2m1_encode4(float a, float b, float c, float d)
{
    const float x[4] = {a, b, c, d};
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        y[j] = x[j] != x[j] ? __builtin_copysignf(0.0f, x[j])
                            : __builtin_fminf(__builtin_fmaxf(x[j], -6.0f), 6.0f);
    uint32_t r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, y[0], y[1], 1.0f, 0);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(r, y[2], y[3], 1.0f, 1);
    return r & 0xFFFFu;
}

// Exact floor(log2 a) and 23 fraction bits for a finite a > 0.
__device__ __forceinline__ void log2_parts(float a, int& E, uint32_t& frac)
{
    uint32_t u = __float_as_uint(a) & 0x7FFFFFFFu;
    int ef = (int)(u >> 23);
    if (ef > 0) {
        E = ef - 127;
        frac = u & 0x7FFFFFu;
    } else {
        uint32_t mant = u & 0x7FFFFFu;
        int msb = 31 - __clz(mant);
        E = msb - 149;
        frac = (mant << (23 - msb)) & 0x7FFFFFu;
    }
}

// E8M0 exponent of an MX block whose element format has largest value
// (1 + FRAC/2^23) * 2^EMAX: rule 0: floor(log2(amax/max)), 1: ceil, 2: OCP
// floor(log2 amax) - EMAX. Zero block -> -127.
template <uint32_t FRAC, int EMAX>
__device__ __forceinline__ int mx_scale_exp_t(float amax, int rule)
{
    if (!(amax > 0.0f))
        return -127;
    if (__float_as_uint(amax) == 0x7F800000u)
        return 127;
    int E;
    uint32_t f;
    log2_parts(amax, E, f);
    int e;
    if (rule == 0)
        e = (f >= FRAC) ? E - EMAX : E - EMAX - 1;
    else if (rule == 1)
        e = (f <= FRAC) ? E - EMAX : E - EMAX + 1;
    else
        e = E - EMAX;
    return e < -127 ? -127 : (e > 127 ? 127 : e);
}

// E4M3: 448 = 1.75 * 2^8.
__device__ __forceinline__ int mx_scale_exp(float amax, int rule)
{
    return mx_scale_exp_t<0x600000u, 8>(amax, rule);
}

// E5M2: 57344 = 1.75 * 2^15.
__device__ __forceinline__ int mx5_scale_exp(float amax, int rule)
{
    return mx_scale_exp_t<0x600000u, 15>(amax, rule);
}

// E2M1: 6 = 1.5 * 2^2.
__device__ __forceinline__ int mx4_scale_exp(float amax, int rule)
{
    return mx_scale_exp_t<0x400000u, 2>(amax, rule);
}

// OCP E2M1 encode (MXFP4 element; values 0, .5, 1, 1.5, 2, 3, 4, 6, sign in
// bit 3): round to nearest, ties to the even code, saturate to +-6. E2M1 has
// no NaN: NaN gives a zero with its sign bit.
__device__ __forceinline__ uint32_t e2m1_encode(float x)
{
    const uint32_t u = __float_as_uint(x);
    const float a = __uint_as_float(u & 0x7FFFFFFFu);
    const uint32_t c = (uint32_t)(a > 0.25f) + (uint32_t)(a >= 0.75f) + (uint32_t)(a > 1.25f) +
                       (uint32_t)(a >= 1.75f) + (uint32_t)(a > 2.5f) + (uint32_t)(a >= 3.5f) +
                       (uint32_t)(a > 5.0f);
    return ((u >> 28) & 8u) | c;
}

// Linear tile id -> (tile_m, tile_n) on a gdx x gdy tile grid. Workgroup ids
// are dispatched round-robin over the 8 XCDs; the remap gives each XCD a
// contiguous range of tiles, swept column by column inside groups of
// `group_m` M-tiles so the workgroups resident on one XCD share A and B
// panels in its L2.
__device__ __forceinline__ void map_tile_lin(int lin, int gdx, int gdy, int group_m, int& tm,
                                             int& tn)
{
    const int total = gdx * gdy;
    const int full = (total / 8) * 8;
    if (lin < full)
        lin = (lin % 8) * (total / 8) + lin / 8;
    const int per_group = group_m * gdx;
    const int g = lin / per_group;
    const int first_m = g * group_m;
    const int gsize = min(gdy - first_m, group_m);
    const int r = lin - g * per_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

__device__ __forceinline__ void map_tile(int bx, int by, int gdx, int gdy, int group_m, int& tm,
                                         int& tn)
{
    map_tile_lin(by * gdx + bx, gdx, gdy, group_m, tm, tn);
}

} // namespace ga

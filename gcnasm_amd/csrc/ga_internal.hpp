// ga_internal.hpp -- host-side internals shared by the library's translation
// units: error reporting, the compiled kernel registry, workspace handling.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>

#include "../../include/gcnasm_amd.h"

namespace ga {

// Records a formatted detail message for ga_last_error() and returns `s`.
ga_status fail(ga_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
ga_status hip_fail(hipError_t e, const char* what);

#define GA_HIP_CHECK(call)                                  \
    do {                                                    \
        hipError_t e_ = (call);                             \
        if (e_ != hipSuccess)                               \
            return ::ga::hip_fail(e_, #call);               \
    } while (0)

// One compiled MX kernel: the manifest row plus its launcher.
// ws: the split-K workspace, or (wsh set) found through the device slot wsh at
// kernel entry, where a slot shorter than the layout makes the kernel write nothing.
typedef void (*mx_launch_fn)(const ga_f4gemm_kargs& args, float* ws,
                             const ga_splitk_ws_handle* wsh, int gdx, int gdy, int gdz,
                             hipStream_t stream);
struct MxKernel {
    ga_tile_config cfg;
    mx_launch_fn launch;
    int small_m_stream; // M up to this many rows goes to the decode path (launch_mx_decode)
    int elem_bits;      // 8: E4M3 operands, 4: e2m1 packed two per byte
    bool by_shape;      // a tile known by name: runs the compiled tile the heuristic picks
};
// 256x256 eight-wave kernels (gemm_mx_pp.hip), preshuffled / plain B.
void launch_mx_pp_bps(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                      int gdx, int gdy, int gdz, hipStream_t stream);
void launch_mx_pp_nobps(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                        int gdx, int gdy, int gdz, hipStream_t stream);
// The same tile for MXFP4 operands (e2m1, packed two per byte).
void launch_mx4_pp_bps(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                       int gdx, int gdy, int gdz, hipStream_t stream);
void launch_mx4_pp_nobps(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                         int gdx, int gdy, int gdz, hipStream_t stream);
// Small-M (decode) path shared by the kernels (gemm_mx_decode.hip): streams B
// into registers, K slices summed in the workgroup (no workspace). Results
// equal the tile kernels' (one fp32 chain of 128-K steps per slice).
bool mx_decode_applies(const ga_f4gemm_kargs& args, int gdz);
void launch_mx_decode(const ga_f4gemm_kargs& args, int gdz, bool bps, bool fp4, int fmt,
                      int num_cu, hipStream_t stream);
// 17-64 rows, each wave over ng (2-8) 16-column groups, the caller's gdz K
// slices on phys workgroups along K, each running ceil(gdz / phys)
// consecutive slices as separate fp32 chains (gemm_mx_decode.hip):
// mx_decode_split_groups gives ng and phys for the shape (ng 0: not this
// path). With phys > 1 each slice's fp32 partials go to the split-K
// workspace (ws, or the slot wsh) for the split-K reduce; with phys = 1 the
// kernel sums the slices in order and applies the epilogue, no workspace
// (33-64 rows: in the shared-A variant, four waves per workgroup sharing A
// through LDS, sized from num_cu).
int mx_decode_split_groups(const ga_f4gemm_kargs& args, int gdz, int num_cu, int* phys);
void launch_mx_decode_split(const ga_f4gemm_kargs& args, int gdz, int phys, int ng, bool bps,
                            bool fp4, int fmt, float* ws, const ga_splitk_ws_handle* wsh,
                            int num_cu, hipStream_t stream);
// fmt (the decode entry points and launch_mx_pp_fmt): MXFP8 operand element
// formats, fmt(A) | fmt(B) << 1 with 0 E4M3, 1 E5M2; 0 for MXFP4.
// 256x256 eight-wave kernel with operand formats fmt, grid of its own tiles.
void launch_mx_pp_fmt(const ga_f4gemm_kargs& args, float* ws, const ga_splitk_ws_handle* wsh,
                      int gdz, bool bps, int fmt, hipStream_t stream);

// Compute units of the current device (queried once per device).
ga_status device_cu_count(int* num_cu);
// 256x256 eight-wave fp32-scaled FP8 GEMM (gemm_bs_pp.hip); mode 0 = block
// scale GROUP_N 128, 1 = GROUP_N 1, 2 = per-tensor.
void launch_bs_pp(const ga_opus_gemm_kargs& ka, int mode, int out_dtype, hipStream_t stream);
// The same kernel's stream-K form (batch 1): workgroups it would use on
// num_cu CUs (0: the whole-tile form is the better one), its workspace
// (per-tile counters, zero between calls, then 2 * nwg fp32 partial tiles),
// the counters' share of it, and the launch.
int bs_sk_workgroups(const ga_opus_gemm_kargs& ka, int num_cu);
size_t bs_sk_counter_bytes(const ga_opus_gemm_kargs& ka);
size_t bs_sk_workspace_bytes(const ga_opus_gemm_kargs& ka, int nwg);
void launch_bs_pp_sk(const ga_opus_gemm_kargs& ka, int mode, int out_dtype, int nwg, void* ws,
                     hipStream_t stream);
// The same GEMMs for up to 64 rows, streaming B (gemm_bs_decode.hip); same
// mode numbering.
ga_status launch_bs_decode(const ga_opus_gemm_kargs& ka, int mode, int out_dtype,
                           hipStream_t stream);
// 128-K groups per K slice of that kernel (slices are summed in order).
int bs_decode_groups_per_slice(const ga_opus_gemm_kargs& ka, int num_cu);
int mx_registry_count();  // MXFP8 manifest rows (registry entries [0, count))
int mx_registry_total();  // every registry entry (manifests + kernels reachable by name)
const MxKernel* mx_registry_get(int idx);
int mx4_registry_first(); // MXFP4 manifest rows: entries [first, first + count)
int mx4_registry_count();

// Current bytes of a workspace slot made by ga_ws_handle_create (host mirror);
// false for a slot the caller made itself.
bool ws_slot_bytes(const ga_splitk_ws_handle* slot, size_t* bytes);

// Library-owned per-device fp32 workspace, grown on demand.
ga_status default_workspace(size_t bytes, void** ptr);

// Split-K reduce with the MX epilogue folded in:
//   out[b, m, n] = alpha * sum_s ws[s, b, m, n] (+ bias[n]) (+ beta * c_in[b, m, n])
// ws[s, b, m, n] is at (s * batch + b) * ws_batch + m * ws_ld + n; out/c_in
// rows are `ldc` elements apart and batches `c_batch_stride` elements apart.
// With `wsh` set, ws is read from that device slot at kernel entry (and
// nothing is written when the slot's bytes are short of the layout).
struct ReduceArgs {
    const float* ws;
    const ga_splitk_ws_handle* wsh;
    void* out;
    const void* c_in;  // bf16, may be null
    const void* bias;  // may be null
    int out_dtype;
    int bias_dtype;
    int split_k, M, N, batch, ldc;
    long long ws_ld, ws_batch;
    long long c_batch_stride;
    int bias_stride_batch;
    float alpha, beta;
    int tpr_log2;  // threads per output row (set by splitk_reduce_launch)
};
ga_status splitk_reduce_launch(const ReduceArgs& a, hipStream_t stream);

} // namespace ga

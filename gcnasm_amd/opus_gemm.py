"""Host interface of the fp32-scale FP8 GEMMs, mirroring the reference's opus_gemm drivers.

  opus_gemm_kargs               opus_gemm/block_scale_gemm/gemm_a8w8_blockscale_common.h:4-25
  gemm_a8w8_blockscale          opus_gemm/block_scale_gemm/gemm_a8w8_blockscale_host.cc:228-257
                                (GROUP 1x128x128)
  gemm_a8w8_1x128x1_blockscale  opus_gemm/block_scale_1x128x1_gemm/..._host.cc:202-231
                                (GROUP 1x1x128)
  fp8_gemm                      opus_gemm/fp8_gemm/rebuild.sh:3-11 (per-tensor scales)

Argument validation mirrors the reference drivers' checks (positive sizes,
K % GROUP_K) and raises GaError instead of returning 1.
"""
import ctypes

from . import _lib
from ._lib import OpusGemmKargs as opus_gemm_kargs  # noqa: N813 (reference name)
from ._lib import check, lib
from .f4gemm import _stream_handle


def make_kargs(a, b, c, sfa, sfb, m, n, k, batch=1, group_n=128):
    """kargs with the reference drivers' dense strides (host.cc:228-247).

    a [batch, M, K], b [batch, N, K] E4M3 (uint8 tensors); c [batch, M, N];
    sfa [batch, K/128, M] fp32; sfb [batch, ceil(N/128), K/128] (group_n 128)
    or [batch, K/128, N] (group_n 1). Per-tensor: sfa, sfb one fp32 each.
    The struct keeps the tensors alive for as long as it lives.
    """
    kg = k // 128
    ka = opus_gemm_kargs()
    ka.ptr_a, ka.ptr_b, ka.ptr_c = a.data_ptr(), b.data_ptr(), c.data_ptr()
    ka.m, ka.n, ka.k, ka.batch = m, n, k, batch
    ka.stride_a, ka.stride_b, ka.stride_c = k, k, n
    ka.stride_a_batch, ka.stride_b_batch, ka.stride_c_batch = m * k, n * k, m * n
    ka.ptr_sfa, ka.ptr_sfb = sfa.data_ptr(), sfb.data_ptr()
    if group_n == 128:
        ng = (n + 127) // 128
        ka.stride_sfa, ka.stride_sfb = m, kg
        ka.stride_sfa_batch, ka.stride_sfb_batch = m * kg, ng * kg
    elif group_n == 1:
        ka.stride_sfa, ka.stride_sfb = m, n
        ka.stride_sfa_batch, ka.stride_sfb_batch = m * kg, n * kg
    else:  # per-tensor: one scalar each
        ka.stride_sfa = ka.stride_sfb = ka.stride_sfa_batch = ka.stride_sfb_batch = 0
    # the struct holds raw device pointers: keep the tensors alive with it
    ka._tensors = (a, b, c, sfa, sfb)
    return ka


def _out_dtype(c):
    import torch
    if c.dtype == torch.float32:
        return _lib.GA_DTYPE_F32
    if c.dtype == torch.bfloat16:
        return _lib.GA_DTYPE_BF16
    raise TypeError("C must be float32 or bfloat16")


def gemm_a8w8_blockscale(kargs, out_dtype, group_n=128, stream=None, workspace=None):
    """gemm_a8w8_blockscale_kernel; with `workspace` (a zero-filled device
    tensor of workspace_bytes(kargs) bytes, kept zero-filled by the calls)
    ga_gemm_a8w8_blockscale_ws, which may run the stream-K form."""
    if workspace is None:
        check(lib().ga_gemm_a8w8_blockscale(ctypes.byref(kargs), group_n, out_dtype,
                                            _stream_handle(stream)))
        return
    check(lib().ga_gemm_a8w8_blockscale_ws(ctypes.byref(kargs), group_n, out_dtype,
                                           ctypes.c_void_p(workspace.data_ptr()),
                                           workspace.numel() * workspace.element_size(),
                                           _stream_handle(stream)))


def workspace_check(kargs, workspace, stream=None):
    """ga_blockscale_workspace_check: raises (GA_ERR_WORKSPACE) when a
    stream-K call on `workspace` found its tile counters not zero-filled, and
    zero-fills them again; waits for the stream."""
    check(lib().ga_blockscale_workspace_check(ctypes.byref(kargs),
                                              ctypes.c_void_p(workspace.data_ptr()),
                                              workspace.numel() * workspace.element_size(),
                                              _stream_handle(stream)))


def workspace_bytes(kargs):
    """Bytes ga_gemm_a8w8_blockscale_ws can use for these kargs (0: none)."""
    n = ctypes.c_size_t(0)
    check(lib().ga_blockscale_workspace_bytes(ctypes.byref(kargs), ctypes.byref(n)))
    return n.value


def stream_k_workgroups(m, n, k, batch=1):
    """Workgroups of the stream-K form ga_gemm_a8w8_blockscale_ws runs for
    these sizes on the current device (0: whole tiles)."""
    ka = opus_gemm_kargs()
    ka.m, ka.n, ka.k, ka.batch = m, n, k, batch
    w = ctypes.c_int(0)
    check(lib().ga_blockscale_stream_k(ctypes.byref(ka), ctypes.byref(w)))
    return w.value


def stream_k_cuts(m, n, k, workgroups):
    """{(tile_m, tile_n): [first 128-K group of each K piece]} of the stream-K
    plan (ga_blockscale_stream_k's documented order) with `workgroups`
    workgroups: a tile's K pieces are summed in this order."""
    tn, tm, G = (n + 255) // 256, (m + 255) // 256, k // 128
    T = tn * tm * G
    begins = [v * T // workgroups for v in range(workgroups)]
    cuts = {}
    for t in range(tn * tm):
        band = 4 * tn
        first_m = 4 * (t // band)
        h = min(tm - first_m, 4)
        r = t % band
        key = (first_m + r % h, r // h)
        cuts[key] = [0] + sorted(b - t * G for b in begins if t * G < b < (t + 1) * G)
    return cuts


def gemm_a8w8_1x128x1_blockscale(kargs, out_dtype, stream=None):
    gemm_a8w8_blockscale(kargs, out_dtype, group_n=1, stream=stream)


def fp8_gemm(kargs, out_dtype, stream=None):
    check(lib().ga_fp8_gemm_per_tensor(ctypes.byref(kargs), out_dtype, _stream_handle(stream)))


def blockscale_gemm(a, b, sfa, sfb, c, group_n=128, stream=None, workspace=None):
    """Tensor-level wrapper: a [B,M,K] or [M,K] uint8 E4M3, c fp32/bf16;
    `workspace` as for gemm_a8w8_blockscale."""
    batch = a.shape[0] if a.dim() == 3 else 1
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-2]
    ka = make_kargs(a, b, c, sfa, sfb, m, n, k, batch, group_n)
    gemm_a8w8_blockscale(ka, _out_dtype(c), group_n, stream, workspace)
    return c


def per_tensor_gemm(a, b, sa, sb, c, stream=None):
    batch = a.shape[0] if a.dim() == 3 else 1
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-2]
    ka = make_kargs(a, b, c, sa, sb, m, n, k, batch, group_n=0)
    fp8_gemm(ka, _out_dtype(c), stream)
    return c


def k_slices(m, n, k, batch=1):
    """128-K groups per K slice of the kernel these sizes run on the current
    device (ga_blockscale_k_slices; K // 128 means one fp32 chain)."""
    ka = opus_gemm_kargs()
    ka.m, ka.n, ka.k, ka.batch = m, n, k, batch
    g = ctypes.c_int(0)
    check(lib().ga_blockscale_k_slices(ctypes.byref(ka), ctypes.byref(g)))
    return g.value

"""Host interface of the bf16 split-K GEMM and its graph-safe workspace handle.

Mirrors the reference's a16w16 flatmm split-K path:

  opus_splitk_ws_handle             opus_gemm_dist/opus_gemm_mem_gemm_a2a/include/gfx950/
                                    opus_gemm_traits_a16w16_gfx950.cuh:588-597
  opus_gemm_flatmm_splitk_kargs     (same file):599-634
  gemm_a16w16_flatmm_splitk_kernel  .../opus_gemm_pipeline_a16w16_flatmm_splitk_gfx950.cuh:204-563
  splitk_reduce_kernel              .../splitk_reduce_gfx950.cuh:68-259
  launch_once (GEMM + reduce)       opus_gemm_dist/opus_gemm_mem_gemm_a2a/main.cc:299-318

The workspace is reached through a device slot {ptr, bytes} that the kernels
read at entry, so a HIP graph captured once keeps working after the slot's
workspace is grown (and moved) by WorkspaceHandle.reserve.
"""
import ctypes

from . import _lib
from ._lib import FlatmmSplitkKargs, SplitkWsHandle, check, lib  # noqa: F401
from .f4gemm import _stream_handle

# Padding of the workspace rows/columns in the reference's layout: its tile,
# B_M = B_N = 64 (opus_gemm_mem_gemm_a2a.h:9-17, main.cc:178-181).
WS_PAD = 64


class WorkspaceHandle:
    """A device slot made by ga_ws_handle_create; `address` is what kargs.ws_handle
    and the reduce take. reserve() grows the workspace (never during capture)."""

    def __init__(self, nbytes=0):
        h = ctypes.c_void_p()
        check(lib().ga_ws_handle_create(ctypes.byref(h)))
        self.address = h.value
        if nbytes:
            self.reserve(nbytes)

    def reserve(self, nbytes):
        check(lib().ga_ws_handle_reserve(self.address, int(nbytes)))

    def query(self):
        """(device pointer, capacity in bytes) of the current workspace."""
        ptr, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
        check(lib().ga_ws_handle_query(self.address, ctypes.byref(ptr), ctypes.byref(nbytes)))
        return ptr.value, nbytes.value

    def close(self):
        if self.address:
            check(lib().ga_ws_handle_destroy(self.address))
            self.address = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _round_up(x, m):
    return (x + m - 1) // m * m


def make_kargs(a, b, c, split_k, handle, bias=None, bias_per_batch=False):
    """kargs with the reference driver's dense layout (main.cc:262-280).

    a [batch, M, K] or [M, K] bf16, b [batch, N, K] or [N, K] bf16, c [.., M, N]
    bf16; workspace [split_k, batch, round_up(M, 64), round_up(N, 64)] fp32;
    bias bf16 [N] (or [batch, N] with bias_per_batch). The struct keeps the
    tensors and the handle alive for as long as it lives.
    """
    batch = a.shape[0] if a.dim() == 3 else 1
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-2]
    pm, pn = _round_up(m, WS_PAD), _round_up(n, WS_PAD)
    ka = FlatmmSplitkKargs()
    ka.ptr_a, ka.ptr_b = a.data_ptr(), b.data_ptr()
    ka.ws_handle = handle.address if handle is not None else None
    ka.ptr_c = c.data_ptr() if c is not None else None
    ka.ptr_bias = bias.data_ptr() if bias is not None else None
    ka.m, ka.n, ka.k, ka.batch, ka.split_k = m, n, k, batch, split_k
    ka.stride_a, ka.stride_b = a.stride(-2), b.stride(-2)
    ka.stride_ws, ka.stride_c = pn, n if c is None else c.stride(-2)
    ka.stride_a_batch = a.stride(0) if a.dim() == 3 else m * ka.stride_a
    ka.stride_b_batch = b.stride(0) if b.dim() == 3 else n * ka.stride_b
    ka.stride_ws_batch = pm * pn
    ka.stride_c_batch = (c.stride(0) if c is not None and c.dim() == 3 else m * n)
    ka.stride_bias_batch = n if bias_per_batch else 0
    # the struct holds raw device pointers: keep the tensors alive with it
    ka._tensors = (a, b, c, bias, handle)
    return ka


def workspace_bytes(kargs):
    return lib().ga_a16w16_splitk_workspace_bytes(ctypes.byref(kargs))


def gemm_a16w16_flatmm_splitk(kargs, stream=None):
    """The split-K kernel alone: fp32 partials into the handle's workspace."""
    check(lib().ga_gemm_a16w16_flatmm_splitk(ctypes.byref(kargs), _stream_handle(stream)))


def gemm_a16w16_splitk(kargs, stream=None):
    """Split-K kernel + reduce into bf16 C (+ kargs.ptr_bias); split_k 1 writes C
    directly."""
    check(lib().ga_gemm_a16w16_splitk(ctypes.byref(kargs), _stream_handle(stream)))


def splitk_reduce_ws_handle(handle, c, split_k, M, N, batch, padded_M, padded_N, bias=None,
                            bias_stride_batch=0, stream=None):
    """splitk_reduce_kernel reading the workspace through the handle; c bf16 or fp32."""
    import torch
    out_dtype = _lib.GA_DTYPE_F32 if c.dtype == torch.float32 else _lib.GA_DTYPE_BF16
    bias_dtype = _lib.GA_DTYPE_BF16
    if bias is not None and bias.dtype == torch.float32:
        bias_dtype = _lib.GA_DTYPE_F32
    check(lib().ga_splitk_reduce_ws_handle(
        handle.address, c.data_ptr(), out_dtype, split_k, M, N, batch, padded_M, padded_N,
        bias.data_ptr() if bias is not None else None, bias_dtype, bias_stride_batch,
        _stream_handle(stream)))


def splitk_gemm(a, b, c, split_k, handle, bias=None, bias_per_batch=False, stream=None):
    """Tensor-level C = A B^T (+ bias) in bf16 through the split-K path; grows the
    handle's workspace first when it is too small (so not inside a capture)."""
    ka = make_kargs(a, b, c, split_k, handle, bias, bias_per_batch)
    if split_k > 1:
        need = workspace_bytes(ka)
        if handle.query()[1] < need:
            handle.reserve(need)
    gemm_a16w16_splitk(ka, stream)
    return c

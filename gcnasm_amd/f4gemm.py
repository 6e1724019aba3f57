"""Host interface of the MXFP8 path, mirroring the reference's f4gemm namespace.

Names, argument meaning and error behaviour follow asm_f4gemm/f4gemm.hpp and
asm_f4gemm/f4gemm_ref.hpp; every call goes through libgcnasm_amd.so. Where the
reference exits the process, these raise GaError with the same condition.

  Config, load_configs        f4gemm.hpp:120-200
  select_kernel               f4gemm.hpp:210-267
  Kernel.load / Kernel.launch f4gemm.hpp:272-317 (compiled kernels, no .co files)
  LaunchDesc, make_launch     f4gemm.hpp:322-349
  fill_args                   f4gemm.hpp:355-392
  Shape                       f4gemm_ref.hpp:61-73
  shuffle_weight_16x16        f4gemm_ref.hpp:81-96
  shuffle_scale               f4gemm_ref.hpp:108-130
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import F4gemmKargs as KernelArgs  # noqa: F401  (reference name)
from ._lib import GaError, check, lib


@dataclass
class Config:
    tile_M: int = 0
    tile_N: int = 0
    splitK: int = 0
    bpreshuffle: int = 0
    knl_name: str = ""
    co_name: str = ""

    def to_c(self):
        c = _lib.TileConfig()
        c.tile_M, c.tile_N, c.splitK, c.bpreshuffle = (self.tile_M, self.tile_N, self.splitK,
                                                        self.bpreshuffle)
        c.knl_name = self.knl_name.encode()[: _lib.GA_NAME_MAX - 1]
        c.co_name = self.co_name.encode()[: _lib.GA_NAME_MAX - 1]
        return c

    @staticmethod
    def from_c(c):
        return Config(c.tile_M, c.tile_N, c.splitK, c.bpreshuffle, c.knl_name.decode(),
                      c.co_name.decode())


def manifest():
    """The compiled kernel manifest, in manifest order."""
    l = lib()
    out = []
    for i in range(l.ga_manifest_count()):
        c = _lib.TileConfig()
        check(l.ga_manifest_get(i, ctypes.byref(c)))
        out.append(Config.from_c(c))
    return out


def manifest_csv():
    l = lib()
    need = ctypes.c_size_t(0)
    check(l.ga_manifest_csv(None, 0, ctypes.byref(need)))
    buf = ctypes.create_string_buffer(need.value)
    check(l.ga_manifest_csv(buf, need.value, ctypes.byref(need)))
    return buf.value.decode()


def manifest_fp4():
    """The compiled MXFP4 manifest (e2m1 operands), in manifest order."""
    l = lib()
    out = []
    for i in range(l.ga_manifest_fp4_count()):
        c = _lib.TileConfig()
        check(l.ga_manifest_fp4_get(i, ctypes.byref(c)))
        out.append(Config.from_c(c))
    return out


def manifest_fp4_csv():
    l = lib()
    need = ctypes.c_size_t(0)
    check(l.ga_manifest_fp4_csv(None, 0, ctypes.byref(need)))
    buf = ctypes.create_string_buffer(need.value)
    check(l.ga_manifest_fp4_csv(buf, need.value, ctypes.byref(need)))
    return buf.value.decode()


def load_configs(csv_path):
    l = lib()
    n = ctypes.c_int(0)
    check(l.ga_load_configs(str(csv_path).encode(), None, 0, ctypes.byref(n)))
    arr = (_lib.TileConfig * max(n.value, 1))()
    check(l.ga_load_configs(str(csv_path).encode(), arr, n.value, ctypes.byref(n)))
    return [Config.from_c(arr[i]) for i in range(n.value)]


def _cfg_array(cfgs):
    if cfgs is None:
        return None, 0
    arr = (_lib.TileConfig * max(len(cfgs), 1))()
    for i, c in enumerate(cfgs):
        arr[i] = c.to_c()
    return arr, len(cfgs)


def select_kernel(M, N, K, num_cu, log2_k_split, bpreshuffle, cfgs=None):
    """Returns (index, log2 split); index -1 when nothing fits (as the reference)."""
    arr, n = _cfg_array(cfgs)
    idx, l2 = ctypes.c_int(-1), ctypes.c_int(0)
    st = lib().ga_select_kernel(M, N, K, num_cu, log2_k_split, bpreshuffle, arr, n,
                                ctypes.byref(idx), ctypes.byref(l2))
    if st not in (_lib.GA_OK, _lib.GA_ERR_NO_KERNEL):
        check(st)
    return idx.value, l2.value


@dataclass
class LaunchDesc:
    gdx: int = 0
    gdy: int = 0
    gdz: int = 1
    log2_k_split: int = 0
    zero_out: bool = False

    def to_c(self):
        return _lib.LaunchDesc(self.gdx, self.gdy, self.gdz, self.log2_k_split, int(self.zero_out))


def make_launch(cfg, M, N, K, log2_k_split):
    c = cfg.to_c()
    d = _lib.LaunchDesc()
    check(lib().ga_make_launch(ctypes.byref(c), M, N, K, log2_k_split, ctypes.byref(d)))
    return LaunchDesc(d.gdx, d.gdy, d.gdz, d.log2_k_split, bool(d.zero_out))


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def fill_args(d_D, d_C, d_A, d_B, d_ScaleA, d_ScaleB, M, N, K, stride_D0, stride_ScaleA0,
              stride_ScaleB0, alpha, beta, log2_k_split):
    args = KernelArgs()
    lib().ga_fill_args(ctypes.byref(args), _ptr(d_D), _ptr(d_C), _ptr(d_A), _ptr(d_B),
                       _ptr(d_ScaleA), _ptr(d_ScaleB), M, N, K, stride_D0, stride_ScaleA0,
                       stride_ScaleB0, alpha, beta, log2_k_split)
    return args


class Shape:
    """Padded geometry; elem_bits 8 for FP8 (Kp = K), 4 for FP4."""

    def __init__(self, M, N, K, elem_bits=8):
        s = _lib.MxShape()
        check(lib().ga_mx_shape_init(M, N, K, elem_bits, ctypes.byref(s)))
        self.M, self.N, self.K = M, N, K
        self._s = s

    def Kp(self):
        return self._s.Kp

    def Ks(self):
        return self._s.Ks

    def scale_cols(self):
        return self._s.scale_cols

    def a_rows_pad(self):
        return self._s.a_rows_pad

    def b_rows_pad(self):
        return self._s.b_rows_pad

    def scale_a_rows(self):
        return self._s.scale_a_rows

    def scale_b_rows(self):
        return self._s.scale_b_rows

    def d_rows_pad(self):
        return self._s.d_rows_pad


def _np_ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def shuffle_weight_16x16(src, N, Kp):
    src = np.ascontiguousarray(src, dtype=np.uint8).reshape(-1)
    dst = np.empty(N * Kp, dtype=np.uint8)
    check(lib().ga_shuffle_weight_16x16(_np_ptr(src), _np_ptr(dst), N, Kp))
    return dst


def shuffle_scale(src, rows, cols, sm, sn):
    src = np.ascontiguousarray(src, dtype=np.uint8).reshape(-1)
    dst = np.empty(sm * sn, dtype=np.uint8)
    check(lib().ga_shuffle_scale(_np_ptr(src), _np_ptr(dst), rows, cols, sm, sn))
    return dst


def _stream_handle(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class Kernel:
    """Compiled-kernel handle; load() finds a manifest row by knl_name or co_name."""

    def __init__(self):
        self.idx = -1
        self.cfg = None

    def load(self, co_dir_or_none, cfg):
        del co_dir_or_none  # kernels are compiled into the library
        idx = ctypes.c_int(-1)
        check(lib().ga_kernel_find(cfg.knl_name.encode(), ctypes.byref(idx)))
        self.idx = idx.value
        self.cfg = cfg
        return self

    def workspace_bytes(self, ld, M, N):
        d = ld.to_c()
        return lib().ga_kernel_workspace_bytes(self.idx, ctypes.byref(d), M, N)

    def launch(self, args, gdx, gdy, gdz, stream=None, workspace=None, ws_handle=None,
               fmt_a=0, fmt_b=0):
        """Kernel::launch. The split-K workspace is `workspace` (a tensor; None:
        the library's own), or with `ws_handle` (a flatmm_splitk.WorkspaceHandle
        or a device slot address) found through that slot when the kernels run
        (ga_kernel_launch_ws_handle: safe to capture into a HIP graph).
        fmt_a / fmt_b: the MXFP8 operands' element formats, 0 E4M3 (default)
        or 1 E5M2 (ga_kernel_launch_fmt; with a workspace buffer or the
        library's)."""
        if fmt_a or fmt_b:
            if ws_handle is not None:
                raise ValueError("element formats take a workspace buffer, not a slot")
            ws_ptr, ws_bytes = None, 0
            if workspace is not None:
                ws_ptr = _ptr(workspace)
                ws_bytes = workspace.numel() * workspace.element_size()
            check(lib().ga_kernel_launch_fmt(self.idx, ctypes.byref(args), gdx, gdy, gdz,
                                             int(fmt_a), int(fmt_b), ws_ptr, ws_bytes,
                                             _stream_handle(stream)))
            return
        if ws_handle is not None:
            addr = getattr(ws_handle, "address", ws_handle)
            check(lib().ga_kernel_launch_ws_handle(self.idx, ctypes.byref(args), gdx, gdy, gdz,
                                                   addr, _stream_handle(stream)))
            return
        ws_ptr, ws_bytes = None, 0
        if workspace is not None:
            ws_ptr = _ptr(workspace)
            ws_bytes = workspace.numel() * workspace.element_size()
        check(lib().ga_kernel_launch(self.idx, ctypes.byref(args), gdx, gdy, gdz, ws_ptr,
                                     ws_bytes, _stream_handle(stream)))


__all__ = ["Config", "KernelArgs", "LaunchDesc", "Shape", "Kernel", "GaError", "load_configs",
           "select_kernel", "make_launch", "fill_args", "shuffle_weight_16x16", "shuffle_scale",
           "manifest", "manifest_csv"]

"""ctypes binding of libgcnasm_amd.so (the C ABI in include/gcnasm_amd.h).

The library is the product: every compute call below goes to the HIP kernels
in that shared object. Loading fails loudly when it has not been built; there
is no fallback implementation.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgcnasm_amd.so")

GA_OK = 0
GA_ERR_ARG = 1
GA_ERR_SHAPE = 2
GA_ERR_NO_KERNEL = 3
GA_ERR_SPLITK = 4
GA_ERR_MANIFEST = 5
GA_ERR_WORKSPACE = 6
GA_ERR_HIP = 7
GA_ERR_GROUP = 8
GA_ERR_CAPACITY = 9

GA_DTYPE_BF16 = 0
GA_DTYPE_F32 = 1
GA_IN_F32 = 0
GA_IN_BF16 = 1
GA_MX_SCALE_FLOOR_448 = 0
GA_MX_SCALE_CEIL_448 = 1
GA_MX_SCALE_OCP = 2
GA_NAME_MAX = 96


class GaError(RuntimeError):
    """A non-zero ga_status; .status holds the code."""

    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


class OpusGemmKargs(ctypes.Structure):
    """opus_gemm_kargs (opus_gemm/block_scale_gemm/gemm_a8w8_blockscale_common.h:4-25)."""

    _fields_ = [
        ("ptr_a", ctypes.c_void_p),
        ("ptr_b", ctypes.c_void_p),
        ("ptr_c", ctypes.c_void_p),
        ("m", ctypes.c_int),
        ("n", ctypes.c_int),
        ("k", ctypes.c_int),
        ("batch", ctypes.c_int),
        ("stride_a", ctypes.c_int),
        ("stride_b", ctypes.c_int),
        ("stride_c", ctypes.c_int),
        ("stride_a_batch", ctypes.c_int),
        ("stride_b_batch", ctypes.c_int),
        ("stride_c_batch", ctypes.c_int),
        ("ptr_sfa", ctypes.c_void_p),
        ("ptr_sfb", ctypes.c_void_p),
        ("stride_sfa", ctypes.c_int),
        ("stride_sfb", ctypes.c_int),
        ("stride_sfa_batch", ctypes.c_int),
        ("stride_sfb_batch", ctypes.c_int),
    ]


def _slot_fields():
    """f4gemm::KernelArgs (asm_f4gemm/f4gemm.hpp:64-115): one arg per 16-byte slot."""
    u32 = ctypes.c_uint32
    f = []

    def ptr(name, i):
        f.append((name, ctypes.c_void_p))
        f.append(("_p%d" % i, u32 * 2))

    def scal(name, ty, i):
        f.append((name, ty))
        f.append(("_p%d" % i, u32 * 3))

    ptr("ptr_D", 0)
    ptr("ptr_C", 1)
    ptr("ptr_A", 2)
    ptr("ptr_B", 3)
    scal("alpha", ctypes.c_float, 4)
    scal("beta", ctypes.c_float, 5)
    for i, n in enumerate(["stride_D0", "stride_D1", "stride_C0", "stride_C1", "stride_A0",
                           "stride_A1", "stride_B0", "stride_B1", "M", "N", "K"]):
        scal(n, u32, 6 + i)
    ptr("ptr_ScaleA", 17)
    ptr("ptr_ScaleB", 18)
    for i, n in enumerate(["stride_ScaleA0", "stride_ScaleA1", "stride_ScaleB0",
                           "stride_ScaleB1"]):
        scal(n, u32, 19 + i)
    f.append(("log2_k_split", ctypes.c_int))
    return f


class F4gemmKargs(ctypes.Structure):
    _pack_ = 1
    _fields_ = _slot_fields()


class TileConfig(ctypes.Structure):
    """f4gemm::Config (asm_f4gemm/f4gemm.hpp:120-128)."""

    _fields_ = [
        ("tile_M", ctypes.c_int),
        ("tile_N", ctypes.c_int),
        ("splitK", ctypes.c_int),
        ("bpreshuffle", ctypes.c_int),
        ("knl_name", ctypes.c_char * GA_NAME_MAX),
        ("co_name", ctypes.c_char * GA_NAME_MAX),
    ]


class LaunchDesc(ctypes.Structure):
    """f4gemm::LaunchDesc (asm_f4gemm/f4gemm.hpp:322-327)."""

    _fields_ = [
        ("gdx", ctypes.c_int),
        ("gdy", ctypes.c_int),
        ("gdz", ctypes.c_int),
        ("log2_k_split", ctypes.c_int),
        ("zero_out", ctypes.c_int),
    ]


class MxShape(ctypes.Structure):
    """f4gemm::Shape (asm_f4gemm/f4gemm_ref.hpp:61-73)."""

    _fields_ = [(n, ctypes.c_int) for n in
                ["M", "N", "K", "Kp", "Ks", "scale_cols", "a_rows_pad", "b_rows_pad",
                 "scale_a_rows", "scale_b_rows", "d_rows_pad"]]


class SplitkWsHandle(ctypes.Structure):
    """opus_splitk_ws_handle (opus_gemm_dist/opus_gemm_mem_gemm_a2a/include/gfx950/
    opus_gemm_traits_a16w16_gfx950.cuh:588-597)."""

    _fields_ = [("ptr", ctypes.c_void_p), ("bytes", ctypes.c_uint64)]


class FlatmmSplitkKargs(ctypes.Structure):
    """opus_gemm_flatmm_splitk_kargs_gfx950 (opus_gemm_traits_a16w16_gfx950.cuh:599-634)."""

    _fields_ = [
        ("ptr_a", ctypes.c_void_p),
        ("ptr_b", ctypes.c_void_p),
        ("ws_handle", ctypes.c_void_p),
        ("ptr_c", ctypes.c_void_p),
        ("ptr_bias", ctypes.c_void_p),
    ] + [(n, ctypes.c_int) for n in
         ["m", "n", "k", "batch", "split_k", "stride_a", "stride_b", "stride_ws", "stride_c",
          "stride_a_batch", "stride_b_batch", "stride_ws_batch", "stride_c_batch",
          "stride_bias_batch"]]


assert ctypes.sizeof(OpusGemmKargs) == 96
assert ctypes.sizeof(F4gemmKargs) == 0x174
assert ctypes.sizeof(SplitkWsHandle) == 16
assert ctypes.sizeof(FlatmmSplitkKargs) == 96

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_f = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "ga_status_string": (ctypes.c_char_p, [_i]),
    "ga_last_error": (ctypes.c_char_p, []),
    "ga_version": (ctypes.c_char_p, []),
    "ga_manifest_count": (_i, []),
    "ga_manifest_get": (_i, [_i, ctypes.POINTER(TileConfig)]),
    "ga_manifest_csv": (_i, [ctypes.c_char_p, _sz, ctypes.POINTER(_sz)]),
    "ga_manifest_fp4_count": (_i, []),
    "ga_manifest_fp4_get": (_i, [_i, ctypes.POINTER(TileConfig)]),
    "ga_manifest_fp4_csv": (_i, [ctypes.c_char_p, _sz, ctypes.POINTER(_sz)]),
    "ga_load_configs": (_i, [ctypes.c_char_p, ctypes.POINTER(TileConfig), _i,
                             ctypes.POINTER(_i)]),
    "ga_select_kernel": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(TileConfig), _i,
                              ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "ga_make_launch": (_i, [ctypes.POINTER(TileConfig), _i, _i, _i, _i,
                            ctypes.POINTER(LaunchDesc)]),
    "ga_fill_args": (None, [ctypes.POINTER(F4gemmKargs), _vp, _vp, _vp, _vp, _vp, _vp, _i, _i,
                            _i, _i, _i, _i, _f, _f, _i]),
    "ga_mx_shape_init": (_i, [_i, _i, _i, _i, ctypes.POINTER(MxShape)]),
    "ga_shuffle_weight_16x16": (_i, [_vp, _vp, _i, _i]),
    "ga_shuffle_scale": (_i, [_vp, _vp, _i, _i, _i, _i]),
    "ga_shuffle_weight_16x16_device": (_i, [_vp, _vp, _i, _i, _vp]),
    "ga_shuffle_scale_device": (_i, [_vp, _vp, _i, _i, _i, _i, _vp]),
    "ga_quant_mxfp8": (_i, [_vp, _i, _i, _i, _i, _vp, _i, _vp, _i, _i, _vp]),
    "ga_quant_mx8": (_i, [_vp, _i, _i, _i, _i, _vp, _i, _vp, _i, _i, _i, _vp]),
    "ga_quant_mxfp4": (_i, [_vp, _i, _i, _i, _i, _vp, _i, _vp, _i, _i, _vp]),
    "ga_quant_fp8_1x128": (_i, [_vp, _i, _i, _i, _i, _vp, _i, _vp, _i, _vp]),
    "ga_quant_fp8_128x128": (_i, [_vp, _i, _i, _i, _i, _vp, _i, _vp, _i, _vp]),
    "ga_quant_fp8_per_tensor": (_i, [_vp, _i, _sz, _vp, _vp, _vp, _vp]),
    "ga_kernel_find": (_i, [ctypes.c_char_p, ctypes.POINTER(_i)]),
    "ga_kernel_workspace_bytes": (_sz, [_i, ctypes.POINTER(LaunchDesc), _i, _i]),
    "ga_kernel_launch": (_i, [_i, ctypes.POINTER(F4gemmKargs), _i, _i, _i, _vp, _sz, _vp]),
    "ga_kernel_launch_ws_handle": (_i, [_i, ctypes.POINTER(F4gemmKargs), _i, _i, _i, _vp, _vp]),
    "ga_kernel_launch_noalloc": (_i, [_i, ctypes.POINTER(F4gemmKargs), _i, _i, _i, _vp]),
    "ga_kernel_launch_fmt": (_i, [_i, ctypes.POINTER(F4gemmKargs), _i, _i, _i, _i, _i, _vp, _sz,
                                  _vp]),
    "ga_mxfp8_gemm": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _sz,
                           ctypes.POINTER(_i), ctypes.POINTER(LaunchDesc), _vp]),
    "ga_mxfp4_gemm": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _sz,
                           ctypes.POINTER(_i), ctypes.POINTER(LaunchDesc), _vp]),
    "ga_gemm_a8w8_blockscale": (_i, [ctypes.POINTER(OpusGemmKargs), _i, _i, _vp]),
    "ga_blockscale_k_slices": (_i, [ctypes.POINTER(OpusGemmKargs), ctypes.POINTER(_i)]),
    "ga_gemm_a8w8_blockscale_ws": (_i, [ctypes.POINTER(OpusGemmKargs), _i, _i, _vp, _sz, _vp]),
    "ga_blockscale_workspace_bytes": (_i, [ctypes.POINTER(OpusGemmKargs), ctypes.POINTER(_sz)]),
    "ga_blockscale_workspace_check": (_i, [ctypes.POINTER(OpusGemmKargs), _vp, _sz, _vp]),
    "ga_blockscale_stream_k": (_i, [ctypes.POINTER(OpusGemmKargs), ctypes.POINTER(_i)]),
    "ga_fp8_gemm_per_tensor": (_i, [ctypes.POINTER(OpusGemmKargs), _i, _vp]),
    "ga_splitk_reduce": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _i, _vp]),
    "ga_splitk_reduce_ws_handle": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _i,
                                        _vp]),
    "ga_gemm_a16w16_flatmm_splitk": (_i, [ctypes.POINTER(FlatmmSplitkKargs), _vp]),
    "ga_gemm_a16w16_splitk": (_i, [ctypes.POINTER(FlatmmSplitkKargs), _vp]),
    "ga_a16w16_splitk_workspace_bytes": (_sz, [ctypes.POINTER(FlatmmSplitkKargs)]),
    "ga_ws_handle_create": (_i, [ctypes.POINTER(_vp)]),
    "ga_ws_handle_reserve": (_i, [_vp, _sz]),
    "ga_ws_handle_query": (_i, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_sz)]),
    "ga_ws_handle_destroy": (_i, [_vp]),
    "ga_device_num_cu": (_i, [ctypes.POINTER(_i)]),
}

_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                "libgcnasm_amd.so is not built (%s); run "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`make -C gcnasm_amd/csrc`" % LIB_PATH)
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(status):
    """Raise GaError for a non-zero status, with the library's detail text."""
    if status != GA_OK:
        l = lib()
        raise GaError(status, "%s: %s" % (l.ga_status_string(status).decode(),
                                          l.ga_last_error().decode()))
    return status

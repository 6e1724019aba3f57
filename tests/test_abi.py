"""The C ABI library (CPU only, no compute on a GPU): it loads, exports every
entry point declared in include/gcnasm_amd.h, its structs have the reference's
byte layout, and argument errors come back as status codes (validated before
any HIP call, so these run without a GPU)."""
import ctypes
import os
import re

import pytest

from gcnasm_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "gcnasm_amd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ga_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 25
    l = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in names if not hasattr(l, n)]
    assert not missing, missing
    # and the Python binding covers all of them
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_struct_sizes():
    assert ctypes.sizeof(_lib.OpusGemmKargs) == 96
    assert ctypes.sizeof(_lib.F4gemmKargs) == 0x174
    assert ctypes.sizeof(_lib.TileConfig) == 16 + 2 * _lib.GA_NAME_MAX


def test_status_strings():
    l = _lib.lib()
    for s in range(10):
        assert l.ga_status_string(s)
    assert b"gfx950" in l.ga_version()


def test_null_arguments_are_rejected_before_any_device_call():
    l = _lib.lib()
    assert l.ga_kernel_launch(0, None, 1, 1, 1, None, 0, None) == _lib.GA_ERR_ARG
    assert l.ga_kernel_launch(-1, None, 1, 1, 1, None, 0, None) == _lib.GA_ERR_ARG
    assert l.ga_gemm_a8w8_blockscale(None, 128, 0, None) == _lib.GA_ERR_ARG
    assert l.ga_fp8_gemm_per_tensor(None, 0, None) == _lib.GA_ERR_ARG
    assert l.ga_quant_mxfp8(None, 0, 1, 32, 32, None, 32, None, 1, 0, None) == _lib.GA_ERR_ARG
    assert l.ga_quant_fp8_1x128(None, 0, 1, 128, 128, None, 128, None, 1, None) == _lib.GA_ERR_ARG
    assert l.ga_quant_fp8_128x128(None, 0, 1, 128, 128, None, 128, None, 1, None) == _lib.GA_ERR_ARG
    assert l.ga_quant_fp8_per_tensor(None, 0, 4, None, None, None, None) == _lib.GA_ERR_ARG
    assert l.ga_splitk_reduce(None, None, 0, 1, 1, 1, 1, 1, 1, None, 0, 0, None) == _lib.GA_ERR_ARG
    assert l.ga_shuffle_weight_16x16_device(None, None, 16, 32, None) == _lib.GA_ERR_ARG
    assert l.ga_shuffle_scale_device(None, None, 1, 1, 32, 8, None) == _lib.GA_ERR_ARG
    assert l.ga_manifest_get(10 ** 6, None) == _lib.GA_ERR_ARG
    assert b"range" in l.ga_last_error()


def test_opus_kargs_validation():
    l = _lib.lib()
    ka = _lib.OpusGemmKargs()
    ka.ptr_a = ka.ptr_b = ka.ptr_c = ka.ptr_sfa = ka.ptr_sfb = 0x1000
    ka.m, ka.n, ka.k, ka.batch = 64, 64, 200, 1  # K % 128 != 0
    ka.stride_a = ka.stride_b = 208
    ka.stride_c = 64
    assert l.ga_gemm_a8w8_blockscale(ctypes.byref(ka), 128, 0, None) == _lib.GA_ERR_GROUP
    ka.k = 0
    assert l.ga_gemm_a8w8_blockscale(ctypes.byref(ka), 128, 0, None) == _lib.GA_ERR_ARG
    ka.k = ka.stride_a = ka.stride_b = 256
    assert l.ga_gemm_a8w8_blockscale(ctypes.byref(ka), 64, 0, None) == _lib.GA_ERR_ARG
    # 256 rows of A (or B) beyond the 4 GiB a buffer descriptor addresses
    ka.stride_a = 1 << 24
    assert l.ga_gemm_a8w8_blockscale(ctypes.byref(ka), 128, 0, None) == _lib.GA_ERR_SHAPE
    assert l.ga_fp8_gemm_per_tensor(ctypes.byref(ka), 0, None) == _lib.GA_ERR_SHAPE
    ka.stride_a = 256
    ka.stride_b = 1 << 24
    assert l.ga_gemm_a8w8_blockscale(ctypes.byref(ka), 128, 0, None) == _lib.GA_ERR_SHAPE


def test_mx_extent_beyond_4gib_is_rejected():
    """512 rows of a row stride past 2^23 bytes, or a scale matrix past 4 GiB,
    cannot be addressed from a tile's buffer descriptor: GA_ERR_SHAPE before
    any device call."""
    l = _lib.lib()
    args = _lib.F4gemmKargs()
    l.ga_fill_args(ctypes.byref(args), 0x1000, None, 0x1000, 0x1000, 0x1000, 0x1000,
                   256, 256, 1024, 256, 32, 32, 1.0, 0.0, 0)
    args.stride_A0 = 1 << 23
    assert l.ga_kernel_launch(0, ctypes.byref(args), 1, 1, 1, None, 0, None) == _lib.GA_ERR_SHAPE
    args.stride_A0 = 1024
    args.stride_B0 = 1 << 23
    idx = ctypes.c_int()
    assert l.ga_kernel_find(b"ga_mxfp8_bf16_noBpreShuffle_256x256", ctypes.byref(idx)) == 0
    assert l.ga_kernel_launch(idx.value, ctypes.byref(args), 1, 1, 1, None, 0, None) == \
        _lib.GA_ERR_SHAPE


def test_mx_launch_validation_without_gpu():
    l = _lib.lib()
    args = _lib.F4gemmKargs()
    l.ga_fill_args(ctypes.byref(args), 8, None, 8, 8, 8, 8, 64, 64, 256, 64, 8, 8, 1.0, 0.0, 0)
    assert l.ga_kernel_launch(0, ctypes.byref(args), 99, 1, 1, None, 0, None) == _lib.GA_ERR_ARG
    l.ga_fill_args(ctypes.byref(args), 8, None, 8, 8, 8, 8, 64, 60, 256, 64, 8, 8, 1.0, 0.0, 0)
    assert l.ga_kernel_launch(0, ctypes.byref(args), 1, 1, 1, None, 0, None) == _lib.GA_ERR_SHAPE


def test_flatmm_splitk_structs_match_reference_layout():
    """opus_splitk_ws_handle / opus_gemm_flatmm_splitk_kargs_gfx950 byte layout
    (opus_gemm_traits_a16w16_gfx950.cuh:588-634)."""
    K = _lib.FlatmmSplitkKargs
    assert ctypes.sizeof(_lib.SplitkWsHandle) == 16
    assert ctypes.sizeof(K) == 96
    want = dict(ptr_a=0, ptr_b=8, ws_handle=16, ptr_c=24, ptr_bias=32, m=40, n=44, k=48,
                batch=52, split_k=56, stride_a=60, stride_b=64, stride_ws=68, stride_c=72,
                stride_a_batch=76, stride_b_batch=80, stride_ws_batch=84, stride_c_batch=88,
                stride_bias_batch=92)
    for name, off in want.items():
        assert getattr(K, name).offset == off, name


def test_flatmm_splitk_validation_without_gpu():
    l = _lib.lib()
    assert l.ga_gemm_a16w16_flatmm_splitk(None, None) == _lib.GA_ERR_ARG
    assert l.ga_gemm_a16w16_splitk(None, None) == _lib.GA_ERR_ARG
    ka = _lib.FlatmmSplitkKargs()
    ka.ptr_a = ka.ptr_b = ka.ptr_c = 0x10000
    ka.ws_handle = 0x20000
    ka.m, ka.n, ka.k, ka.batch, ka.split_k = 64, 64, 100, 1, 2   # K % 8 != 0
    ka.stride_a = ka.stride_b = 104
    ka.stride_ws, ka.stride_c, ka.stride_ws_batch = 64, 64, 64 * 64
    assert l.ga_gemm_a16w16_flatmm_splitk(ctypes.byref(ka), None) == _lib.GA_ERR_SHAPE
    ka.k = 96
    ka.stride_a = 90                                              # < K
    assert l.ga_gemm_a16w16_flatmm_splitk(ctypes.byref(ka), None) == _lib.GA_ERR_SHAPE
    ka.stride_a = 96
    ka.ptr_a = 0x10008                                            # not 16-byte aligned
    assert l.ga_gemm_a16w16_flatmm_splitk(ctypes.byref(ka), None) == _lib.GA_ERR_ARG
    ka.ptr_a = 0x10000
    ka.stride_ws = 32                                             # < N
    assert l.ga_gemm_a16w16_flatmm_splitk(ctypes.byref(ka), None) == _lib.GA_ERR_SHAPE
    ka.stride_ws, ka.stride_ws_batch = 64, 63 * 64                # < M * stride_ws
    assert l.ga_gemm_a16w16_flatmm_splitk(ctypes.byref(ka), None) == _lib.GA_ERR_SHAPE
    ka.stride_ws_batch = 64 * 64
    ka.ws_handle = None
    assert l.ga_gemm_a16w16_flatmm_splitk(ctypes.byref(ka), None) == _lib.GA_ERR_ARG
    ka.split_k = 0
    assert l.ga_gemm_a16w16_flatmm_splitk(ctypes.byref(ka), None) == _lib.GA_ERR_ARG
    ka.split_k, ka.batch = 3, 2
    assert l.ga_a16w16_splitk_workspace_bytes(ctypes.byref(ka)) == 3 * 2 * 64 * 64 * 4
    assert l.ga_splitk_reduce_ws_handle(None, None, 0, 2, 1, 1, 1, 1, 1, None, 0, 0,
                                        None) == _lib.GA_ERR_ARG
    # slots are only those made by ga_ws_handle_create
    assert l.ga_ws_handle_reserve(0x1234, 64) == _lib.GA_ERR_ARG
    assert l.ga_ws_handle_query(0x1234, None, None) == _lib.GA_ERR_ARG
    assert l.ga_ws_handle_destroy(0x1234) == _lib.GA_ERR_ARG
    assert l.ga_ws_handle_create(None) == _lib.GA_ERR_ARG


def test_element_formats_are_validated_without_gpu():
    """ga_kernel_launch_fmt: format codes other than 0 (E4M3) / 1 (E5M2), and
    any E5M2 request on an MXFP4 kernel, are GA_ERR_ARG before a device call;
    a valid request still meets the usual argument checks (bad grid)."""
    l = _lib.lib()
    args = _lib.F4gemmKargs()
    l.ga_fill_args(ctypes.byref(args), 8, None, 8, 8, 8, 8, 64, 64, 256, 64, 8, 8, 1.0, 0.0, 0)
    for fa, fb in ((2, 0), (0, 2), (-1, 0), (4, 4)):
        assert l.ga_kernel_launch_fmt(0, ctypes.byref(args), 1, 1, 1, fa, fb, None, 0, None) == \
            _lib.GA_ERR_ARG
        assert b"E5M2" in l.ga_last_error()
    idx = ctypes.c_int()
    assert l.ga_kernel_find(b"ga_mxfp4_bf16_BpreShuffle_256x256", ctypes.byref(idx)) == 0
    assert l.ga_kernel_launch_fmt(idx.value, ctypes.byref(args), 1, 1, 1, 1, 0, None, 0,
                                  None) == _lib.GA_ERR_ARG
    assert b"e2m1" in l.ga_last_error()
    assert l.ga_kernel_launch_fmt(0, ctypes.byref(args), 99, 1, 1, 1, 1, None, 0, None) == \
        _lib.GA_ERR_ARG


def test_kargs_keep_their_tensors_alive():
    """The kargs structs hold raw device pointers; the Python builders keep
    the tensors with them, so kargs built from temporaries never point at
    memory the allocator has handed to something else."""
    import gc
    import weakref
    import torch
    from gcnasm_amd import flatmm_splitk, opus_gemm

    def build_opus():
        a, b = torch.zeros((1, 4, 128), dtype=torch.uint8), torch.zeros((1, 4, 128), dtype=torch.uint8)
        c = torch.zeros((1, 4, 4))
        sfa, sfb = torch.ones((1, 1, 4)), torch.ones((1, 1, 1))
        return opus_gemm.make_kargs(a, b, c, sfa, sfb, 4, 4, 128), [weakref.ref(x) for x in (a, b, c, sfa, sfb)]

    def build_flatmm():
        a, b = torch.zeros((4, 64), dtype=torch.bfloat16), torch.zeros((4, 64), dtype=torch.bfloat16)
        c = torch.zeros((4, 4), dtype=torch.bfloat16)
        return flatmm_splitk.make_kargs(a, b, c, 1, None), [weakref.ref(x) for x in (a, b, c)]

    for build in (build_opus, build_flatmm):
        ka, refs = build()
        gc.collect()
        assert all(r() is not None for r in refs)
        del ka
        gc.collect()
        assert all(r() is None for r in refs)

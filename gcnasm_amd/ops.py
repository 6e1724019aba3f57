"""Tensor-level entry points over the C ABI (torch tensors as device buffers).

These are conveniences for tests, the benchmark and Python callers; every
function is a thin call into libgcnasm_amd.so.
"""
import ctypes

import torch

from . import _lib
from ._lib import check, lib
from .f4gemm import Shape, _stream_handle


def _rows(x, what="x"):
    """Checks that x is a [rows, K] matrix whose rows are contiguous (the
    quantisers take a row stride, not a column stride)."""
    if x.dim() != 2 or x.stride(1) != 1 or x.stride(0) < x.shape[1]:
        raise ValueError("%s must be a [rows, K] matrix with contiguous rows "
                         "(shape %s, strides %s)" % (what, tuple(x.shape), tuple(x.stride())))
    return x.shape


def _in_dtype(x):
    if x.dtype == torch.float32:
        return _lib.GA_IN_F32
    if x.dtype == torch.bfloat16:
        return _lib.GA_IN_BF16
    raise TypeError("input must be float32 or bfloat16")


def quant_mxfp8(x, scale_rule=_lib.GA_MX_SCALE_FLOOR_448, stream=None):
    """x [rows, K] -> (q uint8 [rows, K] E4M3, scales uint8 [rows, K/32] E8M0, unshuffled)."""
    rows, K = _rows(x)
    q = torch.empty((rows, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((rows, K // 32), dtype=torch.uint8, device=x.device)
    check(lib().ga_quant_mxfp8(x.data_ptr(), _in_dtype(x), rows, K, x.stride(0), q.data_ptr(),
                               K, s.data_ptr(), K // 32, scale_rule, _stream_handle(stream)))
    return q, s


def quant_mx8(x, fmt, scale_rule=_lib.GA_MX_SCALE_FLOOR_448, stream=None):
    """x [rows, K] -> (q uint8 [rows, K] codes of format fmt: 0 E4M3, 1 E5M2;
    scales uint8 [rows, K/32] E8M0, unshuffled); rule numbers as for MXFP8
    with the format's maximum (448 or 57344)."""
    rows, K = _rows(x)
    q = torch.empty((rows, K), dtype=torch.uint8, device=x.device)
    s = torch.empty((rows, K // 32), dtype=torch.uint8, device=x.device)
    check(lib().ga_quant_mx8(x.data_ptr(), _in_dtype(x), rows, K, x.stride(0), q.data_ptr(), K,
                             s.data_ptr(), K // 32, scale_rule, int(fmt), _stream_handle(stream)))
    return q, s


def quant_mxfp4(x, scale_rule=_lib.GA_MX_SCALE_FLOOR_448, stream=None):
    """x [rows, K] -> (q uint8 [rows, K/2] packed e2m1, low nibble = even element;
    scales uint8 [rows, K/32] E8M0, unshuffled). Rule numbers as for MXFP8 with
    the e2m1 maximum 6 in place of 448."""
    rows, K = _rows(x)
    q = torch.empty((rows, K // 2), dtype=torch.uint8, device=x.device)
    s = torch.empty((rows, K // 32), dtype=torch.uint8, device=x.device)
    check(lib().ga_quant_mxfp4(x.data_ptr(), _in_dtype(x), rows, K, x.stride(0), q.data_ptr(),
                               K // 2, s.data_ptr(), K // 32, scale_rule, _stream_handle(stream)))
    return q, s


def quant_fp8_1x128(x, stream=None):
    """x [rows, K] -> (q [rows, K], sfa fp32 [K/128, rows])."""
    rows, K = _rows(x)
    q = torch.empty((rows, K), dtype=torch.uint8, device=x.device)
    sfa = torch.empty((K // 128, rows), dtype=torch.float32, device=x.device)
    check(lib().ga_quant_fp8_1x128(x.data_ptr(), _in_dtype(x), rows, K, x.stride(0),
                                   q.data_ptr(), K, sfa.data_ptr(), rows,
                                   _stream_handle(stream)))
    return q, sfa


def quant_fp8_128x128(x, stream=None):
    """x [rows, K] -> (q [rows, K], sfb fp32 [ceil(rows/128), K/128])."""
    rows, K = _rows(x)
    q = torch.empty((rows, K), dtype=torch.uint8, device=x.device)
    sfb = torch.empty(((rows + 127) // 128, K // 128), dtype=torch.float32, device=x.device)
    check(lib().ga_quant_fp8_128x128(x.data_ptr(), _in_dtype(x), rows, K, x.stride(0),
                                     q.data_ptr(), K, sfb.data_ptr(), K // 128,
                                     _stream_handle(stream)))
    return q, sfb


def quant_fp8_per_tensor(x, stream=None):
    """x (contiguous) -> (q uint8 same shape, scale fp32 [1])."""
    x = x.contiguous()
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scale = torch.empty((1,), dtype=torch.float32, device=x.device)
    ws = torch.empty((1,), dtype=torch.int32, device=x.device)
    check(lib().ga_quant_fp8_per_tensor(x.data_ptr(), _in_dtype(x), x.numel(), q.data_ptr(),
                                        scale.data_ptr(), ws.data_ptr(),
                                        _stream_handle(stream)))
    return q, scale


def shuffle_weight_16x16(w, stream=None):
    """Device preshuffle of B [N, Kp] bytes (shuffle_weight(layout=(16,16)))."""
    w = w.contiguous()
    N, Kp = w.shape
    out = torch.empty((N, Kp), dtype=w.dtype, device=w.device)
    check(lib().ga_shuffle_weight_16x16_device(w.data_ptr(), out.data_ptr(), N, Kp,
                                               _stream_handle(stream)))
    return out


def shuffle_scale(s, sm, sn, stream=None):
    """Device pad-to-[sm, sn] (0x7F) + shuffle of an E8M0 scale matrix [rows, cols]."""
    s = s.contiguous()
    rows, cols = s.shape
    out = torch.empty((sm * sn,), dtype=torch.uint8, device=s.device)
    check(lib().ga_shuffle_scale_device(s.data_ptr(), out.data_ptr(), rows, cols, sm, sn,
                                        _stream_handle(stream)))
    return out


class MxOperand:
    """An MXFP8 operand in the kernel layout: codes (rows padded to 256 for A,
    16x16-preshuffled for B) and padded + shuffled E8M0 scales."""

    def __init__(self, codes, scales, rows, K):
        self.codes, self.scales, self.rows, self.K = codes, scales, rows, K


def prepare_mx_a(x, scale_rule=_lib.GA_MX_SCALE_FLOOR_448, stream=None):
    """Activation [M, K] -> MxOperand (A rows zero-padded to 256)."""
    M, K = x.shape
    sh = Shape(M, 1, K)
    q, s = quant_mxfp8(x, scale_rule, stream)
    codes = torch.zeros((sh.a_rows_pad(), K), dtype=torch.uint8, device=x.device)
    codes[:M].copy_(q)
    ss = shuffle_scale(s, sh.scale_a_rows(), sh.scale_cols(), stream)
    return MxOperand(codes, ss, M, K)


def prepare_mx_b(w, scale_rule=_lib.GA_MX_SCALE_FLOOR_448, bpreshuffle=True, stream=None):
    """Weight [N, K] -> MxOperand (16x16 preshuffled codes when bpreshuffle)."""
    N, K = w.shape
    sh = Shape(1, N, K)
    q, s = quant_mxfp8(w, scale_rule, stream)
    codes = shuffle_weight_16x16(q, stream) if bpreshuffle else q
    ss = shuffle_scale(s, sh.scale_b_rows(), sh.scale_cols(), stream)
    return MxOperand(codes, ss, N, K)


def prepare_mx4_a(x, scale_rule=_lib.GA_MX_SCALE_FLOOR_448, stream=None):
    """Activation [M, K] -> MXFP4 MxOperand: packed e2m1 [round_up(M, 256), K/2]."""
    M, K = x.shape
    sh = Shape(M, 1, K, elem_bits=4)
    q, s = quant_mxfp4(x, scale_rule, stream)
    codes = torch.zeros((sh.a_rows_pad(), K // 2), dtype=torch.uint8, device=x.device)
    codes[:M].copy_(q)
    ss = shuffle_scale(s, sh.scale_a_rows(), sh.scale_cols(), stream)
    return MxOperand(codes, ss, M, K)


def prepare_mx4_b(w, scale_rule=_lib.GA_MX_SCALE_FLOOR_448, bpreshuffle=True, stream=None):
    """Weight [N, K] -> MXFP4 MxOperand (packed bytes 16x16 preshuffled over Kp = K/2)."""
    N, K = w.shape
    sh = Shape(1, N, K, elem_bits=4)
    q, s = quant_mxfp4(w, scale_rule, stream)
    codes = shuffle_weight_16x16(q, stream) if bpreshuffle else q
    ss = shuffle_scale(s, sh.scale_b_rows(), sh.scale_cols(), stream)
    return MxOperand(codes, ss, N, K)


def mxfp4_gemm(a, b, bpreshuffle=True, log2_k_split=0, out=None, num_cu=0, workspace=None,
               stream=None):
    """D [M, N] bf16 = A * B^T for MXFP4 operands (prepare_mx4_a/b) through the
    MXFP4 manifest. Returns (D, registry index, launch desc)."""
    M, N, K = a.rows, b.rows, a.K
    sh = Shape(M, N, K, elem_bits=4)
    if out is None:
        out = torch.empty((sh.d_rows_pad(), N), dtype=torch.bfloat16, device=a.codes.device)
    chosen = ctypes.c_int(-1)
    ld = _lib.LaunchDesc()
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    check(lib().ga_mxfp4_gemm(out.data_ptr(), a.codes.data_ptr(), b.codes.data_ptr(),
                              a.scales.data_ptr(), b.scales.data_ptr(), M, N, K, out.stride(0),
                              int(bpreshuffle), log2_k_split, num_cu, ws_ptr, ws_bytes,
                              ctypes.byref(chosen), ctypes.byref(ld), _stream_handle(stream)))
    return out, chosen.value, ld


def mxfp8_gemm(a, b, bpreshuffle=True, log2_k_split=0, out=None, num_cu=0, workspace=None,
               stream=None):
    """D [M, N] bf16 = A * B^T through the heuristic-chosen compiled kernel.
    Returns (D, kernel index, launch desc)."""
    M, N, K = a.rows, b.rows, a.K
    sh = Shape(M, N, K)
    if out is None:
        out = torch.empty((sh.d_rows_pad(), N), dtype=torch.bfloat16, device=a.codes.device)
    chosen = ctypes.c_int(-1)
    ld = _lib.LaunchDesc()
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    check(lib().ga_mxfp8_gemm(out.data_ptr(), a.codes.data_ptr(), b.codes.data_ptr(),
                              a.scales.data_ptr(), b.scales.data_ptr(), M, N, K, out.stride(0),
                              int(bpreshuffle), log2_k_split, num_cu, ws_ptr, ws_bytes,
                              ctypes.byref(chosen), ctypes.byref(ld), _stream_handle(stream)))
    return out, chosen.value, ld


def splitk_reduce(ws, out, split_k, M, N, batch=1, padded_M=None, padded_N=None, bias=None,
                  stream=None):
    padded_M = padded_M or M
    padded_N = padded_N or N
    out_dtype = _lib.GA_DTYPE_BF16 if out.dtype == torch.bfloat16 else _lib.GA_DTYPE_F32
    bias_dtype = _lib.GA_DTYPE_F32
    bptr, bstride = None, 0
    if bias is not None:
        bias_dtype = _lib.GA_DTYPE_BF16 if bias.dtype == torch.bfloat16 else _lib.GA_DTYPE_F32
        bptr = bias.data_ptr()
        bstride = bias.shape[-1] if bias.dim() == 2 else 0
    check(lib().ga_splitk_reduce(ws.data_ptr(), out.data_ptr(), out_dtype, split_k, M, N, batch,
                                 padded_M, padded_N, bptr, bias_dtype, bstride,
                                 _stream_handle(stream)))
    return out

"""GPU parity of MXFP8 GEMMs with E5M2 (bf8) operands and mixed E4M3 x E5M2
pairs (ga_kernel_launch_fmt: the f8f6f4 format codes of the reference's
scaled-MFMA dispatch, wmma_opus_rdna4/opus/opus.hpp:1785-1786, at the GEMM
level) against oracle.gemm_mx8_mfma (the MFMA step model with each format's
significand, pinned on recorded hardware outputs of every format pair in
tests/test_oracle_mfma.py), under the north-star rule of tests/helpers.py.

Covered: the 256x256 eight-wave kernel (every M > 64 launch, whichever tile
the index names; preshuffled and row-major B; split-K through the workspace),
the decode kernels at 1-64 rows (in-workgroup, and the split variant with the
slices in separate workgroups, with and without K splits), and a 4096^3
problem checked on one row of every 256-row tile.
"""
import numpy as np
import pytest
import torch

import oracle
from gcnasm_amd import f4gemm
from helpers import assert_parity, bf16_compare, tile_rows

pytestmark = pytest.mark.gpu

PAIRS = [(1, 1), (0, 1), (1, 0)]


def operands(M, N, K, fa, fb, seed, std_b=1.0):
    xa = oracle.gen_mx_input(M, K, seed * 7919 + 1, 1.0, 4)
    xb = oracle.gen_mx_input(N, K, seed * 7919 + 2, std_b, 4)
    qa, sa = oracle.quant_mx8(xa, fa)
    qb, sb = oracle.quant_mx8(xb, fb)
    return qa, sa, qb, sb


def cfg_named(name):
    return [c for c in f4gemm.manifest() if c.knl_name == name][0]


def run_fmt(dev, qa, sa, qb, sb, cfg, l2, fa, fb):
    M, K = qa.shape
    N = qb.shape[0]
    sh = f4gemm.Shape(M, N, K)
    a_pad = np.zeros((sh.a_rows_pad(), K), dtype=np.uint8)
    a_pad[:M] = qa
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    A = t(a_pad)
    B = t(f4gemm.shuffle_weight_16x16(qb, N, K) if cfg.bpreshuffle else qb.reshape(-1))
    SA = t(f4gemm.shuffle_scale(sa, M, K // 32, sh.scale_a_rows(), sh.scale_cols()))
    SB = t(f4gemm.shuffle_scale(sb, N, K // 32, sh.scale_b_rows(), sh.scale_cols()))
    D = torch.full((sh.d_rows_pad(), N), float("nan"), dtype=torch.bfloat16, device=dev)
    ld = f4gemm.make_launch(cfg, M, N, K, l2)
    args = f4gemm.fill_args(D, None, A, B, SA, SB, M, N, K, N, sh.scale_cols(), sh.scale_cols(),
                            1.0, 0.0, ld.log2_k_split)
    ws = torch.empty(max(1, ld.gdz * M * N), dtype=torch.float32, device=dev)
    print("launch %s M=%d N=%d K=%d gdz=%d formats %d x %d" % (cfg.knl_name, M, N, K, ld.gdz,
                                                                fa, fb), flush=True)
    f4gemm.Kernel().load(None, cfg).launch(args, ld.gdx, ld.gdy, ld.gdz, workspace=ws,
                                            fmt_a=fa, fmt_b=fb)
    torch.cuda.synchronize()
    return D[:M].view(torch.int16).cpu().numpy().view(np.uint16), ld


def check(got, qa, sa, qb, sb, fa, fb, l2, label, rows=None):
    if rows is not None:
        qa, sa, got = qa[rows], sa[rows], got[rows]
    want = oracle.to_bf16_bits(oracle.gemm_mx8_mfma(qa, sa, qb, sb, fa, fb, l2))
    ok, st = bf16_compare(got, want, oracle.mx_absdot(qa, sa, qb, sb, fa, fb))
    assert_parity(st, label)


@pytest.mark.parametrize("fa,fb", PAIRS)
@pytest.mark.parametrize("name,l2", [("ga_mxfp8_bf16_BpreShuffle_256x256", 0),
                                     ("ga_mxfp8_bf16_BpreShuffle_128x128", 0),
                                     ("ga_mxfp8_bf16_BpreShuffle_256x256_splitK", 2),
                                     ("ga_mxfp8_bf16_noBpreShuffle_256x256", 0),
                                     ("ga_mxfp8_bf16_noBpreShuffle_128x128_splitK", 1)])
def test_formats_large_m(dev, fa, fb, name, l2):
    """More than 64 rows: the 256x256 kernel with the requested formats,
    partial tiles in M and N, whatever tile the index names."""
    M, N, K = 300, 784, 1536
    qa, sa, qb, sb = operands(M, N, K, fa, fb, seed=11 + 2 * fa + fb)
    got, ld = run_fmt(dev, qa, sa, qb, sb, cfg_named(name), l2, fa, fb)
    check(got, qa, sa, qb, sb, fa, fb, l2, "formats %dx%d %s gdz=%d" % (fa, fb, name, ld.gdz))


@pytest.mark.parametrize("fa,fb", PAIRS)
@pytest.mark.parametrize("M", [1, 16, 40, 64])
@pytest.mark.parametrize("NKL", [(1040, 2048, 0), (1040, 2048, 2), (28672 - 16, 512, 0),
                                 (8192, 2048, 3)])
def test_formats_decode(dev, fa, fb, M, NKL):
    """1-64 rows: the decode kernels with the requested formats (in-workgroup
    at 1-16 rows and narrow N, the split variant at 17-64 rows with a split or
    over wide N), preshuffled B."""
    N, K, l2 = NKL
    name = "ga_mxfp8_bf16_BpreShuffle_256x256" + ("_splitK" if l2 else "")
    qa, sa, qb, sb = operands(M, N, K, fa, fb, seed=M + N + 3 * fa + fb, std_b=0.02)
    got, ld = run_fmt(dev, qa, sa, qb, sb, cfg_named(name), l2, fa, fb)
    check(got, qa, sa, qb, sb, fa, fb, l2,
          "formats %dx%d decode M=%d N=%d K=%d gdz=%d" % (fa, fb, M, N, K, ld.gdz))


@pytest.mark.parametrize("fa,fb", [(1, 1), (0, 1)])
def test_formats_decode_plain_b(dev, fa, fb):
    M, N, K = 40, 1040, 1024
    qa, sa, qb, sb = operands(M, N, K, fa, fb, seed=5)
    got, _ = run_fmt(dev, qa, sa, qb, sb, cfg_named("ga_mxfp8_bf16_noBpreShuffle_128x128_splitK"),
                     2, fa, fb)
    check(got, qa, sa, qb, sb, fa, fb, 2, "formats %dx%d decode plain B" % (fa, fb))


def test_e5m2_4096_cube(dev):
    """E5M2 x E5M2 at 4096^3 on the heuristic's kernel, one row of every
    256-row tile checked on every column."""
    n = 4096
    qa, sa, qb, sb = operands(n, n, n, 1, 1, seed=4096)
    idx, l2 = f4gemm.select_kernel(n, n, n, 256, 0, 1)
    got, _ = run_fmt(dev, qa, sa, qb, sb, f4gemm.manifest()[idx], l2, 1, 1)
    rows = tile_rows(n)
    check(got, qa, sa, qb, sb, 1, 1, l2, "E5M2 4096^3 (%d rows)" % len(rows), rows=rows)


def test_default_formats_equal_plain_launch(dev):
    """ga_kernel_launch_fmt with formats 0 x 0 (E4M3 both) writes exactly what
    ga_kernel_launch writes, on a tile other than 256x256 and with a split."""
    import ctypes
    from gcnasm_amd import _lib
    M, N, K, l2 = 130, 512, 1024, 1
    qa, sa, qb, sb = operands(M, N, K, 0, 0, seed=21)
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_128x128_splitK")
    sh = f4gemm.Shape(M, N, K)
    a_pad = np.zeros((sh.a_rows_pad(), K), dtype=np.uint8)
    a_pad[:M] = qa
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    A, B = t(a_pad), t(f4gemm.shuffle_weight_16x16(qb, N, K))
    SA = t(f4gemm.shuffle_scale(sa, M, K // 32, sh.scale_a_rows(), sh.scale_cols()))
    SB = t(f4gemm.shuffle_scale(sb, N, K // 32, sh.scale_b_rows(), sh.scale_cols()))
    ld = f4gemm.make_launch(cfg, M, N, K, l2)
    idx = f4gemm.Kernel().load(None, cfg).idx
    ws = torch.empty(ld.gdz * M * N, dtype=torch.float32, device=dev)
    outs = []
    for use_fmt in (False, True):
        D = torch.full((sh.d_rows_pad(), N), float("nan"), dtype=torch.bfloat16, device=dev)
        args = f4gemm.fill_args(D, None, A, B, SA, SB, M, N, K, N, sh.scale_cols(),
                                sh.scale_cols(), 1.0, 0.0, ld.log2_k_split)
        if use_fmt:
            st = _lib.lib().ga_kernel_launch_fmt(idx, ctypes.byref(args), ld.gdx, ld.gdy, ld.gdz,
                                                 0, 0, ws.data_ptr(), ws.numel() * 4, None)
        else:
            st = _lib.lib().ga_kernel_launch(idx, ctypes.byref(args), ld.gdx, ld.gdy, ld.gdz,
                                             ws.data_ptr(), ws.numel() * 4, None)
        _lib.check(st)
        torch.cuda.synchronize()
        outs.append(D[:M].view(torch.int16).cpu().numpy().view(np.uint16))
    np.testing.assert_array_equal(outs[1], outs[0])
    check(outs[1], qa, sa, qb, sb, 0, 0, l2, "formats 0x0 via ga_kernel_launch_fmt")


@pytest.mark.parametrize("l2", [0, 1])
def test_every_tile_writes_the_same_bits(dev, l2):
    """Above the decode path every MXFP8 kernel (all tiles, preshuffled and
    row-major B) chains the same 128-K MFMA steps per K slice from zero, so
    the bf16 output is bit-identical whichever entry runs; this is what lets
    ga_kernel_launch_fmt run the 256x256 kernel for any index. Checked over
    the whole manifest (split entries at l2 = 1), and against the oracle."""
    M, N, K = 300, 784, 1536
    qa, sa, qb, sb = operands(M, N, K, 0, 0, seed=31 + l2)
    cfgs = [c for c in f4gemm.manifest() if l2 == 0 or c.splitK]
    outs = [run_fmt(dev, qa, sa, qb, sb, c, l2, 0, 0)[0] for c in cfgs]
    for c, got in zip(cfgs[1:], outs[1:]):
        np.testing.assert_array_equal(got, outs[0], err_msg="%s vs %s" % (c.knl_name,
                                                                         cfgs[0].knl_name))
    check(outs[0], qa, sa, qb, sb, 0, 0, l2, "every tile l2=%d" % l2)

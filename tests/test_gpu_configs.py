"""GPU parity at the benchmark configurations' own sizes.

The reference's drivers verify the very shape they benchmark
(opus_gemm/block_scale_gemm/gemm_a8w8_blockscale_host.cc:260-281). These tests
do the same for every configuration bench.py times: MXFP8 4096^3 and 8192^3
(heuristic tile: the persistent 256x256 kernel, several tiles per
workgroup), the per-tensor and block-scale 8192^3 GEMMs, and the six decode
shapes M in {1, 16, 64} x (N=28672, K=8192) / (N=8192, K=28672) at every
log2_k_split 0-3 (0 is the reference driver's default; the heuristic picks 1
or 3).

Inputs come from the benchmark's own generators (bench.mx_inputs,
bench.scaled_inputs) on the GPU. The GPU quantisers' codes and scales are
compared byte for byte with the oracle's quantisation of the same fp32
values; the GEMM outputs are checked against the MFMA-model oracle on every
row for decode shapes and, for the square shapes, on helpers.tile_rows (one
row in every 256-row tile, a different offset in each, plus the first and
last row), so every output tile is checked. The MXFP8 outputs are also held
against the reference's own reference_gemm (asm_f4gemm/f4gemm_ref.hpp:181-222,
oracle/_ref) under the north-star rule (helpers.hold_to_reference).
"""
import numpy as np
import pytest
import torch

import bench
import oracle
from gcnasm_amd import f4gemm, opus_gemm, ops
from helpers import (assert_parity, bf16_compare, dequant_mx_f32, f32_compare, hold_to_reference,
                     reference_gemm, tile_rows)

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def bf16_host(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def quantise_both(x):
    """MX quantisation of the device tensor x on the GPU and in the oracle;
    asserts they agree byte for byte and returns (device q, s, host q, s)."""
    qd, sd = ops.quant_mxfp8(x)
    q, s = oracle.quant_mxfp8(host(x))
    np.testing.assert_array_equal(host(qd), q)
    np.testing.assert_array_equal(host(sd), s)
    return qd, sd, q, s


def operand_a(q, s, K):
    sh = f4gemm.Shape(q.shape[0], 1, K)
    codes = torch.zeros((sh.a_rows_pad(), K), dtype=torch.uint8, device=q.device)
    codes[:q.shape[0]].copy_(q)
    return ops.MxOperand(codes, ops.shuffle_scale(s, sh.scale_a_rows(), sh.scale_cols()),
                         q.shape[0], K)


def operand_b(q, s, K):
    sh = f4gemm.Shape(1, q.shape[0], K)
    return ops.MxOperand(ops.shuffle_weight_16x16(q),
                         ops.shuffle_scale(s, sh.scale_b_rows(), sh.scale_cols()),
                         q.shape[0], K)


def mx_case(M, N, K, b_std, log2_k_split, seed, rows=None):
    print("config MXFP8 M=%d N=%d K=%d l2=%d seed=%d" % (M, N, K, log2_k_split, seed), flush=True)
    xa, xbs = bench.mx_inputs(torch, M, N, K, b_std=b_std, nsets=1, seed=seed)
    qad, sad, qa, sa = quantise_both(xa)
    del xa
    qbd, sbd, qb, sb = quantise_both(xbs[0])
    del xbs
    a, b = operand_a(qad, sad, K), operand_b(qbd, sbd, K)
    D, idx, ld = ops.mxfp8_gemm(a, b, log2_k_split=log2_k_split)
    torch.cuda.synchronize()
    name = f4gemm.manifest()[idx].knl_name
    rows = np.arange(M) if rows is None else rows
    got = bf16_host(D[:M])[rows]
    del D, a, b, qad, sad, qbd, sbd
    torch.cuda.empty_cache()
    qa_r, sa_r = np.ascontiguousarray(qa[rows]), np.ascontiguousarray(sa[rows])
    want = oracle.to_bf16_bits(oracle.gemm_mx_mfma(qa_r, sa_r, qb, sb, ld.log2_k_split))
    ok, st = bf16_compare(got, want, oracle.mx_absdot(qa_r, sa_r, qb, sb))
    label = "MXFP8 %dx%dx%d %s grid=(%d,%d,%d) rows=%d" % (
        M, N, K, name, ld.gdx, ld.gdy, ld.gdz, len(rows))
    assert_parity(st, label)
    # the reference's own CPU reference (reference_gemm, f64 sums) and the
    # north-star rule: misses are counted, each bounded, capped by the MFMA
    # model's own misses on the same rows
    R = oracle.load_ref()
    if R is None:
        print("%s: oracle/_ref not built, reference_gemm check skipped" % label, flush=True)
        return
    A, B = dequant_mx_f32(qa_r, sa_r), dequant_mx_f32(qb, sb)
    hold_to_reference(label, got, reference_gemm(R, A, B), A, B, want)


@pytest.mark.parametrize("n", [4096, 8192])
def test_mxfp8_square(dev, n):
    """Configurations 2a/2b: the benchmark's inputs (seed 0, as bench.py's
    8192^3 leg), heuristic tile and split."""
    mx_case(n, n, n, 1.0, 0, seed=0, rows=tile_rows(n))


@pytest.mark.parametrize("M", [1, 16, 64])
@pytest.mark.parametrize("NK", [(28672, 8192), (8192, 28672)])
@pytest.mark.parametrize("l2", [0, 1, 2, 3])
def test_mxfp8_decode(dev, M, NK, l2):
    """Configuration 5: decode shapes, weights N(0, 0.02) (bench.py's decode
    legs use seed 1), every output row checked, at each log2 split the
    benchmark times (the heuristic's is 1 for K = 8192 and 3 for K = 28672)."""
    N, K = NK
    mx_case(M, N, K, 0.02, l2, seed=1)


def test_per_tensor_8192(dev):
    """Configuration 3: per-tensor FP8 8192^3, bf16 C, bench.py's inputs."""
    n = 8192
    print("config per-tensor %d^3" % n, flush=True)
    xa, xb = bench.scaled_inputs(torch, n, n, n)
    qad, sad = ops.quant_fp8_per_tensor(xa)
    qbd, sbd = ops.quant_fp8_per_tensor(xb)
    qa, sa = oracle.quant_fp8_per_tensor(host(xa))
    qb, sb = oracle.quant_fp8_per_tensor(host(xb))
    np.testing.assert_array_equal(host(sad), sa)
    np.testing.assert_array_equal(host(sbd), sb)
    np.testing.assert_array_equal(host(qad), qa)
    np.testing.assert_array_equal(host(qbd), qb)
    del xa, xb
    C = torch.empty((n, n), dtype=torch.bfloat16, device=dev)
    opus_gemm.per_tensor_gemm(qad, qbd, sad, sbd, C)
    torch.cuda.synchronize()
    rows = tile_rows(n)
    got = bf16_host(C)[rows]
    del C, qad, qbd
    torch.cuda.empty_cache()
    want = oracle.gemm_per_tensor_mfma(np.ascontiguousarray(qa[rows]), qb, sa[0], sb[0],
                                       opus_gemm.k_slices(n, n, n))
    absdot = oracle.fp8_absdot(np.ascontiguousarray(qa[rows]), qb) * float(sa[0]) * float(sb[0])
    ok, st = bf16_compare(got, oracle.to_bf16_bits(want), absdot)
    assert_parity(st, "per-tensor %d^3 rows=%d" % (n, len(rows)))


def test_blockscale_8192(dev):
    """The benchmark's block-scale leg: DeepSeek 1x128 / 128x128 scales,
    fp32 C, 8192^3, bench.py's inputs."""
    n = 8192
    print("config block-scale %d^3" % n, flush=True)
    xa, xb = bench.scaled_inputs(torch, n, n, n)
    qad, sfad = ops.quant_fp8_1x128(xa)
    qbd, sfbd = ops.quant_fp8_128x128(xb)
    qa, sfa = oracle.quant_fp8_1x128(host(xa))
    qb, sfb = oracle.quant_fp8_128x128(host(xb))
    np.testing.assert_array_equal(host(qad), qa)
    np.testing.assert_array_equal(host(qbd), qb)
    np.testing.assert_array_equal(host(sfad), sfa)
    np.testing.assert_array_equal(host(sfbd), sfb)
    del xa, xb
    C = torch.empty((n, n), dtype=torch.float32, device=dev)
    opus_gemm.blockscale_gemm(qad, qbd, sfad, sfbd, C)
    torch.cuda.synchronize()
    rows = tile_rows(n)
    got = host(C)[rows]
    del C, qad, qbd
    torch.cuda.empty_cache()
    qa_r, sfa_r = np.ascontiguousarray(qa[rows]), np.ascontiguousarray(sfa[:, rows])
    want = oracle.gemm_blockscale_mfma(qa_r, qb, sfa_r, sfb, 128, opus_gemm.k_slices(n, n, n))
    ok, st = f32_compare(got, want, absdot=oracle.blockscale_absdot(qa_r, qb, sfa_r, sfb, 128))
    assert_parity(st, "block-scale %d^3 rows=%d" % (n, len(rows)))

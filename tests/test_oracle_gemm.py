"""Pins the oracle's reference GEMMs (CPU only).

  reference_gemm   bit-identical to the reference's own reference_gemm
                   (asm_f4gemm/f4gemm_ref.hpp:181-222, compiled into oracle/_ref)
  MXFP8 exact      vs numpy float64 matmul of the dequantised operands
                   (products of E4M3 values times power-of-two scales are exact)
  MXFP8 fp32acc    within the fp32 accumulation bound of the exact value;
                   split-K slices partition K exactly (f4gemm.hpp:342-344)
  block-scale      the per-product fp32 reference (host.cc:66-90), the
                   kernel-order fp32 accumulation and the f64 value agree
                   within fp32 bounds; scale indexing checked against a numpy
                   formulation for GROUP_N 128 and 1, including a partial last
                   N group; a planted transposed-SFB mistake is detected
  per-tensor       vs numpy
  split-K reduce   vs an in-order numpy sum
  golden fixture   tests/golden/mx_config1.npz (made by tests/golden/make_golden.py)
"""
import os

import numpy as np
import pytest

import oracle
from helpers import mx_operands

HERE = os.path.dirname(os.path.abspath(__file__))


def test_reference_gemm_bit_identical(R):
    rng = np.random.default_rng(0)
    A = rng.standard_normal((37, 300), dtype=np.float32)
    B = rng.standard_normal((50, 300), dtype=np.float32)
    ours = oracle.reference_gemm(A, B, 0.75)
    ref = np.empty((37, 50), np.float32)
    R.ref_reference_gemm(oracle.p(A), oracle.p(B), 37, 50, 300, 0.75, oracle.p(ref))
    np.testing.assert_array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_reference_gemm_on_reference_operands(R):
    """The reference's own seeded MXFP4 operand generator (make_operand) feeds both
    GEMMs; its products are exact, so both equal the f64 numpy value."""
    M, N, K = 16, 24, 256
    pa, sa, da = np.empty(M * K // 2, np.uint8), np.empty(M * K // 32, np.uint8), np.empty((M, K), np.float32)
    pb, sb, db = np.empty(N * K // 2, np.uint8), np.empty(N * K // 32, np.uint8), np.empty((N, K), np.float32)
    R.ref_make_operand(M, K, 1234, oracle.p(pa), oracle.p(sa), oracle.p(da))
    R.ref_make_operand(N, K, 5678, oracle.p(pb), oracle.p(sb), oracle.p(db))
    # the oracle's FP4/E8M0 decode reproduces the reference's dequantised values
    O = oracle.load()
    lo = np.array([O.or_fp4_decode(v & 15) for v in pa], np.float32)
    hi = np.array([O.or_fp4_decode(v >> 4) for v in pa], np.float32)
    deq = np.stack([lo, hi], 1).reshape(M, K) * np.repeat(
        oracle.e8m0_decode_table()[sa.reshape(M, K // 32)], 32, axis=1)
    np.testing.assert_array_equal(deq, da)
    np.testing.assert_array_equal(oracle.reference_gemm(da, db),
                                  (da.astype(np.float64) @ db.astype(np.float64).T).astype(np.float32))


def test_mx_exact_vs_numpy():
    qa, sa, qb, sb = mx_operands(64, 48, 512, seed=3)
    want = oracle.mx_dequant(qa, sa) @ oracle.mx_dequant(qb, sb).T
    got = oracle.gemm_mxfp8_exact(qa, sa, qb, sb)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())


@pytest.mark.parametrize("l2", [0, 1, 2, 3])
def test_mx_fp32acc_close_to_exact(l2):
    qa, sa, qb, sb = mx_operands(32, 40, 1024, seed=4 + l2)
    ex = oracle.gemm_mxfp8_exact(qa, sa, qb, sb)
    got = oracle.gemm_mxfp8_fp32acc(qa, sa, qb, sb, l2).astype(np.float64)
    absdot = oracle.mx_absdot(qa, sa, qb, sb)
    # fp32 accumulation of (K/128 + 2^l2) roundings of magnitude <= absdot
    bound = (1024 / 128 + (1 << l2) + 1) * 2.0 ** -24 * absdot
    assert np.all(np.abs(got - ex) <= bound)


def test_mx_fp32acc_matches_numpy_step_model():
    """Independent numpy restatement: fp32 accumulator, one rounding per 128-K step."""
    qa, sa, qb, sb = mx_operands(16, 16, 768, seed=9)
    A, B = oracle.mx_dequant(qa, sa), oracle.mx_dequant(qb, sb)
    acc = np.zeros((16, 16), np.float32)
    for k in range(0, 768, 128):
        acc = (acc.astype(np.float64) + A[:, k:k + 128] @ B[:, k:k + 128].T).astype(np.float32)
    np.testing.assert_array_equal(oracle.gemm_mxfp8_fp32acc(qa, sa, qb, sb, 0), acc)


def test_mx_planted_scale_mistake_is_caught():
    qa, sa, qb, sb = mx_operands(16, 16, 256, seed=5)
    good = oracle.gemm_mxfp8_exact(qa, sa, qb, sb)
    bad_sa = sa.copy()
    bad_sa[:, 1] += 1  # one K-block's scale off by a factor 2
    bad = oracle.gemm_mxfp8_exact(qa, bad_sa, qb, sb)
    assert np.abs(bad - good).max() > 1e-3 * np.abs(good).max()


def ds_case(M, N, K, group_n, seed):
    xa = oracle.randn(M * K, seed).reshape(M, K)
    xb = oracle.randn(N * K, seed + 1).reshape(N, K)
    qa, sfa = oracle.quant_fp8_1x128(xa)
    if group_n == 128:
        qb, sfb = oracle.quant_fp8_128x128(xb)
    else:
        qb, sfb = oracle.quant_fp8_1x128(xb)
    return qa, qb, sfa, sfb


def numpy_blockscale(qa, qb, sfa, sfb, group_n):
    t = oracle.e4m3_decode_table().astype(np.float64)
    A, B = t[qa], t[qb]
    M, K = qa.shape
    N = qb.shape[0]
    out = np.zeros((M, N))
    for g in range(K // 128):
        p = A[:, g * 128:(g + 1) * 128] @ B[:, g * 128:(g + 1) * 128].T
        sb = sfb[np.arange(N) // 128, g] if group_n == 128 else sfb[g, :]
        out += p * sfa[g, :][:, None] * sb[None, :]
    return out


@pytest.mark.parametrize("group_n", [128, 1])
@pytest.mark.parametrize("shape", [(32, 200, 512), (17, 2112, 256)])
def test_blockscale_variants_agree(group_n, shape):
    M, N, K = shape
    qa, qb, sfa, sfb = ds_case(M, N, K, group_n, seed=M)
    want = numpy_blockscale(qa, qb, sfa, sfb, group_n)
    ex = oracle.gemm_blockscale_exact(qa, qb, sfa, sfb, group_n)
    np.testing.assert_allclose(ex, want, rtol=1e-12, atol=1e-10 * np.abs(want).max())
    absdot = oracle.blockscale_absdot(qa, qb, sfa, sfb, group_n)
    for f in (oracle.gemm_blockscale_ref, oracle.gemm_blockscale_fp32acc):
        got = f(qa, qb, sfa, sfb, group_n).astype(np.float64)
        assert np.all(np.abs(got - ex) <= (K + 4) * 2.0 ** -23 * absdot)


def test_blockscale_planted_sfb_transpose_is_caught():
    M, N, K = 16, 256, 256
    qa, qb, sfa, sfb = ds_case(M, N, K, 128, seed=2)
    good = oracle.gemm_blockscale_exact(qa, qb, sfa, sfb, 128)
    bad = numpy_blockscale(qa, qb, sfa, np.ascontiguousarray(sfb[::-1]), 128)
    assert np.abs(bad - good).max() > 1e-3 * np.abs(good).max()


def test_per_tensor_vs_numpy():
    xa = oracle.randn(24 * 384, 1).reshape(24, 384)
    xb = oracle.randn(40 * 384, 2).reshape(40, 384)
    qa, sa = oracle.quant_fp8_per_tensor(xa)
    qb, sb = oracle.quant_fp8_per_tensor(xb)
    t = oracle.e4m3_decode_table().astype(np.float64)
    acc = np.zeros((24, 40), np.float32)
    for k in range(0, 384, 128):
        acc = (acc.astype(np.float64) + t[qa[:, k:k + 128]] @ t[qb[:, k:k + 128]].T).astype(np.float32)
    want = acc * np.float32(sa[0] * sb[0])
    np.testing.assert_array_equal(oracle.gemm_per_tensor_fp32acc(qa, qb, sa[0], sb[0]), want)


def test_splitk_reduce_in_order():
    rng = np.random.default_rng(1)
    split, M, N, batch, pM, pN = 4, 3, 50, 2, 4, 64
    ws = rng.standard_normal((split, batch, pM, pN)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    out = np.empty((batch, M, N), np.float32)
    oracle.load().or_splitk_reduce(oracle.p(ws), oracle.p(out), split, M, N, batch, pM, pN,
                                   oracle.p(bias), 0)
    acc = ws[0, :, :M, :N].copy()
    for s in range(1, split):
        acc = (acc + ws[s, :, :M, :N]).astype(np.float32)
    np.testing.assert_array_equal(out, (acc + bias).astype(np.float32))


def test_golden_config1():
    path = os.path.join(HERE, "golden", "mx_config1.npz")
    g = np.load(path)
    qa, sa = oracle.quant_mxfp8(g["xa"])
    qb, sb = oracle.quant_mxfp8(g["xb"])
    np.testing.assert_array_equal(qa, g["qa"])
    np.testing.assert_array_equal(sa, g["sa"])
    np.testing.assert_array_equal(qb, g["qb"])
    np.testing.assert_array_equal(sb, g["sb"])
    np.testing.assert_array_equal(oracle.gemm_mxfp8_fp32acc(qa, sa, qb, sb, 0), g["d_fp32acc"])
    np.testing.assert_allclose(g["d_fp32acc"], oracle.mx_dequant(qa, sa) @ oracle.mx_dequant(qb, sb).T,
                               rtol=1e-5, atol=1e-5 * np.abs(g["d_fp32acc"]).max())

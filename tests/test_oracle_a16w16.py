"""Pins the oracle's bf16 split-K GEMM (CPU only).

  slices         the reference's partition (opus_gemm_pipeline_a16w16_flatmm_
                 splitk_gfx950.cuh:234-247: K in 128-wide iterations,
                 ceil(iters / split_k) per slice, the last takes the rest),
                 worked out by hand for each table row below, including the
                 cases that leave slices empty; one-hot K columns land in
                 exactly the slice the table names
  partials       integer-valued bf16 operands make every sum exact in fp32:
                 each slice's partial equals the integer product over its K
                 range, and their sum equals A B^T; a transposed B (planted
                 in the oracle call) does not
  accumulation   on N(0,1) data the summed partials stay within the fp32
                 rounding bound (one rounding per 32-K group and per slice
                 sum) of the float64 product
  reduce         splitk_reduce_gfx950.cuh:105-170: slices summed in order plus
                 a [N] or [batch, N] bias, exact on integer data
"""
import numpy as np
import pytest

import oracle

# (K, split_k) -> slices, computed by hand from pipeline .cuh:234-247
SLICE_TABLE = {
    (7168, 2): [(0, 3584), (3584, 7168)],                   # main.cc defaults
    (1000, 3): [(0, 384), (384, 768), (768, 1000)],         # iters 8, per 3
    (640, 4): [(0, 256), (256, 512), (512, 640), (640, 640)],  # iters 5, per 2
    (128, 3): [(0, 128), (128, 128), (128, 128)],           # iters 1, per 1
    (2048, 16): [(i * 128, i * 128 + 128) for i in range(16)],
    (200, 1): [(0, 200)],
    (4096, 5): [(0, 896), (896, 1792), (1792, 2688), (2688, 3584), (3584, 4096)],
}


@pytest.mark.parametrize("key", sorted(SLICE_TABLE))
def test_slice_table(key):
    K, split_k = key
    assert oracle.a16w16_slices(K, split_k) == SLICE_TABLE[key]


def bf16(x):
    return oracle.to_bf16_bits(np.asarray(x, np.float32))


@pytest.mark.parametrize("key", [(1000, 3), (640, 4), (128, 3), (4096, 5)])
def test_onehot_column_lands_in_its_slice(key):
    K, split_k = key
    M, N = 3, 5
    for k0 in sorted(k for k in {0, 127, 128, 383, 384, K - 8, K - 1, K // 2} if k < K):
        a = np.zeros((M, K), np.float32)
        b = np.zeros((N, K), np.float32)
        a[:, k0] = 1.0
        b[:, k0] = 1.0
        ws = oracle.a16w16_splitk_ws(bf16(a), bf16(b), split_k)
        want = [1.0 if kb <= k0 < ke else 0.0 for kb, ke in SLICE_TABLE[key]]
        assert sum(want) == 1.0
        for s in range(split_k):
            assert np.all(ws[s] == want[s]), (key, k0, s)


def int_operands(M, N, K, seed):
    rng = np.random.default_rng(seed)
    a = rng.integers(-8, 9, (M, K)).astype(np.float32)
    b = rng.integers(-8, 9, (N, K)).astype(np.float32)
    return a, b


@pytest.mark.parametrize("shape", [(7, 9, 1000, 3), (16, 12, 640, 4), (5, 33, 4096, 5)])
def test_integer_partials_are_exact(shape):
    M, N, K, split_k = shape
    a, b = int_operands(M, N, K, seed=K)
    ws = oracle.a16w16_splitk_ws(bf16(a), bf16(b), split_k)
    ai, bi = a.astype(np.int64), b.astype(np.int64)
    for s, (kb, ke) in enumerate(oracle.a16w16_slices(K, split_k)):
        want = ai[:, kb:ke] @ bi[:, kb:ke].T
        np.testing.assert_array_equal(ws[s], want.astype(np.float32))
    np.testing.assert_array_equal(ws.astype(np.float64).sum(0), (ai @ bi.T).astype(np.float64))


def test_planted_transpose_is_caught():
    M = N = K = 256
    a, b = int_operands(M, N, K, seed=3)
    exact = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float32)
    good = oracle.a16w16_splitk_ws(bf16(a), bf16(b), 2).sum(0)
    bad = oracle.a16w16_splitk_ws(bf16(a), bf16(b.T.copy()), 2).sum(0)
    np.testing.assert_array_equal(good, exact)
    assert not np.array_equal(bad, exact)


@pytest.mark.parametrize("split_k", [1, 2, 7])
def test_randn_within_fp32_bound(split_k):
    M, N, K = 24, 40, 2048
    a = oracle.randn(M * K, 11).reshape(M, K)
    b = oracle.randn(N * K, 12).reshape(N, K)
    ab, bb = bf16(a), bf16(b)
    A = oracle.bf16_bits_to_f32(ab).astype(np.float64)
    B = oracle.bf16_bits_to_f32(bb).astype(np.float64)
    exact = A @ B.T
    absdot = np.abs(A) @ np.abs(B).T
    ws = oracle.a16w16_splitk_ws(ab, bb, split_k)
    red = oracle.splitk_reduce(ws[:, None])[0]
    # one rounding per 32-K group and one per slice addition, each at most
    # 2^-24 of a partial sum bounded by sum |a b|
    bound = (K // 32 + split_k) * 2.0 ** -24 * absdot
    assert np.all(np.abs(red - exact) <= bound)
    # and not trivially: the accumulation does round
    assert np.any(red != exact.astype(np.float32)) or split_k == 1


def test_reduce_bias_broadcast_and_per_batch():
    split_k, batch, M, N = 3, 2, 4, 6
    rng = np.random.default_rng(0)
    ws = rng.integers(-50, 50, (split_k, batch, M, N)).astype(np.float32)
    bias = rng.integers(-9, 9, N).astype(np.float32)
    got = oracle.splitk_reduce(ws, bias, 0)
    np.testing.assert_array_equal(got, ws.sum(0) + bias[None, None, :])
    bias2 = rng.integers(-9, 9, (batch, N)).astype(np.float32)
    got = oracle.splitk_reduce(ws, bias2, N)
    np.testing.assert_array_equal(got, ws.sum(0) + bias2[:, None, :])
    np.testing.assert_array_equal(oracle.splitk_reduce(ws), ws.sum(0))

"""Pins the B / scale preshuffles (CPU only): the oracle, the product's host
shuffles and the reference's own functions (compiled from
asm_f4gemm/f4gemm_ref.hpp into oracle/_ref) must agree byte for byte, and all
must equal the documented view/permute formulation (f4gemm_ref.hpp:78, 102)
written independently in numpy. The maps are bijections (round trip).
"""
import numpy as np
import pytest

import oracle
from gcnasm_amd import f4gemm

W_SHAPES = [(16, 32), (32, 64), (256, 512), (48, 96), (272, 4096)]
S_SHAPES = [(1, 8, 256, 8), (17, 5, 32, 8), (300, 32, 512, 32), (256, 16, 256, 16),
            (33, 7, 256, 8)]


def numpy_shuffle_weight(w, N, Kp):
    return w.reshape(N // 16, 16, Kp // 32, 2, 16).transpose(0, 2, 3, 1, 4).reshape(-1)


def numpy_shuffle_scale(s, rows, cols, sm, sn):
    pad = np.full((sm, sn), 0x7F, np.uint8)
    pad[:rows, :cols] = s
    return pad.reshape(sm // 32, 2, 16, sn // 8, 2, 4).transpose(0, 3, 5, 2, 4, 1).reshape(-1)


@pytest.mark.parametrize("shape", W_SHAPES)
def test_shuffle_weight(shape):
    N, Kp = shape
    w = np.random.default_rng(N * Kp).integers(0, 256, (N, Kp), dtype=np.uint8)
    want = numpy_shuffle_weight(w, N, Kp)
    np.testing.assert_array_equal(oracle.shuffle_weight_16x16(w, N, Kp), want)
    np.testing.assert_array_equal(f4gemm.shuffle_weight_16x16(w, N, Kp), want)
    # bijection: shuffling a ramp of indices gives a permutation
    idx = np.arange(N * Kp, dtype=np.int64)
    perm = idx.reshape(N // 16, 16, Kp // 32, 2, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
    assert np.array_equal(np.sort(perm), idx)
    inv = np.empty_like(perm)
    inv[perm] = idx
    np.testing.assert_array_equal(want[inv], w.reshape(-1))


@pytest.mark.parametrize("shape", W_SHAPES)
def test_shuffle_weight_vs_reference(R, shape):
    N, Kp = shape
    w = np.random.default_rng(N + Kp).integers(0, 256, (N, Kp), dtype=np.uint8)
    ref = np.empty(N * Kp, np.uint8)
    R.ref_shuffle_weight_16x16(oracle.p(w), oracle.p(ref), N, Kp)
    np.testing.assert_array_equal(oracle.shuffle_weight_16x16(w, N, Kp), ref)


@pytest.mark.parametrize("shape", S_SHAPES)
def test_shuffle_scale(shape):
    rows, cols, sm, sn = shape
    s = np.random.default_rng(rows).integers(0, 256, (rows, cols), dtype=np.uint8)
    want = numpy_shuffle_scale(s, rows, cols, sm, sn)
    np.testing.assert_array_equal(oracle.shuffle_scale(s, rows, cols, sm, sn), want)
    np.testing.assert_array_equal(f4gemm.shuffle_scale(s, rows, cols, sm, sn), want)
    # padding is 0x7F everywhere outside [rows, cols]
    assert (want == 0x7F).sum() >= sm * sn - rows * cols


@pytest.mark.parametrize("shape", S_SHAPES)
def test_shuffle_scale_vs_reference(R, shape):
    rows, cols, sm, sn = shape
    s = np.random.default_rng(cols).integers(0, 256, (rows, cols), dtype=np.uint8)
    ref = np.empty(sm * sn, np.uint8)
    R.ref_shuffle_scale(oracle.p(s), oracle.p(ref), rows, cols, sm, sn)
    np.testing.assert_array_equal(oracle.shuffle_scale(s, rows, cols, sm, sn), ref)


def test_scale_layout_serves_mfma_lanes():
    """Dword l of each 256-byte block holds the scales of lane l of the 16x16x128
    MFMA: row l%16, K-block l/16, for (row half d1, 128-K half d4) at byte
    2*d4 + d1 -- the property the kernels' op_sel addressing relies on."""
    rows, cols = 64, 16
    s = np.random.default_rng(0).integers(0, 256, (rows, cols), dtype=np.uint8)
    sh = oracle.shuffle_scale(s, rows, cols, 64, 16).reshape(-1, 64, 4)
    for blk in range(sh.shape[0]):
        d0, d3 = blk // 2, blk % 2
        for lane in range(64):
            for d4 in range(2):
                for d1 in range(2):
                    r = d0 * 32 + d1 * 16 + lane % 16
                    c = d3 * 8 + d4 * 4 + lane // 16
                    assert sh[blk, lane, 2 * d4 + d1] == s[r, c]


def test_shuffle_rejects_bad_shapes():
    from gcnasm_amd._lib import GaError
    with pytest.raises(GaError):
        f4gemm.shuffle_weight_16x16(np.zeros(24 * 32, np.uint8), 24, 32)
    with pytest.raises(GaError):
        f4gemm.shuffle_scale(np.zeros(10, np.uint8), 2, 5, 30, 8)

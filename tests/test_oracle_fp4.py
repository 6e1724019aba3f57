"""Pins the oracle's MXFP4 (OCP e2m1) functions (CPU only).

  e2m1 decode      equals the reference's kFp4Lut (f4gemm_ref.hpp:24-26,
                   compiled into oracle/_ref) and the OCP value table
  e2m1 encode      brute-force nearest value over the 16 codes, ties to the
                   even code, saturation at +-6, signed zero for NaN
  scale rules      closed-form brackets of amax / 2^e against the e2m1 max 6
  quantiser        every code equals the brute-force nearest code of x * 2^-e;
                   the packing (element 2i in the low nibble of byte i,
                   asm_f4gemm/README.md:97-99) decodes to the reference's own
                   make_operand dequantised values (f4gemm_ref.hpp:132-176)
  MXFP4 GEMMs      the exact GEMM equals the reference's reference_gemm on the
                   reference's make_operand operands and numpy float64; the
                   fp32-accumulated GEMM follows the same 128-K step model as
                   MXFP8 (checked against a numpy restatement); a planted
                   nibble-order mistake is caught
"""
import numpy as np
import pytest

import oracle

OCP_E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], np.float32)


def test_e2m1_decode_table(O):
    got = oracle.fp4_decode_table()
    np.testing.assert_array_equal(got.view(np.uint32), OCP_E2M1.view(np.uint32))


def test_e2m1_decode_vs_reference(R, O):
    for c in range(16):
        assert np.float32(O.or_fp4_decode(c)).view(np.uint32) == \
            np.float32(R.ref_fp4_lut(c)).view(np.uint32)


def brute_e2m1(x):
    """Nearest e2m1 code by exhaustive search; ties -> even code; |x| > 6 -> 6."""
    if np.isnan(x):
        return 8 if np.signbit(x) else 0
    sign = 8 if np.signbit(x) else 0
    a = abs(float(x))
    if a >= 6.0:
        return sign | 7
    vals = OCP_E2M1[:8].astype(np.float64)
    d = np.abs(vals - a)
    best = np.flatnonzero(d == d.min())
    c = int(best[0]) if len(best) == 1 else int(best[best % 2 == 0][0])
    return sign | c


def test_e2m1_encode_bruteforce(O):
    vals = [0.0, -0.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 7.0, 1e30,
            float("inf"), -float("inf"), float("nan"), 1e-45, -1e-40, 0.2500001, 0.2499999]
    vals += list(np.linspace(-8, 8, 4097))
    mids = (OCP_E2M1[:7] + OCP_E2M1[1:8]) / 2
    for m in mids:
        for d in (0.0, 1e-6, -1e-6):
            vals += [m + d, -(m + d)]
    rng = np.random.default_rng(4)
    vals += list(rng.standard_normal(5000) * 3)
    for v in np.array(vals, np.float32):
        assert O.or_e2m1_encode(float(v)) == brute_e2m1(v), v


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_mx4_scale_rule_brackets(O, rule):
    rng = np.random.default_rng(rule)
    amax = np.concatenate([np.abs(rng.standard_normal(3000)) * 2.0 ** rng.integers(-30, 30, 3000),
                           6.0 * 2.0 ** np.arange(-20, 20), 2.0 ** np.arange(-20, 20),
                           [1e-40, 3e-39]]).astype(np.float32)
    for a in amax:
        e = O.or_mx4_scale_exp(float(a), rule)
        a = float(a)
        # the unclamped exponent, from frexp of a/6 in float64 (a/6 lands on a
        # power of two only when a = 6*2^k, where the division is exact)
        m, ex = np.frexp(a / 6.0 if rule < 2 else a)
        if rule == 0:
            want = ex - 1                        # largest e with 6*2^e <= amax
        elif rule == 1:
            want = ex - 1 if m == 0.5 else ex    # smallest e with 6*2^e >= amax
        else:
            want = ex - 1 - 2                    # OCP: floor(log2 amax) - 2
        assert e == min(127, max(-127, want)), (a, e, want)
        if -127 < e < 127:
            if rule == 0:
                assert 6.0 * 2.0 ** e <= a < 6.0 * 2.0 ** (e + 1), (a, e)
            elif rule == 1:
                assert 6.0 * 2.0 ** (e - 1) < a <= 6.0 * 2.0 ** e, (a, e)
            else:
                assert 2.0 ** (e + 2) <= a < 2.0 ** (e + 3), (a, e)
    assert O.or_mx4_scale_exp(0.0, 0) == -127


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_quant_mxfp4_bruteforce(O, rule):
    rows, K = 6, 256
    x = oracle.gen_mx_input(rows, K, 11 + rule, 1.0, 4)
    x[0, :32] = 0.0                 # zero block
    x[1, 3] = 6.0 * 2.0 ** 5        # exact maximum
    q, s = oracle.quant_mxfp4(x, rule)
    codes = oracle.unpack_fp4(q)
    for r in range(rows):
        for b in range(K // 32):
            blk = x[r, b * 32:(b + 1) * 32]
            e = O.or_mx4_scale_exp(float(np.abs(blk).max()), rule)
            assert s[r, b] == e + 127
            for i in range(32):
                want = brute_e2m1(np.float32(np.ldexp(np.float64(blk[i]), -e)))
                assert codes[r, b * 32 + i] == want, (r, b, i)


def test_mxfp4_packing_vs_reference(R):
    """Packed bytes + scales of the reference's make_operand decode to its own
    dequantised values under the oracle's unpacking."""
    M, K = 40, 512
    pa, sa, da = (np.empty(M * K // 2, np.uint8), np.empty(M * K // 32, np.uint8),
                  np.empty((M, K), np.float32))
    R.ref_make_operand(M, K, 99, oracle.p(pa), oracle.p(sa), oracle.p(da))
    deq = oracle.mx4_dequant(pa.reshape(M, K // 2), sa.reshape(M, K // 32))
    np.testing.assert_array_equal(deq.astype(np.float32), da)


def ref_operands(R, M, N, K, seeds=(1234, 5678)):
    out = []
    for rows, seed in ((M, seeds[0]), (N, seeds[1])):
        p, s, d = (np.empty(rows * K // 2, np.uint8), np.empty(rows * K // 32, np.uint8),
                   np.empty((rows, K), np.float32))
        R.ref_make_operand(rows, K, seed, oracle.p(p), oracle.p(s), oracle.p(d))
        out += [p.reshape(rows, K // 2), s.reshape(rows, K // 32), d]
    return out


def test_mxfp4_exact_gemm_vs_reference_gemm(R):
    M, N, K = 24, 40, 512
    qa, sa, da, qb, sb, db = ref_operands(R, M, N, K)
    exact = oracle.gemm_mx_exact(qa, sa, qb, sb, 4)
    ref = np.empty((M, N), np.float32)
    R.ref_reference_gemm(oracle.p(da), oracle.p(db), M, N, K, 1.0, oracle.p(ref))
    np.testing.assert_array_equal(exact.astype(np.float32), ref)
    np.testing.assert_array_equal(exact, da.astype(np.float64) @ db.astype(np.float64).T)


def mx4_operands(M, N, K, seed=1, rule=0):
    xa = oracle.gen_mx_input(M, K, seed * 7919 + 1, 1.0, 4)
    xb = oracle.gen_mx_input(N, K, seed * 7919 + 2, 1.0, 4)
    qa, sa = oracle.quant_mxfp4(xa, rule)
    qb, sb = oracle.quant_mxfp4(xb, rule)
    return qa, sa, qb, sb


@pytest.mark.parametrize("l2", [0, 1, 2])
def test_mxfp4_fp32acc_step_model(l2):
    """fp32acc = per 128-K step fp32(acc + exact step sum), slices of
    round_up(K/2^L, 256) summed in order (the MXFP8 model, f4gemm.hpp:342-344)."""
    M, N, K = 8, 12, 1024
    qa, sa, qb, sb = mx4_operands(M, N, K, seed=5)
    got = oracle.gemm_mx_fp32acc(qa, sa, qb, sb, 4, l2)
    A, B = oracle.mx4_dequant(qa, sa), oracle.mx4_dequant(qb, sb)
    kpt = ((K >> l2) + 255) // 256 * 256
    want = np.zeros((M, N), np.float32)
    for z in range(0, K, kpt):
        acc = np.zeros((M, N), np.float32)
        for k in range(z, min(K, z + kpt), 128):
            step = A[:, k:k + 128] @ B[:, k:k + 128].T     # exact in f64 here
            acc = (acc.astype(np.float64) + step).astype(np.float32)
        want = acc if z == 0 else (want + acc).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_mxfp4_planted_nibble_swap_is_caught(R):
    """Decoding with the nibbles swapped (high = even element) must not match the
    reference's dequantised values."""
    M, K = 8, 256
    qa, sa, da, _, _, _ = ref_operands(R, M, 8, K)
    swapped = ((qa & 15) << 4) | (qa >> 4)
    deq = oracle.mx4_dequant(swapped.astype(np.uint8), sa).astype(np.float32)
    assert not np.array_equal(deq, da)

"""Shared helpers for the parity tests: operand preparation and the tolerance rule."""
import numpy as np

import oracle

# bf16 outputs must be within 1 bf16 ULP or relative error <= 2^-7 of the
# oracle's fp32-accumulated result, whichever is looser (north-star rule).
REL_TOL = 2.0 ** -7
MAX_ULP = 1

# The gfx950 FP8 MFMA does not add its 128 products exactly: measured on the
# GPU, each group of 8 consecutive K products is aligned to the group's largest
# operand-exponent sum and truncated toward zero to 13 fractional bits, so one
# output can be off by up to 8 * 2^-13 * max|p| per group, i.e. at most
# 2^-10 * sum_k |a_k b_k| (with the block scales applied). Where an output
# cancels (|C| << sum |a b|) that exceeds 1 ULP / 2^-7 of |C| for any
# MFMA-based kernel, so such outputs are accepted when within
# MFMA_BOUND_FACTOR * sum |a b| (a factor 2 above the derived bound) and are
# counted separately ("bounded").
MFMA_BOUND_FACTOR = 2.0 ** -9


def bf16_compare(got_bits, want_bits, absdot=None):
    """Returns (ok mask, stats) for bf16 bit arrays under the tolerance rule;
    absdot (sum |a b| per output) enables the MFMA truncation bound."""
    got_bits = np.asarray(got_bits, dtype=np.uint16)
    want_bits = np.asarray(want_bits, dtype=np.uint16)
    g = oracle.bf16_bits_to_f32(got_bits).astype(np.float64)
    w = oracle.bf16_bits_to_f32(want_bits).astype(np.float64)
    # ULP distance on the monotone integer line of bf16 codes
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    ulp = np.abs(ordered(got_bits) - ordered(want_bits))
    rel = np.abs(g - w) / np.maximum(np.abs(w), 1e-38)
    strict = (ulp <= MAX_ULP) | (rel <= REL_TOL)
    ok = strict.copy()
    if absdot is not None:
        # the bound also covers the final bf16 rounding of the result
        ok |= np.abs(g - w) <= MFMA_BOUND_FACTOR * absdot + np.abs(w) * 2.0 ** -8
    stats = dict(n=int(got_bits.size), exact=float((ulp == 0).mean()) if got_bits.size else 1.0,
                 max_ulp=int(ulp.max()) if got_bits.size else 0,
                 bounded=int((ok & ~strict).sum()), bad=int((~ok).sum()))
    return ok, stats


def f32_compare(got, want, rel_tol=REL_TOL, absdot=None):
    """fp32 outputs: exact-match fraction and violations of |d| <= rel_tol*|want|
    or 1 fp32 ulp, or (absdot given) the MFMA truncation bound."""
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    gi = got.view(np.int32).astype(np.int64)
    wi = want.view(np.int32).astype(np.int64)
    def ordered(i):
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    ulp = np.abs(ordered(gi) - ordered(wi))
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), 1e-38)
    strict = (ulp <= 1) | (rel <= rel_tol)
    ok = strict.copy()
    if absdot is not None:
        ok |= np.abs(got.astype(np.float64) - want) <= MFMA_BOUND_FACTOR * absdot
    return ok, dict(n=int(got.size), exact=float((ulp == 0).mean()), max_ulp=int(ulp.max()),
                    bounded=int((ok & ~strict).sum()), bad=int((~ok).sum()))


def mx_operands(M, N, K, seed=1, std_b=1.0, rule=0, spread=4):
    """Seeded MX operands: x ~ N(0, std) * 2^u per 1x32 block, quantised by the oracle."""
    xa = oracle.gen_mx_input(M, K, seed * 7919 + 1, 1.0, spread)
    xb = oracle.gen_mx_input(N, K, seed * 7919 + 2, std_b, spread)
    qa, sa = oracle.quant_mxfp8(xa, rule)
    qb, sb = oracle.quant_mxfp8(xb, rule)
    return qa, sa, qb, sb

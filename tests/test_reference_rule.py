"""The reference-rule helpers on the CPU: the MFMA model's own outputs held
against the reference's reference_gemm (asm_f4gemm/f4gemm_ref.hpp:181-222,
oracle/_ref) as the GPU tests hold the kernels' outputs, and planted mistakes
that the checks must catch. Also the block-scale drivers' check
(gemm_a8w8_blockscale_host.cc:47-63, 273-274: |C - gemm_ref| <= 1e-3 on fp32
C) applied to the MFMA model on the drivers' operand distribution, which is
what the GPU test of that check expects of the kernels."""
import numpy as np
import pytest
import torch

import oracle
from helpers import (MFMA_TRUNC_BOUND, dequant_mx_f32, hold_to_reference, mx_operands,
                     north_star_misses, reference_gemm)


def config1():
    M, N, K = 256, 256, 512
    qa, sa = oracle.quant_mxfp8(oracle.gen_mx_input(M, K, seed=1234))
    qb, sb = oracle.quant_mxfp8(oracle.gen_mx_input(N, K, seed=5678))
    return qa, sa, qb, sb


def test_north_star_misses_hand_cases():
    ref = np.array([1.0, 1.0, 1.0, 1.0, 0.0, -3.0, 1e-30], np.float32)
    got = np.array([1.0, 1.0 + 2.0 ** -7, 1.0 + 2.0 ** -6, 1.0 - 2.0 ** -7, 2.0 ** -20,
                    -3.0 - 2.0 ** -6, 0.0], np.float32)
    miss, ulp = north_star_misses(oracle.to_bf16_bits(got), ref)
    # 0 ULP; 1 ULP; 2 ULP at relative 2^-6; 2 ULP below 1.0 (ULP 2^-8 there)
    # at relative 2^-7; a non-zero output for an exact zero; 1 ULP (2^-6) at -3;
    # 0 for 1e-30 (many ULP, relative error 1)
    np.testing.assert_array_equal(miss, [False, False, True, False, True, False, True])
    np.testing.assert_array_equal(ulp[:4], [0, 1, 2, 2])


def test_mx_dequant_f32_is_exact():
    qa, sa, _, _ = mx_operands(64, 32, 512, seed=3)
    np.testing.assert_array_equal(dequant_mx_f32(qa, sa).astype(np.float64),
                                  oracle.mx_dequant(qa, sa))


def test_model_against_reference_gemm_config1(R):
    """The MFMA model's config-1 output (bit-identical to the GPU's on all but
    a few outputs) under the north-star rule against reference_gemm: 40 of
    65536 outputs miss, all of them outputs that cancel."""
    qa, sa, qb, sb = config1()
    A, B = dequant_mx_f32(qa, sa), dequant_mx_f32(qb, sb)
    ref = reference_gemm(R, A, B)
    # reference_gemm sums in f64: it equals the exact oracle rounded to fp32
    np.testing.assert_array_equal(ref, oracle.gemm_mxfp8_exact(qa, sa, qb, sb).astype(np.float32))
    model = oracle.to_bf16_bits(oracle.gemm_mx_mfma(qa, sa, qb, sb, 0))
    out = hold_to_reference("model config 1", model, ref, A, B, model)
    assert out["misses"] == 40
    assert out["model_misses"] == 40 and out["gpu_model_differ"] == 0
    # every miss cancels by more than 9 binades (|ref| < 2^-9 sum |a b|)
    assert out["max_ref_over_absdot_miss"] < 2.0 ** -9
    assert out["worst_err_over_absdot"] < MFMA_TRUNC_BOUND / 16
    # the exact result rounded to bf16 misses nothing
    exact_bits = oracle.to_bf16_bits(ref)
    assert hold_to_reference("exact config 1", exact_bits, ref, A, B)["misses"] == 0


def test_planted_mistakes_are_caught(R):
    qa, sa, qb, sb = config1()
    A, B = dequant_mx_f32(qa, sa), dequant_mx_f32(qb, sb)
    ref = reference_gemm(R, A, B)
    model = oracle.to_bf16_bits(oracle.gemm_mx_mfma(qa, sa, qb, sb, 0))
    # an output that does not cancel, 4 bf16 ULP off: beyond the truncation bound
    absdot = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)).T
    i, j = np.unravel_index(np.argmax(np.abs(ref) / absdot), ref.shape)
    bad = model.copy()
    bad[i, j] = bad[i, j] + 4
    with pytest.raises(AssertionError):
        hold_to_reference("planted 4 ULP", bad, ref, A, B)
    # a dropped K block (one 1x32 scale block of A zeroed): many misses
    qz = qa.copy()
    qz[:, 64:96] = 0
    dropped = oracle.to_bf16_bits(oracle.gemm_mx_mfma(qz, sa, qb, sb, 0))
    with pytest.raises(AssertionError):
        hold_to_reference("planted dropped block", dropped, ref, A, B)
    # the cap: 20 more cancelling outputs pushed off by 2^-12 sum |a b| (within
    # the truncation bound, outside the rule) than the model's 40 misses
    miss, _ = north_star_misses(model, ref)
    cand = np.argwhere(~miss & (np.abs(ref) < 2.0 ** -6 * absdot))[:20]
    assert len(cand) == 20
    off = model.copy()
    for i, j in cand:
        off[i, j] = oracle.to_bf16_bits(np.array([ref[i, j] + 2.0 ** -12 * absdot[i, j]],
                                                  np.float32))[0]
    with pytest.raises(AssertionError, match="allow"):
        hold_to_reference("planted cap", off, ref, A, B, model)


def driver_operands(batch, M, N, K, seed):
    g = torch.Generator()
    g.manual_seed(seed)
    a = torch.rand((batch, M, K), generator=g).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    b = (torch.rand((batch, N, K), generator=g) - 0.5).to(torch.float8_e4m3fn).view(
        torch.uint8).numpy()
    sfa = (torch.rand((batch, K // 128, M), generator=g) * 0.4 + 0.8).numpy()
    sfb = (torch.rand((batch, (N + 127) // 128, K // 128), generator=g) * 0.4 + 0.8).numpy()
    return a, b, sfa, sfb


@pytest.mark.parametrize("MNK", [(256, 512, 256), (16, 1024, 8192)])
def test_blockscale_driver_check_holds_for_the_model(MNK):
    """The MFMA model of the block-scale kernels is within the drivers' 1e-3
    of gemm_ref on their data, also at K = 8192 (max measured ~3e-4); a
    planted SFB transpose is not."""
    M, N, K = MNK
    a, b, sfa, sfb = driver_operands(1, M, N, K, 11)
    ref = oracle.gemm_blockscale_ref(a[0], b[0], sfa[0], sfb[0], 128)
    model = oracle.gemm_blockscale_mfma(a[0], b[0], sfa[0], sfb[0], 128, 0)
    d = np.abs(model.astype(np.float64) - ref)
    assert d.max() <= 1e-3
    if sfb.shape[1] == sfb.shape[2]:
        planted = oracle.gemm_blockscale_mfma(a[0], b[0], sfa[0],
                                              np.ascontiguousarray(sfb[0].T), 128, 0)
        assert np.abs(planted.astype(np.float64) - ref).max() > 1e-3

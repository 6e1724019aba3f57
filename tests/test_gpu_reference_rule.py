"""GPU GEMM outputs held against the reference's own CPU references and its
own pass rules (the other GPU tests hold them against the oracle's model of
the MFMA).

* MXFP8, config 1 (256x256x512, every output): reference_gemm
  (asm_f4gemm/f4gemm_ref.hpp:181-222, the reference's own header compiled
  into oracle/_ref) under the north-star rule. The FP8 MFMA truncates
  products inside a 128-K step (helpers.MFMA_TRUNC_BOUND), so outputs that
  cancel to far below sum |a b| miss the rule; helpers.hold_to_reference
  counts them, bounds each one and caps their number by the MFMA model's own
  misses on the same data. The benchmark's 4096^3, 8192^3 and decode shapes
  get the same check in test_gpu_configs.py.
* MXFP4 on the reference's own operand generator (make_operand,
  f4gemm_ref.hpp:132-176, seeds 1234 / 5678 as main.cpp:189-190) under the
  reference's pass rule (main.cpp:256-290: |d| <= atol + 2e-2 |ref|, atol =
  2e-4 max|ref|, 2e-2 max|ref| with split-K), on run_tests.sh:37-57's shapes.
* Block scale on the reference drivers' own operand distribution (A ~
  U[0,1), B ~ U[-0.5,0.5) as E4M3, SFA / SFB ~ U[0.8,1.2):
  gemm_a8w8_blockscale_host.cc:207-210) under their -v check, |d| <= 1e-3
  on fp32 C against gemm_ref (:66-90; restated as or_gemm_blockscale_ref, its
  file needing aiter's absent headers): the driver's default problem
  (256x512x256, batch 8), the 1x128x1 driver's default (4096x12288x2048,
  gemm_a8w8_1x128x1_blockscale_host.cc:162-169, verify on), and the
  benchmark's 8192^3 reference-data leg.
"""
import numpy as np
import pytest
import torch

import bench
import oracle
from gcnasm_amd import f4gemm, opus_gemm
from helpers import (dequant_mx_f32, hold_to_reference, mx_operands, reference_gemm,
                     tile_rows)

pytestmark = pytest.mark.gpu


def run_mx(dev, qa, sa, qb, sb, l2):
    """MXFP8 GEMM through the heuristic's kernel at log2 split l2 (-1: the
    heuristic's split); bf16 output bits [M, N]."""
    M, K = qa.shape
    N = qb.shape[0]
    idx, l2 = f4gemm.select_kernel(M, N, K, 256, l2, 1)
    cfg = f4gemm.manifest()[idx]
    sh = f4gemm.Shape(M, N, K)
    a_pad = np.zeros((sh.a_rows_pad(), K), dtype=np.uint8)
    a_pad[:M] = qa
    A = torch.from_numpy(a_pad).to(dev)
    B = torch.from_numpy(f4gemm.shuffle_weight_16x16(qb, N, K)).to(dev)
    SA = torch.from_numpy(f4gemm.shuffle_scale(sa, M, K // 32, sh.scale_a_rows(),
                                               sh.scale_cols())).to(dev)
    SB = torch.from_numpy(f4gemm.shuffle_scale(sb, N, K // 32, sh.scale_b_rows(),
                                               sh.scale_cols())).to(dev)
    D = torch.full((sh.d_rows_pad(), N), float("nan"), dtype=torch.bfloat16, device=dev)
    ld = f4gemm.make_launch(cfg, M, N, K, l2)
    args = f4gemm.fill_args(D, None, A, B, SA, SB, M, N, K, N, sh.scale_cols(), sh.scale_cols(),
                            1.0, 0.0, ld.log2_k_split)
    print("launch %s M=%d N=%d K=%d grid=(%d,%d,%d)" % (cfg.knl_name, M, N, K, ld.gdx, ld.gdy,
                                                         ld.gdz), flush=True)
    f4gemm.Kernel().load(None, cfg).launch(args, ld.gdx, ld.gdy, ld.gdz)
    torch.cuda.synchronize()
    return D[:M].view(torch.int16).cpu().numpy().view(np.uint16), ld.log2_k_split


@pytest.mark.parametrize("seeds", [(1234, 5678), (1, 2), (3, 4), (5, 6)])
def test_mxfp8_config1_vs_reference_gemm(dev, R, seeds):
    """Config 1, every output; the first seed pair is the smoke run's."""
    M, N, K = 256, 256, 512
    if seeds == (1234, 5678):
        qa, sa = oracle.quant_mxfp8(oracle.gen_mx_input(M, K, seed=1234))
        qb, sb = oracle.quant_mxfp8(oracle.gen_mx_input(N, K, seed=5678))
    else:
        qa, sa, qb, sb = mx_operands(M, N, K, seed=seeds[0] * 100 + seeds[1])
    got, l2 = run_mx(dev, qa, sa, qb, sb, 0)
    A, B = dequant_mx_f32(qa, sa), dequant_mx_f32(qb, sb)
    ref = reference_gemm(R, A, B)
    model = oracle.to_bf16_bits(oracle.gemm_mx_mfma(qa, sa, qb, sb, l2))
    hold_to_reference("MXFP8 config 1 seeds %s" % (seeds,), got, ref, A, B, model)


# ---- MXFP4 on the reference's own operands and pass rule ---------------------
def make_operand(R, rows, K, seed):
    """The reference's make_operand (f4gemm_ref.hpp:145-176): packed e2m1
    [rows, K/2], E8M0 scales [rows, K/32], dequantised fp32 [rows, K]."""
    p = np.empty(rows * K // 2, np.uint8)
    s = np.empty(rows * K // 32, np.uint8)
    d = np.empty((rows, K), np.float32)
    R.ref_make_operand(rows, K, seed, oracle.p(p), oracle.p(s), oracle.p(d))
    return p.reshape(rows, K // 2), s.reshape(rows, K // 32), d


def run_mx4(dev, qa, sa, qb, sb, cfg, l2):
    M, Kp = qa.shape
    K = 2 * Kp
    N = qb.shape[0]
    sh = f4gemm.Shape(M, N, K, elem_bits=4)
    a_pad = np.zeros((sh.a_rows_pad(), Kp), dtype=np.uint8)
    a_pad[:M] = qa
    A = torch.from_numpy(a_pad).to(dev)
    bh = f4gemm.shuffle_weight_16x16(qb, N, Kp) if cfg.bpreshuffle else qb.reshape(-1)
    B = torch.from_numpy(np.ascontiguousarray(bh)).to(dev)
    SA = torch.from_numpy(f4gemm.shuffle_scale(sa, M, K // 32, sh.scale_a_rows(),
                                               sh.scale_cols())).to(dev)
    SB = torch.from_numpy(f4gemm.shuffle_scale(sb, N, K // 32, sh.scale_b_rows(),
                                               sh.scale_cols())).to(dev)
    D = torch.full((sh.d_rows_pad(), N), float("nan"), dtype=torch.bfloat16, device=dev)
    ld = f4gemm.make_launch(cfg, M, N, K, l2)
    args = f4gemm.fill_args(D, None, A, B, SA, SB, M, N, K, N, sh.scale_cols(), sh.scale_cols(),
                            1.0, 0.0, ld.log2_k_split)
    print("launch %s M=%d N=%d K=%d grid=(%d,%d,%d)" % (cfg.knl_name, M, N, K, ld.gdx, ld.gdy,
                                                         ld.gdz), flush=True)
    f4gemm.Kernel().load(None, cfg).launch(args, ld.gdx, ld.gdy, ld.gdz)
    torch.cuda.synchronize()
    return D[:M].view(torch.int16).cpu().numpy().view(np.uint16), ld


def verify_like_main_cpp(label, got_bits, ref, split):
    """main.cpp:256-290: |got - ref| <= atol + 2e-2 |ref| with atol = 2e-4
    max|ref| (2e-2 max|ref| with split-K); returns the worst relative error
    over outputs above atol (its max_rel_err)."""
    got = oracle.bf16_bits_to_f32(got_bits).astype(np.float64)
    r = ref.astype(np.float64)
    max_abs_ref = float(np.abs(r).max())
    atol = (2e-2 if split else 2e-4) * max_abs_ref
    d = np.abs(got - r)
    bad = int((d > atol + 2e-2 * np.abs(r)).sum())
    big = np.abs(r) > atol
    worst_rel = float((d[big] / np.abs(r[big])).max()) if big.any() else 0.0
    print("%s: max|ref|=%.4g max_abs_err=%.4g max_rel_err=%.4g mismatches=%d/%d" % (
        label, max_abs_ref, float(d.max()), worst_rel, bad, d.size), flush=True)
    assert bad == 0, "%s: %d mismatches under main.cpp's rule" % (label, bad)
    return worst_rel


# run_tests.sh:37-41 (heuristic sweep)
MX4_HEURISTIC_SHAPES = [(128, 1024, 1024), (256, 2048, 2048), (300, 2048, 1024), (1, 4096, 2048),
                        (17, 512, 256), (512, 1024, 2048), (2048, 8192, 1024), (4096, 4096, 512)]


@pytest.mark.parametrize("shape", MX4_HEURISTIC_SHAPES)
def test_mxfp4_reference_operands_heuristic(dev, R, shape):
    M, N, K = shape
    qa, sa, da = make_operand(R, M, K, 1234)
    qb, sb, db = make_operand(R, N, K, 5678)
    idx, l2 = f4gemm.select_kernel(M, N, K, 256, 0, 1, f4gemm.manifest_fp4())
    cfg = f4gemm.manifest_fp4()[idx]
    got, ld = run_mx4(dev, qa, sa, qb, sb, cfg, l2)
    ref = reference_gemm(R, da, db)
    worst = verify_like_main_cpp("MXFP4 heuristic %dx%dx%d %s" % (M, N, K, cfg.knl_name), got,
                                 ref, ld.gdz > 1)
    # products of e2m1 codes are exact and the MFMA adds them exactly: the
    # only error left is the output's bf16 rounding (asm_f4gemm/README.md:151
    # reports max_rel_err 0.003891 = 2^-8)
    assert worst <= 2.0 ** -8


@pytest.mark.parametrize("name", [c.knl_name for c in f4gemm.manifest_fp4()])
def test_mxfp4_reference_operands_every_kernel(dev, R, name):
    """run_tests.sh:43-49: every manifest kernel at M=300 N=2048 K=1024."""
    M, N, K = 300, 2048, 1024
    cfg = [c for c in f4gemm.manifest_fp4() if c.knl_name == name][0]
    qa, sa, da = make_operand(R, M, K, 1234)
    qb, sb, db = make_operand(R, N, K, 5678)
    got, ld = run_mx4(dev, qa, sa, qb, sb, cfg, 0)
    worst = verify_like_main_cpp("MXFP4 %s" % name, got, reference_gemm(R, da, db), ld.gdz > 1)
    assert worst <= 2.0 ** -8


@pytest.mark.parametrize("tile", ["256x256", "128x512"])
@pytest.mark.parametrize("l2", [1, 2, 3, 4])
def test_mxfp4_reference_operands_splitk(dev, R, tile, l2):
    """run_tests.sh:51-57: split-K 1-4 on two tiles at 256x1024x4096. The
    slices here are summed in fp32 (the reference's kernels add bf16
    partials), so the no-split rule holds as well."""
    M, N, K = 256, 1024, 4096
    cfg = [c for c in f4gemm.manifest_fp4()
           if c.knl_name.endswith("BpreShuffle_%s_splitK" % tile)][0]
    qa, sa, da = make_operand(R, M, K, 1234)
    qb, sb, db = make_operand(R, N, K, 5678)
    got, ld = run_mx4(dev, qa, sa, qb, sb, cfg, l2)
    assert ld.gdz == 1 << l2
    ref = reference_gemm(R, da, db)
    verify_like_main_cpp("MXFP4 %s split %d" % (tile, l2), got, ref, True)
    worst = verify_like_main_cpp("MXFP4 %s split %d (no-split rule)" % (tile, l2), got, ref,
                                 False)
    assert worst <= 2.0 ** -8


# ---- block scale on the reference drivers' data and -v check ------------------
def driver_operands(dev, batch, M, N, K, group_n, seed):
    """The reference drivers' distribution (gemm_a8w8_blockscale_host.cc:
    207-210), generated on the GPU: A [batch, M, K], B [batch, N, K] E4M3
    bytes; SFA [batch, K/128, M]; SFB [batch, ceil(N/128), K/128] (group_n
    128) or [batch, K/128, N] (group_n 1)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.rand((batch, M, K), device=dev, generator=g).to(torch.float8_e4m3fn).view(
        torch.uint8)
    b = (torch.rand((batch, N, K), device=dev, generator=g) - 0.5).to(
        torch.float8_e4m3fn).view(torch.uint8)
    sfa = torch.rand((batch, K // 128, M), device=dev, generator=g) * 0.4 + 0.8
    shape_b = (batch, (N + 127) // 128, K // 128) if group_n == 128 else (batch, K // 128, N)
    sfb = torch.rand(shape_b, device=dev, generator=g) * 0.4 + 0.8
    return a, b, sfa, sfb


def driver_check(label, got, qa, qb, sfa, sfb, group_n, rows):
    """The drivers' -v check on `rows`: |C - gemm_ref| <= 1e-3 on fp32 C
    (valid_vector, gemm_a8w8_blockscale_host.cc:47-63, 273-274)."""
    qa_r = np.ascontiguousarray(qa[rows])
    sfa_r = np.ascontiguousarray(sfa[:, rows])
    want = oracle.gemm_blockscale_ref(qa_r, qb, sfa_r, sfb, group_n)
    d = np.abs(got.astype(np.float64) - want)
    bad = int((d > 1e-3).sum())
    print("%s: max |C - gemm_ref| = %.3g over %d outputs (rule 1e-3), above it: %d" % (
        label, float(d.max()), d.size, bad), flush=True)
    assert bad == 0


def test_blockscale_driver_default(dev):
    """gemm_a8w8_blockscale_host.cc's default problem: 256x512x256, batch 8,
    every output of every batch."""
    batch, M, N, K = 8, 256, 512, 256
    a, b, sfa, sfb = driver_operands(dev, batch, M, N, K, 128, 11)
    c = torch.full((batch, M, N), float("nan"), dtype=torch.float32, device=dev)
    opus_gemm.blockscale_gemm(a, b, sfa, sfb, c)
    torch.cuda.synchronize()
    got, qa, qb = c.cpu().numpy(), a.cpu().numpy(), b.cpu().numpy()
    fa, fb = sfa.cpu().numpy(), sfb.cpu().numpy()
    for i in range(batch):
        driver_check("block scale driver default, batch %d" % i, got[i], qa[i], qb[i], fa[i],
                     fb[i], 128, np.arange(M))


def test_blockscale_1x128x1_driver_default(dev):
    """gemm_a8w8_1x128x1_blockscale_host.cc's default (4096x12288x2048, one
    SFB per output column and 128-K group, verify on); every 256-row tile
    checked on one row (helpers.tile_rows)."""
    M, N, K = 4096, 12288, 2048
    a, b, sfa, sfb = driver_operands(dev, 1, M, N, K, 1, 12)
    c = torch.empty((M, N), dtype=torch.float32, device=dev)
    opus_gemm.blockscale_gemm(a[0], b[0], sfa[0], sfb[0], c, group_n=1)
    torch.cuda.synchronize()
    rows = tile_rows(M)
    driver_check("block scale 1x128x1 driver default (%d rows)" % len(rows),
                 c.cpu().numpy()[rows], a[0].cpu().numpy(), b[0].cpu().numpy(),
                 sfa[0].cpu().numpy(), sfb[0].cpu().numpy(), 1, rows)


def test_blockscale_8192_reference_data(dev):
    """The benchmark's block-scale reference-data leg (bench.ref_bs_operands,
    its seed), 8192^3, fp32 C, under the driver's check on tile_rows."""
    n = 8192
    ra, rb, rsfa, rsfb = bench.ref_bs_operands(torch, n, 7)
    c = torch.empty((n, n), dtype=torch.float32, device=dev)
    opus_gemm.blockscale_gemm(ra, rb, rsfa, rsfb, c)
    torch.cuda.synchronize()
    rows = tile_rows(n)
    got = c.cpu().numpy()[rows]
    del c
    driver_check("block scale 8192^3 reference data (%d rows)" % len(rows), got,
                 ra.cpu().numpy(), rb.cpu().numpy(), rsfa.cpu().numpy(), rsfb.cpu().numpy(),
                 128, rows)

"""GPU parity of the MXFP8 GEMM (f4gemm ABI) against the CPU oracle.

Cases follow the reference's regression sweep (asm_f4gemm/run_tests.sh:37-57):
a heuristic shape sweep, every manifest kernel at M=300 N=2048 K=1024, and
split-K with log2 splits 1..4; plus config 1 of the benchmark, decode shapes,
alpha/beta and error paths. Expected values come from oracle.gemm_mx_mfma
(the FP8 MFMA's own 128-K step sum, accumulated in fp32 in the kernel's K
order, slices summed in order) rounded to bf16; the tolerance is the
north-star rule (helpers.bf16_compare / assert_parity).
"""
import ctypes
import re

import numpy as np
import pytest
import torch

import oracle
from gcnasm_amd import _lib, f4gemm
from gcnasm_amd._lib import GaError
from helpers import assert_parity, bf16_compare, mx_operands

pytestmark = pytest.mark.gpu


def run_mx(dev, qa, sa, qb, sb, cfg, log2_k_split=0, alpha=1.0, beta=0.0, c_in=None,
           workspace=None):
    M, K = qa.shape
    N = qb.shape[0]
    sh = f4gemm.Shape(M, N, K)
    a_pad = np.zeros((sh.a_rows_pad(), K), dtype=np.uint8)
    a_pad[:M] = qa
    A = torch.from_numpy(a_pad).to(dev)
    bh = f4gemm.shuffle_weight_16x16(qb, N, K) if cfg.bpreshuffle else qb.reshape(-1)
    B = torch.from_numpy(np.ascontiguousarray(bh)).to(dev)
    SA = torch.from_numpy(f4gemm.shuffle_scale(sa, M, K // 32, sh.scale_a_rows(),
                                               sh.scale_cols())).to(dev)
    SB = torch.from_numpy(f4gemm.shuffle_scale(sb, N, K // 32, sh.scale_b_rows(),
                                               sh.scale_cols())).to(dev)
    D = torch.full((sh.d_rows_pad(), N), float("nan"), dtype=torch.bfloat16, device=dev)
    C = None
    if c_in is not None:
        C = torch.from_numpy(c_in.view(np.int16)).to(dev).view(torch.bfloat16)
    ld = f4gemm.make_launch(cfg, M, N, K, log2_k_split)
    args = f4gemm.fill_args(D, C, A, B, SA, SB, M, N, K, N, sh.scale_cols(), sh.scale_cols(),
                            alpha, beta, ld.log2_k_split)
    k = f4gemm.Kernel().load(None, cfg)
    k.launch(args, ld.gdx, ld.gdy, ld.gdz, workspace=workspace)
    torch.cuda.synchronize()
    out = D[:M].view(torch.int16).cpu().numpy().view(np.uint16)
    return out, ld


def expect(qa, sa, qb, sb, log2_k_split=0, alpha=1.0):
    return oracle.to_bf16_bits(oracle.gemm_mx_mfma(qa, sa, qb, sb, log2_k_split, alpha))


def check(got, want, label, absdot):
    ok, st = bf16_compare(got, want, absdot)
    assert_parity(st, label)
    return st


def cfg_named(name):
    """Manifest row of `name`, or for kernels reachable only by name
    (ga_kernel_find) a row built from the tile encoded in the name."""
    for c in f4gemm.manifest():
        if c.knl_name == name:
            return c
    m = re.search(r"_(\d+)x(\d+)", name)
    return f4gemm.Config(int(m.group(1)), int(m.group(2)), int("_splitK" in name),
                         int("noBpreShuffle" not in name), name, name + ".co")


# Kernels outside the manifest, reachable by name.
NAMED_ONLY = ["ga_mxfp8_bf16_BpreShuffle_256x256_ns2"]

# The 256x256 eight-wave tiles, run on shapes with partial tiles, a single K
# step and one row.
PP_KERNELS = ["ga_mxfp8_bf16_BpreShuffle_256x256", "ga_mxfp8_bf16_BpreShuffle_256x256_splitK",
              "ga_mxfp8_bf16_noBpreShuffle_256x256"]


def test_config1_heuristic(dev):
    """Benchmark config 1: M=256 N=256 K=512 through the heuristic choice."""
    M, N, K = 256, 256, 512
    qa, sa, qb, sb = mx_operands(M, N, K, seed=1)
    idx, l2 = f4gemm.select_kernel(M, N, K, 256, 0, 1)
    cfg = f4gemm.manifest()[idx]
    got, _ = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    st = check(got, expect(qa, sa, qb, sb, l2), "config1 " + cfg.knl_name,
               oracle.mx_absdot(qa, sa, qb, sb))
    # bf16 outputs bit-identical to the MFMA-model oracle but for rounding
    # boundaries the model's residual crosses
    assert st["exact"] > 0.999


@pytest.mark.parametrize("shape", [(128, 1024, 1024), (256, 2048, 2048), (300, 2048, 1024),
                                   (1, 4096, 2048), (17, 512, 256), (512, 1024, 2048),
                                   (2048, 8192, 1024), (4096, 4096, 512)])
def test_heuristic_sweep(dev, shape):
    M, N, K = shape
    qa, sa, qb, sb = mx_operands(M, N, K, seed=M + N + K)
    idx, l2 = f4gemm.select_kernel(M, N, K, 256, 0, 1)
    cfg = f4gemm.manifest()[idx]
    rows = slice(None) if M * N * K <= 2 ** 32 else slice(0, 256)
    got, _ = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    want = expect(qa[rows], sa[rows], qb, sb, l2)
    check(got[rows], want, "sweep %s %s" % (shape, cfg.knl_name),
          oracle.mx_absdot(qa[rows], sa[rows], qb, sb))


@pytest.mark.parametrize("name", [c.knl_name for c in f4gemm.manifest()])
def test_every_kernel(dev, name):
    M, N, K = 300, 2048, 1024
    cfg = cfg_named(name)
    qa, sa, qb, sb = mx_operands(M, N, K, seed=3)
    got, _ = run_mx(dev, qa, sa, qb, sb, cfg, 0)
    check(got, expect(qa, sa, qb, sb, 0), name, oracle.mx_absdot(qa, sa, qb, sb))


@pytest.mark.parametrize("name", NAMED_ONLY + PP_KERNELS)
@pytest.mark.parametrize("shape", [(300, 2048, 1024), (520, 784, 1536), (256, 256, 128),
                                   (1, 256, 256), (777, 1040, 2048)])
def test_large_tiles_edge_shapes(dev, name, shape):
    """Large tiles (in the manifest or found by name only) on shapes with
    partial M and N tiles, a single K step and a single row."""
    M, N, K = shape
    cfg = cfg_named(name)
    assert (cfg in f4gemm.manifest()) == (name not in NAMED_ONLY)
    qa, sa, qb, sb = mx_operands(M, N, K, seed=M + 7 * N + K)
    got, _ = run_mx(dev, qa, sa, qb, sb, cfg, 0)
    check(got, expect(qa, sa, qb, sb, 0), "%s %s" % (name, shape),
          oracle.mx_absdot(qa, sa, qb, sb))


@pytest.mark.parametrize("name", ["ga_mxfp8_bf16_BpreShuffle_256x128_splitK",
                                  "ga_mxfp8_bf16_BpreShuffle_32x256_splitK",
                                  "ga_mxfp8_bf16_BpreShuffle_256x256_splitK"])
@pytest.mark.parametrize("l2", [1, 2, 3, 4])
def test_splitk(dev, name, l2):
    M, N, K = 256, 1024, 4096
    cfg = cfg_named(name)
    qa, sa, qb, sb = mx_operands(M, N, K, seed=10 + l2)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    assert ld.gdz == 1 << l2
    check(got, expect(qa, sa, qb, sb, l2), "%s splitk=%d" % (name, l2),
          oracle.mx_absdot(qa, sa, qb, sb))


@pytest.mark.parametrize("M", [1, 16, 64])
@pytest.mark.parametrize("NK", [(2048, 4096), (1024, 8192)])
def test_decode_shapes(dev, M, NK):
    """Decode-shaped GEMMs (weights from N(0, 0.02)) with the heuristic's split-K."""
    N, K = NK
    qa, sa, qb, sb = mx_operands(M, N, K, seed=M, std_b=0.02)
    idx, l2 = f4gemm.select_kernel(M, N, K, 256, -1, 1)
    cfg = f4gemm.manifest()[idx]
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    check(got, expect(qa, sa, qb, sb, l2), "decode M=%d N=%d K=%d %s gdz=%d" %
          (M, N, K, cfg.knl_name, ld.gdz), oracle.mx_absdot(qa, sa, qb, sb))


def test_alpha_beta(dev):
    M, N, K = 128, 256, 512
    qa, sa, qb, sb = mx_operands(M, N, K, seed=77)
    rng = np.random.default_rng(5)
    c = oracle.to_bf16_bits(rng.standard_normal((M, N)).astype(np.float32))
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_128x128")
    got, _ = run_mx(dev, qa, sa, qb, sb, cfg, 0, alpha=0.5, beta=2.0, c_in=c)
    acc = oracle.gemm_mx_mfma(qa, sa, qb, sb, 0, 1.0)
    v = (np.float32(0.5) * acc).astype(np.float32)
    v = (v + (np.float32(2.0) * oracle.bf16_bits_to_f32(c)).astype(np.float32)).astype(np.float32)
    check(got, oracle.to_bf16_bits(v), "alpha/beta", 0.5 * oracle.mx_absdot(qa, sa, qb, sb))


def test_explicit_workspace_and_too_small(dev):
    M, N, K = 64, 512, 2048
    qa, sa, qb, sb = mx_operands(M, N, K, seed=9)
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_64x256_splitK")
    ws = torch.empty(4 * M * N, dtype=torch.float32, device=dev)
    got, _ = run_mx(dev, qa, sa, qb, sb, cfg, 2, workspace=ws)
    check(got, expect(qa, sa, qb, sb, 2), "explicit workspace", oracle.mx_absdot(qa, sa, qb, sb))
    small = torch.empty(16, dtype=torch.float32, device=dev)
    with pytest.raises(GaError) as e:
        run_mx(dev, qa, sa, qb, sb, cfg, 2, workspace=small)
    assert e.value.status == _lib.GA_ERR_WORKSPACE


def test_rejects_bad_shapes(dev):
    l = _lib.lib()
    args = _lib.F4gemmKargs()
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    l.ga_fill_args(ctypes.byref(args), buf.data_ptr(), None, buf.data_ptr(), buf.data_ptr(),
                   buf.data_ptr(), buf.data_ptr(), 64, 64, 200, 64, 8, 8, 1.0, 0.0, 0)
    st = l.ga_kernel_launch(0, ctypes.byref(args), 1, 1, 1, None, 0, None)
    assert st == _lib.GA_ERR_SHAPE  # K % 128


def test_one_call_mxfp8_gemm_from_float(dev):
    """ga_mxfp8_gemm over operands prepared on the GPU (quantiser + shuffles)."""
    from gcnasm_amd import ops
    M, N, K = 192, 768, 1024
    xa = oracle.gen_mx_input(M, K, 42, 1.0, 4)
    xb = oracle.gen_mx_input(N, K, 43, 1.0, 4)
    a = ops.prepare_mx_a(torch.from_numpy(xa).to(dev))
    b = ops.prepare_mx_b(torch.from_numpy(xb).to(dev))
    D, idx, ld = ops.mxfp8_gemm(a, b)
    torch.cuda.synchronize()
    qa, sa = oracle.quant_mxfp8(xa)
    qb, sb = oracle.quant_mxfp8(xb)
    got = D[:M].view(torch.int16).cpu().numpy().view(np.uint16)
    check(got, expect(qa, sa, qb, sb, ld.log2_k_split), "one-call",
          oracle.mx_absdot(qa, sa, qb, sb))


# Small-M streaming path of the 256x256 kernels: every M row tile count
# (M = 1, 16, 17, 33, 64), odd 16-column group counts (N = 784 -> 49 groups),
# K not a multiple of 256, and each split factor the path handles in-kernel.
@pytest.mark.parametrize("M", [1, 16, 17, 33, 64])
@pytest.mark.parametrize("NKL", [(784, 1152, 0), (784, 1152, 1), (4096, 2048, 0),
                                 (4096, 2048, 1), (4096, 2048, 2), (4096, 2048, 3),
                                 (1808, 3072, 2)])
def test_decode_path(dev, M, NKL):
    N, K, l2 = NKL
    name = "ga_mxfp8_bf16_BpreShuffle_256x256" + ("_splitK" if l2 else "")
    cfg = cfg_named(name)
    qa, sa, qb, sb = mx_operands(M, N, K, seed=100 + M + l2, std_b=0.02)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    check(got, expect(qa, sa, qb, sb, l2), "decode path M=%d N=%d K=%d gdz=%d" %
          (M, N, K, ld.gdz), oracle.mx_absdot(qa, sa, qb, sb))


# 1-16 rows with a split: one wave runs all K slices of its column task in
# turn, one fp32 chain per slice, the slices summed in order. Every N has
# one group per wave at 1 row and two at 16 (N = 16384 / 28672: 4-7 groups
# per workgroup; N = 784 and 4096: 1-2); K = 1152 at l2 = 2 is 3 slices
# (512, 512, 128), the last one step.
@pytest.mark.parametrize("M", [1, 12, 16])
@pytest.mark.parametrize("NKL", [(16384, 2048, 1), (16384, 2048, 3), (16384, 1152, 2),
                                 (28672, 1024, 2), (784, 1152, 2), (4096, 3072, 3),
                                 (4096, 1152, 2)])
def test_decode_sequential_slices(dev, M, NKL):
    N, K, l2 = NKL
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_128x512_splitK")
    qa, sa, qb, sb = mx_operands(M, N, K, seed=300 + M + l2, std_b=0.02)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    check(got, expect(qa, sa, qb, sb, l2), "decode sequential slices M=%d N=%d K=%d gdz=%d" %
          (M, N, K, ld.gdz), oracle.mx_absdot(qa, sa, qb, sb))


# 9-16 rows with at least four 16-column groups per CU and K <= 8192: the
# workgroup's A panel (16 rows x K) is copied into LDS once and the waves read
# their A fragments there. K = 8192 fills the 128 KB panel; K = 1152 is 9
# steps; N = 20480 gives five groups per CU; N = 16384 + 64 gives 4 or 5
# groups per CU on five waves, so most workgroups hold a wave without columns
# (it takes its share of the copies and the barrier); M = 9 leaves 7 rows of
# the panel zero.
@pytest.mark.parametrize("M", [9, 12, 16])
@pytest.mark.parametrize("NKL", [(16384, 8192, 0), (20480, 1152, 0), (20480, 1152, 1),
                                 (16384 + 64, 2048, 2), (28672, 8192, 3)])
def test_decode_a_panel_in_lds(dev, M, NKL):
    N, K, l2 = NKL
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_128x512" + ("_splitK" if l2 else ""))
    qa, sa, qb, sb = mx_operands(M, N, K, seed=400 + M + l2, std_b=0.02)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    check(got, expect(qa, sa, qb, sb, l2), "decode A panel in LDS M=%d N=%d K=%d gdz=%d" %
          (M, N, K, ld.gdz), oracle.mx_absdot(qa, sa, qb, sb))


@pytest.mark.parametrize("MNK", [(40, 8192, 8192), (64, 8192, 8192), (64, 16384, 1024),
                                 (48, 4096, 2048), (24, 8192, 8192)])
def test_decode_64_rows_paths(dev, MNK):
    """17-64 rows in the decode kernel: more steps in flight with one two-group
    task per CU and long K (N = 8192, K = 8192), eight waves of two groups
    (N = 16384), one group per wave (N = 4096)."""
    M, N, K = MNK
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_256x128_splitK")
    qa, sa, qb, sb = mx_operands(M, N, K, seed=M + N, std_b=0.02)
    got, _ = run_mx(dev, qa, sa, qb, sb, cfg, 0)
    check(got, expect(qa, sa, qb, sb, 0), "decode 64-row path M=%d N=%d K=%d" % (M, N, K),
          oracle.mx_absdot(qa, sa, qb, sb))


@pytest.mark.parametrize("M", [33, 64])
@pytest.mark.parametrize("name", ["ga_mxfp8_bf16_BpreShuffle_256x128_splitK",
                                  "ga_mxfp8_bf16_BpreShuffle_32x512_splitK"])
def test_few_rows_wide_n(dev, M, name):
    """33-64 rows over N wide enough for 32x256 B-streaming tiles on 3/4 of
    the CUs (the path ga_kernel_launch takes there instead of the decode
    kernel), N not a multiple of 256."""
    N, K = 28672 - 16, 512
    cfg = cfg_named(name)
    qa, sa, qb, sb = mx_operands(M, N, K, seed=M + 3, std_b=0.02)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, 0)
    assert ld.gdz == 1
    check(got, expect(qa, sa, qb, sb, 0), "few rows wide N M=%d %s" % (M, name),
          oracle.mx_absdot(qa, sa, qb, sb))


@pytest.mark.parametrize("M", [1, 40])
def test_decode_path_plain_b_and_epilogue(dev, M):
    """Row-major B and alpha/beta through the small-M path."""
    N, K = 512, 1024
    cfg = cfg_named("ga_mxfp8_bf16_noBpreShuffle_256x256")
    qa, sa, qb, sb = mx_operands(M, N, K, seed=7 + M)
    rng = np.random.default_rng(M)
    c_in = oracle.to_bf16_bits(rng.standard_normal((M, N)).astype(np.float32))
    got, _ = run_mx(dev, qa, sa, qb, sb, cfg, 0, alpha=0.5, beta=2.0, c_in=c_in)
    acc = oracle.gemm_mx_mfma(qa, sa, qb, sb, 0, 1.0)
    want_f = (np.float32(0.5) * acc).astype(np.float32) + np.float32(2.0) * \
        oracle.bf16_bits_to_f32(c_in)
    check(got, oracle.to_bf16_bits(want_f.astype(np.float32)), "decode plain-B alpha/beta M=%d" % M,
          0.5 * oracle.mx_absdot(qa, sa, qb, sb))


@pytest.mark.parametrize("name", PP_KERNELS)
def test_persistent_many_tiles(dev, name):
    """More 256x256 tiles (17 x 16 = 272) than the persistent grid has
    workgroups (one per CU, 256 on MI355X), so workgroups compute a second
    tile after the first (LDS reuse, staged epilogue, split-K partials of a
    later tile); every output checked."""
    M, N, K = 4352, 4096, 256
    cfg = cfg_named(name)
    l2 = 1 if cfg.splitK else 0
    qa, sa, qb, sb = mx_operands(M, N, K, seed=4352)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    check(got, expect(qa, sa, qb, sb, l2), "persistent %s gdz=%d" % (name, ld.gdz),
          oracle.mx_absdot(qa, sa, qb, sb))


@pytest.mark.parametrize("MNKL", [(64, 8192, 28672, 1), (64, 8192, 32768, 2),
                                  (24, 8192, 16384, 1)])
def test_decode_deep_k_split(dev, MNKL):
    """The decode kernel's four-steps-in-flight variant with K split across
    the waves of a workgroup (2 or 4 slices of at least 64 steps each), for
    the 33-64-row and 17-32-row instantiations."""
    M, N, K, l2 = MNKL
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_256x128_splitK")
    qa, sa, qb, sb = mx_operands(M, N, K, seed=M + l2, std_b=0.02)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    assert ld.gdz == 1 << l2
    check(got, expect(qa, sa, qb, sb, l2), "decode deep M=%d N=%d K=%d gdz=%d" %
          (M, N, K, ld.gdz), oracle.mx_absdot(qa, sa, qb, sb))


# (N, K, log2 split) -> 16-column groups per wave on 256 CUs, slices: every
# groups-per-wave instantiation, ragged last waves, whole rounds of waves.
SPLIT_DECODE_SHAPES = [
    (1040, 4096, 2),        # 65 groups x 4 slices: 2 groups, last wave holds one
    (8192 + 48, 2048, 3),   # 515 groups x 8: 6 groups, three rounds
    (4096, 1152, 1),        # 2 groups; second slice shorter (768 + 384)
    (8192, 2048, 1),        # 4 groups
    (8192, 2048, 2),        # 8 groups
    (19216, 512, 0),        # one slice, 1201 groups: 5 per wave, last holds one
    (22400, 512, 0),        # one slice: 6 groups
    (28672 - 16, 512, 0),   # one slice: 7 groups, last wave holds six
    (28672 - 16, 1024, 1),  # 2 slices x 1791 groups: 7 groups, two rounds
    (19216, 2048, 2),       # 4 slices x 1201 groups: 5 groups, four rounds
    (22400, 1152, 1),       # 2 slices of 768 + 384: 6 groups
    (28672 - 16, 2048, 3),  # 8 slices: 8 groups, seven rounds
]


@pytest.mark.parametrize("M", [20, 40, 64])
@pytest.mark.parametrize("bps", [True, False])
@pytest.mark.parametrize("NKL", SPLIT_DECODE_SHAPES)
def test_decode_split_across_workgroups(dev, M, bps, NKL):
    """17-64 rows with each wave over several 16-column groups and one K
    slice, the slices in separate workgroups: partials summed by the split-K
    reduce in slice order, or with one slice the epilogue in the kernel;
    preshuffled and row-major B."""
    N, K, l2 = NKL
    name = ("ga_mxfp8_bf16_BpreShuffle_256x256_splitK" if bps else
            "ga_mxfp8_bf16_noBpreShuffle_128x128_splitK")
    cfg = cfg_named(name)
    qa, sa, qb, sb = mx_operands(M, N, K, seed=3 * M + l2, std_b=0.02)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2)
    assert ld.gdz == 1 << l2
    check(got, expect(qa, sa, qb, sb, l2), "decode split %s M=%d N=%d K=%d gdz=%d" %
          ("bps" if bps else "plain", M, N, K, ld.gdz), oracle.mx_absdot(qa, sa, qb, sb))


# 33-64 rows at one slice over wide N: the shared-A variant (A through an LDS
# ring). (M, N, K, preshuffled B): eight waves of one group (shares of 6, 5
# and 7 groups: waves without a group) with the ring (6 steps) longer than the
# slice (5 steps), 33 rows; 9 steps (one pass of the main loop and a three-step
# tail); 7 groups per workgroup as at N = 28672; four waves of 4 groups (N >
# 32768: the five-step ring without paired scale loads) over 13 steps (two
# passes, a three-step tail) and 9, with one workgroup of 9 groups among 8s.
SHARED_A_CASES = [(33, 24576, 640, True), (33, 24576, 640, False), (40, 20480, 1152, True),
                  (64, 28672, 1152, True), (64, 32784, 1664, True), (64, 32784, 1152, False)]


@pytest.mark.parametrize("MNKB", SHARED_A_CASES)
def test_decode_shared_a(dev, MNKB):
    M, N, K, bps = MNKB
    name = ("ga_mxfp8_bf16_BpreShuffle_256x256" if bps else
            "ga_mxfp8_bf16_noBpreShuffle_256x256")
    cfg = cfg_named(name)
    qa, sa, qb, sb = mx_operands(M, N, K, seed=5 * M + K, std_b=0.02)
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, 0)
    assert ld.gdz == 1
    check(got, expect(qa, sa, qb, sb, 0), "decode shared-A %s M=%d N=%d K=%d" %
          ("bps" if bps else "plain", M, N, K), oracle.mx_absdot(qa, sa, qb, sb))


def test_decode_split_epilogue(dev):
    """alpha/beta through the split variant (applied by the split-K reduce)."""
    M, N, K, l2 = 40, 512, 2048, 2
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_256x256_splitK")
    qa, sa, qb, sb = mx_operands(M, N, K, seed=41)
    rng = np.random.default_rng(41)
    c_in = oracle.to_bf16_bits(rng.standard_normal((M, N)).astype(np.float32))
    got, ld = run_mx(dev, qa, sa, qb, sb, cfg, l2, alpha=0.5, beta=2.0, c_in=c_in)
    assert ld.gdz == 4
    acc = oracle.gemm_mx_mfma(qa, sa, qb, sb, l2, 1.0)
    want_f = (np.float32(0.5) * acc).astype(np.float32) + np.float32(2.0) * \
        oracle.bf16_bits_to_f32(c_in)
    check(got, oracle.to_bf16_bits(want_f.astype(np.float32)), "decode split alpha/beta",
          0.5 * oracle.mx_absdot(qa, sa, qb, sb))


def _mx_device_problem(dev, M, N, K, cfg, l2, seed):
    qa, sa, qb, sb = mx_operands(M, N, K, seed=seed)
    sh = f4gemm.Shape(M, N, K)
    a_pad = np.zeros((sh.a_rows_pad(), K), dtype=np.uint8)
    a_pad[:M] = qa
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    A, B = t(a_pad), t(f4gemm.shuffle_weight_16x16(qb, N, K))
    SA = t(f4gemm.shuffle_scale(sa, M, K // 32, sh.scale_a_rows(), sh.scale_cols()))
    SB = t(f4gemm.shuffle_scale(sb, N, K // 32, sh.scale_b_rows(), sh.scale_cols()))
    D = torch.full((sh.d_rows_pad(), N), float("nan"), dtype=torch.bfloat16, device=dev)
    ld = f4gemm.make_launch(cfg, M, N, K, l2)
    args = f4gemm.fill_args(D, None, A, B, SA, SB, M, N, K, N, sh.scale_cols(), sh.scale_cols(),
                            1.0, 0.0, ld.log2_k_split)
    keep = (A, B, SA, SB)
    return (qa, sa, qb, sb), D, ld, args, keep


@pytest.mark.parametrize("name,M", [("ga_mxfp8_bf16_BpreShuffle_256x256_splitK", 256),
                                    ("ga_mxfp8_bf16_BpreShuffle_128x128_splitK", 256),
                                    ("ga_mxfp8_bf16_BpreShuffle_64x256_splitK", 256),
                                    ("ga_mxfp8_bf16_BpreShuffle_256x256_splitK", 48)])
def test_ws_handle_graph_replay_survives_grow(dev, name, M):
    """ga_kernel_launch_ws_handle: a split-K GEMM captured into a HIP graph
    with its workspace found through a device slot keeps giving the eager
    result after the slot's buffer is grown (and moved) between replays; a
    slot never reserved is refused on the host. M = 48 runs the decode
    kernel's split variant (slices in separate workgroups)."""
    from gcnasm_amd import flatmm_splitk as fs
    N, K, l2 = 1024, 4096, 2
    cfg = cfg_named(name)
    (qa, sa, qb, sb), D, ld, args, keep = _mx_device_problem(dev, M, N, K, cfg, l2, 21)
    assert ld.gdz == 4
    kern = f4gemm.Kernel().load(None, cfg)
    need = kern.workspace_bytes(ld, M, N)
    h = fs.WorkspaceHandle()
    try:
        with pytest.raises(GaError) as e:
            kern.launch(args, ld.gdx, ld.gdy, ld.gdz, ws_handle=h)
        assert e.value.status == _lib.GA_ERR_WORKSPACE
        h.reserve(need)
        kern.launch(args, ld.gdx, ld.gdy, ld.gdz, ws_handle=h)
        torch.cuda.synchronize()
        eager = D[:M].view(torch.int16).cpu().numpy().view(np.uint16).copy()
        check(eager, expect(qa, sa, qb, sb, l2), "ws handle eager %s M=%d" % (name, M),
              oracle.mx_absdot(qa, sa, qb, sb))
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            kern.launch(args, ld.gdx, ld.gdy, ld.gdz, stream=s, ws_handle=h)
        ptr0 = h.query()[0]
        for rep in range(6):
            if rep == 3:
                h.reserve(3 * need)  # grows and moves the workspace
                assert h.query()[0] != ptr0
            D.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = D[:M].view(torch.int16).cpu().numpy().view(np.uint16)
            np.testing.assert_array_equal(got, eager, err_msg="replay %d" % rep)
            kern.launch(args, ld.gdx, ld.gdy, ld.gdz, ws_handle=h)  # eager work between
            torch.cuda.synchronize()
        del g
    finally:
        h.close()
    del keep


def test_library_workspace_refused_under_capture(dev):
    """A split-K launch with no caller workspace uses the library's own buffer,
    which a later call may reallocate: refused while the stream captures."""
    M, N, K, l2 = 256, 1024, 4096, 2
    cfg = cfg_named("ga_mxfp8_bf16_BpreShuffle_256x256_splitK")
    _, D, ld, args, keep = _mx_device_problem(dev, M, N, K, cfg, l2, 22)
    kern = f4gemm.Kernel().load(None, cfg)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with pytest.raises(GaError) as e:
        with torch.cuda.graph(g, stream=s):
            kern.launch(args, ld.gdx, ld.gdy, ld.gdz, stream=s)
    assert e.value.status == _lib.GA_ERR_WORKSPACE
    torch.cuda.synchronize()
    del g, keep

"""GPU parity of the fp32-scale FP8 GEMMs (opus kargs ABI) against the CPU oracle.

Block-scale (DeepSeek 1x128 activation / 128x128 weight, and the 1x128x1
per-column variant) and per-tensor. Expected values: the oracle's kernel-order
fp32 accumulation with the FP8 MFMA's own 128-K step sum, in the K slices the
library reports for the call (oracle.gemm_blockscale_mfma /
gemm_per_tensor_mfma with opus_gemm.k_slices); fp32 outputs are also checked
against the reference's own gemm_ref semantics
(per-product fp32 sum, opus_gemm/block_scale_gemm/..._host.cc:66-90) with the
reference's absolute tolerance scaled to the output magnitude.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from gcnasm_amd import opus_gemm, ops
from helpers import assert_parity, bf16_compare, f32_compare, mx_operands, tile_rows

pytestmark = pytest.mark.gpu


def ds_operands(M, N, K, seed, group_n=128, batch=1):
    xa = oracle.randn(batch * M * K, seed).reshape(batch, M, K)
    xb = oracle.randn(batch * N * K, seed + 1).reshape(batch, N, K)
    qa = np.empty((batch, M, K), np.uint8)
    qb = np.empty((batch, N, K), np.uint8)
    sfa = []
    sfb = []
    for b in range(batch):
        qa[b], s = oracle.quant_fp8_1x128(xa[b])
        sfa.append(s)
        if group_n == 128:
            qb[b], s = oracle.quant_fp8_128x128(xb[b])
        else:  # per-column scales over 128-K groups: [K/128, N]
            qb[b], s = oracle.quant_fp8_1x128(xb[b])
        sfb.append(s)
    return qa, qb, np.stack(sfa), np.stack(sfb)


def expect_bs(qa, qb, sfa, sfb, group_n, M_full=None, batch=1):
    """fp32 result of the kernel the library picks for [M_full, N, K] (rows of
    qa may be a subset of those)."""
    M = qa.shape[0] if M_full is None else M_full
    N, K = qb.shape
    gps = opus_gemm.k_slices(M, N, K, batch)
    return oracle.gemm_blockscale_mfma(qa, qb, sfa, sfb, group_n, gps)


def expect_pt(qa, qb, sa, sb, M_full=None):
    M = qa.shape[0] if M_full is None else M_full
    N, K = qb.shape
    return oracle.gemm_per_tensor_mfma(qa, qb, sa, sb, opus_gemm.k_slices(M, N, K))


def run_bs(dev, qa, qb, sfa, sfb, out_dtype, group_n):
    batch, M, K = qa.shape
    N = qb.shape[1]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    C = torch.full((batch, M, N), float("nan"), dtype=out_dtype, device=dev)
    opus_gemm.blockscale_gemm(t(qa), t(qb), t(sfa), t(sfb), C, group_n)
    torch.cuda.synchronize()
    return C


@pytest.mark.parametrize("group_n", [128, 1])
@pytest.mark.parametrize("shape", [(256, 512, 256), (384, 2112, 1024), (96, 1000, 512),
                                   (33, 7168, 512), (1, 256, 384), (520, 784, 1152),
                                   (65, 300, 640),
                                   # up to 64 rows: the B-streaming kernel (K slices,
                                   # ragged N, one or two column groups per wave) ...
                                   (16, 1000, 2048), (64, 7168, 1024), (8, 3000, 1536),
                                   (1, 8200, 4096),
                                   # ... or the 64x256 tile when it has enough tiles
                                   (40, 16640, 256),
                                   # more rows: the 128x128 tile while its tiles fit on
                                   # the CUs in one round (all the shapes above with
                                   # M > 64), the 256x256 kernel here
                                   (1024, 7168, 256)])
def test_blockscale(dev, group_n, shape):
    M, N, K = shape
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=M + N, group_n=group_n)
    want = expect_bs(qa[0], qb[0], sfa[0], sfb[0], group_n)
    C = run_bs(dev, qa, qb, sfa, sfb, torch.float32, group_n)
    got = C[0].cpu().numpy()
    absdot = oracle.blockscale_absdot(qa[0], qb[0], sfa[0], sfb[0], group_n)
    ok, st = f32_compare(got, want, absdot=absdot)
    assert_parity(st, "bs f32 %s g%d" % (shape, group_n))
    # reference gemm_ref semantics (per-product fp32 sums): the reference's own
    # check is |diff| <= 1e-3 on its U[0,1) x U[-.5,.5) data; on N(0,1) data the
    # same check scaled to the output magnitude
    ref = oracle.gemm_blockscale_ref(qa[0], qb[0], sfa[0], sfb[0], group_n)
    assert np.max(np.abs(got - ref)) <= 2e-4 * max(1.0, float(np.max(np.abs(ref))))
    Cb = run_bs(dev, qa, qb, sfa, sfb, torch.bfloat16, group_n)
    gb = Cb[0].view(torch.int16).cpu().numpy().view(np.uint16)
    ok, st = bf16_compare(gb, oracle.to_bf16_bits(want), absdot)
    assert_parity(st, "bs bf16 %s g%d" % (shape, group_n))


def check_rows_fp32_bf16(dev, shape, group_n, seed):
    """Runs a whole GEMM on the GPU (fp32 and bf16 C) and checks the first and
    last 8 rows and one row of every 256-row tile against the oracle (the CPU
    oracle on every row would take minutes)."""
    M, N, K = shape
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=seed, group_n=group_n)
    rows = np.unique(np.concatenate([np.arange(8), np.arange(M - 8, M), tile_rows(M)]))
    qa_r = np.ascontiguousarray(qa[0][rows])
    sfa_r = np.ascontiguousarray(sfa[0][:, rows])
    want = expect_bs(qa_r, qb[0], sfa_r, sfb[0], group_n, M_full=M)
    absdot = oracle.blockscale_absdot(qa_r, qb[0], sfa_r, sfb[0], group_n)
    C = run_bs(dev, qa, qb, sfa, sfb, torch.float32, group_n)
    ok, st = f32_compare(C[0].cpu().numpy()[rows], want, absdot=absdot)
    assert_parity(st, "bs f32 %s g%d" % (shape, group_n))
    del C
    Cb = run_bs(dev, qa, qb, sfa, sfb, torch.bfloat16, group_n)
    gb = Cb[0].view(torch.int16).cpu().numpy().view(np.uint16)[rows]
    ok, st = bf16_compare(gb, oracle.to_bf16_bits(want), absdot)
    assert_parity(st, "bs bf16 %s g%d" % (shape, group_n))


@pytest.mark.parametrize("shape", [(4096, 7168, 2048), (4096, 2112, 7168), (4096, 24576, 1536)])
def test_blockscale_deepseek_configs(dev, shape):
    """The DeepSeek shapes the benchmark configuration names (4096x24576x1536
    with fp32 C passes the non-temporal store limit below)."""
    check_rows_fp32_bf16(dev, shape, 128, 17)


@pytest.mark.parametrize("group_n", [128, 1])
def test_blockscale_nontemporal_stores(dev, group_n):
    """C, A and B together above 320 MiB: the 256x256 kernel writes its staged
    C rows with non-temporal stores, bf16 C as well as fp32 (16384 x 12288:
    384 MiB of bf16 C, 768 MiB of fp32)."""
    check_rows_fp32_bf16(dev, (16384, 12288, 512), group_n, 23)


def _rows_checked(M):
    return np.unique(np.concatenate([np.arange(4), np.arange(M - 4, M), tile_rows(M)]))


@pytest.mark.parametrize("group_n", [128, 1])
@pytest.mark.parametrize("shape,ldc_pad", [((4100, 4100, 256), 0), ((4100, 4100, 384), 12),
                                           ((2304, 7680, 512), 0), ((2304, 7680, 128), 0),
                                           ((4100, 4098, 256), 2)])
def test_blockscale_more_tiles_than_cus(dev, group_n, shape, ldc_pad):
    """More 256x256 tiles than CUs (more than one round of workgroups), K of
    one to four 128-K groups, ragged last tiles in M and N, a row stride above
    N whose padding must stay untouched and no write past row M, fp32 and bf16
    C, N % 4 != 0 included. Checked on the first and last rows and one row of
    every 256-row tile, against the oracle."""
    M, N, K = shape
    ldc = N + ldc_pad
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=M + N + K, group_n=group_n)
    rows = _rows_checked(M)
    qa_r = np.ascontiguousarray(qa[0][rows])
    sfa_r = np.ascontiguousarray(sfa[0][:, rows])
    want = expect_bs(qa_r, qb[0], sfa_r, sfb[0], group_n, M_full=M)
    absdot = oracle.blockscale_absdot(qa_r, qb[0], sfa_r, sfb[0], group_n)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    A, B, SA, SB = t(qa), t(qb), t(sfa), t(sfb)
    for dt in (torch.float32, torch.bfloat16):
        # one spare row past M: nothing may be written there either
        Cbuf = torch.full((M + 1, ldc), float("nan"), dtype=dt, device=dev)
        ka = opus_gemm.make_kargs(A, B, Cbuf, SA, SB, M, N, K, 1, group_n)
        ka.stride_c = ldc
        ka.stride_c_batch = M * ldc
        print("bs %s ldc=%d group_n=%d %s" % (shape, ldc, group_n, dt), flush=True)
        opus_gemm.gemm_a8w8_blockscale(ka, opus_gemm._out_dtype(Cbuf), group_n)
        torch.cuda.synchronize()
        if dt == torch.float32:
            full = Cbuf.cpu().numpy()
            ok, st = f32_compare(full[:M, :N][rows], want, absdot=absdot)
            pad = full[:, N:]
            tail = full[M]
        else:
            full = Cbuf.view(torch.int16).cpu().numpy().view(np.uint16)
            ok, st = bf16_compare(full[:M, :N][rows], oracle.to_bf16_bits(want), absdot)
            pad = oracle.bf16_bits_to_f32(full[:, N:])
            tail = oracle.bf16_bits_to_f32(full[M])
        assert_parity(st, "bs %s ldc=%d g%d %s" % (shape, ldc, group_n, dt))
        assert np.all(np.isnan(pad)), "row padding written"
        assert np.all(np.isnan(tail)), "row past M written"


def test_blockscale_batched_more_tiles_than_cus(dev):
    """Batched launch with more tiles per batch entry than CUs (2 x 289
    tiles)."""
    M, N, K, batch = 4100, 4100, 256, 2
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=41, batch=batch)
    C = run_bs(dev, qa, qb, sfa, sfb, torch.float32, 128)
    rows = _rows_checked(M)
    for b in range(batch):
        qa_r = np.ascontiguousarray(qa[b][rows])
        sfa_r = np.ascontiguousarray(sfa[b][:, rows])
        want = expect_bs(qa_r, qb[b], sfa_r, sfb[b], 128, M_full=M, batch=batch)
        absdot = oracle.blockscale_absdot(qa_r, qb[b], sfa_r, sfb[b], 128)
        ok, st = f32_compare(C[b].cpu().numpy()[rows], want, absdot=absdot)
        assert_parity(st, "batched, more tiles than CUs %d" % b)


@pytest.mark.parametrize("shape", [(4100, 4100, 512), (2304, 7680, 256)])
def test_per_tensor_more_tiles_than_cus(dev, shape):
    """Per-tensor with more tiles than CUs (one fp32 chain, scale in the
    epilogue), ragged tiles, fp32 and bf16 C, rows checked as above."""
    M, N, K = shape
    xa = oracle.randn(M * K, 31).reshape(M, K)
    xb = oracle.randn(N * K, 32).reshape(N, K)
    qa, sa = oracle.quant_fp8_per_tensor(xa)
    qb, sb = oracle.quant_fp8_per_tensor(xb)
    rows = _rows_checked(M)
    want = expect_pt(np.ascontiguousarray(qa[rows]), qb, sa[0], sb[0], M_full=M)
    absdot = oracle.fp8_absdot(np.ascontiguousarray(qa[rows]), qb) * float(sa[0]) * float(sb[0])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    for dt in (torch.float32, torch.bfloat16):
        C = torch.full((M, N), float("nan"), dtype=dt, device=dev)
        opus_gemm.per_tensor_gemm(t(qa), t(qb), t(sa), t(sb), C)
        torch.cuda.synchronize()
        if dt == torch.float32:
            ok, st = f32_compare(C.cpu().numpy()[rows], want, absdot=absdot)
        else:
            ok, st = bf16_compare(C.view(torch.int16).cpu().numpy().view(np.uint16)[rows],
                                  oracle.to_bf16_bits(want), absdot)
        assert_parity(st, "per-tensor, more tiles than CUs %s %s" % (shape, dt))


def expect_bs_stream_k(qa, qb, sfa, sfb, group_n, rows, M):
    """Oracle for ga_gemm_a8w8_blockscale_ws on rows `rows` of [M, N, K]:
    each 256x256 tile with its own stream-K K pieces (opus_gemm.stream_k_cuts
    of the library's plan), or the whole-tile kernel's slices without one."""
    N, K = qb.shape
    P = opus_gemm.stream_k_workgroups(M, N, K)
    if P == 0:
        return expect_bs(qa[rows], qb, sfa[:, rows], sfb, group_n, M_full=M), 0
    cuts = opus_gemm.stream_k_cuts(M, N, K, P)
    out = np.empty((len(rows), N), np.float32)
    for tn in range((N + 255) // 256):
        cols = slice(256 * tn, min(N, 256 * tn + 256))
        qb_t = np.ascontiguousarray(qb[cols])
        sfb_t = np.ascontiguousarray(sfb[2 * tn:2 * tn + 2] if group_n == 128 else sfb[:, cols])
        for tm in sorted(set(int(r) // 256 for r in rows)):
            sel = np.nonzero(np.asarray(rows) // 256 == tm)[0]
            r = np.asarray(rows)[sel]
            out[sel, cols] = oracle.gemm_blockscale_mfma(
                np.ascontiguousarray(qa[r]), qb_t, np.ascontiguousarray(sfa[:, r]), sfb_t,
                group_n, cuts=cuts[(tm, tn)])
    return out, P


def run_bs_ws(dev, qa, qb, sfa, sfb, out_dtype, group_n, ws):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    M, K = qa.shape
    N = qb.shape[0]
    C = torch.full((M, N), float("nan"), dtype=out_dtype, device=dev)
    opus_gemm.blockscale_gemm(t(qa), t(qb), t(sfa), t(sfb), C, group_n, workspace=ws)
    torch.cuda.synchronize()
    return C


@pytest.mark.parametrize("group_n", [128, 1])
@pytest.mark.parametrize("shape", [(2048, 2560, 8192), (2100, 2600, 6144), (2304, 2304, 6656),
                                   (1536, 4096, 8192)])
def test_blockscale_stream_k(dev, group_n, shape):
    """ga_gemm_a8w8_blockscale_ws: tile counts that fit the CUs badly run in
    stream-K form (every CU an equal share of the tiles' 128-K groups; a tile
    cut between CUs summed from fp32 partials in K order by the last one):
    long-K shapes whose tiles keep at most 40 % of the CUs busy, with three
    to five K pieces per tile, ragged edges, at least 16 K groups per CU, fp32 and bf16 C, each tile
    against the oracle with its own cuts; a second call gives the same bits
    (the tile counters were left at zero)."""
    M, N, K = shape
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=M + 3 * N + K, group_n=group_n)
    qa, qb, sfa, sfb = qa[0], qb[0], sfa[0], sfb[0]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    C0 = torch.empty((M, N), dtype=torch.float32, device=dev)
    ka = opus_gemm.make_kargs(t(qa[None]), t(qb[None]), C0, t(sfa[None]), t(sfb[None]),
                              M, N, K, 1, group_n)
    nbytes = opus_gemm.workspace_bytes(ka)
    ws = torch.zeros(max(nbytes, 4), dtype=torch.uint8, device=dev)
    rows = _rows_checked(M)
    want, P = expect_bs_stream_k(qa, qb, sfa, sfb, group_n, rows, M)
    assert P > 0 and nbytes > 0, "shape %s does not take the stream-K form" % (shape,)
    absdot = oracle.blockscale_absdot(np.ascontiguousarray(qa[rows]), qb,
                                      np.ascontiguousarray(sfa[:, rows]), sfb, group_n)
    for dt in (torch.float32, torch.bfloat16):
        print("stream-K %s group_n=%d %s P=%d" % (shape, group_n, dt, P), flush=True)
        C = run_bs_ws(dev, qa, qb, sfa, sfb, dt, group_n, ws)
        C2 = run_bs_ws(dev, qa, qb, sfa, sfb, dt, group_n, ws)
        whole = run_bs_ws(dev, qa, qb, sfa, sfb, dt, group_n, None)
        if dt == torch.float32:
            got = C.cpu().numpy()
            ok, st = f32_compare(got[rows], want, absdot=absdot)
            np.testing.assert_array_equal(C2.cpu().numpy().view(np.uint32), got.view(np.uint32))
            g64, w64 = got.astype(np.float64), whole.cpu().numpy().astype(np.float64)
        else:
            got = C.view(torch.int16).cpu().numpy().view(np.uint16)
            ok, st = bf16_compare(got[rows], oracle.to_bf16_bits(want), absdot)
            np.testing.assert_array_equal(C2.view(torch.int16).cpu().numpy(), got.view(np.int16))
            g64 = oracle.bf16_bits_to_f32(got).astype(np.float64)
            w64 = oracle.bf16_bits_to_f32(
                whole.view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.float64)
        assert_parity(st, "stream-K %s g%d %s" % (shape, group_n, dt))
        # every output against the whole-tile kernel's: the two differ only
        # in where a tile's K chain is cut (fp32 rounding of the pieces' sum,
        # far below 2^-14 of the row's largest output; a bf16 output may also
        # round to the neighbouring code), so a partial slot or quadrant
        # mixed up anywhere in a cut tile shows
        tol = 2.0 ** -14 * np.abs(w64).max(axis=1, keepdims=True)
        if dt == torch.bfloat16:
            tol = tol + np.abs(w64) * 2.0 ** -7
        far = np.abs(g64 - w64) > tol
        print("stream-K %s g%d %s against the whole-tile kernel: %d of %d outputs differ, "
              "%d beyond the bound" % (shape, group_n, dt, int((g64 != w64).sum()), g64.size,
                                       int(far.sum())), flush=True)
        assert not far.any()
    assert int(ws[:((M + 255) // 256) * ((N + 255) // 256) * 4].sum()) == 0, "counters not reset"


def test_blockscale_stream_k_reports_a_dirty_workspace(dev):
    """A workspace first used as an MX split-K workspace (fp32 partials where
    the tile counters live) and then given to a stream-K call without
    zero-filling it: the call's misuse is reported by
    ga_blockscale_workspace_check, which zero-fills the counters again, and
    the next stream-K call on it is right (the whole-tile kernel's result
    within the cut's fp32 rounding) and leaves it clean."""
    from gcnasm_amd import _lib, f4gemm
    from gcnasm_amd._lib import GaError
    M, N, K = 2048, 2560, 8192
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=91)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    ka = opus_gemm.make_kargs(t(qa[0][None]), t(qb[0][None]), C, t(sfa[0][None]),
                              t(sfb[0][None]), M, N, K, 1, 128)
    nbytes = opus_gemm.workspace_bytes(ka)
    assert nbytes > 0
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    # an MX split-K GEMM writes its fp32 partials from the workspace's start
    mM, mN, mK, l2 = 256, 1024, 4096, 2
    mqa, msa, mqb, msb = mx_operands(mM, mN, mK, seed=92)
    cfg = [c for c in f4gemm.manifest() if c.knl_name == "ga_mxfp8_bf16_BpreShuffle_256x256_splitK"][0]
    sh = f4gemm.Shape(mM, mN, mK)
    D = torch.empty((sh.d_rows_pad(), mN), dtype=torch.bfloat16, device=dev)
    a_pad = np.zeros((sh.a_rows_pad(), mK), dtype=np.uint8)
    a_pad[:mM] = mqa
    bufs = [t(a_pad), t(f4gemm.shuffle_weight_16x16(mqb, mN, mK)),
            t(f4gemm.shuffle_scale(msa, mM, mK // 32, sh.scale_a_rows(), sh.scale_cols())),
            t(f4gemm.shuffle_scale(msb, mN, mK // 32, sh.scale_b_rows(), sh.scale_cols()))]
    ld = f4gemm.make_launch(cfg, mM, mN, mK, l2)
    args = f4gemm.fill_args(D, None, *bufs, mM, mN, mK, mN, sh.scale_cols(), sh.scale_cols(),
                            1.0, 0.0, ld.log2_k_split)
    ws32 = ws.view(torch.float32)
    assert ld.gdz * mM * mN <= ws32.numel()
    f4gemm.Kernel().load(None, cfg).launch(args, ld.gdx, ld.gdy, ld.gdz, workspace=ws32)
    torch.cuda.synchronize()
    assert int((ws[:64] != 0).sum()) > 0, "the MX partials should leave the counters dirty"
    whole = run_bs_ws(dev, qa[0], qb[0], sfa[0], sfb[0], torch.float32, 128, None)
    opus_gemm.gemm_a8w8_blockscale(ka, _lib.GA_DTYPE_F32, 128, workspace=ws)
    with pytest.raises(GaError) as e:
        opus_gemm.workspace_check(ka, ws)
    assert e.value.status == _lib.GA_ERR_WORKSPACE
    print("dirty workspace reported: %s" % e.value, flush=True)
    C.fill_(float("nan"))
    opus_gemm.gemm_a8w8_blockscale(ka, _lib.GA_DTYPE_F32, 128, workspace=ws)
    opus_gemm.workspace_check(ka, ws)
    got = C.cpu().numpy().astype(np.float64)
    w64 = whole.cpu().numpy().astype(np.float64)
    tol = 2.0 ** -14 * np.abs(w64).max(axis=1, keepdims=True)
    assert not np.any(np.abs(got - w64) > tol)
    tiles = ((M + 255) // 256) * ((N + 255) // 256)
    assert int(ws[:(tiles + 1) * 4].sum()) == 0, "counters and misuse word left zero"


def test_blockscale_ws_whole_tiles_where_they_fit():
    """Tile counts that keep over 40 % of the CUs busy (the three DeepSeek
    configuration shapes: 144, 448 and 1536 tiles) keep the whole-tile
    kernel with or without a workspace: no stream-K plan, no workspace asked
    for."""
    for M, N, K in ((4096, 2112, 7168), (4096, 7168, 2048), (4096, 24576, 1536),
                    (8192, 8192, 8192), (4096, 1792, 6144)):
        assert opus_gemm.stream_k_workgroups(M, N, K) == 0, (M, N, K)


def test_blockscale_ws_without_workspace_and_short_workspace(dev):
    """ga_gemm_a8w8_blockscale_ws with no workspace is the plain call, bit for
    bit; a workspace short of ga_blockscale_workspace_bytes is an error."""
    M, N, K = 2048, 2560, 8192
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=77)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    A, B, SA, SB = t(qa), t(qb), t(sfa), t(sfb)
    C1 = torch.full((1, M, N), float("nan"), device=dev)
    C2 = torch.full((1, M, N), float("nan"), device=dev)
    opus_gemm.blockscale_gemm(A, B, SA, SB, C1, 128)
    ka = opus_gemm.make_kargs(A, B, C2, SA, SB, M, N, K, 1, 128)
    from gcnasm_amd import _lib
    _lib.check(_lib.lib().ga_gemm_a8w8_blockscale_ws(ctypes.byref(ka), 128, _lib.GA_DTYPE_F32,
                                                     None, 0, None))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(C2.cpu().numpy().view(np.uint32),
                                  C1.cpu().numpy().view(np.uint32))
    need = opus_gemm.workspace_bytes(ka)
    assert need > 0
    short = torch.zeros(need - 256, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="workspace"):
        opus_gemm.gemm_a8w8_blockscale(ka, _lib.GA_DTYPE_F32, 128, workspace=short)


def test_blockscale_batched(dev):
    M, N, K, batch = 128, 384, 512, 3
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=5, batch=batch)
    C = run_bs(dev, qa, qb, sfa, sfb, torch.float32, 128)
    for b in range(batch):
        want = expect_bs(qa[b], qb[b], sfa[b], sfb[b], 128, batch=batch)
        absdot = oracle.blockscale_absdot(qa[b], qb[b], sfa[b], sfb[b], 128)
        ok, st = f32_compare(C[b].cpu().numpy(), want, absdot=absdot)
        assert_parity(st, "batch %d" % b)


def test_blockscale_batched_small_m(dev):
    M, N, K, batch = 20, 700, 1024, 3
    qa, qb, sfa, sfb = ds_operands(M, N, K, seed=9, batch=batch)
    C = run_bs(dev, qa, qb, sfa, sfb, torch.float32, 128)
    for b in range(batch):
        want = expect_bs(qa[b], qb[b], sfa[b], sfb[b], 128, batch=batch)
        absdot = oracle.blockscale_absdot(qa[b], qb[b], sfa[b], sfb[b], 128)
        ok, st = f32_compare(C[b].cpu().numpy(), want, absdot=absdot)
        assert_parity(st, "batch %d" % b)


@pytest.mark.parametrize("shape", [(256, 256, 512), (200, 1040, 1024), (1, 512, 256),
                                   (600, 1000, 768), (16, 4000, 2048), (48, 600, 1024),
                                   (1024, 7168, 256)])
def test_per_tensor(dev, shape):
    M, N, K = shape
    xa = oracle.randn(M * K, 11).reshape(M, K)
    xb = oracle.randn(N * K, 12).reshape(N, K)
    qa, sa = oracle.quant_fp8_per_tensor(xa)
    qb, sb = oracle.quant_fp8_per_tensor(xb)
    want = expect_pt(qa, qb, sa[0], sb[0])
    absdot = oracle.fp8_absdot(qa, qb) * float(sa[0]) * float(sb[0])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    for dt in (torch.float32, torch.bfloat16):
        C = torch.full((M, N), float("nan"), dtype=dt, device=dev)
        opus_gemm.per_tensor_gemm(t(qa), t(qb), t(sa), t(sb), C)
        torch.cuda.synchronize()
        if dt == torch.float32:
            ok, st = f32_compare(C.cpu().numpy(), want, absdot=absdot)
        else:
            ok, st = bf16_compare(C.view(torch.int16).cpu().numpy().view(np.uint16),
                                  oracle.to_bf16_bits(want), absdot)
        assert_parity(st, "per-tensor %s %s" % (shape, dt))


def test_per_tensor_from_float_on_gpu(dev):
    """GPU per-tensor quantiser feeding the GEMM."""
    M, N, K = 128, 256, 512
    xa = oracle.randn(M * K, 21).reshape(M, K)
    xb = oracle.randn(N * K, 22).reshape(N, K)
    qa, sa = ops.quant_fp8_per_tensor(torch.from_numpy(xa).to(dev))
    qb, sb = ops.quant_fp8_per_tensor(torch.from_numpy(xb).to(dev))
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    opus_gemm.per_tensor_gemm(qa, qb, sa, sb, C)
    torch.cuda.synchronize()
    oa, osa = oracle.quant_fp8_per_tensor(xa)
    ob, osb = oracle.quant_fp8_per_tensor(xb)
    want = expect_pt(oa, ob, osa[0], osb[0])
    absdot = oracle.fp8_absdot(oa, ob) * float(osa[0]) * float(osb[0])
    ok, st = f32_compare(C.cpu().numpy(), want, absdot=absdot)
    assert_parity(st, "per-tensor from float")


def test_splitk_reduce(dev):
    split, M, N, batch, pM, pN = 3, 5, 1000, 2, 8, 1024
    rng = np.random.default_rng(3)
    ws = rng.standard_normal((split, batch, pM, pN)).astype(np.float32)
    bias = rng.standard_normal((N,)).astype(np.float32)
    want = np.empty((batch, M, N), dtype=np.float32)
    O = oracle.load()
    O.or_splitk_reduce(oracle.p(ws), oracle.p(want), split, M, N, batch, pM, pN,
                       oracle.p(bias), 0)
    out = torch.empty((batch, M, N), dtype=torch.float32, device=dev)
    ops.splitk_reduce(torch.from_numpy(ws).to(dev), out, split, M, N, batch, pM, pN,
                      bias=torch.from_numpy(bias).to(dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    outb = torch.empty((batch, M, N), dtype=torch.bfloat16, device=dev)
    ops.splitk_reduce(torch.from_numpy(ws).to(dev), outb, split, M, N, batch, pM, pN)
    torch.cuda.synchronize()
    O.or_splitk_reduce(oracle.p(ws), oracle.p(want), split, M, N, batch, pM, pN, None, 0)
    np.testing.assert_array_equal(outb.view(torch.int16).cpu().numpy().view(np.uint16),
                                  oracle.to_bf16_bits(want))


@pytest.mark.parametrize("dims", [(5, 3, 5000, 2, 8, 5008), (2, 70, 37, 1, 72, 40),
                                  (9, 1, 2048, 3, 1, 2048), (1, 300, 8, 1, 300, 8)])
def test_splitk_reduce_shapes(dev, dims):
    """Rows wider than one workgroup (several along N), rows packed several to
    a workgroup, N tails that are not a multiple of 8, one slice."""
    split, M, N, batch, pM, pN = dims
    rng = np.random.default_rng(split * 1000 + N)
    ws = rng.standard_normal((split, batch, pM, pN)).astype(np.float32)
    bias = rng.standard_normal((batch, N)).astype(np.float32)
    want = np.empty((batch, M, N), dtype=np.float32)
    O = oracle.load()
    O.or_splitk_reduce(oracle.p(ws), oracle.p(want), split, M, N, batch, pM, pN,
                       oracle.p(bias), N)
    out = torch.full((batch, M, N), float("nan"), dtype=torch.float32, device=dev)
    ops.splitk_reduce(torch.from_numpy(ws).to(dev), out, split, M, N, batch, pM, pN,
                      bias=torch.from_numpy(bias).to(dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))

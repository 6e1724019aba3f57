"""GPU parity of the bf16 split-K GEMM behind the opus flatmm split-K ABI, its
reduce, and the graph-safe workspace handle, against the CPU oracle.

  partials   ga_gemm_a16w16_flatmm_splitk writes ws[s, b, m, n] (fp32) for
             every slice of the reference's partition (pipeline .cuh:234-247);
             compared with oracle.a16w16_splitk_ws under the fp32 rule plus the
             MFMA bound; padding of the workspace is never written
  GEMM       ga_gemm_a16w16_splitk (split-K kernel + reduce, or the direct
             split_k == 1 path) against the oracle's reduce of its partials,
             bf16 rule plus the MFMA bound
  reference  the reference driver's own data and check (main.cc:93-118,
             366-391): M, N, K = 1024, 512, 7168, split_k 2, sampled outputs
             within 0.2 of a sequential fp32 sum
  slots      the one-call GEMM gives bit-identical C through a slot made by
             ga_ws_handle_create and through a caller-made {ptr, bytes} slot,
             launch after launch
  reduce     ga_splitk_reduce_ws_handle bit-exact against oracle.splitk_reduce
  handle     a captured HIP graph replays correctly after the workspace was
             grown and moved; a slot too small for the layout makes both
             kernels write nothing
"""
import numpy as np
import pytest
import torch

import oracle
from gcnasm_amd import flatmm_splitk as fs
from helpers import BF16_MFMA_BOUND, assert_parity, bf16_compare, f32_compare

pytestmark = pytest.mark.gpu


def bf16_bits(shape, seed):
    x = oracle.randn(int(np.prod(shape)), seed).reshape(shape)
    return oracle.to_bf16_bits(x)


def dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(dev).view(torch.bfloat16)


def host_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def caller_slot(ws, dev, nbytes=None):
    """A device slot {ptr, bytes} made the reference driver's way (main.cc:252-259)."""
    n = ws.numel() * 4 if nbytes is None else nbytes
    return torch.tensor([ws.data_ptr(), n], dtype=torch.int64, device=dev)


def slice_absdot(ab, bb, split_k):
    A = np.abs(oracle.bf16_bits_to_f32(ab).astype(np.float64))
    B = np.abs(oracle.bf16_bits_to_f32(bb).astype(np.float64))
    return np.stack([A[:, kb:ke] @ B[:, kb:ke].T
                     for kb, ke in oracle.a16w16_slices(ab.shape[1], split_k)])


SHAPES = [
    (1024, 512, 7168, 2),   # the reference driver's defaults (64x64 tiles)
    (100, 200, 1000, 3),    # K tail inside a 64-wide step, ragged M and N
    (64, 64, 640, 4),       # the last slice is empty
    (1, 1000, 4096, 8),     # one row
    (333, 257, 2048, 5),
    (256, 512, 1024, 1),
    (300, 40, 8, 1),        # K = 8
    (1024, 1024, 3000, 4),  # 128x128 tiles, K tail
    (2048, 1536, 1024, 2),  # 128x128 tiles
    (2048, 2048, 1000, 2),  # 128x256 tiles, K tail
    (520, 1000, 1024, 4),   # 64x128 tiles, ragged M and N
    # few rows (64-row tiles over mostly zero rows), wide N
    (16, 7168, 2048, 1),
    (48, 3000, 1000, 2),    # N % 16 == 8, K tail
    (8, 65536, 256, 2),     # 64x128 tiles
    (64, 8192, 512, 4),     # 64x128 tiles
    (33, 520, 4104, 3),     # 8-element K tail in the last slice
    (24, 16384, 512, 2),
    (40, 32768, 256, 2),
]


@pytest.mark.parametrize("shape", SHAPES)
def test_partials(dev, shape):
    M, N, K, split_k = shape
    print("a16w16 partials", shape, flush=True)
    ab, bb = bf16_bits((M, K), M + K), bf16_bits((N, K), N + K + 1)
    a, b = dev_bf16(ab, dev), dev_bf16(bb, dev)
    pm, pn = (M + 63) // 64 * 64, (N + 63) // 64 * 64
    ws = torch.full((split_k, pm, pn), float("nan"), dtype=torch.float32, device=dev)
    slot = caller_slot(ws, dev)
    ka = fs.make_kargs(a, b, None, split_k, None)
    ka.ws_handle = slot.data_ptr()
    fs.gemm_a16w16_flatmm_splitk(ka)
    torch.cuda.synchronize()
    got = ws.cpu().numpy()
    assert np.all(np.isnan(got[:, M:, :])) and np.all(np.isnan(got[:, :, N:]))
    want = oracle.a16w16_splitk_ws(ab, bb, split_k)
    absdot = slice_absdot(ab, bb, split_k)
    ok, st = f32_compare(got[:, :M, :N], want, absdot=absdot, bound=BF16_MFMA_BOUND)
    assert_parity(st, "  a16w16", cap_frac=1.0)


@pytest.mark.parametrize("shape", SHAPES[:6] + SHAPES[7:])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm(dev, shape, with_bias):
    M, N, K, split_k = shape
    print("a16w16 gemm", shape, with_bias, flush=True)
    ab, bb = bf16_bits((M, K), 7 * M + K), bf16_bits((N, K), 7 * N + K + 1)
    a, b = dev_bf16(ab, dev), dev_bf16(bb, dev)
    bias_bits = bf16_bits((N,), 99) if with_bias else None
    bias = dev_bf16(bias_bits, dev) if with_bias else None
    c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    with fs.WorkspaceHandle() as h:
        fs.splitk_gemm(a, b, c, split_k, h, bias=bias)
        torch.cuda.synchronize()
    ws = oracle.a16w16_splitk_ws(ab, bb, split_k)
    bias_f = oracle.bf16_bits_to_f32(bias_bits) if with_bias else None
    want = oracle.splitk_reduce(ws[:, None], bias_f)[0]
    absdot = slice_absdot(ab, bb, split_k).sum(0)
    ok, st = bf16_compare(host_bits(c), oracle.to_bf16_bits(want), absdot,
                          bound=BF16_MFMA_BOUND)
    assert_parity(st, "  a16w16", cap_frac=1.0)


def test_batched_strided_per_batch_bias(dev):
    batch, M, N, K, split_k = 3, 130, 384, 512, 2
    ab, bb = bf16_bits((batch, M, K + 8), 5), bf16_bits((batch, N, K), 6)
    a = dev_bf16(ab, dev)[:, :, :K]              # row stride K + 8
    b = dev_bf16(bb, dev)
    bias_bits = bf16_bits((batch, N), 7)
    bias = dev_bf16(bias_bits, dev)
    cbig = torch.full((batch, M, N + 16), float("nan"), dtype=torch.bfloat16, device=dev)
    c = cbig[:, :, :N]                           # row stride N + 16
    with fs.WorkspaceHandle() as h:
        fs.splitk_gemm(a, b, c, split_k, h, bias=bias, bias_per_batch=True)
        torch.cuda.synchronize()
    got = host_bits(cbig)
    assert np.all(np.isnan(oracle.bf16_bits_to_f32(got[:, :, N:])))
    for i in range(batch):
        ws = oracle.a16w16_splitk_ws(ab[i, :, :K], bb[i], split_k)
        want = oracle.splitk_reduce(ws[:, None], oracle.bf16_bits_to_f32(bias_bits[i]))[0]
        absdot = slice_absdot(np.ascontiguousarray(ab[i, :, :K]), bb[i], split_k).sum(0)
        ok, st = bf16_compare(got[i, :, :N], oracle.to_bf16_bits(want), absdot,
                              bound=BF16_MFMA_BOUND)
        assert st["bad"] == 0, (i, st)


def reference_driver_values(M, N, K):
    """fill_a / fill_b of main.cc:93-118 (rank 0), evaluated in fp32 like the C++."""
    f = np.float32
    row = np.arange(M, dtype=np.float32)[:, None]
    col = np.arange(N, dtype=np.float32)[:, None]
    ka = np.arange(K, dtype=np.float32)[None, :]
    a = (f(0.001) * f(1.0) + f(0.0002) * ((row % 17) - f(8))) + f(0.0001) * ((ka % 29) - f(14))
    b = f(0.0003) * ((col % 23) - f(11)) + f(0.0001) * ((ka % 31) - f(15))
    return oracle.to_bf16_bits(a.astype(np.float32)), oracle.to_bf16_bits(b.astype(np.float32))


def test_reference_driver_check(dev):
    M, N, K, split_k = 1024, 512, 7168, 2
    ab, bb = reference_driver_values(M, N, K)
    a, b = dev_bf16(ab, dev), dev_bf16(bb, dev)
    c = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
    with fs.WorkspaceHandle() as h:
        fs.splitk_gemm(a, b, c, split_k, h)
        torch.cuda.synchronize()
    got = oracle.bf16_bits_to_f32(host_bits(c))
    A, B = oracle.bf16_bits_to_f32(ab), oracle.bf16_bits_to_f32(bb)
    bad = 0
    for row in (0, 17, 255, 511, 1023):
        for col in (0, 127, 255, 511):
            # sample_ref: sequential fp32 sum, then bf16
            acc = np.add.accumulate((A[row] * B[col]).astype(np.float32), dtype=np.float32)[-1]
            ref = oracle.bf16_bits_to_f32(oracle.to_bf16_bits(np.float32(acc))).reshape(-1)[0]
            bad += abs(float(got[row, col]) - float(ref)) > 0.2
    assert bad == 0


@pytest.mark.parametrize("shape", [(1024, 512, 7168, 2), (100, 200, 1000, 3), (64, 64, 640, 4),
                                   (1024, 1024, 3000, 4), (333, 257, 2048, 5), (1, 4096, 4096, 8)])
def test_library_slot_equals_caller_slot(dev, shape):
    M, N, K, split_k = shape
    print("a16w16 slots", shape, flush=True)
    ab, bb = bf16_bits((M, K), 3 * M + K), bf16_bits((N, K), 3 * N + K + 1)
    a, b = dev_bf16(ab, dev), dev_bf16(bb, dev)
    bias = dev_bf16(bf16_bits((N,), 5), dev)
    # reference protocol: caller-made slot -> split-K kernel + reduce kernel
    c_ref = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    ka = fs.make_kargs(a, b, c_ref, split_k, None, bias)
    ws = torch.empty(fs.workspace_bytes(ka) // 4, dtype=torch.float32, device=dev)
    slot = caller_slot(ws, dev)
    ka.ws_handle = slot.data_ptr()
    fs.gemm_a16w16_splitk(ka)
    torch.cuda.synchronize()
    want = host_bits(c_ref)
    assert not np.any(np.isnan(oracle.bf16_bits_to_f32(want)))
    # the caller-slot result against the oracle (partials, then reduce with bias)
    ws_o = oracle.a16w16_splitk_ws(ab, bb, split_k)
    expect = oracle.splitk_reduce(ws_o[:, None], oracle.bf16_bits_to_f32(bf16_bits((N,), 5)))[0]
    ok, st = bf16_compare(want, oracle.to_bf16_bits(expect),
                          slice_absdot(ab, bb, split_k).sum(0), bound=BF16_MFMA_BOUND)
    assert_parity(st, "  a16w16 caller slot", cap_frac=1.0)
    # library slot, repeated launches: bit-identical to the caller slot
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    with fs.WorkspaceHandle() as h:
        kf = fs.make_kargs(a, b, c, split_k, h, bias)
        h.reserve(fs.workspace_bytes(kf))
        for rep in range(5):
            c.fill_(float("nan"))
            for _ in range(3):
                fs.gemm_a16w16_splitk(kf)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(host_bits(c), want, err_msg="launch %d" % rep)


def test_reduce_ws_handle_bit_exact(dev):
    split_k, batch, M, N = 3, 2, 70, 200
    pm, pn = 128, 256
    rng = np.random.default_rng(1)
    ws_h = rng.standard_normal((split_k, batch, pm, pn)).astype(np.float32)
    ws = torch.from_numpy(ws_h).to(dev)
    slot = caller_slot(ws, dev)
    bias_h = rng.standard_normal((batch, N)).astype(np.float32)
    bias = torch.from_numpy(bias_h).to(dev)

    class Slot:
        address = slot.data_ptr()

    c = torch.empty((batch, M, N), dtype=torch.float32, device=dev)
    fs.splitk_reduce_ws_handle(Slot, c, split_k, M, N, batch, pm, pn, bias, N)
    torch.cuda.synchronize()
    want = oracle.splitk_reduce(ws_h[:, :, :M, :N], bias_h, N)
    np.testing.assert_array_equal(c.cpu().numpy().view(np.uint32), want.view(np.uint32))
    cb = torch.empty((batch, M, N), dtype=torch.bfloat16, device=dev)
    fs.splitk_reduce_ws_handle(Slot, cb, split_k, M, N, batch, pm, pn)
    torch.cuda.synchronize()
    want = oracle.to_bf16_bits(oracle.splitk_reduce(ws_h[:, :, :M, :N]))
    np.testing.assert_array_equal(host_bits(cb), want)


def test_slot_too_small_writes_nothing(dev):
    M, N, K, split_k = 256, 256, 512, 2
    ab, bb = bf16_bits((M, K), 1), bf16_bits((N, K), 2)
    a, b = dev_bf16(ab, dev), dev_bf16(bb, dev)
    ws = torch.full((split_k, M, N), 7.0, dtype=torch.float32, device=dev)
    slot = caller_slot(ws, dev, nbytes=ws.numel() * 4 - 4)
    c = torch.full((M, N), 3.0, dtype=torch.bfloat16, device=dev)
    ka = fs.make_kargs(a, b, c, split_k, None)
    ka.ws_handle = slot.data_ptr()
    fs.gemm_a16w16_splitk(ka)
    torch.cuda.synchronize()
    assert torch.all(ws == 7.0).item() and torch.all(c == 3.0).item()


def test_graph_replay_survives_workspace_grow(dev):
    M, N, K, split_k = 512, 384, 2048, 4
    ab, bb = bf16_bits((M, K), 11), bf16_bits((N, K), 12)
    a, b = dev_bf16(ab, dev), dev_bf16(bb, dev)
    bias = dev_bf16(bf16_bits((N,), 13), dev)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    h = fs.WorkspaceHandle()
    try:
        ka = fs.make_kargs(a, b, c, split_k, h, bias)
        need = fs.workspace_bytes(ka)
        h.reserve(need)
        fs.gemm_a16w16_splitk(ka)                 # eager result
        torch.cuda.synchronize()
        eager = host_bits(c).copy()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            fs.gemm_a16w16_splitk(ka, stream=s)
        ptr0 = h.query()[0]
        for rep in range(6):
            if rep == 3:
                h.reserve(3 * need)               # grows and moves the workspace
                assert h.query()[0] != ptr0 and h.query()[1] == 3 * need
            c.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(host_bits(c), eager, err_msg="replay %d" % rep)
            # eager work on the same buffers between replays
            fs.gemm_a16w16_splitk(ka)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(host_bits(c), eager)
        del g
    finally:
        h.close()
    ws = oracle.a16w16_splitk_ws(ab, bb, split_k)
    want = oracle.splitk_reduce(ws[:, None], oracle.bf16_bits_to_f32(host_bits(bias)))[0]
    ok, st = bf16_compare(eager, oracle.to_bf16_bits(want), slice_absdot(ab, bb, split_k).sum(0),
                          bound=BF16_MFMA_BOUND)
    assert st["bad"] == 0


def test_handle_query_and_reserve(dev):
    h = fs.WorkspaceHandle()
    try:
        assert h.query() == (None, 0)
        h.reserve(1 << 20)
        p1, n1 = h.query()
        assert p1 and n1 == 1 << 20
        h.reserve(1000)                           # smaller: unchanged
        assert h.query() == (p1, n1)
        h.reserve((1 << 20) + 1)                  # larger: a new buffer
        p2, n2 = h.query()
        assert p2 != p1 and n2 == (1 << 20) + 1
    finally:
        h.close()
    assert h.address is None


def test_unreserved_slot_is_refused(dev):
    """A slot made by ga_ws_handle_create but never reserved (or reserved
    short of the layout) is refused on the host outside capture, for the
    partials-only kernel and for the GEMM + reduce."""
    from gcnasm_amd import _lib
    from gcnasm_amd._lib import GaError
    M, N, K, split_k = 128, 256, 1024, 2
    a = dev_bf16(bf16_bits((M, K), 31), dev)
    b = dev_bf16(bf16_bits((N, K), 32), dev)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    with fs.WorkspaceHandle() as h:
        ka = fs.make_kargs(a, b, c, split_k, h)
        for fn in (fs.gemm_a16w16_splitk, fs.gemm_a16w16_flatmm_splitk):
            with pytest.raises(GaError) as e:
                fn(ka)
            assert e.value.status == _lib.GA_ERR_WORKSPACE
        h.reserve(fs.workspace_bytes(ka) - 4)
        with pytest.raises(GaError) as e:
            fs.gemm_a16w16_splitk(ka)
        assert e.value.status == _lib.GA_ERR_WORKSPACE
        h.reserve(fs.workspace_bytes(ka))
        fs.gemm_a16w16_splitk(ka)
        torch.cuda.synchronize()

"""ga_kernel_launch_noalloc (split-K partials in the library's fixed device
scratch array, no allocation) against ga_kernel_launch (caller workspace) on
the same operands: bit-identical bf16 outputs, for two calls in a row, the
second smaller than the first, and a call whose partials exceed the scratch
is refused."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from gcnasm_amd import _lib, f4gemm
from helpers import mx_operands

pytestmark = pytest.mark.gpu


def _problem(dev, M, N, K, name, l2, seed):
    qa, sa, qb, sb = mx_operands(M, N, K, seed=seed)
    sh = f4gemm.Shape(M, N, K)
    a_pad = np.zeros((sh.a_rows_pad(), K), dtype=np.uint8)
    a_pad[:M] = qa
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    bufs = [t(a_pad), t(f4gemm.shuffle_weight_16x16(qb, N, K)),
            t(f4gemm.shuffle_scale(sa, M, K // 32, sh.scale_a_rows(), sh.scale_cols())),
            t(f4gemm.shuffle_scale(sb, N, K // 32, sh.scale_b_rows(), sh.scale_cols()))]
    cfg = [c for c in f4gemm.manifest() if c.knl_name == name][0]
    ld = f4gemm.make_launch(cfg, M, N, K, l2)
    outs = []
    for _ in range(2):
        D = torch.full((sh.d_rows_pad(), N), float("nan"), dtype=torch.bfloat16, device=dev)
        args = f4gemm.fill_args(D, None, bufs[0], bufs[1], bufs[2], bufs[3], M, N, K, N,
                                sh.scale_cols(), sh.scale_cols(), 1.0, 0.0, ld.log2_k_split)
        outs.append((D, args))
    idx = f4gemm.Kernel().load(None, cfg).idx
    return idx, ld, outs, bufs


def _bits(D, M):
    return D[:M].view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("name", ["ga_mxfp8_bf16_BpreShuffle_256x256_splitK",
                                  "ga_mxfp8_bf16_BpreShuffle_128x128_splitK",
                                  "ga_mxfp8_bf16_BpreShuffle_64x256_splitK"])
def test_noalloc_matches_workspace_launch(dev, name):
    lib = _lib.lib()
    # the 256x256 kernel also at 17-64 rows (the decode kernel's split variant)
    cases = [(512, 2048, 4096, 2, 1), (256, 1024, 2048, 1, 2)]
    if name.endswith("256x256_splitK"):
        cases += [(64, 4096, 8192, 3, 4), (40, 2064, 4096, 2, 5), (64, 28672, 1024, 1, 6)]
    for (M, N, K, l2, seed) in cases:
        idx, ld, outs, bufs = _problem(dev, M, N, K, name, l2, seed)
        assert ld.gdz == 1 << l2
        (D0, a0), (D1, a1) = outs
        ws = torch.empty(ld.gdz * M * N, dtype=torch.float32, device=dev)
        print("noalloc %s M=%d N=%d K=%d gdz=%d" % (name, M, N, K, ld.gdz), flush=True)
        _lib.check(lib.ga_kernel_launch(idx, ctypes.byref(a0), ld.gdx, ld.gdy, ld.gdz,
                                        ws.data_ptr(), ws.numel() * 4, None))
        _lib.check(lib.ga_kernel_launch_noalloc(idx, ctypes.byref(a1), ld.gdx, ld.gdy, ld.gdz,
                                                None))
        torch.cuda.synchronize()
        want = _bits(D0, M)
        got = _bits(D1, M)
        assert not np.any(np.isnan(oracle.bf16_bits_to_f32(got)))
        np.testing.assert_array_equal(got, want)
        del ws, outs, bufs


def test_noalloc_rejects_partials_beyond_the_scratch(dev):
    lib = _lib.lib()
    M, N, K, l2 = 2048, 4096, 1024, 1  # 2 * 2048 * 4096 * 4 = 64 MiB > 32 MiB
    name = "ga_mxfp8_bf16_BpreShuffle_256x256_splitK"
    idx, ld, outs, bufs = _problem(dev, M, N, K, name, l2, 3)
    st = lib.ga_kernel_launch_noalloc(idx, ctypes.byref(outs[0][1]), ld.gdx, ld.gdy, ld.gdz,
                                      None)
    assert st == _lib.GA_ERR_WORKSPACE
    torch.cuda.synchronize()


def test_noalloc_under_graph_capture(dev):
    """ga_kernel_launch_noalloc captured into a HIP graph (global capture
    mode, in which the library-owned workspace path is refused) and replayed:
    every replay gives the eager caller-workspace launch's bits, with other
    no-alloc calls (a smaller problem, which rewrites the scratch array)
    between the replays."""
    lib = _lib.lib()
    name = "ga_mxfp8_bf16_BpreShuffle_256x256_splitK"
    M, N, K, l2 = 256, 1024, 4096, 2
    idx, ld, outs, bufs = _problem(dev, M, N, K, name, l2, 7)
    (D0, a0), (D1, a1) = outs
    ws = torch.empty(ld.gdz * M * N, dtype=torch.float32, device=dev)
    _lib.check(lib.ga_kernel_launch(idx, ctypes.byref(a0), ld.gdx, ld.gdy, ld.gdz,
                                    ws.data_ptr(), ws.numel() * 4, None))
    # the eager no-alloc call first: the scratch array's address is looked up
    # outside capture
    _lib.check(lib.ga_kernel_launch_noalloc(idx, ctypes.byref(a1), ld.gdx, ld.gdy, ld.gdz, None))
    torch.cuda.synchronize()
    want = _bits(D0, M)
    np.testing.assert_array_equal(_bits(D1, M), want)
    sidx, sld, souts, sbufs = _problem(dev, 128, 512, 2048, name, 1, 8)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _lib.check(lib.ga_kernel_launch_noalloc(idx, ctypes.byref(a1), ld.gdx, ld.gdy, ld.gdz,
                                                ctypes.c_void_p(s.cuda_stream)))
    for rep in range(4):
        D1.fill_(float("nan"))
        torch.cuda.synchronize()
        print("noalloc graph replay %d" % rep, flush=True)
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(D1, M), want, err_msg="replay %d" % rep)
        _lib.check(lib.ga_kernel_launch_noalloc(sidx, ctypes.byref(souts[0][1]), sld.gdx, sld.gdy,
                                                sld.gdz, None))
        torch.cuda.synchronize()
    del g, ws, outs, bufs, souts, sbufs

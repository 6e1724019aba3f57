"""Host launch logic (CPU only): tile heuristic, split-K geometry, kernarg
filling, padded shapes and the manifest parser of libgcnasm_amd, checked
against the reference's own f4gemm.hpp / f4gemm_ref.hpp (compiled in place
into oracle/_ref) and against the oracle's restatement.

Shapes follow the reference's regression sweep (asm_f4gemm/run_tests.sh:37-57).
"""
import ctypes
import itertools

import numpy as np
import pytest

import oracle
from gcnasm_amd import _lib, f4gemm
from gcnasm_amd._lib import GaError

SWEEP = [(128, 1024, 1024), (256, 2048, 2048), (300, 2048, 1024), (1, 4096, 2048),
         (17, 512, 256), (512, 1024, 2048), (2048, 8192, 1024), (4096, 4096, 512),
         (16, 28672, 8192), (16, 8192, 28672), (64, 28672, 8192), (8192, 8192, 8192),
         (4096, 7168, 2048), (4096, 2112, 7168), (1, 256, 256), (257, 129, 768)]


def aiter_like_manifest():
    """A manifest shaped like aiter's 35-kernel MXFP4 list: many tiles, some
    splitK, the 128x512 quirk, one non-preshuffled tile."""
    tiles = [(32, 128), (32, 256), (32, 512), (64, 128), (64, 256), (64, 512), (96, 256),
             (96, 640), (128, 128), (128, 256), (128, 512), (160, 256), (192, 256),
             (224, 256), (256, 128), (256, 256)]
    cfgs = []
    for i, (m, n) in enumerate(tiles):
        cfgs.append(f4gemm.Config(m, n, i % 2, 1, "k%d" % i, "k%d.co" % i))
        cfgs.append(f4gemm.Config(m, n, 1, 1, "k%ds" % i, "k%ds.co" % i))
    cfgs.append(f4gemm.Config(256, 256, 0, 0, "noBps", "noBps.co"))
    return cfgs


def manifests():
    return [("compiled", f4gemm.manifest()), ("aiter_like", aiter_like_manifest())]


def ref_select(R, cfgs, M, N, K, num_cu, l2, bps):
    arr = lambda f: np.array([getattr(c, f) for c in cfgs], np.int32)  # noqa: E731
    tm, tn, sk, bp = arr("tile_M"), arr("tile_N"), arr("splitK"), arr("bpreshuffle")
    out = ctypes.c_int(0)
    idx = R.ref_select_kernel(M, N, K, num_cu, l2, bps, oracle.p(tm), oracle.p(tn), oracle.p(sk),
                              oracle.p(bp), len(cfgs), ctypes.byref(out))
    return idx, out.value


def oracle_select(cfgs, M, N, K, num_cu, l2, bps):
    arr = (ctypes.c_int * (4 * len(cfgs)))(
        *itertools.chain.from_iterable((c.tile_M, c.tile_N, c.splitK, c.bpreshuffle) for c in cfgs))
    out = ctypes.c_int(0)
    idx = oracle.load().or_select_kernel(M, N, K, num_cu, l2, bps, ctypes.cast(arr, ctypes.c_void_p),
                                         len(cfgs), ctypes.byref(out))
    return idx, out.value


@pytest.mark.parametrize("name,cfgs", manifests())
def test_select_kernel_vs_reference(R, name, cfgs):
    n = 0
    for (M, N, K), num_cu, l2, bps in itertools.product(SWEEP, (80, 256, 304), (-1, 0, 1, 2, 4),
                                                        (0, 1)):
        ours = f4gemm.select_kernel(M, N, K, num_cu, l2, bps, cfgs)
        ref = ref_select(R, cfgs, M, N, K, num_cu, l2, bps)
        assert ours == ref, (M, N, K, num_cu, l2, bps)
        assert oracle_select(cfgs, M, N, K, num_cu, l2, bps) == ref
        n += 1
    assert n > 400


def test_select_kernel_random_shapes(R):
    rng = np.random.default_rng(0)
    cfgs = aiter_like_manifest()
    for _ in range(2000):
        M, N = int(rng.integers(1, 20000)), int(rng.integers(1, 40000))
        K = int(rng.integers(1, 64)) * 256
        l2 = int(rng.integers(-1, 5))
        ours = f4gemm.select_kernel(M, N, K, 256, l2, 1, cfgs)
        assert ours == ref_select(R, cfgs, M, N, K, 256, l2, 1)


def test_select_kernel_none_fits():
    only_split = [f4gemm.Config(256, 256, 1, 1, "a", "a.co")]
    assert f4gemm.select_kernel(64, 64, 256, 256, 0, 0, only_split)[0] == -1
    l = _lib.lib()
    idx, l2 = ctypes.c_int(), ctypes.c_int()
    arr = (_lib.TileConfig * 1)(only_split[0].to_c())
    st = l.ga_select_kernel(64, 64, 256, 256, 0, 0, arr, 1, ctypes.byref(idx), ctypes.byref(l2))
    assert st == _lib.GA_ERR_NO_KERNEL and idx.value == -1


def test_make_launch_vs_reference(R):
    for (M, N, K), (tm, tn), sk, l2 in itertools.product(
            SWEEP, [(32, 256), (256, 256), (96, 640), (128, 512)], (0, 1), range(0, 5)):
        if K % (1 << l2):
            continue
        cfg = f4gemm.Config(tm, tn, sk, 1, "x", "x.co")
        d = f4gemm.make_launch(cfg, M, N, K, l2)
        out = np.zeros(5, np.int32)
        R.ref_make_launch(tm, tn, sk, 1, M, N, K, l2, oracle.p(out))
        assert [d.gdx, d.gdy, d.gdz, d.log2_k_split, int(d.zero_out)] == list(out)


def test_make_launch_splitk_error():
    cfg = f4gemm.Config(32, 256, 1, 1, "x", "x.co")
    with pytest.raises(GaError) as e:
        f4gemm.make_launch(cfg, 16, 256, 1000, 4)  # 1000 % 16 != 0
    assert e.value.status == _lib.GA_ERR_SPLITK
    d = oracle.load()
    gdx, gdy, gdz, z = (ctypes.c_int() for _ in range(4))
    c = (ctypes.c_int * 4)(32, 256, 1, 1)
    assert d.or_make_launch(ctypes.cast(c, ctypes.c_void_p), 16, 256, 1000, 4, ctypes.byref(gdx),
                            ctypes.byref(gdy), ctypes.byref(gdz), ctypes.byref(z)) == -1


def test_fill_args_bytes_vs_reference(R):
    assert R.ref_kernelargs_size() == ctypes.sizeof(_lib.F4gemmKargs) == 0x174
    ptrs = [0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000]
    ours = f4gemm.fill_args(*ptrs, 300, 2048, 1024, 2048, 32, 40, 0.5, 2.0, 3)
    ref = (ctypes.c_uint8 * 0x174)()
    R.ref_fill_args(ref, *[ctypes.c_void_p(p) for p in ptrs], 300, 2048, 1024, 2048, 32, 40, 0.5,
                    2.0, 3)
    assert bytes(ours) == bytes(ref)


def test_kernarg_offsets():
    K = _lib.F4gemmKargs
    want = dict(ptr_D=0x00, ptr_C=0x10, ptr_A=0x20, ptr_B=0x30, alpha=0x40, beta=0x50,
                stride_D0=0x60, stride_D1=0x70, stride_C0=0x80, stride_C1=0x90, stride_A0=0xA0,
                stride_A1=0xB0, stride_B0=0xC0, stride_B1=0xD0, M=0xE0, N=0xF0, K=0x100,
                ptr_ScaleA=0x110, ptr_ScaleB=0x120, stride_ScaleA0=0x130, stride_ScaleA1=0x140,
                stride_ScaleB0=0x150, stride_ScaleB1=0x160, log2_k_split=0x170)
    for f, off in want.items():
        assert getattr(K, f).offset == off, f
    O = _lib.OpusGemmKargs
    assert ctypes.sizeof(O) == 96
    assert (O.ptr_a.offset, O.ptr_b.offset, O.ptr_c.offset, O.m.offset) == (0, 8, 16, 24)
    assert (O.ptr_sfa.offset, O.ptr_sfb.offset, O.stride_sfa.offset,
            O.stride_sfb_batch.offset) == (64, 72, 80, 92)


def test_shape_vs_reference(R):
    for M, N, K in SWEEP:
        s = f4gemm.Shape(M, N, K, elem_bits=4)
        out = np.zeros(7, np.int32)
        R.ref_shape(M, N, K, oracle.p(out))
        assert [s.Kp(), s.Ks(), s.scale_cols(), s.a_rows_pad(), s.b_rows_pad(),
                s.scale_a_rows(), s.d_rows_pad()] == list(out)
        s8 = f4gemm.Shape(M, N, K)
        assert s8.Kp() == K and s8.scale_cols() == s.scale_cols()


CSV_CASES = {
    "plain": "tile_M,tile_N,splitK,bpreshuffle,knl_name,co_name\n"
             "256,256,0,1,kA,a.co\n32,512,1,1,kB,b.co\n",
    "reordered": "co_name, knl_name ,bpreshuffle,splitK,tile_N,tile_M\n"
                 "a.co,kA,1,0,256,256\n\n b.co , kB ,1,1,512,32\n",
    "ragged": "tile_M,tile_N,splitK,bpreshuffle,knl_name,co_name\n"
              "256,256,0,1,kA,a.co\n1,2,3\n32,512,1,1,kB,b.co,extra\n64,128,1,1,kC,c.co\n",
    "extra_col": "tile_M,tile_N,foo,splitK,bpreshuffle,knl_name,co_name\n"
                 "96,640,x,1,1,kD,d.co\n",
}


@pytest.mark.parametrize("case", list(CSV_CASES))
def test_load_configs_vs_reference(R, tmp_path, case):
    p = tmp_path / ("%s.csv" % case)
    p.write_text(CSV_CASES[case])
    ours = f4gemm.load_configs(p)
    cap = 16
    arrs = [np.zeros(cap, np.int32) for _ in range(4)]
    n = R.ref_load_configs(str(p).encode(), *[oracle.p(a) for a in arrs], cap)
    assert len(ours) == n
    assert [(c.tile_M, c.tile_N, c.splitK, c.bpreshuffle) for c in ours] == \
        [tuple(int(a[i]) for a in arrs) for i in range(n)]


def test_load_configs_errors(tmp_path):
    with pytest.raises(GaError) as e:
        f4gemm.load_configs(tmp_path / "missing.csv")
    assert e.value.status == _lib.GA_ERR_MANIFEST
    empty = tmp_path / "empty.csv"
    empty.write_text("")
    with pytest.raises(GaError) as e:
        f4gemm.load_configs(empty)
    assert e.value.status == _lib.GA_ERR_MANIFEST
    noname = tmp_path / "noname.csv"
    noname.write_text("tile_M,tile_N,splitK,bpreshuffle,knl_name,co_name\n32,256,0,1,,x.co\n")
    assert f4gemm.load_configs(noname) == []


def test_manifest_csv_round_trip(tmp_path):
    p = tmp_path / "m.csv"
    p.write_text(f4gemm.manifest_csv())
    assert f4gemm.load_configs(p) == f4gemm.manifest()
    names = [c.knl_name for c in f4gemm.manifest()]
    assert len(set(names)) == len(names)
    for c in f4gemm.manifest():
        assert f4gemm.Kernel().load(None, c).idx >= 0
    with pytest.raises(GaError):
        f4gemm.Kernel().load(None, f4gemm.Config(1, 1, 0, 0, "nope", "nope.co"))

"""GPU quantisers and device shuffles: bit-exact against the CPU oracle."""
import numpy as np
import pytest
import torch

import oracle
from gcnasm_amd import f4gemm, ops

pytestmark = pytest.mark.gpu


def edge_values():
    """Ties, subnormal boundaries, saturation, zeros of both signs, infinities
    (NaNs: test_quant_nan_blocks)."""
    vals = [0.0, -0.0, 448.0, -448.0, 464.0, 480.0, 1e30, -1e30, np.inf, -np.inf,
            2.0 ** -6, 2.0 ** -7, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -10, 1.0625, 1.1875,
            1.0 + 2.0 ** -4, 1.0 + 3 * 2.0 ** -4, 3.0e-45]
    # midpoints between consecutive E4M3 values (exact ties)
    t = oracle.e4m3_decode_table()
    pos = np.sort(t[np.isfinite(t) & (t > 0)])
    mids = (pos[:-1] + pos[1:]) / 2
    return np.concatenate([np.array(vals, dtype=np.float32), mids.astype(np.float32),
                           -mids.astype(np.float32)])


@pytest.mark.parametrize("rule", [0, 1, 2])
@pytest.mark.parametrize("in_bf16", [False, True])
def test_quant_mx(dev, rule, in_bf16):
    rows, K = 96, 1024
    x = oracle.gen_mx_input(rows, K, 100 + rule, 1.0, 6)
    e = edge_values()
    x.reshape(-1)[: e.size] = e
    if in_bf16:
        xb = oracle.to_bf16_bits(x)
        x = oracle.bf16_bits_to_f32(xb)
        xt = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xt = torch.from_numpy(x).to(dev)
    q, s = ops.quant_mxfp8(xt, rule)
    torch.cuda.synchronize()
    qo, so = oracle.quant_mxfp8(x, rule)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)


@pytest.mark.parametrize("in_bf16", [False, True])
def test_quant_1x128_128x128_per_tensor(dev, in_bf16):
    rows, K = 300, 1024
    x = oracle.randn(rows * K, 7).reshape(rows, K) * np.float32(3.0)
    x[5, :128] = 0.0  # an all-zero group
    x.reshape(-1)[1000:1000 + 40] = edge_values()[:40]
    x[np.isinf(x)] = 1000.0
    if in_bf16:
        xb = oracle.to_bf16_bits(x)
        x = oracle.bf16_bits_to_f32(xb)
        xt = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xt = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    q1, s1 = ops.quant_fp8_1x128(xt)
    q2, s2 = ops.quant_fp8_128x128(xt)
    q3, s3 = ops.quant_fp8_per_tensor(xt)
    torch.cuda.synchronize()
    o1, os1 = oracle.quant_fp8_1x128(x)
    o2, os2 = oracle.quant_fp8_128x128(x)
    o3, os3 = oracle.quant_fp8_per_tensor(x)
    np.testing.assert_array_equal(s1.cpu().numpy().view(np.uint32), os1.view(np.uint32))
    np.testing.assert_array_equal(q1.cpu().numpy(), o1)
    np.testing.assert_array_equal(s2.cpu().numpy().view(np.uint32), os2.view(np.uint32))
    np.testing.assert_array_equal(q2.cpu().numpy(), o2)
    np.testing.assert_array_equal(s3.cpu().numpy().view(np.uint32), os3.view(np.uint32))
    np.testing.assert_array_equal(q3.cpu().numpy(), o3)


@pytest.mark.parametrize("in_bf16", [False, True])
def test_quant_strided_rows_and_tails(dev, in_bf16):
    """Rows whose stride is a multiple of 4 but not 8 elements (bf16 takes the
    8-byte load path), a block count that leaves a partial last workgroup, and a
    per-tensor size with n % 4 != 0."""
    rows, K = 97, 1152
    base = oracle.gen_mx_input(rows, K + 4, 55, 1.0, 6)
    x = np.ascontiguousarray(base[:, :K])
    if in_bf16:
        bb = oracle.to_bf16_bits(base)
        x = oracle.bf16_bits_to_f32(np.ascontiguousarray(bb[:, :K]))
        xt = torch.from_numpy(bb.view(np.int16)).to(dev).view(torch.bfloat16)[:, :K]
    else:
        xt = torch.from_numpy(base).to(dev)[:, :K]
    assert xt.stride(0) == K + 4
    q, s = ops.quant_mxfp8(xt, 0)
    q4, s4 = ops.quant_mxfp4(xt, 2)
    q1, s1 = ops.quant_fp8_1x128(xt)
    q2, s2 = ops.quant_fp8_128x128(xt)
    torch.cuda.synchronize()
    qo, so = oracle.quant_mxfp8(x, 0)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    q4o, s4o = oracle.quant_mxfp4(x, 2)
    np.testing.assert_array_equal(s4.cpu().numpy(), s4o)
    np.testing.assert_array_equal(q4.cpu().numpy(), q4o)
    o1, os1 = oracle.quant_fp8_1x128(x)
    np.testing.assert_array_equal(s1.cpu().numpy().view(np.uint32), os1.view(np.uint32))
    np.testing.assert_array_equal(q1.cpu().numpy(), o1)
    o2, os2 = oracle.quant_fp8_128x128(x)
    np.testing.assert_array_equal(s2.cpu().numpy().view(np.uint32), os2.view(np.uint32))
    np.testing.assert_array_equal(q2.cpu().numpy(), o2)
    flat = x.reshape(-1)[:12345]
    ft = xt.contiguous().reshape(-1)[:12345]
    q3, s3 = ops.quant_fp8_per_tensor(ft)
    torch.cuda.synchronize()
    o3, os3 = oracle.quant_fp8_per_tensor(flat)
    np.testing.assert_array_equal(s3.cpu().numpy().view(np.uint32), os3.view(np.uint32))
    np.testing.assert_array_equal(q3.cpu().numpy(), o3)


def test_e4m3_encoder_every_bf16_value(dev):
    """Per-tensor quantisation with amax = 448 has scale 1, so q = e4m3(x): every
    bf16 bit pattern of magnitude <= 448 (and every NaN) goes through the
    device encoder and is compared with the oracle's."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = oracle.bf16_bits_to_f32(bits)
    keep = np.isnan(vals) | (np.abs(vals) <= 448.0)
    xb = bits[keep]
    xb = np.concatenate([xb, oracle.to_bf16_bits(np.array([448.0], np.float32))])
    x = oracle.bf16_bits_to_f32(xb)
    for t in (torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16),
              torch.from_numpy(np.ascontiguousarray(x)).to(dev)):
        q, s = ops.quant_fp8_per_tensor(t)
        torch.cuda.synchronize()
        assert s.cpu().numpy()[0] == np.float32(1.0)
        np.testing.assert_array_equal(q.cpu().numpy(), oracle.e4m3_encode(x))


@pytest.mark.parametrize("in_bf16", [False, True])
def test_quant_nan_blocks(dev, in_bf16):
    """Block maxima ignore NaNs (the CPU reference's `a > amax` scan): NaNs,
    quiet, signalling and negative, as the first or last element of a 1x32
    block, next to the block's largest value, filling a whole 1x32 / 1x128
    block, and in one 128x128 tile only, among blocks without NaNs in the same
    wave; every quantiser against the oracle, codes and scales."""
    rows, K = 256, 1024
    x = oracle.gen_mx_input(rows, K, 91, 1.0, 6)
    nans = np.array([0x7FC00000, 0x7F800001, 0xFFC00000, 0xFFBFFFFF], np.uint32).view(np.float32)
    x[0, 0] = nans[0]                  # first of its 1x32 block
    x[1, 31] = nans[1]                 # last of its block (signalling)
    x[2, 40] = nans[2]                 # negative
    x[2, 41] = 300.0                   # beside the block's maximum
    x[3, 64:96] = nans[3]              # a whole 1x32 block
    x[4, 128:256] = nans[0]            # a whole 1x128 block
    x[200, 900] = nans[1]              # one NaN in tile (1, 7)
    if in_bf16:
        xb = oracle.to_bf16_bits(x)
        x = oracle.bf16_bits_to_f32(xb)
        xt = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xt = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    assert np.isnan(x).sum() == 3 + 32 + 128 + 1
    for rule in (0, 1, 2):
        q, sc = ops.quant_mxfp8(xt, rule)
        q4, s4 = ops.quant_mxfp4(xt, rule)
        torch.cuda.synchronize()
        qo, so = oracle.quant_mxfp8(x, rule)
        np.testing.assert_array_equal(sc.cpu().numpy(), so)
        np.testing.assert_array_equal(q.cpu().numpy(), qo)
        q4o, s4o = oracle.quant_mxfp4(x, rule)
        np.testing.assert_array_equal(s4.cpu().numpy(), s4o)
        np.testing.assert_array_equal(q4.cpu().numpy(), q4o)
    q1, s1 = ops.quant_fp8_1x128(xt)
    q2, s2 = ops.quant_fp8_128x128(xt)
    torch.cuda.synchronize()
    o1, os1 = oracle.quant_fp8_1x128(x)
    o2, os2 = oracle.quant_fp8_128x128(x)
    np.testing.assert_array_equal(s1.cpu().numpy().view(np.uint32), os1.view(np.uint32))
    np.testing.assert_array_equal(q1.cpu().numpy(), o1)
    np.testing.assert_array_equal(s2.cpu().numpy().view(np.uint32), os2.view(np.uint32))
    np.testing.assert_array_equal(q2.cpu().numpy(), o2)


@pytest.mark.parametrize("amax", [1000.5, 3.7e-5, 1.7 * 2.0 ** -50, 2.0 ** -60, 3.0e38])
def test_quant_division_every_bf16_value(dev, amax):
    """The 1x128, 128x128 and per-tensor quantisers divide by s = amax/448,
    which is not a power of two: blocks whose first element is the maximum
    and whose other elements run through every bf16 value of magnitude <=
    amax (both signs, zeros included), at scales on both sides of the 2^-64
    bound of the shared-reciprocal division (1.7 * 2^-50 / 448 above it,
    2^-60 / 448 below), checked bit for bit against the oracle's fp32 division
    for fp32 and bf16 input."""
    top = oracle.bf16_bits_to_f32(oracle.to_bf16_bits(np.array([amax], np.float32)))[0]
    allv = oracle.bf16_bits_to_f32(np.arange(0x7F80, dtype=np.uint32).astype(np.uint16))
    vals = allv[allv <= top]
    vals = np.concatenate([vals, -vals]).astype(np.float32)
    nblk = -(-len(vals) // 127)
    nblk = -(-nblk // 8) * 8  # whole rows of K = 1024
    body = np.zeros(nblk * 127, np.float32)
    body[:len(vals)] = vals
    x = np.concatenate([np.full((nblk, 1), top, np.float32), body.reshape(nblk, 127)], axis=1)
    x = np.ascontiguousarray(x.reshape(-1, 1024))
    xb = oracle.to_bf16_bits(x)
    assert np.array_equal(oracle.bf16_bits_to_f32(xb), x)
    o1, os1 = oracle.quant_fp8_1x128(x)
    o2, os2 = oracle.quant_fp8_128x128(x)
    o3, os3 = oracle.quant_fp8_per_tensor(x)
    for t in (torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16),
              torch.from_numpy(x).to(dev)):
        q1, s1 = ops.quant_fp8_1x128(t)
        q2, s2 = ops.quant_fp8_128x128(t)
        q3, s3 = ops.quant_fp8_per_tensor(t)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(s1.cpu().numpy().view(np.uint32), os1.view(np.uint32))
        np.testing.assert_array_equal(q1.cpu().numpy(), o1)
        np.testing.assert_array_equal(s2.cpu().numpy().view(np.uint32), os2.view(np.uint32))
        np.testing.assert_array_equal(q2.cpu().numpy(), o2)
        np.testing.assert_array_equal(s3.cpu().numpy().view(np.uint32), os3.view(np.uint32))
        np.testing.assert_array_equal(q3.cpu().numpy(), o3)


@pytest.mark.parametrize("NK", [(16, 32), (256, 512), (272, 4096)])
def test_device_shuffle_weight(dev, NK):
    N, Kp = NK
    rng = np.random.default_rng(N + Kp)
    w = rng.integers(0, 256, size=(N, Kp), dtype=np.uint8)
    got = ops.shuffle_weight_16x16(torch.from_numpy(w).to(dev)).cpu().numpy().reshape(-1)
    np.testing.assert_array_equal(got, oracle.shuffle_weight_16x16(w, N, Kp))


@pytest.mark.parametrize("shape", [(1, 8, 256, 8), (300, 32, 512, 32), (17, 5, 32, 8)])
def test_device_shuffle_scale(dev, shape):
    rows, cols, sm, sn = shape
    rng = np.random.default_rng(rows)
    s = rng.integers(100, 140, size=(rows, cols), dtype=np.uint8)
    got = ops.shuffle_scale(torch.from_numpy(s).to(dev), sm, sn).cpu().numpy()
    np.testing.assert_array_equal(got, oracle.shuffle_scale(s, rows, cols, sm, sn))


def test_prepare_matches_host_path(dev):
    """prepare_mx_b on the GPU == oracle quantiser + host shuffles."""
    N, K = 256, 768
    x = oracle.gen_mx_input(N, K, 5, 0.02, 4)
    b = ops.prepare_mx_b(torch.from_numpy(x).to(dev))
    q, s = oracle.quant_mxfp8(x)
    sh = f4gemm.Shape(1, N, K)
    np.testing.assert_array_equal(b.codes.cpu().numpy().reshape(-1),
                                  oracle.shuffle_weight_16x16(q, N, K))
    np.testing.assert_array_equal(b.scales.cpu().numpy(),
                                  oracle.shuffle_scale(s, N, K // 32, sh.scale_b_rows(),
                                                       sh.scale_cols()))


@pytest.mark.parametrize("rule", [0, 1, 2])
@pytest.mark.parametrize("in_bf16", [False, True])
def test_quant_mx8_e5m2(dev, rule, in_bf16):
    """MX 1x32 with E5M2 elements (ga_quant_mx8 fmt 1) byte for byte against
    the oracle, codes and scales, fp32 and bf16 inputs, a partial 16-byte tail
    of rows; fmt 0 equals the E4M3 quantiser."""
    rows, K = 77, 1056
    x = oracle.gen_mx_input(rows, K, 55 + rule, 1.0, 6)
    x[0, :32] = 0.0
    x[1, 5] = np.nan
    x[2, :32] = 57344.0
    if in_bf16:
        xb = oracle.to_bf16_bits(x)
        t = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
        x = oracle.bf16_bits_to_f32(xb)
    else:
        t = torch.from_numpy(x).to(dev)
    q, s = ops.quant_mx8(t, 1, rule)
    q8, s8 = ops.quant_mx8(t, 0, rule)
    q0, s0 = ops.quant_mxfp8(t, rule)
    torch.cuda.synchronize()
    qo, so = oracle.quant_mx8(x, 1, rule)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    np.testing.assert_array_equal(q8.cpu().numpy(), q0.cpu().numpy())
    np.testing.assert_array_equal(s8.cpu().numpy(), s0.cpu().numpy())


def test_e5m2_encoder_every_bf16_value(dev):
    """Every bf16 bit pattern of magnitude <= 57344 (and every NaN) through the
    device E5M2 encoder at scale 1: each 32-block holds 57344 first, so the
    floor rule gives exponent 0, then 31 of the test values."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = oracle.bf16_bits_to_f32(bits)
    keep = np.isnan(vals) | (np.abs(vals) <= 57344.0)
    v = vals[keep]
    per = 31
    nblk = (len(v) + per - 1) // per
    pad = np.zeros(nblk * per, np.float32)
    pad[:len(v)] = v
    blocks = np.concatenate([np.full((nblk, 1), 57344.0, np.float32), pad.reshape(nblk, per)],
                            axis=1)
    rows = (nblk + 31) // 32
    x = np.zeros((rows * 32, 32), np.float32)
    x[:nblk] = blocks
    x = x.reshape(rows, 32 * 32)
    xb = oracle.to_bf16_bits(x)
    assert np.array_equal(oracle.bf16_bits_to_f32(xb)[np.isfinite(x)], x[np.isfinite(x)])
    t = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    q, s = ops.quant_mx8(t, 1, 0)
    torch.cuda.synchronize()
    xf = oracle.bf16_bits_to_f32(xb)
    sc = s.cpu().numpy()[:, :]
    assert np.all(sc.reshape(-1)[:nblk] == 127)
    np.testing.assert_array_equal(q.cpu().numpy(), oracle.quant_mx8(xf, 1, 0)[0])
    np.testing.assert_array_equal(q.cpu().numpy().reshape(-1, 32)[:nblk, 1:].reshape(-1)[:len(v)],
                                  oracle.e5m2_encode(v))

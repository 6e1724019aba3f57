"""Pins the oracle's quantisers (CPU only).

Each code is checked by brute force: it must decode (times the block scale) to
the E4M3 value nearest the input among all 254 finite codes, ties to the even
code, saturating at +-448. Scales are checked against the closed forms
(MX: the rule bracket of amax/2^e; DeepSeek/per-tensor: s = amax/448 in fp32,
an all-zero block gets s = 1) and the codes against torch's float8_e4m3fn
conversion of the same scaled values.
"""
import numpy as np
import pytest
import torch

import oracle


def nearest_codes(v):
    """Brute-force RNE-saturating E4M3 code of each float32 value in v."""
    t = oracle.e4m3_decode_table().astype(np.float64)
    codes = np.array([c for c in range(256) if np.isfinite(t[c]) and c != 0x80])  # +0 only
    vals = t[codes]
    v = np.clip(np.asarray(v, np.float64).ravel(), -448.0, 448.0)
    d = np.abs(v[:, None] - vals[None, :])
    best = d.min(1, keepdims=True)
    cand = d == best
    # ties: prefer the code with an even mantissa lsb
    pick = np.where(cand & ((codes[None, :] & 1) == 0), 1, 0) + cand
    out = codes[np.argmax(pick, axis=1)]
    # signed zero: the encoder keeps the sign of zero results
    neg0 = (t[out] == 0) & (np.signbit(np.asarray(v)))
    return np.where(neg0, 0x80, out).astype(np.uint8)


def mx_inputs(rows, K, seed):
    x = oracle.gen_mx_input(rows, K, seed, 1.0, 6)
    x[0, :32] = 0.0                     # all-zero block
    x[1, :32] = 448.0                   # block at the saturation edge
    x[2, 5] = 1e-30                     # tiny element
    x[3, :32] = np.linspace(-3, 3, 32)  # mixed signs incl. exact zero
    return x


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_mx_quant_brute_force(rule):
    x = mx_inputs(24, 256, 10 + rule)
    q, s = oracle.quant_mxfp8(x, rule)
    O = oracle.load()
    for r in range(x.shape[0]):
        for b in range(x.shape[1] // 32):
            blk = x[r, b * 32:(b + 1) * 32]
            e = O.or_mx_scale_exp(float(np.abs(blk).max()), rule)
            assert s[r, b] == e + 127
            scaled = (blk.astype(np.float64) * 2.0 ** -e).astype(np.float32)
            np.testing.assert_array_equal(q[r, b * 32:(b + 1) * 32], nearest_codes(scaled))


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_mx_quant_vs_torch(rule):
    x = mx_inputs(64, 512, 20 + rule)
    q, s = oracle.quant_mxfp8(x, rule)
    e = s.astype(np.int32) - 127
    scaled = (x.reshape(64, -1, 32).astype(np.float64) * np.exp2(-e)[..., None]).astype(np.float32)
    ref = torch.from_numpy(np.clip(scaled, -448, 448).reshape(64, 512)).to(torch.float8_e4m3fn)
    np.testing.assert_array_equal(q, ref.view(torch.uint8).numpy())


def test_mx_floor_rule_saturates_block_max():
    """The literal config rule e = floor(log2(amax/448)) puts amax/2^e in [448, 896),
    so the block maximum always encodes as +-448 (0x7E / 0xFE)."""
    x = mx_inputs(16, 256, 5)[4:]
    q, s = oracle.quant_mxfp8(x, 0)
    for r in range(x.shape[0]):
        for b in range(8):
            blk = x[r, b * 32:(b + 1) * 32]
            i = int(np.argmax(np.abs(blk)))
            assert q[r, b * 32 + i] & 0x7F == 0x7E


def test_planted_scale_mistake_is_caught():
    """A quantiser with an off-by-one scale exponent fails the brute-force check."""
    x = mx_inputs(4, 64, 3)
    q, s = oracle.quant_mxfp8(x, 0)
    e = s.astype(np.int32) - 127 + 1  # planted mistake
    scaled = (x.reshape(4, -1, 32).astype(np.float64) * np.exp2(-e)[..., None]).astype(np.float32)
    assert not np.array_equal(q, nearest_codes(scaled).reshape(q.shape))


def ds_inputs(rows, K, seed):
    x = (oracle.randn(rows * K, seed).reshape(rows, K) * 3).astype(np.float32)
    x[0, :128] = 0.0
    x[1, 7] = 1e-20
    return x


def test_quant_1x128():
    x = ds_inputs(40, 512, 1)
    q, sfa = oracle.quant_fp8_1x128(x)
    for r in range(40):
        for g in range(4):
            blk = x[r, g * 128:(g + 1) * 128]
            amax = np.float32(np.abs(blk).max())
            want = np.float32(amax / np.float32(448.0)) if amax > 0 else np.float32(1.0)
            assert sfa[g, r] == want
            np.testing.assert_array_equal(q[r, g * 128:(g + 1) * 128],
                                          nearest_codes((blk / want).astype(np.float32)))


def test_quant_128x128():
    x = ds_inputs(300, 256, 2)
    q, sfb = oracle.quant_fp8_128x128(x)
    assert sfb.shape == (3, 2)
    for rb in range(3):
        for g in range(2):
            tile = x[rb * 128:(rb + 1) * 128, g * 128:(g + 1) * 128]
            amax = np.float32(np.abs(tile).max())
            want = np.float32(amax / np.float32(448.0))
            assert sfb[rb, g] == want
            ref = torch.from_numpy(np.clip(tile / want, -448, 448)).to(torch.float8_e4m3fn)
            np.testing.assert_array_equal(q[rb * 128:(rb + 1) * 128, g * 128:(g + 1) * 128],
                                          ref.view(torch.uint8).numpy())


def test_quant_per_tensor():
    x = ds_inputs(33, 128, 3)
    q, s = oracle.quant_fp8_per_tensor(x)
    want = np.float32(np.float32(np.abs(x).max()) / np.float32(448.0))
    assert s[0] == want
    np.testing.assert_array_equal(q.ravel(), nearest_codes((x / want).astype(np.float32)))
    q0, s0 = oracle.quant_fp8_per_tensor(np.zeros((4, 4), np.float32))
    assert s0[0] == 1.0 and not q0.any()


def nearest_codes_e5m2(v):
    """Brute-force RNE-saturating E5M2 code of each float32 value in v."""
    t = oracle.e5m2_decode_table().astype(np.float64)
    codes = np.array([c for c in range(256) if np.isfinite(t[c]) and c != 0x80])
    vals = t[codes]
    v = np.clip(np.asarray(v, np.float64).ravel(), -57344.0, 57344.0)
    d = np.abs(v[:, None] - vals[None, :])
    best = d.min(1, keepdims=True)
    cand = d == best
    pick = np.where(cand & ((codes[None, :] & 1) == 0), 1, 0) + cand
    out = codes[np.argmax(pick, axis=1)]
    neg0 = (t[out] == 0) & (np.signbit(np.asarray(v)))
    return np.where(neg0, 0x80, out).astype(np.uint8)


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_mx_quant_e5m2_brute_force(rule):
    """MX 1x32 with E5M2 elements: scales by the E5M2 rule (format maximum
    57344), every code the brute-force nearest E5M2 value of x * 2^-e; the
    E4M3 format of the same quantiser equals quant_mxfp8."""
    x = mx_inputs(24, 256, 30 + rule)
    q, s = oracle.quant_mx8(x, 1, rule)
    O = oracle.load()
    for r in range(x.shape[0]):
        for b in range(x.shape[1] // 32):
            blk = x[r, b * 32:(b + 1) * 32]
            e = O.or_mx8_scale_exp(float(np.abs(blk).max()), rule, 1)
            assert s[r, b] == e + 127
            scaled = (blk.astype(np.float64) * 2.0 ** -e).astype(np.float32)
            np.testing.assert_array_equal(q[r, b * 32:(b + 1) * 32], nearest_codes_e5m2(scaled))
    q8, s8 = oracle.quant_mx8(x, 0, rule)
    q0, s0 = oracle.quant_mxfp8(x, rule)
    np.testing.assert_array_equal(q8, q0)
    np.testing.assert_array_equal(s8, s0)


def test_mx_e5m2_floor_rule_saturates_block_max():
    x = mx_inputs(16, 256, 7)[4:]
    q, s = oracle.quant_mx8(x, 1, 0)
    for r in range(x.shape[0]):
        for b in range(8):
            blk = x[r, b * 32:(b + 1) * 32]
            i = int(np.argmax(np.abs(blk)))
            assert q[r, b * 32 + i] & 0x7F == 0x7B


def test_shared_scale_division_is_exact(tmp_path):
    """The 1x128 / 128x128 / per-tensor quantisers divide by a block scale
    with a shared reciprocal and two FMA corrections (quant.hip, ScaleDiv):
    scale_div_check.c restates that arithmetic on the CPU and compares it with
    IEEE division for every bf16 value and random fp32 values under 300
    scales (~1.5e7 quotients)."""
    import os
    import subprocess
    src = os.path.join(os.path.dirname(__file__), "scale_div_check.c")
    exe = str(tmp_path / "scale_div_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
    out = subprocess.run([exe, "300"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout
    assert " 0 mismatches" in out.stdout

"""Writes tests/golden/mx_config1.npz: benchmark config 1 (MXFP8 M=256 N=256
K=512) inputs, the oracle's quantised codes/scales and its fp32-accumulated
output. Run from the repository root: python tests/golden/make_golden.py"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import numpy as np  # noqa: E402

import oracle  # noqa: E402

M, N, K = 256, 256, 512
xa = oracle.gen_mx_input(M, K, 1234, 1.0, 4)
xb = oracle.gen_mx_input(N, K, 5678, 1.0, 4)
qa, sa = oracle.quant_mxfp8(xa)
qb, sb = oracle.quant_mxfp8(xb)
d = oracle.gemm_mxfp8_fp32acc(qa, sa, qb, sb, 0)
np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)), "mx_config1.npz"),
                    xa=xa, xb=xb, qa=qa, sa=sa, qb=qb, sb=sb, d_fp32acc=d)
print("wrote mx_config1.npz")

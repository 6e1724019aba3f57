"""gcnasm_amd -- block-scaled FP8 GEMM library for MI355X (gfx950).

The product is libgcnasm_amd.so (C ABI in include/gcnasm_amd.h): hand-written
HIP kernels for the MXFP8/MXFP4, DeepSeek block-scale and per-tensor FP8
GEMMs, the bf16 split-K GEMM with its graph-safe workspace handle, the
quantisers and layout shuffles that feed them, and the host launch logic
(tile manifest, heuristic, split-K geometry, kernarg blocks).

Python modules:
  f4gemm     mirror of the reference's f4gemm host namespace (MXFP8 path)
  opus_gemm  mirror of the reference's opus_gemm drivers (fp32-scale paths)
  flatmm_splitk  mirror of the reference's a16w16 split-K driver, workspace
             handle and split-K reduce
  ops        tensor-level conveniences (torch tensors as device buffers)
"""
from ._lib import GaError, lib  # noqa: F401

__all__ = ["GaError", "lib"]

"""turbocider_amd -- MI355X (gfx950) GGUF Q4_K/Q6_K quantized-linear path.

* ``turbocider_amd.gguf``: K-quant type registry, device decode (decode_into / decode_gather),
  device quantizer.
* ``turbocider_amd.qlinear``: ``QuantizedLinear`` (fused dequant + bf16 MFMA GEMM, skinny
  GEMV for M <= 8, runtime LoRA and bias epilogue) and the ``Weights`` container.
* ``turbocider_amd.build``: compiles ``libtc_qlinear.so`` (the C ABI of include/tc_qlinear.h).
"""
from . import _lib  # noqa: F401

__all__ = ["gguf", "qlinear", "build"]

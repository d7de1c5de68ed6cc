"""MI355X (gfx950) int8-weight matrix product with telmo's operator surface.

The compute is the HIP library ``lib/libtelmo_hip.so`` behind the C ABI of
``include/telmo_hip.h``; this package mirrors the reference's Python-visible names over it.
"""
from .kernels import (Act, Epilogue, Kernels, PackedWeights, Precision, TdtDecoder, TelmoError, Token, decode, encode,
                      random)
from .pack import Pack

__all__ = ["Act", "Epilogue", "Kernels", "Pack", "PackedWeights", "Precision", "TdtDecoder", "TelmoError", "Token",
           "decode", "encode", "random"]

"""Apertura decode attention for MI355X (gfx950).

The compute path is libesda.so (hand-written HIP, C ABI in include/esda.h); this
package is its Python front end.  There is no CPU or PyTorch fallback: every entry
point raises if the library is missing or the device is not gfx950.
"""
from ._lib import EsdaError, lib, library_path  # noqa: F401
from .decode import DecodeStep, decode_step, workspace_bytes  # noqa: F401

__all__ = ["EsdaError", "lib", "library_path", "DecodeStep", "decode_step", "workspace_bytes"]

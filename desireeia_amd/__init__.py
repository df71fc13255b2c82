"""MI355X-native (gfx950) quantized-weight compute path of DesireeIA.

The product is libdesireeia_hip.so (C ABI: include/desireeia_hip.h). This
package holds its sources (csrc/), its build recipe (build.py), a ctypes
binding (_lib.py), a host-side mirror of the reference operators over torch
device tensors (ops.py) and seeded synthetic GGUF inputs (synth.py).
"""
from . import _lib  # noqa: F401

__all__ = ["ops", "synth", "build"]

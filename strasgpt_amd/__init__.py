"""StrasGPT transformer forward pass on AMD Instinct MI355X (gfx950).

The product is the C-ABI library strasgpt_amd/lib/libstrasgpt_hip.so
(include/transformer.h, include/transformer_hip.h, include/safetensors.h).
This package holds its sources (csrc/), a ctypes binding (runtime.py) and
the seeded synthetic model writer (synth.py).
"""
__all__ = ["runtime", "synth"]

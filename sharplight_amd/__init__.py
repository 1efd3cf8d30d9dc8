"""Sharplight HIP execution provider for MI355X (gfx950).

``native``   -- ctypes binding of libsharplight_hip (the C ABI in include/sharplight_hip.h).
``synth``    -- seeded synthetic inputs of the benchmark configurations.
``build``    -- builds libsharplight_hip.so in-tree with hipcc.
"""
__all__ = ["native", "synth"]

"""fortai_amd: MI355X-native (gfx950) backend for FortAI's device-resident
Qwen3.5 Q8_0 decode step.

The product is the C ABI in ``include/fortai_hip_backend.h`` implemented by
``fortai_amd/lib/libfortai_hip.so`` (hand-written HIP kernels for gfx950).
This Python package is host-side plumbing: a ctypes mirror of the ABI
(``backend``), a GGUF v3 reader/writer (``gguf``), the seeded synthetic model
generator (``synth``) and a host driver that mirrors the reference's Qwen3.5
model step (``qwen35``).
"""

__all__ = ["backend", "gguf", "synth", "qwen35", "build"]

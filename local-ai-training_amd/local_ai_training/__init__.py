"""MI355X-native ratchet-linear training path (host mirror of LoomNode/local-ai-training).

The compute lives in libratchet_hip.so (hand-written gfx950 HIP kernels behind the C ABI
of include/ratchet_hip.h); these modules keep the reference's Python surface.
"""

__version__ = "0.1.0"

"""arthip_amd: MI355X (gfx950) engine for ArtCNN-style conv-chain upscalers.

The compute lives in the native library libarthip.so (C ABI in
include/arthip.h); this package is the host-side mirror of the reference's
engine interface plus ONNX model tooling. See ``arthip_amd.engine.Engine``.
"""

__version__ = "0.1.0"

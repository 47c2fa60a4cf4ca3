"""soklyn_amd — MI355X-native (gfx950) DenseBlock hot path of Felix1G/soklyn.

The product is libsoklyn_hip.so (include/soklyn_hip.h): hand-written HIP
kernels for CDNA4 behind a C ABI that replaces the reference's device layer
(src/io/device/ffn_device.rs, util_device.rs).  `abi` is its ctypes binding;
`devblock` lays out one DenseBlock's device buffers for it; `build` compiles
it with hipcc for gfx950.
"""
from . import abi  # noqa: F401

__all__ = ["abi"]

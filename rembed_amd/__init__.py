"""rembed_amd — MI355X (gfx950) GEMM backend for rembed's encoder path.

The product is librembed_hip.so (C ABI in include/rembed_hip.h: hand-written
HIP kernels plus the C++ model runtime). This package is its Python binding:
`tensor` mirrors internal/tensor's GEMM family, `model` mirrors the encoder
API, `checkpoint` reads .safetensors weights for it, `synthetic` generates
the benchmark's random-init weights and tokens.
Importing `rembed_amd.tensor` or `rembed_amd.model` loads the library and
raises if it is not built: there is no CPU fallback.
"""
__all__ = ["tensor", "model", "checkpoint", "synthetic"]

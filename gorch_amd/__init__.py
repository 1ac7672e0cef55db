"""gorch_amd — MI355X (gfx950) backend for gorch's BF16-weight inference path.

- ``csrc/``: hand-written HIP kernels and the C-ABI (include/gorch_hip.h),
  built into ``libgorch_hip.so`` by ``gorch_amd.build``.
- ``hip``: the ctypes binding (the metal/metal.go analogue).
- ``bf16``: gorch's host bf16 codec (tensor.go:85-121) for preparing uploads.
- ``synthetic``: seeded synthetic weights/inputs at the benchmark shapes.
"""
from . import bf16  # noqa: F401

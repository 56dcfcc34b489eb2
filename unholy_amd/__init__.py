"""gfx950 quantized-MoE hot path: MXFP4 routed experts and the fp8 block-scaled dense GEMM.

The compute lives in libunholy_amd.so (hand-written HIP for gfx950 behind a C ABI, include/unholy_amd.h; the C++
drop-ins of the reference's src/kernels entry points are declared under include/unholy/kernels/). This package is
the host-side binding: `_lib` binds every C entry point from the header with ctypes (`call(name, *args)`),
`device` holds device buffers, streams, events and graphs, and `build` compiles the library in-tree.
"""
from ._lib import UhError, call, lib  # noqa: F401

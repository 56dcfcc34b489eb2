"""gfx950 quantized-MoE hot path: MXFP4 routed experts and the fp8 block-scaled dense GEMM.

The compute lives in libunholy_amd.so (hand-written HIP for gfx950 behind a C ABI, include/unholy_amd.h);
this package is the host-side binding: `kernels` mirrors the reference's src/kernels entry points one to one,
`device` holds device buffers and streams, `moe` composes the routed-expert FFN as the reference's model layer
does.
"""
from ._lib import UhError, call, lib  # noqa: F401

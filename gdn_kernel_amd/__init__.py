"""MI355X (gfx950) Gated DeltaNet decode and varlen chunked prefill.

Entry points (destination-passing, reference argument order):
  gdn_kernel_amd.decode.kernel          -- solution/cuda/kernel.cu::kernel
  gdn_kernel_amd.decode.kernel_pooled   -- decode over an indexed state pool
  gdn_kernel_amd.prefill.kernel         -- solution/cuda/kernel_prefill.cu::kernel
The compute runs in libgdn_kernel_amd.so (hand-written HIP for gfx950), reached
through the C ABI declared in include/gdn_kernel_amd.h.
"""
from .binding import GDNError, decode_kernel, decode_pooled_kernel, prefill_kernel  # noqa: F401

__version__ = "0.1.0"

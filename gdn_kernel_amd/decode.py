"""``kernel`` for the decode definition: the drop-in for the reference's
``solution/cuda/kernel.cu::kernel`` (DPS, 11 arguments, kernel.cu:101-113)."""
from .binding import decode_kernel as kernel, decode_pooled_kernel as kernel_pooled  # noqa: F401

__all__ = ["kernel", "kernel_pooled"]

"""``kernel`` for the prefill definition: the drop-in for the reference's
``solution/cuda/kernel_prefill.cu::kernel`` (DPS, 12 arguments,
kernel_prefill.cu:300-306)."""
from .binding import prefill_kernel as kernel  # noqa: F401

__all__ = ["kernel"]

"""Drop-in Python binding for the MI355X GDN kernels (destination-passing style).

Mirrors the reference's entry points argument for argument:

* ``decode_kernel(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state)``
  -- the TVM-FFI ``kernel`` of solution/cuda/kernel.cu:101-113,150 (also the
  Triton ``kernel`` of solution/triton/kernel.py:61).
* ``prefill_kernel(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale,
  output, new_state)`` -- the TVM-FFI ``kernel`` of
  solution/cuda/kernel_prefill.cu:300-306,339.
* ``decode_pooled_kernel(q, k, v, state_pool, A_log, a, dt_bias, b, scale,
  output, state_indices)`` -- no reference counterpart; decode over an indexed
  state pool, updated in place.
* ``prefill_kernel_with_workspace(..., new_state, workspace)`` -- no reference
  counterpart; ``prefill_kernel`` with a caller-owned workspace, which batches of
  few chains use to prepare each chunk once.

Semantics kept from the reference: outputs are preallocated and written in
place; ``scale`` None or 0 selects 1/sqrt(dk); ``state`` None means a zero
initial state; ``new_state`` may be the same tensor as ``state``; launches are
asynchronous on the current stream.  Unlike the reference (which checks
nothing), shapes, dtypes, devices and contiguity are validated and reported as
``ValueError``; device errors raise ``GDNError``.

Tensors travel to the C ABI as raw device pointers; torch is used only for
tensor metadata and the current HIP stream.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

__all__ = ["decode_kernel", "decode_pooled_kernel", "prefill_kernel", "prefill_kernel_with_workspace",
           "prefill_workspace_bytes", "prefill_giveups", "decode_pool_conflicts", "GDNError"]

GDNError = _lib.GDNError
_BF16 = torch.bfloat16
_F32 = torch.float32


def _need(t, name: str, dtype: torch.dtype, shape: tuple, device) -> None:
    # Fast path first: one attribute read per property, no allocation.
    try:
        if (t.dtype is dtype and t.shape == shape and t.device == device
                and t.is_contiguous()):
            return
    except AttributeError:
        raise ValueError(f"{name} must be a torch.Tensor") from None
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} (got {t.dtype})")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)} (got {tuple(t.shape)})")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    raise ValueError(f"{name} must be contiguous")


class _on_device:
    """Make ``device`` current for the call; a no-op when it already is."""

    __slots__ = ("idx", "prev")

    def __init__(self, device: torch.device):
        self.idx = device.index if device.index is not None else torch.cuda.current_device()

    def __enter__(self):
        self.prev = torch.cuda.current_device()
        if self.prev != self.idx:
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev != self.idx:
            torch.cuda.set_device(self.prev)
        return False


def _device_of(q: torch.Tensor) -> torch.device:
    if not isinstance(q, torch.Tensor):
        raise ValueError("q must be a torch.Tensor")
    if q.device.type != "cuda":
        raise ValueError(f"tensors must be on a ROCm GPU device (got {q.device})")
    return q.device


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _scale(scale) -> float:
    return 0.0 if scale is None else float(scale)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def decode_kernel(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state) -> None:
    """GDN decode step (T = 1).  Shapes (design.md:97-121):
    q,k [B,1,H{q,k},128] bf16; v [B,1,Hv,128] bf16; state [B,Hv,128,128] fp32 or
    None; A_log,dt_bias [Hv] fp32; a,b [B,1,Hv] bf16; output [B,1,Hv,128] bf16;
    new_state [B,Hv,128,128] fp32 (may be ``state``)."""
    dev = _device_of(q)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D [B, 1, H, d]")
    B, T, Hq, dk = q.shape
    Hk = k.shape[2]
    Hv, dv = v.shape[2], v.shape[3]
    if T != 1:
        raise ValueError(f"decode expects T == 1 (got {T})")
    _need(q, "q", _BF16, (B, 1, Hq, dk), dev)
    _need(k, "k", _BF16, (B, 1, Hk, dk), dev)
    _need(v, "v", _BF16, (B, 1, Hv, dv), dev)
    if state is not None:
        _need(state, "state", _F32, (B, Hv, dv, dk), dev)
    _need(A_log, "A_log", _F32, (Hv,), dev)
    _need(a, "a", _BF16, (B, 1, Hv), dev)
    _need(dt_bias, "dt_bias", _F32, (Hv,), dev)
    _need(b, "b", _BF16, (B, 1, Hv), dev)
    _need(output, "output", _BF16, (B, 1, Hv, dv), dev)
    _need(new_state, "new_state", _F32, (B, Hv, dv, dk), dev)
    lib = _lib.load()
    with _on_device(dev):
        rc = lib.gdn_decode(_ptr(q), _ptr(k), _ptr(v), _ptr(state), _ptr(A_log), _ptr(a),
                            _ptr(dt_bias), _ptr(b), _scale(scale), _ptr(output), _ptr(new_state),
                            B, Hq, Hk, Hv, dk, dv, _stream(dev))
    _lib.check(rc)


def decode_pooled_kernel(q, k, v, state_pool, A_log, a, dt_bias, b, scale, output,
                         state_indices) -> None:
    """Decode step with the state of batch row i held in ``state_pool[state_indices[i]]``
    (updated in place).  state_pool [S,Hv,128,128] fp32; state_indices [B] int32;
    an index outside [0, S) is a padding row (zero output, no slot touched).  Rows
    whose slot another row of the batch also names are skipped the same way, on the
    device, and counted (``decode_pool_conflicts``)."""
    dev = _device_of(q)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D [B, 1, H, d]")
    B, T, Hq, dk = q.shape
    Hk = k.shape[2]
    Hv, dv = v.shape[2], v.shape[3]
    if T != 1:
        raise ValueError(f"decode expects T == 1 (got {T})")
    if state_pool.dim() != 4:
        raise ValueError("state_pool must be 4-D [slots, Hv, dv, dk]")
    slots = state_pool.shape[0]
    _need(q, "q", _BF16, (B, 1, Hq, dk), dev)
    _need(k, "k", _BF16, (B, 1, Hk, dk), dev)
    _need(v, "v", _BF16, (B, 1, Hv, dv), dev)
    _need(state_pool, "state_pool", _F32, (slots, Hv, dv, dk), dev)
    _need(state_indices, "state_indices", torch.int32, (B,), dev)
    _need(A_log, "A_log", _F32, (Hv,), dev)
    _need(a, "a", _BF16, (B, 1, Hv), dev)
    _need(dt_bias, "dt_bias", _F32, (Hv,), dev)
    _need(b, "b", _BF16, (B, 1, Hv), dev)
    _need(output, "output", _BF16, (B, 1, Hv, dv), dev)
    lib = _lib.load()
    with _on_device(dev):
        rc = lib.gdn_decode_pooled(_ptr(q), _ptr(k), _ptr(v), _ptr(state_pool), slots,
                                   _ptr(state_indices), _ptr(A_log), _ptr(a), _ptr(dt_bias),
                                   _ptr(b), _scale(scale), _ptr(output), B, Hq, Hk, Hv, dk, dv,
                                   _stream(dev))
    _lib.check(rc)


def _prefill_args(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, output, new_state):
    """Validate the prefill arguments; returns (device, C-ABI argument list without the
    stream)."""
    dev = _device_of(q)

    def squeeze1(t, nd):
        if t is not None and t.dim() == nd + 1 and t.shape[0] == 1:
            return t[0]
        return t

    q, k, v = squeeze1(q, 3), squeeze1(k, 3), squeeze1(v, 3)
    a, b, output = squeeze1(a, 2), squeeze1(b, 2), squeeze1(output, 3)
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be [T, H, d] (optionally with a leading 1)")
    T, Hq, dk = q.shape
    Hk = k.shape[1]
    Hv, dv = v.shape[1], v.shape[2]
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 1:
        raise ValueError("cu_seqlens must be a 1-D tensor [N + 1]")
    if cu_seqlens.dtype == torch.int32:
        cu_code = _lib.GDN_INDEX_INT32
    elif cu_seqlens.dtype == torch.int64:
        cu_code = _lib.GDN_INDEX_INT64
    else:
        raise ValueError(f"cu_seqlens must be int32 or int64 (got {cu_seqlens.dtype})")
    if cu_seqlens.device != dev or not cu_seqlens.is_contiguous():
        raise ValueError("cu_seqlens must be contiguous and on the same device as q")
    N = cu_seqlens.numel() - 1
    _need(q, "q", _BF16, (T, Hq, dk), dev)
    _need(k, "k", _BF16, (T, Hk, dk), dev)
    _need(v, "v", _BF16, (T, Hv, dv), dev)
    if state is not None:
        _need(state, "state", _F32, (N, Hv, dv, dk), dev)
    _need(A_log, "A_log", _F32, (Hv,), dev)
    _need(a, "a", _BF16, (T, Hv), dev)
    _need(dt_bias, "dt_bias", _F32, (Hv,), dev)
    _need(b, "b", _BF16, (T, Hv), dev)
    _need(output, "output", _BF16, (T, Hv, dv), dev)
    _need(new_state, "new_state", _F32, (N, Hv, dv, dk), dev)
    return dev, [_ptr(q), _ptr(k), _ptr(v), _ptr(state), _ptr(A_log), _ptr(a), _ptr(dt_bias),
                 _ptr(b), cu_seqlens.data_ptr(), cu_code, N, T, None, _ptr(output),
                 _ptr(new_state), Hq, Hk, Hv, dk, dv]


def prefill_kernel(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                   new_state) -> None:
    """Varlen chunked prefill over packed sequences (kernel_prefill.cu:300-306), the
    drop-in ``kernel``.  q,k [T,H{q,k},128] bf16 (a leading batch dim of 1 is
    accepted); v [T,Hv,128] bf16; state [N,Hv,128,128] fp32 or None; a,b [T,Hv] bf16;
    cu_seqlens [N+1] int32 or int64 on the device; output [T,Hv,128] bf16; new_state
    [N,Hv,128,128] fp32 (may be ``state``).  Calls gdn_prefill, as the TVM-FFI shim
    does: nothing is allocated, and calls on any streams give correct results (one long
    sequence runs two kernels in a scratch of the library, whose launches the library
    orders on the device)."""
    dev, args = _prefill_args(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, output, new_state)
    args[12] = _scale(scale)
    lib = _lib.load()
    with _on_device(dev):
        rc = lib.gdn_prefill(*args, _stream(dev))
    _lib.check(rc)


def prefill_workspace_bytes(num_seqs: int, total_tokens: int, num_v_heads: int, device=None) -> int:
    """Bytes of workspace ``prefill_kernel_with_workspace`` uses for a batch of this size on
    ``device`` (gdn_prefill_workspace_size); 0 when the batch runs one kernel anyway."""
    lib = _lib.load()
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    with _on_device(dev):
        return int(lib.gdn_prefill_workspace_size(num_seqs, total_tokens, num_v_heads))


def prefill_kernel_with_workspace(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                                  new_state, workspace) -> None:
    """``prefill_kernel`` with a caller-owned device workspace (gdn_prefill_with_workspace;
    no reference counterpart): batches of few (sequence, v-head) chains then prepare
    each chunk once in a first kernel, for the same results bit for bit.  ``workspace``
    is a contiguous uint8 tensor of at least ``prefill_workspace_bytes(N, T, Hv)`` bytes
    on the same device (or None: ``prefill_kernel``); launches that may overlap must
    not share one."""
    dev, args = _prefill_args(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, output, new_state)
    args[12] = _scale(scale)
    if workspace is not None:
        if not isinstance(workspace, torch.Tensor) or workspace.dtype != torch.uint8 or \
                workspace.dim() != 1 or workspace.device != dev or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous 1-D uint8 tensor on the device of q")
    lib = _lib.load()
    with _on_device(dev):
        rc = lib.gdn_prefill_with_workspace(*args, _ptr(workspace),
                                            0 if workspace is None else workspace.numel(),
                                            _stream(dev))
    _lib.check(rc)


def prefill_giveups(reset: bool = False, device=None) -> int:
    """Number of prefill wavefronts on ``device`` (default: the current one) whose
    hand-off wait gave up since the library was loaded or the last reset
    (gdn_prefill_giveups).  Synchronises the device.  A give-up, which only a defect
    could cause, leaves NaN in the affected outputs and final states; 0 means every
    launch so far completed its hand-offs."""
    import ctypes
    lib = _lib.load()
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    count = ctypes.c_uint64(0)
    with _on_device(dev):
        rc = lib.gdn_prefill_giveups(ctypes.byref(count), 1 if reset else 0)
    _lib.check(rc)
    return int(count.value)


def decode_pool_conflicts(reset: bool = False, device=None) -> int:
    """Number of pooled-decode rows on ``device`` (default: the current one) skipped
    because another row of their batch named the same state slot, since the library
    was loaded or the last reset (gdn_decode_pool_conflicts).  Synchronises the
    device.  A skipped row's output is zero and its slot is left as it was."""
    import ctypes
    lib = _lib.load()
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    count = ctypes.c_uint64(0)
    with _on_device(dev):
        rc = lib.gdn_decode_pool_conflicts(ctypes.byref(count), 1 if reset else 0)
    _lib.check(rc)
    return int(count.value)

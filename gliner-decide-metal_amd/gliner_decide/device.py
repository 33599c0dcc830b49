"""Device-buffer plumbing: torch tensors supply HIP memory and streams.

The arithmetic is in the HIP library; torch is only the allocator and the
stream handle.  Every helper refuses CPU tensors so a call can never run
anywhere but the GPU.
"""

from __future__ import annotations

import torch


def require_gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of a contiguous GPU tensor (None passes through)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("expected a GPU tensor")
    return t.data_ptr()


def stream_handle(stream: torch.cuda.Stream | None = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def as_f16(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be on the GPU")
    if t.dtype != torch.float16:
        raise TypeError(f"{name} must be float16 (got {t.dtype})")
    return t.contiguous()


def as_i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be on the GPU")
    if t.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{name} must be an integer tensor (got {t.dtype})")
    return t.to(torch.int32).contiguous()

"""Device plumbing for driving the gfx950 packs from Python.

PyTorch is used only for device memory and streams.  Every entry point of
the packs rejects stream 0 (the reference's "explicit engine stream" rule,
src/backend/cuda/gemm_plan.cpp:181-184), so callers run under
``engine_stream()``, which makes a dedicated (default-priority) HIP stream
current for both torch allocations and pack launches.
"""
from __future__ import annotations

import contextlib
from typing import Optional

import torch

_stream: Optional["torch.cuda.Stream"] = None


def require_gpu() -> None:
    if not torch.cuda.is_available():
        raise RuntimeError("pih_amd: no HIP device visible; the gfx950 packs have no CPU fallback")


def stream() -> "torch.cuda.Stream":
    global _stream
    require_gpu()
    if _stream is None:
        _stream = torch.cuda.Stream()
    return _stream


@contextlib.contextmanager
def engine_stream():
    s = stream()
    with torch.cuda.stream(s):
        yield s


def stream_handle() -> int:
    h = torch.cuda.current_stream().cuda_stream
    if h == 0:
        raise RuntimeError("pih_amd: launches need an explicit stream; run under pih_amd.device.engine_stream()")
    return h


def ptr(t: Optional[torch.Tensor]) -> int:
    if t is None:
        return 0
    if not t.is_cuda:
        raise ValueError("pih_amd: tensor must live on the HIP device")
    if not t.is_contiguous():
        raise ValueError("pih_amd: tensor must be contiguous")
    return t.data_ptr()


def error_flag() -> torch.Tensor:
    return torch.zeros(1, dtype=torch.int32, device="cuda")


def flag_value(flag: torch.Tensor) -> int:
    return int(flag.item()) & 0xFFFFFFFF

"""Graph capture and host-to-device copies shared by the decoders.

Restates ``CapturedGraph`` and ``to_device`` of the reference's
``transcription.py:133-179``.  On PyTorch-ROCm ``torch.cuda.CUDAGraph`` is a
hipGraph: capture records the decoder step's kernel launches -- the HIP
attention kernels included, which launch on the current stream, read lengths
from device memory and never allocate or synchronize -- and ``replay`` issues
them as one graph launch.
"""

from __future__ import annotations

from typing import Callable

import torch


def to_device(data, device: torch.device) -> torch.Tensor:
    """``data`` copied to ``device`` from pinned memory without waiting for the
    work queued there (``transcription.py:133-139``)."""
    tensor = torch.as_tensor(data)
    if device.type == "cuda":
        tensor = tensor.pin_memory()
    return tensor.to(device, non_blocking=True)


class CapturedGraph:
    """A function of fixed-address tensors captured once as a hipGraph
    (``transcription.py:158-179``): three warm-up calls on a side stream keep
    lazy initialization out of the graph, then one captured call."""

    def __init__(self, function: Callable[[], None], pool=None) -> None:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(3):
                function()
        torch.cuda.current_stream().wait_stream(stream)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=pool, capture_error_mode="thread_local"):
            function()

    def replay(self) -> None:
        self.graph.replay()

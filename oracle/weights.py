"""Seeded random weights addressed by parameter name (test infrastructure).

Every parameter is drawn from its own generator, seeded by (seed, parameter
name), so a state dict does not depend on the order modules register their
parameters and loads into the oracle's and the product's modules alike.
"""

from __future__ import annotations

import math
import zlib

import torch
from torch import Tensor, nn


def named_weights(module: nn.Module, seed: int) -> dict[str, Tensor]:
    """A state dict drawn parameter by parameter from generators seeded by
    (``seed``, parameter name), so it does not depend on registration order:
    norm weights 1 + N(0, 0.1^2), biases and other vectors N(0, 0.02^2),
    matrices N(0, 1 / fan_in)."""
    state = {}
    for name, param in module.named_parameters():
        g = torch.Generator().manual_seed((seed * 1_000_003 + zlib.crc32(name.encode())) % (2**62))
        shape = param.shape
        if param.dim() == 1 and "norm" in name and name.endswith("weight"):
            value = 1.0 + 0.1 * torch.randn(shape, generator=g)
        elif param.dim() == 1:
            value = 0.02 * torch.randn(shape, generator=g)
        else:
            fan_in = math.prod(shape[1:])
            value = torch.randn(shape, generator=g) / math.sqrt(fan_in)
        state[name] = value
    return state

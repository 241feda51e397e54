"""SenseVoiceSmall's SAN-M encoder on the MI355X attention kernels.

Drop-in for the network classes of the reference's ``models/sensevoice.py``
(``:66-212``): same class names, parameter names (FunASR checkpoint names)
and ``forward(x, mask, lengths)`` signatures.  ``SANMAttention`` runs its
attention and its FSMN memory in one kernel call
(:func:`asrback_amd.attention.flash_fsmn`) directly over views of the fused
``linear_q_k_v`` output (token stride ``3 * size``), with the padding
expressed as ``seqused_k = lengths``: the reference's ``varlen_attn`` path
(``sensevoice.py:110-125``), its masked-SDPA fallback (``:126-133``) and the
masked depthwise convolution (``:99-107``) become one launch, and
``linear_out(attention) + memory`` one GEMM accumulating into the memory
(which carries ``linear_out``'s bias).

Padded frames: the attention of a padded frame (a query at or past its
row's length) is not computed; it is zero, so that frame's output is
``linear_out``'s bias alone.  No valid frame can see the difference: every
later op on a padded frame is row-local (norms, linear layers, the FFN), the
FSMN convolution reads values through the frame mask (``sensevoice.py:99-107``:
padded frames contribute zeros) and attention reads keys ``0 .. n_b - 1`` only
(``:115-125``).  Valid frames are bit-identical with or without the skip
(``SANMAttention.zero_padded_rows``).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from .attention import flash_fsmn


class SANMAttention(nn.Module):
    """Self-attention plus a depthwise convolution (FSMN memory) over the
    values (``sensevoice.py:66-135``)."""

    # Padded frames' attention rows are zeros instead of computed (see the
    # module docstring); valid frames are unchanged.
    zero_padded_rows = True

    def __init__(self, in_size: int, size: int, heads: int, kernel_size: int) -> None:
        super().__init__()
        self.heads = heads
        self.size = size
        self.linear_q_k_v = nn.Linear(in_size, size * 3)
        self.linear_out = nn.Linear(size, size)
        self.fsmn_block = nn.Conv1d(size, size, kernel_size, padding=0, groups=size, bias=False)
        if not 1 <= kernel_size <= 15:
            raise ValueError(f"FSMN kernel_size {kernel_size} is outside the supported 1..15")

    def forward(self, x: Tensor, mask: Tensor | None, lengths: Tensor | None) -> Tensor:
        """``mask`` is ``(batch, length)``, True for the first ``lengths[b]``
        frames of row b (the frame mask ``sensevoice.py:548-550`` builds), and
        ``lengths`` (int32) counts them; both are None when every frame is
        real."""
        qkv = self.linear_q_k_v(x)
        query, key, value = qkv.split(self.size, dim=-1)
        batch, length, _ = x.shape
        if lengths is None and mask is not None:
            lengths = mask.sum(dim=1, dtype=torch.int32)
        shape = (batch, length, self.heads, self.size // self.heads)
        output, memory = flash_fsmn(
            query.view(shape),
            key.view(shape),
            value.view(shape),
            self.fsmn_block.weight,
            seqused_k=lengths,
            bias=self.linear_out.bias,
            zero_padded_rows=self.zero_padded_rows and lengths is not None,
        )
        # linear_out(output) + memory: the bias is in memory already.
        memory.view(-1, self.size).addmm_(output.view(-1, self.size), self.linear_out.weight.t())
        return memory


class FeedForward(nn.Module):
    def __init__(self, size: int, hidden: int) -> None:
        super().__init__()
        self.w_1 = nn.Linear(size, hidden)
        self.w_2 = nn.Linear(hidden, size)

    def forward(self, x: Tensor) -> Tensor:
        return self.w_2(F.relu(self.w_1(x)))


class EncoderLayer(nn.Module):
    """``sensevoice.py:148-163``; the first layer changes width and has no
    residual path."""

    def __init__(self, in_size: int, size: int, heads: int, hidden: int, kernel_size: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(in_size)
        self.self_attn = SANMAttention(in_size, size, heads, kernel_size)
        self.norm2 = nn.LayerNorm(size)
        self.feed_forward = FeedForward(size, hidden)
        self.residual = in_size == size

    def forward(self, x: Tensor, mask: Tensor | None, lengths: Tensor | None) -> Tensor:
        attention = self.self_attn(self.norm1(x), mask, lengths)
        x = x + attention if self.residual else attention
        return x + self.feed_forward(self.norm2(x))


def sinusoidal_positions(length: int, depth: int, device: torch.device) -> Tensor:
    """FunASR's sinusoidal encoding of positions ``1..length``
    (``sensevoice.py:166-174``)."""
    positions = torch.arange(1, length + 1, device=device, dtype=torch.float32)
    increment = math.log(10000.0) / (depth / 2 - 1)
    inverse = torch.exp(torch.arange(depth // 2, device=device, dtype=torch.float32) * -increment)
    scaled = positions[:, None] * inverse[None, :]
    return torch.cat((torch.sin(scaled), torch.cos(scaled)), dim=1)


class SenseVoiceEncoder(nn.Module):
    """``sensevoice.py:177-212``: ``encoders0`` (width change), ``num_blocks - 1``
    ``encoders``, ``after_norm``, ``tp_blocks`` ``tp_encoders``, ``tp_norm``."""

    def __init__(self, input_size: int, config: dict) -> None:
        super().__init__()
        size = config["output_size"]
        heads = config["attention_heads"]
        hidden = config["linear_units"]
        kernel = config["kernel_size"]
        if config.get("sanm_shfit", 0):
            raise ValueError("sanm_shfit is not supported")
        self.size = size
        self.encoders0 = nn.ModuleList([EncoderLayer(input_size, size, heads, hidden, kernel)])
        self.encoders = nn.ModuleList(
            EncoderLayer(size, size, heads, hidden, kernel) for _ in range(config["num_blocks"] - 1)
        )
        self.tp_encoders = nn.ModuleList(
            EncoderLayer(size, size, heads, hidden, kernel) for _ in range(config["tp_blocks"])
        )
        self.after_norm = nn.LayerNorm(size)
        self.tp_norm = nn.LayerNorm(size)

    def forward(self, x: Tensor, mask: Tensor | None) -> Tensor:
        positions = sinusoidal_positions(x.shape[1], x.shape[2], x.device)
        x = x * self.size**0.5 + positions.to(x.dtype)
        lengths = None if mask is None else mask.sum(dim=1, dtype=torch.int32)
        for layer in self.encoders0:
            x = layer(x, mask, lengths)
        for layer in self.encoders:
            x = layer(x, mask, lengths)
        x = self.after_norm(x)
        for layer in self.tp_encoders:
            x = layer(x, mask, lengths)
        return self.tp_norm(x)

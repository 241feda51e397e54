"""SenseVoiceSmall's SAN-M encoder restated on the CPU
(``models/sensevoice.py:66-212``) on its masked-SDPA path (``:126-133``),
which is what the reference runs on the CPU and in float32.  Parameter names
match the reference's (FunASR's), so one state dict loads into this encoder
and into ``asrback_amd.sensevoice``.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import attention as oa


class SANMAttention(nn.Module):
    def __init__(self, in_size: int, size: int, heads: int, kernel_size: int) -> None:
        super().__init__()
        self.heads = heads
        self.size = size
        self.kernel_size = kernel_size
        self.linear_q_k_v = nn.Linear(in_size, size * 3)
        self.linear_out = nn.Linear(size, size)
        self.fsmn_block = nn.Conv1d(size, size, kernel_size, padding=0, groups=size, bias=False)

    def forward(self, x: Tensor, mask: Tensor | None, lengths: Tensor | None) -> Tensor:
        del lengths  # the masked-SDPA path reads the mask
        qkv = self.linear_q_k_v(x)
        value = qkv[..., 2 * self.size :]
        memory = oa.fsmn_memory(value, mask, self.fsmn_block.weight, self.kernel_size)
        return self.linear_out(oa.sensevoice_attention(qkv, self.heads, mask)) + memory


class EncoderLayer(nn.Module):
    def __init__(self, in_size: int, size: int, heads: int, hidden: int, kernel_size: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(in_size)
        self.self_attn = SANMAttention(in_size, size, heads, kernel_size)
        self.norm2 = nn.LayerNorm(size)
        self.feed_forward = nn.Module()
        self.feed_forward.w_1 = nn.Linear(size, hidden)
        self.feed_forward.w_2 = nn.Linear(hidden, size)
        self.residual = in_size == size

    def forward(self, x: Tensor, mask: Tensor | None, lengths: Tensor | None) -> Tensor:
        attention = self.self_attn(self.norm1(x), mask, lengths)
        x = x + attention if self.residual else attention
        h = self.norm2(x)
        return x + self.feed_forward.w_2(F.relu(self.feed_forward.w_1(h)))


def sinusoidal_positions(length: int, depth: int) -> Tensor:
    """Positions ``1..length`` (``sensevoice.py:166-174``)."""
    positions = torch.arange(1, length + 1, dtype=torch.float32)
    increment = math.log(10000.0) / (depth / 2 - 1)
    inverse = torch.exp(torch.arange(depth // 2, dtype=torch.float32) * -increment)
    scaled = positions[:, None] * inverse[None, :]
    return torch.cat((torch.sin(scaled), torch.cos(scaled)), dim=1)


class SenseVoiceEncoder(nn.Module):
    """``sensevoice.py:177-212``."""

    def __init__(self, input_size: int, config: dict) -> None:
        super().__init__()
        size, heads = config["output_size"], config["attention_heads"]
        hidden, kernel = config["linear_units"], config["kernel_size"]
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
        x = x * self.size**0.5 + sinusoidal_positions(x.shape[1], x.shape[2]).to(x.dtype)
        lengths = None if mask is None else mask.sum(dim=1, dtype=torch.int32)
        for layer in self.encoders0:
            x = layer(x, mask, lengths)
        for layer in self.encoders:
            x = layer(x, mask, lengths)
        x = self.after_norm(x)
        for layer in self.tp_encoders:
            x = layer(x, mask, lengths)
        return self.tp_norm(x)


def frame_mask(lengths: Tensor, queries: int, frames: int) -> Tensor:
    """``(B, queries + frames)`` mask of real frames, the four query
    embeddings included (``sensevoice.py:548-550``)."""
    return oa.key_padding_mask(lengths + queries, queries + frames)

"""Qwen3-ASR's attention modules on the MI355X kernels.

Drop-in for the attention side of the reference's ``models/qwen3_asr.py``:
``Segments``/``attend`` (``:123-181``), ``AudioAttention`` (``:207-221``),
``RMSNorm``/``rotate`` (``:316-330``), ``KVCache`` (``:333-347``),
``TextAttention`` (``:350-432``) and ``TextModel`` (``:463-524``), with the
same names, parameter names and signatures, and the cache layout
``(layers, batch, length, kv_heads, head_dim)``.

* Packed prompts and audio windows attend through
  :func:`asrback_amd.attention.varlen_attn` in every dtype (the reference
  falls back to a padded, gathered SDPA off CUDA/bf16, ``:167-181``).
* A decoder step attends with :func:`asrback_amd.attention.decode` straight
  over the row's cache slab, ``seqused_k = position + 1`` read on the device,
  grouped-query attention in the kernel (16 query heads share 8 kv heads,
  query head h reads kv head h // 2).  ``TextAttention.step`` accepts the
  reference's ``mask`` in both of its forms -- the varlen tuple
  ``(query_starts, key_starts, lengths)`` and the boolean ``(batch, 1, 1,
  length)`` mask -- and a :class:`~asrback_amd.attention.KeyPrefix`.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from .attention import KeyPrefix, decode, varlen_attn
from .transcription import to_device

# Positions per row of the KV cache (qwen3_asr.py:57-59).
CACHE_LENGTH = 1024


@dataclass
class Segments:
    """Boundaries of sequences laid out back to back in a packed tensor
    (``qwen3_asr.py:123-149``): ``starts`` are int32 cumulative lengths from
    0 and ``longest`` the longest sequence.  ``varlen`` is kept for the
    reference's signature; the kernels always read packed sequences."""

    starts: Tensor
    longest: int
    varlen: bool = True

    @classmethod
    def from_lengths(cls, lengths: list[int], device: torch.device, varlen: bool = True) -> Segments:
        sizes = to_device(lengths, device)
        starts = F.pad(sizes.cumsum(0), (1, 0)).to(torch.int32)
        return cls(starts, max(lengths), varlen)


def attend(q: Tensor, k: Tensor, v: Tensor, segments: Segments, causal: bool) -> Tensor:
    """Attention within each segment of packed ``(tokens, heads, head_dim)``
    tensors; ``k``/``v`` may have fewer heads (``qwen3_asr.py:152-181``)."""
    return varlen_attn(
        q,
        k,
        v,
        segments.starts,
        segments.starts,
        segments.longest,
        segments.longest,
        window_size=(-1, 0) if causal else (-1, -1),
        enable_gqa=k.shape[1] != q.shape[1],
    )


class AudioAttention(nn.Module):
    """Windowed non-causal encoder attention (``qwen3_asr.py:207-221``)."""

    def __init__(self, width: int, heads: int) -> None:
        super().__init__()
        self.heads = heads
        self.q_proj = nn.Linear(width, width)
        self.k_proj = nn.Linear(width, width)
        self.v_proj = nn.Linear(width, width)
        self.out_proj = nn.Linear(width, width)

    def forward(self, x: Tensor, segments: Segments) -> Tensor:
        q, k, v = (projection(x).view(len(x), self.heads, -1) for projection in (self.q_proj, self.k_proj, self.v_proj))
        return self.out_proj(attend(q, k, v, segments, causal=False).flatten(1))


class RMSNorm(nn.Module):
    def __init__(self, width: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(width))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        return F.rms_norm(x, self.weight.shape, self.weight, self.eps)


def rotate(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Half-split rotary embedding of ``(..., heads, head_dim)`` with
    ``cos``/``sin`` ``(..., head_dim)`` (``qwen3_asr.py:326-330``)."""
    first, second = x.chunk(2, dim=-1)
    rotated = torch.cat((-second, first), dim=-1)
    return x * cos[..., None, :] + rotated * sin[..., None, :]


def rope_tables(config: dict, length: int, device: torch.device, dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    """``cos``/``sin`` ``(length, head_dim)`` in the model dtype
    (``qwen3_asr.py:795-803``)."""
    head_dim = config["head_dim"]
    inverse = 1.0 / (config["rope_theta"] ** (torch.arange(0, head_dim, 2).float() / head_dim))
    angles = torch.arange(length).float()[:, None] * inverse[None, :]
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos().to(device, dtype), angles.sin().to(device, dtype)


@dataclass
class KVCache:
    """Preallocated keys and values, ``(layers, batch, length, kv_heads,
    head_dim)`` (``qwen3_asr.py:333-347``); written in place, so the tensors
    keep fixed addresses across graph replays."""

    keys: Tensor
    values: Tensor

    @classmethod
    def allocate(cls, config: dict, batch: int, length: int, device, dtype) -> KVCache:
        shape = (config["num_hidden_layers"], batch, length, config["num_key_value_heads"], config["head_dim"])
        return cls(torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device))

    def narrow(self, batch_size: int, length: int) -> KVCache:
        return KVCache(self.keys[:, :batch_size, :length], self.values[:, :batch_size, :length])


def _step_lengths(mask, positions: Tensor, length: int) -> Tensor:
    """Keys per row for a decoder step from any of the reference's mask forms."""
    if isinstance(mask, KeyPrefix):
        return mask.lengths if mask.lengths is not None else (mask.positions + 1).clamp(max=length).to(torch.int32)
    if isinstance(mask, tuple):
        return mask[2]  # (query_starts, key_starts, lengths) of qwen3_asr.py:510-512
    if isinstance(mask, Tensor):
        return KeyPrefix.from_mask(mask).lengths
    return (positions + 1).clamp(max=length).to(torch.int32)


class TextAttention(nn.Module):
    """``qwen3_asr.py:350-432``: fused qkv projection, per-head RMSNorm on q
    and k, RoPE, grouped-query attention."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        width = config["hidden_size"]
        self.head_dim = config["head_dim"]
        self.heads = config["num_attention_heads"]
        self.kv_heads = config["num_key_value_heads"]
        self.sizes = [size * self.head_dim for size in (self.heads, self.kv_heads, self.kv_heads)]
        self.qkv_proj = nn.Linear(width, sum(self.sizes), bias=False)
        self.o_proj = nn.Linear(self.heads * self.head_dim, width, bias=False)
        self.q_norm = RMSNorm(self.head_dim, config["rms_norm_eps"])
        self.k_norm = RMSNorm(self.head_dim, config["rms_norm_eps"])

    def _project(self, x: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, ...]:
        shape = (len(x), -1, self.head_dim)
        q, k, v = self.qkv_proj(x).split(self.sizes, dim=-1)
        q = rotate(self.q_norm(q.reshape(shape)), cos, sin)
        k = rotate(self.k_norm(k.reshape(shape)), cos, sin)
        return q, k, v.reshape(shape)

    def prefill(self, x, keys, values, rows, positions, segments: Segments, cos, sin) -> Tensor:
        """Causal attention within each packed prompt; every token's key and
        value go to its row and position of the cache (``:374-390``)."""
        q, k, v = self._project(x, cos, sin)
        keys[rows, positions] = k
        values[rows, positions] = v
        return self.o_proj(attend(q, k, v, segments, causal=True).flatten(1))

    def step(self, x, keys, values, positions, mask, cos, sin) -> Tensor:
        """One token per row at its own position, attending over the cache
        view ``keys``/``values`` ``(batch, length, kv_heads, head_dim)``
        (``:392-432``)."""
        q, k, v = self._project(x, cos, sin)
        rows = torch.arange(len(x), device=x.device)
        keys[rows, positions] = k
        values[rows, positions] = v
        lengths = _step_lengths(mask, positions, keys.shape[1])
        output = decode(q, keys, values, seqused_k=lengths)
        return self.o_proj(output.flatten(1))


class TextMLP(nn.Module):
    def __init__(self, config: dict) -> None:
        super().__init__()
        width, hidden = config["hidden_size"], config["intermediate_size"]
        self.gate_up_proj = nn.Linear(width, 2 * hidden, bias=False)
        self.down_proj = nn.Linear(hidden, width, bias=False)

    def forward(self, x: Tensor) -> Tensor:
        gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)


class DecoderLayer(nn.Module):
    def __init__(self, config: dict) -> None:
        super().__init__()
        self.input_layernorm = RMSNorm(config["hidden_size"], config["rms_norm_eps"])
        self.self_attn = TextAttention(config)
        self.post_attention_layernorm = RMSNorm(config["hidden_size"], config["rms_norm_eps"])
        self.mlp = TextMLP(config)

    def forward(self, x: Tensor, attention: Callable[[TextAttention, Tensor], Tensor]) -> Tensor:
        x = x + attention(self.self_attn, self.input_layernorm(x))
        return x + self.mlp(self.post_attention_layernorm(x))


class TextModel(nn.Module):
    """``qwen3_asr.py:463-524``."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(config["vocab_size"], config["hidden_size"])
        self.layers = nn.ModuleList(DecoderLayer(config) for _ in range(config["num_hidden_layers"]))
        self.norm = RMSNorm(config["hidden_size"], config["rms_norm_eps"])

    def prefill(self, x, cache: KVCache, rows, positions, segments: Segments, cos, sin) -> Tensor:
        for index, layer in enumerate(self.layers):
            keys, values = cache.keys[index], cache.values[index]
            x = layer(x, lambda attention, h: attention.prefill(h, keys, values, rows, positions, segments, cos, sin))
        return self.norm(x)

    def step(self, tokens, positions, cache: KVCache, cos, sin, varlen: bool = True) -> Tensor:
        """Hidden states for one token per row over a fixed-shape cache view;
        ``cos``/``sin`` are the full tables.  Each row reads its keys
        ``0 .. position`` whatever the view's length (``varlen`` is kept for
        the reference's signature)."""
        del varlen
        x = self.embed_tokens(tokens)
        cos, sin = cos[positions], sin[positions]
        mask = KeyPrefix(lengths=(positions + 1).clamp(max=cache.keys.shape[2]).to(torch.int32))
        for index, layer in enumerate(self.layers):
            keys, values = cache.keys[index], cache.values[index]
            x = layer(x, lambda attention, h: attention.step(h, keys, values, positions, mask, cos, sin))
        return self.norm(x)

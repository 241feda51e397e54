"""The reference's attention calls, restated on the CPU with torch's SDPA.

Each function reproduces one call pattern of the reference -- the mask it
builds, the layout it passes, the GQA grouping -- around the library routine
``F.scaled_dot_product_attention`` (torch's CPU kernels), the same routine the
reference itself runs on the CPU and in float32.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor


def sdpa(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    attn_mask: Tensor | None = None,
    is_causal: bool = False,
    enable_gqa: bool = False,
    scale: float | None = None,
) -> Tensor:
    """``F.scaled_dot_product_attention`` on ``(B, H, L, D)`` tensors, as called
    at ``whisper.py:102-104``, ``sensevoice.py:128-133``,
    ``qwen3_asr.py:176-180``/``:429-431`` and (``scale=1.0``)
    ``gemma4.py:552-559``/``:580-586``."""
    return F.scaled_dot_product_attention(
        query, key, value, attn_mask=attn_mask, is_causal=is_causal, enable_gqa=enable_gqa, scale=scale
    )


def split_heads(x: Tensor, heads: int) -> Tensor:
    """``(B, L, W)`` -> ``(B, H, L, W / H)`` view (``whisper.py:85-87``,
    ``sensevoice.py:90-92``)."""
    batch, length, width = x.shape
    return x.view(batch, length, heads, width // heads).transpose(1, 2)


def whisper_step_mask(positions: Tensor, length: int) -> Tensor:
    """Mask of a fixed-shape decoder step over ``length`` cache positions:
    key ``j`` visible to row ``b`` iff ``j <= positions[b]``
    (``whisper.py:263-264``).  Shape ``(B, 1, 1, length)``."""
    key_positions = torch.arange(length, device=positions.device)
    return (key_positions[None, :] <= positions[:, None])[:, None, None, :]


def gemma_step_mask(positions: Tensor, length: int, window: int | None) -> Tensor:
    """Mask of a Gemma 4 decoder step (``gemma4.py:717-725``): key ``j``
    visible to row ``b`` iff ``j <= positions[b]`` and, on sliding-window
    layers, ``j > positions[b] - window``.  Shape ``(B, 1, 1, length)``."""
    key_positions = torch.arange(length, device=positions.device)[None, :]
    mask = key_positions <= positions[:, None]
    if window is not None:
        mask = mask & (key_positions > positions[:, None] - window)
    return mask[:, None, None, :]


def gemma_prefill_mask(sizes: Tensor, longest: int, window: int | None) -> Tensor:
    """Mask of the Gemma 4 padded prompt pass (``gemma4.py:1227-1235``):
    causal, keys before each prompt's size, and on sliding-window layers
    keys within ``window`` of the query.  Shape ``(B, 1, longest, longest)``."""
    positions = torch.arange(longest, device=sizes.device)
    causal = (positions[None, :] <= positions[:, None]) & (positions[None, None, :] < sizes[:, None, None])
    if window is not None:
        causal = causal & (positions[None, :] > positions[:, None] - window)
    return causal[:, None]


def key_padding_mask(lengths: Tensor, length: int) -> Tensor:
    """``(B, length)`` mask, True for the first ``lengths[b]`` frames
    (``sensevoice.py:548-550``)."""
    frames = torch.arange(length, device=lengths.device)
    return frames[None, :] < lengths[:, None]


def fsmn_memory(value: Tensor, mask: Tensor | None, weight: Tensor, kernel_size: int) -> Tensor:
    """SAN-M's FSMN memory (``sensevoice.py:99-107``): a depthwise convolution
    (``weight`` ``(C, 1, kernel_size)``, no bias) over the masked values, plus
    the masked values, masked again."""
    keep = None if mask is None else mask[..., None].to(value.dtype)
    masked = value if keep is None else value * keep
    left = (kernel_size - 1) // 2
    padded = F.pad(masked.transpose(1, 2), (left, kernel_size - 1 - left))
    memory = F.conv1d(padded, weight, groups=value.shape[-1]).transpose(1, 2) + masked
    return memory if keep is None else memory * keep


def sensevoice_attention(qkv: Tensor, heads: int, mask: Tensor | None) -> Tensor:
    """SAN-M attention core on the fused projection ``qkv`` ``(B, L, 3W)``
    (``sensevoice.py:97``, ``:126-134``): key-padding mask ``(B, 1, 1, L)``;
    returns ``(B, L, W)``."""
    size = qkv.shape[-1] // 3
    query, key, value = qkv.split(size, dim=-1)
    attention_mask = None if mask is None else mask[:, None, None, :]
    out = sdpa(
        split_heads(query, heads),
        split_heads(key, heads),
        split_heads(value, heads),
        attn_mask=attention_mask,
    ).transpose(1, 2)
    return out.reshape(qkv.shape[0], qkv.shape[1], size)


@dataclass
class Segments:
    """Packed-sequence boundaries on the padded path (``qwen3_asr.py:123-149``):
    ``starts`` (int32 cumulative lengths), ``gather`` ``(S, longest)`` token
    indices padded with each sequence's last token, ``valid`` its real ones."""

    starts: Tensor
    longest: int
    gather: Tensor
    valid: Tensor

    @classmethod
    def from_lengths(cls, lengths: list[int]) -> Segments:
        sizes = torch.tensor(lengths)
        starts = F.pad(sizes.cumsum(0), (1, 0)).to(torch.int32)
        longest = max(lengths)
        offsets = torch.arange(longest)
        valid = offsets < sizes[:, None]
        last = (starts[1:] - 1)[:, None]
        gather = torch.minimum(starts[:-1, None] + offsets, last)
        return cls(starts, longest, gather, valid)


def qwen_attend(q: Tensor, k: Tensor, v: Tensor, segments: Segments, causal: bool) -> Tensor:
    """Attention within packed sequences of ``(tokens, heads, D)`` tensors, GQA
    when ``k`` has fewer heads (``qwen3_asr.py:167-181``)."""
    mask = segments.valid[:, None, None, :]
    if causal:
        mask = mask & torch.ones((segments.longest,) * 2, dtype=torch.bool).tril()
    out = sdpa(
        *(t[segments.gather].transpose(1, 2) for t in (q, k, v)),
        attn_mask=mask,
        enable_gqa=True,
    )
    return out.transpose(1, 2)[segments.valid]


def qwen_step_mask(positions: Tensor, length: int) -> Tensor:
    """``(B, 1, 1, length)`` mask of a Qwen3 decoder step (``qwen3_asr.py:514-515``)."""
    return whisper_step_mask(positions, length)


def qwen_step_attention(q: Tensor, keys: Tensor, values: Tensor, mask: Tensor) -> Tensor:
    """GQA decode on the padded path (``qwen3_asr.py:427-432``): ``q`` (B, Hq, D)
    viewed as (B, Hkv, Hq / Hkv, D) -- the query heads of one kv head attend as
    one group of queries -- over ``keys``/``values`` (B, L, Hkv, D).
    Returns (B, Hq, D)."""
    batch, heads_q, head_dim = q.shape
    heads_kv = keys.shape[2]
    grouped = q.view(batch, heads_kv, heads_q // heads_kv, head_dim)
    out = sdpa(grouped, keys.transpose(1, 2), values.transpose(1, 2), attn_mask=mask)
    return out.reshape(batch, heads_q, head_dim)


def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """``F.rms_norm`` over the last axis (``qwen3_asr.py:322-323``)."""
    return F.rms_norm(x, weight.shape, weight, eps)


def rotate(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Half-split rotary embedding of ``(..., heads, D)`` with ``cos``/``sin``
    ``(..., D)`` (``qwen3_asr.py:326-330``)."""
    first, second = x.chunk(2, dim=-1)
    rotated = torch.cat((-second, first), dim=-1)
    return x * cos[..., None, :] + rotated * sin[..., None, :]


def rope_tables(theta: float, head_dim: int, length: int, dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    """``cos``/``sin`` tables ``(length, head_dim)`` rounded to the model dtype
    (``qwen3_asr.py:795-803``)."""
    inverse = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    angles = torch.arange(length).float()[:, None] * inverse[None, :]
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos().to(dtype), angles.sin().to(dtype)

"""Gemma 4's attention modules on the MI355X kernels.

Drop-in for the attention side of the reference's ``models/gemma4.py``:
``RMSNorm``, ``ClippedLinear`` (``:166-197``), the audio encoder's
``AudioAttention`` (``:199-282``), ``rotate``/``rotary_tables``
(``:440-465``), ``LayerKV`` (``:469-483``) and the language model's
``TextAttention`` (``:486-587``), with the same names, parameter names and
signatures.

* ``AudioAttention`` keeps its projections in PyTorch and runs the blocked
  local attention -- context gathering, content and relative scores, the
  Transformer-XL relative shift, the soft cap, the mask and the softmax --
  as one kernel (:func:`~asrback_amd.attention.local_attention`).
* ``TextAttention.prefill`` attends over the padded prompts with the
  multi-row kernel (causal, each prompt's size, the 512-key window on
  sliding layers, ``scale=1.0``, grouped-query attention, head_dim 256 or
  512); ``step`` with the decode kernel over the ``(batch, length, kv_heads,
  head_dim)`` cache, keys ``0 .. position`` (the window's last keys on
  sliding layers).  KV-shared layers read the cache (or the prompt's keys)
  of the last earlier layer of their type, as the reference passes them.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _lib
from .attention import KeyPrefix, decode, decode_append, decode_supported, flash, local_attention


class RMSNorm(nn.Module):
    """Root-mean-square normalization as Gemma 4 applies it
    (``gemma4.py:166-180``): the statistics in float32, then an optional
    learned scale (none when ``scale=False``)."""

    def __init__(self, width: int, eps: float, scale: bool = True) -> None:
        super().__init__()
        self.width = width
        self.eps = eps
        if scale:
            self.weight = nn.Parameter(torch.ones(width))
        else:
            self.register_parameter("weight", None)

    def forward(self, x: Tensor) -> Tensor:
        weight = None if self.weight is None else self.weight.float()
        return F.rms_norm(x.float(), (self.width,), weight, self.eps).type_as(x)


class ClippedLinear(nn.Module):
    """``nn.Linear`` between two clamps whose bounds come with the checkpoint
    (``gemma4.py:183-197``)."""

    def __init__(self, inputs: int, outputs: int) -> None:
        super().__init__()
        self.linear = nn.Linear(inputs, outputs, bias=False)
        for name in ("input_min", "output_min"):
            self.register_buffer(name, torch.tensor(-math.inf))
        for name in ("input_max", "output_max"):
            self.register_buffer(name, torch.tensor(math.inf))

    def forward(self, x: Tensor) -> Tensor:
        x = self.linear(x.clamp(self.input_min, self.input_max))
        return x.clamp(self.output_min, self.output_max)


def _lengths_from_blocked_mask(mask: Tensor, chunk: int, past: int) -> Tensor:
    """Valid tokens per sequence from the ``(batch, 1, blocks, chunk,
    context)`` mask of ``AudioAttention.blocked_mask`` (True = may not
    attend): one more than the last key any query may see (the key at the
    last valid position is visible to itself)."""
    blocks, context = mask.shape[2], mask.shape[4]
    keys = (torch.arange(blocks, device=mask.device) * chunk - past)[:, None, None] + torch.arange(
        context, device=mask.device
    )
    seen = torch.where(~mask[:, 0], keys, torch.full_like(keys, -1))
    return (seen.flatten(1).amax(dim=1) + 1).to(torch.int32)


class AudioAttention(nn.Module):
    """Gemma 4's audio attention (``gemma4.py:199-282``): frames are grouped
    in blocks of ``chunk``; a frame attends to itself and its ``past - 1``
    predecessors, scores get a learned bias by relative distance."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        width = config["hidden_size"]
        self.heads = config["num_attention_heads"]
        self.head_dim = width // self.heads
        self.q_scale = self.head_dim**-0.5 / math.log(2)
        self.k_scale = math.log(1 + math.e) / math.log(2)
        self.chunk = config["attention_chunk_size"]
        self.past = config["attention_context_left"] - 1
        self.future = config["attention_context_right"]
        self.context = self.chunk + self.past + self.future
        self.softcap = config["attention_logit_cap"]
        self.invalid = config["attention_invalid_logits_value"]
        self.q_proj = ClippedLinear(width, width)
        self.k_proj = ClippedLinear(width, width)
        self.v_proj = ClippedLinear(width, width)
        self.post = ClippedLinear(width, width)
        self.relative_k_proj = nn.Linear(width, width, bias=False)
        self.per_dim_scale = nn.Parameter(torch.zeros(self.head_dim))

    def blocked_mask(self, lengths: Tensor, frames: int) -> Tensor:
        """The blocked layout's exclusion mask (``gemma4.py:223-240``): shape
        ``(batch, 1, blocks, chunk, context)``, True for each (query, context
        slot) pair that is out of reach or past the sequence's length."""
        blocks = -(-frames // self.chunk)
        device = lengths.device
        query = torch.arange(blocks * self.chunk, device=device).view(blocks, self.chunk, 1)
        key = (torch.arange(blocks, device=device) * self.chunk - self.past).view(blocks, 1, 1) + torch.arange(
            self.context, device=device
        )
        distance = query - key
        allowed = (distance >= 0) & (distance < self.past) & (key >= 0)
        if self.future:
            allowed |= (distance < 0) & (-distance < self.future)
        allowed = allowed & (key < lengths.view(-1, 1, 1, 1))
        return ~allowed[:, None]

    def forward(self, x: Tensor, positions: Tensor, mask: Tensor | KeyPrefix) -> Tensor:
        """``positions``: the relative-distance sinusoids; ``mask``: the
        blocked mask (or a :class:`KeyPrefix` of the valid token counts)."""
        batch, frames, _ = x.shape
        shape = (batch, frames, self.heads, self.head_dim)
        q = self.q_proj(x).float().view(shape)
        q = q * self.q_scale * F.softplus(self.per_dim_scale)
        k = self.k_proj(x).float().view(shape) * self.k_scale
        v = self.v_proj(x).float().view(shape)
        relative = self.relative_k_proj(positions).float().view(-1, self.heads, self.head_dim)
        if isinstance(mask, KeyPrefix):
            lengths = mask.lengths
        else:
            lengths = _lengths_from_blocked_mask(mask, self.chunk, self.past)
        output = local_attention(
            q, k, v, relative.contiguous(), lengths, chunk=self.chunk, past=self.past, future=self.future,
            softcap=float(self.softcap), invalid=float(self.invalid),
        )
        return self.post(output.reshape(batch, frames, -1).to(x.dtype))


def rotate(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Half-split rotary embedding (``gemma4.py:440-445``): ``x`` is
    ``(..., heads, head_dim)``; ``cos`` and ``sin`` are ``(..., head_dim)``,
    broadcast over the heads."""
    first, second = x.chunk(2, dim=-1)
    rotated = torch.cat((-second, first), dim=-1)
    return x * cos[..., None, :] + rotated * sin[..., None, :]


def rotary_tables(text: dict, layer_type: str, head_dim: int, length: int) -> tuple[Tensor, Tensor]:
    """``cos``/``sin`` ``(length, head_dim)`` of a layer type; proportional
    RoPE rotates the first ``partial_rotary_factor`` of the frequencies
    (``gemma4.py:448-465``)."""
    parameters = text["rope_parameters"][layer_type]
    angles = head_dim // 2
    if parameters["rope_type"] == "proportional":
        angles = int(parameters.get("partial_rotary_factor", 1.0) * head_dim // 2)
    elif parameters["rope_type"] != "default":
        raise ValueError(f"unsupported RoPE type {parameters['rope_type']!r}")
    inverse = 1.0 / (parameters["rope_theta"] ** (torch.arange(0, 2 * angles, 2).float() / head_dim))
    inverse = F.pad(inverse, (0, head_dim // 2 - angles))
    angles = torch.arange(length).float()[:, None] * inverse[None, :]
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos(), angles.sin()


@dataclass
class LayerKV:
    """One layer's cache tensors, ``(batch, length, kv_heads, head_dim)``,
    allocated once and updated in place (``gemma4.py:469-483``)."""

    keys: Tensor
    values: Tensor

    def narrow(self, batch_size: int, length: int) -> LayerKV:
        return LayerKV(self.keys[:batch_size, :length], self.values[:batch_size, :length])


def _prompt_sizes(mask: Tensor) -> Tensor:
    """Each prompt's size from the prompt pass's ``(batch, 1, length,
    length)`` mask: its diagonal is True exactly on the prompt's tokens."""
    return mask[:, 0].diagonal(dim1=-2, dim2=-1).sum(dim=-1, dtype=torch.int32)


class TextAttention(nn.Module):
    """Gemma 4's text attention (``gemma4.py:486-587``): RMS norms on the
    queries, keys and values, softmax without a 1/sqrt(d) factor.  The final
    ``num_kv_shared_layers`` layers project queries only and reuse the cache
    of the nearest earlier layer of the same kind."""

    def __init__(self, text: dict, layer_type: str, shared: bool) -> None:
        super().__init__()
        width = text["hidden_size"]
        eps = text["rms_norm_eps"]
        full = layer_type == "full_attention"
        self.head_dim = text["global_head_dim"] if full else text["head_dim"]
        self.heads = text["num_attention_heads"]
        self.kv_heads = text["num_key_value_heads"]
        if full and text.get("attention_k_eq_v") and text["num_global_key_value_heads"]:
            self.kv_heads = text["num_global_key_value_heads"]
        self.window = None if full else text["sliding_window"]
        self.layer_type = layer_type
        self.shared = shared
        self.q_norm = RMSNorm(self.head_dim, eps)
        if shared:
            self.q_proj = nn.Linear(width, self.heads * self.head_dim, bias=False)
        else:
            self.sizes = [size * self.head_dim for size in (self.heads, self.kv_heads, self.kv_heads)]
            self.qkv_proj = nn.Linear(width, sum(self.sizes), bias=False)
            self.k_norm = RMSNorm(self.head_dim, eps)
            self.v_norm = RMSNorm(self.head_dim, eps, scale=False)
        self.o_proj = nn.Linear(self.heads * self.head_dim, width, bias=False)

    def _project(self, x: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor | None, Tensor | None]:
        shape = (*x.shape[:-1], -1, self.head_dim)
        if self.shared:
            return rotate(self.q_norm(self.q_proj(x).view(shape)), cos, sin), None, None
        q, k, v = self.qkv_proj(x).split(self.sizes, dim=-1)
        q = rotate(self.q_norm(q.reshape(shape)), cos, sin)
        k = rotate(self.k_norm(k.reshape(shape)), cos, sin)
        return q, k, self.v_norm(v.reshape(shape))

    def prefill(self, x: Tensor, cache: LayerKV, rows: Tensor, kv: dict[str, tuple[Tensor, Tensor]],
                mask: Tensor | KeyPrefix, cos: Tensor, sin: Tensor) -> Tensor:
        """The prompt pass: padded prompts ``x`` ``(batch, length, width)``
        attend causally (within the window on sliding layers) and their keys
        and values go to cache ``rows``.  ``mask`` is either the reference's
        prompt mask or a :class:`KeyPrefix` holding each prompt's size."""
        q, k, v = self._project(x, cos, sin)
        if self.shared:
            k, v = kv[self.layer_type]
        else:
            length = x.shape[1]
            cache.keys[rows, :length] = k
            cache.values[rows, :length] = v
            kv[self.layer_type] = k, v
        sizes = mask.lengths if isinstance(mask, KeyPrefix) else _prompt_sizes(mask)
        output = flash(q, k, v, causal=_lib.CAUSAL_TOP_LEFT, seqused_k=sizes, scale=1.0, window=self.window)
        return self.o_proj(output.flatten(2))

    def step(self, x: Tensor, cache: LayerKV, positions: Tensor, mask, cos: Tensor, sin: Tensor) -> Tensor:
        """One token per row at its own position over the cache; ``mask`` is
        the step's (causal at ``positions``, the window on sliding layers, as
        ``TextModel.step`` builds it from the same positions)."""
        del mask  # keys 0 .. position, and the window: from positions
        if not self.shared and decode_supported(x.dtype, self.head_dim, self.heads // self.kv_heads):
            # One launch: the q/k/v norms, the rotation, the cache writes at
            # each row's position and the attention (asrattn_decode_append).
            q, k, v = self.qkv_proj(x).split(self.sizes, dim=-1)
            shape = (len(x), -1, self.head_dim)
            output = decode_append(q.view(shape), k.view(shape), v.view(shape), cache.keys, cache.values, positions,
                                   q_norm=self.q_norm.weight, k_norm=self.k_norm.weight, eps=self.q_norm.eps,
                                   cos=cos, sin=sin, scale=1.0, window=self.window, v_norm=True)
            return self.o_proj(output.reshape(len(x), -1))
        q, k, v = self._project(x, cos, sin)
        if not self.shared:
            rows = torch.arange(len(x), device=x.device)
            cache.keys[rows, positions] = k
            cache.values[rows, positions] = v
        if decode_supported(q.dtype, self.head_dim, self.heads // self.kv_heads):
            output = decode(q, cache.keys, cache.values, positions=positions, scale=1.0, window=self.window)
        else:
            # float32 at head_dim 512 (a key row is wider than a wave's 16-byte
            # lanes): the multi-row kernel with one query per row, which sees
            # keys 0 .. position as the bottom-right-aligned causal mask.
            used = (positions + 1).clamp(max=cache.keys.shape[1]).to(torch.int32)
            output = flash(q[:, None], cache.keys, cache.values, causal=_lib.CAUSAL_BOTTOM_RIGHT, seqused_k=used,
                           scale=1.0, window=self.window)
        return self.o_proj(output.reshape(len(x), -1))

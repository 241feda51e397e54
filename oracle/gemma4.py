"""Gemma 4's attention restated on the CPU (``models/gemma4.py:199-282``,
``:440-587``): test infrastructure, the CPU reference the GPU modules of
``asrback_amd.gemma4`` are compared with.

``local_attention`` follows the reference's route through the blocked audio
attention -- padding, ``unfold`` into per-block contexts, content scores,
relative scores against the distance sinusoids' keys and the
Transformer-XL relative shift, the soft cap, the mask, softmax -- and
``local_attention_loops`` computes the same from its definition, query by
query and key by key, so that the tests pin the shift and the masks.
``TextAttention`` is the language model's attention on torch SDPA with the
reference's masks (``oracle.attention.gemma_*_mask``) and ``scale=1.0``.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import attention as oa


def relative_positions(width: int, chunk: int, context_left: int, context_right: int) -> Tensor:
    """Sinusoids ``[sin, cos]`` of the relative distances ``context // 2 .. 0``
    (``gemma4.py:380-396``)."""
    context = chunk + context_left - 1 + context_right
    timescales = width // 2
    increment = math.log(10000) / max(timescales - 1, 1)
    inverse = torch.exp(torch.arange(timescales) * -increment)
    distances = torch.arange(context // 2, -1, -1)[:, None]
    scaled = distances * inverse[None, :]
    return torch.cat((torch.sin(scaled), torch.cos(scaled)), dim=-1)


def blocked_mask(lengths: Tensor, frames: int, chunk: int, past: int, future: int) -> Tensor:
    """``(batch, 1, blocks, chunk, context)``, True where a query may not
    attend (``gemma4.py:223-240``)."""
    blocks = -(-frames // chunk)
    context = chunk + past + future
    query = torch.arange(blocks * chunk).view(blocks, chunk, 1)
    key = (torch.arange(blocks) * chunk - past).view(blocks, 1, 1) + torch.arange(context)
    distance = query - key
    allowed = (distance >= 0) & (distance < past) & (key >= 0)
    if future:
        allowed |= (distance < 0) & (-distance < future)
    allowed = allowed & (key < lengths.view(-1, 1, 1, 1))
    return ~allowed[:, None]


def local_attention(q: Tensor, k: Tensor, v: Tensor, relative: Tensor, mask: Tensor, chunk: int, past: int,
                    future: int, softcap: float, invalid: float) -> Tensor:
    """The attention of ``AudioAttention.forward`` (``gemma4.py:256-282``) on
    scaled ``q``/``k``/``v`` ``(batch, frames, heads, head_dim)`` and the
    relative keys ``relative`` ``(positions, heads, head_dim)``; returns
    ``(batch, frames, heads, head_dim)``."""
    batch, frames, heads, head_dim = q.shape
    context = chunk + past + future
    blocks = mask.shape[2]

    def contexts(x: Tensor) -> Tensor:  # (batch, blocks, context, heads, head_dim)
        x = F.pad(x, (0, 0, 0, 0, past, future + chunk - 1))
        return torch.movedim(x.unfold(1, context, chunk), -1, 2)

    qb = F.pad(q, (0, 0, 0, 0, 0, blocks * chunk - frames))
    qb = qb.view(batch, blocks, chunk, heads, head_dim).permute(0, 3, 1, 2, 4)
    kb = contexts(k).permute(0, 3, 1, 4, 2)
    vb = contexts(v).permute(0, 3, 1, 2, 4)
    rel = relative.permute(1, 2, 0)  # (heads, head_dim, positions)

    content = qb @ kb
    position = qb.reshape(batch, heads, -1, head_dim) @ rel
    # Transformer-XL relative shift: rows padded to context + 1, flattened,
    # cut to chunk * context and viewed back.
    position = position.view(batch, heads, blocks, chunk, -1)
    position = F.pad(position, (0, context + 1 - position.shape[-1]))
    position = position.view(batch, heads, blocks, chunk * (context + 1))[..., : chunk * context]
    position = position.view(batch, heads, blocks, chunk, context)
    scores = torch.tanh((content + position) / softcap) * softcap
    scores = scores.masked_fill(mask, invalid)
    out = F.softmax(scores, dim=-1) @ vb
    out = out.permute(0, 2, 3, 1, 4).reshape(batch, blocks * chunk, heads, head_dim)
    return out[:, :frames]


def local_attention_loops(q: Tensor, k: Tensor, v: Tensor, relative: Tensor, lengths: Tensor, chunk: int,
                          past: int, future: int, softcap: float, invalid: float) -> Tensor:
    """The same attention from its definition, in float64 loops: query i of
    block u = i // chunk sees context slots t (key u chunk - past + t); the
    relative term of slot t is q . relative[t - i % chunk] when that row
    exists (relative row r belongs to distance past - r, and i - key = past -
    (t - i % chunk)); slots the mask hides score ``invalid``."""
    batch, frames, heads, head_dim = q.shape
    context = chunk + past + future
    out = torch.zeros(batch, frames, heads, head_dim, dtype=torch.float64)
    for b in range(batch):
        n = int(lengths[b])
        for i in range(frames):
            u, c = divmod(i, chunk)
            for h in range(heads):
                scores, values = [], []
                for t in range(context):
                    key = u * chunk - past + t
                    kv_ok = 0 <= key < frames
                    kk = k[b, key, h].double() if kv_ok else torch.zeros(head_dim, dtype=torch.float64)
                    vv = v[b, key, h].double() if kv_ok else torch.zeros(head_dim, dtype=torch.float64)
                    s = float(q[b, i, h].double() @ kk)
                    if 0 <= t - c < relative.shape[0]:
                        s += float(q[b, i, h].double() @ relative[t - c, h].double())
                    s = math.tanh(s / softcap) * softcap
                    d = i - key
                    allowed = (0 <= d < past) or (future > 0 and d < 0 and -d < future)
                    if not (allowed and 0 <= key < n):
                        s = invalid
                    scores.append(s)
                    values.append(vv)
                weights = torch.tensor(scores, dtype=torch.float64).softmax(0)
                out[b, i, h] = sum(w * vv for w, vv in zip(weights, values))
    return out


class TextAttention(nn.Module):
    """The language model's attention (``gemma4.py:486-587``): q/k/v RMS norms
    (v without weight), rotary embedding, no scaling, grouped-query SDPA
    with the prompt pass's or the step's mask."""

    def __init__(self, text: dict, layer_type: str, shared: bool) -> None:
        super().__init__()
        width = text["hidden_size"]
        eps = text["rms_norm_eps"]
        full = layer_type == "full_attention"
        self.head_dim = text["global_head_dim"] if full else text["head_dim"]
        self.heads = text["num_attention_heads"]
        self.kv_heads = text["num_key_value_heads"]
        self.window = None if full else text["sliding_window"]
        self.layer_type = layer_type
        self.shared = shared
        self.eps = eps
        self.q_norm = _Norm(self.head_dim, eps)
        if shared:
            self.q_proj = nn.Linear(width, self.heads * self.head_dim, bias=False)
        else:
            self.sizes = [size * self.head_dim for size in (self.heads, self.kv_heads, self.kv_heads)]
            self.qkv_proj = nn.Linear(width, sum(self.sizes), bias=False)
            self.k_norm = _Norm(self.head_dim, eps)
            self.v_norm = _Norm(self.head_dim, eps, scale=False)
        self.o_proj = nn.Linear(self.heads * self.head_dim, width, bias=False)

    def _project(self, x: Tensor, cos: Tensor, sin: Tensor):
        shape = (*x.shape[:-1], -1, self.head_dim)
        if self.shared:
            return rotate(self.q_norm(self.q_proj(x).view(shape)), cos, sin), None, None
        q, k, v = self.qkv_proj(x).split(self.sizes, dim=-1)
        q = rotate(self.q_norm(q.reshape(shape)), cos, sin)
        k = rotate(self.k_norm(k.reshape(shape)), cos, sin)
        return q, k, self.v_norm(v.reshape(shape))

    def prefill(self, x, cache_keys, cache_values, rows, kv, mask, cos, sin) -> Tensor:
        q, k, v = self._project(x, cos, sin)
        if self.shared:
            k, v = kv[self.layer_type]
        else:
            length = x.shape[1]
            cache_keys[rows, :length] = k
            cache_values[rows, :length] = v
            kv[self.layer_type] = k, v
        output = oa.sdpa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), attn_mask=mask, scale=1.0,
                         enable_gqa=True)
        return self.o_proj(output.transpose(1, 2).flatten(2))

    def step(self, x, cache_keys, cache_values, positions, mask, cos, sin) -> Tensor:
        q, k, v = self._project(x, cos, sin)
        if not self.shared:
            rows = torch.arange(len(x))
            cache_keys[rows, positions] = k
            cache_values[rows, positions] = v
        q = q.view(len(x), self.kv_heads, -1, self.head_dim)
        output = oa.sdpa(q, cache_keys.transpose(1, 2), cache_values.transpose(1, 2), attn_mask=mask, scale=1.0)
        return self.o_proj(output.reshape(len(x), -1))


class _Norm(nn.Module):
    """Gemma 4's RMS norm in float32 (``gemma4.py:166-180``); parameter name
    ``weight`` as the reference's."""

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


def rotate(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """``gemma4.py:440-445``."""
    first, second = x.chunk(2, dim=-1)
    return x * cos[..., None, :] + torch.cat((-second, first), dim=-1) * sin[..., None, :]

"""Qwen3-ASR's text attention and audio-window attention restated on the CPU
on the reference's SDPA fallback paths (``models/qwen3_asr.py:167-181``,
``:427-432``): packed prompts gathered into a padded batch with a
``valid & tril`` mask, and decoder steps with the query heads of a kv head
grouped as one query block over a ``(batch, 1, 1, length)`` mask.  Parameter
names match the reference's, so one state dict loads into this model and
into ``asrback_amd.qwen3_asr``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import attention as oa


class RMSNorm(nn.Module):
    def __init__(self, width: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(width))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        return oa.rms_norm(x, self.weight, self.eps)


class TextAttention(nn.Module):
    """``qwen3_asr.py:350-432`` on the padded path."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        width = config["hidden_size"]
        self.head_dim = config["head_dim"]
        self.heads = config["num_attention_heads"]
        self.kv_heads = config["num_key_value_heads"]
        self.sizes = [s * self.head_dim for s in (self.heads, self.kv_heads, self.kv_heads)]
        self.qkv_proj = nn.Linear(width, sum(self.sizes), bias=False)
        self.o_proj = nn.Linear(self.heads * self.head_dim, width, bias=False)
        self.q_norm = RMSNorm(self.head_dim, config["rms_norm_eps"])
        self.k_norm = RMSNorm(self.head_dim, config["rms_norm_eps"])

    def _project(self, x, cos, sin):
        shape = (len(x), -1, self.head_dim)
        q, k, v = self.qkv_proj(x).split(self.sizes, dim=-1)
        q = oa.rotate(self.q_norm(q.reshape(shape)), cos, sin)
        k = oa.rotate(self.k_norm(k.reshape(shape)), cos, sin)
        return q, k, v.reshape(shape)

    def prefill(self, x, keys, values, rows, positions, segments: oa.Segments, cos, sin):
        q, k, v = self._project(x, cos, sin)
        keys[rows, positions] = k
        values[rows, positions] = v
        return self.o_proj(oa.qwen_attend(q, k, v, segments, causal=True).flatten(1))

    def step(self, x, keys, values, positions, mask, cos, sin):
        q, k, v = self._project(x, cos, sin)
        rows = torch.arange(len(x))
        keys[rows, positions] = k
        values[rows, positions] = v
        return self.o_proj(oa.qwen_step_attention(q, keys, values, mask).reshape(len(x), -1))


class DecoderLayer(nn.Module):
    def __init__(self, config: dict) -> None:
        super().__init__()
        self.input_layernorm = RMSNorm(config["hidden_size"], config["rms_norm_eps"])
        self.self_attn = TextAttention(config)
        self.post_attention_layernorm = RMSNorm(config["hidden_size"], config["rms_norm_eps"])
        self.mlp = nn.Module()
        self.mlp.gate_up_proj = nn.Linear(config["hidden_size"], 2 * config["intermediate_size"], bias=False)
        self.mlp.down_proj = nn.Linear(config["intermediate_size"], config["hidden_size"], bias=False)

    def forward(self, x, attention):
        x = x + attention(self.self_attn, self.input_layernorm(x))
        gate, up = self.mlp.gate_up_proj(self.post_attention_layernorm(x)).chunk(2, dim=-1)
        return x + self.mlp.down_proj(F.silu(gate) * up)


class TextModel(nn.Module):
    """``qwen3_asr.py:463-524``; steps use the ``(batch, 1, 1, length)`` mask."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(config["vocab_size"], config["hidden_size"])
        self.layers = nn.ModuleList(DecoderLayer(config) for _ in range(config["num_hidden_layers"]))
        self.norm = RMSNorm(config["hidden_size"], config["rms_norm_eps"])

    def prefill(self, x, keys, values, rows, positions, segments, cos, sin):
        for index, layer in enumerate(self.layers):
            k, v = keys[index], values[index]
            x = layer(x, lambda att, h: att.prefill(h, k, v, rows, positions, segments, cos, sin))
        return self.norm(x)

    def step(self, tokens, positions, keys, values, cos, sin):
        x = self.embed_tokens(tokens)
        cos, sin = cos[positions], sin[positions]
        mask = oa.qwen_step_mask(positions, keys.shape[2])
        for index, layer in enumerate(self.layers):
            k, v = keys[index], values[index]
            x = layer(x, lambda att, h: att.step(h, k, v, positions, mask, cos, sin))
        return self.norm(x)


class AudioAttention(nn.Module):
    """``qwen3_asr.py:207-221`` on the padded path."""

    def __init__(self, width: int, heads: int) -> None:
        super().__init__()
        self.heads = heads
        self.q_proj = nn.Linear(width, width)
        self.k_proj = nn.Linear(width, width)
        self.v_proj = nn.Linear(width, width)
        self.out_proj = nn.Linear(width, width)

    def forward(self, x: Tensor, segments: oa.Segments) -> Tensor:
        q, k, v = (p(x).view(len(x), self.heads, -1) for p in (self.q_proj, self.k_proj, self.v_proj))
        return self.out_proj(oa.qwen_attend(q, k, v, segments, causal=False).flatten(1))

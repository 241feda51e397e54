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


def greedy_decode(model: TextModel, lm_head: Tensor, config: dict, prompt: list[int], max_new_tokens: int,
                  eos_ids: list[int], cache_length: int = 1024) -> dict:
    """The Qwen3-ASR transcriber's token loop for one window, greedy
    (``qwen3_asr.py:1017-1090``, ``:1179-1198``, ``:1131-1155``): the prompt
    pass picks the first token at position ``len(prompt)``; each step decodes
    the latest token at its position and picks the next; a window stops at an
    EOS id or when its position reaches ``len(prompt) - 1 + limit``, with
    ``limit = min(max_new_tokens, cache_length - len(prompt))``; a trailing EOS
    is dropped.  Returns the tokens and the smallest top-2 logit gap met (how
    far the argmaxes are from ties)."""
    n = len(prompt)
    end = n - 1 + min(max_new_tokens, cache_length - n)
    shape = (config["num_hidden_layers"], 1, cache_length, config["num_key_value_heads"], config["head_dim"])
    keys, values = torch.zeros(shape), torch.zeros(shape)
    cos, sin = oa.rope_tables(config["rope_theta"], config["head_dim"], cache_length, torch.float32)
    positions = torch.arange(n)
    gaps = []

    def pick(hidden: Tensor) -> int:
        logits = hidden @ lm_head.T
        top = torch.topk(logits, 2).values
        gaps.append(float(top[0] - top[1]))
        return int(logits.argmax())

    with torch.inference_mode():
        x = model.embed_tokens(torch.tensor(prompt))
        hidden = model.prefill(x, keys, values, torch.zeros(n, dtype=torch.long), positions,
                               oa.Segments.from_lengths([n]), cos[positions], sin[positions])
        token, position = pick(hidden[-1]), n
        tokens = [token]
        while token not in eos_ids and position < end:
            hidden = model.step(torch.tensor([token]), torch.tensor([position]), keys, values, cos, sin)
            token, position = pick(hidden[0]), position + 1
            tokens.append(token)
    if tokens[-1] in eos_ids:
        tokens.pop()
    return {"tokens": tokens, "min_gap": min(gaps)}

"""Qwen3-ASR's attention modules on the MI355X kernels.

Drop-in for the attention side of the reference's ``models/qwen3_asr.py``:
``Segments``/``attend`` (``:123-181``), ``AudioAttention`` (``:207-221``),
``RMSNorm``/``rotate`` (``:316-330``), ``KVCache`` (``:333-347``),
``TextAttention`` (``:350-432``) and ``TextModel`` (``:463-524``), with the
same names, parameter names and signatures, and the cache layout
``(layers, batch, length, kv_heads, head_dim)``; and the transcriber's
decode loop around them (``DecodeState``, ``choose``, ``TextGreedyDecoder``:
``:659-699``, ``:1017-1214``).

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
* :class:`PagedKVCache` replaces the fixed 1024-slot rows with pages from a
  shared pool and a block table (``TextGreedyDecoder(page_size=...)``):
  rows hold the pages their prompt and generation limit need.  Its layers
  index like the slab (``keys[rows, positions] = k``), so the attention
  modules take either cache.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import attention
from .attention import KeyPrefix, PageTable, decode, decode_append, greedy_choice, varlen_attn
from .transcription import CapturedGraph, to_device

# Positions per row of the KV cache (qwen3_asr.py:57-59).
CACHE_LENGTH = 1024
# Decoder steps between host checks for finished rows (qwen3_asr.py:56).
EOS_CHECK_INTERVAL = 4
# Default cap on generated tokens per window (qwen3_asr.py:63).
MAX_NEW_TOKENS = 512


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
    """``varlen_attn`` over packed ``(tokens, heads, head_dim)`` segments
    (``qwen3_asr.py:152-181``), grouped-query when ``k``/``v`` carry fewer
    heads than ``q``."""
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
    """RoPE in the half-split convention (``qwen3_asr.py:326-330``): ``x``
    ``(..., heads, head_dim)``, tables ``(..., head_dim)`` shared by the
    heads."""
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
    """The slab cache (``qwen3_asr.py:333-347``): one
    ``(layers, batch, length, kv_heads, head_dim)`` tensor each for keys and
    values, allocated once; every write is in place, so captured graphs keep
    valid addresses."""

    keys: Tensor
    values: Tensor

    @classmethod
    def allocate(cls, config: dict, batch: int, length: int, device, dtype) -> KVCache:
        shape = (config["num_hidden_layers"], batch, length, config["num_key_value_heads"], config["head_dim"])
        return cls(torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device))

    def narrow(self, batch_size: int, length: int) -> KVCache:
        return KVCache(self.keys[:, :batch_size, :length], self.values[:, :batch_size, :length])


class PagedLayer:
    """One layer's keys (or values) of a :class:`PagedKVCache`, addressed as
    the slab ``(batch, length, kv_heads, head_dim)`` would be: ``layer[rows,
    positions] = x`` writes each token to its row's page."""

    def __init__(self, pool: Tensor, table: PageTable, page_size: int) -> None:
        # (num_pages + 1, page_size, kv_heads, head_dim): the last page is a
        # sink that no table entry names.
        self.pool = pool
        self.table = table
        self.page_size = page_size
        self.dtype = pool.dtype
        self.device = pool.device
        batch, reach = table.block_table.shape[0], table.max_len
        self.shape = (batch, reach, pool.shape[2], pool.shape[3])

    def __setitem__(self, index: tuple[Tensor, Tensor], value: Tensor) -> None:
        rows, positions = index
        pages = self.table.block_table[rows, positions // self.page_size].long()
        # A row without a page there (-1: a free row of the bucket) writes to
        # the sink page, so it cannot land in a page another row owns; no
        # data-dependent shapes, so the write can be graph-captured.
        sink = self.pool.shape[0] - 1
        pages = torch.where((pages >= 0) & (pages < sink), pages, sink)
        self.pool[pages, positions % self.page_size] = value


@dataclass
class PagedKVCache:
    """Keys and values in pages of ``page_size`` positions from one pool per
    layer, ``(layers, num_pages + 1, page_size, kv_heads, head_dim)`` (the
    last page a write sink that no row owns), and a block
    table ``(batch, CACHE_LENGTH / page_size)`` (int32, on the device; -1 for
    no page) mapping each row's logical pages to pool pages.  Generalizes the
    reference's ``row * 1024`` slab (``qwen3_asr.py:511-512``): a row holds
    only the pages its keys need, so the pool -- not ``CACHE_LENGTH`` times
    the batch -- bounds how many rows fit.  Pages are handed out on the host
    (:meth:`assign`, :meth:`release`); the tensors keep fixed addresses."""

    pool_keys: Tensor
    pool_values: Tensor
    block_table: Tensor
    page_size: int
    free_pages: list[int]

    @classmethod
    def allocate(cls, config: dict, batch: int, num_pages: int, page_size: int, device, dtype) -> PagedKVCache:
        if CACHE_LENGTH % page_size:
            raise ValueError(f"page_size must divide {CACHE_LENGTH}")
        # One page more than the table hands out: the sink of PagedLayer.
        shape = (config["num_hidden_layers"], num_pages + 1, page_size, config["num_key_value_heads"],
                 config["head_dim"])
        table = torch.full((batch, CACHE_LENGTH // page_size), -1, dtype=torch.int32, device=device)
        return cls(torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device),
                   table, page_size, list(range(num_pages - 1, -1, -1)))

    def __post_init__(self) -> None:
        # Per layer, indexed like KVCache.keys / .values.
        table = PageTable(self.block_table, CACHE_LENGTH)
        self.keys = [PagedLayer(pool, table, self.page_size) for pool in self.pool_keys]
        self.values = [PagedLayer(pool, table, self.page_size) for pool in self.pool_values]

    def narrow(self, batch_size: int, length: int) -> PagedKVCache:
        del length  # every row reads only its own pages
        return PagedKVCache(self.pool_keys, self.pool_values, self.block_table[:batch_size], self.page_size,
                            self.free_pages)

    def pages_for(self, positions: int) -> int:
        return -(-positions // self.page_size)

    def assign(self, row: int, positions: int) -> list[int]:
        """Pages for positions ``0 .. positions - 1`` of ``row`` (whose
        previous pages must have been released)."""
        count = self.pages_for(positions)
        if count > len(self.free_pages):
            raise RuntimeError(f"paged cache exhausted: {count} pages wanted, {len(self.free_pages)} free")
        pages = [self.free_pages.pop() for _ in range(count)]
        entries = torch.full((self.block_table.shape[1],), -1, dtype=torch.int32)
        entries[:count] = torch.tensor(pages, dtype=torch.int32)
        self.block_table[row].copy_(entries.to(self.block_table.device))
        return pages

    def release(self, row: int, pages: list[int]) -> None:
        self.block_table[row].fill_(-1)
        self.free_pages.extend(reversed(pages))


def _cache_layer(layer) -> tuple[Tensor, PageTable | None]:
    """The tensor the kernels read for one layer's keys or values, and its
    page table (None for the slab)."""
    if isinstance(layer, PagedLayer):
        return layer.pool, layer.table
    return layer, None


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
        """The prompt pass (``:374-390``): keys and values of the packed
        prompts are stored at (row, position) in the cache, then each prompt
        attends causally within itself."""
        q, k, v = self._project(x, cos, sin)
        keys[rows, positions] = k
        values[rows, positions] = v
        return self.o_proj(attend(q, k, v, segments, causal=True).flatten(1))

    def _fused_step(self, x: Tensor, keys: Tensor) -> bool:
        return (
            x.dtype in (torch.float32, torch.bfloat16)
            and self.head_dim in (64, 128)
            and self.heads // self.kv_heads in (1, 2, 4)
            and keys.dtype == x.dtype
        )

    def step(self, x, keys, values, positions, mask, cos, sin) -> Tensor:
        """One token per row at its own position, attending over the cache
        view ``keys``/``values`` ``(batch, length, kv_heads, head_dim)``
        (``:392-432``).  With the step mask built on these positions (a
        :class:`KeyPrefix` of ``positions``, as :meth:`TextModel.step`
        passes), the norms, the rotation, the cache write and the attention
        run as one kernel (:func:`~asrback_amd.attention.decode_append`);
        other mask forms take the reference's sequence of ops."""
        key_cache, pages = _cache_layer(keys)
        value_cache, _ = _cache_layer(values)
        if isinstance(mask, KeyPrefix) and mask.positions is positions and self._fused_step(x, key_cache):
            batch = len(x)
            q, k, v = self.qkv_proj(x).split(self.sizes, dim=-1)
            output = decode_append(
                q.view(batch, self.heads, self.head_dim),
                k.view(batch, self.kv_heads, self.head_dim),
                v.view(batch, self.kv_heads, self.head_dim),
                key_cache, value_cache, positions,
                q_norm=self.q_norm.weight, k_norm=self.k_norm.weight, eps=self.q_norm.eps,
                cos=cos, sin=sin, pages=pages,
            )
            return self.o_proj(output.flatten(1))
        q, k, v = self._project(x, cos, sin)
        rows = torch.arange(len(x), device=x.device)
        keys[rows, positions] = k
        values[rows, positions] = v
        lengths = _step_lengths(mask, positions, keys.shape[1])
        output = decode(q, key_cache, value_cache, seqused_k=lengths, pages=pages)
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
        mask = KeyPrefix(positions=positions)
        for index, layer in enumerate(self.layers):
            keys, values = cache.keys[index], cache.values[index]
            x = layer(x, lambda attention, h: attention.step(h, keys, values, positions, mask, cos, sin))
        return self.norm(x)


@dataclass
class DecodeState:
    """Per-row decoding state updated in place by every step
    (``qwen3_asr.py:659-699``).  ``position`` is each row's position of its
    latest token; a step writes the next token to ``generated`` at
    ``position + 1``.  Finished rows, and free rows (marked finished), keep
    their token and position."""

    tokens: Tensor  # (batch,)
    position: Tensor  # (batch,)
    end: Tensor  # (batch,): each row's final writable position
    finished: Tensor  # (batch,)
    sum_logprobs: Tensor  # (batch,)
    generated: Tensor  # (batch, CACHE_LENGTH)

    @classmethod
    def allocate(cls, batch_size: int, device: torch.device) -> DecodeState:
        return cls(
            torch.zeros(batch_size, dtype=torch.long, device=device),
            torch.zeros(batch_size, dtype=torch.long, device=device),
            torch.zeros(batch_size, dtype=torch.long, device=device),
            torch.ones(batch_size, dtype=torch.bool, device=device),
            torch.zeros(batch_size, device=device),
            torch.zeros((batch_size, CACHE_LENGTH), dtype=torch.long, device=device),
        )

    def narrow(self, batch_size: int) -> DecodeState:
        return DecodeState(*(t[:batch_size] for t in (
            self.tokens, self.position, self.end, self.finished, self.sum_logprobs, self.generated
        )))

    def free(self, rows: Tensor) -> None:
        """Return ``rows`` to the pool of free slots (finished, back at
        position 0)."""
        self.finished[rows] = True
        self.position[rows] = 0
        self.tokens[rows] = 0


def choose(logits: Tensor, temperatures: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """Next token per row -- greedy, or sampled where the row's temperature is
    positive -- and its log-probability (``qwen3_asr.py:1200-1210``).  All
    greedy over fp32 logits on the GPU: one fused pass
    (:func:`~asrback_amd.attention.greedy_choice`)."""
    if temperatures is None and logits.is_cuda and logits.dtype == torch.float32 and logits.dim() == 2:
        return greedy_choice(logits)
    token = logits.argmax(dim=-1)
    if temperatures is not None:
        scaled = logits / temperatures.clamp(min=1e-6)[:, None]
        sampled = torch.multinomial(F.softmax(scaled, dim=-1), 1).squeeze(1)
        token = torch.where(temperatures > 0, sampled, token)
    logprob = F.log_softmax(logits, dim=-1).gather(1, token[:, None]).squeeze(1)
    return token, logprob


class TextGreedyDecoder:
    """Decoding of Qwen3-ASR windows in a pool of ``max_batch_size`` cache
    rows, the step replayed from a HIP graph per batch bucket.

    Restates the decode path of the reference's ``Qwen3ASRTranscriber``
    without its request queue, audio encoder and tokenizer: :meth:`admit`
    runs prompts packed back to back straight into free rows and picks their
    first tokens (``_admit``, ``qwen3_asr.py:1017-1090``), :meth:`step` is
    ``_step`` (``:1179-1198``), :meth:`advance` runs up to
    ``EOS_CHECK_INTERVAL`` steps from the graphs (``_advance``,
    ``:1101-1128``; graphs as ``_capture_graphs``, ``:930-948``) and
    :meth:`finished_rows` returns and frees finished rows (``_finish``,
    ``:1131-1155``).  Attention reads each row's own keys, so one KV bucket
    (the whole 1024-position slab) serves every length, as with the
    reference's varlen path.  With ``page_size`` the cache is a
    :class:`PagedKVCache` of ``num_pages`` pages (default: as many
    positions as the slab): a row holds the pages for its prompt and its
    generation limit from admission until it finishes.
    """

    def __init__(self, text: TextModel, lm_head: nn.Module, config: dict, max_batch_size: int,
                 eos_ids: list[int], graphs: bool = True, page_size: int | None = None,
                 num_pages: int | None = None) -> None:
        self.text = text
        self.lm_head = lm_head
        self.config = config
        weight = text.embed_tokens.weight
        self.device, self.dtype = weight.device, weight.dtype
        self.max_batch_size = max_batch_size
        self.cos, self.sin = rope_tables(config, CACHE_LENGTH, self.device, self.dtype)
        self.buckets = sorted(
            {min(2**p, max_batch_size) for p in range(max_batch_size.bit_length())} | {max_batch_size}
        )
        self.kv_buckets = [CACHE_LENGTH]
        if page_size is None:
            self.cache = KVCache.allocate(config, max_batch_size, CACHE_LENGTH, self.device, self.dtype)
        else:
            pages = max_batch_size * CACHE_LENGTH // page_size if num_pages is None else num_pages
            self.cache = PagedKVCache.allocate(config, max_batch_size, pages, page_size, self.device, self.dtype)
        self.state = DecodeState.allocate(max_batch_size, self.device)
        self.eos_ids = torch.tensor(eos_ids, dtype=torch.long, device=self.device)
        self.workspace = torch.empty(self._workspace_bytes(), dtype=torch.uint8, device=self.device)
        self.rows: dict[int, dict] = {}
        self.graphs: dict[tuple[int, int], CapturedGraph] = {}
        if graphs:
            self._capture_graphs()

    def _workspace_bytes(self) -> int:
        """Split partials of the largest step over the buckets: the decode
        launch per layer and the greedy choice over the logits."""
        config = self.config
        vocab = self.lm_head.weight.shape[0]
        need = 256
        for batch in self.buckets:
            for length in self.kv_buckets:
                need = max(need, attention.decode_workspace_size(
                    batch, config["num_attention_heads"], config["num_key_value_heads"], config["head_dim"],
                    length, self.dtype))
            need = max(need, attention.choice_workspace_size(batch, vocab))
        return need

    @torch.inference_mode()
    def _capture_graphs(self) -> None:
        """One greedy step per (batch bucket, KV bucket); warm-up steps advance
        the rows, so they start inside the cache."""
        pool = torch.cuda.graph_pool_handle()
        for batch_size in self.buckets:
            state = self.state.narrow(batch_size)
            for length in self.kv_buckets:
                cache = self.cache.narrow(batch_size, length)
                state.finished.zero_()
                state.position.zero_()
                state.end.fill_(CACHE_LENGTH - 1)
                self.graphs[batch_size, length] = CapturedGraph(
                    lambda state=state, cache=cache: self.step(state, cache), pool
                )
        self.state.free(torch.arange(self.max_batch_size, device=self.device))

    def logits(self, hidden: Tensor) -> Tensor:
        return self.lm_head(hidden).float()

    @torch.inference_mode()
    def admit(self, prompts: list[list[int]], max_new_tokens: int | list[int] = MAX_NEW_TOKENS,
              embeddings: Tensor | None = None, audio_id: int | None = None,
              temperatures: Tensor | None = None) -> list[int]:
        """Prompt pass for new windows, packed back to back into free cache
        rows, and their first tokens; returns their slots.  ``embeddings``
        (one row per ``audio_id`` token of the packed prompts, in order)
        replace those tokens' embeddings, as the audio encoder's output does."""
        count = len(prompts)
        slots = [s for s in range(self.max_batch_size) if s not in self.rows][:count]
        if len(slots) < count:
            raise RuntimeError("no free rows")
        if isinstance(max_new_tokens, int):
            max_new_tokens = [max_new_tokens] * count
        lengths = [len(prompt) for prompt in prompts]
        if min(lengths) < 1 or max(lengths) >= CACHE_LENGTH:
            raise ValueError(f"prompt lengths must lie in [1, {CACHE_LENGTH})")
        ids = np.concatenate([np.asarray(prompt, dtype=np.int64) for prompt in prompts])
        offsets = np.cumsum(lengths) - lengths
        positions = np.arange(len(ids)) - np.repeat(offsets, lengths)
        limits = [min(n, CACHE_LENGTH - length) for n, length in zip(max_new_tokens, lengths)]
        ends = [length - 1 + limit for length, limit in zip(lengths, limits)]
        audio = np.flatnonzero(ids == audio_id) if audio_id is not None else None
        if isinstance(self.cache, PagedKVCache):
            wanted = sum(self.cache.pages_for(end + 1) for end in ends)
            if wanted > len(self.cache.free_pages):
                raise RuntimeError(f"paged cache exhausted: {wanted} pages wanted, {len(self.cache.free_pages)} free")
            held = [self.cache.assign(slot, end + 1) for slot, end in zip(slots, ends)]
        else:
            held = [[] for _ in slots]
        ids_d, rows, positions_d, slot_rows, start, end = (
            to_device(data, self.device)
            for data in (ids, np.repeat(slots, lengths), positions, slots, lengths, ends)
        )
        x = self.text.embed_tokens(ids_d)
        if embeddings is not None:
            x[to_device(audio, self.device)] = embeddings.to(x.dtype)
        segments = Segments.from_lengths(lengths, self.device)
        hidden = self.text.prefill(x, self.cache, rows, positions_d, segments,
                                   self.cos[positions_d], self.sin[positions_d])
        last = segments.starts[1:].long() - 1
        with attention.workspace(self.workspace):
            token, logprob = choose(self.logits(hidden[last]), temperatures)
        state = self.state
        state.tokens[slot_rows] = token
        state.position[slot_rows] = start
        state.end[slot_rows] = end
        state.finished[slot_rows] = torch.isin(token, self.eos_ids) | (start >= end)
        state.sum_logprobs[slot_rows] = logprob
        state.generated[slot_rows, start] = token
        for slot, length, end_position, pages in zip(slots, lengths, ends, held):
            self.rows[slot] = {"prompt_length": length, "end": end_position, "bound": length, "pages": pages}
        return slots

    def step(self, state: DecodeState, cache: KVCache, temperatures: Tensor | None = None) -> None:
        """Decode ``state.tokens`` and select every row's next token
        (``qwen3_asr.py:1179-1198``).  Split partials go to the decoder's
        own workspace, sized at construction for the largest bucket."""
        with attention.workspace(self.workspace):
            hidden = self.text.step(state.tokens, state.position, cache, self.cos, self.sin)
            token, logprob = choose(self.logits(hidden), temperatures)
        active = ~state.finished
        position = state.position + active
        token = torch.where(active, token, state.tokens)
        state.sum_logprobs.add_(logprob.masked_fill(state.finished, 0.0))
        state.generated.scatter_(1, position[:, None], token[:, None])
        state.finished.logical_or_(torch.isin(token, self.eos_ids) | (position >= state.end))
        state.position.copy_(position)
        state.tokens.copy_(token)

    @torch.inference_mode()
    def advance(self, temperatures: Tensor | None = None) -> int:
        """Up to ``EOS_CHECK_INTERVAL`` steps over the occupied rows, from the
        graph of the smallest covering batch bucket when every row is greedy;
        returns the count."""
        bucket = next(size for size in self.buckets if size > max(self.rows))
        rows = self.rows.values()
        count = max(1, min(EOS_CHECK_INTERVAL, max(r["end"] - r["bound"] for r in rows)))
        length = max(min(r["bound"] + count, r["end"]) for r in rows) + 1
        kv_bucket = next(size for size in self.kv_buckets if size >= length)
        if self.graphs and temperatures is None:
            graph = self.graphs[bucket, kv_bucket]
            for _ in range(count):
                graph.replay()
        else:
            state = self.state.narrow(bucket)
            cache = self.cache.narrow(bucket, kv_bucket)
            for _ in range(count):
                self.step(state, cache, temperatures)
        for r in rows:
            r["bound"] = min(r["bound"] + count, r["end"])
        return count

    @torch.inference_mode()
    def finished_rows(self) -> dict[int, tuple[list[int], float]]:
        """Generated tokens and mean log-probability of the rows that finished,
        which are freed (``qwen3_asr.py:1131-1155``; a trailing EOS is
        dropped)."""
        finished = self.state.finished[: max(self.rows) + 1].tolist()
        done = [slot for slot in self.rows if finished[slot]]
        if not done:
            return {}
        rows = torch.tensor(done, device=self.device)
        positions = self.state.position[rows].tolist()
        sums = self.state.sum_logprobs[rows].tolist()
        generated = self.state.generated[rows, : max(positions) + 1].tolist()
        self.state.free(rows)
        eos = set(self.eos_ids.tolist())
        out = {}
        for slot, position, total, tokens in zip(done, positions, sums, generated):
            row = self.rows.pop(slot)
            if isinstance(self.cache, PagedKVCache):
                self.cache.release(slot, row["pages"])
            tokens = tokens[row["prompt_length"] : position + 1]
            if tokens and tokens[-1] in eos:
                tokens.pop()
            out[slot] = (tokens, total / (len(tokens) + 1))
        return out

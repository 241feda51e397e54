"""Whisper's attention modules on the MI355X kernels.

Drop-in for the network classes of the reference's ``models/whisper.py``
(``:73-342``): same class names, parameter names (so Hugging Face state dicts
load unchanged), method signatures and cache layout
``(layers, batch, heads, length, head_dim)``.  What changes is underneath:

* ``MultiHeadAttention.attend`` calls :func:`asrback_amd.attention.sdpa`
  (the HIP kernels) instead of ``F.scaled_dot_product_attention``, and gets
  the output already in ``(batch, length, heads, head_dim)`` order, so the
  reference's transpose copy before ``out_proj`` disappears.
* ``WhisperDecoder.forward`` passes the step's key mask as a
  :class:`~asrback_amd.attention.KeyPrefix` over the device-resident
  ``positions`` instead of materializing the boolean ``(batch, 1, 1,
  length)`` mask (``whisper.py:263-264``); a boolean mask passed by a caller
  still works.  There is no SDPA backend priority to set.

The greedy decoding machinery of the reference's ``Transcriber``
(``whisper.py:402-448``, ``:710-726``, ``:828-974``) is restated by
:class:`GreedyDecoder`, with the decoder step captured in a HIP graph
(``torch.cuda.CUDAGraph`` is hipGraph on ROCm).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import attention
from .attention import KeyPrefix, decode_append, greedy_choice, sdpa
from .transcription import CapturedGraph, to_device

# Key buckets of the graphed decoder step; max_target_positions is the last
# one (whisper.py:54).
KV_BUCKETS = (64, 128, 256)
# Decoder steps between host checks for finished rows (whisper.py:52).
EOS_CHECK_INTERVAL = 4


class MultiHeadAttention(nn.Module):
    """``whisper.py:73-110``; ``k_proj`` has no bias."""

    def __init__(self, width: int, heads: int) -> None:
        super().__init__()
        if width % heads:
            raise ValueError(f"d_model ({width}) must be divisible by heads ({heads})")
        self.heads = heads
        self.head_dim = width // heads
        self.k_proj = nn.Linear(width, width, bias=False)
        self.v_proj = nn.Linear(width, width)
        self.q_proj = nn.Linear(width, width)
        self.out_proj = nn.Linear(width, width)

    def _split_heads(self, x: Tensor) -> Tensor:
        batch, length, width = x.shape
        return x.view(batch, length, self.heads, width // self.heads).transpose(1, 2)

    def project_key_value(self, x: Tensor) -> tuple[Tensor, Tensor]:
        """Keys and values of ``x`` as ``(batch, heads, length, head_dim)``
        views of the projections (no copy)."""
        return self._split_heads(self.k_proj(x)), self._split_heads(self.v_proj(x))

    def step(self, x: Tensor, key: Tensor, value: Tensor, keys: Tensor, values: Tensor, positions: Tensor) -> Tensor:
        """One query token per row (``x`` ``(batch, 1, width)``) whose own key
        and value (``(batch, heads, 1, head_dim)``) go into the self-attention
        cache ``keys``/``values`` ``(batch, heads, length, head_dim)`` at
        ``positions`` before the row attends keys ``0 .. positions[b]``: the
        reference's ``scatter_`` pair and masked SDPA (``whisper.py:224-237``)
        as one ``decode_append`` launch."""
        query = self._split_heads(self.q_proj(x))[:, :, 0]
        output = decode_append(query, key[:, :, 0], value[:, :, 0], keys.transpose(1, 2), values.transpose(1, 2),
                               positions)
        return self.out_proj(output.reshape(x.shape[0], 1, -1))

    def attend(
        self,
        x: Tensor,
        key: Tensor,
        value: Tensor,
        mask: KeyPrefix | Tensor | None = None,
        is_causal: bool = False,
    ) -> Tensor:
        query = self._split_heads(self.q_proj(x))
        output = sdpa(query, key, value, mask, is_causal)  # (batch, length, heads, head_dim)
        return self.out_proj(output.reshape(x.shape[0], x.shape[1], -1))

    def forward(self, x: Tensor) -> Tensor:
        """Self-attention of ``x`` over itself, no mask (the encoder's)."""
        return self.attend(x, *self.project_key_value(x))


class EncoderLayer(nn.Module):
    """``whisper.py:113-125``."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        width = config["d_model"]
        self.self_attn = MultiHeadAttention(width, config["encoder_attention_heads"])
        self.self_attn_layer_norm = nn.LayerNorm(width)
        self.fc1 = nn.Linear(width, config["encoder_ffn_dim"])
        self.fc2 = nn.Linear(config["encoder_ffn_dim"], width)
        self.final_layer_norm = nn.LayerNorm(width)

    def forward(self, x: Tensor) -> Tensor:
        x = x + self.self_attn(self.self_attn_layer_norm(x))
        return x + self.fc2(F.gelu(self.fc1(self.final_layer_norm(x))))


class WhisperEncoder(nn.Module):
    """``whisper.py:128-153``: two convolutions, positions, the layers."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        width = config["d_model"]
        self.conv1 = nn.Conv1d(config["num_mel_bins"], width, 3, padding=1)
        self.conv2 = nn.Conv1d(width, width, 3, stride=2, padding=1)
        self.embed_positions = nn.Embedding(config["max_source_positions"], width)
        self.layers = nn.ModuleList(EncoderLayer(config) for _ in range(config["encoder_layers"]))
        self.layer_norm = nn.LayerNorm(width)

    def forward(self, mel: Tensor) -> Tensor:
        x = F.gelu(self.conv1(mel))
        x = F.gelu(self.conv2(x)).transpose(1, 2).contiguous()
        if x.shape[1] != self.embed_positions.num_embeddings:
            raise ValueError(
                f"expected {self.embed_positions.num_embeddings * 2} mel frames, got {mel.shape[-1]}"
            )
        x = x + self.embed_positions.weight
        for layer in self.layers:
            x = layer(x)
        return self.layer_norm(x)


@dataclass
class DecoderCache:
    """Self- and cross-attention caches, ``(layers, batch, heads, length,
    head_dim)`` each (``whisper.py:156-196``), allocated once and updated in
    place so that captured graphs keep valid addresses."""

    self_keys: Tensor
    self_values: Tensor
    cross_keys: Tensor
    cross_values: Tensor

    @property
    def batch_size(self) -> int:
        return self.self_keys.shape[1]

    def narrow(self, batch_size: int, length: int | None = None) -> DecoderCache:
        return self.rows(0, batch_size, length)

    def rows(self, start: int, stop: int, length: int | None = None) -> DecoderCache:
        return DecoderCache(
            self.self_keys[:, start:stop, :, :length],
            self.self_values[:, start:stop, :, :length],
            self.cross_keys[:, start:stop],
            self.cross_values[:, start:stop],
        )

    def copy_rows(self, source: DecoderCache, rows: Tensor, length: int) -> None:
        for target, values in (
            (self.self_keys[:, :, :, :length], source.self_keys[:, :, :, :length]),
            (self.self_values[:, :, :, :length], source.self_values[:, :, :, :length]),
            (self.cross_keys, source.cross_keys),
            (self.cross_values, source.cross_values),
        ):
            target.index_copy_(1, rows, values)


class DecoderLayer(nn.Module):
    """``whisper.py:199-241``.  ``fused_step`` (on by default): the graphed
    step writes the new key and value in its attention launch; off, it runs
    the reference's two ``scatter_`` writes before the attention (the same
    results; kept for comparisons)."""

    fused_step = True

    def __init__(self, config: dict) -> None:
        super().__init__()
        width = config["d_model"]
        heads = config["decoder_attention_heads"]
        self.self_attn = MultiHeadAttention(width, heads)
        self.self_attn_layer_norm = nn.LayerNorm(width)
        self.encoder_attn = MultiHeadAttention(width, heads)
        self.encoder_attn_layer_norm = nn.LayerNorm(width)
        self.fc1 = nn.Linear(width, config["decoder_ffn_dim"])
        self.fc2 = nn.Linear(config["decoder_ffn_dim"], width)
        self.final_layer_norm = nn.LayerNorm(width)

    def forward(
        self,
        x: Tensor,
        cache: tuple[Tensor, Tensor, Tensor, Tensor],
        positions: Tensor,
        length: int | None,
        mask: KeyPrefix | Tensor | None,
    ) -> Tensor:
        self_keys, self_values, cross_keys, cross_values = cache
        hidden = self.self_attn_layer_norm(x)
        key, value = self.self_attn.project_key_value(hidden)
        if self.fused_step and length is None and isinstance(mask, KeyPrefix) and mask.positions is positions:
            # The graphed step (one token per row, rows at different
            # positions, each seeing keys up to its own): cache write and
            # attention in one launch.
            x = x + self.self_attn.step(hidden, key, value, self_keys, self_values, positions)
        else:
            if length is None:
                # Per-row positions with another mask form: write each row's
                # token at its own position, then attend as the mask says.
                index = positions[:, None, None, None].expand_as(key)
                self_keys.scatter_(2, index, key)
                self_values.scatter_(2, index, value)
            else:
                # Prompt pass: every row writes the same positions and attends
                # causally over the prefix written so far.
                self_keys.index_copy_(2, positions, key)
                self_values.index_copy_(2, positions, value)
                self_keys = self_keys[:, :, :length]
                self_values = self_values[:, :, :length]
            x = x + self.self_attn.attend(hidden, self_keys, self_values, mask=mask, is_causal=x.shape[1] > 1)
        hidden = self.encoder_attn_layer_norm(x)
        x = x + self.encoder_attn.attend(hidden, cross_keys, cross_values)
        return x + self.fc2(F.gelu(self.fc1(self.final_layer_norm(x))))


class WhisperDecoder(nn.Module):
    """``whisper.py:244-277``."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        width = config["d_model"]
        self.embed_tokens = nn.Embedding(config["vocab_size"], width)
        self.embed_positions = nn.Embedding(config["max_target_positions"], width)
        self.layers = nn.ModuleList(DecoderLayer(config) for _ in range(config["decoder_layers"]))
        self.layer_norm = nn.LayerNorm(width)

    def forward(self, tokens: Tensor, positions: Tensor, cache: DecoderCache, length: int | None) -> Tensor:
        mask = None
        if length is None:
            # Graphed step over the bucket's cache view: row b is at
            # positions[b] and sees keys 0 .. positions[b] (read on the device).
            x = self.embed_tokens(tokens) + self.embed_positions(positions)[:, None]
            mask = KeyPrefix(positions=positions)
        else:
            x = self.embed_tokens(tokens) + self.embed_positions(positions)
        for index, layer in enumerate(self.layers):
            layer_cache = (
                cache.self_keys[index],
                cache.self_values[index],
                cache.cross_keys[index],
                cache.cross_values[index],
            )
            x = layer(x, layer_cache, positions, length, mask)
        return self.layer_norm(x)


class WhisperModel(nn.Module):
    def __init__(self, config: dict) -> None:
        super().__init__()
        self.encoder = WhisperEncoder(config)
        self.decoder = WhisperDecoder(config)


class WhisperForConditionalGeneration(nn.Module):
    """``whisper.py:287-342``."""

    def __init__(self, config: dict) -> None:
        super().__init__()
        self.config = config
        self.model = WhisperModel(config)

    def allocate_cache(self, batch_size: int) -> DecoderCache:
        config = self.config
        weight = self.model.decoder.embed_tokens.weight
        heads = config["decoder_attention_heads"]

        def empty(length: int) -> Tensor:
            size = (config["decoder_layers"], batch_size, heads, length, config["d_model"] // heads)
            return torch.zeros(size, dtype=weight.dtype, device=weight.device)

        target = config["max_target_positions"]
        source = config["max_source_positions"]
        return DecoderCache(empty(target), empty(target), empty(source), empty(source))

    def set_encoder_output(self, cache: DecoderCache, encoder_output: Tensor) -> None:
        batch_size = encoder_output.shape[0]
        for index, layer in enumerate(self.model.decoder.layers):
            key, value = layer.encoder_attn.project_key_value(encoder_output)
            cache.cross_keys[index, :batch_size] = key
            cache.cross_values[index, :batch_size] = value

    def decode(self, tokens: Tensor, positions: Tensor, cache: DecoderCache, length: int | None = None) -> Tensor:
        return self.model.decoder(tokens, positions, cache, length)

    def logits(self, hidden: Tensor) -> Tensor:
        weight = self.model.decoder.embed_tokens.weight
        rows = hidden.flatten(0, -2)
        return (weight @ rows.T).T.unflatten(0, hidden.shape[:-1])


@dataclass
class DecodeState:
    """Per-row decoding state updated in place by every step
    (``whisper.py:401-447``).  ``position`` is each row's position of
    ``tokens``; a step writes the next token to ``generated`` at
    ``position + 1``.  Finished and free rows keep their token and position."""

    tokens: Tensor  # (batch, 1)
    position: Tensor  # (batch,)
    end: Tensor  # (batch,)
    finished: Tensor  # (batch,)
    sum_logprobs: Tensor  # (batch,)
    generated: Tensor  # (batch, max_target_positions)

    @classmethod
    def allocate(cls, batch_size: int, max_target: int, device: torch.device) -> DecodeState:
        return cls(
            torch.zeros((batch_size, 1), dtype=torch.long, device=device),
            torch.zeros(batch_size, dtype=torch.long, device=device),
            torch.zeros(batch_size, dtype=torch.long, device=device),
            torch.ones(batch_size, dtype=torch.bool, device=device),
            torch.zeros(batch_size, device=device),
            torch.zeros((batch_size, max_target), dtype=torch.long, device=device),
        )

    def narrow(self, batch_size: int) -> DecodeState:
        return DecodeState(*(t[:batch_size] for t in (
            self.tokens, self.position, self.end, self.finished, self.sum_logprobs, self.generated
        )))

    def free(self, rows: Tensor) -> None:
        self.finished[rows] = True
        self.position[rows] = 0
        self.tokens[rows] = 0


def choose(logits: Tensor, suppress: Tensor, temperatures: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """Next token per row -- greedy, or sampled where the row's temperature is
    positive -- and its log-probability (``whisper.py:962-974``).  All greedy
    over fp32 logits on the GPU: one fused pass
    (:func:`~asrback_amd.attention.greedy_choice`; ``logits`` stays
    unmodified).  Otherwise the reference's ops, suppressed tokens filled
    with -inf in ``logits`` as the reference does."""
    if (temperatures is None and logits.is_cuda and logits.dtype == torch.float32 and logits.dim() == 2
            and suppress.dim() == 1):
        return greedy_choice(logits, suppress)
    logits.masked_fill_(suppress, -math.inf)
    token = logits.argmax(dim=-1)
    if temperatures is not None:
        scaled = logits / temperatures.clamp(min=1e-6)[:, None]
        sampled = torch.multinomial(F.softmax(scaled, dim=-1), 1).squeeze(1)
        token = torch.where(temperatures > 0, sampled, token)
    logprob = F.log_softmax(logits, dim=-1).gather(1, token[:, None]).squeeze(1)
    return token, logprob


class GreedyDecoder:
    """Greedy decoding of Whisper windows in a pool of ``max_batch_size`` rows,
    the decoder step replayed from a HIP graph per (batch bucket, KV bucket).

    Restates the decode path of the reference's ``Transcriber`` without its
    request queue and tokenizer: :meth:`detect_languages` picks a language
    token per window (``_detect_languages``, ``whisper.py:976-984``),
    :meth:`admit` runs the prompts (``_prefill``, ``:828-878``, with the
    first token's temperatures and the no-speech probability),
    :meth:`advance` runs up to ``EOS_CHECK_INTERVAL`` steps (``:887-915``),
    :meth:`finished_rows` returns finished rows' tokens (``:917-940``).
    Token ids come from the caller (the tokenizer stays outside).
    """

    def __init__(
        self,
        model: WhisperForConditionalGeneration,
        max_batch_size: int,
        suppress: Tensor,
        first_suppress: Tensor,
        eos: int,
        graphs: bool = True,
    ) -> None:
        self.model = model
        self.config = model.config
        self.device = model.model.decoder.embed_tokens.weight.device
        self.max_batch_size = max_batch_size
        self.eos = eos
        self._suppress = suppress.to(self.device)
        self._first_suppress = first_suppress.to(self.device)
        max_target = self.config["max_target_positions"]
        self._positions = torch.arange(max_target, device=self.device)
        self.buckets = sorted(
            {min(2**p, max_batch_size) for p in range(max_batch_size.bit_length())} | {max_batch_size}
        )
        self.kv_buckets = sorted({s for s in KV_BUCKETS if s < max_target} | {max_target})
        self.cache = model.allocate_cache(max_batch_size)
        self.staging = model.allocate_cache(max_batch_size)
        self.state = DecodeState.allocate(max_batch_size, max_target, self.device)
        # Per row: the prompt pass's no-speech probability (admit's no_speech_id).
        self.no_speech = torch.zeros(max_batch_size, dtype=torch.float32, device=self.device)
        self.workspace = torch.empty(self._workspace_bytes(), dtype=torch.uint8, device=self.device)
        self.rows: dict[int, dict] = {}
        self.graphs: dict[tuple[int, int], CapturedGraph] = {}
        if graphs:
            self._capture_graphs()

    def _workspace_bytes(self) -> int:
        """Split partials of the largest step over the buckets: each layer's
        self-attention over its KV bucket and cross-attention over the
        encoder frames, and the greedy choice over the logits."""
        config = self.config
        heads = config["decoder_attention_heads"]
        head_dim = config["d_model"] // heads
        dtype = self.model.model.decoder.embed_tokens.weight.dtype
        need = 256
        for batch in self.buckets:
            for length in [*self.kv_buckets, config["max_source_positions"]]:
                need = max(need, attention.decode_workspace_size(batch, heads, heads, head_dim, length, dtype))
            need = max(need, attention.choice_workspace_size(batch, config["vocab_size"]))
        return need

    @torch.inference_mode()
    def _capture_graphs(self) -> None:
        """``whisper.py:710-726``: warm-up steps advance active rows, so they
        stay inside the shortest length."""
        max_target = self.config["max_target_positions"]
        for batch_size in self.buckets:
            state = self.state.narrow(batch_size)
            for length in self.kv_buckets:
                cache = self.cache.narrow(batch_size, length)
                state.finished.zero_()
                state.position.zero_()
                state.end.fill_(max_target - 1)
                self.graphs[batch_size, length] = CapturedGraph(
                    lambda state=state, cache=cache: self.step(state, cache)
                )
        self.state.free(torch.arange(self.max_batch_size, device=self.device))

    @torch.inference_mode()
    def detect_languages(self, encoder_output: Tensor, start_id: int, language_ids: list[int]) -> list[int]:
        """The language of each window (``whisper.py:976-984``): one decoder
        pass over ``start_id`` (<|startoftranscript|>) at position 0 of the
        staging rows, whose cross-attention takes ``encoder_output``; returns,
        per window, the index into ``language_ids`` of the largest logit among
        those tokens.  Position 0 is overwritten by the next :meth:`admit`."""
        count = len(encoder_output)
        staging = self.staging.narrow(count)
        self.model.set_encoder_output(staging, encoder_output)
        tokens = torch.full((count, 1), start_id, dtype=torch.long, device=self.device)
        hidden = self.model.decode(tokens, self._positions[:1], staging, length=1)
        ids = torch.as_tensor(language_ids, dtype=torch.long, device=self.device)
        return self.model.logits(hidden[:, -1])[:, ids].argmax(dim=-1).tolist()

    @torch.inference_mode()
    def admit(
        self,
        encoder_output: Tensor,
        prefixes: list[list[int]],
        max_new_tokens: int,
        temperatures: Tensor | None = None,
        sot_index: int | None = None,
        no_speech_id: int | None = None,
    ) -> list[int]:
        """Prompt pass for windows that share a prefix length, then move them
        (with their first token) into free rows; returns their slots.

        ``temperatures`` (one per window, or None for greedy) pick the first
        token as the reference's ``_choose`` does.  With ``no_speech_id`` the
        pass also keeps each window's probability of that token after the
        prompt's <|startoftranscript|> at index ``sot_index``
        (``whisper.py:848-858``; :meth:`no_speech_probs`)."""
        count = len(prefixes)
        prefix_length = len(prefixes[0])
        if any(len(p) != prefix_length for p in prefixes):
            raise ValueError("admit() takes prompts of one length")
        if no_speech_id is not None and not (sot_index is not None and 0 <= sot_index < prefix_length):
            raise ValueError("no_speech_id needs sot_index, the position of <|startoftranscript|> in the prompt")
        slots = [s for s in range(self.max_batch_size) if s not in self.rows][:count]
        if len(slots) < count:
            raise RuntimeError("no free rows")
        staging = self.staging.narrow(count)
        self.model.set_encoder_output(staging, encoder_output)
        tokens = to_device(prefixes, self.device)
        hidden = self.model.decode(tokens, self._positions[:prefix_length], staging, length=prefix_length)
        rows = to_device(slots, self.device)
        if no_speech_id is None:
            logits = self.model.logits(hidden[:, -1:]).float()[:, 0]
            self.no_speech[rows] = 0.0
        else:
            both = self.model.logits(torch.stack((hidden[:, sot_index], hidden[:, -1]), dim=1)).float()
            self.no_speech[rows] = both[:, 0].softmax(dim=-1)[:, no_speech_id]
            logits = both[:, 1]
        if temperatures is not None:
            temperatures = torch.as_tensor(temperatures, dtype=torch.float32).to(self.device)
        with attention.workspace(self.workspace):
            token, logprob = choose(logits, self._first_suppress, temperatures)
        available = self.config["max_target_positions"] - prefix_length
        end = prefix_length - 1 + min(max_new_tokens, available)
        self.cache.copy_rows(staging, rows, prefix_length)
        state = self.state
        state.tokens[rows] = token[:, None]
        state.position[rows] = prefix_length
        state.end[rows] = end
        state.finished[rows] = (token == self.eos) | (prefix_length >= end)
        state.sum_logprobs[rows] = logprob
        state.generated[rows, prefix_length] = token
        for slot in slots:
            self.rows[slot] = {"prefix_length": prefix_length, "end": end, "bound": prefix_length}
        return slots

    def step(self, state: DecodeState, cache: DecoderCache) -> None:
        """One greedy step for every row (``whisper.py:942-960``); split
        partials go to the decoder's own workspace, sized at construction for
        the largest bucket."""
        with attention.workspace(self.workspace):
            hidden = self.model.decode(state.tokens, state.position, cache)
            logits = self.model.logits(hidden[:, -1]).float()
            token, logprob = choose(logits, self._suppress)
        active = ~state.finished
        position = state.position + active
        token = torch.where(active, token, state.tokens[:, 0])
        state.sum_logprobs.add_(logprob.masked_fill(state.finished, 0.0))
        state.generated.scatter_(1, position[:, None], token[:, None])
        state.finished.logical_or_((token == self.eos) | (position >= state.end))
        state.position.copy_(position)
        state.tokens.copy_(token[:, None])

    @torch.inference_mode()
    def advance(self) -> int:
        """Up to ``EOS_CHECK_INTERVAL`` steps over the occupied rows, from the
        graph of the smallest covering (batch, KV) bucket; returns the count."""
        bucket = next(size for size in self.buckets if size > max(self.rows))
        rows = self.rows.values()
        count = max(1, min(EOS_CHECK_INTERVAL, max(r["end"] - r["bound"] for r in rows)))
        length = max(min(r["bound"] + count, r["end"]) for r in rows) + 1
        kv_bucket = next(size for size in self.kv_buckets if size >= length)
        if self.graphs:
            graph = self.graphs[bucket, kv_bucket]
            for _ in range(count):
                graph.replay()
        else:
            state = self.state.narrow(bucket)
            cache = self.cache.narrow(bucket, kv_bucket)
            for _ in range(count):
                self.step(state, cache)
        for r in rows:
            r["bound"] = min(r["bound"] + count, r["end"])
        return count

    def no_speech_probs(self, slots: list[int]) -> list[float]:
        """The no-speech probability :meth:`admit` kept for each slot (0.0
        when it was given no ``no_speech_id``, as in the reference)."""
        return self.no_speech[to_device(slots, self.device)].tolist()

    @torch.inference_mode()
    def finished_rows(self) -> dict[int, list[int]]:
        """Generated tokens of the rows that finished, which are freed
        (``whisper.py:917-940``; the trailing EOS is dropped)."""
        finished = self.state.finished[: max(self.rows) + 1].tolist()
        done = [slot for slot in self.rows if finished[slot]]
        if not done:
            return {}
        rows = torch.tensor(done, device=self.device)
        positions = self.state.position[rows].tolist()
        generated = self.state.generated[rows, : max(positions) + 1].tolist()
        self.state.free(rows)
        out = {}
        for slot, position, tokens in zip(done, positions, generated):
            row = self.rows.pop(slot)
            tokens = tokens[row["prefix_length"] : position + 1]
            if tokens and tokens[-1] == self.eos:
                tokens.pop()
            out[slot] = tokens
        return out

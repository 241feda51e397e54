#!/usr/bin/env python3
"""Throughput of the asrback attention hot path on one MI355X.

Prints progress lines, then one JSON line holding every line below in full
(``"detail": true``), then the result line, last and compact: the headline
with its roofline and CPU baseline, and ``configs``, one entry per
benchmark configuration (1 Whisper-tiny fp32 encoder and decoder step, 2
SenseVoice, 3 Whisper-small decoder step, 4 Whisper large-v3-turbo encoder,
5 Qwen3-ASR-1.7B decode) with its rate, median ms per step, steps timed,
work per step, roofline fraction, HBM traffic per launch and CPU baseline.
Workloads that advance positions through a fixed schedule (Qwen3's 128
decode steps, Whisper-tiny's 32) time the whole schedule whatever --steps
says.  The headline workload is SenseVoiceSmall's SAN-M
encoder self-attention in bf16 (4 heads x 128, 70 layers, batch 32 with
ragged lengths of 104-504 frames and key padding): a step is the attention of
all 70 layers over one batch, q/k/v read in place from per-layer fused
projection buffers (token stride 1536) already resident in HBM, the 70
launches replayed from one hipGraph.  As ``SANMAttention`` runs it, padded
query rows (t >= L_b) are not computed and get zeros.  ``value`` is
algorithmic TFLOP/s: sum_b 4 * L_b^2 * 512 per layer over valid queries x
valid keys.  Every figure is the median over the timed steps, each step
bracketed by HIP events on the stream the graph replays on.

Decode is reported beside it (``decode``): Qwen3-ASR-1.7B's GQA decoder step
(28 layers, 16 query / 8 kv heads x 128, batch 64, prompts of 400-430 tokens,
a (28, 64, 1024, 8, 128) cache, 128 steps; also over a paged cache of
64-position pages holding only what the rows use) and Whisper-small's decoder step
(12 layers, 12 heads x 64, batch 16, self keys 1-224, cross-attention over
1500 frames), in algorithmic HBM GB/s (K and V of the keys each row uses,
plus q and o), and the Qwen3 step with its prologue (per-head RMSNorm and
rotary embedding of q and k, the cache write) fused into the decode launch,
timed beside the unfused sequence of ops, and the greedy token choice over
Qwen3's (64, 151936) logits in one pass.  ``secondary`` adds the SenseVoice
attention with its FSMN memory fused into the same launch (timed beside the
reference's ops for both outputs), Whisper large-v3-turbo's encoder
attention (20 heads x 64, 1500 frames, batch 16, 32 layers), and Qwen3's
causal grouped-query prompt pass and its audio encoder's windowed
attention.  Gemma 4's lines (its decoder step: sliding layers over a
512-key window at head_dim 256, full layers at 512; its blocked local audio
attention; its windowed prompt pass) run with --only gemma4-decode,
gemma4-audio, gemma4-prefill.  ``whisper_tiny`` holds Whisper-tiny's float32 lines
(encoder attention against the fp32 matrix peak, the greedy decoder step's
attention), ``whole_step`` Whisper-small's whole greedy decoder step with
the cache write fused into the attention launch against the reference's
separate writes.  ``calibration`` times what the card reaches with the
vendor's libraries in the same run: an 8192^3 GEMM in bf16 and in float32
(torch.matmul) and a 1 GiB device copy; each bf16 matrix-core line's
roofline also carries ``frac_of_library_gemm``, its rate over that GEMM's
(the 2.5 PFLOP/s datasheet peak assumes the 2.4 GHz peak engine clock, which
the card does not hold under a full bf16 matrix-core load).

``cpu_baseline`` times the CPU restatement of the reference's attention
(torch SDPA with the reference's masks, float32, the reference's CPU path)
on a bounded sample of the same workload on this machine's host cores: the
headline and each of the other configurations' lines carry one.

``roofline.traffic`` is the HBM bytes per launch of the dominant kernel from
the FETCH_SIZE / WRITE_SIZE counter runs that ``--profile`` records in
profiles/hbm_traffic.md, used only while the kernel sources still hash to
what that run measured (else null, with a note).

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--only NAME]
    python bench.py --profile DIR [--only NAME]   (rocprofv3 runs; no GPU use in this process)
"""

from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import statistics
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 matrix
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
MFMA_FILE = ROOT / "profiles" / "mfma_utilisation.md"
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic.md"
METRIC = "attn TFLOP/s (encoder) & HBM GB/s (decode step), % of MI355X roofline"


def log(*args) -> None:
    """Progress, on stdout before the result lines (so that the last line
    printed is the result)."""
    print(*args, flush=True)


class Workload:
    """A step of attention launches over inputs resident in HBM."""

    name: str
    unit: str
    bound: str
    kernel: str  # the dominant kernel (rocprof name prefix)
    launches: int  # launches of ``kernel`` per step
    work_per_step: float  # flop or bytes
    peak: float = 0.0  # the roofline's peak; 0: bf16 MFMA for TFLOP/s, HBM for GB/s
    dtype: str = "bf16"
    counters: bool = True  # whether --profile runs its counter passes

    def run(self) -> None:
        raise NotImplementedError

    def config(self) -> dict:
        raise NotImplementedError


class SenseVoiceEncoder(Workload):
    """SAN-M encoder self-attention (sensevoice.py:94-135): fused qkv
    ``(B, L, 1536)`` per layer, key padding by ``lengths = T + 4``."""

    name = "sensevoice-small-encoder-attention"
    unit = "TFLOP/s"
    bound = "mfma"
    kernel = "fwd_ring_kernel"

    def __init__(self, torch, attention, seed: int = 1) -> None:
        rng = np.random.default_rng(seed)
        self.batch, self.heads, self.head_dim, self.layers = 32, 4, 128, 70
        frames = rng.integers(100, 501, size=self.batch)  # LFR frames, U{100..500}
        self.lengths_host = (frames + 4).astype(np.int32)  # four query embeddings in front
        self.length = int(self.lengths_host.max())
        width = self.heads * self.head_dim
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.qkv = [
            torch.randn((self.batch, self.length, 3 * width), generator=g, device="cuda", dtype=torch.bfloat16)
            for _ in range(self.layers)
        ]
        self.lengths = torch.from_numpy(self.lengths_host).cuda()
        self.out = torch.empty((self.batch, self.length, self.heads, self.head_dim), device="cuda", dtype=torch.bfloat16)
        self.attention = attention
        self.launches = self.layers
        per_layer = float(sum(4 * int(n) ** 2 * width for n in self.lengths_host))
        self.work_per_step = per_layer * self.layers

    def views(self, layer: int):
        q, k, v = self.qkv[layer].split(self.heads * self.head_dim, dim=-1)
        shape = (self.batch, self.length, self.heads, self.head_dim)
        return q.view(shape), k.view(shape), v.view(shape)

    def run(self) -> None:
        for layer in range(self.layers):
            q, k, v = self.views(layer)
            self.attention.flash(q, k, v, seqused_k=self.lengths, out=self.out, zero_padded_rows=True)

    def config(self) -> dict:
        return {
            "workload": self.name,
            "batch": self.batch,
            "heads": self.heads,
            "head_dim": self.head_dim,
            "layers": self.layers,
            "frames": "L=U{100..500}+4, key padding",
            "lengths_mean": round(float(self.lengths_host.mean()), 1),
            "max_length": self.length,
            "padded_rows": "zeroed, not computed",
        }


class SenseVoiceAttentionFsmn(SenseVoiceEncoder):
    """The SAN-M attention and its FSMN memory (sensevoice.py:97-135) on the
    headline batch, one ``flash_fsmn`` launch per layer (kernel 11).  Value:
    attention FLOPs per second as for the attention alone.
    ``unfused_ms_per_step`` times the reference's ops for the same two
    outputs (mask multiply, pad, depthwise conv1d, add, mask multiply, then
    the attention kernel); ``module_ms_per_step`` / ``module_unfused_ms_per_step``
    add ``linear_out(attention) + memory`` (one GEMM accumulating into the
    memory, against linear and add)."""

    name = "sensevoice-small-attention-fsmn"

    def __init__(self, torch, attention, seed: int = 1) -> None:
        super().__init__(torch, attention, seed)
        g = torch.Generator(device="cuda").manual_seed(seed + 7)
        width = self.heads * self.head_dim
        self.weight = [(torch.randn((width, 1, 11), generator=g, device="cuda") * 0.3).to(torch.bfloat16)
                       for _ in range(self.layers)]
        self.bias = [torch.randn(width, generator=g, device="cuda").to(torch.bfloat16) for _ in range(self.layers)]
        self.w_out = [(torch.randn((width, width), generator=g, device="cuda") / width ** 0.5).to(torch.bfloat16)
                      for _ in range(self.layers)]
        frames = torch.arange(self.length, device="cuda")[None, :] < self.lengths[:, None].long()
        self.keep = frames[..., None].to(torch.bfloat16)
        self.memory = torch.empty((self.batch, self.length, width), device="cuda", dtype=torch.bfloat16)
        self.torch = torch
        self.mode = "fused"

    def run(self) -> None:
        F = self.torch.nn.functional
        width = self.heads * self.head_dim
        module = self.mode.startswith("module")
        for layer in range(self.layers):
            q, k, v = self.views(layer)
            if self.mode in ("fused", "module"):
                self.attention.flash_fsmn(q, k, v, self.weight[layer], seqused_k=self.lengths,
                                          bias=self.bias[layer] if module else None, out=self.out,
                                          memory=self.memory, zero_padded_rows=True)
                if module:
                    self.memory.view(-1, width).addmm_(self.out.view(-1, width), self.w_out[layer].t())
                continue
            masked = self.qkv[layer][..., 2 * width:] * self.keep
            memory = F.pad(masked.transpose(1, 2), (5, 5))
            memory = F.conv1d(memory, self.weight[layer], groups=width).transpose(1, 2) + masked
            memory = memory * self.keep
            self.attention.flash(q, k, v, seqused_k=self.lengths, out=self.out, zero_padded_rows=True)
            if module:
                memory = F.linear(self.out.view(self.batch, self.length, width), self.w_out[layer],
                                  self.bias[layer]) + memory
            self.memory.copy_(memory)

    def config(self) -> dict:
        return {**super().config(), "workload": self.name, "fsmn_kernel": 11}


class WhisperTurboEncoder(Workload):
    """Whisper large-v3-turbo encoder self-attention (whisper.py:102-110):
    q/k/v ``(16, 20, 1500, 64)`` views of ``(16, 1500, 1280)`` projections."""

    name = "whisper-large-v3-turbo-encoder-attention"
    unit = "TFLOP/s"
    bound = "mfma"
    kernel = "fwd_ring_kernel"

    def __init__(self, torch, attention, seed: int = 2) -> None:
        self.batch, self.heads, self.head_dim, self.layers, self.length = 16, 20, 64, 32, 1500
        width = self.heads * self.head_dim
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.qkv = [
            torch.randn((self.batch, self.length, 3 * width), generator=g, device="cuda", dtype=torch.bfloat16)
            for _ in range(self.layers)
        ]
        self.out = torch.empty((self.batch, self.length, self.heads, self.head_dim), device="cuda", dtype=torch.bfloat16)
        self.attention = attention
        self.launches = self.layers
        self.work_per_step = 4.0 * self.length**2 * width * self.batch * self.layers

    def run(self) -> None:
        width = self.heads * self.head_dim
        shape = (self.batch, self.length, self.heads, self.head_dim)
        for layer in range(self.layers):
            q, k, v = (t.view(shape) for t in self.qkv[layer].split(width, dim=-1))
            self.attention.flash(q, k, v, out=self.out)

    def config(self) -> dict:
        return {"workload": self.name, "batch": self.batch, "heads": self.heads, "head_dim": self.head_dim,
                "layers": self.layers, "frames": self.length}


class Qwen3Prefill(Workload):
    """Qwen3-ASR-1.7B prompt pass (qwen3_asr.py:374-390 via ``attend``,
    :152-166): 8 packed prompts of 390 + U{10..40} tokens, q ``(tokens, 16,
    128)`` over k/v ``(tokens, 8, 128)``, causal (``window_size=(-1, 0)``)
    and grouped-query, 28 layers.  Value: causal TFLOP/s, ``4 * 128 * 16 *
    P (P + 1) / 2`` per prompt and layer (each query over the keys it sees)."""

    name = "qwen3-asr-1.7b-prefill-attention"
    unit = "TFLOP/s"
    bound = "mfma"
    kernel = "fwd_ring_kernel"

    def __init__(self, torch, attention, seed: int = 4) -> None:
        rng = np.random.default_rng(seed)
        self.prompts = (390 + rng.integers(10, 41, size=8)).astype(np.int64)
        self.heads_q, self.heads_kv, self.head_dim, self.layers = 16, 8, 128, 28
        tokens = int(self.prompts.sum())
        starts = np.concatenate(([0], np.cumsum(self.prompts))).astype(np.int32)
        self.cu = torch.from_numpy(starts).cuda()
        self.longest = int(self.prompts.max())
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.q = [torch.randn((tokens, self.heads_q, self.head_dim), generator=g, device="cuda", dtype=torch.bfloat16)
                  for _ in range(self.layers)]
        self.kv = [torch.randn((2, tokens, self.heads_kv, self.head_dim), generator=g, device="cuda",
                               dtype=torch.bfloat16) for _ in range(self.layers)]
        self.attention = attention
        self.launches = self.layers
        per_layer = float(sum(4 * self.head_dim * self.heads_q * int(p) * (int(p) + 1) // 2 for p in self.prompts))
        self.work_per_step = per_layer * self.layers

    def run(self) -> None:
        for layer in range(self.layers):
            k, v = self.kv[layer]
            self.attention.varlen_attn(self.q[layer], k, v, self.cu, self.cu, self.longest, self.longest,
                                       window_size=(-1, 0), enable_gqa=True)

    def config(self) -> dict:
        return {"workload": self.name, "prompts": 8, "prompt_tokens": "390 + U{10..40}", "heads_q": self.heads_q,
                "heads_kv": self.heads_kv, "head_dim": self.head_dim, "layers": self.layers, "causal": "bottom-right"}


class Qwen3AudioAttention(Workload):
    """Qwen3-ASR's audio encoder attention (qwen3_asr.py:216-221 over the
    windows of :303-310) with transformers' ``Qwen3ASRAudioEncoderConfig``
    defaults: 16 heads x 64, 24 layers, chunks of 13 tokens in attention
    windows of 8 chunks (104 tokens); 8 audio windows of 30 s (390 tokens:
    segments of 104, 104, 104, 78), packed, non-causal.  Value: TFLOP/s over
    each segment's queries x keys."""

    name = "qwen3-asr-audio-encoder-attention"
    unit = "TFLOP/s"
    bound = "mfma"
    kernel = "fwd_ring_kernel"

    def __init__(self, torch, attention, seed: int = 8) -> None:
        self.heads, self.head_dim, self.layers, self.windows = 16, 64, 24, 8
        segments = [104, 104, 104, 78] * self.windows
        tokens = sum(segments)
        self.cu = torch.from_numpy(np.concatenate(([0], np.cumsum(segments))).astype(np.int32)).cuda()
        self.longest = max(segments)
        g = torch.Generator(device="cuda").manual_seed(seed)
        width = self.heads * self.head_dim
        self.qkv = [torch.randn((tokens, 3 * width), generator=g, device="cuda", dtype=torch.bfloat16)
                    for _ in range(self.layers)]
        self.attention = attention
        self.launches = self.layers
        self.work_per_step = float(sum(4 * n * n * width for n in segments)) * self.layers
        self.segments = len(segments)

    def run(self) -> None:
        width = self.heads * self.head_dim
        for layer in range(self.layers):
            q, k, v = (t.view(-1, self.heads, self.head_dim) for t in self.qkv[layer].split(width, dim=-1))
            self.attention.varlen_attn(q, k, v, self.cu, self.cu, self.longest, self.longest)

    def config(self) -> dict:
        return {"workload": self.name, "windows": self.windows, "segments": self.segments,
                "segment_tokens": "104, 104, 104, 78 per 30 s window", "heads": self.heads,
                "head_dim": self.head_dim, "layers": self.layers}


class Gemma4AudioAttention(Workload):
    """Gemma 4's blocked local audio attention (gemma4.py:240-282) with
    transformers' ``Gemma4AudioConfig`` defaults: 8 heads x 128, 12 layers,
    blocks of 12 tokens seeing the 12 before them, 13 relative keys, soft cap
    50, float32 as the reference computes it; 8 windows of 30 s (750 tokens,
    one a shorter tail).  Value: algorithmic HBM GB/s (q, k, v read and the
    output written once, plus the relative keys).  ``unfused_ms_per_step``
    times the reference's ops for the same output (pad, unfold into block
    contexts, content and relative products, the relative shift, soft cap,
    mask, softmax, product with the values)."""

    name = "gemma4-audio-local-attention"
    unit = "GB/s"
    bound = "hbm"
    kernel = "local_mfma_kernel"

    def __init__(self, torch, attention, seed: int = 5) -> None:
        self.batch, self.tokens, self.heads, self.head_dim, self.layers = 8, 750, 8, 128, 12
        self.chunk, self.past, self.rel_positions = 12, 12, 13
        lengths = np.full(self.batch, self.tokens, dtype=np.int32)
        lengths[-1] = 412
        self.lengths = torch.from_numpy(lengths).cuda()
        shape = (self.batch, self.tokens, self.heads, self.head_dim)
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.qkv = [[torch.randn(shape, generator=g, device="cuda") for _ in range(3)] for _ in range(self.layers)]
        self.rel = [torch.randn((self.rel_positions, self.heads, self.head_dim), generator=g, device="cuda")
                    for _ in range(self.layers)]
        self.out = torch.empty(shape, device="cuda")
        self.attention = attention
        self.torch = torch
        self.unfused = False
        blocks = -(-self.tokens // self.chunk)
        context = self.chunk + self.past
        query = torch.arange(blocks * self.chunk, device="cuda").view(blocks, self.chunk, 1)
        key = (torch.arange(blocks, device="cuda") * self.chunk - self.past).view(blocks, 1, 1) + torch.arange(
            context, device="cuda")
        allowed = (query - key >= 0) & (query - key < self.past) & (key >= 0)
        self.mask = ~(allowed & (key < self.lengths.view(-1, 1, 1, 1)))[:, None]
        self.launches = self.layers
        elements = self.batch * self.tokens * self.heads * self.head_dim
        per_layer = 4.0 * (4 * elements + self.rel_positions * self.heads * self.head_dim)
        self.work_per_step = per_layer * self.layers

    def run(self) -> None:
        for layer in range(self.layers):
            q, k, v = self.qkv[layer]
            if self.unfused:
                self.out.copy_(self.reference_ops(q, k, v, self.rel[layer]))
                continue
            self.attention.local_attention(q, k, v, self.rel[layer], self.lengths, chunk=self.chunk, past=self.past,
                                           future=0, softcap=50.0, invalid=-1e9, out=self.out)

    def reference_ops(self, q, k, v, rel):
        """The reference's sequence of ops (gemma4.py:256-282)."""
        F = self.torch.nn.functional
        batch, tokens, heads, dim = q.shape
        chunk, past = self.chunk, self.past
        context, blocks = chunk + past, self.mask.shape[2]

        def contexts(x):
            x = F.pad(x, (0, 0, 0, 0, past, chunk - 1))
            return self.torch.movedim(x.unfold(1, context, chunk), -1, 2)

        qb = F.pad(q, (0, 0, 0, 0, 0, blocks * chunk - tokens)).view(batch, blocks, chunk, heads, dim)
        qb = qb.permute(0, 3, 1, 2, 4)
        content = qb @ contexts(k).permute(0, 3, 1, 4, 2)
        position = qb.reshape(batch, heads, -1, dim) @ rel.permute(1, 2, 0)
        position = F.pad(position.view(batch, heads, blocks, chunk, -1), (0, context + 1 - rel.shape[0]))
        position = position.view(batch, heads, blocks, chunk * (context + 1))[..., : chunk * context]
        scores = self.torch.tanh((content + position.view(batch, heads, blocks, chunk, context)) / 50.0) * 50.0
        weights = F.softmax(scores.masked_fill(self.mask, -1e9), dim=-1)
        out = weights @ contexts(v).permute(0, 3, 1, 2, 4)
        return out.permute(0, 2, 3, 1, 4).reshape(batch, blocks * chunk, heads, dim)[:, :tokens]

    def config(self) -> dict:
        return {"workload": self.name, "batch": self.batch, "tokens": self.tokens, "heads": self.heads,
                "head_dim": self.head_dim, "layers": self.layers, "chunk": self.chunk, "past": self.past,
                "dtype": "float32"}


class Gemma4Prefill(Workload):
    """Gemma 4's prompt pass (gemma4.py:534-561, ``scale=1.0``) with
    transformers' ``Gemma4TextConfig`` defaults, as the reference admits
    windows: 8 padded prompts (``PREFILL_ROWS``, gemma4.py:66) of 800 +
    U{0..40} tokens, 8 query heads over 4 kv heads, causal; sliding layers
    head_dim 256 within a 512-key window, full layers head_dim 512; 30
    layers, five sliding to one full.  Value: TFLOP/s over each valid
    query's visible keys, ``4 * head_dim * 8`` per (query, key)."""

    name = "gemma4-prefill-attention"
    unit = "TFLOP/s"
    bound = "mfma"
    kernel = "fwd_ring_kernel"

    def __init__(self, torch, attention, seed: int = 7) -> None:
        rng = np.random.default_rng(seed)
        self.batch, self.heads_q, self.heads_kv, self.layers, self.window = 8, 8, 4, 30, 512
        self.full = [(i + 1) % 6 == 0 for i in range(self.layers)]
        sizes = (800 + rng.integers(0, 41, size=self.batch)).astype(np.int64)
        self.length = int(sizes.max())
        self.sizes = torch.from_numpy(sizes.astype(np.int32)).cuda()
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.q, self.kv = [], []
        for full in self.full:
            hd = 512 if full else 256
            self.q.append(torch.randn((self.batch, self.length, self.heads_q, hd), generator=g, device="cuda",
                                      dtype=torch.bfloat16))
            self.kv.append(torch.randn((2, self.batch, self.length, self.heads_kv, hd), generator=g, device="cuda",
                                       dtype=torch.bfloat16))
        self.out = {hd: torch.empty((self.batch, self.length, self.heads_q, hd), device="cuda", dtype=torch.bfloat16)
                    for hd in (256, 512)}
        self.attention = attention
        self.launches = self.layers
        work = 0.0
        for full in self.full:
            hd = 512 if full else 256
            for n in sizes:
                visible = np.arange(1, int(n) + 1)
                keys = visible.sum() if full else np.minimum(visible, self.window).sum()
                work += 4.0 * hd * self.heads_q * float(keys)
        self.work_per_step = work

    def run(self) -> None:
        for layer, full in enumerate(self.full):
            k, v = self.kv[layer]
            hd = k.shape[-1]
            self.attention.flash(self.q[layer], k, v, causal=1, seqused_k=self.sizes, scale=1.0,
                                 window=None if full else self.window, out=self.out[hd])

    def config(self) -> dict:
        return {"workload": self.name, "prompts": self.batch, "prompt_tokens": "800 + U{0..40}",
                "heads_q": self.heads_q, "heads_kv": self.heads_kv,
                "head_dim": "256 (sliding, window 512) / 512 (full)", "layers": self.layers,
                "full_layers": sum(self.full), "causal": "top-left"}


class Gemma4TextDecode(Workload):
    """Gemma 4's decoder step (gemma4.py:534-587, ``scale=1.0``) with
    transformers' ``Gemma4TextConfig`` defaults: 30 layers, five sliding to
    one full, 8 query heads over 4 kv heads; sliding layers head_dim 256 over
    the last 512 keys, full layers head_dim 512 over every key.  32 rows
    (the reference's default batch in bfloat16, gemma4.py:874-875) of a
    ``(32, 1280, 4, head_dim)`` cache per layer, prompts of 800 + U{0..40}
    tokens (a 30 s window's prompt), 128 steps.  Value: algorithmic HBM GB/s
    (K and V of the keys each row's window holds, plus q and o)."""

    name = "gemma4-text-decode-attention"
    unit = "GB/s"
    bound = "hbm"
    kernel = "decode_kernel"
    # Its 128-step schedule is ~8,100 dispatches, too many for a counter
    # pass within the profiler run's time limit.
    counters = False

    def __init__(self, torch, attention, seed: int = 6, steps: int = 128) -> None:
        rng = np.random.default_rng(seed)
        self.torch = torch
        self.batch, self.heads_q, self.heads_kv, self.layers = 32, 8, 4, 30
        self.cache_length, self.steps, self.window = 1280, steps, 512
        self.full = [(i + 1) % 6 == 0 for i in range(self.layers)]
        self.prompts = (800 + rng.integers(0, 41, size=self.batch)).astype(np.int64)
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.cache, self.q = [], []
        for full in self.full:
            hd = 512 if full else 256
            shape = (2, self.batch, self.cache_length, self.heads_kv, hd)
            self.cache.append(torch.randn(shape, generator=g, device="cuda", dtype=torch.bfloat16))
            self.q.append(torch.randn((self.batch, self.heads_q, hd), generator=g, device="cuda", dtype=torch.bfloat16))
        self.out = {hd: torch.empty((self.batch, self.heads_q, hd), device="cuda", dtype=torch.bfloat16)
                    for hd in (256, 512)}
        self.start = torch.from_numpy(self.prompts - 1).cuda()
        self.positions = self.start.clone()
        self.used = torch.empty(self.batch, dtype=torch.int32, device="cuda")
        self.attention = attention
        self.launches = self.layers
        self.step_bytes = []
        for t in range(self.steps):
            total = 0.0
            for full in self.full:
                hd = 512 if full else 256
                for p in self.prompts:
                    keys = int(p) + t + 1
                    keys = keys if full else min(keys, self.window)
                    total += 2 * self.heads_kv * hd * 2 * keys + 2 * self.heads_q * hd * 2
            self.step_bytes.append(total)
        self.work_per_step = float(np.mean(self.step_bytes))

    def reset(self) -> None:
        self.positions.copy_(self.start)

    def run(self) -> None:
        self.positions.add_(1)
        self.used.copy_(self.positions + 1)
        for layer, full in enumerate(self.full):
            k, v = self.cache[layer]
            hd = k.shape[-1]
            self.attention.decode(self.q[layer], k, v, seqused_k=self.used, scale=1.0,
                                  window=None if full else self.window, out=self.out[hd])

    def config(self) -> dict:
        return {"workload": self.name, "batch": self.batch, "heads_q": self.heads_q, "heads_kv": self.heads_kv,
                "head_dim": "256 (sliding, window 512) / 512 (full)", "layers": self.layers,
                "full_layers": sum(self.full), "cache_length": self.cache_length, "prompt_tokens": "800 + U{0..40}",
                "steps": self.steps}


class Qwen3Decode(Workload):
    """Qwen3-ASR-1.7B GQA decoder step (qwen3_asr.py:392-432): q ``(64, 16,
    128)`` over the ``(28, 64, 1024, 8, 128)`` cache, keys ``0 ..
    position`` (the kernel reads the positions, as the decoders pass them);
    each step advances every row by one position, 128 steps from prompts of
    390 + U{10..40} tokens."""

    name = "qwen3-asr-1.7b-decode-attention"
    unit = "GB/s"
    bound = "hbm"
    kernel = "decode_kernel"

    def __init__(self, torch, attention, seed: int = 3, steps: int = 128, slab: bool = True) -> None:
        rng = np.random.default_rng(seed)
        self.torch = torch
        self.batch, self.heads_q, self.heads_kv, self.head_dim, self.layers = 64, 16, 8, 128, 28
        self.cache_length, self.steps = 1024, steps
        self.prompts = (390 + rng.integers(10, 41, size=self.batch)).astype(np.int64)
        shape = (self.layers, self.batch, self.cache_length, self.heads_kv, self.head_dim)
        g = torch.Generator(device="cuda").manual_seed(seed)
        if slab:
            self.keys = torch.randn(shape, generator=g, device="cuda", dtype=torch.bfloat16)
            self.values = torch.randn(shape, generator=g, device="cuda", dtype=torch.bfloat16)
        self.q = torch.randn((self.layers, self.batch, self.heads_q, self.head_dim), generator=g, device="cuda",
                             dtype=torch.bfloat16)
        self.out = torch.empty((self.batch, self.heads_q, self.head_dim), device="cuda", dtype=torch.bfloat16)
        self.start = torch.from_numpy(self.prompts - 1).cuda()  # position of the last prompt token
        self.positions = self.start.clone()
        self.used = torch.empty(self.batch, dtype=torch.int32, device="cuda")
        self.attention = attention
        self.launches = self.layers
        # Step t attends P_b + t + 1 keys (the new token's key included).
        row_bytes = 2 * self.heads_kv * self.head_dim * 2  # K and V, bf16
        qo_bytes = 2 * self.heads_q * self.head_dim * 2
        self.step_bytes = [
            self.layers * float(sum(row_bytes * (int(p) + t + 1) + qo_bytes for p in self.prompts))
            for t in range(self.steps)
        ]
        self.work_per_step = float(np.mean(self.step_bytes))

    def reset(self) -> None:
        self.positions.copy_(self.start)

    def run(self) -> None:
        self.positions.add_(1)
        # Keys 0 .. position: the kernel reads the positions, as the decoders
        # pass them (KeyPrefix(positions=...)); no separate length tensor.
        for layer in range(self.layers):
            self.attention.decode(self.q[layer], self.keys[layer], self.values[layer], positions=self.positions,
                                  out=self.out)

    def config(self) -> dict:
        return {"workload": self.name, "batch": self.batch, "heads_q": self.heads_q, "heads_kv": self.heads_kv,
                "head_dim": self.head_dim, "layers": self.layers, "cache": list(self.keys.shape[1:]),
                "prompt_tokens": "390 + U{10..40}", "steps": self.steps}


class Qwen3DecodePaged(Qwen3Decode):
    """The Qwen3-ASR-1.7B decode workload over a paged cache: 64-position
    pages in random pool order, each row holding the pages for its prompt
    and the 128 steps (9 per row, 576 pages: 56% of the slab's 1024
    positions per row), the block table read on the device
    (``asrattn_decode_paged``).  Same prompts, positions and bytes."""

    name = "qwen3-asr-1.7b-decode-attention-paged"
    page_size = 64

    def __init__(self, torch, attention, seed: int = 3, steps: int = 128) -> None:
        super().__init__(torch, attention, seed, steps, slab=False)
        per_row = [-(-(int(p) + steps + 1) // self.page_size) for p in self.prompts]
        pages = sum(per_row)
        order = np.random.default_rng(seed + 11).permutation(pages)
        table = np.full((self.batch, self.cache_length // self.page_size), -1, dtype=np.int32)
        i = 0
        for b, count in enumerate(per_row):
            table[b, :count] = order[i : i + count]
            i += count
        shape = (self.layers, pages, self.page_size, self.heads_kv, self.head_dim)
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.keys = torch.randn(shape, generator=g, device="cuda", dtype=torch.bfloat16)
        self.values = torch.randn(shape, generator=g, device="cuda", dtype=torch.bfloat16)
        self.pages = attention.PageTable(torch.from_numpy(table).cuda(), self.cache_length)

    def run(self) -> None:
        self.positions.add_(1)
        for layer in range(self.layers):
            self.attention.decode(self.q[layer], self.keys[layer], self.values[layer], positions=self.positions,
                                  out=self.out, pages=self.pages)

    def config(self) -> dict:
        return {**super().config(), "workload": self.name, "page_size": self.page_size,
                "pool_pages": int(self.keys.shape[1]), "cache": list(self.keys.shape[1:])}


class Qwen3DecodeStepFused(Qwen3Decode):
    """The Qwen3-ASR-1.7B decoder step's attention sub-step with its prologue
    (qwen3_asr.py:366-372, :409-432): per layer, RMSNorm and rotary embedding
    of q (64, 16, 128) and the new key (64, 8, 128), the key/value write at
    each row's position and the GQA attention over keys 0..position -- one
    ``decode_append`` launch per layer.  Same cache, prompts and positions as
    the decode workload; ``unfused_ms_per_step`` times the reference's
    sequence of ops (norms, rotation, index writes, then the decode kernel)
    on the same inputs.  Bytes: the old keys' K and V, the new key and
    value (read and written), q and o."""

    name = "qwen3-asr-1.7b-decode-step-fused-prologue"

    def __init__(self, torch, attention, seed: int = 3, steps: int = 128) -> None:
        super().__init__(torch, attention, seed, steps)
        g = torch.Generator(device="cuda").manual_seed(seed + 1)
        kv_shape = (self.layers, self.batch, self.heads_kv, self.head_dim)
        self.k_new = torch.randn(kv_shape, generator=g, device="cuda", dtype=torch.bfloat16)
        self.v_new = torch.randn(kv_shape, generator=g, device="cuda", dtype=torch.bfloat16)
        self.q_norm = (torch.rand((self.layers, self.head_dim), generator=g, device="cuda") + 0.5).to(torch.bfloat16)
        self.k_norm = (torch.rand((self.layers, self.head_dim), generator=g, device="cuda") + 0.5).to(torch.bfloat16)
        inverse = 1.0 / (1e6 ** (torch.arange(0, self.head_dim, 2, device="cuda").float() / self.head_dim))
        angles = torch.arange(self.cache_length, device="cuda").float()[:, None] * inverse[None, :]
        angles = torch.cat((angles, angles), dim=-1)
        self.cos, self.sin = angles.cos().to(torch.bfloat16), angles.sin().to(torch.bfloat16)
        self.rows = torch.arange(self.batch, device="cuda")
        row_bytes = 2 * self.heads_kv * self.head_dim * 2
        qo_bytes = 2 * self.heads_q * self.head_dim * 2
        self.step_bytes = [
            self.layers * float(sum(row_bytes * (int(p) + t) + 2 * row_bytes + qo_bytes for p in self.prompts))
            for t in range(self.steps)
        ]
        self.work_per_step = float(np.mean(self.step_bytes))
        self.unfused = False

    def run(self) -> None:
        torch = self.torch
        self.positions.add_(1)
        cos, sin = self.cos[self.positions], self.sin[self.positions]
        if not self.unfused:
            for layer in range(self.layers):
                self.attention.decode_append(
                    self.q[layer], self.k_new[layer], self.v_new[layer], self.keys[layer], self.values[layer],
                    self.positions, q_norm=self.q_norm[layer], k_norm=self.k_norm[layer], eps=1e-6,
                    cos=cos, sin=sin, out=self.out)
            return
        F = torch.nn.functional
        self.used.copy_(self.positions + 1)

        def rotate(x):
            first, second = x.chunk(2, dim=-1)
            return x * cos[:, None, :] + torch.cat((-second, first), dim=-1) * sin[:, None, :]

        for layer in range(self.layers):
            q = rotate(F.rms_norm(self.q[layer], (self.head_dim,), self.q_norm[layer], 1e-6))
            k = rotate(F.rms_norm(self.k_new[layer], (self.head_dim,), self.k_norm[layer], 1e-6))
            self.keys[layer][self.rows, self.positions] = k
            self.values[layer][self.rows, self.positions] = self.v_new[layer]
            self.attention.decode(q, self.keys[layer], self.values[layer], seqused_k=self.used, out=self.out)


class GreedyChoice(Workload):
    """The greedy token choice of a Qwen3-ASR-1.7B decoder step
    (qwen3_asr.py:1200-1210): argmax and log_softmax at it over fp32 logits
    (64, 151936): each row read by 32 workgroups, their partials folded
    by a second launch; ``unfused_ms_per_step`` times torch's argmax,
    log_softmax and gather on the same logits.  A step is the choices of
    eight decoder steps over eight logits buffers (311 MB, more than the
    Infinity Cache), so that one graph replay is not just its own launch
    overhead.  Bytes: the logits read once, tokens and log-probabilities
    written."""

    name = "qwen3-asr-1.7b-greedy-choice"
    unit = "GB/s"
    bound = "hbm"
    kernel = "choose_kernel"

    def __init__(self, torch, attention, seed: int = 5) -> None:
        self.torch = torch
        self.rows, self.vocab, self.choices = 64, 151936, 8
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.logits = [torch.randn((self.rows, self.vocab), generator=g, device="cuda") * 4 for _ in range(self.choices)]
        self.attention = attention
        self.launches = self.choices
        self.work_per_step = float(self.choices * (self.rows * self.vocab * 4 + self.rows * 12))
        self.unfused = False

    def run(self) -> None:
        torch = self.torch
        for logits in self.logits:
            if not self.unfused:
                self.token, self.logprob = self.attention.greedy_choice(logits)
            else:
                self.token = logits.argmax(dim=-1)
                self.logprob = torch.log_softmax(logits, dim=-1).gather(1, self.token[:, None]).squeeze(1)

    def config(self) -> dict:
        return {"workload": self.name, "rows": self.rows, "vocab": self.vocab, "dtype": "float32 logits",
                "choices_per_step": self.choices}


class WhisperSmallDecoderStep(Workload):
    """Whisper-small decoder step (whisper.py:212-277): per layer, self-attention
    over the ``(16, 12, 256, 64)`` KV bucket view (keys 0..position, positions
    U{0..223}) and cross-attention over ``(16, 12, 1500, 64)``."""

    name = "whisper-small-decoder-step-attention"
    unit = "GB/s"
    bound = "hbm"
    kernel = "decode_kernel"

    def __init__(self, torch, attention, seed: int = 4) -> None:
        rng = np.random.default_rng(seed)
        self.batch, self.heads, self.head_dim, self.layers = 16, 12, 64, 12
        self.positions_host = rng.integers(0, 224, size=self.batch).astype(np.int64)
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.self_keys = torch.randn((self.layers, self.batch, self.heads, 448, self.head_dim), generator=g,
                                     device="cuda", dtype=torch.bfloat16)
        self.self_values = torch.randn_like(self.self_keys)
        self.cross_keys = torch.randn((self.layers, self.batch, self.heads, 1500, self.head_dim), generator=g,
                                      device="cuda", dtype=torch.bfloat16)
        self.cross_values = torch.randn_like(self.cross_keys)
        self.q = torch.randn((self.layers, 2, self.batch, self.heads, self.head_dim), generator=g, device="cuda",
                             dtype=torch.bfloat16)
        self.out = torch.empty((self.batch, self.heads, self.head_dim), device="cuda", dtype=torch.bfloat16)
        self.positions = torch.from_numpy(self.positions_host).cuda()
        self.attention = attention
        self.launches = 2 * self.layers
        row = self.heads * self.head_dim * 2
        qo = 2 * row
        self_bytes = sum(2 * row * (int(p) + 1) + qo for p in self.positions_host)
        cross_bytes = self.batch * (2 * row * 1500 + qo)
        self.work_per_step = float(self.layers * (self_bytes + cross_bytes))

    def run(self) -> None:
        bucket = 256
        for layer in range(self.layers):
            k = self.self_keys[layer, :, :, :bucket].transpose(1, 2)
            v = self.self_values[layer, :, :, :bucket].transpose(1, 2)
            self.attention.decode(self.q[layer, 0], k, v, positions=self.positions, out=self.out)
            self.attention.decode(self.q[layer, 1], self.cross_keys[layer].transpose(1, 2),
                                  self.cross_values[layer].transpose(1, 2), out=self.out)

    def config(self) -> dict:
        return {"workload": self.name, "batch": self.batch, "heads": self.heads, "head_dim": self.head_dim,
                "layers": self.layers, "self_keys": "U{1..224} in a 256 bucket", "cross_frames": 1500}


WHISPER_TINY = {"d_model": 384, "heads": 6, "layers": 4, "frames": 1500, "prefix": 4, "steps": 32}


class WhisperTinyEncoder(Workload):
    """Whisper-tiny's encoder self-attention in float32 (whisper.py:102-110):
    one 30 s window, 6 heads x 64 over 1500 frames, 4 layers, q/k/v views of
    per-layer ``(1, 1500, 1152)`` projections.  Value: TFLOP/s of ``4 * 1500^2
    * 384`` per layer against the fp32 matrix peak."""

    name = "whisper-tiny-encoder-attention-fp32"
    unit = "TFLOP/s"
    bound = "mfma"
    kernel = "fwd_"
    peak = PEAK_FP32_TFLOPS
    dtype = "f32"

    def __init__(self, torch, attention, seed: int = 9) -> None:
        self.width, self.heads, self.layers, self.length = (WHISPER_TINY[k] for k in ("d_model", "heads", "layers",
                                                                                      "frames"))
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.qkv = [torch.randn((1, self.length, 3 * self.width), generator=g, device="cuda")
                    for _ in range(self.layers)]
        self.out = torch.empty((1, self.length, self.heads, self.width // self.heads), device="cuda")
        self.attention = attention
        self.launches = self.layers
        self.work_per_step = 4.0 * self.length**2 * self.width * self.layers

    def run(self) -> None:
        shape = (1, self.length, self.heads, self.width // self.heads)
        for layer in range(self.layers):
            q, k, v = (t.view(shape) for t in self.qkv[layer].split(self.width, dim=-1))
            self.attention.flash(q, k, v, out=self.out)

    def config(self) -> dict:
        return {"workload": self.name, "batch": 1, "heads": self.heads, "head_dim": self.width // self.heads,
                "layers": self.layers, "frames": self.length, "dtype": "float32"}


class WhisperTinyDecodeStep(Workload):
    """Whisper-tiny's greedy decoder step in float32 (whisper.py:212-277),
    one row: per layer, self-attention over keys 0..position of the ``(1, 6,
    448, 64)`` cache (the 4-token prompt, then 32 steps: positions 4..35) and
    cross-attention over the 1500 encoder frames.  Value: algorithmic HBM
    GB/s (K and V of the keys each launch uses, plus q and o)."""

    name = "whisper-tiny-decoder-step-attention-fp32"
    unit = "GB/s"
    bound = "hbm"
    kernel = "decode_kernel"
    dtype = "f32"

    def __init__(self, torch, attention, seed: int = 10) -> None:
        self.width, self.heads, self.layers = WHISPER_TINY["d_model"], WHISPER_TINY["heads"], WHISPER_TINY["layers"]
        self.steps = WHISPER_TINY["steps"]
        hd = self.width // self.heads
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.self_kv = torch.randn((2, self.layers, 1, self.heads, 448, hd), generator=g, device="cuda")
        self.cross_kv = torch.randn((2, self.layers, 1, self.heads, 1500, hd), generator=g, device="cuda")
        self.q = torch.randn((self.layers, 2, 1, self.heads, hd), generator=g, device="cuda")
        self.out = torch.empty((1, self.heads, hd), device="cuda")
        self.start = torch.full((1,), WHISPER_TINY["prefix"] - 1, dtype=torch.int64, device="cuda")
        self.positions = self.start.clone()
        self.attention = attention
        self.launches = 2 * self.layers
        row = self.width * 4
        self.step_bytes = [
            float(self.layers * (2 * row * (WHISPER_TINY["prefix"] + t + 1) + 2 * row * 1500 + 4 * row))
            for t in range(self.steps)
        ]
        self.work_per_step = float(np.mean(self.step_bytes))

    def reset(self) -> None:
        self.positions.copy_(self.start)

    def run(self) -> None:
        self.positions.add_(1)
        for layer in range(self.layers):
            keys, values = (t[layer, :, :, :64].transpose(1, 2) for t in self.self_kv)
            self.attention.decode(self.q[layer, 0], keys, values, positions=self.positions, out=self.out)
            keys, values = (t[layer].transpose(1, 2) for t in self.cross_kv)
            self.attention.decode(self.q[layer, 1], keys, values, out=self.out)

    def config(self) -> dict:
        return {"workload": self.name, "batch": 1, "heads": self.heads, "head_dim": self.width // self.heads,
                "layers": self.layers, "self_keys": "5..36 in a 64 bucket (4-token prompt, 32 steps)",
                "cross_frames": 1500, "steps": self.steps, "dtype": "float32"}


class WhisperSmallWholeStep(Workload):
    """Whisper-small's whole greedy decoder step (whisper.py:942-960: token and
    position embeddings, 12 decoder layers, the logits, the greedy choice and
    the state update) in bf16 with random-init weights: 16 rows at positions
    U{0..223} over the 256-position KV bucket, cross-attention over 1500
    frames, one hipGraph per form.  With ``DecoderLayer.fused_step`` each
    layer's new key and value are written by its attention launch
    (``decode_append``); without it, by the reference's two ``scatter_``
    writes before the attention launch.  Value: decoder steps per second of
    the fused form; ``kernels_per_step`` counts the graph's kernel nodes."""

    name = "whisper-small-decoder-whole-step"
    unit = "steps/s"
    bound = "hbm"
    kernel = "decode_kernel"

    def __init__(self, torch, attention, seed: int = 4, steps: int = 32) -> None:
        from asrback_amd import whisper as aw

        self.torch, self.aw, self.steps = torch, aw, steps
        config = {"d_model": 768, "encoder_attention_heads": 12, "decoder_attention_heads": 12,
                  "encoder_layers": 12, "decoder_layers": 12, "encoder_ffn_dim": 3072, "decoder_ffn_dim": 3072,
                  "num_mel_bins": 80, "max_source_positions": 1500, "max_target_positions": 448,
                  "vocab_size": 51865, "eos_token_id": 50257}
        torch.manual_seed(seed)
        with torch.device("cuda"):
            model = aw.WhisperForConditionalGeneration(config)
        model = model.to(torch.bfloat16).eval().requires_grad_(False)
        vocab = config["vocab_size"]
        suppress = torch.zeros(vocab, dtype=torch.bool)
        suppress[50257:] = True  # special tokens, as the reference's suppress list holds them
        self.batch = 16
        self.decoder = aw.GreedyDecoder(model, self.batch, suppress, suppress, config["eos_token_id"], graphs=False)
        cache = self.decoder.cache
        g = torch.Generator(device="cuda").manual_seed(seed)
        for tensor in (cache.self_keys, cache.self_values, cache.cross_keys, cache.cross_values):
            tensor.copy_(torch.randn(tensor.shape, generator=g, device="cuda", dtype=torch.bfloat16))
        rng = np.random.default_rng(seed)
        self.start = torch.from_numpy(rng.integers(0, 224, size=self.batch).astype(np.int64)).cuda()
        self.tokens = torch.from_numpy(rng.integers(0, 50257, size=(self.batch, 1)).astype(np.int64)).cuda()
        self.state = self.decoder.state.narrow(self.batch)
        self.view = cache.narrow(self.batch, 256)
        self.state.end.fill_(255)
        self.reset()
        self.attention = attention
        self.launches = 2 * config["decoder_layers"]
        self.work_per_step = 1.0  # one step

    def reset(self) -> None:
        self.state.position.copy_(self.start)
        self.state.tokens.copy_(self.tokens)
        self.state.finished.zero_()

    def run(self) -> None:
        with self.torch.no_grad():
            self.decoder.step(self.state, self.view)

    def config(self) -> dict:
        return {"workload": self.name, "model": "whisper-small decoder (random init)", "batch": self.batch,
                "heads": 12, "head_dim": 64, "layers": 12, "self_keys": "U{1..224} in a 256 bucket",
                "cross_frames": 1500}


class CopyCalibration(Workload):
    """A plain device-to-device copy of 1 GiB: the known-size kernel that
    scales the HBM traffic counters (FETCH_SIZE / WRITE_SIZE)."""

    name = "copy-1GiB"
    unit = "GB/s"
    bound = "hbm"
    kernel = "copy"

    def __init__(self, torch, attention) -> None:
        del attention
        self.src = torch.ones(1 << 29, dtype=torch.bfloat16, device="cuda")
        self.dst = torch.empty_like(self.src)
        self.launches = 1
        self.work_per_step = 2.0 * (1 << 30)  # read + write

    def run(self) -> None:
        self.dst.copy_(self.src)

    def config(self) -> dict:
        return {"workload": self.name, "bytes_read": 1 << 30, "bytes_written": 1 << 30}


class GemmCalibration(Workload):
    """torch.matmul of two (8192, 8192) bf16 matrices (the vendor's tuned
    GEMM library), four per step: the matrix-core rate a library reaches on
    this card, beside the datasheet peak, which assumes the 2.4 GHz peak
    engine clock."""

    name = "gemm-bf16-8192-calibration"
    unit = "TFLOP/s"
    bound = "mfma"
    kernel = "Cijk_"
    size = 8192
    per_step = 4

    def __init__(self, torch, attention) -> None:
        del attention
        self.torch = torch
        g = torch.Generator(device="cuda").manual_seed(5)
        dt = torch.float32 if self.dtype == "f32" else torch.bfloat16
        self.a, self.b = (torch.randn((self.size, self.size), generator=g, device="cuda", dtype=dt) for _ in range(2))
        self.c = torch.empty((self.size, self.size), device="cuda", dtype=dt)
        self.launches = self.per_step
        self.work_per_step = self.per_step * 2.0 * self.size**3

    def run(self) -> None:
        for _ in range(self.per_step):
            self.torch.matmul(self.a, self.b, out=self.c)

    def config(self) -> dict:
        return {"workload": self.name, "m_n_k": [self.size] * 3, "per_step": self.per_step, "dtype": self.dtype}


class GemmCalibrationF32(GemmCalibration):
    """The same in float32 (no reduced-precision inner products): against the
    fp32 matrix peak."""

    name = "gemm-f32-8192-calibration"
    peak = PEAK_FP32_TFLOPS
    dtype = "f32"
    per_step = 2

    def __init__(self, torch, attention) -> None:
        torch.backends.cuda.matmul.allow_tf32 = False
        super().__init__(torch, attention)


_hip = None


def hip_runtime():
    """The HIP runtime torch loaded (the same library handle, found by path)."""
    global _hip
    if _hip is None:
        for line in open("/proc/self/maps"):
            if "libamdhip64" in line:
                _hip = ctypes.CDLL(line.split()[-1])
                break
    return _hip


def kernel_nodes(graph) -> int | None:
    """Kernel nodes of a captured graph (hipGraphGetNodes / hipGraphNodeGetType)."""
    hip = hip_runtime()
    if hip is None:
        return None
    handle = ctypes.c_void_p(graph.raw_cuda_graph())
    count = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(handle, None, ctypes.byref(count)) != 0:
        return None
    nodes = (ctypes.c_void_p * count.value)()
    if hip.hipGraphGetNodes(handle, nodes, ctypes.byref(count)) != 0:
        return None
    kernels = 0
    kind = ctypes.c_int(-1)
    for node in nodes:
        if hip.hipGraphNodeGetType(ctypes.c_void_p(node), ctypes.byref(kind)) != 0:
            return None
        kernels += kind.value == 0  # hipGraphNodeTypeKernel
    return kernels


def time_graph(torch, workload: Workload, steps: int, warmup: int) -> dict:
    """The step captured once as a hipGraph, ``warmup`` untimed replays, then
    ``steps`` replays, each between HIP events on the replaying stream, with
    a device synchronization on both sides.  Returns the median and mean
    milliseconds per step and the graph's kernel nodes."""
    reset = getattr(workload, "reset", None)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            workload.run()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        workload.run()
    graph.instantiate()
    kernels = kernel_nodes(graph)
    if reset is not None:
        reset()
    for _ in range(warmup):
        graph.replay()
    if reset is not None:
        reset()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    events[0].record()
    for i in range(steps):
        graph.replay()
        events[i + 1].record()
    torch.cuda.synchronize()
    per_step = [events[i].elapsed_time(events[i + 1]) for i in range(steps)]
    return {"median": statistics.median(per_step), "mean": events[0].elapsed_time(events[-1]) / steps,
            "kernels": kernels}


def sources_digest() -> str:
    """Hash of the kernel library's sources (csrc and the C header)."""
    csrc = ROOT / "asrback_amd" / "csrc"
    h = hashlib.sha256()
    for path in sorted(list(csrc.glob("*.hip")) + list(csrc.glob("*.hpp"))) + [ROOT / "include" / "asrattn.h"]:
        h.update(path.name.encode())
        h.update(path.read_bytes())
    return h.hexdigest()[:16]


def read_traffic(path: Path | None = None) -> dict:
    """The JSON block of profiles/hbm_traffic.md, or of ``path`` ({} when absent)."""
    try:
        text = (path or TRAFFIC_FILE).read_text()
        return json.loads(text.split("```json", 1)[1].split("```", 1)[0])
    except (OSError, IndexError, ValueError):
        return {}


def measured_traffic(key: str) -> tuple[float | None, str | None]:
    """HBM bytes per launch of ``key``'s dominant kernel from the counter
    runs, or None and the reason."""
    record = read_traffic()
    if not record:
        return None, "no counter run recorded"
    if record.get("sources") != sources_digest():
        return None, "the counter run measured other kernel sources"
    entry = record.get("workloads", {}).get(key)
    if not entry:
        return None, "not in the counter run"
    return entry["bytes_per_launch"], None


def roofline(workload: Workload, key: str, ms_per_step: float, work_per_step: float) -> dict:
    seconds = ms_per_step / 1e3
    if workload.unit == "TFLOP/s":
        achieved = work_per_step / seconds / 1e12
        peak = workload.peak or PEAK_BF16_TFLOPS
    else:
        achieved = work_per_step / seconds / 1e9
        peak = workload.peak or PEAK_HBM_GBS
    traffic, note = measured_traffic(key)
    line = {
        "bound": workload.bound,
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": workload.unit,
        "frac": round(achieved / peak, 4),
        "traffic": traffic,
        "kernel": workload.kernel,
        "launches_per_step": workload.launches,
        "avg_launch_us": round(ms_per_step * 1e3 / workload.launches, 2),
    }
    if note:
        line["traffic_note"] = note
    if workload.unit == "TFLOP/s" and traffic:
        # The attainable rate given the launch's measured HBM traffic: flops
        # per byte times the HBM peak, capped by the matrix-core peak.
        intensity = work_per_step / workload.launches / traffic
        ceiling = min(peak, intensity * PEAK_HBM_GBS / 1e3)
        line["flop_per_byte"] = round(intensity, 1)
        line["ceiling"] = round(ceiling, 1)
        line["frac_of_ceiling"] = round(achieved / ceiling, 4)
    return line


def timed_against(torch, workload: Workload, steps: int, warmup: int, result: dict, attr: str, value,
                  prefix: str = "unfused") -> None:
    """Time ``workload`` again with ``attr`` set to ``value`` and add it to
    ``result`` as ``{prefix}_ms_per_step`` (and its kernel count)."""
    owner = workload.aw.DecoderLayer if attr == "fused_step" else workload
    saved = getattr(owner, attr)
    setattr(owner, attr, value)
    try:
        other = time_graph(torch, workload, steps, warmup)
    finally:
        setattr(owner, attr, saved)
    result[f"{prefix}_ms_per_step"] = round(other["median"], 4)
    result[f"{prefix}_kernels_per_step"] = other["kernels"]
    if prefix == "unfused":
        result["speedup_vs_unfused"] = round(other["median"] / result["ms_per_step"], 3)


def measure(torch, workload: Workload, key: str, steps: int, warmup: int, compare: bool = True) -> dict:
    if hasattr(workload, "steps"):
        # Workloads that advance positions through a fixed schedule (Qwen3's
        # 128 decode steps, Whisper's 32) time the whole schedule, whatever
        # --steps asks, so that the bytes per step are the schedule's mean.
        steps = workload.steps
        warmup = min(warmup, workload.steps)
    timing = time_graph(torch, workload, steps, warmup)
    ms = timing["median"]
    step_bytes = getattr(workload, "step_bytes", None)
    work = float(np.mean(step_bytes[:steps])) if step_bytes else workload.work_per_step
    if workload.unit == "steps/s":
        value = 1e3 / ms
    else:
        value = work / (ms / 1e3) / (1e12 if workload.unit == "TFLOP/s" else 1e9)
    result = {
        "workload": workload.name,
        "value": round(value, 2),
        "unit": workload.unit,
        "dtype": workload.dtype,
        "ms_per_step": round(ms, 4),
        "ms_per_step_mean": round(timing["mean"], 4),
        "steps_timed": steps,
        "kernels_per_step": timing["kernels"],
        "roofline": None if workload.unit == "steps/s" else roofline(workload, key, ms, work),
        "config": workload.config(),
        "work_per_launch": work / workload.launches,
    }
    if not compare:
        return result
    if isinstance(workload, (GreedyChoice, Gemma4AudioAttention, Qwen3DecodeStepFused)):
        timed_against(torch, workload, steps, warmup, result, "unfused", True)
    if isinstance(workload, WhisperSmallWholeStep):
        timed_against(torch, workload, steps, warmup, result, "fused_step", False)
        result["saved_kernels_per_step"] = (None if result["kernels_per_step"] is None
                                            or result["unfused_kernels_per_step"] is None
                                            else result["unfused_kernels_per_step"] - result["kernels_per_step"])
    if isinstance(workload, SenseVoiceAttentionFsmn):
        for mode in ("unfused", "module", "module_unfused"):
            timed_against(torch, workload, steps, warmup, result, "mode", mode, prefix=mode)
        result.pop("unfused_kernels_per_step", None)
        result["speedup_vs_unfused"] = round(result["unfused_ms_per_step"] / ms, 3)
        result["module_speedup_vs_unfused"] = round(result["module_unfused_ms_per_step"] /
                                                    result["module_ms_per_step"], 3)
    return result


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _cpu_timed(fn, work: float, scale: float, unit: str, sample: str, budget_s: float) -> dict:
    """``fn`` once untimed, then repeatedly until ``budget_s`` seconds (at
    least three runs); the rate is ``work`` over the median run time."""
    import torch

    fn()
    times = []
    start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - start < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    median = statistics.median(times)
    return {
        "value": round(work / median / scale, 4),
        "unit": unit,
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{sample}; median of {len(times)} runs of {median * 1e3:.1f} ms; {_cpu_model()}",
        "seconds": round(sum(times), 2),
    }


def cpu_sensevoice(budget_s: float) -> dict:
    """SAN-M attention of one layer over the headline batch (oracle: torch
    SDPA with the key-padding mask, sensevoice.py:128-133)."""
    import torch

    from oracle import attention as oa

    rng = np.random.default_rng(1)
    lengths = torch.from_numpy((rng.integers(100, 501, size=32) + 4).astype(np.int64))
    length = int(lengths.max())
    qkv = torch.randn((32, length, 3 * 512), generator=torch.Generator().manual_seed(1))
    mask = oa.key_padding_mask(lengths, length)
    work = float(sum(4 * int(n) ** 2 * 512 for n in lengths))
    return _cpu_timed(lambda: oa.sensevoice_attention(qkv, 4, mask), work, 1e12, "TFLOP/s",
                      f"one layer, B=32, lengths {int(lengths.min())}-{length}, float32",
                      budget_s)


def cpu_turbo(budget_s: float) -> dict:
    """Whisper large-v3-turbo encoder attention of one layer (whisper.py:102-104)."""
    import torch

    from oracle import attention as oa

    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn((16, 20, 1500, 64), generator=g) for _ in range(3))
    return _cpu_timed(lambda: oa.sdpa(q, k, v), 4.0 * 1500**2 * 1280 * 16, 1e12, "TFLOP/s",
                      "one layer (B=16, 20 heads x 64, 1500 frames), float32", budget_s)


def cpu_whisper_tiny_encoder(budget_s: float) -> dict:
    """Whisper-tiny's encoder attention, all 4 layers (whisper.py:102-104)."""
    import torch

    from oracle import attention as oa

    g = torch.Generator().manual_seed(9)
    layers = [[torch.randn((1, 6, 1500, 64), generator=g) for _ in range(3)] for _ in range(4)]
    return _cpu_timed(lambda: [oa.sdpa(*qkv) for qkv in layers], 4.0 * 1500**2 * 384 * 4, 1e12, "TFLOP/s",
                      "the 4 layers of one window (6 heads x 64, 1500 frames), float32", budget_s)


def _decode_sample(batch, heads_q, heads_kv, head_dim, cache, keys_used, seed):
    """Inputs of one decode launch on the CPU: q, keys/values ``(B, H, L, D)``
    and the step mask for ``keys_used`` (None: every key)."""
    import torch

    from oracle import attention as oa

    g = torch.Generator().manual_seed(seed)
    q = torch.randn((batch, heads_q, 1, head_dim), generator=g)
    k, v = (torch.randn((batch, heads_kv, cache, head_dim), generator=g) for _ in range(2))
    mask = None
    if keys_used is not None:
        mask = oa.whisper_step_mask(torch.as_tensor(keys_used, dtype=torch.int64) - 1, cache)
    return q, k, v, mask


def cpu_whisper_small(budget_s: float) -> dict:
    """Whisper-small decoder step attention of one layer: self-attention with
    the step mask over the 256 bucket (whisper.py:235-237) and
    cross-attention over 1500 frames (:239-240)."""
    from oracle import attention as oa

    rng = np.random.default_rng(4)
    used = rng.integers(0, 224, size=16) + 1
    self_in = _decode_sample(16, 12, 12, 64, 256, used, 4)
    cross_in = _decode_sample(16, 12, 12, 64, 1500, None, 5)
    row = 12 * 64 * 2
    work = float(sum(2 * row * int(n) + 2 * row for n in used) + 16 * (2 * row * 1500 + 2 * row))

    def layer():
        oa.sdpa(*self_in[:3], attn_mask=self_in[3])
        oa.sdpa(*cross_in[:3])

    return _cpu_timed(layer, work, 1e9, "GB/s",
                      "one layer (B=16, self keys U{1..224} in a 256 bucket, cross 1500), float32; bytes "
                      "counted as the bf16 workload's", budget_s)


def cpu_whisper_tiny_step(budget_s: float) -> dict:
    """Whisper-tiny decoder step attention, all 4 layers, at the 32-step
    decode's middle position (keys 0..19 of a 64 bucket; cross 1500)."""
    from oracle import attention as oa

    layers = [(_decode_sample(1, 6, 6, 64, 64, [20], 10 + i), _decode_sample(1, 6, 6, 64, 1500, None, 20 + i))
              for i in range(4)]
    row = 384 * 4
    work = float(4 * (2 * row * 20 + 2 * row * 1500 + 4 * row))

    def step():
        for self_in, cross_in in layers:
            oa.sdpa(*self_in[:3], attn_mask=self_in[3])
            oa.sdpa(*cross_in[:3])

    return _cpu_timed(step, work, 1e9, "GB/s", "the 4 layers of one step (20 self keys, cross 1500), float32",
                      budget_s)


def cpu_qwen3_decode(budget_s: float) -> dict:
    """Qwen3-ASR GQA decode of one layer at the 128-step decode's middle
    step (qwen3_asr.py:427-432 on the padded path: query heads grouped per kv
    head, the step mask over the 1024-position cache)."""
    import torch

    from oracle import attention as oa

    rng = np.random.default_rng(3)
    used = (390 + rng.integers(10, 41, size=64)) + 64
    g = torch.Generator().manual_seed(3)
    q = torch.randn((64, 16, 128), generator=g)
    keys, values = (torch.randn((64, 1024, 8, 128), generator=g) for _ in range(2))
    mask = oa.qwen_step_mask(torch.from_numpy(used - 1), 1024)
    row = 2 * 8 * 128 * 2
    work = float(sum(row * int(n) + 2 * 16 * 128 * 2 for n in used))
    return _cpu_timed(lambda: oa.qwen_step_attention(q, keys, values, mask), work, 1e9, "GB/s",
                      "one layer at step 64 (B=64, 16q/8kv x 128, 1024-position cache), float32; bytes counted "
                      "as the bf16 workload's", budget_s)


# Workloads (by --only key) that carry a CPU baseline: the headline and one
# line per other configuration.
CPU_BASELINES = {
    "sensevoice": cpu_sensevoice,
    "turbo": cpu_turbo,
    "whisper-small": cpu_whisper_small,
    "qwen3": cpu_qwen3_decode,
    "whisper-tiny-encoder": cpu_whisper_tiny_encoder,
    "whisper-tiny-step": cpu_whisper_tiny_step,
}


def cpu_baseline(key: str, budget_s: float) -> dict:
    import torch

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    with torch.inference_mode():
        return CPU_BASELINES[key](budget_s)


def shape_sweep(torch, attention) -> None:
    """Average launch time of the encoder kernel over shapes: where its time
    goes (fixed cost per launch, per-sequence critical path, throughput)."""

    def launch_us(fn, reps=20):
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(5):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e3 / (5 * reps)

    rng = np.random.default_rng(1)
    ragged = list((rng.integers(100, 501, size=32) + 4).astype(int))
    cases = [
        ("SenseVoice ragged B=32 (headline)", 32, 4, max(ragged), 128, ragged),
        ("uniform B=32 L=504", 32, 4, 504, 128, None),
        ("uniform B=32 L=128", 32, 4, 128, 128, None),
        ("uniform B=128 L=504", 128, 4, 504, 128, None),
        ("uniform B=8 L=504", 8, 4, 504, 128, None),
        ("one 64-row tile, 64 keys", 1, 1, 64, 128, None),
        ("B=4 H=16 L=4096 hd=128", 4, 16, 4096, 128, None),
        ("Whisper turbo B=16 H=20 L=1500 hd=64", 16, 20, 1500, 64, None),
    ]
    print("| Shape | us per launch | TFLOP/s |")
    print("|---|---|---|")
    for name, batch, heads, length, hd, lengths in cases:
        q, k, v = (torch.randn(batch, length, heads, hd, device="cuda", dtype=torch.bfloat16) for _ in range(3))
        used = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device="cuda")
        out = torch.empty_like(q)
        us = launch_us(lambda: attention.flash(q, k, v, seqused_k=used, out=out))
        lens = lengths if lengths is not None else [length] * batch
        flops = sum(4 * n * n * heads * hd for n in lens)
        print(f"| {name} | {us:.2f} | {flops / us / 1e6:.1f} |", flush=True)


WORKLOADS = {
    "sensevoice": SenseVoiceEncoder,
    "sensevoice-fsmn": SenseVoiceAttentionFsmn,
    "turbo": WhisperTurboEncoder,
    "qwen3": Qwen3Decode,
    "qwen3-paged": Qwen3DecodePaged,
    "qwen3-fused": Qwen3DecodeStepFused,
    "qwen3-prefill": Qwen3Prefill,
    "qwen3-audio": Qwen3AudioAttention,
    "gemma4-audio": Gemma4AudioAttention,
    "gemma4-decode": Gemma4TextDecode,
    "gemma4-prefill": Gemma4Prefill,
    "choice": GreedyChoice,
    "whisper-small": WhisperSmallDecoderStep,
    "whisper-tiny-encoder": WhisperTinyEncoder,
    "whisper-tiny-step": WhisperTinyDecodeStep,
    "whisper-small-step": WhisperSmallWholeStep,
    "copy": CopyCalibration,
    "gemm-bf16": GemmCalibration,
    "gemm-f32": GemmCalibrationF32,
}
# The lines of the default run after the headline, by group.  Gemma 4's
# lines (gemma4-decode, gemma4-audio, gemma4-prefill) run with --only.
GROUPS = {
    "decode": ["qwen3", "qwen3-paged", "qwen3-fused", "whisper-small", "choice"],
    "secondary": ["sensevoice-fsmn", "turbo", "qwen3-prefill", "qwen3-audio"],
    "whisper_tiny": ["whisper-tiny-encoder", "whisper-tiny-step"],
    "whole_step": ["whisper-small-step"],
    # What the card reaches with the vendor's libraries: bf16 and fp32 GEMMs
    # and a 1 GiB device copy (the same card and run as the lines above).
    "calibration": ["gemm-bf16", "gemm-f32", "copy"],
}
# The five benchmark configurations and the line that measures each: 1
# Whisper-tiny fp32 (encoder attention and the greedy step's attention), 2
# SenseVoice (the headline), 3 Whisper-small's decoder step, 4 Whisper
# large-v3-turbo's encoder, 5 Qwen3-ASR-1.7B's decode.
CONFIG_LINES = [(1, "whisper-tiny-encoder"), (1, "whisper-tiny-step"), (2, "sensevoice"), (3, "whisper-small"),
                (4, "turbo"), (5, "qwen3")]


def config_entry(cfg: int, key: str, result: dict) -> dict:
    """One configuration's figures in the final line, compact: its line (the
    --only name of its workload), rate, median ms per step, steps timed,
    algorithmic work per step (flop or bytes), roofline fraction, HBM
    traffic per launch and CPU baseline rate (same unit; host cores as the
    headline's)."""
    roof = result.get("roofline") or {}
    cpu = result.get("cpu_baseline") or {}
    work = result["work_per_launch"] * (roof.get("launches_per_step") or 1)
    return {"cfg": cfg, "line": key, "value": result["value"], "unit": result["unit"],
            "ms_per_step": result["ms_per_step"], "steps": result["steps_timed"], "work_per_step": f"{work:.3g}",
            "frac": roof.get("frac"), "traffic": roof.get("traffic"), "cpu": cpu.get("value")}


def _run_child(cmd: list[str], limit: float) -> tuple[int, str, str]:
    """Run ``cmd`` in its own process group; kill the group at ``limit`` s."""
    proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, start_new_session=True)
    try:
        out, err = proc.communicate(timeout=limit)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, 9)
        out, err = proc.communicate()
        return 124, out, err
    return proc.returncode, out, err


def _result_line(stdout: str) -> dict | None:
    for line in reversed(stdout.splitlines()):
        if line.startswith("{"):
            return json.loads(line)
    return None


def _csv_rows(directory: Path, suffix: str) -> list[dict]:
    import csv

    rows = []
    for path in sorted(directory.rglob(f"*{suffix}")):
        with open(path, newline="") as f:
            rows.extend(csv.DictReader(f))
    return rows


def _dispatch_counters(directory: Path, counter: str) -> list[tuple[int, str, float]]:
    """(dispatch id, kernel, value) of ``counter`` per dispatch, in dispatch order."""
    values: dict[int, list] = {}
    for row in _csv_rows(directory, "counter_collection.csv"):
        if row.get("Counter_Name") != counter:
            continue
        dispatch = int(row["Dispatch_Id"])
        entry = values.setdefault(dispatch, [row["Kernel_Name"], 0.0])
        entry[1] += float(row["Counter_Value"])
    return [(d, k, v) for d, (k, v) in sorted(values.items())]


def _dispatch_ns(directory: Path) -> dict[int, int]:
    """Duration (ns) of each dispatch of a counter run."""
    spans = {}
    for row in _csv_rows(directory, "counter_collection.csv"):
        spans[int(row["Dispatch_Id"])] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
    return spans


def profile(out: Path, keys: list[str], steps: int, warmup: int) -> int:
    """rocprofv3 runs of each workload in child processes (this process
    never touches the GPU): a plain run, a kernel trace, and one counter pass
    each for FETCH_SIZE and WRITE_SIZE (plus the 1 GiB copy that scales
    them).  Writes a summary per workload and hbm_traffic.md to
    ``out/profiles``."""
    out = out.resolve()
    summaries = out / "profiles"
    summaries.mkdir(parents=True, exist_ok=True)
    digest = sources_digest()
    bench = [sys.executable, "-u", str(ROOT / "bench.py")]

    def child(key: str, tag: str, prof: list[str], n_steps: int, n_warmup: int) -> tuple[dict, Path, str]:
        directory = out / key / tag
        directory.mkdir(parents=True, exist_ok=True)
        args = ["--only", key, "--steps", str(n_steps), "--warmup", str(n_warmup), "--no-cpu-baseline",
                "--no-compare"]
        cmd = bench + args
        if prof:
            cmd = ["rocprofv3", *prof, "--output-format", "csv", "-d", str(directory), "-o", "run", "--"] + cmd
        shown = " ".join(["python3 -u bench.py", *args] if not prof else
                         ["rocprofv3", *prof, "--output-format", "csv", "-d", "<dir>", "-o", "run", "--",
                          "python3 -u bench.py", *args])
        log(f"profile: {key} {tag}")
        rc, stdout, stderr = _run_child(cmd, 240)
        (directory / "stdout.txt").write_text(stdout)
        (directory / "stderr.txt").write_text(stderr[-20000:])
        result = _result_line(stdout)
        # rocprofv3 may exit with a signal after the program has finished and
        # its files are complete; the program's own result line decides.
        if result is None:
            raise RuntimeError(f"{key} {tag}: exit {rc} without a result line; see {directory}/stderr.txt")
        log(f"profile: {key} {tag} done (exit {rc})")
        return result, directory, shown

    def counter(key: str, name: str) -> tuple[list[tuple[int, str, float]], str, dict]:
        result, directory, shown = child(key, name.lower(), ["--pmc", name], 2, 1)
        return _dispatch_counters(directory, name), shown, result

    scale = {}
    calibration = {}
    for name in ("FETCH_SIZE", "WRITE_SIZE"):
        values, shown, _ = counter("copy", name)
        kib = max(v for _, _, v in values)
        scale[name] = (1 << 30) / (kib * 1024.0)
        calibration[name] = {"kib_per_1GiB_copy": kib, "scale": round(scale[name], 4), "command": shown}

    # Earlier --profile calls into the same directory (same sources) merge,
    # else the committed table does.
    record = read_traffic(summaries / "hbm_traffic.md")
    if record.get("sources") != digest:
        record = read_traffic()
    workloads = record.get("workloads", {}) if record.get("sources") == digest else {}
    mfma = read_traffic(summaries / MFMA_FILE.name)
    if mfma.get("sources") != digest:
        mfma = read_traffic(MFMA_FILE)
    mfma_rows = mfma.get("workloads", {}) if mfma.get("sources") == digest else {}
    mfma_counters = ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU",
                     "GRBM_GUI_ACTIVE"]
    mfma_command = None
    for key in keys:
        cls = WORKLOADS[key]
        plain, _, plain_cmd = child(key, "plain", [], steps, warmup)
        traced, directory, trace_cmd = child(key, "trace", ["--kernel-trace", "--stats"], steps, warmup)
        trace = sorted(_csv_rows(directory, "kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
        per_step = traced["kernels_per_step"] or 0
        n_timed = traced["steps_timed"]
        timed = trace[-per_step * n_timed:] if per_step else []
        durations = [(r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3) for r in timed]
        dominant = [d for name, d in durations if cls.kernel in name]
        kernel_name = next((name for name, _ in durations if cls.kernel in name), cls.kernel)
        per_step_us = sum(d for _, d in durations) / max(n_timed, 1)
        stats = sorted(_csv_rows(directory, "kernel_stats.csv"), key=lambda r: -float(r["TotalDurationNs"]))[:6]

        traffic = {"FETCH_SIZE": None, "WRITE_SIZE": None}
        commands = {"FETCH_SIZE": "(no counter pass for this workload)", "WRITE_SIZE": ""}
        counted = None  # a counter run's own result: the same steps as its counters
        for name in ("FETCH_SIZE", "WRITE_SIZE") if cls.counters else ():
            values, commands[name], counted = counter(key, name)
            mine = [v for _, kernel, v in values if cls.kernel in kernel]
            # The counter run's timed steps: its last two, or a fixed
            # schedule (Qwen3's 128 decode steps) whole.
            mine = mine[-counted["steps_timed"] * cls_launches(plain):] or mine
            traffic[name] = statistics.mean(mine) * 1024.0 * scale[name] if mine else None
        short = short_kernel(kernel_name)
        entry = {"kernel": short, "launches_per_step": cls_launches(plain),
                 "fetch_bytes": round(traffic["FETCH_SIZE"]) if traffic["FETCH_SIZE"] else None,
                 "write_bytes": round(traffic["WRITE_SIZE"]) if traffic["WRITE_SIZE"] else None}
        entry["bytes_per_launch"] = (entry["fetch_bytes"] + entry["write_bytes"]
                                     if entry["fetch_bytes"] is not None and entry["write_bytes"] is not None
                                     else None)
        # Algorithmic bytes of the launches the counters saw.
        if counted and counted.get("work_per_launch") and counted["unit"] == "GB/s":
            entry["algorithmic_bytes_per_launch"] = round(counted["work_per_launch"])
        if cls.counters:
            workloads[key] = entry

        if cls.bound == "mfma":
            # One counter pass: matrix-core busy and VALU co-execution cycles,
            # per dispatch of the dominant kernel (mean over the last two steps).
            _, mdir, mfma_command = child(key, "mfma", ["--pmc", *mfma_counters], 2, 1)
            per = {}
            spans = _dispatch_ns(mdir)
            clocks = []
            for name in mfma_counters:
                rows = [(d, v) for d, kernel, v in _dispatch_counters(mdir, name) if cls.kernel in kernel]
                rows = rows[-2 * cls_launches(plain):] or rows
                per[name] = statistics.mean(v for _, v in rows) if rows else None
                if name == "GRBM_GUI_ACTIVE":
                    # Busy cycles per XCD over the dispatch's duration: the
                    # engine clock the kernel ran at.  The counter's window
                    # is not tight around short dispatches (it reads above
                    # 2.4 GHz for 20 us ones), so only dispatches of 100 us
                    # and more give a clock.
                    clocks = [v / 8 / spans[d] for d, v in rows if spans.get(d, 0) >= 100_000]
            if all(per.get(n) for n in ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_INSTS_MFMA")):
                cycles = per["GRBM_GUI_ACTIVE"] / 8  # summed over the 8 XCDs
                mfma_rows[key] = {
                    "clock_ghz": round(statistics.mean(clocks), 3) if clocks else None,
                    "kernel": short_kernel(kernel_name),
                    "mfma_busy": round(per["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles * 1024), 4),
                    "coexec_of_busy": round((per["SQ_VALU_MFMA_COEXEC_CYCLES"] or 0) /
                                            per["SQ_VALU_MFMA_BUSY_CYCLES"], 4),
                    "valu_per_mfma": round(((per["SQ_INSTS_VALU"] or 0) - per["SQ_INSTS_MFMA"]) /
                                           per["SQ_INSTS_MFMA"], 2),
                    "mfma_per_dispatch": round(per["SQ_INSTS_MFMA"]),
                    "us_per_launch": round(statistics.mean(dominant), 2) if dominant else None,
                }

        lines = [
            f"# `{short}` — {cls.name}",
            "",
            f"Kernel sources digest `{digest}` (bench.py `sources_digest`).  Commands, from the repository root "
            "on one MI355X (this summary: `python3 bench.py --profile <dir> --only " + key + "`):",
            "",
            f"    {plain_cmd}",
            f"    {trace_cmd}",
            *[f"    {c}" for c in (commands["FETCH_SIZE"], commands["WRITE_SIZE"]) if c],
            "",
            "| Figure | Value |",
            "|---|---|",
            f"| bench, plain run: median ms per step ({plain['steps_timed']} steps) | {plain['ms_per_step']} |",
            f"| bench, plain run: µs per launch of the dominant kernel (step ÷ {cls_launches(plain)}) | "
            f"{plain['ms_per_step'] * 1e3 / cls_launches(plain):.2f} |",
            f"| bench inside the traced run: median ms per step | {traced['ms_per_step']} |",
            f"| profiler overhead (traced ÷ plain − 1) | {traced['ms_per_step'] / plain['ms_per_step'] - 1:+.1%} |",
            f"| trace, timed steps: `{short}` launches, mean / min / max µs | {len(dominant)}, "
            + (f"{statistics.mean(dominant):.2f} / {min(dominant):.2f} / {max(dominant):.2f} |"
               if dominant else "— |"),
            f"| trace, timed steps: kernel time per step, all kernels (ms) | {per_step_us / 1e3:.4f} "
            f"(≤ {traced['ms_per_step_mean']} mean ms per step of the same run: "
            f"{'yes' if per_step_us / 1e3 <= traced['ms_per_step_mean'] * 1.001 else 'no'}) |",
            f"| FETCH_SIZE per launch (scaled ×{scale['FETCH_SIZE']:.3f}) | "
            + (f"{entry['fetch_bytes'] / 1e6:.2f} MB |" if entry["fetch_bytes"] else "— |"),
            f"| WRITE_SIZE per launch (scaled ×{scale['WRITE_SIZE']:.3f}) | "
            + (f"{entry['write_bytes'] / 1e6:.2f} MB |" if entry["write_bytes"] else "— |"),
        ]
        if counted:
            lines.append(f"| counter runs: steps timed (the counters' mean is over their launches) | "
                         f"{counted['steps_timed']} |")
        if "algorithmic_bytes_per_launch" in entry:
            lines.append(f"| algorithmic bytes per launch | {entry['algorithmic_bytes_per_launch'] / 1e6:.2f} MB |")
        lines += ["", "Kernel stats of the traced run (every launch, warm-up and untimed runs included):", "",
                  "| Kernel | Calls | Average µs | Min µs | Max µs |", "|---|---|---|---|---|"]
        for row in stats:
            lines.append(f"| `{row['Name'][:110]}` | {row['Calls']} | {float(row['AverageNs']) / 1e3:.2f} | "
                         f"{float(row['MinNs']) / 1e3:.2f} | {float(row['MaxNs']) / 1e3:.2f} |")
        (summaries / f"{short}_{key}.md").write_text("\n".join(lines) + "\n")

    block = {"sources": digest, "calibration": calibration, "workloads": workloads}
    table = ["| Workload | Kernel | FETCH MB | WRITE MB | Per launch MB | Algorithmic MB |", "|---|---|---|---|---|---|"]
    for key, e in sorted(workloads.items()):
        alg = e.get("algorithmic_bytes_per_launch")
        table.append(f"| {key} | `{e['kernel']}` | {(e['fetch_bytes'] or 0) / 1e6:.2f} | "
                     f"{(e['write_bytes'] or 0) / 1e6:.2f} | {(e['bytes_per_launch'] or 0) / 1e6:.2f} | "
                     f"{alg / 1e6 if alg else float('nan'):.2f} |")
    text = "\n".join([
        "# HBM traffic per launch of each workload's dominant kernel",
        "",
        "FETCH_SIZE and WRITE_SIZE (KiB per dispatch, one rocprofv3 `--pmc` pass each, mean over the launches "
        "of the counter run's timed steps: its last two, or a fixed schedule whole), scaled by what the same "
        "counter reads for a 1 GiB device copy "
        f"(FETCH ×{scale['FETCH_SIZE']:.3f}, WRITE ×{scale['WRITE_SIZE']:.3f}).  Made by "
        "`python3 bench.py --profile <dir>`; bench.py uses these figures only while the kernel sources hash "
        f"to `{digest}`.",
        "",
        *table,
        "",
        "```json",
        json.dumps(block, indent=1),
        "```",
        "",
    ])
    (summaries / "hbm_traffic.md").write_text(text)
    if mfma_rows:
        rows = ["| Workload | Kernel | µs per launch | Engine clock GHz | MFMA busy | VALU co-executing (share of busy "
                "cycles) | VALU per MFMA | MFMA per dispatch |", "|---|---|---|---|---|---|---|---|"]
        for key, e in sorted(mfma_rows.items()):
            clock = e.get("clock_ghz")
            rows.append(f"| {key} | `{e['kernel']}` | {e['us_per_launch']} | {clock if clock else '—'} | "
                        f"{e['mfma_busy']:.1%} | {e['coexec_of_busy']:.1%} | {e['valu_per_mfma']} | "
                        f"{e['mfma_per_dispatch']} |")
        shown = mfma_command or "rocprofv3 --pmc " + " ".join(mfma_counters) + " -- python3 -u bench.py --only <W> ..."
        (summaries / MFMA_FILE.name).write_text("\n".join([
            "# Matrix-core utilisation of the encoder kernels",
            "",
            "One rocprofv3 counter pass per workload, per dispatch of its dominant kernel (mean over the last "
            "two steps' launches); made by `python3 bench.py --profile <dir>` with, per workload W:",
            "",
            f"    {shown}",
            "",
            "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs); co-executing = "
            "SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES (matrix cycles during which the same SIMD also "
            "issued vector ALU work); VALU per MFMA = (SQ_INSTS_VALU - SQ_INSTS_MFMA) / SQ_INSTS_MFMA; engine "
            "clock = GRBM_GUI_ACTIVE / 8 / the dispatch's duration, for dispatches of 100 µs and more (the "
            "datasheet's 2.5 PFLOP/s bf16 and 157.3 TFLOP/s fp32 matrix peaks assume 2.4 GHz); the busy share of "
            "short dispatches is a lower bound (the counter's window is wider than the dispatch).  "
            f"Kernel sources digest `{digest}`.",
            "",
            *rows,
            "",
            "```json",
            json.dumps({"sources": digest, "workloads": mfma_rows}, indent=1),
            "```",
            "",
        ]))
    log(f"profile: wrote {summaries}")
    return 0


def short_kernel(name: str) -> str:
    """``void ns::(anonymous namespace)::fwd_ring_kernel<...>(...)`` -> ``fwd_ring_kernel``; a library
    kernel's long generated name (``Cijk_...``) -> its first 24 characters."""
    depth, kept = 0, []
    for ch in name:
        if ch in "<(":
            depth += 1
        if depth == 0:
            kept.append(ch)
        if ch in ">)":
            depth -= 1
    short = "".join(kept).split()[-1].split("::")[-1] if "".join(kept).split() else name
    return short if len(short) <= 48 else short[:24]


def cls_launches(result: dict) -> int:
    return result["roofline"]["launches_per_step"] if result.get("roofline") else 1


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--only", default=None,
                        help="comma-separated workloads to measure alone: " + ", ".join(WORKLOADS))
    parser.add_argument("--no-compare", action="store_true",
                        help="with --only: skip the unfused/reference comparison runs")
    parser.add_argument("--profile", metavar="DIR", default=None,
                        help="rocprofv3 trace and counter runs of the workloads, summaries under DIR/profiles")
    parser.add_argument("--sweep", action="store_true",
                        help="time the encoder kernel over a table of shapes (one launch per line)")
    args = parser.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one GPU: the attention path runs one model per process on one device "
            f"(asked for --gpus {args.gpus}, WORLD_SIZE {world}); run it with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    keys = args.only.split(",") if args.only else None
    for key in keys or []:
        if key not in WORKLOADS:
            print(f"unknown workload {key!r}; one of {', '.join(WORKLOADS)}", file=sys.stderr)
            return 2
    if args.profile:
        chosen = keys or ["sensevoice", *(k for group in GROUPS.values() for k in group)]
        return profile(Path(args.profile), chosen, args.steps, args.warmup)

    import torch

    from asrback_amd import attention

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    if args.sweep:
        shape_sweep(torch, attention)
        return 0

    # One caller-owned workspace for every workload's decode and choice
    # partials, as the decoders hold theirs: a fixed address in the graphs.
    workspace = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")

    def run(key: str, compare: bool = True) -> dict:
        log(f"bench: {key}")
        with attention.workspace(workspace):
            workload = WORKLOADS[key](torch, attention)
            result = measure(torch, workload, key, args.steps, args.warmup, compare)
        del workload
        torch.cuda.empty_cache()
        return result

    if keys:
        for key in keys:
            result = run(key, compare=not args.no_compare)
            if not args.no_cpu_baseline and key in CPU_BASELINES:
                result["cpu_baseline"] = cpu_baseline(key, 5.0)
            print(json.dumps(result), flush=True)
        return 0

    head = run("sensevoice")
    groups = {name: [run(key) for key in group] for name, group in GROUPS.items()}
    baseline = None
    if not args.no_cpu_baseline:
        log("bench: cpu baselines")
        baseline = cpu_baseline("sensevoice", 8.0)
        head["cpu_baseline"] = baseline
        for lines in groups.values():
            for result in lines:
                key = next(k for k, cls in WORKLOADS.items() if cls.name == result["workload"])
                if key in CPU_BASELINES:
                    result["cpu_baseline"] = cpu_baseline(key, 5.0)

    # Each bf16 matrix-core line against the same run's library GEMM too
    # (the datasheet peak assumes a clock the card does not hold under a
    # full matrix-core load).
    gemm = next((r for r in groups.get("calibration", []) if r["workload"] == GemmCalibration.name), None)
    if gemm:
        for result in [head, *(r for lines in groups.values() for r in lines)]:
            roof = result.get("roofline")
            if roof and roof["unit"] == "TFLOP/s" and result["dtype"] == "bf16" and result is not gemm:
                roof["frac_of_library_gemm"] = round(roof["achieved"] / gemm["value"], 4)
    by_key = {"sensevoice": head}
    for lines in groups.values():
        for result in lines:
            by_key[next(k for k, cls in WORKLOADS.items() if cls.name == result["workload"])] = result
    # Every line, in full, on one line of its own; the result line follows it.
    print(json.dumps({"detail": True, "headline": head, **groups}), flush=True)
    roof = {k: v for k, v in head["roofline"].items()
            if k not in ("launches_per_step", "flop_per_byte", "ceiling", "frac_of_ceiling")}
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs resident in HBM)",
        "config": head["config"],
        "roofline": roof,
        "cpu_baseline": None if baseline is None else {k: v for k, v in baseline.items() if k != "seconds"},
        "configs": [config_entry(cfg, key, by_key[key]) for cfg, key in CONFIG_LINES if key in by_key],
    }
    print(json.dumps(line, separators=(",", ":")), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

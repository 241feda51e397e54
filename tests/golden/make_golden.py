"""Writes the attention golden vectors (``attention_cases.npz``).

Inputs are drawn from seeded N(0, 1) generators and rounded to bfloat16
values (exactly representable in both float32 and bfloat16, so the same
inputs serve the fp32 and bf16 kernels); outputs are the float64 closed form
of ``oracle.brute``.  Each case mirrors one attention call site of the
reference, at a small size:

    enc        whisper.py:102-104 (encoder self-attention, no mask)
    prefix     whisper.py:235-237 (causal prompt prefix, q len == k len)
    step       whisper.py:235-237 (decoder step, mask key <= position)
    cross      whisper.py:239-240 (cross-attention, one query per row)
    padded     sensevoice.py:115-133 (key-padding mask / seqused_k)
    packed     qwen3_asr.py:156-180 (packed causal GQA prefill)
    gqa_step   qwen3_asr.py:414-431 (GQA decode, seqused_k = position + 1)

It also writes ``whisper_tiny_greedy.json``: the greedy token ids the CPU
oracle (``oracle.whisper``, float32) decodes for whisper-tiny's shape with
seeded named random weights (``attention_heavy_weights``) and a log-mel input
drawn from N(0, 1), with the top-2 logit gap of every pick (how far each
argmax is from a tie).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import brute  # noqa: E402

WHISPER_SEEDS = {"weights": 0, "mel": 1}
WHISPER_STEPS = 32


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even)."""
    bits = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return bits.astype(np.uint32).view(np.float32)


def normal(rng: np.random.Generator, *shape: int) -> np.ndarray:
    return bf16_round(rng.standard_normal(shape).astype(np.float32))


def cases() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    rng = np.random.default_rng(20261201)

    # enc: (B, H, L, D) non-causal.
    q, k, v = (normal(rng, 2, 3, 37, 64) for _ in range(3))
    out.update(enc_q=q, enc_k=k, enc_v=v, enc_out=brute.attention_bhld(q, k, v))

    # prefix: causal, top-left, q len == k len.
    q, k, v = (normal(rng, 2, 2, 29, 64) for _ in range(3))
    out.update(
        prefix_q=q, prefix_k=k, prefix_v=v,
        prefix_out=brute.attention_bhld(q, k, v, causal="top_left"),
    )

    # step: one query per row over a 40-slot cache, keys 0..position.
    positions = np.array([0, 17, 39], dtype=np.int64)
    q = normal(rng, 3, 2, 1, 64)
    k, v = (normal(rng, 3, 2, 40, 64) for _ in range(2))
    out.update(
        step_q=q, step_k=k, step_v=v, step_positions=positions,
        step_out=brute.attention_bhld(q, k, v, n_keys=positions + 1),
    )

    # cross: one query per row over 50 encoder frames.
    q = normal(rng, 2, 2, 1, 64)
    k, v = (normal(rng, 2, 2, 50, 64) for _ in range(2))
    out.update(cross_q=q, cross_k=k, cross_v=v, cross_out=brute.attention_bhld(q, k, v))

    # padded: SenseVoice shapes, key padding by lengths; every query row
    # (padding rows too) attends to the valid keys.
    lengths = np.array([21, 9, 14], dtype=np.int32)
    q, k, v = (normal(rng, 3, 2, 21, 128) for _ in range(3))
    out.update(
        padded_q=q, padded_k=k, padded_v=v, padded_lengths=lengths,
        padded_out=brute.attention_bhld(q, k, v, n_keys=lengths),
    )

    # packed: three prompts back to back, causal (bottom-right == top-left
    # for q len == k len), 4 query heads over 2 kv heads.
    seqlens = np.array([7, 13, 5], dtype=np.int32)
    tokens = int(seqlens.sum())
    q = normal(rng, tokens, 4, 128)
    k, v = (normal(rng, tokens, 2, 128) for _ in range(2))
    starts = np.concatenate([[0], np.cumsum(seqlens)]).astype(np.int32)
    packed_out = np.zeros((tokens, 4, 128))
    for s in range(len(seqlens)):
        a, b = starts[s], starts[s + 1]
        seq = brute.attention_bhld(
            q[None, a:b].transpose(0, 2, 1, 3),
            k[None, a:b].transpose(0, 2, 1, 3),
            v[None, a:b].transpose(0, 2, 1, 3),
            causal="bottom_right",
        )
        packed_out[a:b] = seq[0].transpose(1, 0, 2)
    out.update(packed_q=q, packed_k=k, packed_v=v, packed_starts=starts, packed_out=packed_out)

    # gqa_step: q (B, 4, 128) over a (B, 24, 2, 128) cache, seqused_k.
    used = np.array([1, 11, 24], dtype=np.int32)
    q = normal(rng, 3, 4, 128)
    k, v = (normal(rng, 3, 24, 2, 128) for _ in range(2))
    gqa = brute.attention_bhld(
        q[:, :, None, :], k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3), n_keys=used
    )
    out.update(
        gqa_step_q=q, gqa_step_k=k, gqa_step_v=v, gqa_step_used=used, gqa_step_out=gqa[:, :, 0]
    )
    return out


def whisper_mel(seed: int):
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, 80, 3000, generator=g)


def whisper_greedy() -> dict:
    import torch

    from oracle import whisper as ow

    torch.set_num_threads(min(8, torch.get_num_threads()))
    model = ow.WhisperForConditionalGeneration(ow.WHISPER_TINY).eval()
    model.load_state_dict(ow.attention_heavy_weights(model, WHISPER_SEEDS["weights"]))
    result = ow.greedy_decode(model, whisper_mel(WHISPER_SEEDS["mel"]), WHISPER_STEPS)
    return {
        "config": ow.WHISPER_TINY,
        "seeds": WHISPER_SEEDS,
        "steps": WHISPER_STEPS,
        "prefix": [ow.SOT, ow.EN, ow.TRANSCRIBE, ow.NO_TIMESTAMPS],
        "tokens": result["tokens"][0],
        "top2_gaps": [round(g, 6) for g in result["gaps"][0]],
    }


def main() -> None:
    import json

    path = HERE / "attention_cases.npz"
    np.savez_compressed(path, **cases())
    print(path)
    path = HERE / "whisper_tiny_greedy.json"
    path.write_text(json.dumps(whisper_greedy(), indent=1) + "\n")
    print(path)


if __name__ == "__main__":
    main()

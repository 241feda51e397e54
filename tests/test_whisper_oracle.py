"""CPU: the Whisper restatement in the oracle reproduces the committed greedy
token fixture, and its decoder steps are invariant to the cache length
they run over (the reference's KV buckets, ``whisper.py:54``, ``:893-896``).
"""

from __future__ import annotations

import json

import pytest
import torch

from conftest import GOLDEN, max_rel_err
from oracle import attention as oa
from oracle import whisper as ow


@pytest.fixture(scope="module")
def fixture():
    return json.loads((GOLDEN / "whisper_tiny_greedy.json").read_text())


def test_fixture_is_not_degenerate(fixture):
    assert len(fixture["tokens"]) == fixture["steps"] == 32
    assert len(set(fixture["tokens"])) >= 5
    assert min(fixture["top2_gaps"]) > 0.05  # far from argmax ties


def test_oracle_reproduces_greedy_fixture(fixture):
    torch.set_num_threads(min(8, torch.get_num_threads()))
    model = ow.WhisperForConditionalGeneration(fixture["config"]).eval()
    model.load_state_dict(ow.attention_heavy_weights(model, fixture["seeds"]["weights"]))
    g = torch.Generator().manual_seed(fixture["seeds"]["mel"])
    mel = torch.randn(1, 80, 3000, generator=g)
    result = ow.greedy_decode(model, mel, fixture["steps"])
    assert result["tokens"][0] == fixture["tokens"]


def test_step_attention_is_bucket_invariant():
    """A decoder step over a 64-slot view equals one over the whole 448-slot
    cache: masked slots contribute nothing."""
    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 6, 1, 64, generator=g, dtype=torch.float64)
    k, v = (torch.randn(2, 6, 448, 64, generator=g, dtype=torch.float64) for _ in range(2))
    positions = torch.tensor([5, 63])
    short = oa.sdpa(q, k[:, :, :64], v[:, :, :64], attn_mask=oa.whisper_step_mask(positions, 64))
    full = oa.sdpa(q, k, v, attn_mask=oa.whisper_step_mask(positions, 448))
    assert max_rel_err(short, full) < 1e-12


def test_decoder_steps_equal_prompt_pass():
    """Pins the oracle's decoder loop (cache writes, step mask, positions):
    feeding a prompt one token at a time through the fixed-shape step path
    (whisper.py:224-228, :260-264) gives the hidden states of the eager
    causal prompt pass (whisper.py:229-237)."""
    config = dict(ow.WHISPER_TINY, vocab_size=600, decoder_layers=2, encoder_layers=1)
    model = ow.WhisperForConditionalGeneration(config).double().eval()
    model.load_state_dict({k: v.double() for k, v in ow.named_weights(model, 3).items()})
    g = torch.Generator().manual_seed(4)
    encoded = torch.randn(2, 1500, 384, generator=g, dtype=torch.float64)
    tokens = torch.randint(0, 600, (2, 6), generator=g)
    with torch.inference_mode():
        cache = model.allocate_cache(2, torch.float64)
        model.set_encoder_output(cache, encoded)
        full = model.model.decoder(tokens, torch.arange(6), cache, 6)
        cache = model.allocate_cache(2, torch.float64)
        model.set_encoder_output(cache, encoded)
        for p in range(6):
            step = model.model.decoder(tokens[:, p : p + 1], torch.full((2,), p), cache, None)
            assert max_rel_err(step[:, 0], full[:, p]) < 1e-10, p


def test_suppress_masks_follow_the_config():
    """whisper.py:536-544: the configured suppress_tokens and every token
    after <|notimestamps|> are never chosen; the first step also suppresses
    begin_suppress_tokens; a config without the lists suppresses only the
    timestamps.  Checked element for element, and through the greedy choice
    on logits that favour a suppressed token."""
    vocab = ow.WHISPER_TINY["vocab_size"]
    config = {"vocab_size": vocab, "suppress_tokens": [1, 2, 7, 50362], "begin_suppress_tokens": [220, 50257]}
    suppress, first = ow.suppress_masks(config)
    expected = torch.zeros(vocab, dtype=torch.bool)
    expected[[1, 2, 7, 50362]] = True
    expected[ow.NO_TIMESTAMPS + 1 :] = True
    assert torch.equal(suppress, expected)
    expected_first = expected.clone()
    expected_first[[220, 50257]] = True
    assert torch.equal(first, expected_first)
    assert not suppress[ow.NO_TIMESTAMPS] and not suppress[220] and suppress[ow.NO_TIMESTAMPS + 1]

    bare, bare_first = ow.suppress_masks({"vocab_size": vocab})
    timestamps = torch.zeros(vocab, dtype=torch.bool)
    timestamps[ow.NO_TIMESTAMPS + 1 :] = True
    assert torch.equal(bare, timestamps) and torch.equal(bare_first, timestamps)

    logits = torch.zeros(2, vocab)
    logits[:, 7] = 5.0  # configured suppression: never chosen
    logits[:, 220] = 4.0  # begin token: not chosen on the first step only
    logits[:, 3] = 1.0
    assert ow.choose(logits, suppress)[0].tolist() == [220, 220]
    assert ow.choose(logits, first)[0].tolist() == [3, 3]

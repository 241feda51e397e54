"""CPU: pins the oracle's Qwen3 text-attention restatement by an invariant
of causal decoding: the packed prefill (gather/valid/tril path,
qwen3_asr.py:167-181) and token-by-token steps over the cache (grouped query
view and step mask, qwen3_asr.py:427-432, :514-515) give the same hidden
states, for prompts of different lengths packed together and written to
arbitrary cache rows."""

from __future__ import annotations

import torch

from conftest import max_rel_err
from oracle import attention as oa
from oracle import qwen3 as oq
from oracle.weights import named_weights

CONFIG = {
    "hidden_size": 256,
    "head_dim": 128,
    "num_attention_heads": 4,
    "num_key_value_heads": 2,
    "intermediate_size": 512,
    "num_hidden_layers": 2,
    "vocab_size": 300,
    "rms_norm_eps": 1e-6,
    "rope_theta": 1e6,
}


def test_packed_prefill_equals_token_by_token_steps():
    model = oq.TextModel(CONFIG).double().eval()
    model.load_state_dict({k: v.double() for k, v in named_weights(model, 2).items()})
    lengths, rows = [5, 9, 3], [1, 2, 0]
    g = torch.Generator().manual_seed(3)
    tokens = [torch.randint(0, 300, (n,), generator=g) for n in lengths]
    cos, sin = oa.rope_tables(1e6, 128, 32, torch.float64)
    shape = (2, 3, 32, 2, 128)
    with torch.inference_mode():
        ids = torch.cat(tokens)
        row_ids = torch.cat([torch.full((n,), r) for n, r in zip(lengths, rows)])
        positions = torch.cat([torch.arange(n) for n in lengths])
        keys, values = torch.zeros(shape, dtype=torch.float64), torch.zeros(shape, dtype=torch.float64)
        packed = model.prefill(model.embed_tokens(ids), keys, values, row_ids, positions,
                               oa.Segments.from_lengths(lengths), cos[positions], sin[positions])
        keys2, values2 = torch.zeros(shape, dtype=torch.float64), torch.zeros(shape, dtype=torch.float64)
        by_row = {r: t for r, t in zip(rows, tokens)}
        starts = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)[:-1]))
        for p in range(max(lengths)):
            active = [r for r in range(3) if p < len(by_row[r])]
            step_tokens = torch.tensor([by_row[r][p] if p < len(by_row[r]) else 0 for r in range(3)])
            out = model.step(step_tokens, torch.full((3,), p), keys2, values2, cos, sin)
            for r in active:
                seg = rows.index(r)
                assert max_rel_err(out[r], packed[starts[seg] + p]) < 1e-10, (r, p)


def _greedy_setup():
    model = oq.TextModel(CONFIG).eval()
    model.load_state_dict(named_weights(model, 5))
    g = torch.Generator().manual_seed(6)
    head = torch.randn(CONFIG["vocab_size"], CONFIG["hidden_size"], generator=g) * 16 * CONFIG["hidden_size"] ** -0.5
    prompt = torch.randint(0, CONFIG["vocab_size"], (23,), generator=g).tolist()
    return model, head, prompt


def test_greedy_loop_equals_teacher_forced_prefill():
    """Pins the oracle's transcriber loop (qwen3_asr.py:1017-1090,
    :1179-1198): each token it emits is the argmax, at the previous
    position, of one causal prefill over the prompt and the tokens before
    it -- so the first token comes from the prompt's last row and every step
    decodes the latest token at its own position."""
    model, head, prompt = _greedy_setup()
    out = oq.greedy_decode(model, head, CONFIG, prompt, 10, eos_ids=[])
    tokens = out["tokens"]
    assert len(tokens) == 10 and out["min_gap"] > 1e-3
    seq = prompt + tokens[:-1]
    n = len(seq)
    shape = (CONFIG["num_hidden_layers"], 1, 64, CONFIG["num_key_value_heads"], CONFIG["head_dim"])
    keys, values = torch.zeros(shape), torch.zeros(shape)
    cos, sin = oa.rope_tables(CONFIG["rope_theta"], CONFIG["head_dim"], 64, torch.float32)
    pos = torch.arange(n)
    with torch.inference_mode():
        hidden = model.prefill(model.embed_tokens(torch.tensor(seq)), keys, values, torch.zeros(n, dtype=torch.long),
                               pos, oa.Segments.from_lengths([n]), cos[pos], sin[pos])
    forced = (hidden[len(prompt) - 1:] @ head.T).argmax(-1).tolist()
    assert forced == tokens


def test_greedy_loop_stops_at_eos_and_limit():
    """A window ends at an EOS id (dropped from the result) or once its
    position reaches len(prompt) - 1 + min(max_new_tokens, cache - len(prompt))
    (qwen3_asr.py:1031-1035, :1193-1195, :1150-1152)."""
    model, head, prompt = _greedy_setup()
    full = oq.greedy_decode(model, head, CONFIG, prompt, 10, eos_ids=[])["tokens"]
    k = next(i for i in range(1, 10) if full[i] not in full[:i])  # first occurrence of a later token
    stopped = oq.greedy_decode(model, head, CONFIG, prompt, 10, eos_ids=[full[k]])["tokens"]
    assert stopped == full[:k]
    assert oq.greedy_decode(model, head, CONFIG, prompt, 4, eos_ids=[])["tokens"] == full[:4]
    # The cache bounds the window too: 23 prompt positions + 5 in a 28-slot cache.
    assert oq.greedy_decode(model, head, CONFIG, prompt, 10, eos_ids=[], cache_length=28)["tokens"] == full[:5]

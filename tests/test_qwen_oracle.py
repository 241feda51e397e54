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

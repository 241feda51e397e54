"""GPU: Gemma 4's attention (``models/gemma4.py:199-282``, ``:486-587``) on the
HIP kernels against the CPU oracle (``oracle/gemma4.py``) with the same
weights and inputs.

Bar: the blocked audio attention (float32, as the reference computes it)
to 1e-5 relative; the text attention modules in float32 to 1e-4 (the
projections and norms run in a different summation order on the GPU), and
in bfloat16 to 2e-2 against the oracle module run in bfloat16 on the CPU
(the same chain of roundings: projections, norms, rotation, attention
output; against a float32 oracle those alone reach ~2.5%).
"""

from __future__ import annotations

import math

import pytest
import torch

from conftest import assert_close, max_rel_err
from oracle import gemma4 as og
from oracle import attention as oa

pytestmark = pytest.mark.gpu

AUDIO = {
    "hidden_size": 256,
    "num_attention_heads": 2,
    "attention_chunk_size": 12,
    "attention_context_left": 13,
    "attention_context_right": 0,
    "attention_logit_cap": 50.0,
    "attention_invalid_logits_value": -1e9,
}
TEXT = {
    "hidden_size": 256,
    "rms_norm_eps": 1e-6,
    "head_dim": 256,
    "global_head_dim": 512,
    "num_attention_heads": 8,
    "num_key_value_heads": 1,
    "sliding_window": 24,
}


def say(*args):
    print(*args, flush=True)


def randn(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


@pytest.mark.parametrize("heads,head_dim,future", [(8, 128, 0), (4, 192, 0), (2, 64, 3), (2, 40, 0)])
def test_local_attention_matches_oracle(device, heads, head_dim, future):
    """Blocks of 12 audio tokens, each seeing itself and the 11 before it
    (Gemma 4 E2B/E4B's audio layers), ragged lengths including tokens past a
    sequence's end, relative keys of 13 distances, soft cap 50.  Head sizes
    64, 128 and 192 run on the matrix-core kernel that takes runs of blocks
    (the last run reaching past the final block); head_dim 40 on the
    one-wave-per-block kernel."""
    from asrback_amd import attention

    say("local attention", heads, head_dim, future)
    chunk, past = 12, 12
    frames, lengths = 75, torch.tensor([75, 40, 7], dtype=torch.int32)
    q = randn(3, frames, heads, head_dim, seed=1, scale=0.3)
    k = randn(3, frames, heads, head_dim, seed=2)
    v = randn(3, frames, heads, head_dim, seed=3)
    rel = randn((chunk + past + future) // 2 + 1, heads, head_dim, seed=4, scale=0.3)
    mask = og.blocked_mask(lengths, frames, chunk, past, future)
    ref = og.local_attention(q, k, v, rel, mask, chunk, past, future, 50.0, -1e9)
    out = attention.local_attention(q.to(device), k.to(device), v.to(device), rel.to(device), lengths.to(device),
                                    chunk=chunk, past=past, future=future, softcap=50.0, invalid=-1e9)
    assert_close(out.cpu(), ref, "f32")


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("chunk,past,future", [(8, 4, 0), (6, 12, 2), (8, 8, 0), (4, 12, 1)])
def test_local_attention_small_contexts(device, head_dim, chunk, past, future):
    """Contexts of 12-24 slots on the matrix-core kernel: at most 16 slots
    (the second score tile empty) and 17-23 (the second tile partly filled,
    its slots packed into other rows), against the oracle."""
    from asrback_amd import attention

    say("local attention small context", head_dim, chunk, past, future)
    heads, frames = 2, 61
    lengths = torch.tensor([61, 33, 5], dtype=torch.int32)
    q = randn(3, frames, heads, head_dim, seed=11, scale=0.3)
    k = randn(3, frames, heads, head_dim, seed=12)
    v = randn(3, frames, heads, head_dim, seed=13)
    rel = randn(past + future + 1, heads, head_dim, seed=14, scale=0.3)
    mask = og.blocked_mask(lengths, frames, chunk, past, future)
    ref = og.local_attention(q, k, v, rel, mask, chunk, past, future, 50.0, -1e9)
    out = attention.local_attention(q.to(device), k.to(device), v.to(device), rel.to(device), lengths.to(device),
                                    chunk=chunk, past=past, future=future, softcap=50.0, invalid=-1e9)
    assert_close(out.cpu(), ref, "f32")


@pytest.mark.parametrize("head_dim,frames,future", [(128, 500, 0), (64, 620, 0), (64, 620, 3)])
def test_local_attention_workgroups_walk_runs(device, head_dim, frames, future):
    """Enough runs of four blocks that a workgroup takes two in a row,
    loading the second while it computes the first (8 sequences x 8 heads of
    500 tokens: 11 runs per (sequence, head), 704 in all for 512 resident
    workgroups; the last workgroup of each pair of heads gets one), with
    ragged lengths; also with three keys past each block (14 relative
    rows)."""
    from asrback_amd import attention

    say("local attention runs", head_dim, frames, future)
    chunk, past, heads, batch = 12, 12, 8, 8
    lengths = torch.tensor([frames, 431, 17, frames - 1, 250, 1, frames, 333], dtype=torch.int32)
    q = randn(batch, frames, heads, head_dim, seed=11, scale=0.3)
    k = randn(batch, frames, heads, head_dim, seed=12)
    v = randn(batch, frames, heads, head_dim, seed=13)
    rel = randn((chunk + past + future) // 2 + 1, heads, head_dim, seed=14, scale=0.3)
    mask = og.blocked_mask(lengths, frames, chunk, past, future)
    ref = og.local_attention(q, k, v, rel, mask, chunk, past, future, 50.0, -1e9)
    out = attention.local_attention(q.to(device), k.to(device), v.to(device), rel.to(device), lengths.to(device),
                                    chunk=chunk, past=past, future=future, softcap=50.0, invalid=-1e9)
    assert_close(out.cpu(), ref, "f32")


def test_audio_attention_module_matches_oracle(device):
    """``AudioAttention.forward(x, positions, mask)`` with its clipped
    projections, per-dimension query scale and relative-key projection
    (gemma4.py:199-282), the mask as the encoder builds it."""
    from asrback_amd import gemma4 as ag

    say("gemma audio attention module")
    torch.manual_seed(5)
    module = ag.AudioAttention(AUDIO)
    with torch.no_grad():
        for p in module.parameters():
            p.copy_(torch.randn_like(p) * 0.05)
    frames, lengths = 50, torch.tensor([50, 23])
    x = randn(2, frames, AUDIO["hidden_size"], seed=6)
    positions = og.relative_positions(AUDIO["hidden_size"], 12, 13, 0)
    mask = og.blocked_mask(lengths, frames, 12, 12, 0)
    with torch.no_grad():
        shape = (2, frames, module.heads, module.head_dim)
        q = module.q_proj(x).view(shape) * module.q_scale * torch.nn.functional.softplus(module.per_dim_scale)
        k = module.k_proj(x).view(shape) * module.k_scale
        v = module.v_proj(x).view(shape)
        rel = module.relative_k_proj(positions).view(-1, module.heads, module.head_dim)
        core = og.local_attention(q, k, v, rel, mask, 12, 12, 0, 50.0, -1e9)
        expected = module.post(core.reshape(2, frames, -1))
        gpu = module.to(device)
        out = gpu(x.to(device), positions.to(device), mask.to(device))
        assert torch.equal(gpu.blocked_mask(lengths.to(device), frames).cpu(), mask)
    assert_close(out.cpu(), expected, "f32")


def _text_pair(layer_type, shared, dtype, device, seed):
    from asrback_amd import gemma4 as ag

    ref = og.TextAttention(TEXT, layer_type, shared)
    g = torch.Generator().manual_seed(seed)
    state = {name: torch.randn(p.shape, generator=g) * (0.5 if "norm" in name else 0.06)
             for name, p in ref.state_dict().items()}
    state = {name: (t + 1.0 if "norm" in name else t).to(dtype).float() for name, t in state.items()}
    ref.load_state_dict(state)
    model = ag.TextAttention(TEXT, layer_type, shared)
    model.load_state_dict(state, strict=True)
    return ref.eval().to(dtype), model.eval().to(device=device, dtype=dtype)


def _tables(head_dim, length, theta, dtype):
    inverse = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    angles = torch.arange(length).float()[:, None] * inverse[None, :]
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos().to(dtype), angles.sin().to(dtype)


@pytest.mark.parametrize("layer_type", ["sliding_attention", "full_attention"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_text_attention_prefill_and_steps_match_oracle(device, layer_type, dtype):
    """Prompt pass over padded prompts (sizes 40, 17, 3) into cache rows,
    then decoder steps at each row's own position (gemma4.py:534-587): q/k/v
    norms, rotary embedding, no scaling, 8 query heads over 1 kv head,
    head_dim 256 with a 24-key window (sliding) or 512 (full); and a KV-shared
    layer reading the same cache and prompt keys.  Steps of layers with their
    own keys run the fused prologue (norms, rotation and cache writes in the
    decode launch) where the decode kernel takes the head size; the cache
    holds what the oracle's holds."""
    from asrback_amd import gemma4 as ag

    say("gemma text attention", layer_type, dtype)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    ref, model = _text_pair(layer_type, False, dtype, device, 7)
    ref_shared, model_shared = _text_pair(layer_type, True, dtype, device, 8)
    window = None if layer_type == "full_attention" else TEXT["sliding_window"]
    hd = model.head_dim
    sizes, longest, cache_len = torch.tensor([40, 17, 3]), 40, 64
    cos, sin = _tables(hd, cache_len, 1e4, dtype)
    x = randn(3, longest, TEXT["hidden_size"], seed=9).to(dtype)
    rows = torch.tensor([2, 0, 1])
    keys = torch.zeros(3, cache_len, 1, hd, dtype=dtype)  # the oracle's cache
    values = torch.zeros_like(keys)
    mask = oa.gemma_prefill_mask(sizes, longest, window)
    with torch.no_grad():
        kv = {}
        expected = ref.prefill(x, keys, values, rows, kv, mask, cos[:longest], sin[:longest]).float()
        expected_shared = ref_shared.prefill(x, keys, values, rows, kv, mask, cos[:longest], sin[:longest]).float()
        cache = ag.LayerKV(torch.zeros(3, cache_len, 1, hd, dtype=dtype, device=device),
                           torch.zeros(3, cache_len, 1, hd, dtype=dtype, device=device))
        kv_d = {}
        out = model.prefill(x.to(device), cache, rows.to(device), kv_d, mask.to(device), cos[:longest].to(device),
                            sin[:longest].to(device))
        out_shared = model_shared.prefill(x.to(device), cache, rows.to(device), kv_d, mask.to(device),
                                          cos[:longest].to(device), sin[:longest].to(device))
    for b, n in enumerate(sizes.tolist()):
        assert_close(out[b, :n].float().cpu(), expected[b, :n], "f32" if tol == 1e-5 else "bf16", tol)
        assert_close(out_shared[b, :n].float().cpu(), expected_shared[b, :n], "f32" if tol == 1e-5 else "bf16", tol)
    # Steps: each cache row continues after its prompt (row 2 holds prompt 0, ...).
    positions = torch.zeros(3, dtype=torch.long)
    positions[rows] = sizes
    for step in range(3):
        xs = randn(3, TEXT["hidden_size"], seed=20 + step).to(dtype)
        step_mask = oa.gemma_step_mask(positions, cache_len, window)
        with torch.no_grad():
            expected = ref.step(xs, keys, values, positions, step_mask, cos[positions], sin[positions]).float()
            expected_shared = ref_shared.step(xs, keys, values, positions, step_mask, cos[positions],
                                              sin[positions]).float()
            out = model.step(xs.to(device), cache, positions.to(device), step_mask.to(device),
                             cos[positions].to(device), sin[positions].to(device))
            out_shared = model_shared.step(xs.to(device), cache, positions.to(device), step_mask.to(device),
                                           cos[positions].to(device), sin[positions].to(device))
        assert_close(out.float().cpu(), expected, "f32" if tol == 1e-5 else "bf16", tol)
        assert_close(out_shared.float().cpu(), expected_shared, "f32" if tol == 1e-5 else "bf16", tol)
        positions += 1
    assert max_rel_err(cache.keys.float().cpu(), keys.float()) < (1e-5 if dtype == torch.float32 else 1e-2)
    assert max_rel_err(cache.values.float().cpu(), values.float()) < (1e-5 if dtype == torch.float32 else 1e-2)

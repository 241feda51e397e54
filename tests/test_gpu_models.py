"""GPU: the SenseVoice and Qwen3-ASR modules on the HIP kernels against their
CPU restatements in the oracle, with the same seeded named weights.

Whole-module outputs include GEMMs, norms and convolutions that run in a
different summation order on the GPU, so float32 module outputs are held to
1e-4 relative (the attention kernels alone meet 1e-5 in test_gpu_configs);
structural invariants (padding, GQA mask forms, graph replay) are held
tighter where the arithmetic is identical.
"""

from __future__ import annotations

import pytest
import torch

from conftest import assert_close, max_rel_err
from oracle import attention as oa
from oracle import qwen3 as oq
from oracle import sensevoice as osv
from oracle.weights import named_weights

pytestmark = pytest.mark.gpu

SENSEVOICE = {
    "output_size": 512,
    "attention_heads": 4,
    "linear_units": 2048,
    "kernel_size": 11,
    "num_blocks": 2,
    "tp_blocks": 1,
}
QWEN3 = {
    "hidden_size": 512,
    "head_dim": 128,
    "num_attention_heads": 4,
    "num_key_value_heads": 2,
    "intermediate_size": 1024,
    "num_hidden_layers": 2,
    "vocab_size": 1000,
    "rms_norm_eps": 1e-6,
    "rope_theta": 1e6,
}


def say(*args):
    print(*args, flush=True)


# --- SenseVoice ----------------------------------------------------------------


def sensevoice_pair(device):
    from asrback_amd import sensevoice as asv

    ref = osv.SenseVoiceEncoder(560, SENSEVOICE).eval()
    state = named_weights(ref, 5)
    ref.load_state_dict(state)
    model = asv.SenseVoiceEncoder(560, SENSEVOICE)
    model.load_state_dict(state, strict=True)
    return ref, model.eval().to(device)


def test_sensevoice_encoder_matches_oracle(device):
    """Padded ragged batch with the frame mask (sensevoice.py:543-561)."""
    say("sensevoice encoder")
    ref, model = sensevoice_pair(device)
    frames = torch.tensor([80, 40, 120, 7])
    g = torch.Generator().manual_seed(6)
    x = torch.randn(4, 4 + 120, 560, generator=g)
    mask = osv.frame_mask(frames, 4, 120)
    with torch.inference_mode():
        expected = ref(x, mask)
        out = model(x.to(device), mask.to(device))
    valid = mask[..., None]
    assert_close(out.cpu() * valid, expected * valid, "module", 1e-4)


def test_sensevoice_padding_invariance(device):
    """A padded batch gives each row what it gets alone (docs/architecture.md:427-429)."""
    say("sensevoice padding invariance")
    _, model = sensevoice_pair(device)
    frames = [60, 23, 91]
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 4 + 91, 560, generator=g)
    for b, n in enumerate(frames):
        x[b, 4 + n :] = 0
    mask = osv.frame_mask(torch.tensor(frames), 4, 91).to(device)
    with torch.inference_mode():
        batched = model(x.to(device), mask)
        for b, n in enumerate(frames):
            alone = model(x[b : b + 1, : 4 + n].to(device), None)
            assert_close(batched[b, : 4 + n].cpu(), alone[0].cpu(), "f32")


def test_sensevoice_layer_bf16_matches_oracle(device):
    """One SAN-M attention module in bfloat16 (fused attention + FSMN, one
    GEMM for linear_out + memory) against the oracle's module in float32 on
    the same bf16-rounded weights and inputs, on the valid frames; padded
    frames carry linear_out's bias alone (their attention is skipped)."""
    from asrback_amd import sensevoice as asv

    say("sensevoice layer bf16")
    ref = osv.SANMAttention(512, 512, 4, 11).eval()
    state = {k: v.to(torch.bfloat16).float() for k, v in named_weights(ref, 8).items()}
    ref.load_state_dict(state)
    model = asv.SANMAttention(512, 512, 4, 11)
    model.load_state_dict(state, strict=True)
    model = model.eval().to(device=device, dtype=torch.bfloat16)
    frames = torch.tensor([300, 120, 9, 257])
    g = torch.Generator().manual_seed(9)
    x = torch.randn(4, 300, 512, generator=g).to(torch.bfloat16)
    mask = osv.frame_mask(frames, 0, 300)
    with torch.inference_mode():
        expected = ref(x.float(), mask, None)
        out = model(x.to(device), mask.to(device), None)
        model.zero_padded_rows = False
        computed = model(x.to(device), mask.to(device), None)
    valid = mask[..., None]
    assert_close(out.float().cpu() * valid, expected * valid, "bf16")
    assert_close(out.float().cpu()[mask], expected[mask], "bf16")
    # Skipping the padded frames changes no valid frame, bit for bit.
    assert torch.equal(out[mask.to(device)], computed[mask.to(device)])
    bias = model.linear_out.bias.detach()
    for b, n in enumerate(frames.tolist()):
        assert torch.equal(out[b, n:], bias.expand(300 - n, 512))


# --- Qwen3-ASR -------------------------------------------------------------------


def qwen_pair(device):
    from asrback_amd import qwen3_asr as aq

    ref = oq.TextModel(QWEN3).eval()
    state = named_weights(ref, 8)
    ref.load_state_dict(state)
    model = aq.TextModel(QWEN3)
    model.load_state_dict(state, strict=True)
    return ref, model.eval().to(device)


def test_qwen_prefill_and_steps_match_oracle(device):
    """Packed causal GQA prefill into cache rows, then decoder steps over the
    cache with seqused_k = position + 1 (qwen3_asr.py:374-432, :472-524)."""
    from asrback_amd import qwen3_asr as aq

    say("qwen3 prefill + steps")
    ref, model = qwen_pair(device)
    lengths = [37, 52, 29]
    rows = [2, 0, 1]
    batch, cache_len = 3, 128
    g = torch.Generator().manual_seed(9)
    x = torch.randn(sum(lengths), QWEN3["hidden_size"], generator=g)
    row_ids = torch.cat([torch.full((n,), r) for n, r in zip(lengths, rows)])
    positions = torch.cat([torch.arange(n) for n in lengths])
    cos, sin = oa.rope_tables(QWEN3["rope_theta"], 128, cache_len, torch.float32)
    shape = (2, batch, cache_len, 2, 128)
    keys_ref, values_ref = torch.zeros(shape), torch.zeros(shape)
    cache = aq.KVCache.allocate(QWEN3, batch, cache_len, device, torch.float32)
    with torch.inference_mode():
        h_ref = ref.prefill(x, keys_ref, values_ref, row_ids, positions, oq.oa.Segments.from_lengths(lengths),
                            cos[positions], sin[positions])
        segments = aq.Segments.from_lengths(lengths, device)
        cos_d, sin_d = cos.to(device), sin.to(device)
        pos_d = positions.to(device)
        h = model.prefill(x.to(device), cache, row_ids.to(device), pos_d, segments, cos_d[pos_d], sin_d[pos_d])
        assert_close(h.cpu(), h_ref, "module", 1e-4)
        assert_close(cache.keys.cpu(), keys_ref, "module", 1e-4)

        step_pos = torch.tensor([lengths[rows.index(r)] for r in range(batch)])
        for step in range(5):
            tokens = torch.randint(0, QWEN3["vocab_size"], (batch,), generator=g)
            s_ref = ref.step(tokens, step_pos, keys_ref, values_ref, cos, sin)
            s = model.step(tokens.to(device), step_pos.to(device), cache, cos_d, sin_d)
            assert_close(s.cpu(), s_ref, "module", 1e-4, f"step {step}")
            step_pos = step_pos + 1


def test_qwen_step_mask_forms_agree(device):
    """The reference's three step masks -- varlen tuple, boolean mask over a
    shorter bucket view, KeyPrefix -- give the same attention."""
    from asrback_amd import qwen3_asr as aq
    from asrback_amd.attention import KeyPrefix

    say("qwen3 mask forms")
    torch.manual_seed(10)
    attn = aq.TextAttention(QWEN3).to(device).eval()
    batch = 4
    keys = torch.randn(batch, 1024, 2, 128, device=device)
    values = torch.randn(batch, 1024, 2, 128, device=device)
    positions = torch.tensor([3, 100, 511, 255], device=device)
    x = torch.randn(batch, QWEN3["hidden_size"], device=device)
    cos, sin = aq.rope_tables(QWEN3, 1024, device, torch.float32)
    cos, sin = cos[positions], sin[positions]
    lengths = (positions + 1).to(torch.int32)
    starts = torch.arange(batch + 1, dtype=torch.int32, device=device)
    with torch.inference_mode():
        a = attn.step(x, keys.clone(), values.clone(), positions, (starts, starts * 1024, lengths), cos, sin)
        mask = oa.qwen_step_mask(positions, 512)
        b = attn.step(x, keys.clone()[:, :512], values.clone()[:, :512], positions, mask, cos, sin)
        c = attn.step(x, keys.clone(), values.clone(), positions, KeyPrefix(lengths=lengths), cos, sin)
        # The step mask of these very positions takes the fused kernel
        # (norms, rotation, cache write and attention in one launch).
        fused_keys, fused_values = keys.clone(), values.clone()
        d = attn.step(x, fused_keys, fused_values, positions, KeyPrefix(positions=positions), cos, sin)
        ref_keys = keys.clone()
        attn.step(x, ref_keys, values.clone(), positions, KeyPrefix(lengths=lengths), cos, sin)
    assert max_rel_err(b, a) < 1e-6
    assert torch.equal(a, c)
    assert_close(d, a, "f32")
    assert max_rel_err(fused_keys, ref_keys) < 1e-6


def test_qwen_step_replays_from_graph(device):
    """The decoder step of TextModel captured in a hipGraph and replayed at
    advancing positions matches eager steps."""
    from asrback_amd import qwen3_asr as aq
    from asrback_amd.transcription import CapturedGraph

    say("qwen3 graph replay")
    _, model = qwen_pair(device)
    batch = 4
    cache = aq.KVCache.allocate(QWEN3, batch, 256, device, torch.float32)
    torch.nn.init.normal_(cache.keys)
    torch.nn.init.normal_(cache.values)
    snapshot = (cache.keys.clone(), cache.values.clone())
    cos, sin = aq.rope_tables(QWEN3, 256, device, torch.float32)
    tokens = torch.tensor([1, 2, 3, 4], device=device)
    positions = torch.tensor([10, 50, 0, 200], device=device)
    out = torch.empty(batch, QWEN3["hidden_size"], device=device)

    def step():
        out.copy_(model.step(tokens, positions, cache, cos, sin))
        positions.add_(1)

    with torch.inference_mode():
        graph = CapturedGraph(step)
        # Reset after warm-up and capture, then replay 3 steps.
        cache.keys.copy_(snapshot[0])
        cache.values.copy_(snapshot[1])
        positions.copy_(torch.tensor([10, 50, 0, 200]))
        replayed = []
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            replayed.append(out.clone())
        cache.keys.copy_(snapshot[0])
        cache.values.copy_(snapshot[1])
        pos = torch.tensor([10, 50, 0, 200], device=device)
        for i in range(3):
            eager = model.step(tokens, pos, cache, cos, sin)
            assert torch.equal(eager, replayed[i]), i
            pos = pos + 1


def test_qwen_audio_attention_windows(device):
    """Windowed non-causal audio attention, 16 heads x 64 (qwen3_asr.py:207-221, :303-310)."""
    from asrback_amd import qwen3_asr as aq

    say("qwen3 audio windows")
    ref = oq.AudioAttention(1024, 16).eval()
    state = named_weights(ref, 11)
    ref.load_state_dict(state)
    model = aq.AudioAttention(1024, 16)
    model.load_state_dict(state, strict=True)
    model = model.eval().to(device)
    lengths = [104, 104, 37, 81]
    g = torch.Generator().manual_seed(12)
    x = torch.randn(sum(lengths), 1024, generator=g)
    with torch.inference_mode():
        expected = ref(x, oa.Segments.from_lengths(lengths))
        out = model(x.to(device), aq.Segments.from_lengths(lengths, device))
    assert_close(out.cpu(), expected, "module", 1e-4)


def _qwen_decoder(device, graphs, eos_ids, **cache):
    from asrback_amd import qwen3_asr as aq

    ref, model = qwen_pair(device)
    g = torch.Generator().manual_seed(21)
    head = torch.randn(QWEN3["vocab_size"], QWEN3["hidden_size"], generator=g) * 16 * QWEN3["hidden_size"] ** -0.5
    prompts = [torch.randint(0, QWEN3["vocab_size"], (n,), generator=g).tolist() for n in (37, 52, 29)]
    lm_head = torch.nn.Linear(QWEN3["hidden_size"], QWEN3["vocab_size"], bias=False)
    lm_head.weight.data.copy_(head)
    decoder = aq.TextGreedyDecoder(model, lm_head.to(device), QWEN3, 4, eos_ids, graphs=graphs, **cache)
    expected = [oq.greedy_decode(ref, head, QWEN3, p, 12, eos_ids) for p in prompts]
    for e in expected:
        assert e["min_gap"] > 0.1  # far from argmax ties
    return decoder, prompts, [e["tokens"] for e in expected]


def _drain(decoder, results):
    while decoder.rows:
        decoder.advance()
        for slot, (tokens, _) in decoder.finished_rows().items():
            results[slot] = tokens


def test_qwen_greedy_decoder_matches_oracle(device):
    """Qwen3 transcriber loop on the kernels -- packed prompts prefilled into
    free rows, graph-replayed steps, EOS checks every few steps -- emits the
    oracle's greedy tokens; EOS id 989 ends the third window early."""
    say("qwen3 greedy decoder, graphs")
    decoder, prompts, expected = _qwen_decoder(device, True, [989])
    assert 989 not in expected[2] and len(expected[2]) < 12 and len(expected[0]) == 12
    slots = decoder.admit(prompts, 12)
    results = {}
    _drain(decoder, results)
    assert [results[s] for s in slots] == expected


def test_qwen_greedy_decoder_staggered_rows(device):
    """Windows admitted while others are mid-decode get the same tokens as
    alone: rows do not interact."""
    say("qwen3 greedy decoder, staggered admission")
    decoder, prompts, expected = _qwen_decoder(device, True, [])
    first = decoder.admit(prompts[:2], 12)
    results = {}
    decoder.advance()
    third = decoder.admit(prompts[2:], 12)
    _drain(decoder, results)
    assert [results[s] for s in first + third] == expected


def test_qwen_greedy_decoder_paged_cache(device):
    """The same windows on a paged cache of 16-position pages, with a pool of
    only 14 pages (224 positions, against the slab's 4 x 1024): each row
    holds the pages for its prompt and 12 new tokens, staggered admissions
    reuse the pages freed by finished rows, and the tokens are the oracle's
    (qwen3_asr.py:511-512 generalized)."""
    say("qwen3 greedy decoder, paged cache")
    decoder, prompts, expected = _qwen_decoder(device, True, [], page_size=16, num_pages=14)
    cache = decoder.cache
    first = decoder.admit(prompts[:2], 12)  # (37 + 12) and (52 + 12) positions: 4 + 4 pages
    assert len(cache.free_pages) == 14 - 8
    results = {}
    decoder.advance()
    with pytest.raises(RuntimeError, match="exhausted"):
        decoder.admit([prompts[1], prompts[1]], 12)  # 8 pages wanted, 6 free
    assert len(cache.free_pages) == 6
    third = decoder.admit(prompts[2:], 12)  # 29 + 12 positions: 3 pages
    _drain(decoder, results)
    assert [results[s] for s in first + third] == expected
    assert sorted(cache.free_pages) == list(range(14)) and bool((cache.block_table == -1).all())
    again = decoder.admit(prompts, 12)
    results = {}
    _drain(decoder, results)
    assert [results[s] for s in again] == expected


def test_qwen_greedy_decoder_eager_equals_graphs(device):
    """Eager steps give the graphs' tokens."""
    say("qwen3 greedy decoder, eager")
    decoder, prompts, expected = _qwen_decoder(device, False, [])
    slots = decoder.admit(prompts, 12)
    results = {}
    _drain(decoder, results)
    assert [results[s] for s in slots] == expected

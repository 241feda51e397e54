"""CPU: pins the oracle (``oracle/``) before any GPU result is compared with it.

The oracle's attention calls go through torch's CPU SDPA; here they are
checked against the independent float64 brute force (``oracle.brute``) and
the committed golden vectors, and the brute force itself against special
cases with known answers.  Mistakes these catch: a transposed mask, causal
alignment off by one, the wrong kv head for a query head, a missing scale.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import GOLDEN, max_rel_err
from oracle import attention as oa
from oracle import brute


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN / "attention_cases.npz")


def t64(x):
    return torch.from_numpy(np.asarray(x)).double()


# --- the brute force against answers the mathematics fixes ---------------


def test_brute_single_key_returns_its_value():
    rng = np.random.default_rng(0)
    q, k, v = rng.standard_normal((3, 1, 8))
    out = brute.attention_rows(q, k, v, np.ones((1, 1), bool))
    np.testing.assert_allclose(out, v, rtol=0, atol=1e-15)


def test_brute_identical_keys_average_values():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((2, 8))
    k = np.repeat(rng.standard_normal((1, 8)), 5, axis=0)
    v = rng.standard_normal((5, 8))
    out = brute.attention_rows(q, k, v, np.ones((2, 5), bool))
    np.testing.assert_allclose(out, np.repeat(v.mean(0, keepdims=True), 2, 0), atol=1e-14)


def test_brute_two_keys_closed_form():
    # softmax of two scores is a logistic function of their difference.
    q = np.array([[1.0, 2.0, 0.0, 0.0]])
    k = np.array([[1.0, 0.0, 0.0, 0.0], [0.0, 1.0, 0.0, 0.0]])
    v = np.array([[1.0, 0.0, 0.0, 0.0], [0.0, 1.0, 0.0, 0.0]])
    scale = 0.5
    w1 = 1.0 / (1.0 + math.exp(-(2.0 - 1.0) * scale))
    out = brute.attention_rows(q, k, v, np.ones((1, 2), bool), scale)
    np.testing.assert_allclose(out[0, :2], [1 - w1, w1], atol=1e-15)


def test_brute_masks():
    top = brute.visible_mask(3, 3, causal="top_left")
    assert top.tolist() == [[1, 0, 0], [1, 1, 0], [1, 1, 1]]
    bottom = brute.visible_mask(2, 4, causal="bottom_right")
    assert bottom.tolist() == [[1, 1, 1, 0], [1, 1, 1, 1]]
    padded = brute.visible_mask(2, 4, n_keys=2)
    assert padded.tolist() == [[1, 1, 0, 0], [1, 1, 0, 0]]


# --- the oracle's call patterns against the golden vectors ---------------


def test_oracle_encoder_matches_golden(golden):
    q, k, v = (t64(golden[f"enc_{n}"]) for n in "qkv")
    assert max_rel_err(oa.sdpa(q, k, v), golden["enc_out"]) < 1e-12


def test_oracle_prefix_matches_golden(golden):
    q, k, v = (t64(golden[f"prefix_{n}"]) for n in "qkv")
    assert max_rel_err(oa.sdpa(q, k, v, is_causal=True), golden["prefix_out"]) < 1e-12


def test_oracle_step_matches_golden(golden):
    q, k, v = (t64(golden[f"step_{n}"]) for n in "qkv")
    positions = torch.from_numpy(golden["step_positions"])
    mask = oa.whisper_step_mask(positions, k.shape[2])
    assert max_rel_err(oa.sdpa(q, k, v, attn_mask=mask), golden["step_out"]) < 1e-12


def test_oracle_cross_matches_golden(golden):
    q, k, v = (t64(golden[f"cross_{n}"]) for n in "qkv")
    assert max_rel_err(oa.sdpa(q, k, v), golden["cross_out"]) < 1e-12


def test_oracle_sensevoice_padding_matches_golden(golden):
    q, k, v = (t64(golden[f"padded_{n}"]) for n in "qkv")  # (B, H, L, D)
    lengths = torch.from_numpy(golden["padded_lengths"])
    batch, heads, length, dim = q.shape
    fused = torch.cat([t.transpose(1, 2).reshape(batch, length, heads * dim) for t in (q, k, v)], -1)
    mask = oa.key_padding_mask(lengths, length)
    out = oa.sensevoice_attention(fused, heads, mask)
    ref = torch.from_numpy(golden["padded_out"]).transpose(1, 2).reshape(batch, length, heads * dim)
    assert max_rel_err(out, ref) < 1e-12


def test_oracle_packed_gqa_matches_golden(golden):
    q, k, v = (t64(golden[f"packed_{n}"]) for n in "qkv")
    starts = golden["packed_starts"]
    segments = oa.Segments.from_lengths(np.diff(starts).tolist())
    out = oa.qwen_attend(q, k, v, segments, causal=True)
    assert max_rel_err(out, golden["packed_out"]) < 1e-12


def test_oracle_gqa_step_matches_golden(golden):
    q, k, v = (t64(golden[f"gqa_step_{n}"]) for n in "qkv")
    used = torch.from_numpy(golden["gqa_step_used"]).long()
    mask = oa.qwen_step_mask(used - 1, k.shape[1])
    out = oa.qwen_step_attention(q, k, v, mask)
    assert max_rel_err(out, golden["gqa_step_out"]) < 1e-12


# --- invariants -------------------------------------------------------------


def test_step_equals_last_row_of_causal_prefill():
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 3, 17, 64, generator=g, dtype=torch.float64) for _ in range(3))
    full = oa.sdpa(q, k, v, is_causal=True)
    for p in (0, 5, 16):
        mask = oa.whisper_step_mask(torch.tensor([p, p]), 17)
        step = oa.sdpa(q[:, :, p : p + 1], k, v, attn_mask=mask)
        assert max_rel_err(step, full[:, :, p : p + 1]) < 1e-12


def test_gemma_masks_match_explicit_loops():
    """gemma4.py:717-725 (step) and :1227-1235 (prompt pass), restated as
    loops over (row, query, key)."""
    positions, length, window = torch.tensor([0, 3, 9, 15]), 16, 5
    for w in (None, window):
        step = oa.gemma_step_mask(positions, length, w)
        for b, p in enumerate(positions.tolist()):
            for j in range(length):
                want = j <= p and (w is None or j > p - w)
                assert bool(step[b, 0, 0, j]) == want
    sizes, longest = torch.tensor([16, 7, 1]), 16
    for w in (None, window):
        mask = oa.gemma_prefill_mask(sizes, longest, w)
        assert mask.shape == (3, 1, 16, 16)
        for b, n in enumerate(sizes.tolist()):
            for i in range(longest):
                for j in range(longest):
                    want = j <= i and j < n and (w is None or j > i - w)
                    assert bool(mask[b, 0, i, j]) == want


def test_gemma_window_step_equals_prefill_row_and_window_slice():
    """Unscaled (scale=1.0) windowed attention: a step at position p equals
    row p of the windowed prompt pass, and equals plain attention over the
    keys p - w + 1 .. p alone."""
    g = torch.Generator().manual_seed(12)
    q, k, v = (torch.randn(1, 2, 20, 16, generator=g, dtype=torch.float64) * 0.3 for _ in range(3))
    w = 6
    full = oa.sdpa(q, k, v, attn_mask=oa.gemma_prefill_mask(torch.tensor([20]), 20, w), scale=1.0)
    for p in (0, 4, 5, 6, 19):
        step = oa.sdpa(q[:, :, p : p + 1], k, v, attn_mask=oa.gemma_step_mask(torch.tensor([p]), 20, w), scale=1.0)
        assert max_rel_err(step, full[:, :, p : p + 1]) < 1e-12
        lo = max(0, p - w + 1)
        sliced = oa.sdpa(q[:, :, p : p + 1], k[:, :, lo : p + 1], v[:, :, lo : p + 1], scale=1.0)
        assert max_rel_err(step, sliced) < 1e-12
        # closed form, scale 1: per head, softmax of the raw dot products
        weights = torch.einsum("hd,hjd->hj", q[0, :, p], k[0, :, lo : p + 1]).softmax(-1)
        assert max_rel_err(step[0, :, 0], torch.einsum("hj,hjd->hd", weights, v[0, :, lo : p + 1])) < 1e-12


def test_step_is_independent_of_cache_bucket():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(3, 2, 1, 64, generator=g, dtype=torch.float64)
    k, v = (torch.randn(3, 2, 448, 64, generator=g, dtype=torch.float64) for _ in range(2))
    positions = torch.tensor([3, 40, 63])
    outs = [
        oa.sdpa(q, k[:, :, :L], v[:, :, :L], attn_mask=oa.whisper_step_mask(positions, L))
        for L in (64, 128, 256, 448)
    ]
    for out in outs[1:]:
        assert max_rel_err(out, outs[0]) < 1e-12


def test_padded_batch_equals_per_sequence_runs():
    g = torch.Generator().manual_seed(5)
    lengths = torch.tensor([11, 4, 8])
    fused = torch.randn(3, 11, 3 * 256, generator=g, dtype=torch.float64)
    out = oa.sensevoice_attention(fused, 2, oa.key_padding_mask(lengths, 11))
    for b, n in enumerate(lengths.tolist()):
        alone = oa.sensevoice_attention(fused[b : b + 1, :n], 2, None)
        assert max_rel_err(out[b, :n], alone[0]) < 1e-12


def test_gqa_equals_repeated_kv_heads():
    g = torch.Generator().manual_seed(6)
    q = torch.randn(2, 4, 128, generator=g, dtype=torch.float64)
    k, v = (torch.randn(2, 30, 2, 128, generator=g, dtype=torch.float64) for _ in range(2))
    mask = oa.qwen_step_mask(torch.tensor([10, 29]), 30)
    grouped = oa.qwen_step_attention(q, k, v, mask)
    # MHA with kv head h // 2 repeated for query head h.
    k_rep = k.repeat_interleave(2, dim=2).transpose(1, 2)
    v_rep = v.repeat_interleave(2, dim=2).transpose(1, 2)
    mha = oa.sdpa(q[:, :, None], k_rep, v_rep, attn_mask=mask)[:, :, 0]
    assert max_rel_err(grouped, mha) < 1e-12


def test_rope_identity_at_position_zero_and_norm_preserving():
    cos, sin = oa.rope_tables(1e6, 128, 1024, torch.float64)
    x = torch.randn(5, 16, 128, dtype=torch.float64, generator=torch.Generator().manual_seed(40))
    assert torch.equal(oa.rotate(x, cos[0].expand(5, 128), sin[0].expand(5, 128)), x)
    positions = torch.tensor([1, 7, 100, 555, 1023])
    rotated = oa.rotate(x, cos[positions], sin[positions])
    # The angles are float32 (as the reference computes them): cos^2 + sin^2
    # is 1 to about 1e-8.
    torch.testing.assert_close(rotated.norm(dim=-1), x.norm(dim=-1), rtol=1e-7, atol=0)


def test_rope_scores_depend_only_on_position_difference():
    cos, sin = oa.rope_tables(1e6, 128, 1024, torch.float64)
    g = torch.Generator().manual_seed(41)
    q = torch.randn(1, 1, 128, dtype=torch.float64, generator=g)
    k = torch.randn(1, 1, 128, dtype=torch.float64, generator=g)

    def score(m, n):
        qm = oa.rotate(q, cos[m : m + 1], sin[m : m + 1])
        kn = oa.rotate(k, cos[n : n + 1], sin[n : n + 1])
        return float((qm * kn).sum())

    # The angles are float32 (as the reference computes them): each is off
    # by at most 2^-24 of its value (frequencies <= 1), so the two scores
    # differ by at most twice that at position 507 times |q| |k|.
    bound = 2 * 507 * 2.0**-24 * float(q.norm() * k.norm())
    assert abs(score(10, 3) - score(507, 500)) < bound
    assert abs(score(0, 0) - float((q * k).sum())) < 1e-12


def test_rms_norm_formula():
    g = torch.Generator().manual_seed(42)
    x = torch.randn(4, 16, 128, dtype=torch.float64, generator=g)
    w = torch.randn(128, dtype=torch.float64, generator=g)
    ref = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
    torch.testing.assert_close(oa.rms_norm(x, w, 1e-6), ref, rtol=1e-12, atol=1e-12)


def test_fsmn_matches_explicit_loop():
    g = torch.Generator().manual_seed(7)
    value = torch.randn(2, 9, 4, generator=g, dtype=torch.float64)
    weight = torch.randn(4, 1, 11, generator=g, dtype=torch.float64)
    mask = oa.key_padding_mask(torch.tensor([9, 6]), 9)
    out = oa.fsmn_memory(value, mask, weight, 11)
    keep = mask[..., None].double()
    masked = value * keep
    ref = torch.zeros_like(value)
    for b in range(2):
        for t in range(9):
            for c in range(4):
                acc = 0.0
                for i in range(11):
                    s = t + i - 5  # left padding (11 - 1) // 2 = 5
                    if 0 <= s < 9:
                        acc += float(weight[c, 0, i]) * float(masked[b, s, c])
                ref[b, t, c] = acc
    ref = (ref + masked) * keep
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)


# --- Gemma 4 blocked audio attention ------------------------------------------


@pytest.mark.parametrize("frames,lengths,future", [(29, [29, 17, 1], 0), (25, [25, 9], 3)])
def test_gemma_local_attention_matches_definition(frames, lengths, future):
    """The reference's unfold + relative-shift route (gemma4.py:256-282)
    equals the definition evaluated query by query (relative row t - c,
    i.e. distance past - r; invalid score outside each query's window and the
    sequence's length), including padded queries that see no key."""
    from oracle import gemma4 as og

    chunk, past, heads, head_dim = 4, 5, 2, 8
    g = torch.Generator().manual_seed(14)
    q, k, v = (torch.randn(len(lengths), frames, heads, head_dim, generator=g, dtype=torch.float64)
               for _ in range(3))
    rel_rows = (chunk + past + future) // 2 + 1
    relative = torch.randn(rel_rows, heads, head_dim, generator=g, dtype=torch.float64)
    lengths_t = torch.tensor(lengths)
    mask = og.blocked_mask(lengths_t, frames, chunk, past, future)
    out = og.local_attention(q, k, v, relative, mask, chunk, past, future, 7.0, -1e9)
    ref = og.local_attention_loops(q, k, v, relative, lengths_t, chunk, past, future, 7.0, -1e9)
    assert max_rel_err(out, ref) < 1e-12


def test_gemma_relative_positions_and_window():
    """Relative row r holds the sinusoids of distance context // 2 - r, and a
    query's visible keys are itself and the past - 1 before it
    (gemma4.py:380-396, :223-240)."""
    from oracle import gemma4 as og

    table = og.relative_positions(8, chunk=12, context_left=13, context_right=0)
    assert table.shape == (13, 8)
    assert torch.equal(table[-1], torch.cat((torch.zeros(4), torch.ones(4))))  # distance 0: sin 0, cos 0
    inverse = torch.exp(torch.arange(4) * -(math.log(10000) / 3))
    assert torch.allclose(table[0, :4], torch.sin(12 * inverse))
    mask = og.blocked_mask(torch.tensor([40]), 40, 12, 12, 0)
    allowed = ~mask[0, 0]
    for i in range(40):
        u, c = divmod(i, 12)
        keys = [u * 12 - 12 + t for t in range(24) if bool(allowed[u, c, t])]
        assert keys == list(range(max(0, i - 11), i + 1))


@pytest.mark.parametrize("source", ["oracle", "asrback_amd"])
def test_sinusoidal_positions_closed_form(source):
    """SenseVoice's position encoding (sensevoice.py:166-174) against values
    the definition fixes, at the model's depth 512: column i < 256 of
    position p (rows are positions 1, 2, ...) is sin(p * 10000^(-i/255)),
    column 256 + i its cosine.  Pinned: row 0 is position 1 (not 0), column
    0 is sin(p) (frequency 1), the last frequency is exactly 1e-4 (the
    exponent's denominator is depth/2 - 1), sines come before cosines in
    two halves (not interleaved), and sin^2 + cos^2 = 1."""
    if source == "oracle":
        from oracle.sensevoice import sinusoidal_positions as encode

        table = encode(600, 512).double()
    else:
        from asrback_amd.sensevoice import sinusoidal_positions as encode

        table = encode(600, 512, torch.device("cpu")).double()
    assert table.shape == (600, 512)
    p = torch.arange(1, 601, dtype=torch.float64)
    # float32 phases up to 600 rad carry ~4e-5 rad of rounding.
    assert torch.allclose(table[0, :256], torch.sin(torch.tensor([10000.0 ** (-i / 255) for i in range(256)],
                                                                 dtype=torch.float64)), atol=1e-6)
    assert torch.allclose(table[:, 0], torch.sin(p), atol=1e-4)
    assert torch.allclose(table[:, 256], torch.cos(p), atol=1e-4)
    assert torch.allclose(table[:, 255], torch.sin(p * 1e-4), atol=1e-6)
    assert torch.allclose(table[:, 511], torch.cos(p * 1e-4), atol=1e-6)
    assert math.isclose(float(table[0, 255]), math.sin(1e-4), rel_tol=1e-5)
    freq = torch.tensor([10000.0 ** (-i / 255) for i in range(256)], dtype=torch.float64)
    phase = p[:, None] * freq[None, :]
    assert torch.allclose(table[:, :256], torch.sin(phase), atol=1e-4)
    assert torch.allclose(table[:, 256:], torch.cos(phase), atol=1e-4)
    assert torch.allclose(table[:, :256] ** 2 + table[:, 256:] ** 2, torch.ones(600, 256, dtype=torch.float64),
                          atol=1e-6)

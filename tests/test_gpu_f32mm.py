"""GPU parity of the fp32 matrix-core forward kernel (fwd_f32mm.hip).

Every float32 ``flash`` call with head_dim 64 or 128 and no sliding window
runs on it.  Bar: within 1e-5 of the CPU oracle (torch SDPA in float32 with
the reference's masks), normwise and element-wise (conftest.assert_close),
and within the same bound of the vector-ALU kernel (``force_valu``), the
exact-arithmetic fp32 twin.  The shapes reach every key-split count the
launcher picks (1, 2, 4, 8 waves per row block), query and key counts that
are not multiples of the 32-key sub-tile, and the edge rows of each layout.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import attention as oa

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from asrback_amd import attention

    return attention


def say(*args):
    print(*args, flush=True)


def randn(*shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g)


@pytest.mark.parametrize(
    "batch,heads,length,hd",
    [
        (1, 6, 1500, 64),   # Whisper-tiny encoder layer: 282 row blocks, four key splits
        (1, 1, 1, 64),      # one query, one key
        (2, 3, 33, 64),     # one key split, a partial sub-tile
        (1, 2, 300, 128),   # head_dim 128, four key splits
        (2, 2, 200, 128),   # head_dim 128, two key splits
        (4, 2, 95, 128),    # head_dim 128, one key split
        (8, 8, 257, 64),    # two key splits
        (2, 4, 1000, 64),   # eight key splits
    ],
)
def test_noncausal_matches_oracle_and_valu(ops, device, batch, heads, length, hd):
    say("f32mm noncausal", batch, heads, length, hd)
    q, k, v = (randn(batch, length, heads, hd, seed=300 + i) for i in range(3))
    ref = oa.sdpa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)
    qd, kd, vd = (t.to(device) for t in (q, k, v))
    out = ops.flash(qd, kd, vd)
    assert_close(out, ref, "f32", label="oracle")
    twin = ops.flash(qd, kd, vd, force_valu=True)
    assert_close(out, twin, "f32", label="vector-ALU twin")


@pytest.mark.parametrize("length", [1, 2, 31, 32, 33, 64, 65, 127, 448])
@pytest.mark.parametrize("hd", [64, 128])
def test_causal_prefix_matches_oracle(ops, device, length, hd):
    """Whisper's fp32 prompt prefix: causal, q len == k len (whisper.py:229-237)."""
    say("f32mm causal", length, hd)
    q, k, v = (randn(3, 6, length, hd, seed=320 + i) for i in range(3))
    ref = oa.sdpa(q, k, v, is_causal=length > 1)
    out = ops.sdpa(q.to(device), k.to(device), v.to(device), is_causal=length > 1)
    assert_close(out.transpose(1, 2), ref, "f32")


def test_cross_attention_prompt_matches_oracle(ops, device):
    """A prompt's rows over 1500 encoder frames (cross-attention, whisper.py:238-240)."""
    say("f32mm cross")
    q = randn(2, 6, 7, 64, seed=330)
    k, v = (randn(2, 6, 1500, 64, seed=331 + i) for i in range(2))
    ref = oa.sdpa(q, k, v)
    out = ops.sdpa(q.to(device), k.to(device), v.to(device))
    assert_close(out.transpose(1, 2), ref, "f32")


@pytest.mark.parametrize("zero_padded", [False, True])
def test_ragged_keys_match_oracle(ops, device, zero_padded):
    """Key padding by seqused_k (SenseVoice's layout, sensevoice.py:110-133),
    with the padded rows computed (as the reference does) or zeroed."""
    say("f32mm ragged", zero_padded)
    rng = np.random.default_rng(21)
    lengths = torch.from_numpy(rng.integers(1, 300, size=9).astype(np.int32))
    length = int(lengths.max())
    fused = randn(9, length, 3 * 256, seed=340)
    ref = oa.sensevoice_attention(fused, 2, oa.key_padding_mask(lengths, length))
    x = fused.to(device)
    q, k, v = (t.view(9, length, 2, 128) for t in x.split(256, dim=-1))
    out = ops.flash(q, k, v, seqused_k=lengths.to(device), zero_padded_rows=zero_padded)
    out = out.reshape(9, length, 256).cpu()
    if zero_padded:
        keep = torch.arange(length)[None, :] < lengths[:, None].long()
        assert torch.count_nonzero(out[~keep]) == 0
        ref = ref * keep[..., None]
    assert_close(out, ref, "f32")


def test_packed_gqa_causal_matches_oracle(ops, device):
    """Qwen3's packed varlen prefill in fp32: bottom-right causal, 16 query
    heads over 8 kv heads (qwen3_asr.py:367-372)."""
    say("f32mm packed gqa")
    sizes = [5, 64, 131, 33]
    segs = oa.Segments.from_lengths(sizes)
    total = sum(sizes)
    q = randn(total, 16, 128, seed=350)
    k, v = (randn(total, 8, 128, seed=351 + i) for i in range(2))
    ref = oa.qwen_attend(q, k, v, segs, causal=True)
    starts = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]), dtype=torch.int32, device=device)
    out = ops.flash(q.to(device), k.to(device), v.to(device), causal=2, cu_seqlens_q=starts, cu_seqlens_k=starts,
                    max_len_q=max(sizes), max_len_k=max(sizes))
    assert_close(out, ref, "f32")


def test_padded_key_slots_never_reach_the_output(ops, device):
    """K/V slots past each sequence's key count hold NaN; the output must not
    see them (the buffer resources end at the block's last visible key)."""
    say("f32mm nan slots")
    lengths = torch.tensor([40, 97, 1], dtype=torch.int32)
    q, k, v = (randn(3, 128, 2, 64, seed=360 + i) for i in range(3))
    for b, n in enumerate(lengths.tolist()):
        k[b, n:] = float("nan")
        v[b, n:] = float("nan")
    ref = oa.sdpa(q.transpose(1, 2), k.nan_to_num().transpose(1, 2), v.nan_to_num().transpose(1, 2),
                  attn_mask=oa.key_padding_mask(lengths, 128)[:, None, None, :]).transpose(1, 2)
    out = ops.flash(q.to(device), k.to(device), v.to(device), seqused_k=lengths.to(device))
    assert torch.isfinite(out).all()
    assert_close(out, ref, "f32")

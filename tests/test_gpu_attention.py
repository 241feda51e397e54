"""GPU parity of the attention kernels, called through the C ABI.

Bar (stated per test): fp32 outputs within 1e-5 and bf16 outputs within 2e-2
of a float32/float64 reference on the same (bf16-rounded) inputs, measured as
max |out - ref| / max |ref|.  References: the committed golden vectors
(float64 closed form) and, at the reference's configuration shapes, the CPU
oracle (torch SDPA with the reference's masks).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import GOLDEN, assert_close, max_rel_err
from oracle import attention as oa

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
KIND = {torch.float32: "f32", torch.bfloat16: "bf16"}  # tolerance classes of conftest.assert_close
DTYPES = [torch.float32, torch.bfloat16]


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN / "attention_cases.npz")


@pytest.fixture(scope="module")
def ops():
    from asrback_amd import attention

    return attention


def dev(x, dtype, device):
    return torch.from_numpy(np.asarray(x)).to(device=device, dtype=dtype)


def say(*args):
    print(*args, flush=True)


# --- golden vectors -----------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("force_valu", [False, True])
def test_encoder_golden(golden, ops, device, dtype, force_valu):
    say("encoder golden", dtype, force_valu)
    q, k, v = (dev(golden[f"enc_{n}"], dtype, device) for n in "qkv")
    out = ops.flash(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), force_valu=force_valu)
    assert_close(out.transpose(1, 2), golden["enc_out"], KIND[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("force_valu", [False, True])
def test_prefix_golden(golden, ops, device, dtype, force_valu):
    say("prefix golden", dtype, force_valu)
    q, k, v = (dev(golden[f"prefix_{n}"], dtype, device) for n in "qkv")
    out = ops.flash(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), causal=1, force_valu=force_valu
    )
    assert_close(out.transpose(1, 2), golden["prefix_out"], KIND[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
def test_step_golden(golden, ops, device, dtype):
    say("step golden", dtype)
    q, k, v = (dev(golden[f"step_{n}"], dtype, device) for n in "qkv")
    positions = torch.from_numpy(golden["step_positions"]).to(device)
    out = ops.sdpa(q, k, v, ops.KeyPrefix(positions=positions))  # (B, 1, H, D)
    assert_close(out.transpose(1, 2), golden["step_out"], KIND[dtype])
    # The boolean mask the reference builds gives the same result.
    mask = oa.whisper_step_mask(positions, k.shape[2])
    out2 = ops.sdpa(q, k, v, mask)
    assert_close(out2.transpose(1, 2), golden["step_out"], KIND[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
def test_cross_golden(golden, ops, device, dtype):
    say("cross golden", dtype)
    q, k, v = (dev(golden[f"cross_{n}"], dtype, device) for n in "qkv")
    out = ops.sdpa(q, k, v)
    assert_close(out.transpose(1, 2), golden["cross_out"], KIND[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("force_valu", [False, True])
def test_padded_golden(golden, ops, device, dtype, force_valu):
    say("padded golden", dtype, force_valu)
    q, k, v = (dev(golden[f"padded_{n}"], dtype, device) for n in "qkv")
    lengths = torch.from_numpy(golden["padded_lengths"]).to(device)
    out = ops.flash(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), seqused_k=lengths, force_valu=force_valu
    )
    assert_close(out.transpose(1, 2), golden["padded_out"], KIND[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("force_valu", [False, True])
def test_packed_gqa_golden(golden, ops, device, dtype, force_valu):
    say("packed golden", dtype, force_valu)
    q, k, v = (dev(golden[f"packed_{n}"], dtype, device) for n in "qkv")
    starts = torch.from_numpy(golden["packed_starts"]).to(device)
    longest = int(np.diff(golden["packed_starts"]).max())
    out = ops.flash(
        q, k, v, causal=2, cu_seqlens_q=starts, cu_seqlens_k=starts,
        max_len_q=longest, max_len_k=longest, force_valu=force_valu,
    )
    assert_close(out, golden["packed_out"], KIND[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
def test_gqa_step_golden(golden, ops, device, dtype):
    say("gqa step golden", dtype)
    q, k, v = (dev(golden[f"gqa_step_{n}"], dtype, device) for n in "qkv")
    used = torch.from_numpy(golden["gqa_step_used"]).to(device)
    out = ops.decode(q, k, v, seqused_k=used)
    assert_close(out, golden["gqa_step_out"], KIND[dtype])


# --- running-max paths of the matrix-core kernel --------------------------------


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("pattern", ["growing", "shrinking", "spike", "large"])
def test_running_max_paths(ops, device, hd, pattern):
    """Score patterns that drive the matrix-core kernel's running max off its
    common path, 16 key tiles of 64: row maxima that grow along the keys
    (rescales after the first tile), that shrink (probabilities far below
    the first tile's), one late key far above every other for every row
    (its tile's probabilities overflow the slack: at head_dim 64 the first,
    max-free exponentiation is thrown away and redone), and scores large
    throughout.  bf16 against the float32 oracle (torch SDPA)."""
    say("running max", hd, pattern)
    g = torch.Generator().manual_seed(70 + hd)
    batch, heads, length = 2, 3, 1000
    q, k, v = (torch.randn(batch, heads, length, hd, generator=g) for _ in range(3))
    ramp = torch.linspace(0.0, 1.0, length)[None, None, :, None]
    if pattern == "growing":
        k = k * (1 + 5 * ramp)
    elif pattern == "shrinking":
        k = k * (6 - 5 * ramp)
    elif pattern == "spike":
        # A direction every query shares, and key 777 along it: its score is
        # ~18 sqrt(hd) for every row, far above the rest.
        u = torch.randn(batch, heads, 1, hd, generator=g)
        q = q + 3 * u
        k[:, :, 777:778] = 6 * u
    else:
        q = q * 6
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    ref = oa.sdpa(q.float(), k.float(), v.float())
    out = ops.flash(*(t.transpose(1, 2).to(device) for t in (q, k, v)))
    assert torch.isfinite(out).all()
    assert_close(out.transpose(1, 2), ref, "bf16")


@pytest.mark.parametrize("batch", [5, 12, 24, 40, 64, 65])
@pytest.mark.parametrize("hd", [64, 128])
def test_ragged_work_order_batches(ops, device, batch, hd):
    """Ragged batches of every size class of the longest-first work order
    (the ranking's 8-, 16-, 32- and 64-sequence bounds; 65 sequences are
    not ranked), key counts 1-300 with ties, bf16 against the oracle."""
    say("ragged work order", batch, hd)
    rng = np.random.default_rng(200 + batch)
    lengths = rng.integers(1, 301, size=batch).astype(np.int32)
    lengths[: batch // 3] = lengths[batch // 3]  # ties: index order decides
    length = int(lengths.max())
    heads = 8
    g = torch.Generator().manual_seed(210 + batch + hd)
    q, k, v = (torch.randn(batch, length, heads, hd, generator=g).to(torch.bfloat16) for _ in range(3))
    used = torch.from_numpy(lengths)
    ref = oa.sdpa(*(t.float().transpose(1, 2) for t in (q, k, v)),
                  attn_mask=oa.key_padding_mask(used, length)[:, None, None, :]).transpose(1, 2)
    out = ops.flash(q.to(device), k.to(device), v.to(device), seqused_k=used.to(device))
    assert_close(out.float().cpu(), ref, "bf16")

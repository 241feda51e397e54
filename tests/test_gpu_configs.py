"""GPU parity at the reference's configuration shapes, edge cases and graph
replays, against the CPU oracle (torch SDPA with the reference's masks) on
the same inputs.

Bar: max |out - ref| / max |ref| <= 1e-5 (fp32) and <= 2e-2 (bf16, against
an fp32 reference on the bf16-rounded inputs).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_close, max_rel_err
from oracle import attention as oa

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
KIND = {torch.float32: "f32", torch.bfloat16: "bf16"}  # tolerance classes of conftest.assert_close


@pytest.fixture(scope="module")
def ops():
    from asrback_amd import attention

    return attention


def say(*args):
    print(*args, flush=True)


def randn(*shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


# --- encoder self-attention ----------------------------------------------------


@pytest.mark.parametrize("zero_padded", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sensevoice_ragged_batch(ops, device, dtype, zero_padded):
    """SenseVoice SAN-M: B=32, 4 x 128, lengths 4 + U{100..500}, key padding
    through seqused_k on views of the fused (B, L, 1536) projection
    (sensevoice.py:97, :110-133).  With ``zero_padded_rows`` -- the launch
    the headline line times (bench.py's SenseVoice workload, as
    SANMAttention runs it) -- the valid rows are checked against the oracle
    and every padded row must be exactly zero."""
    say("sensevoice ragged", dtype, "zero_padded", zero_padded)
    rng = np.random.default_rng(11)
    lengths = torch.from_numpy((rng.integers(100, 501, size=32) + 4).astype(np.int32))
    length = int(lengths.max())
    fused = randn(32, length, 1536, seed=11, dtype=dtype)
    ref = oa.sensevoice_attention(fused.float(), 4, oa.key_padding_mask(lengths, length))
    x = fused.to(device)
    q, k, v = (t.view(32, length, 4, 128) for t in x.split(512, dim=-1))
    out = ops.flash(q, k, v, seqused_k=lengths.to(device), zero_padded_rows=zero_padded).reshape(32, length, 512)
    if not zero_padded:
        assert_close(out, ref, KIND[dtype])
        return
    valid = torch.arange(length)[None, :] < lengths[:, None]  # (32, length)
    out = out.float().cpu()
    assert_close(out[valid], ref[valid], KIND[dtype], label="valid rows")
    assert not out[~valid].any(), "padded rows must be exactly zero"


def test_sensevoice_unmasked_equals_masked_full_length(ops, device):
    """No mask when every row is full length (sensevoice.py:99-103, :550)."""
    x = randn(3, 130, 1536, seed=12, dtype=torch.bfloat16).to(device)
    q, k, v = (t.view(3, 130, 4, 128) for t in x.split(512, dim=-1))
    full = ops.flash(q, k, v)
    masked = ops.flash(q, k, v, seqused_k=torch.full((3,), 130, dtype=torch.int32, device=device))
    assert torch.equal(full, masked)


def _fsmn_reference(fused, heads, lengths, weight, bias):
    """The oracle's FSMN memory (sensevoice.py:99-107) in float32 on the
    values of ``fused``, plus ``bias`` on every row."""
    size = fused.shape[-1] // 3
    mask = None if lengths is None else oa.key_padding_mask(lengths, fused.shape[1])
    memory = oa.fsmn_memory(fused[..., 2 * size :].float(), mask, weight.float(), weight.shape[-1])
    return memory if bias is None else memory + bias.float()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sensevoice_fsmn_fused_matches_oracle(ops, device, dtype):
    """Attention plus FSMN memory in one call at the SenseVoice batch shape
    (B=32, 4 x 128, lengths 4 + U{100..500}, kernel 11, linear_out's bias
    folded in): the attention output equals asrattn_fwd's, the memory
    matches the oracle's masked depthwise convolution, and padded rows hold
    the bias alone."""
    say("sensevoice fsmn fused", dtype)
    rng = np.random.default_rng(13)
    lengths = torch.from_numpy((rng.integers(100, 501, size=32) + 4).astype(np.int32))
    length = int(lengths.max())
    fused = randn(32, length, 1536, seed=13, dtype=dtype)
    weight = (randn(512, 1, 11, seed=14) * 0.3).to(dtype)
    bias = randn(512, seed=15, dtype=dtype)
    x = fused.to(device)
    q, k, v = (t.view(32, length, 4, 128) for t in x.split(512, dim=-1))
    used = lengths.to(device)
    out, memory = ops.flash_fsmn(q, k, v, weight.to(device), seqused_k=used, bias=bias.to(device))
    assert torch.equal(out, ops.flash(q, k, v, seqused_k=used))
    ref = _fsmn_reference(fused, 4, lengths, weight, bias)
    assert_close(memory.cpu(), ref, KIND[dtype])
    for b in (int(lengths.argmin()), 0):
        n = int(lengths[b])
        assert torch.equal(memory[b, n:].cpu(), bias.expand(length - n, 512))


@pytest.mark.parametrize(
    "dtype,heads,head_dim,kernel,force_valu",
    [
        (torch.bfloat16, 4, 128, 11, False),
        (torch.bfloat16, 4, 128, 5, False),
        (torch.bfloat16, 4, 128, 4, False),
        (torch.bfloat16, 4, 128, 15, False),
        (torch.bfloat16, 8, 64, 11, False),
        (torch.bfloat16, 4, 128, 11, True),
        (torch.float32, 4, 128, 11, False),
        (torch.float32, 2, 64, 10, False),
        (torch.float32, 4, 128, 1, False),
        (torch.float32, 2, 64, 15, False),
    ],
)
def test_fsmn_kernel_sizes_and_edges(ops, device, dtype, heads, head_dim, kernel, force_valu):
    """Filter sizes 1..15 (odd and even: left padding (K - 1) // 2), both
    head sizes, the fused epilogue and the separate kernel; rows of 0, 2
    and 37 frames (shorter than the filter's reach) and one full row of 130
    (two row blocks, the second of two rows)."""
    say("fsmn", dtype, heads, head_dim, kernel, force_valu)
    lengths = torch.tensor([37, 130, 2, 0], dtype=torch.int32)
    width = heads * head_dim
    fused = randn(4, 130, 3 * width, seed=16, dtype=dtype)
    weight = (randn(width, 1, kernel, seed=17) * 0.3).to(dtype)
    x = fused.to(device)
    q, k, v = (t.view(4, 130, heads, head_dim) for t in x.split(width, dim=-1))
    out, memory = ops.flash_fsmn(
        q, k, v, weight.to(device), seqused_k=lengths.to(device), force_valu=force_valu
    )
    ref = _fsmn_reference(fused, heads, lengths, weight, None)
    assert_close(memory.cpu(), ref, KIND[dtype])
    assert not memory[3].any() and not memory[2, 2:].any()
    # (the frame-less row's reference is NaN: softmax over no keys)
    valid = oa.key_padding_mask(lengths, 130)
    attention = oa.sensevoice_attention(fused.float(), heads, valid)
    assert_close(out.reshape(4, 130, width).cpu()[valid], attention[valid], KIND[dtype])
    # Without frame counts every frame is real.
    _, full = ops.flash_fsmn(q, k, v, weight.to(device), force_valu=force_valu)
    assert_close(full.cpu(), _fsmn_reference(fused, heads, None, weight, None), KIND[dtype])


def test_fsmn_fused_epilogue_equals_separate_kernel(ops, device):
    """The attention kernel's FSMN epilogue and the FSMN kernel of its own
    compute the same sums in the same order: identical bits."""
    lengths = torch.tensor([300, 17, 256, 129], dtype=torch.int32, device=device)
    x = randn(4, 300, 1536, seed=18, dtype=torch.bfloat16).to(device)
    weight = (randn(512, 1, 11, seed=19) * 0.3).to(torch.bfloat16).to(device)
    bias = randn(512, seed=20, dtype=torch.bfloat16).to(device)
    q, k, v = (t.view(4, 300, 4, 128) for t in x.split(512, dim=-1))
    _, fused = ops.flash_fsmn(q, k, v, weight, seqused_k=lengths, bias=bias)
    _, separate = ops.flash_fsmn(q, k, v, weight, seqused_k=lengths, bias=bias, force_valu=True)
    assert torch.equal(fused, separate)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_whisper_encoder_shapes(ops, device, dtype):
    """Whisper encoder self-attention over 1500 frames: one layer of
    large-v3-turbo's, all 16 rows of 20 heads x 64 in bf16 (the benchmark's
    3,840-item launch), and whisper-tiny's 6 heads in fp32 (whisper.py:102-110)."""
    heads = 20 if dtype == torch.bfloat16 else 6
    batch = 16 if dtype == torch.bfloat16 else 1
    say("whisper encoder", dtype, heads)
    x = randn(batch, 1500, 3 * heads * 64, seed=13, dtype=dtype)
    q, k, v = (oa.split_heads(t, heads) for t in x.float().split(heads * 64, dim=-1))
    ref = oa.sdpa(q, k, v)
    xd = x.to(device)
    qd, kd, vd = (oa.split_heads(t, heads) for t in xd.split(heads * 64, dim=-1))
    out = ops.sdpa(qd, kd, vd)  # (B, L, H, D)
    assert_close(out.transpose(1, 2), ref, KIND[dtype])


@pytest.mark.parametrize("length", [1, 2, 31, 63, 64, 65, 127, 129, 448])
def test_causal_prefix_lengths(ops, device, length):
    """Causal prompt prefix, q len == k len (whisper.py:229-237)."""
    say("causal prefix", length)
    q, k, v = (randn(3, 6, length, 64, seed=14 + i, dtype=torch.bfloat16) for i in range(3))
    ref = oa.sdpa(q.float(), k.float(), v.float(), is_causal=length > 1)
    out = ops.sdpa(q.to(device), k.to(device), v.to(device), is_causal=length > 1)
    assert_close(out.transpose(1, 2), ref, "bf16")


def test_qwen_packed_causal_prefill(ops, device):
    """Qwen3 prompts packed back to back, causal GQA 16/8 x 128
    (qwen3_asr.py:152-181, :374-390)."""
    lengths = [417, 402, 430, 425]
    tokens = sum(lengths)
    q = randn(tokens, 16, 128, seed=15, dtype=torch.bfloat16)
    k = randn(tokens, 8, 128, seed=16, dtype=torch.bfloat16)
    v = randn(tokens, 8, 128, seed=17, dtype=torch.bfloat16)
    segments = oa.Segments.from_lengths(lengths)
    ref = oa.qwen_attend(q.float(), k.float(), v.float(), segments, causal=True)
    starts = segments.starts.to(device)
    out = ops.varlen_attn(q.to(device), k.to(device), v.to(device), starts, starts, max(lengths),
                          max(lengths), window_size=(-1, 0), enable_gqa=True)
    assert_close(out, ref, "bf16")


def test_qwen_audio_windows_noncausal(ops, device):
    """Audio encoder windows of <= 104 tokens, non-causal varlen
    (qwen3_asr.py:216-221, :303-310)."""
    lengths = [104, 104, 37, 104, 81]
    tokens = sum(lengths)
    q, k, v = (randn(tokens, 16, 64, seed=18 + i, dtype=torch.bfloat16) for i in range(3))
    segments = oa.Segments.from_lengths(lengths)
    ref = oa.qwen_attend(q.float(), k.float(), v.float(), segments, causal=False)
    starts = segments.starts.to(device)
    out = ops.varlen_attn(q.to(device), k.to(device), v.to(device), starts, starts, 104, 104)
    assert_close(out, ref, "bf16")


# --- decoder steps ---------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_whisper_small_decoder_step(ops, device, dtype):
    """Whisper-small step: 16 rows x 12 heads x 64; self-attention over the
    256 bucket with keys 0..position (positions U{0..223}), cross-attention
    over 1500 frames (whisper.py:235-240, mask :263-264)."""
    say("whisper small step", dtype)
    rng = np.random.default_rng(19)
    positions = torch.from_numpy(rng.integers(0, 224, size=16).astype(np.int64))
    q = randn(16, 12, 1, 64, seed=19, dtype=dtype)
    cache_k = randn(16, 12, 448, 64, seed=20, dtype=dtype)
    cache_v = randn(16, 12, 448, 64, seed=21, dtype=dtype)
    cross_k = randn(16, 12, 1500, 64, seed=22, dtype=dtype)
    cross_v = randn(16, 12, 1500, 64, seed=23, dtype=dtype)
    mask = oa.whisper_step_mask(positions, 256)
    ref_self = oa.sdpa(q.float(), cache_k[:, :, :256].float(), cache_v[:, :, :256].float(), attn_mask=mask)
    ref_cross = oa.sdpa(q.float(), cross_k.float(), cross_v.float())
    qd, kd, vd = q.to(device), cache_k.to(device), cache_v.to(device)
    out_self = ops.sdpa(qd, kd[:, :, :256], vd[:, :, :256], ops.KeyPrefix(positions=positions.to(device)))
    out_cross = ops.sdpa(qd, cross_k.to(device), cross_v.to(device))
    assert_close(out_self.transpose(1, 2), ref_self, KIND[dtype])
    assert_close(out_cross.transpose(1, 2), ref_cross, KIND[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_qwen_gqa_decode(ops, device, dtype):
    """Qwen3-1.7B step: 64 rows, 16 query / 8 kv heads x 128 over the
    (64, 1024, 8, 128) cache with seqused_k = position + 1, positions
    400-557 (qwen3_asr.py:392-432)."""
    say("qwen decode", dtype)
    rng = np.random.default_rng(24)
    positions = torch.from_numpy((390 + rng.integers(10, 41, size=64) + rng.integers(0, 128, size=64)).astype(np.int64))
    q = randn(64, 16, 128, seed=24, dtype=dtype)
    keys = randn(64, 1024, 8, 128, seed=25, dtype=dtype)
    values = randn(64, 1024, 8, 128, seed=26, dtype=dtype)
    ref = oa.qwen_step_attention(q.float(), keys.float(), values.float(), oa.qwen_step_mask(positions, 1024))
    used = (positions + 1).to(torch.int32).to(device)
    out = ops.decode(q.to(device), keys.to(device), values.to(device), seqused_k=used)
    assert_close(out, ref, KIND[dtype])


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16, 64])
def test_decode_split_count_does_not_change_result(ops, device, splits):
    """Any split count gives the same output (the last split merges)."""
    q = randn(5, 8, 128, seed=27, dtype=torch.bfloat16).to(device)
    k = randn(5, 700, 4, 128, seed=28, dtype=torch.bfloat16).to(device)
    v = randn(5, 700, 4, 128, seed=29, dtype=torch.bfloat16).to(device)
    used = torch.tensor([1, 64, 65, 333, 700], dtype=torch.int32, device=device)
    base = ops.decode(q, k, v, seqused_k=used, num_splits=1).float()
    out = ops.decode(q, k, v, seqused_k=used, num_splits=splits).float()
    assert max_rel_err(out, base) < 1e-2


def test_caller_owned_workspace_gives_the_same_bits(ops, device):
    """Split partials in a caller-owned buffer (sized with
    decode_workspace_size, installed with ``workspace``) or in a per-call
    temporary: identical outputs, for decode, decode_append and the greedy
    choice; a buffer smaller than the call needs is refused."""
    q = randn(2, 16, 128, seed=90, dtype=torch.bfloat16).to(device)
    k = randn(2, 1024, 8, 128, seed=91, dtype=torch.bfloat16).to(device)
    v = randn(2, 1024, 8, 128, seed=92, dtype=torch.bfloat16).to(device)
    used = torch.tensor([1000, 37], dtype=torch.int32, device=device)
    need = ops.decode_workspace_size(2, 16, 8, 128, 1024, torch.bfloat16)
    assert need > 0
    buffer = torch.full((need,), 255, dtype=torch.uint8, device=device)
    base = ops.decode(q, k, v, seqused_k=used)
    with ops.workspace(buffer):
        assert torch.equal(ops.decode(q, k, v, seqused_k=used), base)
        with pytest.raises(ValueError, match="workspace"):
            ops.decode(q, k, v, seqused_k=used, workspace=buffer[: need // 2])
    logits = randn(3, 50000, seed=93).to(device)
    choice = ops.greedy_choice(logits)
    held = torch.empty(ops.choice_workspace_size(3, 50000), dtype=torch.uint8, device=device)
    with ops.workspace(held):
        again = ops.greedy_choice(logits)
    assert torch.equal(choice[0], again[0]) and torch.equal(choice[1], again[1])
    positions = torch.tensor([700, 5], dtype=torch.int64, device=device)
    k_new = randn(2, 8, 128, seed=94, dtype=torch.bfloat16).to(device)
    caches = [(k.clone(), v.clone()) for _ in range(2)]
    outs = [ops.decode_append(q, k_new, k_new, ck, cv, positions) for ck, cv in caches[:1]]
    with ops.workspace(buffer):
        outs += [ops.decode_append(q, k_new, k_new, ck, cv, positions) for ck, cv in caches[1:]]
    assert torch.equal(outs[0], outs[1]) and torch.equal(caches[0][0], caches[1][0])


def test_decode_zero_keys_gives_zeros(ops, device):
    q = randn(3, 4, 64, seed=32).to(device)
    k = randn(3, 50, 4, 64, seed=33).to(device)
    used = torch.tensor([0, 5, 0], dtype=torch.int32, device=device)
    out = ops.decode(q, k, k, seqused_k=used, num_splits=4)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0
    assert torch.count_nonzero(out[1]) > 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd,heads_q,heads_kv", [(128, 16, 8), (64, 12, 12)])
@pytest.mark.parametrize("splits", [1, 3])
def test_decode_ignores_cache_slots_past_each_row(ops, device, dtype, hd, heads_q, heads_kv, splits):
    """Cache slots at and past each row's length hold NaN (a slab row used
    before, or never written).  With one split the first load batch reads
    the whole row before its length is known; the outputs still equal the
    oracle's over each row's own keys, for plain decode (seqused_k) and the
    append variant (the step's key at the row's position), and a row of
    length 0 gives zeros."""
    say("decode past rows", dtype, hd, heads_q, heads_kv, splits)
    batch, length = 6, 320
    n = torch.tensor([0, 1, 37, 64, 200, 319])
    q = randn(batch, heads_q, hd, seed=81, dtype=dtype)
    keys = randn(batch, length, heads_kv, hd, seed=82, dtype=dtype)
    values = randn(batch, length, heads_kv, hd, seed=83, dtype=dtype)
    past = torch.arange(length)[None, :] >= n[:, None]
    keys_nan, values_nan = keys.clone(), values.clone()
    keys_nan[past] = float("nan")
    values_nan[past] = float("nan")
    mask = torch.arange(length)[None, :] < n[:, None]
    ref = oa.qwen_step_attention(q.float(), keys.float(), values.float(), mask[:, None, None, :])
    used = n.to(torch.int32).to(device)
    out = ops.decode(q.to(device), keys_nan.to(device), values_nan.to(device), seqused_k=used,
                     num_splits=splits).float().cpu()
    assert torch.count_nonzero(out[0]) == 0
    assert_close(out[1:], ref[1:], KIND[dtype])

    # Append: row b's step key goes to slot n_b and attends keys 0..n_b.
    positions = n.clone()
    k_new = randn(batch, heads_kv, hd, seed=84, dtype=dtype)
    v_new = randn(batch, heads_kv, hd, seed=85, dtype=dtype)
    rows = torch.arange(batch)
    keys_ref, values_ref = keys.clone(), values.clone()
    keys_ref[rows, positions] = k_new
    values_ref[rows, positions] = v_new
    ref = oa.qwen_step_attention(q.float(), keys_ref.float(), values_ref.float(), oa.qwen_step_mask(positions, length))
    kd, vd = keys_nan.to(device), values_nan.to(device)
    out = ops.decode_append(q.to(device), k_new.to(device), v_new.to(device), kd, vd, positions.to(device),
                            num_splits=splits)
    assert_close(out.float().cpu(), ref, KIND[dtype])
    assert torch.equal(kd.cpu()[rows, positions], k_new) and torch.equal(vd.cpu()[rows, positions], v_new)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_speculative_first_batch_ignores_slots_past_each_row(ops, device, dtype):
    """At the Qwen3 shape (64 rows x 8 kv heads of 128 over a 1024-slot
    cache: one split) the first load batch (32 keys per workgroup) is
    issued before the row's key count is read, over the whole cache's
    extent.  Slots at and past each row's count hold NaN and +-inf; lengths
    0, 1, 31, 32, 33 (around that batch) and 1023 among random ones.  The
    outputs equal the oracle's over each row's own keys, the empty row gives
    zeros, and a graph replay with other counts agrees with an eager call."""
    say("decode speculative first batch", dtype)
    batch, length, heads_q, heads_kv, hd = 64, 1024, 16, 8, 128
    rng = np.random.default_rng(91)
    lengths = rng.integers(1, length, size=batch)
    lengths[:6] = [0, 1, 31, 32, 33, 1023]
    n = torch.from_numpy(lengths)
    q = randn(batch, heads_q, hd, seed=92, dtype=dtype)
    keys = randn(batch, length, heads_kv, hd, seed=93, dtype=dtype)
    values = randn(batch, length, heads_kv, hd, seed=94, dtype=dtype)
    past = torch.arange(length)[None, :] >= n[:, None]
    garbage = torch.tensor([float("nan"), float("inf"), -float("inf")])[torch.arange(length) % 3]
    keys_bad, values_bad = keys.clone(), values.clone()
    keys_bad[past] = garbage.expand(batch, length)[past][:, None, None].to(dtype)
    values_bad[past] = garbage.expand(batch, length)[past].flip(0)[:, None, None].to(dtype)
    mask = torch.arange(length)[None, :] < n[:, None]
    ref = oa.qwen_step_attention(q.float(), keys.float(), values.float(), mask[:, None, None, :])
    qd, kd, vd = q.to(device), keys_bad.to(device), values_bad.to(device)
    used = n.to(torch.int32).to(device)
    out = ops.decode(qd, kd, vd, seqused_k=used)
    assert torch.isfinite(out).all()
    assert torch.count_nonzero(out[0]) == 0
    assert_close(out[1:].float().cpu(), ref[1:], KIND[dtype])

    # Positions instead of counts (keys 0..positions[b]), replayed from a graph.
    positions = (n - 1).clamp(min=0).to(torch.int64).to(device)
    static_out = torch.empty_like(out)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        ops.decode(qd, kd, vd, positions=positions, out=static_out)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.decode(qd, kd, vd, positions=positions, out=static_out)
    for shift in (0, -7, -20):  # within each row's own keys
        positions.copy_(((n - 1 + shift).clamp(0, length - 1)).to(torch.int64).to(device))
        graph.replay()
        torch.cuda.synchronize()
        eager = ops.decode(qd, kd, vd, positions=positions)
        assert torch.equal(static_out, eager), shift
        assert torch.isfinite(static_out).all()


def test_encoder_zero_keys_gives_zeros(ops, device):
    q = randn(2, 40, 2, 128, seed=34, dtype=torch.bfloat16).to(device)
    used = torch.tensor([0, 17], dtype=torch.int32, device=device)
    out = ops.flash(q, q, q, seqused_k=used)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[1]) > 0


def test_step_matches_last_row_of_prefill_on_gpu(ops, device):
    """Invariant: a decoder step at position p equals row p of the causal
    prefill over the same keys."""
    q, k, v = (randn(2, 6, 40, 64, seed=35 + i, dtype=torch.bfloat16).to(device) for i in range(3))
    full = ops.sdpa(q, k, v, is_causal=True)  # (B, L, H, D)
    for p in (0, 17, 39):
        pos = torch.full((2,), p, dtype=torch.int64, device=device)
        step = ops.sdpa(q[:, :, p : p + 1], k, v, ops.KeyPrefix(positions=pos))
        assert_close(step[:, 0].float(), full[:, p].float(), "bf16")


def test_decode_replays_from_a_graph(ops, device):
    """A captured decode sees new positions on every replay; each replay
    matches the eager call (graph replays interleaved with eager work)."""
    q = randn(8, 12, 1, 64, seed=38, dtype=torch.bfloat16).to(device)
    k = randn(8, 12, 448, 64, seed=39, dtype=torch.bfloat16).to(device)
    v = randn(8, 12, 448, 64, seed=40, dtype=torch.bfloat16).to(device)
    positions = torch.zeros(8, dtype=torch.int64, device=device)
    out = torch.empty(8, 1, 12, 64, dtype=torch.bfloat16, device=device)

    def step():
        out.copy_(ops.sdpa(q, k[:, :, :256], v[:, :, :256], ops.KeyPrefix(positions=positions)))

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    rng = np.random.default_rng(41)
    for _ in range(4):
        positions.copy_(torch.from_numpy(rng.integers(0, 256, size=8)).to(device))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = ops.sdpa(q, k[:, :, :256], v[:, :, :256], ops.KeyPrefix(positions=positions))
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)


def test_errors_raise_runtime_error(ops, device):
    from asrback_amd._lib import AttentionError

    q = randn(2, 3, 96, seed=42).to(device)  # head_dim 96: no kernel
    with pytest.raises(AttentionError, match="head_dim"):
        ops.decode(q, q[:, None].expand(2, 5, 3, 96), q[:, None].expand(2, 5, 3, 96))
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.decode(q.cpu(), q.cpu()[:, None], q.cpu()[:, None])


# --- decoder step with its prologue fused (asrattn_decode_append) ----------------


def _ulp_diff_ok(got: torch.Tensor, want: torch.Tensor, dtype) -> bool:
    """Equal, or (bf16) at most one unit in the last place apart on a small
    fraction of elements: the kernel rounds where torch rounds, but sums the
    squares in another order."""
    if dtype == torch.float32:
        return max_rel_err(got, want) < 1e-6
    diff = (got.float() - want.float()).abs()
    ulp = torch.clamp(want.float().abs(), min=1e-30) * 2.0**-7
    return bool((diff <= ulp).all()) and float((diff > 0).float().mean()) < 0.01


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch,heads_q,heads_kv,splits", [(64, 16, 8, 0), (2, 4, 2, 0), (3, 8, 2, 5)])
def test_decode_append_matches_oracle(ops, device, dtype, batch, heads_q, heads_kv, splits):
    """Qwen3 step path fused (qwen3_asr.py:366-372, :409-432): RMSNorm and
    rotary embedding of q and the new key, the cache write at each row's
    position and the attention over keys 0..position, against the oracle's
    norm/rotate (torch CPU, in the cache dtype) and SDPA.  Small batches split
    the keys: the last split folds the new key in, the first writes it."""
    say("decode append", dtype, batch, heads_q, heads_kv, splits)
    hd, length, eps = 128, 1024, 1e-6
    rng = np.random.default_rng(60 + batch)
    positions = torch.from_numpy(rng.integers(0, 600, size=batch).astype(np.int64))
    positions[0] = 0  # only the new key
    q = randn(batch, heads_q, hd, seed=61, dtype=dtype)
    k_new = randn(batch, heads_kv, hd, seed=62, dtype=dtype)
    v_new = randn(batch, heads_kv, hd, seed=63, dtype=dtype)
    keys = randn(batch, length, heads_kv, hd, seed=64, dtype=dtype)
    values = randn(batch, length, heads_kv, hd, seed=65, dtype=dtype)
    g = torch.Generator().manual_seed(66)
    q_w = (torch.rand(hd, generator=g) + 0.5).to(dtype)
    k_w = (torch.rand(hd, generator=g) + 0.5).to(dtype)
    cos, sin = oa.rope_tables(1e6, hd, length, dtype)
    cos, sin = cos[positions], sin[positions]
    qn = oa.rotate(oa.rms_norm(q, q_w, eps), cos, sin)
    kn = oa.rotate(oa.rms_norm(k_new, k_w, eps), cos, sin)
    rows = torch.arange(batch)
    keys_ref, values_ref = keys.clone(), values.clone()
    keys_ref[rows, positions] = kn
    values_ref[rows, positions] = v_new
    ref = oa.qwen_step_attention(qn.float(), keys_ref.float(), values_ref.float(), oa.qwen_step_mask(positions, length))

    kd, vd = keys.to(device), values.to(device)
    out = ops.decode_append(q.to(device), k_new.to(device), v_new.to(device), kd, vd, positions.to(device),
                            q_norm=q_w.to(device), k_norm=k_w.to(device), eps=eps, cos=cos.to(device),
                            sin=sin.to(device), num_splits=splits)
    assert_close(out, ref, KIND[dtype])
    assert _ulp_diff_ok(kd.cpu()[rows, positions], kn, dtype)
    assert torch.equal(vd.cpu()[rows, positions], v_new)
    untouched = torch.ones(batch, length, dtype=torch.bool)
    untouched[rows, positions] = False
    assert torch.equal(kd.cpu()[untouched], keys[untouched]) and torch.equal(vd.cpu()[untouched], values[untouched])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_append_gemma_prologue_matches_oracle(ops, device, dtype):
    """Gemma 4's step prologue fused into the decode launch (gemma4.py:515,
    :522-532, :563-587): q/k norms with weights, the value norm without
    (v_norm), the rotation, the cache writes, then 8 query heads over 4 kv
    heads at head_dim 256 over a 512-key window, scale 1.0; against the
    oracle module's norms (oracle.gemma4) and SDPA with the step's mask."""
    from oracle import gemma4 as og

    say("decode append gemma", dtype)
    hd, length, eps, window = 256, 1280, 1e-6, 512
    batch, heads_q, heads_kv = 5, 8, 4
    positions = torch.tensor([0, 37, 511, 512, 1000], dtype=torch.int64)
    q = randn(batch, heads_q, hd, seed=71, dtype=dtype)
    k_new = randn(batch, heads_kv, hd, seed=72, dtype=dtype)
    v_new = randn(batch, heads_kv, hd, seed=73, dtype=dtype)
    keys = randn(batch, length, heads_kv, hd, seed=74, dtype=dtype)
    values = randn(batch, length, heads_kv, hd, seed=75, dtype=dtype)
    g = torch.Generator().manual_seed(76)
    q_norm, k_norm, v_norm = og._Norm(hd, eps), og._Norm(hd, eps), og._Norm(hd, eps, scale=False)
    with torch.no_grad():
        q_norm.weight.copy_(torch.rand(hd, generator=g) + 0.5)
        k_norm.weight.copy_(torch.rand(hd, generator=g) + 0.5)
    q_w, k_w = q_norm.weight.detach().to(dtype), k_norm.weight.detach().to(dtype)
    q_norm.weight.data, k_norm.weight.data = q_w.float(), k_w.float()
    cos, sin = oa.rope_tables(1e4, hd, length, dtype)
    cos, sin = cos[positions], sin[positions]
    with torch.no_grad():
        qn = og.rotate(q_norm(q), cos, sin)
        kn = og.rotate(k_norm(k_new), cos, sin)
        vn = v_norm(v_new)
    rows = torch.arange(batch)
    keys_ref, values_ref = keys.clone(), values.clone()
    keys_ref[rows, positions] = kn
    values_ref[rows, positions] = vn
    mask = oa.gemma_step_mask(positions, length, window)
    ref = oa.sdpa(qn.float().view(batch, heads_kv, -1, hd), keys_ref.float().transpose(1, 2),
                  values_ref.float().transpose(1, 2), attn_mask=mask, scale=1.0).reshape(batch, heads_q, hd)

    kd, vd = keys.to(device), values.to(device)
    out = ops.decode_append(q.to(device), k_new.to(device), v_new.to(device), kd, vd, positions.to(device),
                            q_norm=q_w.to(device), k_norm=k_w.to(device), eps=eps, cos=cos.to(device),
                            sin=sin.to(device), scale=1.0, window=window, v_norm=True)
    assert_close(out, ref, KIND[dtype])
    assert _ulp_diff_ok(kd.cpu()[rows, positions], kn, dtype)
    assert _ulp_diff_ok(vd.cpu()[rows, positions], vn, dtype)


def _paginate(cache_k, cache_v, needed, page_size, seed, spare=3):
    """Pools ``(num_pages, page_size, H, D)`` holding each slab row's first
    ``needed[b]`` positions in randomly placed pages, and the block table
    (-1 past a row's pages).  Every other pool slot -- the tail of a row's
    last page and ``spare`` pages no row owns -- holds NaN, which any read
    of it would carry into the output."""
    batch, length, heads, hd = cache_k.shape
    per_row = [-(-int(n) // page_size) for n in needed]
    total = sum(per_row) + spare
    order = np.random.default_rng(seed).permutation(total)
    pool_k = torch.full((total, page_size, heads, hd), float("nan"), dtype=cache_k.dtype)
    pool_v = torch.full_like(pool_k, float("nan"))
    table = torch.full((batch, length // page_size), -1, dtype=torch.int32)
    i = 0
    for b in range(batch):
        for page in range(per_row[b]):
            table[b, page] = int(order[i])
            lo, hi = page * page_size, min((page + 1) * page_size, int(needed[b]))
            pool_k[int(order[i]), : hi - lo] = cache_k[b, lo:hi]
            pool_v[int(order[i]), : hi - lo] = cache_v[b, lo:hi]
            i += 1
    return pool_k, pool_v, table


@pytest.mark.parametrize(
    "dtype,hd,heads_q,heads_kv,page,splits,batch",
    [
        (torch.bfloat16, 128, 16, 8, 64, 0, 64),
        (torch.bfloat16, 128, 16, 8, 16, 0, 8),
        (torch.bfloat16, 128, 16, 8, 256, 0, 3),
        (torch.bfloat16, 128, 16, 8, 64, 7, 5),
        (torch.bfloat16, 64, 12, 12, 32, 0, 16),
        (torch.float32, 128, 16, 8, 16, 0, 4),
        (torch.float32, 64, 6, 6, 16, 1, 2),
    ],
)
def test_paged_decode_matches_slab_and_oracle(ops, device, dtype, hd, heads_q, heads_kv, page, splits, batch):
    """Decode over a paged cache (pages in random pool order, NaN in every
    slot no row owns) against the oracle on the slab it was cut from
    (qwen3_asr.py:412-432, :511-512); lengths 1, one page exactly, 1023 and
    random; split counts that do and do not align with pages.  At the
    Qwen3 batch (64 rows, 64-position pages) the workgroup shape equals the
    slab's and the output is bit-identical to decode over the slab."""
    say("paged decode", dtype, hd, heads_q, heads_kv, page, splits, batch)
    length = 1024
    rng = np.random.default_rng(80 + batch)
    lengths = rng.integers(1, length, size=batch).astype(np.int32)
    lengths[0] = 1
    if batch > 2:
        lengths[1], lengths[2] = page, length - 1
    q = randn(batch, heads_q, hd, seed=81, dtype=dtype)
    keys = randn(batch, length, heads_kv, hd, seed=82, dtype=dtype)
    values = randn(batch, length, heads_kv, hd, seed=83, dtype=dtype)
    pool_k, pool_v, table = _paginate(keys, values, lengths, page, seed=84)
    used = torch.from_numpy(lengths)
    ref = oa.qwen_step_attention(q.float(), keys.float(), values.float(),
                                 oa.qwen_step_mask(used.long() - 1, length))
    pages = ops.PageTable(table.to(device), length)
    out = ops.decode(q.to(device), pool_k.to(device), pool_v.to(device), seqused_k=used.to(device),
                     num_splits=splits, pages=pages)
    assert torch.isfinite(out).all()
    assert_close(out, ref, KIND[dtype])
    if batch == 64:
        slab = ops.decode(q.to(device), keys.to(device), values.to(device), seqused_k=used.to(device))
        assert torch.equal(out, slab)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_decode_append_matches_slab(ops, device, dtype):
    """The fused Qwen3 step on a paged cache: the new key and value land in
    slot positions % page_size of page table[b, positions // page_size] (page
    starts and ends included), nothing else changes, and the output equals
    the same step on the slab."""
    say("paged decode append", dtype)
    batch, heads_q, heads_kv, hd, length, page, eps = 64, 16, 8, 128, 1024, 64, 1e-6
    rng = np.random.default_rng(90)
    positions = torch.from_numpy(rng.integers(0, 1000, size=batch).astype(np.int64))
    positions[:4] = torch.tensor([0, 63, 64, 1023])
    q = randn(batch, heads_q, hd, seed=91, dtype=dtype)
    k_new = randn(batch, heads_kv, hd, seed=92, dtype=dtype)
    v_new = randn(batch, heads_kv, hd, seed=93, dtype=dtype)
    keys = randn(batch, length, heads_kv, hd, seed=94, dtype=dtype)
    values = randn(batch, length, heads_kv, hd, seed=95, dtype=dtype)
    g = torch.Generator().manual_seed(96)
    q_w = (torch.rand(hd, generator=g) + 0.5).to(dtype)
    k_w = (torch.rand(hd, generator=g) + 0.5).to(dtype)
    cos, sin = oa.rope_tables(1e6, hd, length, dtype)
    cos, sin = cos[positions].to(device), sin[positions].to(device)
    pool_k, pool_v, table = _paginate(keys, values, (positions + 1).numpy(), page, seed=97)
    # The slot the step writes must not hold an old key: poison it too.
    rows = torch.arange(batch)
    slots = table[rows, positions // page].long(), positions % page
    pool_k[slots] = float("nan")
    pool_v[slots] = float("nan")
    args = dict(q_norm=q_w.to(device), k_norm=k_w.to(device), eps=eps, cos=cos, sin=sin)
    kd, vd = keys.to(device), values.to(device)
    slab = ops.decode_append(q.to(device), k_new.to(device), v_new.to(device), kd, vd, positions.to(device), **args)
    pk, pv = pool_k.to(device), pool_v.to(device)
    out = ops.decode_append(q.to(device), k_new.to(device), v_new.to(device), pk, pv, positions.to(device),
                            pages=ops.PageTable(table.to(device), length), **args)
    assert torch.equal(out, slab)
    assert torch.equal(pk.cpu()[slots], kd.cpu()[rows, positions])
    assert torch.equal(pv.cpu()[slots], v_new)
    written = torch.zeros(pool_k.shape[:2], dtype=torch.bool)
    written[slots] = True
    for before, after in ((pool_k, pk.cpu()), (pool_v, pv.cpu())):
        before, after = before[~written], after[~written]
        assert bool(((after == before) | (before.isnan() & after.isnan())).all())


@pytest.mark.parametrize(
    "dtype,hd,heads_q,heads_kv,window,page,splits",
    [
        (torch.bfloat16, 256, 8, 1, 512, 0, 0),
        (torch.bfloat16, 512, 8, 1, 0, 0, 0),
        (torch.bfloat16, 512, 8, 2, 0, 0, 3),
        (torch.bfloat16, 256, 8, 2, 512, 64, 0),
        (torch.bfloat16, 256, 8, 1, 512, 16, 5),
        (torch.float32, 256, 8, 1, 512, 0, 0),
        (torch.float32, 256, 8, 2, 100, 0, 4),
        (torch.bfloat16, 128, 16, 8, 300, 0, 0),
    ],
)
def test_gemma_decode_window_and_head_sizes(ops, device, dtype, hd, heads_q, heads_kv, window, page, splits):
    """Gemma 4 text steps (gemma4.py:563-587, masks :717-725): head_dim 256
    (sliding layers, 512-key window) and 512 (full layers), 8 query heads
    over 1 or 2 kv heads, scale 1.0, against the oracle's masked SDPA;
    lengths around the window and the 1280-position cache end, slab and
    paged caches, split keys."""
    say("gemma decode", dtype, hd, heads_q, heads_kv, window, page, splits)
    batch, length = 7, 1280
    lengths = np.array([1, 511, 512, 513, 1279, 1280, 700], dtype=np.int32)
    q = randn(batch, heads_q, hd, seed=101, dtype=dtype) * 0.1
    keys = randn(batch, length, heads_kv, hd, seed=102, dtype=dtype)
    values = randn(batch, length, heads_kv, hd, seed=103, dtype=dtype)
    positions = torch.from_numpy(lengths.astype(np.int64) - 1)
    mask = oa.gemma_step_mask(positions, length, window or None)
    grouped = q.float().view(batch, heads_kv, heads_q // heads_kv, hd)
    ref = oa.sdpa(grouped, keys.float().transpose(1, 2), values.float().transpose(1, 2), attn_mask=mask, scale=1.0)
    ref = ref.reshape(batch, heads_q, hd)
    used = torch.from_numpy(lengths).to(device)
    if page:
        pool_k, pool_v, table = _paginate(keys, values, lengths, page, seed=104)
        out = ops.decode(q.to(device), pool_k.to(device), pool_v.to(device), seqused_k=used, scale=1.0,
                         window=window, num_splits=splits, pages=ops.PageTable(table.to(device), length))
    else:
        out = ops.decode(q.to(device), keys.to(device), values.to(device), seqused_k=used, scale=1.0,
                         window=window, num_splits=splits)
    assert torch.isfinite(out).all()
    assert_close(out, ref, KIND[dtype])


@pytest.mark.parametrize(
    "dtype,hd,heads_q,heads_kv,window",
    [
        (torch.bfloat16, 256, 8, 1, 512),
        (torch.bfloat16, 512, 8, 1, None),
        (torch.bfloat16, 512, 8, 2, None),
        (torch.float32, 256, 8, 2, 512),
        (torch.float32, 512, 8, 1, 100),
        (torch.bfloat16, 128, 16, 8, 100),
        (torch.bfloat16, 512, 8, 2, 100),
        (torch.bfloat16, 64, 8, 8, 33),
    ],
)
def test_gemma_prefill_window_and_head_sizes(ops, device, dtype, hd, heads_q, heads_kv, window):
    """Gemma 4's padded prompt pass (gemma4.py:552-559, masks :1227-1235):
    causal, keys before each prompt's size, the sliding window, scale 1.0,
    grouped-query attention, head_dim 256/512, against the oracle's masked
    SDPA on the prompts' own rows.  bf16 runs on the matrix-core kernel
    (head_dim 512 with its dimensions split over two waves), float32 on the
    vector-ALU kernel."""
    say("gemma prefill", dtype, hd, heads_q, heads_kv, window)
    batch, length = 3, 700
    sizes = torch.tensor([700, 513, 37])
    q = randn(batch, length, heads_q, hd, seed=121, dtype=dtype) * 0.1
    k = randn(batch, length, heads_kv, hd, seed=122, dtype=dtype)
    v = randn(batch, length, heads_kv, hd, seed=123, dtype=dtype)
    mask = oa.gemma_prefill_mask(sizes, length, window)
    ref = oa.sdpa(q.float().transpose(1, 2), k.float().transpose(1, 2), v.float().transpose(1, 2),
                  attn_mask=mask, scale=1.0, enable_gqa=True).transpose(1, 2)
    out = ops.flash(q.to(device), k.to(device), v.to(device), causal=1, seqused_k=sizes.int().to(device),
                    scale=1.0, window=window).cpu()
    for b, n in enumerate(sizes.tolist()):
        assert_close(out[b, :n], ref[b, :n], KIND[dtype])


def test_gemma_decode_append_window(ops, device):
    """The appending step with a window: the new key is the last of the
    window's keys, and only cache keys position - window + 1 .. position - 1
    join it."""
    say("gemma decode append, window")
    batch, heads_q, heads_kv, hd, length, window = 6, 8, 1, 256, 1280, 512
    positions = torch.tensor([0, 510, 511, 512, 1000, 1279])
    q = randn(batch, heads_q, hd, seed=111, dtype=torch.bfloat16) * 0.1
    k_new = randn(batch, heads_kv, hd, seed=112, dtype=torch.bfloat16)
    v_new = randn(batch, heads_kv, hd, seed=113, dtype=torch.bfloat16)
    keys = randn(batch, length, heads_kv, hd, seed=114, dtype=torch.bfloat16)
    values = randn(batch, length, heads_kv, hd, seed=115, dtype=torch.bfloat16)
    rows = torch.arange(batch)
    ref_k, ref_v = keys.clone(), values.clone()
    ref_k[rows, positions] = k_new
    ref_v[rows, positions] = v_new
    mask = oa.gemma_step_mask(positions, length, window)
    grouped = q.float().view(batch, heads_kv, heads_q // heads_kv, hd)
    ref = oa.sdpa(grouped, ref_k.float().transpose(1, 2), ref_v.float().transpose(1, 2), attn_mask=mask, scale=1.0)
    kd, vd = keys.to(device), values.to(device)
    out = ops.decode_append(q.to(device), k_new.to(device), v_new.to(device), kd, vd, positions.to(device),
                            scale=1.0, window=window)
    assert_close(out, ref.reshape(batch, heads_q, hd), KIND[torch.bfloat16])
    assert torch.equal(kd.cpu()[rows, positions], k_new) and torch.equal(vd.cpu()[rows, positions], v_new)


def test_decode_append_whisper_cache_without_norm(ops, device):
    """The Whisper step's scatter + attention (whisper.py:224-237) fused, no
    norm or rotation, into a (batch, heads, length, head_dim) cache through
    its transposed view."""
    say("decode append, whisper layout")
    rng = np.random.default_rng(70)
    positions = torch.from_numpy(rng.integers(0, 224, size=16).astype(np.int64))
    q = randn(16, 12, 64, seed=71, dtype=torch.bfloat16)
    k_new = randn(16, 12, 64, seed=72, dtype=torch.bfloat16)
    v_new = randn(16, 12, 64, seed=73, dtype=torch.bfloat16)
    cache_k = randn(16, 12, 448, 64, seed=74, dtype=torch.bfloat16)
    cache_v = randn(16, 12, 448, 64, seed=75, dtype=torch.bfloat16)
    rows = torch.arange(16)
    ref_k, ref_v = cache_k.clone(), cache_v.clone()
    ref_k[rows, :, positions] = k_new
    ref_v[rows, :, positions] = v_new
    ref = oa.sdpa(q[:, :, None].float(), ref_k[:, :, :256].float(), ref_v[:, :, :256].float(),
                  attn_mask=oa.whisper_step_mask(positions, 256))[:, :, 0]
    kd, vd = cache_k.to(device), cache_v.to(device)
    out = ops.decode_append(q.to(device), k_new.to(device), v_new.to(device), kd[:, :, :256].transpose(1, 2),
                            vd[:, :, :256].transpose(1, 2), positions.to(device))
    assert_close(out, ref, KIND[torch.bfloat16])
    assert torch.equal(kd.cpu(), ref_k) and torch.equal(vd.cpu(), ref_v)


# --- greedy choice (asrattn_choose) ---------------------------------------------


def _torch_choice(logits: torch.Tensor, suppress: torch.Tensor | None):
    x = logits.clone()
    if suppress is not None:
        x.masked_fill_(suppress, float("-inf"))
    token = x.argmax(dim=-1)
    return token, torch.log_softmax(x, dim=-1).gather(1, token[:, None]).squeeze(1)


@pytest.mark.parametrize("vocab", [1000, 51865, 151936])
def test_greedy_choice_matches_torch(ops, device, vocab):
    """argmax + log_softmax at it in one pass (whisper.py:962-974,
    qwen3_asr.py:1200-1210) against torch on the CPU: tokens exact,
    log-probabilities to 1e-5; rows with ties, a suppress mask, NaN, +inf
    and all -inf rows (and a NaN among -inf values only, which a plain max
    skips); odd vocabularies take the element-wise path."""
    say("greedy choice", vocab)
    g = torch.Generator().manual_seed(80 + vocab % 97)
    logits = torch.randn(12, vocab, generator=g) * 4
    logits[1, 7] = logits[1, vocab - 3] = logits[1].max() + 1.0  # tie: first index wins
    logits[2, :] = 0.5  # all equal
    logits[3, 5] = float("nan")
    logits[3, 9] = float("nan")
    logits[4, :] = float("-inf")
    logits[5, : vocab // 2] = float("-inf")
    logits[9, :] = float("-inf")
    logits[9, vocab // 3] = float("nan")  # the only non -inf value
    logits[10, 11] = logits[10, vocab - 5] = float("inf")  # +inf twice: the first wins
    logits[11, : vocab // 2] = float("-inf")
    logits[11, vocab // 4] = float("nan")  # inside the -inf half
    suppress = torch.zeros(vocab, dtype=torch.bool)
    suppress[torch.randperm(vocab, generator=g)[: vocab // 10]] = True
    suppress[int(logits[6].argmax())] = True  # the row's max is suppressed
    for mask in (None, suppress):
        want_t, want_p = _torch_choice(logits, mask)
        got_t, got_p = ops.greedy_choice(logits.to(device), None if mask is None else mask.to(device))
        got_t, got_p = got_t.cpu(), got_p.cpu()
        assert torch.equal(got_t, want_t), (got_t, want_t)
        nan = torch.isnan(want_p)
        assert torch.equal(torch.isnan(got_p), nan)
        assert torch.allclose(got_p[~nan], want_p[~nan], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("offset,vocab,stride", [(1, 1000, 1003), (0, 1001, 1004), (0, 4093, 4096)])
def test_greedy_choice_strided_rows(ops, device, offset, vocab, stride):
    """Rows inside a wider buffer: unaligned (4-byte loads), and aligned with
    a vocabulary that is not a multiple of four (16-byte loads plus the
    element-wise tail)."""
    buf = randn(6, stride, seed=85 + vocab) * 3
    buf[2, offset + vocab - 1] = 50.0  # the max sits in the tail
    mask = torch.zeros(vocab, dtype=torch.bool)
    mask[vocab - 2] = True
    for m in (None, mask):
        want_t, want_p = _torch_choice(buf[:, offset:offset + vocab], m)
        got_t, got_p = ops.greedy_choice(buf.to(device)[:, offset:offset + vocab], None if m is None else m.to(device))
        assert torch.equal(got_t.cpu(), want_t)
        assert torch.allclose(got_p.cpu(), want_p, rtol=1e-5, atol=1e-5)


def test_greedy_choice_column_major_logits(ops, device):
    """Logits of a transposed product (Whisper's head computes (W h^T)^T)."""
    w = randn(700, 64, seed=86)
    h = randn(5, 64, seed=87)
    logits = (w.to(device) @ h.to(device).T).T
    assert logits.stride(-1) != 1
    want_t, want_p = _torch_choice(logits.cpu(), None)
    got_t, got_p = ops.greedy_choice(logits)
    assert torch.equal(got_t.cpu(), want_t)
    assert torch.allclose(got_p.cpu(), want_p, rtol=1e-5, atol=1e-5)


def test_flash_refuses_out_without_unit_last_stride(ops, device):
    """The forward kernels write each head's head_dim elements contiguously:
    an out view with a non-unit last stride is refused, not written wrongly."""
    q = randn(1, 4, 2, 64, seed=30, dtype=torch.bfloat16).to(device)
    out = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16, device=device)[..., ::2]
    with pytest.raises(ValueError, match="unit last stride"):
        ops.flash(q, q, q, out=out)
    with pytest.raises(ValueError, match="unit last stride"):
        ops.flash_fsmn(q, q, q, torch.zeros(128, 11, dtype=torch.bfloat16, device=device), out=out)

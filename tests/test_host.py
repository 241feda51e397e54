"""CPU: host-side logic of the attention wrappers -- argument handling, mask
conversion and error mapping -- without launching kernels.

Failure injection follows the reference's own tests (host-side monkeypatching,
``tests/test_models.py:36-45``): a nonzero C-ABI status must surface as a
Python ``RuntimeError`` carrying the library's message.
"""

from __future__ import annotations

import subprocess
import sys

import pytest
import torch

from conftest import ROOT


def test_key_prefix_validation_and_mask_conversion():
    from asrback_amd.attention import KeyPrefix

    with pytest.raises(ValueError):
        KeyPrefix()
    with pytest.raises(ValueError):
        KeyPrefix(positions=torch.zeros(2, dtype=torch.int64), lengths=torch.zeros(2, dtype=torch.int32))
    with pytest.raises(TypeError):
        KeyPrefix(positions=torch.zeros(2, dtype=torch.int32))
    mask = torch.arange(10)[None, :] <= torch.tensor([0, 4, 9])[:, None]  # whisper.py:263-264
    prefix = KeyPrefix.from_mask(mask[:, None, None, :])
    assert prefix.lengths.tolist() == [1, 5, 10]
    with pytest.raises(TypeError):
        KeyPrefix.from_mask(mask.float())
    # A hole (False before True) is not a prefix: refused, not reduced to a count.
    holed = mask.clone()
    holed[2, 3] = False
    with pytest.raises(ValueError, match="prefix"):
        KeyPrefix.from_mask(holed[:, None, None, :])
    # Masks with more than one query row per sequence are not key prefixes.
    with pytest.raises(ValueError, match="mask"):
        KeyPrefix.from_mask(torch.ones(3, 1, 2, 10, dtype=torch.bool))
    assert KeyPrefix.from_mask(torch.zeros(2, 5, dtype=torch.bool)).lengths.tolist() == [0, 0]


def test_ops_refuse_cpu_tensors_instead_of_falling_back():
    from asrback_amd import attention

    q = torch.zeros(2, 4, 64)
    k = torch.zeros(2, 8, 4, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        attention.decode(q, k, k)
    with pytest.raises(RuntimeError, match="GPU only"):
        attention.flash(q[:, None], k, k)
    with pytest.raises(TypeError, match="float32 and bfloat16"):
        attention.decode(q.half(), k.half(), k.half())


def test_shape_errors_are_reported():
    from asrback_amd import attention

    with pytest.raises(ValueError):
        attention.decode(torch.zeros(2, 4, 64), torch.zeros(2, 8, 3, 64), torch.zeros(2, 8, 3, 64))
    with pytest.raises(ValueError, match="window_size"):
        attention.varlen_attn(torch.zeros(4, 2, 64), torch.zeros(4, 2, 64), torch.zeros(4, 2, 64),
                              torch.zeros(2, dtype=torch.int32), torch.zeros(2, dtype=torch.int32), 4, 4,
                              window_size=(8, 8))


def test_nonzero_status_raises_runtime_error(monkeypatch):
    from asrback_amd import _lib

    class FakeLib:
        def asrattn_last_error(self):
            return b"no decode kernel for head_dim 96"

    monkeypatch.setattr(_lib, "_handle", FakeLib())
    with pytest.raises(RuntimeError, match="head_dim 96") as info:
        _lib.check(_lib.ERR_UNSUPPORTED, "asrattn_decode")
    assert isinstance(info.value, _lib.AttentionError)
    assert info.value.status == _lib.ERR_UNSUPPORTED
    _lib.check(_lib.OK, "asrattn_decode")  # no exception


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from asrback_amd import _lib

    monkeypatch.setattr(_lib, "_handle", None)
    monkeypatch.setattr(_lib, "LIBRARY", tmp_path / "libasrattn.so")
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


def test_qwen_step_lengths_from_every_mask_form():
    from asrback_amd.attention import KeyPrefix
    from asrback_amd.qwen3_asr import _step_lengths
    from oracle import attention as oa

    positions = torch.tensor([0, 7, 300])
    lengths = torch.tensor([1, 8, 301], dtype=torch.int32)
    starts = torch.arange(4, dtype=torch.int32)
    assert torch.equal(_step_lengths((starts, starts * 1024, lengths), positions, 1024), lengths)
    assert torch.equal(_step_lengths(oa.qwen_step_mask(positions, 512), positions, 512), lengths)
    assert torch.equal(_step_lengths(KeyPrefix(positions=positions), positions, 1024), lengths)
    assert _step_lengths(None, positions, 256).tolist() == [1, 8, 256]


def test_segments_from_lengths_on_cpu():
    from asrback_amd.qwen3_asr import Segments

    segments = Segments.from_lengths([3, 5, 2], torch.device("cpu"))
    assert segments.starts.tolist() == [0, 3, 8, 10]
    assert segments.starts.dtype == torch.int32
    assert segments.longest == 5


def test_bench_refuses_more_than_one_gpu():
    result = subprocess.run(
        [sys.executable, str(ROOT / "bench.py"), "--gpus", "8"], capture_output=True, text=True, timeout=120
    )
    assert result.returncode == 2
    assert "one GPU" in result.stderr


def test_bench_gemma_audio_reference_ops_match_oracle():
    """The Gemma 4 audio line times the reference's sequence of ops as its
    unfused baseline; on the CPU that sequence equals the oracle's blocked
    attention (pad, unfold, relative shift, soft cap, mask, softmax)."""
    import types

    import bench
    from oracle import gemma4 as og

    torch.manual_seed(0)
    lengths = torch.tensor([50, 23])
    w = types.SimpleNamespace(torch=torch, chunk=12, past=12, mask=og.blocked_mask(lengths, 50, 12, 12, 0))
    q, k, v = (torch.randn(2, 50, 2, 16) for _ in range(3))
    rel = torch.randn(13, 2, 16)
    got = bench.Gemma4AudioAttention.reference_ops(w, q, k, v, rel)
    ref = og.local_attention(q, k, v, rel, w.mask, 12, 12, 0, 50.0, -1e9)
    assert torch.equal(got, ref)


def test_paged_layer_write_skips_rows_without_pages():
    """A bucket's free row (block table -1) must not write into a page another
    row owns: with the last pool page assigned to row 0, the unfused step's
    cache write for rows [0, 1] leaves row 0's keys intact (qwen3_asr.py
    ``PagedLayer.__setitem__``; torch indexing would map -1 to the last page)."""
    from asrback_amd.qwen3_asr import PagedKVCache

    config = {"num_hidden_layers": 1, "num_key_value_heads": 2, "head_dim": 8}
    cache = PagedKVCache.allocate(config, batch=2, num_pages=3, page_size=16, device="cpu", dtype=torch.float32)
    # Hand out pages until row 0 holds the last real page (2).
    cache.assign(0, 16 * 3)
    assert cache.block_table[0, :3].tolist() == [0, 1, 2]
    layer = cache.keys[0]
    rows = torch.tensor([0, 1])
    positions = torch.tensor([32, 0])  # row 0: page 2, slot 0; row 1: no page
    value = torch.stack([torch.full((2, 8), 7.0), torch.full((2, 8), -5.0)])
    layer[rows, positions] = value
    assert torch.equal(cache.pool_keys[0, 2, 0], torch.full((2, 8), 7.0))
    assert not (cache.pool_keys[0, :3] == -5.0).any()  # the free row's write went to the sink page



def test_workspace_sizes_and_scoped_buffer():
    """Split-K workspace sizing through the C ABI, and the caller-owned
    buffer a ``workspace`` block installs (checked before any device call)."""
    from asrback_amd import attention

    # 64 rows x 8 kv heads fill the GPU without splits; one row over 4096
    # keys splits (16 query heads x splits x 128 floats, plus the maxima and
    # sums).
    assert attention.decode_workspace_size(64, 16, 8, 128, 1024) == 0
    one = attention.decode_workspace_size(1, 16, 8, 128, 4096)
    assert one >= 16 * 16 * 128 * 4 and one % 256 == 0
    assert attention.decode_workspace_size(1, 16, 8, 128, 4096, num_splits=2) < one
    with pytest.raises(ValueError):
        attention.decode_workspace_size(1, 16, 8, 96, 4096)  # no kernel for head_dim 96
    assert attention.choice_workspace_size(64, 151936) > 0

    device = torch.device("cpu")
    small = torch.empty(64, dtype=torch.uint8)
    big = torch.empty(1 << 16, dtype=torch.uint8)
    assert attention._split_workspace(0, None, device) is None
    temporary = attention._split_workspace(1000, None, device)
    assert temporary.numel() == 1000 and temporary.dtype == torch.uint8
    with attention.workspace(big):
        assert attention._split_workspace(1000, None, device) is big
        assert attention._split_workspace(1000, small.new_empty(2000), device).numel() == 2000
        with attention.workspace(small):
            with pytest.raises(ValueError, match="needs 1000 workspace bytes"):
                attention._split_workspace(1000, None, device)
        assert attention._split_workspace(1000, None, device) is big
    assert attention._split_workspace(1000, None, device) is not big
    with pytest.raises(ValueError):
        with attention.workspace(torch.empty(8, dtype=torch.float32)):
            pass


def test_whisper_choose_samples_where_temperature_is_positive():
    """Whisper's choose takes the reference's temperatures (whisper.py:962-974):
    rows at temperature 0 take the argmax, rows above it sample, suppressed
    tokens are never chosen, and the log-probability is log_softmax at the
    chosen token."""
    import torch

    from asrback_amd.whisper import choose

    g = torch.Generator().manual_seed(5)
    logits = torch.randn(6, 50, generator=g)
    suppress = torch.zeros(50, dtype=torch.bool)
    suppress[[3, 7, 11]] = True
    temperatures = torch.tensor([0.0, 1.0, 0.0, 2.0, 0.5, 0.0])
    masked = logits.masked_fill(suppress, float("-inf"))
    torch.manual_seed(9)
    token, logprob = choose(logits.clone(), suppress, temperatures)
    greedy = temperatures == 0
    assert torch.equal(token[greedy], masked.argmax(dim=-1)[greedy])
    assert not suppress[token].any()
    ref_lp = torch.log_softmax(masked, dim=-1).gather(1, token[:, None]).squeeze(1)
    assert torch.allclose(logprob, ref_lp)
    # The same seed reproduces the reference's sampling ops exactly.
    torch.manual_seed(9)
    scaled = masked / temperatures.clamp(min=1e-6)[:, None]
    sampled = torch.multinomial(torch.softmax(scaled, dim=-1), 1).squeeze(1)
    assert torch.equal(token, torch.where(temperatures > 0, sampled, masked.argmax(dim=-1)))


def test_whisper_admit_checks_the_no_speech_arguments():
    """admit() with a no_speech_id needs the prompt position of
    <|startoftranscript|> (whisper.py:848-858); the check comes before any
    device work, so a wrong call fails on any machine."""
    import json

    from conftest import GOLDEN

    from asrback_amd import whisper as aw

    config = json.loads((GOLDEN / "whisper_tiny_greedy.json").read_text())["config"]
    model = aw.WhisperForConditionalGeneration(config).eval()
    suppress = torch.zeros(config["vocab_size"], dtype=torch.bool)
    dec = aw.GreedyDecoder(model, 2, suppress, suppress, config["eos_token_id"], graphs=False)
    encoded = torch.zeros(1, config["max_source_positions"], config["d_model"])
    for sot_index in (None, 4, -1):
        with pytest.raises(ValueError, match="sot_index"):
            dec.admit(encoded, [[1, 2, 3, 4]], 8, no_speech_id=5, sot_index=sot_index)

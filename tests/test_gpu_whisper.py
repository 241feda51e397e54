"""GPU: Whisper on the HIP attention kernels (``asrback_amd.whisper``).

The seeded float32 whisper-tiny model must decode exactly the committed
greedy token ids of the CPU oracle (``tests/golden/whisper_tiny_greedy.json``)
-- with the decoder step replayed from hipGraphs per (batch, KV) bucket and
eagerly; both paths must agree token for token.  Encoder and decoder hidden
states are compared with the oracle within 1e-4 relative (fp32 GEMMs and
LayerNorms differ from the CPU's in summation order; attention alone is held
to 1e-5 in test_gpu_configs).
"""

from __future__ import annotations

import json

import pytest
import torch

from conftest import GOLDEN, assert_close, max_rel_err
from oracle import whisper as ow

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fixture():
    return json.loads((GOLDEN / "whisper_tiny_greedy.json").read_text())


@pytest.fixture(scope="module")
def weights(fixture):
    model = ow.WhisperForConditionalGeneration(fixture["config"])
    return ow.attention_heavy_weights(model, fixture["seeds"]["weights"])


def mel_for(seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, 80, 3000, generator=g)


def gpu_model(fixture, weights, device, dtype=torch.float32):
    from asrback_amd import whisper as aw

    model = aw.WhisperForConditionalGeneration(fixture["config"])
    model.load_state_dict(weights, strict=True)
    return model.eval().to(device, dtype)


def decoder(model, fixture, device, batch, graphs):
    from asrback_amd import whisper as aw

    suppress, first = ow.suppress_masks(fixture["config"])
    return aw.GreedyDecoder(model, batch, suppress, first, fixture["config"]["eos_token_id"], graphs=graphs)


def run_rows(dec, model, mels, fixture, device):
    with torch.inference_mode():
        encoded = model.model.encoder(torch.cat(mels).to(device, next(model.parameters()).dtype))
        slots = dec.admit(encoded, [fixture["prefix"]] * len(mels), fixture["steps"])
        done = {}
        for _ in range(64):
            dec.advance()
            done.update(dec.finished_rows())
            if len(done) == len(slots):
                break
    return [done[s] for s in slots]


@pytest.mark.parametrize("graphs", [True, False])
def test_greedy_tokens_match_oracle_fixture(fixture, weights, device, graphs):
    print("whisper greedy, graphs =", graphs, flush=True)
    model = gpu_model(fixture, weights, device)
    dec = decoder(model, fixture, device, batch=1, graphs=graphs)
    (tokens,) = run_rows(dec, model, [mel_for(fixture["seeds"]["mel"])], fixture, device)
    assert tokens == fixture["tokens"]


def test_batch_rows_decode_independently(fixture, weights, device):
    """Two windows in one batch: the fixture's window decodes to the fixture
    tokens whatever shares its batch."""
    print("whisper batch of two", flush=True)
    model = gpu_model(fixture, weights, device)
    dec = decoder(model, fixture, device, batch=4, graphs=True)
    rows = run_rows(dec, model, [mel_for(fixture["seeds"]["mel"]), mel_for(77)], fixture, device)
    assert rows[0] == fixture["tokens"]
    assert rows[1] != fixture["tokens"]


def test_encoder_and_prefix_hidden_states_match_oracle(fixture, weights, device):
    print("whisper hidden states", flush=True)
    torch.set_num_threads(min(8, torch.get_num_threads()))
    ref = ow.WhisperForConditionalGeneration(fixture["config"]).eval()
    ref.load_state_dict(weights)
    model = gpu_model(fixture, weights, device)
    mel = mel_for(fixture["seeds"]["mel"])
    with torch.inference_mode():
        enc_ref = ref.model.encoder(mel)
        enc = model.model.encoder(mel.to(device))
        assert_close(enc.cpu(), enc_ref, "module", 1e-4)
        cache_ref = ref.allocate_cache(1)
        ref.set_encoder_output(cache_ref, enc_ref)
        prefix = torch.tensor([fixture["prefix"]])
        hid_ref = ref.model.decoder(prefix, torch.arange(4), cache_ref, 4)
        cache = model.allocate_cache(1)
        model.set_encoder_output(cache, enc)
        hid = model.decode(prefix.to(device), torch.arange(4, device=device), cache, length=4)
        assert_close(hid.cpu(), hid_ref, "module", 1e-4)


def test_bf16_model_decodes(fixture, weights, device):
    """bfloat16 (the reference's CUDA default) runs the same path, graphs
    included; its tokens need not equal the float32 ones."""
    print("whisper bf16", flush=True)
    model = gpu_model(fixture, weights, device, torch.bfloat16)
    dec = decoder(model, fixture, device, batch=1, graphs=True)
    (tokens,) = run_rows(dec, model, [mel_for(fixture["seeds"]["mel"])], fixture, device)
    assert len(tokens) == fixture["steps"]
    assert all(0 <= t < fixture["config"]["vocab_size"] for t in tokens)


def test_prompt_pass_side_outputs_match_oracle(fixture, weights, device):
    """The prompt pass's no-speech probability (softmax of the logits after
    <|startoftranscript|>, whisper.py:848-858) and the detected language
    (argmax over the language tokens after <|startoftranscript|> alone,
    :976-984) against the float32 CPU oracle on the same weights, two
    windows; a temperature of 0 keeps the greedy first token."""
    print("whisper prompt side outputs", flush=True)
    torch.set_num_threads(min(8, torch.get_num_threads()))
    ref = ow.WhisperForConditionalGeneration(fixture["config"]).eval()
    ref.load_state_dict(weights)
    model = gpu_model(fixture, weights, device)
    mel = torch.cat([mel_for(fixture["seeds"]["mel"]), mel_for(77)])
    languages = list(range(ow.EN, ow.EN + 99))  # the multilingual vocabulary's language tokens
    no_speech = ow.NO_TIMESTAMPS - 1  # <|nospeech|> there
    prefix = fixture["prefix"]
    with torch.inference_mode():
        enc_ref = ref.model.encoder(mel)
        cache_ref = ref.allocate_cache(2)
        ref.set_encoder_output(cache_ref, enc_ref)
        hid_ref = ref.model.decoder(torch.tensor([prefix] * 2), torch.arange(len(prefix)), cache_ref, len(prefix))
        probs_ref = ref.logits(hid_ref[:, prefix.index(ow.SOT)]).softmax(dim=-1)[:, no_speech]
        hid_lang = ref.model.decoder(torch.full((2, 1), ow.SOT), torch.arange(1), cache_ref, 1)
        lang_logits = ref.logits(hid_lang[:, -1])[:, languages]
        top2 = lang_logits.topk(2, dim=-1).values
        assert bool((top2[:, 0] - top2[:, 1] > 1e-3 * top2.abs().max()).all()), "near-tie in the oracle's languages"

        enc = model.model.encoder(mel.to(device))
        dec = decoder(model, fixture, device, batch=2, graphs=False)
        detected = dec.detect_languages(enc, ow.SOT, languages)
        slots = dec.admit(enc, [prefix] * 2, fixture["steps"], temperatures=[0.0, 0.0],
                          sot_index=prefix.index(ow.SOT), no_speech_id=no_speech)
        probs = torch.tensor(dec.no_speech_probs(slots))
        first = dec.state.tokens[slots[0], 0].item()
    assert detected == lang_logits.argmax(dim=-1).tolist()
    assert_close(probs, probs_ref, "module", 1e-4)
    assert first == fixture["tokens"][0]


def test_choose_samples_only_where_temperature_is_positive(device):
    """whisper.py:962-974 with temperatures (0, 0.8): the product's choose
    runs the reference's ops for the whole batch -- the zero-temperature
    row takes the greedy token (the fused greedy pass's choice), the other
    samples under a seeded generator, and each row's log-probability is the
    unscaled log_softmax at its token, suppressed tokens included as -inf."""
    from asrback_amd import attention
    from asrback_amd import whisper as aw

    vocab = ow.WHISPER_TINY["vocab_size"]
    g = torch.Generator().manual_seed(31)
    logits = (torch.randn(2, vocab, generator=g) * 3).to(device)
    suppress, _ = ow.suppress_masks(ow.WHISPER_TINY)
    suppress = suppress.to(device)
    greedy_token, greedy_logprob = attention.greedy_choice(logits.clone(), suppress)
    reference = torch.log_softmax(logits.masked_fill(suppress, float("-inf")), dim=-1).cpu()
    temperatures = torch.tensor([0.0, 0.8], device=device)
    torch.manual_seed(32)
    token, logprob = aw.choose(logits.clone(), suppress, temperatures)
    token, logprob = token.cpu(), logprob.cpu()
    assert token[0] == greedy_token[0].cpu()
    assert torch.allclose(logprob[0], greedy_logprob[0].cpu(), rtol=1e-5, atol=1e-5)
    assert not suppress[token[1]]
    assert torch.allclose(logprob, reference.gather(1, token[:, None]).squeeze(1), rtol=1e-5, atol=1e-5)
    torch.manual_seed(32)
    again, _ = aw.choose(logits.clone(), suppress, temperatures)
    assert torch.equal(again.cpu(), token)  # the seeded draw repeats

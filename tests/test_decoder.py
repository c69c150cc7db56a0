"""The decode harnesses (the reference's runtime_8b.py Starcoder2Block /
Starcoder2, runtime_1b.py BigCodeBlock / GPTBigCode and runtime_shared.py
CachedDecoding / _beam_sample) on small configurations.

Teacher forcing pins the cache machinery: decoding token t after a prefill
of L positions must give the logits that a prefill of the L + 1 positions
gives at its last position (same RoPE angles or position embedding, same
keys and values, same mask). On the GPU, graph replays are compared with
eager decode steps; the fused HIP decode against a pure-torch restatement is
tests/test_gpu_decoder_parity.py.
"""
from __future__ import annotations

import pytest
import torch

import starvector_amd.quantization as quantization
import starvector_amd.decoder as decoder
from starvector_amd.decoder import (BigCodeConfig, DecoderConfig, GPTBigCodeDecoder,
                                    Starcoder2Decoder, beam_steps, beam_steps_reference)

# head_dim 128, as every StarVector decoder (the fused decode attention
# kernel's head size); 2 query heads per key/value head.
SMALL = DecoderConfig(hidden=512, heads=4, kv_heads=2, inner=1024, layers=2, vocab=320,
                      window=4096, context=512)
SMALL_1B = BigCodeConfig(hidden=512, heads=4, inner=1024, layers=2, vocab=320, context=512)


def small_model(device, qtype="Q4_0"):
    model = Starcoder2Decoder(SMALL, qtype=qtype, seed=3, device=device)
    return model.to_host() if device == "cpu" else model


def prompt(length, device, dtype):
    g = torch.Generator(device=device).manual_seed(7)
    return torch.randn((1, length, SMALL.hidden), generator=g, device=device).to(dtype)


def teacher_forced(model, emb, token):
    """(decode-step logits, prefill logits) for `token` after `emb`."""
    with torch.inference_mode():
        decoding, _ = model.prefill(emb, 2, emb.shape[1] + 4)
        stepped = decoding.step(torch.tensor([token, token], device=emb.device)).clone()
        extended = torch.cat((emb, model.embed(torch.tensor([[token]], device=emb.device)).to(emb.dtype)), 1)
        _, full = model.prefill(extended, 1, extended.shape[1] + 1)
    return stepped, full


@pytest.mark.parametrize("qtype", ("Q4_0", "Q5_0", "Q8_0"))
def test_decode_step_matches_prefill_cpu(qtype):
    model = small_model("cpu", qtype)
    stepped, full = teacher_forced(model, prompt(9, "cpu", torch.float32), 17)
    assert torch.equal(stepped[0], stepped[1])
    err = ((stepped[0] - full[0]).abs().max() / full.abs().max()).item()
    assert err <= 1e-4, err


@pytest.mark.parametrize("qtype", ("Q4_0", "Q5_0", "Q8_0"))
def test_bigcode_decode_step_matches_prefill_cpu(qtype):
    """GPTBigCode-1B: the decode step at position L (token embedding plus
    position embedding L, the new key/value slot, multi-query attention over
    the cache) equals the last position of a prefill of L + 1 tokens."""
    model = GPTBigCodeDecoder(SMALL_1B, qtype=qtype, embed_qtype="Q8_0", seed=5,
                              device="cpu").to_host()
    stepped, full = teacher_forced(model, prompt(9, "cpu", torch.float32), 17)
    assert torch.equal(stepped[0], stepped[1])
    err = ((stepped[0] - full[0]).abs().max() / full.abs().max()).item()
    assert err <= 1e-4, err


def test_bigcode_cache_layout_and_masking_cpu():
    """The 1B cache is [layers, rows, 1, capacity, head_dim]; a decode step
    writes exactly slot `position` of every layer and row."""
    model = GPTBigCodeDecoder(SMALL_1B, qtype="Q4_0", seed=5, device="cpu").to_host()
    emb = prompt(6, "cpu", torch.float32)
    with torch.inference_mode():
        decoding, _ = model.prefill(emb, 2, 10)
        assert decoding.keys.shape == (2, 2, 1, 10, 128)
        before = decoding.kv.clone()
        decoding.step(torch.tensor([3, 4]))
    changed = (decoding.kv != before).flatten(0, 3).any(-1)  # [2 * layers * rows, slots]
    assert changed.all(0).tolist() == [False] * 6 + [True] + [False] * 3


def test_beam_steps_cpu():
    model = small_model("cpu")
    torch.manual_seed(0)
    with torch.inference_mode():
        tokens, scores = beam_steps(model, prompt(5, "cpu", torch.float32), 4, beams=2)
    assert len(tokens) == 4 and all(0 <= t < SMALL.vocab for t in tokens)
    assert len(scores) == 2


@pytest.mark.gpu
def test_decode_step_matches_prefill_gpu(cuda_device):
    model = small_model(cuda_device)
    stepped, full = teacher_forced(model, prompt(9, cuda_device, torch.float16), 17)
    err = ((stepped[0].float() - full[0].float()).abs().max() / full.float().abs().max()).item()
    assert err <= 2e-2, err


@pytest.mark.gpu
def test_graph_replays_match_eager_decode(cuda_device):
    """CachedDecoding replays one captured graph per span; every replay, with
    eager work and synchronization between replays, matches an eager decode of
    the same step."""
    model = small_model(cuda_device)
    emb = prompt(12, cuda_device, torch.float16)
    tokens = [(5, 6), (300, 2), (17, 17), (1, 319)]
    with torch.inference_mode():
        decoding, _ = model.prefill(emb, 2, 40)
        eager, _ = model.prefill(emb, 2, 40)
        for a, b in tokens:
            t = torch.tensor([a, b], device=cuda_device)
            got = decoding.step(t).float().clone()
            torch.cuda.synchronize()
            eager.tokens.copy_(t)
            want = eager._decode(decoding.span()).float()
            eager.position += 1
            eager.length += 1
            assert len(decoding.graphs) == 1
            err = ((got - want).abs().max() / want.abs().max()).item()
            assert err <= 1e-3, err


@pytest.mark.parametrize("parents", ([0, 0, 2], [1, 1, 1], [1, 0, 2], [2, 0, 1], [0, 1, 2]))
def test_reorder_matches_indexing(parents):
    """Slice copies and the gather path give each row its parent's cache, as
    indexing the cache with the parent list does (runtime_shared.py:388-394)."""
    from starvector_amd.decoder import CachedDecoding
    g = torch.Generator().manual_seed(4)
    keys = torch.randn((2, 3, 2, 10, 4), generator=g)
    values = torch.randn((2, 3, 2, 10, 4), generator=g)
    decoding = CachedDecoding.__new__(CachedDecoding)
    decoding.keys, decoding.values, decoding.length = keys.clone(), values.clone(), 7
    decoding.reorder(parents)
    for cache, original in ((decoding.keys, keys), (decoding.values, values)):
        want = original.clone()
        want[:, :, :, :7] = original[:, parents, :, :7]
        assert torch.equal(cache, want)


def _scores(rows, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.log_softmax(torch.randn((rows, vocab), generator=g) * 3, -1)


@pytest.mark.parametrize("temperature,top_p,keep", ((1.5, 0.9, 2), (1.0, 0.9, 4), (0.7, 0.5, 2),
                                                    (1.5, 1.0, 2), (2.0, 0.99, 2)))
def test_warp_candidates_matches_warp(temperature, top_p, keep):
    """The candidate warper against the whole-vocabulary restatement of the
    reference's warpers, on seeded log-probabilities without ties."""
    for seed in range(6):
        scores = _scores(2, 49152, seed)
        want = decoder.warp(scores, temperature, top_p, keep)
        got, overflow = decoder.warp_candidates(scores, temperature, top_p, keep)
        assert not bool(overflow)
        assert torch.equal(got, want), seed
        assert int(torch.isfinite(got).sum(-1).min()) >= keep


def test_warp_candidates_ties():
    """Values tied with the k-th largest: within the candidate room they are
    kept as the reference keeps them; beyond it the overflow flag is set."""
    scores = _scores(2, 1000, 11)
    top = torch.topk(scores[0], decoder.TOP_K).values
    few = scores.clone()
    few[0, :5] = top[-1]  # 5 extra entries equal to the threshold
    got, overflow = decoder.warp_candidates(few, 1.0, 1.0, 2)
    assert not bool(overflow)
    assert torch.equal(got, decoder.warp(few, 1.0, 1.0, 2))
    many = scores.clone()
    many[1, :40] = torch.topk(scores[1], decoder.TOP_K).values[-1]
    _, overflow = decoder.warp_candidates(many, 1.0, 0.9, 2)
    assert bool(overflow)


def test_beam_steps_overflow_uses_warp(monkeypatch):
    """A tie overflow on every step sends beam sampling to the reference form."""
    calls = []
    real = decoder.warp

    def counting(*args):
        calls.append(1)
        return real(*args)

    monkeypatch.setattr(decoder, "warp", counting)
    monkeypatch.setattr(decoder, "TIE_ROOM", 0)
    model = small_model("cpu")
    torch.manual_seed(0)
    with torch.inference_mode():
        emb = prompt(5, "cpu", torch.float32)
        tokens, _ = beam_steps(model, emb, 3, beams=2)
    assert len(tokens) == 3
    assert len(calls) == 3  # TIE_ROOM 0: the k-th value always fills the last slot


def beam_steps_host_selection(decoder_model, embeddings, steps, beams=2, temperature=1.5,
                              top_p=0.9):
    """The beam loop with the survivors chosen on the host, as the reference
    does (runtime_shared.py:214-265: Python lists, `sorted`, a host list of
    parents for the cache reorder) -- the checker for `beam_steps`, whose
    selection stays on the device."""
    keep = 2 * beams
    decoding, logits = decoder_model.prefill(embeddings, beams, embeddings.shape[1] + steps + 1)
    device, vocab = logits.device, logits.shape[-1]
    running = [[] for _ in range(beams)]
    running_scores = [0.0] + [-1e9] * (beams - 1)
    seen = torch.zeros((beams, vocab), dtype=torch.bool, device=device)
    for _ in range(steps):
        penalized = decoder.penalize(torch.log_softmax(logits.float(), -1), seen)
        log_probs, overflow = decoder.warp_candidates(penalized, temperature, top_p, 2)
        if bool(overflow):
            log_probs = decoder.warp(penalized, temperature, top_p, 2)
        scores = (log_probs + torch.tensor(running_scores, device=device)[:, None]).view(1, -1)
        probs = scores.softmax(-1)
        picks = torch.multinomial(probs, min(keep, int(torch.count_nonzero(probs))))
        picked = scores.gather(1, picks)[0].tolist()
        parents, tokens = zip(*(divmod(pick, vocab) for pick in picks[0].tolist()))
        order = sorted(range(len(picked)), key=picked.__getitem__, reverse=True)[:beams]
        running_scores = [picked[j] for j in order] + [-1e9] * (beams - len(order))
        order += [order[0]] * (beams - len(order))
        running = [running[parents[j]] + [tokens[j]] for j in order]
        selected = torch.tensor([parents[j] for j in order], device=device)
        next_tokens = torch.tensor([tokens[j] for j in order], device=device)
        seen = seen[selected]
        seen[torch.arange(beams, device=device), next_tokens] = True
        decoding.reorder([parents[j] for j in order])
        logits = decoding.step(next_tokens)
    return running[0], running_scores


def test_beam_steps_reference_loop_matches_beam_steps_cpu():
    """The reference's loop as it runs it (whole-vocabulary warpers,
    torch.multinomial, host survivor selection) and the loop of the fused
    path (candidate warpers, the multinomial draws restated, device-side
    selection) give the same tokens and scores from the same seed."""
    model = small_model("cpu")
    emb = prompt(5, "cpu", torch.float32)
    with torch.inference_mode():
        torch.manual_seed(9)
        want = beam_steps_reference(model, emb, 6, beams=2)
        torch.manual_seed(9)
        got = beam_steps(model, emb, 6, beams=2)
    assert got[0] == want[0], (got, want)
    torch.testing.assert_close(torch.tensor(got[1]), torch.tensor(want[1]), rtol=1e-6, atol=1e-5)


@pytest.mark.parametrize("loop", (beam_steps, beam_steps_reference))
def test_beam_steps_nan_logits_raise_as_multinomial_does(monkeypatch, loop):
    """NaN logits make NaN probabilities: the reference's torch.multinomial
    rejects them, and both loops raise that error instead of drawing."""
    model = small_model("cpu")
    real = type(model.lm_head).forward

    def nan_logits(self, x):
        return torch.full_like(real(self, x), float("nan"))

    monkeypatch.setattr(type(model.lm_head), "forward", nan_logits)
    with torch.inference_mode(), pytest.raises(RuntimeError):
        loop(model, prompt(5, "cpu", torch.float32), 2, beams=2)


def test_possible_draws_counts_positive_and_flags_nan():
    probs = torch.tensor([[0.5, 0.0, 0.25, 0.25]])
    assert int(decoder.possible_draws(probs)) == 3
    assert int(decoder.possible_draws(torch.tensor([[0.5, float("nan"), 0.5, 0.0]]))) == -1


def test_beam_steps_matches_host_selection_cpu():
    """Device-side survivor selection and cache reorder give the sequence and
    scores of the host-side bookkeeping (same seed, same draws)."""
    model = small_model("cpu")
    emb = prompt(5, "cpu", torch.float32)
    with torch.inference_mode():
        torch.manual_seed(4)
        want = beam_steps_host_selection(model, emb, 6, beams=2)
        torch.manual_seed(4)
        got = beam_steps(model, emb, 6, beams=2)
    assert got[0] == want[0] and got[1] == want[1], (got, want)


@pytest.mark.gpu
def test_beam_steps_matches_host_selection_gpu(cuda_device):
    """The same on the GPU: the candidate and selection kernels, the
    svq_cache_reorder kernel and graph-replayed steps against torch warpers,
    torch.multinomial, host-chosen parents and torch slice copies."""
    model = small_model(cuda_device)
    emb = prompt(9, cuda_device, torch.float16)
    with torch.inference_mode():
        torch.manual_seed(5)
        want = beam_steps_host_selection(model, emb, 8, beams=2)
        torch.manual_seed(5)
        got = beam_steps(model, emb, 8, beams=2)
    # The candidate kernels' sums add in another order than torch's: the
    # running scores agree to rounding, the tokens exactly.
    assert got[0] == want[0], (got, want)
    torch.testing.assert_close(torch.tensor(got[1]), torch.tensor(want[1]), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("values", ([3.0, 1.0, 3.0, 2.0], [1.0, 1.0, 1.0, 1.0], [0.5],
                                    [-1e9, 2.0, 2.0, -1e9], [5.0, 4.0, 3.0, 2.0, 4.0, 5.0]))
def test_stable_descending_is_python_sorted(values):
    """The survivors' order: Python's sorted(..., reverse=True), ties in index
    order (the reference's selection, runtime_shared.py:245)."""
    got_values, got_order = decoder.stable_descending(torch.tensor(values))
    want = sorted(range(len(values)), key=values.__getitem__, reverse=True)
    assert got_order.tolist() == want
    assert got_values.tolist() == [values[i] for i in want]


def _rope_table_matches(device, dtype):
    model = Starcoder2Decoder(SMALL, qtype="Q4_0", seed=3, device=device)
    cos_t, sin_t = model._rope(torch.arange(600, device=device), dtype)
    for p in (0, 1, 17, 511, 599):
        cos, sin = model._rope(torch.tensor([p], device=device), dtype)
        assert torch.equal(cos_t[p:p + 1], cos) and torch.equal(sin_t[p:p + 1], sin), p


def test_rope_table_rows_equal_per_position_angles_cpu():
    """A decode step gathers its RoPE row from a table of every slot: the rows
    must be the per-position values bit for bit."""
    _rope_table_matches("cpu", torch.float32)


@pytest.mark.gpu
def test_rope_table_rows_equal_per_position_angles_gpu(cuda_device):
    _rope_table_matches(cuda_device, torch.float16)

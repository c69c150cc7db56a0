"""svq_beam_select (the survivor selection of a beam-sampling step) against
the torch formulation of runtime_shared.py:233-262 on the same inputs, and
its draws against torch.multinomial itself (same generator state).

Inputs are built as a beam step builds them: each beam has `ncand` candidate
tokens (a top-k of random logits); probabilities and scores are zero / -inf
elsewhere. Scores are rounded to a coarse grid in some cases so that drawn
scores tie and the stable order matters. Everything is exact: results must
be equal, not close.
"""
from __future__ import annotations

import pytest
import torch

import starvector_amd._native as native

pytestmark = pytest.mark.gpu


def make_case(device, beams, vocab, ncand, seed, ties=False, dead=0):
    g = torch.Generator(device=device).manual_seed(seed)
    logits = torch.randn((beams, vocab), generator=g, device=device)
    candidates = torch.topk(logits, ncand).indices
    scores = torch.full((beams, vocab), float("-inf"), device=device)
    vals = torch.randn((beams, ncand), generator=g, device=device) * 2
    if ties:
        vals = torch.round(vals * 2) / 2
    # `dead` candidates per beam carry no probability (masked by top-p).
    if dead:
        vals[:, ncand - dead:] = float("-inf")
    scores.scatter_(1, candidates, vals)
    scores = scores.view(1, -1)
    probs = scores.softmax(-1)
    noise = torch.empty_like(probs).exponential_(generator=g)
    pitch = (vocab + 15) // 16 * 16
    seen = torch.rand((beams, pitch), generator=g, device=device) < 0.1
    return probs, noise, scores, candidates.contiguous(), seen


def torch_select(probs, noise, scores, draws, seen, beams, vocab):
    q = probs / noise
    picks = torch.argmax(q, -1, keepdim=True)[0] if draws == 1 else torch.topk(q, draws).indices[0]
    picked = scores[0].gather(0, picks)
    ordered, order = torch.sort(picked, descending=True, stable=True)
    kept = min(beams, draws)
    chosen = picks[order[:kept]]
    running = ordered[:kept]
    if kept < beams:
        chosen = torch.cat((chosen, chosen[:1].expand(beams - kept)))
        running = torch.cat((running, torch.full((beams - kept,), -1e9, device=probs.device)))
    parents, tokens = chosen // vocab, chosen % vocab
    seen_next = seen[parents].clone()
    seen_next[torch.arange(beams, device=probs.device), tokens] = True
    return parents, tokens, running, seen_next


def run_select(probs, noise, scores, candidates, draws, seen, beams):
    dev = probs.device
    seen_out = torch.ones_like(seen)  # every byte must be overwritten
    running = torch.full((beams,), 7.0, device=dev)
    parents = torch.full((beams,), -5, dtype=torch.long, device=dev)
    tokens = torch.full((beams,), -5, dtype=torch.long, device=dev)
    copy = torch.full((beams,), -5, dtype=torch.long, device=dev)
    native.beam_select(probs, noise, scores, candidates, draws, seen, seen_out, running, parents,
                       tokens, copy)
    torch.cuda.synchronize()
    return parents, tokens, running, seen_out, copy


CASES = [
    # beams, vocab, ncand, draws, ties, dead
    (1, 320, 64, 1, False, 0),
    (1, 320, 64, 2, True, 0),
    (2, 320, 64, 4, False, 0),
    (2, 1001, 64, 4, True, 0),
    (2, 49152, 64, 4, False, 0),
    (2, 49157, 64, 3, True, 0),
    (2, 49152, 64, 1, False, 0),
    (3, 1001, 64, 6, True, 10),
    (4, 4096, 64, 2, False, 0),   # fewer draws than beams: padded survivors
    (4, 4096, 64, 8, True, 0),
    (8, 49152, 128, 16, True, 0),
    (8, 777, 100, 5, False, 90),
]


@pytest.mark.parametrize("beams,vocab,ncand,draws,ties,dead", CASES)
@pytest.mark.parametrize("seed", (1, 2))
def test_beam_select_matches_torch(cuda_device, beams, vocab, ncand, draws, ties, dead, seed):
    probs, noise, scores, candidates, seen = make_case(cuda_device, beams, vocab, ncand, seed,
                                                       ties, dead)
    want = torch_select(probs, noise, scores, draws, seen, beams, vocab)
    parents, tokens, running, seen_out, copy = run_select(probs, noise, scores, candidates, draws,
                                                          seen, beams)
    assert torch.equal(parents, want[0]), (parents, want[0])
    assert torch.equal(tokens, want[1]), (tokens, want[1])
    assert torch.equal(copy, want[1])
    assert torch.equal(running, want[2]), (running, want[2])
    assert torch.equal(seen_out, want[3])


@pytest.mark.parametrize("beams,draws", ((1, 1), (2, 4), (2, 1), (4, 8), (3, 2)))
def test_beam_select_draws_are_torch_multinomial(cuda_device, beams, draws):
    """The race with the Exp(1) draws that torch.multinomial would make from
    the same generator state picks what torch.multinomial picks."""
    vocab, ncand = 2048, 64
    probs, _, scores, candidates, seen = make_case(cuda_device, beams, vocab, ncand, 11)
    torch.manual_seed(123)
    picks = torch.multinomial(probs, draws)[0]
    torch.manual_seed(123)
    noise = torch.empty_like(probs).exponential_()
    parents, tokens, _, _, _ = run_select(probs, noise, scores, candidates, draws, seen, beams)
    picked = scores[0].gather(0, picks)
    order = torch.sort(picked, descending=True, stable=True).indices[:min(beams, draws)]
    survivors = picks[order]
    kept = survivors.numel()
    assert torch.equal(parents[:kept] * vocab + tokens[:kept], survivors)


def test_beam_select_twice_in_a_row(cuda_device):
    """Two calls that swap the seen buffers, as the decode loop does."""
    beams, vocab = 2, 1001
    a = make_case(cuda_device, beams, vocab, 64, 5)
    b = make_case(cuda_device, beams, vocab, 64, 6)
    seen0 = a[4]
    start = seen0.clone()
    seen1 = torch.zeros_like(seen0)
    run = lambda case, src, dst: native.beam_select(
        case[0], case[1], case[2], case[3], 4, src, dst, torch.zeros(beams, device=cuda_device),
        torch.zeros(beams, dtype=torch.long, device=cuda_device),
        torch.zeros(beams, dtype=torch.long, device=cuda_device))
    run(a, seen0, seen1)
    run(b, seen1, seen0)
    torch.cuda.synchronize()
    first = torch_select(a[0], a[1], a[2], 4, start, beams, vocab)[3]
    second = torch_select(b[0], b[1], b[2], 4, first, beams, vocab)[3]
    assert torch.equal(seen0, second)


def test_beam_select_rejects_mismatched_tensors(cuda_device):
    probs, noise, scores, candidates, seen = make_case(cuda_device, 2, 320, 64, 1)
    out = torch.zeros_like(seen)
    f = torch.zeros(2, device=cuda_device)
    i = torch.zeros(2, dtype=torch.long, device=cuda_device)
    with pytest.raises(ValueError):
        native.beam_select(probs.half(), noise, scores, candidates, 4, seen, out, f, i, i)
    with pytest.raises(ValueError):
        native.beam_select(probs, noise, scores, candidates, 4, seen, out[:1], f, i, i)
    with pytest.raises(native.SVQError):
        native.beam_select(probs, noise, scores, candidates, 5, seen, out, f, i, i)


# --- svq_beam_candidates against the torch formulation of the warpers ---

from starvector_amd import decoder  # noqa: E402


def torch_candidates(logits, seen, running, temperature, top_p, keep=2):
    beams, vocab = logits.shape
    penalized = decoder.penalize(torch.log_softmax(logits.float(), -1), seen[:, :vocab])
    log_probs, overflow, index = decoder.warp_candidates(penalized, temperature, top_p, keep,
                                                         with_index=True)
    scores = (log_probs + running[:, None]).view(1, -1)
    probs = scores.softmax(-1)
    count = torch.count_nonzero(probs.view(beams, vocab).gather(1, index))
    return scores.view(beams, vocab), probs.view(beams, vocab), int(count), bool(overflow)


def run_candidates(logits, seen, running, temperature, top_p, keep=2):
    beams, vocab = logits.shape
    k = max(decoder.TOP_K, keep)
    kc = min(k + decoder.TIE_ROOM, vocab)
    dev = logits.device
    cand = torch.full((beams, kc), -7, dtype=torch.long, device=dev)
    scores = torch.full((beams, kc), 7.0, device=dev)
    probs = torch.full((beams * kc,), 7.0, device=dev)
    status = torch.full((2 + beams,), -7, dtype=torch.long, device=dev)
    ws = native.beam_candidates_workspace(beams, vocab, kc, dev)
    native.beam_candidates(logits, seen, running, k, kc, keep, decoder.REPETITION_PENALTY,
                           temperature, top_p, cand, scores, probs, status, ws)
    torch.cuda.synchronize()
    return cand, scores, probs.view(beams, kc), status


def logits_case(device, beams, vocab, seed, ties=False, seen_rate=0.05):
    g = torch.Generator(device=device).manual_seed(seed)
    logits = torch.randn((beams, vocab), generator=g, device=device) * 3
    if ties:
        logits = torch.round(logits)
    pitch = (vocab + 15) // 16 * 16
    seen = torch.rand((beams, pitch), generator=g, device=device) < seen_rate
    # Seen tokens among the top ones, so the penalty reorders the top-k.
    top = torch.topk(logits, 8).indices
    seen.scatter_(1, top[:, ::2], True)
    running = torch.randn(beams, generator=g, device=device) * 4
    return logits.half(), seen, running


CAND_CASES = [
    # beams, vocab, temperature, top_p
    (1, 320, 1.0, 1.0),
    (2, 320, 1.5, 0.9),
    (2, 1001, 1.5, 0.9),
    (2, 49152, 1.5, 0.9),
    (2, 49157, 0.7, 0.5),
    (4, 4096, 1.0, 0.9),
    (8, 49152, 1.5, 0.95),
    (3, 65536, 1.5, 0.9),
]


@pytest.mark.parametrize("beams,vocab,temperature,top_p", CAND_CASES)
@pytest.mark.parametrize("seed", (1, 2))
def test_beam_candidates_match_torch(cuda_device, beams, vocab, temperature, top_p, seed):
    logits, seen, running = logits_case(cuda_device, beams, vocab, seed)
    if beams > 1:
        running[1] = -1e9  # a dead beam, as in the first steps
    want_scores, want_probs, want_count, want_overflow = torch_candidates(
        logits, seen, running, temperature, top_p)
    cand, scores, probs, status = run_candidates(logits, seen, running, temperature, top_p)
    assert bool(status[1]) == want_overflow is False
    assert int(status[0]) == want_count
    for r in range(beams):
        got_s, got_p = scores[r], probs[r]
        ws = want_scores[r].gather(0, cand[r])
        wp = want_probs[r].gather(0, cand[r])
        # Same kept tokens (finite scores), scores and probabilities to rounding.
        assert torch.equal(torch.isfinite(got_s), torch.isfinite(ws))
        assert int(torch.isfinite(got_s).sum()) == int(torch.isfinite(want_scores[r]).sum())
        fin = torch.isfinite(ws)
        torch.testing.assert_close(got_s[fin], ws[fin], rtol=1e-6, atol=1e-5)
        torch.testing.assert_close(got_p, wp, rtol=1e-5, atol=1e-7)
        # Candidates are distinct, in range, and their warped values descend.
        assert cand[r].unique().numel() == cand.shape[1]
        assert int(cand[r].min()) >= 0 and int(cand[r].max()) < vocab
        vals = (scores[r] - running[r])[fin]
        assert bool((vals[1:] <= vals[:-1]).all())


def test_beam_candidates_report_tie_overflow(cuda_device):
    """Rounded logits tie at the top-k threshold beyond the candidate room:
    both forms report the overflow."""
    logits, seen, running = logits_case(cuda_device, 2, 49152, 3, ties=True, seen_rate=0.0)
    want = torch_candidates(logits, seen, running, 1.5, 0.9)
    _, _, _, status = run_candidates(logits, seen, running, 1.5, 0.9)
    assert want[3] is True
    assert bool(status[1]) and (bool(status[2]) or bool(status[3]))

"""Decode-step parity of the fused HIP decoders against a pure-torch
restatement (tests/torch_reference.py: oracle-decoded fp32 weights, F.linear
in fp32, torch LayerNorm, attention and GELU; no libsvq kernel).

Both decodings start from the same prefilled cache (the product's prefill,
cloned), so each compared step differs only in how the step itself is
computed; teacher forcing feeds both the same tokens, and each writes its
own new cache slot. The fused kernels round to fp16 where the torch ops do
(LayerNorm output, every linear, GELU, residual add, attention scores and
probabilities), so the two differ only by fp32 summation order inside those
ops: a few fp16 ulps per op, compounded over the layers. The stated bound is
the largest relative logit difference, max|hip - ref| / max|ref|.

Reference: runtime_8b.py:20-110 (StarCoder2), runtime_1b.py:17-91
(GPTBigCode), runtime_shared.py:345-386 (CachedDecoding).
"""
from __future__ import annotations

import pytest
import torch

from starvector_amd.decoder import (BigCodeConfig, CachedDecoding, DecoderConfig,
                                    GPTBigCodeDecoder, Starcoder2Decoder)
from torch_reference import dense_reference, rel_err

pytestmark = pytest.mark.gpu

SMALL8 = DecoderConfig(hidden=512, heads=4, kv_heads=2, inner=1024, layers=2, vocab=320,
                       window=4096, context=512)
SMALL1 = BigCodeConfig(hidden=512, heads=4, inner=1024, layers=2, vocab=320, context=512)
# Small models: two layers.
SMALL_TOL = 4e-3


def prompt(hidden, length, device, seed=7):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn((1, length, hidden), generator=g, device=device).half()


def decode_pair(model, emb, rows, tokens, capacity):
    """(fused HIP logits, torch reference logits) [steps, rows, vocab] of the
    teacher-forced steps `tokens` after one shared prefill."""
    device = emb.device
    with torch.inference_mode():
        decoding, _ = model.prefill(emb, rows, capacity)
        kv = decoding.kv.clone()
        length = decoding.length
        hip = []
        for t in tokens:
            hip.append(decoding.step(torch.tensor(t, device=device)).float().clone())
        with dense_reference(model):
            ref_decoding = CachedDecoding(model, kv[0], kv[1], length, kv)
            assert ref_decoding.workspaces is None  # the torch path, no HIP step
            ref = []
            for t in tokens:
                ref.append(ref_decoding.step(torch.tensor(t, device=device)).float().clone())
    return torch.stack(hip), torch.stack(ref)


@pytest.mark.parametrize("qtype", ("Q4_0", "Q5_0", "Q8_0"))
def test_starcoder2_decode_matches_torch_reference(cuda_device, qtype):
    model = Starcoder2Decoder(SMALL8, qtype=qtype, seed=3, device=cuda_device)
    emb = prompt(SMALL8.hidden, 12, cuda_device)
    hip, ref = decode_pair(model, emb, 2, [(5, 6), (300, 2), (17, 17), (1, 319)], 40)
    errs = [rel_err(h, r) for h, r in zip(hip, ref)]
    print(f"starcoder2 {qtype}: per-step rel err {errs}")
    assert max(errs) <= SMALL_TOL, errs


@pytest.mark.parametrize("qtype", ("Q4_0", "Q5_0", "Q8_0"))
def test_bigcode_decode_matches_torch_reference(cuda_device, qtype):
    model = GPTBigCodeDecoder(SMALL1, qtype=qtype, embed_qtype="Q8_0", seed=4,
                              device=cuda_device)
    emb = prompt(SMALL1.hidden, 12, cuda_device)
    hip, ref = decode_pair(model, emb, 2, [(5, 6), (300, 2), (17, 17), (1, 319)], 40)
    errs = [rel_err(h, r) for h, r in zip(hip, ref)]
    print(f"bigcode {qtype}: per-step rel err {errs}")
    assert max(errs) <= SMALL_TOL, errs


@pytest.mark.parametrize("model_kind", ("starcoder2", "bigcode"))
def test_prefill_matches_torch_reference(cuda_device, model_kind):
    """The product's prefill runs its linears as HIP dequantization to fp16
    plus an fp16 GEMM (the reference's `_soa_mm` arithmetic, quantization.py:
    130-169); the restatement multiplies exact fp32 weights. The difference is
    the fp16 rounding of the weights, about 2^-11 relative each."""
    if model_kind == "starcoder2":
        model = Starcoder2Decoder(SMALL8, qtype="Q4_0", seed=3, device=cuda_device)
        hidden = SMALL8.hidden
    else:
        model = GPTBigCodeDecoder(SMALL1, qtype="Q4_0", embed_qtype="Q8_0", seed=4,
                                  device=cuda_device)
        hidden = SMALL1.hidden
    emb = prompt(hidden, 24, cuda_device)
    with torch.inference_mode():
        _, hip = model.prefill(emb, 2, 32)
        hip = hip.float().clone()
        with dense_reference(model):
            _, ref = model.prefill(emb, 2, 32)
    err = rel_err(hip, ref)
    print(f"{model_kind} prefill rel err {err}")
    assert err <= 1e-2, err


# Layer by layer at full size: a layer's output is the fp16 residual stream,
# rounded once more than its increment, so the bound is relative to the
# output's largest element: about 8 fp16 ulps (2^-11 each). The increments'
# own relative error (printed) grows with the stream's magnitude through that
# last rounding, which both paths make alike.
LAYER_TOL = 4e-3


def layerwise(model, layers, embed, decode_layer, head, tokens, cuda_device):
    """Per-layer parity of one decode step at full size: every layer gets the
    torch restatement's input (its previous layer's output), then the fused
    HIP layer and the torch layer each compute it over their own copy of the
    prefilled cache. Returns (relative errors of the layer outputs, relative
    errors of the layers' increments out - x, error of the logits)."""
    out_err, delta_err = [], []
    with torch.inference_mode(), dense_reference(model):
        x = embed(torch.tensor(tokens, device=cuda_device))[:, None]
        for layer_index, layer in enumerate(layers):
            hip, ref = decode_layer(layer_index, layer, x)
            out_err.append(rel_err(hip, ref))
            delta_err.append(rel_err(hip.float() - x.float(), ref.float() - x.float()))
            x = ref
        hip_logits, ref_logits = head(x)
    return out_err, delta_err, rel_err(hip_logits, ref_logits)


def test_starcoder2_8b_full_size_layers_match_torch_reference(cuda_device):
    """The benchmark's decoder at full size (32 layers, hidden 4608, 36 / 4
    heads, inner 18432, vocab 49152, Q4_0, beam 2) after a 1024-token
    prefill: the decode step at cache position 1024, layer by layer.

    End to end, the two paths' logits differ by several percent: with
    random weights the attention scores have a spread of about 11, so the
    softmax over 1024 slots is nearly one-hot, and a one-ulp fp16 difference
    in a score near a tie moves most of a head's weight; 32 layers compound
    that. Layer by layer, each difference is a few fp16 ulps of the layer's
    own arithmetic."""
    cfg = DecoderConfig()
    model = Starcoder2Decoder(cfg, qtype="Q4_0", seed=0, device=cuda_device)
    emb = prompt(cfg.hidden, 1024, cuda_device, seed=1)
    with torch.inference_mode():
        decoding, _ = model.prefill(emb, 2, 1032)
    span, position = decoding.span(), decoding.position
    hip_kv, ref_kv = decoding.kv, decoding.kv.clone()
    ws = decoding.workspaces
    cos, sin = model._rope(position, torch.float16)
    slots = torch.arange(span, device=cuda_device)
    bias = torch.zeros(span, device=cuda_device, dtype=torch.float16).masked_fill_(
        (slots > position) | (slots <= position - cfg.window), float("-inf"))

    def decode_layer(i, layer, x):
        cache = lambda kv: (kv[0][i][:, :, :span], kv[1][i][:, :, :span])
        hip = layer(x, cos, sin, *cache(hip_kv), position, None, ws)
        ref = layer(x, cos, sin, *cache(ref_kv), position, bias, None)
        return hip, ref

    def head(x):
        from starvector_amd.decoder import fused_linear
        return fused_linear(model.lm_head, x[:, 0], norm=model.norm), model.lm_head(model.norm(x[:, 0]))

    out_err, delta_err, logit_err = layerwise(model, model.layers, model.embed_tokens,
                                              decode_layer, head, [17, 40000], cuda_device)
    print(f"8B layer outputs: max rel err {max(out_err):.2e}; increments: max {max(delta_err):.2e}; "
          f"head {logit_err:.2e}")
    print("per layer:", [f"{e:.1e}" for e in delta_err])
    assert max(out_err) <= LAYER_TOL, out_err
    assert logit_err <= 1e-3, logit_err


def test_bigcode_1b_full_size_layers_match_torch_reference(cuda_device):
    """GPTBigCode-1B at full size (24 layers, hidden 2048, 16 heads with one
    key/value head, inner 8192, vocab 49152; Q4_0 linears, Q8_0 tables)
    after a 600-token prefill: the decode step at position 600, layer by
    layer, as the StarCoder2 test."""
    cfg = BigCodeConfig()
    model = GPTBigCodeDecoder(cfg, qtype="Q4_0", embed_qtype="Q8_0", seed=0,
                              device=cuda_device)
    emb = prompt(cfg.hidden, 600, cuda_device, seed=2)
    with torch.inference_mode():
        decoding, _ = model.prefill(emb, 2, 608)
    span, position = decoding.span(), decoding.position
    hip_kv, ref_kv = decoding.kv, decoding.kv.clone()
    ws = decoding.workspaces
    slots = torch.arange(span, device=cuda_device)
    bias = torch.zeros(span, device=cuda_device, dtype=torch.float16).masked_fill_(
        slots > position, float("-inf"))

    def embed(tokens):
        return model.wte(tokens) + model.wpe(position)

    def decode_layer(i, block, x):
        cache = lambda kv: (kv[0][i][:, :, :span], kv[1][i][:, :, :span])
        hip = block(x, *cache(hip_kv), position, None, ws)
        ref = block(x, *cache(ref_kv), position, bias, None)
        return hip, ref

    def head(x):
        from starvector_amd.decoder import fused_linear
        return fused_linear(model.lm_head, x[:, 0], norm=model.ln_f), model.lm_head(model.ln_f(x[:, 0]))

    out_err, delta_err, logit_err = layerwise(model, model.h, embed, decode_layer, head,
                                              [17, 40000], cuda_device)
    print(f"1B layer outputs: max rel err {max(out_err):.2e}; increments: max {max(delta_err):.2e}; "
          f"head {logit_err:.2e}")
    print("per layer:", [f"{e:.1e}" for e in delta_err])
    assert max(out_err) <= LAYER_TOL, out_err
    assert logit_err <= 1e-3, logit_err


def test_interleaved_decodings_keep_their_own_workspaces(cuda_device):
    """Two decodings of different row counts and capacities, stepped in
    turn: each replays graphs captured with its own attention and GEMV
    workspaces, so every replay still matches an eager decode of the same
    step (a workspace shared through a cache and replaced by the larger one
    would leave the first decoding's graphs writing freed memory)."""
    model = Starcoder2Decoder(SMALL8, qtype="Q4_0", seed=3, device=cuda_device)
    emb = prompt(SMALL8.hidden, 12, cuda_device)
    with torch.inference_mode():
        small, _ = model.prefill(emb, 2, 40)
        small_twin, _ = model.prefill(emb, 2, 40)
        large, _ = model.prefill(emb, 4, 600)
        large_twin, _ = model.prefill(emb, 4, 600)
        assert small.workspaces["attention"].data_ptr() != large.workspaces["attention"].data_ptr()
        for i, (a, b) in enumerate([(5, 6), (300, 2), (17, 17)]):
            for decoding, twin, toks in ((small, small_twin, [a, b]),
                                         (large, large_twin, [a, b, b, a])):
                t = torch.tensor(toks, device=cuda_device)
                got = decoding.step(t).float().clone()
                twin.tokens.copy_(t)
                want = twin._decode(decoding.span()).float()
                twin.position += 1
                twin.length += 1
                err = rel_err(got, want)
                assert err <= 1e-3, (i, len(toks), err)

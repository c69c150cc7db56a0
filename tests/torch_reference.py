"""A pure-torch restatement of a decoder's decode path, for parity tests.

Every quantized weight is decoded once by the oracle's torch restatement of
the SoA decode (`oracle.soa_oracle.dequant_torch`, exact fp32 weights) and
every op around it is a plain torch op: the quantized linears become
`F.linear` in fp32 on the fp16 activations (the GEMV's arithmetic: exact
weights, fp32 accumulation, one rounding to fp16), the quantized embeddings
a dense row gather, and LayerNorm, attention and GELU the reference's ops
(the decoders' `fused = False` path). No HIP kernel of libsvq runs inside
`dense_reference()`.
"""
from __future__ import annotations

from contextlib import contextmanager

import torch
import torch.nn.functional as F

from oracle import soa_oracle as orc
from starvector_amd.quantization import GGUFEmbedding, GGUFLinear


def _dense(module, cache):
    key = id(module.weight)
    if key not in cache:
        spec = module._specs["weight"]
        cache[key] = orc.dequant_torch(module.weight.detach(), module.weight_scales.detach(),
                                       spec.qtype, spec.shape)
    return cache[key]


@contextmanager
def dense_reference(model):
    """Within the block, `model` computes with dense fp32 weights and torch
    ops only: GGUFLinear and GGUFEmbedding forwards are replaced for the
    duration, and the decoder's fused HIP step is switched off."""
    cache = {}

    def linear_forward(self, x):
        w = _dense(self, cache)
        b = self.bias
        y = F.linear(x.float(), w, None if b is None else b.float())
        return y.to(x.dtype)

    def embedding_forward(self, ids):
        w = _dense(self, cache)
        return w[ids.reshape(-1)].reshape(*ids.shape, w.shape[1]).to(self.output_dtype)

    saved = (GGUFLinear.forward, GGUFEmbedding.forward)
    GGUFLinear.forward = linear_forward
    GGUFEmbedding.forward = embedding_forward
    model.fused = False
    try:
        yield model
    finally:
        GGUFLinear.forward, GGUFEmbedding.forward = saved
        del model.fused  # back to the class default
        cache.clear()


def rel_err(got, want):
    got, want = got.float(), want.float()
    return ((got - want).abs().max() / want.abs().max()).item()

"""A GGUF checkpoint through this package's reader onto the GPU: the
reference's load path (TensorStore.linear, runtime_shared.py:68-75:
`set_gguf` of weight and bias) then the HIP GEMV, against the oracle's
decode of the written bytes (fp32 product, tolerance 1e-3 x max|ref|)."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import starvector_amd.gguf_support as gs
from gguf_writer import GGML, gguf_bytes
from oracle import soa_oracle as orc
from starvector_amd.quantization import GGUFLinear

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("qtype", ("Q4_0", "Q5_0", "Q8_0"))
def test_gguf_linear_from_file(cuda_device, tmp_path, qtype):
    n, k = 1000, 4096
    raw = orc.packed_matrix(qtype, n, k, seed=9)
    bias = np.random.default_rng(1).standard_normal(n).astype(np.float16)
    path = tmp_path / "m.gguf"
    path.write_bytes(gguf_bytes([], [("l.weight", GGML[qtype], (k, n), raw.tobytes()),
                                     ("l.bias", GGML["F16"], (n,), bias.tobytes())]))
    reader = gs.GGUFReader(path, "c")
    layer = GGUFLinear(k, n)
    layer.set_gguf("weight", reader.tensors[0])
    layer.set_gguf("bias", reader.tensors[1])
    layer = layer.to(cuda_device)
    x = torch.randn((2, k), generator=torch.Generator().manual_seed(2)).half()
    y = layer(x.to(cuda_device)).float().cpu()
    w = torch.from_numpy(orc.dequantize_aos(raw, qtype, (n, k)))
    ref = F.linear(x.float(), w, torch.from_numpy(bias).float())
    err = ((y - ref).abs().max() / ref.abs().max()).item()
    assert err <= 1e-3, err

"""INTEGRATION.md's reference-side binding runs as written: its Python
blocks are executed against the built libsvq.so, and every launch wrapper
they define is called with arguments the library rejects before any HIP
call (no GPU needed). This keeps the documented binding in step with the
ABI (version, element type codes, signatures)."""
from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

import starvector_amd._native as native

ROOT = Path(__file__).resolve().parents[1]


def python_blocks():
    return re.findall(r"```python\n(.*?)```", (ROOT / "INTEGRATION.md").read_text(), re.S)


class _Stream:
    cuda_stream = None


@pytest.fixture
def binding(monkeypatch):
    monkeypatch.setenv("SVQ_LIB", str(native.LIB_PATH))
    # The launch wrappers read the current stream; with no GPU, the null stream.
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a, **k: _Stream())
    # The reference module's kernel codes (quantization.py:120).
    ns = {"_QTYPE_CODE": {"Q4_0": 4, "Q5_0": 5, "Q8_0": 8}}
    blocks = python_blocks()
    assert len(blocks) == 4
    for i, block in enumerate(blocks):
        exec(compile(block, f"INTEGRATION.md block {i}", "exec"), ns)
    return ns


def test_binding_loads_the_library_at_this_abi(binding):
    assert binding["_svq"].svq_abi_version() == native.ABI_VERSION
    assert (binding["_SVQ_F16"], binding["_SVQ_F32"], binding["_SVQ_BF16"]) == (0, 1, 2)


def test_binding_gemv_reaches_the_library(binding):
    x = torch.zeros(2, 40, dtype=torch.float16)  # K = 40: not a multiple of 32
    q = torch.zeros(8 * 16, dtype=torch.uint8)
    s = torch.zeros(8, dtype=torch.float16)
    out = torch.zeros(2, 8, dtype=torch.float16)
    with pytest.raises(RuntimeError, match=r"libsvq error -2: invalid matrix dimensions"):
        binding["_launch_soa_gemv"](x, q, s, out, "Q4_0", None)
    x = torch.zeros(9, 64, dtype=torch.float16)  # M = 9: more rows than the GEMV takes
    with pytest.raises(RuntimeError, match=r"libsvq error -2: m=9"):
        binding["_launch_soa_gemv"](x, q, s, out, "Q4_0", None)


def test_binding_dequantize_reaches_the_library(binding):
    q = torch.zeros(32, dtype=torch.uint8)
    s = torch.zeros(4, dtype=torch.uint8)  # two blocks
    out = torch.zeros(64, dtype=torch.float32)
    binding["_QTYPE_CODE"]["Q6_X"] = 6  # not a quantization the library decodes
    with pytest.raises(RuntimeError, match=r"libsvq error -1"):
        binding["_launch_dequantize_soa"](q, s, "Q6_X", (2, 32), out)
    out = torch.zeros(64, dtype=torch.float32)[1:]  # misaligned output
    with pytest.raises(RuntimeError, match=r"libsvq error -6"):
        binding["_launch_dequantize_soa"](q, s, "Q4_0", (2, 32), out)


def test_binding_attention_reorder_and_beam_reach_the_library(binding):
    qkv = torch.zeros(2, (35 + 8) * 128, dtype=torch.float16)
    keys = torch.zeros(2, 4, 16, 128, dtype=torch.float16)
    position = torch.zeros(1, dtype=torch.int64)
    ws = torch.zeros(1 << 16, dtype=torch.uint8)
    # 35 query heads over 4 key/value heads: rejected (SVQ_E_SHAPE)
    with pytest.raises(RuntimeError, match=r"libsvq error -2"):
        binding["_attend"](qkv, None, None, keys, keys, position, 4096, 35, 4, ws)

    class Decoding:
        keys = values = torch.zeros(2, 9, 4, 16, 128, dtype=torch.float16)  # 9 rows > 8
        length = 4

    with pytest.raises(RuntimeError, match=r"libsvq error -2"):
        binding["reorder"](Decoding(), torch.zeros(9, dtype=torch.int64))
    logits = torch.zeros(9, 320, dtype=torch.float16)  # 9 beams > 8
    z = torch.zeros(64)
    with pytest.raises(RuntimeError, match=r"libsvq error -2"):
        binding["_beam_step"](logits, torch.zeros(9, 320, dtype=torch.bool),
                              torch.zeros(9, 320, dtype=torch.bool), z, z, z, z, z, z,
                              torch.zeros(11, dtype=torch.int64), torch.zeros(64, dtype=torch.uint8),
                              1.5, 0.9)

"""The reference's quantized-op API on this implementation (mirrors the
reference's tests/test_quantization.py, with the CPU oracle as the reference
arithmetic). CPU tests exercise the CPU branch and the Python-side contract;
`gpu` tests exercise the HIP path behind the same API."""
from __future__ import annotations

import struct
from unittest.mock import patch

import numpy as np
import pytest
import torch

from package_alias import GGUFType as QType, fake_tensor
from oracle import soa_oracle as orc
import starvector_amd.quantization as quant
from starvector_amd.quantization import (
    GGUFConv2d, GGUFEmbedding, GGUFLinear, dequantize, dequantize_soa, graph_io,
    pack_gguf_soa, soa_gemv, tensor_payload, tied_head,
)

QTYPES = ("Q4_0", "Q5_0", "Q8_0")
KIND = {"Q4_0": QType.Q4_0, "Q5_0": QType.Q5_0, "Q8_0": QType.Q8_0}


def fake(name, qtype, shape, raw):
    return fake_tensor(name, np.frombuffer(bytes(raw), dtype=np.uint8).copy(), qtype, shape)


def packed(qtype, n, k, seed=321):
    return fake("test.weight", KIND[qtype], (n, k), orc.packed_matrix(qtype, n, k, seed))


def u8(raw):
    return torch.tensor(list(raw), dtype=torch.uint8)


# --- known answers (reference tests/test_quantization.py:21-59) ------------

def test_q8_0_decode_blocks():
    raw = struct.pack("<e", 0.5) + bytes(range(32))
    result = dequantize(u8(raw), "Q8_0", (1, 32), torch.float32)
    assert torch.equal(result[0], torch.arange(32).float() * 0.5)


def test_q4_0_unpack_nibble_halves():
    raw = struct.pack("<e", 1.0) + bytes([0xF0] * 16)
    result = dequantize(u8(raw), "Q4_0", (1, 32), torch.float32)
    assert torch.equal(result[0, :16], torch.full((16,), -8.0))
    assert torch.equal(result[0, 16:], torch.full((16,), 7.0))


def test_q5_0_fifth_bits():
    raw = struct.pack("<e", 1.0) + struct.pack("<I", 0xFFFF0000) + bytes(range(16))
    result = dequantize(u8(raw), "Q5_0", (1, 32), torch.float32)
    assert torch.equal(result[0, :16], torch.arange(16).float() - 16)
    assert torch.equal(result[0, 16:], torch.zeros(16))


def test_q8_linear():
    raw = struct.pack("<e", 0.25) + bytes([4] * 32)
    layer = GGUFLinear(32, 1)
    layer.set_gguf("weight", fake("test.weight", QType.Q8_0, (1, 32), raw))
    assert torch.allclose(layer(torch.ones((1, 32))), torch.tensor([[32.0]]))
    assert layer.weight.dtype == torch.uint8 and layer.weight_scales.dtype == torch.uint8
    assert layer.weight.numel() + layer.weight_scales.numel() == len(raw)


def test_quant_embedding_selects_only_requested_rows():
    raw = (struct.pack("<e", 1.0) + bytes([0x99] * 16)) + (struct.pack("<e", 2.0) + bytes([0x99] * 16))
    emb = GGUFEmbedding(2, 32)
    emb.set_gguf("weight", fake("tokens.weight", QType.Q4_0, (2, 32), raw))
    x = emb(torch.tensor([[1, 0, 1]]))
    assert tuple(x.shape) == (1, 3, 32)
    assert torch.equal(x[0, 0], torch.full((32,), 2.0))
    assert torch.equal(x[0, 1], torch.ones(32))


# --- seeded matrices against the oracle -------------------------------------

SHAPES = ((1, 9, 64), (2, 33, 192), (8, 17, 256), (16, 13, 64))


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_quantized_linear_matches_dequantized_reference_cpu(qtype, shape):
    m, n, k = shape
    original = packed(qtype, n, k)
    layer = GGUFLinear(k, n)
    layer.set_gguf("weight", original)
    bias = np.linspace(-0.5, 0.5, n, dtype=np.float32)
    layer.set_gguf("bias", fake_tensor("test.bias", bias.copy()))
    unpacked = orc.dequantize_aos(np.asarray(original.data), qtype, (n, k))
    assert np.array_equal(layer.unpack("weight", torch.float32, "cpu").numpy().view(np.int32),
                          unpacked.view(np.int32))
    assert layer.weight.numel() + layer.weight_scales.numel() == tensor_payload(original).numel()
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m * n))
    expected = x.double().numpy() @ unpacked.astype(np.float64).T + bias
    assert np.allclose(layer(x).numpy(), expected, rtol=2e-5, atol=2e-4)


@pytest.mark.parametrize("qtype", QTYPES)
def test_soa_payload_exact_and_dtype_stable(qtype):
    tensor = packed(qtype, 13, 128)
    q, scale_bits = pack_gguf_soa(tensor)
    reference = orc.dequantize_aos(np.asarray(tensor.data), qtype, (13, 128))
    assert q.numel() + scale_bits.numel() == tensor_payload(tensor).numel()
    got = dequantize_soa(q, scale_bits, qtype, (13, 128), torch.float32)
    assert np.array_equal(got.numpy().view(np.int32), reference.view(np.int32))
    oq, os_ = orc.pack_soa(np.asarray(tensor.data), qtype, (13, 128))
    assert np.array_equal(q.numpy(), oq) and np.array_equal(scale_bits.numpy(), os_)
    layer = GGUFLinear(128, 13)
    layer.set_gguf("weight", tensor)
    layer.to(dtype=torch.bfloat16)
    assert layer.weight.dtype == torch.uint8 and layer.weight_scales.dtype == torch.uint8
    assert torch.equal(layer.unpack("weight", torch.float32, "cpu"), torch.from_numpy(reference))


@pytest.mark.parametrize("qtype", ("Q4_0", "Q8_0"))
def test_tied_soa_embedding_and_head_share_both_parameters(qtype):
    tensor = packed(qtype, 12, 128)
    emb = GGUFEmbedding(12, 128)
    emb.set_gguf("weight", tensor)
    head = tied_head(emb)
    model = torch.nn.Module()
    model.add_module("embed", emb)
    model.add_module("head", head)
    model.to(dtype=torch.float16)
    assert head.weight is emb.weight and head.weight_scales is emb.weight_scales
    assert len(list(model.parameters())) == 2
    selected = torch.tensor([[0, 5, 5, 1, 10, 0, 8, 7, 3]])
    dense = torch.from_numpy(orc.dequantize_aos(np.asarray(tensor.data), qtype, (12, 128)))
    assert torch.equal(emb(selected), dense[selected])
    x = torch.randn(2, 128)
    assert torch.allclose(head(x), torch.nn.functional.linear(x, dense), rtol=1e-5, atol=1e-4)


def test_conv_weights_stay_floating_point():
    conv = GGUFConv2d(stride=2)
    conv.set_gguf("weight", fake_tensor("patch.weight", np.ones((2, 3, 2, 2), np.float32)))
    conv.set_gguf("bias", fake_tensor("patch.bias", np.array([1, 2], np.float32)))
    output = conv(torch.ones(1, 3, 2, 2))
    assert output.dtype == torch.float32
    assert torch.equal(output.flatten(), torch.tensor([13.0, 14.0]))


def test_short_embedding_decode_avoids_unique_sort():
    raw = (struct.pack("<e", 1.0) + bytes([0x99] * 16)) * 3
    emb = GGUFEmbedding(3, 32)
    emb.set_gguf("weight", fake("tokens.weight", QType.Q4_0, (3, 32), raw))
    with patch.object(torch, "unique", side_effect=AssertionError("unnecessary unique")):
        output = emb(torch.tensor([[2, 1, 2]]))
    assert tuple(output.shape) == (1, 3, 32)
    assert torch.equal(output, torch.ones_like(output))


def test_long_embedding_prefill_deduplicates():
    raw = (struct.pack("<e", 1.0) + bytes([0x99] * 16)) * 3
    emb = GGUFEmbedding(3, 32)
    emb.set_gguf("weight", fake("tokens.weight", QType.Q4_0, (3, 32), raw))
    out = emb(torch.tensor([[0, 1, 2, 0, 1, 2, 0, 1, 2]]))
    assert tuple(out.shape) == (1, 9, 32)
    assert torch.equal(out, torch.ones_like(out))


def test_bf16_gguf_tensor_becomes_f32_once():
    layer = GGUFLinear(4, 2)
    data = torch.tensor([[1.5, -2.0, 0.25, 3.0], [0.0, 1.0, -1.0, 2.0]], dtype=torch.bfloat16)
    bf16 = fake_tensor("w", data.view(torch.int16).numpy().view(np.uint8).reshape(2, 8),
                       type("T", (), {"name": "BF16"}), (2, 4))
    layer.set_gguf("weight", bf16)
    assert layer._specs["weight"].qtype == "F32"
    assert torch.equal(layer.weight, data.float())


# --- Python-side contract of the GPU entry points (no GPU needed) -----------

def test_soa_gemv_validates_like_the_reference():
    x = torch.zeros(2, 64, dtype=torch.float16)
    q = torch.zeros(2 * 2 * 16, dtype=torch.uint8)
    s = torch.zeros(4, dtype=torch.float16)
    out = torch.zeros(2, 2, dtype=torch.float16)
    with pytest.raises(ValueError, match="Unsupported GGUF type"):
        soa_gemv(x, q, s, out, "Q6_K")
    with pytest.raises(ValueError, match="rank-2"):
        soa_gemv(torch.zeros(9, 64, dtype=torch.float16), q, s, torch.zeros(9, 2), "Q4_0")
    with pytest.raises(ValueError, match="Invalid matrix dimensions"):
        soa_gemv(torch.zeros(2, 48, dtype=torch.float16), q, s, out, "Q4_0")
    with pytest.raises(ValueError, match="tile size"):
        soa_gemv(x, q, s, out, "Q4_0", bn=3)
    with pytest.raises(ValueError, match="num_warps"):
        soa_gemv(x, q, s, out, "Q4_0", num_warps=16)
    with pytest.raises(ValueError, match="CUDA tensors"):
        soa_gemv(x, q, s, out, "Q4_0")


def test_fused_path_declines_cpu_and_non_fp16():
    spec = quant.PackedSpec("Q4_0", (2, 64))
    q = torch.zeros(64, dtype=torch.uint8)
    s = torch.zeros(8, dtype=torch.uint8)
    assert quant._fused_soa_linear(torch.zeros(1, 64, dtype=torch.float16), q, s, spec, None) is None
    assert quant._fused_soa_linear(torch.zeros(1, 64), q, s, spec, None) is None


def test_graph_io_records_buffers_in_call_order():
    buffers = []
    with graph_io(buffers):
        assert quant._GRAPH_IO.get() == (buffers, True, [0])
    assert quant._GRAPH_IO.get() is None


# --- the same API on the GPU (HIP path) --------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("shape", SHAPES + ((5, 40, 4608), (577, 64, 256)))
def test_quantized_linear_gpu(cuda_device, qtype, shape):
    m, n, k = shape
    print(f"GGUFLinear gpu {qtype} {shape}", flush=True)
    original = packed(qtype, n, k)
    layer = GGUFLinear(k, n)
    layer.set_gguf("weight", original)
    bias = np.linspace(-0.5, 0.5, n, dtype=np.float32)
    layer.set_gguf("bias", fake_tensor("test.bias", bias.copy()))
    unpacked = orc.dequantize_aos(np.asarray(original.data), qtype, (n, k))
    gpu_layer = layer.to(cuda_device)
    assert gpu_layer.weight_scales.dtype == torch.uint8
    assert np.array_equal(gpu_layer.unpack("weight", torch.float32, cuda_device).cpu().numpy().view(np.int32),
                          unpacked.view(np.int32))
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(7))
    for dtype in (torch.float16, torch.float32):
        xg = x.to(device=cuda_device, dtype=dtype)
        ref = xg.double().cpu().numpy() @ unpacked.astype(np.float64).T + bias.astype(np.float16 if dtype == torch.float16 else np.float32)
        out = gpu_layer(xg)
        assert out.dtype == dtype
        assert orc.rel_err(out.float().cpu().numpy(), ref) <= (1e-3 if dtype == torch.float16 else 1e-5)
        if dtype == torch.float16:
            fused = quant._fused_soa_linear(xg, gpu_layer.weight, gpu_layer.weight_scales,
                                            gpu_layer._specs["weight"],
                                            gpu_layer.unpack("bias", dtype, xg.device))
            assert fused is not None, "fused path unexpectedly declined"
            assert orc.rel_err(fused.float().cpu().numpy(), ref) <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", QTYPES)
def test_graph_capture_with_static_io(cuda_device, qtype):
    print(f"graph capture {qtype}", flush=True)
    layer = GGUFLinear(256, 96)
    layer.set_gguf("weight", packed(qtype, 96, 256))
    layer = layer.to(cuda_device)
    x = torch.randn(2, 256, device=cuda_device, dtype=torch.float16)
    buffers = []
    with graph_io(buffers):
        layer(x)
    assert len(buffers) == 1
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph), graph_io(buffers):
        captured = layer(x)
    assert captured.data_ptr() == buffers[0][1].data_ptr()
    w = layer.unpack("weight", torch.float32, cuda_device)
    for step in range(4):
        x.copy_(torch.randn_like(x))
        graph.replay()
        eager = layer(x)  # eager work between replays
        torch.cuda.synchronize()
        reference = x.float() @ w.t()
        assert ((captured.float() - reference).abs().max() / reference.abs().max()).item() <= 1e-3, step
        assert torch.equal(captured, eager), step


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", QTYPES)
def test_embedding_gpu(cuda_device, qtype):
    tensor = packed(qtype, 12, 128)
    emb = GGUFEmbedding(12, 128)
    emb.set_gguf("weight", tensor)
    emb = emb.to(cuda_device)
    dense = torch.from_numpy(orc.dequantize_aos(np.asarray(tensor.data), qtype, (12, 128)))
    selected = torch.tensor([[0, 5, 5, 1, 10, 0, 8, 7, 3]], device=cuda_device)
    with patch.object(torch, "unique", side_effect=AssertionError("unnecessary unique")):
        got = emb(selected)
    assert torch.equal(got.cpu(), dense[selected.cpu()])
    emb.output_dtype = torch.float16
    assert torch.equal(emb(selected).cpu(), dense[selected.cpu()].half())


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("m", (2, 4, 8))
def test_soa_gemv_long_rows_split_k_against_oracle(cuda_device, qtype, m):
    """`soa_gemv` itself on the 8B c_proj shape (4608 x 18432), where fp16
    output splits K across workgroups through the per-stream workspace
    (svq_gemv_split: fp32 partial sums per slice, added in slice order by
    the finish kernel): the fp64 oracle at the 1e-3 bar of
    tools/tune_kernels.py:83. fp32 output runs the one-pass kernel and meets
    the 1e-5 bar of the fp32 GEMV tests."""
    n, k = 4608, 18432
    print(f"soa_gemv split-K {qtype} M={m}", flush=True)
    q, s = orc.synthetic_soa(qtype, n, k, seed=40 + m)
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, k)).astype(np.float16)
    bias = (0.02 * rng.standard_normal(n)).astype(np.float16)
    ref = orc.gemv_ref(x, q, s, qtype, n, k, bias)
    assert quant._native.gemv_workspace_bytes(m, n, k, qtype) > 0  # this shape splits
    qt = torch.from_numpy(q).to(cuda_device)
    st = torch.from_numpy(s).to(cuda_device).view(torch.float16)
    xt = torch.from_numpy(x).to(cuda_device)
    bt = torch.from_numpy(bias).to(cuda_device)
    out16 = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda_device)
    soa_gemv(xt, qt, st, out16, qtype, bias=bt)
    out32 = torch.full((m, n), float("nan"), dtype=torch.float32, device=cuda_device)
    soa_gemv(xt, qt, st, out32, qtype, bias=bt)
    torch.cuda.synchronize()
    assert orc.rel_err(out16.float().cpu().numpy(), ref) <= 1e-3
    assert orc.rel_err(out32.cpu().numpy(), ref) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("dtype", (torch.float32, torch.float16, torch.bfloat16))
def test_dequantize_aos_on_gpu_bit_exact(cuda_device, qtype, dtype):
    """`dequantize` of GGUF AoS blocks already on the GPU (split to SoA, then
    the HIP decode; quantization.py:50-65) equals the oracle's exact fp32
    product, rounded once to `dtype`."""
    n, k = 257, 96
    raw = orc.packed_matrix(qtype, n, k, seed=11)
    want = torch.from_numpy(orc.dequantize_aos(raw, qtype, (n, k))).to(dtype)
    got = dequantize(torch.from_numpy(raw).to(cuda_device), qtype, (n, k), dtype)
    assert got.device.type == "cuda" and got.dtype == dtype and got.shape == (n, k)
    assert torch.equal(got.cpu().view(torch.int16 if dtype != torch.float32 else torch.int32),
                       want.view(torch.int16 if dtype != torch.float32 else torch.int32))
    with pytest.raises(ValueError):
        dequantize(torch.from_numpy(raw[:-1]).to(cuda_device), qtype, (n, k), dtype)


@pytest.mark.gpu
def test_no_fallback_by_default_and_reference_switch(cuda_device, monkeypatch):
    """Without STARVECTOR_DISABLE_TRITON the GPU fp16 path is the fused HIP
    GEMV and never the tiled dequantize + F.linear fallback; with the
    reference's switch set to "1" it is the fallback (quantization.py:286-291,
    390-407), with the same result to the GEMV's bar."""
    m, n, k = 2, 96, 256
    layer = GGUFLinear(k, n)
    layer.set_gguf("weight", packed("Q5_0", n, k))
    layer = layer.to(cuda_device)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(3)).half().to(cuda_device)
    monkeypatch.delenv("STARVECTOR_DISABLE_TRITON", raising=False)
    real_dequant = quant.dequantize_soa

    def no_dequant(*args, **kwargs):
        raise AssertionError("the tiled fallback ran")

    monkeypatch.setattr(quant, "dequantize_soa", no_dequant)
    fused = layer(x)
    monkeypatch.setattr(quant, "dequantize_soa", real_dequant)
    monkeypatch.setenv("STARVECTOR_DISABLE_TRITON", "1")

    def no_gemv(*args, **kwargs):
        raise AssertionError("the fused GEMV ran")

    monkeypatch.setattr(quant._native, "gemv", no_gemv)
    tiled = layer(x)
    w = orc.dequantize_aos(np.asarray(packed("Q5_0", n, k).data), "Q5_0", (n, k))
    ref = x.double().cpu().numpy() @ w.astype(np.float64).T
    assert orc.rel_err(fused.float().cpu().numpy(), ref) <= 1e-3
    assert orc.rel_err(tiled.float().cpu().numpy(), ref) <= 1e-3

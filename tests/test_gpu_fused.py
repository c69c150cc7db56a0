"""svq_gemv_fused: the GEMV with the decoder-layer ops around it (LayerNorm
before, GELU and the residual add after), against the same ops done by torch
on the GPU in fp16, as the reference's decode step runs them
(runtime_8b.py:37, 53-54; runtime_1b.py:33, 46-47).

* Residual only: bit-exact with svq_gemv followed by the fp16 add.
* GELU: within one fp16 ulp of svq_gemv followed by F.gelu(approximate='tanh')
  (the tanh and the order of the fp32 operations may differ by an fp32 ulp).
* LayerNorm: the fused statistics are fp32 two-pass sums in a different order
  from torch's Welford pass, so normalized values may differ by an fp16 ulp;
  the result is compared with F.layer_norm + svq_gemv within 2e-3 x max|y|.
* Every combination against the fp32 dequantize + matmul reference within
  3e-3 x max|y|.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import starvector_amd._native as native
from oracle import soa_oracle as orc

pytestmark = pytest.mark.gpu


def ulp16(v):
    """fp16 ulp of each element of v (fp32 tensor)."""
    a = v.abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def make(m, n, k, qtype, device, seed=0, x_shift=0.0):
    """Seeded SoA weights (scales U[1e-3, 2e-2]), activations, bias, LayerNorm
    parameters and residual on the GPU, plus the oracle's fp32 weights."""
    g = torch.Generator(device=device).manual_seed(seed)
    blocks = n * k // 32
    d = (torch.rand(blocks, generator=g, device=device) * (2e-2 - 1e-3) + 1e-3).half()
    if qtype == "Q8_0":
        q = torch.randint(-127, 128, (blocks * 32,), generator=g, device=device,
                          dtype=torch.int8).view(torch.uint8)
    else:
        q = torch.randint(0, 256, (blocks * orc.PAYLOAD_BYTES[qtype],), generator=g,
                          device=device, dtype=torch.uint8)
    s = d.view(torch.uint8)
    rand = lambda *shape: torch.randn(shape, generator=g, device=device)
    return dict(x=(rand(m, k) + x_shift).half(), q=q, s=s, bias=(rand(n) * 0.5).half(),
                w_ln=(1 + 0.2 * rand(k)).half(), b_ln=(0.1 * rand(k)).half(),
                res=rand(m, n).half(), w=orc.dequant_torch(q, s, qtype, (n, k)))


def plain(c, x, qtype):
    y = torch.empty((x.shape[0], c["w"].shape[0]), dtype=torch.float16, device=x.device)
    native.gemv(x.contiguous(), c["q"], c["s"], y, qtype, c["bias"])
    return y


def fused(c, qtype, ln=False, ln_bias=True, res=False, gelu=False, eps=1e-5, y=None):
    n = c["w"].shape[0]
    y = torch.empty((c["x"].shape[0], n), dtype=torch.float16, device=c["x"].device) if y is None else y
    native.gemv_fused(c["x"], c["q"], c["s"], y, qtype, bias=c["bias"],
                      ln_weight=c["w_ln"] if ln else None,
                      ln_bias=c["b_ln"] if ln and ln_bias else None, ln_eps=eps,
                      residual=c["res"] if res else None,
                      activation="gelu_tanh" if gelu else None)
    return y


def torch_ref(c, ln=False, ln_bias=True, res=False, gelu=False, eps=1e-5):
    """fp32 product of fp16 ops: LayerNorm (fp16 out), W.x + b (rounded), GELU, +res."""
    x = c["x"]
    if ln:
        x = F.layer_norm(x, (x.shape[1],), c["w_ln"], c["b_ln"] if ln_bias else None, eps)
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        t = F.linear(x.float(), c["w"], c["bias"].float()).half()
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    if gelu:
        t = F.gelu(t, approximate="tanh")
    if res:
        t = c["res"] + t
    return t


SHAPES = [
    (2, 5632, 4608, "Q4_0"),   # 8B fused q/k/v at beam 2
    (2, 5632, 4608, "Q5_0"),   # Q5_0 q/k/v: one row tile per tile slot, short prologue
    (2, 4608, 18432, "Q5_0"),  # 8B c_proj: K = 18432 staged in LDS
    (1, 1000, 4608, "Q8_0"),
    (4, 300, 2048, "Q5_0"),
    (8, 257, 1024, "Q4_0"),    # M = 8: the LayerNorm runs in the vector kernel
    (3, 64, 32, "Q4_0"),       # one block per row
]


@pytest.mark.parametrize("m,n,k,qtype", SHAPES)
def test_residual_is_exact_and_gelu_within_one_ulp(cuda_device, m, n, k, qtype):
    c = make(m, n, k, qtype, cuda_device)
    base = plain(c, c["x"], qtype)
    assert torch.equal(fused(c, qtype, res=True), c["res"] + base)
    want = F.gelu(base, approximate="tanh").float()
    got = fused(c, qtype, gelu=True).float()
    assert ((got - want).abs() <= ulp16(want)).all()
    want = (c["res"] + F.gelu(base, approximate="tanh")).float()
    got = fused(c, qtype, gelu=True, res=True).float()
    assert ((got - want).abs() <= 2 * ulp16(want)).all()


@pytest.mark.parametrize("m,n,k,qtype", SHAPES)
@pytest.mark.parametrize("ln_bias", (True, False))
def test_layer_norm_matches_torch(cuda_device, m, n, k, qtype, ln_bias):
    c = make(m, n, k, qtype, cuda_device, seed=1)
    got = fused(c, qtype, ln=True, ln_bias=ln_bias).float()
    h = F.layer_norm(c["x"], (k,), c["w_ln"], c["b_ln"] if ln_bias else None, 1e-5)
    want = plain(c, h, qtype).float()
    assert (got - want).abs().max().item() <= 2e-3 * want.abs().max().item()


def test_layer_norm_with_large_mean(cuda_device):
    """Rows with mean 50 and unit spread: the two-pass variance keeps the
    normalized values accurate."""
    c = make(2, 512, 4608, "Q4_0", cuda_device, seed=2, x_shift=50.0)
    got = fused(c, "Q4_0", ln=True).float()
    want = torch_ref(c, ln=True).float()
    assert (got - want).abs().max().item() <= 3e-3 * want.abs().max().item()


@pytest.mark.parametrize("path", ("auto", "mfma4", "stream", "mfma", "chunked"))
@pytest.mark.parametrize("m,n,k,qtype", [(2, 5632, 4608, "Q4_0"), (4, 300, 2048, "Q5_0"),
                                         (1, 1000, 4608, "Q8_0"), (6, 96, 512, "Q8_0")])
def test_every_fusion_on_every_kernel(cuda_device, monkeypatch, path, m, n, k, qtype):
    if path != "auto":
        monkeypatch.setenv("SVQ_PATH", path)
    c = make(m, n, k, qtype, cuda_device, seed=3)
    for kw in (dict(ln=True, gelu=True), dict(res=True), dict(ln=True, res=True, gelu=True),
               dict(gelu=True)):
        got = fused(c, qtype, **kw).float()
        want = torch_ref(c, **kw).float()
        err = (got - want).abs().max().item()
        assert err <= 3e-3 * want.abs().max().item(), (kw, err)


def test_residual_in_place(cuda_device):
    c = make(2, 4608, 4608, "Q5_0", cuda_device, seed=4)
    want = c["res"] + plain(c, c["x"], "Q5_0")
    y = c["res"].clone()
    c["res"] = y
    fused(c, "Q5_0", res=True, y=y)
    assert torch.equal(y, want)


def test_decoder_layer_sequence(cuda_device):
    """One StarCoder2-8B-style MLP half at beam 2: LayerNorm + c_fc + GELU,
    then c_proj + residual, against the torch ops."""
    fc = make(2, 18432, 4608, "Q4_0", cuda_device, seed=6)
    proj = make(2, 4608, 18432, "Q4_0", cuda_device, seed=7)
    h = fused(fc, "Q4_0", ln=True, gelu=True)
    proj["x"] = h
    proj["res"] = fc["x"]
    got = fused(proj, "Q4_0", res=True).float()
    want_h = torch_ref(fc, ln=True, gelu=True)
    proj_ref = dict(proj, x=want_h)
    want = torch_ref(proj_ref, res=True).float()
    assert (got - want).abs().max().item() <= 3e-3 * want.abs().max().item()


SPLIT_SHAPES = [
    (2, 4608, 18432, "Q5_0"),  # 8B c_proj at beam 2: four slices of 4608
    (2, 4608, 18432, "Q4_0"),
    (2, 4608, 18432, "Q8_0"),
    (4, 130, 18432, "Q4_0"),   # ragged rows
    (3, 77, 9216, "Q8_0"),     # two slices
    (2, 300, 12288, "Q5_0"),   # three slices
    (4, 64, 18432, "Q5_0"),
    (8, 4608, 18432, "Q5_0"),  # 8B c_proj at beam 8: x rows 4..7 in the second A half
    (8, 4608, 18432, "Q4_0"),
    (5, 130, 18432, "Q8_0"),
    (7, 77, 9216, "Q4_0"),
    (6, 300, 12288, "Q8_0"),
]


def split(c, qtype, ws, res=False, gelu=False):
    y = torch.empty((c["x"].shape[0], c["w"].shape[0]), dtype=torch.float16, device=c["x"].device)
    native.gemv_fused(c["x"], c["q"], c["s"], y, qtype, bias=c["bias"],
                      residual=c["res"] if res else None,
                      activation="gelu_tanh" if gelu else None, workspace=ws)
    return y


@pytest.mark.parametrize("m,n,k,qtype", SPLIT_SHAPES)
def test_split_k_matches_torch_and_one_pass(cuda_device, m, n, k, qtype):
    """svq_gemv_split (K slices across workgroups, then the finish kernel)
    against the fp32 torch reference and the one-pass kernels, with every
    epilogue; the slices only reorder fp32 sums."""
    c = make(m, n, k, qtype, cuda_device, seed=8)
    ws = native.split_workspace(cuda_device, m, n, k, qtype)
    # cached per stream and only grown: at least this shape's size
    assert ws is not None and ws.numel() >= native.load().svq_gemv_split_workspace(
        m, n, k, native.QTYPE_CODE[qtype])
    for kw in (dict(), dict(res=True), dict(gelu=True), dict(res=True, gelu=True)):
        got = split(c, qtype, ws, **kw).float()
        want = torch_ref(c, **kw).float()
        assert (got - want).abs().max().item() <= 3e-3 * want.abs().max().item(), kw
        one = fused(c, qtype, **kw).float()
        assert (got - one).abs().max().item() <= 1e-3 * one.abs().max().item(), kw
    # svq_gemv with a workspace takes the same path
    y = torch.empty((m, n), dtype=torch.float16, device=cuda_device)
    native.gemv(c["x"], c["q"], c["s"], y, qtype, c["bias"], ws)
    assert torch.equal(y, split(c, qtype, ws))


def test_split_k_residual_in_place_and_graph_replays(cuda_device):
    """In-place residual (y is the residual) and graph replays of the split
    launches on the stream that allocated the workspace: every replay equals
    the eager result."""
    m, n, k, qtype = 2, 4608, 18432, "Q4_0"
    c = make(m, n, k, qtype, cuda_device, seed=9)
    stream = torch.cuda.Stream(cuda_device)
    with torch.cuda.stream(stream):
        ws = native.split_workspace(cuda_device, m, n, k, qtype)
        y = c["res"].clone()
        native.gemv_fused(c["x"], c["q"], c["s"], y, qtype, bias=c["bias"], residual=y,
                          workspace=ws)
        stream.synchronize()
        eager = y.clone()
        assert torch.equal(eager, (c["res"] + split(c, qtype, ws)))
        out = torch.empty((m, n), dtype=torch.float16, device=cuda_device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out.copy_(c["res"])
            native.gemv_fused(c["x"], c["q"], c["s"], out, qtype, bias=c["bias"], residual=out,
                              workspace=native.split_workspace(cuda_device, m, n, k, qtype))
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)

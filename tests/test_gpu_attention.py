"""Decode attention kernel (svq_decode_attention) against the reference's
decode-branch ops (runtime_8b.py:38-55, runtime_1b.py:30-45) restated in torch.

* The rotation and the cache write are compared bit for bit: the reference's
  fp16 elementwise ops (`_rotate`, `index_copy_`) run on the CPU, where torch
  forms each fp16 product and sum in fp32 and rounds once, as the kernel does.
* The attention output is compared with an fp32 restatement: scores
  alpha * q.k + bias rounded to fp16 (the reference's fp16 baddbmm output),
  fp32 softmax, fp32 weighted sum of V. Tolerance: 2e-3 x max|reference|
  (fp32 summation order, the exponential, and the final fp16 rounding).
* Against the reference's own rounding of the probabilities to fp16 before
  its bmm, the tolerance is 4e-3 x max|reference|.
"""
from __future__ import annotations

import pytest
import torch

import starvector_amd._native as native

pytestmark = pytest.mark.gpu

HD = 128


def rotate(x, cos, sin):
    first, second = x.chunk(2, dim=-1)
    return x * cos + torch.cat((-second, first), dim=-1) * sin


def rope_tables(position, theta=1e6):
    inv_freq = 1.0 / (theta ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))
    angles = torch.tensor([float(position)])[:, None] * inv_freq
    angles = torch.cat((angles, angles), -1)
    return angles.cos().half()[0], angles.sin().half()[0]


def make_case(rows, heads, kvh, capacity, span, position, rope=True, window=None,
              bias_kind="causal", seed=0, spread=1.0):
    g = torch.Generator().manual_seed(seed)
    width = (heads + 2 * kvh) * HD
    qkv = (torch.randn(rows, width, generator=g) * spread).half()
    keys = torch.randn(rows, kvh, capacity, HD, generator=g).half()
    values = torch.randn(rows, kvh, capacity, HD, generator=g).half()
    cos, sin = rope_tables(position) if rope else (None, None)
    slots = torch.arange(span)
    if bias_kind is None:
        bias = None
    elif bias_kind == "zeros":
        bias = torch.zeros(span).half()
    else:
        hidden = slots > position
        if window is not None:
            hidden |= slots <= position - window
        bias = torch.zeros(span).half().masked_fill_(hidden, float("-inf"))
    return dict(qkv=qkv, keys=keys, values=values, cos=cos, sin=sin, bias=bias, span=span,
                position=position, rows=rows, heads=heads, kvh=kvh)


def reference(case, round_probs=False):
    """(keys, values after the write, attention output fp32 [rows, heads*HD])."""
    rows, heads, kvh, span = case["rows"], case["heads"], case["kvh"], case["span"]
    hidden = heads * HD
    qkv = case["qkv"]
    q, k, v = qkv[:, :hidden], qkv[:, hidden:hidden + kvh * HD], qkv[:, hidden + kvh * HD:]
    q = q.view(rows, heads, HD)
    k = k.view(rows, kvh, HD)
    v = v.view(rows, kvh, HD)
    if case["cos"] is not None:
        q = rotate(q, case["cos"], case["sin"])
        k = rotate(k, case["cos"], case["sin"])
    keys, values = case["keys"].clone(), case["values"].clone()
    pos = case["position"]
    if 0 <= pos < span:
        keys[:, :, pos] = k
        values[:, :, pos] = v
    group = heads // kvh
    kf = keys[:, :, :span].float()
    vf = values[:, :, :span].float()
    qf = q.float().view(rows, kvh, group, HD)
    scores = torch.einsum("rkgd,rksd->rkgs", qf, kf) * (HD ** -0.5)
    if case["bias"] is not None:
        scores = scores + case["bias"].float()
    scores = scores.half().float()
    probs = torch.softmax(scores, -1)
    if round_probs:
        probs = probs.half().float()
    out = torch.einsum("rkgs,rksd->rkgd", probs, vf).reshape(rows, heads * HD)
    return keys, values, out


def run_kernel(case, device, out=None, workspace=None, window=0):
    dev = lambda t: None if t is None else t.to(device)
    keys, values = dev(case["keys"]), dev(case["values"])
    span = case["span"]
    rows, heads, kvh = case["rows"], case["heads"], case["kvh"]
    out = torch.full((rows, heads * HD), float("nan"), dtype=torch.float16, device=device)
    position = torch.tensor([case["position"]], dtype=torch.int64, device=device)
    ws = workspace if workspace is not None else native.attention_workspace(
        device, rows, heads, kvh, span)
    native.decode_attention(dev(case["qkv"]), dev(case["cos"]), dev(case["sin"]),
                            keys[:, :, :span], values[:, :, :span], position, dev(case["bias"]),
                            out, heads, kvh, HD ** -0.5, ws, window=window)
    torch.cuda.synchronize()
    return keys.cpu(), values.cpu(), out.float().cpu()


def check(case, device):
    keys, values, out = run_kernel(case, device)
    rkeys, rvalues, ref = reference(case)
    assert torch.equal(keys, rkeys), "key cache differs"
    assert torch.equal(values, rvalues), "value cache differs"
    assert torch.isfinite(out).all()
    scale = ref.abs().max().item()
    err = (out - ref).abs().max().item()
    assert err <= 2e-3 * scale, (err, scale)
    _, _, ref16 = reference(case, round_probs=True)
    err16 = (out - ref16).abs().max().item()
    assert err16 <= 4e-3 * scale, (err16, scale)


# (rows, heads, kv_heads, capacity, span, position, rope, window, bias)
CASES = [
    (2, 36, 4, 1600, 1537, 1100, True, 4096, "causal"),   # StarCoder2-8B, beam 2
    (2, 36, 4, 1600, 1537, 1536, True, 4096, "causal"),   # last slot of the span
    (2, 36, 4, 2048, 2048, 1500, True, 1000, "causal"),   # sliding window cuts the front
    (1, 36, 4, 64, 64, 0, True, 4096, "causal"),          # first slot: one key attended
    (4, 36, 4, 200, 130, 63, True, 4096, "causal"),       # chunk edge, beam 4
    (3, 36, 4, 200, 130, 64, True, 4096, "causal"),       # next chunk's first slot
    (2, 16, 1, 600, 512, 300, False, None, "causal"),     # GPTBigCode-1B multi-query
    (2, 8, 8, 100, 77, 76, True, None, None),             # one query head per kv head, no bias
    (2, 8, 2, 100, 33, 10, True, None, None),             # no bias: slots past position attended
    (2, 8, 2, 300, 290, 100, True, None, "zeros"),        # zero bias: slots past position attended
    (2, 36, 4, 600, 512, 450, True, 100, "causal"),       # window: masked slots before position
]


@pytest.mark.parametrize("rows,heads,kvh,cap,span,pos,rope,window,bias",
                         [c for c in CASES if c[-1] == "causal"])
def test_decode_attention_window_mask_equals_bias(cuda_device, rows, heads, kvh, cap, span, pos,
                                                   rope, window, bias):
    """The kernel's own causal sliding-window mask (bias NULL, window w; the
    decode step's form) gives what the explicit -inf bias gives, bit for bit."""
    case = make_case(rows, heads, kvh, cap, span, pos, rope, window, bias)
    w = window if window is not None else 1 << 20
    keys, values, out = run_kernel(case, cuda_device)
    masked = dict(case, bias=None)
    mkeys, mvalues, mout = run_kernel(masked, cuda_device, window=w)
    assert torch.equal(keys, mkeys) and torch.equal(values, mvalues)
    assert torch.equal(out, mout)


@pytest.mark.parametrize("rows,heads,kvh,cap,span,pos,rope,window,bias", CASES)
def test_decode_attention_matches_reference(cuda_device, rows, heads, kvh, cap, span, pos, rope,
                                            window, bias):
    check(make_case(rows, heads, kvh, cap, span, pos, rope, window, bias), cuda_device)


def test_decode_attention_peaked_scores(cuda_device):
    """Large activations: near one-hot softmax, scores far from zero."""
    check(make_case(2, 36, 4, 300, 257, 200, spread=4.0, seed=5), cuda_device)


def test_decode_attention_every_group_size(cuda_device):
    for group in range(1, 17):
        check(make_case(2, 2 * group, 2, 150, 129, 100, seed=group), cuda_device)


def test_decode_attention_consecutive_calls_share_workspace(cuda_device):
    """Back-to-back calls on one workspace, the second with a shorter span and
    a new position, each see only their own partial results."""
    ws = native.attention_workspace(cuda_device, 2, 36, 4, 1537)
    for span, pos, seed in ((1537, 1000, 1), (700, 699, 2), (1537, 1536, 3)):
        case = make_case(2, 36, 4, 1600, span, pos, seed=seed)
        keys, values, out = run_kernel(case, cuda_device, workspace=ws)
        rkeys, _, ref = reference(case)
        assert torch.equal(keys, rkeys)
        assert (out - ref).abs().max().item() <= 2e-3 * ref.abs().max().item()


def test_decode_attention_shapes_share_workspace(cuda_device):
    """Calls of different shapes (rows, heads, kv heads, span) on one
    workspace, each seeing only its own partial results."""
    ws = native.attention_workspace(cuda_device, 4, 36, 4, 1537)
    for rows, heads, kvh, cap, span, pos, seed in ((4, 36, 4, 1600, 1537, 900, 11),
                                                   (1, 16, 1, 300, 64, 63, 12),
                                                   (2, 32, 2, 700, 700, 650, 13),
                                                   (3, 36, 4, 200, 129, 128, 14)):
        print(f"attention shapes share workspace rows={rows} heads={heads} kvh={kvh} span={span}",
              flush=True)
        case = make_case(rows, heads, kvh, cap, span, pos, seed=seed)
        keys, values, out = run_kernel(case, cuda_device, workspace=ws)
        _, _, ref = reference(case)
        assert torch.isfinite(out).all()
        assert (out - ref).abs().max().item() <= 2e-3 * ref.abs().max().item()


def test_decode_attention_graph_replays(cuda_device):
    """Captured once, replayed with the position advanced between replays
    (eager work and synchronization in between): each replay writes the new
    slot and matches the reference for its position."""
    rows, heads, kvh, cap, span = 2, 36, 4, 600, 512
    base = make_case(rows, heads, kvh, cap, span, 400, seed=9)
    keys = base["keys"].to(cuda_device)
    values = base["values"].to(cuda_device)
    qkv = base["qkv"].to(cuda_device)
    cos = torch.empty(HD, dtype=torch.float16, device=cuda_device)
    sin = torch.empty_like(cos)
    bias = torch.empty(span, dtype=torch.float16, device=cuda_device)
    position = torch.tensor([400], dtype=torch.int64, device=cuda_device)
    out = torch.empty((rows, heads * HD), dtype=torch.float16, device=cuda_device)
    ws = native.attention_workspace(cuda_device, rows, heads, kvh, span)

    def set_position(p):
        c, s = rope_tables(p)
        cos.copy_(c)
        sin.copy_(s)
        bias.copy_(torch.zeros(span).half().masked_fill_(torch.arange(span) > p, float("-inf")))
        position.fill_(p)

    def call():
        native.decode_attention(qkv, cos, sin, keys[:, :, :span], values[:, :, :span], position,
                                bias, out, heads, kvh, HD ** -0.5, ws)

    set_position(400)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        call()  # warm-up
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    host_keys, host_values = keys.cpu(), values.cpu()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for p in (401, 402, 450):
        set_position(p)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        case = dict(base, keys=host_keys, values=host_values, position=p)
        case["cos"], case["sin"] = rope_tables(p)
        case["bias"] = bias.cpu()
        rkeys, rvalues, ref = reference(case)
        assert torch.equal(keys.cpu(), rkeys)
        got = out.float().cpu()
        assert (got - ref).abs().max().item() <= 2e-3 * ref.abs().max().item(), p
        host_keys, host_values = rkeys, rvalues


@pytest.mark.parametrize("rows,parents", [(2, (0, 1)), (2, (0, 0)), (2, (1, 1)), (2, (1, 0)),
                                          (4, (2, 2, 0, 1)), (8, (7, 0, 1, 2, 3, 4, 5, 6)),
                                          (3, (5, -1, 0))])
def test_cache_reorder_matches_indexing(cuda_device, rows, parents):
    """svq_cache_reorder against the reference's index copy (rows whose parent
    differs take the parent's first `length` slots; rows may exchange
    caches); parents outside [0, rows) leave their row unchanged."""
    planes, heads, capacity, length = 3, 2, 40, 29
    g = torch.Generator().manual_seed(rows)
    cache = torch.randn(planes, rows, heads, capacity, HD, generator=g).half()
    fixed = [p if 0 <= p < rows else r for r, p in enumerate(parents)]
    want = cache.clone()
    moved = [r for r, p in enumerate(fixed) if p != r]
    if moved:
        want[:, moved, :, :length] = cache[:, [fixed[r] for r in moved], :, :length]
    got = cache.to(cuda_device)
    native.cache_reorder(got, torch.tensor(parents, dtype=torch.int64, device=cuda_device), length)
    assert torch.equal(got.cpu(), want)

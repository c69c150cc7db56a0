"""GPU parity of the HIP kernels, called through the C ABI (libsvq.so).

Bars: dequantization bit-exact with the oracle and the golden fixtures (fp32
bits; fp16/bf16 as round-to-nearest-even of the exact fp32 value). GEMV:
max|y - ref| / max|ref| <= 1e-3 for fp16 outputs (the BASELINE bar; the
reference's own GPU test allows 0.06) and <= 1e-5 for fp32 outputs, where ref
is the float64 oracle (small shapes) or a plain torch fp32 dequant + matmul
with TF32 disabled (full decoder shapes).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import starvector_amd._native as native
from oracle import soa_oracle as orc

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
QTYPES = ("Q4_0", "Q5_0", "Q8_0")
FP16_TOL = 1e-3
FP32_TOL = 1e-5


def say(msg):
    print(msg, flush=True)


def golden_cases(qtype):
    data = np.load(GOLDEN / f"{qtype.lower()}.npz")
    names = sorted({key.split("/")[0] for key in data.files})
    return [(name, {key.split("/")[1]: data[key] for key in data.files if key.startswith(name + "/")})
            for name in names]


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def hip_gemv(x, q, s, qtype, n, bias=None, out_dtype=torch.float16):
    y = torch.empty((x.shape[0], n), dtype=out_dtype, device=x.device)
    native.gemv(x, q, s, y, qtype, bias)
    return y


def assert_bits(got: np.ndarray, want: np.ndarray, label: str) -> None:
    """Bit equality; on failure report the first mismatches compactly."""
    got = np.ascontiguousarray(got).reshape(-1)
    want = np.ascontiguousarray(want).reshape(-1)
    assert got.shape == want.shape, (label, got.shape, want.shape)
    bad = np.nonzero(got != want)[0]
    if bad.size:
        head = ", ".join(f"[{i}] got {int(got[i]):#x} want {int(want[i]):#x}" for i in bad[:8])
        raise AssertionError(f"{label}: {bad.size} of {got.size} differ: {head}")


def bf16_rne_bits(f32: np.ndarray) -> np.ndarray:
    b = f32.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f32)
    r[nan] = 0x7FC0
    return r


def test_native_library_is_the_loaded_code(cuda_device):
    native.load()
    maps = Path("/proc/self/maps").read_text()
    assert str(native.LIB_PATH) in maps


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_golden_bit_exact(cuda_device, qtype):
    for name, fx in golden_cases(qtype):
        say(f"dequant golden {qtype} {name}")
        n, k, _ = (int(v) for v in fx["shape"])
        q, s = to_dev(fx["q"], cuda_device), to_dev(fx["s"], cuda_device)
        want = fx["dequant_bits"].reshape(-1)
        out32 = torch.empty(n * k, dtype=torch.float32, device=cuda_device)
        native.dequant(q, s, out32, qtype)
        assert_bits(out32.cpu().numpy().view(np.uint32), want.view(np.uint32), f"{name} fp32")
        f32 = want.view(np.float32)
        out16 = torch.empty(n * k, dtype=torch.float16, device=cuda_device)
        native.dequant(q, s, out16, qtype)
        with np.errstate(over="ignore"):
            want16 = f32.astype(np.float16).view(np.uint16)
        assert_bits(out16.cpu().numpy().view(np.uint16), want16, f"{name} fp16")
        outb = torch.empty(n * k, dtype=torch.bfloat16, device=cuda_device)
        native.dequant(q, s, outb, qtype)
        assert_bits(outb.view(torch.int16).cpu().numpy().view(np.uint16), bf16_rne_bits(f32), f"{name} bf16")


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_seeded_matrix_bit_exact(cuda_device, qtype):
    n, k = 1031, 4608
    say(f"dequant seeded {qtype} {n}x{k}")
    q, s = orc.synthetic_soa(qtype, n, k, seed=21)
    want = orc.dequantize_soa(q, s, qtype, (n, k)).reshape(-1)
    out = torch.empty(n * k, dtype=torch.float32, device=cuda_device)
    native.dequant(to_dev(q, cuda_device), to_dev(s, cuda_device), out, qtype)
    assert_bits(out.cpu().numpy().view(np.uint32), want.view(np.uint32), f"{qtype} seeded")


@pytest.mark.parametrize("qtype", QTYPES)
def test_dequant_rows_gather(cuda_device, qtype):
    n, k = 50, 256
    q, s = orc.synthetic_soa(qtype, n, k, seed=8)
    dense = orc.dequantize_soa(q, s, qtype, (n, k))
    ids = np.array([3, 0, 49, 3, 3, 17, 2, 48, 0, 1, 5], dtype=np.int64)
    say(f"dequant rows {qtype}")
    qd, sd = to_dev(q, cuda_device), to_dev(s, cuda_device)
    out = torch.empty((ids.size, k), dtype=torch.float32, device=cuda_device)
    native.dequant_rows(qd, sd, to_dev(ids, cuda_device), n, k, out, qtype)
    assert np.array_equal(out.cpu().numpy().view(np.int32), dense[ids].view(np.int32))
    bad = np.array([1, -1, 50, 2], dtype=np.int64)
    out = torch.empty((bad.size, k), dtype=torch.float16, device=cuda_device)
    native.dequant_rows(qd, sd, to_dev(bad, cuda_device), n, k, out, qtype)
    got = out.float().cpu().numpy()
    assert np.isnan(got[1]).all() and np.isnan(got[2]).all()
    assert np.array_equal(got[0], dense[1].astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("qtype", QTYPES)
def test_gemv_golden(cuda_device, qtype):
    for name, fx in golden_cases(qtype):
        n, k, m = (int(v) for v in fx["shape"])
        say(f"gemv golden {qtype} {name} m={m} n={n} k={k}")
        q, s = to_dev(fx["q"], cuda_device), to_dev(fx["s"], cuda_device)
        x, b = to_dev(fx["x"], cuda_device), to_dev(fx["bias"], cuda_device)
        y32 = hip_gemv(x, q, s, qtype, n, b, torch.float32)
        assert orc.rel_err(y32.cpu().numpy(), fx["y_exact"]) <= FP32_TOL, name
        if name.startswith("edge"):
            continue  # the largest-scale block overflows fp16 outputs
        y16 = hip_gemv(x, q, s, qtype, n, b, torch.float16)
        assert orc.rel_err(y16.float().cpu().numpy(), fx["y_exact"]) <= FP16_TOL, name


SMALL_SHAPES = [(1, 32), (3, 64), (13, 128), (33, 192), (17, 256), (96, 256), (7, 1024),
                (129, 2048), (65, 4608), (40, 18432)]


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("m", range(1, 9))
def test_gemv_small_shapes_against_oracle(cuda_device, qtype, m):
    rng = np.random.default_rng(100 + m)
    for n, k in SMALL_SHAPES:
        say(f"gemv small {qtype} m={m} n={n} k={k}")
        q, s = orc.synthetic_soa(qtype, n, k, seed=n * 7 + k + m)
        x = rng.standard_normal((m, k)).astype(np.float16)
        bias = rng.standard_normal(n).astype(np.float16) if n % 2 else None
        ref = orc.gemv_ref(x, q, s, qtype, n, k, bias)
        qd, sd, xd = to_dev(q, cuda_device), to_dev(s, cuda_device), to_dev(x, cuda_device)
        bd = None if bias is None else to_dev(bias, cuda_device)
        y32 = hip_gemv(xd, qd, sd, qtype, n, bd, torch.float32)
        assert orc.rel_err(y32.cpu().numpy(), ref) <= FP32_TOL, (n, k)
        y16 = hip_gemv(xd, qd, sd, qtype, n, bd, torch.float16)
        assert orc.rel_err(y16.float().cpu().numpy(), ref) <= FP16_TOL, (n, k)


def gpu_soa(qtype, n, k, seed, dev):
    """Benchmark-distribution SoA arrays generated on the GPU."""
    g = torch.Generator(device=dev).manual_seed(seed)
    blocks = n * k // 32
    d = (torch.rand(blocks, generator=g, device=dev) * (2e-2 - 1e-3) + 1e-3).half()
    if qtype == "Q8_0":
        q = torch.randint(-127, 128, (blocks * 32,), generator=g, device=dev, dtype=torch.int8).view(torch.uint8)
    else:
        q = torch.randint(0, 256, (blocks * orc.PAYLOAD_BYTES[qtype],), generator=g, device=dev,
                          dtype=torch.uint8)
    return q, d.view(torch.uint8)


def torch_ref(x, q, s, qtype, n, k, bias):
    """Plain torch fp32 dequant + matmul on the GPU (TF32 off)."""
    w = orc.dequant_torch(q, s, qtype, (n, k))
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        return F.linear(x.float(), w, None if bias is None else bias.float())
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev


def decoder_cases():
    cases = [("Q8_0", 8192, 2048, 1, True)]
    for n, k in ((2304, 2048), (2048, 2048), (8192, 2048), (2048, 8192), (49152, 2048), (49156, 2048)):
        for m in (1, 2):
            cases.append(("Q4_0", n, k, m, n < 49152))
    for n, k in ((5632, 4608), (4608, 4608), (512, 4608), (18432, 4608), (4608, 18432),
                 (49152, 4608), (49157, 4608)):
        cases.append(("Q5_0", n, k, 2, n < 49152))
    for qtype in QTYPES:
        for n, k, bias in ((18432, 4608, True), (49152, 4608, False)):
            for m in (1, 2, 4, 8):
                cases.append((qtype, n, k, m, bias))
    return cases


@pytest.mark.parametrize("qtype,n,k,m,has_bias", decoder_cases())
def test_gemv_persistent_launch_shape(cuda_device, qtype, n, k, m, has_bias):
    """Automatic streaming launches (both persistent kernels, no split K) use
    a whole number of workgroups per CU, at most two: every CU holds the
    same share of tiles."""
    plan = native.gemv_plan(m, n, k, qtype)
    if plan["kernel"] not in ("stream", "mfma4") or (plan["kernel"] == "mfma4" and plan["lg_g"] > 1):
        return
    cus = torch.cuda.get_device_properties(cuda_device).multi_processor_count
    say(f"launch shape {qtype} m={m} n={n} k={k} plan={plan} cus={cus}")
    assert plan["groups"] % cus == 0 and plan["groups"] <= 2 * cus, plan


@pytest.mark.parametrize("kernel_path", ["auto", "mfma", "mfma4"], indirect=True)
@pytest.mark.parametrize("qtype,n,k,m,has_bias", decoder_cases())
def test_gemv_decoder_shapes(cuda_device, kernel_path, qtype, n, k, m, has_bias):
    say(f"gemv decoder shape {kernel_path} {qtype} m={m} n={n} k={k} bias={has_bias}")
    if kernel_path == "mfma":
        assert native.gemv_plan(m, n, k, qtype)["kernel"] == "mfma"
    if kernel_path == "mfma4" and stream_eligible(qtype, m, n, k):
        assert native.gemv_plan(m, n, k, qtype)["kernel"] == "mfma4"
    q, s = gpu_soa(qtype, n, k, seed=n + k + m, dev=cuda_device)
    g = torch.Generator(device=cuda_device).manual_seed(m)
    x = torch.randn((m, k), generator=g, device=cuda_device).half()
    bias = torch.randn(n, generator=g, device=cuda_device).half() if has_bias else None
    ref = torch_ref(x, q, s, qtype, n, k, bias)
    y = hip_gemv(x, q, s, qtype, n, bias, torch.float16)
    err = ((y.float() - ref).abs().max() / ref.abs().max()).item()
    assert err <= FP16_TOL, err
    y32 = hip_gemv(x, q, s, qtype, n, bias, torch.float32)
    err32 = ((y32 - ref).abs().max() / ref.abs().max()).item()
    assert err32 <= FP32_TOL, err32


def test_gemv_dequant_consistency_full_head(cuda_device):
    """At the largest shape, the GEMV equals the product of the bit-exact
    dequantization (a size-independent property)."""
    for qtype in QTYPES:
        n, k = 49152, 4608
        say(f"gemv vs dequant full head {qtype}")
        q, s = gpu_soa(qtype, n, k, seed=5, dev=cuda_device)
        w = torch.empty(n * k, dtype=torch.float32, device=cuda_device)
        native.dequant(q, s, w, qtype)
        assert torch.equal(w.view(n, k), orc.dequant_torch(q, s, qtype, (n, k)))
        x = torch.randn((2, k), device=cuda_device).half()
        y = hip_gemv(x, q, s, qtype, n, None, torch.float32)
        ref = x.double() @ w.view(n, k).double().t()
        assert ((y.double() - ref).abs().max() / ref.abs().max()).item() <= FP32_TOL


def test_gemv_is_deterministic(cuda_device):
    q, s = gpu_soa("Q4_0", 18432, 4608, seed=3, dev=cuda_device)
    x = torch.randn((2, 4608), device=cuda_device).half()
    a = hip_gemv(x, q, s, "Q4_0", 18432, None, torch.float32)
    b = hip_gemv(x, q, s, "Q4_0", 18432, None, torch.float32)
    assert torch.equal(a, b)


def test_gemv_fp16_denormal_activations(cuda_device):
    """Activations in the fp16 subnormal range and exact zeros."""
    n, k = 64, 512
    q, s = orc.synthetic_soa("Q5_0", n, k, seed=2)
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((2, k)) * 1e-6).astype(np.float16)
    x[0, ::3] = 0
    ref = orc.gemv_ref(x, q, s, "Q5_0", n, k)
    y = hip_gemv(to_dev(x, cuda_device), to_dev(q, cuda_device), to_dev(s, cuda_device), "Q5_0", n,
                 None, torch.float32)
    assert orc.rel_err(y.cpu().numpy(), ref) <= FP32_TOL


@pytest.fixture
def kernel_path(request, monkeypatch):
    """Force the MFMA, streaming or chunked GEMV kernel (read per call)."""
    monkeypatch.setenv("SVQ_PATH", request.param)
    return request.param


def mfma_eligible(qtype, m, n, k):
    """Shapes the MFMA kernel takes: whole steps of K, x in LDS."""
    kb = k // 32
    bps = 2 if qtype == "Q8_0" else 4
    lds = kb * 4 * m * 16 + kb * (m + 3) // 4 * 4 * 4
    return kb % bps == 0 and lds <= 156 * 1024


def stream_eligible(qtype, m, n, k):
    """Shapes the streaming kernels take: x and its offset sums in LDS."""
    units = k // 32 * (2 if qtype == "Q8_0" else 1)
    per_unit = (16 if qtype == "Q8_0" else 32) * 2 + 4
    return m * units * per_unit <= 156 * 1024


@pytest.mark.parametrize("kernel_path", ["mfma4", "mfma", "stream", "chunked"], indirect=True)
@pytest.mark.parametrize("qtype", QTYPES)
def test_gemv_every_kernel_against_oracle(cuda_device, kernel_path, qtype):
    rng = np.random.default_rng(7)
    for m in (1, 2, 3, 4, 5, 7, 8):
        for n, k in ((1, 32), (13, 128), (33, 192), (129, 2048), (515, 4608), (40, 18432)):
            say(f"gemv {kernel_path} {qtype} m={m} n={n} k={k}")
            plan = native.gemv_plan(m, n, k, qtype)
            if kernel_path == "mfma":
                assert (plan["kernel"] == "mfma") == mfma_eligible(qtype, m, n, k), plan
            if kernel_path == "mfma4":
                assert (plan["kernel"] == "mfma4") == stream_eligible(qtype, m, n, k), plan
            q, s = orc.synthetic_soa(qtype, n, k, seed=n + k + m)
            x = rng.standard_normal((m, k)).astype(np.float16)
            bias = rng.standard_normal(n).astype(np.float16)
            ref = orc.gemv_ref(x, q, s, qtype, n, k, bias)
            y = hip_gemv(to_dev(x, cuda_device), to_dev(q, cuda_device), to_dev(s, cuda_device), qtype, n,
                         to_dev(bias, cuda_device), torch.float32)
            assert orc.rel_err(y.cpu().numpy(), ref) <= FP32_TOL, (kernel_path, m, n, k)


@pytest.mark.parametrize("lg_g", range(0, 7))
@pytest.mark.parametrize("rows", (1, 2))
def test_gemv_every_launch_shape(cuda_device, monkeypatch, lg_g, rows):
    """Every lanes-per-row / rows-per-group choice, on ragged shapes."""
    monkeypatch.setenv("SVQ_LG_G", str(lg_g))
    monkeypatch.setenv("SVQ_ROWS", str(rows))
    rng = np.random.default_rng(lg_g * 10 + rows)
    for path in ("stream", "chunked"):
        monkeypatch.setenv("SVQ_PATH", path)
        for qtype in QTYPES:
            for m, n, k in ((1, 77, 320), (2, 130, 1056), (5, 3, 96)):
                say(f"gemv shape lg_g={lg_g} rows={rows} {path} {qtype} m={m} n={n} k={k}")
                q, s = orc.synthetic_soa(qtype, n, k, seed=m * n + k)
                x = rng.standard_normal((m, k)).astype(np.float16)
                ref = orc.gemv_ref(x, q, s, qtype, n, k)
                y = hip_gemv(to_dev(x, cuda_device), to_dev(q, cuda_device), to_dev(s, cuda_device), qtype,
                             n, None, torch.float32)
                assert orc.rel_err(y.cpu().numpy(), ref) <= FP32_TOL, (lg_g, rows, path, qtype, m, n, k)


@pytest.mark.parametrize("rows", (1, 2))
@pytest.mark.parametrize("ksplit", (1, 2, 3, 5, 8, 16))
def test_gemv_every_mfma_launch_shape(cuda_device, monkeypatch, rows, ksplit):
    """Every MFMA tile / K-split / tile-slot choice, on ragged row counts."""
    monkeypatch.setenv("SVQ_PATH", "mfma")
    monkeypatch.setenv("SVQ_MFMA_R", str(rows))
    monkeypatch.setenv("SVQ_MFMA_S", str(ksplit))
    rng = np.random.default_rng(rows * 100 + ksplit)
    for slots in (1, 2, 4):
        if slots * ksplit > 16:
            continue
        monkeypatch.setenv("SVQ_MFMA_P", str(slots))
        for qtype in QTYPES:
            for m, n, k in ((1, 77, 2048), (2, 130, 1152), (5, 35, 512), (8, 200, 4608)):
                say(f"gemv mfma rows={rows} ksplit={ksplit} slots={slots} {qtype} m={m} n={n} k={k}")
                plan = native.gemv_plan(m, n, k, qtype)
                steps = k // 32 // (2 if qtype == "Q8_0" else 4)
                assert plan["kernel"] == "mfma", plan
                assert plan["lg_g"] == min(ksplit, steps), plan  # K splits in use
                q, s = orc.synthetic_soa(qtype, n, k, seed=m * n + k)
                x = rng.standard_normal((m, k)).astype(np.float16)
                bias = rng.standard_normal(n).astype(np.float16)
                ref = orc.gemv_ref(x, q, s, qtype, n, k, bias)
                y = hip_gemv(to_dev(x, cuda_device), to_dev(q, cuda_device), to_dev(s, cuda_device),
                             qtype, n, to_dev(bias, cuda_device), torch.float32)
                assert orc.rel_err(y.cpu().numpy(), ref) <= FP32_TOL, (rows, ksplit, slots, qtype, m, n, k)
                y16 = hip_gemv(to_dev(x, cuda_device), to_dev(q, cuda_device), to_dev(s, cuda_device),
                               qtype, n, to_dev(bias, cuda_device), torch.float16)
                assert orc.rel_err(y16.float().cpu().numpy(), ref) <= FP16_TOL


@pytest.mark.parametrize("rows", (1, 2, 3))
def test_gemv_mfma4_row_sets(cuda_device, monkeypatch, rows):
    """Every variant of the streaming MFMA kernel on ragged shapes (3:
    consecutive units per lane: three Q4_0 / Q5_0 blocks, for K a multiple of
    1536, or one Q8_0 block)."""
    monkeypatch.setenv("SVQ_PATH", "mfma4")
    monkeypatch.setenv("SVQ_MFMA_R", str(rows))
    rng = np.random.default_rng(rows)
    for qtype in QTYPES:
        shapes = ((1, 77, 320), (2, 130, 1056), (3, 3, 96), (4, 261, 2048), (5, 19, 1056),
                  (6, 130, 320), (7, 261, 96), (8, 515, 2048))
        if rows == 3:
            shapes = ((1, 77, 1536), (2, 130, 4608), (3, 3, 3072), (4, 261, 1536), (5, 19, 3072),
                      (6, 130, 1536), (7, 261, 4608), (8, 515, 1536))
        for m, n, k in shapes:
            say(f"gemv mfma4 rows={rows} {qtype} m={m} n={n} k={k}")
            assert native.gemv_plan(m, n, k, qtype)["rows"] == rows
            q, s = orc.synthetic_soa(qtype, n, k, seed=m * n + k)
            x = rng.standard_normal((m, k)).astype(np.float16)
            bias = rng.standard_normal(n).astype(np.float16)
            ref = orc.gemv_ref(x, q, s, qtype, n, k, bias)
            y = hip_gemv(to_dev(x, cuda_device), to_dev(q, cuda_device), to_dev(s, cuda_device), qtype, n,
                         to_dev(bias, cuda_device), torch.float32)
            assert orc.rel_err(y.cpu().numpy(), ref) <= FP32_TOL, (rows, qtype, m, n, k)


@pytest.mark.parametrize("ksplit", (1, 2, 4))
@pytest.mark.parametrize("rows", (1, 2, 3))
def test_gemv_mfma4_ksplit(cuda_device, monkeypatch, rows, ksplit):
    """Split-K of the streaming MFMA kernel (waves of a workgroup sharing a
    tile and adding their partial sums in LDS), every variant, ragged rows."""
    monkeypatch.setenv("SVQ_PATH", "mfma4")
    monkeypatch.setenv("SVQ_MFMA_R", str(rows))
    monkeypatch.setenv("SVQ_MFMA_S", str(ksplit))
    rng = np.random.default_rng(10 * rows + ksplit)
    for qtype in QTYPES:
        for m, n, k in ((1, 37, 1536), (2, 130, 4608), (3, 9, 18432), (6, 21, 3072), (8, 130, 4608)):
            plan = native.gemv_plan(m, n, k, qtype)
            say(f"gemv mfma4 rows={rows} ksplit={ksplit} {qtype} m={m} n={n} k={k} plan={plan}")
            assert plan["kernel"] == "mfma4" and plan["lg_g"] in (1, ksplit), plan
            q, s = orc.synthetic_soa(qtype, n, k, seed=m + n + k)
            x = rng.standard_normal((m, k)).astype(np.float16)
            bias = rng.standard_normal(n).astype(np.float16)
            ref = orc.gemv_ref(x, q, s, qtype, n, k, bias)
            y = hip_gemv(to_dev(x, cuda_device), to_dev(q, cuda_device), to_dev(s, cuda_device), qtype, n,
                         to_dev(bias, cuda_device), torch.float32)
            assert orc.rel_err(y.cpu().numpy(), ref) <= FP32_TOL, (rows, ksplit, qtype, m, n, k)

"""Pins of the CPU oracle (CPU only).

Each oracle function is checked against something other than itself:
the reference's known-answer tests (tests/test_quantization.py:21-59 of the
reference), exhaustive enumeration of every lane value against the block
layout's closed forms, Python's own fp16 decoding, the exact-rational golden
fixtures (tests/golden/make_golden.py), brute-force rational GEMV, the C
restatement, and byte-permutation invariants. The planted-mistake tests at
the end show that each pin rejects a plausible wrong decoder.
"""
from __future__ import annotations

import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import c_oracle
from oracle import soa_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"
QTYPES = ("Q4_0", "Q5_0", "Q8_0")


def raw_block(d: float, payload: bytes) -> np.ndarray:
    return np.frombuffer(struct.pack("<e", d) + payload, dtype=np.uint8)


# --- the reference's known-answer tests ------------------------------------

def test_q8_0_known_answer():
    w = orc.dequantize_aos(raw_block(0.5, bytes(range(32))), "Q8_0", (1, 32))
    assert np.array_equal(w[0], np.arange(32, dtype=np.float32) * 0.5)


def test_q4_0_nibble_halves_known_answer():
    w = orc.dequantize_aos(raw_block(1.0, bytes([0xF0] * 16)), "Q4_0", (1, 32))
    assert np.array_equal(w[0, :16], np.full(16, -8.0, np.float32))
    assert np.array_equal(w[0, 16:], np.full(16, 7.0, np.float32))


def test_q5_0_fifth_bits_known_answer():
    payload = struct.pack("<I", 0xFFFF0000) + bytes(range(16))
    w = orc.dequantize_aos(raw_block(1.0, payload), "Q5_0", (1, 32))
    assert np.array_equal(w[0, :16], np.arange(16, dtype=np.float32) - 16)
    assert np.array_equal(w[0, 16:], np.zeros(16, np.float32))


def test_q8_0_linear_known_answer():
    raw = raw_block(0.25, bytes([4] * 32))
    q, s = orc.pack_soa(raw, "Q8_0", (1, 32))
    y = orc.gemv_ref(np.ones((1, 32), np.float16), q, s, "Q8_0", 1, 32)
    assert y[0, 0] == 32.0
    assert q.size + s.size == raw.size


def test_q4_0_embedding_rows_known_answer():
    raw = np.concatenate((raw_block(1.0, bytes([0x99] * 16)), raw_block(2.0, bytes([0x99] * 16))))
    w = orc.dequantize_aos(raw, "Q4_0", (2, 32))
    assert np.array_equal(w[0], np.ones(32, np.float32))
    assert np.array_equal(w[1], np.full(32, 2.0, np.float32))


# --- exhaustive lane enumeration against the closed forms ------------------

def closed_form_code(qtype: str, payload: bytes, j: int) -> int:
    """Weight j's integer code from the GGUF block layout, bit by bit."""
    if qtype == "Q8_0":
        b = payload[j]
        return b - 256 if b >= 128 else b
    if qtype == "Q4_0":
        b = payload[j % 16]
        return (b & 15 if j < 16 else b >> 4) - 8
    mask = payload[0] | payload[1] << 8 | payload[2] << 16 | payload[3] << 24
    b = payload[4 + j % 16]
    nib = b & 15 if j < 16 else b >> 4
    return (nib | ((mask >> j) & 1) << 4) - 16


def enumerated_payloads(qtype: str):
    """Every byte value at every byte position (Q8_0, Q4_0); for Q5_0 every
    nibble value at every weight with its mask bit clear and set."""
    width = orc.PAYLOAD_BYTES[qtype]
    out = []
    if qtype in ("Q8_0", "Q4_0"):
        for pos in range(width):
            for v in range(256):
                p = bytearray([0x5A] * width)
                p[pos] = v
                out.append(bytes(p))
    else:
        for j in range(32):
            for nib in range(16):
                for bit in (0, 1):
                    p = bytearray(20)
                    mask = (bit << j) | (0xA5A5A5A5 & ~(1 << j) & 0xFFFFFFFF)
                    p[0:4] = struct.pack("<I", mask)
                    for t in range(16):
                        p[4 + t] = 0x3C
                    cur = p[4 + j % 16]
                    p[4 + j % 16] = (cur & 0xF0) | nib if j < 16 else (cur & 0x0F) | (nib << 4)
                    out.append(bytes(p))
    return out


@pytest.mark.parametrize("qtype", QTYPES)
def test_block_codes_exhaustive(qtype):
    payloads = enumerated_payloads(qtype)
    arr = np.frombuffer(b"".join(payloads), dtype=np.uint8).reshape(len(payloads), -1)
    codes = orc.block_codes(arr, qtype)
    expect = np.array([[closed_form_code(qtype, p, j) for j in range(32)] for p in payloads])
    assert np.array_equal(codes, expect)


def test_scales_match_python_half_decoding_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint16)
    got = orc.scales_f32(bits.view(np.uint8))
    want = np.array([struct.unpack("<e", struct.pack("<H", int(b)))[0] for b in bits],
                    dtype=np.float64)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].astype(np.float64), want[finite])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_c_half_conversion_all_bit_patterns():
    lib = c_oracle.load()
    for b in range(65536):
        want = struct.unpack("<e", struct.pack("<H", b))[0]
        got = lib.svqo_half_to_float(b)
        if want != want:
            assert got != got
        else:
            assert got == want, hex(b)


def test_dequantized_products_are_exact():
    """float32(code) * float32(d) is the exact rational product for every code
    and a sample of scales spanning subnormal to largest finite."""
    scale_bits = [0x0001, 0x0017, 0x03FF, 0x0400, 0x1C00, 0x2E66, 0x3C00, 0x5555, 0x7BFF,
                  0x8001, 0xBC00, 0xFBFF]
    codes = np.arange(-128, 128, dtype=np.int32)
    for sb in scale_bits:
        d = orc.scales_f32(np.array([sb], np.uint16).view(np.uint8))[0]
        prod = codes.astype(np.float32) * d
        for c, p in zip(codes, prod):
            assert Fraction(float(p)) == int(c) * Fraction(float(d))


# --- SoA repack invariants ---------------------------------------------------

@pytest.mark.parametrize("qtype", QTYPES)
def test_pack_soa_is_a_byte_permutation(qtype):
    raw = orc.packed_matrix(qtype, 13, 128)
    q, s = orc.pack_soa(raw, qtype, (13, 128))
    assert q.size + s.size == raw.size
    assert np.array_equal(orc.unpack_soa(q, s, qtype), raw)
    aos = orc.dequantize_aos(raw, qtype, (13, 128))
    soa = orc.dequantize_soa(q, s, qtype, (13, 128))
    assert np.array_equal(aos.view(np.int32), soa.view(np.int32))


def test_pack_soa_rejects_bad_shapes():
    raw = orc.packed_matrix("Q4_0", 2, 64)
    with pytest.raises(ValueError):
        orc.pack_soa(raw, "Q4_0", (2, 48))
    with pytest.raises(ValueError):
        orc.pack_soa(raw[:-1], "Q4_0", (2, 64))
    with pytest.raises(ValueError):
        orc.dequantize_soa(raw[:10], raw[:4], "Q4_0", (2, 64))


# --- golden fixtures (exact rationals from an independent decoder) ----------

def golden_cases(qtype):
    data = np.load(GOLDEN / f"{qtype.lower()}.npz")
    names = sorted({key.split("/")[0] for key in data.files})
    return [(name, {key.split("/")[1]: data[key] for key in data.files if key.startswith(name + "/")})
            for name in names]


@pytest.mark.parametrize("qtype", QTYPES)
def test_oracle_matches_golden(qtype):
    for name, fx in golden_cases(qtype):
        n, k, m = (int(v) for v in fx["shape"])
        q, s = orc.pack_soa(fx["aos"], qtype, (n, k))
        assert np.array_equal(q, fx["q"]) and np.array_equal(s, fx["s"]), name
        w = orc.dequantize_soa(fx["q"], fx["s"], qtype, (n, k))
        assert np.array_equal(w.view(np.int32), fx["dequant_bits"]), name
        y = orc.gemv_ref(fx["x"], fx["q"], fx["s"], qtype, n, k, fx["bias"])
        assert orc.rel_err(y, fx["y_exact"]) < 1e-12, name
        yc = c_oracle.gemv_f64(fx["x"], fx["q"], fx["s"], qtype, n, k, fx["bias"])
        assert orc.rel_err(yc, fx["y_exact"]) < 1e-12, name
        wc = c_oracle.dequant(fx["q"], fx["s"], qtype).reshape(n, k)
        assert np.array_equal(wc.view(np.int32), fx["dequant_bits"]), name


@pytest.mark.parametrize("qtype", QTYPES)
def test_c_oracle_matches_numpy_oracle(qtype):
    n, k = 37, 320
    q, s = orc.synthetic_soa(qtype, n, k, seed=5)
    w = orc.dequantize_soa(q, s, qtype, (n, k))
    wc = c_oracle.dequant(q, s, qtype).reshape(n, k)
    assert np.array_equal(w.view(np.int32), wc.view(np.int32))
    x = np.random.default_rng(5).standard_normal((3, k)).astype(np.float16)
    assert orc.rel_err(c_oracle.gemv_f64(x, q, s, qtype, n, k), orc.gemv_ref(x, q, s, qtype, n, k)) < 1e-12


def test_gemv_brute_force_rational():
    """Tiny GEMV in exact rationals, one weight at a time, vs gemv_ref."""
    for qtype in QTYPES:
        n, k, m = 3, 64, 2
        raw = orc.packed_matrix(qtype, n, k, seed=99)
        q, s = orc.pack_soa(raw, qtype, (n, k))
        x = np.random.default_rng(1).standard_normal((m, k)).astype(np.float16)
        bb = orc.BLOCK_BYTES[qtype]
        for mi in range(m):
            for row in range(n):
                acc = Fraction(0)
                for kk in range(k):
                    blk = raw[(row * (k // 32) + kk // 32) * bb:][:bb].tobytes()
                    d = Fraction(struct.unpack("<e", blk[:2])[0])
                    acc += closed_form_code(qtype, blk[2:], kk % 32) * d * Fraction(float(x[mi, kk]))
                y = orc.gemv_ref(x, q, s, qtype, n, k)[mi, row]
                assert abs(y - float(acc)) <= 1e-12 * max(1.0, abs(float(acc)))


def test_tiled_cpu_path_matches_reference_gemv():
    torch = pytest.importorskip("torch")
    for qtype in QTYPES:
        n, k = 300, 4160  # several 2 MiB / K row slices and a ragged last one
        q, s = orc.synthetic_soa(qtype, n, k, seed=3)
        x = np.random.default_rng(3).standard_normal((2, k)).astype(np.float16)
        bias = np.random.default_rng(4).standard_normal(n).astype(np.float16)
        y = orc.tiled_linear_cpu(torch.from_numpy(x).float(), torch.from_numpy(q), torch.from_numpy(s),
                                 qtype, n, k, torch.from_numpy(bias).float())
        assert orc.rel_err(y.numpy(), orc.gemv_ref(x, q, s, qtype, n, k, bias)) < 1e-5


# --- planted mistakes: each pin rejects a plausible wrong decoder -----------

def swapped_halves(payload, qtype):
    c = orc.block_codes(payload, qtype)
    return np.concatenate((c[:, 16:], c[:, :16]), axis=1) if qtype != "Q8_0" else c


def reversed_mask_bits(payload, qtype):
    if qtype != "Q5_0":
        return orc.block_codes(payload, qtype)
    p = np.array(payload, dtype=np.uint8, copy=True)
    p[:, :4] = p[:, 3::-1]  # big-endian mask read
    return orc.block_codes(p, qtype)


def wrong_offset(payload, qtype):
    return orc.block_codes(payload, qtype) + 1


def unsigned_q8(payload, qtype):
    if qtype != "Q8_0":
        return orc.block_codes(payload, qtype)
    return np.ascontiguousarray(payload, dtype=np.uint8).astype(np.int32)


def golden_decode_ok() -> bool:
    """Whole-decode pin: the oracle's dequantization equals every golden bit."""
    for qtype in QTYPES:
        for _, fx in golden_cases(qtype):
            n, k, _m = (int(v) for v in fx["shape"])
            w = orc.dequantize_soa(fx["q"], fx["s"], qtype, (n, k))
            if not np.array_equal(w.view(np.int32), fx["dequant_bits"]):
                return False
    return True


def enumeration_ok() -> bool:
    """Lane pin: the oracle's codes equal the closed forms for every value."""
    for qtype in QTYPES:
        payloads = enumerated_payloads(qtype)
        arr = np.frombuffer(b"".join(payloads), dtype=np.uint8).reshape(len(payloads), -1)
        expect = np.array([[closed_form_code(qtype, p, j) for j in range(32)] for p in payloads])
        if not np.array_equal(orc.block_codes(arr, qtype), expect):
            return False
    return True


def known_answers_ok() -> bool:
    for test in (test_q8_0_known_answer, test_q4_0_nibble_halves_known_answer,
                 test_q5_0_fifth_bits_known_answer, test_q4_0_embedding_rows_known_answer):
        try:
            test()
        except AssertionError:
            return False
    return True


def test_pins_pass_on_the_oracle():
    assert golden_decode_ok() and enumeration_ok() and known_answers_ok()


@pytest.mark.parametrize("mutant", [swapped_halves, reversed_mask_bits, wrong_offset, unsigned_q8])
def test_pins_reject_planted_mistakes(mutant, monkeypatch):
    """Plant the mistake in the oracle's decoder; every pin must fail."""
    original = orc.block_codes
    monkeypatch.setattr(orc, "block_codes", lambda p, q: mutant(p, q) if q in QTYPES else original(p, q))
    # `mutant` calls orc.block_codes internally; route those calls to the original.
    monkeypatch.setattr(orc, "block_codes",
                        lambda p, q, _mutant=mutant: _call_mutant(_mutant, original, p, q))
    assert not golden_decode_ok()
    assert not enumeration_ok()


def _call_mutant(mutant, original, payload, qtype):
    saved = orc.block_codes
    orc.block_codes = original
    try:
        return mutant(payload, qtype)
    finally:
        orc.block_codes = saved


def test_golden_rejects_transposed_gemv():
    name, fx = golden_cases("Q4_0")[0]
    n, k, m = (int(v) for v in fx["shape"])
    w = orc.dequantize_soa(fx["q"], fx["s"], "Q4_0", (n, k)).astype(np.float64)
    # A transposed-operand mistake: reading W column-major.
    wt = w.reshape(-1).reshape(k, n).T
    y_bad = fx["x"].astype(np.float64) @ wt.T + fx["bias"].astype(np.float64)
    assert orc.rel_err(y_bad, fx["y_exact"]) > 1e-2

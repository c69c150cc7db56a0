"""Write the golden fixtures of the SoA decode and GEMV (tests/golden/*.npz).

The expected values come from a pure-Python, bit-level decoder written from
the GGUF block layout (struct + integer shifts, one weight at a time) and an
exact rational GEMV (fractions.Fraction), so they are independent of the
numpy oracle, of the C oracle and of any floating-point summation order:

* Inputs: the reference tests' seeded packing recipe
  (tests/test_quantization.py:62-85: default_rng(321), fp16 scales uniform in
  [0.02, 0.22]) at the reference tests' matrix shapes (:89, :137), plus the
  reference's known-answer blocks (:21-37) and edge blocks (zero, negative,
  subnormal and largest fp16 scales; all-0x00 / all-0xFF payloads; the int8
  value -128).
* dequant_bits: float32 bits of float(code) * float(d), exact by construction
  (|code| <= 128 and an 11-bit significand fit in 24 bits).
* y_exact: sum_k x * W + bias in exact rationals, rounded once to float64.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import struct
from fractions import Fraction
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent
BLOCK = {"Q4_0": 18, "Q5_0": 22, "Q8_0": 34}


def half_to_fraction(bits: int) -> Fraction:
    sign = -1 if bits >> 15 else 1
    exp = (bits >> 10) & 31
    man = bits & 1023
    if exp == 31:
        raise ValueError("inf/nan not representable")
    if exp == 0:
        return sign * Fraction(man, 1 << 24)
    return sign * Fraction(1024 + man, 1 << 10) * Fraction(2) ** (exp - 15)


def decode_block(raw: bytes, qtype: str) -> tuple[int, list[int]]:
    """(fp16 scale bits, 32 signed codes) of one AoS block, weight by weight."""
    (d_bits,) = struct.unpack_from("<H", raw, 0)
    body = raw[2:]
    codes = []
    for j in range(32):
        if qtype == "Q8_0":
            (v,) = struct.unpack_from("<b", body, j)
        elif qtype == "Q4_0":
            byte = body[j % 16]
            v = ((byte >> (4 * (j // 16))) & 15) - 8
        else:
            (mask,) = struct.unpack_from("<I", body, 0)
            byte = body[4 + j % 16]
            nib = (byte >> (4 * (j // 16))) & 15
            v = (nib | (((mask >> j) & 1) << 4)) - 16
        codes.append(v)
    return d_bits, codes


def f32_bits(code: int, d_bits: int) -> int:
    """fp32 bits of the IEEE product float(code) * float(d): the exact value,
    and for a zero product the sign bit sign(code) XOR sign(d), as IEEE
    multiplication gives it (code 0 is +0)."""
    value = code * half_to_fraction(d_bits)
    if value == 0:
        return ((d_bits >> 15) ^ (1 if code < 0 else 0)) << 31
    f = np.float32(float(value))
    if Fraction(float(f)) != value:
        raise AssertionError("dequantized value not exact in fp32")
    return int(np.array(f, dtype=np.float32).view(np.uint32))


def packed_matrix(qtype: str, n: int, k: int, seed: int = 321) -> bytes:
    """The seeded recipe of tests/test_quantization.py:62-85, block by block."""
    rng = np.random.default_rng(seed)
    blocks = n * k // 32
    scales = rng.uniform(0.02, 0.22, size=blocks).astype(np.float16)
    if qtype == "Q4_0":
        signed = rng.integers(-8, 8, size=(blocks, 32), dtype=np.int8)
        unsigned = (signed.astype(np.int16) + 8).astype(np.uint8)
        payload = unsigned[:, :16] | (unsigned[:, 16:] << 4)
    elif qtype == "Q5_0":
        unsigned = rng.integers(0, 32, size=(blocks, 32)).astype(np.uint32)
        fifth = ((unsigned >> 4) << np.arange(32, dtype=np.uint32)).sum(axis=1).astype("<u4")
        nibbles = (unsigned[:, :16] & 15) | ((unsigned[:, 16:] & 15) << 4)
        payload = np.concatenate((fifth.view(np.uint8).reshape(blocks, 4),
                                  nibbles.astype(np.uint8)), axis=1)
    else:
        payload = rng.integers(-127, 128, size=(blocks, 32), dtype=np.int8).view(np.uint8)
    return b"".join(struct.pack("<e", float(scales[i])) + payload[i].tobytes()
                    for i in range(blocks))


def edge_blocks(qtype: str) -> bytes:
    """Known-answer and edge blocks (4 rows of 64 weights = 8 blocks)."""
    w = BLOCK[qtype] - 2
    blocks = []
    if qtype == "Q8_0":
        blocks.append(struct.pack("<e", 0.5) + bytes(range(32)))          # :21-24
        blocks.append(struct.pack("<e", 0.25) + bytes([4] * 32))          # :39-45
    elif qtype == "Q4_0":
        blocks.append(struct.pack("<e", 1.0) + bytes([0xF0] * 16))        # :26-30
        blocks.append(struct.pack("<e", 1.0) + bytes([0x99] * 16))        # :51-59
    else:
        blocks.append(struct.pack("<e", 1.0) + struct.pack("<I", 0xFFFF0000) + bytes(range(16)))  # :32-37
        blocks.append(struct.pack("<e", 2.0) + struct.pack("<I", 0x0000FFFF) + bytes(range(16)))
    blocks.append(struct.pack("<H", 0x0000) + bytes([0xFF] * w))   # +0 scale
    blocks.append(struct.pack("<H", 0x8000) + bytes([0x37] * w))   # -0 scale
    blocks.append(struct.pack("<H", 0x0001) + bytes([0xFF] * w))   # smallest subnormal
    blocks.append(struct.pack("<H", 0x7BFF) + bytes([0x80] * w))   # largest finite; int8 -128
    blocks.append(struct.pack("<e", -0.0123) + bytes([0x00] * w))  # negative scale
    blocks.append(struct.pack("<H", 0x03FF) + bytes(range(0x10, 0x10 + w)))  # largest subnormal
    return b"".join(blocks)


def fixture(qtype: str, raw: bytes, n: int, k: int, m: int, seed: int) -> dict:
    bb = BLOCK[qtype]
    nblocks = n * k // 32
    assert len(raw) == nblocks * bb
    weights = []
    q_parts, s_parts, bits = [], [], []
    for b in range(nblocks):
        block = raw[b * bb:(b + 1) * bb]
        d_bits, codes = decode_block(block, qtype)
        d = half_to_fraction(d_bits)
        vals = [c * d for c in codes]
        weights.append(vals)
        bits.extend(f32_bits(c, d_bits) for c in codes)
        q_parts.append(block[2:])
        s_parts.append(block[:2])
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float16)
    bias = rng.standard_normal(n).astype(np.float16)
    xf = [[Fraction(float(v)) for v in row] for row in x]
    bf = [Fraction(float(v)) for v in bias]
    y = np.empty((m, n), dtype=np.float64)
    kb = k // 32
    for mi in range(m):
        for row in range(n):
            acc = bf[row]
            for blk in range(kb):
                wrow = weights[row * kb + blk]
                xs = xf[mi][blk * 32:(blk + 1) * 32]
                acc += sum(wv * xv for wv, xv in zip(wrow, xs))
            y[mi, row] = float(acc)
    return {
        "aos": np.frombuffer(raw, dtype=np.uint8),
        "q": np.frombuffer(b"".join(q_parts), dtype=np.uint8),
        "s": np.frombuffer(b"".join(s_parts), dtype=np.uint8),
        "dequant_bits": np.array(bits, dtype=np.int64).astype(np.uint32).view(np.int32).reshape(n, k),
        "x": x, "bias": bias, "y_exact": y,
        "shape": np.array([n, k, m], dtype=np.int64),
    }


CASES = [
    # name, qtype, source, n, k, m, seed
    ("seeded_13x128", None, "seeded", 13, 128, 2, 11),
    ("seeded_33x192", None, "seeded", 33, 192, 5, 12),
    ("seeded_9x64", None, "seeded", 9, 64, 1, 13),
    ("edge_4x64", None, "edge", 4, 64, 3, 14),
]


def main() -> None:
    for qtype in BLOCK:
        arrays = {}
        for name, _, source, n, k, m, seed in CASES:
            raw = packed_matrix(qtype, n, k) if source == "seeded" else edge_blocks(qtype)
            fx = fixture(qtype, raw, n, k, m, seed)
            for key, value in fx.items():
                arrays[f"{name}/{key}"] = value
        path = OUT / f"{qtype.lower()}.npz"
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()

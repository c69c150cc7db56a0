"""CPU oracle of the GGUF SoA dequantize + GEMV path.

TEST INFRASTRUCTURE ONLY. This module is the checker: only tests/,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of bench.py may import
it. The product (comfyui-starvector-gguf_amd/) never imports or calls it.

It restates, with numpy (and, for the CPU baseline, torch CPU ops), the
algorithm of the reference's quantization.py for this path:

  block_codes      quantization.py:34-47   (_block_values)
  dequantize_aos   quantization.py:50-65   (dequantize, quantized types)
  pack_soa         quantization.py:67-90   (pack_gguf_soa)
  dequantize_soa   quantization.py:93-105  (dequantize_soa)
  gemv_ref         quantization.py:171-229 (_soa_gemv) semantics, evaluated in
                   float64: y = x @ W^T + bias over the exactly dequantized W
  tiled_linear_cpu quantization.py:390-407 (GGUFLinear.forward CPU branch),
                   the reference's CPU path, timed as the CPU baseline
  packed_matrix    tests/test_quantization.py:62-85 (seeded packing recipe)

How each function is pinned (tests/test_oracle.py): the reference's
known-answer tests (tests/test_quantization.py:21-59), exhaustive per-lane
enumeration of every byte/nibble/mask-bit value against the closed forms of
the GGUF block layout, an independent pure-Python bit-level decoder, exact
rational (fractions) GEMV on tiny inputs, the SoA byte-permutation invariants
of tests/test_quantization.py:135-145, and the C restatement in
svq_oracle.c. Planted-mistake tests check that each pin catches a plausible
error (swapped nibble halves, wrong mask bit order, wrong offset, transposed
operand).
"""
from __future__ import annotations

import numpy as np

BLOCK_BYTES = {"Q4_0": 18, "Q5_0": 22, "Q8_0": 34}
PAYLOAD_BYTES = {q: b - 2 for q, b in BLOCK_BYTES.items()}
QTYPES = ("Q4_0", "Q5_0", "Q8_0")


def block_codes(payload: np.ndarray, qtype: str) -> np.ndarray:
    """Signed integer weights [B, 32] of block payloads [B, W] (no scales).

    Q8_0: int8 bytes. Q4_0: byte j low nibble -> weight j, high nibble ->
    weight j + 16, minus 8. Q5_0: bytes 0-3 are a little-endian uint32 mask
    whose bit j is weight j's fifth bit; nibbles as Q4_0 from byte 4; minus 16.
    """
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    if qtype == "Q8_0":
        return payload.view(np.int8).astype(np.int32)
    nib = payload[:, -16:].astype(np.int32)
    codes = np.concatenate((nib & 15, nib >> 4), axis=1)
    if qtype == "Q4_0":
        return codes - 8
    if qtype != "Q5_0":
        raise ValueError(qtype)
    mask = payload[:, :4].astype(np.uint32)
    mask = mask[:, 0] | (mask[:, 1] << 8) | (mask[:, 2] << 16) | (mask[:, 3] << 24)
    fifth = (mask[:, None] >> np.arange(32, dtype=np.uint32)) & 1
    return (codes | (fifth.astype(np.int32) << 4)) - 16


def scales_f32(scale_bytes: np.ndarray) -> np.ndarray:
    """fp16 scale bits (2 little-endian bytes per block) -> float32 [B]."""
    flat = np.ascontiguousarray(scale_bytes, dtype=np.uint8).reshape(-1)
    return flat.view("<f2").astype(np.float32)


def dequantize_aos(raw: np.ndarray, qtype: str, shape) -> np.ndarray:
    """GGUF AoS blocks [fp16 d][payload] -> float32 weights of `shape`; each
    weight is the exact fp32 product float(code) * float(d)."""
    bb = BLOCK_BYTES[qtype]
    n = int(np.prod(shape))
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    if n % 32 or raw.size != n // 32 * bb:
        raise ValueError(f"Invalid {qtype} payload for shape {shape}")
    blocks = raw.reshape(-1, bb)
    d = scales_f32(blocks[:, :2].copy())
    w = block_codes(blocks[:, 2:], qtype).astype(np.float32) * d[:, None]
    return w.reshape(shape)


def pack_soa(raw: np.ndarray, qtype: str, shape) -> tuple[np.ndarray, np.ndarray]:
    """AoS -> SoA: (payloads without scales, flat; scale bytes, flat)."""
    if qtype not in BLOCK_BYTES or len(shape) != 2 or shape[1] % 32:
        raise ValueError("Expected rank-2 Q4_0/Q5_0/Q8_0 matrix")
    bb = BLOCK_BYTES[qtype]
    blocks = shape[0] * (shape[1] // 32)
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    if raw.size != blocks * bb:
        raise ValueError("Invalid packed GGUF payload")
    rows = raw.reshape(blocks, bb)
    return rows[:, 2:].reshape(-1).copy(), rows[:, :2].reshape(-1).copy()


def unpack_soa(q: np.ndarray, s: np.ndarray, qtype: str) -> np.ndarray:
    """SoA -> AoS, the inverse byte permutation of pack_soa."""
    w = PAYLOAD_BYTES[qtype]
    q = np.ascontiguousarray(q, dtype=np.uint8).reshape(-1, w)
    s = np.ascontiguousarray(s, dtype=np.uint8).reshape(-1, 2)
    return np.concatenate((s, q), axis=1).reshape(-1)


def dequantize_soa(q: np.ndarray, s: np.ndarray, qtype: str, shape) -> np.ndarray:
    """Decode the SoA arrays to float32 weights of `shape` (exact products)."""
    n = int(np.prod(shape))
    w = PAYLOAD_BYTES[qtype]
    q = np.ascontiguousarray(q, dtype=np.uint8).reshape(-1)
    s = np.ascontiguousarray(s, dtype=np.uint8).reshape(-1)
    if n % 32 or q.size != n // 32 * w or s.size != n // 32 * 2:
        raise ValueError(f"Invalid SoA payload for shape {shape}")
    d = scales_f32(s)
    vals = block_codes(q.reshape(-1, w), qtype).astype(np.float32) * d[:, None]
    return vals.reshape(shape)


def gemv_ref(x: np.ndarray, q: np.ndarray, s: np.ndarray, qtype: str,
             n: int, k: int, bias: np.ndarray | None = None) -> np.ndarray:
    """float64 y[m, n] = sum_k x[m, k] W[n, k] + bias[n] for fp16 x / bias."""
    w = dequantize_soa(q, s, qtype, (n, k)).astype(np.float64)
    y = np.asarray(x, dtype=np.float16).astype(np.float64) @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float16).astype(np.float64)[None, :]
    return y


def rel_err(y, ref) -> float:
    """max|y - ref| / max|ref|, the error metric of tools/tune_kernels.py:83."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.abs(ref).max()
    return float(np.abs(y - ref).max() / (denom if denom > 0 else 1.0))


# ---------------------------------------------------------------------------
# Seeded inputs.

def packed_matrix(qtype: str, n: int, k: int, seed: int = 321) -> np.ndarray:
    """AoS GGUF bytes of the reference tests' seeded matrix
    (tests/test_quantization.py:62-85): default_rng(321); fp16 scales uniform in
    [0.02, 0.22]; Q4_0 codes uniform in [-8, 8); Q5_0 unsigned codes uniform in
    [0, 32); Q8_0 codes uniform in [-127, 127]."""
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
    elif qtype == "Q8_0":
        payload = rng.integers(-127, 128, size=(blocks, 32), dtype=np.int8).view(np.uint8)
    else:
        raise ValueError(qtype)
    raw = np.concatenate((scales.reshape(-1, 1).view(np.uint8), payload.astype(np.uint8)), axis=1)
    return raw.reshape(-1)


def synthetic_soa(qtype: str, n: int, k: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """SoA arrays with the benchmark distributions: fp16 scales uniform in
    [1e-3, 2e-2]; Q4_0/Q5_0 payload bytes uniform (uniform codes); Q8_0 int8
    uniform in [-127, 127]."""
    rng = np.random.default_rng(seed)
    blocks = n * k // 32
    d = rng.uniform(1e-3, 2e-2, size=blocks).astype(np.float16)
    if qtype == "Q8_0":
        q = rng.integers(-127, 128, size=blocks * 32, dtype=np.int8).view(np.uint8)
    else:
        q = rng.integers(0, 256, size=blocks * PAYLOAD_BYTES[qtype], dtype=np.uint8)
    return q, d.view(np.uint8).copy()


# ---------------------------------------------------------------------------
# The reference's CPU path (GGUFLinear.forward on CPU, quantization.py:390-407),
# used as the CPU baseline.

def tiled_linear_cpu(x, q, s, qtype: str, n: int, k: int, bias=None):
    """fp32 CPU GEMV the way the reference's CPU branch runs it: slices of
    max(1, 2 MiB / K) rows are dequantized to fp32 and multiplied with
    F.linear, then concatenated. x, q, s, bias are CPU torch tensors."""
    import torch
    import torch.nn.functional as F

    width = PAYLOAD_BYTES[qtype]
    kb = k // 32
    rows_per_chunk = max(1, 2 * 1024 * 1024 // k)
    payload = q.reshape(n, kb * width)
    scales = s.reshape(n, kb * 2)
    outputs = []
    for start in range(0, n, rows_per_chunk):
        end = min(start + rows_per_chunk, n)
        w = _dequant_torch(payload[start:end].reshape(-1), scales[start:end].reshape(-1),
                           qtype, (end - start, k))
        outputs.append(F.linear(x, w, None if bias is None else bias[start:end]))
    return torch.cat(outputs, -1)


def _dequant_torch(q, s, qtype, shape):
    """fp32 weights from SoA torch tensors (torch restatement of
    quantization.py:34-47, 93-105); runs on the tensors' device."""
    import torch

    w = PAYLOAD_BYTES[qtype]
    blocks = q.reshape(-1, w)
    d = s.contiguous().view(torch.float16).float().reshape(-1, 1)
    if qtype == "Q8_0":
        codes = blocks.view(torch.int8).float()
    else:
        nib = blocks[:, -16:]
        codes = torch.cat((nib & 15, nib >> 4), -1).to(torch.int32)
        if qtype == "Q4_0":
            codes = (codes - 8).float()
        else:
            m = blocks[:, :4].to(torch.int64)
            mask = m[:, 0] | (m[:, 1] << 8) | (m[:, 2] << 16) | (m[:, 3] << 24)
            bits = (mask[:, None] >> torch.arange(32, device=q.device)) & 1
            codes = ((codes | (bits.to(torch.int32) << 4)) - 16).float()
    return (codes * d).reshape(shape)


def dequant_torch(q, s, qtype: str, shape):
    """Public torch restatement of the SoA decode: a plain torch fp32
    reference of the dequantization, usable on CPU or GPU tensors."""
    return _dequant_torch(q.reshape(-1), s.reshape(-1), qtype, shape)

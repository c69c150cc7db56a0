"""StarVector GGUF quantized ops for MI355X: compact SoA parameters and gfx950 HIP GEMV.

Drop-in for the reference's L2 module (quantization.py of
ComfyUI-StarVector-GGUF): the same public names, signatures, parameter layout
(`weight` = uint8 SoA payload, `weight_scales` = uint8 fp16 scale bits) and
validation messages. What changes is the device code: every computation on a
GPU tensor runs in the hand-written HIP kernels of libsvq.so (through
`_native`), never in Triton and never in a torch fallback. If the library is
missing the GPU calls raise. CPU tensors keep the reference's tiled torch
path, which is what a CPU-resident (offloaded) model runs.
"""
from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
import logging
import os

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native

SUPPORTED_TYPES = {"Q4_0", "Q5_0", "Q8_0", "F16", "F32", "BF16"}
# Bytes of one GGUF block of 32 weights: an FP16 scale followed by the payload
# (reference quantization.py:15).
BLOCK_BYTES = {"Q4_0": 18, "Q5_0": 22, "Q8_0": 34}
_LOG = logging.getLogger(__name__)

# Largest number of activation rows served by the fused GEMV; more rows
# (prefill, vision) take the dequantize + GEMM path.
GEMV_MAX_ROWS = 8
# Rows of a weight matrix dequantized at a time by the GEMM path: bounds its
# fp16 scratch to 64 MiB.
_GEMM_CHUNK_ELEMS = 32 * 1024 * 1024


def type_name(tensor):
    """GGUF tensor type name (reference quantization.py:18-19)."""
    return tensor.tensor_type.name


def tensor_shape(tensor):
    """Row-major shape of a GGUF tensor, whose reader stores it reversed (:21-22)."""
    return tuple(int(x) for x in reversed(tensor.shape))


def tensor_payload(tensor):
    """Owned copy of a GGUF tensor's data; quantized and BF16 data as flat
    bytes (reference quantization.py:24-31)."""
    qtype = type_name(tensor)
    if qtype not in SUPPORTED_TYPES:
        raise ValueError(f"Unsupported GGUF type {qtype}: {tensor.name}")
    data = np.array(tensor.data, copy=True)
    if qtype in BLOCK_BYTES or qtype == "BF16":
        data = data.view(np.uint8).reshape(-1)
    return torch.from_numpy(data)


def _block_values(payload, qtype):
    """Signed integer weights [blocks, 32] (as float32) of CPU block payloads
    [blocks, W] without scales (reference quantization.py:34-47)."""
    if qtype == "Q8_0":
        return payload.contiguous().view(torch.int8).float()
    low = (payload[:, -16:] & 15).to(torch.int32)
    high = (payload[:, -16:] >> 4).to(torch.int32)
    codes = torch.cat((low, high), -1)
    if qtype == "Q4_0":
        return (codes - 8).float()
    # Q5_0: the first four bytes are a little-endian mask whose bit j is the
    # fifth bit of weight j.
    mask = payload[:, :4].to(torch.int64)
    mask = mask[:, 0] | (mask[:, 1] << 8) | (mask[:, 2] << 16) | (mask[:, 3] << 24)
    fifth = (mask[:, None] >> torch.arange(32, dtype=torch.int64)) & 1
    return ((codes | (fifth.to(torch.int32) << 4)) - 16).float()


def _numel(shape):
    n = 1
    for dim in shape:
        n *= dim
    return n


def dequantize(data, qtype, shape, dtype):
    """Dense weights of a GGUF payload (reference quantization.py:50-65).

    Quantized payloads are GGUF AoS blocks `[fp16 d][payload]`; on a GPU they
    are split into the SoA arrays and decoded by the HIP kernel.
    """
    if qtype in ("F16", "F32"):
        return data.reshape(shape).to(dtype)
    if qtype == "BF16":
        return data.reshape(-1).view(torch.bfloat16).reshape(shape).to(dtype)
    if qtype not in BLOCK_BYTES:
        raise ValueError(f"Unsupported GGUF quantization: {qtype}")
    block_bytes = BLOCK_BYTES[qtype]
    n = _numel(shape)
    if n % 32 or data.numel() != n // 32 * block_bytes:
        raise ValueError(f"Invalid {qtype} payload for shape {shape}")
    blocks = data.contiguous().view(torch.uint8).reshape(-1, block_bytes)
    if blocks.device.type == "cuda":
        q = blocks[:, 2:].contiguous().reshape(-1)
        scale_bits = blocks[:, :2].contiguous().reshape(-1)
        return dequantize_soa(q, scale_bits, qtype, shape, dtype)
    scales = blocks[:, :2].contiguous().view(torch.float16).float().reshape(-1, 1)
    return (_block_values(blocks[:, 2:], qtype) * scales).reshape(shape).to(dtype)


def pack_gguf_soa(tensor):
    """Split a GGUF Q4_0/Q5_0/Q8_0 matrix on the CPU into its SoA arrays
    (reference quantization.py:67-90): the block payloads without scales, and
    the fp16 scale bits stored as bytes so that `module.to(dtype)` never
    converts them. Tensors of `gguf_support.GGUFReader` are repacked by the
    library's multithreaded C++ shuffle; other tensor objects by torch."""
    qtype = type_name(tensor)
    shape = tensor_shape(tensor)
    if qtype not in BLOCK_BYTES or len(shape) != 2 or shape[1] % 32:
        raise ValueError(f"Expected rank-2 GGUF Q4_0/Q5_0/Q8_0 matrix: {tensor.name}")
    block_bytes = BLOCK_BYTES[qtype]
    blocks = shape[0] * (shape[1] // 32)
    address = getattr(tensor, "native_address", None)
    if address is not None:
        # A tensor of this package's GGUF reader: the library repacks straight
        # from its file mapping on the host threads (svq_pack_soa).
        if tensor.n_bytes != blocks * block_bytes:
            raise ValueError(f"Invalid packed GGUF payload: {tensor.name}")
        q = torch.empty(blocks * (block_bytes - 2), dtype=torch.uint8)
        scales = torch.empty(blocks * 2, dtype=torch.uint8)
        _native.pack_soa(address, blocks, qtype, q, scales)
        return q, scales
    src = torch.from_numpy(np.asarray(tensor.data).view(np.uint8))
    if src.numel() != blocks * block_bytes:
        raise ValueError(f"Invalid packed GGUF payload: {tensor.name}")
    raw = src.reshape(blocks, block_bytes)
    q = raw[:, 2:].clone(memory_format=torch.contiguous_format).reshape(-1)
    scales = raw[:, :2].clone(memory_format=torch.contiguous_format).reshape(-1)
    return q, scales


def dequantize_soa(qbytes, scale_bits, qtype, shape, dtype):
    """Decode the SoA arrays (reference quantization.py:93-105): each weight is
    the exact fp32 product of its integer code and block scale, then cast to
    `dtype`. GPU tensors are decoded by the HIP kernel."""
    if qtype not in BLOCK_BYTES:
        raise ValueError(f"Unsupported SoA quantization: {qtype}")
    n = _numel(shape)
    width = BLOCK_BYTES[qtype] - 2
    if (n % 32 or qbytes.numel() != (n // 32) * width or
            scale_bits.numel() * scale_bits.element_size() != (n // 32) * 2):
        raise ValueError(f"Invalid SoA payload for shape {shape}")
    if qbytes.device.type == "cuda":
        q = _aligned(qbytes.contiguous().view(torch.uint8).reshape(-1), 16)
        s = scale_bits.contiguous().reshape(-1).view(torch.uint8)
        direct = dtype in _native.DTYPE_CODE
        out = torch.empty(n, dtype=dtype if direct else torch.float32, device=q.device)
        _native.dequant(q, s, out, qtype)
        out = out.reshape(shape)
        return out if direct else out.to(dtype)
    scale = scale_bits.contiguous().view(torch.uint8).view(torch.float16).float().reshape(-1, 1)
    return (_block_values(qbytes.reshape(-1, width), qtype) * scale).reshape(shape).to(dtype)


def _aligned(t, alignment):
    """`t` itself, or an aligned copy when its data pointer is not aligned
    (only views with odd storage offsets)."""
    return t if t.data_ptr() % alignment == 0 else t.clone()


@dataclass(frozen=True)
class PackedSpec:
    qtype: str
    shape: tuple[int, ...]


# Kernel codes of the quantizations (reference quantization.py:120); they are
# also the qtype codes of the C ABI.
_QTYPE_CODE = dict(_native.QTYPE_CODE)
# Launch tuples of the reference's Triton GEMV (quantization.py:121-127), kept
# so that callers indexing them still work. The HIP library picks its own
# launch shape from (qtype, M, N, K); these values are validated, not used.
SOA_GEMV_CONFIG = {
    ("Q4_0", 1): (4, 32, 4), ("Q4_0", 2): (1, 32, 2),
    ("Q5_0", 1): (4, 16, 2), ("Q5_0", 2): (8, 16, 2),
    ("Q8_0", 1): (1, 32, 2), ("Q8_0", 2): (1, 16, 2),
}


def soa_gemv(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor,
             out: torch.Tensor, qtype: str, *, bn: int = 4,
             blocks: int = 16, num_warps: int = 4, bias=None) -> None:
    """GEMV over the SoA layout into `out` (reference quantization.py:232-265).

    Same arguments, checks and messages as the reference; M may be 1..8 rather
    than 1..2. `out` may also be fp32 (same kernel, no final fp16 rounding).
    `bn`, `blocks` and `num_warps` are validated for compatibility and ignored.
    """
    if qtype not in ("Q4_0", "Q5_0", "Q8_0"):
        raise ValueError(f"Unsupported GGUF type: {qtype}")
    if x.ndim != 2 or out.ndim != 2 or not 1 <= x.shape[0] <= GEMV_MAX_ROWS:
        raise ValueError("SOA kernel requires rank-2 input with M=1..8")
    m, k = x.shape
    n = out.shape[1]
    if k <= 0 or k % 32 or n <= 0 or out.shape[0] != m:
        raise ValueError("Invalid matrix dimensions")
    if bn not in (1, 2, 4, 8, 16) or blocks not in (4, 8, 16, 32, 64):
        raise ValueError("Unsupported GEMV tile size")
    if num_warps not in (2, 4, 8):
        raise ValueError("num_warps must be 2, 4 or 8")
    if x.device.type != "cuda" or q.device != x.device or s.device != x.device or out.device != x.device:
        raise ValueError("Expected CUDA tensors on the same device")
    if (x.dtype != torch.float16 or out.dtype not in (torch.float16, torch.float32)
            or q.dtype != torch.uint8 or s.dtype != torch.float16):
        raise ValueError("Expected FP16 input/output/scales and uint8 Q bytes")
    if not (x.is_contiguous() and q.is_contiguous() and s.is_contiguous() and out.is_contiguous()):
        raise ValueError("Expected contiguous tensors")
    if bias is not None and (bias.shape != (n,) or
                             bias.device != x.device or
                             bias.dtype != torch.float16 or
                             not bias.is_contiguous()):
        raise ValueError("SoA GEMV bias must be contiguous FP16 on input device")
    total = n * (k // 32)
    if q.numel() != total * (BLOCK_BYTES[qtype] - 2) or s.numel() != total:
        raise ValueError("Incorrect repacked weight size")
    # Long rows split K across workgroups through a per-stream workspace
    # (svq_gemv_split); during graph capture without one, a single pass.
    workspace = _native.split_workspace(x.device, x.shape[0], n, k, qtype)
    _native.gemv(_aligned(x, 16), _aligned(q, 16), s, out, qtype, bias, workspace)


# Static activation/output pairs of decode graphs (reference
# quantization.py:268-283): the eager warm-up of a step allocates them in call
# order and the capture that follows reuses them, so a captured step reads and
# writes memory that outlives the capture.
_GRAPH_IO = ContextVar("starvector_graph_io", default=None)


@contextmanager
def graph_io(buffers):
    """Warm-up (empty `buffers`) allocates static input/output pairs in call
    order; the graph capture that follows reuses them."""
    token = _GRAPH_IO.set((buffers, not buffers, [0]))
    try:
        yield
    finally:
        _GRAPH_IO.reset(token)


def _soa_gemm(inp, qbytes, scales_u8, spec, bias, out):
    """M > GEMV_MAX_ROWS (prefill, vision): HIP dequantization of row chunks
    to fp16, then an fp16 GEMM with fp32 accumulation (hipBLASLt), i.e. the
    arithmetic of the reference's `_soa_mm` (quantization.py:130-169)."""
    n, k = spec.shape
    width = BLOCK_BYTES[spec.qtype] - 2
    kb = k // 32
    rows = max(1, _GEMM_CHUNK_ELEMS // k)
    for start in range(0, n, rows):
        end = min(start + rows, n)
        w = dequantize_soa(qbytes[start * kb * width:end * kb * width],
                           scales_u8[start * kb * 2:end * kb * 2],
                           spec.qtype, (end - start, k), torch.float16)
        part = F.linear(inp, w, None if bias is None else bias[start:end])
        if end - start == n:
            out.copy_(part)
        else:
            out[:, start:end].copy_(part)
    return out


def _fused_soa_linear(x, qbytes, scale_bits, spec, bias):
    """GPU fp16 dispatch (reference quantization.py:286-323): the fused HIP
    GEMV for up to GEMV_MAX_ROWS rows, dequantize + GEMM beyond. Returns None
    -- the caller then runs the tiled dequantize + F.linear path -- for
    inputs this path does not take (CPU tensors, non-fp16 activations) and
    when the reference's switch STARVECTOR_DISABLE_TRITON is "1" (off by
    default), as the reference does. Unlike the reference, a kernel error
    propagates instead of being logged and answered with that path: a failed
    launch is an invalid argument or a broken device, not a reason to change
    arithmetic silently."""
    if (x.device.type != "cuda" or os.getenv("STARVECTOR_DISABLE_TRITON") == "1" or
            x.dtype != torch.float16 or x.numel() % spec.shape[1]):
        return None
    nrows = x.numel() // spec.shape[1]
    n, k = spec.shape
    inp = x.reshape(nrows, k)
    io = _GRAPH_IO.get()
    if io is None:
        inp = inp.contiguous()
        out = torch.empty((nrows, n), dtype=inp.dtype, device=inp.device)
    else:
        buffers, warmup, calls = io
        if warmup:
            buffers.append((torch.empty((nrows, k), dtype=inp.dtype, device=inp.device),
                            torch.empty((nrows, n), dtype=inp.dtype, device=inp.device)))
        static_in, out = buffers[calls[0]]
        calls[0] += 1
        inp = static_in.copy_(inp)
    scales = scale_bits.view(torch.float16)
    if nrows <= GEMV_MAX_ROWS:
        soa_gemv(inp, qbytes, scales, out, spec.qtype, bias=bias)
    else:
        _soa_gemm(inp, qbytes, scale_bits, spec, bias, out)
    return out.reshape(*x.shape[:-1], n)


class GGUFWeights(nn.Module):
    """Parameters of one GGUF-backed layer (reference quantization.py:326-366)."""

    def __init__(self):
        super().__init__()
        self.register_parameter("weight", None)
        self.register_parameter("weight_scales", None)
        self.register_parameter("bias", None)
        self._specs: dict[str, PackedSpec] = {}

    def set_gguf(self, key, tensor):
        if key not in ("weight", "bias"):
            raise ValueError("Unexpected weight key")
        qtype, shape = type_name(tensor), tensor_shape(tensor)
        payload = tensor_payload(tensor)
        if qtype == "BF16":
            # Converted once, so the model dtype cast applies at load time.
            payload, qtype = dequantize(payload, qtype, shape, torch.float32), "F32"
        self.register_parameter(key, nn.Parameter(payload, requires_grad=False))
        self._specs[key] = PackedSpec(qtype, shape)

    def _set_soa_weight(self, tensor):
        if type_name(tensor) not in BLOCK_BYTES:
            return False
        q, scales = pack_gguf_soa(tensor)
        self.register_parameter("weight", nn.Parameter(q, requires_grad=False))
        self.register_parameter("weight_scales", nn.Parameter(scales, requires_grad=False))
        self._specs["weight"] = PackedSpec(type_name(tensor), tensor_shape(tensor))
        return True

    def set_soa(self, qtype, shape, qbytes, scale_bits):
        """Install already-split SoA arrays (uint8 payload, uint8 scale bits),
        e.g. generated or repacked on the GPU."""
        if qtype not in BLOCK_BYTES or len(shape) != 2 or shape[1] % 32:
            raise ValueError(f"Expected rank-2 Q4_0/Q5_0/Q8_0 shape, got {qtype} {shape}")
        blocks = shape[0] * shape[1] // 32
        if (qbytes.dtype != torch.uint8 or scale_bits.dtype != torch.uint8 or
                qbytes.numel() != blocks * (BLOCK_BYTES[qtype] - 2) or
                scale_bits.numel() != blocks * 2):
            raise ValueError("Invalid SoA arrays")
        self.register_parameter("weight", nn.Parameter(qbytes.reshape(-1), requires_grad=False))
        self.register_parameter("weight_scales", nn.Parameter(scale_bits.reshape(-1), requires_grad=False))
        self._specs["weight"] = PackedSpec(qtype, tuple(int(d) for d in shape))

    def set_dense(self, key, value):
        """Install a floating-point parameter (bias, or an unquantized weight)."""
        self.register_parameter(key, nn.Parameter(value, requires_grad=False))
        self._specs[key] = PackedSpec({torch.float16: "F16"}.get(value.dtype, "F32"),
                                      tuple(value.shape))

    def unpack(self, key, dtype, device):
        data = getattr(self, key)
        if data is None:
            return None
        spec = self._specs[key]
        if key == "weight" and self.weight_scales is not None:
            return dequantize_soa(
                data.to(device=device), self.weight_scales.to(device=device),
                spec.qtype, spec.shape, dtype)
        return dequantize(data.to(device=device), spec.qtype, spec.shape, dtype)


class GGUFLinear(GGUFWeights):
    """Quantized linear layer (reference quantization.py:368-408)."""

    def __init__(self, in_features, out_features):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features

    def set_gguf(self, key, tensor):
        if key == "weight" and self._set_soa_weight(tensor):
            return
        super().set_gguf(key, tensor)

    def forward(self, x):
        spec = self._specs.get("weight")
        if spec is None:
            raise RuntimeError("GGUFLinear missing weight")
        if spec.shape != (self.out_features, self.in_features):
            raise ValueError(f"Unexpected weight shape {spec.shape}")
        bias = self.unpack("bias", x.dtype, x.device)
        if spec.qtype in BLOCK_BYTES:
            fused = _fused_soa_linear(x, self.weight, self.weight_scales, spec, bias)
            if fused is not None:
                return fused
            # Non-fp16 activations, or CPU tensors: dequantize slices of the
            # resident SoA arrays (on a GPU with the HIP kernel) and multiply.
            rows_per_chunk = max(1, 2 * 1024 * 1024 // self.in_features)
            x_flat = x.reshape(-1, self.in_features)
            blocks_per_row = self.in_features // 32
            payload = self.weight.reshape(
                self.out_features, blocks_per_row * (BLOCK_BYTES[spec.qtype] - 2))
            scales = self.weight_scales.reshape(self.out_features, blocks_per_row * 2)
            outputs = []
            for start in range(0, self.out_features, rows_per_chunk):
                end = min(start + rows_per_chunk, self.out_features)
                weights = dequantize_soa(
                    payload[start:end].flatten(), scales[start:end].flatten(),
                    spec.qtype, (end - start, self.in_features), x.dtype)
                outputs.append(F.linear(
                    x_flat, weights, bias[start:end] if bias is not None else None))
            return torch.cat(outputs, -1).reshape(*x.shape[:-1], self.out_features)
        return F.linear(x, self.unpack("weight", x.dtype, x.device), bias)


class GGUFEmbedding(GGUFWeights):
    """Quantized embedding table (reference quantization.py:410-446). On a GPU
    the requested rows are gathered and decoded by one HIP kernel, so
    duplicate ids need no torch.unique and nothing synchronizes."""

    def __init__(self, num_embeddings, embedding_dim):
        super().__init__()
        self.num_embeddings, self.embedding_dim = num_embeddings, embedding_dim
        self.output_dtype = torch.float32

    def set_gguf(self, key, tensor):
        if key == "weight" and self._set_soa_weight(tensor):
            return
        super().set_gguf(key, tensor)

    def forward(self, ids):
        spec = self._specs.get("weight")
        if spec is None:
            raise RuntimeError("GGUFEmbedding missing weight")
        if spec.qtype in ("F16", "F32", "BF16"):
            return F.embedding(ids, self.unpack("weight", self.output_dtype, ids.device))
        if spec.shape[-1] % 32:
            raise ValueError("GGUF embedding hidden dimension must be divisible by 32")
        rows, width = spec.shape
        blocks_per_row = width // 32
        flat_ids = ids.reshape(-1)
        if self.weight.device.type == "cuda":
            direct = self.output_dtype in _native.DTYPE_CODE
            out = torch.empty((flat_ids.numel(), width),
                              dtype=self.output_dtype if direct else torch.float32,
                              device=self.weight.device)
            _native.dequant_rows(self.weight, self.weight_scales,
                                 flat_ids.to(device=self.weight.device, dtype=torch.int64).contiguous(),
                                 rows, width, out, spec.qtype)
            out = out if direct else out.to(self.output_dtype)
            return out.reshape(*ids.shape, width)
        stride = blocks_per_row * (BLOCK_BYTES[spec.qtype] - 2)
        if flat_ids.numel() <= 8:
            selected, inverse = flat_ids, None
        else:
            selected, inverse = torch.unique(flat_ids, return_inverse=True)
        q = self.weight.reshape(rows, stride).index_select(0, selected)
        scales = self.weight_scales.reshape(rows, blocks_per_row * 2).index_select(0, selected)
        decoded = dequantize_soa(q.flatten(), scales.flatten(), spec.qtype,
                                 (selected.numel(), width), self.output_dtype)
        if inverse is not None:
            decoded = decoded.index_select(0, inverse)
        return decoded.reshape(*ids.shape, width)


def tied_head(embedding):
    """Output projection sharing both SoA arrays of its embedding
    (reference quantization.py:448-454)."""
    head = GGUFLinear(embedding.embedding_dim, embedding.num_embeddings)
    head.weight = embedding.weight
    head.weight_scales = embedding.weight_scales
    head._specs["weight"] = embedding._specs["weight"]
    return head


class GGUFConv2d(GGUFWeights):
    """Patch embedding convolution with stride equal to the patch size
    (reference quantization.py:456-465)."""

    def __init__(self, stride):
        super().__init__()
        self.stride = stride

    def forward(self, x):
        return F.conv2d(x, self.unpack("weight", x.dtype, x.device),
                        self.unpack("bias", x.dtype, x.device), stride=self.stride)

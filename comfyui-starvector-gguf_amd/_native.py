"""ctypes binding of libsvq.so, the gfx950 HIP library behind the quantized ops.

Only this module touches the C ABI (include/svq.h). Tensors cross the boundary
as raw device pointers plus sizes, and every call is enqueued on the current
torch stream of the tensors' device, so calls made while a graph is captured
become kernel nodes of that graph. A missing or unloadable library raises
`RuntimeError`: there is no other GPU code path.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libsvq.so")
ABI_VERSION = 1

QTYPE_CODE = {"Q4_0": 4, "Q5_0": 5, "Q8_0": 8}
DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_lib = None
_lock = threading.Lock()


class SVQError(RuntimeError):
    """A libsvq call returned a non-zero status."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed with status {code}: {message}")
        self.code = code


def load() -> ctypes.CDLL:
    """Load libsvq.so once and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; build it with "
                f"`python {LIB_PATH.parent / '_build.py'}`")
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        lib.svq_abi_version.argtypes = []
        lib.svq_abi_version.restype = i32
        lib.svq_last_error.argtypes = []
        lib.svq_last_error.restype = ctypes.c_char_p
        lib.svq_gemv.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]
        lib.svq_gemv.restype = i32
        lib.svq_gemv_plan.argtypes = [i32, i32, i32, i32, ctypes.POINTER(ctypes.c_int32)]
        lib.svq_gemv_plan.restype = i32
        lib.svq_dequant.argtypes = [vp, vp, vp, i64, i32, i32, vp]
        lib.svq_dequant.restype = i32
        lib.svq_dequant_rows.argtypes = [vp, vp, vp, i64, i64, i32, vp, i32, i32, vp]
        lib.svq_dequant_rows.restype = i32
        version = lib.svq_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libsvq ABI {version}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def _check(lib, fn: str, rc: int) -> None:
    if rc != 0:
        raise SVQError(fn, rc, lib.svq_last_error().decode(errors="replace"))


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _on_device:
    """Make `device` current for the launch if it is not already."""

    def __init__(self, device: torch.device):
        self.device = device
        self.ctx = None

    def __enter__(self):
        if self.device.index is not None and self.device.index != torch.cuda.current_device():
            self.ctx = torch.cuda.device(self.device)
            self.ctx.__enter__()

    def __exit__(self, *exc):
        if self.ctx is not None:
            self.ctx.__exit__(*exc)


def gemv(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor, y: torch.Tensor,
         qtype: str, bias: torch.Tensor | None = None) -> None:
    """y[m, n] = x[m, k] @ W[n, k]^T (+ bias); all tensors contiguous on one GPU."""
    lib = load()
    m, k = x.shape
    n = y.shape[1]
    with _on_device(x.device):
        rc = lib.svq_gemv(x.data_ptr(), q.data_ptr(), s.data_ptr(),
                          None if bias is None else bias.data_ptr(), y.data_ptr(),
                          m, n, k, QTYPE_CODE[qtype], DTYPE_CODE[y.dtype],
                          _stream(x.device))
    _check(lib, "svq_gemv", rc)


PLAN_FIELDS = ("kernel", "lg_g", "rows", "waves_per_group", "waves", "groups",
               "wave_capacity", "chunk_units")


def gemv_plan(m: int, n: int, k: int, qtype: str) -> dict:
    """The launch svq_gemv would make for this shape on the current device."""
    lib = load()
    out = (ctypes.c_int32 * 8)()
    _check(lib, "svq_gemv_plan", lib.svq_gemv_plan(m, n, k, QTYPE_CODE[qtype], out))
    plan = dict(zip(PLAN_FIELDS, list(out)))
    plan["kernel"] = {1: "stream", 2: "chunked", 3: "mfma", 4: "mfma4"}[plan["kernel"]]
    return plan


def dequant(q: torch.Tensor, s: torch.Tensor, out: torch.Tensor, qtype: str) -> None:
    """out (flat, fp32/fp16/bf16) = every weight of the SoA arrays q, s."""
    lib = load()
    nblocks = s.numel() * s.element_size() // 2
    with _on_device(q.device):
        rc = lib.svq_dequant(q.data_ptr(), s.data_ptr(), out.data_ptr(), nblocks,
                             QTYPE_CODE[qtype], DTYPE_CODE[out.dtype], _stream(q.device))
    _check(lib, "svq_dequant", rc)


def dequant_rows(q: torch.Tensor, s: torch.Tensor, ids: torch.Tensor, nrows: int,
                 k: int, out: torch.Tensor, qtype: str) -> None:
    """out[i, :] = dequantized row ids[i] of an nrows x k SoA matrix."""
    lib = load()
    with _on_device(q.device):
        rc = lib.svq_dequant_rows(q.data_ptr(), s.data_ptr(), ids.data_ptr(),
                                  ids.numel(), nrows, k, out.data_ptr(),
                                  QTYPE_CODE[qtype], DTYPE_CODE[out.dtype],
                                  _stream(q.device))
    _check(lib, "svq_dequant_rows", rc)

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
ABI_VERSION = 3

QTYPE_CODE = {"Q4_0": 4, "Q5_0": 5, "Q8_0": 8}
DTYPE_CODE = {torch.float16: 0, torch.float32: 1, torch.bfloat16: 2}

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
        lib.svq_gemv_fused.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, vp,
                                       ctypes.c_float, vp, i32, vp]
        lib.svq_gemv_fused.restype = i32
        lib.svq_gemv_plan.argtypes = [i32, i32, i32, i32, ctypes.POINTER(ctypes.c_int32)]
        lib.svq_gemv_plan.restype = i32
        lib.svq_dequant.argtypes = [vp, vp, vp, i64, i32, i32, vp]
        lib.svq_dequant.restype = i32
        lib.svq_dequant_rows.argtypes = [vp, vp, vp, i64, i64, i32, vp, i32, i32, vp]
        lib.svq_dequant_rows.restype = i32
        lib.svq_decode_attention_workspace.argtypes = [i32, i32, i32, i32]
        lib.svq_decode_attention_workspace.restype = i64
        lib.svq_decode_attention.argtypes = [vp, i64, vp, vp, vp, vp, i64, vp, vp, i32, i32,
                                             vp, i32, i32, i32, i32, ctypes.c_float, vp, i64,
                                             vp]
        lib.svq_decode_attention.restype = i32
        lib.svq_gemv_split.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32, vp,
                                       i64, vp]
        lib.svq_gemv_split.restype = i32
        lib.svq_gemv_split_workspace.argtypes = [i32, i32, i32, i32]
        lib.svq_gemv_split_workspace.restype = i64
        lib.svq_cache_reorder.argtypes = [vp, i64, i32, i32, i64, i32, i64, vp, vp]
        lib.svq_cache_reorder.restype = i32
        lib.svq_beam_select.argtypes = [vp, vp, vp, vp, i32, i64, i32, i32, vp, vp, i64, vp, vp,
                                        vp, vp, i32, vp]
        lib.svq_beam_select.restype = i32
        f32 = ctypes.c_float
        lib.svq_beam_candidates.argtypes = [vp, vp, i64, vp, i32, i32, i32, i32, i32, f32, f32,
                                            ctypes.c_double, vp, vp, vp, vp, vp, i64, vp]
        lib.svq_beam_candidates.restype = i32
        lib.svq_beam_candidates_workspace.argtypes = [i32, i32, i32]
        lib.svq_beam_candidates_workspace.restype = i64
        cp = ctypes.c_char_p
        lib.svq_gguf_open.argtypes = [cp, i32, ctypes.POINTER(vp)]
        lib.svq_gguf_open.restype = i32
        lib.svq_gguf_close.argtypes = [vp]
        lib.svq_gguf_close.restype = None
        lib.svq_gguf_version.argtypes = [vp]
        lib.svq_gguf_version.restype = i32
        lib.svq_gguf_alignment.argtypes = [vp]
        lib.svq_gguf_alignment.restype = i64
        lib.svq_gguf_kv_count.argtypes = [vp]
        lib.svq_gguf_kv_count.restype = i64
        lib.svq_gguf_find_kv.argtypes = [vp, cp]
        lib.svq_gguf_find_kv.restype = i64
        lib.svq_gguf_kv.argtypes = [vp, i64, ctypes.POINTER(cp), ctypes.POINTER(i32),
                                    ctypes.POINTER(vp), ctypes.POINTER(i64), ctypes.POINTER(i32),
                                    ctypes.POINTER(i64)]
        lib.svq_gguf_kv.restype = i32
        lib.svq_gguf_tensor_count.argtypes = [vp]
        lib.svq_gguf_tensor_count.restype = i64
        lib.svq_gguf_find_tensor.argtypes = [vp, cp]
        lib.svq_gguf_find_tensor.restype = i64
        lib.svq_gguf_tensor.argtypes = [vp, i64, ctypes.POINTER(cp), ctypes.POINTER(i32),
                                        ctypes.POINTER(i32), ctypes.POINTER(i64),
                                        ctypes.POINTER(i64), ctypes.POINTER(i64)]
        lib.svq_gguf_tensor.restype = i32
        lib.svq_gguf_tensor_data.argtypes = [vp, i64]
        lib.svq_gguf_tensor_data.restype = vp
        lib.svq_pack_soa.argtypes = [vp, i64, i32, vp, vp, i32]
        lib.svq_pack_soa.restype = i32
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
         qtype: str, bias: torch.Tensor | None = None,
         workspace: torch.Tensor | None = None) -> None:
    """y[m, n] = x[m, k] @ W[n, k]^T (+ bias); all tensors contiguous on one GPU.
    With a workspace (see split_workspace) and fp16 y, long rows split K
    across workgroups (svq_gemv_split)."""
    lib = load()
    m, k = x.shape
    n = y.shape[1]
    if workspace is not None and y.dtype == torch.float16:
        _split(lib, x, q, s, y, qtype, bias, None, None, workspace)
        return
    with _on_device(x.device):
        rc = lib.svq_gemv(x.data_ptr(), q.data_ptr(), s.data_ptr(),
                          None if bias is None else bias.data_ptr(), y.data_ptr(),
                          m, n, k, QTYPE_CODE[qtype], DTYPE_CODE[y.dtype],
                          _stream(x.device))
    _check(lib, "svq_gemv", rc)


def _split(lib, x, q, s, y, qtype, bias, residual, activation, workspace) -> None:
    if workspace.device != x.device or workspace.dtype != torch.uint8:
        raise ValueError("workspace must be a uint8 tensor on the device of x")
    m, k = x.shape
    n = y.shape[1]
    ptr = lambda t: None if t is None else t.data_ptr()
    with _on_device(x.device):
        rc = lib.svq_gemv_split(x.data_ptr(), q.data_ptr(), s.data_ptr(), ptr(bias),
                                y.data_ptr(), m, n, k, QTYPE_CODE[qtype], ptr(residual),
                                ACTIVATION_CODE[activation], workspace.data_ptr(),
                                workspace.numel(), _stream(x.device))
    _check(lib, "svq_gemv_split", rc)


_split_workspaces: dict = {}
# Workspaces replaced by larger ones. They stay allocated until the process
# ends: a graph captured earlier keeps their addresses in its kernel nodes.
_retired_workspaces: list = []


def gemv_workspace_bytes(m: int, n: int, k: int, qtype: str) -> int:
    """Bytes of workspace svq_gemv_split uses for this shape: the partial sums
    when long rows split K across workgroups, 0 when the shape runs in one
    pass."""
    lib = load()
    need = lib.svq_gemv_split_workspace(m, n, k, QTYPE_CODE[qtype])
    _check(lib, "svq_gemv_split_workspace", min(need, 0))
    return need


def split_workspace(device: torch.device, m: int, n: int, k: int, qtype: str,
                    allocate: bool = True, per_stream: bool = True) -> torch.Tensor | None:
    """A workspace for svq_gemv_split of this shape, cached per (device,
    stream) -- per device with per_stream False, for callers that keep all
    their launches on one stream -- and grown as needed; None when the shape
    runs in one pass, or when the workspace would have to grow while the
    stream is being captured into a graph or `allocate` is False (the call
    then runs in one pass). Calls that share it are ordered by their stream. A workspace that is replaced by a larger one
    is kept allocated, since graphs captured with it still use it."""
    if device.type != "cuda":
        return None
    need = gemv_workspace_bytes(m, n, k, qtype)
    if need == 0:
        return None
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, torch.cuda.current_stream(index).cuda_stream if per_stream else None)
    ws = _split_workspaces.get(key)
    if ws is None or ws.numel() < need:
        if not allocate or torch.cuda.is_current_stream_capturing():
            return None
        if ws is not None:
            _retired_workspaces.append(ws)
        ws = torch.empty(need, dtype=torch.uint8, device=torch.device("cuda", index))
        _split_workspaces[key] = ws
    return ws


ACTIVATION_CODE = {None: 0, "gelu_tanh": 1}


def gemv_fused(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor, y: torch.Tensor,
               qtype: str, bias: torch.Tensor | None = None,
               ln_weight: torch.Tensor | None = None, ln_bias: torch.Tensor | None = None,
               ln_eps: float = 1e-5, residual: torch.Tensor | None = None,
               activation: str | None = None, workspace: torch.Tensor | None = None) -> None:
    """y = residual + act(x' @ W^T + bias), x' = LayerNorm(x) when ln_weight or
    ln_bias is given (svq_gemv_fused); fp16 tensors, contiguous, on one GPU.
    Without a LayerNorm and with a workspace, long rows split K across
    workgroups (svq_gemv_split)."""
    lib = load()
    m, k = x.shape
    n = y.shape[1]
    for name, t in (("ln_weight", ln_weight), ("ln_bias", ln_bias)):
        if t is not None and (t.shape != (k,) or t.dtype != torch.float16 or
                              not t.is_contiguous() or t.device != x.device):
            raise ValueError(f"{name} must be a contiguous float16 [{k}] tensor on {x.device}")
    if residual is not None and (residual.shape != y.shape or residual.dtype != torch.float16
                                 or not residual.is_contiguous() or
                                 residual.device != x.device):
        raise ValueError(f"residual must be a contiguous float16 {tuple(y.shape)} tensor")
    if y.dtype != torch.float16:
        raise ValueError("svq_gemv_fused writes float16")
    if workspace is not None and ln_weight is None and ln_bias is None:
        _split(lib, x, q, s, y, qtype, bias, residual, activation, workspace)
        return
    ptr = lambda t: None if t is None else t.data_ptr()
    with _on_device(x.device):
        rc = lib.svq_gemv_fused(x.data_ptr(), q.data_ptr(), s.data_ptr(), ptr(bias),
                                y.data_ptr(), m, n, k, QTYPE_CODE[qtype], ptr(ln_weight),
                                ptr(ln_bias), ln_eps, ptr(residual),
                                ACTIVATION_CODE[activation], _stream(x.device))
    _check(lib, "svq_gemv_fused", rc)


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


_workspaces: dict = {}


def attention_workspace_bytes(rows: int, heads: int, kv_heads: int, span: int) -> int:
    """Bytes of workspace svq_decode_attention needs for this shape."""
    lib = load()
    need = lib.svq_decode_attention_workspace(rows, heads, kv_heads, span)
    _check(lib, "svq_decode_attention_workspace", min(need, 0))
    return need


def attention_workspace(device: torch.device, rows: int, heads: int, kv_heads: int,
                        span: int) -> torch.Tensor:
    """A workspace for svq_decode_attention, cached per device and grown as
    needed; a replaced one stays allocated (graphs captured with it still use
    it). Calls that share it must be ordered (one stream)."""
    need = attention_workspace_bytes(rows, heads, kv_heads, span)
    key = (device.type, device.index if device.index is not None else torch.cuda.current_device())
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _retired_workspaces.append(ws)
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def decode_attention(qkv: torch.Tensor, cos: torch.Tensor | None, sin: torch.Tensor | None,
                     keys: torch.Tensor, values: torch.Tensor, position: torch.Tensor,
                     bias: torch.Tensor | None, out: torch.Tensor, heads: int, kv_heads: int,
                     scale: float, workspace: torch.Tensor, window: int = 0) -> None:
    """One layer's decode attention (svq_decode_attention). qkv [rows, >= (heads +
    2 kv_heads) * 128] fp16 with unit stride in its last dim; keys/values the
    layer's cache or a slot-prefix view of it, [rows, kv_heads, span, 128];
    position a device int64 scalar; out [rows, heads * 128]; window > 0 masks
    the slots outside (position - window, position]."""
    lib = load()
    if keys.dim() != 4 or values.shape != keys.shape or values.stride() != keys.stride():
        raise ValueError("keys and values must be [rows, kv_heads, span, head_dim] views "
                         "of the same layout")
    rows, span, head_dim = keys.shape[0], keys.shape[2], keys.shape[3]
    st = keys.stride()
    if st[3] != 1 or st[2] != head_dim or st[1] % head_dim or st[0] != kv_heads * st[1]:
        raise ValueError("keys/values must be slot-prefix views of a contiguous "
                         "[rows, kv_heads, capacity, head_dim] cache")
    capacity = st[1] // head_dim
    if qkv.dim() != 2 or qkv.stride(1) != 1 or qkv.shape[0] != rows:
        raise ValueError("qkv must be [rows, width] with unit stride in its last dim")
    if not out.is_contiguous() or out.numel() != rows * heads * head_dim:
        raise ValueError("out must be a contiguous [rows, heads * head_dim] tensor")
    for name, t in (("cos", cos), ("sin", sin), ("bias", bias)):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if position.dtype != torch.int64 or position.numel() != 1:
        raise ValueError("position must be a one-element int64 tensor")
    tensors = [qkv, keys, values, out, position] + [t for t in (cos, sin, bias) if t is not None]
    if any(t.dtype != torch.float16 for t in tensors if t is not position):
        raise ValueError("qkv, keys, values, out, cos, sin and bias must be float16")
    if any(t.device != qkv.device for t in tensors + [workspace]):
        raise ValueError("all tensors must be on one device")
    with _on_device(qkv.device):
        rc = lib.svq_decode_attention(
            qkv.data_ptr(), qkv.stride(0), None if cos is None else cos.data_ptr(),
            None if sin is None else sin.data_ptr(), keys.data_ptr(), values.data_ptr(),
            capacity, position.data_ptr(), None if bias is None else bias.data_ptr(),
            int(window), span, out.data_ptr(), rows, heads, kv_heads, head_dim, scale,
            workspace.data_ptr(),
            workspace.numel(), _stream(qkv.device))
    _check(lib, "svq_decode_attention", rc)


def cache_reorder(cache: torch.Tensor, parents: torch.Tensor, length: int) -> None:
    """Beam reorder of a contiguous fp16 cache [planes, rows, heads, capacity,
    128] (svq_cache_reorder): row r takes the first `length` slots of row
    parents[r] (a device int64 [rows] tensor) wherever the two differ."""
    lib = load()
    if cache.dim() != 5 or not cache.is_contiguous() or cache.dtype != torch.float16:
        raise ValueError("cache must be a contiguous float16 [planes, rows, heads, capacity, "
                         "head_dim] tensor")
    planes, rows, heads, capacity, head_dim = cache.shape
    if parents.dtype != torch.int64 or parents.shape != (rows,) or not parents.is_contiguous():
        raise ValueError("parents must be a contiguous int64 tensor of one entry per row")
    if parents.device != cache.device:
        raise ValueError("cache and parents must be on one device")
    with _on_device(cache.device):
        rc = lib.svq_cache_reorder(cache.data_ptr(), planes, rows, heads, capacity, head_dim,
                                   int(length), parents.data_ptr(), _stream(cache.device))
    _check(lib, "svq_cache_reorder", rc)


def beam_select(probs, noise, scores, candidates, draws, seen_in, seen_out, running, parents,
                tokens, tokens_copy=None) -> None:
    """Survivor selection of a beam-sampling step (svq_beam_select) on the
    device, asynchronously: `draws` multinomial draws without replacement
    from probs (the exponential race with the given Exp(1) noise, over the
    candidate token ids [beams, ncand] only), the first `beams` of them by
    score (descending, stable), their parents and tokens, running scores, and
    seen rows seen_out[b] = seen_in[parent b] with token b set. noise is
    float32 with beams * vocab entries; probs and scores have as many, or one
    per candidate (`beam_candidates`' outputs); seen_in / seen_out are
    distinct bool [beams, pitch] buffers, pitch >= vocab a multiple of 16."""
    lib = load()
    beams, ncand = candidates.shape
    compact = probs.numel() == candidates.numel()
    vocab = noise.numel() // beams
    tensors = (probs, noise, scores, candidates, seen_in, seen_out, running, parents, tokens) + (
        (tokens_copy,) if tokens_copy is not None else ())
    if any(not t.is_contiguous() or t.device != probs.device for t in tensors):
        raise ValueError("beam_select tensors must be contiguous and on one device")
    if any(t.dtype != torch.float32 for t in (probs, noise, scores, running)):
        raise ValueError("probs, noise, scores and running must be float32")
    if any(t.dtype != torch.int64 for t in tensors[7:] + (candidates,)):
        raise ValueError("candidates, parents and tokens must be int64")
    if seen_in.dtype != torch.bool or seen_out.dtype != torch.bool or seen_in.dim() != 2:
        raise ValueError("seen_in and seen_out must be bool [beams, pitch]")
    if noise.numel() % beams or scores.numel() != probs.numel() or (
            not compact and probs.numel() != noise.numel()):
        raise ValueError("noise must hold beams * vocab entries, probs and scores as many or "
                         "one per candidate")
    if seen_out.shape != seen_in.shape or seen_in.shape[0] != beams:
        raise ValueError("seen_in and seen_out must be [beams, pitch]")
    if any(t.numel() != beams for t in (running, parents, tokens)):
        raise ValueError("running, parents and tokens must hold one entry per beam")
    with _on_device(probs.device):
        rc = lib.svq_beam_select(
            probs.data_ptr(), noise.data_ptr(), scores.data_ptr(), candidates.data_ptr(), beams,
            vocab, ncand, int(draws), seen_in.data_ptr(), seen_out.data_ptr(),
            seen_in.shape[1], running.data_ptr(), parents.data_ptr(), tokens.data_ptr(),
            tokens_copy.data_ptr() if tokens_copy is not None else None, int(compact),
            _stream(probs.device))
    _check(lib, "svq_beam_select", rc)


def beam_candidates_workspace(beams: int, vocab: int, kc: int, device) -> torch.Tensor:
    """A workspace for `beam_candidates` (uint8, written and read within a call)."""
    lib = load()
    need = lib.svq_beam_candidates_workspace(beams, vocab, kc)
    _check(lib, "svq_beam_candidates_workspace", min(need, 0))
    return torch.empty(need, dtype=torch.uint8, device=device)


def beam_candidates(logits, seen, running, k, kc, keep, penalty, temperature, top_p,
                    candidates, scores, probs, status, workspace) -> None:
    """Candidates of a beam-sampling step (svq_beam_candidates) on the
    device, asynchronously: from fp16 logits [beams, vocab], the seen rows
    (bool [beams, pitch]) and running scores, each row's kc largest warped
    log-probabilities (token ids into `candidates` [beams, kc] int64, value +
    running score into `scores` [beams, kc] float32), their joint softmax
    (`probs`, float32 [beams * kc]) and `status` (int64 [2 + beams]: number
    of non-zero probs, overflow flag, flag per row)."""
    lib = load()
    beams, vocab = logits.shape
    tensors = (logits, seen, running, candidates, scores, probs, status, workspace)
    if any(not t.is_contiguous() or t.device != logits.device for t in tensors):
        raise ValueError("beam_candidates tensors must be contiguous and on one device")
    if logits.dtype != torch.float16 or seen.dtype != torch.bool or seen.dim() != 2 or \
            seen.shape[0] != beams:
        raise ValueError("logits must be float16 [beams, vocab] and seen bool [beams, pitch]")
    if candidates.dtype != torch.int64 or status.dtype != torch.int64 or any(
            t.dtype != torch.float32 for t in (running, scores, probs)):
        raise ValueError("candidates and status must be int64; running, scores and probs float32")
    if candidates.shape != (beams, kc) or scores.numel() != beams * kc or \
            probs.numel() != beams * kc or status.numel() != 2 + beams or running.numel() != beams:
        raise ValueError("output shapes do not match beams and kc")
    with _on_device(logits.device):
        rc = lib.svq_beam_candidates(
            logits.data_ptr(), seen.data_ptr(), seen.shape[1], running.data_ptr(), beams, vocab,
            int(k), int(kc), int(keep), float(penalty), float(temperature), float(top_p),
            candidates.data_ptr(), scores.data_ptr(), probs.data_ptr(), status.data_ptr(),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(),
            _stream(logits.device))
    _check(lib, "svq_beam_candidates", rc)


def pack_soa(aos_ptr: int, nblocks: int, qtype: str, q: torch.Tensor, s: torch.Tensor,
             threads: int = 0) -> None:
    """Host AoS blocks at aos_ptr -> SoA payload q and scale bytes s (uint8 CPU
    tensors of nblocks * W and nblocks * 2 bytes), on `threads` host threads."""
    lib = load()
    _check(lib, "svq_pack_soa", lib.svq_pack_soa(aos_ptr, nblocks, QTYPE_CODE[qtype],
                                                  q.data_ptr(), s.data_ptr(), threads))


class GGUFFile:
    """A GGUF file opened by the library's reader (svq_gguf_*): metadata and
    tensor infos, parsed and bounds-checked in C++. Closed on close() or when
    garbage collected."""

    def __init__(self, path: str, writable_copy: bool = False):
        self._lib = load()
        handle = ctypes.c_void_p()
        rc = self._lib.svq_gguf_open(str(path).encode(), int(writable_copy), ctypes.byref(handle))
        _check(self._lib, "svq_gguf_open", rc)
        self._h = handle

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.svq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def version(self) -> int:
        return self._lib.svq_gguf_version(self._h)

    @property
    def alignment(self) -> int:
        return self._lib.svq_gguf_alignment(self._h)

    def kv_count(self) -> int:
        return self._lib.svq_gguf_kv_count(self._h)

    def kv(self, i: int):
        """(key, type, address, nbytes, element type, count) of metadata entry i."""
        key, typ, val = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_void_p()
        nbytes, et, count = ctypes.c_int64(), ctypes.c_int(), ctypes.c_int64()
        _check(self._lib, "svq_gguf_kv", self._lib.svq_gguf_kv(
            self._h, i, ctypes.byref(key), ctypes.byref(typ), ctypes.byref(val),
            ctypes.byref(nbytes), ctypes.byref(et), ctypes.byref(count)))
        return (key.value.decode("utf-8", errors="replace"), typ.value, val.value or 0,
                nbytes.value, et.value, count.value)

    def find_kv(self, key: str) -> int:
        return self._lib.svq_gguf_find_kv(self._h, key.encode())

    def tensor_count(self) -> int:
        return self._lib.svq_gguf_tensor_count(self._h)

    def tensor(self, i: int):
        """(name, ggml type, dims in file order, file offset, nbytes) of tensor i."""
        name, typ, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        dims = (ctypes.c_int64 * 4)()
        off, nbytes = ctypes.c_int64(), ctypes.c_int64()
        _check(self._lib, "svq_gguf_tensor", self._lib.svq_gguf_tensor(
            self._h, i, ctypes.byref(name), ctypes.byref(typ), ctypes.byref(nd), dims,
            ctypes.byref(off), ctypes.byref(nbytes)))
        return (name.value.decode("utf-8", errors="replace"), typ.value,
                tuple(dims[: nd.value]), off.value, nbytes.value)

    def tensor_address(self, i: int) -> int:
        return self._lib.svq_gguf_tensor_data(self._h, i) or 0

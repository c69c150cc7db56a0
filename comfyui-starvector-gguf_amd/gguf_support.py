"""Local GGUF discovery and structural validation for StarVector.

Mirrors the reference's gguf_support.py (same names, arguments, results and
error messages) with one change: the file is opened by this package's own
reader (`GGUFReader` below: the C++ reader in libsvq.so, svq_gguf_*) instead
of the PyPI `gguf` package, which the reference needs installed
(gguf_support.py:101-121).

`GGUFReader` offers the part of PyPI gguf's reader interface that the
reference uses: `.tensors` (objects with `name`, `tensor_type` whose `.name`
is the ggml type name, `shape` in file order, `data` as a NumPy view of the
mapping) and `get_field(key).contents()`.
"""
from __future__ import annotations

import ctypes
import enum
import json
import mmap
from dataclasses import dataclass, field
from pathlib import Path
from typing import Iterable

import numpy as np

from . import _native

# Tensor-name prefix of each StarVector part; a file must hold all three.
REQUIRED_COMPONENTS = {
    "vision": "model.image_encoder.",
    "adapter": "model.image_projection.",
    "decoder": "model.svg_transformer.transformer.",
}
# Embedded files read back from the metadata: the tokenizer and its config
# (the EOS token). Anything else embedded is left alone.
EMBEDDED_TOKENIZER_FILES = ("tokenizer.json", "tokenizer_config.json")
EMBEDDED_ASSET_PREFIX = "starvector.embedded_file."
MAX_EMBEDDED_ASSET_BYTES = 16 * 1024 * 1024


class GGMLQuantizationType(enum.IntEnum):
    """ggml tensor type codes of the GGUF format (the names PyPI gguf uses)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    BF16 = 30


class GGUFValueType(enum.IntEnum):
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


_SCALAR = {
    GGUFValueType.UINT8: np.uint8, GGUFValueType.INT8: np.int8,
    GGUFValueType.UINT16: np.uint16, GGUFValueType.INT16: np.int16,
    GGUFValueType.UINT32: np.uint32, GGUFValueType.INT32: np.int32,
    GGUFValueType.FLOAT32: np.float32, GGUFValueType.BOOL: np.bool_,
    GGUFValueType.UINT64: np.uint64, GGUFValueType.INT64: np.int64,
    GGUFValueType.FLOAT64: np.float64,
}
# NumPy element type of tensor data; packed types are exposed as bytes.
_TENSOR_DTYPE = {
    GGMLQuantizationType.F32: np.float32, GGMLQuantizationType.F16: np.float16,
    GGMLQuantizationType.F64: np.float64, GGMLQuantizationType.I8: np.int8,
    GGMLQuantizationType.I16: np.int16, GGMLQuantizationType.I32: np.int32,
    GGMLQuantizationType.I64: np.int64,
}


class ReaderField:
    """One metadata entry; `contents()` is its Python value (str, int, float,
    bool, or a list for arrays)."""

    def __init__(self, name, value_type, contents):
        self.name = name
        self.types = [GGUFValueType(value_type)]
        self._contents = contents

    def contents(self):
        return self._contents


class ReaderTensor:
    """One tensor of a GGUF file; `data` is a view of the file mapping, valid
    while its reader is alive (the tensor keeps a reference to it)."""

    def __init__(self, reader, index, name, tensor_type, dims, offset, nbytes):
        self._reader = reader
        self.index = index
        self.name = name
        self.tensor_type = GGMLQuantizationType(tensor_type)
        self.shape = np.array(dims, dtype=np.uint64)  # file order: dims[0] varies fastest
        self.n_elements = int(np.prod(dims))
        self.n_bytes = nbytes
        self.data_offset = offset

    @property
    def data(self) -> np.ndarray:
        dtype = _TENSOR_DTYPE.get(self.tensor_type)
        buf = self._reader._mm
        if dtype is None:  # block-packed and BF16 data: raw bytes
            return np.frombuffer(buf, dtype=np.uint8, count=self.n_bytes, offset=self.data_offset)
        return np.frombuffer(buf, dtype=dtype, count=self.n_elements,
                             offset=self.data_offset).reshape(tuple(int(d) for d in self.shape[::-1]))

    @property
    def native_address(self) -> int:
        """Address of the data in the library reader's own mapping."""
        return self._reader._native.tensor_address(self.index)


class GGUFReader:
    """GGUF file reader backed by libsvq.so. mode "r" maps the file read-only,
    "c" copy-on-write (writes stay in memory), as PyPI gguf's reader modes."""

    def __init__(self, path, mode: str = "r"):
        if mode not in ("r", "c"):
            raise ValueError(f"unsupported mode {mode!r}")
        self.path = Path(path)
        self._native = _native.GGUFFile(str(self.path), writable_copy=mode == "c")
        with open(self.path, "rb") as f:
            access = mmap.ACCESS_COPY if mode == "c" else mmap.ACCESS_READ
            self._mm = mmap.mmap(f.fileno(), 0, access=access)
        self.fields = {}
        for i in range(self._native.kv_count()):
            key, typ, addr, nbytes, elem, count = self._native.kv(i)
            self.fields[key] = ReaderField(key, typ, self._decode(typ, addr, nbytes, elem, count))
        self.tensors = [ReaderTensor(self, i, *self._native.tensor(i))
                        for i in range(self._native.tensor_count())]

    def get_field(self, key: str):
        return self.fields.get(key)

    def get_tensor(self, index: int) -> ReaderTensor:
        return self.tensors[index]

    def _bytes(self, addr: int, nbytes: int) -> bytes:
        return ctypes.string_at(addr, nbytes) if nbytes else b""

    def _decode(self, typ, addr, nbytes, elem, count):
        raw = self._bytes(addr, nbytes)
        typ = GGUFValueType(typ)
        if typ == GGUFValueType.STRING:
            try:
                return raw.decode("utf-8")
            except UnicodeDecodeError:
                return raw  # callers report undecodable text themselves
        if typ != GGUFValueType.ARRAY:
            value = np.frombuffer(raw, dtype=_SCALAR[typ], count=1)[0]
            return value.item()
        return _decode_array(raw, GGUFValueType(elem), count)


def _decode_array(raw: bytes, elem: GGUFValueType, count: int):
    """Elements of an array value (lengths already validated by the reader).
    Arrays of arrays are not decoded: their contents are None."""
    if elem in _SCALAR:
        return np.frombuffer(raw, dtype=_SCALAR[elem], count=count).tolist()
    if elem != GGUFValueType.STRING:
        return None
    out, pos = [], 0
    for _ in range(count):
        n = int.from_bytes(raw[pos:pos + 8], "little")
        text = raw[pos + 8:pos + 8 + n]
        try:
            out.append(text.decode("utf-8"))
        except UnicodeDecodeError:
            out.append(text)
        pos += 8 + n
    return out


@dataclass(frozen=True)
class GGUFReference:
    """What `inspect_local_gguf` hands the loader: the checked file's path,
    its tensors keyed by name (views of the file mapping), the model config
    it carries and the tokenizer files it carries (names of the reference's
    result type, gguf_support.py:19-26)."""

    path: Path
    tensor_index: dict = field(repr=False)
    model_config: dict = field(repr=False)
    model_assets: dict[str, str] = field(repr=False)


def inspect_tensor_index(tensors: Iterable) -> int:
    """Number of tensors in the file, after checking that each StarVector part
    (vision encoder, adapter, decoder) owns at least one of them by its name
    prefix. The error text is the reference's (gguf_support.py:29-47)."""
    names = [tensor.name for tensor in tensors]
    absent = [part for part, prefix in REQUIRED_COMPONENTS.items()
              if not any(name.startswith(prefix) for name in names)]
    if absent:
        raise ValueError("This is not a full StarVector GGUF pack: missing tensor groups "
                         f"{', '.join(absent)}. A GGUF containing only an LLM or a diffusion "
                         "UNet is unsupported.")
    return len(names)


def _metadata_text(reader, key):
    """A string metadata entry's contents (str, or bytes the caller decodes),
    or None when the file has no such key."""
    entry = reader.get_field(key)
    return None if entry is None else entry.contents()


def read_embedded_config(reader) -> dict:
    """The model config JSON object the exporter stores under
    starvector.config_json, parsed; the reference's errors for a missing,
    non-string, non-JSON or non-object entry (gguf_support.py:50-67)."""
    raw = _metadata_text(reader, "starvector.config_json")
    if raw is None:
        raise ValueError("This StarVector GGUF has no starvector.config_json metadata. "
                         "The model architecture cannot be constructed from this export.")
    text = raw.decode("utf-8") if isinstance(raw, bytes) else raw
    if not isinstance(text, str):
        raise ValueError("starvector.config_json must be a JSON string")
    try:
        config = json.loads(text)
    except json.JSONDecodeError as exc:
        raise ValueError("Invalid JSON in GGUF starvector.config_json") from exc
    if not isinstance(config, dict):
        raise ValueError("GGUF starvector.config_json must contain a JSON object")
    return config


def read_embedded_assets(reader) -> dict[str, str]:
    """The tokenizer files stored under starvector.embedded_file.<name>, as
    text: each must be UTF-8, non-empty and at most 16 MiB, and
    tokenizer.json must be present (the reference's checks and messages,
    gguf_support.py:70-95)."""
    assets = {}
    for filename in EMBEDDED_TOKENIZER_FILES:
        contents = _metadata_text(reader, EMBEDDED_ASSET_PREFIX + filename)
        if contents is None:
            continue
        if isinstance(contents, bytes):
            try:
                contents = contents.decode("utf-8")
            except UnicodeDecodeError as exc:
                raise ValueError(
                    f"Invalid StarVector GGUF: embedded {filename} is not UTF-8") from exc
        if not isinstance(contents, str):
            raise ValueError(f"Invalid StarVector GGUF: embedded {filename} is not a string")
        size = len(contents.encode("utf-8"))
        if size == 0 or size > MAX_EMBEDDED_ASSET_BYTES:
            raise ValueError(
                f"Invalid StarVector GGUF: embedded {filename} is empty or too large")
        assets[filename] = contents
    if "tokenizer.json" not in assets:
        raise ValueError("Invalid StarVector GGUF: embedded tokenizer metadata is missing "
                         "(expected starvector.embedded_file.tokenizer.json)")
    return assets


def inspect_local_gguf(path: Path) -> GGUFReference:
    """Open a local .gguf with this package's reader and check it is a whole
    StarVector export: config, tokenizer, every model part, unique tensor
    names (gguf_support.py:98-121, without the PyPI `gguf` dependency)."""
    path = Path(path).resolve(strict=True)
    if not path.is_file() or path.suffix.lower() != ".gguf":
        raise ValueError("Expected a local .gguf file")
    # Mode "c" maps the file copy-on-write: tensors built on the mapping are
    # writable, and writes never reach the file.
    reader = GGUFReader(str(path), "c")
    config = read_embedded_config(reader)
    assets = read_embedded_assets(reader)
    count = inspect_tensor_index(reader.tensors)
    tensor_index = {tensor.name: tensor for tensor in reader.tensors}
    if len(tensor_index) != count:
        raise ValueError("Duplicate tensor names in GGUF checkpoint")
    return GGUFReference(path=path, tensor_index=tensor_index, model_config=config,
                         model_assets=assets)

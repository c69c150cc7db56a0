"""Fakes shared by the tests, mirroring the reference's tests/package_alias.py:
GGUF tensor type ids (ggml's numbering) and GGUF tensors as the reader
returns them, with the shape stored reversed."""
from enum import Enum
from types import SimpleNamespace


class GGUFType(Enum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q5_0 = 6
    Q8_0 = 8


def fake_tensor(name, data=None, tensor_type=GGUFType.F32, shape=None):
    """GGUF tensor as the reader returns it: `shape` (default data.shape) reversed."""
    if shape is None:
        shape = () if data is None else data.shape
    return SimpleNamespace(name=name, tensor_type=tensor_type,
                           shape=tuple(reversed(shape)), data=data)

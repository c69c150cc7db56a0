"""The GGUF container reader (svq_gguf_*, gguf_support.GGUFReader) and the
C++ AoS -> SoA repack, on the CPU.

* Files written by tests/gguf_writer.py (every metadata value type, the
  tensor types StarVector packs hold, custom alignment) read back exactly:
  metadata values, tensor names, types, shapes in file order, data bytes.
* Malformed files (bad magic or version, truncation at every point, data past
  the end, misaligned data, unknown tensor types, absurd counts) fail with
  SVQ_E_FORMAT / SVQ_E_DTYPE / SVQ_E_IO, never with a crash.
* The repack is bit-exact with the oracle's `pack_soa` (the reference's
  `pack_gguf_soa`, quantization.py:67-90) and with the torch path it replaces.
* The reference's own gguf_support tests (tests/test_gguf_support.py: fake
  readers for the config, tokenizer and component checks) are restated
  against this package's gguf_support, plus the same checks on a real file.
"""
from __future__ import annotations

import json
import struct
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import starvector_amd._native as native
import starvector_amd.gguf_support as gs
import starvector_amd.quantization as quantization
from gguf_writer import ARRAY, GGML, STRING, gguf_bytes
from oracle import soa_oracle as orc

BB = {"Q4_0": 18, "Q5_0": 22, "Q8_0": 34}


def random_blocks(qtype, n, k, seed):
    """Seeded AoS payload of an n x k matrix (scales: valid fp16 numbers)."""
    return orc.packed_matrix(qtype, n, k, seed=seed).tobytes()


def sample_file(tmp_path, alignment=32, extra_kvs=(), name="model.gguf"):
    rng = np.random.default_rng(5)
    f32 = rng.standard_normal((3, 64)).astype(np.float32)
    f16 = rng.standard_normal(64).astype(np.float16)
    bf16 = rng.integers(0, 65535, 128, dtype=np.uint16)
    tensors = [
        ("model.image_encoder.conv.weight", GGML["F32"], (64, 3), f32.tobytes()),
        ("model.image_projection.c_fc.weight", GGML["Q4_0"], (64, 5), random_blocks("Q4_0", 5, 64, 1)),
        ("model.svg_transformer.transformer.wte.weight", GGML["Q8_0"], (96, 7),
         random_blocks("Q8_0", 7, 96, 2)),
        ("model.svg_transformer.transformer.h.0.c_fc.weight", GGML["Q5_0"], (32, 9),
         random_blocks("Q5_0", 9, 32, 3)),
        ("model.svg_transformer.transformer.h.0.ln.bias", GGML["F16"], (64,), f16.tobytes()),
        ("model.svg_transformer.transformer.h.0.bf", GGML["BF16"], (128,), bf16.tobytes()),
    ]
    kvs = [
        ("general.architecture", STRING, "starvector"),
        ("general.alignment", 4, alignment),
        ("starvector.config_json", STRING, json.dumps({"hidden_size": 2048, "n": [1, 2]})),
        ("starvector.embedded_file.tokenizer.json", STRING, '{"model":{"type":"BPE"}}'),
        ("t.u8", 0, 200), ("t.i8", 1, -5), ("t.u16", 2, 60000), ("t.i16", 3, -300),
        ("t.i32", 5, -70000), ("t.f32", 6, 1.5), ("t.bool", 7, True), ("t.u64", 10, 1 << 40),
        ("t.i64", 11, -(1 << 40)), ("t.f64", 12, 0.125),
        ("t.arr_i32", ARRAY, [1, -2, 3], 5), ("t.arr_str", ARRAY, ["a", "bc", ""], STRING),
        ("t.empty", ARRAY, [], 4),
        *extra_kvs,
    ]
    path = tmp_path / name
    path.write_bytes(gguf_bytes(kvs, tensors, alignment=alignment))
    return path, {t[0]: t for t in tensors}


@pytest.mark.parametrize("alignment", (32, 64, 256))
def test_round_trip(tmp_path, alignment):
    path, tensors = sample_file(tmp_path, alignment)
    reader = gs.GGUFReader(path)
    assert reader._native.version == 3 and reader._native.alignment == alignment
    want = {"general.architecture": "starvector", "t.u8": 200, "t.i8": -5, "t.u16": 60000,
            "t.i16": -300, "t.i32": -70000, "t.f32": 1.5, "t.bool": True, "t.u64": 1 << 40,
            "t.i64": -(1 << 40), "t.f64": 0.125, "t.arr_i32": [1, -2, 3],
            "t.arr_str": ["a", "bc", ""], "t.empty": [], "general.alignment": alignment}
    for key, value in want.items():
        assert reader.get_field(key).contents() == value, key
    assert reader.get_field("missing") is None
    assert [t.name for t in reader.tensors] == list(tensors)
    for t in reader.tensors:
        name, gtype, dims, data = tensors[t.name]
        assert int(t.tensor_type) == gtype
        assert tuple(int(d) for d in t.shape) == dims
        assert quantization.tensor_shape(t) == tuple(reversed(dims))
        assert t.data_offset % alignment == 0
        assert np.asarray(t.data).view(np.uint8).tobytes() == data
    f32 = reader.tensors[0].data
    assert f32.dtype == np.float32 and f32.shape == (3, 64)
    assert reader.tensors[1].tensor_type.name == "Q4_0"


def test_payload_and_dense_decode_match_the_bytes(tmp_path):
    """tensor_payload / dequantize over reader tensors (the reference's load
    path) give the values the written bytes hold."""
    path, tensors = sample_file(tmp_path)
    reader = gs.GGUFReader(path)
    for t in reader.tensors:
        qtype = quantization.type_name(t)
        shape = quantization.tensor_shape(t)
        dense = quantization.dequantize(quantization.tensor_payload(t), qtype, shape,
                                        torch.float32)
        raw = tensors[t.name][3]
        if qtype in BB:
            want = orc.dequantize_aos(np.frombuffer(raw, np.uint8), qtype, shape)
        elif qtype == "F32":
            want = np.frombuffer(raw, np.float32).reshape(shape)
        elif qtype == "F16":
            want = np.frombuffer(raw, np.float16).astype(np.float32).reshape(shape)
        else:  # BF16: the high half of an fp32
            bits = np.frombuffer(raw, np.uint16).astype(np.uint32) << 16
            want = bits.view(np.float32).reshape(shape)
        np.testing.assert_array_equal(dense.numpy(), want)


@pytest.mark.parametrize("qtype", ("Q4_0", "Q5_0", "Q8_0"))
def test_pack_soa_is_the_reference_repack(tmp_path, qtype):
    n, k = 37, 256
    raw = random_blocks(qtype, n, k, 11)
    path = tmp_path / "m.gguf"
    path.write_bytes(gguf_bytes([], [("w", GGML[qtype], (k, n), raw)]))
    tensor = gs.GGUFReader(path).tensors[0]
    q, s = quantization.pack_gguf_soa(tensor)
    want_q, want_s = orc.pack_soa(np.frombuffer(raw, np.uint8), qtype, (n, k))
    np.testing.assert_array_equal(q.numpy(), want_q)
    np.testing.assert_array_equal(s.numpy(), want_s)
    # The torch path (any tensor object with .data) gives the same bytes.
    fake = SimpleNamespace(name="w", tensor_type=tensor.tensor_type, shape=tensor.shape,
                           data=np.frombuffer(raw, np.uint8).copy())
    q2, s2 = quantization.pack_gguf_soa(fake)
    assert torch.equal(q, q2) and torch.equal(s, s2)


@pytest.mark.parametrize("threads", (1, 3, 0))
def test_pack_soa_threads(threads):
    nblocks = 70001
    aos = np.random.default_rng(3).integers(0, 256, nblocks * 22, dtype=np.uint8)
    q = torch.empty(nblocks * 20, dtype=torch.uint8)
    s = torch.empty(nblocks * 2, dtype=torch.uint8)
    native.pack_soa(aos.ctypes.data, nblocks, "Q5_0", q, s, threads)
    blocks = aos.reshape(nblocks, 22)
    np.testing.assert_array_equal(q.numpy(), blocks[:, 2:].reshape(-1))
    np.testing.assert_array_equal(s.numpy(), blocks[:, :2].reshape(-1))


def test_pack_soa_rejects_bad_arguments():
    lib = native.load()
    assert lib.svq_pack_soa(None, 4, 3, None, None, 1) == -1
    assert lib.svq_pack_soa(None, -1, 4, None, None, 1) == -2
    assert lib.svq_pack_soa(None, 4, 4, None, None, 1) == -3
    assert lib.svq_pack_soa(None, 0, 4, None, None, 1) == 0


def open_error(path):
    with pytest.raises(native.SVQError) as info:
        native.GGUFFile(str(path))
    return info.value.code, str(info.value)


def test_rejects_malformed_files(tmp_path):
    good = gguf_bytes([("a", STRING, "x")], [("w", GGML["F32"], (8,), bytes(32))])
    cases = {
        "magic": (b"GGUX" + good[4:], -8, "magic"),
        "version": (good[:4] + struct.pack("<I", 1) + good[8:], -8, "version"),
        "counts": (good[:8] + struct.pack("<Q", 1 << 60) + good[16:], -8, "counts"),
        "tiny": (b"GGUF", -8, "too small"),
    }
    for name, (data, code, text) in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        got, msg = open_error(p)
        assert got == code and text in msg, (name, got, msg)
    assert open_error(tmp_path / "absent.gguf")[0] == -9


def test_rejects_bad_tensor_infos(tmp_path):
    def write(tensors, **kw):
        p = tmp_path / "t.gguf"
        p.write_bytes(gguf_bytes([], tensors, **kw))
        return p

    # Unknown ggml type (an i-quant code) -> SVQ_E_DTYPE.
    assert open_error(write([("w", 19, (256,), bytes(100))]))[0] == -4
    # Row not whole blocks.
    assert open_error(write([("w", GGML["Q4_0"], (48,), bytes(27))]))[0] == -8
    # Data past the end: declare 64 rows of Q8_0 but write one block.
    data = gguf_bytes([], [("w", GGML["Q8_0"], (32, 64), bytes(34))])
    p = tmp_path / "short.gguf"
    p.write_bytes(data[: len(data)])  # the writer emits only what it was given
    assert open_error(p)[0] == -8
    # Misaligned data offset: patch the stored offset to 4.
    ok = gguf_bytes([], [("w", GGML["F32"], (4,), bytes(16)), ("v", GGML["F32"], (4,), bytes(16))])
    i = ok.index(b"v") + 1 + 4 + 8 + 4  # name, n_dims, dims[0], type
    bad = ok[:i] + struct.pack("<Q", 4) + ok[i + 8:]
    p.write_bytes(bad)
    code, msg = open_error(p)
    assert code == -8 and "aligned" in msg
    # general.alignment that is not a power of two.
    p.write_bytes(gguf_bytes([("general.alignment", 4, 24)], []))
    assert open_error(p)[0] == -8


def test_every_truncation_is_an_error(tmp_path):
    """Cut the file at every length below its size: opening fails cleanly."""
    path, _ = sample_file(tmp_path)
    data = path.read_bytes()
    p = tmp_path / "cut.gguf"
    for cut in list(range(0, 600)) + list(range(600, len(data), 97)):
        p.write_bytes(data[:cut])
        with pytest.raises(native.SVQError):
            native.GGUFFile(str(p))
    native.GGUFFile(str(path)).close()


def test_copy_on_write_mapping_keeps_the_file(tmp_path):
    path, tensors = sample_file(tmp_path)
    before = path.read_bytes()
    reader = gs.GGUFReader(path, "c")
    arr = reader.tensors[0].data
    arr[0, 0] = 123.0  # writable, private
    assert reader.tensors[0].data[0, 0] == 123.0
    assert path.read_bytes() == before
    ro = gs.GGUFReader(path, "r").tensors[0].data
    assert not ro.flags.writeable


# The reference's gguf_support tests (tests/test_gguf_support.py), restated.

def fake_tensor(name):
    return SimpleNamespace(name=name)


def test_full_pack_reports_all_components():
    items = [fake_tensor("model.image_encoder.visual_encoder.conv1.weight"),
             fake_tensor("model.image_projection.c_fc.weight"),
             fake_tensor("model.svg_transformer.transformer.transformer.wte.weight")]
    assert gs.inspect_tensor_index(items) == 3


@pytest.mark.parametrize("names", (["diffusion_model.input_blocks.0.weight"],
                                   ["model.svg_transformer.transformer.transformer.wte.weight"]))
def test_rejects_partial_packs(names):
    with pytest.raises(ValueError, match="full StarVector GGUF"):
        gs.inspect_tensor_index([fake_tensor(n) for n in names])


def reader_with(fields):
    return SimpleNamespace(get_field=lambda key: fields.get(key))


def field_of(value):
    return SimpleNamespace(contents=lambda: value)


def test_embedded_config_parsing():
    reader = reader_with({"starvector.config_json": field_of('{"hidden_size": 2048}')})
    assert gs.read_embedded_config(reader)["hidden_size"] == 2048
    for raw in ("not-json", "[]", "null"):
        with pytest.raises(ValueError, match="starvector.config_json"):
            gs.read_embedded_config(reader_with({"starvector.config_json": field_of(raw)}))
    with pytest.raises(ValueError, match="starvector.config_json"):
        gs.read_embedded_config(reader_with({}))


def test_embedded_tokenizer_assets():
    payload = '{"version":"1.0","model":{"type":"BPE"}}'
    reader = reader_with({"starvector.embedded_file.tokenizer.json": field_of(payload),
                          "starvector.embedded_file.tokenizer_config.json": field_of("{}")})
    assert gs.read_embedded_assets(reader)["tokenizer.json"] == payload
    for fields in ({}, {"starvector.embedded_file.vocab.json": field_of('{"a":0}')}):
        with pytest.raises(ValueError, match="Invalid StarVector GGUF.*embedded tokenizer"):
            gs.read_embedded_assets(reader_with(fields))
    for contents in ("", bytes([255]), 10):
        with pytest.raises(ValueError, match="Invalid StarVector GGUF"):
            gs.read_embedded_assets(
                reader_with({"starvector.embedded_file.tokenizer.json": field_of(contents)}))


def test_inspect_local_gguf_on_a_real_file(tmp_path):
    path, tensors = sample_file(tmp_path)
    ref = gs.inspect_local_gguf(path)
    assert ref.path == path.resolve()
    assert ref.model_config == {"hidden_size": 2048, "n": [1, 2]}
    assert "tokenizer.json" in ref.model_assets
    assert set(ref.tensor_index) == set(tensors)
    q, s = quantization.pack_gguf_soa(ref.tensor_index["model.image_projection.c_fc.weight"])
    assert q.numel() == 5 * 2 * 16 and s.numel() == 5 * 2 * 2


def test_inspect_local_gguf_rejects(tmp_path):
    wrong = tmp_path / "model.bin"
    wrong.write_bytes(b"")
    with pytest.raises(ValueError, match="Expected a local .gguf file"):
        gs.inspect_local_gguf(wrong)
    dup = [("model.image_encoder.same.weight", GGML["F32"], (4,), bytes(16)),
           ("model.image_encoder.same.weight", GGML["F32"], (4,), bytes(16)),
           ("model.image_projection.c_fc.weight", GGML["F32"], (4,), bytes(16)),
           ("model.svg_transformer.transformer.transformer.wte.weight", GGML["F32"], (4,), bytes(16))]
    kvs = [("starvector.config_json", STRING, "{}"),
           ("starvector.embedded_file.tokenizer.json", STRING, '{"model":{}}')]
    p = tmp_path / "dup.gguf"
    p.write_bytes(gguf_bytes(kvs, dup))
    with pytest.raises(ValueError, match="Duplicate tensor"):
        gs.inspect_local_gguf(p)
    p.write_bytes(gguf_bytes(kvs[1:], dup[2:]))
    with pytest.raises(ValueError, match="starvector.config_json"):
        gs.inspect_local_gguf(p)

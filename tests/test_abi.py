"""The C ABI without a GPU: libsvq.so loads, exports every function that
include/svq.h declares, and rejects bad arguments before any HIP call."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

import starvector_amd._native as native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "svq.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int64_t|int|void|const char \*|const void \*)\s*(svq_\w+)\s*\(",
                                  text, re.M)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    assert {"svq_abi_version", "svq_last_error", "svq_gemv", "svq_dequant",
            "svq_dequant_rows", "svq_decode_attention", "svq_gemv_fused", "svq_gguf_open",
            "svq_gguf_close", "svq_gguf_tensor", "svq_gguf_tensor_data", "svq_pack_soa",
            "svq_decode_attention_workspace"} <= set(names)


TIMELINE_ONLY = {"svq_timeline_stamps", "svq_timeline_read"}
TIMELINE_LIB = Path(native.__file__).resolve().parent / "libsvq_timeline.so"


def test_library_exports_every_declared_function():
    lib = native.load()
    for name in declared_functions():
        if name in TIMELINE_ONLY:
            continue
        assert hasattr(lib, name), name
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_timeline_library_exports_everything_and_libsvq_no_timeline():
    """libsvq_timeline.so (the SVQ_TIMELINE build) exports every declared
    function; libsvq.so carries no timeline entry point."""
    names = declared_functions()
    assert TIMELINE_ONLY <= set(names)
    timeline = ctypes.CDLL(str(TIMELINE_LIB))
    for name in names:
        assert hasattr(timeline, name), name
    lib = native.load()
    for name in TIMELINE_ONLY:
        assert not hasattr(lib, name), name


def test_timeline_read_rejects_bad_arguments():
    timeline = ctypes.CDLL(str(TIMELINE_LIB))
    f = timeline.svq_timeline_read
    f.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p,
                  ctypes.c_void_p, ctypes.c_void_p]
    assert f(X, 1000, 512, Y, B, None) == -2  # not a multiple of 1024
    assert f(X, 1 << 31, 512, Y, B, None) == -2  # too large
    assert f(X, 1024, 0, Y, B, None) == -2  # no workgroups
    assert f(None, 1024, 512, Y, B, None) == -2


def test_abi_version():
    assert native.load().svq_abi_version() == native.ABI_VERSION == 3


FAKE = 1 << 20  # a 16-byte aligned non-null address; never dereferenced
# Distinct fake arrays, 1 MiB apart: no two of them overlap at the sizes used.
X, Q, S, Y, B, W, R = (FAKE * i for i in range(2, 9))


def test_dtype_codes_are_the_fp32_flags():
    """SVQ_F16 = 0 and SVQ_F32 = 1: svq_gemv's y_is_fp32 and svq_dequant's
    out_is_fp32 flags (the boundary's suggested signatures) are the codes."""
    text = HEADER.read_text()
    codes = dict(re.findall(r"#define (SVQ_F16|SVQ_F32|SVQ_BF16) (\d+)", text))
    assert codes == {"SVQ_F16": "0", "SVQ_F32": "1", "SVQ_BF16": "2"}
    assert native.DTYPE_CODE == {__import__("torch").float16: 0, __import__("torch").float32: 1,
                                 __import__("torch").bfloat16: 2}
    assert re.search(r"int svq_gemv\(.*?int y_is_fp32, void \*stream\);", text, re.S)


def gemv(**kw):
    args = dict(x=X, q=Q, s=S, bias=None, y=Y, m=1, n=8, k=64, qtype=4, y_is_fp32=0,
                stream=None)
    args.update(kw)
    lib = native.load()
    return lib.svq_gemv(args["x"], args["q"], args["s"], args["bias"], args["y"], args["m"],
                        args["n"], args["k"], args["qtype"], args["y_is_fp32"], args["stream"])


@pytest.mark.parametrize("kw,code", [
    (dict(qtype=2), -1), (dict(qtype=6), -1),
    (dict(m=0), -2), (dict(m=9), -2), (dict(n=0), -2), (dict(k=0), -2), (dict(k=48), -2),
    (dict(k=1 << 25), -5), (dict(n=(1 << 30) + 1), -5),
    (dict(x=None), -3), (dict(q=None), -3), (dict(s=None), -3), (dict(y=None), -3),
    (dict(y_is_fp32=2), -4), (dict(y_is_fp32=7), -4), (dict(y_is_fp32=-1), -4),
    (dict(x=X + 8), -6), (dict(q=Q + 4), -6), (dict(q=Q + 4, qtype=5), None),
    (dict(s=S + 1), -6), (dict(bias=B + 1), -6), (dict(y=Y + 1), -6),
    # y may share no byte with an input (workgroups write y while others read)
    (dict(y=X), -2), (dict(y=X + 112), -2), (dict(x=Y - 112), -2), (dict(y=Q + 240), -2),
    (dict(y=S + 16), -2), (dict(bias=Y + 8), -2),
])
def test_gemv_rejects_bad_arguments(kw, code):
    if code is None:
        # Q5_0 only needs 4-byte payload alignment: pair it with a rejected
        # shape so the call still returns before any launch.
        kw = dict(kw, k=48)
        code = -2
    assert gemv(**kw) == code
    assert native.load().svq_last_error().decode()


def test_dequant_rejects_bad_arguments():
    lib = native.load()
    assert lib.svq_dequant(FAKE, FAKE, FAKE, 4, 3, 0, None) == -1
    assert lib.svq_dequant(FAKE, FAKE, FAKE, -1, 4, 0, None) == -2
    assert lib.svq_dequant(FAKE, FAKE, FAKE, 4, 4, 3, None) == -4
    assert lib.svq_dequant(None, FAKE, FAKE, 4, 4, 0, None) == -3
    assert lib.svq_dequant(FAKE, FAKE, FAKE + 4, 4, 4, 0, None) == -6
    assert lib.svq_dequant(FAKE, FAKE, FAKE, 0, 4, 0, None) == 0  # empty: no launch


def test_dequant_rows_rejects_bad_arguments():
    lib = native.load()
    call = lambda **kw: lib.svq_dequant_rows(
        kw.get("q", FAKE), kw.get("s", FAKE), kw.get("ids", FAKE), kw.get("nids", 2),
        kw.get("nrows", 5), kw.get("k", 64), kw.get("out", FAKE), kw.get("qtype", 8),
        kw.get("dt", 1), None)
    assert call(qtype=1) == -1
    assert call(k=40) == -2
    assert call(nrows=0) == -2
    assert call(dt=5) == -4
    assert call(ids=None) == -3
    assert call(ids=FAKE + 4) == -6
    assert call(nids=0) == 0


def test_error_message_names_the_problem():
    gemv(m=11)
    assert "m=11" in native.load().svq_last_error().decode()


def test_gemv_plan_rejects_bad_arguments():
    lib = native.load()
    plan = (ctypes.c_int32 * 8)()
    assert lib.svq_gemv_plan(2, 64, 64, 3, plan) == -1
    assert lib.svq_gemv_plan(9, 64, 64, 4, plan) == -2
    assert lib.svq_gemv_plan(2, 64, 40, 4, plan) == -2
    assert lib.svq_gemv_plan(2, 0, 64, 4, plan) == -2
    assert lib.svq_gemv_plan(2, 64, 64, 4, None) == -3


def attention(**kw):
    args = dict(qkv=FAKE, stride=(36 + 8) * 128, cos=FAKE, sin=FAKE, keys=FAKE, values=FAKE,
                capacity=64, position=FAKE, bias=FAKE, span=64, out=FAKE, rows=2, heads=36,
                kv_heads=4, head_dim=128, scale=128 ** -0.5, workspace=FAKE,
                workspace_bytes=1 << 20)
    args.update(kw)
    lib = native.load()
    return lib.svq_decode_attention(
        args["qkv"], args["stride"], args["cos"], args["sin"], args["keys"], args["values"],
        args["capacity"], args["position"], args["bias"], args.get("window", 0), args["span"],
        args["out"], args["rows"], args["heads"], args["kv_heads"], args["head_dim"],
        args["scale"], args["workspace"], args["workspace_bytes"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(heads=35), -2), (dict(kv_heads=0), -2), (dict(heads=34, kv_heads=2), -2),
    (dict(head_dim=64), -2), (dict(span=0), -2), (dict(capacity=32), -2), (dict(rows=0), -2),
    (dict(stride=44 * 128 - 8), -2), (dict(stride=44 * 128 + 4), -2),
    (dict(span=1 << 23, capacity=1 << 23), -5),
    (dict(qkv=None), -3), (dict(keys=None), -3), (dict(position=None), -3),
    (dict(workspace=None), -3), (dict(cos=None), -3),
    (dict(qkv=FAKE + 8), -6), (dict(cos=FAKE + 2), -6), (dict(bias=FAKE + 1), -6),
    (dict(position=FAKE + 4), -6), (dict(workspace=FAKE + 16), -6),
    (dict(workspace_bytes=1024), -7),
])
def test_decode_attention_rejects_bad_arguments(kw, code):
    assert attention(**kw) == code
    assert native.load().svq_last_error().decode()


def test_decode_attention_workspace_size():
    lib = native.load()
    # Per (row, query head) and chunk of 64 slots (25 for span 1537): (max,
    # sum) as 8 bytes, padded to 256 bytes in all, then 128 fp32 weighted-V
    # sums.
    assert lib.svq_decode_attention_workspace(2, 36, 4, 1537) == 14592 + 2 * 36 * 25 * 512
    assert lib.svq_decode_attention_workspace(2, 16, 1, 64) == 256 + 2 * 16 * 512
    assert lib.svq_decode_attention_workspace(2, 36, 5, 64) == -2
    assert lib.svq_decode_attention_workspace(2, 34, 2, 64) == -2  # 17 heads per kv head


def cache_reorder(**kw):
    args = dict(cache=FAKE, planes=32, rows=2, heads=4, capacity=64, head_dim=128, length=10,
                parents=FAKE)
    args.update(kw)
    return native.load().svq_cache_reorder(
        args["cache"], args["planes"], args["rows"], args["heads"], args["capacity"],
        args["head_dim"], args["length"], args["parents"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(rows=0), -2), (dict(rows=9), -2), (dict(planes=0), -2), (dict(heads=0), -2),
    (dict(head_dim=64), -2), (dict(length=65), -2), (dict(length=-1), -2),
    (dict(planes=70000, heads=1), -2),
    (dict(cache=None), -3), (dict(parents=None), -3),
    (dict(cache=FAKE + 8), -6), (dict(parents=FAKE + 4), -6),
])
def test_cache_reorder_rejects_bad_arguments(kw, code):
    assert cache_reorder(**kw) == code
    assert native.load().svq_last_error().decode()


def test_cache_reorder_empty_length_is_a_no_op():
    # Nothing to move: returns before any launch (no device needed).
    assert cache_reorder(length=0) == 0


def gemv_fused(**kw):
    args = dict(x=X, q=Q, s=S, bias=None, y=Y, m=2, n=8, k=64, qtype=4,
                ln_w=None, ln_b=None, eps=1e-5, res=None, act=0)
    args.update(kw)
    return native.load().svq_gemv_fused(
        args["x"], args["q"], args["s"], args["bias"], args["y"], args["m"], args["n"],
        args["k"], args["qtype"], args["ln_w"], args["ln_b"], args["eps"], args["res"],
        args["act"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(act=2), -4), (dict(ln_w=W + 2), -6), (dict(ln_b=W + 8), -6),
    (dict(res=R + 1), -6), (dict(ln_w=W, eps=-1.0), -2),
    (dict(y=X, res=R), -2), (dict(y=X + 64, res=X + 64), -2), (dict(ln_w=Y - 64), -2),
    (dict(ln_b=Y + 16), -2), (dict(res=Y + 2), -2), (dict(res=Y - 30), -2),
    (dict(qtype=3), -1), (dict(m=9), -2), (dict(k=40), -2), (dict(x=None), -3),
    # x of 8 rows x 18432 does not fit the LDS staging the LayerNorm needs
    (dict(m=8, k=18432, n=64, ln_w=W), -2),
])
def test_gemv_fused_rejects_bad_arguments(kw, code):
    assert gemv_fused(**kw) == code
    assert native.load().svq_last_error().decode()


def gemv_split(**kw):
    args = dict(x=X, q=Q, s=S, bias=None, y=Y, m=2, n=8, k=64, qtype=4,
                res=None, act=0, ws=FAKE * 9, ws_bytes=1 << 16)
    args.update(kw)
    return native.load().svq_gemv_split(
        args["x"], args["q"], args["s"], args["bias"], args["y"], args["m"], args["n"],
        args["k"], args["qtype"], args["res"], args["act"], args["ws"], args["ws_bytes"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(act=2), -4), (dict(res=R + 1), -6), (dict(ws=FAKE * 9 + 8), -6),
    (dict(y=X, res=R), -2), (dict(res=Y + 4), -2), (dict(ws_bytes=-1), -7),
    # the workspace is written: it may share no byte with y or an input
    (dict(ws=Y - 64, ws_bytes=128), -2), (dict(ws=X + 16), -2), (dict(ws=Q), -2),
    (dict(ws=R - 16, ws_bytes=32, res=R), -2),
    (dict(qtype=3), -1), (dict(m=9), -2), (dict(k=40), -2), (dict(x=None), -3),
])
def test_gemv_split_rejects_bad_arguments(kw, code):
    assert gemv_split(**kw) == code
    assert native.load().svq_last_error().decode()


def test_gemv_split_workspace_size():
    """fp32 partial sums of every slice: K > 8192 at m = 2..4 is cut into the
    fewest slices of at most 4608 columns that divide K / 32."""
    lib = native.load()
    assert lib.svq_gemv_split_workspace(2, 4608, 18432, 5) == 4 * 2 * 4608 * 4
    assert lib.svq_gemv_split_workspace(1, 4608, 18432, 4) == 0   # m = 1: one pass
    assert lib.svq_gemv_split_workspace(8, 4608, 18432, 4) == 4 * 8 * 4608 * 4
    assert lib.svq_gemv_split_workspace(5, 100, 9216, 8) == 2 * 5 * 100 * 4
    assert lib.svq_gemv_split_workspace(4, 100, 9216, 8) == 2 * 4 * 100 * 4
    assert lib.svq_gemv_split_workspace(2, 100, 12288, 4) == 3 * 2 * 100 * 4
    assert lib.svq_gemv_split_workspace(2, 4608, 4608, 5) == 0   # one pass
    assert lib.svq_gemv_split_workspace(2, 2048, 8192, 4) == 0   # K <= 8192
    assert lib.svq_gemv_split_workspace(5, 4608, 18432, 5) == 4 * 5 * 4608 * 4
    assert lib.svq_gemv_split_workspace(9, 4608, 18432, 5) < 0   # m > 8
    assert lib.svq_gemv_split_workspace(2, 64, 40, 4) == -2
    assert lib.svq_gemv_split_workspace(2, 64, 64, 3) == -1


def beam_select(**kw):
    args = dict(probs=FAKE, noise=FAKE, scores=FAKE, candidates=FAKE, beams=2, vocab=320,
                ncand=64, draws=4, seen_in=FAKE, seen_out=FAKE + 4096, pitch=320, running=FAKE,
                parents=FAKE, tokens=FAKE, tokens_copy=None)
    args.update(kw)
    return native.load().svq_beam_select(
        args["probs"], args["noise"], args["scores"], args["candidates"], args["beams"],
        args["vocab"], args["ncand"], args["draws"], args["seen_in"], args["seen_out"],
        args["pitch"], args["running"], args["parents"], args["tokens"], args["tokens_copy"],
        args.get("compact", 0), None)


@pytest.mark.parametrize("kw,code", [
    (dict(beams=0), -2), (dict(beams=9), -2), (dict(vocab=0), -2), (dict(ncand=0), -2),
    (dict(ncand=321), -2), (dict(beams=8, ncand=129), -2), (dict(draws=0), -2),
    (dict(draws=5), -2), (dict(beams=1, ncand=1, draws=2), -2), (dict(pitch=304), -2),
    (dict(pitch=328), -2), (dict(probs=None), -3), (dict(seen_out=None), -3),
    (dict(tokens=None), -3), (dict(candidates=FAKE + 4), -6), (dict(seen_in=FAKE + 8), -6),
    (dict(tokens_copy=FAKE + 4), -6), (dict(seen_out=FAKE + 320), -2),  # overlaps seen_in
    (dict(beams=1, ncand=65, draws=2, compact=1), -2),
])
def test_beam_select_rejects_bad_arguments(kw, code):
    assert beam_select(**kw) == code
    assert native.load().svq_last_error().decode()


def beam_candidates(**kw):
    args = dict(logits=FAKE, seen=FAKE, pitch=320, running=FAKE, beams=2, vocab=320, k=50, kc=64,
                keep=2, penalty=3.1, temperature=1.5, top_p=0.9, candidates=FAKE, scores=FAKE,
                probs=FAKE, status=FAKE, workspace=FAKE, workspace_bytes=1 << 20)
    args.update(kw)
    return native.load().svq_beam_candidates(
        args["logits"], args["seen"], args["pitch"], args["running"], args["beams"],
        args["vocab"], args["k"], args["kc"], args["keep"], args["penalty"],
        args["temperature"], args["top_p"], args["candidates"], args["scores"], args["probs"],
        args["status"], args["workspace"], args["workspace_bytes"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(beams=0), -2), (dict(beams=9), -2), (dict(vocab=65537, pitch=65552), -2),
    (dict(k=0), -2), (dict(k=65, kc=64), -2), (dict(kc=65), -2), (dict(vocab=60, pitch=64), -2),
    (dict(keep=65), -2), (dict(keep=-1), -2), (dict(pitch=304), -2), (dict(pitch=328), -2),
    (dict(temperature=0.0), -2), (dict(penalty=-1.0), -2), (dict(top_p=1.5), -2),
    (dict(logits=None), -3), (dict(status=None), -3), (dict(logits=FAKE + 1), -6),
    (dict(candidates=FAKE + 4), -6), (dict(status=FAKE + 4), -6), (dict(workspace=None), -3),
    (dict(workspace=FAKE + 4), -6), (dict(workspace_bytes=100), -7),
])
def test_beam_candidates_rejects_bad_arguments(kw, code):
    assert beam_candidates(**kw) == code
    assert native.load().svq_last_error().decode()


def test_beam_candidates_workspace_size():
    lib = native.load()
    # Per row and slice of 4096 tokens: (max, sum), two counts, and kc
    # (logit, token) pairs per class.
    assert lib.svq_beam_candidates_workspace(2, 49152, 64) == 2 * 12 * (16 + 2 * 64 * 8)
    assert lib.svq_beam_candidates_workspace(1, 320, 64) == 16 + 2 * 64 * 8
    assert lib.svq_beam_candidates_workspace(9, 320, 64) == -2
    assert lib.svq_beam_candidates_workspace(2, 320, 65) == -2

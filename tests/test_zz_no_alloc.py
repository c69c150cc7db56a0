"""svq_gemv_split_static, the GEMV entry point that allocates nothing: the
K split's partial sums live in the library's static device array instead of
a caller's workspace. Checked against svq_gemv_split with a workspace (same
kernels and slices, so the same bits) and against the fp64 oracle, on two
calls in a row, the second with a smaller input."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import starvector_amd._native as native
from oracle import soa_oracle as orc

FAKE = 1 << 32  # fake device arrays 4 GiB apart: never dereferenced
QCODE = {"Q4_0": 4, "Q5_0": 5, "Q8_0": 8}


def lib():
    lib = native.load()
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    lib.svq_gemv_split_static.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32, vp]
    lib.svq_gemv_split_static.restype = i32
    return lib


def test_static_scratch_limit_is_a_clear_error():
    """A split whose partial sums exceed the static scratch (8 rows x 40000
    outputs x 4 slices x 4 bytes > 4 MiB) is rejected before any HIP call."""
    rc = lib().svq_gemv_split_static(2 * FAKE, 3 * FAKE, 4 * FAKE, None, 5 * FAKE, 8, 40000, 18432,
                                     4, None, 0, None)
    assert rc == -7
    assert "static scratch holds 4194304" in native.load().svq_last_error().decode()
    assert lib().svq_gemv_split_static(2 * FAKE, 3 * FAKE, 4 * FAKE, None, 2 * FAKE, 2, 64, 64,
                                       4, None, 0, None) == -2  # y overlaps x


@pytest.mark.gpu
def test_split_static_matches_split_with_workspace(cuda_device):
    l = lib()
    stream = torch.cuda.current_stream(cuda_device).cuda_stream
    # The 8B c_proj at beam 4 with GELU and a residual, then a smaller shape.
    for m, n, k, qtype, act, with_res in ((4, 4608, 18432, "Q5_0", 1, True),
                                          (2, 1000, 9216, "Q4_0", 0, False)):
        print(f"split static {qtype} M={m} {n}x{k}", flush=True)
        need = native.gemv_workspace_bytes(m, n, k, qtype)
        assert 0 < need <= 4 << 20  # this shape splits K, within the scratch
        q, s = orc.synthetic_soa(qtype, n, k, seed=n)
        rng = np.random.default_rng(m)
        x = rng.standard_normal((m, k)).astype(np.float16)
        bias = (0.02 * rng.standard_normal(n)).astype(np.float16)
        qt = torch.from_numpy(q).to(cuda_device)
        st = torch.from_numpy(s).to(cuda_device)
        xt = torch.from_numpy(x).to(cuda_device)
        bt = torch.from_numpy(bias).to(cuda_device)
        res = torch.randn((m, n), device=cuda_device).half() if with_res else None
        ptr = lambda t: None if t is None else t.data_ptr()
        ws = torch.empty(need, dtype=torch.uint8, device=cuda_device)
        want = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda_device)
        got = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda_device)
        assert l.svq_gemv_split(xt.data_ptr(), qt.data_ptr(), st.data_ptr(), bt.data_ptr(),
                                want.data_ptr(), m, n, k, QCODE[qtype], ptr(res), act,
                                ws.data_ptr(), need, stream) == 0
        assert l.svq_gemv_split_static(xt.data_ptr(), qt.data_ptr(), st.data_ptr(), bt.data_ptr(),
                                       got.data_ptr(), m, n, k, QCODE[qtype], ptr(res), act,
                                       stream) == 0, native.load().svq_last_error()
        torch.cuda.synchronize()
        assert not torch.isnan(got).any()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        if not act and not with_res:
            ref = orc.gemv_ref(x, q, s, qtype, n, k, bias)
            assert orc.rel_err(got.float().cpu().numpy(), ref) <= 1e-3

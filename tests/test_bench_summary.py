"""bench.py's rocprofv3 summaries on synthetic traces (no GPU): a K-split
GEMV's finish kernel is part of the GEMV before it, in durations, shape
mapping and counters."""
from __future__ import annotations

import csv
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

GEMV = "void svq::(anonymous namespace)::gemv_mfma4_kernel<5, 2, 1, 3, 4, 3, false>(svq::GemvArgs)"
STREAM = "void svq::(anonymous namespace)::gemv_stream_kernel<5, 2, 2, 4, 4, false>(svq::GemvArgs)"
FINISH = "svq::(anonymous namespace)::split_finish_kernel(svq::GemvArgs, int, float)"
COPY = "__amd_rocclr_copyBuffer"


def write_trace(path, names):
    """Dispatches of 10 us each, 1 us apart, in the order given. An entry is a
    kernel name (launched as 1 slice x 512 workgroups of 256 threads) or a
    (name, slices, workgroups per slice) tuple."""
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Start_Timestamp",
                                          "End_Timestamp", "Workgroup_Size_X", "Grid_Size_X",
                                          "Grid_Size_Y", "Grid_Size_Z", "VGPR_Count",
                                          "LDS_Block_Size"])
        w.writeheader()
        for i, entry in enumerate(names):
            name, slices, groups = entry if isinstance(entry, tuple) else (entry, 1, 512)
            w.writerow(dict(Dispatch_Id=i + 1, Kernel_Name=name, Start_Timestamp=i * 11000,
                            End_Timestamp=i * 11000 + 10000, Workgroup_Size_X=256,
                            Grid_Size_X=256 * slices, Grid_Size_Y=groups, Grid_Size_Z=1,
                            VGPR_Count=56, LDS_Block_Size=2048))


def profile_order():
    """bench.py --profile: two passes over 8 copies of the 5 step shapes; c_proj
    (the fourth) is a K split: GEMV + finish."""
    names = []
    for _ in range(2 * bench.COPIES):
        for name, *_ in bench.STEP_SHAPES:
            if name == "c_proj":
                names += [(GEMV, 4, 128), (FINISH, 18, 1)]
            else:
                names.append(GEMV)
    return names + [COPY] * 16


def test_profile_trace_maps_split_gemv_to_its_shape(tmp_path, capsys):
    write_trace(tmp_path / "ktp_kernel_trace.csv", profile_order())
    bench.summarize(tmp_path)
    out = capsys.readouterr().out
    lines = {line.split(" | ")[0]: line for line in out.splitlines() if line.startswith("| ")}
    assert "split_finish_kernel" in lines["| c_proj 4608x18432"]
    assert " 20.00 " in lines["| c_proj 4608x18432"]   # both kernels: 10 + 10 us
    assert " 10.00 " in lines["| qkv 5632x4608"]
    assert " 131072 (4x128 wg) " in lines["| c_proj 4608x18432"]   # 2-D launch: K slices x groups
    assert " 131072 (1x512 wg) " in lines["| qkv 5632x4608"]
    assert f"({2 * bench.COPIES * len(bench.STEP_SHAPES)} GEMV dispatches)" in out


def test_decode_summary_counts_finish_as_gemv(tmp_path, capsys):
    names = ["void svq::(anonymous namespace)::dequant_kernel<4>(x)", STREAM, FINISH,
             "other_kernel", GEMV]
    write_trace(tmp_path / "dec_kernel_trace.csv", names)
    bench.summarize_decode(tmp_path / "dec_kernel_trace.csv")
    out = capsys.readouterr().out
    assert "GEMV kernels: 30 us = 75.0% of kernel time" in out

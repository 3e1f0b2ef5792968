"""stage_report on a hand-made trace: kernels go to the innermost range open at their launch,
the first step is skipped, per-step averages."""

import importlib

import pytest


def _write(d, name, header, rows):
    with open(d / name, "w") as f:
        f.write(",".join(header) + "\n")
        for r in rows:
            f.write(",".join(str(x) for x in r) + "\n")


def test_innermost_range_attribution(tmp_path):
    sr = importlib.import_module("inference-engine_amd.stage_report")
    mh = ["Domain", "Function", "Process_Id", "Thread_Id", "Correlation_Id", "Start_Timestamp",
          "End_Timestamp"]
    marks, hips, kerns = [], [], []
    for step in range(3):
        t = 1000 * step
        marks += [("M", "embed", 1, 1, 0, t, t + 10), ("M", "layer", 1, 1, 0, t + 20, t + 90),
                  ("M", "attn", 1, 1, 0, t + 30, t + 60)]
        for j, lt in enumerate((t + 5, t + 40, t + 70)):  # embed, attn, layer (outside attn)
            cid = 100 * step + j
            hips.append(("H", "hipLaunchKernel", 1, 1, cid, lt, lt + 1))
            kerns.append(("KERNEL_DISPATCH", f"k{j}(int)", cid, 5000 + 100 * cid,
                          5000 + 100 * cid + 1000 * (j + 1)))
    _write(tmp_path, "s_marker_api_trace.csv", mh, marks)
    _write(tmp_path, "s_hip_api_trace.csv", mh, hips)
    _write(tmp_path, "s_kernel_trace.csv",
           ["Kind", "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp"], kerns)
    out = sr.report(str(tmp_path), skip=1)
    lines = {l.split("|")[1].strip(): l for l in out.splitlines() if l.startswith("| ")}
    assert "steps: 2" in out
    assert "| 1 | 1.0 |" in lines["embed"] and "k0 x1" in lines["embed"]
    assert "| 1 | 2.0 |" in lines["attn"] and "k1 x1" in lines["attn"]
    assert "| 1 | 3.0 |" in lines["layer"] and "k2 x1" in lines["layer"]
    with pytest.raises(SystemExit):
        sr.report(str(tmp_path), skip=3)

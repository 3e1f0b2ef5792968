"""Per-stage GPU time from a rocprofv3 trace of eager steps (the stage ranges are the
`torch.cuda.nvtx` / roctx ranges that attention_layer.py and decode_step.py open at the
reference's stage points, qwen3-1.7b/architecture.py:84-200 and engine.py:145-223).

    rocprofv3 --marker-trace --hip-runtime-trace --kernel-trace -d DIR -o s \\
        --output-format csv -- python3 -m inference-engine_amd.decode_step --eager 5
    python3 -m inference-engine_amd.stage_report DIR

Each kernel is attributed to the innermost range open on the host thread when its launch call
started (the kernel record and its launch call share a correlation id); the first `--skip`
steps (a step starts at its "embed" or "embed+metadata" range) are left out. Ranges are
recorded while a graph is captured, not when it replays, hence the eager steps. Prints a
markdown table.
"""

import argparse
import collections
import csv
import glob


def _rows(d, suffix):
    files = glob.glob(f"{d}/*{suffix}")
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def report(d: str, skip: int = 1) -> str:
    marks = _rows(d, "marker_api_trace.csv")
    launch_t = {r["Correlation_Id"]: int(r["Start_Timestamp"])
                for r in _rows(d, "hip_api_trace.csv")}
    kernels = _rows(d, "kernel_trace.csv")
    ranges = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Function"]) for r in marks]
    steps = sorted(r for r in ranges if r[2].startswith("embed"))
    if len(steps) <= skip:
        raise SystemExit(f"{len(steps)} steps in the trace, {skip} skipped")
    t_first, n = steps[skip][0], len(steps) - skip
    per, cnt = collections.defaultdict(float), collections.Counter()
    names = collections.defaultdict(collections.Counter)
    for k in kernels:
        t = launch_t.get(k["Correlation_Id"])
        if t is None or t < t_first:
            continue
        inner = None
        for a, b, name in ranges:
            if a <= t <= b and (inner is None or b - a < inner[1] - inner[0]):
                inner = (a, b, name)
        stage = inner[2] if inner else "(outside ranges)"
        per[stage] += (int(k["End_Timestamp"]) - int(k["Start_Timestamp"])) / 1e3
        cnt[stage] += 1
        kname = k["Kernel_Name"].split("(")[0].split("<")[0].replace("void ", "")
        names[stage][kname] += 1
    total = sum(per.values())
    out = [f"steps: {n}; kernel time per step {total / n:.1f} us", "",
           "| stage (innermost range) | kernels/step | GPU us/step | share | kernels |",
           "|---|---|---|---|---|"]
    for stage, v in sorted(per.items(), key=lambda kv: -kv[1]):
        ks = ", ".join(f"{k} x{c / n:g}" for k, c in names[stage].most_common(4))
        out.append(f"| {stage} | {cnt[stage] / n:g} | {v / n:.1f} | {v / total * 100:.1f} % | "
                   f"{ks} |")
    return "\n".join(out)


def _main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace_dir")
    ap.add_argument("--skip", type=int, default=1, help="leading steps left out")
    args = ap.parse_args()
    print(report(args.trace_dir, args.skip))


if __name__ == "__main__":
    _main()

"""Markdown table of the raw parity errors of the BASELINE configs from a GPU test run.

    LLATTN_PARITY_LOG=gpurun_out/parity.jsonl python -m pytest tests -m gpu
    python tests/parity_table.py gpurun_out/parity.jsonl

Each row is one comparison that ``tests/gpu_helpers.py`` made: the raw max|got - ref| (no scaling), max|ref|,
the scaled max-abs (raw / max(1, max|ref|)) and the mean-relative error mean|got - ref| / mean|ref| that the
bars apply to, and the bars themselves.
"""
from __future__ import annotations

import json
import sys

CONFIGS = (("config 1 fp32", "C1 (fp32, golden from the reference)"),
           ("c2 reference row", "C2 out/dx, batch rows vs fp32 CPU reference"),
           ("c2 weight grads", "C2 parameter gradients (B=2) vs fp32 CPU reference"),
           ("c3 reference row", "C3 out/dx rows"), ("c3 parameter gradients", "C3 parameter gradients per row"),
           ("c4 reference row", "C4 out/dx rows"), ("c4 parameter gradients", "C4 parameter gradients per row"))


def main(path: str) -> None:
    rows = [json.loads(line) for line in open(path)]
    bars = [r for r in rows if "scaled_max_abs" in r]
    # raw max-abs of the reference's own math under CPU bf16 autocast, by (config, tensor)
    floors = {(r["case"].split()[0], r["tensor"]): r["floor_raw_max_abs"] for r in rows if "floor_raw_max_abs" in r}
    print("| config | tensor | raw max-abs | max abs ref | scaled max-abs | mean-rel | bar (max-abs / mean-rel) | "
          "reference bf16 floor (raw) | raw / floor |")
    print("|---|---|---:|---:|---:|---:|---|---:|---:|")
    for prefix, label in CONFIGS:
        for r in bars:
            if not r["case"].startswith(prefix):
                continue
            bar = f"{r['max_abs_bar']:.0e}" + ("" if r["mean_rel_bar"] is None else f" / {r['mean_rel_bar']:.0e}")
            fl = floors.get((r["case"].split()[0], r["tensor"]))
            fl_s = "" if fl is None else f"{fl:.3e}"
            ratio = "" if not fl else f"{r['raw_max_abs'] / fl:.2f}"
            print(f"| {label} | {r['tensor']} | {r['raw_max_abs']:.3e} | {r['max_ref']:.3e} | "
                  f"{r['scaled_max_abs']:.3e} | {r['mean_rel']:.3e} | {bar} | {fl_s} | {ratio} |")


if __name__ == "__main__":
    main(sys.argv[1])

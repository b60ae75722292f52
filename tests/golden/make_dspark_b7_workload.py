"""Writes tests/golden/dspark_b7_workload.json from the reference's published attention study.

Source (read as data, in this container only): the `workload`, `dimensions`, `timing_contract`,
`timings` and `errors` of docs/assets/dspark-attention-training/benchmark-evidence.json in the
reference checkout (the study behind docs/dspark_attn_kernel_optimization.md:49-61 and
tools/performance/bench_dspark_b7_attention.py). The fixture keeps the document lengths, block
size and the captured anchor positions (document-local, in the sampler's order), and the median
and window figures of the study's routes, so the same workload can be timed on MI355X.

    python tests/golden/make_dspark_b7_workload.py [/root/reference]
"""

import json
import sys
from pathlib import Path

EVIDENCE = "docs/assets/dspark-attention-training/benchmark-evidence.json"


def main(reference="/root/reference"):
    src = json.loads((Path(reference) / EVIDENCE).read_text())
    w = src["workload"]
    routes = {}
    for route, phases in src["timings"].items():
        routes[route] = {phase: {k: t[k] for k in ("median_ms", "min_ms", "max_ms")}
                         for phase, t in phases.items()}
    out = {
        "source": EVIDENCE,
        "study": src["study"],
        "architecture": src["architecture"],
        "lengths": w["lengths"],
        "block": w["block"],
        "anchors_per_document": w["anchors"],
        "anchor_policy": w["anchor_policy"],
        "anchor_positions": w["anchor_positions"],
        "dimensions": src["dimensions"],
        "timing_contract": src["timing_contract"],
        "published_ms": routes,
        "published_errors_vs_torch": {r: e["values"] for r, e in src["errors"].items()},
    }
    dst = Path(__file__).resolve().parent / "dspark_b7_workload.json"
    dst.write_text(json.dumps(out, separators=(",", ":")) + "\n")
    print(dst, dst.stat().st_size)


if __name__ == "__main__":
    main(*sys.argv[1:])

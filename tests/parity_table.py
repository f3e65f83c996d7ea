"""Render the parity records ``test_benchmark_configuration`` writes (``$AYAKA_PARITY_DIR``)
as a markdown table: per configuration, the raw max-abs and relative-L2 error against the
float32 gather-then-softmax oracle of our launches, beside the reference's own rounding of
that float32 result (the error any implementation that returns the dtype carries).

Usage: python tests/parity_table.py DIR > profiles/parity.md
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

COLUMNS = (("reference_rounding", "reference (fp32 oracle rounded once)"), ("auto", "ours, library's launch"),
           ("v1-mfma", "ours, v1"), ("v2-mfma", "ours, v2 (partitions of 512)"))


def main(directory: str) -> int:
    records = [json.loads(p.read_text()) for p in sorted(Path(directory).glob("parity_c*.json"))]
    print("| config | rows | launch | result | max-abs vs fp32 oracle | rel-L2 vs fp32 oracle | "
          "max-abs excess vs fp64 (net of half an ulp) | rel-L2 vs fp64 rounded once |")
    print("|---|---|---|---|---|---|---|---|")
    for r in records:
        for key, label in COLUMNS:
            m = r[key]
            print(f"| {r['config']} ({r['dtype']}) | {r['rows']} | {r['auto_launch']} | {label} | {m['max_abs']:.3e} | "
                  f"{m['rel_l2']:.3e} | {m['max_abs_excess_fp64']:.3e} | {m['rel_l2_rounded_fp64']:.3e} |")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1]))

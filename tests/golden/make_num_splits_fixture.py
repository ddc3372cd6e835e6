"""Extract the known-answer table for get_num_splits from the reference's results.

The reference's `triton-mla-bench --csv` writes one row per (batch, seqlen)
with the split count it used, get_num_splits(batch, heads, seqlen, num_sms)
(src/triton_mla/bench.py:66), measured on an H100 (num_sms = 132). This script
reads the two committed CSVs of the reference and writes their
(batch, seqlen, heads, num_splits) columns as a JSON fixture. It only reads
data files; it imports nothing from the reference.

    python tests/golden/make_num_splits_fixture.py /root/reference/results
"""

import csv
import json
import os
import sys


def main(results_dir: str) -> None:
    rows = []
    for name in ("bench_h100.csv", "bench_h100_untuned.csv"):
        with open(os.path.join(results_dir, name), newline="") as f:
            for rec in csv.DictReader(f):
                rows.append({"source": f"results/{name}", "gpu": rec["gpu"], "batch": int(rec["batch"]),
                             "seqlen": int(rec["seqlen"]), "heads": int(rec["heads"]),
                             "num_splits": int(rec["num_splits"])})
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "num_splits_h100.json")
    with open(out, "w") as f:
        json.dump({"num_sms": 132, "rows": rows}, f, indent=1)
    print(f"wrote {len(rows)} rows to {out}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/results")

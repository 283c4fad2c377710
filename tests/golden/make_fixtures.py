"""Writes tests/golden/reference_synth_metrics.json: the per-case metrics that the reference's saved runs of kcholf
hold (results/synth_kcholf.json on an RTX 4080 Laptop, results/synth_kcholf_rtx5060ti.json on an RTX 5060 Ti).

Only data is taken: for every (K, r, case) row the input's condition number (which fingerprints the generated
matrix) and the metrics of the reference's Q (orth, span_n, hh_span_n, bad_cols, deterministic). No reference code
is imported or run. Run from the repository root with the reference checked out at /root/reference:

    python tests/golden/make_fixtures.py [/root/reference]
"""
import json
import os
import sys

FILES = {"rtx4080_laptop": "results/synth_kcholf.json", "rtx5060ti": "results/synth_kcholf_rtx5060ti.json"}
KEYS = ("cond", "orth", "span_n", "hh_span_n", "bad_cols", "deterministic", "hard")


def main(ref_root="/root/reference"):
    out = {"source": {k: v for k, v in FILES.items()}, "rows": {}}
    for dev, rel in FILES.items():
        with open(os.path.join(ref_root, rel)) as f:
            data = json.load(f)
        for row in data["rows"]:
            if row.get("method") != "kcholf":
                continue
            key = f'{row["K"]}x{row["r"]}/{row["case"]}'
            ent = out["rows"].setdefault(key, {})
            ent[dev] = {k: row.get(k) for k in KEYS}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_synth_metrics.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(f"{len(out['rows'])} rows -> {dst}")


if __name__ == "__main__":
    main(*sys.argv[1:])

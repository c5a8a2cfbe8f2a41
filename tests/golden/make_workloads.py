"""Writes reference_workloads.json: the workload tables of the reference's evaluation as data, for
tests/test_workloads.py.  Run in a container that holds the reference (read as data, nothing of it is imported):

    python tests/golden/make_workloads.py /path/to/reference

Sources: kda/mi350x/workloads/workloads.json (the eval's tables, exported from eval_kda_mi350x.py:92-130,715-767) and
kda/mi350x/workloads/legacy_{prefill,decode}_baseline_sota.json (the recorded phase-1 baselines)."""
import json
import sys
from pathlib import Path

TABLES = ("PREFILL_WORKLOADS", "DECODE_WORKLOADS", "LEGACY_PREFILL", "LEGACY_DECODE", "DECODE_HELDOUT",
          "NUMERIC_PROBES")


def main(ref):
    wl = Path(ref) / "kda" / "mi350x" / "workloads"
    src = json.loads((wl / "workloads.json").read_text())
    out = {"source": "kda/mi350x/workloads/workloads.json, legacy_prefill_baseline_sota.json, "
                     "legacy_decode_baseline_sota.json",
           "constants": src["constants"],
           "tables": {t: src["tables"][t]["data"] for t in TABLES},
           "legacy_prefill_baseline_ms": json.loads((wl / "legacy_prefill_baseline_sota.json").read_text())["latency_ms"],
           "legacy_decode_baseline_us": json.loads((wl / "legacy_decode_baseline_sota.json").read_text())["latency_us"]}
    dst = Path(__file__).resolve().parent / "reference_workloads.json"
    dst.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {dst}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

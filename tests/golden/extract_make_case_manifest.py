"""Extract the published make_case SHA-256 manifests into a fixture.

Reads the reference's own benchmark record
reports/data/engine_comparison_20261026.json (cases B1/ctx128, B8/ctx512,
B32/ctx2048; seed 20261026, fp16, block 256) and writes the input-tensor
hashes to tests/golden/make_case_manifest.json.  Run in the container that
has the reference checkout; no GPU run uses this script.
"""

import json
from pathlib import Path

SOURCE = Path("/root/reference/reports/data/engine_comparison_20261026.json")
TARGET = Path(__file__).resolve().parent / "make_case_manifest.json"


def find_cases(node, found):
    if isinstance(node, dict):
        if "case_sha256" in node and "tensors" in node and "shape" in node:
            found.append({"shape": node["shape"], "tensors": node["tensors"], "case_sha256": node["case_sha256"]})
        for value in node.values():
            find_cases(value, found)
    elif isinstance(node, list):
        for value in node:
            find_cases(value, found)


def main():
    found = []
    find_cases(json.loads(SOURCE.read_text()), found)
    unique = {json.dumps(case, sort_keys=True) for case in found}
    cases = sorted((json.loads(u) for u in unique), key=lambda c: (c["shape"]["batch"], c["shape"]["context"]))
    TARGET.write_text(json.dumps({"source": "reports/data/engine_comparison_20261026.json",
                                  "cases": cases}, indent=1) + "\n")
    print(f"wrote {len(cases)} cases to {TARGET}")


if __name__ == "__main__":
    main()

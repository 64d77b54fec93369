"""Extract the reference's recorded MoE known-answer data into a small fixture.

Reads only the JSON result records that ship with the reference
(``results/m4-moe-20261006T094645Z-376040740.json``: written by
``moe_benchmark.py:_case_metadata`` :411-418 and ``validate_dispatch`` :139-190)
and keeps, per case, the generator arguments together with the recorded
``routing_sha256`` / ``input_sha256`` digests and the expected per-expert
counts and offsets.  Nothing from the reference is imported or executed.

Run in the build container (the reference is not present on the GPU box):
    python tests/golden/make_reference_records.py
"""
import json
from pathlib import Path

SOURCE = Path("/root/reference/results/m4-moe-20261006T094645Z-376040740.json")
OUT = Path(__file__).with_name("m4_reference_records.json")

FUNCTIONAL_EXTRA = {  # moe_benchmark.py:356-377 flags that are not in the record
    "nonpower_experts_signed_weights": {"signed_weights": True},
}


def main():
    record = json.loads(SOURCE.read_text())
    cases = []
    for family in ("functional_cases", "performance_cases"):
        for case in record[family]:
            entry = {k: case[k] for k in ("name", "T", "E", "topk", "H", "I", "id_dtype",
                                           "route_pattern", "seed", "routing_sha256",
                                           "input_sha256")}
            entry["family"] = family
            entry.update(FUNCTIONAL_EXTRA.get(case["name"], {}))
            dv = case.get("dispatch_validation") or {}
            if "expected_counts" in dv:
                entry["expected_counts"] = dv["expected_counts"]
                entry["expected_offsets"] = dv["expected_offsets"]
            cases.append(entry)
    OUT.write_text(json.dumps({"source": str(SOURCE.name), "cases": cases}, indent=1) + "\n")
    print(f"wrote {len(cases)} cases to {OUT}")


if __name__ == "__main__":
    main()

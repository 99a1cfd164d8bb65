"""Writes tests/golden/saved_mugraphs/qknorm_gqa_bs1_subset.json: the first
graph of each distinct operator structure (kernel op types and threadblock
op types, in order) of the reference's benchmark/saved_mugraphs/cuda/
qknorm_gqa_bs1.json (190 saved candidates, 1.8 MB), up to 12 graphs.  The
graphs are copied unchanged; run once, in a container holding the
reference, from the repository root."""
import json
import os
import sys

SRC = os.path.join(sys.argv[1] if len(sys.argv) > 1 else "/root/reference",
                   "benchmark", "saved_mugraphs", "cuda", "qknorm_gqa_bs1.json")
DST = os.path.join(os.path.dirname(__file__), "saved_mugraphs", "qknorm_gqa_bs1_subset.json")


def structure(graph):
    sig = []
    for op in graph:
        sig.append(op["op_type"])
        if op["op_type"] == "kn_customized_op":
            sig.append(tuple(t["op_type"] for t in op["bgraph"]["operators"]))
    return tuple(sig)


def main():
    with open(SRC) as f:
        graphs = json.load(f)
    seen, keep = set(), []
    for g in graphs:
        s = structure(g)
        if s not in seen:
            seen.add(s)
            keep.append(g)
        if len(keep) == 12:
            break
    with open(DST, "w") as f:
        json.dump(keep, f)
    print(f"{len(keep)} of {len(graphs)} graphs -> {DST}")


if __name__ == "__main__":
    main()

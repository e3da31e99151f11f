"""Copy the reference's captured decode graph into tests/golden/ as fixtures.

Data only: k0/schedule.csv (one row per ggml node of the Qwen3.6-27B decode
graph), k0/leaves.csv (one row per leaf tensor) and the compiled program's
meta block from k0/program.json (structural counts of the reference's own
schedule compile: nodes emitted and dropped, boundaries per pass, the DRAM
bytes formula).  Run from the repository root where the reference checkout
is mounted at /root/reference:

    python tests/golden/copy_graph_fixtures.py [--check]

--check only verifies that the committed copies equal the reference's files.
"""
import hashlib
import json
import os
import shutil
import sys

REF = "/root/reference/k0"
HERE = os.path.dirname(os.path.abspath(__file__))
FILES = {"schedule.csv": "k0_schedule.csv", "leaves.csv": "k0_leaves.csv"}
SHA256 = {
    "k0_schedule.csv": "98e488b2332ed69eee87056a8aad2cc7cb7524961b05bcc416084524c08bff75",
    "k0_leaves.csv": "ad3c7e1e792f09f8aa5499c8998135c071783822a77d8091fab5c3a512e46540",
}


def sha(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def main():
    check = "--check" in sys.argv
    for src, dst in FILES.items():
        d = os.path.join(HERE, dst)
        if not check:
            shutil.copyfile(os.path.join(REF, src), d)
        assert sha(d) == SHA256[dst], dst
        if os.path.exists(os.path.join(REF, src)):
            assert sha(os.path.join(REF, src)) == SHA256[dst], src
    meta_out = os.path.join(HERE, "k0_program_meta.json")
    with open(os.path.join(REF, "program.json")) as f:
        meta = json.load(f)["meta"]
    keep = {k: meta[k] for k in ("source", "isa", "split", "coverage", "per_pass")}
    keep["drops"] = [{"reason": d["reason"], "count": d["count"]} for d in meta["drops"]]
    text = json.dumps(keep, indent=1, sort_keys=True) + "\n"
    if check:
        assert open(meta_out).read() == text, "k0_program_meta.json differs"
    else:
        with open(meta_out, "w") as f:
            f.write(text)
    print("ok")


if __name__ == "__main__":
    main()

"""Writes tests/golden/bank/: the dev split of the reference's challenge bank
(evidence/inputs/challenge-bank-v1.jsonl, 90 of its 270 JSON lines, copied
unchanged) and the published dev-split evaluations of it
(evidence/inputs/bank-{original,geometry,goal,static,dynamic}.csv, trimmed to
the level id, protocol and outcome columns), plus tests/golden/actors/
<policy>.npz for the two checkpoints those evaluations name besides the
guided one: the actor parameters and SimConfig bytes, SHA-256 checked
against the evaluations' checkpoint_sha256 column.  The bank is checked
against their bank_sha256.  Reads the reference tree; run it where that tree
is present:

    python tests/golden/make_bank_fixtures.py [/root/reference]
"""
import csv
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
INPUTS = os.path.join(REF, "evidence", "inputs")
EVALUATIONS = ["original", "geometry", "goal", "static", "dynamic"]
KEEP = ["failure_id", "split", "family", "seed", "base_seed", "environment_index", "distance_m", "mode", "speed_mps",
        "max_steps", "episodes", "success", "collision", "timeout", "progress", "path_m", "elapsed_s", "goal_time_s",
        "mean_speed_mps", "peak_speed_mps", "min_clearance_m", "checkpoint_sha256", "bank_sha256"]
CHECKPOINTS = {"clean_stress": "guided-clean-stress.bin.best", "threat_joint": "guided-threat-joint.bin.best",
               "table_memory": "guided-table-memory.bin.best"}


def sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def main():
    out = os.path.join(HERE, "bank")
    os.makedirs(out, exist_ok=True)
    bank = os.path.join(INPUTS, "challenge-bank-v1.jsonl")
    bank_sha = sha(bank)
    named = set()
    for name in EVALUATIONS:
        rows = list(csv.DictReader(open(os.path.join(INPUTS, "bank-%s.csv" % name))))
        assert all(r["bank_sha256"] == bank_sha for r in rows), name
        named.update(r["checkpoint_sha256"] for r in rows)
        with open(os.path.join(out, "bank-%s.csv" % name), "w", newline="") as f:
            w = csv.DictWriter(f, KEEP)
            w.writeheader()
            for r in rows:
                w.writerow({k: r[k] for k in KEEP})
    import json
    with open(os.path.join(out, "challenge-bank-v1-dev.jsonl"), "w") as f:
        for line in open(bank):
            if json.loads(line)["split"] == "dev":
                f.write(line)
    for cand, name in CHECKPOINTS.items():
        path = os.path.join(REF, "assets", "checkpoints", name)
        digest = sha(path)
        assert digest in named, name
        if cand == "table_memory":
            continue  # the full checkpoint is a fixture already
        data = open(path, "rb").read()
        assert data[:8] == b"PPOFIX1\0" and int(np.frombuffer(data[12:16], np.uint32)[0]) == 12104
        np.savez(os.path.join(HERE, "actors", cand + ".npz"), actor=np.frombuffer(data[136:136 + 4 * 12104], np.float32),
                 config=np.frombuffer(data[48:132], np.uint8), sha256=np.frombuffer(bytes.fromhex(digest), np.uint8))
    print("bank fixtures ok", bank_sha[:12])


if __name__ == "__main__":
    main()

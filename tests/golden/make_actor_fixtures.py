"""Writes tests/golden/actors/<checkpoint>.npz: the actor parameters and the
simulator config of the reference's trained PPOFIX1 checkpoints whose
evaluations the reference published in assets/continuation-evaluation.csv
(checked by SHA-256 against that file), and of the goal-arrival checkpoint of
evidence/inputs/arrival-training (checked against its manifest), so the tests carry 48 KB per policy
instead of the 1.6 MB checkpoints.  Reads the reference tree; run it where
that tree is present:

    python tests/golden/make_actor_fixtures.py [/root/reference]
"""
import csv
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
CHECKPOINTS = {"broad_stress": "guided-stress.bin.best", "door_stress": "guided-door-stress.bin.best",
               "rehearsal": "guided-rehearsal.bin.best"}


# the goal-arrival policy of the reference's task-training evidence, checked
# against evidence/inputs/arrival-training/manifest.json
ARRIVAL = ("arrival", "arrival-open-domain-experimental.bin.best")


def arrival_fixture():
    import json
    manifest = json.load(open(os.path.join(REF, "evidence", "inputs", "arrival-training", "manifest.json")))
    name = ARRIVAL[1]
    data = open(os.path.join(REF, "assets", "checkpoints", name), "rb").read()
    assert hashlib.sha256(data).hexdigest() == manifest["source_hashes"]["assets/checkpoints/" + name], name
    assert data[:8] == b"PPOFIX1\0"
    actor_count = int(np.frombuffer(data[12:16], np.uint32)[0])
    assert actor_count == 12104
    config = np.frombuffer(data[48:132], np.uint8).copy()
    actor = np.frombuffer(data[136:136 + 4 * 12104], np.float32).copy()
    sha = hashlib.sha256(data).hexdigest()
    np.savez(os.path.join(HERE, "actors", ARRIVAL[0] + ".npz"), actor=actor, config=config,
             sha256=np.frombuffer(bytes.fromhex(sha), np.uint8))
    print(ARRIVAL[0], name, "ok")


def main():
    rows = list(csv.DictReader(open(os.path.join(REF, "assets", "continuation-evaluation.csv"))))
    sha = {r["candidate"]: r["checkpoint_sha256"] for r in rows}
    os.makedirs(os.path.join(HERE, "actors"), exist_ok=True)
    for cand, name in CHECKPOINTS.items():
        data = open(os.path.join(REF, "assets", "checkpoints", name), "rb").read()
        assert hashlib.sha256(data).hexdigest() == sha[cand], (cand, name)
        assert data[:8] == b"PPOFIX1\0"
        version, actor_count = np.frombuffer(data[8:16], np.uint32)
        assert version == 6 and actor_count == 12104
        config = np.frombuffer(data[48:132], np.uint8).copy()  # SimConfig, 84 bytes
        actor = np.frombuffer(data[136:136 + 4 * 12104], np.float32).copy()
        np.savez(os.path.join(HERE, "actors", cand + ".npz"), actor=actor, config=config,
                 sha256=np.frombuffer(bytes.fromhex(sha[cand]), np.uint8))
        print(cand, name, "ok")
    arrival_fixture()


if __name__ == "__main__":
    main()

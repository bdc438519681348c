"""Challenge-bank levels (challenge_evaluation.hpp:163-283) parsed from the
dev split of the reference's bank (tests/golden/bank): the seed derivation
holds for every level, starts and goals are clear of obstacles under the
oracle's clearance (the parser's own safety contract, 0.04 m), and the
stored direct routes are blocked while the witness routes are clear."""
import json
import os

import numpy as np

from mdnav import abi, load_bank
from oracle_lib import GOLDEN, oracle, ptr

BANK = os.path.join(GOLDEN, "bank", "challenge-bank-v1-dev.jsonl")


def test_bank_dev_split_parses():
    levels = load_bank(BANK, "dev")
    assert len(levels) == 90
    assert sorted({lv["family"] for lv in levels}) == [14, 15, 16]
    assert load_bank(BANK, "train") == []


def test_bank_levels_satisfy_their_contracts():
    levels = load_bank(BANK, "dev")
    recs = [json.loads(line) for line in open(BANK)]
    worlds = np.array([lv["world"] for lv in levels], abi.WORLD)
    pts = np.array([[0, 0, 1.5] for _ in levels] + [lv["world"]["goal"] for lv in levels], np.float32)
    w2 = np.concatenate([worlds, worlds])
    out = np.zeros(len(pts), np.float32)
    oracle().orc_clearance_batch(ptr(w2), ptr(pts), ptr(np.zeros(len(pts), np.float32)), ptr(out), len(pts))
    assert (out > 0.04).all(), out.min()
    # stored route clearances: the direct line is blocked, the witness route clear,
    # sampled every 2 cm here (the bank's own sampling is not stated)
    for lv, rec in zip(levels, recs):
        route = np.array(rec["witness_route"], np.float32)
        seg = []
        for a, b in zip(route[:-1], route[1:]):
            k = max(2, int(np.linalg.norm(b - a) / 0.02))
            seg.append(a + (b - a) * np.linspace(0, 1, k, dtype=np.float32)[:, None])
        p = np.concatenate(seg).astype(np.float32)
        ww = np.repeat(lv["world"][None], len(p))
        cl = np.zeros(len(p), np.float32)
        oracle().orc_clearance_batch(ptr(ww), ptr(p), ptr(np.zeros(len(p), np.float32)), ptr(cl), len(p))
        assert cl.min() > 0.0, (lv["failure_id"], cl.min(), rec["witness_min_clearance_m"])
        assert abs(cl.min() - rec["witness_min_clearance_m"]) < 0.05
        assert rec["direct_route_clearance_m"] < -0.02

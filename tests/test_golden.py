"""Determinism of the seeded inputs and the oracle across hosts: digests of
generated weights, positions and oracle outputs must match the committed
fixtures bit for bit (tests/golden/make_golden.py)."""

import hashlib
import json
import os

import numpy as np

import oracle
from metalfish_amd import synth

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "seeded.json")))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_cpu_plumbing_weights_and_oracle():
    spec = synth.SPECS["cpu_plumbing"]
    w = synth.make_weights(spec, seed=0)
    assert sha(np.concatenate([w[k].reshape(-1) for k in sorted(w)])) == \
        GOLD["cpu_plumbing_weights_sha256"]
    planes, legal, moves = synth.playout_positions(16, seed=0, with_moves=True)
    assert sha(planes) == GOLD["playout16_planes_sha256"]
    assert sha(legal) == GOLD["playout16_legal_sha256"]
    assert moves[:3] == GOLD["playout16_moves_first3"]
    ref = oracle.OracleNet(oracle.NetFormat(body_heads=spec.heads), w).evaluate_batch(planes)
    assert [float(x) for x in ref["policy"][0, :4]] == GOLD["cpu_plumbing_policy0_first4"]
    assert sha(ref["policy"]) == GOLD["cpu_plumbing_policy_sha256"]
    assert sha(ref["wdl"]) == GOLD["cpu_plumbing_wdl_sha256"]


def test_bt4_weights_and_oracle_first_positions():
    spec = synth.SPECS["bt4"]
    w = synth.make_weights(spec, seed=0)
    assert sha(np.concatenate([w[k].reshape(-1) for k in sorted(w)])) == GOLD["bt4_weights_sha256"]
    planes, _ = synth.playout_positions(4, seed=0)
    ref = oracle.OracleNet(oracle.NetFormat(body_heads=spec.heads), w).evaluate_batch(planes)
    gold = np.load(os.path.join(HERE, "golden", "bt4_seed0_4pos.npz"))
    assert np.array_equal(ref["policy"], gold["policy"])
    assert np.array_equal(ref["wdl"], gold["wdl"])
    assert sha(ref["policy"]) == GOLD["bt4_policy_sha256"]

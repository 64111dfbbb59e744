"""Writes the golden fixtures under tests/golden/ (run in the build container).

* reference_tables.json -- SHA-256 digests of the reference's own policy
  tables, dumped by oracle/_ref/ref_tables_dump (compiled from the
  reference's src/nn/policy_map.cpp and tables/attention_policy_map.h by
  oracle/Makefile): kAttnPolicyMap (4288 int16), MoveToNNIndex over every
  (from, to, promotion) (64*64*5 int16), IndexToNNMove (1858 x 3 int16), and both again under
  the input transforms 1..7.
  Digests only: the tables themselves are not copied into this repository.
* seeded.json -- digests of this repository's seeded inputs and of the CPU
  oracle's outputs on them (pins the generator, the encoder and the oracle
  across hosts), plus a few literal values for readable failures.
* bt4_seed0_4pos.npz -- oracle policy logits and WDL for the first 4
  seeded positions of the BT4-shape net (seed 0).

Usage: python tests/golden/make_golden.py
"""

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from metalfish_amd import synth  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def reference_tables():
    path = os.path.join(ROOT, "oracle", "_ref", "ref_tables.bin")
    n16 = 4288 + 64 * 64 * 5 + 1858 * 3
    data = open(path, "rb").read()
    raw = np.frombuffer(data[:2 * n16], dtype=np.int16)
    amap = raw[:4288]
    idx = raw[4288:4288 + 64 * 64 * 5]
    inv = raw[4288 + 64 * 64 * 5:]
    pos = np.frombuffer(data[2 * n16:2 * n16 + 4 * 64 * 64], dtype=np.float32)
    rest = np.frombuffer(data[2 * n16 + 4 * 64 * 64:], dtype=np.int16)
    idx_t = rest[:7 * 64 * 64 * 5]
    inv_t = rest[7 * 64 * 64 * 5:]
    assert inv.size == 1858 * 3 and pos.size == 64 * 64 and inv_t.size == 7 * 1858 * 3
    return {"source": "oracle/_ref/ref_tables.bin (reference policy_map.cpp + "
                      "tables/attention_policy_map.h)",
            "attn_policy_map_sha256": sha(amap),
            "move_to_nn_index_sha256": sha(idx),
            "index_to_nn_move_sha256": sha(inv),
            "pos_encoding_sha256": sha(pos),
            "move_to_nn_index_transforms_1_7_sha256": sha(idx_t),
            "index_to_nn_move_transforms_1_7_sha256": sha(inv_t)}


def seeded():
    out = {}
    spec = synth.SPECS["cpu_plumbing"]
    w = synth.make_weights(spec, seed=0)
    out["cpu_plumbing_weights_sha256"] = sha(np.concatenate(
        [w[k].reshape(-1) for k in sorted(w)]))
    planes, legal, moves = synth.playout_positions(16, seed=0, with_moves=True)
    out["playout16_planes_sha256"] = sha(planes)
    out["playout16_legal_sha256"] = sha(legal)
    out["playout16_moves_first3"] = moves[:3]
    ref = oracle.OracleNet(oracle.NetFormat(body_heads=spec.heads), w).evaluate_batch(planes)
    out["cpu_plumbing_policy_sha256"] = sha(ref["policy"])
    out["cpu_plumbing_wdl_sha256"] = sha(ref["wdl"])
    out["cpu_plumbing_policy0_first4"] = [float(x) for x in ref["policy"][0, :4]]
    out["cpu_plumbing_wdl0"] = [float(x) for x in ref["wdl"][0]]
    bt4 = synth.SPECS["bt4"]
    wb = synth.make_weights(bt4, seed=0)
    out["bt4_weights_sha256"] = sha(np.concatenate([wb[k].reshape(-1) for k in sorted(wb)]))
    refb = oracle.OracleNet(oracle.NetFormat(body_heads=bt4.heads), wb).evaluate_batch(planes[:4])
    np.savez_compressed(os.path.join(HERE, "bt4_seed0_4pos.npz"), policy=refb["policy"],
                        wdl=refb["wdl"])
    out["bt4_policy_sha256"] = sha(refb["policy"])
    out["bt4_wdl_sha256"] = sha(refb["wdl"])
    return out


def main():
    with open(os.path.join(HERE, "reference_tables.json"), "w") as f:
        json.dump(reference_tables(), f, indent=1)
    with open(os.path.join(HERE, "seeded.json"), "w") as f:
        json.dump(seeded(), f, indent=1)
    print("golden fixtures written")


if __name__ == "__main__":
    main()

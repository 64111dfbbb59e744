"""Policy move index and attention gather table against the reference's own
tables (digests of oracle/_ref's dump of reference src/nn/policy_map.cpp and
tables/attention_policy_map.h; see tests/golden/make_golden.py)."""

import hashlib
import json
import os

import numpy as np
import pytest

from metalfish_amd import synth
from oracle import policy_tables as opt

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "reference_tables.json")))
REF_BIN = os.path.join(os.path.dirname(HERE), "oracle", "_ref", "ref_tables.bin")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _move_to_index_table(move_to_index):
    out = np.full((64, 64, 5), -1, dtype=np.int16)
    for f in range(64):
        for t in range(64):
            if f == t:
                continue
            for p, ch in enumerate(("", "q", "r", "b", "n")):
                out[f, t, p] = move_to_index(f, t, ch)
    return out


def _index_to_move_table(moves):
    kind = {"": 0, "q": 5, "r": 4, "b": 3}  # reference PieceType values
    return np.array([[f, t, kind[p]] for f, t, p in moves], dtype=np.int16)


def test_product_attention_map_matches_reference():
    amap, gather, names = synth.policy_tables()
    assert sha(amap) == GOLD["attn_policy_map_sha256"]
    assert len(names) == 1858 and names[0] == "a1b1" and names[1792] == "a7a8q"
    # gather is the inverse of the map on every policy index.
    assert all(amap[gather[i]] == i for i in range(1858))


def test_oracle_attention_map_matches_reference():
    assert sha(opt.attention_map()) == GOLD["attn_policy_map_sha256"]


def test_oracle_move_index_matches_reference():
    moves = opt.move_list()
    lookup = {}
    for i, (f, t, p) in enumerate(moves):
        lookup[(f, t, p)] = i

    def move_to_index(f, t, p):
        if p == "n":
            p = ""  # knight promotion is the plain move (policy_map.cpp:338-340)
        return lookup.get((f, t, p), -1)

    assert sha(_move_to_index_table(move_to_index)) == GOLD["move_to_nn_index_sha256"]
    assert sha(_index_to_move_table(moves)) == GOLD["index_to_nn_move_sha256"]


@pytest.mark.skipif(not os.path.exists(REF_BIN), reason="oracle/_ref not built")
def test_reference_dump_matches_committed_digests():
    data = open(REF_BIN, "rb").read()
    raw = np.frombuffer(data, dtype=np.int16)
    assert sha(raw[:4288]) == GOLD["attn_policy_map_sha256"]
    assert sha(raw[4288:4288 + 64 * 64 * 5]) == GOLD["move_to_nn_index_sha256"]
    n16 = 4288 + 64 * 64 * 5 + 1858 * 3
    pos = np.frombuffer(data[2 * n16:2 * n16 + 4 * 64 * 64], dtype=np.float32)
    assert sha(pos) == GOLD["pos_encoding_sha256"]
    rest = np.frombuffer(data[2 * n16 + 4 * 64 * 64:], dtype=np.int16)
    assert sha(rest[:7 * 64 * 64 * 5]) == GOLD["move_to_nn_index_transforms_1_7_sha256"]
    assert sha(rest[7 * 64 * 64 * 5:]) == GOLD["index_to_nn_move_transforms_1_7_sha256"]


def test_product_move_index_under_transforms_matches_reference():
    """MoveToNNIndex / IndexToNNMove with the canonical formats' input
    transforms 1..7 (reference policy_map.cpp:305-410), every (from, to,
    promotion) and every index, against digests of the reference's own
    functions.  Under a transpose the reference maps squares by a half turn
    rather than by the planes' reflection; the digests hold it to that."""
    fwd = np.concatenate([
        _move_to_index_table(lambda f, t, p, tr=tr: synth.move_to_index(f, t, p, tr)).ravel()
        for tr in range(1, 8)])
    assert sha(fwd) == GOLD["move_to_nn_index_transforms_1_7_sha256"]
    inv = np.concatenate([
        _index_to_move_table([synth.index_to_move(i, tr) for i in range(1858)]).ravel()
        for tr in range(1, 8)])
    assert sha(inv) == GOLD["index_to_nn_move_transforms_1_7_sha256"]
    # Transform 0 through the same entry points: the plain tables.
    assert sha(_move_to_index_table(synth.move_to_index)) == GOLD["move_to_nn_index_sha256"]
    assert sha(_index_to_move_table([synth.index_to_move(i) for i in range(1858)])) == \
        GOLD["index_to_nn_move_sha256"]


def test_static_position_encoding_matches_reference():
    """PE_MAP table (reference tables/attention_policy_map.h:377, kPosEncoding)
    rebuilt from its rule, in the product and in the oracle."""
    assert sha(synth.static_position_encoding()) == GOLD["pos_encoding_sha256"]
    assert sha(opt.pos_encoding()) == GOLD["pos_encoding_sha256"]


def test_encoder_policy_roundtrip_g1f3():
    """reference tests/test_nn_comparison.cpp:224-245: g1f3 has a valid
    index that maps back to g1f3."""
    _, _, names = synth.policy_tables()
    _, legal = synth.encode_game("", "")
    idx = [i for i in legal if names[i] == "g1f3"]
    assert len(idx) == 1

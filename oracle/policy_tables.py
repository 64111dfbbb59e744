"""CPU ORACLE -- TEST INFRASTRUCTURE ONLY.

Independent Python construction of the 1858-move policy list and the
attention-policy gather table used by the oracle's policy-map step.  It
restates the definition behind reference ``src/nn/policy_map.cpp:35-245``
(move list) and ``src/nn/tables/attention_policy_map.h:15`` (kAttnPolicyMap):
queen-line and knight moves ordered by from-square then to-square, then the
q/r/b promotions ordered by from-file, to-file, piece; raw attention index
from*64+to for plain moves and 4096 + from_file*24 + to_file*3 + piece for
promotions.  Pinned bit-exact against the reference's compiled table by
tests/test_policy_tables.py.
"""

import numpy as np


def _queen_line(f, t):
    df, dr = (t & 7) - (f & 7), (t >> 3) - (f >> 3)
    return f != t and (df == 0 or dr == 0 or abs(df) == abs(dr))


def _knight(f, t):
    df, dr = abs((t & 7) - (f & 7)), abs((t >> 3) - (f >> 3))
    return (df, dr) in ((1, 2), (2, 1))


def move_list():
    moves = []
    for f in range(64):
        for t in range(64):
            if _queen_line(f, t) or _knight(f, t):
                moves.append((f, t, ""))
    for ff in range(8):
        for tf in (ff - 1, ff, ff + 1):
            if 0 <= tf < 8:
                for p in "qrb":
                    moves.append((48 + ff, 56 + tf, p))
    assert len(moves) == 1858
    return moves


def attention_map():
    amap = np.full(64 * 64 + 192, -1, dtype=np.int16)
    for i, (f, t, p) in enumerate(move_list()):
        if p:
            amap[4096 + (f & 7) * 24 + (t & 7) * 3 + "qrb".index(p)] = i
        else:
            amap[f * 64 + t] = i
    return amap


def gather_table():
    """policy index -> raw attention index (AttentionPolicyGatherMap,
    reference src/nn/cpu/cpu_network.cpp:91-103)."""
    g = np.full(1858, -1, dtype=np.int32)
    for raw, idx in enumerate(attention_map()):
        if idx >= 0:
            g[idx] = raw
    return g


def uci_strings():
    names = []
    for f, t, p in move_list():
        names.append("%s%d%s%d%s" % ("abcdefgh"[f & 7], (f >> 3) + 1, "abcdefgh"[t & 7],
                                     (t >> 3) + 1, p))
    return names


def pos_encoding():
    """Static position encoding of PE_MAP nets, [square][channel] float32:
    -1 on the square itself, 1 where a queen or knight move from the square
    lands, 0 elsewhere (the rule behind reference
    src/nn/tables/attention_policy_map.h:377, kPosEncoding).  Pinned against
    the digest of the reference's table by tests/test_policy_tables.py."""
    t = np.zeros((64, 64), dtype=np.float32)
    for s_ in range(64):
        for c in range(64):
            t[s_, c] = -1.0 if s_ == c else (1.0 if _queen_line(s_, c) or _knight(s_, c)
                                             else 0.0)
    return t

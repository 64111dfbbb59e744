"""Input generation and the packed-input contract.

Pins: perft counts (published values for the standard test positions), the
start-position packed fixture (reference tests/nn_input_fixture.h:35-58,
nn_input_fixture.cpp:60-106), the repetition plane (reference
tests/test_nn_comparison.cpp:304-341), black-to-move board flip, and
PackInputPlanesRaw (reference src/nn/input_plane_packing.h:30-83) between the
oracle and the product's C ABI packer.
"""

import numpy as np
import pytest

import oracle
from metalfish_amd import backend, synth

START = "rnbqkbnr/pppppppp/8/8/8/8/PPPPPPPP/RNBQKBNR w KQkq - 0 1"
FULL = 0xFFFFFFFFFFFFFFFF

PERFT = [
    (START, [20, 400, 8902, 197281]),
    ("r3k2r/p1ppqpb1/bn2pnp1/3PN3/1p2P3/2N2Q1p/PPPBBPPP/R3K2R w KQkq - 0 1", [48, 2039, 97862]),
    ("8/2p5/3p4/KP5r/1R3p1k/8/4P1P1/8 w - - 0 1", [14, 191, 2812, 43238]),
    ("r3k2r/Pppp1ppp/1b3nbN/nP6/BBP1P3/q4N2/Pp1P2PP/R2Q1RK1 w kq - 0 1", [6, 264, 9467]),
    ("rnbq1k1r/pp1Pbppp/2p5/8/2B5/8/PPP1NnPP/RNBQK2R w KQ - 1 8", [44, 1486, 62379]),
]


@pytest.mark.parametrize("fen,counts", PERFT)
def test_perft(fen, counts):
    for depth, want in enumerate(counts, start=1):
        assert synth.perft(fen, depth) == want


def test_start_position_packed_fixture():
    planes, _ = synth.encode_game(START, "")
    masks, values = oracle.pack_planes(planes[None])
    masks, values = masks[0], values[0]
    checks = [(0, 0x000000000000FF00), (1, 0x42), (2, 0x24), (3, 0x81), (4, 0x08), (5, 0x10),
              (6, 0x00FF000000000000), (7, 0x4200000000000000), (8, 0x2400000000000000),
              (9, 0x8100000000000000), (10, 0x0800000000000000), (11, 0x1000000000000000),
              (12, 0), (104, FULL), (105, FULL), (106, FULL), (107, FULL), (111, FULL)]
    for plane, mask in checks:
        assert int(masks[plane]) == mask, plane
        assert values[plane] == (1.0 if mask else 0.0)
    assert int(np.count_nonzero(masks)) == 17
    assert int(np.sum(masks == np.uint64(FULL))) == 5
    assert not masks[13:104].any()  # no synthetic history through the start position
    for plane in (108, 109, 110):
        assert masks[plane] == 0 and values[plane] == 0.0


def test_repetition_plane_after_knight_dance():
    planes, _ = synth.encode_game(START, "g1f3 g8f6 f3g1 f6g8")
    assert np.all(planes[12] == 1.0)      # current position repeats the start
    assert np.all(planes[13 + 12] == 0.0)  # previous position has no repetition


def test_black_to_move_is_flipped():
    planes, _ = synth.encode_game(START, "e2e4")
    # Black to move: "our" pawns (black) appear on rank 2 after the flip.
    assert int(np.flatnonzero(planes[0]).min()) == 8
    assert np.all(planes[108] == 1.0)


def test_playouts_are_deterministic_and_legal():
    a, la = synth.playout_positions(8, seed=5)
    b, lb = synth.playout_positions(8, seed=5)
    c, _ = synth.playout_positions(8, seed=6)
    assert np.array_equal(a, b) and np.array_equal(la, lb)
    assert not np.array_equal(a, c)
    assert all((row >= 0).sum() > 0 for row in la)
    # First game of a batch does not depend on the batch it is generated in.
    d, _ = synth.playout_positions(3, seed=5, first_game=2)
    assert np.array_equal(d[0], a[2])


def test_product_packer_matches_oracle_packer():
    planes, _ = synth.playout_positions(32, seed=9)
    planes[3, 40, 5] = 2.5  # a non-binary plane exercises first-nonzero value
    m1, v1 = oracle.pack_planes(planes)
    m2, v2 = backend.pack_planes(planes)
    assert np.array_equal(m1, m2) and np.array_equal(v1.view(np.uint32), v2.view(np.uint32))

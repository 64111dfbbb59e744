"""The position encoder for every network input format (reference
src/nn/encoder.cpp:249-475): castling-plane, canonical, hectoplies,
armageddon and canonical-v2 formats, and the canonical transform.

Pins:
* the reference's own test: the v2 repetition plane after Nf3 Nf6 Ng1 Ng8
  (tests/test_nn_comparison.cpp:304-341);
* what the mathematics fixes: a canonical form is the same for every
  symmetric image of a position.  For white to move, pawnless and without
  castling rights the 8 images under the board's symmetries encode to equal
  planes; with pawns the file flip alone leaves them equal;
* the classical encoding (itself pinned in test_inputs.py): the history sets
  a canonical format keeps are the classical ones, v2 keeps exactly the
  repeated positions, a capture ends canonical history;
* the policy indices of the legal moves under a flip transform land on the
  transformed squares of the moving pieces.

The en-passant plane and the transform choice use board coordinates when
black is to move, as the reference does (encoder.cpp:94-157, 316-323); for
those two the checks below restate the reference (parity unpinned beyond it).
"""

import numpy as np
import pytest

from metalfish_amd import synth

START = "rnbqkbnr/pppppppp/8/8/8/8/PPPPPPPP/RNBQKBNR w KQkq - 0 1"
AUX = 104


def _board(fen):
    rows = fen.split()[0].split("/")
    sq = {}
    for r, row in enumerate(rows):
        rank = 7 - r
        f = 0
        for ch in row:
            if ch.isdigit():
                f += int(ch)
            else:
                sq[rank * 8 + f] = ch
                f += 1
    return sq


def _fen(sq, rest):
    rows = []
    for rank in range(7, -1, -1):
        row, empty = "", 0
        for f in range(8):
            ch = sq.get(rank * 8 + f)
            if ch is None:
                empty += 1
            else:
                if empty:
                    row += str(empty)
                    empty = 0
                row += ch
        if empty:
            row += str(empty)
        rows.append(row)
    return "/".join(rows) + " " + rest


def _sym(s, k):
    """Square s under symmetry k of the board (8 elements: file flip, rank
    flip, diagonal reflection and their compositions)."""
    r, f = s >> 3, s & 7
    if k & 1:
        f = 7 - f
    if k & 2:
        r = 7 - r
    if k & 4:
        r, f = f, r
    return r * 8 + f


def _image(fen, k):
    parts = fen.split()
    sq = {_sym(s, k): p for s, p in _board(fen).items()}
    return _fen(sq, " ".join(parts[1:]))


def _random_pawnless(rng):
    while True:
        squares = rng.choice(64, size=6, replace=False)
        wk, bk = int(squares[0]), int(squares[1])
        if abs((wk >> 3) - (bk >> 3)) <= 1 and abs((wk & 7) - (bk & 7)) <= 1:
            continue
        pieces = {wk: "K", bk: "k"}
        for s, p in zip(squares[2:], rng.choice(list("QRBNqrbn"), size=4)):
            pieces[int(s)] = str(p)
        fen = _fen(pieces, "w - - 0 1")
        try:
            _, legal, _ = synth.encode_game_format(fen, "", "canonical")
        except ValueError:
            continue
        if len(legal):
            return fen


def test_reference_v2_repetition_plane():
    planes, _, t = synth.encode_game_format(START, "g1f3 g8f6 f3g1 f6g8", "canonical_v2")
    assert t == 0  # castling rights remain
    assert np.all(planes[12] == 1.0)


@pytest.mark.parametrize("seed", range(12))
def test_canonical_planes_equal_for_all_symmetric_images(seed):
    fen = _random_pawnless(np.random.default_rng(seed))
    ref, _, _ = synth.encode_game_format(fen, "", "canonical")
    for k in range(1, 8):
        planes, _, _ = synth.encode_game_format(_image(fen, k), "", "canonical")
        assert np.array_equal(planes, ref), (fen, k)


@pytest.mark.parametrize("fen", [
    "8/2p5/3p4/KP5r/1R3p1k/8/4P1P1/8 w - - 0 1",
    "4k3/pp6/8/8/8/8/5PPP/2K5 w - - 0 1",
    "r3k3/8/8/8/8/8/P7/1K6 w - - 0 1"])
def test_canonical_planes_with_pawns_equal_under_file_flip(fen):
    a, _, ta = synth.encode_game_format(fen, "", "canonical")
    b, _, tb = synth.encode_game_format(_image(fen, 1), "", "canonical")
    assert np.array_equal(a, b)
    assert {ta, tb} <= {0, 1} and ta != tb  # exactly one of them is flipped


def test_castling_rights_keep_the_board_untransformed():
    fen = "r3k2r/8/8/8/8/8/8/R3K2R w KQkq - 0 1"
    canon, _, t = synth.encode_game_format(fen, "", "canonical")
    classic, _, _ = synth.encode_game_format(fen, "", "classical")
    assert t == 0
    assert np.array_equal(canon[:13], classic[:13])
    # A rule-50 count of 0 ends canonical history after the current
    # position; classical FEN_ONLY fill repeats it.
    assert not canon[13:AUX].any()
    assert np.array_equal(classic[13:25], classic[:12])


def test_castling_plane_formats_mark_rook_squares():
    for fmt in ("castling_plane", "canonical", "canonical_v2"):
        for moves in ("", "e2e4"):
            p, _, _ = synth.encode_game_format(START, moves, fmt)
            assert set(np.flatnonzero(p[AUX + 0])) == {0, 56}
            assert set(np.flatnonzero(p[AUX + 1])) == {7, 63}
            assert not p[AUX + 2].any() and not p[AUX + 3].any()
    # Only the side to move's queenside right left: a1 of its frame.
    p, _, _ = synth.encode_game_format("r3k2r/8/8/8/8/8/8/R3K2R b q - 0 1", "", "canonical")
    assert set(np.flatnonzero(p[AUX + 0])) == {0}
    assert not p[AUX + 1].any()


def test_side_rule50_and_armageddon_planes():
    fen_b = "4k3/8/8/8/8/8/8/R3K3 b - - 30 40"
    fen_w = "4k3/8/8/8/8/8/8/R3K3 w - - 30 40"
    p, _, _ = synth.encode_game_format(fen_b, "", "castling_plane")
    assert np.all(p[AUX + 4] == 1.0) and np.all(p[AUX + 5] == 30.0)
    for fmt, rule50 in (("canonical", 30.0), ("canonical_hectoplies", np.float32(0.3)),
                        ("canonical_v2", np.float32(0.3))):
        p, _, _ = synth.encode_game_format(fen_b, "", fmt)
        assert np.all(p[AUX + 5] == np.float32(rule50)), fmt
        assert not p[AUX + 6].any() and np.all(p[AUX + 7] == 1.0)
    for fmt in ("canonical_hectoplies_armageddon", "canonical_v2_armageddon"):
        pb, _, _ = synth.encode_game_format(fen_b, "", fmt)
        pw, _, _ = synth.encode_game_format(fen_w, "", fmt)
        assert np.all(pb[AUX + 6] == 1.0) and not pw[AUX + 6].any()


def test_canonical_en_passant_plane():
    # Black to move can take e3 en passant; the square is marked in board
    # coordinates (e3 = 20), castling rights keep the board untransformed.
    fen = "rnbqkbnr/ppp1pppp/8/8/3pP3/8/PPPP1PPP/RNBQKBNR b KQkq e3 0 3"
    p, _, t = synth.encode_game_format(fen, "", "canonical")
    assert t == 0 and list(np.flatnonzero(p[AUX + 4])) == [20]
    p, _, _ = synth.encode_game_format(fen, "", "classical")
    assert np.all(p[AUX + 4] == 1.0)  # classical: the side-to-move plane


def test_v2_keeps_only_repeated_history():
    moves = "g1f3 g8f6 f3g1 f6g8 g1f3 g8f6"
    v2, _, _ = synth.encode_game_format(START, moves, "canonical_v2")
    classic, _, _ = synth.encode_game_format(START, moves, "classical")
    # Plies 6, 5 and 4 repeat plies 2, 1 and 0; 3, 2, 1 do not, ply 0 ends
    # the search (rule-50 count 0).
    assert np.array_equal(v2[:39], classic[:39])
    assert not v2[39:AUX].any()
    for i in range(3):
        assert np.all(v2[13 * i + 12] == 1.0)


def test_canonical_history_stops_at_a_capture():
    moves = "e2e4 d7d5 e4d5 d8d5 b1c3"
    canon, _, t = synth.encode_game_format(START, moves, "canonical")
    classic, _, _ = synth.encode_game_format(START, moves, "classical")
    assert t == 0
    assert np.array_equal(canon[:26], classic[:26])  # current + the capture
    assert not canon[26:AUX].any()
    assert classic[26:AUX].any()


def test_fill_modes():
    fen = "4k3/8/8/8/8/8/8/R3K3 w - - 5 40"
    no, _, _ = synth.encode_game_format(fen, "", "classical", fill="no")
    fen_only, _, _ = synth.encode_game_format(fen, "", "classical", fill="fen_only")
    assert not no[13:AUX].any()
    for i in range(1, 8):  # FEN_ONLY repeats a non-start position
        assert np.array_equal(fen_only[13 * i:13 * i + 12], fen_only[:12])
    start_always, _, _ = synth.encode_game_format(START, "", "classical", fill="always")
    assert np.array_equal(start_always[13:25], start_always[:12])


def test_legal_move_indices_follow_a_flip_transform():
    # King on the d-file, pawns on the board, no castling: the flip.
    fen = "3k4/pp6/8/8/8/8/5PPP/3K4 w - - 0 1"
    planes, legal, t = synth.encode_game_format(fen, "", "canonical")
    assert t == 1
    ours = planes[:6].sum(axis=0)
    for idx in legal:
        assert idx >= 0
        frm, to, _ = synth.index_to_move(int(idx), 0)
        assert ours[frm] == 1.0  # a piece of ours on the transformed square


def test_black_to_move_transform_uses_board_coordinates():
    # Black king on e8, pawnless, no castling: ranks 5-8 in board
    # coordinates take the mirror (the reference does not flip the king to
    # the side to move's frame first).
    _, _, t = synth.encode_game_format("4k3/8/8/8/8/8/8/R2K4 b - - 0 1", "", "canonical")
    assert t == 2


def test_bad_format_rejected():
    with pytest.raises(ValueError):
        synth.encode_game_format(START, "", 6)

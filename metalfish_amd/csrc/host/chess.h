// Chess position model used to synthesise benchmark and parity inputs.
//
// This is input generation, not part of the evaluation hot path: MetalFish's
// MCTS hands `InputPlanes` to `NN::Network::EvaluateBatch`
// (reference src/nn/network.h:44-45); the positions those planes come from are
// produced upstream by `NN::EncodePositionForNN` (reference
// src/nn/encoder.cpp:249-475).  This module plays seeded random games and
// encodes them the same way so that the GPU backend and the CPU oracle see
// identical, realistic inputs.
//
// Square numbering follows the reference: a1 = 0, b1 = 1, ..., h8 = 63.
#pragma once

#include <array>
#include <cstdint>
#include <string>
#include <vector>

namespace mfh_chess {

using Bitboard = std::uint64_t;

enum Color : int { WHITE = 0, BLACK = 1 };
enum PieceType : int { PAWN = 0, KNIGHT, BISHOP, ROOK, QUEEN, KING, NO_PIECE_TYPE };
enum CastlingRight : int { WHITE_OO = 1, WHITE_OOO = 2, BLACK_OO = 4, BLACK_OOO = 8 };
constexpr int SQ_NONE = 64;

enum MoveKind : std::uint8_t { MK_NORMAL = 0, MK_EN_PASSANT, MK_CASTLE, MK_PROMOTION };

struct Move {
  std::uint8_t from = 0;
  std::uint8_t to = 0;
  std::uint8_t promo = NO_PIECE_TYPE;  // piece type for MK_PROMOTION
  std::uint8_t kind = MK_NORMAL;
  bool operator==(const Move &o) const {
    return from == o.from && to == o.to && promo == o.promo && kind == o.kind;
  }
  std::string Uci() const;
};

// One position plus the bookkeeping the encoder needs (rule-50 counter,
// plies since the game start, repetition distance as Stockfish-style
// `StateInfo::repetition`, reference src/core/position.cpp:865-877).
struct State {
  Bitboard by_color[2] = {0, 0};
  Bitboard by_type[6] = {0, 0, 0, 0, 0, 0};
  int stm = WHITE;
  int castling = 0;
  int ep = SQ_NONE;  // set only when an en-passant capture is playable
  int rule50 = 0;
  int plies_from_null = 0;
  int game_ply = 0;
  std::uint64_t key = 0;
  int repetition = 0;

  Bitboard Pieces() const { return by_color[0] | by_color[1]; }
  Bitboard Pieces(int c, int pt) const { return by_color[c] & by_type[pt]; }
  int KingSquare(int c) const;
  bool CanCastle(int right) const { return (castling & right) != 0; }
  bool IsRepetition() const { return repetition != 0; }
};

// A game: the start state and every state reached by do_move, so that
// repetition detection and history encoding can look back.
class Game {
public:
  Game();
  bool SetFen(const std::string &fen);  // resets history to one state
  std::string Fen() const;

  const State &Current() const { return states_.back(); }
  const std::vector<State> &History() const { return states_; }

  void LegalMoves(std::vector<Move> &out) const;
  void DoMove(const Move &m);
  void UndoMove();
  bool ParseUci(const std::string &uci, Move &out) const;

private:
  std::vector<State> states_;
};

std::uint64_t Perft(Game &game, int depth);

// Input formats of a network file (reference src/nn/proto/net.proto:256-263).
enum InputFormat : int {
  INPUT_CLASSICAL_112_PLANE = 1,
  INPUT_112_WITH_CASTLING_PLANE = 2,
  INPUT_112_WITH_CANONICALIZATION = 3,
  INPUT_112_WITH_CANONICALIZATION_HECTOPLIES = 4,
  INPUT_112_WITH_CANONICALIZATION_HECTOPLIES_ARMAGEDDON = 132,
  INPUT_112_WITH_CANONICALIZATION_V2 = 5,
  INPUT_112_WITH_CANONICALIZATION_V2_ARMAGEDDON = 133,
};
// How missing history is filled (reference src/nn/encoder.h:20).
enum FillEmptyHistory : int { FILL_NO = 0, FILL_FEN_ONLY = 1, FILL_ALWAYS = 2 };

// Plane transforms of the canonical formats (reference input_planes.h:16-20).
constexpr int kFlipTransform = 1;
constexpr int kMirrorTransform = 2;
constexpr int kTransposeTransform = 4;

bool IsCanonicalFormat(int input_format);
bool IsHectopliesFormat(int input_format);
bool IsCanonicalArmageddonFormat(int input_format);

// The transform a canonical format applies to the current position
// (reference ChooseTransform, src/nn/encoder.cpp:94-157).
int ChooseTransform(const State &s);

// NN::EncodePositionForNN (reference src/nn/encoder.cpp:249-475): the 112
// planes of the last position of `history` with up to `history_planes` (8
// at most) earlier positions, for any of the input formats above.  Returns
// the transform applied (0 outside the canonical formats).  `planes`
// receives 112*64 floats.
int EncodePositionForNN(const std::vector<State> &history, int input_format,
                        int history_planes, int fill_empty_history, float *planes);

// Classical 112-plane encoding with 8-ply history and FEN_ONLY fill of
// missing history, as the MCTS evaluator calls it for classical nets
// (reference src/mcts/evaluator.cpp:155-157).
void EncodeClassical112(const std::vector<State> &history, float *planes);

bool IsStartPosition(const State &s);

}  // namespace mfh_chess

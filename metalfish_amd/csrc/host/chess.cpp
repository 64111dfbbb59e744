// Chess rules for synthetic input generation (see chess.h for scope).
#include "chess.h"

#include <cstring>
#include <sstream>

namespace mfh_chess {
namespace {

inline int FileOf(int sq) { return sq & 7; }
inline int RankOf(int sq) { return sq >> 3; }
inline Bitboard Bit(int sq) { return 1ULL << sq; }
inline int Lsb(Bitboard b) { return __builtin_ctzll(b); }
inline int PopLsb(Bitboard &b) {
  const int s = Lsb(b);
  b &= b - 1;
  return s;
}
inline bool MoreThanOne(Bitboard b) { return (b & (b - 1)) != 0; }
inline Bitboard FileBB(int sq) { return 0x0101010101010101ULL << FileOf(sq); }

struct Tables {
  Bitboard knight[64];
  Bitboard king[64];
  Bitboard pawn[2][64];  // squares attacked by a pawn of colour c on sq
  std::uint64_t z_psq[2][6][64];
  std::uint64_t z_castle[16];
  std::uint64_t z_ep[8];
  std::uint64_t z_side;
  Tables() {
    for (int sq = 0; sq < 64; ++sq) {
      knight[sq] = king[sq] = pawn[0][sq] = pawn[1][sq] = 0;
      const int f = FileOf(sq), r = RankOf(sq);
      static const int kn[8][2] = {{1, 2}, {2, 1}, {2, -1}, {1, -2},
                                   {-1, -2}, {-2, -1}, {-2, 1}, {-1, 2}};
      for (auto &d : kn) {
        const int nf = f + d[0], nr = r + d[1];
        if (nf >= 0 && nf < 8 && nr >= 0 && nr < 8)
          knight[sq] |= Bit(nr * 8 + nf);
      }
      for (int df = -1; df <= 1; ++df)
        for (int dr = -1; dr <= 1; ++dr) {
          if (!df && !dr)
            continue;
          const int nf = f + df, nr = r + dr;
          if (nf >= 0 && nf < 8 && nr >= 0 && nr < 8)
            king[sq] |= Bit(nr * 8 + nf);
        }
      for (int df : {-1, 1}) {
        const int nf = f + df;
        if (nf < 0 || nf > 7)
          continue;
        if (r + 1 < 8)
          pawn[WHITE][sq] |= Bit((r + 1) * 8 + nf);
        if (r - 1 >= 0)
          pawn[BLACK][sq] |= Bit((r - 1) * 8 + nf);
      }
    }
    // Fixed-seed SplitMix64 stream for hashing; only equality matters.
    std::uint64_t s = 0x4D46484953484131ULL;
    auto next = [&s]() {
      std::uint64_t z = (s += 0x9E3779B97F4A7C15ULL);
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
      return z ^ (z >> 31);
    };
    for (auto &c : z_psq)
      for (auto &p : c)
        for (auto &v : p)
          v = next();
    for (auto &v : z_castle)
      v = next();
    for (auto &v : z_ep)
      v = next();
    z_side = next();
  }
};

const Tables &T() {
  static const Tables t;
  return t;
}

Bitboard RayAttacks(int sq, Bitboard occ, const int (*dirs)[2], int ndirs) {
  Bitboard out = 0;
  const int f0 = FileOf(sq), r0 = RankOf(sq);
  for (int i = 0; i < ndirs; ++i) {
    int f = f0 + dirs[i][0], r = r0 + dirs[i][1];
    while (f >= 0 && f < 8 && r >= 0 && r < 8) {
      const int s = r * 8 + f;
      out |= Bit(s);
      if (occ & Bit(s))
        break;
      f += dirs[i][0];
      r += dirs[i][1];
    }
  }
  return out;
}

const int kRookDirs[4][2] = {{1, 0}, {-1, 0}, {0, 1}, {0, -1}};
const int kBishopDirs[4][2] = {{1, 1}, {1, -1}, {-1, 1}, {-1, -1}};

Bitboard RookAttacks(int sq, Bitboard occ) { return RayAttacks(sq, occ, kRookDirs, 4); }
Bitboard BishopAttacks(int sq, Bitboard occ) { return RayAttacks(sq, occ, kBishopDirs, 4); }

// Squares strictly between a and b on a shared line, or 0.
Bitboard Between(int a, int b) {
  const int df = FileOf(b) - FileOf(a), dr = RankOf(b) - RankOf(a);
  if (a == b)
    return 0;
  if (!(df == 0 || dr == 0 || df == dr || df == -dr))
    return 0;
  const int sf = (df > 0) - (df < 0), sr = (dr > 0) - (dr < 0);
  Bitboard out = 0;
  int f = FileOf(a) + sf, r = RankOf(a) + sr;
  while (r * 8 + f != b) {
    out |= Bit(r * 8 + f);
    f += sf;
    r += sr;
  }
  return out;
}

Bitboard AttackersTo(const State &s, int sq, Bitboard occ) {
  const Tables &t = T();
  return (t.pawn[BLACK][sq] & s.Pieces(WHITE, PAWN)) |
         (t.pawn[WHITE][sq] & s.Pieces(BLACK, PAWN)) |
         (t.knight[sq] & s.by_type[KNIGHT]) | (t.king[sq] & s.by_type[KING]) |
         (RookAttacks(sq, occ) & (s.by_type[ROOK] | s.by_type[QUEEN])) |
         (BishopAttacks(sq, occ) & (s.by_type[BISHOP] | s.by_type[QUEEN]));
}

// Pieces of either colour that are the only blocker between king `c` and an
// enemy slider (Stockfish's blockers_for_king).
Bitboard BlockersForKing(const State &s, int c) {
  const int ksq = s.KingSquare(c);
  const int them = c ^ 1;
  const Bitboard occ = s.Pieces();
  Bitboard snipers =
      (RookAttacks(ksq, 0) & (s.Pieces(them, ROOK) | s.Pieces(them, QUEEN))) |
      (BishopAttacks(ksq, 0) &
       (s.Pieces(them, BISHOP) | s.Pieces(them, QUEEN)));
  Bitboard blockers = 0;
  while (snipers) {
    const int sn = PopLsb(snipers);
    const Bitboard b = Between(ksq, sn) & occ;
    if (b && !MoreThanOne(b))
      blockers |= b;
  }
  return blockers;
}

int PieceOn(const State &s, int sq, int &color) {
  const Bitboard b = Bit(sq);
  if (!(s.Pieces() & b))
    return NO_PIECE_TYPE;
  color = (s.by_color[WHITE] & b) ? WHITE : BLACK;
  for (int pt = 0; pt < 6; ++pt)
    if (s.by_type[pt] & b)
      return pt;
  return NO_PIECE_TYPE;
}

void PutPiece(State &s, int c, int pt, int sq) {
  s.by_color[c] |= Bit(sq);
  s.by_type[pt] |= Bit(sq);
}
void RemovePiece(State &s, int c, int pt, int sq) {
  s.by_color[c] &= ~Bit(sq);
  s.by_type[pt] &= ~Bit(sq);
}

std::uint64_t ComputeKey(const State &s) {
  const Tables &t = T();
  std::uint64_t k = 0;
  for (int c = 0; c < 2; ++c)
    for (int pt = 0; pt < 6; ++pt) {
      Bitboard b = s.Pieces(c, pt);
      while (b)
        k ^= t.z_psq[c][pt][PopLsb(b)];
    }
  k ^= t.z_castle[s.castling & 15];
  if (s.ep != SQ_NONE)
    k ^= t.z_ep[FileOf(s.ep)];
  if (s.stm == BLACK)
    k ^= t.z_side;
  return k;
}

bool KingAttacked(const State &s, int c) {
  return (AttackersTo(s, s.KingSquare(c), s.Pieces()) & s.by_color[c ^ 1]) != 0;
}

// Applies the piece movement of `m` to the boards only.
void MovePieces(State &s, const Move &m) {
  const int us = s.stm, them = us ^ 1;
  int pc_color = us;
  const int pt = PieceOn(s, m.from, pc_color);
  if (m.kind == MK_CASTLE) {
    const bool king_side = m.to > m.from;
    const int rank_base = us == WHITE ? 0 : 56;
    const int rook_from = rank_base + (king_side ? 7 : 0);
    const int rook_to = rank_base + (king_side ? 5 : 3);
    RemovePiece(s, us, KING, m.from);
    RemovePiece(s, us, ROOK, rook_from);
    PutPiece(s, us, KING, m.to);
    PutPiece(s, us, ROOK, rook_to);
    return;
  }
  if (m.kind == MK_EN_PASSANT) {
    const int cap = us == WHITE ? m.to - 8 : m.to + 8;
    RemovePiece(s, them, PAWN, cap);
  } else {
    int cc = them;
    const int captured = PieceOn(s, m.to, cc);
    if (captured != NO_PIECE_TYPE)
      RemovePiece(s, cc, captured, m.to);
  }
  RemovePiece(s, us, pt, m.from);
  PutPiece(s, us, m.kind == MK_PROMOTION ? m.promo : pt, m.to);
}

void AddPawnMoves(int from, int to, bool promo_rank, std::vector<Move> &out) {
  if (promo_rank) {
    for (int pt : {QUEEN, ROOK, BISHOP, KNIGHT})
      out.push_back(Move{static_cast<std::uint8_t>(from),
                         static_cast<std::uint8_t>(to),
                         static_cast<std::uint8_t>(pt), MK_PROMOTION});
  } else {
    out.push_back(Move{static_cast<std::uint8_t>(from),
                       static_cast<std::uint8_t>(to), NO_PIECE_TYPE, MK_NORMAL});
  }
}

void PseudoLegal(const State &s, std::vector<Move> &out) {
  const Tables &t = T();
  const int us = s.stm, them = us ^ 1;
  const Bitboard occ = s.Pieces();
  const Bitboard own = s.by_color[us];
  const Bitboard enemy = s.by_color[them];
  const int push = us == WHITE ? 8 : -8;
  const int start_rank = us == WHITE ? 1 : 6;
  const int promo_from_rank = us == WHITE ? 6 : 1;

  Bitboard pawns = s.Pieces(us, PAWN);
  while (pawns) {
    const int from = PopLsb(pawns);
    const bool promo = RankOf(from) == promo_from_rank;
    const int one = from + push;
    if (!(occ & Bit(one))) {
      AddPawnMoves(from, one, promo, out);
      const int two = one + push;
      if (RankOf(from) == start_rank && !(occ & Bit(two)))
        AddPawnMoves(from, two, false, out);
    }
    Bitboard caps = t.pawn[us][from] & enemy;
    while (caps)
      AddPawnMoves(from, PopLsb(caps), promo, out);
    if (s.ep != SQ_NONE && (t.pawn[us][from] & Bit(s.ep)))
      out.push_back(Move{static_cast<std::uint8_t>(from),
                         static_cast<std::uint8_t>(s.ep), NO_PIECE_TYPE,
                         MK_EN_PASSANT});
  }
  for (int pt = KNIGHT; pt <= KING; ++pt) {
    Bitboard pieces = s.Pieces(us, pt);
    while (pieces) {
      const int from = PopLsb(pieces);
      Bitboard att = 0;
      switch (pt) {
      case KNIGHT: att = t.knight[from]; break;
      case BISHOP: att = BishopAttacks(from, occ); break;
      case ROOK: att = RookAttacks(from, occ); break;
      case QUEEN: att = RookAttacks(from, occ) | BishopAttacks(from, occ); break;
      default: att = t.king[from]; break;
      }
      att &= ~own;
      while (att)
        out.push_back(Move{static_cast<std::uint8_t>(from),
                           static_cast<std::uint8_t>(PopLsb(att)),
                           NO_PIECE_TYPE, MK_NORMAL});
    }
  }
  // Castling: king and rook on their original squares are implied by rights.
  const int rank_base = us == WHITE ? 0 : 56;
  const int ksq = rank_base + 4;
  const int oo = us == WHITE ? WHITE_OO : BLACK_OO;
  const int ooo = us == WHITE ? WHITE_OOO : BLACK_OOO;
  auto attacked = [&](int sq) {
    return (AttackersTo(s, sq, occ) & enemy) != 0;
  };
  if ((s.castling & (oo | ooo)) && s.KingSquare(us) == ksq && !attacked(ksq)) {
    if ((s.castling & oo) && !(occ & (Bit(ksq + 1) | Bit(ksq + 2))) &&
        !attacked(ksq + 1) && !attacked(ksq + 2))
      out.push_back(Move{static_cast<std::uint8_t>(ksq),
                         static_cast<std::uint8_t>(ksq + 2), NO_PIECE_TYPE,
                         MK_CASTLE});
    if ((s.castling & ooo) &&
        !(occ & (Bit(ksq - 1) | Bit(ksq - 2) | Bit(ksq - 3))) &&
        !attacked(ksq - 1) && !attacked(ksq - 2))
      out.push_back(Move{static_cast<std::uint8_t>(ksq),
                         static_cast<std::uint8_t>(ksq - 2), NO_PIECE_TYPE,
                         MK_CASTLE});
  }
}

int CastlingMaskFor(int sq) {
  switch (sq) {
  case 0: return WHITE_OOO;
  case 4: return WHITE_OO | WHITE_OOO;
  case 7: return WHITE_OO;
  case 56: return BLACK_OOO;
  case 60: return BLACK_OO | BLACK_OOO;
  case 63: return BLACK_OO;
  default: return 0;
  }
}

// En-passant square after a double push of `us` landing on `to`, following
// the Stockfish rule used by the reference (src/core/position.cpp:823-860):
// the square is recorded only if a capture there is playable.
int EpSquareAfterDoublePush(const State &s, int us, int to) {
  const Tables &t = T();
  const int them = us ^ 1;
  const int ep = us == WHITE ? to - 8 : to + 8;
  Bitboard pawns = t.pawn[us][ep] & s.Pieces(them, PAWN);
  if (!pawns)
    return SQ_NONE;
  const int ksq = s.KingSquare(them);
  const Bitboard checkers = AttackersTo(s, ksq, s.Pieces()) & s.by_color[us];
  if (checkers & ~Bit(to))
    return SQ_NONE;
  if (MoreThanOne(pawns)) {
    if (!MoreThanOne(BlockersForKing(s, them) & pawns))
      return ep;
    if (!(FileBB(ksq) & pawns))
      return SQ_NONE;
    pawns &= ~FileBB(ksq);
  }
  const Bitboard occupied = (s.Pieces() ^ Bit(Lsb(pawns)) ^ Bit(to)) | Bit(ep);
  const Bitboard our_rq = s.Pieces(us, QUEEN) | s.Pieces(us, ROOK);
  const Bitboard our_bq = s.Pieces(us, QUEEN) | s.Pieces(us, BISHOP);
  if (!(RookAttacks(ksq, occupied) & our_rq) &&
      !(BishopAttacks(ksq, occupied) & our_bq))
    return ep;
  return SQ_NONE;
}

const char kPieceChars[] = "pnbrqk";

}  // namespace

std::string Move::Uci() const {
  std::string s;
  s += static_cast<char>('a' + FileOf(from));
  s += static_cast<char>('1' + RankOf(from));
  s += static_cast<char>('a' + FileOf(to));
  s += static_cast<char>('1' + RankOf(to));
  if (kind == MK_PROMOTION)
    s += kPieceChars[promo];
  return s;
}

int State::KingSquare(int c) const {
  const Bitboard k = Pieces(c, KING);
  return k ? Lsb(k) : SQ_NONE;
}

Game::Game() {
  SetFen("rnbqkbnr/pppppppp/8/8/8/8/PPPPPPPP/RNBQKBNR w KQkq - 0 1");
}

bool Game::SetFen(const std::string &fen) {
  State s;
  std::istringstream in(fen);
  std::string board, side, castle, ep;
  int r50 = 0, fullmove = 1;
  if (!(in >> board >> side >> castle >> ep))
    return false;
  in >> r50 >> fullmove;
  int rank = 7, file = 0;
  for (char ch : board) {
    if (ch == '/') {
      --rank;
      file = 0;
    } else if (ch >= '1' && ch <= '8') {
      file += ch - '0';
    } else {
      const char lower = static_cast<char>(ch | 0x20);
      const char *p = std::strchr(kPieceChars, lower);
      if (!p || rank < 0 || file > 7)
        return false;
      PutPiece(s, (ch == lower) ? BLACK : WHITE,
               static_cast<int>(p - kPieceChars), rank * 8 + file);
      ++file;
    }
  }
  s.stm = side == "b" ? BLACK : WHITE;
  s.castling = 0;
  for (char ch : castle) {
    if (ch == 'K') s.castling |= WHITE_OO;
    if (ch == 'Q') s.castling |= WHITE_OOO;
    if (ch == 'k') s.castling |= BLACK_OO;
    if (ch == 'q') s.castling |= BLACK_OOO;
  }
  s.ep = SQ_NONE;
  if (ep.size() == 2 && ep[0] >= 'a' && ep[0] <= 'h') {
    // Keep the FEN ep square only if a capture there is playable, as the
    // reference's Position::set does (src/core/position.cpp:274-288).
    const int sq = (ep[1] - '1') * 8 + (ep[0] - 'a');
    const int us = s.stm, them = us ^ 1;
    const int push = us == WHITE ? 8 : -8;
    const bool ok = (T().pawn[them][sq] & s.Pieces(us, PAWN)) &&
                    (s.Pieces(them, PAWN) & Bit(sq - push)) &&
                    !(s.Pieces() & (Bit(sq) | Bit(sq + push)));
    if (ok)
      s.ep = sq;
  }
  s.rule50 = r50;
  s.plies_from_null = 0;
  s.game_ply = (fullmove > 0 ? 2 * (fullmove - 1) : 0) + (s.stm == BLACK);
  s.key = ComputeKey(s);
  s.repetition = 0;
  states_.assign(1, s);
  return true;
}

std::string Game::Fen() const {
  const State &s = Current();
  std::string out;
  for (int r = 7; r >= 0; --r) {
    int empty = 0;
    for (int f = 0; f < 8; ++f) {
      int c = WHITE;
      const int pt = PieceOn(s, r * 8 + f, c);
      if (pt == NO_PIECE_TYPE) {
        ++empty;
        continue;
      }
      if (empty)
        out += static_cast<char>('0' + empty);
      empty = 0;
      const char ch = kPieceChars[pt];
      out += c == WHITE ? static_cast<char>(ch & ~0x20) : ch;
    }
    if (empty)
      out += static_cast<char>('0' + empty);
    if (r)
      out += '/';
  }
  out += s.stm == WHITE ? " w " : " b ";
  std::string c;
  if (s.castling & WHITE_OO) c += 'K';
  if (s.castling & WHITE_OOO) c += 'Q';
  if (s.castling & BLACK_OO) c += 'k';
  if (s.castling & BLACK_OOO) c += 'q';
  out += c.empty() ? "-" : c;
  out += ' ';
  if (s.ep == SQ_NONE) {
    out += '-';
  } else {
    out += static_cast<char>('a' + FileOf(s.ep));
    out += static_cast<char>('1' + RankOf(s.ep));
  }
  out += ' ' + std::to_string(s.rule50) + ' ' +
         std::to_string(1 + s.game_ply / 2);
  return out;
}

void Game::LegalMoves(std::vector<Move> &out) const {
  out.clear();
  const State &s = Current();
  std::vector<Move> pseudo;
  pseudo.reserve(64);
  PseudoLegal(s, pseudo);
  for (const Move &m : pseudo) {
    State tmp = s;
    MovePieces(tmp, m);
    if (!KingAttacked(tmp, s.stm))
      out.push_back(m);
  }
}

void Game::DoMove(const Move &m) {
  const State &prev = states_.back();
  State s = prev;
  const int us = prev.stm;
  int cc = us ^ 1;
  const bool capture = m.kind == MK_EN_PASSANT ||
                       PieceOn(prev, m.to, cc) != NO_PIECE_TYPE;
  int mc = us;
  const bool pawn_move = PieceOn(prev, m.from, mc) == PAWN;
  MovePieces(s, m);
  s.castling &= ~(CastlingMaskFor(m.from) | CastlingMaskFor(m.to));
  s.rule50 = (capture || pawn_move) ? 0 : prev.rule50 + 1;
  s.plies_from_null = prev.plies_from_null + 1;
  s.game_ply = prev.game_ply + 1;
  s.stm = us ^ 1;
  s.ep = SQ_NONE;
  if (pawn_move && (m.to ^ m.from) == 16)
    s.ep = EpSquareAfterDoublePush(s, us, m.to);
  s.key = ComputeKey(s);
  states_.push_back(s);

  // Repetition distance (reference src/core/position.cpp:865-877).
  State &cur = states_.back();
  cur.repetition = 0;
  const int n = static_cast<int>(states_.size()) - 1;
  const int end = cur.rule50 < cur.plies_from_null ? cur.rule50
                                                   : cur.plies_from_null;
  for (int i = 4; i <= end && n - i >= 0; i += 2) {
    const State &old = states_[n - i];
    if (old.key == cur.key) {
      cur.repetition = old.repetition ? -i : i;
      break;
    }
  }
}

void Game::UndoMove() {
  if (states_.size() > 1)
    states_.pop_back();
}

bool Game::ParseUci(const std::string &uci, Move &out) const {
  std::vector<Move> moves;
  LegalMoves(moves);
  for (const Move &m : moves) {
    if (m.Uci() == uci) {
      out = m;
      return true;
    }
  }
  return false;
}

std::uint64_t Perft(Game &game, int depth) {
  std::vector<Move> moves;
  game.LegalMoves(moves);
  if (depth <= 1)
    return depth == 1 ? moves.size() : 1;
  std::uint64_t total = 0;
  for (const Move &m : moves) {
    game.DoMove(m);
    total += Perft(game, depth - 1);
    game.UndoMove();
  }
  return total;
}

bool IsStartPosition(const State &s) {
  return s.stm == WHITE && s.game_ply == 0 && s.rule50 == 0 &&
         s.ep == SQ_NONE && s.castling == 15 &&
         s.Pieces(WHITE, PAWN) == 0x000000000000FF00ULL &&
         s.Pieces(BLACK, PAWN) == 0x00FF000000000000ULL &&
         s.Pieces(WHITE, KNIGHT) == 0x0000000000000042ULL &&
         s.Pieces(BLACK, KNIGHT) == 0x4200000000000000ULL &&
         s.Pieces(WHITE, BISHOP) == 0x0000000000000024ULL &&
         s.Pieces(BLACK, BISHOP) == 0x2400000000000000ULL &&
         s.Pieces(WHITE, ROOK) == 0x0000000000000081ULL &&
         s.Pieces(BLACK, ROOK) == 0x8100000000000000ULL &&
         s.Pieces(WHITE, QUEEN) == 0x0000000000000008ULL &&
         s.Pieces(BLACK, QUEEN) == 0x0800000000000000ULL &&
         s.Pieces(WHITE, KING) == 0x0000000000000010ULL &&
         s.Pieces(BLACK, KING) == 0x1000000000000000ULL;
}

namespace {
// Byte-order reversal flips the board vertically (rank r -> 7 - r).
inline Bitboard ReverseBytes(Bitboard b) { return __builtin_bswap64(b); }

// Bit reversal within each byte flips the board horizontally (file f ->
// 7 - f).
inline Bitboard ReverseBitsInBytes(Bitboard v) {
  v = ((v >> 1) & 0x5555555555555555ULL) | ((v & 0x5555555555555555ULL) << 1);
  v = ((v >> 2) & 0x3333333333333333ULL) | ((v & 0x3333333333333333ULL) << 2);
  return ((v >> 4) & 0x0F0F0F0F0F0F0F0FULL) | ((v & 0x0F0F0F0F0F0F0F0FULL) << 4);
}

// Reflection in the a8-h1 diagonal: square (rank r, file f) -> (rank 7 - f,
// file 7 - r), as three block swaps of 1, 2 and 4 squares (the reference's
// TransposeBitsInBytes, encoder.cpp:47-55, does the same).
inline Bitboard TransposeAntiDiagonal(Bitboard v) {
  v = ((v & 0xAA00AA00AA00AA00ULL) >> 9) | ((v & 0x0055005500550055ULL) << 9) |
      (v & 0x55AA55AA55AA55AAULL);
  v = ((v & 0xCCCC0000CCCC0000ULL) >> 18) | ((v & 0x0000333300003333ULL) << 18) |
      (v & 0x3333CCCC3333CCCCULL);
  return ((v & 0xF0F0F0F000000000ULL) >> 36) | ((v & 0x000000000F0F0F0FULL) << 36) |
         (v & 0x0F0F0F0FF0F0F0F0ULL);
}

// Flip, then mirror, then transpose (reference encoder.cpp:57-73).
Bitboard ApplyTransform(Bitboard b, int transform) {
  if (b == 0 || b == ~0ULL)
    return b;
  if (transform & kFlipTransform)
    b = ReverseBitsInBytes(b);
  if (transform & kMirrorTransform)
    b = ReverseBytes(b);
  if (transform & kTransposeTransform)
    b = TransposeAntiDiagonal(b);
  return b;
}

// -1 / 0 / 1 as `board` (after the flip / mirror of `transform`) is below,
// equal to or above its transpose (reference encoder.cpp:75-92).
int CompareTransposing(Bitboard board, int transform) {
  if (transform & kFlipTransform)
    board = ReverseBitsInBytes(board);
  if (transform & kMirrorTransform)
    board = ReverseBytes(board);
  const Bitboard alt = TransposeAntiDiagonal(board);
  return board < alt ? -1 : board > alt ? 1 : 0;
}

void SetBits(float *plane, Bitboard b) {
  while (b)
    plane[PopLsb(b)] = 1.0f;
}
void Fill(float *plane, float v) {
  for (int i = 0; i < 64; ++i)
    plane[i] = v;
}
}  // namespace

bool IsCanonicalFormat(int f) {
  return f == INPUT_112_WITH_CANONICALIZATION || f == INPUT_112_WITH_CANONICALIZATION_HECTOPLIES ||
         f == INPUT_112_WITH_CANONICALIZATION_HECTOPLIES_ARMAGEDDON ||
         f == INPUT_112_WITH_CANONICALIZATION_V2 ||
         f == INPUT_112_WITH_CANONICALIZATION_V2_ARMAGEDDON;
}

bool IsHectopliesFormat(int f) {
  return f == INPUT_112_WITH_CANONICALIZATION_HECTOPLIES ||
         f == INPUT_112_WITH_CANONICALIZATION_HECTOPLIES_ARMAGEDDON ||
         f == INPUT_112_WITH_CANONICALIZATION_V2 ||
         f == INPUT_112_WITH_CANONICALIZATION_V2_ARMAGEDDON;
}

bool IsCanonicalArmageddonFormat(int f) {
  return f == INPUT_112_WITH_CANONICALIZATION_HECTOPLIES_ARMAGEDDON ||
         f == INPUT_112_WITH_CANONICALIZATION_V2_ARMAGEDDON;
}

// No transform while any castling right remains.  Otherwise the side to
// move's king goes to files e-h (flip); without pawns also to ranks 1-4
// (mirror) and below the a8-h1 diagonal (transpose), a king on that
// diagonal breaking the tie by comparing whole-board, own, king, queen,
// rook, knight and bishop bitboards with their transposes.  The king and
// the tie-break boards are taken in board coordinates, not flipped for
// black to move, as the reference takes them.
int ChooseTransform(const State &s) {
  if (s.castling != 0)
    return 0;
  const int us = s.stm;
  Bitboard king = s.Pieces(us, KING);
  int t = 0;
  if (king & 0x0F0F0F0F0F0F0F0FULL) {
    t |= kFlipTransform;
    king = ReverseBitsInBytes(king);
  }
  if (s.by_type[PAWN] != 0)
    return t;
  if (king & 0xFFFFFFFF00000000ULL) {
    t |= kMirrorTransform;
    king = ReverseBytes(king);
  }
  if (king & 0xE0C08000ULL)
    return t | kTransposeTransform;
  if (king & 0x10204080ULL) {
    const Bitboard boards[7] = {s.Pieces(), s.by_color[us], s.by_type[KING], s.by_type[QUEEN],
                                s.by_type[ROOK], s.by_type[KNIGHT], s.by_type[BISHOP]};
    for (Bitboard b : boards) {
      const int c = CompareTransposing(b, t);
      if (c < 0)
        return t;
      if (c > 0)
        return t | kTransposeTransform;
    }
  }
  return t;
}

int EncodePositionForNN(const std::vector<State> &history, int fmt, int history_planes,
                        int fill, float *planes) {
  std::memset(planes, 0, sizeof(float) * 112 * 64);
  if (history.empty())
    return 0;
  const State &cur = history.back();
  const int us = cur.stm, them = us ^ 1;
  const bool canonical = IsCanonicalFormat(fmt);
  const bool skip_non_repeats = fmt == INPUT_112_WITH_CANONICALIZATION_V2 ||
                                fmt == INPUT_112_WITH_CANONICALIZATION_V2_ARMAGEDDON;
  const int transform = canonical ? ChooseTransform(cur) : 0;
  const int our_oo = us == WHITE ? WHITE_OO : BLACK_OO;
  const int our_ooo = us == WHITE ? WHITE_OOO : BLACK_OOO;
  const int their_oo = us == WHITE ? BLACK_OO : WHITE_OO;
  const int their_ooo = us == WHITE ? BLACK_OOO : WHITE_OOO;

  // Aux planes (reference encoder.cpp:283-339).
  float *aux = planes + 104 * 64;
  if (fmt == INPUT_CLASSICAL_112_PLANE) {
    Fill(aux + 0 * 64, cur.CanCastle(our_ooo) ? 1.f : 0.f);
    Fill(aux + 1 * 64, cur.CanCastle(our_oo) ? 1.f : 0.f);
    Fill(aux + 2 * 64, cur.CanCastle(their_ooo) ? 1.f : 0.f);
    Fill(aux + 3 * 64, cur.CanCastle(their_oo) ? 1.f : 0.f);
  } else {
    // The castling rook's square: the side to move's on the first rank of
    // its frame, the other side's on the last.
    aux[0 * 64 + 0] = cur.CanCastle(our_ooo) ? 1.f : 0.f;
    aux[1 * 64 + 7] = cur.CanCastle(our_oo) ? 1.f : 0.f;
    aux[0 * 64 + 56] = cur.CanCastle(their_ooo) ? 1.f : 0.f;
    aux[1 * 64 + 63] = cur.CanCastle(their_oo) ? 1.f : 0.f;
  }
  if (canonical) {
    // The en-passant square in board coordinates (not flipped for black).
    if (cur.ep != SQ_NONE)
      aux[4 * 64 + cur.ep] = 1.f;
  } else {
    Fill(aux + 4 * 64, us == BLACK ? 1.f : 0.f);
  }
  Fill(aux + 5 * 64, IsHectopliesFormat(fmt) ? static_cast<float>(cur.rule50) / 100.0f
                                             : static_cast<float>(cur.rule50));
  Fill(aux + 6 * 64, IsCanonicalArmageddonFormat(fmt) && us == BLACK ? 1.f : 0.f);
  Fill(aux + 7 * 64, 1.f);

  // Castling rights relative to the side to move (reference encoder.cpp:
  // 341-367): a history position with other rights cannot repeat.
  auto rights = [&](const State &p) {
    return (p.CanCastle(our_oo) ? 1 : 0) | (p.CanCastle(our_ooo) ? 2 : 0) |
           (p.CanCastle(their_oo) ? 4 : 0) | (p.CanCastle(their_ooo) ? 8 : 0);
  };
  const int root_rights = rights(cur);
  const int planes_wanted = history_planes < 8 ? history_planes : 8;
  const int actual = static_cast<int>(history.size());
  for (int i = 0, idx = actual - 1; i < planes_wanted; ++i, --idx) {
    const State &pos = history[idx >= 0 ? idx : 0];
    // Without fill, one earlier position is inferred only from an en-passant
    // square (reference encoder.cpp:378-389).
    if (fill == FILL_NO && (idx < -1 || (idx == -1 && pos.ep == SQ_NONE)))
      break;
    // FEN_ONLY fill: repeat the oldest known position unless it is the
    // standard start position.
    if (idx < 0 && fill == FILL_FEN_ONLY && IsStartPosition(pos))
      break;
    if (canonical && idx < actual - 1) {
      if (rights(pos) != root_rights || pos.ep != SQ_NONE)
        break;
    }
    const bool rep = pos.IsRepetition();
    // Canonical v2: history planes only for repeated positions, the plane
    // index kept while non-repeats are skipped (reference encoder.cpp:
    // 399-404).  Synthesised history (before the first position) repeats
    // that position, which never is a repetition: the reference would skip
    // it without end, this stops there.
    if (skip_non_repeats && i > 0 && !rep) {
      if (pos.rule50 == 0 || idx < 0)
        break;
      --i;
      continue;
    }
    Bitboard ours[6], theirs[6];
    for (int pt = 0; pt < 6; ++pt) {
      ours[pt] = pos.Pieces(us, pt);
      theirs[pt] = pos.Pieces(them, pt);
      if (us == BLACK) {
        ours[pt] = ReverseBytes(ours[pt]);
        theirs[pt] = ReverseBytes(theirs[pt]);
      }
    }
    float *base = planes + i * 13 * 64;
    for (int pt = 0; pt < 6; ++pt) {
      SetBits(base + pt * 64, ours[pt]);
      SetBits(base + (6 + pt) * 64, theirs[pt]);
    }
    Fill(base + 12 * 64, rep ? 1.f : 0.f);
    // Synthesised-history en-passant adjustment (reference encoder.cpp:
    // 440-451); it only fires for ep squares on the first or last rank.
    if (idx < 0 && pos.ep != SQ_NONE) {
      const int ep_idx = pos.ep;
      if (ep_idx < 8) {
        const Bitboard mask = (0x0000000000000100ULL - 0x0000000001000000ULL)
                              << ep_idx;
        Fill(base + 0 * 64, 0.f);
        SetBits(base + 0 * 64, ours[0] + mask);
      } else if (ep_idx >= 56) {
        const Bitboard mask = (0x0001000000000000ULL - 0x0000000100000000ULL)
                              << (ep_idx - 56);
        Fill(base + 6 * 64, 0.f);
        SetBits(base + 6 * 64, theirs[0] + mask);
      }
    }
    if (canonical && pos.rule50 == 0)
      break;
  }

  // The transform acts on every 0/1 plane up to the en-passant plane
  // (reference encoder.cpp:456-469).
  if (transform != 0) {
    for (int p = 0; p <= 104 + 4; ++p) {
      float *plane = planes + p * 64;
      Bitboard b = 0;
      for (int sq = 0; sq < 64; ++sq)
        if (plane[sq] > 0.5f)
          b |= 1ULL << sq;
      if (b == 0 || b == ~0ULL)
        continue;
      Fill(plane, 0.f);
      SetBits(plane, ApplyTransform(b, transform));
    }
  }
  return transform;
}

void EncodeClassical112(const std::vector<State> &history, float *planes) {
  EncodePositionForNN(history, INPUT_CLASSICAL_112_PLANE, 8, FILL_FEN_ONLY, planes);
}

}  // namespace mfh_chess

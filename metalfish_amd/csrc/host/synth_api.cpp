// C ABI of libmfhost.so: seeded nets and chess positions (see mfh_synth.h).
#include "../../../include/mfh_synth.h"

#include <cmath>
#include <cstring>
#include <sstream>
#include <string>
#include <vector>

#include "chess.h"
#include "policy_tables.h"

namespace {

constexpr std::uint64_t kGamma = 0x9E3779B97F4A7C15ULL;

inline std::uint64_t Mix(std::uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

struct SplitMix64 {
  std::uint64_t state;
  std::uint64_t Next() { return Mix(state += kGamma); }
};

std::uint64_t Fnv1a(const char *s) {
  std::uint64_t h = 0xCBF29CE484222325ULL;
  for (; *s; ++s) {
    h ^= static_cast<unsigned char>(*s);
    h *= 0x100000001B3ULL;
  }
  return h;
}

void LegalIndices(const mfh_chess::Game &game, int transform, int16_t *out, int cap,
                  int *count) {
  std::vector<mfh_chess::Move> moves;
  game.LegalMoves(moves);
  const bool black = game.Current().stm == mfh_chess::BLACK;
  int n = 0;
  for (const auto &m : moves) {
    if (n >= cap)
      break;
    // The policy is read in the side-to-move frame: black moves are mirrored
    // vertically (reference src/mcts/evaluator.cpp:196-208).
    const int from = black ? (m.from ^ 56) : m.from;
    const int to = black ? (m.to ^ 56) : m.to;
    char promo = 0;
    if (m.kind == mfh_chess::MK_PROMOTION)
      promo = "pnbrqk"[m.promo];
    out[n++] = static_cast<int16_t>(mfh_policy::MoveToIndex(from, to, promo, transform));
  }
  for (int i = n; i < cap; ++i)
    out[i] = -1;
  *count = n;
}

}  // namespace

extern "C" {

void mfs_fill_tensor(uint64_t seed, const char *name, int init_kind,
                     double fan_in, float *out, uint64_t count) {
  const std::uint64_t base = seed ^ Fnv1a(name ? name : "");
  const double scale = fan_in > 0.0 ? 1.0 / std::sqrt(fan_in) : 1.0;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < static_cast<long long>(count); ++i) {
    if (init_kind == MFS_INIT_ZERO) {
      out[i] = 0.0f;
      continue;
    }
    // Element i consumes draws 12*i .. 12*i+11 of the stream; SplitMix64's
    // state is a counter, so the draws are addressed directly.
    std::uint64_t state = base + kGamma * (12ULL * static_cast<std::uint64_t>(i));
    std::int64_t sum = 0;
    for (int k = 0; k < 12; ++k)
      sum += static_cast<std::int64_t>(Mix(state += kGamma) >> 40);
    const double normal =
        static_cast<double>(sum - 6 * (1LL << 24)) / static_cast<double>(1LL << 24);
    double v = 0.0;
    switch (init_kind) {
    case MFS_INIT_NORMAL_FAN_IN: v = normal * scale; break;
    case MFS_INIT_ONE_PLUS_TENTH: v = 1.0 + 0.1 * normal; break;
    case MFS_INIT_TENTH: v = 0.1 * normal; break;
    default: v = 0.0; break;
    }
    out[i] = static_cast<float>(v);
  }
}

void mfs_round_bf16(float *data, uint64_t count) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < static_cast<long long>(count); ++i) {
    std::uint32_t u;
    std::memcpy(&u, &data[i], 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
    std::memcpy(&data[i], &u, 4);
  }
}

int mfs_playout_batch(uint64_t seed, int first_game, int count, int min_plies,
                      int max_plies, float *planes, int16_t *legal, char *text,
                      int text_stride) {
  if (count < 0 || min_plies < 0 || max_plies < min_plies || !planes)
    return -1;
  int failures = 0;
#pragma omp parallel for schedule(dynamic, 1)
  for (int i = 0; i < count; ++i) {
    const std::uint64_t g = static_cast<std::uint64_t>(first_game + i);
    SplitMix64 rng{Mix(seed * kGamma + (g + 1) * 0xD1B54A32D192ED03ULL)};
    const int target =
        min_plies + static_cast<int>(rng.Next() % static_cast<std::uint64_t>(
                                                      max_plies - min_plies + 1));
    mfh_chess::Game game;
    std::vector<mfh_chess::Move> moves;
    std::string played;
    bool done = false;
    for (int attempt = 0; attempt < 1000 && !done; ++attempt) {
      game = mfh_chess::Game();
      played.clear();
      bool dead_end = false;
      for (int ply = 0; ply < target; ++ply) {
        game.LegalMoves(moves);
        if (moves.empty()) {
          dead_end = true;
          break;
        }
        const auto &m = moves[rng.Next() % moves.size()];
        if (!played.empty())
          played += ' ';
        played += m.Uci();
        game.DoMove(m);
      }
      if (dead_end)
        continue;
      game.LegalMoves(moves);
      done = !moves.empty();
    }
    if (!done) {
#pragma omp atomic
      ++failures;
      continue;
    }
    mfh_chess::EncodeClassical112(game.History(),
                                  planes + static_cast<size_t>(i) * 112 * 64);
    if (legal) {
      int n = 0;
      LegalIndices(game, 0, legal + static_cast<size_t>(i) * 256, 256, &n);
    }
    if (text && text_stride > 0) {
      char *dst = text + static_cast<size_t>(i) * text_stride;
      std::strncpy(dst, played.c_str(), static_cast<size_t>(text_stride - 1));
      dst[text_stride - 1] = '\0';
    }
  }
  return failures ? -2 : 0;
}

int mfs_encode_game(const char *fen, const char *moves, float *planes,
                    int16_t *legal, int legal_cap) {
  return mfs_encode_game_format(fen, moves, mfh_chess::INPUT_CLASSICAL_112_PLANE,
                                mfh_chess::FILL_FEN_ONLY, 8, planes, legal, legal_cap, nullptr);
}

int mfs_encode_game_format(const char *fen, const char *moves, int input_format,
                           int fill_empty_history, int history_planes, float *planes,
                           int16_t *legal, int legal_cap, int *transform_out) {
  const int f = input_format;
  if ((f < mfh_chess::INPUT_CLASSICAL_112_PLANE || f > mfh_chess::INPUT_112_WITH_CANONICALIZATION_V2) &&
      f != mfh_chess::INPUT_112_WITH_CANONICALIZATION_HECTOPLIES_ARMAGEDDON &&
      f != mfh_chess::INPUT_112_WITH_CANONICALIZATION_V2_ARMAGEDDON)
    return -1;
  if (fill_empty_history < mfh_chess::FILL_NO || fill_empty_history > mfh_chess::FILL_ALWAYS ||
      history_planes < 1)
    return -1;
  mfh_chess::Game game;
  if (fen && *fen && !game.SetFen(fen))
    return -1;
  if (moves) {
    std::istringstream in(moves);
    std::string tok;
    while (in >> tok) {
      mfh_chess::Move m;
      if (!game.ParseUci(tok, m))
        return -1;
      game.DoMove(m);
    }
  }
  std::vector<float> scratch;
  if (!planes) {
    scratch.resize(112 * 64);
    planes = scratch.data();
  }
  const int transform = mfh_chess::EncodePositionForNN(game.History(), input_format,
                                                       history_planes, fill_empty_history, planes);
  if (transform_out)
    *transform_out = transform;
  int n = 0;
  if (legal && legal_cap > 0)
    LegalIndices(game, transform, legal, legal_cap, &n);
  return n;
}

int mfs_move_to_index(int from, int to, char promo, int transform) {
  return mfh_policy::MoveToIndex(from, to, promo, transform);
}

int mfs_index_to_move(int index, int transform, int *from, int *to, char *promo) {
  return mfh_policy::IndexToMove(index, transform, from, to, promo) ? 0 : -1;
}

int64_t mfs_perft(const char *fen, int depth) {
  mfh_chess::Game game;
  if (fen && *fen && !game.SetFen(fen))
    return -1;
  return static_cast<int64_t>(mfh_chess::Perft(game, depth));
}

void mfs_static_position_encoding(float *out) {
  const auto &t = mfh_policy::StaticPositionEncoding();
  if (out)
    std::memcpy(out, t.data(), sizeof(float) * t.size());
}

void mfs_policy_tables(int16_t *attention_map, int16_t *gather,
                       char *move_strings) {
  const auto &map = mfh_policy::AttentionMap();
  const auto &inv = mfh_policy::AttentionGather();
  const auto &moves = mfh_policy::MoveList();
  if (attention_map)
    std::memcpy(attention_map, map.data(), sizeof(int16_t) * map.size());
  if (gather)
    std::memcpy(gather, inv.data(), sizeof(int16_t) * inv.size());
  if (move_strings) {
    for (int i = 0; i < mfh_policy::kPolicyOutputs; ++i) {
      char *dst = move_strings + 6 * i;
      std::memset(dst, 0, 6);
      const auto &m = moves[i];
      dst[0] = static_cast<char>('a' + (m.from & 7));
      dst[1] = static_cast<char>('1' + (m.from >> 3));
      dst[2] = static_cast<char>('a' + (m.to & 7));
      dst[3] = static_cast<char>('1' + (m.to >> 3));
      dst[4] = m.promo;
    }
  }
}

}  // extern "C"

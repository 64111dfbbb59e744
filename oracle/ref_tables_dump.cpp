// Checker-only program: dumps the reference's own policy tables (and the
// static position encoding table) so the tests
// can pin this repository's independently generated tables against them.
// Built by oracle/Makefile from the reference sources where they lie
// (/root/reference/src/nn/policy_map.cpp and
// src/nn/tables/attention_policy_map.h); outputs go to oracle/_ref/ only.
#include <cstdio>
#include <cstdint>

#include "nn/input_planes.h"
#include "nn/policy_map.h"
#include "nn/tables/attention_policy_map.h"

using namespace MetalFish;

int main(int argc, char **argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s OUT.bin\n", argv[0]);
    return 2;
  }
  std::FILE *f = std::fopen(argv[1], "wb");
  if (!f)
    return 1;
  // Section 1: kAttnPolicyMap, 4288 little-endian int16.
  const std::size_t n = sizeof(NN::Tables::kAttnPolicyMap) /
                        sizeof(NN::Tables::kAttnPolicyMap[0]);
  for (std::size_t i = 0; i < n; ++i) {
    const std::int16_t v = NN::Tables::kAttnPolicyMap[i];
    std::fwrite(&v, 2, 1, f);
  }
  // Section 2: MoveToNNIndex for every (from, to, promotion) with promotion
  // in {none, q, r, b, n}: 64*64*5 int16 (-1 when unmapped).
  for (int from = 0; from < 64; ++from)
    for (int to = 0; to < 64; ++to)
      for (int p = 0; p < 5; ++p) {
        std::int16_t v = -1;
        if (from != to) {
          Move m = Move(Square(from), Square(to));
          if (p > 0) {
            static const PieceType kPt[4] = {QUEEN, ROOK, BISHOP, KNIGHT};
            m = Move::make<PROMOTION>(Square(from), Square(to), kPt[p - 1]);
          }
          v = static_cast<std::int16_t>(NN::MoveToNNIndex(m, 0));
        }
        std::fwrite(&v, 2, 1, f);
      }
  // Section 3: IndexToNNMove(i) -> (from, to, promotion piece type or 0).
  for (int i = 0; i < NN::kPolicyOutputs; ++i) {
    const Move m = NN::IndexToNNMove(i, 0);
    std::int16_t rec[3] = {static_cast<std::int16_t>(m.from_sq()),
                           static_cast<std::int16_t>(m.to_sq()),
                           static_cast<std::int16_t>(
                               m.type_of() == PROMOTION ? m.promotion_type() : 0)};
    std::fwrite(rec, 2, 3, f);
  }
  // Section 4: kPosEncoding, 64 x 64 little-endian float32.
  for (int sq = 0; sq < 64; ++sq)
    for (int c = 0; c < NN::Tables::kNumPosEncodingChannels; ++c) {
      const float v = NN::Tables::kPosEncoding[sq][c];
      std::fwrite(&v, 4, 1, f);
    }
  // Section 5: MoveToNNIndex as in section 2 under the input transforms 1..7
  // (flip 1, mirror 2, transpose 4 and their combinations).
  for (int t = 1; t < 8; ++t)
    for (int from = 0; from < 64; ++from)
      for (int to = 0; to < 64; ++to)
        for (int p = 0; p < 5; ++p) {
          std::int16_t v = -1;
          if (from != to) {
            Move m = Move(Square(from), Square(to));
            if (p > 0) {
              static const PieceType kPt[4] = {QUEEN, ROOK, BISHOP, KNIGHT};
              m = Move::make<PROMOTION>(Square(from), Square(to), kPt[p - 1]);
            }
            v = static_cast<std::int16_t>(NN::MoveToNNIndex(m, t));
          }
          std::fwrite(&v, 2, 1, f);
        }
  // Section 6: IndexToNNMove as in section 3 under the transforms 1..7.
  for (int t = 1; t < 8; ++t)
    for (int i = 0; i < NN::kPolicyOutputs; ++i) {
      const Move m = NN::IndexToNNMove(i, t);
      std::int16_t rec[3] = {static_cast<std::int16_t>(m.from_sq()),
                             static_cast<std::int16_t>(m.to_sq()),
                             static_cast<std::int16_t>(
                                 m.type_of() == PROMOTION ? m.promotion_type() : 0)};
      std::fwrite(rec, 2, 3, f);
    }
  std::fclose(f);
  return 0;
}

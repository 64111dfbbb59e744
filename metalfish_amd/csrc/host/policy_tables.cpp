#include "policy_tables.h"

namespace mfh_policy {
namespace {

bool QueenLine(int from, int to) {
  const int df = (to & 7) - (from & 7), dr = (to >> 3) - (from >> 3);
  if (from == to)
    return false;
  return df == 0 || dr == 0 || df == dr || df == -dr;
}

bool KnightJump(int from, int to) {
  int df = (to & 7) - (from & 7), dr = (to >> 3) - (from >> 3);
  df = df < 0 ? -df : df;
  dr = dr < 0 ? -dr : dr;
  return (df == 1 && dr == 2) || (df == 2 && dr == 1);
}

struct Built {
  std::array<PolicyMove, kPolicyOutputs> moves{};
  std::array<std::int16_t, kAttentionRaw> attention{};
  std::array<std::int16_t, kPolicyOutputs> gather{};
  std::array<std::int16_t, 64 * 64> regular{};      // from*64+to -> index
  std::array<std::int16_t, 8 * 8 * 3> promotion{};  // ff*24+tf*3+p -> index
  Built() {
    regular.fill(-1);
    promotion.fill(-1);
    int n = 0;
    for (int from = 0; from < 64; ++from)
      for (int to = 0; to < 64; ++to)
        if (QueenLine(from, to) || KnightJump(from, to)) {
          regular[from * 64 + to] = static_cast<std::int16_t>(n);
          moves[n++] = PolicyMove{static_cast<std::int16_t>(from),
                                  static_cast<std::int16_t>(to), 0};
        }
    static const char kPromo[3] = {'q', 'r', 'b'};
    for (int ff = 0; ff < 8; ++ff)
      for (int tf = ff - 1; tf <= ff + 1; ++tf) {
        if (tf < 0 || tf > 7)
          continue;
        for (int p = 0; p < 3; ++p) {
          promotion[ff * 24 + tf * 3 + p] = static_cast<std::int16_t>(n);
          moves[n++] = PolicyMove{static_cast<std::int16_t>(48 + ff),
                                  static_cast<std::int16_t>(56 + tf), kPromo[p]};
        }
      }
    for (int i = 0; i < 64 * 64; ++i)
      attention[i] = regular[i];
    for (int i = 0; i < 8 * 24; ++i)
      attention[64 * 64 + i] = promotion[i];
    gather.fill(-1);
    for (int raw = 0; raw < kAttentionRaw; ++raw)
      if (attention[raw] >= 0)
        gather[attention[raw]] = static_cast<std::int16_t>(raw);
  }
};

const Built &B() {
  static const Built b;
  return b;
}

}  // namespace

const std::array<PolicyMove, kPolicyOutputs> &MoveList() { return B().moves; }
const std::array<std::int16_t, kAttentionRaw> &AttentionMap() {
  return B().attention;
}
const std::array<std::int16_t, kPolicyOutputs> &AttentionGather() {
  return B().gather;
}

const std::array<float, 64 * kPosEncodingChannels> &StaticPositionEncoding() {
  static const std::array<float, 64 * kPosEncodingChannels> table = [] {
    std::array<float, 64 * kPosEncodingChannels> t{};
    for (int sq = 0; sq < 64; ++sq)
      for (int c = 0; c < kPosEncodingChannels; ++c)
        t[sq * kPosEncodingChannels + c] =
            sq == c ? -1.0f : (QueenLine(sq, c) || KnightJump(sq, c) ? 1.0f : 0.0f);
    return t;
  }();
  return table;
}

namespace {
// The square map of the reference's MoveToNNIndex / IndexToNNMove
// (policy_map.cpp:305-314): the rank is reversed under the mirror or the
// transpose transform, the file under the flip or the transpose.  For the
// transpose that is a half turn, not the anti-diagonal reflection the
// encoder applies to the input planes (encoder.cpp:47-55); it is kept as
// the reference has it, since the policy indices must equal the
// reference's.
int TransformSquare(int sq, int transform) {
  int file = sq & 7, rank = sq >> 3;
  if (transform & (kMirrorTransform | kTransposeTransform))
    rank = 7 - rank;
  if (transform & (kFlipTransform | kTransposeTransform))
    file = 7 - file;
  return rank * 8 + file;
}
}  // namespace

int MoveToIndex(int from, int to, char promo, int transform) {
  if (from < 0 || from > 63 || to < 0 || to > 63)
    return -1;
  if (transform != 0) {
    from = TransformSquare(from, transform);
    to = TransformSquare(to, transform);
  }
  if (promo == 'q' || promo == 'r' || promo == 'b') {
    if ((from >> 3) != 6 || (to >> 3) != 7)
      return -1;
    const int p = promo == 'q' ? 0 : (promo == 'r' ? 1 : 2);
    return B().promotion[(from & 7) * 24 + (to & 7) * 3 + p];
  }
  return B().regular[from * 64 + to];
}

// Reference IndexToNNMove (policy_map.cpp:362-410): the inverse of the
// square map above (a transpose with one of flip / mirror takes the other).
bool IndexToMove(int index, int transform, int *from, int *to, char *promo) {
  if (index < 0 || index >= kPolicyOutputs)
    return false;
  const PolicyMove &m = MoveList()[index];
  int f = m.from, t = m.to;
  if (transform != 0) {
    int inv = transform;
    if (transform & kTransposeTransform) {
      inv = kTransposeTransform;
      if (transform & kFlipTransform)
        inv |= kMirrorTransform;
      if (transform & kMirrorTransform)
        inv |= kFlipTransform;
    }
    t = TransformSquare(t, inv);
    f = TransformSquare(f, inv);
  }
  *from = f;
  *to = t;
  *promo = m.promo;
  return true;
}

}  // namespace mfh_policy

// The 1858-entry policy move index and the attention-policy gather table.
//
// Both are rebuilt here from the rules that define them rather than stored:
//  * move index: every queen-line or knight move from->to (1792 entries,
//    ordered by from-square then to-square, a1 = 0), followed by the q/r/b
//    promotions from the 7th rank to the 8th (66 entries, ordered by
//    from-file, to-file, piece) -- the list in reference
//    src/nn/policy_map.cpp:35-245; knight promotions reuse the plain move
//    (policy_map.cpp:338-340).
//  * attention map: 64*64 raw QK logits (from*64+to) plus 8*24 promotion
//    logits (from_file*24 + to_file*3 + {q,r,b}) mapped to the 1858 index or
//    -1 -- reference src/nn/tables/attention_policy_map.h:15 (kAttnPolicyMap).
// Tests compare both against digests of the reference's own tables.
#pragma once

#include <array>
#include <cstdint>

namespace mfh_policy {

constexpr int kPolicyOutputs = 1858;
constexpr int kAttentionRaw = 64 * 64 + 8 * 24;  // 4288

struct PolicyMove {
  std::int16_t from;
  std::int16_t to;
  char promo;  // 0, 'q', 'r' or 'b'
};

const std::array<PolicyMove, kPolicyOutputs> &MoveList();
// raw attention-logit index (0..4287) -> policy index or -1.
const std::array<std::int16_t, kAttentionRaw> &AttentionMap();
// policy index -> raw attention-logit index (inverse of AttentionMap).
const std::array<std::int16_t, kPolicyOutputs> &AttentionGather();

// Static position encoding of INPUT_EMBEDDING_PE_MAP nets, [square][64]:
// -1 at the square itself, 1 at every square a queen or a knight reaches
// from it, 0 elsewhere -- the rule behind reference
// src/nn/tables/attention_policy_map.h:377 (kPosEncoding), checked against a
// digest of that table.
constexpr int kPosEncodingChannels = 64;
const std::array<float, 64 * kPosEncodingChannels> &StaticPositionEncoding();

// Input-plane transforms of the canonical input formats (reference
// src/nn/input_planes.h:16-20).
constexpr int kFlipTransform = 1;       // files a <-> h
constexpr int kMirrorTransform = 2;     // ranks 1 <-> 8
constexpr int kTransposeTransform = 4;  // the planes' anti-diagonal reflection

// Index of a move given in the side-to-move-relative frame, or -1
// (reference MoveToNNIndex, src/nn/policy_map.cpp:316-360).  `promo` is 0
// for no promotion or one of 'q','r','b','n'; `transform` is the one the
// encoder chose for the position (its squares are mapped as the reference
// maps them, see policy_tables.cpp).
int MoveToIndex(int from, int to, char promo, int transform = 0);

// Move of a policy index under `transform` (reference IndexToNNMove,
// policy_map.cpp:362-410): from/to squares and promo 0 / 'q' / 'r' / 'b'.
// False for an index outside 0..1857.
bool IndexToMove(int index, int transform, int *from, int *to, char *promo);

}  // namespace mfh_policy

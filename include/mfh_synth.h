/*
 * mfh_synth.h -- seeded synthetic inputs for the MI355X transformer backend.
 *
 * Host-only C ABI of libmfhost.so.  Nothing here is on the evaluation hot
 * path; these functions produce the deterministic nets and chess positions
 * that the benchmark and the parity tests feed to both the GPU backend
 * (mfhip.h) and the CPU oracle.  The reference has no counterpart for the net
 * generator (it loads trained .pb files, reference src/nn/loader.cpp:156-179);
 * the position encoder follows NN::EncodePositionForNN
 * (reference src/nn/encoder.cpp:249-475) for every input format.
 */
#ifndef MFH_SYNTH_H
#define MFH_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Initialisation kinds for mfs_fill_tensor. */
enum {
  MFS_INIT_NORMAL_FAN_IN = 0, /* N(0,1) / sqrt(fan_in)  (matrices, biases)   */
  MFS_INIT_ONE_PLUS_TENTH = 1, /* 1 + 0.1 N(0,1)        (LN gammas, mult gate) */
  MFS_INIT_TENTH = 2,          /* 0.1 N(0,1)            (LN betas, add gate)   */
  MFS_INIT_ZERO = 3
};

/* Deterministic fill: SplitMix64 stream seeded with seed ^ FNV-1a(name);
 * N(0,1) is the Irwin-Hall sum of twelve 24-bit uniforms minus 6, formed in
 * integer and double arithmetic only, so every IEEE host gets the same bits. */
void mfs_fill_tensor(uint64_t seed, const char *name, int init_kind,
                     double fan_in, float *out, uint64_t count);

/* Round fp32 values in place to the nearest bf16 (ties to even). */
void mfs_round_bf16(float *data, uint64_t count);

/* Seeded random playouts from the start position.  Game g (first_game <= g <
 * first_game + count) plays a uniformly random legal move each ply for a
 * length drawn uniformly from [min_plies, max_plies]; a game that reaches a
 * position without legal moves is replayed with fresh draws.  Writes, per
 * game: planes[112*64] (classical encoding of the final position with its
 * history), legal[256] policy indices of the legal moves in the
 * side-to-move frame padded with -1, and optionally the UCI move list
 * (NUL-terminated, space separated, `text_stride` bytes per game).
 * Returns 0 on success, a negative value on error. */
int mfs_playout_batch(uint64_t seed, int first_game, int count, int min_plies,
                      int max_plies, float *planes, int16_t *legal,
                      char *text, int text_stride);

/* Encode the position reached from `fen` after the space-separated UCI
 * `moves` (may be empty), with history.  Returns the number of legal moves
 * written to legal[] (policy indices, side-to-move frame) or -1 on error. */
int mfs_encode_game(const char *fen, const char *moves, float *planes,
                    int16_t *legal, int legal_cap);

/* The same for any input format of a network file (net.proto InputFormat:
 * 1 classical, 2 castling plane, 3 canonical, 4 canonical hectoplies, 132
 * canonical hectoplies armageddon, 5 canonical v2, 133 canonical v2
 * armageddon), fill_empty_history 0 NO / 1 FEN_ONLY / 2 ALWAYS, and
 * history_planes earlier positions at most (8 used).  The legal moves'
 * policy indices take the transform the encoder chose, written to
 * *transform_out when given (reference src/mcts/evaluator.cpp:152-160,
 * 194-200).  planes may be null.  Returns the legal-move count or -1. */
int mfs_encode_game_format(const char *fen, const char *moves, int input_format,
                           int fill_empty_history, int history_planes, float *planes,
                           int16_t *legal, int legal_cap, int *transform_out);

/* Policy index of the move from -> to (side-to-move frame; promo 0 or one
 * of 'q','r','b','n') under an input transform, or -1 (reference
 * NN::MoveToNNIndex, src/nn/policy_map.cpp:316-360). */
int mfs_move_to_index(int from, int to, char promo, int transform);

/* Move of a policy index under an input transform (reference
 * NN::IndexToNNMove, policy_map.cpp:362-410); -1 for a bad index. */
int mfs_index_to_move(int index, int transform, int *from, int *to, char *promo);

/* Legal-move tree size of `fen` at `depth`; -1 if the FEN is invalid. */
int64_t mfs_perft(const char *fen, int depth);

/* Policy tables: raw attention-logit index -> policy index (4288 entries),
 * policy index -> raw index (1858), and the 1858 UCI move strings (6 bytes
 * each, NUL padded). */
void mfs_policy_tables(int16_t *attention_map, int16_t *gather,
                       char *move_strings);

/* The static position encoding of PE_MAP nets, out[64*64] ([square][channel]). */
void mfs_static_position_encoding(float *out);

#ifdef __cplusplus
}
#endif

#endif /* MFH_SYNTH_H */

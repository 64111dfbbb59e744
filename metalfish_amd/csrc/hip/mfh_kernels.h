// Host-side launch wrappers for the gfx950 kernels of libmfhip.  Every
// wrapper validates the shapes and alignment its kernel and grid assume
// before launching, and returns hipErrorInvalidValue with a message in *err
// when they do not hold.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace mfh {

// Fixed power-of-two scale of the e4m3 lo parts of activations in the
// BF16X2_FP8LO precision: code = e4m3(lo * 2^kLo8Shift).  |lo| <= 2^-9 |x|
// for lo = x - bf16(x), so codes saturate (448) only for |x| > 224, far above
// the LayerNorm, attention and FFN outputs that carry them; lo parts below
// 2^-16 (|x| below ~2^-7) lose bits to e4m3 subnormals, an absolute error
// under 2^-20.
constexpr int kLo8Shift = 10;

// Column block of the per-row partial sums of a LayerNorm folded into GEMM
// epilogues (GemmParams::ln_stats / out_stats): 128 columns, or 64 where
// the residual GEMMs take 64-wide tiles (GemmParams::ln_part).
constexpr int kLnStatCols = 128;

// Activation ids used by kernel epilogues (the C ABI maps the
// reference's ActivationFunction values onto these).
enum Act : int {
  ACT_NONE = -1,
  ACT_RELU = 0,
  ACT_RELU2 = 1,
  ACT_TANH = 2,
  ACT_SIGMOID = 3,
  ACT_SWISH = 4,
  ACT_MISH = 5,
  ACT_SELU = 6,
};


enum GemmOut : int {
  GEMM_OUT_BF16 = 0,       // C = act(A.W^T + b) as bf16
  GEMM_OUT_F32 = 1,        // C = act(A.W^T + b) as fp32
  GEMM_OUT_RESID_F32 = 2,  // C = resid + alpha * (A.W^T + b) as fp32
};
// The residual of GEMM_OUT_RESID_F32 is fp32 `resid`, or, when resid16 is
// set, the split pair resid16 + resid16_lo (bf16 hi and lo planes, same ldr):
// the split-precision activation that the previous LayerNorm wrote for the
// next layer's input.

// C[M,N] = A[M,K] . W[N,K]^T with bf16 operands and fp32 accumulation.
// Columns >= split_n are written to C2 (column index minus split_n) so one
// launch can fill two tensors that share an input (e.g. Q|K|V and the
// smolgen compression).  Split precision: A_lo (same lda) holds the bf16
// residual of each activation (x = A + A_lo); C_lo / C2_lo receive the
// residuals of bf16 outputs.
struct GemmParams {
  const std::uint16_t *A = nullptr;
  const std::uint16_t *A_lo = nullptr;
  int lda = 0;
  const std::uint16_t *W = nullptr;
  // Alternatively e4m3 weight codes [N][ldw] with fp32 row scales (the
  // accumulated row is multiplied by wscale[n]).
  const std::uint8_t *W8 = nullptr;
  const float *wscale = nullptr;
  int ldw = 0;
  int M = 0, N = 0, K = 0;
  const float *bias = nullptr;
  int act = -1;
  int out_mode = GEMM_OUT_BF16;
  void *C = nullptr;
  void *C_lo = nullptr;
  int ldc = 0;
  void *C2 = nullptr;
  void *C2_lo = nullptr;
  int ldc2 = 0;
  int split_n = 1 << 30;
  const float *resid = nullptr;
  const std::uint16_t *resid16 = nullptr;
  const std::uint16_t *resid16_lo = nullptr;
  int ldr = 0;
  float alpha = 1.0f;
  // K split over blockIdx.y; each slice writes fp32 partials to
  // C + slice * M * ldc (GEMM_OUT_F32, no bias/activation).
  int k_splits = 1;
  // Optional fp32 scratch of partials_floats elements: lets LaunchGemm split
  // K for small problems (partials summed by a second kernel).
  float *partials = nullptr;
  size_t partials_floats = 0;
  // fp8 activations: A8 holds e4m3 codes [M][lda] of the rows A / ascale[m]
  // (the weights then are W8 with their row scales); the product runs on the
  // fp8 MFMA and output row m is scaled by ascale[m] * wscale[n].  K % 128
  // == 0, lda % 16 == 0, M >= 2048 rows.
  const std::uint8_t *A8 = nullptr;
  const float *ascale = nullptr;
  // fp8 lo correction (the BF16X2_FP8LO precision): the activation is hi + lo
  // with hi = A (bf16) and lo = A_lo8 / 2^kLo8Shift (e4m3 codes [M][lda8]),
  // and the product is hi . W^T on the bf16 MFMA plus A_lo8 . W_lo8^T
  // (e4m3 codes [N][ldw8]) on the fp8 MFMA, accumulated together; W then
  // holds the weights times 2^kLo8Shift / s_n and W_lo8 the e4m3 codes of
  // W_n / s_n, and wscale[n] = s_n / 2^kLo8Shift brings the sum back.
  // K % 128 == 0; whole 256 x 256 tiles over one K slice.
  const std::uint8_t *A_lo8 = nullptr;
  int lda8 = 0;
  const std::uint8_t *W_lo8 = nullptr;
  int ldw8 = 0;
  // bf16 outputs: the lo part as e4m3 codes of lo * 2^kLo8Shift [M][ldc8]
  // (instead of the bf16 C_lo plane), the A_lo8 of a following GEMM.
  std::uint8_t *C_lo8 = nullptr;
  int ldc8 = 0;
  // A LayerNorm folded into the GEMMs around it (the LayerNorm kernel then
  // does not run).  The rows x it normalises, y = LN(x) = (x - mu) r gamma +
  // beta with r = 1 / sqrt(E[x^2] - mu^2 + eps), are stored as x o gamma
  // (bf16 hi + lo planes) with per-row partial sums (sum x, sum x^2) over
  // blocks of ln_part columns (ln_width / ln_part pairs per row):
  // * producer (residual mode, out_gamma set): x = resid + alpha (acc + b) is
  //   written as x o out_gamma to C / C_lo (bf16 planes, C_lo8 codes) and
  //   its partial sums to out_stats, instead of x in fp32;
  // * consumer of y as the A operand (fold_c set): A holds x o gamma,
  //   fold_c[n] = sum_k gamma_k W[n][k] and the bias is b + W beta, so
  //   out = act(r (acc - mu fold_c[n]) + bias[n]) with the stats ln_stats;
  // * residual y (res_stats set): resid16 / resid16_lo hold x o gamma, and
  //   resid = r (x o gamma - mu res_gamma) + res_beta.
  // Residual modes with out_gamma or res_stats take whole tiles of 256 or
  // (ln_part 64) 64 columns (LaunchGemm rejects other shapes).
  const float *ln_stats = nullptr;
  const float *fold_c = nullptr;
  float ln_eps = 0.f;
  const float *res_stats = nullptr;
  const float *res_gamma = nullptr;
  const float *res_beta = nullptr;
  float res_eps = 0.f;
  const float *out_gamma = nullptr;
  float *out_stats = nullptr;
  int ln_width = 0;  // width of the normalised rows (K for ln_stats, N otherwise)
  int ln_part = kLnStatCols;  // columns per partial-sum block: 128 or 64
  // Tiles that leave room for a concurrent launch on another stream (bf16
  // weights).  beside_chain (split precision): whole-round 256 x 256 tiles
  // take two LDS stages (96 KiB) instead of three (144 KiB).  small_lds:
  // below the large-problem rows, 64 x 64 tiles over BK = 32 with two
  // stages (24 KiB split, 16 KiB single bf16) instead of BK = 64 with three
  // (72 / 48 KiB), so they fit on a CU beside a two-stage split or a
  // four-stage single-bf16 256 x 256 tile.  Neither changes the result
  // bits (the K order of the MFMAs is the same).
  bool beside_chain = false;
  bool small_lds = false;
  // Set by LaunchGemm: every output row start allows 4-column vector stores
  // (vec), and 8-column groups allow 16-byte accesses everywhere (vec8).
  bool vec = false;
  bool vec8 = false;
};

hipError_t LaunchGemm(const GemmParams &p, hipStream_t stream, std::string *err);
// Number of K slices LaunchGemm splits this (small-M) problem into when
// p.partials is set and p.k_splits == 1, or 1.  A caller that sums the
// partials itself (in a kernel it launches anyway, such as the LayerNorm
// after a residual GEMM) passes summed_by_consumer and launches with
// k_splits set to this value instead.
int GemmAutoSplits(const GemmParams &p, bool summed_by_consumer = false);
// Workgroup limits of those splits (64 x 64 tiles times slices): slices that
// need a reduce launch, and the two-way split a consumer sums.  The partials
// of one split GEMM therefore hold at most kSplitPairMaxGroups * 64 * 64
// floats.
constexpr long kSplitMaxGroups = 256;
constexpr long kSplitPairMaxGroups = 384;

// Whether LaunchGemm runs `p` (bf16 activations) on 256 x 256 tiles that
// fill whole rounds of 256 workgroups.
bool GemmWholeRoundTiles(const GemmParams &p);

// Whether LaunchGemm can run `p` with a folded LayerNorm (fold_c as a
// consumer in the bf16 mode, out_gamma / res_stats in the residual mode):
// a tile whose instance compiles that epilogue exists for its shape and
// operands.  (The pointers and widths are checked at the launch.)
bool GemmLnFoldOk(const GemmParams &p);

// Row-panel GEMM: one workgroup of eight waves owns 64 whole output rows
// and a panel of 128 * TN columns (TN = 2, 4, 6 or 8), so a row's outputs
// never leave the workgroup.  The activation panel goes through LDS (every
// wave reads all 64 rows); each wave streams its own 16 * TN weight rows
// from L2 straight into registers, one K step ahead.  Two epilogues:
//   PANEL_OUT_BF16: C = act(A.W^T + b) as bf16 (+ lo plane), row stride ldc;
//   PANEL_OUT_LN:   y = LayerNorm(resid + alpha * (A.W^T + b)) over the N
//                   columns of each row (N = 128 * TN, one column panel):
//                   mean = sum/N, var = sum(x^2)/N - mean^2 clamped at 0,
//                   y = (x - mean) / sqrt(var + eps) * gamma + beta
//                   (reference cpu_network.cpp:424-460, 1399-1457), written
//                   as bf16 hi (+ lo) planes to C / C_lo (ldc = N) and
//                   optionally fp32 to y_f32.  The residual is fp32 `resid`
//                   or the split pair resid16 + resid16_lo, stride N; it may
//                   alias the outputs (each element is read before the
//                   workgroup's statistics barrier and written after it by
//                   the same lane).
// Operands as GemmParams (A / A_lo K-contiguous, W bf16 or W8 e4m3 codes
// with row scales).  Constraints, checked by LaunchPanelGemm: M >= 1;
// K % 64 == 0 and K >= 128; N a multiple of the panel width.
enum PanelOut : int { PANEL_OUT_BF16 = 0, PANEL_OUT_LN = 1 };
struct PanelGemmParams {
  const std::uint16_t *A = nullptr;
  const std::uint16_t *A_lo = nullptr;
  int lda = 0;
  const std::uint16_t *W = nullptr;
  const std::uint8_t *W8 = nullptr;
  const float *wscale = nullptr;
  int ldw = 0;
  int M = 0, N = 0, K = 0;
  const float *bias = nullptr;
  int act = -1;
  int out_mode = PANEL_OUT_BF16;
  std::uint16_t *C = nullptr;
  std::uint16_t *C_lo = nullptr;
  int ldc = 0;
  const float *resid = nullptr;
  const std::uint16_t *resid16 = nullptr;
  const std::uint16_t *resid16_lo = nullptr;
  float alpha = 1.0f;
  float eps = 1e-3f;
  const float *gamma = nullptr, *beta = nullptr;
  float *y_f32 = nullptr;
};
// True when LaunchPanelGemm takes this shape (panel width for N exists).
bool PanelGemmShapeOk(int out_mode, int N, int K);
hipError_t LaunchPanelGemm(const PanelGemmParams &p, hipStream_t stream, std::string *err);

// Few-row GEMM (M <= 64, the single-position smolgen chain): C = A . W^T with
// the whole K per workgroup, so no split-K partials and no reduce launch.  A
// workgroup of 16 waves owns 16 * NT output columns for all M rows; its
// waves split the M rows into 16-row tiles and K into equal parts, load
// their fragments straight from global memory into registers, and sum the
// K parts through LDS in a fixed order.
//   A operand: the bf16 planes a16 (+ a16_lo), or, with `x` set, the
//   LayerNorm of fp32 rows computed on the fly:
//     A[r][k] = (x[s][c0 + k] - mean_s) * inv_std_s * gamma[c0 + k]
//               + beta[c0 + k],  s = r / rows_per_src,
//               c0 = (r % rows_per_src) * K,
//   with mean / variance from ln_parts partial (sum, sum of squares) pairs
//   per source row (ln_stats[part * ln_rows + s], as written by stats_out)
//   over ln_width columns: var = E[x^2] - mean^2 clamped at 0, inv_std =
//   1 / sqrt(var + eps) (reference cpu_network.cpp:424-460).  ln_split adds
//   the bf16 lo plane of the normalised value to the product.  With y16 set
//   the normalised rows are also stored (hi to y16, lo to y16_lo, fp32 to
//   y32, stride ldy; rows_per_src must be 1), each 64-wide K block by one
//   workgroup.
//   Outputs (row m, columns n .. n + 3 per lane):
//     SKINNY_OUT_BF16   act(acc + bias) -> bf16 hi (+ lo) planes, columns at
//                       or past split_n to C2 / C2_lo (ldc2)
//     SKINNY_OUT_F32    act(acc + bias) -> fp32
//     SKINNY_OUT_RESID  resid + alpha * (acc + bias) -> fp32, the residual
//                       fp32 `resid` or the planes resid16 + resid16_lo
//   stats_out (fp32 modes): per workgroup and row, the sum and sum of squares
//   of the stored values over its columns, at stats_out[2 * (blockIdx * M +
//   m)], for a later LayerNorm of these rows.
// Constraints (checked by LaunchSkinnyGemm): SkinnyShapeOk(M, N, K)
// (1 <= M <= 64, N % 4 == 0, K % 64 == 0 with the K parts dividing K / 64),
// 16-byte aligned operands, lda / ldw / ldy % 8 == 0, ldx % 4 == 0.
enum SkinnyOut : int { SKINNY_OUT_BF16 = 0, SKINNY_OUT_F32 = 1, SKINNY_OUT_RESID = 2 };
constexpr int kSkinnyMaxRows = 64;
struct SkinnyParams {
  const std::uint16_t *a16 = nullptr;
  const std::uint16_t *a16_lo = nullptr;
  int lda = 0;
  const float *x = nullptr;
  int ldx = 0;
  int rows_per_src = 1;
  const float *ln_stats = nullptr;
  int ln_parts = 0, ln_rows = 0, ln_width = 0;
  float ln_eps = 1e-5f;
  const float *gamma = nullptr, *beta = nullptr;
  bool ln_split = false;
  std::uint16_t *y16 = nullptr;
  std::uint16_t *y16_lo = nullptr;
  float *y32 = nullptr;
  int ldy = 0;
  const std::uint16_t *W = nullptr;
  int ldw = 0;
  int M = 0, N = 0, K = 0;
  int out_mode = SKINNY_OUT_BF16;
  const float *bias = nullptr;
  int act = -1;
  void *C = nullptr;
  std::uint16_t *C_lo = nullptr;
  int ldc = 0;
  int split_n = 1 << 30;
  void *C2 = nullptr;
  std::uint16_t *C2_lo = nullptr;
  int ldc2 = 0;
  const float *resid = nullptr;
  const std::uint16_t *resid16 = nullptr;
  const std::uint16_t *resid16_lo = nullptr;
  int ldr = 0;
  float alpha = 1.0f;
  float *stats_out = nullptr;
};
// Workgroups LaunchSkinnyGemm uses for N columns (the ln_parts of a
// LayerNorm that reads its stats_out).
int SkinnyGemmParts(int N);
bool SkinnyShapeOk(int M, int N, int K);
hipError_t LaunchSkinnyGemm(const SkinnyParams &p, hipStream_t stream, std::string *err);

// Rows of bf16 activations (x, plus the lo plane x_lo when given; stride
// ldx) as OCP e4m3 codes q (stride ldq) with one fp32 scale per row:
// scale = max|row| / 448 (1 for a zero row), q = e4m3(x / scale) rounded to
// nearest even.  16 <= cols <= 2048, cols % 16 == 0, 16-byte aligned rows.
hipError_t LaunchQuantizeRowsE4m3(const std::uint16_t *x, const std::uint16_t *x_lo, int ldx,
                                  int rows, int cols, std::uint8_t *q, int ldq, float *scale,
                                  hipStream_t stream, std::string *err);

// Packed planes -> embedding input rows and the dynamic-PE input.
//   emb_in [B*64, emb_ld] bf16: cols 0..111 plane values; with static_pe
//   ([64][pe_ch] fp32, PE_MAP nets) cols 112..111+pe_ch the square's table
//   row; the rest zero (PE_DENSE columns are filled by LaunchScatterPe);
//   emb_in_lo (split precision, may be null) gets the zero residual of those
//   exact values (planes and the table's -1/0/1 are exact in bf16).
//   pos_in [B, 64*12] bf16: square-major first 12 planes (exact in bf16).
hipError_t LaunchExpandInputs(const std::uint64_t *masks, const float *values,
                              int batch, std::uint16_t *emb_in,
                              std::uint16_t *emb_in_lo, int emb_ld,
                              const float *static_pe, int pe_ch,
                              std::uint16_t *pos_in, hipStream_t stream,
                              std::string *err);

// Debug view: packed planes -> fp32 planes [B,112,64].
hipError_t LaunchUnpackPlanes(const std::uint64_t *masks, const float *values,
                              int batch, float *planes, hipStream_t stream,
                              std::string *err);

// pe [B, 64*P] fp32 -> emb_in[b*64+sq][112 + c] (bf16, plus residual in
// emb_in_lo when not null).
hipError_t LaunchScatterPe(const float *pe, int batch, int pe_channels,
                           std::uint16_t *emb_in, std::uint16_t *emb_in_lo,
                           int emb_ld, hipStream_t stream, std::string *err);

// Row LayerNorm: y = (x - mean) * rstd * gamma + beta with the reference's
// E[x^2] - mean^2 variance (cpu_network.cpp:424-460), optionally followed by
// the input gates y = y * mult[c][sq] + add[c][sq] (cpu_network.cpp:
// 1268-1316, gate layout [width][64], sq = row % 64).  Writes fp32 and/or
// bf16 copies (y_bf16_lo: bf16 residual for split precision).  x may be a
// stack of `parts` partial sums [parts][rows][width] (split-K GEMM output)
// that are added together with `bias` and passed through `act` first.
struct LayerNormParams {
  const float *x = nullptr;
  int parts = 1;
  const float *bias = nullptr;
  int act = -1;
  // Residual LayerNorm input: x = resid + alpha * (sum of parts + bias), the
  // residual fp32 or the split pair resid16 + resid16_lo (row stride width;
  // may alias the outputs).  No activation with a residual.
  const float *resid = nullptr;
  const std::uint16_t *resid16 = nullptr;
  const std::uint16_t *resid16_lo = nullptr;
  float alpha = 1.0f;
  int rows = 0, width = 0;
  float eps = 1e-3f;
  const float *gamma = nullptr, *beta = nullptr;
  // Embedding gates (square rows): [64][width], square-major, 16-byte
  // aligned; y = y * mult_gate[sq][c] + add_gate[sq][c], sq = row % 64.
  const float *mult_gate = nullptr, *add_gate = nullptr;
  float *y_f32 = nullptr;
  std::uint16_t *y_bf16 = nullptr;
  std::uint16_t *y_bf16_lo = nullptr;
  // The lo part of each bf16 output as e4m3 codes of lo * 2^kLo8Shift
  // ([rows][width] bytes), beside or instead of y_bf16_lo.
  std::uint8_t *y_lo8 = nullptr;
};
hipError_t LaunchLayerNorm(const LayerNormParams &lp, hipStream_t stream,
                           std::string *err);

// Multi-head 64x64 attention per (position, head), head depth 32:
//   ctx = softmax(Q K^T / sqrt(32) + bias) V
// qkv [B*64, 3E] bf16 (Q | K | V, head h at columns h*32..), bias [B,H,4096]
// (bf16, or fp32 when bias_f32; each head's 64 x 64 in SmolgenBiasIndex
// order) or null, ctx [B*64, E] bf16.  Split
// precision inputs when qkv_lo is set (then ctx_lo is required); ctx_lo
// alone splits only the output.
// Element order of one (position, head)'s 64 x 64 smolgen bias in the
// tensor attention reads: lane 16 g + f of a wave holds, for query tile q,
// the four keys 16 t + 4 g .. + 3 of query 16 q + f in each key tile t, so
// those four are contiguous and a wave's loads for one key tile cover 256
// contiguous values.  The global projection's output rows are packed in
// this order, so its GEMM writes the bias directly in it.
constexpr int SmolgenBiasIndex(int query, int key) {
  return ((query >> 4) * 4 + (key >> 4)) * 256 + ((((key >> 2) & 3) << 4) + (query & 15)) * 4 +
         (key & 3);
}

struct AttentionParams {
  const std::uint16_t *qkv = nullptr;
  const std::uint16_t *qkv_lo = nullptr;
  // Alternatively the lo plane as e4m3 codes of lo * 2^kLo8Shift ([B*64][3E]
  // bytes, BF16X2_FP8LO), converted exactly to bf16 as it loads.
  const std::uint8_t *qkv_lo8 = nullptr;
  const void *bias = nullptr;
  int bias_f32 = 0;
  // With e4m3 lo inputs: the bias as bf16 hi (bias, bias_f32 0) plus the
  // e4m3 codes of its lo parts times 2^kLo8Shift, in the same order.
  const std::uint8_t *bias_lo8 = nullptr;
  int batch = 0, heads = 0;
  std::uint16_t *ctx = nullptr;
  std::uint16_t *ctx_lo = nullptr;
  // With split outputs: the lo plane as e4m3 codes of lo * 2^kLo8Shift
  // ([B*64][E] bytes) instead of ctx_lo.
  std::uint8_t *ctx_lo8 = nullptr;
  // Query tiles (of 4) per workgroup: 4, 2 or 1 (the rest over grid.y), or
  // 0 to choose by batch (fewer per workgroup when there are few of them).
  int q_tiles = 0;
};
hipError_t LaunchAttention(const AttentionParams &ap, hipStream_t stream,
                           std::string *err);

// The same attention for smolgen nets with the per-head bias generated in
// the kernel (reference cpu_network.cpp:1164-1218): for (position b, head
// h), bias[q][k] = sum_j gen[b][h*G + j] * Wg[q*64 + k][j], where gen is
// the smolgen dense2 output after its LayerNorm ([B, H*G] bf16, gen_lo its
// residual plane or null) and Wg the shared global projection [4096, G]
// (bf16, or e4m3 codes wg8 with row scales wg_scale).  A workgroup takes 16
// (position, head) pairs and q_tiles of the 4 query tiles; G is 64, 128 or 256.
struct AttentionSmolgenParams {
  const std::uint16_t *qkv = nullptr;
  const std::uint16_t *qkv_lo = nullptr;
  const std::uint16_t *gen = nullptr;
  const std::uint16_t *gen_lo = nullptr;
  const std::uint16_t *wg = nullptr;
  const std::uint8_t *wg8 = nullptr;
  const float *wg_scale = nullptr;
  int gen_width = 0;  // G
  int batch = 0, heads = 0;
  int q_tiles = 4;    // query tiles per workgroup: 1, 2 or 4
  std::uint16_t *ctx = nullptr;
  std::uint16_t *ctx_lo = nullptr;
};
hipError_t LaunchAttentionSmolgen(const AttentionSmolgenParams &ap, hipStream_t stream,
                                  std::string *err);
// Dynamic LDS bytes the kernel needs for a gen width (and whether gen has a
// lo plane); the launcher checks it against the device limit.
size_t AttentionSmolgenLds(int gen_width, bool gen_split);

// Attention policy map: raw[q,k] = Q_q.K_k / sqrt(Dp), the 8x24 promotion
// logits, and the 1858-entry gather (cpu_network.cpp:892-1025).
// qk [B*64, 2*Dp] bf16 (Q | K; qk_lo residual plane or null), promo [4, Dp]
// fp32, policy [B, 1858] fp32.
hipError_t LaunchPolicyMap(const std::uint16_t *qk, const std::uint16_t *qk_lo,
                           int batch, int dp, const float *promo,
                           const std::int16_t *gather, float *policy,
                           hipStream_t stream, std::string *err);

// MCTS priors over each position's legal moves (reference
// src/mcts/search.cpp:127-199): policy [B, 1858] raw logits, offsets [B + 1]
// into indices (policy indices, at most 256 per position; an index outside
// [0, 1858) reads logit 0), priors written at the same offsets.
hipError_t LaunchPolicyPriors(const float *policy, const std::int32_t *offsets,
                              const std::int16_t *indices, int batch, float inv_temp,
                              float *priors, hipStream_t stream, std::string *err);

// Value / moves-left head output: hidden = act(sum of `parts` partials
// [parts][B][vh] + b1), then dense2 and the output function: tanh (scalar
// value, 1 output), softmax (WDL, 3 outputs) or relu (moves left, 1 output).
enum { kHeadTanh = 0, kHeadSoftmax3 = 1, kHeadRelu = 2 };
hipError_t LaunchValueHead(const float *hidden, int parts, const float *b1,
                           int act, int batch, int vh, const float *w2,
                           const float *b2, int mode, float *out,
                           hipStream_t stream, std::string *err);

}  // namespace mfh

// Fused 64-token multi-head attention for gfx950 (head depth 32):
//   ctx_h = softmax(Q_h K_h^T / sqrt(32) + bias_h) V_h
// restating reference src/nn/cpu/cpu_network.cpp:1175-1254.
//
// One wave owns one (position, head); a workgroup holds 4 heads of one
// position and 4, 2 or 1 of its 4 query tiles (each tile's softmax is its
// own, so the split changes no result; at small batches it spreads the work
// over more workgroups and shortens each wave's chain).  The wave computes the transposed scores S^T = K Q^T with
// v_mfma_f32_16x16x32_bf16 (the MFMA's K dimension is exactly the head
// depth), K and Q fragments coming straight from HBM as 16-byte loads.  In
// that layout a lane holds, for one query, four consecutive keys of every
// 16-key tile, so:
//   * the smolgen bias for those keys is one 16-byte (fp32) or 8-byte (bf16)
//     load;
//   * the softmax over a query's 64 keys is 16 values in the lane plus two
//     cross-lane shuffles;
//   * the probabilities never leave registers: the eight keys a lane holds
//     for a pair of key tiles are exactly the eight K-slots that lane feeds
//     to the next MFMA (the MFMA sums over K, so only the pairing of P and V
//     slots matters), and ctx^T = V^T P^T takes them as its B operand.
// Only V^T goes through LDS (4 KiB per head, two 8-byte reads per fragment).
// ctx^T leaves each lane with four consecutive depths of one query; each
// query tile's context goes through a small LDS tile so that the workgroup
// stores its 4 heads' rows whole (256 contiguous bytes per row and plane,
// 16 bytes per lane).  Scores, softmax statistics and accumulation stay in
// fp32.
//
// Split precision: with SPLIT_IN, Q, K and V arrive as hi + lo bf16 planes,
// P is split the same way in registers, and each product takes three MFMAs
// (hi.hi + hi.lo + lo.hi; the lo.lo term is below fp32 resolution).  With
// SPLIT_OUT the context leaves as hi + lo planes (it feeds a split GEMM).
#include "mfh_device.h"
#include "mfh_kernels.h"

#include <mutex>
#include <type_traits>

namespace mfh {
namespace {

constexpr int kSq = 64;
constexpr int kDepth = 32;
constexpr int kHeadsPerBlock = 4;
// V^T rows: 64 keys plus 4 of padding (34 dwords per depth).  The P.V
// fragment reads (8 bytes per lane at dword 34 (16 dt + fr) + 16 u + 2 g)
// then spread each quarter wave over all 32 four-byte banks: with 36-dword
// rows (8 of padding) lanes fr and fr + 8 shared banks, and the counters read
// 4 conflict cycles per LDS instruction.
constexpr int kVtStride = kSq + 4;
// Context staging tile: 16 queries x (4 heads x 32 depths) bf16 per plane,
// rows of 16 chunks of 16 bytes, chunk c of row r stored at c ^ r.
constexpr int kCtxCols = kHeadsPerBlock * kDepth;


__device__ __forceinline__ f32x4 Mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 Join(u32x2 a, u32x2 b) {
  const u32x4 v{a[0], a[1], b[0], b[1]};
  return __builtin_bit_cast(bf16x8, v);
}

template <bool SPLIT, bool SPLIT_OUT, bool BIAS_F32, bool LO8_IN = false>
__global__ __launch_bounds__(256) void AttentionKernel(AttentionParams ap) {
  static_assert(!LO8_IN || SPLIT, "e4m3 lo inputs are the lo planes of split inputs");
  constexpr int PLANES = SPLIT ? 2 : 1;
  constexpr int OUT_PLANES = SPLIT_OUT ? 2 : 1;
  __shared__ __attribute__((aligned(16))) std::uint16_t vt_lds[kHeadsPerBlock][PLANES]
                                                                [kDepth * kVtStride];
  __shared__ __attribute__((aligned(16))) std::uint16_t ctx_lds[2][OUT_PLANES][16 * kCtxCols];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int heads = ap.heads;
  const int groups = heads / kHeadsPerBlock;
  const int b = blockIdx.x / groups;
  const int h = (blockIdx.x % groups) * kHeadsPerBlock + wave;
  const int qn = ap.q_tiles;              // query tiles of this workgroup
  const int q0 = blockIdx.y * qn;         // its first one
  const int E = heads * kDepth;
  const size_t ld = static_cast<size_t>(3) * E;
  const size_t pos = static_cast<size_t>(b) * kSq * ld;
  const int qcol = h * kDepth, kcol = E + h * kDepth, vcol = 2 * E + h * kDepth;
  const int fr = lane & 15, g = lane >> 4;

  // The head's V rows (for V^T), its K fragments and the first query tile's
  // Q fragments and bias go out first, so their latencies overlap; each
  // later query tile's Q fragments and bias are fetched while the tile
  // before it is processed.  Lane l's V rows: the key pair 2 (l % 32),
  // 2 (l % 32) + 1, depths 16 (l / 32) .. + 16.
  const int kp = lane & 31, dh = (lane >> 5) * 16;
  u32x4 vrow[PLANES][4];
#pragma unroll
  for (int pl = 0; pl < PLANES; ++pl) {
    if (LO8_IN && pl == 1) {
      // The lo plane from its e4m3 codes (16 per row), converted exactly.
      const std::uint8_t *base = ap.qkv_lo8 + pos + vcol + dh;
      const u32x4 c0 = *reinterpret_cast<const u32x4 *>(base + (2 * kp) * ld);
      const u32x4 c1 = *reinterpret_cast<const u32x4 *>(base + (2 * kp + 1) * ld);
      vrow[1][0] = __builtin_bit_cast(u32x4, Lo8x8ToBf16(u32x2{c0[0], c0[1]}));
      vrow[1][1] = __builtin_bit_cast(u32x4, Lo8x8ToBf16(u32x2{c0[2], c0[3]}));
      vrow[1][2] = __builtin_bit_cast(u32x4, Lo8x8ToBf16(u32x2{c1[0], c1[1]}));
      vrow[1][3] = __builtin_bit_cast(u32x4, Lo8x8ToBf16(u32x2{c1[2], c1[3]}));
      continue;
    }
    const std::uint16_t *base = (pl ? ap.qkv_lo : ap.qkv) + pos + vcol + dh;
    const u32x4 *r0 = reinterpret_cast<const u32x4 *>(base + (2 * kp) * ld);
    const u32x4 *r1 = reinterpret_cast<const u32x4 *>(base + (2 * kp + 1) * ld);
    vrow[pl][0] = r0[0];
    vrow[pl][1] = r0[1];
    vrow[pl][2] = r1[0];
    vrow[pl][3] = r1[1];
  }
  // S^T = K Q^T operands: tile (t, q) holds keys 16 t + 4 g + r (rows) for
  // queries 16 q + fr (columns).
  const std::uint16_t *qh = ap.qkv + pos;
  const std::uint16_t *ql = SPLIT && !LO8_IN ? ap.qkv_lo + pos : ap.qkv + pos;
  const std::uint8_t *q8 = LO8_IN ? ap.qkv_lo8 + pos : nullptr;
  // Eight lo values of row `row` from column `col` (bf16 plane or codes).
  auto load_lo = [&](size_t row, int col) {
    if constexpr (LO8_IN)
      return Lo8x8ToBf16(*reinterpret_cast<const u32x2 *>(q8 + row * ld + col));
    else
      return *reinterpret_cast<const bf16x8 *>(ql + row * ld + col);
  };
  bf16x8 kf[4], kl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kf[i] = *reinterpret_cast<const bf16x8 *>(qh + (i * 16 + fr) * ld + kcol + g * 8);
    if constexpr (SPLIT)
      kl[i] = load_lo(i * 16 + fr, kcol + g * 8);
  }
  // A query tile's Q lo fragment as loaded (bf16, or e4m3 codes converted
  // where the scores use them, so that the next tile's loads stay in flight
  // while this one is processed).
  using QLo = std::conditional_t<LO8_IN, u32x2, bf16x8>;
  auto load_q = [&](int q, bf16x8 &hi, QLo &lo) {
    hi = *reinterpret_cast<const bf16x8 *>(qh + (q * 16 + fr) * ld + qcol + g * 8);
    if constexpr (LO8_IN)
      lo = *reinterpret_cast<const u32x2 *>(q8 + (q * 16 + fr) * ld + qcol + g * 8);
    else if constexpr (SPLIT)
      lo = load_lo(q * 16 + fr, qcol + g * 8);
  };
  auto q_lo = [&](const QLo &lo) -> bf16x8 {
    if constexpr (LO8_IN)
      return Lo8x8ToBf16(lo);
    else
      return lo;
  };
  const size_t bias_off = (static_cast<size_t>(b) * heads + h) * kSq * kSq;
  // Bias of query tile q for the lane's keys 16 t + 4 g .. + 3, t = 0..3:
  // SmolgenBiasIndex(16 q + fr, 16 t + 4 g) = (4 q + t) 256 + 4 lane.  Kept
  // as loaded (fp32, bf16 pairs, or bf16 pairs + e4m3 lo codes) until the
  // scores use it, like Q's lo fragment.
  struct BiasWords {
    f32x4 f[4];
    u32x2 h[4];
    unsigned c[4];
  };
  auto load_bias = [&](int q, BiasWords &w) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const size_t e = bias_off + (q * 4 + t) * 256 + lane * 4;
      if constexpr (BIAS_F32) {
        w.f[t] = ap.bias ? *reinterpret_cast<const f32x4 *>(static_cast<const float *>(ap.bias) + e)
                         : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        w.h[t] = ap.bias ? *reinterpret_cast<const u32x2 *>(
                               static_cast<const std::uint16_t *>(ap.bias) + e)
                         : u32x2{0u, 0u};
        if constexpr (LO8_IN)
          w.c[t] = ap.bias ? *reinterpret_cast<const unsigned *>(ap.bias_lo8 + e) : 0u;
      }
    }
  };
  auto bias_tile = [&](const BiasWords &w, int t) -> f32x4 {
    if constexpr (BIAS_F32) {
      return w.f[t];
    } else {
      f32x4 x{__uint_as_float(w.h[t][0] << 16), __uint_as_float(w.h[t][0] & 0xFFFF0000u),
              __uint_as_float(w.h[t][1] << 16), __uint_as_float(w.h[t][1] & 0xFFFF0000u)};
      if constexpr (LO8_IN) {
        // The e4m3 codes of the lo parts times 2^kLo8Shift (BF16X2_FP8LO).
        constexpr float kInv = 1.0f / static_cast<float>(1 << kLo8Shift);
        const auto l01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w.c[t], kInv, false);
        const auto l23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w.c[t], kInv, true);
        x[0] += l01[0];
        x[1] += l01[1];
        x[2] += l23[0];
        x[3] += l23[1];
      }
      return x;
    }
  };
  bf16x8 qcur;
  QLo qlcur;
  BiasWords bcur;
  load_q(q0, qcur, qlcur);
  load_bias(q0, bcur);

  // V^T into LDS, one packed dword (two keys) per depth.  Each wave reads
  // only its own head's V^T.
#pragma unroll
  for (int pl = 0; pl < PLANES; ++pl) {
    std::uint32_t *vt = reinterpret_cast<std::uint32_t *>(vt_lds[wave][pl]);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const std::uint32_t x = vrow[pl][e < 8 ? 0 : 1][(e & 7) >> 1];
      const std::uint32_t y = vrow[pl][e < 8 ? 2 : 3][(e & 7) >> 1];
      const std::uint32_t lo = (e & 1) ? (x >> 16) : (x & 0xFFFFu);
      const std::uint32_t hi = (e & 1) ? (y >> 16) : (y & 0xFFFFu);
      vt[((dh + e) * kVtStride) / 2 + kp] = lo | (hi << 16);
    }
  }
  __syncthreads();

  // One query tile at a time: scores, scale + bias, softmax over the 64 keys
  // of each query 16 q + fr (the lane holds 16 of them, lanes fr, fr + 16,
  // fr + 32, fr + 48 the rest), then ctx^T = V^T P^T for the tile and its
  // store.  Only one tile's scores and probabilities are live at a time.
  const float scale = 0.17677669529663687f;  // 1 / sqrt(32)
  const size_t out_off =
      static_cast<size_t>(b) * kSq * E + (blockIdx.x % groups) * kHeadsPerBlock * kDepth;
#pragma unroll
  for (int qi = 0; qi < 4; ++qi) {
    if (qi >= qn)
      break;
    const int q = q0 + qi;
    bf16x8 qnext;
    QLo qlnext;
    BiasWords bnext;
    if (qi + 1 < qn) {
      load_q(q + 1, qnext, qlnext);
      load_bias(q + 1, bnext);
    }
    f32x4 s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      s[t] = Mfma(kf[t], qcur, f32x4{0.f, 0.f, 0.f, 0.f});
    if constexpr (SPLIT) {
      const bf16x8 ql_cur = q_lo(qlcur);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        s[t] = Mfma(kl[t], qcur, Mfma(kf[t], ql_cur, s[t]));
    }
    float v[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f32x4 bt = bias_tile(bcur, t);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[t][r] = s[t][r] * scale + bt[r];
    }
    float m = v[0][0];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        m = fmaxf(m, v[t][r]);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[t][r] = __expf(v[t][r] - m);
        sum += v[t][r];
      }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float inv = 1.f / sum;
    // B operands of ctx^T: K-slot j of pair u is key 32 u + 4 g + (j % 4) +
    // 16 (j / 4), i.e. tile t = 2 u + j / 4, element r = j % 4 (the MFMA
    // sums over K, so only the pairing of P and V slots matters).
    bf16x8 pf[2], plo[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      std::uint32_t hw[4], lw[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const float p0 = v[2 * u + j / 4][j % 4] * inv;
        const float p1 = v[2 * u + j / 4][j % 4 + 1] * inv;
        if constexpr (SPLIT)
          split_bf16x2(p0, p1, hw[j / 2], lw[j / 2]);
        else
          hw[j / 2] = pack_bf16x2(p0, p1);
      }
      pf[u] = __builtin_bit_cast(bf16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
      if constexpr (SPLIT)
        plo[u] = __builtin_bit_cast(bf16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
    }
    // ctx^T = V^T P^T: A = V^T fragment (depth 16 dt + fr, the lane's 8
    // keys), B = P fragment; tile dt holds depths 16 dt + 4 g + r for query
    // 16 q + fr.
    f32x4 o[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const int row = (dt * 16 + fr) * kVtStride + 32 * u + 4 * g;
        const std::uint16_t *vh = vt_lds[wave][0];
        const bf16x8 va = Join(*reinterpret_cast<const u32x2 *>(vh + row),
                               *reinterpret_cast<const u32x2 *>(vh + row + 16));
        o[dt] = Mfma(va, pf[u], o[dt]);
        if constexpr (SPLIT) {
          const std::uint16_t *vl = vt_lds[wave][1];
          const bf16x8 vb = Join(*reinterpret_cast<const u32x2 *>(vl + row),
                                 *reinterpret_cast<const u32x2 *>(vl + row + 16));
          o[dt] = Mfma(vb, pf[u], Mfma(va, plo[u], o[dt]));
        }
      }
    // Context of the tile into the staging buffer (lane: query fr, depths
    // 16 dt + 4 g .. + 3 of this wave's head = half of 16-byte chunk
    // 4 wave + 2 dt + g / 2), then one 16-byte store per plane and thread:
    // thread t takes chunk t % 16 of query row t / 16.  Rows 8-15 hold each
    // chunk's two 8-byte halves swapped: the 16 lanes of one g (queries
    // 0-15) then write distinct LDS banks (rows fr and fr + 8 share their
    // chunk's banks, and now take its other half), and the reader swaps
    // them back.
    std::uint16_t(*stage)[16 * kCtxCols] = ctx_lds[qi & 1];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int chunk = (4 * wave + 2 * dt + (g >> 1)) ^ fr;
      const int off = fr * kCtxCols + chunk * 8 + ((g & 1) ^ (fr >> 3)) * 4;
      std::uint32_t hw[2], lw[2];
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        if constexpr (SPLIT_OUT)
          split_bf16x2(o[dt][r], o[dt][r + 1], hw[r / 2], lw[r / 2]);
        else
          hw[r / 2] = pack_bf16x2(o[dt][r], o[dt][r + 1]);
      }
      *reinterpret_cast<u32x2 *>(stage[0] + off) = u32x2{hw[0], hw[1]};
      if constexpr (SPLIT_OUT)
        *reinterpret_cast<u32x2 *>(stage[1] + off) = u32x2{lw[0], lw[1]};
    }
    // Two staging buffers: the barrier of a tile also orders every read of
    // the previous tile's buffer before the next tile overwrites it.
    __syncthreads();
    {
      const int row = threadIdx.x >> 4, chunk = threadIdx.x & 15;
      const int src = row * kCtxCols + (chunk ^ row) * 8;
      const size_t idx = out_off + static_cast<size_t>(q * 16 + row) * E + chunk * 8;
      auto unswap = [&](u32x4 x) { return row >= 8 ? u32x4{x[2], x[3], x[0], x[1]} : x; };
      *reinterpret_cast<u32x4 *>(ap.ctx + idx) =
          unswap(*reinterpret_cast<const u32x4 *>(stage[0] + src));
      if constexpr (OUT_PLANES > 1) {
        const u32x4 l = unswap(*reinterpret_cast<const u32x4 *>(stage[1] + src));
        if (ap.ctx_lo8) {
          // The lo plane as e4m3 codes of lo * 2^kLo8Shift (rounded from
          // its bf16 value).
          float f[8];
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            f[2 * h] = __uint_as_float(l[h] << 16);
            f[2 * h + 1] = __uint_as_float(l[h] & 0xFFFF0000u);
          }
          *reinterpret_cast<u32x2 *>(ap.ctx_lo8 + idx) =
              u32x2{Lo8Pack4(f[0], f[1], f[2], f[3]), Lo8Pack4(f[4], f[5], f[6], f[7])};
        } else {
          *reinterpret_cast<u32x4 *>(ap.ctx_lo + idx) = l;
        }
      }
    }
    if (qi + 1 < qn) {
      qcur = qnext;
      qlcur = qlnext;
      bcur = bnext;
    }
  }
}

template <bool SPLIT, bool SPLIT_OUT, bool BIAS_F32, bool LO8_IN = false>
hipError_t Launch(const AttentionParams &ap, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((AttentionKernel<SPLIT, SPLIT_OUT, BIAS_F32, LO8_IN>),
                     dim3(grid, 4 / ap.q_tiles), dim3(256), 0, stream, ap);
  return hipGetLastError();
}

bool Misaligned(const void *p, std::uintptr_t bytes) {
  return (reinterpret_cast<std::uintptr_t>(p) & (bytes - 1)) != 0;
}

// ---- Attention with the smolgen bias generated in the kernel ---------------
//
// bias[p][q][k] = sum_j gen[p][j] Wg[64 q + k][j] for pair p = (position,
// head) (reference cpu_network.cpp:1164-1173) is a GEMM whose N dimension is
// the pairs: Wg is shared by every position and head.  A workgroup of 16
// waves takes 16 consecutive pairs of the flattened batch x heads list, so
// one MFMA column tile covers them all: per query tile, wave w computes the
// bias of query 16 qt + w for the 64 keys and 16 pairs (four 16-row tiles of
// Wg rows as the A operand, the pairs' gen vectors from LDS as B), and the
// result goes through LDS to the layout of the score tiles, where wave w
// runs the attention of pair w.  Two bias buffers: the bias of tile qt + 1
// is computed while other waves still run tile qt's attention, one barrier
// per tile.
//
// Wg rows stream from L2 (2 MiB, shared by every workgroup and layer); each
// lane loads 32 contiguous bytes per row and step pair, so a wave load
// covers whole 128-byte lines: K-slots 8 g .. 8 g + 7 of the two MFMAs of a
// step pair are elements 64 s2 + 16 g + 8 e .. + 7 (e = 0, 1) of both
// operands (the MFMA sums over K, so only the pairing matters).
//
// V^T, the A operand of ctx^T = V^T P^T, is gathered into registers once
// (eight 16-bit loads per fragment: lane (fr, g) holds depth 16 dt + fr of
// the keys 32 u + 4 g + (j % 4) + 16 (j / 4), the same key order as the
// probabilities it meets), so no LDS is spent on it.
constexpr int kPairs = 16;                     // pairs (= waves) per workgroup
constexpr int kBiasQS = kSq + 4;               // floats per staged query row
constexpr int kBiasPS = 16 * kBiasQS + 4;      // floats per pair (bank spread)
constexpr int kBiasFloats = kPairs * kBiasPS;  // one query tile's bias

template <int G, bool SPLIT, bool SPLIT_OUT, bool W8>
__global__ __launch_bounds__(1024) void AttentionSmolgenKernel(AttentionSmolgenParams ap) {
  constexpr int PLANES = SPLIT ? 2 : 1;
  constexpr int GP = G + 8;  // gen rows padded: 16-byte bank step
  constexpr int STEPS = G / 64;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float *bias_lds = reinterpret_cast<float *>(smem);  // [2][kBiasFloats]
  std::uint16_t *gen_lds = reinterpret_cast<std::uint16_t *>(smem + 2 * kBiasFloats * 4);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const int heads = ap.heads, E = heads * kDepth;
  const int pairs = ap.batch * heads;
  const int pair0 = blockIdx.x * kPairs;
  // Waves past the last pair compute on a clamped pair and store nothing.
  const bool valid = pair0 + w < pairs;
  const int p = min(pair0 + w, pairs - 1);
  const int b = p / heads, h = p % heads;
  const size_t ld = static_cast<size_t>(3) * E;
  const size_t pos = static_cast<size_t>(b) * kSq * ld;
  const int qt_begin = blockIdx.y * ap.q_tiles, qt_end = qt_begin + ap.q_tiles;

  // The 16 pairs' gen vectors (rows p * G of [B, H * G]) into LDS.
  {
    const int chunks = G / 8;  // 16-byte chunks per row
    for (int c = threadIdx.x; c < PLANES * kPairs * chunks; c += 1024) {
      const int pl = c / (kPairs * chunks), rem = c % (kPairs * chunks);
      const int pr = rem / chunks, ch = rem % chunks;
      const std::uint16_t *src = (pl ? ap.gen_lo : ap.gen) +
                                 static_cast<size_t>(min(pair0 + pr, pairs - 1)) * G + ch * 8;
      *reinterpret_cast<u32x4 *>(gen_lds + (pl * kPairs + pr) * GP + ch * 8) =
          *reinterpret_cast<const u32x4 *>(src);
    }
  }
  const std::uint16_t *qh = ap.qkv + pos;
  const std::uint16_t *ql = SPLIT ? ap.qkv_lo + pos : ap.qkv + pos;
  const int qcol = h * kDepth, kcol = E + h * kDepth, vcol = 2 * E + h * kDepth;
  // V^T fragments (dt, u): slot j holds V[32 u + 4 g + (j % 4) + 16 (j / 4)][16 dt + fr].
  bf16x8 vt[PLANES][2][2];
#pragma unroll
  for (int pl = 0; pl < PLANES; ++pl)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const std::uint16_t *col = (pl ? ql : qh) + vcol + 16 * dt + fr;
        std::uint32_t wd[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int j0 = 2 * jj, j1 = 2 * jj + 1;
          const int k0 = 32 * u + 4 * g + (j0 & 3) + 16 * (j0 >> 2);
          const int k1 = 32 * u + 4 * g + (j1 & 3) + 16 * (j1 >> 2);
          wd[jj] = static_cast<std::uint32_t>(col[k0 * ld]) |
                   (static_cast<std::uint32_t>(col[k1 * ld]) << 16);
        }
        vt[pl][dt][u] = __builtin_bit_cast(bf16x8, u32x4{wd[0], wd[1], wd[2], wd[3]});
      }
  __syncthreads();  // gen vectors in LDS

  // Bias of query tile qt into buffer qt & 1.
  auto bias_phase = [&](int qt) {
    const int qq = qt * 16 + w;
    f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const size_t row0 = static_cast<size_t>(qq) * kSq + fr;  // Wg row of tile i: row0 + 16 i
    // Wg fragments of step pair s2 for the four row tiles (32 bytes per lane
    // and row; e4m3: 16 codes), requested one step pair ahead of their MFMAs.
    auto load_a = [&](int s2, u32x4 (&raw)[4][2]) {
      const int kc = 64 * s2 + 16 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (W8) {
          raw[i][0] = *reinterpret_cast<const u32x4 *>(ap.wg8 + (row0 + 16 * i) * G + kc);
        } else {
          const u32x4 *src = reinterpret_cast<const u32x4 *>(ap.wg + (row0 + 16 * i) * G + kc);
          raw[i][0] = src[0];
          raw[i][1] = src[1];
        }
      }
    };
    u32x4 cur[4][2], nxt[4][2];
    load_a(0, cur);
#pragma unroll
    for (int s2 = 0; s2 < STEPS; ++s2) {
      if (s2 + 1 < STEPS)
        load_a(s2 + 1, nxt);
      const int kc = 64 * s2 + 16 * g;
      bf16x8 bh[2], bl[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        bh[e] = *reinterpret_cast<const bf16x8 *>(gen_lds + fr * GP + kc + 8 * e);
        if constexpr (SPLIT)
          bl[e] = *reinterpret_cast<const bf16x8 *>(gen_lds + (kPairs + fr) * GP + kc + 8 * e);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x8 a[2];
        if constexpr (W8) {
          a[0] = Fp8x8ToBf16(u32x2{cur[i][0][0], cur[i][0][1]});
          a[1] = Fp8x8ToBf16(u32x2{cur[i][0][2], cur[i][0][3]});
        } else {
          a[0] = __builtin_bit_cast(bf16x8, cur[i][0]);
          a[1] = __builtin_bit_cast(bf16x8, cur[i][1]);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          acc[i] = Mfma(a[e], bh[e], acc[i]);
          if constexpr (SPLIT)
            acc[i] = Mfma(a[e], bl[e], acc[i]);
        }
      }
      if (s2 + 1 < STEPS) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          cur[i][0] = nxt[i][0];
          cur[i][1] = nxt[i][1];
        }
      }
    }
    // Lane (fr, g) holds bias rows 16 i + 4 g + r (keys) of query qq for
    // pair fr.
    float *dst = bias_lds + (qt & 1) * kBiasFloats + fr * kBiasPS + w * kBiasQS + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 v = acc[i];
      if constexpr (W8) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          v[r] *= ap.wg_scale[qq * kSq + 16 * i + 4 * g + r];
      }
      *reinterpret_cast<f32x4 *>(dst + 16 * i) = v;
    }
  };

  const float scale = 0.17677669529663687f;  // 1 / sqrt(32)
  const size_t out_row0 = static_cast<size_t>(b) * kSq;
  bias_phase(qt_begin);
  for (int qt = qt_begin; qt < qt_end; ++qt) {
    // Bias of tile qt visible; every wave is past tile qt - 1's attention,
    // so buffer (qt + 1) & 1 may be overwritten.
    __syncthreads();
    if (qt + 1 < qt_end)
      bias_phase(qt + 1);
    // K fragments (A operand of S^T = K Q^T: keys 16 t + fr, depths 8 g ..)
    // and this tile's Q fragments, from L2 for each tile: registers for K
    // would not survive the bias phase without spilling.
    bf16x8 kf[4], kl[4], qf, qfl;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      kf[t] = *reinterpret_cast<const bf16x8 *>(qh + (t * 16 + fr) * ld + kcol + g * 8);
      if constexpr (SPLIT)
        kl[t] = *reinterpret_cast<const bf16x8 *>(ql + (t * 16 + fr) * ld + kcol + g * 8);
    }
    qf = *reinterpret_cast<const bf16x8 *>(qh + (qt * 16 + fr) * ld + qcol + g * 8);
    if constexpr (SPLIT)
      qfl = *reinterpret_cast<const bf16x8 *>(ql + (qt * 16 + fr) * ld + qcol + g * 8);
    f32x4 s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
      s[t] = Mfma(kf[t], qf, f32x4{0.f, 0.f, 0.f, 0.f});
    if constexpr (SPLIT) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        s[t] = Mfma(kl[t], qf, Mfma(kf[t], qfl, s[t]));
    }
    const float *bsrc = bias_lds + (qt & 1) * kBiasFloats + w * kBiasPS + fr * kBiasQS + 4 * g;
    float v[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f32x4 bb = *reinterpret_cast<const f32x4 *>(bsrc + 16 * t);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[t][r] = s[t][r] * scale + bb[r];
    }
    float m = v[0][0];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        m = fmaxf(m, v[t][r]);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[t][r] = __expf(v[t][r] - m);
        sum += v[t][r];
      }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float inv = 1.f / sum;
    bf16x8 pf[2], plo[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      std::uint32_t hw[4], lw[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const float p0 = v[2 * u + j / 4][j % 4] * inv;
        const float p1 = v[2 * u + j / 4][j % 4 + 1] * inv;
        if constexpr (SPLIT)
          split_bf16x2(p0, p1, hw[j / 2], lw[j / 2]);
        else
          hw[j / 2] = pack_bf16x2(p0, p1);
      }
      pf[u] = __builtin_bit_cast(bf16x8, u32x4{hw[0], hw[1], hw[2], hw[3]});
      if constexpr (SPLIT)
        plo[u] = __builtin_bit_cast(bf16x8, u32x4{lw[0], lw[1], lw[2], lw[3]});
    }
    f32x4 o[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        o[dt] = Mfma(vt[0][dt][u], pf[u], o[dt]);
        if constexpr (SPLIT)
          o[dt] = Mfma(vt[1][dt][u], pf[u], Mfma(vt[0][dt][u], plo[u], o[dt]));
      }
    // Lane (fr, g): depths 16 dt + 4 g .. + 3 of query 16 qt + fr.
    if (valid) {
      const size_t off = (out_row0 + qt * 16 + fr) * E + h * kDepth + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        std::uint32_t hw[2], lw[2];
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          if constexpr (SPLIT_OUT)
            split_bf16x2(o[dt][r], o[dt][r + 1], hw[r / 2], lw[r / 2]);
          else
            hw[r / 2] = pack_bf16x2(o[dt][r], o[dt][r + 1]);
        }
        *reinterpret_cast<u32x2 *>(ap.ctx + off + 16 * dt) = u32x2{hw[0], hw[1]};
        if constexpr (SPLIT_OUT)
          *reinterpret_cast<u32x2 *>(ap.ctx_lo + off + 16 * dt) = u32x2{lw[0], lw[1]};
      }
    }
  }
}

template <int G, bool SPLIT, bool SPLIT_OUT, bool W8>
hipError_t LaunchSmolgenG(const AttentionSmolgenParams &ap, dim3 grid, size_t lds,
                          hipStream_t stream) {
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&AttentionSmolgenKernel<G, SPLIT, SPLIT_OUT, W8>),
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  });
  if (attr != hipSuccess)
    return attr;
  hipLaunchKernelGGL((AttentionSmolgenKernel<G, SPLIT, SPLIT_OUT, W8>), grid, dim3(1024), lds,
                     stream, ap);
  return hipGetLastError();
}

// Gen widths of Lc0-style smolgen nets: 64, 128, 256.
template <bool SPLIT, bool SPLIT_OUT, bool W8>
hipError_t LaunchSmolgen(const AttentionSmolgenParams &ap, dim3 grid, size_t lds,
                         hipStream_t stream) {
  switch (ap.gen_width) {
  case 64: return LaunchSmolgenG<64, SPLIT, SPLIT_OUT, W8>(ap, grid, lds, stream);
  case 128: return LaunchSmolgenG<128, SPLIT, SPLIT_OUT, W8>(ap, grid, lds, stream);
  default: return LaunchSmolgenG<256, SPLIT, SPLIT_OUT, W8>(ap, grid, lds, stream);
  }
}

}  // namespace

size_t AttentionSmolgenLds(int gen_width, bool gen_split) {
  return static_cast<size_t>(2) * kBiasFloats * 4 +
         static_cast<size_t>(gen_split ? 2 : 1) * kPairs * (gen_width + 8) * 2;
}

hipError_t LaunchAttentionSmolgen(const AttentionSmolgenParams &ap, hipStream_t stream,
                                  std::string *err) {
  const bool split = ap.qkv_lo != nullptr;
  const bool split_out = ap.ctx_lo != nullptr;
  const bool w8 = ap.wg8 != nullptr;
  const size_t lds = AttentionSmolgenLds(ap.gen_width, ap.gen_lo != nullptr);
  if (ap.batch <= 0 || ap.heads <= 0 || !ap.qkv || !ap.ctx || !ap.gen ||
      (!ap.wg && !ap.wg8) || (ap.wg && ap.wg8) || (w8 && !ap.wg_scale) ||
      (ap.gen_width != 64 && ap.gen_width != 128 && ap.gen_width != 256) ||
      lds > 160 * 1024 ||
      (ap.q_tiles != 1 && ap.q_tiles != 2 && ap.q_tiles != 4) ||
      (split != (ap.gen_lo != nullptr)) || (split && !split_out) ||
      Misaligned(ap.qkv, 16) || Misaligned(ap.ctx, 8) || Misaligned(ap.gen, 16) ||
      (ap.wg && Misaligned(ap.wg, 16)) || (ap.wg8 && Misaligned(ap.wg8, 16)) ||
      (split && (Misaligned(ap.qkv_lo, 16) || Misaligned(ap.gen_lo, 16))) ||
      (split_out && Misaligned(ap.ctx_lo, 8))) {
    if (err)
      *err = "attention_smolgen: needs batch, heads > 0, gen width 64, 128 or 256, "
             "q_tiles 1/2/4, one of wg / wg8 (with scales), aligned operands, and "
             "gen / qkv / ctx lo planes together";
    return hipErrorInvalidValue;
  }
  const int groups = (ap.batch * ap.heads + kPairs - 1) / kPairs;
  const dim3 grid(groups, 4 / ap.q_tiles);
  if (w8)
    return split ? LaunchSmolgen<true, true, true>(ap, grid, lds, stream)
           : split_out ? LaunchSmolgen<false, true, true>(ap, grid, lds, stream)
                       : LaunchSmolgen<false, false, true>(ap, grid, lds, stream);
  return split ? LaunchSmolgen<true, true, false>(ap, grid, lds, stream)
         : split_out ? LaunchSmolgen<false, true, false>(ap, grid, lds, stream)
                     : LaunchSmolgen<false, false, false>(ap, grid, lds, stream);
}

hipError_t LaunchAttention(const AttentionParams &ap, hipStream_t stream, std::string *err) {
  const bool lo8_in = ap.qkv_lo8 != nullptr;
  const bool split = ap.qkv_lo != nullptr || lo8_in;
  const bool split_out = ap.ctx_lo != nullptr || ap.ctx_lo8 != nullptr;
  if (ap.batch <= 0 || ap.heads <= 0 || ap.heads % kHeadsPerBlock || !ap.qkv || !ap.ctx ||
      Misaligned(ap.qkv, 16) || Misaligned(ap.ctx, 16) ||
      (ap.bias && Misaligned(ap.bias, ap.bias_f32 ? 16 : 8)) ||
      (split && !split_out) || (ap.qkv_lo && Misaligned(ap.qkv_lo, 16)) ||
      (lo8_in && (ap.qkv_lo || Misaligned(ap.qkv_lo8, 16))) ||
      (ap.bias_lo8 && (!lo8_in || ap.bias_f32 || !ap.bias || Misaligned(ap.bias_lo8, 4))) ||
      (ap.ctx_lo && Misaligned(ap.ctx_lo, 16)) || (ap.ctx_lo && ap.ctx_lo8) ||
      (ap.ctx_lo8 && Misaligned(ap.ctx_lo8, 8))) {
    if (err)
      *err = "attention: needs batch > 0, heads % 4 == 0, 16-byte aligned qkv and ctx, "
             "8-byte aligned bias, and one lo output plane (bf16 or e4m3) whenever the "
             "input has one";
    return hipErrorInvalidValue;
  }
  if (ap.q_tiles != 0 && ap.q_tiles != 1 && ap.q_tiles != 2 && ap.q_tiles != 4) {
    if (err)
      *err = "attention: q_tiles must be 0 (by batch), 1, 2 or 4";
    return hipErrorInvalidValue;
  }
  const int grid = ap.batch * (ap.heads / kHeadsPerBlock);
  AttentionParams a = ap;
  // By batch: whole heads from 512 workgroups up (two rounds of the CUs),
  // below that the query tiles split over two or four workgroups (batch 1
  // forward 1.36 -> 1.29 ms; batch 40 3.18 -> 3.15).
  if (a.q_tiles == 0)
    a.q_tiles = grid >= 512 ? 4 : grid >= 128 ? 2 : 1;
  // e4m3 lo inputs (BF16X2_FP8LO): an fp32 bias, or bf16 hi + e4m3 lo.
  if (lo8_in && a.bias && !a.bias_f32 && !a.bias_lo8) {
    if (err)
      *err = "attention: e4m3 lo inputs take an fp32 bias or a bf16 one with e4m3 lo codes";
    return hipErrorInvalidValue;
  }
  if (lo8_in && a.bias_lo8)
    return Launch<true, true, false, true>(a, grid, stream);
  if (lo8_in)
    return Launch<true, true, true, true>(a, grid, stream);
  if (split)
    return a.bias_f32 ? Launch<true, true, true>(a, grid, stream)
                      : Launch<true, true, false>(a, grid, stream);
  if (split_out)
    return a.bias_f32 ? Launch<false, true, true>(a, grid, stream)
                      : Launch<false, true, false>(a, grid, stream);
  return a.bias_f32 ? Launch<false, false, true>(a, grid, stream)
                    : Launch<false, false, false>(a, grid, stream);
}

}  // namespace mfh

// Attention policy head for gfx950: the 64x64 query-key logits, the 8x24
// promotion logits and the gather into the 1858-move policy
// (reference src/nn/cpu/cpu_network.cpp:892-1025, gather table 91-103).
//
// One workgroup of 16 waves per position, or up to 64 positions four, one
// per block of 16 query rows (a single position's Q K^T on one workgroup
// waited on that CU's loads: 45 us at batch 1).  A wave computes 16 query
// rows against all 64 keys over an interleaved quarter (one workgroup) or
// sixteenth (four) of the Dp dimension, with v_mfma_f32_16x16x32_bf16
// straight from global memory (Q and K rows are K-contiguous); the partial
// blocks go to LDS and are summed in a fixed order, then scaled by
// 1 / sqrt(Dp).  The promotion logit for p in [0,192) is, as in the
// reference,
//   raw[48 + (p%64)/8][56 + (p%64)%8] + K[56 + (p%24)/3] . (promo[p%3] + promo[3]).
// The 24 promotion-offset dot products are formed once per position, by the
// workgroup of query rows 48-63.
// Split precision: Q and K arrive as hi + lo planes and each fragment product
// takes three MFMAs (hi.hi + hi.lo + lo.hi).
#include "mfh_device.h"
#include "mfh_kernels.h"

namespace mfh {
namespace {

constexpr int kSq = 64;
constexpr int kOutputs = 1858;
constexpr int kMaxMoves = 256;

template <bool SPLIT, int NQB>
__global__ __launch_bounds__(1024) void PolicyMapKernel(
    const std::uint16_t *__restrict__ qk, const std::uint16_t *__restrict__ qk_lo, int dp,
    float scale, const float *__restrict__ promo, const std::int16_t *__restrict__ gather,
    float *__restrict__ policy) {
  // NQB workgroups per position; each takes QBW blocks of 16 query rows,
  // its waves DC interleaved parts of the depth.
  constexpr int QBW = 4 / NQB, DC = 16 / QBW;
  __shared__ float part[DC][QBW * 16 * kSq];
  __shared__ float pk_term[24];
  __shared__ float pk_wave[16][24];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int qbl = wave % QBW, dc = wave / QBW;
  const int qb = blockIdx.x * QBW + qbl, b = blockIdx.y;
  const int row0 = 16 * QBW * blockIdx.x;  // the workgroup's first query row
  const size_t ld = static_cast<size_t>(2) * dp;
  const size_t pos = static_cast<size_t>(b) * kSq * ld;
  const std::uint16_t *base = qk + pos;
  const int fr = lane & 15, fc = (lane >> 4) * 8;

  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const size_t qoff = (qb * 16 + fr) * ld + fc;
#pragma unroll 2
  for (int k0 = dc * 32; k0 < dp; k0 += 32 * DC) {
    const bf16x8 a = *reinterpret_cast<const bf16x8 *>(base + qoff + k0);
    bf16x8 kb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      kb[j] = *reinterpret_cast<const bf16x8 *>(base + (j * 16 + fr) * ld + dp + fc + k0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, kb[j], acc[j], 0, 0, 0);
    if constexpr (SPLIT) {
      const bf16x8 a_lo = *reinterpret_cast<const bf16x8 *>(qk_lo + pos + qoff + k0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8 kl = *reinterpret_cast<const bf16x8 *>(qk_lo + pos + (j * 16 + fr) * ld +
                                                            dp + fc + k0);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, kl, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_lo, kb[j], acc[j], 0, 0, 0);
      }
    }
  }
  // Query row q of the workgroup at (q - row0) * 64.
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      part[dc][(qbl * 16 + (lane >> 4) * 4 + r) * kSq + j * 16 + fr] = acc[j][r];

  // Promotion offsets (the workgroup of query rows 48-63 only; the branch
  // is uniform over the workgroup): term[t][tf] = K[56+tf] . (promo[t] +
  // promo[3]).  Thread c takes depth c (c, c + 1024, ...) of all 24
  // products, so every load is issued before any sum waits on one; then one
  // wave sum per product and a fixed-order sum over the 16 waves.
  const bool promos = blockIdx.x == NQB - 1;
  if (promos) {
    float term[24];
#pragma unroll
    for (int d = 0; d < 24; ++d)
      term[d] = 0.f;
    for (int c = threadIdx.x; c < dp; c += 1024) {
      float pr[3];
      const float p3 = promo[static_cast<size_t>(3) * dp + c];
#pragma unroll
      for (int t = 0; t < 3; ++t)
        pr[t] = promo[static_cast<size_t>(t) * dp + c] + p3;
#pragma unroll
      for (int tf = 0; tf < 8; ++tf) {
        const size_t koff = (56 + tf) * ld + dp + c;
        float kv = bf16_to_f32(base[koff]);
        if constexpr (SPLIT)
          kv += bf16_to_f32(qk_lo[pos + koff]);
#pragma unroll
        for (int t = 0; t < 3; ++t)
          term[t * 8 + tf] += kv * pr[t];
      }
    }
#pragma unroll
    for (int d = 0; d < 24; ++d) {
      const float w = wave_sum(term[d]);
      if (lane == 0)
        pk_wave[wave][d] = w;
    }
  }
  __syncthreads();
  if (promos && threadIdx.x < 24) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w)
      sum += pk_wave[w][threadIdx.x];
    pk_term[threadIdx.x] = sum;
  }
  __syncthreads();

  // Each workgroup writes the outputs whose logit lies in its query rows
  // (the first also the ones with no logit; the last the promotions,
  // queries 48-55).
  float *out = policy + static_cast<size_t>(b) * kOutputs;
  auto raw = [&](int q, int k) {
    const int i = (q - row0) * kSq + k;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < DC; ++w)
      v += part[w][i];
    return v * scale;
  };
  for (int i = threadIdx.x; i < kOutputs; i += 1024) {
    const int r = gather[i];
    if (r >= 0 && r < kSq * kSq) {
      if (r / kSq / (16 * QBW) == static_cast<int>(blockIdx.x))
        out[i] = raw(r / kSq, r % kSq);
    } else if (r >= kSq * kSq) {
      if (promos) {
        const int p = r - kSq * kSq;
        const int pair = p % kSq;
        out[i] = raw(48 + pair / 8, 56 + pair % 8) + pk_term[(p % 3) * 8 + (p % 24) / 3];
      }
    } else if (blockIdx.x == 0) {
      out[i] = 0.f;
    }
  }
}

// Schraudolph's exponential (N. N. Schraudolph, "A fast, compact
// approximation of the exponential function", Neural Computation 11(4),
// 1999): the binary32 pattern int(x * 2^23 / ln 2) + 127 * 2^23, with x
// clamped to [-88, 88] as the reference's MCTS does (src/mcts/core.h:38-44).
// The clamp keeps the comparisons of std::min / std::max (a NaN becomes 88).
__device__ __forceinline__ float SchraudolphExp(float x) {
  x = x < 88.0f ? x : 88.0f;
  x = -88.0f < x ? x : -88.0f;
  const int bits = static_cast<int>(x * 12102203.0f) + 1065353216;
  return __int_as_float(bits);
}

// MCTS priors of the legal moves (reference ApplyNNPolicyToNode,
// src/mcts/search.cpp:127-199, fed as NNMCTSEvaluator::BuildResult feeds it,
// src/mcts/evaluator.cpp:181-224): logit = policy[idx] for an index inside
// [0, 1858) and 0 otherwise; max over the moves; p = exp((logit - max) /
// temperature) with Schraudolph's exponential; a sequential sum in move order;
// p / sum, or 1 / n when the sum is not positive.  Every step is the same IEEE
// operation in the same order as on the CPU, so the priors match the CPU
// computation bit for bit.  One wave per position, at most 256 moves
// (search.cpp:49 kMaxEdges); the moves of position b are
// indices[offsets[b] .. offsets[b + 1]).
__global__ __launch_bounds__(64) void PolicyPriorsKernel(
    const float *__restrict__ policy, const std::int32_t *__restrict__ offsets,
    const std::int16_t *__restrict__ indices, float inv_temp, float *__restrict__ priors) {
  __shared__ float e[kMaxMoves];
  __shared__ float total;
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int start = offsets[b];
  int n = offsets[b + 1] - start;
  n = n < 0 ? 0 : (n > kMaxMoves ? kMaxMoves : n);
  const float *logits = policy + static_cast<size_t>(b) * kOutputs;
  float l[kMaxMoves / 64];
  float m = -__builtin_inff();
#pragma unroll
  for (int r = 0; r < kMaxMoves / 64; ++r) {
    const int i = r * 64 + lane;
    l[r] = 0.0f;
    if (i < n) {
      const int k = indices[start + i];
      l[r] = k >= 0 && k < kOutputs ? logits[k] : 0.0f;
      m = l[r] > m ? l[r] : m;  // a NaN never replaces the running maximum
    }
  }
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    const float o = __shfl_xor(m, s);
    m = o > m ? o : m;
  }
#pragma unroll
  for (int r = 0; r < kMaxMoves / 64; ++r) {
    const int i = r * 64 + lane;
    if (i < n)
      e[i] = SchraudolphExp((l[r] - m) * inv_temp);
  }
  __syncthreads();
  if (lane == 0) {
    float sum = 0.0f;
    for (int i = 0; i < n; ++i)
      sum += e[i];
    total = sum;
  }
  __syncthreads();
  const float sum = total;
  const bool uniform = sum <= 0.0f;
  const float scale = uniform ? 1.0f / static_cast<float>(n > 0 ? n : 1) : 1.0f / sum;
#pragma unroll
  for (int r = 0; r < kMaxMoves / 64; ++r) {
    const int i = r * 64 + lane;
    if (i < n)
      priors[start + i] = uniform ? scale : e[i] * scale;
  }
}

}  // namespace

hipError_t LaunchPolicyPriors(const float *policy, const std::int32_t *offsets,
                              const std::int16_t *indices, int batch, float inv_temp,
                              float *priors, hipStream_t stream, std::string *err) {
  if (batch <= 0 || !policy || !offsets || !indices || !priors) {
    if (err)
      *err = "policy_priors: needs batch > 0 and non-null buffers";
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(PolicyPriorsKernel, dim3(batch), dim3(64), 0, stream, policy, offsets,
                     indices, inv_temp, priors);
  return hipGetLastError();
}

hipError_t LaunchPolicyMap(const std::uint16_t *qk, const std::uint16_t *qk_lo, int batch,
                           int dp, const float *promo, const std::int16_t *gather,
                           float *policy, hipStream_t stream, std::string *err) {
  if (batch <= 0 || batch > 65535 || dp <= 0 || dp % 32 || !qk || !promo || !gather || !policy ||
      (reinterpret_cast<std::uintptr_t>(qk) & 15u) ||
      (qk_lo && (reinterpret_cast<std::uintptr_t>(qk_lo) & 15u))) {
    if (err)
      *err = "policy_map: needs 0 < batch <= 65535, Dp % 32 == 0 and 16-byte aligned Q|K";
    return hipErrorInvalidValue;
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(dp));
  // Four workgroups per position while they fit on the CUs at once (up to
  // 64 positions: batch 1 1.179 -> 1.150 ms, batch 32 +1.1 %), one above
  // (four at batch 256 were 0.4 % slower: K read by every workgroup).
  const bool four = batch <= 64;
  const dim3 grid(four ? 4 : 1, batch);
  if (qk_lo && four)
    hipLaunchKernelGGL((PolicyMapKernel<true, 4>), grid, dim3(1024), 0, stream, qk, qk_lo, dp,
                       scale, promo, gather, policy);
  else if (qk_lo)
    hipLaunchKernelGGL((PolicyMapKernel<true, 1>), grid, dim3(1024), 0, stream, qk, qk_lo, dp,
                       scale, promo, gather, policy);
  else if (four)
    hipLaunchKernelGGL((PolicyMapKernel<false, 4>), grid, dim3(1024), 0, stream, qk, qk_lo, dp,
                       scale, promo, gather, policy);
  else
    hipLaunchKernelGGL((PolicyMapKernel<false, 1>), grid, dim3(1024), 0, stream, qk, qk_lo, dp,
                       scale, promo, gather, policy);
  return hipGetLastError();
}

}  // namespace mfh

// Fused 64-token multi-head attention for gfx950 (head depth 32):
//   ctx_h = softmax(Q_h K_h^T / sqrt(32) + bias_h) V_h
// restating reference src/nn/cpu/cpu_network.cpp:1175-1254.
//
// One wave owns one (position, head); a workgroup holds 4 heads of one
// position.  S = Q K^T is 16 v_mfma_f32_16x16x32_bf16 (the K dimension of the
// MFMA is exactly the head depth); the softmax runs on the accumulator layout
// with 16-lane shuffles; P (bf16) and V^T are staged in LDS and O = P V is 16
// more MFMAs.  Scores, softmax statistics and accumulation stay in fp32.
//
// Split precision: Q, K, V and the context arrive/leave as hi + lo bf16
// planes, P is staged as hi + lo, and each product takes three MFMAs
// (hi.hi + hi.lo + lo.hi; the lo.lo term is below fp32 resolution).
#include "mfh_device.h"
#include "mfh_kernels.h"

#include <mutex>

namespace mfh {
namespace {

constexpr int kSq = 64;
constexpr int kDepth = 32;
constexpr int kHeadsPerBlock = 4;

// 64-column bf16 tiles in LDS: 8 chunks of 16 bytes per row, chunk index
// XOR-swizzled by row for conflict-free ds_read_b128 fragment loads.
__device__ __forceinline__ int Swz(int row, int col) {
  return row * 64 + ((((col >> 3) ^ (row & 7))) << 3) + (col & 7);
}

__device__ __forceinline__ f32x4 Mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <bool SPLIT, bool BIAS_F32>
__global__ __launch_bounds__(256) void AttentionKernel(AttentionParams ap) {
  constexpr int PLANES = SPLIT ? 2 : 1;
  // Dynamic LDS: P planes [4][PLANES][64*64] then V^T planes [4][PLANES][32*64].
  extern __shared__ __attribute__((aligned(16))) std::uint16_t smem[];
  typedef std::uint16_t PTile[PLANES][kSq * kSq];
  typedef std::uint16_t VTile[PLANES][kDepth * kSq];
  PTile *p_lds = reinterpret_cast<PTile *>(smem);
  VTile *vt_lds = reinterpret_cast<VTile *>(smem + kHeadsPerBlock * PLANES * kSq * kSq);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int heads = ap.heads;
  const int groups = heads / kHeadsPerBlock;
  const int b = blockIdx.x / groups;
  const int h = (blockIdx.x % groups) * kHeadsPerBlock + wave;
  const int E = heads * kDepth;
  const size_t ld = static_cast<size_t>(3) * E;
  const size_t pos = static_cast<size_t>(b) * kSq * ld;
  const int qcol = h * kDepth, kcol = E + h * kDepth, vcol = 2 * E + h * kDepth;

  // V^T into LDS: each lane moves 4 chunks of 8 depths for one key.
#pragma unroll
  for (int pl = 0; pl < PLANES; ++pl) {
    const std::uint16_t *base = (pl ? ap.qkv_lo : ap.qkv) + pos;
    std::uint16_t *vt = vt_lds[wave][pl];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane + i * 64;  // 256 chunks = 64 keys x 4 chunks
      const int key = c >> 2, d0 = (c & 3) * 8;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(base + key * ld + vcol + d0);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vt[Swz(d0 + e, key)] = static_cast<std::uint16_t>(v[e >> 1] >> ((e & 1) * 16));
    }
  }

  // S = Q K^T.
  const int fr = lane & 15, fc = (lane >> 4) * 8;
  const std::uint16_t *qh = ap.qkv + pos;
  bf16x8 qa[4], kb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qa[i] = *reinterpret_cast<const bf16x8 *>(qh + (i * 16 + fr) * ld + qcol + fc);
    kb[i] = *reinterpret_cast<const bf16x8 *>(qh + (i * 16 + fr) * ld + kcol + fc);
  }
  f32x4 s[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      s[i][j] = Mfma(qa[i], kb[j], f32x4{0.f, 0.f, 0.f, 0.f});
  if constexpr (SPLIT) {
    const std::uint16_t *ql = ap.qkv_lo + pos;
    bf16x8 qlo[4], klo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qlo[i] = *reinterpret_cast<const bf16x8 *>(ql + (i * 16 + fr) * ld + qcol + fc);
      klo[i] = *reinterpret_cast<const bf16x8 *>(ql + (i * 16 + fr) * ld + kcol + fc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s[i][j] = Mfma(qlo[i], kb[j], Mfma(qa[i], klo[j], s[i][j]));
  }

  // Scale, add the smolgen bias, softmax over keys.  Lane holds rows
  // q = 16 i + 4 (lane / 16) + r, key = 16 j + lane % 16.
  const float scale = 0.17677669529663687f;  // 1 / sqrt(32)
  const size_t bias_off = (static_cast<size_t>(b) * heads + h) * kSq * kSq;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = i * 16 + (lane >> 4) * 4 + r;
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = s[i][j][r] * scale;
        if (ap.bias) {
          const int bi = q * kSq + j * 16 + fr;
          if constexpr (BIAS_F32)
            v[j] += static_cast<const float *>(ap.bias)[bias_off + bi];
          else
            v[j] += bf16_to_f32(static_cast<const std::uint16_t *>(ap.bias)[bias_off + bi]);
        }
      }
      float m = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
      for (int o = 1; o < 16; o <<= 1)
        m = fmaxf(m, __shfl_xor(m, o, 64));
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = __expf(v[j] - m);
        sum += v[j];
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1)
        sum += __shfl_xor(sum, o, 64);
      const float inv = 1.f / sum;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p = v[j] * inv;
        const std::uint16_t hi = f32_to_bf16(p);
        p_lds[wave][0][Swz(q, j * 16 + fr)] = hi;
        if constexpr (SPLIT)
          p_lds[wave][PLANES - 1][Swz(q, j * 16 + fr)] = f32_to_bf16(p - bf16_to_f32(hi));
      }
    }
  __syncthreads();

  // O = P V: M = 64 queries, N = 32 depths, K = 64 keys.
  f32x4 o[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      o[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    bf16x8 pa[4], vb[2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pa[i] = *reinterpret_cast<const bf16x8 *>(&p_lds[wave][0][Swz(i * 16 + fr, kk * 32 + fc)]);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      vb[j] = *reinterpret_cast<const bf16x8 *>(&vt_lds[wave][0][Swz(j * 16 + fr, kk * 32 + fc)]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        o[i][j] = Mfma(pa[i], vb[j], o[i][j]);
    if constexpr (SPLIT) {
      bf16x8 pl[4], vl[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pl[i] = *reinterpret_cast<const bf16x8 *>(&p_lds[wave][1][Swz(i * 16 + fr, kk * 32 + fc)]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        vl[j] = *reinterpret_cast<const bf16x8 *>(&vt_lds[wave][1][Swz(j * 16 + fr, kk * 32 + fc)]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          o[i][j] = Mfma(pl[i], vb[j], Mfma(pa[i], vl[j], o[i][j]));
    }
  }
  const size_t out_off = static_cast<size_t>(b) * kSq * E + h * kDepth;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = i * 16 + (lane >> 4) * 4 + r;
        const size_t idx = out_off + static_cast<size_t>(q) * E + j * 16 + fr;
        const std::uint16_t hi = f32_to_bf16(o[i][j][r]);
        ap.ctx[idx] = hi;
        if constexpr (SPLIT)
          ap.ctx_lo[idx] = f32_to_bf16(o[i][j][r] - bf16_to_f32(hi));
      }
}

template <bool SPLIT, bool BIAS_F32>
hipError_t Launch(const AttentionParams &ap, int grid, hipStream_t stream) {
  constexpr int PLANES = SPLIT ? 2 : 1;
  constexpr int kLds = kHeadsPerBlock * PLANES * (kSq * kSq + kDepth * kSq) * 2;
  auto kernel = AttentionKernel<SPLIT, BIAS_F32>;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&]() {
    attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  });
  if (attr != hipSuccess)
    return attr;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), kLds, stream, ap);
  return hipGetLastError();
}

}  // namespace

hipError_t LaunchAttention(const AttentionParams &ap, hipStream_t stream, std::string *err) {
  const bool split = ap.qkv_lo != nullptr;
  if (ap.batch <= 0 || ap.heads <= 0 || ap.heads % kHeadsPerBlock || !ap.qkv || !ap.ctx ||
      (reinterpret_cast<std::uintptr_t>(ap.qkv) & 15u) ||
      (split && (!ap.ctx_lo || (reinterpret_cast<std::uintptr_t>(ap.qkv_lo) & 15u)))) {
    if (err)
      *err = "attention: needs batch > 0, heads % 4 == 0, 16-byte aligned qkv, and "
             "lo planes for both input and output in split mode";
    return hipErrorInvalidValue;
  }
  const int grid = ap.batch * (ap.heads / kHeadsPerBlock);
  if (split) {
    if (ap.bias_f32)
      return Launch<true, true>(ap, grid, stream);
    return Launch<true, false>(ap, grid, stream);
  }
  if (ap.bias_f32)
    return Launch<false, true>(ap, grid, stream);
  return Launch<false, false>(ap, grid, stream);
}

}  // namespace mfh

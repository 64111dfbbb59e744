// Fused 64-token multi-head attention for gfx950 (head depth 32):
//   ctx_h = softmax(Q_h K_h^T / sqrt(32) + bias_h) V_h
// restating reference src/nn/cpu/cpu_network.cpp:1175-1254.
//
// One wave owns one (position, head); a workgroup holds 4 heads of one
// position.  S = Q K^T is 16 v_mfma_f32_16x16x32_bf16 (the K dimension of the
// MFMA is exactly the head depth); the softmax runs on the accumulator layout
// with 16-lane shuffles; P (bf16) and V^T are staged in LDS and O = P V is 16
// more MFMAs.  Scores, softmax statistics and accumulation stay in fp32.
#include "mfh_device.h"
#include "mfh_kernels.h"

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

__global__ __launch_bounds__(256) void AttentionKernel(
    const std::uint16_t *__restrict__ qkv, const std::uint16_t *__restrict__ bias,
    int heads, std::uint16_t *__restrict__ ctx) {
  __shared__ __attribute__((aligned(16))) std::uint16_t p_lds[kHeadsPerBlock][kSq * kSq];
  __shared__ __attribute__((aligned(16))) std::uint16_t vt_lds[kHeadsPerBlock][kDepth * kSq];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int groups = heads / kHeadsPerBlock;
  const int b = blockIdx.x / groups;
  const int h = (blockIdx.x % groups) * kHeadsPerBlock + wave;
  const int E = heads * kDepth;
  const size_t ld = static_cast<size_t>(3) * E;
  const std::uint16_t *base = qkv + static_cast<size_t>(b) * kSq * ld;
  const int qcol = h * kDepth, kcol = E + h * kDepth, vcol = 2 * E + h * kDepth;

  // V^T into LDS: each lane moves 4 chunks of 8 depths for one key.
  std::uint16_t *vt = vt_lds[wave];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane + i * 64;  // 256 chunks = 64 keys x 4 chunks
    const int key = c >> 2, d0 = (c & 3) * 8;
    const uint4 v = *reinterpret_cast<const uint4 *>(base + key * ld + vcol + d0);
    const std::uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      vt[Swz(d0 + e, key)] = static_cast<std::uint16_t>(w[e >> 1] >> ((e & 1) * 16));
  }

  // S = Q K^T.
  const int fr = lane & 15, fc = (lane >> 4) * 8;
  bf16x8 qa[4], kb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qa[i] = *reinterpret_cast<const bf16x8 *>(base + (i * 16 + fr) * ld + qcol + fc);
    kb[i] = *reinterpret_cast<const bf16x8 *>(base + (i * 16 + fr) * ld + kcol + fc);
  }
  f32x4 s[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      s[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i], kb[j],
                                                        f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);

  // Scale, add the smolgen bias, softmax over keys.  Lane holds rows
  // q = 16 i + 4 (lane / 16) + r, key = 16 j + lane % 16.
  const float scale = 0.17677669529663687f;  // 1 / sqrt(32)
  const std::uint16_t *bh =
      bias ? bias + (static_cast<size_t>(b) * heads + h) * kSq * kSq : nullptr;
  std::uint16_t *pl = p_lds[wave];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = i * 16 + (lane >> 4) * 4 + r;
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = s[i][j][r] * scale;
        if (bh)
          v[j] += bf16_to_f32(bh[q * kSq + j * 16 + fr]);
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
      for (int j = 0; j < 4; ++j)
        pl[Swz(q, j * 16 + fr)] = f32_to_bf16(v[j] * inv);
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
      pa[i] = *reinterpret_cast<const bf16x8 *>(&pl[Swz(i * 16 + fr, kk * 32 + fc)]);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      vb[j] = *reinterpret_cast<const bf16x8 *>(&vt[Swz(j * 16 + fr, kk * 32 + fc)]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        o[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[i], vb[j], o[i][j], 0, 0, 0);
  }
  std::uint16_t *out = ctx + static_cast<size_t>(b) * kSq * E + h * kDepth;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int q = i * 16 + (lane >> 4) * 4 + r;
        out[static_cast<size_t>(q) * E + j * 16 + fr] = f32_to_bf16(o[i][j][r]);
      }
}

}  // namespace

hipError_t LaunchAttention(const std::uint16_t *qkv, const std::uint16_t *bias, int batch,
                           int heads, std::uint16_t *ctx, hipStream_t stream,
                           std::string *err) {
  if (batch <= 0 || heads <= 0 || heads % kHeadsPerBlock || !qkv || !ctx ||
      (reinterpret_cast<std::uintptr_t>(qkv) & 15u)) {
    if (err)
      *err = "attention: needs batch > 0, heads % 4 == 0 and 16-byte aligned qkv";
    return hipErrorInvalidValue;
  }
  const int grid = batch * (heads / kHeadsPerBlock);
  hipLaunchKernelGGL(AttentionKernel, dim3(grid), dim3(256), 0, stream, qkv, bias, heads,
                     ctx);
  return hipGetLastError();
}

}  // namespace mfh

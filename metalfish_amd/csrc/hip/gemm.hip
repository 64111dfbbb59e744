// bf16 MFMA GEMM for gfx950 with fused bias / activation / residual
// epilogues: the dense layers of the transformer body and heads
// (reference src/nn/cpu/cpu_network.cpp:822-890, 1057-1062, 1256-1259,
// 1318-1397).
//
// C[M,N] = A[M,K] . W[N,K]^T.  Both operands are K-contiguous (activations
// row-major, weights in the reference's [out][in] layout), so every lane
// fetches 16-byte chunks along K for both.  A workgroup of 4 waves owns a
// BM x BN tile; each wave owns a (BM/2) x (BN/2) sub-tile built from
// v_mfma_f32_16x16x32_bf16 instructions.  K advances in 64-wide steps through
// a double-buffered LDS stage whose 16-byte chunks are XOR-swizzled by row so
// the ds_read_b128 fragment reads are bank-conflict free.
#include "mfh_device.h"
#include "mfh_kernels.h"

namespace mfh {
namespace {

constexpr int kBK = 64;
constexpr int kThreads = 256;

__device__ __forceinline__ int SwizzledOffset(int row, int chunk) {
  return row * kBK + ((chunk ^ (row & 7)) << 3);
}

__device__ __forceinline__ void StoreOut(const GemmParams &p, int row, int col,
                                         float v) {
  if (p.out_mode == GEMM_OUT_RESID_F32) {
    const float r = p.resid[static_cast<size_t>(row) * p.ldr + col];
    static_cast<float *>(p.C)[static_cast<size_t>(row) * p.ldc + col] =
        r + p.alpha * v;
    return;
  }
  v = activate(v, p.act);
  void *base = p.C;
  int ld = p.ldc;
  int c = col;
  if (col >= p.split_n) {
    base = p.C2;
    ld = p.ldc2;
    c = col - p.split_n;
  }
  if (p.out_mode == GEMM_OUT_F32)
    static_cast<float *>(base)[static_cast<size_t>(row) * ld + c] = v;
  else
    static_cast<std::uint16_t *>(base)[static_cast<size_t>(row) * ld + c] =
        f32_to_bf16(v);
}

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void GemmBf16Kernel(GemmParams p) {
  constexpr int WTM = BM / 2, WTN = BN / 2;  // wave tile (2 x 2 waves)
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int A_PER_T = BM * kBK / 8 / kThreads;  // 16-byte chunks
  constexpr int B_PER_T = BN * kBK / 8 / kThreads;
  static_assert(A_PER_T >= 1 && B_PER_T >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) std::uint16_t lds[2][(BM + BN) * kBK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int nbm = (p.M + BM - 1) / BM;
  const int nbn = (p.N + BN - 1) / BN;
  const int nb = nbm * nbn;
  // Consecutive workgroup ids land on different XCDs (round robin over 8);
  // remap so each XCD works on a contiguous range of tiles, then walk the
  // range in groups of 8 M-tiles to keep the shared A/W panels in its L2.
  int bid = blockIdx.x;
  if ((nb & 7) == 0)
    bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  constexpr int kGroupM = 8;
  const int group = bid / (kGroupM * nbn);
  const int first_m = group * kGroupM;
  const int group_m = min(nbm - first_m, kGroupM);
  const int bm = first_m + (bid % (kGroupM * nbn)) % group_m;
  const int bn = (bid % (kGroupM * nbn)) / group_m;
  const int m0 = bm * BM, n0 = bn * BN;

  u32x4 ra[A_PER_T], rb[B_PER_T];
  const std::uint16_t *a_rows[A_PER_T];
  const std::uint16_t *w_rows[B_PER_T];
  int a_lds[A_PER_T], w_lds[B_PER_T];
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i) {
    const int c = tid + i * kThreads;
    // Rows past M read a clamped valid row: they only feed output rows that
    // are never stored, so no zeroing (and no select) is needed.
    const int gr = min(m0 + (c >> 3), p.M - 1);
    a_rows[i] = p.A + static_cast<size_t>(gr) * p.lda + (c & 7) * 8;
    a_lds[i] = SwizzledOffset(c >> 3, c & 7);
  }
#pragma unroll
  for (int i = 0; i < B_PER_T; ++i) {
    const int c = tid + i * kThreads;
    const int gr = min(n0 + (c >> 3), p.N - 1);  // columns past N are never stored
    w_rows[i] = p.W + static_cast<size_t>(gr) * p.ldw + (c & 7) * 8;
    w_lds[i] = BM * kBK + SwizzledOffset(c >> 3, c & 7);
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = p.K / kBK;
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i)
    ra[i] = *reinterpret_cast<const u32x4 *>(a_rows[i]);
#pragma unroll
  for (int i = 0; i < B_PER_T; ++i)
    rb[i] = *reinterpret_cast<const u32x4 *>(w_rows[i]);
#pragma unroll
  for (int i = 0; i < A_PER_T; ++i)
    *reinterpret_cast<u32x4 *>(&lds[0][a_lds[i]]) = ra[i];
#pragma unroll
  for (int i = 0; i < B_PER_T; ++i)
    *reinterpret_cast<u32x4 *>(&lds[0][w_lds[i]]) = rb[i];
  __syncthreads();

  const int frag_row = lane & 15;
  const int frag_chunk = lane >> 4;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) {
      const int k0 = (kt + 1) * kBK;
#pragma unroll
      for (int i = 0; i < A_PER_T; ++i)
        ra[i] = *reinterpret_cast<const u32x4 *>(a_rows[i] + k0);
#pragma unroll
      for (int i = 0; i < B_PER_T; ++i)
        rb[i] = *reinterpret_cast<const u32x4 *>(w_rows[i] + k0);
    }
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      bf16x8 af[TM], bw[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8 *>(&lds[cur][SwizzledOffset(
            wm * WTM + i * 16 + frag_row, kk * 4 + frag_chunk)]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bw[j] = *reinterpret_cast<const bf16x8 *>(&lds[cur][BM * kBK + SwizzledOffset(
            wn * WTN + j * 16 + frag_row, kk * 4 + frag_chunk)]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bw[j],
                                                              acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) {
#pragma unroll
      for (int i = 0; i < A_PER_T; ++i)
        *reinterpret_cast<u32x4 *>(&lds[cur ^ 1][a_lds[i]]) = ra[i];
#pragma unroll
      for (int i = 0; i < B_PER_T; ++i)
        *reinterpret_cast<u32x4 *>(&lds[cur ^ 1][w_lds[i]]) = rb[i];
    }
    __syncthreads();
  }

  // Accumulator layout of the 16x16 MFMA: lane holds rows 4*(lane/16)+r,
  // column lane%16 of its tile.
  const int row_base = m0 + wm * WTM + (lane >> 4) * 4;
  const int col_base = n0 + wn * WTN + (lane & 15);
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = col_base + j * 16;
    if (col >= p.N)
      continue;
    const float b = p.bias ? p.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row_base + i * 16 + r;
        if (row < p.M)
          StoreOut(p, row, col, acc[i][j][r] + b);
      }
  }
}

bool Aligned16(const void *ptr) {
  return (reinterpret_cast<std::uintptr_t>(ptr) & 15u) == 0;
}

}  // namespace

hipError_t LaunchGemm(const GemmParams &p, hipStream_t stream, std::string *err) {
  auto fail = [&](const char *why) {
    if (err)
      *err = std::string("gemm: ") + why;
    return hipErrorInvalidValue;
  };
  if (p.M <= 0 || p.N <= 0 || p.K <= 0)
    return fail("non-positive shape");
  if (p.K % kBK)
    return fail("K must be a multiple of 64");
  if (!p.A || !p.W || !p.C)
    return fail("null operand");
  if (!Aligned16(p.A) || !Aligned16(p.W) || p.lda % 8 || p.ldw % 8 ||
      p.lda < p.K || p.ldw < p.K)
    return fail("operands must be 16-byte aligned with ld >= K, ld % 8 == 0");
  if (p.out_mode == GEMM_OUT_RESID_F32 && (!p.resid || p.split_n < p.N))
    return fail("residual mode needs resid and no split");
  if (p.split_n < p.N && (!p.C2 || p.ldc2 < p.N - p.split_n))
    return fail("split output needs C2 wide enough");
  if (p.ldc < (p.split_n < p.N ? p.split_n : p.N))
    return fail("ldc too small");
  const bool large = p.M >= 2048 && p.N >= 128;
  if (large) {
    const int grid = ((p.M + 127) / 128) * ((p.N + 127) / 128);
    hipLaunchKernelGGL((GemmBf16Kernel<128, 128>), dim3(grid), dim3(kThreads), 0,
                       stream, p);
  } else {
    const int grid = ((p.M + 63) / 64) * ((p.N + 63) / 64);
    hipLaunchKernelGGL((GemmBf16Kernel<64, 64>), dim3(grid), dim3(kThreads), 0,
                       stream, p);
  }
  return hipGetLastError();
}

}  // namespace mfh

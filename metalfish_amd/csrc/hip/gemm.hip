// bf16 MFMA GEMM for gfx950 with fused bias / activation / residual
// epilogues: the dense layers of the transformer body and heads
// (reference src/nn/cpu/cpu_network.cpp:822-890, 1057-1062, 1256-1259,
// 1318-1397).
//
// C[M,N] = A[M,K] . W[N,K]^T.  Both operands are K-contiguous (activations
// row-major, weights in the reference's [out][in] layout).  A workgroup of
// WM x WN waves owns a BM x BN tile; each wave owns a (BM/WM) x (BN/WN)
// sub-tile of v_mfma_f32_16x16x32_bf16 instructions.  K advances in 64-wide
// steps through a two-stage LDS ring filled by global_load_lds_dwordx4
// (direct global->LDS, no VGPR round trip): the next step's tiles are in
// flight while the current one feeds the MFMAs.  LDS rows are 128 bytes with
// their 16-byte chunks XOR-swizzled by (row & 7), which keeps the
// ds_read_b128 fragment reads free of bank conflicts; the swizzle is applied
// on the global side (each lane fetches the chunk that belongs in its LDS
// slot).
//
// Split precision: when A_lo is set, the activation is carried as
// hi + lo bf16 planes (lo = bf16(x - hi)) and every fragment pair issues two
// MFMAs, giving ~16-bit activation precision against exact bf16 weights.
#include "mfh_device.h"
#include "mfh_kernels.h"

#include <mutex>

namespace mfh {
namespace {

constexpr int kBK = 64;
#define MFH_LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

__device__ __forceinline__ int Swz(int row, int chunk) {
  return row * kBK + ((chunk ^ (row & 7)) << 3);
}

// Activation with a compile-time kind; ACT_RUNTIME defers to p.act.
constexpr int ACT_RUNTIME = -2;
template <int ACT>
__device__ __forceinline__ float Act(float v, int runtime_act) {
  if constexpr (ACT == ACT_RUNTIME)
    return activate(v, runtime_act);
  else
    return activate(v, ACT);
}

template <int BM, int BN, int WM, int WN, bool SPLIT, int MODE, int ACT>
__global__ __launch_bounds__(WM *WN * 64) void GemmKernel(GemmParams p) {
  constexpr int NWAVES = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int A_ROWS = SPLIT ? 2 * BM : BM;     // hi rows then lo rows
  constexpr int STAGE = (A_ROWS + BN) * kBK;      // bf16 elements per stage
  constexpr int LOADS = (A_ROWS + BN) * kBK * 2 / 1024;  // 1 KiB wave-loads
  static_assert(LOADS % NWAVES == 0, "stage loads must split evenly over waves");
  constexpr int LPW = LOADS / NWAVES;
  extern __shared__ __attribute__((aligned(1024))) std::uint16_t lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int nbm = (p.M + BM - 1) / BM;
  const int nbn = (p.N + BN - 1) / BN;
  const int nb = nbm * nbn;
  // Consecutive workgroup ids go round-robin over the 8 XCDs; remap so each
  // XCD owns a contiguous range of tiles, walked in groups of 8 M-tiles so
  // the A and W panels a group shares stay in that XCD's L2.
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
  // Split-K: slice blockIdx.y covers K range [ks * kslice, (ks + 1) * kslice)
  // and writes its fp32 partial tile to C + ks * M * ldc.
  const int kslice = p.K / p.k_splits;
  const int k_begin = blockIdx.y * kslice;

  // Each lane's source pointer for its LPW wave-loads.  A wave-load fills
  // 1 KiB = 8 rows x 128 B of LDS; lane l lands in row l/8, physical chunk
  // l%8, so it fetches logical chunk (l%8) ^ (row & 7).  Rows past M or N
  // read a clamped valid row: they only feed outputs that are never stored.
  const std::uint16_t *src[LPW];
  int dst[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int L = wave * LPW + j;
    const int row = L * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ (row & 7);
    if (row < BM) {
      src[j] = p.A + static_cast<size_t>(min(m0 + row, p.M - 1)) * p.lda + k_begin + chunk * 8;
    } else if (SPLIT && row < 2 * BM) {
      src[j] = p.A_lo + static_cast<size_t>(min(m0 + row - BM, p.M - 1)) * p.lda + k_begin +
               chunk * 8;
    } else {
      src[j] = p.W + static_cast<size_t>(min(n0 + row - A_ROWS, p.N - 1)) * p.ldw + k_begin +
               chunk * 8;
    }
    dst[j] = L * 512;
  }

  const int KT = kslice / kBK;
  // Stage 0 in flight before the loop.
#pragma unroll
  for (int j = 0; j < LPW; ++j)
    __builtin_amdgcn_global_load_lds(static_cast<const void *>(src[j]),
                                     MFH_LDS_PTR(lds + dst[j]), 16, 0, 0);

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, fc = lane >> 4;
  for (int kt = 0; kt < KT; ++kt) {
    // This wave's loads for step kt are done; the barrier makes every
    // wave's loads visible and guarantees the other stage is no longer read.
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("s_barrier" ::: "memory");
    if (kt + 1 < KT) {
      std::uint16_t *next = lds + ((kt + 1) & 1) * STAGE;
#pragma unroll
      for (int j = 0; j < LPW; ++j)
        __builtin_amdgcn_global_load_lds(static_cast<const void *>(src[j] + (kt + 1) * kBK),
                                         MFH_LDS_PTR(next + dst[j]), 16, 0, 0);
    }
    const std::uint16_t *sa = lds + (kt & 1) * STAGE;
    const std::uint16_t *sw = sa + A_ROWS * kBK;
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      bf16x8 af[TM], bw[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8 *>(sa + Swz(wm * WTM + i * 16 + fr, kk * 4 + fc));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bw[j] = *reinterpret_cast<const bf16x8 *>(sw + Swz(wn * WTN + j * 16 + fr, kk * 4 + fc));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bw[j], acc[i][j], 0, 0, 0);
      if constexpr (SPLIT) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const bf16x8 *>(
              sa + Swz(BM + wm * WTM + i * 16 + fr, kk * 4 + fc));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bw[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // Accumulator layout of the 16x16 MFMA: lane holds rows 4*(lane/16)+r,
  // column lane%16 of its tile.
  const int row_base = m0 + wm * WTM + (lane >> 4) * 4;
  const int col_base = n0 + wn * WTN + (lane & 15);
  if (p.k_splits > 1) {
    float *part = static_cast<float *>(p.C) + static_cast<size_t>(blockIdx.y) * p.M * p.ldc;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = col_base + j * 16;
      if (col >= p.N)
        continue;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row_base + i * 16 + r;
          if (row < p.M)
            part[static_cast<size_t>(row) * p.ldc + col] = acc[i][j][r];
        }
    }
    return;
  }
  // Epilogue, specialised at compile time on the output mode and activation;
  // the split-column target and the residual plane are resolved per column.
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = col_base + j * 16;
    if (col >= p.N)
      continue;
    const float b = p.bias ? p.bias[col] : 0.f;
    if constexpr (MODE == GEMM_OUT_RESID_F32) {
      float *c = static_cast<float *>(p.C) + col;
      const float *res = p.resid + col;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row_base + i * 16 + r;
          if (row < p.M)
            c[static_cast<size_t>(row) * p.ldc] =
                res[static_cast<size_t>(row) * p.ldr] + p.alpha * (acc[i][j][r] + b);
        }
    } else {
      const bool second = col >= p.split_n;
      const int cc = second ? col - p.split_n : col;
      const int ld = second ? p.ldc2 : p.ldc;
      if constexpr (MODE == GEMM_OUT_F32) {
        float *c = static_cast<float *>(second ? p.C2 : p.C) + cc;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = row_base + i * 16 + r;
            if (row < p.M)
              c[static_cast<size_t>(row) * ld] = Act<ACT>(acc[i][j][r] + b, p.act);
          }
      } else {
        std::uint16_t *c = static_cast<std::uint16_t *>(second ? p.C2 : p.C) + cc;
        std::uint16_t *c_lo = static_cast<std::uint16_t *>(second ? p.C2_lo : p.C_lo);
        if (c_lo) {
          c_lo += cc;
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = row_base + i * 16 + r;
              if (row < p.M) {
                const float v = Act<ACT>(acc[i][j][r] + b, p.act);
                const std::uint16_t hi = f32_to_bf16(v);
                c[static_cast<size_t>(row) * ld] = hi;
                c_lo[static_cast<size_t>(row) * ld] = f32_to_bf16(v - bf16_to_f32(hi));
              }
            }
        } else {
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = row_base + i * 16 + r;
              if (row < p.M)
                c[static_cast<size_t>(row) * ld] = f32_to_bf16(Act<ACT>(acc[i][j][r] + b, p.act));
            }
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, bool SPLIT, int MODE, int ACT>
hipError_t LaunchVariant(const GemmParams &p, hipStream_t stream) {
  constexpr int A_ROWS = SPLIT ? 2 * BM : BM;
  constexpr size_t kLds = 2ull * (A_ROWS + BN) * kBK * 2;
  auto kernel = GemmKernel<BM, BN, WM, WN, SPLIT, MODE, ACT>;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&]() {
    attr = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(kLds));
  });
  if (attr != hipSuccess)
    return attr;
  const int grid = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  hipLaunchKernelGGL(kernel, dim3(grid, p.k_splits), dim3(WM * WN * 64), kLds, stream, p);
  return hipGetLastError();
}

// Epilogue dispatch: the activations the network uses (none, mish) get
// dedicated instances, anything else the runtime switch.
template <int BM, int BN, int WM, int WN, bool SPLIT>
hipError_t Launch(const GemmParams &p, hipStream_t stream) {
  if (p.k_splits > 1 || (p.out_mode == GEMM_OUT_F32 && p.act == ACT_NONE))
    return LaunchVariant<BM, BN, WM, WN, SPLIT, GEMM_OUT_F32, ACT_NONE>(p, stream);
  if (p.out_mode == GEMM_OUT_RESID_F32)
    return LaunchVariant<BM, BN, WM, WN, SPLIT, GEMM_OUT_RESID_F32, ACT_NONE>(p, stream);
  if (p.out_mode == GEMM_OUT_F32)
    return p.act == ACT_MISH
               ? LaunchVariant<BM, BN, WM, WN, SPLIT, GEMM_OUT_F32, ACT_MISH>(p, stream)
               : LaunchVariant<BM, BN, WM, WN, SPLIT, GEMM_OUT_F32, ACT_RUNTIME>(p, stream);
  if (p.act == ACT_NONE)
    return LaunchVariant<BM, BN, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_NONE>(p, stream);
  if (p.act == ACT_MISH)
    return LaunchVariant<BM, BN, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_MISH>(p, stream);
  return LaunchVariant<BM, BN, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_RUNTIME>(p, stream);
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
  if (p.k_splits < 1 || p.K % (p.k_splits * kBK))
    return fail("K must split into multiples of 64");
  if (p.k_splits > 1 && (p.out_mode != GEMM_OUT_F32 || p.bias || p.act != ACT_NONE ||
                         p.split_n < p.N))
    return fail("split-K writes raw fp32 partials only (no bias, activation or split)");
  if (!p.A || !p.W || !p.C)
    return fail("null operand");
  if (!Aligned16(p.A) || !Aligned16(p.W) || (p.A_lo && !Aligned16(p.A_lo)) || p.lda % 8 ||
      p.ldw % 8 || p.lda < p.K || p.ldw < p.K)
    return fail("operands must be 16-byte aligned with ld >= K, ld % 8 == 0");
  if (p.out_mode == GEMM_OUT_RESID_F32 && (!p.resid || p.split_n < p.N))
    return fail("residual mode needs resid and no split");
  if (p.split_n < p.N && (!p.C2 || p.ldc2 < p.N - p.split_n))
    return fail("split output needs C2 wide enough");
  if (p.split_n < p.N && (p.C_lo != nullptr) != (p.C2_lo != nullptr))
    return fail("split output needs lo planes for both parts or neither");
  if (p.ldc < (p.split_n < p.N ? p.split_n : p.N))
    return fail("ldc too small");
  const bool split = p.A_lo != nullptr;
  const bool large = p.M >= 2048 && p.N >= 128;
  if (large)
    return split ? Launch<128, 128, 2, 2, true>(p, stream)
                 : Launch<128, 128, 2, 2, false>(p, stream);
  return split ? Launch<64, 64, 2, 2, true>(p, stream) : Launch<64, 64, 2, 2, false>(p, stream);
}

}  // namespace mfh

// Row-panel bf16 MFMA GEMM for gfx950 with a fused residual + LayerNorm
// epilogue: the out-projection + ln1 and FFN2 + ln2 steps of every encoder
// layer (reference src/nn/cpu/cpu_network.cpp:1256-1259, 1318-1397 followed
// by 1399-1457), and wide bias + activation GEMMs (Q|K|V, FFN1).
//
// C[M,N] = A[M,K] . W[N,K]^T.  A workgroup of eight waves owns 64 whole
// rows of A and a panel of 128 * TN output columns; wave w owns columns
// w * 16 * TN .. + 16 * TN - 1 of the panel for all 64 rows (4 x TN
// v_mfma_f32_16x16x32_bf16 tiles, computed transposed, D = W . A^T, so a
// lane holds four consecutive columns of one row).
//
// * The 64-row activation panel (hi and lo planes in split precision) is
//   shared by all eight waves: each lane buffer-loads 16 bytes of a K step
//   two steps ahead into registers and writes them to a two-slot LDS ring
//   one step ahead, rows XOR-swizzled so a fragment read hits every bank
//   group once.  (Direct global->LDS loads would save the register hop, but
//   the compiler then waits for every outstanding load before each LDS read,
//   weight prefetches included.)
// * A weight row is used by exactly one wave, so weights skip LDS: each lane
//   buffer-loads its 16-byte (bf16) or 8-byte (e4m3) fragment piece from L2
//   into registers one K step ahead of the MFMAs.  All workgroups walk K in
//   the same order, so each XCD's L2 serves the weight panel to its 32 CUs.
// * One barrier per K step; the loop is unrolled by two so the register sets
//   alternate without copies.
// * With whole rows in one workgroup, the LayerNorm statistics need one LDS
//   exchange of per-wave row partial sums: the pre-LayerNorm rows never go
//   to HBM.
#include "mfh_device.h"
#include "mfh_kernels.h"

#include <type_traits>

namespace mfh {
namespace {

constexpr int kRows = 64;    // rows per workgroup
constexpr int kWaves = 8;    // waves per workgroup, side by side along N
constexpr int kBK = 32;      // K per step (one MFMA deep)

// Element offset of 16-byte chunk `chunk` (0..3) of 32-element LDS row
// `row`: two rows per 128 bytes, chunk XOR (row >> 1) & 3, so the 16 rows of
// a fragment read cover all eight 16-byte bank groups twice.
__device__ __forceinline__ int PanelSwz(int row, int chunk) {
  return row * kBK + ((chunk ^ ((row >> 1) & 3)) << 3);
}

template <int TN, bool SPLIT, bool W8, int MODE, int ACT>
__global__ __launch_bounds__(kWaves * 64) void PanelGemmKernel(PanelGemmParams p) {
  constexpr int TM = kRows / 16;
  constexpr int A_ROWS = SPLIT ? 2 * kRows : kRows;  // hi rows, then lo rows
  constexpr int STAGE = A_ROWS * kBK;                // bf16 elements per stage
  constexpr int A_LOADERS = A_ROWS * kBK * 2 / 16;   // lanes with a 16-B piece
  static_assert(A_LOADERS % 64 == 0 && A_LOADERS <= kWaves * 64, "panel load split");
  __shared__ __attribute__((aligned(1024))) std::uint16_t lds[2 * STAGE];
  __shared__ float red[2][kWaves][kRows];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fc = lane >> 4;
  const int m0 = blockIdx.x * kRows;
  const int n_wave = blockIdx.y * (kWaves * 16 * TN) + wave * 16 * TN;
  const int KT = p.K / kBK;

  // Activation panel: lane t = tid % A_LOADERS owns row t / 4 of the stage
  // (hi rows, then lo rows: a wave-uniform choice) and physical chunk t % 4,
  // which holds the logical chunk the swizzle maps there.  With single
  // activations the upper four waves repeat the lower four's pieces (same
  // bytes to the same LDS address), so every wave runs the same code.  Rows
  // past M read a clamped valid row; they only feed outputs never stored.
  const int t = tid % A_LOADERS;
  __amdgpu_buffer_rsrc_t arsrc;
  int avoff;
  {
    const int row = t / 4;
    const int chunk = (t % 4) ^ ((row >> 1) & 3);
    const bool lo_plane = (wave % (A_LOADERS / 64)) >= kRows * 4 / 64;
    const std::uint16_t *base = lo_plane ? p.A_lo : p.A;
    arsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<std::uint16_t *>(base), 0,
                                              0x7FFFFFFF, 0x00020000);
    avoff = (min(m0 + (row % kRows), p.M - 1) * p.lda + chunk * 8) * 2;
  }
  auto load_a = [&](int kt) {
    return __builtin_amdgcn_raw_buffer_load_b128(arsrc, avoff, min(kt, KT - 1) * kBK * 2, 0);
  };
  auto store_a = [&](int slot, u32x4 v) {
    *reinterpret_cast<u32x4 *>(lds + slot * STAGE + t * 8) = v;
  };

  // Weights: fragment j is row n_wave + 16 j + fr at K offset 8 fc of the
  // step (16 bytes of bf16, or 8 bytes of e4m3 codes).
  constexpr int WB = W8 ? 1 : 2;  // bytes per weight
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      W8 ? const_cast<std::uint8_t *>(p.W8)
         : reinterpret_cast<std::uint8_t *>(const_cast<std::uint16_t *>(p.W)),
      0, 0x7FFFFFFF, 0x00020000);
  const int wvoff = ((n_wave + fr) * p.ldw + fc * 8) * WB;
  typedef typename std::conditional<W8, u32x2, u32x4>::type WFrag;
  auto load_w = [&](int kt, WFrag (&w)[TN]) {
    const int koff = min(kt, KT - 1) * kBK * WB;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int soff = j * 16 * p.ldw * WB + koff;
      if constexpr (W8)
        w[j] = __builtin_amdgcn_raw_buffer_load_b64(wrsrc, wvoff, soff, 0);
      else
        w[j] = __builtin_amdgcn_raw_buffer_load_b128(wrsrc, wvoff, soff, 0);
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Step kt: prefetch the next step's weights into `wnext`, read stage kt
  // from slot kt % 2 and run the MFMAs on `wcur`; then write stage kt + 1
  // (loaded two steps ago into `anext`) to the other slot, start the load of
  // stage kt + 3 into `anext`, and meet at the barrier.  Past the end of K
  // the loads repeat the last step; their data is never used.
  auto step = [&](int kt, const WFrag (&wcur)[TN], WFrag (&wnext)[TN], u32x4 &anext) {
    load_w(kt + 1, wnext);
    // Keep the prefetch at the top of the step: the scheduler would
    // otherwise sink it below the MFMAs, shortening the time it has to land.
    __builtin_amdgcn_sched_barrier(0);
    const std::uint16_t *sa = lds + (kt & 1) * STAGE;
    bf16x8 af[TM], al[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      af[i] = *reinterpret_cast<const bf16x8 *>(sa + PanelSwz(i * 16 + fr, fc));
      if constexpr (SPLIT)
        al[i] = *reinterpret_cast<const bf16x8 *>(sa + PanelSwz(kRows + i * 16 + fr, fc));
    }
    // All hi-plane MFMAs, then all lo-plane ones: the two MFMAs into one
    // accumulator are TM * TN instructions apart, never back to back.
    bf16x8 bw[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (W8)
        bw[j] = Fp8x8ToBf16(wcur[j]);
      else
        bw[j] = __builtin_bit_cast(bf16x8, wcur[j]);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw[j], af[i], acc[i][j], 0, 0, 0);
    if constexpr (SPLIT) {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw[j], al[i], acc[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    store_a((kt + 1) & 1, anext);
    anext = load_a(kt + 3);
    __syncthreads();
  };

  WFrag wa[TN], wb[TN];
  u32x4 a0 = load_a(0), a1 = load_a(1);
  load_w(0, wa);
  store_a(0, a0);
  a0 = load_a(2);
  __syncthreads();
  // K % 64 == 0: whole pairs of steps.  Stage kt + 1 sits in a1 for even kt
  // and in a0 for odd kt.
  for (int kt = 0; kt < KT; kt += 2) {
    step(kt, wa, wb, a1);
    step(kt + 1, wb, wa, a0);
  }

  // Lane holds rows m0 + 16 i + fr, columns col0 + 16 j + r (r = 0..3).
  const int col0 = n_wave + fc * 4;
  float bias[TN][4];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const f32x4 b = p.bias ? *reinterpret_cast<const f32x4 *>(p.bias + col0 + j * 16)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 s = p.wscale ? *reinterpret_cast<const f32x4 *>(p.wscale + col0 + j * 16)
                             : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bias[j][r] = b[r];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        acc[i][j][r] *= s[r];
    }
  }

  if constexpr (MODE == PANEL_OUT_BF16) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + i * 16 + fr;
      if (row >= p.M)
        continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const size_t off = static_cast<size_t>(row) * p.ldc + col0 + j * 16;
        std::uint32_t hi[2], lo[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float v0 = Act<ACT>(acc[i][j][2 * h] + bias[j][2 * h], p.act);
          const float v1 = Act<ACT>(acc[i][j][2 * h + 1] + bias[j][2 * h + 1], p.act);
          split_bf16x2(v0, v1, hi[h], lo[h]);
        }
        *reinterpret_cast<u32x2 *>(p.C + off) = u32x2{hi[0], hi[1]};
        if (p.C_lo)
          *reinterpret_cast<u32x2 *>(p.C_lo + off) = u32x2{lo[0], lo[1]};
      }
    }
  } else {
    // x = resid + alpha * (acc + bias), then per-row sums over this lane's
    // 4 TN columns, the four lanes that share a row (xor 16, 32), and the
    // eight waves (fixed order through LDS).
    float s[TM], ss[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = min(m0 + i * 16 + fr, p.M - 1);
      s[i] = 0.f;
      ss[i] = 0.f;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const size_t off = static_cast<size_t>(row) * p.N + col0 + j * 16;
        float rv[4];
        if (p.resid16) {
          const u32x2 h = *reinterpret_cast<const u32x2 *>(p.resid16 + off);
          const u32x2 l = *reinterpret_cast<const u32x2 *>(p.resid16_lo + off);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const unsigned hw = h[r >> 1], lw = l[r >> 1];
            rv[r] = __uint_as_float((r & 1) ? (hw & 0xFFFF0000u) : (hw << 16)) +
                    __uint_as_float((r & 1) ? (lw & 0xFFFF0000u) : (lw << 16));
          }
        } else {
          const f32x4 x = *reinterpret_cast<const f32x4 *>(p.resid + off);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            rv[r] = x[r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = rv[r] + p.alpha * (acc[i][j][r] + bias[j][r]);
          acc[i][j][r] = v;
          s[i] += v;
          ss[i] += v * v;
        }
      }
      s[i] += __shfl_xor(s[i], 16, 64);
      ss[i] += __shfl_xor(ss[i], 16, 64);
      s[i] += __shfl_xor(s[i], 32, 64);
      ss[i] += __shfl_xor(ss[i], 32, 64);
      if (lane < 16) {
        red[0][wave][i * 16 + lane] = s[i];
        red[1][wave][i * 16 + lane] = ss[i];
      }
    }
    __syncthreads();
    float gam[TN][4], bet[TN][4];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const f32x4 g = *reinterpret_cast<const f32x4 *>(p.gamma + col0 + j * 16);
      const f32x4 b = *reinterpret_cast<const f32x4 *>(p.beta + col0 + j * 16);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        gam[j][r] = g[r];
        bet[j][r] = b[r];
      }
    }
    const float inv_n = 1.f / static_cast<float>(p.N);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float S = 0.f, SS = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        S += red[0][w][i * 16 + fr];
        SS += red[1][w][i * 16 + fr];
      }
      const int row = m0 + i * 16 + fr;
      if (row >= p.M)
        continue;
      const float mean = S * inv_n;
      float var = SS * inv_n - mean * mean;
      var = var < 0.f ? 0.f : var;
      const float inv_std = 1.f / sqrtf(var + p.eps);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const size_t off = static_cast<size_t>(row) * p.N + col0 + j * 16;
        float y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          y[r] = (acc[i][j][r] - mean) * inv_std * gam[j][r] + bet[j][r];
        std::uint32_t hi[2], lo[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          split_bf16x2(y[2 * h], y[2 * h + 1], hi[h], lo[h]);
        }
        *reinterpret_cast<u32x2 *>(p.C + off) = u32x2{hi[0], hi[1]};
        if (p.C_lo)
          *reinterpret_cast<u32x2 *>(p.C_lo + off) = u32x2{lo[0], lo[1]};
        if (p.y_f32)
          *reinterpret_cast<f32x4 *>(p.y_f32 + off) = f32x4{y[0], y[1], y[2], y[3]};
      }
    }
  }
}

template <int TN, bool SPLIT, bool W8, int MODE, int ACT>
hipError_t LaunchPanel(const PanelGemmParams &p, hipStream_t stream) {
  const dim3 grid((p.M + kRows - 1) / kRows, p.N / (kWaves * 16 * TN));
  hipLaunchKernelGGL((PanelGemmKernel<TN, SPLIT, W8, MODE, ACT>), grid, dim3(kWaves * 64), 0,
                     stream, p);
  return hipGetLastError();
}

template <int TN, bool SPLIT, bool W8>
hipError_t LaunchPanelW(const PanelGemmParams &p, hipStream_t stream) {
  if (p.out_mode == PANEL_OUT_LN)
    return LaunchPanel<TN, SPLIT, W8, PANEL_OUT_LN, ACT_NONE>(p, stream);
  if (p.act == ACT_NONE)
    return LaunchPanel<TN, SPLIT, W8, PANEL_OUT_BF16, ACT_NONE>(p, stream);
  if (p.act == ACT_MISH)
    return LaunchPanel<TN, SPLIT, W8, PANEL_OUT_BF16, ACT_MISH>(p, stream);
  return LaunchPanel<TN, SPLIT, W8, PANEL_OUT_BF16, ACT_RUNTIME>(p, stream);
}

template <int TN>
hipError_t LaunchPanelTN(const PanelGemmParams &p, hipStream_t stream) {
  const bool split = p.A_lo != nullptr;
  if (p.W8)
    return split ? LaunchPanelW<TN, true, true>(p, stream)
                 : LaunchPanelW<TN, false, true>(p, stream);
  return split ? LaunchPanelW<TN, true, false>(p, stream)
               : LaunchPanelW<TN, false, false>(p, stream);
}

// Panel width (in units of 128 columns) for a shape, or 0 if none fits.
// LayerNorm needs the whole row in one panel; bias + activation outputs take
// the widest panel that divides N.
int PanelTN(int out_mode, int N) {
  if (N <= 0 || N % 128)
    return 0;
  const int units = N / 128;
  if (out_mode == PANEL_OUT_LN)
    return (units == 2 || units == 4 || units == 6 || units == 8) ? units : 0;
  for (int tn : {8, 6, 4})
    if (units % tn == 0)
      return tn;
  return 0;
}

bool Aligned(const void *ptr, std::uintptr_t bytes) {
  return (reinterpret_cast<std::uintptr_t>(ptr) & (bytes - 1)) == 0;
}

}  // namespace

bool PanelGemmShapeOk(int out_mode, int N, int K) {
  return PanelTN(out_mode, N) != 0 && K % (2 * kBK) == 0 && K >= 4 * kBK;
}

hipError_t LaunchPanelGemm(const PanelGemmParams &p, hipStream_t stream, std::string *err) {
  auto fail = [&](const char *why) {
    if (err)
      *err = std::string("panel gemm: ") + why;
    return hipErrorInvalidValue;
  };
  if (p.M <= 0 || p.N <= 0 || p.K <= 0)
    return fail("non-positive shape");
  if (p.out_mode != PANEL_OUT_BF16 && p.out_mode != PANEL_OUT_LN)
    return fail("unknown output mode");
  if (!PanelGemmShapeOk(p.out_mode, p.N, p.K))
    return fail("N has no panel width (LayerNorm: N in {256, 512, 768, 1024}; else a "
                "multiple of 512 or 768) or K is not a multiple of 64 of at least 128");
  if (!p.A || (!p.W && !p.W8) || (p.W && p.W8) || !p.C)
    return fail("null operand (or both W and W8)");
  if (p.W8 && !p.wscale)
    return fail("fp8 weights need row scales");
  if (!Aligned(p.A, 16) || (p.A_lo && !Aligned(p.A_lo, 16)) || (p.W && !Aligned(p.W, 16)) ||
      (p.W8 && !Aligned(p.W8, 8)) || p.lda % 8 || p.ldw % 8 || p.lda < p.K || p.ldw < p.K)
    return fail("operands must be 16-byte aligned (e4m3 weights 8) with ld >= K, ld % 8 == 0");
  // Buffer loads address the operands with 32-bit byte offsets.
  if (static_cast<long long>(p.M) * p.lda * 2 >= (1ll << 31) ||
      static_cast<long long>(p.N) * p.ldw * 2 >= (1ll << 31))
    return fail("operands must be under 2 GiB");
  if ((p.bias && !Aligned(p.bias, 16)) || (p.wscale && !Aligned(p.wscale, 16)))
    return fail("bias and row scales must be 16-byte aligned");
  if (!Aligned(p.C, 8) || (p.C_lo && !Aligned(p.C_lo, 8)))
    return fail("outputs must be 8-byte aligned");
  if (p.out_mode == PANEL_OUT_BF16) {
    if (p.ldc < p.N || p.ldc % 4)
      return fail("ldc must be >= N and a multiple of 4");
  } else {
    if (p.ldc != p.N)
      return fail("LayerNorm output stride must equal N");
    if ((!p.resid && !p.resid16) || (p.resid && p.resid16) ||
        (p.resid16 != nullptr) != (p.resid16_lo != nullptr))
      return fail("LayerNorm mode needs resid (fp32) or resid16 + resid16_lo (split)");
    if ((p.resid && !Aligned(p.resid, 16)) ||
        (p.resid16 && (!Aligned(p.resid16, 8) || !Aligned(p.resid16_lo, 8))))
      return fail("residual must be 16-byte (fp32) or 8-byte (split) aligned");
    if (!p.gamma || !p.beta || !Aligned(p.gamma, 16) || !Aligned(p.beta, 16))
      return fail("LayerNorm needs 16-byte aligned gamma and beta");
    if (p.y_f32 && !Aligned(p.y_f32, 16))
      return fail("fp32 output must be 16-byte aligned");
  }
  switch (PanelTN(p.out_mode, p.N)) {
  case 2:
    return LaunchPanelTN<2>(p, stream);
  case 4:
    return LaunchPanelTN<4>(p, stream);
  case 6:
    return LaunchPanelTN<6>(p, stream);
  default:
    return LaunchPanelTN<8>(p, stream);
  }
}

}  // namespace mfh

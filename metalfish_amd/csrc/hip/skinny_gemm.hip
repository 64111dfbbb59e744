// Few-row GEMM (M <= 64 rows, one position): the single-position smolgen
// chain (reference src/nn/cpu/cpu_network.cpp:1065-1173: dense1, its
// LayerNorm, dense2, its LayerNorm, the global projection) as three
// launches instead of six, with the LayerNorm of 424-460 applied by the GEMM
// that reads the normalised rows.
//
// A workgroup of 16 waves owns 16 * NT output columns for all rows and the
// whole K: each wave takes one 16-row tile and a contiguous part of K and
// issues the loads of up to CHUNK 64-wide K blocks at once (weight and
// activation fragments straight from global memory into registers), then
// runs the MFMAs; the K parts are summed through LDS in a fixed order.
//
// The activation operand is either bf16 planes, or the LayerNorm of fp32
// rows computed on the fly: the producing GEMM writes each row's partial
// (sum, sum of squares) over its columns, the consuming GEMM's waves add
// them up in a fixed order, and every workgroup normalises the rows it reads
// (gamma / beta staged in LDS).  The kernel can also store the normalised
// rows (one workgroup per K block).
//
// Measured on MI355X at batch 1 (BT4 shape): the smolgen chain takes 24 us
// per layer this way against 29.5 us as split-K GEMMs with LayerNorm and
// reduce launches.  Running every dense layer of the encoder layer this way
// (8 launches per layer instead of 15, residual LayerNorms deferred into the
// next GEMM) was slower (1.78 vs 1.52 ms per forward): every workgroup reads
// all 64 activation rows, about 290 KB per CU for the body GEMMs.  Splitting
// K over workgroups, with the last one of a column block summing the
// partials, was slower still.
#include "mfh_device.h"
#include "mfh_kernels.h"

#include <string>

namespace mfh {
namespace {

constexpr int kSkWaves = 16;

__device__ __forceinline__ bf16x8 AsBf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

template <int NT, bool LN>
__global__ __launch_bounds__(1024) void SkinnyGemmKernel(SkinnyParams p) {
  // The K loop runs in blocks of 64: lane (r, c) of a wave loads 32
  // contiguous bytes, elements 16 c .. 16 c + 15 of the block, of its
  // activation row r and of weight row r, and feeds the two halves to two
  // MFMAs.  Both operands take the same permutation of k, so the sum is the
  // product; a wave's load then covers whole 128-byte lines of 16 rows.
  // CHUNK blocks have their loads in flight together (register budget: 128
  // VGPRs per lane at 16 waves per workgroup).
  constexpr int CHUNK = NT > 1 || LN ? 2 : 4;
  __shared__ f32x4 red[kSkWaves][NT][64];
  extern __shared__ float gb[];  // LN: gamma then beta, gb_len floats each
  const int lane = threadIdx.x & 63;
  // Wave-uniform values in scalar registers: every branch around an MFMA
  // is then a scalar branch (an MFMA runs whatever the EXEC mask holds, so
  // a block it sits in must be skipped, not masked).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fr = lane & 15, fc = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT;
  const int mt = (p.M + 15) >> 4;
  const int mtp = mt <= 1 ? 1 : mt <= 2 ? 2 : 4;  // row tiles laid out
  const int wpt = kSkWaves / mtp;                  // waves per row tile
  const int blocks = p.K >> 6;                     // 64-wide K blocks
  const int ks = wpt < blocks ? wpt : blocks;      // K parts
  const int bpw = blocks / ks;                     // K blocks per wave
  const int mtile = wave / wpt, kpart = wave % wpt;
  const bool active = mtile < mt && kpart < ks;
  const int m = mtile * 16 + fr;
  const int mrow = m < p.M ? m : p.M - 1;

  f32x4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
    acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const float *xrow = nullptr;
  int c0 = 0;
  float mean = 0.f, inv_std = 0.f;
  if constexpr (LN) {
    __shared__ float row_stat[2][kSkinnyMaxRows];
    const int gb_len = p.rows_per_src * p.K;
    for (int i = threadIdx.x; i < gb_len / 4; i += blockDim.x) {
      reinterpret_cast<f32x4 *>(gb)[i] = reinterpret_cast<const f32x4 *>(p.gamma)[i];
      reinterpret_cast<f32x4 *>(gb + gb_len)[i] = reinterpret_cast<const f32x4 *>(p.beta)[i];
    }
    // Statistics of the source rows this workgroup reads: wave w sums the
    // parts of rows w, w + 16, ...; lane l takes parts l, l + 64, ... in
    // order, then a butterfly sum over the wave (a fixed order).
    const int srcs = (p.M - 1) / p.rows_per_src + 1;
    for (int r = wave; r < srcs; r += kSkWaves) {
      float s = 0.f, ss = 0.f;
      for (int q = lane; q < p.ln_parts; q += 64) {
        const float2 v = *reinterpret_cast<const float2 *>(
            p.ln_stats + 2 * (static_cast<size_t>(q) * p.ln_rows + r));
        s += v.x;
        ss += v.y;
      }
      s = wave_sum(s);
      ss = wave_sum(ss);
      if (lane == 0) {
        const float mu = s / static_cast<float>(p.ln_width);
        float var = ss / static_cast<float>(p.ln_width) - mu * mu;
        var = var < 0.f ? 0.f : var;
        row_stat[0][r] = mu;
        row_stat[1][r] = 1.f / sqrtf(var + p.ln_eps);
      }
    }
    __syncthreads();
    const int src = mrow / p.rows_per_src;
    c0 = (mrow % p.rows_per_src) * p.K;
    xrow = p.x + static_cast<size_t>(src) * p.ldx + c0;
    mean = row_stat[0][src];
    inv_std = row_stat[1][src];
  }

  if (active) {
    const int kbeg = kpart * bpw;  // first K block of this wave
    const std::uint16_t *wrow[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = n0 + j * 16 + fr;
      wrow[j] = p.W + static_cast<size_t>(n < p.N ? n : p.N - 1) * p.ldw + fc * 16;
    }
    const std::uint16_t *arow = nullptr, *arow_lo = nullptr;
    if constexpr (!LN) {
      arow = p.a16 + static_cast<size_t>(mrow) * p.lda + fc * 16;
      if (p.a16_lo)
        arow_lo = p.a16_lo + static_cast<size_t>(mrow) * p.lda + fc * 16;
    }
    const bool has_lo = LN ? p.ln_split : p.a16_lo != nullptr;
    const bool store_rows = LN && p.y16 != nullptr && m < p.M;
    for (int c = 0; c < bpw; c += CHUNK) {
      u32x4 wv[CHUNK][NT][2];
      u32x4 av[CHUNK][2], al[CHUNK][2] = {};
      f32x4 xv[CHUNK][4];
#pragma unroll
      for (int s = 0; s < CHUNK; ++s) {
        if (c + s < bpw) {
          const int k = (kbeg + c + s) * 64;
#pragma unroll
          for (int j = 0; j < NT; ++j) {
            wv[s][j][0] = *reinterpret_cast<const u32x4 *>(wrow[j] + k);
            wv[s][j][1] = *reinterpret_cast<const u32x4 *>(wrow[j] + k + 8);
          }
          if constexpr (LN) {
            const float *xp = xrow + k + fc * 16;
#pragma unroll
            for (int q = 0; q < 4; ++q)
              xv[s][q] = *reinterpret_cast<const f32x4 *>(xp + 4 * q);
          } else {
            av[s][0] = *reinterpret_cast<const u32x4 *>(arow + k);
            av[s][1] = *reinterpret_cast<const u32x4 *>(arow + k + 8);
            if (has_lo) {
              al[s][0] = *reinterpret_cast<const u32x4 *>(arow_lo + k);
              al[s][1] = *reinterpret_cast<const u32x4 *>(arow_lo + k + 8);
            }
          }
        }
      }
#pragma unroll
      for (int s = 0; s < CHUNK; ++s) {
        if (c + s < bpw) {
          const int gblock = kbeg + c + s;
          u32x4 hv[2], lv[2];
          if constexpr (LN) {
            const int kc = c0 + gblock * 64 + fc * 16;
            const int gb_len = p.rows_per_src * p.K;
            float y[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x4 g = *reinterpret_cast<const f32x4 *>(gb + kc + 4 * q);
              const f32x4 b = *reinterpret_cast<const f32x4 *>(gb + gb_len + kc + 4 * q);
#pragma unroll
              for (int e = 0; e < 4; ++e)
                y[4 * q + e] = (xv[s][q][e] - mean) * inv_std * g[e] + b[e];
            }
            unsigned h[8], l[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const std::uint16_t ha = f32_to_bf16(y[2 * e]), hb = f32_to_bf16(y[2 * e + 1]);
              h[e] = ha | (static_cast<unsigned>(hb) << 16);
              l[e] = f32_to_bf16(y[2 * e] - bf16_to_f32(ha)) |
                     (static_cast<unsigned>(f32_to_bf16(y[2 * e + 1] - bf16_to_f32(hb))) << 16);
            }
            hv[0] = u32x4{h[0], h[1], h[2], h[3]};
            hv[1] = u32x4{h[4], h[5], h[6], h[7]};
            lv[0] = u32x4{l[0], l[1], l[2], l[3]};
            lv[1] = u32x4{l[4], l[5], l[6], l[7]};
            // One workgroup stores each K block of the normalised rows.
            if (store_rows &&
                gblock % static_cast<int>(gridDim.x) == static_cast<int>(blockIdx.x)) {
              const size_t off = static_cast<size_t>(m) * p.ldy + gblock * 64 + fc * 16;
              *reinterpret_cast<u32x4 *>(p.y16 + off) = hv[0];
              *reinterpret_cast<u32x4 *>(p.y16 + off + 8) = hv[1];
              if (p.y16_lo) {
                *reinterpret_cast<u32x4 *>(p.y16_lo + off) = lv[0];
                *reinterpret_cast<u32x4 *>(p.y16_lo + off + 8) = lv[1];
              }
              if (p.y32) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                  *reinterpret_cast<f32x4 *>(p.y32 + off + 4 * q) =
                      f32x4{y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]};
              }
            }
          } else {
            hv[0] = av[s][0];
            hv[1] = av[s][1];
            lv[0] = al[s][0];
            lv[1] = al[s][1];
          }
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
            for (int j = 0; j < NT; ++j)
              acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(AsBf16x8(wv[s][j][h2]),
                                                               AsBf16x8(hv[h2]), acc[j], 0, 0, 0);
          if (has_lo) {
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
              for (int j = 0; j < NT; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    AsBf16x8(wv[s][j][h2]), AsBf16x8(lv[h2]), acc[j], 0, 0, 0);
          }
        }
      }
    }
  }

  // Sum of the K parts, part 0 first.
  if (ks > 1) {
    if (active) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
        red[wave][j][lane] = acc[j];
    }
    __syncthreads();
    if (active && kpart == 0) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        f32x4 t = red[wave][j][lane];
        for (int kp = 1; kp < ks; ++kp)
          t += red[wave + kp][j][lane];
        acc[j] = t;
      }
    }
  }
  if (!active || kpart != 0)
    return;

  // Epilogue: lane holds rows m, columns n .. n + 3 of tile j (the MFMA
  // computes W . A^T, so D[n][m] with n = 4 * (lane / 16) + r).
  float s = 0.f, ss = 0.f;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int n = n0 + j * 16 + fc * 4;
    if (n >= p.N)
      continue;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      v[r] = acc[j][r] + (p.bias ? p.bias[n + r] : 0.f);
    if (p.out_mode == SKINNY_OUT_RESID) {
      const size_t roff = static_cast<size_t>(mrow) * p.ldr + n;
      float rv[4];
      if (p.resid) {
        const f32x4 x = *reinterpret_cast<const f32x4 *>(p.resid + roff);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          rv[r] = x[r];
      } else {
        const u32x2 h = *reinterpret_cast<const u32x2 *>(p.resid16 + roff);
        const u32x2 l = *reinterpret_cast<const u32x2 *>(p.resid16_lo + roff);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const unsigned hw = h[r >> 1], lw = l[r >> 1];
          rv[r] = __uint_as_float((r & 1) ? (hw & 0xFFFF0000u) : (hw << 16)) +
                  __uint_as_float((r & 1) ? (lw & 0xFFFF0000u) : (lw << 16));
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = rv[r] + p.alpha * v[r];
    } else if (p.act != ACT_NONE) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = activate(v[r], p.act);
    }
    if (m < p.M) {
      if (p.out_mode == SKINNY_OUT_BF16) {
        const bool second = n >= p.split_n;
        const int cc = second ? n - p.split_n : n;
        const size_t off = static_cast<size_t>(m) * (second ? p.ldc2 : p.ldc) + cc;
        std::uint16_t *c = static_cast<std::uint16_t *>(second ? p.C2 : p.C) + off;
        std::uint16_t *c_lo = second ? p.C2_lo : p.C_lo;
        std::uint16_t hi[4], lo[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          hi[r] = f32_to_bf16(v[r]);
          lo[r] = f32_to_bf16(v[r] - bf16_to_f32(hi[r]));
        }
        *reinterpret_cast<u32x2 *>(c) = u32x2{hi[0] | (static_cast<unsigned>(hi[1]) << 16),
                                              hi[2] | (static_cast<unsigned>(hi[3]) << 16)};
        if (c_lo)
          *reinterpret_cast<u32x2 *>(c_lo + off) =
              u32x2{lo[0] | (static_cast<unsigned>(lo[1]) << 16),
                    lo[2] | (static_cast<unsigned>(lo[3]) << 16)};
      } else {
        *reinterpret_cast<f32x4 *>(static_cast<float *>(p.C) + static_cast<size_t>(m) * p.ldc +
                                   n) = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s += v[r];
      ss += v[r] * v[r];
    }
  }
  if (p.stats_out) {
    // Lanes fr, fr + 16, fr + 32, fr + 48 hold the same row.
    s += __shfl_xor(s, 16);
    ss += __shfl_xor(ss, 16);
    s += __shfl_xor(s, 32);
    ss += __shfl_xor(ss, 32);
    if (fc == 0 && m < p.M)
      *reinterpret_cast<float2 *>(p.stats_out +
                                  2 * (static_cast<size_t>(blockIdx.x) * p.M + m)) =
          make_float2(s, ss);
  }
}

int SkinnyNt(int N) { return N > 4096 ? 2 : 1; }



bool Aligned16(const void *ptr) { return (reinterpret_cast<std::uintptr_t>(ptr) & 15) == 0; }
// Null, or 8-byte aligned (the u32x2 stores and loads of bf16 planes).
bool Aligned8OrNull(const void *ptr) { return (reinterpret_cast<std::uintptr_t>(ptr) & 7) == 0; }

template <int NT, bool LN>
hipError_t LaunchSkinnyVariant(const SkinnyParams &p, hipStream_t stream) {
  const size_t lds = LN ? 2 * sizeof(float) * static_cast<size_t>(p.rows_per_src) * p.K : 0;
  if (lds > 48 * 1024) {
    static hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(SkinnyGemmKernel<NT, LN>),
        hipFuncAttributeMaxDynamicSharedMemorySize, 120 * 1024);
    if (attr != hipSuccess)
      return attr;
  }
  const int grid = (p.N + 16 * NT - 1) / (16 * NT);
  hipLaunchKernelGGL((SkinnyGemmKernel<NT, LN>), dim3(grid), dim3(1024), lds, stream, p);
  return hipGetLastError();
}

}  // namespace

bool SkinnyShapeOk(int M, int N, int K) {
  if (M < 1 || M > kSkinnyMaxRows || N < 4 || N % 4 || K < 64 || K % 64)
    return false;
  const int mt = (M + 15) / 16;
  const int mtp = mt <= 1 ? 1 : mt <= 2 ? 2 : 4;
  const int blocks = K / 64;
  const int ks = kSkWaves / mtp < blocks ? kSkWaves / mtp : blocks;
  return blocks % ks == 0;
}

int SkinnyGemmParts(int N) {
  const int nt = SkinnyNt(N);
  return (N + 16 * nt - 1) / (16 * nt);
}

hipError_t LaunchSkinnyGemm(const SkinnyParams &p, hipStream_t stream, std::string *err) {
  auto fail = [&](const char *why) {
    if (err)
      *err = std::string("skinny gemm: ") + why;
    return hipErrorInvalidValue;
  };
  if (!SkinnyShapeOk(p.M, p.N, p.K))
    return fail("shape (1 <= M <= 64, N % 4 == 0, K % 64 == 0 splitting evenly over the "
                "waves of a row tile)");
  if (!p.W || !Aligned16(p.W) || p.ldw % 8 || p.ldw < p.K || !p.C)
    return fail("weights (16-byte aligned, ldw % 8 == 0, ldw >= K) and output required");
  const bool ln = p.x != nullptr;
  if (ln) {
    if (!Aligned16(p.x) || p.ldx % 4 || p.rows_per_src < 1 || !p.ln_stats || p.ln_parts < 1 ||
        p.ln_rows < 1 || p.ln_width < 1 || !p.gamma || !p.beta || !Aligned16(p.gamma) ||
        !Aligned16(p.beta) || p.rows_per_src * p.K > 8192)
      return fail("LayerNorm operand (x, stats, gamma, beta; row segments up to 8192)");
    if (p.y16 && (p.rows_per_src != 1 || !Aligned16(p.y16) || p.ldy % 8 ||
                  (p.y16_lo && !Aligned16(p.y16_lo)) || (p.y32 && !Aligned16(p.y32))))
      return fail("normalised-row outputs need rows_per_src == 1 and 16-byte alignment");
  } else if (!p.a16 || !Aligned16(p.a16) || p.lda % 8 || p.lda < p.K ||
             (p.a16_lo && !Aligned16(p.a16_lo))) {
    return fail("activation planes (16-byte aligned, lda % 8 == 0, lda >= K)");
  }
  if (p.out_mode == SKINNY_OUT_BF16) {
    if (p.ldc % 4 || (p.split_n < p.N && (p.split_n % 16 || !p.C2 || p.ldc2 % 4)) ||
        p.stats_out)
      return fail("bf16 output (ldc % 4 == 0, split_n % 16 == 0, no statistics)");
    if (!Aligned8OrNull(p.C) || !Aligned8OrNull(p.C_lo) || !Aligned8OrNull(p.C2) ||
        !Aligned8OrNull(p.C2_lo))
      return fail("bf16 output planes must be 8-byte aligned");
  } else if (p.out_mode == SKINNY_OUT_F32 || p.out_mode == SKINNY_OUT_RESID) {
    if (!Aligned16(p.C) || p.ldc % 4 || p.split_n < p.N)
      return fail("fp32 output (16-byte aligned, ldc % 4 == 0, no column split)");
    if (p.out_mode == SKINNY_OUT_RESID &&
        ((!p.resid && !p.resid16) || (p.resid && p.resid16) || (p.resid16 && !p.resid16_lo) ||
         p.ldr % 4))
      return fail("residual (fp32 or hi + lo planes, ldr % 4 == 0)");
    if (p.out_mode == SKINNY_OUT_RESID &&
        ((p.resid && !Aligned16(p.resid)) || !Aligned8OrNull(p.resid16) ||
         !Aligned8OrNull(p.resid16_lo)))
      return fail("residual alignment (fp32 16 bytes, bf16 planes 8 bytes)");
  } else {
    return fail("output mode");
  }
  if (SkinnyNt(p.N) == 2)
    return ln ? LaunchSkinnyVariant<2, true>(p, stream) : LaunchSkinnyVariant<2, false>(p, stream);
  return ln ? LaunchSkinnyVariant<1, true>(p, stream) : LaunchSkinnyVariant<1, false>(p, stream);
}

}  // namespace mfh

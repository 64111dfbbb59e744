// bf16 MFMA GEMM for gfx950 with fused bias / activation / residual
// epilogues: the dense layers of the transformer body and heads
// (reference src/nn/cpu/cpu_network.cpp:822-890, 1057-1062, 1256-1259,
// 1318-1397).
//
// C[M,N] = A[M,K] . W[N,K]^T.  Both operands are K-contiguous (activations
// row-major, weights in the reference's [out][in] layout).  A workgroup of
// WM x WN waves owns a BM x BN tile; each wave owns a (BM/WM) x (BN/WN)
// sub-tile of v_mfma_f32_16x16x32_bf16 instructions.  K advances in BK-wide
// steps (BK = 32 or 64) through an ST-stage LDS ring filled by
// global_load_lds_dwordx4 (direct global->LDS, no VGPR round trip): ST - 1
// steps' tiles are in flight while the current one feeds the MFMAs, enough
// bytes in flight to cover the L2/HBM latency.  LDS rows
// are BK bf16 wide with their 16-byte chunks XOR-swizzled so that the 16 rows
// a fragment read touches spread over all bank groups; the swizzle is applied
// on the global side (each lane fetches the chunk that belongs in its LDS
// slot).
//
// The MFMA computes the transposed tile, D = W_frag . A_frag^T, so each lane
// ends up holding four consecutive output columns of one row: the epilogue
// stores 8 bytes (bf16) or 16 bytes (fp32) per lane instead of 2 or 4.
//
// FP8 weights (W8): the weight tile skips LDS.  Each wave loads its own
// fragments (8 e4m3 codes = 8 bytes per lane) from global memory one K step
// ahead, converts them exactly to bf16 with v_cvt_scalef32_pk_bf16_fp8, and
// the row scale multiplies the accumulators in the epilogue (or the split-K
// partials).
//
// Split precision: when A_lo is set, the activation is carried as
// hi + lo bf16 planes (lo = bf16(x - hi)) and every fragment pair issues two
// MFMAs, giving ~16-bit activation precision against exact bf16 weights.
#include "mfh_device.h"
#include "mfh_kernels.h"

#include <mutex>
#include <type_traits>

namespace mfh {
namespace {

// Element offset of 16-byte chunk `chunk` of LDS row `row` (rows of BK bf16).
// BK = 64: 8 chunks per 128-byte row, XOR with row & 7 and with 5 when bit 3
// of the row is set.  Measured on MI355X (LDS bank-conflict cycles per
// 16-byte read, fragment reads of 16 rows by 4 lane groups, every XOR-linear
// swizzle of the row's 4 bits tried): row & 7 alone is conflict-free for the
// bf16 reads (chunks c and 4 + c of lane group c) but costs 4 for the 8-bit
// K-step reads (chunks 2c and 2c + 1); XOR 1 for bit 3 the reverse; XOR 5
// none for both.  BK = 32: two rows per 128 bytes, XOR with (row >> 1) & 3,
// so rows r..r+7 cover all eight 16-byte bank groups.
__device__ __forceinline__ int Swz64Chunk(int row, int chunk) {
  return chunk ^ (row & 7) ^ (((row >> 3) & 1) * 5);
}
template <int BK>
__device__ __forceinline__ int Swz(int row, int chunk) {
  if constexpr (BK == 64)
    return row * 64 + (Swz64Chunk(row, chunk) << 3);
  else
    return row * 32 + ((chunk ^ ((row >> 1) & 3)) << 3);
}

// mu and r = 1 / sqrt(var + eps) of row `row` of a folded LayerNorm from
// its partial sums (width / part (sum x, sum x^2) pairs, added in order),
// with the reference formula var = E[x^2] - mu^2 clamped at 0.
__device__ __forceinline__ void RowLnStats(const float *stats, int width, int part, float eps,
                                           int row, float &mu, float &r) {
  const int pairs2 = width / (2 * part);
  const f32x4 *q = reinterpret_cast<const f32x4 *>(stats) + static_cast<size_t>(row) * pairs2;
  float s = 0.f, s2 = 0.f;
  // Eight quads at a time, loaded together.
  for (int i0 = 0; i0 < pairs2; i0 += 8) {
    f32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i0 + i < pairs2)
        v[i] = q[i0 + i];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i0 + i < pairs2) {
        s += v[i][0];
        s2 += v[i][1];
        s += v[i][2];
        s2 += v[i][3];
      }
  }
  mu = s / static_cast<float>(width);
  float var = s2 / static_cast<float>(width) - mu * mu;
  var = var < 0.f ? 0.f : var;
  r = 1.f / sqrtf(var + eps);
}

// Eight consecutive floats of a per-column vector.
__device__ __forceinline__ void LoadVec8(const float *v, int col, float (&o)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4 *>(v + col);
  const f32x4 b = *reinterpret_cast<const f32x4 *>(v + col + 4);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    o[r] = a[r];
    o[4 + r] = b[r];
  }
}

// A consumer of a folded LayerNorm: v = r (v - mu fold_c) for the row.
// (fold_c is loaded here, per row, from L1: holding it across the row loop
// costs registers the 256 x 128 tiles do not have.)
__device__ __forceinline__ void FoldLn8(const GemmParams &p, int row, int col, float (&v)[8]) {
  float mu, rr;
  RowLnStats(p.ln_stats, p.ln_width, p.ln_part, p.ln_eps, row, mu, rr);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const f32x4 c = *reinterpret_cast<const f32x4 *>(p.fold_c + col + 4 * h);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      v[4 * h + r] = rr * (v[4 * h + r] - mu * c[r]);
  }
}

// Epilogue for four consecutive outputs (row, col .. col + 3) of C, given
// the fp32 accumulators and bias: bias + activation to bf16 (with the lo
// plane and the split column) or fp32, or resid + alpha * (acc + bias).
// Columns at or past N are skipped; vector stores when the whole group is
// inside and the rows allow it (p.vec).
template <int MODE, int ACT, bool LN = false>
__device__ __forceinline__ void Epilogue4(const GemmParams &p, int row, int col, f32x4 acc,
                                          const float (&b)[4]) {
  const bool full = p.vec && col + 3 < p.N;
  if (p.wscale) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      acc[r] *= col + r < p.N ? p.wscale[col + r] : 0.f;
  }
  if (LN && p.fold_c) {
    // Consumer of a folded LayerNorm (never in the residual mode).
    float mu, rr;
    RowLnStats(p.ln_stats, p.ln_width, p.ln_part, p.ln_eps, row, mu, rr);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      acc[r] = rr * (acc[r] - mu * (col + r < p.N ? p.fold_c[col + r] : 0.f));
  }
  float v[4];
  if constexpr (MODE == GEMM_OUT_RESID_F32) {
    float *c = static_cast<float *>(p.C) + static_cast<size_t>(row) * p.ldc + col;
    const size_t roff = static_cast<size_t>(row) * p.ldr + col;
    float rv[4];
    if (p.resid16) {
      // Split residual: hi + lo bf16 planes.
      if (full) {
        const u32x2 h = *reinterpret_cast<const u32x2 *>(p.resid16 + roff);
        const u32x2 l = *reinterpret_cast<const u32x2 *>(p.resid16_lo + roff);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const unsigned hw = h[r >> 1], lw = l[r >> 1];
          rv[r] = __uint_as_float((r & 1) ? (hw & 0xFFFF0000u) : (hw << 16)) +
                  __uint_as_float((r & 1) ? (lw & 0xFFFF0000u) : (lw << 16));
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          rv[r] = col + r < p.N
                      ? bf16_to_f32(p.resid16[roff + r]) + bf16_to_f32(p.resid16_lo[roff + r])
                      : 0.f;
      }
    } else if (full) {
      const f32x4 x = *reinterpret_cast<const f32x4 *>(p.resid + roff);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        rv[r] = x[r];
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        rv[r] = col + r < p.N ? p.resid[roff + r] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      v[r] = rv[r] + p.alpha * (acc[r] + b[r]);
    if (full) {
      *reinterpret_cast<f32x4 *>(c) = f32x4{v[0], v[1], v[2], v[3]};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (col + r < p.N)
          c[r] = v[r];
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      v[r] = Act<ACT>(acc[r] + b[r], p.act);
    // split_n is a multiple of 4, so a group never straddles it.
    const bool second = col >= p.split_n;
    const int cc = second ? col - p.split_n : col;
    const size_t off = static_cast<size_t>(row) * (second ? p.ldc2 : p.ldc) + cc;
    const int valid = p.N - col;
    if constexpr (MODE == GEMM_OUT_F32) {
      float *c = static_cast<float *>(second ? p.C2 : p.C) + off;
      if (full) {
        *reinterpret_cast<f32x4 *>(c) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (r < valid)
            c[r] = v[r];
      }
    } else {
      std::uint16_t *c = static_cast<std::uint16_t *>(second ? p.C2 : p.C) + off;
      std::uint16_t *c_lo = static_cast<std::uint16_t *>(second ? p.C2_lo : p.C_lo);
      std::uint16_t hi[4], lo[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        hi[r] = f32_to_bf16(v[r]);
        lo[r] = f32_to_bf16(v[r] - bf16_to_f32(hi[r]));
      }
      // The lo parts as e4m3 codes (C_lo8, never beside a split output).
      std::uint8_t *c8 = p.C_lo8 ? p.C_lo8 + static_cast<size_t>(row) * p.ldc8 + col : nullptr;
      const unsigned q8 =
          c8 ? Lo8Pack4(v[0] - bf16_to_f32(hi[0]), v[1] - bf16_to_f32(hi[1]),
                        v[2] - bf16_to_f32(hi[2]), v[3] - bf16_to_f32(hi[3]))
             : 0u;
      if (full) {
        *reinterpret_cast<u32x2 *>(c) = u32x2{hi[0] | (static_cast<unsigned>(hi[1]) << 16),
                                              hi[2] | (static_cast<unsigned>(hi[3]) << 16)};
        if (c_lo)
          *reinterpret_cast<u32x2 *>(c_lo + off) =
              u32x2{lo[0] | (static_cast<unsigned>(lo[1]) << 16),
                    lo[2] | (static_cast<unsigned>(lo[3]) << 16)};
        if (c8)
          *reinterpret_cast<unsigned *>(c8) = q8;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (r < valid) {
            c[r] = hi[r];
            if (c_lo)
              c_lo[off + r] = lo[r];
            if (c8)
              c8[r] = static_cast<std::uint8_t>(q8 >> (8 * r));
          }
      }
    }
  }
}

// Output of eight consecutive columns (row, col .. col + 7) of a whole,
// aligned group on one side of split_n: v holds the scaled accumulators, b
// the bias and rv the residual (residual mode only).  One 16-byte store per
// output plane (two for fp32).
template <int MODE, int ACT>
__device__ __forceinline__ void Finish8(const GemmParams &p, int row, int col, float (&v)[8],
                                        const float (&b)[8], const float (&rv)[8]) {
  if constexpr (MODE == GEMM_OUT_RESID_F32) {
#pragma unroll
    for (int r = 0; r < 8; ++r)
      v[r] = rv[r] + p.alpha * (v[r] + b[r]);
    float *c = static_cast<float *>(p.C) + static_cast<size_t>(row) * p.ldc + col;
    *reinterpret_cast<f32x4 *>(c) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4 *>(c + 4) = f32x4{v[4], v[5], v[6], v[7]};
  } else {
#pragma unroll
    for (int r = 0; r < 8; ++r)
      v[r] = Act<ACT>(v[r] + b[r], p.act);
    const bool second = col >= p.split_n;
    const int cc = second ? col - p.split_n : col;
    const size_t off = static_cast<size_t>(row) * (second ? p.ldc2 : p.ldc) + cc;
    if constexpr (MODE == GEMM_OUT_F32) {
      float *c = static_cast<float *>(second ? p.C2 : p.C) + off;
      *reinterpret_cast<f32x4 *>(c) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4 *>(c + 4) = f32x4{v[4], v[5], v[6], v[7]};
    } else {
      std::uint16_t *c = static_cast<std::uint16_t *>(second ? p.C2 : p.C) + off;
      std::uint16_t *c_lo = static_cast<std::uint16_t *>(second ? p.C2_lo : p.C_lo);
      u32x4 hi, lo;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        std::uint32_t hw, lw;
        split_bf16x2(v[2 * h], v[2 * h + 1], hw, lw);
        hi[h] = hw;
        lo[h] = lw;
      }
      *reinterpret_cast<u32x4 *>(c) = hi;
      if (c_lo)
        *reinterpret_cast<u32x4 *>(c_lo + off) = lo;
      if (p.C_lo8) {
        float l[8];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          l[2 * h] = v[2 * h] - __uint_as_float(hi[h] << 16);
          l[2 * h + 1] = v[2 * h + 1] - __uint_as_float(hi[h] & 0xFFFF0000u);
        }
        *reinterpret_cast<u32x2 *>(p.C_lo8 + static_cast<size_t>(row) * p.ldc8 + col) =
            u32x2{Lo8Pack4(l[0], l[1], l[2], l[3]), Lo8Pack4(l[4], l[5], l[6], l[7])};
      }
    }
  }
}

// The residual of eight consecutive columns as fp32 (hi + lo bf16 planes,
// or fp32).
__device__ __forceinline__ void LoadResid8(const GemmParams &p, int row, int col,
                                           float (&rv)[8]) {
  const size_t roff = static_cast<size_t>(row) * p.ldr + col;
  if (p.resid16) {
    const u32x4 h = *reinterpret_cast<const u32x4 *>(p.resid16 + roff);
    const u32x4 l = *reinterpret_cast<const u32x4 *>(p.resid16_lo + roff);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const unsigned hw = h[r >> 1], lw = l[r >> 1];
      rv[r] = __uint_as_float((r & 1) ? (hw & 0xFFFF0000u) : (hw << 16)) +
              __uint_as_float((r & 1) ? (lw & 0xFFFF0000u) : (lw << 16));
    }
  } else {
    const f32x4 x0 = *reinterpret_cast<const f32x4 *>(p.resid + roff);
    const f32x4 x1 = *reinterpret_cast<const f32x4 *>(p.resid + roff + 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      rv[r] = x0[r];
      rv[4 + r] = x1[r];
    }
  }
}

// Bias and fp8 row scale of eight consecutive columns (zero / one when
// absent).
__device__ __forceinline__ void LoadBiasScale8(const GemmParams &p, int col, float (&b)[8],
                                               float (&sc)[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    b[r] = 0.f;
    sc[r] = 1.f;
  }
  if (p.bias) {
    const f32x4 b0 = *reinterpret_cast<const f32x4 *>(p.bias + col);
    const f32x4 b1 = *reinterpret_cast<const f32x4 *>(p.bias + col + 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      b[r] = b0[r];
      b[4 + r] = b1[r];
    }
  }
  if (p.wscale) {
    const f32x4 s0 = *reinterpret_cast<const f32x4 *>(p.wscale + col);
    const f32x4 s1 = *reinterpret_cast<const f32x4 *>(p.wscale + col + 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sc[r] = s0[r];
      sc[4 + r] = s1[r];
    }
  }
}

// Epilogue for eight consecutive outputs (row, col .. col + 7) given as two
// fp32 accumulator quads: one 16-byte store per output plane when the group
// is whole, aligned (p.vec8) and on one side of split_n; otherwise two
// four-column epilogues.
template <int MODE, int ACT, bool LN = false>
__device__ __forceinline__ void Epilogue8(const GemmParams &p, int row, int col, f32x4 a0,
                                          f32x4 a1) {
  if (!(p.vec8 && col + 7 < p.N && (col >= p.split_n || col + 8 <= p.split_n))) {
    float b[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      b[r] = (p.bias && col + r < p.N) ? p.bias[col + r] : 0.f;
    Epilogue4<MODE, ACT, LN>(p, row, col, a0, b);
    if (col + 4 < p.N) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        b[r] = (p.bias && col + 4 + r < p.N) ? p.bias[col + 4 + r] : 0.f;
      Epilogue4<MODE, ACT, LN>(p, row, col + 4, a1, b);
    }
    return;
  }
  float v[8], b[8], sc[8], rv[8];
  LoadBiasScale8(p, col, b, sc);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    v[r] = a0[r] * sc[r];
    v[4 + r] = a1[r] * sc[4 + r];
  }
  if (LN && p.fold_c)
    FoldLn8(p, row, col, v);
  if constexpr (MODE == GEMM_OUT_RESID_F32)
    LoadResid8(p, row, col, rv);
  Finish8<MODE, ACT>(p, row, col, v, b, rv);
}

// The folded-LayerNorm residual epilogue: a thread keeps one column group
// for the tile (the threads are a multiple of the groups per row and every
// thread runs the same rows) and each 128-column block of a row is 16
// consecutive lanes (tiles 128 or 256 columns wide).
// Rows per pass of the staged epilogue: the fp32 tile rows (BN + 4 floats
// each) that fit the LDS ring of ST stages of STAGE_BYTES.
template <int BM, int BN, int ST, int STAGE_BYTES>
constexpr int StagedRows() {
  constexpr int ring = ST * STAGE_BYTES / 4;
  constexpr int pitch = BN + 4;
  return ring >= BM * pitch    ? BM
         : ring >= 128 * pitch ? 128
         : ring >= 64 * pitch  ? 64
         : ring >= 32 * pitch  ? 32
                               : 16;
}
template <int BN, int THREADS, int RB>
constexpr bool GemmLnEpilogueOk() {
  return (BN == 64 || BN == 128 || BN == 256) && THREADS % (BN / 8) == 0 &&
         (RB * (BN / 8)) % THREADS == 0;
}

// fp8 weights (W8): the e4m3 rows go through the LDS ring as bytes (BK
// codes per row) when a stage's 1 KiB wave-loads split evenly over the
// waves; otherwise each wave loads its own weight fragments from global
// memory.
template <int BM, int BN, int BK, int WM, int WN, bool SPLIT>
constexpr bool W8InLds() {
  return ((SPLIT ? 2 : 1) * BM * BK * 2 + BN * BK) % (1024 * WM * WN) == 0;
}

// Bytes of one LDS ring stage: the activation rows (bf16, hi then lo) and
// the weight rows (bf16, or e4m3 bytes, or none).
template <int BM, int BN, int BK, int WM, int WN, bool SPLIT, bool W8>
constexpr int GemmStageBytes() {
  constexpr int a = (SPLIT ? 2 : 1) * BM * BK * 2;
  return !W8 ? a + BN * BK * 2 : W8InLds<BM, BN, BK, WM, WN, SPLIT>() ? a + BN * BK : a;
}

// Software-pipelined main loop (bf16 weights, BK = 32): LDS fragment reads
// for the next MFMAs are issued while earlier MFMAs run, so neither the LDS
// latency nor the LDS pipe's time opens a gap in the MFMA stream.  In the
// lock-step loop the compiler waited for each group of fragment reads just
// before the MFMAs using them (five exposed LDS latencies per K step).
//
// Split precision (hi + lo activation planes): a K step runs as two halves,
// the hi plane's MFMAs (TM x TN fragment pairs), then the lo plane's.
// During the hi half the lo fragments of the step are read; during the lo
// half the hi fragments of step k + 1 are read, and W_j of step k + 1 is
// read into W_j's registers as soon as its last MFMA of step k is issued.
// Nothing is double-buffered (256 x 256 tile: 128 accumulators + 16 + 16
// activation + 32 weight registers).  Single bf16: the activation
// fragments feed every MFMA of a step, so step k + 1's go into a second
// set; the weight fragments roll the same way.
//
// One barrier per step, before the reads of stage k + 1 begin: this wave's
// loads of stage k + 1 have landed (the loads of the ST - 2 later stages
// may stay in flight), so the barrier makes stage k + 1 visible; and every
// wave has waited for its reads of stage k, so that slot takes stage
// k + ST right after the barrier.  The loop is rotated so that it begins
// right after that barrier: the compiler's wait-count pass waits for every
// outstanding LDS read where a loop begins, and there none is in flight.
// Fragment i of activation plane q sits at a_off + (q BM + 16 i) BK
// elements of a stage and weight fragment j at w_off + 16 j BK (the swizzle
// of Swz repeats every 16 rows).
// (The buffer-resource type exists only in the device pass.)
#if defined(__HIP_DEVICE_COMPILE__)
// Buffer resource over a whole operand (raw addressing: stride 0, byte
// offsets below 2^31; the loads' offsets are clamped to valid rows, so the
// range check never triggers).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t BufferRsrc(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, 0x7FFFFFFF, 0x00020000);
}

template <int BM, int BN, int BK, int ST, int WM, int WN, bool SPLIT, int STAGE>
__device__ __forceinline__ void PipelinedLoop(const GemmParams &p, std::uint16_t *lds, int m0,
                                              int n0, int k_begin, int KT,
                                              f32x4 (&acc)[BM / WM / 16][BN / WN / 16]) {
  static_assert(BK == 32, "one MFMA K step per LDS stage");
  constexpr int NWAVES = WM * WN;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int P = SPLIT ? 2 : 1;
  constexpr int A_ROWS = P * BM;
  constexpr int CPR = BK / 8, RPL = 64 / CPR;  // 16-byte chunks per row, rows per wave-load
  constexpr int LPW = STAGE * 2 / 1024 / NWAVES;
  static_assert(BM % RPL == 0 && BN % RPL == 0, "a wave-load stays inside one operand");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int fr = lane & 15, fc = lane >> 4;

  // Global -> LDS loads of this wave: wave-load L covers rows L RPL ..
  // L RPL + RPL - 1 of the stage (A rows, then A_lo rows, then W rows).
  // They are MUBUF loads (buffer_load_dwordx4 ... lds): a buffer resource
  // per operand, the lane's byte offset in a register and the K step's in
  // a scalar one.  (The FLAT form, global_load_lds, counts as a possible
  // LDS access for the compiler's wait-count pass, which then waits for
  // every outstanding LDS read, lgkmcnt(0), wherever it waits for one.)
  __amdgpu_buffer_rsrc_t rsrc[LPW];
  unsigned goff[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int L = wave * LPW + j;
    const int row = L * RPL + lane / CPR;
    const int chunk = (lane % CPR) ^ ((row >> 1) & 3);
    if (L * RPL < BM) {
      rsrc[j] = BufferRsrc(p.A);
      goff[j] = 2u * (static_cast<unsigned>(min(m0 + row, p.M - 1)) * p.lda + k_begin + chunk * 8);
    } else if (SPLIT && L * RPL < 2 * BM) {
      rsrc[j] = BufferRsrc(p.A_lo);
      goff[j] = 2u * (static_cast<unsigned>(min(m0 + row - BM, p.M - 1)) * p.lda + k_begin +
                      chunk * 8);
    } else {
      rsrc[j] = BufferRsrc(p.W);
      goff[j] = 2u * (static_cast<unsigned>(min(n0 + row - A_ROWS, p.N - 1)) * p.ldw + k_begin +
                      chunk * 8);
    }
  }
  const int ldsw = __builtin_amdgcn_readfirstlane(wave * LPW * 512);  // elements
  auto fill = [&](int s, int slot) {
    std::uint16_t *d = lds + slot * STAGE + ldsw;
#pragma unroll
    for (int j = 0; j < LPW; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc[j], MFH_LDS_PTR(d + j * 512), 16, goff[j],
                                               s * (BK * 2), 0, 0);
  };

  const int a_off = Swz<BK>(wm * (BM / WM) + fr, fc);
  const int w_off = A_ROWS * BK + Swz<BK>(wn * (BN / WN) + fr, fc);
  auto read_a = [&](bf16x8 (&a)[TM], const std::uint16_t *base, int q) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      a[i] = *reinterpret_cast<const bf16x8 *>(base + a_off + (q * BM + i * 16) * BK);
  };
  auto read_w = [&](bf16x8 &w, const std::uint16_t *base, int j) {
    w = *reinterpret_cast<const bf16x8 *>(base + w_off + j * 16 * BK);
  };
  auto mfma_group = [&](const bf16x8 &w, const bf16x8 (&a)[TM], int j) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, a[i], acc[i][j], 0, 0, 0);
  };
  // s_waitcnt encodings (expcnt always left alone): vmcnt(kVmKeep) and
  // lgkmcnt(0); vmcnt(0) and lgkmcnt(0); lgkmcnt(0) alone; the prologue's
  // vmcnt(kPro) alone.
  constexpr int kVmKeep = (ST - 2) * LPW;
  constexpr int kPro = (ST - 1) * LPW;
  static_assert(kPro < 64, "vmcnt holds at most 63");
  constexpr int kWaitKeep = (kVmKeep & 15) | ((kVmKeep >> 4) << 14) | (7 << 4);
  constexpr int kWaitAll = 7 << 4;
  constexpr int kWaitLgkm = 0xC00F | (7 << 4);  // lgkmcnt(0) alone
  constexpr int kWaitPro = (kPro & 15) | ((kPro >> 4) << 14) | (7 << 4) | (15 << 8);

#pragma unroll
  for (int s = 0; s < ST; ++s)
    if (s < KT)
      fill(s, s);
  if (KT >= ST)
    __builtin_amdgcn_s_waitcnt(kWaitPro);
  else
    __builtin_amdgcn_s_waitcnt(0);
  asm volatile("s_barrier" ::: "memory");
  // Scalar loads (kernel arguments) share the LDS read counter and complete
  // out of order; none may be pending once the fragment reads begin, or
  // every wait on those reads becomes lgkmcnt(0).
  __builtin_amdgcn_s_waitcnt(kWaitLgkm);

  // Stage k + 1 visible, slot of stage k refilled with stage k + ST.
  // (The lgkmcnt(0) wait is unconditional: a wait chosen between two
  // branches leaves the wait-count pass a path with no wait at all, and it
  // then waits for every read issued after the barrier.)
  auto sync_next = [&](int k, int fslot) {
    __builtin_amdgcn_s_waitcnt(kWaitKeep);
    if (k + ST - 1 >= KT)
      __builtin_amdgcn_s_waitcnt(kWaitAll);
    asm volatile("s_barrier" ::: "memory");
    if (k + ST < KT)
      fill(k + ST, fslot);
  };

  bf16x8 w[TN];
  // The last step reads nothing more: it is peeled off so that the steady
  // loop's reads are unconditional and the wait counts stay exact.
  using More = std::integral_constant<bool, true>;
  using Last = std::integral_constant<bool, false>;
  int cslot = 0;  // slot of stage k
  if constexpr (SPLIT) {
    // The loop is rotated so that its header follows the step's barrier,
    // whose lgkmcnt(0) already drained the reads: an iteration is the lo
    // half of step k (reading stage k + 1) and the hi half of step k + 1.
    bf16x8 ahi[TM], alo[TM];
    read_a(ahi, lds, 0);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      read_w(w[j], lds, j);
    // hi half of a step whose stage is `cur`: the step's lo fragments are
    // read behind its first MFMA group.
    auto hi_half = [&](const std::uint16_t *cur) {
      mfma_group(w[0], ahi, 0);
      __builtin_amdgcn_sched_barrier(0);
      read_a(alo, cur, 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 1; j < TN; ++j) {
        mfma_group(w[j], ahi, j);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // lo half: behind its first MFMA group the next step's hi fragments
    // are read (the hi half has consumed this step's), and W_j of the next
    // step rolls in behind its last MFMA.  (No read precedes the first
    // group: the wait-count pass waits for every outstanding LDS read
    // where the loop begins, and nothing is in flight there yet.)
    auto lo_half = [&](auto tag, const std::uint16_t *nxt) {
      constexpr bool more = decltype(tag)::value;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        mfma_group(w[j], alo, j);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (more) {
          if (j == 0)
            read_a(ahi, nxt, 0);
          read_w(w[j], nxt, j);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    hi_half(lds);
    if (KT > 1)
      sync_next(0, 0);
    for (int k = 0; k + 2 < KT; ++k) {
      const int nslot = cslot + 1 == ST ? 0 : cslot + 1;
      const std::uint16_t *nxt = lds + nslot * STAGE;
      lo_half(More(), nxt);
      hi_half(nxt);
      sync_next(k + 1, nslot);
      cslot = nslot;
    }
    if (KT > 1) {
      const int nslot = cslot + 1 == ST ? 0 : cslot + 1;
      const std::uint16_t *nxt = lds + nslot * STAGE;
      lo_half(More(), nxt);
      hi_half(nxt);
    }
    lo_half(Last(), lds);
  } else {
    // Single bf16: the step's activation fragments feed every MFMA group,
    // so the next step's go into a second set; the loop is rotated like
    // the split one (an iteration is MFMA groups 1 .. TN-1 of step k,
    // reading stage k + 1, then group 0 of step k + 1 and the barrier).
    bf16x8 a[TM], an[TM];
    read_a(a, lds, 0);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      read_w(w[j], lds, j);
    auto rest = [&](auto tag, const std::uint16_t *nxt) {
      constexpr bool more = decltype(tag)::value;
      // Nothing is in flight here (the barrier's wait drained the reads);
      // saying so keeps the wait-count pass from draining mid-step.
      __builtin_amdgcn_s_waitcnt(kWaitLgkm);
      if constexpr (more) {
        read_a(an, nxt, 0);
        read_w(w[0], nxt, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 1; j < TN; ++j) {
        mfma_group(w[j], a, j);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (more)
          read_w(w[j], nxt, j);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (more) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          a[i] = an[i];
        mfma_group(w[0], a, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    mfma_group(w[0], a, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (KT > 1)
      sync_next(0, 0);
    for (int k = 0; k + 2 < KT; ++k) {
      const int nslot = cslot + 1 == ST ? 0 : cslot + 1;
      rest(More(), lds + nslot * STAGE);
      sync_next(k + 1, nslot);
      cslot = nslot;
    }
    if (KT > 1) {
      const int nslot = cslot + 1 == ST ? 0 : cslot + 1;
      rest(More(), lds + nslot * STAGE);
    }
    rest(Last(), lds);
  }
}

// The fp8 lo-correction pass of the BF16X2_FP8LO precision, run after the
// hi pass (PipelinedLoop) into the same accumulators: A_lo8 . W_lo8^T over
// the whole K on v_mfma_f32_16x16x128_f8f6f4, 128-byte K steps.  A stage is
// the BM activation code rows then the BN weight code rows, 128 bytes each,
// their 16-byte chunks XOR-swizzled with row & 7 (the F8 path's layout) and
// the bit 3 of the row as well; ST2 stages of (BM + BN) * 128 bytes share
// the kernel's LDS ring.  Lane
// (r, c) of a fragment feeds bytes 32 c .. 32 c + 31 of row r's K step
// (chunks 2 c and 2 c + 1), for A and W alike.
template <int BM, int BN, int WM, int WN, int ST2>
__device__ __forceinline__ void Lo8Loop(const GemmParams &p, std::uint16_t *lds, int m0, int n0,
                                        f32x4 (&acc)[BM / WM / 16][BN / WN / 16]) {
  constexpr int NWAVES = WM * WN;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int STAGE = (BM + BN) * 64;        // 16-bit units per stage
  constexpr int LOADS = (BM + BN) * 128 / 1024;  // 1 KiB wave-loads (8 rows)
  static_assert(LOADS % NWAVES == 0, "stage loads must split evenly over waves");
  constexpr int LPW = LOADS / NWAVES;
  static_assert(BM % 8 == 0 && ST2 == 2, "wave-loads inside one operand; two stages");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int fr = lane & 15, fc = lane >> 4;
  const int KT = p.K / 128;

  // A wave's LPW wave-loads are 8 LPW consecutive rows of one operand (BM
  // is a multiple of them), so one buffer resource, one lane offset and a
  // scalar offset per wave-load and K step address them.  The resource
  // covers the operand's rows exactly: rows past M or N read zeros (they
  // only feed outputs that are never stored).  Lane l takes row l / 8 of a
  // wave-load and its logical chunk Swz64Chunk(row, l % 8): a wave's loads
  // start at a multiple of 16 rows, so bit 3 of the row is the parity of
  // the wave-load, and the odd ones flip bits 4 and 6 of the offset (the
  // chunk's bits 0 and 2; the row offsets are multiples of 128 bytes:
  // ld % 128 == 0).
  static_assert(BM % (8 * LPW) == 0, "a wave's loads stay inside one operand");
  static_assert(LPW % 2 == 0 && BM % 16 == 0, "a wave's loads start at a multiple of 16 rows");
  const bool w_rows = wave * LPW * 8 >= BM;
  const int row0 = wave * LPW * 8 - (w_rows ? BM : 0);  // first row of the wave's loads
  const int ld = w_rows ? p.ldw8 : p.lda8;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<std::uint8_t *>(w_rows ? p.W_lo8 : p.A_lo8), 0,
      static_cast<int>((w_rows ? p.N : p.M) * static_cast<long>(ld)), 0x00020000);
  const unsigned goff =
      static_cast<unsigned>((w_rows ? n0 : m0) + row0 + lane / 8) * ld +
      Swz64Chunk(lane / 8, lane % 8) * 16;
  const int ldsw = __builtin_amdgcn_readfirstlane(wave * LPW * 512);  // 16-bit units
  auto fill = [&](int s, int slot) {
    std::uint16_t *d = lds + slot * STAGE + ldsw;
#pragma unroll
    for (int j = 0; j < LPW; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, MFH_LDS_PTR(d + j * 512), 16,
                                               (j & 1) ? goff ^ 80u : goff,
                                               s * 128 + j * 8 * ld, 0, 0);
  };
  // The hi pass's fragment reads of the ring are done before it is refilled.
  __builtin_amdgcn_s_waitcnt(0xC00F | (7 << 4));  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int s = 0; s < ST2 - 1; ++s)
    if (s < KT)
      fill(s, s);
  int slot = 0, fslot = ST2 - 1;
  for (int kt = 0; kt < KT; ++kt) {
    // Stage kt landed (this wave's loads; the barrier makes every wave's
    // visible), and slot fslot, read in step kt - 1, is free again.
    __builtin_amdgcn_s_waitcnt(7 << 4);  // vmcnt(0), lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    if (kt + ST2 - 1 < KT)
      fill(kt + ST2 - 1, fslot);
    const std::uint16_t *sa = lds + slot * STAGE;
    const std::uint16_t *sw = sa + BM * 64;
    slot = slot + 1 == ST2 ? 0 : slot + 1;
    fslot = fslot + 1 == ST2 ? 0 : fslot + 1;
    i32x8 af[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = wm * WTM + i * 16 + fr;
      const u32x4 c0 = *reinterpret_cast<const u32x4 *>(sa + Swz<64>(row, 2 * fc));
      const u32x4 c1 = *reinterpret_cast<const u32x4 *>(sa + Swz<64>(row, 2 * fc + 1));
      af[i] = i32x8{(int)c0[0], (int)c0[1], (int)c0[2], (int)c0[3],
                    (int)c1[0], (int)c1[1], (int)c1[2], (int)c1[3]};
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int row = wn * WTN + j * 16 + fr;
      const u32x4 c0 = *reinterpret_cast<const u32x4 *>(sw + Swz<64>(row, 2 * fc));
      const u32x4 c1 = *reinterpret_cast<const u32x4 *>(sw + Swz<64>(row, 2 * fc + 1));
      const i32x8 bw = i32x8{(int)c0[0], (int)c0[1], (int)c0[2], (int)c0[3],
                             (int)c1[0], (int)c1[1], (int)c1[2], (int)c1[3]};
#pragma unroll
      for (int i = 0; i < TM; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bw, af[i], acc[i][j], 0, 0,
                                                                    0, 0, 0, 0);
    }
  }
}
#endif  // __HIP_DEVICE_COMPILE__

template <int BM, int BN, int BK, int ST, int WM, int WN, bool SPLIT, int MODE, int ACT,
          bool W8, bool F8 = false, bool PIPE = false, bool LO8 = false, bool LN = false>
// (The folded-LayerNorm 256 x 128 tiles are held to 128 VGPRs, two
// workgroups per CU like the others of that shape.)
__global__ __launch_bounds__(WM *WN * 64, (LN && BM == 256 && BN == 128) ? 4 : 1) void GemmKernel(
    GemmParams p) {
  constexpr int NWAVES = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  constexpr int CPR = BK / 8;                      // 16-byte chunks per LDS row
  constexpr int RPL = 64 / CPR;                    // rows per 1 KiB wave-load
  constexpr int A_ROWS = SPLIT ? 2 * BM : BM;      // hi rows then lo rows
  constexpr int A_BYTES = A_ROWS * BK * 2;
  constexpr bool W8L = W8 && W8InLds<BM, BN, BK, WM, WN, SPLIT>();  // e4m3 rows in LDS
  constexpr bool W8G = W8 && !W8L;                 // e4m3 fragments from global
  constexpr int STAGE_BYTES = GemmStageBytes<BM, BN, BK, WM, WN, SPLIT, W8>();
  constexpr int STAGE = STAGE_BYTES / 2;           // bf16 elements per stage
  constexpr int LOADS = STAGE_BYTES / 1024;
  static_assert(STAGE_BYTES % 1024 == 0 && A_BYTES % 1024 == 0, "whole 1 KiB wave-loads");
  static_assert(!W8G || ST == 2, "fp8 weight fragments from global use the two-stage loop");
  // F8: both operands are e4m3 bytes staged like bf16 rows of BK = 64
  // (128-byte rows): one v_mfma_f32_16x16x128_f8f6f4 per fragment pair and
  // K step.  The launcher passes the byte operands with K and the leading
  // dimensions halved.
  static_assert(!F8 || (BK == 64 && !SPLIT && !W8), "fp8 activations: BK = 64 bytes pairs");
  static_assert(BK == 32 || BK == 64, "BK is 32 or 64");
  static_assert(!PIPE || (!W8 && !F8 && BK == 32), "pipelined loop: bf16 weights, BK = 32");
  static_assert(!LO8 || (PIPE && !SPLIT), "fp8 lo correction follows the single-plane hi pass");
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
  // XCD owns a contiguous range of tiles, walked in groups of 2 M-tiles so
  // the A and W panels the tiles in flight share stay in that XCD's L2.
  // With groups of 8, an XCD's 32 concurrent 256 x 256 tiles covered 8 A
  // panels and 4 W panels, and each round of N-tiles fetched the same A
  // panels again (Q|K|V fetched 252 MB against 73 MB of operands).  Groups
  // of 2 cover 2-3 A panels and all W panels per round: batch 128 forward
  // 6.56 -> 6.29 ms, 256 11.08 -> 10.85, 1024 43.76 -> 43.17 (groups of 1,
  // 3, 4 and 16 measured between or slower).
  int bid = blockIdx.x;
  if ((nb & 7) == 0)
    bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  constexpr int kGroupM = 2;
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

  // Each lane's source pointer for its LPW wave-loads.  Lane l lands in row
  // l / CPR of its wave-load, physical chunk l % CPR, so it fetches the
  // logical chunk that the swizzle puts there.  Rows past M or N read a
  // clamped valid row: they only feed outputs that are never stored.  The
  // e4m3 weight rows (W8L) are BK bytes, 1024 / BK per wave-load, lane l
  // fetching the wave-load's l-th 16 bytes unswizzled (a fragment read
  // covers 16 whole consecutive rows).  kstep: bytes per K step.
  const char *src[LPW];
  int kstep[LPW];
  int dst[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int L = wave * LPW + j;
    if (W8L && L * 1024 >= A_BYTES) {
      const int off = L * 1024 - A_BYTES + lane * 16;
      const int row = off / BK;
      src[j] = reinterpret_cast<const char *>(
          p.W8 + static_cast<size_t>(min(n0 + row, p.N - 1)) * p.ldw + k_begin + off % BK);
      kstep[j] = BK;
    } else {
      const int row = L * RPL + lane / CPR;
      const int phys = lane % CPR;
      const int chunk = BK == 64 ? Swz64Chunk(row, phys) : (phys ^ ((row >> 1) & 3));
      const std::uint16_t *s16;
      if (row < BM) {
        s16 = p.A + static_cast<size_t>(min(m0 + row, p.M - 1)) * p.lda + k_begin + chunk * 8;
      } else if (SPLIT && row < 2 * BM) {
        s16 = p.A_lo + static_cast<size_t>(min(m0 + row - BM, p.M - 1)) * p.lda + k_begin +
              chunk * 8;
      } else {
        s16 = p.W + static_cast<size_t>(min(n0 + row - A_ROWS, p.N - 1)) * p.ldw + k_begin +
              chunk * 8;
      }
      src[j] = reinterpret_cast<const char *>(s16);
      kstep[j] = BK * 2;
    }
    dst[j] = L * 512;
  }

  const int KT = kslice / BK;
  constexpr int KK = BK / 32;
  const int fr = lane & 15, fc = lane >> 4;
  // FP8 weight fragments: lane reads 8 codes of row n at k offset 8 fc.
  const std::uint8_t *wsrc[TN];
  u32x2 wq[KK][TN];
  if constexpr (W8G) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
      wsrc[j] = p.W8 + static_cast<size_t>(min(n0 + wn * WTN + j * 16 + fr, p.N - 1)) * p.ldw +
                k_begin + fc * 8;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        wq[kk][j] = *reinterpret_cast<const u32x2 *>(wsrc[j] + kk * 32);
  }
  // Stages 0 .. ST-2 in flight before the loop (the pipelined loop issues
  // its own).
#pragma unroll
  for (int s = 0; s < ST - 1; ++s)
    if (!PIPE && s < KT) {
#pragma unroll
      for (int j = 0; j < LPW; ++j)
        __builtin_amdgcn_global_load_lds(static_cast<const void *>(src[j] + s * kstep[j]),
                                         MFH_LDS_PTR(lds + s * STAGE + dst[j]), 16, 0, 0);
    }

  // acc[i][j]: transposed 16x16 tile, rows = output columns n, cols = rows m.
  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if constexpr (PIPE) {
#if defined(__HIP_DEVICE_COMPILE__)
    PipelinedLoop<BM, BN, BK, ST, WM, WN, SPLIT, STAGE>(p, lds, m0, n0, k_begin, KT, acc);
    if constexpr (LO8)
      Lo8Loop<BM, BN, WM, WN, 2>(p, lds, m0, n0, acc);
#endif
  } else {
  int slot = 0;                       // kt % ST
  int fill = (ST - 1) % ST;           // (kt + ST - 1) % ST
  for (int kt = 0; kt < KT; ++kt) {
    // Wait until this wave's loads of step kt have landed (the ST - 2 later
    // steps may stay in flight; loads complete in issue order), then the
    // barrier makes every wave's loads visible and guarantees that slot
    // `fill`, consumed in step kt - 1, is no longer read.
    if (kt + ST - 2 < KT) {
      constexpr int n = (ST - 2) * LPW;
      static_assert(n < 64, "vmcnt holds at most 63");
      __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    asm volatile("s_barrier" ::: "memory");
    if (kt + ST - 1 < KT) {
      std::uint16_t *next = lds + fill * STAGE;
#pragma unroll
      for (int j = 0; j < LPW; ++j)
        __builtin_amdgcn_global_load_lds(
            static_cast<const void *>(src[j] + (kt + ST - 1) * kstep[j]),
            MFH_LDS_PTR(next + dst[j]), 16, 0, 0);
    }
    const std::uint16_t *sa = lds + slot * STAGE;
    slot = slot + 1 == ST ? 0 : slot + 1;
    fill = fill + 1 == ST ? 0 : fill + 1;
    const std::uint16_t *sw = sa + A_ROWS * BK;
    u32x2 wn_next[KK][TN];
    if constexpr (W8G) {
      if (kt + 1 < KT) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            wn_next[kk][j] =
                *reinterpret_cast<const u32x2 *>(wsrc[j] + (kt + 1) * BK + kk * 32);
      }
    }
    if constexpr (F8) {
      // Lane (r, c) of a fragment holds bytes 32 c .. 32 c + 31 of row r's
      // 128-byte K step: 16-byte chunks 2 c and 2 c + 1.
      i32x8 af[TM], bw[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn * WTN + j * 16 + fr;
        const u32x4 c0 = *reinterpret_cast<const u32x4 *>(sw + Swz<BK>(row, 2 * fc));
        const u32x4 c1 = *reinterpret_cast<const u32x4 *>(sw + Swz<BK>(row, 2 * fc + 1));
        bw[j] = i32x8{(int)c0[0], (int)c0[1], (int)c0[2], (int)c0[3],
                      (int)c1[0], (int)c1[1], (int)c1[2], (int)c1[3]};
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WTM + i * 16 + fr;
        const u32x4 c0 = *reinterpret_cast<const u32x4 *>(sa + Swz<BK>(row, 2 * fc));
        const u32x4 c1 = *reinterpret_cast<const u32x4 *>(sa + Swz<BK>(row, 2 * fc + 1));
        af[i] = i32x8{(int)c0[0], (int)c0[1], (int)c0[2], (int)c0[3],
                      (int)c1[0], (int)c1[1], (int)c1[2], (int)c1[3]};
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bw[j], af[i], acc[i][j], 0,
                                                                      0, 0, 0, 0, 0);
    } else {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      bf16x8 af[TM], bw[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (W8L)
          bw[j] = Fp8x8ToBf16(*reinterpret_cast<const u32x2 *>(
              reinterpret_cast<const std::uint8_t *>(sw) + (wn * WTN + j * 16 + fr) * BK +
              kk * 32 + fc * 8));
        else if constexpr (W8G)
          bw[j] = Fp8x8ToBf16(wq[kk][j]);
        else
          bw[j] = *reinterpret_cast<const bf16x8 *>(
              sw + Swz<BK>(wn * WTN + j * 16 + fr, kk * 4 + fc));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8 *>(
            sa + Swz<BK>(wm * WTM + i * 16 + fr, kk * 4 + fc));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw[j], af[i], acc[i][j], 0, 0, 0);
      if constexpr (SPLIT) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const bf16x8 *>(
              sa + Swz<BK>(BM + wm * WTM + i * 16 + fr, kk * 4 + fc));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw[j], af[i], acc[i][j], 0, 0, 0);
      }
    }
    }  // F8 / bf16 fragments
    if constexpr (W8G) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          wq[kk][j] = wn_next[kk][j];
    }
  }
  }  // PIPE / lock-step loop

  // fp8 activations: each row's quantisation scale (the weight row scale
  // follows in the epilogue).  (Never with a folded LayerNorm.)
  if (!LN && p.ascale) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + wm * WTM + i * 16 + (lane & 15);
      const float rs = p.ascale[row < p.M ? row : p.M - 1];
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] *= rs;
    }
  }
  // Transposed accumulator layout: lane holds output row m_base + lane % 16
  // of its tile, columns n_base + 4 * (lane / 16) + r, r = 0..3.
  const int row_base = m0 + wm * WTM + (lane & 15);
  const int col_base = n0 + wn * WTN + (lane >> 4) * 4;
  if (!LN && p.k_splits > 1) {
    float *part = static_cast<float *>(p.C) + static_cast<size_t>(blockIdx.y) * p.M * p.ldc;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = row_base + i * 16;
      if (row >= p.M)
        continue;
      float *c = part + static_cast<size_t>(row) * p.ldc;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = col_base + j * 16;
        f32x4 v = acc[i][j];
        if (p.wscale) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[r] *= col + r < p.N ? p.wscale[col + r] : 0.f;
        }
        if (p.vec && col + 3 < p.N) {
          *reinterpret_cast<f32x4 *>(c + col) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (col + r < p.N)
              c[col + r] = v[r];
        }
      }
    }
    return;
  }
  // Staged epilogue (bf16 outputs, whole fp32 tiles, and the residual mode,
  // which also reads the residual): the fp32 accumulator tile passes through
  // LDS (reusing the operand ring, in row chunks of RB rows that fit it),
  // then each thread applies the epilogue to eight consecutive columns of a
  // row and stores them with 16-byte accesses: a wave writes whole 128-byte
  // lines of consecutive rows instead of pieces of sixteen rows.
  constexpr int PITCH = BN + 4;  // floats per staged row (+4: bank spread)
  constexpr int RING_FLOATS = ST * STAGE / 2;
  constexpr int RB = StagedRows<BM, BN, ST, STAGE_BYTES>();
  static_assert(RB * PITCH <= RING_FLOATS && BM % RB == 0 && RB % 16 == 0,
                "staged epilogue rows must fit the LDS ring");
  constexpr int GPR = BN / 8;  // 8-column groups per row
  float *tile = reinterpret_cast<float *>(lds);
  // Folded LayerNorm (LN instances): the tile's per-row mu and r (of the A
  // rows' LayerNorm for a consumer, of the residual rows' for a residual
  // GEMM) and per-column constants (fold_c; or the residual's gamma and beta
  // and the output's gamma), fetched once per tile (rows: G lanes each, see
  // ln_load; column t: thread t) and kept in the LDS ring behind the staged
  // rows.
  float *ln_row = tile + RB * PITCH;  // [BM][2]: mu, r
  float *ln_col = ln_row + 2 * BM;    // [3][BN], see ln_col8
  // The eight constants of column group c8 / 8 of plane `plane`: each
  // plane holds the groups' first four columns, then their last four, so a
  // wave's 16-byte reads of consecutive groups are consecutive (each lane's
  // eight in one run had lanes 32 bytes apart: 0.2-0.4 bank-conflict
  // cycles per LDS instruction in the folded epilogues).
  auto ln_col8 = [&](int plane, int c8, float (&o)[8]) {
    const float *b = ln_col + plane * BN + (c8 >> 3) * 4;
    const f32x4 lo = *reinterpret_cast<const f32x4 *>(b);
    const f32x4 hi = *reinterpret_cast<const f32x4 *>(b + BN / 2);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      o[r] = lo[r];
      o[4 + r] = hi[r];
    }
  };
  constexpr int THREADS = NWAVES * 64;
  float ln_c0 = 0.f, ln_c1 = 0.f, ln_c2 = 0.f;
  bool ln_on = false;
  // Load rounds issued before the staging: on 256-wide tiles all of them
  // for rows of up to 4 quads (width 1024), wider rows load the rest in the
  // staging; 128-wide tiles load all there (their registers are full: the
  // FFN1 forward at batch 256 measured 0.9-1.9 % faster so).
  constexpr int kLnPre = LN && BN == 256 ? (BM * 4 + THREADS - 1) / THREADS : 0;
  f32x4 ln_v[kLnPre > 0 ? kLnPre : 1] = {};
  int ln_q = 0, ln_g = 1, ln_rounds = 0;
  const float *st = nullptr;
  // Round k of the row-stat loads: lane idx = k * THREADS + tid reads quad
  // idx % G of tile row idx / G (zeros past the row's quads or the tile).
  auto ln_load = [&](int k) {
    const int idx = k * THREADS + tid, R = idx / ln_g, qd = idx % ln_g;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (k < ln_rounds && R < BM && qd < ln_q)
      v = reinterpret_cast<const f32x4 *>(st)[static_cast<size_t>(min(m0 + R, p.M - 1)) * ln_q +
                                              qd];
    return v;
  };
  // Sums a round's quads over each row's G lanes (a fixed shuffle order)
  // and stores the row's mu and r = 1 / sqrt(var + eps), with the reference
  // formula var = E[x^2] - mu^2 clamped at 0.  Every lane takes part.
  auto ln_reduce = [&](int k, f32x4 v, float eps) {
    float a = v[0] + v[2], a2 = v[1] + v[3];
    for (int m = 1; m < ln_g; m <<= 1) {
      a += __shfl_xor(a, m, 64);
      a2 += __shfl_xor(a2, m, 64);
    }
    const int idx = k * THREADS + tid, R = idx / ln_g;
    if (R < BM && idx % ln_g == 0) {
      const float mu = a / static_cast<float>(p.ln_width);
      float var = a2 / static_cast<float>(p.ln_width) - mu * mu;
      var = var < 0.f ? 0.f : var;
      ln_row[2 * R] = mu;
      ln_row[2 * R + 1] = 1.f / sqrtf(var + eps);
    }
  };
  if constexpr (LN) {
    static_assert(RB * PITCH + 2 * BM + 3 * BN <= RING_FLOATS && BN <= THREADS,
                  "folded LayerNorm constants fit behind the staged rows");
    st = p.fold_c ? p.ln_stats : p.res_stats;
    ln_on = p.fold_c || p.res_stats || p.out_gamma;
    // The rows' partial sums: G lanes per row (G = the row's quads of two
    // (sum, sum^2) pairs, a power of two, 64 at most), the first kLnPre
    // rounds of loads issued here so they are in flight during the staging.
    if (st) {
      ln_q = p.ln_width / (2 * p.ln_part);
      ln_g = 1;
      while (ln_g < ln_q)
        ln_g <<= 1;
      ln_rounds = (BM * ln_g + THREADS - 1) / THREADS;
#pragma unroll
      for (int k = 0; k < kLnPre; ++k)
        ln_v[k] = ln_load(k);
    }
    if (tid < BN) {
      // (A consumer, the bf16 mode, has fold_c only.)
      const int col = min(n0 + tid, p.N - 1);
      if constexpr (MODE != GEMM_OUT_RESID_F32) {
        ln_c0 = p.fold_c[col];
      } else {
        if (p.res_stats) {
          ln_c0 = p.res_gamma[col];
          ln_c1 = p.res_beta[col];
        }
        if (p.out_gamma)
          ln_c2 = p.out_gamma[col];
      }
    }
  }
  // Rows pass * RB .. + RB of the accumulator tile into the ring.
  auto stage = [&](int pass) {
    // The ring is no longer read (first pass) / the previous chunk is stored.
    __syncthreads();
    if constexpr (LN) {
      if (pass == 0 && ln_on) {
        if (st) {
          const float eps = p.fold_c ? p.ln_eps : p.res_eps;
#pragma unroll
          for (int k = 0; k < kLnPre; ++k)
            ln_reduce(k, ln_v[k], eps);
          for (int k = kLnPre; k < ln_rounds; ++k)
            ln_reduce(k, ln_load(k), eps);
        }
        if (tid < BN) {
          const int cs = ((tid & 7) >> 2) * (BN / 2) + (tid >> 3) * 4 + (tid & 3);
          ln_col[cs] = ln_c0;
          if constexpr (MODE == GEMM_OUT_RESID_F32) {
            ln_col[BN + cs] = ln_c1;
            ln_col[2 * BN + cs] = ln_c2;
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int rl = wm * WTM + i * 16 + (lane & 15);
      if (rl / RB != pass)
        continue;
#pragma unroll
      for (int j = 0; j < TN; ++j)
        *reinterpret_cast<f32x4 *>(tile + (rl % RB) * PITCH + wn * WTN + j * 16 +
                                   (lane >> 4) * 4) = acc[i][j];
    }
    __syncthreads();
  };
  // Whole, aligned tiles on one side of split_n, bf16 and fp32 outputs: when
  // the thread count is a multiple of the groups per row, a thread keeps one
  // column group for the whole tile (bias and scale loaded once) and its
  // rows of a chunk are ITER rows RSTEP apart; a wave stores whole rows
  // (fp32: two 16-byte stores per lane).  (The residual mode keeps the loop
  // below: requesting a chunk's residual rows ahead of the staging measured
  // slower.)
  // 256-wide tiles (32 column groups per row): a wave's 64 lanes read two
  // half rows of 16 groups each, lanes 16-31 the next row and lanes 32-63
  // the right halves (a wave reading one whole row measured 4 LDS
  // bank-conflict cycles per 16-byte read on MI355X; this order none).  A
  // thread's group for index g (g % 64 its lane): row 2 (g / 64) + bit 4 of
  // g, group (g % 16) + 16 (bit 5 of g).
  auto group_of = [&](int g, int &rl, int &c8) {
    if constexpr (GPR == 32) {
      rl = 2 * (g >> 6) + ((g >> 4) & 1);
      c8 = ((g & 15) + ((g >> 5) & 1) * 16) * 8;
    } else {
      rl = g / GPR;
      c8 = (g % GPR) * 8;
    }
  };
  if constexpr (MODE != GEMM_OUT_RESID_F32 && THREADS % GPR == 0 &&
                (RB * GPR) % THREADS == 0) {
    constexpr int ITER = RB * GPR / THREADS;
    constexpr int RSTEP = THREADS / GPR;
    int c8, r0;
    group_of(tid, r0, c8);
    const int col = n0 + c8;
    // (The pipelined LN instances take only whole tiles with fold_c, which
    // the launcher checks: their other epilogue paths are not compiled.)
    if ((LN && PIPE) ||
        (p.vec8 && n0 + BN <= p.N && (n0 + BN <= p.split_n || n0 >= p.split_n))) {
      float b[8], sc[8];
      LoadBiasScale8(p, col, b, sc);
      const bool fold = LN && (PIPE || p.fold_c != nullptr);
#pragma unroll 1
      for (int pass = 0; pass < BM / RB; ++pass) {
        const float none[8] = {};
        stage(pass);
#pragma unroll
        for (int k = 0; k < ITER; ++k) {
          const int rl = r0 + k * RSTEP;
          const int row = m0 + pass * RB + rl;
          if (row < p.M) {
            const float *src = tile + rl * PITCH + c8;
            const f32x4 a0 = *reinterpret_cast<const f32x4 *>(src);
            const f32x4 a1 = *reinterpret_cast<const f32x4 *>(src + 4);
            float v[8];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              v[r] = a0[r] * sc[r];
              v[4 + r] = a1[r] * sc[4 + r];
            }
            if (fold) {
              // r (v - mu fold_c) from the tile's LDS constants.
              const int rt = pass * RB + rl;
              const float mu = ln_row[2 * rt], rr = ln_row[2 * rt + 1];
              float fc[8];
              ln_col8(0, c8, fc);
#pragma unroll
              for (int r = 0; r < 8; ++r)
                v[r] = rr * (v[r] - mu * fc[r]);
            }
            Finish8<MODE, ACT>(p, row, col, v, b, none);
          }
        }
      }
      return;
    }
  }
  if constexpr (MODE == GEMM_OUT_F32) {
    // fp32 outputs of partial or unaligned tiles: each lane stores 16 bytes
    // per row straight from the accumulators.
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = col_base + j * 16;
      if (col >= p.N)
        continue;
      float b[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        b[r] = (p.bias && col + r < p.N) ? p.bias[col + r] : 0.f;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = row_base + i * 16;
        if (row < p.M)
          Epilogue4<MODE, ACT, LN>(p, row, col, acc[i][j], b);
      }
    }
    return;
  }
  if constexpr (LN && MODE == GEMM_OUT_RESID_F32 && (BN == 256 || BN == 64) &&
                GemmLnEpilogueOk<BN, THREADS, RB>()) {
    if (PIPE || p.out_gamma || p.res_stats) {
      // Residual mode with a folded LayerNorm on either side (whole tiles,
      // checked by the launcher): the residual is LN(x) of x o gamma rows
      // (res_stats), and/or the result x = resid + alpha (acc + b) leaves
      // as x o out_gamma in bf16 hi + lo (+ e4m3 codes) with the partial
      // sums of x over each block of kPart columns (128 on 256-wide tiles,
      // 64 on 64-wide ones): a block is kPart / 8 consecutive lanes of one
      // row (8 columns each), summed by shuffles in a fixed order.  A
      // thread keeps one column group for the whole tile.
      constexpr int kPartLanes = BN == 64 ? 8 : 16, kPart = 8 * kPartLanes;
      int c8, r0;
      group_of(tid, r0, c8);
      const int col = n0 + c8;
      float b[8], sc[8];
      LoadBiasScale8(p, col, b, sc);
      const int parts = p.ln_width / kPart;
#pragma unroll 1
      for (int pass = 0; pass < BM / RB; ++pass) {
        stage(pass);
        for (int g = tid; g < RB * GPR; g += THREADS) {
          int rl, cc;  // cc == c8: g % 64 is the thread's lane
          group_of(g, rl, cc);
          (void)cc;
          const int row = m0 + pass * RB + rl;
          const bool valid = row < p.M;
          const float *src = tile + rl * PITCH + c8;
          const f32x4 a0 = *reinterpret_cast<const f32x4 *>(src);
          const f32x4 a1 = *reinterpret_cast<const f32x4 *>(src + 4);
          float x[8], rv[8];
          if (valid) {
            LoadResid8(p, row, col, rv);
            if (p.res_stats) {
              // LN of the residual row: r (x o gamma - mu gamma) + beta.
              const int rt = pass * RB + rl;
              const float mu = ln_row[2 * rt], rr = ln_row[2 * rt + 1];
              float g[8], be[8];
              ln_col8(0, c8, g);
              ln_col8(1, c8, be);
#pragma unroll
              for (int r = 0; r < 8; ++r)
                rv[r] = rr * (rv[r] - mu * g[r]) + be[r];
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            x[r] = valid ? rv[r] + p.alpha * (a0[r] * sc[r] + b[r]) : 0.f;
            x[4 + r] = valid ? rv[4 + r] + p.alpha * (a1[r] * sc[4 + r] + b[4 + r]) : 0.f;
          }
          if (!p.out_gamma) {
            if (valid) {
              float *c = static_cast<float *>(p.C) + static_cast<size_t>(row) * p.ldc + col;
              *reinterpret_cast<f32x4 *>(c) = f32x4{x[0], x[1], x[2], x[3]};
              *reinterpret_cast<f32x4 *>(c + 4) = f32x4{x[4], x[5], x[6], x[7]};
            }
            continue;
          }
          float s = 0.f, s2 = 0.f;
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            s += x[r];
            s2 += x[r] * x[r];
          }
#pragma unroll
          for (int m = 1; m < kPartLanes; m <<= 1) {
            s += __shfl_xor(s, m, 64);
            s2 += __shfl_xor(s2, m, 64);
          }
          if (!valid)
            continue;
          if ((lane & (kPartLanes - 1)) == 0)
            *reinterpret_cast<f32x2 *>(p.out_stats + (static_cast<size_t>(row) * parts +
                                                      col / kPart) * 2) = f32x2{s, s2};
          float y[8], og[8], none[8] = {};
          ln_col8(2, c8, og);
#pragma unroll
          for (int r = 0; r < 8; ++r)
            y[r] = x[r] * og[r];
          Finish8<GEMM_OUT_BF16, ACT_NONE>(p, row, col, y, none, none);
        }
      }
      return;
    }
  }
  if constexpr (!(LN && PIPE)) {
#pragma unroll 1
    for (int pass = 0; pass < BM / RB; ++pass) {
      stage(pass);
      for (int g = tid; g < RB * GPR; g += NWAVES * 64) {
        int rl, c8;
        group_of(g, rl, c8);
        const int row = m0 + pass * RB + rl, col = n0 + c8;
        if (row >= p.M || col >= p.N)
          continue;
        const float *src = tile + rl * PITCH + c8;
        Epilogue8<MODE, ACT, LN>(p, row, col, *reinterpret_cast<const f32x4 *>(src),
                                 *reinterpret_cast<const f32x4 *>(src + 4));
      }
    }
  }
}

// Sums the k_splits fp32 partial tiles of a split-K launch in slice order
// and applies the epilogue: one thread per four consecutive outputs.  With
// LN, the GEMM read folded rows (x o gamma) and the epilogue applies their
// LayerNorm (p.fold_c, p.ln_stats) before the bias.
template <int MODE, int ACT, bool LN = false>
__global__ __launch_bounds__(256) void ReduceEpilogueKernel(GemmParams p, const float *part,
                                                            int splits) {
  const int groups = (p.N + 3) / 4;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int row = idx / groups;
  if (row >= p.M)
    return;
  const int col = (idx % groups) * 4;
  const size_t plane = static_cast<size_t>(p.M) * p.N;
  const float *src = part + static_cast<size_t>(row) * p.N + col;
  f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
  if (p.vec && col + 3 < p.N) {
    a = sum_parts4(src, plane, splits);
  } else {
    for (int s = 0; s < splits; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (col + r < p.N)
          a[r] += src[s * plane + r];
  }
  float b[4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    b[r] = (p.bias && col + r < p.N) ? p.bias[col + r] : 0.f;
  Epilogue4<MODE, ACT, LN>(p, row, col, a, b);
}

template <int BM, int BN, int BK, int ST, int WM, int WN, bool SPLIT, int MODE, int ACT,
          bool W8 = false, bool F8 = false, bool PIPE = false, bool LO8 = false, bool LN = false>
hipError_t LaunchVariant(const GemmParams &p, hipStream_t stream) {
  // The LDS ring: ST stages of the main loop, or two stages of the fp8 lo
  // pass's 128-byte rows when larger.
  constexpr size_t kRing =
      static_cast<size_t>(ST) * GemmStageBytes<BM, BN, BK, WM, WN, SPLIT, W8>();
  constexpr size_t kLo8Ring = LO8 ? static_cast<size_t>(2) * (BM + BN) * 128 : 0;
  constexpr size_t kLds = kRing > kLo8Ring ? kRing : kLo8Ring;
  auto kernel = GemmKernel<BM, BN, BK, ST, WM, WN, SPLIT, MODE, ACT, W8, F8, PIPE, LO8, LN>;
  constexpr int kRb = StagedRows<BM, BN, ST, GemmStageBytes<BM, BN, BK, WM, WN, SPLIT, W8>()>();
  if constexpr (MODE == GEMM_OUT_RESID_F32) {
    // The folded-LayerNorm residual epilogue takes whole 256-wide tiles.
    // (Partial sums per 128 columns on 256-wide tiles, per 64 on 64-wide.)
    if ((p.out_gamma || p.res_stats) &&
        !(LN && (BN == 256 || BN == 64) && GemmLnEpilogueOk<BN, WM * WN * 64, kRb>() &&
          p.vec8 && p.N % BN == 0 && p.ln_part == (BN == 64 ? 64 : 128)))
      return hipErrorInvalidValue;
    if (LN && PIPE && !p.out_gamma && !p.res_stats)
      return hipErrorInvalidValue;
  } else if constexpr (LN && PIPE) {
    // The pipelined consumer instances compile only the whole-tile epilogue.
    constexpr int kGpr = BN / 8, kThreads = WM * WN * 64;
    if (!p.fold_c || !p.vec8 || p.N % BN || (p.split_n < p.N && p.split_n % BN) ||
        kThreads % kGpr || (kRb * kGpr) % kThreads)
      return hipErrorInvalidValue;
  }
  if (LN && (p.ascale || p.k_splits != 1))
    return hipErrorInvalidValue;
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

template <int MODE, int ACT, bool LN = false>
hipError_t LaunchReduce(const GemmParams &p, const float *part, int splits,
                        hipStream_t stream) {
  const long threads = static_cast<long>(p.M) * ((p.N + 3) / 4);
  hipLaunchKernelGGL((ReduceEpilogueKernel<MODE, ACT, LN>), dim3((threads + 255) / 256),
                     dim3(256), 0, stream, p, part, splits);
  return hipGetLastError();
}

hipError_t Reduce(const GemmParams &p, const float *part, int splits, hipStream_t stream) {
  if (p.fold_c) {
    // A folded LayerNorm's consumer (bf16 output only).
    if (p.out_mode != GEMM_OUT_BF16 || !p.ln_stats)
      return hipErrorInvalidValue;
    return p.act == ACT_NONE
               ? LaunchReduce<GEMM_OUT_BF16, ACT_NONE, true>(p, part, splits, stream)
               : LaunchReduce<GEMM_OUT_BF16, ACT_RUNTIME, true>(p, part, splits, stream);
  }
  if (p.out_mode == GEMM_OUT_RESID_F32)
    return LaunchReduce<GEMM_OUT_RESID_F32, ACT_NONE>(p, part, splits, stream);
  if (p.out_mode == GEMM_OUT_F32)
    return p.act == ACT_NONE ? LaunchReduce<GEMM_OUT_F32, ACT_NONE>(p, part, splits, stream)
                             : LaunchReduce<GEMM_OUT_F32, ACT_RUNTIME>(p, part, splits, stream);
  if (p.act == ACT_NONE)
    return LaunchReduce<GEMM_OUT_BF16, ACT_NONE>(p, part, splits, stream);
  if (p.act == ACT_MISH)
    return LaunchReduce<GEMM_OUT_BF16, ACT_MISH>(p, part, splits, stream);
  return LaunchReduce<GEMM_OUT_BF16, ACT_RUNTIME>(p, part, splits, stream);
}

// Epilogue dispatch: the activations the network uses (none, mish) get
// dedicated instances, anything else the runtime switch.
template <int BM, int BN, int BK, int ST, int WM, int WN, bool SPLIT, bool W8, bool F8 = false,
          bool PIPE = false, bool LO8 = false>
hipError_t LaunchW(const GemmParams &p, hipStream_t stream) {
  // A folded LayerNorm (GemmParams::fold_c / out_gamma / res_stats): its
  // epilogue code is compiled only into the tiles that take it (LnFoldTile:
  // the pipelined split-precision and BF16X2_FP8LO tiles of the large
  // batches, the small-LDS split 64 x 64 tile of the smolgen compression
  // beside Q|K|V and at 24-62 positions where its K is not split, and the
  // split 64 x 64 tiles of 24-62 positions), bf16 outputs and the residual
  // mode; the split-K reduce applies it for split consumers.
  constexpr bool kLn = !W8 && !F8 && (SPLIT || LO8) && (PIPE || (BM == 64 && BN == 64));
  if (p.fold_c || p.out_gamma || p.res_stats) {
    if constexpr (kLn) {
      if (p.k_splits == 1 && p.out_mode == GEMM_OUT_RESID_F32)
        return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_RESID_F32, ACT_NONE, W8, F8,
                             PIPE, LO8, true>(p, stream);
      if (p.k_splits == 1 && p.out_mode == GEMM_OUT_BF16 && p.act == ACT_NONE)
        return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_NONE, W8, F8,
                             PIPE, LO8, true>(p, stream);
      if (p.k_splits == 1 && p.out_mode == GEMM_OUT_BF16 && p.act == ACT_MISH)
        return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_MISH, W8, F8,
                             PIPE, LO8, true>(p, stream);
      if (p.k_splits == 1 && p.out_mode == GEMM_OUT_BF16)
        return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_RUNTIME, W8, F8,
                             PIPE, LO8, true>(p, stream);
    }
    return hipErrorInvalidValue;
  }
  if (p.k_splits > 1 || (p.out_mode == GEMM_OUT_F32 && p.act == ACT_NONE))
    return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_F32, ACT_NONE, W8, F8, PIPE, LO8>(p, stream);
  if (p.out_mode == GEMM_OUT_RESID_F32)
    return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_RESID_F32, ACT_NONE, W8, F8, PIPE, LO8>(p, stream);
  if (p.out_mode == GEMM_OUT_F32)
    return p.act == ACT_MISH
               ? LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_F32, ACT_MISH, W8, F8, PIPE, LO8>(p, stream)
               : LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_F32, ACT_RUNTIME, W8, F8, PIPE, LO8>(p, stream);
  if (p.act == ACT_NONE)
    return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_NONE, W8, F8, PIPE, LO8>(p, stream);
  if (p.act == ACT_MISH)
    return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_MISH, W8, F8, PIPE, LO8>(p, stream);
  return LaunchVariant<BM, BN, BK, ST, WM, WN, SPLIT, GEMM_OUT_BF16, ACT_RUNTIME, W8, F8, PIPE, LO8>(p, stream);
}

template <int BM, int BN, int BK, int ST, int WM, int WN, bool SPLIT>
hipError_t Launch(const GemmParams &p, hipStream_t stream) {
  // fp8 weights: the ring's stages when their rows go through LDS, else two
  // (fragments from global memory).
  if (p.W8)
    return LaunchW<BM, BN, BK, W8InLds<BM, BN, BK, WM, WN, SPLIT>() ? ST : 2, WM, WN, SPLIT,
                   true>(p, stream);
  return LaunchW<BM, BN, BK, ST, WM, WN, SPLIT, false>(p, stream);
}

bool Aligned(const void *ptr, std::uintptr_t bytes) {
  return (reinterpret_cast<std::uintptr_t>(ptr) & (bytes - 1)) == 0;
}

}  // namespace

// Rows from which the tile rules for large problems apply (below them,
// 64 x 64 tiles over the whole K or split-K).  From 1536 rows (24
// positions) Q|K|V takes 256 x 128 split tiles instead of 1176-1519
// whole-K 64 x 64 ones: forward at batch 24 2.47 -> 2.41 ms, 28 2.60 ->
// 2.50, 31 2.84 -> 2.56; from 1024 rows it was slower (batch 16 2.07 ->
// 2.34).
constexpr int kLargeRows = 1536;

// 256 x 256 tiles where they fill whole rounds of 256 workgroups (bf16
// activations, one K slice, from the large-problem rows).
bool GemmWholeRoundTiles(const GemmParams &p) {
  const long big_tiles = static_cast<long>((p.M + 255) / 256) * ((p.N + 255) / 256);
  return p.M >= kLargeRows && p.N >= 128 && p.k_splits == 1 && big_tiles % 256 == 0 && !p.A8;
}

namespace {

// The instances that compile a folded LayerNorm's epilogue, and the one a
// GEMM with a folded LayerNorm runs on (the tiles the same shapes take
// without it, where those are among them): split precision (bf16 hi + lo
// activations, or the BF16X2_FP8LO codes), bf16 weights, one K slice.
enum class LnTile { kNone, kLo8, k256, k256Beside, k256x128, k64, k64x64, kSplitK };

LnTile LnFoldTile(const GemmParams &p) {
  const bool res = p.out_mode == GEMM_OUT_RESID_F32;
  if ((!p.A_lo && !p.A_lo8) || p.W8 || p.A8 || p.k_splits != 1 || p.K % 64)
    return LnTile::kNone;
  if (!res && p.out_mode != GEMM_OUT_BF16)
    return LnTile::kNone;
  // Whole rounds of 256-wide whole tiles.
  if (p.A_lo8)
    return p.N % 256 == 0 ? LnTile::kLo8 : LnTile::kNone;
  if (p.N % 256 == 0 && GemmWholeRoundTiles(p))
    return p.beside_chain && !res ? LnTile::k256Beside : LnTile::k256;
  // Fewer 128 x 128 tiles than CUs (24-62 positions at the BT4 widths): the
  // 64 x 64 tiles over the whole K that these shapes take without the fold.
  // Consumers up to 2048 wide also up to two rounds of them (FFN1 at 43-62
  // positions, 128 x 128 tiles without the fold; on 256 x 128 ones with it
  // the forward was 3.4 % slower at batch 48, 0.5 % at 56).
  const long tiles128 = static_cast<long>((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (p.M >= kLargeRows && p.N >= 128 && p.N % 64 == 0 &&
      (tiles128 < 256 || (!res && p.N <= 2048 && tiles128 < 512)))
    return LnTile::k64x64;
  if (res)
    return LnTile::kNone;
  // Consumers: the small-LDS 64 x 64 tiles beside Q|K|V (any width); narrow
  // ones (the smolgen compression at 24-62 positions) split over K where
  // the launcher splits them (the split GEMM sums x o gamma and the reduce
  // kernel applies the LayerNorm before the bias), else on those 64 x 64
  // tiles; else 256 x 128 pipelined tiles.
  if (p.small_lds)
    return LnTile::k64;
  if (p.N < 128)
    return GemmAutoSplits(p) > 1 ? LnTile::kSplitK : LnTile::k64;
  return p.N % 128 == 0 ? LnTile::k256x128 : LnTile::kNone;
}

}  // namespace

bool GemmLnFoldOk(const GemmParams &p) { return LnFoldTile(p) != LnTile::kNone; }

// Split-K at few positions (64 x 64 tiles, K in 64-wide steps).  A GEMM
// kernel here costs ~5 us however short its K loop, and a separate reduce
// launch another ~4.5 us, so:
// * the slices fill at most one workgroup per CU (256): beyond that the
//   extra slices lengthen the kernel more than they shorten each loop;
// * a split whose partials need their own reduce launch (LaunchGemm) is
//   taken for long K loops only (>= 16 steps) and at least four ways: a
//   two-way split of FFN1 at 256 rows (10.1 + 4.8 us against 11.9 us whole)
//   and any split of the smolgen global projection (K = 256) lost;
// * a caller whose next kernel sums the partials anyway (the LayerNorm
//   after a residual GEMM) also takes a two-way split up to 384 workgroups.
// Measured forward (with the three-stage rings below): batch 1 1.29 ->
// 1.20 ms, 2 1.43 -> 1.26, 4 1.58 -> 1.33, 8 1.62 -> 1.48, 12 1.79 -> 1.76.
// (kSplitMaxGroups and kSplitPairMaxGroups are in mfh_kernels.h.)
constexpr int kSplitMinSteps = 16;
constexpr int kSplitMinParts = 4;

int GemmAutoSplits(const GemmParams &p, bool summed_by_consumer) {
  const bool large = p.M >= kLargeRows && p.N >= 128;
  if (large || p.k_splits != 1 || !p.partials || p.N % 4 || p.K % 64 || p.M <= 0 || p.N <= 0)
    return 1;
  const long tiles = static_cast<long>((p.M + 63) / 64) * ((p.N + 63) / 64);
  const int steps = p.K / 64;
  const auto fits = [&](int s) {
    return static_cast<size_t>(s) * p.M * p.N <= p.partials_floats;
  };
  int splits = 1;
  if (summed_by_consumer || steps >= kSplitMinSteps)
    for (int s = 2; s <= steps; ++s)
      if (steps % s == 0 && tiles * s <= kSplitMaxGroups && fits(s))
        splits = s;
  if (!summed_by_consumer && splits < kSplitMinParts)
    splits = 1;
  if (splits == 1 && summed_by_consumer && steps % 2 == 0 && tiles * 2 <= kSplitPairMaxGroups &&
      fits(2))
    splits = 2;
  return splits;
}

hipError_t LaunchGemm(const GemmParams &p_in, hipStream_t stream, std::string *err) {
  auto fail = [&](const char *why) {
    if (err)
      *err = std::string("gemm: ") + why;
    return hipErrorInvalidValue;
  };
  GemmParams p = p_in;
  const bool lo8 = p.A_lo8 != nullptr;
  if (lo8 && (!p.A || p.A_lo || !p.W || p.W8 || !p.wscale || !p.W_lo8 || p.A8 ||
              p.k_splits != 1 || p.K % 128 || p.lda8 % 128 || p.ldw8 % 128 || p.lda8 < p.K ||
              p.ldw8 < p.K || !Aligned(p.A_lo8, 16) || !Aligned(p.W_lo8, 16)))
    return fail("fp8 lo correction needs A (hi) + A_lo8 with W (bf16) + W_lo8 + wscale, "
                "one K slice, K % 128 == 0, lda8 / ldw8 % 128 == 0 and 16-byte aligned codes");
  const bool f8 = p.A8 != nullptr;
  if (f8) {
    // fp8 activations x fp8 weights: the byte operands go through the bf16
    // data path as 16-bit units (K and leading dimensions halved); the F8
    // kernels run one fp8 MFMA per 128-byte K step.
    if (p.A || p.A_lo || !p.W8 || p.W || !p.wscale || !p.ascale || p.k_splits != 1 ||
        p.K % 128 || p.lda % 16 || p.ldw % 16 || p.lda < p.K || p.ldw < p.K ||
        !Aligned(p.A8, 16) || !Aligned(p.W8, 16) || p.M < 2048)
      return fail("fp8 activations need A8 + ascale with W8 + wscale, K % 128 == 0, "
                  "lda / ldw % 16 == 0, 16-byte aligned operands and M >= 2048");
    p.A = reinterpret_cast<const std::uint16_t *>(p.A8);
    p.lda /= 2;
    p.W = reinterpret_cast<const std::uint16_t *>(p.W8);
    p.W8 = nullptr;
    p.ldw /= 2;
    p.K /= 2;
    p.partials = nullptr;
  }
  if (p.M <= 0 || p.N <= 0 || p.K <= 0)
    return fail("non-positive shape");
  if (p.K % 32)
    return fail("K must be a multiple of 32");
  if (p.k_splits < 1 || p.K % (p.k_splits * 32))
    return fail("K must split into multiples of 32");
  if (p.k_splits > 1 && (p.out_mode != GEMM_OUT_F32 || p.bias || p.act != ACT_NONE ||
                         p.split_n < p.N))
    return fail("split-K writes raw fp32 partials only (no bias, activation or split)");
  if (!p.A || (!p.W && !p.W8) || (p.W && p.W8) || !p.C)
    return fail("null operand (or both W and W8)");
  if (p.W8 && !p.wscale)
    return fail("fp8 weights need row scales");
  if (!Aligned(p.A, 16) || (p.W && !Aligned(p.W, 16)) || (p.W8 && !Aligned(p.W8, 8)) ||
      (p.A_lo && !Aligned(p.A_lo, 16)) || p.lda % 8 || p.ldw % 8 || p.lda < p.K ||
      p.ldw < p.K)
    return fail("operands must be 16-byte aligned with ld >= K, ld % 8 == 0");
  if (p.out_mode == GEMM_OUT_RESID_F32 &&
      ((!p.resid && !p.resid16) || (p.resid && p.resid16) ||
       (p.resid16 != nullptr) != (p.resid16_lo != nullptr) || p.split_n < p.N))
    return fail("residual mode needs resid (fp32) or resid16 + resid16_lo (split), and no "
                "split output");
  if (p.out_mode == GEMM_OUT_RESID_F32 && p.resid16 &&
      (!Aligned(p.resid16, 2) || !Aligned(p.resid16_lo, 2)))
    return fail("split residual planes must be 2-byte aligned");
  if (p.split_n < p.N && (!p.C2 || p.ldc2 < p.N - p.split_n || p.split_n % 4))
    return fail("split output needs C2 wide enough and split_n % 4 == 0");
  if (p.split_n < p.N && (p.C_lo != nullptr) != (p.C2_lo != nullptr))
    return fail("split output needs lo planes for both parts or neither");
  if (p.ldc < (p.split_n < p.N ? p.split_n : p.N))
    return fail("ldc too small");
  // Folded LayerNorm (see GemmParams): consumer and residual sides.
  const bool ln_res = p.out_mode == GEMM_OUT_RESID_F32 && (p.out_gamma || p.res_stats);
  if (p.fold_c && (!p.ln_stats || p.out_mode == GEMM_OUT_RESID_F32 || p.ln_width != p.K ||
                   (p.ln_part != 64 && p.ln_part != 128) || p.K % (2 * p.ln_part) ||
                   p.K > 128 * p.ln_part ||
                   !Aligned(p.fold_c, 16) ||
                   !Aligned(p.ln_stats, 16) || p.k_splits != 1))
    return fail("folded LayerNorm consumer: ln_stats, fold_c (16-byte aligned), ln_part 64 or "
                "128, K = ln_width a multiple of 2 ln_part up to 128 ln_part, one K slice, not "
                "the residual mode");
  if ((p.out_gamma || p.res_stats) && !ln_res)
    return fail("folded LayerNorm output / residual: residual mode only");
  if (ln_res && (!p.resid16 || p.k_splits != 1 || p.ln_width != p.N ||
                 (p.ln_part != 64 && p.ln_part != 128) || p.N % (2 * p.ln_part) ||
                 p.N > 128 * p.ln_part ||
                 (p.res_stats && (!p.res_gamma || !p.res_beta || !Aligned(p.res_stats, 16) ||
                                  !Aligned(p.res_gamma, 16) || !Aligned(p.res_beta, 16))) ||
                 (p.out_gamma && (!p.out_stats || !Aligned(p.out_gamma, 16) ||
                                  !Aligned(p.out_stats, 8) || !p.C_lo))))
    return fail("folded LayerNorm residual: split residual, one K slice, ln_part 64 or 128, "
                "N = ln_width a multiple of 2 ln_part up to 128 ln_part, gamma / beta / stats "
                "16-byte aligned, a bf16 lo output plane with out_gamma");
  if (p.C_lo8 && !(p.out_mode == GEMM_OUT_RESID_F32 && p.out_gamma) &&
      (p.out_mode != GEMM_OUT_BF16 || p.C_lo || p.split_n < p.N || p.k_splits != 1 ||
       p.ldc8 < p.N || p.ldc8 % 8 || !Aligned(p.C_lo8, 8)))
    return fail("e4m3 lo output: bf16 mode, one output, no bf16 lo plane, ldc8 >= N, "
                "ldc8 % 8 == 0, 8-byte aligned");
  if (p.C_lo8 && p.out_gamma && (p.ldc8 < p.N || p.ldc8 % 8 || !Aligned(p.C_lo8, 8)))
    return fail("e4m3 lo output: ldc8 >= N, ldc8 % 8 == 0, 8-byte aligned");
  // Vector (4-column) stores need every output row start aligned to 4
  // elements' width; otherwise the epilogue stores element by element.
  const bool f32 = (p.out_mode != GEMM_OUT_BF16 && !p.out_gamma) || p.k_splits > 1;
  const std::uintptr_t vb = f32 ? 16 : 8;
  p.vec = Aligned(p.C, vb) && p.ldc % 4 == 0 && (!p.C_lo || Aligned(p.C_lo, vb)) &&
          (p.split_n >= p.N ||
           (Aligned(p.C2, vb) && p.ldc2 % 4 == 0 && (!p.C2_lo || Aligned(p.C2_lo, vb)))) &&
          (p.out_mode != GEMM_OUT_RESID_F32 ||
           (p.ldr % 4 == 0 && (p.resid16 ? Aligned(p.resid16, 8) && Aligned(p.resid16_lo, 8)
                                          : Aligned(p.resid, 16))));
  // Eight-column groups with 16-byte accesses (staged epilogue).
  const bool out_bf16 = p.out_mode == GEMM_OUT_BF16 || p.out_gamma;
  const int gcols = out_bf16 ? 8 : 4;  // elements per 16 bytes
  p.vec8 = p.vec && Aligned(p.C, 16) && p.ldc % gcols == 0 &&
           (!p.C_lo || Aligned(p.C_lo, 16)) &&
           (p.split_n >= p.N || (p.split_n % 8 == 0 && Aligned(p.C2, 16) &&
                                 p.ldc2 % gcols == 0 && (!p.C2_lo || Aligned(p.C2_lo, 16)))) &&
           (!p.bias || Aligned(p.bias, 16)) && (!p.wscale || Aligned(p.wscale, 16)) &&
           (p.out_mode != GEMM_OUT_RESID_F32 ||
            (p.resid16 ? Aligned(p.resid16, 16) && Aligned(p.resid16_lo, 16) && p.ldr % 8 == 0
                       : Aligned(p.resid, 16) && p.ldr % 4 == 0));
  // fp8 lo correction: 256 x 256 tiles of eight waves, the hi pass on the
  // four-stage single-bf16 pipelined ring (128 KiB), then the lo pass on two
  // 64 KiB stages of code rows.
  // A folded LayerNorm: only the instances that compile its epilogue.
  if (p.fold_c || ln_res) {
    switch (LnFoldTile(p)) {
    case LnTile::kLo8:
      return LaunchW<256, 256, 32, 4, 4, 2, false, false, false, true, true>(p, stream);
    case LnTile::k256Beside:
      return LaunchW<256, 256, 32, 2, 4, 2, true, false, false, true>(p, stream);
    case LnTile::k256:
      return LaunchW<256, 256, 32, 3, 4, 2, true, false, false, true>(p, stream);
    case LnTile::k256x128:
      return LaunchW<256, 128, 32, 2, 4, 2, true, false, false, true>(p, stream);
    case LnTile::k64:
      return LaunchW<64, 64, 32, 2, 2, 2, true, false>(p, stream);
    case LnTile::k64x64:
      return LaunchW<64, 64, 64, 2, 2, 2, true, false>(p, stream);
    case LnTile::kSplitK:
      if (!Aligned(p.partials, 16) || !p.vec || p.N % 4)
        return fail("folded LayerNorm split over K: 16-byte aligned partials, vector stores");
      break;  // the split-K launch below, its reduce applying the LayerNorm
    default:
      return fail("folded LayerNorm: split-precision activations, bf16 weights, one K slice, "
                  "K % 64 == 0 and N a multiple of 256 (residual, BF16X2_FP8LO codes) or "
                  "128 (or small-LDS tiles)");
    }
  }
  if (lo8)
    return LaunchW<256, 256, 32, 4, 4, 2, false, false, false, true, true>(p, stream);
  const bool split = p.A_lo != nullptr;
  const bool large = p.M >= kLargeRows && p.N >= 128;
  // Small problems (few positions): 64 x 64 tiles leave most CUs idle and
  // walk K serially, so the launcher splits K (GemmAutoSplits), writes fp32
  // partials to p.partials through a three-stage ring and sums them in
  // slice order in a second kernel that applies the epilogue.  The split depends on the shape
  // only: a batch size always takes the same path and gives the same bits.
  if (!large && !ln_res && p.k_splits == 1 && p.partials && Aligned(p.partials, 16) && p.vec &&
      p.N % 4 == 0) {
    const int splits = GemmAutoSplits(p);
    if (splits > 1) {
      GemmParams q = p;
      q.bias = nullptr;
      q.act = ACT_NONE;
      q.out_mode = GEMM_OUT_F32;
      q.C = p.partials;
      q.C_lo = q.C2 = q.C2_lo = nullptr;
      q.ldc = p.N;
      q.split_n = 1 << 30;
      q.resid = nullptr;
      q.fold_c = q.ln_stats = nullptr;  // plain sums of x o gamma
      q.k_splits = splits;
      q.vec = true;
      const bool small = p.small_lds && !p.W8;
      const hipError_t e = small ? (split ? Launch<64, 64, 32, 2, 2, 2, true>(q, stream)
                                          : Launch<64, 64, 32, 2, 2, 2, false>(q, stream))
                           : split ? Launch<64, 64, 64, 3, 2, 2, true>(q, stream)
                                   : Launch<64, 64, 64, 3, 2, 2, false>(q, stream);
      if (e != hipSuccess)
        return e;
      // The partials already carry the fp8 row scale.
      GemmParams r = p;
      r.wscale = nullptr;
      return Reduce(r, p.partials, splits, stream);
    }
  }
  if (p.fold_c)
    return fail("folded LayerNorm: no tile for this shape");
  const int kslice = p.K / p.k_splits;
  // Tile choice measured on MI355X at the BT4 body shapes (M = 16384): for
  // K <= 1024, eight waves per workgroup on BK = 32 steps (split precision
  // 128 x 128 tiles as 2 x 4 waves with two 48 KiB stages, bf16 256 x 128
  // tiles as 4 x 2 waves with three 24 KiB stages); for longer K, four waves
  // on BK = 64 (split 64 x 128, bf16 128 x 128).
  // Whole rounds of 256 workgroups: 256 x 256 tiles of eight waves (4 x 2,
  // 64 x 128 per wave) and a three-stage (split) or four-stage (bf16) LDS
  // ring, 144 / 128 KiB, one workgroup per CU.  They halve the L2 traffic
  // per MFMA of the 128-wide tiles; measured faster in the forward on the
  // out-projection, FFN2 and smolgen-global shapes, slower on QKV (832 tiles,
  // a partial last round) and FFN1 (384).  bf16 weights only (the fp8 path
  // keeps two stages).
  const long big_tiles = static_cast<long>((p.M + 255) / 256) * ((p.N + 255) / 256);
  if (f8)
    return big_tiles % 256 == 0 ? LaunchW<256, 256, 64, 2, 4, 2, false, false, true>(p, stream)
                                : LaunchW<128, 128, 64, 2, 2, 4, false, false, true>(p, stream);
  if (GemmWholeRoundTiles(p)) {
    // fp8 weights too: their e4m3 rows share the ring (40 / 24 KiB stages).
    if (p.W8)
      return split ? LaunchW<256, 256, 32, 3, 4, 2, true, true>(p, stream)
                   : LaunchW<256, 256, 32, 4, 4, 2, false, true>(p, stream);
    // Beside the smolgen chain (Q|K|V at large batches): two stages, so
    // the chain's small-LDS tiles run on the same CUs instead of waiting for
    // a round of these tiles to end (batch 256 forward 23.01k -> 23.55k
    // positions/s with the chain on small-LDS tiles; two stages alone
    // 23.15k, batch 1024 unchanged).
    // bf16 weights: the software-pipelined main loop (PipelinedLoop).
    // Isolated at batch 256, split precision: Q|K|V 223 -> 209 us, the
    // out-projection 76.7 -> 70.7, FFN2 103.8 -> 93.6; single bf16 Q|K|V
    // 112 -> 104; the batch-256 forward 23.15k -> 23.64k positions/s
    // (bit-equal outputs: the MFMAs accumulate in the same order).
    if (p.beside_chain && split)
      return LaunchW<256, 256, 32, 2, 4, 2, true, false, false, true>(p, stream);
    return split ? LaunchW<256, 256, 32, 3, 4, 2, true, false, false, true>(p, stream)
                 : LaunchW<256, 256, 32, 4, 4, 2, false, false, false, true>(p, stream);
  }
  // Split precision with fewer 128 x 128 tiles than CUs (the out-projection
  // and FFN at M = 2048 .. 3072): 64 x 64 tiles, four times the workgroups
  // (out-projection at M = 2048: 13.5 instead of 25.4 us; batch 32 forward
  // 3.02 -> 2.78 ms).  64 x 128 tiles between one and three rounds were
  // faster in isolated launches but 2 % slower in the forward at batches 64
  // and 96, so those keep 128 x 128.
  const long tiles128 = static_cast<long>((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (large && kslice % 64 == 0) {
    if (split && tiles128 < 256)
      return Launch<64, 64, 64, 2, 2, 2, true>(p, stream);
    if (kslice <= 1024 && split && !p.W8) {
      // 256 x 128 tiles (eight 64 x 64 waves, two 40 KiB stages, two
      // workgroups per CU) read 12 LDS fragments per 32 MFMAs, 128 x 128
      // tiles 10 per 16; a 256 x 128 tile costs ~1.8 times a 128 x 128
      // one, so it is taken when its rounds of 256 workgroups cost less and
      // it fills at least one round.  Below one round (FFN1 at batches 48
      // and 64, the out-projection at 96) it was 1-5 % slower, except for
      // Q|K|V at 2048 rows (batch 32), where its 192 tiles leave CUs to the
      // smolgen chain running beside it, the longer branch there.
      // Measured forward: batch 32 2.72 -> 2.61 ms, 96 5.32 -> 5.26, 128
      // 6.72 -> 6.66, 256 11.30 -> 11.16; 48 and 64 unchanged.
      const long t256 = static_cast<long>((p.M + 255) / 256) * ((p.N + 127) / 128);
      if ((t256 >= 256 || p.M <= 2048) &&
          9 * ((t256 + 255) / 256) < 5 * ((tiles128 + 255) / 256))
        return LaunchW<256, 128, 32, 2, 4, 2, true, false, false, true>(p, stream);
    }
    // Split precision with fp8 weights: BK = 64, whose stage holds the
    // e4m3 rows in LDS (at BK = 32 the 128 x 128 stage does not split
    // evenly over the waves).
    if (kslice <= 1024)
      return split ? (p.W8 ? Launch<128, 128, 64, 2, 2, 4, true>(p, stream)
                           : Launch<128, 128, 32, 2, 2, 4, true>(p, stream))
             : p.W8 ? Launch<256, 128, 32, 2, 4, 2, false>(p, stream)
                    : LaunchW<256, 128, 32, 3, 4, 2, false, false, false, true>(p, stream);
    return split ? Launch<64, 128, 64, 2, 2, 2, true>(p, stream)
                 : Launch<128, 128, 64, 2, 2, 2, false>(p, stream);
  }
  // 64 x 64 tiles over the whole K (Q|K|V at 4-31 positions, the
  // out-projection and FFN at 16-31, the smolgen dense2 and global
  // projection at some batches): from 256 rows up, or over K >= 1024, a
  // three-stage ring keeps two K steps in flight (batch 16 forward 2.30 ->
  // 2.05 ms, batch 8 1.75 -> 1.68, batch 256 +0.9 %, batch 3 1.51 -> 1.36;
  // Q|K|V took 16.0 us at 192 rows with two stages, 11.6 us at 256 rows
  // with three); for short K at 128 rows (smolgen dense2 at batch 128,
  // beside the Q|K|V GEMM on the other stream) it was 1.7 % slower, and four
  // stages (one workgroup per CU) were slower at every batch.
  if (p.small_lds && !p.W8)
    return split ? Launch<64, 64, 32, 2, 2, 2, true>(p, stream)
                 : Launch<64, 64, 32, 2, 2, 2, false>(p, stream);
  if (kslice % 64 == 0) {
    if (p.M >= 256 || kslice >= 1024)
      return split ? Launch<64, 64, 64, 3, 2, 2, true>(p, stream)
                   : Launch<64, 64, 64, 3, 2, 2, false>(p, stream);
    return split ? Launch<64, 64, 64, 2, 2, 2, true>(p, stream)
                 : Launch<64, 64, 64, 2, 2, 2, false>(p, stream);
  }
  return split ? Launch<64, 64, 32, 2, 2, 2, true>(p, stream)
               : Launch<64, 64, 32, 2, 2, 2, false>(p, stream);
}

}  // namespace mfh

// Memory-bound row kernels: input plane expansion, LayerNorm (+ input gates)
// and the WDL value head.
#include "mfh_device.h"
#include "mfh_kernels.h"

namespace mfh {
namespace {

constexpr int kPlanes = 112;
constexpr int kSquares = 64;
constexpr int kPePlanes = 12;

// One thread per (position, square, 8-column chunk) of the embedding input,
// plus the square-major 12-plane PE input.  Unpacking follows the packed
// plane contract of reference src/nn/input_plane_packing.h:30-58: square sq
// of plane p holds values[p] when bit sq of masks[p] is set, else 0
// (cpu_network.cpp:711-731, 777-790).
__global__ void ExpandInputsKernel(const std::uint64_t *__restrict__ masks,
                                   const float *__restrict__ values, int batch,
                                   std::uint16_t *__restrict__ emb_in,
                                   std::uint16_t *__restrict__ emb_in_lo, int emb_ld,
                                   const float *__restrict__ static_pe, int pe_ch,
                                   std::uint16_t *__restrict__ pos_in) {
  const int chunks = emb_ld / 8;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const int total = batch * kSquares * chunks;
  if (idx < total) {
    const int chunk = idx % chunks;
    const int row = idx / chunks;
    const int b = row / kSquares, sq = row % kSquares;
    std::uint16_t out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int col = chunk * 8 + e;
      float v = 0.f;
      if (col < kPlanes) {
        const std::uint64_t m = masks[static_cast<size_t>(b) * kPlanes + col];
        v = ((m >> sq) & 1ull) ? values[static_cast<size_t>(b) * kPlanes + col] : 0.f;
      } else if (static_pe && col < kPlanes + pe_ch) {
        v = static_pe[sq * pe_ch + col - kPlanes];
      }
      out[e] = f32_to_bf16(v);
    }
    uint4 packed;
    packed.x = out[0] | (static_cast<std::uint32_t>(out[1]) << 16);
    packed.y = out[2] | (static_cast<std::uint32_t>(out[3]) << 16);
    packed.z = out[4] | (static_cast<std::uint32_t>(out[5]) << 16);
    packed.w = out[6] | (static_cast<std::uint32_t>(out[7]) << 16);
    *reinterpret_cast<uint4 *>(emb_in + static_cast<size_t>(row) * emb_ld + chunk * 8) =
        packed;
    if (emb_in_lo) {
      // Plane values (0/1, small integers) are exact in bf16: zero residual.
      const uint4 zero = {0u, 0u, 0u, 0u};
      *reinterpret_cast<uint4 *>(emb_in_lo + static_cast<size_t>(row) * emb_ld + chunk * 8) =
          zero;
    }
  }
  // PE input: [b][sq*12 + p] for p < 12.
  const int pos_total = batch * kSquares * kPePlanes;
  if (idx < pos_total) {
    const int p = idx % kPePlanes;
    const int sq = (idx / kPePlanes) % kSquares;
    const int b = idx / (kPePlanes * kSquares);
    const std::uint64_t m = masks[static_cast<size_t>(b) * kPlanes + p];
    const float v = ((m >> sq) & 1ull) ? values[static_cast<size_t>(b) * kPlanes + p] : 0.f;
    pos_in[idx] = f32_to_bf16(v);
  }
}

__global__ void UnpackPlanesKernel(const std::uint64_t *__restrict__ masks,
                                   const float *__restrict__ values, int batch,
                                   float *__restrict__ planes) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= batch * kPlanes * kSquares)
    return;
  const int sq = idx % kSquares;
  const int bp = idx / kSquares;
  const std::uint64_t m = masks[bp];
  planes[idx] = ((m >> sq) & 1ull) ? values[bp] : 0.f;
}

__global__ void ScatterPeKernel(const float *__restrict__ pe, int batch, int pe_ch,
                                std::uint16_t *__restrict__ emb_in,
                                std::uint16_t *__restrict__ emb_in_lo, int emb_ld) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= batch * kSquares * pe_ch)
    return;
  const int c = idx % pe_ch;
  const int row = idx / pe_ch;  // b*64 + sq, and pe is [b][sq*pe_ch + c]
  const size_t off = static_cast<size_t>(row) * emb_ld + kPlanes + c;
  const std::uint16_t hi = f32_to_bf16(pe[idx]);
  emb_in[off] = hi;
  if (emb_in_lo)
    emb_in_lo[off] = f32_to_bf16(pe[idx] - bf16_to_f32(hi));
}

// Row LayerNorm.  T threads per row (64: one wave; 256 or 1024: one
// workgroup), each holding NV groups of G (4 or 8) consecutive elements of
// the row in registers: element c = G (i T + t) + e of group i of thread t.
// The input is the
// sum of `parts` partial rows plus bias, through the activation, as produced
// by a split-K GEMM; with a residual, x = resid + alpha * (sum + bias) (the
// residual LayerNorm, reference cpu_network.cpp:1399-1457).  Statistics in
// fp32 with the reference formula var = E[x^2] - mean^2 clamped at 0,
// inv_std = 1 / sqrt(var + eps) (cpu_network.cpp:424-460).  Loads are 16
// bytes, bf16 stores 2G bytes per lane.  Each element is read and written by
// the same thread, so the output may alias the residual.

template <int T, int NV, int G = 4>
__global__ __launch_bounds__(T > 256 ? T : 256) void LayerNormKernel(LayerNormParams lp) {
  constexpr int kBlock = T > 256 ? T : 256;
  constexpr int kRowsPerBlock = kBlock / T;
  constexpr int kWaves = T / 64;
  constexpr int Q = G / 4;  // float4 vectors per group
  static_assert(G == 4 || G == 8, "groups of 4 or 8 elements");
  __shared__ float red[2][kWaves > 4 ? kWaves : 4];
  const int t = threadIdx.x % T;
  const int row = blockIdx.x * kRowsPerBlock + threadIdx.x / T;
  const bool active = row < lp.rows;
  const int width = lp.width;
  const size_t plane = static_cast<size_t>(lp.rows) * width;
  const size_t row_off = static_cast<size_t>(row) * width;
  f32x4 v[NV][Q];
  float s = 0.f, ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c0 = G * (i * T + t);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int c = c0 + 4 * q;
      f32x4 x = f32x4{0.f, 0.f, 0.f, 0.f};
      if (active && c0 < width) {
        // Part loads go out 16 at a time in the variants that sum split-K
        // parts (256+ threads per row, or one wave with at most two
        // 4-element groups per lane), 4 at a time otherwise.
        x = sum_parts4<(T >= 256 || (G == 4 && NV <= 2)) ? 16 : 4>(lp.x + row_off + c, plane,
                                                                    lp.parts);
        if (lp.bias)
          x += *reinterpret_cast<const f32x4 *>(lp.bias + c);
        if (lp.resid) {
          const f32x4 r = *reinterpret_cast<const f32x4 *>(lp.resid + row_off + c);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            x[e] = r[e] + lp.alpha * x[e];
        } else if (lp.resid16) {
          const u32x2 h = *reinterpret_cast<const u32x2 *>(lp.resid16 + row_off + c);
          const u32x2 l = *reinterpret_cast<const u32x2 *>(lp.resid16_lo + row_off + c);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const unsigned hw = h[e >> 1], lw = l[e >> 1];
            const float r = __uint_as_float((e & 1) ? (hw & 0xFFFF0000u) : (hw << 16)) +
                            __uint_as_float((e & 1) ? (lw & 0xFFFF0000u) : (lw << 16));
            x[e] = r + lp.alpha * x[e];
          }
        }
        if (lp.act != ACT_NONE) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            x[e] = activate(x[e], lp.act);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s += x[e];
          ss += x[e] * x[e];
        }
      }
      v[i][q] = x;
    }
  }
  // gamma / beta are independent of the statistics: fetch them before the
  // reductions so their latency overlaps.
  f32x4 gm[NV][Q], bt[NV][Q];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c0 = G * (i * T + t);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      if (c0 < width) {
        gm[i][q] = *reinterpret_cast<const f32x4 *>(lp.gamma + c0 + 4 * q);
        bt[i][q] = *reinterpret_cast<const f32x4 *>(lp.beta + c0 + 4 * q);
      }
    }
  }
  s = wave_sum(s);
  ss = wave_sum(ss);
  if (T >= 256) {
    if ((threadIdx.x & 63) == 0) {
      red[0][threadIdx.x >> 6] = s;
      red[1][threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    s = 0.f;
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      s += red[0][w];
      ss += red[1][w];
    }
  }
  if (!active)
    return;
  const float mean = s / static_cast<float>(width);
  float var = ss / static_cast<float>(width) - mean * mean;
  var = var < 0.f ? 0.f : var;
  const float inv_std = 1.f / sqrtf(var + lp.eps);
  const int sq = row % kSquares;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c0 = G * (i * T + t);
    if (c0 >= width)
      break;
    unsigned hi2[2 * Q], lo2[2 * Q];  // bf16 pairs of the group
    unsigned q8[Q];                    // e4m3 lo codes of the group
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int c = c0 + 4 * q;
      f32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        y[e] = (v[i][q][e] - mean) * inv_std * gm[i][q][e] + bt[i][q][e];
      // Gates [64][width], square-major: four consecutive channels.
      const size_t goff = static_cast<size_t>(sq) * width + c;
      if (lp.mult_gate) {
        const f32x4 m = *reinterpret_cast<const f32x4 *>(lp.mult_gate + goff);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = y[e] * m[e];
      }
      if (lp.add_gate) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(lp.add_gate + goff);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          y[e] = y[e] + a[e];
      }
      if (lp.y_f32)
        *reinterpret_cast<f32x4 *>(lp.y_f32 + row_off + c) = y;
      std::uint16_t hi[4], lo[4];
      float lf[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = f32_to_bf16(y[e]);
        lf[e] = y[e] - bf16_to_f32(hi[e]);
        lo[e] = f32_to_bf16(lf[e]);
      }
      q8[q] = lp.y_lo8 ? Lo8Pack4(lf[0], lf[1], lf[2], lf[3]) : 0u;
      hi2[2 * q] = hi[0] | (static_cast<unsigned>(hi[1]) << 16);
      hi2[2 * q + 1] = hi[2] | (static_cast<unsigned>(hi[3]) << 16);
      lo2[2 * q] = lo[0] | (static_cast<unsigned>(lo[1]) << 16);
      lo2[2 * q + 1] = lo[2] | (static_cast<unsigned>(lo[3]) << 16);
    }
    if (lp.y_bf16) {
      if constexpr (G == 8) {
        *reinterpret_cast<u32x4 *>(lp.y_bf16 + row_off + c0) =
            u32x4{hi2[0], hi2[1], hi2[2], hi2[3]};
        if (lp.y_bf16_lo)
          *reinterpret_cast<u32x4 *>(lp.y_bf16_lo + row_off + c0) =
              u32x4{lo2[0], lo2[1], lo2[2], lo2[3]};
      } else {
        *reinterpret_cast<u32x2 *>(lp.y_bf16 + row_off + c0) = u32x2{hi2[0], hi2[1]};
        if (lp.y_bf16_lo)
          *reinterpret_cast<u32x2 *>(lp.y_bf16_lo + row_off + c0) = u32x2{lo2[0], lo2[1]};
      }
      if (lp.y_lo8) {
        if constexpr (G == 8)
          *reinterpret_cast<u32x2 *>(lp.y_lo8 + row_off + c0) = u32x2{q8[0], q8[1]};
        else
          *reinterpret_cast<unsigned *>(lp.y_lo8 + row_off + c0) = q8[0];
      }
    }
  }
}

// Rows of bf16 activations (hi, plus the lo plane when given) as OCP e4m3
// codes with one fp32 scale per row: scale = max|row| / 448 (1 for a zero
// row), code = e4m3(x / scale) rounded to nearest even, the quotient
// clamped to +-448 first (the host weight quantiser's arithmetic).  One wave
// per row; lane l holds columns 16 (l + 64 g) .. + 15 for g < 2.
__global__ __launch_bounds__(256) void QuantizeRowsE4m3Kernel(
    const std::uint16_t *__restrict__ x, const std::uint16_t *__restrict__ x_lo, int ldx,
    int rows, int cols, std::uint8_t *__restrict__ q, int ldq, float *__restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows)
    return;
  float v[2][16];
  float mx = 0.f;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int c = 16 * (lane + 64 * g);
    if (c < cols) {
      const size_t off = static_cast<size_t>(row) * ldx + c;
      const u32x4 h0 = *reinterpret_cast<const u32x4 *>(x + off);
      const u32x4 h1 = *reinterpret_cast<const u32x4 *>(x + off + 8);
      u32x4 l0 = u32x4{0u, 0u, 0u, 0u}, l1 = l0;
      if (x_lo) {
        l0 = *reinterpret_cast<const u32x4 *>(x_lo + off);
        l1 = *reinterpret_cast<const u32x4 *>(x_lo + off + 8);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const unsigned hw = (e < 4 ? h0 : h1)[(e & 3)], lw = (e < 4 ? l0 : l1)[(e & 3)];
        v[g][2 * e] = __uint_as_float(hw << 16) + __uint_as_float(lw << 16);
        v[g][2 * e + 1] = __uint_as_float(hw & 0xFFFF0000u) + __uint_as_float(lw & 0xFFFF0000u);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e)
        mx = fmaxf(mx, fabsf(v[g][e]));
    }
  }
  mx = wave_max(mx);
  const float s = mx > 0.f ? mx / 448.0f : 1.0f;
  if (lane == 0)
    scale[row] = s;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int c = 16 * (lane + 64 * g);
    if (c < cols) {
      unsigned w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          t[e] = fminf(fmaxf(v[g][4 * k + e] / s, -448.0f), 448.0f);
        int packed = __builtin_amdgcn_cvt_pk_fp8_f32(t[0], t[1], 0, false);
        packed = __builtin_amdgcn_cvt_pk_fp8_f32(t[2], t[3], packed, true);
        w[k] = static_cast<unsigned>(packed);
      }
      *reinterpret_cast<u32x4 *>(q + static_cast<size_t>(row) * ldq + c) =
          u32x4{w[0], w[1], w[2], w[3]};
    }
  }
}

// One wave per position: dense2 (vh -> 3 or 1) then softmax or tanh
// (reference network_execution_plan.cpp:1098-1106, cpu_network.cpp:336-351).
__global__ __launch_bounds__(256) void ValueHeadKernel(
    const float *__restrict__ hidden, int parts, const float *__restrict__ b1, int act,
    int batch, int vh, const float *__restrict__ w2, const float *__restrict__ b2, int mode,
    float *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= batch)
    return;
  const int outs = mode == kHeadSoftmax3 ? 3 : 1;
  const float *h = hidden + static_cast<size_t>(b) * vh;
  float acc[3] = {0.f, 0.f, 0.f};
  const size_t plane = static_cast<size_t>(batch) * vh;
  for (int c = lane; c < vh; c += 64) {
    float v = sum_parts1(h + c, plane, parts);
    if (b1)
      v += b1[c];
    v = activate(v, act);
    for (int o = 0; o < outs; ++o)
      acc[o] += v * w2[static_cast<size_t>(o) * vh + c];
  }
  for (int o = 0; o < outs; ++o)
    acc[o] = wave_sum(acc[o]) + b2[o];
  if (lane != 0)
    return;
  if (mode == kHeadSoftmax3) {
    const float m = fmaxf(acc[0], fmaxf(acc[1], acc[2]));
    const float e0 = expf(acc[0] - m), e1 = expf(acc[1] - m), e2 = expf(acc[2] - m);
    const float inv = 1.f / (e0 + e1 + e2);
    out[static_cast<size_t>(b) * 3 + 0] = e0 * inv;
    out[static_cast<size_t>(b) * 3 + 1] = e1 * inv;
    out[static_cast<size_t>(b) * 3 + 2] = e2 * inv;
  } else if (mode == kHeadRelu) {
    out[b] = activate(acc[0], ACT_RELU);
  } else {
    out[b] = tanhf(acc[0]);
  }
}

std::string Fail(std::string *err, const char *what) {
  if (err)
    *err = what;
  return what;
}

}  // namespace

hipError_t LaunchExpandInputs(const std::uint64_t *masks, const float *values,
                              int batch, std::uint16_t *emb_in, std::uint16_t *emb_in_lo,
                              int emb_ld, const float *static_pe, int pe_ch,
                              std::uint16_t *pos_in, hipStream_t stream, std::string *err) {
  if (batch <= 0 || emb_ld % 8 || emb_ld < kPlanes || !masks || !values || !emb_in ||
      !pos_in || (reinterpret_cast<std::uintptr_t>(emb_in) & 15u) ||
      (static_pe && (pe_ch <= 0 || kPlanes + pe_ch > emb_ld))) {
    Fail(err, "expand_inputs: invalid arguments");
    return hipErrorInvalidValue;
  }
  const int total = batch * kSquares * (emb_ld / 8);
  const int pos_total = batch * kSquares * kPePlanes;
  const int n = total > pos_total ? total : pos_total;
  hipLaunchKernelGGL(ExpandInputsKernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                     masks, values, batch, emb_in, emb_in_lo, emb_ld, static_pe, pe_ch, pos_in);
  return hipGetLastError();
}

hipError_t LaunchUnpackPlanes(const std::uint64_t *masks, const float *values,
                              int batch, float *planes, hipStream_t stream,
                              std::string *err) {
  if (batch <= 0 || !masks || !values || !planes) {
    Fail(err, "unpack_planes: invalid arguments");
    return hipErrorInvalidValue;
  }
  const int n = batch * kPlanes * kSquares;
  hipLaunchKernelGGL(UnpackPlanesKernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                     masks, values, batch, planes);
  return hipGetLastError();
}

hipError_t LaunchScatterPe(const float *pe, int batch, int pe_channels,
                           std::uint16_t *emb_in, std::uint16_t *emb_in_lo, int emb_ld,
                           hipStream_t stream, std::string *err) {
  if (batch <= 0 || pe_channels <= 0 || kPlanes + pe_channels > emb_ld || !pe || !emb_in) {
    Fail(err, "scatter_pe: invalid arguments");
    return hipErrorInvalidValue;
  }
  const int n = batch * kSquares * pe_channels;
  hipLaunchKernelGGL(ScatterPeKernel, dim3((n + 255) / 256), dim3(256), 0, stream, pe,
                     batch, pe_channels, emb_in, emb_in_lo, emb_ld);
  return hipGetLastError();
}

hipError_t LaunchLayerNorm(const LayerNormParams &lp, hipStream_t stream, std::string *err) {
  if (lp.rows <= 0 || lp.width <= 0 || lp.parts < 1 || !lp.x || !lp.gamma || !lp.beta ||
      (!lp.y_f32 && !lp.y_bf16)) {
    Fail(err, "layernorm: invalid arguments");
    return hipErrorInvalidValue;
  }
  if ((lp.resid && lp.resid16) || (lp.resid16 != nullptr) != (lp.resid16_lo != nullptr) ||
      ((lp.resid || lp.resid16) && lp.act != ACT_NONE)) {
    Fail(err, "layernorm: residual is fp32 or a hi + lo pair, without an activation");
    return hipErrorInvalidValue;
  }
  if ((lp.mult_gate || lp.add_gate) && lp.rows % kSquares) {
    Fail(err, "layernorm: gates need square rows");
    return hipErrorInvalidValue;
  }
  auto aligned = [](const void *p, std::uintptr_t a) {
    return (reinterpret_cast<std::uintptr_t>(p) & (a - 1)) == 0;
  };
  if (lp.width % 4 || !aligned(lp.x, 16) || (lp.bias && !aligned(lp.bias, 16)) ||
      !aligned(lp.gamma, 16) || !aligned(lp.beta, 16) || (lp.y_f32 && !aligned(lp.y_f32, 16)) ||
      (lp.y_bf16 && !aligned(lp.y_bf16, 8)) || (lp.y_bf16_lo && !aligned(lp.y_bf16_lo, 8)) ||
      (lp.y_lo8 && (!lp.y_bf16 || !aligned(lp.y_lo8, 8))) ||
      (lp.resid && !aligned(lp.resid, 16)) ||
      (lp.resid16 && (!aligned(lp.resid16, 8) || !aligned(lp.resid16_lo, 8))) ||
      (lp.mult_gate && !aligned(lp.mult_gate, 16)) || (lp.add_gate && !aligned(lp.add_gate, 16))) {
    Fail(err, "layernorm: width % 4 == 0 and 16-byte aligned rows required");
    return hipErrorInvalidValue;
  }
  // The thread count per row depends on the width and the number of split-K
  // parts only, so at one batch size a row's reduction order (and result
  // bits) never changes.  Rows that sum split-K parts (few positions) take
  // 256 threads per row, so the part loads spread over more lanes.
  // One wave per row with 8-element groups (16-byte bf16 stores) when the
  // width is a whole number of 512-element chunks and rows are 16-byte
  // aligned in every bf16 output.
  const bool g8 = lp.width % 512 == 0 && lp.width <= 2048 && lp.parts == 1 &&
                  (!lp.y_bf16 || aligned(lp.y_bf16, 16)) &&
                  (!lp.y_bf16_lo || aligned(lp.y_bf16_lo, 16)) &&
                  (!lp.resid16 || (aligned(lp.resid16, 16) && aligned(lp.resid16_lo, 16)));
  const int nv64 = (lp.width + 255) / 256;      // float4s per lane, one wave per row
  const int nv256 = (lp.width + 1023) / 1024;   // float4s per lane, 256 threads per row
  const int nv1024 = (lp.width + 4095) / 4096;  // float4s per lane, 1024 threads per row
  const dim3 g64((lp.rows + 3) / 4), g256(lp.rows), blk(256);
  if (lp.parts > 1 && nv256 <= 1 && lp.width > 256)
    hipLaunchKernelGGL((LayerNormKernel<256, 1>), g256, blk, 0, stream, lp);
  else if (lp.parts > 1 && nv256 <= 2 && lp.width > 256)
    hipLaunchKernelGGL((LayerNormKernel<256, 2>), g256, blk, 0, stream, lp);
  else if (g8 && lp.width == 512)
    hipLaunchKernelGGL((LayerNormKernel<64, 1, 8>), g64, blk, 0, stream, lp);
  else if (g8 && lp.width == 1024)
    hipLaunchKernelGGL((LayerNormKernel<64, 2, 8>), g64, blk, 0, stream, lp);
  else if (g8)
    hipLaunchKernelGGL((LayerNormKernel<64, 4, 8>), g64, blk, 0, stream, lp);
  else if (nv64 <= 1)
    hipLaunchKernelGGL((LayerNormKernel<64, 1>), g64, blk, 0, stream, lp);
  else if (nv64 <= 2)
    hipLaunchKernelGGL((LayerNormKernel<64, 2>), g64, blk, 0, stream, lp);
  else if (nv64 <= 4)
    hipLaunchKernelGGL((LayerNormKernel<64, 4>), g64, blk, 0, stream, lp);
  else if (nv64 <= 8)
    hipLaunchKernelGGL((LayerNormKernel<64, 8>), g64, blk, 0, stream, lp);
  else if (nv256 <= 4)
    hipLaunchKernelGGL((LayerNormKernel<256, 4>), g256, blk, 0, stream, lp);
  else if (nv1024 <= 2)
    hipLaunchKernelGGL((LayerNormKernel<1024, 2>), g256, dim3(1024), 0, stream, lp);
  else {
    Fail(err, "layernorm: row wider than 8192");
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t LaunchValueHead(const float *hidden, int parts, const float *b1, int act,
                           int batch, int vh, const float *w2, const float *b2, int mode,
                           float *out, hipStream_t stream, std::string *err) {
  if (batch <= 0 || vh <= 0 || parts < 1 || !hidden || !w2 || !b2 || !out ||
      (mode != kHeadTanh && mode != kHeadSoftmax3 && mode != kHeadRelu)) {
    Fail(err, "value_head: invalid arguments");
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(ValueHeadKernel, dim3((batch + 3) / 4), dim3(256), 0, stream, hidden,
                     parts, b1, act, batch, vh, w2, b2, mode, out);
  return hipGetLastError();
}

hipError_t LaunchQuantizeRowsE4m3(const std::uint16_t *x, const std::uint16_t *x_lo, int ldx,
                                  int rows, int cols, std::uint8_t *q, int ldq, float *scale,
                                  hipStream_t stream, std::string *err) {
  if (!x || !q || !scale || rows < 1 || cols < 16 || cols % 16 || cols > 2048 || ldx < cols ||
      ldx % 8 || ldq < cols || ldq % 16 || (reinterpret_cast<std::uintptr_t>(x) & 15) ||
      (x_lo && (reinterpret_cast<std::uintptr_t>(x_lo) & 15)) ||
      (reinterpret_cast<std::uintptr_t>(q) & 15)) {
    if (err)
      *err = "quantize rows: 16 <= cols <= 2048, cols % 16 == 0, 16-byte aligned rows";
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(QuantizeRowsE4m3Kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, x, x_lo,
                     ldx, rows, cols, q, ldq, scale);
  return hipGetLastError();
}

}  // namespace mfh

// Shared device-side definitions for the gfx950 kernels of libmfhip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "mfh_kernels.h"

namespace mfh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_to_f32(std::uint16_t h) {
  return __uint_as_float(static_cast<std::uint32_t>(h) << 16);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// bf16 rounding to nearest even on gfx950's v_cvt_pk_bf16_f32, two values
// per instruction (a software rounding, add 0x7FFF plus the kept lsb and
// shift, took three instructions per value).  The same bits for finite
// inputs, denormals included (checked on the device against the integer
// rounding).
__device__ __forceinline__ std::uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(std::uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

__device__ __forceinline__ std::uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(std::uint16_t, static_cast<__bf16>(f));
}

// Two values as bf16 hi + lo pairs (hi = bf16(v), lo = bf16(v - hi)),
// packed low-first: one word of hi parts, one of lo parts.
__device__ __forceinline__ void split_bf16x2(float a, float b, std::uint32_t &hi,
                                             std::uint32_t &lo) {
  hi = pack_bf16x2(a, b);
  lo = pack_bf16x2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

// Activations (reference src/nn/cpu/cpu_network.cpp:302-323).  Mish uses the
// identity tanh(log1p(e^x)) = n / (n + 2) with n = e^x (e^x + 2), which needs
// one exponential; for x > 20 the ratio is 1 to fp32 precision.
__device__ __forceinline__ float activate(float x, int act) {
  switch (act) {
  case ACT_RELU:
    return x > 0.f ? x : 0.f;
  case ACT_RELU2: {
    const float r = x > 0.f ? x : 0.f;
    return r * r;
  }
  case ACT_TANH:
    return tanhf(x);
  case ACT_SIGMOID:
    return 1.f / (1.f + __expf(-x));
  case ACT_SWISH:
    return x / (1.f + __expf(-x));
  case ACT_MISH: {
    if (x > 20.f)
      return x;
    const float e = __expf(x);
    const float n = e * (e + 2.f);
    return x * __fdividef(n, n + 2.f);
  }
  case ACT_SELU:
    return 1.05070098f * (x > 0.f ? x : 1.67326324f * (__expf(x) - 1.f));
  default:
    return x;
  }
}

// Activation with a compile-time kind; ACT_RUNTIME defers to the runtime
// id passed as the second argument.
constexpr int ACT_RUNTIME = -2;
template <int ACT>
__device__ __forceinline__ float Act(float v, int runtime_act) {
  if constexpr (ACT == ACT_RUNTIME)
    return activate(v, runtime_act);
  else
    return activate(v, ACT);
}

// Eight OCP e4m3 codes (bytes of q, lowest first) as eight bf16 values;
// exact, since every e4m3 value is a bf16 value.
__device__ __forceinline__ bf16x8 Fp8x8ToBf16(u32x2 q) {
  const auto a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, false);
  const auto b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, true);
  const auto c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, false);
  const auto d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Eight e4m3 lo codes (bytes of q, lowest first: e4m3(lo * 2^kLo8Shift)) as
// the eight bf16 lo values; exact (an e4m3 value times a power of two is a
// bf16 value), the conversion applying the power-of-two scale.
__device__ __forceinline__ bf16x8 Lo8x8ToBf16(u32x2 q) {
  constexpr float kInv = 1.0f / static_cast<float>(1 << kLo8Shift);
  const auto a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], kInv, false);
  const auto b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], kInv, true);
  const auto c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], kInv, false);
  const auto d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], kInv, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// e4m3 codes of four lo parts scaled by 2^kLo8Shift (the BF16X2_FP8LO
// activation lo plane), round to nearest even, clamped to +-448 first.
__device__ __forceinline__ unsigned Lo8Pack4(float a, float b, float c, float d) {
  constexpr float kScale = static_cast<float>(1 << kLo8Shift);
  const auto q = [](float x) { return fminf(fmaxf(x * kScale, -448.0f), 448.0f); };
  int packed = __builtin_amdgcn_cvt_pk_fp8_f32(q(a), q(b), 0, false);
  packed = __builtin_amdgcn_cvt_pk_fp8_f32(q(c), q(d), packed, true);
  return static_cast<unsigned>(packed);
}

// Generic pointer to LDS memory as the address-space-3 pointer that the
// direct global->LDS load builtin takes.
#define MFH_LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

// Sum of the split-K partials x[0], x[stride], ..., x[(parts - 1) * stride]
// added in that order (a fixed order, whatever the launch shape), with the
// loads of each run of B parts issued together: partials written by
// workgroups on other XCDs come from HBM, and one dependent load per part
// would serialise those misses.
template <int B = 16>
__device__ __forceinline__ f32x4 sum_parts4(const float *x, size_t stride, int parts) {
  f32x4 a = *reinterpret_cast<const f32x4 *>(x);
  for (int k0 = 1; k0 < parts; k0 += B) {
    f32x4 v[B];
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (k0 + j < parts)
        v[j] = *reinterpret_cast<const f32x4 *>(x + (k0 + j) * stride);
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (k0 + j < parts)
        a += v[j];
  }
  return a;
}

template <int B = 16>
__device__ __forceinline__ float sum_parts1(const float *x, size_t stride, int parts) {
  float a = x[0];
  for (int k0 = 1; k0 < parts; k0 += B) {
    float v[B];
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (k0 + j < parts)
        v[j] = x[(k0 + j) * stride];
#pragma unroll
    for (int j = 0; j < B; ++j)
      if (k0 + j < parts)
        a += v[j];
  }
  return a;
}

// Wave-wide (64 lanes) reductions.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
    v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace mfh

// Folded activations on the device, numbered as the plan's `Fused` codes
// (src/engine/plan.rs:148-175): 0 none, 1 ReLU, 2 sigmoid, 3 GELU, 4 swish,
// 5 hard sigmoid, 6 the neck's hard sigmoid, and this backend's 7, hard swish.
//
// The library is compiled with -ffp-contract=off: every fused multiply-add
// below is an explicit fmaf, every other product and sum rounds on its own,
// as in the engine's tier-3 CPU arithmetic (src/engine/kernels/activation.rs:
// 10-60, 151-159; src/engine/layers.rs:20-72, 212-226). Division and sqrt
// are correctly rounded (clang's default for HIP), so each activation gives
// the CPU's bits for the same input.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ppocr {

enum Act : int {
  ACT_NONE = 0, ACT_RELU = 1, ACT_SIGMOID = 2, ACT_GELU = 3, ACT_SWISH = 4,
  ACT_HARDSIGMOID = 5, ACT_HARDSIGMOIDFIFTH = 6, ACT_HARDSWISH = 7,
};

__device__ __forceinline__ float bits_f(uint32_t b) { return __uint_as_float(b); }

// exp(z) for z <= 0, XNNPACK's f32-vsigmoid p5 with one-FMA reduction.
__device__ __forceinline__ float exp_neg(float z) {
  const float magic = bits_f(0x4b40007fu);
  float n = fmaf(z, bits_f(0x3fb8aa3bu), magic);
  float s = __uint_as_float(__float_as_uint(n) << 23);
  n = n - magic;
  float t = fmaf(n, bits_f(0xbf317218u), z);
  float p = fmaf(bits_f(0x3c07cfceu), t, bits_f(0x3d2b9d0du));
  p = fmaf(p, t, bits_f(0x3e2aad40u));
  p = fmaf(p, t, bits_f(0x3efffee3u));
  p = fmaf(p, t, bits_f(0x3f7ffffbu));
  if (z < bits_f(0xc2aeac4fu)) return 0.0f;
  return fmaf(t * s, p, s);
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) {
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

__device__ __forceinline__ float sigmoid(float x) {
  uint32_t u = __float_as_uint(x);
  float e = exp_neg(__uint_as_float(u | 0x80000000u));
  float f = e / (e + 1.0f);
  return (u & 0x80000000u) ? f : 1.0f - f;
}

__device__ __forceinline__ float gelu(float x) {
  float c = clampf(x, -5.5f, 5.5f);
  float s = c * c;
  float p = bits_f(0x32c36a3cu);
  p = fmaf(p, s, bits_f(0x36d52462u));
  p = fmaf(p, s, bits_f(0x39310738u));
  p = fmaf(p, s, bits_f(0x3b9943c9u));
  p = fmaf(p, s, bits_f(0x3d0aa93cu));
  p = fmaf(p, s, bits_f(0x3ecc4228u));
  float q = bits_f(0x35a0b9e3u);
  q = fmaf(q, s, bits_f(0x389a737au));
  q = fmaf(q, s, bits_f(0x3af6ffc6u));
  q = fmaf(q, s, bits_f(0x3ceaaaeeu));
  q = fmaf(q, s, bits_f(0x3e80c788u));
  q = fmaf(q, s, 1.0f);
  return x * clampf(fmaf(c, p / q, 0.5f), 0.0f, 1.0f);
}

__device__ __forceinline__ float act(float v, int a) {
  switch (a) {
    case ACT_RELU: return v < 0.0f ? 0.0f : v;
    case ACT_SIGMOID: return sigmoid(v);
    case ACT_GELU: return gelu(v);
    case ACT_SWISH: return v * sigmoid(v);
    case ACT_HARDSIGMOID: return clampf(v * bits_f(0x3e2aaaadu) + 0.5f, 0.0f, 1.0f);
    case ACT_HARDSIGMOIDFIFTH: return clampf(v * 0.2f + 0.5f, 0.0f, 1.0f);
    case ACT_HARDSWISH: return v * clampf(v * bits_f(0x3e2aaaabu) + 0.5f, 0.0f, 1.0f);
    default: return v;
  }
}

}  // namespace ppocr

// Shared device helpers for the omniserve_amd gfx950 kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, MFMA
// 16x16x32 f16 tiles, 160 KB of LDS per CU.  No other target is supported.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "omniserve_amd.h"

#define OMNI_WAVE 64

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Error codes returned by every extern "C" entry point (0 = success).
// Positive values are hipError_t codes from the launch.
#define OMNI_OK 0
#define OMNI_EINVAL -1      // bad size / shape / null pointer
#define OMNI_EUNSUPPORTED -2 // shape outside what the kernel is built for

#define OMNI_CHECK_LAUNCH()                         \
  do {                                              \
    hipError_t _e = hipGetLastError();              \
    if (_e != hipSuccess) return (int)_e;           \
  } while (0)

// ---------------------------------------------------------------------------
// Wave-level reductions (64 lanes, xor butterfly through ds_swizzle/bpermute).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, OMNI_WAVE);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, OMNI_WAVE));
  return v;
}

// ---------------------------------------------------------------------------
// fp32 -> fp8 e4m3fn (OCP: bias 7, no infinities, max finite 448, NaN 0x7f)
// with round-to-nearest-even, in software so the rounding is fully specified.
// Magnitudes that round above 448 become NaN, matching torch's
// Float8_e4m3fn conversion (callers scale so this never happens).
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint8_t f32_to_e4m3fn(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f);  // NaN
  float af = __builtin_bit_cast(float, a);
  // Largest value that still rounds to 448 (0x7e): 464 is the midpoint to the
  // next (non-existent) step; RNE of exactly 464 goes to even -> 0x7e? 448 has
  // mantissa 110 (even is 110), so 464 rounds down to 448; above 464 -> NaN.
  if (af > 464.0f) return (uint8_t)(sign | 0x7f);
  int exp = (int)(a >> 23) - 127;           // unbiased fp32 exponent
  if (exp < -6) {
    // Subnormal range of e4m3fn: value = m * 2^-9, m in [0, 7].
    // q = af * 2^9, rounded to nearest even integer.
    float q = af * 512.0f;                  // exact (power-of-two scale)
    float r = __builtin_rintf(q);           // RNE (default rounding mode)
    uint32_t m = (uint32_t)r;               // 0..8 (8 -> smallest normal)
    return (uint8_t)(sign | m);             // m == 8 encodes 2^-6 correctly
  }
  // Normal: keep 3 mantissa bits with RNE on the dropped 20 bits.
  uint32_t mant = a & 0x7fffffu;
  uint32_t keep = mant >> 20;
  uint32_t rest = mant & 0xfffffu;
  uint32_t half = 0x80000u;
  uint32_t e = (uint32_t)(exp + 7);
  uint32_t code = (e << 3) | keep;
  if (rest > half || (rest == half && (keep & 1u))) code += 1;  // may carry into exponent
  if (code > 0x7e) return (uint8_t)(sign | 0x7f);
  return (uint8_t)(sign | code);
}

__host__ __device__ __forceinline__ float e4m3fn_to_f32(uint8_t v) {
  uint32_t s = (v & 0x80u) ? 0x80000000u : 0u;
  uint32_t e = (v >> 3) & 0xfu;
  uint32_t m = v & 0x7u;
  if (e == 0xf && m == 0x7) return __builtin_bit_cast(float, s | 0x7fc00000u);
  float mag;
  if (e == 0) mag = (float)m * (1.0f / 512.0f);
  else mag = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, mag) | s);
}

// ---------------------------------------------------------------------------
// int4 (uint4b8) dequant: one 32-bit word carries eight 4-bit codes for eight
// consecutive k of one output column.  The repacked layout stores code e at
// bit 2e (e even) or 16 + 2(e-1) (e odd), so the magic-exponent extraction
//   ((w >> 4r) & 0x000F000F) | 0x64006400   ==  (1024 + q_{2r}, 1024 + q_{2r+1})
// yields the codes in natural k order.  (1024 + q) - 1032 = q - 8 is exact in
// fp16; the multiply by the fp16 group scale rounds once (RNE), which is the
// reference's definition W = fp16((q - 8) * s).
// ---------------------------------------------------------------------------
__device__ __forceinline__ half8_t dequant8(uint32_t w, half2_t s2) {
  const half2_t bias = {(half_t)1032.0f, (half_t)1032.0f};
  half8_t out;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    uint32_t t = ((w >> (4 * r)) & 0x000F000Fu) | 0x64006400u;
    half2_t h = __builtin_bit_cast(half2_t, t);
    h = (h - bias) * s2;
    out[2 * r] = h[0];
    out[2 * r + 1] = h[1];
  }
  return out;
}

__device__ __forceinline__ f32x4 mfma16x16x32(half8_t a, half8_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__host__ __device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

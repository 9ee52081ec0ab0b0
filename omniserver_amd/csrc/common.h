// Shared device helpers for the omniserver_amd gfx950 kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, MFMA
// 16x16x32 f16 tiles, 160 KB of LDS per CU.  No other target is supported.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "omniserver_amd.h"

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
// bit 2e (e even) or 16 + 2(e-1) (e odd), so with u = w >> 8 the four fp16 pairs are
//   (w & 0x000F000F) | 0x64006400  ==  (1024 + q0, 1024 + q1)   (mantissa LSB = 1)
//   (w & 0x00F000F0) | 0x54005400  ==  (  64 + q2,   64 + q3)   (bits 4-7, ulp 1/16)
//   (u & 0x000F000F) | 0x64006400  ==  (1024 + q4, 1024 + q5)
//   (u & 0x00F000F0) | 0x54005400  ==  (  64 + q6,   64 + q7)
// in natural k order; subtracting 1032 / 72 gives q - 8 exactly in fp16, and the
// multiply by the fp16 group scale rounds once (RNE): the reference's definition
// W = fp16((q - 8) * s).  One shift, four v_and_or_b32, four packed subtracts and four
// packed multiplies per eight weights.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t and_or_b32(uint32_t x, uint32_t mask, uint32_t bits) {
  // (x & mask) | bits in one VALU op; mask from an SGPR, bits from a VGPR (the VOP3
  // encoding takes one scalar operand and no 32-bit literal).
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(bits));
  return r;
}

// SwiGLU's silu(g) * u in fp32, from the fp16 (or bf16) roundings g, u of the projections.
// The empty asm makes the product opaque: without it the backend may fold the last multiply
// and the caller's fp16 rounding into one mixed-precision fma (one rounding instead of the
// fp32 product's two), which changes near-tie results from kernel to kernel.
// The sigmoid's reciprocal is the hardware v_rcp_f32 (1 ulp): the correctly rounded division
// is 11 instructions of the 20 per output, and the GEMMs' SiLU epilogues are VALU-bound with
// the matrix cores idle; 1 ulp of fp32 moves the fp16 output only at near ties.  Every SiLU
// kernel (decode GEMVs, prefill GEMMs, the standalone SiLU-mul) uses this one helper, so
// their outputs agree bit for bit.
__device__ __forceinline__ float silu_mul_f32(float g, float u) {
#pragma clang fp contract(off)
  float p = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
  asm("" : "+v"(p));
  return p;
}

__device__ __forceinline__ half8_t dequant8(uint32_t w, half2_t s2) {
  const half2_t b_lo = {(half_t)1032.0f, (half_t)1032.0f};
  const half2_t b_hi = {(half_t)72.0f, (half_t)72.0f};
  const uint32_t u = w >> 8;
  half2_t h[4];
  h[0] = (__builtin_bit_cast(half2_t, and_or_b32(w, 0x000F000Fu, 0x64006400u)) - b_lo) * s2;
  h[1] = (__builtin_bit_cast(half2_t, and_or_b32(w, 0x00F000F0u, 0x54005400u)) - b_hi) * s2;
  h[2] = (__builtin_bit_cast(half2_t, and_or_b32(u, 0x000F000Fu, 0x64006400u)) - b_lo) * s2;
  h[3] = (__builtin_bit_cast(half2_t, and_or_b32(u, 0x00F000F0u, 0x54005400u)) - b_hi) * s2;
  half8_t out;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    out[2 * r] = h[r][0];
    out[2 * r + 1] = h[r][1];
  }
  return out;
}

// XCD-aware workgroup numbering.  The dispatcher places workgroup b on XCD b % 8
// (round robin over the 8 XCDs, each with its own L2).  This maps b to a logical index
// such that every XCD receives one contiguous range of logical indices, so neighbouring
// logical workgroups (which share inputs) share an L2.  A bijection on [0, n) for any n;
// if the placement were different only locality, never correctness, would change.
__device__ __forceinline__ int xcd_logical_block(int b, int n) {
  const int q = n >> 3, r = n & 7;
  const int x = b & 7, local = b >> 3;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + local;
}

// Grouped tile order for GEMMs: logical tile L -> (tm, tn) walking groups of GM tile rows
// column by column, so that a run of consecutive logical tiles (the ones one XCD holds at a
// time under xcd_logical_block) covers a GM x (run / GM) block and shares both operands
// in that XCD's L2.  A bijection on [0, tiles_m * tiles_n).
__device__ __forceinline__ void grouped_tile(int L, int tiles_m, int tiles_n, int GM, int& tm, int& tn) {
  const int per_group = GM * tiles_n;
  const int grp = L / per_group;
  const int idx = L - grp * per_group;
  const int rows = min(GM, tiles_m - grp * GM);
  tm = grp * GM + idx % rows;
  tn = idx / rows;
}

// sum[e] += base[p * stride + e] for p = 0 .. n-1 in ascending order (e = 0..7, fp32 split-K
// slices).  Loads go out in batches of BATCH before the first add of the batch, so n
// slices cost ceil(n/BATCH) memory round trips, not n.  The batch is branch-free: a slot
// past n re-reads slice n - 1 and adds +0.0f (sum is never -0.0f) - a load behind a
// branch leaves the compiler unsure what is outstanding, and it then waits per slice.
template <int BATCH = 8>
__device__ __forceinline__ void sum_slices8(const float* __restrict__ base, int64_t stride, int n,
                                            float sum[8]) {
#pragma clang fp contract(off)
  for (int b = 0; b < n; b += BATCH) {
    float4 lo[BATCH], hi[BATCH];
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int p = b + u < n ? b + u : n - 1;
      const float4* pp = (const float4*)(base + (int64_t)p * stride);
      lo[u] = pp[0];
      hi[u] = pp[1];
    }
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const bool on = b + u < n;
      sum[0] += on ? lo[u].x : 0.f; sum[1] += on ? lo[u].y : 0.f;
      sum[2] += on ? lo[u].z : 0.f; sum[3] += on ? lo[u].w : 0.f;
      sum[4] += on ? hi[u].x : 0.f; sum[5] += on ? hi[u].y : 0.f;
      sum[6] += on ? hi[u].z : 0.f; sum[7] += on ? hi[u].w : 0.f;
    }
  }
}

// Split decode-attention state of one (token, kv head, query head): o[128] (unnormalised,
// relative to m), m (running max of the base-2 scaled scores), l (sum of exp2(s - m)),
// two pad floats; records are 16-byte aligned.
// 16-bit storage that is fp16 or (BF16) bfloat16, read and written through fp32; bf16
// stores round to nearest even and keep NaN quiet.
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
template <bool BF16>
__device__ __forceinline__ float ld16f(unsigned short v) {
  return BF16 ? __builtin_bit_cast(float, (uint32_t)v << 16) : (float)__builtin_bit_cast(half_t, v);
}
template <bool BF16>
__device__ __forceinline__ unsigned short st16f(float f) {
  if (BF16) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    return (unsigned short)((u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) | 0x0040u) : r);
  }
  return __builtin_bit_cast(unsigned short, (half_t)f);
}

#define ATT_REC 132

// Merge of S split states for dims d0..d0+7: the record of split s sits at
// rec0 + s * sstride floats.  Splits are merged 8 at a time (every load of a batch in
// flight before its first use); for S <= 8 this is M = max m_s, l = sum f_s l_s,
// o = sum f_s o_s (f_s = exp2(m_s - M), split order, fused multiply-adds), fp16(o / l).
struct Merge8Loads {
  float mm[8], ll[8];
  float4 oa[8], ob[8];
};
struct Merge8State {
  float M = -INFINITY, lsum = 0.f;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
};

// Issue the loads of splits b .. min(b + 8, S) - 1.
__device__ __forceinline__ void attn_merge8_issue(Merge8Loads& L, const float* __restrict__ rec0,
                                                  int64_t sstride, int b, int S, int d0) {
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (b + u < S) {          // uniform: no load is issued for a missing split
      const float* p = rec0 + (int64_t)(b + u) * sstride;
      const float2 ml = *(const float2*)(p + 128);
      L.mm[u] = ml.x;
      L.ll[u] = ml.y;
      L.oa[u] = *(const float4*)(p + d0);
      L.ob[u] = *(const float4*)(p + d0 + 4);
    } else {
      L.mm[u] = -INFINITY;
      L.ll[u] = 0.f;
      L.oa[u] = L.ob[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
}

__device__ __forceinline__ void attn_merge8_batch(Merge8State& st, const Merge8Loads& L, int nvalid) {
#pragma clang fp contract(off)
  float mb = st.M;
#pragma unroll
  for (int u = 0; u < 8; ++u) mb = fmaxf(mb, L.mm[u]);
  if (mb == -INFINITY) return;
  const float sc = exp2f(st.M - mb);          // M = -inf -> 0
  st.lsum *= sc;
#pragma unroll
  for (int e = 0; e < 8; ++e) st.o[e] *= sc;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (u < nvalid) {
      const float f = exp2f(L.mm[u] - mb);
      st.lsum = fmaf(f, L.ll[u], st.lsum);
      st.o[0] = fmaf(f, L.oa[u].x, st.o[0]); st.o[1] = fmaf(f, L.oa[u].y, st.o[1]);
      st.o[2] = fmaf(f, L.oa[u].z, st.o[2]); st.o[3] = fmaf(f, L.oa[u].w, st.o[3]);
      st.o[4] = fmaf(f, L.ob[u].x, st.o[4]); st.o[5] = fmaf(f, L.ob[u].y, st.o[5]);
      st.o[6] = fmaf(f, L.ob[u].z, st.o[6]); st.o[7] = fmaf(f, L.ob[u].w, st.o[7]);
    }
  }
  st.M = mb;
}

__device__ __forceinline__ half8_t attn_merge8_result(const Merge8State& st) {
  half8_t r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (half_t)(st.lsum > 0.f ? st.o[e] / st.lsum : 0.f);
  return r;
}

__device__ __forceinline__ half8_t attn_merge8(const float* __restrict__ rec0, int64_t sstride,
                                               int S, int d0) {
  Merge8State st;
  for (int b = 0; b < S; b += 8) {
    Merge8Loads L;
    attn_merge8_issue(L, rec0, sstride, b, S, d0);
    attn_merge8_batch(st, L, S - b);
  }
  return attn_merge8_result(st);
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations
// (lgkmcnt(0)) and not for its outstanding global loads, so a stream of global loads issued
// before it stays in flight across the barrier (__syncthreads would first drain them: its
// workgroup-scope fence waits for vmcnt(0)).  Use only where no global memory written by
// another wave of the workgroup is read after the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// MFMA 16x16x32 B operand of 32 k (rows of a row-major fp16 tile in LDS) x 16 n (columns),
// read transposed with two ds_read_b64_tr_b16.  The transpose read works per group of 16
// lanes: if lane i of a group addresses the 4 halves M[i][0..3], lane j receives
// (M[4k + j/4][j%4], k = 0..3).  Lane (q16, c16) needs rows rows(q16) + 0..3 of column
// c16 for its first four k and rows 16 + rows(q16) + 0..3 for the next four, so lane i of
// group q16 addresses row 4 q16 + i/4, columns 4 (i%4) .. +3 (then 16 rows further).
// tile: the 16-column block's first element in row 0; stride: halfs per LDS row (a
// multiple of 4).  Lane slot s of the result holds row 16 (s/4) + 4 q16 + s%4, column c16.
__device__ __forceinline__ half8_t lds_read_b_tr16(const half_t* tile, int stride, int q16, int c16) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const half_t* p0 = tile + (4 * q16 + (c16 >> 2)) * stride + 4 * (c16 & 3);
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0 + 16 * stride));
  const half4_t l = __builtin_bit_cast(half4_t, lo), h = __builtin_bit_cast(half4_t, hi);
  return (half8_t){l[0], l[1], l[2], l[3], h[0], h[1], h[2], h[3]};
}

__device__ __forceinline__ f32x4 mfma16x16x32(half8_t a, half8_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__host__ __device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

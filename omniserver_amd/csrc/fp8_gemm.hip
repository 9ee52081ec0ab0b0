// FP8 (e4m3fn) W8A8 GEMM with row-wise scales on the CDNA4 fp8 matrix cores.
//
// Replaces FP8Linear (omniserve/kernels/fp8_linear.py:66-126) and its activation
// quantiser (:45-63):
//   weights   sw[n] = amax_k |W[n, :]| / 448,  Wq = e4m3(W / sw)          (:83-86)
//   inputs    sa[m] = amax_k |x[m, :]| / 448,  xq = e4m3(x / sa)          (:45-63)
//   product   y[m, n] = bf16((sum_k xq[m,k] * Wq[n,k]) * sa[m] * sw[n])    (:115-118,
//             torch._scaled_mm with fp32 accumulation and a bf16 result), then cast to
//             fp16 by FP8Linear.forward (two roundings), plus bias in fp16.
//
// Kernel: one workgroup (4 waves) per 128 x 128 output tile, K consumed in steps of 128
// through double-buffered LDS (each row padded to 144 bytes so the 16 rows one MFMA
// operand read touches spread over the banks).  The MFMA is
// v_mfma_scale_f32_16x16x128_f8f6f4 with unit block scales (e8m0 127): operand A = 16
// weight rows (n), operand B = 16 token rows (m), so a lane ends up holding four
// consecutive n of one m and stores them as one 8-byte write.  Each lane's 32 operand
// bytes are 32 consecutive k of its row (the same k assignment on both operands, which
// is all the dot product needs).  Each wave owns a 64 (n) x 64 (m) sub-tile: 16 MFMAs
// and 8 operand reads per K step.  Row-wise scales and the bf16 -> fp16 rounding are
// applied in the epilogue.
#include "common.h"

#define F8_BT 128          // tile rows (m) and columns (n) per workgroup
#define F8_BK 128          // K per step (one MFMA)
#define F8_STRIDE 144      // LDS bytes per staged row

typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);   // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

struct Fp8GemmArgs {
  const uint8_t* xq;     // [M, K] e4m3
  const float* sa;       // [M]
  const uint8_t* wq;     // [N, K] e4m3
  const float* sw;       // [N]
  const half_t* bias;    // [N] or NULL
  void* out;             // [M, ldo] fp16 (or bf16)
  int ldo;
  int M, N, K;
  int out_bf16;          // 1: write the bf16 result (forward_prequant); 0: fp16 (+bias)
};

__global__ __launch_bounds__(256, 2) void fp8_gemm_kernel(Fp8GemmArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][F8_BT * F8_STRIDE];  // [buf][x|w]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave & 1;          // n half of the tile
  const int wm = wave >> 1;         // m half
  const int l16 = lane & 15;
  const int g4 = lane >> 4;

  const int tiles_n = a.N / F8_BT;
  const int blk = xcd_logical_block(blockIdx.x, gridDim.x);
  const int tn = blk % tiles_n;
  const int tm = blk / tiles_n;
  const int m0 = tm * F8_BT, n0 = tn * F8_BT;

  // global -> LDS staging: thread t moves rows t/8 + 32u (u < 4), 16-byte chunk t%8, of
  // both the x tile and the w tile.  Rows past M re-read row M-1 (never stored out).
  const int srow = tid >> 3;
  const int schunk = (tid & 7) * 16;
  const uint8_t* xsrc[4];
  const uint8_t* wsrc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int mr = min(m0 + srow + 32 * u, a.M - 1);
    xsrc[u] = a.xq + (int64_t)mr * a.K + schunk;
    wsrc[u] = a.wq + (int64_t)(n0 + srow + 32 * u) * a.K + schunk;
  }
  u32x4 xr[4], wr[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      xr[u] = __builtin_nontemporal_load((const u32x4*)(xsrc[u] + k0));
      wr[u] = __builtin_nontemporal_load((const u32x4*)(wsrc[u] + k0));
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      *(u32x4*)(&lds[buf][0][(srow + 32 * u) * F8_STRIDE + schunk]) = xr[u];
      *(u32x4*)(&lds[buf][1][(srow + 32 * u) * F8_STRIDE + schunk]) = wr[u];
    }
  };

  f32x4 acc[4][4];   // [n sub-tile][m sub-tile]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int nk = a.K / F8_BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int ks = 0; ks < nk; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < nk) gload((ks + 1) * F8_BK);
    // operand fragments: 32 bytes of row (16-row sub-tile base + l16) at k = 32 * g4
    i32x8 wf[4], xf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t* p = &lds[cur][1][(64 * wn + 16 * i + l16) * F8_STRIDE + 32 * g4];
      const u32x4 lo = *(const u32x4*)p, hi = *(const u32x4*)(p + 16);
      wf[i] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint8_t* p = &lds[cur][0][(64 * wm + 16 * j + l16) * F8_STRIDE + 32 * g4];
      const u32x4 lo = *(const u32x4*)p, hi = *(const u32x4*)(p + 16);
      xf[j] = (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[i], xf[j], acc[i][j], 0, 0, 0,
                                                                      127, 0, 127);
    if (ks + 1 < nk) {
      sstore(cur ^ 1);
      __syncthreads();
    }
  }

  // Epilogue: lane holds n = n0 + 64wn + 16i + 4g4 + r (r < 4) of m = m0 + 64wm + 16j + l16.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + 64 * wm + 16 * j + l16;
    if (m >= a.M) continue;
    const float sm = a.sa[m];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = n0 + 64 * wn + 16 * i + 4 * g4;
      const float4 s4 = *(const float4*)(a.sw + n);
      const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
      uint16_t bits[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint16_t b = f32_to_bf16_rne((acc[i][j][r] * sm) * sv[r]);
        if (a.out_bf16) {
          bits[r] = b;
        } else {
          half_t h = (half_t)__builtin_bit_cast(float, (uint32_t)b << 16);
          if (a.bias) h = (half_t)((float)h + (float)a.bias[n + r]);
          bits[r] = __builtin_bit_cast(uint16_t, h);
        }
      }
      uint2 pk;
      pk.x = (uint32_t)bits[0] | ((uint32_t)bits[1] << 16);
      pk.y = (uint32_t)bits[2] | ((uint32_t)bits[3] << 16);
      *(uint2*)((uint16_t*)a.out + (int64_t)m * a.ldo + n) = pk;
    }
  }
}

// Row-wise e4m3 quantisation: s[r] = amax_k |x[r, k]| / 448 (clamped below at clamp_min
// when clamp_min > 0), q[r, k] = e4m3(x[r, k] / s[r]).  One workgroup per row.
__global__ __launch_bounds__(256) void fp8_quant_rows_kernel(const half_t* __restrict__ x, int ldx,
                                                             uint8_t* __restrict__ q,
                                                             float* __restrict__ s, int K,
                                                             float clamp_min) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const half_t* xr = x + (int64_t)row * ldx;
  float amax = 0.f;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    const half8_t v = *(const half8_t*)(xr + k);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)v[e]));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sc = amax / 448.0f;
  if (clamp_min > 0.f) sc = fmaxf(sc, clamp_min);
  if (threadIdx.x == 0) s[row] = sc;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    const half8_t v = *(const half8_t*)(xr + k);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) lo |= (uint32_t)f32_to_e4m3fn((float)v[e] / sc) << (8 * e);
#pragma unroll
    for (int e = 0; e < 4; ++e) hi |= (uint32_t)f32_to_e4m3fn((float)v[4 + e] / sc) << (8 * e);
    *(uint2*)(q + (int64_t)row * K + k) = make_uint2(lo, hi);
  }
}

extern "C" int omni_fp8_quant_rows(const void* x, int ldx, void* xq, float* scale, int rows, int K,
                                   float clamp_min, void* stream) {
  if (rows < 0 || K <= 0) return OMNI_EINVAL;
  if ((K & 7) || ldx < K || (ldx & 7)) return OMNI_EUNSUPPORTED;
  if (rows == 0) return OMNI_OK;
  if (!x || !xq || !scale) return OMNI_EINVAL;
  hipLaunchKernelGGL(fp8_quant_rows_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)x, ldx, (uint8_t*)xq, scale, K, clamp_min);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_fp8_gemm(const void* xq, const float* sa, const void* wq, const float* sw,
                             const void* bias, void* out, int ldo, int M, int N, int K,
                             int out_bf16, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return OMNI_EINVAL;
  if ((N % F8_BT) || (K % F8_BK)) return OMNI_EUNSUPPORTED;
  if (ldo < N || (ldo & 3)) return OMNI_EINVAL;
  if (M == 0) return OMNI_OK;
  if (!xq || !sa || !wq || !sw || !out) return OMNI_EINVAL;
  const int64_t tiles = (int64_t)ceil_div(M, F8_BT) * (N / F8_BT);
  if (tiles > 0x7fffffff) return OMNI_EUNSUPPORTED;
  Fp8GemmArgs a;
  a.xq = (const uint8_t*)xq;
  a.sa = sa;
  a.wq = (const uint8_t*)wq;
  a.sw = sw;
  a.bias = (const half_t*)bias;
  a.out = out;
  a.ldo = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  a.out_bf16 = out_bf16;
  hipLaunchKernelGGL(fp8_gemm_kernel, dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

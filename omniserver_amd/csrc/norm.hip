// Fused residual-add + RMSNorm family, SiLU-mul and the embedding gather.
//
// One 64-lane wavefront owns one row; a 256-thread workgroup carries four
// rows.  Each lane holds 8 consecutive fp16 values per 512-element chunk, so a
// 1536-wide Qwen2 row is three 16-byte loads per lane kept in registers between
// the sum-of-squares and the scaling pass (one HBM read, one write).
//
// Numerics follow omniserve/kernels/fused_ops.py:
//   rms_norm      (:21-29)  y = fp16(x * rstd * w), rstd = 1/sqrt(sum(x^2)/N + eps)
//   add_rms_norm  (:43-57)  r = fp16(res + x) is stored, then normalised
//   add_rms_fp8   (:74-91)  y32 = r*rstd*w; s = max(amax|y32|/448, 1e-12);
//                           q = e4m3fn(y32 / s)
//   silu_mul      (:111-119) out = fp16(silu(g) * u) in fp32
#include "common.h"

#define NORM_MAX_CHUNKS 16   // hidden <= 16 * 512 = 8192

// Address of element (n, k) of an fp16 weight in the packed MFMA layout
// [N/16][K/32][64 lanes][8]: lane = n%16 + 16*((k%32)/8), element k%8.
__device__ __forceinline__ size_t packed16_offset(int64_t n, int k, int K) {
  int64_t nt = n >> 4;
  int ks = k >> 5;
  int lane = (int)(n & 15) + 16 * ((k & 31) >> 3);
  return ((((size_t)nt * (K >> 5) + ks) * 64 + lane) << 3) + (k & 7);
}

// Rotary row of one decode token (lanes 0-15): row[0:64] = cos, row[64:128] = sin of
// p * inv_freq, p = lengths[r] + rope_delta[r] clamped to the tables, read from the same
// fp16 tables the attention would index (qwen2_llm.py:169-177; a decode token has one
// position on all three M-RoPE axes).  A decode step writes these rows once for all of its
// layers' attention launches.
#define ROPE_HALF 64
__device__ __forceinline__ void rope_row(int lane, int64_t r, const int64_t* __restrict__ len,
                                         const int64_t* __restrict__ delta,
                                         const half_t* __restrict__ cos_tab,
                                         const half_t* __restrict__ sin_tab, int max_pos,
                                         half_t* __restrict__ out_row) {
  int64_t pos = len[r] + (delta ? delta[r] : 0);
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const half_t* tab = lane < 8 ? cos_tab : sin_tab;
  *(half8_t*)(out_row + lane * 8) = *(const half8_t*)(tab + pos * ROPE_HALF + (lane & 7) * 8);
}

// PARTS: x is the fp32 split-K partial sums [nparts][rows][H] of the producing
// linear, summed in slice order and rounded to fp16 (= that linear's fp16 output).
// GATHER with rope_rows: the rows' rotary rows for the step are written as well.
template <bool HAS_RES, bool GATHER, bool FP8OUT, bool PARTS = false>
__global__ __launch_bounds__(256) void rmsnorm_kernel(
    const half_t* x, const half_t* residual, const int64_t* __restrict__ ids,
    const half_t* __restrict__ table, int table_packed, int64_t vocab,
    const half_t* __restrict__ w, half_t* y, uint8_t* __restrict__ y8,
    float* __restrict__ scale_out, half_t* res_out, int rows, int H, float eps,
    const float* __restrict__ parts = nullptr, int nparts = 0,
    const int64_t* __restrict__ rr_len = nullptr, const int64_t* __restrict__ rr_delta = nullptr,
    const half_t* __restrict__ rr_cos = nullptr, const half_t* __restrict__ rr_sin = nullptr,
    int rr_max = 0, half_t* __restrict__ rope_rows = nullptr) {
#pragma clang fp contract(off)
  // all arguments in one batch of scalar loads (a wait for one is a wait for all)
  asm volatile("" ::"s"(x), "s"(residual), "s"(ids), "s"(table), "s"(table_packed), "s"(vocab),
               "s"(w), "s"(y), "s"(y8), "s"(scale_out), "s"(res_out), "s"(rows), "s"(H), "s"(eps),
               "s"(parts), "s"(nparts), "s"(rr_len), "s"(rr_delta), "s"(rr_cos), "s"(rr_sin),
               "s"(rr_max), "s"(rope_rows));
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nchunk = H >> 3;

  int64_t tok = 0;
  if (GATHER) {
    tok = ids[row];
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
    if (rope_rows && lane < 16)
      rope_row(lane, row, rr_len, rr_delta, rr_cos, rr_sin, rr_max, rope_rows + (size_t)row * 2 * ROPE_HALF);
  }

  half8_t r[NORM_MAX_CHUNKS];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_MAX_CHUNKS; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunk) {
      half8_t v;
      if (GATHER) {
        size_t off = table_packed ? packed16_offset(tok, c * 8, H) : (size_t)tok * H + c * 8;
        v = *(const half8_t*)(table + off);
      } else if (PARTS) {
        float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int p = 0; p < nparts; ++p) {
          const float4* pp = (const float4*)(parts + ((size_t)p * rows + row) * H + c * 8);
          const float4 lo = pp[0], hi = pp[1];
          sum[0] += lo.x; sum[1] += lo.y; sum[2] += lo.z; sum[3] += lo.w;
          sum[4] += hi.x; sum[5] += hi.y; sum[6] += hi.z; sum[7] += hi.w;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (half_t)sum[e];
      } else {
        v = *(const half8_t*)(x + (size_t)row * H + c * 8);
      }
      if (HAS_RES) {
        half8_t rv = *(const half8_t*)(residual + (size_t)row * H + c * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (half_t)((float)v[e] + (float)rv[e]);
      }
      r[i] = v;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float f = (float)v[e];
        ss += f * f;
      }
    }
  }
  ss = wave_sum(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)H + eps);

  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < NORM_MAX_CHUNKS; ++i) {
    const int c = lane + 64 * i;
    if (c < nchunk) {
      if (HAS_RES || GATHER) *(half8_t*)(res_out + (size_t)row * H + c * 8) = r[i];
      half8_t wv = *(const half8_t*)(w + c * 8);
      if (!FP8OUT) {
        half8_t o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (half_t)(((float)r[i][e] * rstd) * (float)wv[e]);
        *(half8_t*)(y + (size_t)row * H + c * 8) = o;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(((float)r[i][e] * rstd) * (float)wv[e]));
      }
    }
  }
  if (FP8OUT) {
    amax = wave_max(amax);
    const float s = fmaxf(amax / 448.0f, 1e-12f);
#pragma unroll
    for (int i = 0; i < NORM_MAX_CHUNKS; ++i) {
      const int c = lane + 64 * i;
      if (c < nchunk) {
        half8_t wv = *(const half8_t*)(w + c * 8);
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo |= (uint32_t)f32_to_e4m3fn((((float)r[i][e] * rstd) * (float)wv[e]) / s) << (8 * e);
          hi |= (uint32_t)f32_to_e4m3fn((((float)r[i][e + 4] * rstd) * (float)wv[e + 4]) / s) << (8 * e);
        }
        uint2 pk = {lo, hi};
        *(uint2*)(y8 + (size_t)row * H + c * 8) = pk;
      }
    }
    if (lane == 0) scale_out[row] = s;
  }
}

// Many-row add+RMSNorm with every load of a row issued before any arithmetic: H = 512 * NC,
// so each lane owns exactly NC 8-element chunks (no lane divergence, nothing for the compiler
// to keep behind a branch), x fp16 (NP = 0) or NP fp32 split-K partial slices summed in slice
// order.  rmsnorm_kernel's operations in its order (the same per-lane chunk sequence, the
// same wave reduction), so the outputs are bit-identical to it; the residual, the inputs and
// the gains are all in flight together where rmsnorm_kernel waits chunk by chunk and fetches
// the gains after its reduction.  res_out may alias residual (each lane reads its chunks
// before it writes them).
template <int NC, int NP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4))) void addnorm_rows_kernel(const half_t* x,
                                                           const float* __restrict__ parts,
                                                           const half_t* residual,
                                                           const half_t* __restrict__ w, half_t* y,
                                                           half_t* res_out, int rows, float eps) {
#pragma clang fp contract(off)
  asm volatile("" ::"s"(x), "s"(parts), "s"(residual), "s"(w), "s"(y), "s"(res_out), "s"(rows),
               "s"(eps));
  constexpr int H = NC * 512;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t base = (size_t)row * H + lane * 8;
  half8_t rv[NC], xv[NP == 0 ? NC : 1], wv[NC];
  float4 pv[NP > 0 ? NP : 1][NC][2];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    if (NP == 0) {
      xv[i] = *(const half8_t*)(x + base + 512 * i);
    } else {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const float4* pp = (const float4*)(parts + (size_t)p * rows * H + base + 512 * i);
        pv[p][i][0] = pp[0];
        pv[p][i][1] = pp[1];
      }
    }
    rv[i] = *(const half8_t*)(residual + base + 512 * i);
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) wv[i] = *(const half8_t*)(w + lane * 8 + 512 * i);

  half8_t r[NC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    half8_t v;
    if (NP == 0) {
      v = xv[i];
    } else {
      float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        sum[0] += pv[p][i][0].x; sum[1] += pv[p][i][0].y;
        sum[2] += pv[p][i][0].z; sum[3] += pv[p][i][0].w;
        sum[4] += pv[p][i][1].x; sum[5] += pv[p][i][1].y;
        sum[6] += pv[p][i][1].z; sum[7] += pv[p][i][1].w;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (half_t)sum[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (half_t)((float)v[e] + (float)rv[i][e]);
    r[i] = v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float f = (float)v[e];
      ss += f * f;
    }
  }
  ss = wave_sum(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    *(half8_t*)(res_out + base + 512 * i) = r[i];
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (half_t)(((float)r[i][e] * rstd) * (float)wv[i][e]);
    *(half8_t*)(y + base + 512 * i) = o;
  }
}

// The addnorm_rows_kernel instance for (hidden, nparts), or nullptr (rmsnorm_kernel then).
typedef void (*addnorm_rows_fn)(const half_t*, const float*, const half_t*, const half_t*,
                                half_t*, half_t*, int, float);
static addnorm_rows_fn addnorm_rows_for(int hidden, int nparts) {
  if (hidden == 1536) {
    switch (nparts) {
      case 0: return addnorm_rows_kernel<3, 0>;
      case 1: return addnorm_rows_kernel<3, 1>;
      case 2: return addnorm_rows_kernel<3, 2>;
      case 3: return addnorm_rows_kernel<3, 3>;
      case 4: return addnorm_rows_kernel<3, 4>;
    }
  } else if (hidden == 3584) {
    switch (nparts) {
      case 0: return addnorm_rows_kernel<7, 0>;
      case 1: return addnorm_rows_kernel<7, 1>;
      case 2: return addnorm_rows_kernel<7, 2>;
    }
  }
  return nullptr;
}

// Decode-size add+RMSNorm: one workgroup per row, one 8-element chunk per thread
// (H/8 threads, rounded up to whole waves), so every load of the row - including all
// split-K partials - is in flight at once.  x is fp16, or (PARTS) the fp32 partial sums
// [nparts][rows][H] added in slice order and rounded to fp16.
// MAXT: the workgroup size bound (256 covers H <= 2048 and leaves the registers for a
// whole batch of 16 partial slices in flight; 1024 covers the largest H).
template <bool PARTS, int MAXT>
__global__ __launch_bounds__(MAXT) void rownorm_kernel(const half_t* x, const float* __restrict__ parts,
                                                       int nparts, const half_t* residual,
                                                       const half_t* __restrict__ w, half_t* y,
                                                       half_t* res_out, int rows, int H, float eps) {
#pragma clang fp contract(off)
  // all arguments in one batch of scalar loads (a wait for one is a wait for all)
  asm volatile("" ::"s"(x), "s"(parts), "s"(nparts), "s"(residual), "s"(w), "s"(y), "s"(res_out),
               "s"(rows), "s"(H), "s"(eps));
  __shared__ float wsum[16];
  const int row = blockIdx.x;
  const int c = threadIdx.x;
  const int nchunk = H >> 3;
  const bool live = c < nchunk;
  // Every load is issued up front, branch-free: threads past the row re-read its last chunk
  // (their values are dropped), and the gains are fetched with the inputs rather than after
  // the reduction's barrier (which would cost another memory round trip).
  const int cc = live ? c : nchunk - 1;
  const half8_t rv = *(const half8_t*)(residual + (size_t)row * H + cc * 8);
  const half8_t wv = *(const half8_t*)(w + cc * 8);
  half8_t v;
  if (PARTS) {
    float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // 16 slices in flight per batch at 256 threads; 8 at 1024 (a quarter of the registers)
    sum_slices8<MAXT <= 256 ? 16 : 8>(parts + (size_t)row * H + cc * 8, (int64_t)rows * H, nparts,
                                       sum);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (half_t)sum[e];
  } else {
    v = *(const half8_t*)(x + (size_t)row * H + cc * 8);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (half_t)((float)v[e] + (float)rv[e]);
  if (!live) v = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  const int nw = (blockDim.x + 63) >> 6;
  for (int i = 0; i < nw; ++i) tot += wsum[i];
  const float rstd = 1.0f / sqrtf(tot / (float)H + eps);
  if (live) {
    *(half8_t*)(res_out + (size_t)row * H + c * 8) = v;
    half8_t o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (half_t)(((float)v[e] * rstd) * (float)wv[e]);
    *(half8_t*)(y + (size_t)row * H + c * 8) = o;
  }
}

static int check_norm_shape(int rows, int H) {
  if (rows < 0 || H <= 0) return OMNI_EINVAL;
  if ((H & 7) != 0 || H > NORM_MAX_CHUNKS * 512) return OMNI_EUNSUPPORTED;
  return OMNI_OK;
}

extern "C" int omni_rmsnorm(const void* x, const void* weight, void* y, int rows, int hidden,
                            float eps, void* stream) {
  int rc = check_norm_shape(rows, hidden);
  if (rc) return rc;
  if (rows == 0) return OMNI_OK;
  if (!x || !weight || !y) return OMNI_EINVAL;
  hipLaunchKernelGGL((rmsnorm_kernel<false, false, false>), dim3(ceil_div(rows, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const half_t*)x, nullptr, nullptr, nullptr, 0, 0,
                     (const half_t*)weight, (half_t*)y, nullptr, nullptr, nullptr, rows, hidden, eps);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_add_rmsnorm(const void* x, const void* residual, const void* weight, void* y,
                                void* residual_out, int rows, int hidden, float eps, void* stream) {
  int rc = check_norm_shape(rows, hidden);
  if (rc) return rc;
  if (rows == 0) return OMNI_OK;
  if (!x || !residual || !weight || !y || !residual_out) return OMNI_EINVAL;
  if (rows <= 256) {
    const int threads = ceil_div(hidden >> 3, 64) * 64;
    auto kern = threads <= 256 ? rownorm_kernel<false, 256> : rownorm_kernel<false, 1024>;
    hipLaunchKernelGGL(kern, dim3(rows), dim3(threads), 0, (hipStream_t)stream,
                       (const half_t*)x, nullptr, 0, (const half_t*)residual,
                       (const half_t*)weight, (half_t*)y, (half_t*)residual_out, rows, hidden, eps);
  } else if (addnorm_rows_fn kern = addnorm_rows_for(hidden, 0)) {
    hipLaunchKernelGGL(kern, dim3(ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream,
                       (const half_t*)x, nullptr, (const half_t*)residual, (const half_t*)weight,
                       (half_t*)y, (half_t*)residual_out, rows, eps);
  } else {
    hipLaunchKernelGGL((rmsnorm_kernel<true, false, false>), dim3(ceil_div(rows, 4)), dim3(256), 0,
                       (hipStream_t)stream, (const half_t*)x, (const half_t*)residual, nullptr,
                       nullptr, 0, 0, (const half_t*)weight, (half_t*)y, nullptr, nullptr,
                       (half_t*)residual_out, rows, hidden, eps);
  }
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_add_rmsnorm_partials(const float* partials, int nparts, const void* residual,
                                         const void* weight, void* y, void* residual_out, int rows,
                                         int hidden, float eps, void* stream) {
  int rc = check_norm_shape(rows, hidden);
  if (rc) return rc;
  if (rows == 0) return OMNI_OK;
  if (!partials || nparts <= 0 || !residual || !weight || !y || !residual_out) return OMNI_EINVAL;
  if (rows <= 256) {   // the same kernels (and reduction orders) as omni_add_rmsnorm
    const int threads = ceil_div(hidden >> 3, 64) * 64;
    auto kern = threads <= 256 ? rownorm_kernel<true, 256> : rownorm_kernel<true, 1024>;
    hipLaunchKernelGGL(kern, dim3(rows), dim3(threads), 0, (hipStream_t)stream,
                       nullptr, partials, nparts, (const half_t*)residual, (const half_t*)weight,
                       (half_t*)y, (half_t*)residual_out, rows, hidden, eps);
  } else if (addnorm_rows_fn kern = addnorm_rows_for(hidden, nparts)) {
    hipLaunchKernelGGL(kern, dim3(ceil_div(rows, 4)), dim3(256), 0, (hipStream_t)stream,
                       nullptr, partials, (const half_t*)residual, (const half_t*)weight,
                       (half_t*)y, (half_t*)residual_out, rows, eps);
  } else {
    hipLaunchKernelGGL((rmsnorm_kernel<true, false, false, true>), dim3(ceil_div(rows, 4)), dim3(256), 0,
                       (hipStream_t)stream, nullptr, (const half_t*)residual, nullptr, nullptr, 0, 0,
                       (const half_t*)weight, (half_t*)y, nullptr, nullptr, (half_t*)residual_out,
                       rows, hidden, eps, partials, nparts);
  }
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_add_rmsnorm_fp8(const void* x, const void* residual, const void* weight,
                                    void* y_fp8, float* scale, void* residual_out, int rows,
                                    int hidden, float eps, void* stream) {
  int rc = check_norm_shape(rows, hidden);
  if (rc) return rc;
  if (rows == 0) return OMNI_OK;
  if (!x || !residual || !weight || !y_fp8 || !scale || !residual_out) return OMNI_EINVAL;
  hipLaunchKernelGGL((rmsnorm_kernel<true, false, true>), dim3(ceil_div(rows, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const half_t*)x, (const half_t*)residual, nullptr, nullptr,
                     0, 0, (const half_t*)weight, nullptr, (uint8_t*)y_fp8, scale,
                     (half_t*)residual_out, rows, hidden, eps);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_embed_rmsnorm(const int64_t* ids, const void* table, int table_packed,
                                  int64_t vocab, const void* weight, void* y, void* residual_out,
                                  int rows, int hidden, float eps, void* stream) {
  int rc = check_norm_shape(rows, hidden);
  if (rc) return rc;
  if (rows == 0) return OMNI_OK;
  if (!ids || !table || !weight || !y || !residual_out || vocab <= 0) return OMNI_EINVAL;
  if (table_packed && ((hidden & 31) != 0 || (vocab & 15) != 0)) return OMNI_EUNSUPPORTED;
  hipLaunchKernelGGL((rmsnorm_kernel<false, true, false>), dim3(ceil_div(rows, 4)), dim3(256), 0,
                     (hipStream_t)stream, nullptr, nullptr, ids, (const half_t*)table, table_packed,
                     vocab, (const half_t*)weight, (half_t*)y, nullptr, nullptr,
                     (half_t*)residual_out, rows, hidden, eps);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// omni_embed_rmsnorm that also writes the step's rotary rows (see rope_row).
extern "C" int omni_embed_rmsnorm_rope(const int64_t* ids, const void* table, int table_packed,
                                       int64_t vocab, const void* weight, void* y,
                                       void* residual_out, int rows, int hidden, float eps,
                                       const int64_t* lengths, const int64_t* rope_delta,
                                       const void* cos_tab, const void* sin_tab, int max_pos,
                                       void* rope_rows, void* stream) {
  int rc = check_norm_shape(rows, hidden);
  if (rc) return rc;
  if (rows == 0) return OMNI_OK;
  if (!ids || !table || !weight || !y || !residual_out || vocab <= 0) return OMNI_EINVAL;
  if (!lengths || !cos_tab || !sin_tab || !rope_rows || max_pos <= 0) return OMNI_EINVAL;
  if (table_packed && ((hidden & 31) != 0 || (vocab & 15) != 0)) return OMNI_EUNSUPPORTED;
  hipLaunchKernelGGL((rmsnorm_kernel<false, true, false>), dim3(ceil_div(rows, 4)), dim3(256), 0,
                     (hipStream_t)stream, nullptr, nullptr, ids, (const half_t*)table, table_packed,
                     vocab, (const half_t*)weight, (half_t*)y, nullptr, nullptr,
                     (half_t*)residual_out, rows, hidden, eps, nullptr, 0, lengths, rope_delta,
                     (const half_t*)cos_tab, (const half_t*)sin_tab, max_pos, (half_t*)rope_rows);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

__global__ __launch_bounds__(64) void rope_rows_kernel(const int64_t* __restrict__ slots,
                                                       const int64_t* __restrict__ lengths,
                                                       const int64_t* __restrict__ delta,
                                                       const half_t* __restrict__ cos_tab,
                                                       const half_t* __restrict__ sin_tab,
                                                       int max_pos, int pool_rows, int T,
                                                       half_t* __restrict__ out) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 4);
  if (t >= T) return;
  int64_t r = slots ? slots[t] : t;
  r = r < 0 ? 0 : (r >= pool_rows ? pool_rows - 1 : r);
  rope_row(threadIdx.x & 15, r, lengths, delta, cos_tab, sin_tab, max_pos, out + (size_t)t * 2 * ROPE_HALF);
}

// Rotary rows [T][128] of T decode tokens (pool rows slots[t], or t) at their write
// positions lengths[row] + rope_delta[row], for omni_decode_attention_fused.
extern "C" int omni_rope_rows(const int64_t* slots, const int64_t* lengths,
                              const int64_t* rope_delta, const void* cos_tab, const void* sin_tab,
                              int max_pos, int pool_rows, int T, void* rope_rows, void* stream) {
  if (T < 0 || max_pos <= 0 || pool_rows <= 0) return OMNI_EINVAL;
  if (T == 0) return OMNI_OK;
  if (!lengths || !cos_tab || !sin_tab || !rope_rows) return OMNI_EINVAL;
  hipLaunchKernelGGL(rope_rows_kernel, dim3(ceil_div(T, 4)), dim3(64), 0, (hipStream_t)stream,
                     slots, lengths, rope_delta, (const half_t*)cos_tab, (const half_t*)sin_tab,
                     max_pos, pool_rows, T, (half_t*)rope_rows);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// ---------------------------------------------------------------------------
// Embedding gather: out[t, :] = table[ids[t], :]   (models/qwen2_vl.py:93-94)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ ids,
                                                   const half_t* __restrict__ table, int packed,
                                                   int64_t vocab, half_t* __restrict__ out,
                                                   int rows, int H) {
  const int nchunk = H >> 3;
  const int64_t total = (int64_t)rows * nchunk;
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int row = (int)(i / nchunk);
    const int c = (int)(i % nchunk);
    int64_t tok = ids[row];
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
    size_t off = packed ? packed16_offset(tok, c * 8, H) : (size_t)tok * H + c * 8;
    *(half8_t*)(out + (size_t)row * H + c * 8) = *(const half8_t*)(table + off);
  }
}

extern "C" int omni_embedding(const int64_t* ids, const void* table, int table_packed,
                              int64_t vocab, void* out, int rows, int hidden, void* stream) {
  if (rows < 0 || hidden <= 0 || vocab <= 0) return OMNI_EINVAL;
  if ((hidden & 7) != 0) return OMNI_EUNSUPPORTED;
  if (table_packed && ((hidden & 31) != 0 || (vocab & 15) != 0)) return OMNI_EUNSUPPORTED;
  if (rows == 0) return OMNI_OK;
  if (!ids || !table || !out) return OMNI_EINVAL;
  int64_t work = (int64_t)rows * (hidden >> 3);
  int grid = (int)((work + 255) / 256);
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(embed_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, ids,
                     (const half_t*)table, table_packed, vocab, (half_t*)out, rows, hidden);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// ---------------------------------------------------------------------------
// SiLU-mul: gate_up [rows, 2n] (gate first, up second) -> out [rows, n].
// ---------------------------------------------------------------------------
// fp16 (or, BF16, bf16 as the reference's FP8 route feeds it, qwen2_llm.py:130-131) in and out.
template <bool BF16>
__global__ __launch_bounds__(256) void silu_mul_kernel(const unsigned short* __restrict__ gu,
                                                      unsigned short* __restrict__ out, int rows,
                                                      int n) {
#pragma clang fp contract(off)
  const int nchunk = n >> 3;
  const int64_t total = (int64_t)rows * nchunk;
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int row = (int)(i / nchunk);
    const int c = (int)(i % nchunk);
    const u16x8 g = *(const u16x8*)(gu + (size_t)row * 2 * n + c * 8);
    const u16x8 u = *(const u16x8*)(gu + (size_t)row * 2 * n + n + c * 8);
    u16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = st16f<BF16>(silu_mul_f32(ld16f<BF16>(g[e]), ld16f<BF16>(u[e])));
    *(u16x8*)(out + (size_t)row * n + c * 8) = o;
  }
}

static int silu_mul_launch(const void* gate_up, void* out, int rows, int n, bool bf16,
                           void* stream) {
  if (rows < 0 || n <= 0) return OMNI_EINVAL;
  if ((n & 7) != 0) return OMNI_EUNSUPPORTED;
  if (rows == 0) return OMNI_OK;
  if (!gate_up || !out) return OMNI_EINVAL;
  int64_t work = (int64_t)rows * (n >> 3);
  int grid = (int)((work + 255) / 256);
  if (grid > 8192) grid = 8192;
  auto kern = bf16 ? silu_mul_kernel<true> : silu_mul_kernel<false>;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const unsigned short*)gate_up, (unsigned short*)out, rows, n);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_silu_mul(const void* gate_up, void* out, int rows, int n, void* stream) {
  return silu_mul_launch(gate_up, out, rows, n, false, stream);
}

extern "C" int omni_silu_mul_bf16(const void* gate_up, void* out, int rows, int n, void* stream) {
  return silu_mul_launch(gate_up, out, rows, n, true, stream);
}

// Vision tower (Qwen2-VL ViT) kernels: LayerNorm (also over a split-K linear's partial
// sums, with its bias and residual add), the 2-D vision rotary, and non-causal segmented
// attention at head_dim 80.  The tower's linears run on the pipelined fp16 GEMM over packed
// weights (gemm_pipe.hip, omni_f16_gemm_pipe_packed: bias / QuickGELU / GELU / residual /
// partial-sum epilogues) and the patch embedding on the tiled one (gemv.hip).
//
// Replaces, per block of model/qwen2_vit.py:36-69: nn.LayerNorm (norm1 / norm2, and
// the merger's ln_q at :128), the fused rotary of kernels/vision_rope.py:19-47, and
// the varlen flash call at :58-63 (cu_seqlens separate the images; every patch of an
// image attends to every patch of the same image).
#include "common.h"

// ---------------------------------------------------------------------------
// LayerNorm over rows: y = (x - mean) * rsqrt(var + eps) * w + b, fp32 math, fp16 out
// (biased variance, as nn.LayerNorm).  One wave per row; lane holds 16-byte chunks
// lane + 64 u (u < 4), so N <= 2048.
// ---------------------------------------------------------------------------
#define LN_MAXCH 4

// PARTS: x is formed first, as a split-K linear's finish with the residual epilogue would
// form it (gemm_pipe_finish_kernel, GP_RESID): h = fp16(sum of the nparts fp32 slices
// [nparts][M][N] in slice order (+ bias, before the rounding)), x = fp16(res + h), with the
// residual rows read from x (row stride ldx) and x written to x_out (which may alias them:
// each lane reads its chunks before it writes them).
template <bool PARTS>
__global__ __launch_bounds__(256) void layernorm_kernel(const half_t* x, int ldx,
                                                        const half_t* __restrict__ w,
                                                        const half_t* __restrict__ b, int M,
                                                        int N, float eps, half_t* out, int ldo,
                                                        const float* __restrict__ parts = nullptr,
                                                        int nparts = 0,
                                                        const half_t* __restrict__ pbias = nullptr,
                                                        half_t* x_out = nullptr, int ldxo = 0) {
#pragma clang fp contract(off)
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int lane = threadIdx.x & 63;
  const int nc = N >> 3;
  const half_t* xr = x + (int64_t)row * ldx;
  float v[LN_MAXCH][8];
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < LN_MAXCH; ++u) {
    const int c = lane + 64 * u;
    half8_t h = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
    if (c < nc) {
      h = *(const half8_t*)(xr + c * 8);
      if (PARTS) {
        const float* pp = parts + (int64_t)row * N + c * 8;
        const int64_t ps = (int64_t)M * N;
        float a[8];
        const float4 lo = *(const float4*)pp, hi = *(const float4*)(pp + 4);
        a[0] = lo.x; a[1] = lo.y; a[2] = lo.z; a[3] = lo.w;
        a[4] = hi.x; a[5] = hi.y; a[6] = hi.z; a[7] = hi.w;
        for (int p = 1; p < nparts; ++p) {
          const float4 l2 = *(const float4*)(pp + p * ps), h2 = *(const float4*)(pp + p * ps + 4);
          a[0] += l2.x; a[1] += l2.y; a[2] += l2.z; a[3] += l2.w;
          a[4] += h2.x; a[5] += h2.y; a[6] += h2.z; a[7] += h2.w;
        }
        half8_t bb = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
        if (pbias) bb = *(const half8_t*)(pbias + c * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const half_t lin = pbias ? (half_t)(a[e] + (float)bb[e]) : (half_t)a[e];
          h[e] = (half_t)((float)h[e] + (float)lin);
        }
        *(half8_t*)(x_out + (int64_t)row * ldxo + c * 8) = h;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[u][e] = (float)h[e];
      s += v[u][e];
    }
  }
  const float mean = wave_sum(s) / (float)N;
  float q = 0.f;
#pragma unroll
  for (int u = 0; u < LN_MAXCH; ++u) {
    if (lane + 64 * u < nc) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[u][e] - mean;
        q += d * d;
      }
    }
  }
  const float var = wave_sum(q) / (float)N;
  const float rstd = rsqrtf(var + eps);
#pragma unroll
  for (int u = 0; u < LN_MAXCH; ++u) {
    const int c = lane + 64 * u;
    if (c >= nc) continue;
    const half8_t wv = *(const half8_t*)(w + c * 8);
    const half8_t bv = *(const half8_t*)(b + c * 8);
    half8_t y;
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (half_t)((v[u][e] - mean) * rstd * (float)wv[e] + (float)bv[e]);
    *(half8_t*)(out + (int64_t)row * ldo + c * 8) = y;
  }
}

// Rows of N = 256 NC (the tower's 1280: NC = 5): lane l holds the 4-column chunks
// l + 64 u, u < NC, so every lane has the same work and every load of the row - the
// residual / input, NP fp32 partial slices, the linear's bias and the norm's gains - goes out
// before any arithmetic (the kernel above waits chunk by chunk, and its 8-column chunks give
// lanes 2 or 3 of them at N = 1280).  NP = 0: plain LayerNorm of x; NP > 0: x formed first
// from the slices as in the kernel above.  Sums in this kernel's own order (chunks u, then
// the 4 columns), so its outputs agree with the kernel above to fp32 rounding of the mean
// and variance, and its two forms with each other bit for bit.
template <int NC, int NP>
__global__ __launch_bounds__(256) void layernorm4_kernel(const half_t* x, int ldx,
                                                         const half_t* __restrict__ w,
                                                         const half_t* __restrict__ b, int M,
                                                         float eps, half_t* out, int ldo,
                                                         const float* __restrict__ parts,
                                                         const half_t* __restrict__ pbias,
                                                         half_t* x_out, int ldxo) {
#pragma clang fp contract(off)
  constexpr int N = 256 * NC;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int lane = threadIdx.x & 63;
  const half_t* xr = x + (int64_t)row * ldx + 4 * lane;
  half4_t xv[NC], wv[NC], bv[NC], pb[NP > 0 ? NC : 1];
  float4 pv[NP > 0 ? NP : 1][NC];
#pragma unroll
  for (int u = 0; u < NC; ++u) {
    xv[u] = *(const half4_t*)(xr + 256 * u);
    if (NP > 0) {
#pragma unroll
      for (int p = 0; p < NP; ++p)
        pv[p][u] = *(const float4*)(parts + ((int64_t)p * M + row) * N + 4 * lane + 256 * u);
      if (pbias) pb[u] = *(const half4_t*)(pbias + 4 * lane + 256 * u);
    }
  }
#pragma unroll
  for (int u = 0; u < NC; ++u) {
    wv[u] = *(const half4_t*)(w + 4 * lane + 256 * u);
    bv[u] = *(const half4_t*)(b + 4 * lane + 256 * u);
  }
  float v[NC][4];
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < NC; ++u) {
    half4_t h = xv[u];
    if (NP > 0) {
      float a[4] = {pv[0][u].x, pv[0][u].y, pv[0][u].z, pv[0][u].w};
#pragma unroll
      for (int p = 1; p < NP; ++p) {
        a[0] += pv[p][u].x; a[1] += pv[p][u].y; a[2] += pv[p][u].z; a[3] += pv[p][u].w;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const half_t lin = pbias ? (half_t)(a[e] + (float)pb[u][e]) : (half_t)a[e];
        h[e] = (half_t)((float)h[e] + (float)lin);
      }
      *(half4_t*)(x_out + (int64_t)row * ldxo + 4 * lane + 256 * u) = h;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[u][e] = (float)h[e];
      s += v[u][e];
    }
  }
  const float mean = wave_sum(s) / (float)N;
  float q = 0.f;
#pragma unroll
  for (int u = 0; u < NC; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = v[u][e] - mean;
      q += d * d;
    }
  const float var = wave_sum(q) / (float)N;
  const float rstd = rsqrtf(var + eps);
#pragma unroll
  for (int u = 0; u < NC; ++u) {
    half4_t y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = (half_t)((v[u][e] - mean) * rstd * (float)wv[u][e] + (float)bv[u][e]);
    *(half4_t*)(out + (int64_t)row * ldo + 4 * lane + 256 * u) = y;
  }
}

typedef void (*layernorm4_fn)(const half_t*, int, const half_t*, const half_t*, int, float,
                              half_t*, int, const float*, const half_t*, half_t*, int);
// The layernorm4_kernel instance for (N, nparts), or nullptr (the kernel above then).
static layernorm4_fn layernorm4_for(int N, int nparts) {
  if (N != 1280) return nullptr;
  switch (nparts) {
    case 0: return layernorm4_kernel<5, 0>;
    case 1: return layernorm4_kernel<5, 1>;
    case 2: return layernorm4_kernel<5, 2>;
    case 3: return layernorm4_kernel<5, 3>;
    case 4: return layernorm4_kernel<5, 4>;
  }
  return nullptr;
}

// LayerNorm of M rows of N (N % 8 == 0, N <= 2048); w, b fp16 [N]; out may alias x.
extern "C" int omni_layernorm(const void* x, int ldx, const void* weight, const void* bias, int M,
                              int N, float eps, void* out, int ldo, void* stream) {
  if (M < 0 || N <= 0) return OMNI_EINVAL;
  if (M == 0) return OMNI_OK;
  if ((N & 7) || N > 64 * 8 * LN_MAXCH) return OMNI_EUNSUPPORTED;
  if (!x || !weight || !bias || !out) return OMNI_EINVAL;
  if (ldx < N || ldo < N || (ldx & 7) || (ldo & 7)) return OMNI_EINVAL;
  if (layernorm4_fn kern = ((((uintptr_t)x | (uintptr_t)out | (uintptr_t)weight | (uintptr_t)bias) & 7) == 0 &&
                             (ldx & 3) == 0 && (ldo & 3) == 0) ? layernorm4_for(N, 0) : nullptr)
    hipLaunchKernelGGL(kern, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       (const half_t*)x, ldx, (const half_t*)weight, (const half_t*)bias, M, eps,
                       (half_t*)out, ldo, nullptr, nullptr, nullptr, 0);
  else
    hipLaunchKernelGGL(layernorm_kernel<false>, dim3((unsigned)((M + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, (const half_t*)x, ldx, (const half_t*)weight,
                       (const half_t*)bias, M, N, eps, (half_t*)out, ldo, nullptr, 0, nullptr,
                       nullptr, 0);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// The residual add of a split-K linear (fp32 slices [nparts][M][N], 1 <= nparts <= 16,
// optional fp16 bias [N]) followed by a LayerNorm: residual_out = fp16(residual +
// fp16(sum of the slices + bias)), as the linear's finish launch with the residual epilogue
// writes it, then out = LayerNorm(residual_out) as omni_layernorm (model/qwen2_vit.py:66-69:
// x = x + attn(...); norm2(x), and x = x + mlp(...) before the next block's norm1 or the
// merger's ln_q).  residual_out may alias residual.
extern "C" int omni_layernorm_partials(const float* partials, int nparts, const void* lin_bias,
                                       const void* residual, int ldr, void* residual_out, int ldro,
                                       const void* weight, const void* bias, int M, int N,
                                       float eps, void* out, int ldo, void* stream) {
  if (M < 0 || N <= 0 || nparts < 1 || nparts > 16) return OMNI_EINVAL;
  if (M == 0) return OMNI_OK;
  if ((N & 7) || N > 64 * 8 * LN_MAXCH) return OMNI_EUNSUPPORTED;
  if (!partials || !residual || !residual_out || !weight || !bias || !out) return OMNI_EINVAL;
  if (ldr < N || ldro < N || ldo < N || (ldr & 7) || (ldro & 7) || (ldo & 7)) return OMNI_EINVAL;
  if (((uintptr_t)partials & 15) || ((uintptr_t)residual & 15) || ((uintptr_t)residual_out & 15) ||
      ((uintptr_t)out & 15) || (lin_bias && ((uintptr_t)lin_bias & 15)))
    return OMNI_EINVAL;
  if (layernorm4_fn kern = (((uintptr_t)weight | (uintptr_t)bias) & 7) == 0 ? layernorm4_for(N, nparts) : nullptr)
    hipLaunchKernelGGL(kern, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       (const half_t*)residual, ldr, (const half_t*)weight, (const half_t*)bias, M,
                       eps, (half_t*)out, ldo, partials, (const half_t*)lin_bias,
                       (half_t*)residual_out, ldro);
  else
    hipLaunchKernelGGL(layernorm_kernel<true>, dim3((unsigned)((M + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, (const half_t*)residual, ldr, (const half_t*)weight,
                       (const half_t*)bias, M, N, eps, (half_t*)out, ldo, partials, nparts,
                       (const half_t*)lin_bias, (half_t*)residual_out, ldro);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// ---------------------------------------------------------------------------
// 2-D vision rotary, in place on the q and k heads of the qkv rows.
// For head_dim D (half R = D / 2, quarter R / 2): pair (d, d + R), d < R, is rotated by
//   angle_d = pos_h * inv_freq[d]        (d < R/2)
//           = pos_w * inv_freq[d - R/2]  (R/2 <= d < R)
// (model/qwen2_vit.py:96-116: freqs[pos_ids].flatten(1), emb = cat(rpe, rpe)), in fp32:
//   y[d] = x[d] cos - x[d+R] sin,  y[d+R] = x[d+R] cos + x[d] sin
// (kernels/vision_rope.py:19-24), rounded to fp16.  One thread per 8 consecutive d of one
// (token, q|k, head).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void vision_rope_kernel(half_t* __restrict__ qkv, int ld, int S,
                                                          int nh, int hd,
                                                          const int* __restrict__ pos_hw,
                                                          const float* __restrict__ inv_freq) {
#pragma clang fp contract(off)
  const int R = hd >> 1, Q = hd >> 2;
  const int cpr = R >> 3;                                // chunks per rotated half
  const int64_t total = (int64_t)S * 2 * nh * cpr;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int c = (int)(i % cpr);
  const int64_t r = i / cpr;
  const int head = (int)(r % (2 * nh));                  // q heads, then k heads
  const int t = (int)(r / (2 * nh));
  half_t* p = qkv + (int64_t)t * ld + head * hd + c * 8;
  const half8_t x1 = *(const half8_t*)p;
  const half8_t x2 = *(const half8_t*)(p + R);
  const float ph = (float)pos_hw[2 * t], pw = (float)pos_hw[2 * t + 1];
  half8_t y1, y2;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int d = c * 8 + e;
    const float ang = d < Q ? ph * inv_freq[d] : pw * inv_freq[d - Q];
    const float cs = cosf(ang), sn = sinf(ang);
    const float a = (float)x1[e], b = (float)x2[e];
    y1[e] = (half_t)(a * cs - b * sn);
    y2[e] = (half_t)(b * cs + a * sn);
  }
  *(half8_t*)p = y1;
  *(half8_t*)(p + R) = y2;
}

// Rotate q (heads [0, nh)) and k (heads [nh, 2 nh)) of S rows of qkv (row stride ld, head
// dim hd, hd % 16 == 0) in place.  pos_hw int32 [S][2] = (h, w) patch position;
// inv_freq fp32 [hd / 4].
extern "C" int omni_vision_rope(void* qkv, int ld, int S, int n_heads, int head_dim,
                                const int* pos_hw, const float* inv_freq, void* stream) {
  if (S < 0 || n_heads <= 0 || head_dim <= 0) return OMNI_EINVAL;
  if (S == 0) return OMNI_OK;
  if (head_dim & 15) return OMNI_EUNSUPPORTED;
  if (!qkv || !pos_hw || !inv_freq) return OMNI_EINVAL;
  if (ld < 2 * n_heads * head_dim || (ld & 7)) return OMNI_EINVAL;
  const int64_t total = (int64_t)S * 2 * n_heads * (head_dim / 16);
  const int64_t grid = (total + 255) / 256;
  if (grid > 0x7fffffff) return OMNI_EUNSUPPORTED;
  hipLaunchKernelGGL(vision_rope_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (half_t*)qkv, ld, S, n_heads, head_dim, pos_hw, inv_freq);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// ---------------------------------------------------------------------------
// Segmented non-causal attention, head_dim 80 (model/qwen2_vit.py:48-64): for every head
// and every query t of segment [cu[s], cu[s+1]), out[t] = softmax(q_t K^T * scale) V over
// the keys of the same segment.
//
// One workgroup (4 waves) owns 64 consecutive queries of one segment and one head; each
// wave 16 of them.  K and V tiles of 64 keys are staged in LDS once for the 4 waves
// (double buffered, the next tile's loads in flight while the current one is used).  The
// MFMA structure is the decode / prefill kernels': S^T[16 keys x 16 queries] = K . Q^T
// (k = 96: dims 80..95 are zero in both operands), online softmax in fp32 (exp2),
// O[16 queries x 80] += P . V with V read back through the transposing LDS reads.
// The workgroups of one head are contiguous in the XCD-aware order, so that a head's K
// and V are read into one XCD's L2.
// ---------------------------------------------------------------------------
#define VA_HD 80
#define VA_KT 64       // keys per staged tile
#define VA_KSTR 104    // LDS halfs per K row: 80 dims, 16 zeros (dims 80..95), 8 pad
#define VA_VSTR 88     // LDS halfs per V row
#define VA_CPR 10      // 16-byte chunks per 80-dim row
#define VA_NLD 5       // tile chunks per thread: 2 * 64 * 10 / 256

struct VitAttnArgs {
  const half_t* qkv;   // rows [S][ld]: q heads | k heads | v heads, head_dim 80
  int ld;
  const int* cu;       // [nseg + 1]
  const int* tiles;    // [ntiles][2] = (first query, segment)
  int ntiles, nh, S;
  half_t* out;         // [S][ldo], head h at column 80 h
  int ldo;
  float scale_log2;
};

// KH key halves: with KH = 2 the workgroup has 8 waves; waves 4 h .. 4 h + 3 take the
// queries of waves 0 .. 3 against the h-th half of the segment's key tiles (each half with
// its own double-buffered tiles), and the two halves' softmax states are merged through
// LDS at the end - twice the waves per CU on the same queries.
template <int KH>
__global__ __launch_bounds__(256 * KH, 1) void vit_attn_kernel(VitAttnArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) half_t ks_lds[KH][2][VA_KT * VA_KSTR];
  __shared__ __attribute__((aligned(16))) half_t vs_lds[KH][2][VA_KT * VA_VSTR];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kh = wave >> 2;                     // key half
  const int qw = wave & 3;                      // query block of 16
  const int ht = tid & 255;                     // thread index within the half
  const int q16 = lane >> 4, c16 = lane & 15;
  const int L = xcd_logical_block(blockIdx.x, gridDim.x);
  const int h = L / a.ntiles, tile = L - h * a.ntiles;
  const int q0 = a.tiles[2 * tile], seg = a.tiles[2 * tile + 1];
  const int beg = max(a.cu[seg], 0), end = min(a.cu[seg + 1], a.S);
  if (q0 < beg || q0 >= end) return;            // malformed table entry: nothing to do
  const half8_t z8 = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
  // this half's key range, in whole tiles: half 0 takes the first ceil(n/2) tiles
  const int ntile = (end - beg + VA_KT - 1) / VA_KT;
  const int nt0 = (ntile + KH - 1) / KH;
  const int kbeg = beg + (kh == 0 ? 0 : nt0 * VA_KT);
  const int kend = kh == 0 && KH > 1 ? min(end, beg + nt0 * VA_KT) : end;
  const int my_nt = kend > kbeg ? (kend - kbeg + VA_KT - 1) / VA_KT : 0;

  // the K tiles' dims 80..95 are zero for the whole kernel (tile stores never touch them)
  for (int i = tid; i < KH * 2 * VA_KT * 2; i += 256 * KH) {
    const int hb_ = i / (2 * VA_KT * 2), r1 = i - hb_ * (2 * VA_KT * 2);
    const int bsel = r1 / (VA_KT * 2), rem = r1 - bsel * (VA_KT * 2);
    *(half8_t*)(&ks_lds[hb_][bsel][(rem >> 1) * VA_KSTR + VA_HD + 8 * (rem & 1)]) = z8;
  }

  // this wave's query rows q0 + 16 qw + c16 (past the segment: its last row, not stored)
  const int qrow = min(q0 + 16 * qw + c16, end - 1);
  const half_t* qp = a.qkv + (int64_t)qrow * a.ld + h * VA_HD;
  half8_t qf[3];
  qf[0] = *(const half8_t*)(qp + 8 * q16);
  qf[1] = *(const half8_t*)(qp + 32 + 8 * q16);
  qf[2] = *(const half8_t*)(qp + 64 + 8 * (q16 & 1));
  if (q16 >= 2) qf[2] = z8;                     // dims 80..95

  // tile chunk u of this thread: index i = ht + 256 u; i < 640 is K (row i / 10, chunk
  // i % 10), the rest V
  int trow[VA_NLD], tsrc[VA_NLD], tdst[VA_NLD];
  bool tv[VA_NLD];
#pragma unroll
  for (int u = 0; u < VA_NLD; ++u) {
    const int i = ht + 256 * u;
    tv[u] = i >= VA_KT * VA_CPR;
    const int j = tv[u] ? i - VA_KT * VA_CPR : i;
    trow[u] = j / VA_CPR;
    const int ch = j - trow[u] * VA_CPR;
    tsrc[u] = (tv[u] ? 2 : 1) * a.nh * VA_HD + h * VA_HD + ch * 8;
    tdst[u] = tv[u] ? trow[u] * VA_VSTR + ch * 8 : trow[u] * VA_KSTR + ch * 8;
  }
  half8_t tr[VA_NLD];
  const int tok_hi = max(kend, kbeg + 1) - 1;   // a half without tiles re-reads one row
  auto load_tile = [&](int kb) {
#pragma unroll
    for (int u = 0; u < VA_NLD; ++u) {
      const int tok = min(min(kb + trow[u], tok_hi), a.S - 1);
      tr[u] = *(const half8_t*)(a.qkv + (int64_t)tok * a.ld + tsrc[u]);
    }
  };
  auto store_tile = [&](int b) {
#pragma unroll
    for (int u = 0; u < VA_NLD; ++u) {
      half_t* dst = tv[u] ? &vs_lds[kh][b][tdst[u]] : &ks_lds[kh][b][tdst[u]];
      *(half8_t*)dst = tr[u];
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o_acc[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) o_acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // Double buffer per half: tile n is staged in buffer n & 1; the barrier after staging
  // tile n also means every wave has finished reading that buffer's previous tile (n - 2).
  // Both halves run the larger half's tile count so that every wave meets every barrier.
  const int nt_all = nt0;                       // the first half is never the smaller
  int b = 0;
  load_tile(kbeg);
  for (int it = 0; it < nt_all; ++it, b ^= 1) {
    const int kb = kbeg + it * VA_KT;
    store_tile(b);
    __syncthreads();
    if (it + 1 < my_nt) load_tile(kb + VA_KT);
    if (it >= my_nt) continue;                  // this half is done (barriers still met)
    const half_t* kt = ks_lds[kh][b];
    const half_t* vt = vs_lds[kh][b];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {             // 32-key halves of the tile
      const int k0 = kb + 32 * hb;
      if (k0 >= kend) break;
      f32x4 sacc[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 3; ++ks) {
          const half8_t kf = *(const half8_t*)(kt + (32 * hb + 16 * j + c16) * VA_KSTR + 32 * ks + 8 * q16);
          acc = mfma16x16x32(kf, qf[ks], acc);
        }
        sacc[j] = acc;
      }
      // lane holds scores of keys k0 + 16 j + 4 q16 + i for query c16
      float sc[8];
      float mblk = -INFINITY;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + 16 * j + 4 * q16 + i;
          const float s = key < kend ? sacc[j][i] * a.scale_log2 : -INFINITY;
          sc[4 * j + i] = s;
          mblk = fmaxf(mblk, s);
        }
      mblk = fmaxf(mblk, __shfl_xor(mblk, 16, 64));
      mblk = fmaxf(mblk, __shfl_xor(mblk, 32, 64));
      const float m_new = fmaxf(m_run, mblk);      // finite: key k0 < kend is visible
      const float alpha = exp2f(m_run - m_new);
      m_run = m_new;
      half8_t pa;
      float psum = 0.f;
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) {
        const float p = exp2f(sc[s8] - m_new);
        psum += p;
        pa[s8] = (half_t)p;
      }
      l_run = l_run * alpha + psum;
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * q16 + i, 64);
#pragma unroll
      for (int dt = 0; dt < 5; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) o_acc[dt][i] *= al[i];
#pragma unroll
      for (int dt = 0; dt < 5; ++dt) {
        const half8_t vb = lds_read_b_tr16(vt + 32 * hb * VA_VSTR + dt * 16, VA_VSTR, q16, c16);
        o_acc[dt] = mfma16x16x32(pa, vb, o_acc[dt]);
      }
    }
  }
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  // per query row 4 q16 + i of this lane: the half's running max and sum
  float mi[4], li[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mi[i] = __shfl(m_run, 4 * q16 + i, 64);
    li[i] = __shfl(l_run, 4 * q16 + i, 64);
  }
  if constexpr (KH == 2) {
    // merge: the second half hands its (max, sum, O) to the first through LDS (the tile
    // buffers are free once every wave is past the loop)
    __syncthreads();
    float* xch = (float*)&ks_lds[0][0][0];      // [4 query waves][64 lanes][4 m + 4 l + 20 O]
    float* my = xch + (qw * 64 + lane) * 28;
    if (kh == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        my[i] = mi[i];
        my[4 + i] = li[i];
      }
#pragma unroll
      for (int dt = 0; dt < 5; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) my[8 + 4 * dt + i] = o_acc[dt][i];
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float m1 = my[i], l1 = my[4 + i];
      const float m = fmaxf(mi[i], m1);         // finite: the first half is never empty
      const float f0 = exp2f(mi[i] - m), f1 = exp2f(m1 - m);   // m1 = -inf -> 0
      li[i] = li[i] * f0 + l1 * f1;
#pragma unroll
      for (int dt = 0; dt < 5; ++dt) o_acc[dt][i] = o_acc[dt][i] * f0 + my[8 + 4 * dt + i] * f1;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = q0 + 16 * qw + 4 * q16 + i;
    if (t < end && t < q0 + 64) {
      half_t* op = a.out + (int64_t)t * a.ldo + h * VA_HD;
      const float inv = 1.0f / li[i];
#pragma unroll
      for (int dt = 0; dt < 5; ++dt) op[dt * 16 + c16] = (half_t)(o_acc[dt][i] * inv);
    }
  }
}

// Non-causal attention within segments over the qkv rows (q | k | v heads, head_dim 80,
// row stride ld), already rotated.  cu int32 [nseg + 1] (cu[0] = 0, increasing, cu[nseg]
// = S); tiles int32 [ntiles][2] = (first query, segment) covering every segment in steps
// of 64 queries; out fp16 [S][ldo] (head h at column 80 h).
extern "C" int omni_vit_attention(const void* qkv, int ld, int S, int n_heads, int head_dim,
                                  const int* cu_seqlens, const int* tiles, int ntiles, void* out,
                                  int ldo, float scale, void* stream) {
  if (S < 0 || n_heads <= 0 || ntiles < 0) return OMNI_EINVAL;
  if (head_dim != VA_HD) return OMNI_EUNSUPPORTED;
  if (S == 0 || ntiles == 0) return OMNI_OK;
  if (!qkv || !cu_seqlens || !tiles || !out) return OMNI_EINVAL;
  if (ld < 3 * n_heads * VA_HD || (ld & 7) || ldo < n_heads * VA_HD) return OMNI_EINVAL;
  const int64_t grid = (int64_t)ntiles * n_heads;
  if (grid > 0x7fffffff) return OMNI_EUNSUPPORTED;
  VitAttnArgs a;
  a.qkv = (const half_t*)qkv;
  a.ld = ld;
  a.cu = cu_seqlens;
  a.tiles = tiles;
  a.ntiles = ntiles;
  a.nh = n_heads;
  a.S = S;
  a.out = (half_t*)out;
  a.ldo = ldo;
  a.scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(vit_attn_kernel<2>, dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

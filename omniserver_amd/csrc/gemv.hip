// Weight-streaming skinny GEMM for decode (M <= 64 activation rows):
//   out[M, N] = x[M, K] . W^T,  W int4 (GPTQ uint4b8, group 128 along K) or fp16.
//
// Replaces the decode-time calls of the reference's linear modules:
//   GPTQ int4   omniserve/kernels/marlin_linear.py:54-62, 83-96  (W = fp16((q-8)*s),
//               y = fp16(x.W), bias added after the fp16 rounding)
//   fp16        nn.Linear in omniserve/model/qwen2_llm.py:82-83, 120-121, 167
//   lm_head     qwen2_llm.py:167-168, 190 + greedy argmax runners/multimodal.py:306-310
//
// Packed layouts (built once at load time by omni_gptq_repack / omni_f16_pack):
//   int4  qp u32 [N/16][K/128][64 lanes][4]: word j of lane l holds the 8 codes of
//         column 16*nt + l%16, k = 128*kg + 32*j + 8*(l/16) + e, e = 0..7, code e at
//         bit 2e (e even) or 16+2(e-1) (e odd); scales sp fp16 [N/16][K/128][16].
//   fp16  wp     [N/16][K/32][64 lanes][8]: lane l holds column 16*nt + l%16,
//         k = 32*ks + 8*(l/16) + e.
// One 16-byte load per lane is one MFMA 16x16x32 B operand set (four of them for
// int4); a wavefront reads 1 KB contiguous per load; the int4 dequant is the
// magic-exponent trick on packed fp16.
//
// Work split (no cross-workgroup synchronisation anywhere: on this multi-XCD part a
// device-scope fence costs an L2 write-back/invalidate per workgroup, far more than
// the work it would order):
//   * a workgroup owns CW*CPW column tiles of 16 and one K range (all of K, or one of
//     KS slices); it has CW*KW waves: wave (cw, kw) streams its CPW tiles over the
//     kw-th part of the range, issuing its first weight loads before x is staged;
//   * x[:, range] is staged once per workgroup in LDS (loads batched, then stored);
//   * the KW partial accumulators are summed in LDS (fixed order) and the epilogue
//     runs once:
//       STORE    fp16 out (+ bias)                                  KS == 1
//       SILU     tiles (2p, 2p+1) = (gate, up) -> fp16 silu(g)*u    KS == 1
//       PARTIAL  fp32 [KS][M][N] partial sums; the consumer kernel adds them in
//                slice order (deterministic)
//       ARGMAX   per-workgroup (max fp16 logit, lowest index) per row -> candidate
//                arrays reduced by omni_argmax_finalize.
#include "common.h"

#include <mutex>
#include <type_traits>

enum { W_INT4 = 0, W_FP16 = 1 };
enum { EPI_STORE = 0, EPI_SILU = 1, EPI_PARTIAL = 2, EPI_ARGMAX = 3, EPI_QGELU = 4, EPI_GELU = 5,
       EPI_RESID = 6 };

struct GemvArgs {
  const half_t* x;
  int ldx;
  const void* w;
  const half_t* scales;
  const half_t* bias;
  int bias_after_round;  // 1: fp16(fp16(acc) + b) (GPTQ path); 0: fp16(acc + b)
  half_t* out;
  int ldo;
  float* partial;        // EPI_PARTIAL: [KS][M][N]
  float* cand_val;       // EPI_ARGMAX: [gridDim][M]
  int* cand_idx;
  int M, N, K;
  int KS;                // K slices across workgroups
  int KC;                // K per slice (multiple of 128)
  int xl;                // 1: x slice staged in LDS; 0: A fragments read from global
  // x from split decode-attention states (XS == 1): x[m, h*128 + d] = merge over the aS
  // splits of the states [M][a_nkv][aS][aG][ATT_REC] of head h (kv head h / aG).
  const float* apart;
  int aS, a_nkv, aG;
  // tiled kernel only: x columns [kx, K) read as zero (kx % 8 == 0); EPI_RESID adds res
  int kx;
  const half_t* res;
  int ldr;
  // x from an add+RMSNorm of the previous projection's split-K partials (XS == 2):
  //   h[m, :] = fp16(fp16(sum of nparts fp32 slices [nnp][M][K], slice order) + nres[m, :]),
  //   x[m, :] = fp16((h * rstd_m) * ngain), rstd_m = 1 / sqrt(sum(h^2) / K + neps),
  // every workgroup forming its rows' statistics; logical block 0 writes h to nres_out.
  const float* nparts;
  int nnp;
  const half_t* nres;
  const half_t* ngain;
  half_t* nres_out;
  float neps;
};

template <int WF>
struct WFrag;
template <>
struct WFrag<W_INT4> {
  u32x4 q;
  half_t s;
};
template <>
struct WFrag<W_FP16> {
  half8_t h[4];
};

// Per-wave weight stream of one column tile: fragments of consecutive k-groups.
template <int WF>
struct WStream;
template <>
struct WStream<W_INT4> {
  const u32x4* q;      // group g at q + 64 g
  const half_t* s;     // group g at s + 16 g
  __device__ void init(const GemvArgs& a, int nt, int kg0, int lane) {
    const int64_t blk = (int64_t)nt * (a.K >> 7) + kg0;
    q = (const u32x4*)a.w + blk * 64 + lane;
    s = a.scales + blk * 16 + (lane & 15);
  }
  __device__ __forceinline__ void load(WFrag<W_INT4>& f, int g) const {
    f.q = __builtin_nontemporal_load(q + g * 64);
    f.s = s[g * 16];
  }
};
template <>
struct WStream<W_FP16> {
  const half8_t* h;    // group g, sub-block j at h + (4 g + j) * 64
  __device__ void init(const GemvArgs& a, int nt, int kg0, int lane) {
    h = (const half8_t*)a.w + ((int64_t)nt * (a.K >> 5) + kg0 * 4) * 64 + lane;
  }
  __device__ __forceinline__ void load(WFrag<W_FP16>& f, int g) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) f.h[j] = __builtin_nontemporal_load(h + (4 * g + j) * 64);
  }
};


// x * sigmoid(1.702 x) with the three fp16 roundings of the reference's elementwise ops
// (model/qwen2_vit.py:18-19 on fp16 tensors: 1.702 x, sigmoid, product).
__device__ __forceinline__ half_t quick_gelu_ref(half_t h) {
#pragma clang fp contract(off)
  const float t = (float)(half_t)((float)h * 1.702f);
  const float sg = (float)(half_t)(1.0f / (1.0f + expf(-t)));
  return (half_t)((float)h * sg);
}

// Exact (erf) GELU of an fp16 value, fp32 math, one rounding (F.gelu, model/qwen2_vit.py:128).
__device__ __forceinline__ half_t gelu_erf_ref(half_t h) {
#pragma clang fp contract(off)
  const float x = (float)h;
  return (half_t)(0.5f * x * (1.0f + erff(x * 0.70710678118654752f)));
}

__device__ __forceinline__ half_t finish_store(float v, const GemvArgs& a, int n) {
#pragma clang fp contract(off)
  if (a.bias) {
    const float b = (float)a.bias[n];
    if (a.bias_after_round) return (half_t)((float)(half_t)v + b);
    return (half_t)(v + b);
  }
  return (half_t)v;
}

// Dynamic LDS: the x tile [MB*16 rows][KC + 8 halfs], reused for the KW reduction.
// XF = 1: x is staged in LDS before any weight is requested (for a projection whose
// workgroups stage a large x, so that x does not queue behind the grid's weight stream);
// XF = 0: the weight stream is issued first and staging overlaps it.
template <int WF, int MB, int EPI, int CPW, int CW, int KW, int PF, int XS = 0, int XF = 0>
__global__ __launch_bounds__(CW * KW * 64, 1) void gemv_kernel(GemvArgs a) {
#pragma clang fp contract(off)
  static_assert(EPI != EPI_ARGMAX || KW == 1, "argmax epilogue uses every wave of the workgroup");
  constexpr int NW = CW * KW;
  constexpr int NT_WG = CW * CPW;     // column tiles per workgroup
  extern __shared__ __attribute__((aligned(16))) char smem[];
  half_t* xs = (half_t*)smem;

  // Every kernel argument is read into registers in one batch first: scalar loads complete
  // out of order, so a wait for any one of them waits for all, and an argument fetched
  // after the first wait costs the launch another round trip before its loads go out.
  asm volatile("" ::"s"(a.x), "s"(a.ldx), "s"(a.w), "s"(a.scales), "s"(a.bias),
               "s"(a.bias_after_round), "s"(a.out), "s"(a.ldo), "s"(a.partial), "s"(a.M),
               "s"(a.N), "s"(a.K), "s"(a.KS), "s"(a.KC), "s"(a.xl), "s"(a.apart), "s"(a.aS),
               "s"(a.a_nkv), "s"(a.aG), "s"(gridDim.x));
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int cw = wave % CW;
  const int kw = wave / CW;
  const int q16 = lane >> 4;
  const int c16 = lane & 15;
  const int NT = a.N >> 4;
  const int ngroups = (NT + NT_WG - 1) / NT_WG;
  // XCD-aware order: the workgroups of one K slice (same x, different columns) share an L2
  const int blk = xcd_logical_block(blockIdx.x, gridDim.x);
  const int ng = blk % ngroups;
  const int ksi = blk / ngroups;
  const int k0 = ksi * a.KC;
  const int kc = min(a.KC, a.K - k0);          // multiple of 128
  const int xstride = a.KC + 8;
  const int ngk = kc >> 7;                      // k-groups in this slice
  const int per = (ngk + KW - 1) / KW;          // k-groups per wave
  const int g_beg = min(kw * per, ngk);
  const int g_end = min(g_beg + per, ngk);
  const int kg0 = (k0 >> 7) + g_beg;
  const int myg = g_end - g_beg;

  const int tile0 = ng * NT_WG + cw * CPW;
  const bool active = tile0 < NT;

  // x chunk (row r, 8-column chunk c) of the staged slice for flat index i = r*cpr + c:
  // the thread's first index is threadIdx.x and it advances by a whole workgroup each
  // step, so (r, c) is stepped instead of divided (one division per thread).
  const int cpr = kc >> 3;
  const int xtotal = MB * 16 * cpr;
  constexpr int NTH = NW * 64;
  const int step_r = NTH / cpr;
  const int step_c = NTH - step_r * cpr;
  int xr = threadIdx.x / cpr;
  int xc = threadIdx.x - xr * cpr;
  auto xstep = [&]() {
    xc += step_c;
    xr += step_r;
    if (xc >= cpr) {
      xc -= cpr;
      ++xr;
    }
  };

  // 1. The first batch of x loads goes out before the weight loads: x is small and
  //    cache-resident, and loads retire in issue order, so staging it never waits on
  //    the weight stream.  The code is branch-free (clamped addresses) so that the
  //    compiler's wait counts stay exact; a chunk past the slice is marked with the
  //    row-0 pad offset (KC) and not stored.  Rows past M stage row 0's values, stored
  //    as loaded: their products are never stored (every epilogue skips rows >= M, and an
  //    MFMA row depends only on its own A row), and a select on the loaded value would
  //    let the compiler consume - wait for - each x load right after issuing it, ahead
  //    of the weight loads.
  half8_t xv[8];
  int xo[8];
  bool xlive[8];
  // XS == 2: thread t holds chunk n_c of row n_r (t = n_r nch + n_c, whole waves per row);
  // NB partial slices in flight per thread (8 where three waves share a SIMD's registers)
  constexpr int NB = XS == 2 ? (NW > 8 ? 8 : 16) : 1;
  const int n_nch = a.K >> 3;
  const int n_r = XS == 2 ? (int)threadIdx.x / n_nch : 0;
  const int n_c = XS == 2 ? (int)threadIdx.x - n_r * n_nch : 0;
  const int n_rr = n_r < a.M ? n_r : 0;
  float4 n_lo[NB], n_hi[NB];
  half8_t n_rv, n_gv;
  const bool x_single = XS == 1 ? (xtotal <= NTH && a.aS <= 8) : true;
  Merge8Loads ml;
  int m_rec = a.KC;                             // XS: LDS offset of this thread's chunk
  bool m_live = false;
  if constexpr (XS == 1) {
    if (x_single) {
      const bool ok = (int)threadIdx.x < xtotal;
      m_live = ok && xr < a.M;
      m_rec = ok ? xr * xstride + xc * 8 : a.KC;
      const int rr = m_live ? xr : 0;
      const int k = k0 + (ok ? xc : 0) * 8;
      const int head = k >> 7;
      const float* rec0 = a.apart + ((((int64_t)rr * a.a_nkv + head / a.aG) * a.aS) * a.aG +
                                     head % a.aG) * ATT_REC;
      attn_merge8_issue(ml, rec0, (int64_t)a.aG * ATT_REC, 0, a.aS, k & 127);
    }
  } else if (XS == 2) {
    // the rows' first NB partial slices, residual and gain, requested before the weights
    // (loads retire in order: issued after them, the norm would wait for the whole stream)
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int p = u < a.nnp ? u : a.nnp - 1;
      const float4* pp = (const float4*)(a.nparts + ((int64_t)p * a.M + n_rr) * a.K + n_c * 8);
      n_lo[u] = pp[0];
      n_hi[u] = pp[1];
    }
    n_rv = *(const half8_t*)(a.nres + (int64_t)n_rr * a.K + n_c * 8);
    n_gv = *(const half8_t*)(a.ngain + n_c * 8);
  } else if (XS == 0 && a.xl) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool ok = (int)threadIdx.x + u * NTH < xtotal;
      xlive[u] = ok && xr < a.M;
      const int rr = xlive[u] ? xr : 0;
      const int cc = ok ? xc : 0;
      xv[u] = *(const half8_t*)(a.x + (int64_t)rr * a.ldx + k0 + cc * 8);
      xo[u] = ok ? xr * xstride + xc * 8 : a.KC;
      xstep();
    }
  }

  // 2. weight loads: PF groups of every tile in flight.  Issued unconditionally (tiles
  //    and groups past the end re-read the last valid one) so the wait counts of the
  //    code below are exact instead of assuming the worst case.
  WStream<WF> ws[CPW];
  WFrag<WF> buf[PF][CPW];
  auto issue_weights = [&]() {
    // a wave without groups re-reads the slice's first group (loaded by wave kw = 0,
    // so it is served from cache, not HBM)
    const int gmax = myg > 0 ? myg - 1 : 0;
    const int kgb = myg > 0 ? kg0 : (k0 >> 7);
#pragma unroll
    for (int c = 0; c < CPW; ++c) ws[c].init(a, min(tile0 + c, NT - 1), kgb, lane);
#pragma unroll
    for (int p = 0; p < PF; ++p)
#pragma unroll
      for (int c = 0; c < CPW; ++c) ws[c].load(buf[p][c], min(p, gmax));
  };
  if constexpr (!XF || XS == 2) issue_weights();

  // 3. finish staging x[0:M, k0:k0+kc] in LDS (rows >= M zero)
  const half8_t zero8 = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
  auto stage_x = [&]() {
    if constexpr (XS == 1) {
      if (x_single) {
        Merge8State st;
        attn_merge8_batch(st, ml, a.aS);
        if (m_rec != a.KC) *(half8_t*)(xs + m_rec) = m_live ? attn_merge8_result(st) : zero8;
      } else {
        const int64_t sstride = (int64_t)a.aG * ATT_REC;
        for (int i = threadIdx.x; i < xtotal; i += NTH) {
          half8_t v = zero8;
          if (xr < a.M) {
            const int k = k0 + xc * 8;
            const int head = k >> 7;
            const float* rec0 = a.apart + ((((int64_t)xr * a.a_nkv + head / a.aG) * a.aS) * a.aG +
                                           head % a.aG) * ATT_REC;
            v = attn_merge8(rec0, sstride, a.aS, k & 127);
          }
          *(half8_t*)(xs + xr * xstride + xc * 8) = v;
          xstep();
        }
      }
    } else if (XS == 2) {
      // add+RMSNorm of the M rows, one 8-element chunk per thread (row r = t / nch, whole
      // waves per row), in rownorm_kernel's order: the slices summed in order and rounded,
      // the residual added and rounded, the squares summed per chunk, per wave, then over
      // the row's waves in order.  The weights are already in flight: the sums wait for
      // them (loads retire in order), which is at most one round trip.
#pragma clang fp contract(off)
      __shared__ float nws[16];
      const int nch = n_nch;                    // multiple of 64 (host check)
      const int r = n_r;
      const int c = n_c;
      const bool live = r < a.M;                // M nch <= threads (host check)
      const int rr = n_rr;
      float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < NB; ++u) {            // slices 0 .. NB-1 (a slot past nnp adds +0)
        const bool on = u < a.nnp;
        sum[0] += on ? n_lo[u].x : 0.f; sum[1] += on ? n_lo[u].y : 0.f;
        sum[2] += on ? n_lo[u].z : 0.f; sum[3] += on ? n_lo[u].w : 0.f;
        sum[4] += on ? n_hi[u].x : 0.f; sum[5] += on ? n_hi[u].y : 0.f;
        sum[6] += on ? n_hi[u].z : 0.f; sum[7] += on ? n_hi[u].w : 0.f;
      }
      if (a.nnp > NB)                           // the rest, in order (behind the weights)
        sum_slices8<NB>(a.nparts + ((int64_t)NB * a.M + rr) * a.K + c * 8, (int64_t)a.M * a.K,
                        a.nnp - NB, sum);
      const half8_t rv = n_rv;
      const half8_t gv = n_gv;
      half8_t v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (half_t)sum[e];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (half_t)((float)v[e] + (float)rv[e]);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
      ss = wave_sum(ss);
      if ((threadIdx.x & 63) == 0) nws[threadIdx.x >> 6] = ss;
      lds_barrier();
      const int w0 = (rr * nch) >> 6;
      float tot = 0.f;
      for (int i = 0; i < (nch >> 6); ++i) tot += nws[w0 + i];
      const float rstd = 1.0f / sqrtf(tot / (float)a.K + a.neps);
      if (live) {
        if (blk == 0) *(half8_t*)(a.nres_out + (int64_t)r * a.K + c * 8) = v;
        const int kk = c * 8 - k0;
        if (kk >= 0 && kk < kc) {
          half8_t o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (half_t)(((float)v[e] * rstd) * (float)gv[e]);
          *(half8_t*)(xs + r * xstride + kk) = o;
        }
      }
    } else if (a.xl) {
      // (a chunk past the slice stores nothing: many lanes writing one pad address would
      // serialise on its LDS bank)
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (xo[u] != a.KC) *(half8_t*)(xs + xo[u]) = xv[u];
      for (int base = threadIdx.x + 8 * NTH; base < xtotal; base += 8 * NTH) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool ok = base + u * NTH < xtotal;
          xlive[u] = ok && xr < a.M;
          const int rr = xlive[u] ? xr : 0;
          const int cc = ok ? xc : 0;
          xv[u] = *(const half8_t*)(a.x + (int64_t)rr * a.ldx + k0 + cc * 8);
          xo[u] = ok ? xr * xstride + xc * 8 : a.KC;
          xstep();
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (xo[u] != a.KC) *(half8_t*)(xs + xo[u]) = xv[u];
      }
    }
  };
  if constexpr (XF && XS != 2) {
    stage_x();
    __syncthreads();
    issue_weights();
  } else {
    stage_x();
    lds_barrier();   // the weight stream stays in flight across the barrier
  }

  // 3. stream weights, MFMA against x from LDS
  f32x4 acc[CPW][MB];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[c][mb] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // The A-fragment source is chosen once, outside the loop: a runtime branch inside it
  // makes the compiler wait for every outstanding weight load at each fragment read.
  auto stream_weights = [&](auto xl_const) {
    constexpr bool XL = decltype(xl_const)::value;
    auto group = [&](WFrag<WF>(&fr)[CPW], int i) {
      const int kl = (g_beg + i) * 128;           // k offset inside the staged slice
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        half8_t af[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          if constexpr (XL) {
            af[mb] = *(const half8_t*)(xs + (16 * mb + c16) * xstride + kl + 32 * j + 8 * q16);
          } else {
            const int m = 16 * mb + c16;
            af[mb] = m < a.M ? *(const half8_t*)(a.x + (int64_t)m * a.ldx + k0 + kl + 32 * j + 8 * q16)
                             : (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
          }
        }
#pragma unroll
        for (int c = 0; c < CPW; ++c) {
          half8_t bf;
          if constexpr (WF == W_INT4) {
            const half2_t s2 = {fr[c].s, fr[c].s};
            bf = dequant8(fr[c].q[j], s2);
          } else {
            bf = fr[c].h[j];
          }
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[c][mb] = mfma16x16x32(af[mb], bf, acc[c][mb]);
        }
      }
    };
    // The prefetched groups are consumed in straight-line code (a loop carrying the
    // fragment registers would copy them at entry, waiting for every load first).
#pragma unroll
    for (int p = 0; p < PF; ++p)
      if (p < myg) group(buf[p], p);
    // Groups beyond the prefetch depth (long K per wave): load a batch, then use it.
    for (int base = PF; base < myg; base += PF) {
#pragma unroll
      for (int p = 0; p < PF; ++p)
#pragma unroll
        for (int c = 0; c < CPW; ++c) ws[c].load(buf[p][c], min(base + p, myg - 1));
#pragma unroll
      for (int p = 0; p < PF; ++p)
        if (base + p < myg) group(buf[p], base + p);
    }
  };
  if (active) {
    if (XS != 0 || a.xl) stream_weights(std::true_type{});
    else stream_weights(std::false_type{});
  }

  // 4. sum the KW partial accumulators in LDS, in kw order
  if constexpr (KW > 1) {
    __syncthreads();                              // the x tile is no longer read
    f32x4* red = (f32x4*)smem;                    // [KW-1][CW][CPW][MB][64 lanes] x 4
    if (kw > 0) {
#pragma unroll
      for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          red[((((kw - 1) * CW + cw) * CPW + c) * MB + mb) * 64 + lane] = acc[c][mb];
    }
    __syncthreads();
    if (kw > 0) return;                           // no workgroup barrier follows
#pragma unroll
    for (int k2 = 1; k2 < KW; ++k2)
#pragma unroll
      for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[c][mb] += red[((((k2 - 1) * CW + cw) * CPW + c) * MB + mb) * 64 + lane];
  }
  // Lane holds rows 16*mb + 4*q16 + i, column (tile0 + c)*16 + c16.

  if constexpr (EPI == EPI_ARGMAX) {
    __shared__ float red_v[CW][MB * 16];
    __shared__ int red_i[CW][MB * 16];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 16 * mb + 4 * q16 + i;
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        if (active) {
#pragma unroll
          for (int c = 0; c < CPW; ++c) {
            const int n = (tile0 + c) * 16 + c16;
            const half_t h = (half_t)acc[c][mb][i];
            if (a.out && m < a.M) a.out[(int64_t)m * a.ldo + n] = h;
            const float v = (float)h;
            if (v > bv) { bv = v; bi = n; }
          }
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          const float ov = __shfl_xor(bv, o, 64);
          const int oi = __shfl_xor(bi, o, 64);
          if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (c16 == 0) {
          red_v[cw][m] = bv;
          red_i[cw][m] = bi;
        }
      }
    __syncthreads();
    if (threadIdx.x < a.M) {
      const int m = threadIdx.x;
      float bv = red_v[0][m];
      int bi = red_i[0][m];
#pragma unroll
      for (int w = 1; w < CW; ++w) {
        const float ov = red_v[w][m];
        const int oi = red_i[w][m];
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      a.cand_val[(int64_t)blockIdx.x * a.M + m] = bv;
      a.cand_idx[(int64_t)blockIdx.x * a.M + m] = bi;
    }
    return;
  } else {
    if (!active) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 16 * mb + 4 * q16 + i;
        if (m >= a.M) continue;
        if constexpr (EPI == EPI_SILU) {
          // tiles (2p, 2p+1) = (gate, up) columns 16p + c16 of the intermediate.
          const int j = (tile0 >> 1) * 16 + c16;
          const float g = (float)(half_t)acc[0][mb][i];
          const float u = (float)(half_t)acc[1][mb][i];
          a.out[(int64_t)m * a.ldo + j] = (half_t)silu_mul_f32(g, u);
        } else if constexpr (EPI == EPI_PARTIAL) {
#pragma unroll
          for (int c = 0; c < CPW; ++c) {
            const int n = (tile0 + c) * 16 + c16;
            a.partial[((int64_t)ksi * a.M + m) * a.N + n] = acc[c][mb][i];
          }
        } else {
#pragma unroll
          for (int c = 0; c < CPW; ++c) {
            const int n = (tile0 + c) * 16 + c16;
            a.out[(int64_t)m * a.ldo + n] = finish_store(acc[c][mb][i], a, n);
          }
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch.  Presets (CPW, CW, KW):
//   0: (1, 8, 2)  16 waves, 8 tiles = 128 columns per workgroup, K halved in-group
//   1: (1, 8, 1)   8 waves, 8 tiles
//   2: (1, 4, 4)  16 waves, 4 tiles, K in quarters
//   3: (2, 4, 2)   8 waves, 8 tiles
// SiLU (gate/up pairs, CPW = 2): 0: (2, 4, 4), 1: (2, 8, 1), 2: (2, 4, 2), 3: (2, 2, 4),
//   4: (2, 3, 4) (6 tiles: 187 workgroups for the 2B decoder's gate_up), 5: (2, 2, 8);
//   6, 7, 8, 9: (2, 3, 4), (2, 2, 4), (2, 4, 4), (2, 8, 1) with x staged first (XF).
// Argmax: (2, 8, 1) (16 tiles).
// ---------------------------------------------------------------------------
static size_t max_dynamic_lds() {
  static int cached = -1;
  if (cached < 0) {
    int dev = 0, v = 65536;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      v = 65536;
    cached = v;
  }
  return (size_t)cached > 4096 ? (size_t)cached - 4096 : 0;
}

template <int WF, int MB, int EPI, int CPW, int CW, int KW, int PF, int XS, int XF>
static int launch_gemv(GemvArgs a, hipStream_t st) {
  auto kern = gemv_kernel<WF, MB, EPI, CPW, CW, KW, PF, XS, XF>;
  const size_t lim = max_dynamic_lds();
  const size_t xbytes = (size_t)MB * 16 * (a.KC + 8) * sizeof(half_t);
  const size_t rbytes = (size_t)(KW > 1 ? KW - 1 : 0) * CW * CPW * MB * 256 * sizeof(float);
  a.xl = xbytes <= lim;                         // else A fragments come from global/L2
  if (XS != 0 && !a.xl) return OMNI_EUNSUPPORTED;   // merged / normalised input: LDS only
  if (XS == 2 && a.M * (a.K >> 3) > CW * KW * 64) return OMNI_EUNSUPPORTED;   // a chunk a thread
  const size_t lds = a.xl ? (xbytes > rbytes ? xbytes : rbytes) : rbytes;
  if (lds > lim) return OMNI_EUNSUPPORTED;
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lim);
    attr_set = true;
  }
  const int NT = a.N >> 4;
  const int ngroups = (NT + CW * CPW - 1) / (CW * CPW);
  const int grid = ngroups * a.KS;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(CW * KW * 64), lds, st, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

template <int WF, int EPI, int CPW, int CW, int KW, int PF, int XS = 0, int XF = 0>
static int dispatch_mb(const GemvArgs& a, hipStream_t st) {
  switch ((a.M + 15) / 16) {
    case 1: return launch_gemv<WF, 1, EPI, CPW, CW, KW, PF, XS, XF>(a, st);
    case 2: return launch_gemv<WF, 2, EPI, CPW, CW, KW, PF, XS, XF>(a, st);
    case 3: return launch_gemv<WF, 3, EPI, CPW, CW, KW, PF, XS, XF>(a, st);
    case 4: return launch_gemv<WF, 4, EPI, CPW, CW, KW, PF, XS, XF>(a, st);
    default: return OMNI_EUNSUPPORTED;
  }
}

template <int WF, int EPI, int XS = 0>
static int dispatch_preset(const GemvArgs& a, int preset, hipStream_t st) {
  // weight groups in flight per column tile: 4 for int4 (16 bytes per lane and group), 2 for
  // fp16 (64 bytes; 4 kept twice the bytes in flight and measured 12 % slower fp16 steps)
  constexpr int PF = WF == W_FP16 ? 2 : 4;
  // Presets whose register demand at 64 rows exceeds a wave's share (8-wave K splits of
  // two tiles per wave, and every form with the merged attention input but preset 1) are
  // not built: they spilled without being faster at the shapes they were swept on.
  if constexpr (XS == 2) {        // add+RMSNorm input: one row block, the decode plans' shapes
    if constexpr (EPI == EPI_SILU) {
      switch (preset) {
        case 1: return launch_gemv<WF, 1, EPI, 2, 8, 1, PF, 2, 0>(a, st);
        case 4: return launch_gemv<WF, 1, EPI, 2, 3, 4, PF, 2, 0>(a, st);
        default: return OMNI_EINVAL;
      }
    } else {
      return preset == 1 ? launch_gemv<WF, 1, EPI, 1, 8, 1, PF, 2, 0>(a, st) : OMNI_EINVAL;
    }
  } else if constexpr (EPI == EPI_SILU) {
    switch (preset) {
      case 1: return dispatch_mb<WF, EPI, 2, 8, 1, PF>(a, st);
      case 2: return dispatch_mb<WF, EPI, 2, 4, 2, PF>(a, st);
      case 3: return dispatch_mb<WF, EPI, 2, 2, 4, PF>(a, st);
      case 4: return dispatch_mb<WF, EPI, 2, 3, 4, PF>(a, st);
      // x staged before the weights are requested (XF)
      case 6: return dispatch_mb<WF, EPI, 2, 3, 4, PF, 0, 1>(a, st);
      case 7: return dispatch_mb<WF, EPI, 2, 2, 4, PF, 0, 1>(a, st);
      case 9: return dispatch_mb<WF, EPI, 2, 8, 1, PF, 0, 1>(a, st);
      default: return OMNI_EINVAL;
    }
  } else if constexpr (EPI == EPI_ARGMAX) {
    return dispatch_mb<WF, EPI, 2, 8, 1, PF>(a, st);
  } else if constexpr (XS == 1) {
    return preset == 1 ? dispatch_mb<WF, EPI, 1, 8, 1, PF, XS>(a, st) : OMNI_EINVAL;
  } else {
    switch (preset) {
      case 0: return dispatch_mb<WF, EPI, 1, 8, 2, PF, XS>(a, st);
      case 1: return dispatch_mb<WF, EPI, 1, 8, 1, PF, XS>(a, st);
      case 2: return dispatch_mb<WF, EPI, 1, 4, 4, PF, XS>(a, st);
      case 3: return dispatch_mb<WF, EPI, 2, 4, 2, PF, XS>(a, st);
      default: return OMNI_EINVAL;
    }
  }
}

// ---------------------------------------------------------------------------
// Tiled GEMM for many activation rows (prefill: M = packed prompt tokens), same packed
// weight layouts and epilogues (STORE: fp16(acc) + bias, SILU: gate/up tile pairs) as
// the skinny kernel above.
//
// One workgroup (4 waves, 2 x 2) owns a 128 (m) x 128 (n) output tile; wave (wm, wn) owns
// rows 64 wm .. +63 and column tiles 4 wn .. +3 of it (4 x 4 MFMA 16x16x32 accumulators).
// K advances one 128-group at a time: the x tile [128 x 128] fp16 is staged in LDS
// (double buffered, loaded one group ahead into registers), the weight fragments are
// read straight from the packed layout into registers (one 16-byte load per lane and
// column tile for int4, four for fp16), also one group ahead.  Each staged x fragment
// feeds 4 MFMAs and each weight fragment 4, per 32-k step.
// ---------------------------------------------------------------------------
#define GT_BM 128
#define GT_BN 128
#define GT_XSTRIDE 136     // LDS halfs per staged x row (128 + 8 pad)

template <int WF, int EPI>
__global__ __launch_bounds__(256, 1) void gemm_tile_kernel(GemvArgs a) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) half_t xs[2][GT_BM * GT_XSTRIDE];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int q16 = lane >> 4, c16 = lane & 15;
  const int NT = a.N >> 4;
  const int tiles_n = (a.N + GT_BN - 1) / GT_BN;
  const int tiles_m = (a.M + GT_BM - 1) / GT_BM;
  // XCD-aware, grouped order: the tiles one XCD holds at a time form a 4 x 8 block, so
  // both operands are shared in its L2
  // with K slices (EPI_PARTIAL, KS > 1) logical block L is slice L % KS of tile L / KS
  const int Lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int ksl = Lb % a.KS;
  int tm, tn;
  grouped_tile(Lb / a.KS, tiles_m, tiles_n, 4, tm, tn);
  const int m0 = tm * GT_BM;
  const int nt0 = tn * (GT_BN / 16) + wn * 4;   // this wave's first column tile
  const int g0 = ksl * (a.KC >> 7);              // the slice's first 128-group
  const int KG = min(a.K >> 7, g0 + (a.KC >> 7)); // one past its last

  // x staging: thread t moves 16-byte chunks t + 256 u (u < 8) of the 128 x 128 tile:
  // row (t + 256u) / 16, chunk t % 16.  Rows past M re-read row M - 1 (never stored).
  // Columns past kx (a K padded to whole 128-groups) are loaded from column kx - 8, which
  // is in bounds, and staged as zeros.
  const int xc = tid & 15;
  const half_t* xsrc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int r = (tid >> 4) + 16 * u;
    xsrc[u] = a.x + (int64_t)min(m0 + r, a.M - 1) * a.ldx;
  }
  half8_t xr[8];
  auto load_x = [&](int g) {
    const int col = min(g * 128 + xc * 8, a.kx - 8);
#pragma unroll
    for (int u = 0; u < 8; ++u) xr[u] = *(const half8_t*)(xsrc[u] + col);
  };
  auto store_x = [&](int b, int g) {
    const bool live = g * 128 + xc * 8 < a.kx;
    const half8_t z = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < 8; ++u)
      *(half8_t*)(&xs[b][((tid >> 4) + 16 * u) * GT_XSTRIDE + xc * 8]) = live ? xr[u] : z;
  };

  WStream<WF> ws[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) ws[c].init(a, min(nt0 + c, NT - 1), 0, lane);   // group g at g
  WFrag<WF> wb[2][4];
  auto load_w = [&](WFrag<WF>(&f)[4], int g) {
#pragma unroll
    for (int c = 0; c < 4; ++c) ws[c].load(f[c], g);
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[i][c] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const half_t* xb, const WFrag<WF>(&f)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half8_t af[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *(const half8_t*)(xb + (64 * wm + 16 * i + c16) * GT_XSTRIDE + 32 * j + 8 * q16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        half8_t bf;
        if constexpr (WF == W_INT4) {
          const half2_t s2 = {f[c].s, f[c].s};
          bf = dequant8(f[c].q[j], s2);
        } else {
          bf = f[c].h[j];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][c] = mfma16x16x32(af[i], bf, acc[i][c]);
      }
    }
  };

  // Software pipeline over the K groups: group g + 1's x and weights are in flight while
  // group g is multiplied.  Group g is staged in xs[g & 1]; the barrier at the top of an
  // iteration also guarantees every wave finished reading that buffer two groups ago.
  load_x(g0);
  load_w(wb[0], g0);
  for (int g = g0; g < KG; g += 2) {
    store_x(0, g);
    __syncthreads();
    if (g + 1 < KG) {
      load_x(g + 1);
      load_w(wb[1], g + 1);
    }
    compute(xs[0], wb[0]);
    if (g + 1 >= KG) break;
    store_x(1, g + 1);
    __syncthreads();
    if (g + 2 < KG) {
      load_x(g + 2);
      load_w(wb[0], g + 2);
    }
    compute(xs[1], wb[1]);
  }

  // Epilogue.  Lane holds rows m0 + 64 wm + 16 i + 4 q16 + r, column (nt0 + c) * 16 + c16.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 64 * wm + 16 * i + 4 * q16 + r;
      if (m >= a.M) continue;
      if constexpr (EPI == EPI_SILU) {
        // column tiles (2p, 2p+1) = (gate, up) of intermediate columns 16p .. 16p + 15
#pragma unroll
        for (int c = 0; c < 4; c += 2) {
          if (nt0 + c + 1 >= NT) continue;
          const int j = ((nt0 + c) >> 1) * 16 + c16;
          const float gv = (float)(half_t)acc[i][c][r];
          const float uv = (float)(half_t)acc[i][c + 1][r];
          a.out[(int64_t)m * a.ldo + j] = (half_t)silu_mul_f32(gv, uv);
        }
      } else if constexpr (EPI == EPI_PARTIAL) {
        // the slice's fp32 sums, [slice][M][N]
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (nt0 + c >= NT) continue;
          a.partial[((int64_t)ksl * a.M + m) * a.N + (nt0 + c) * 16 + c16] = acc[i][c][r];
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (nt0 + c >= NT) continue;
          const int n = (nt0 + c) * 16 + c16;
          half_t h = finish_store(acc[i][c][r], a, n);
          if constexpr (EPI == EPI_QGELU) h = quick_gelu_ref(h);
          if constexpr (EPI == EPI_GELU) h = gelu_erf_ref(h);
          if constexpr (EPI == EPI_RESID) h = (half_t)((float)a.res[(int64_t)m * a.ldr + n] + (float)h);
          a.out[(int64_t)m * a.ldo + n] = h;
        }
      }
    }
}

template <int WF, int EPI>
static int launch_gemm_tile(const GemvArgs& a, hipStream_t st) {
  const int64_t tiles = (int64_t)((a.M + GT_BM - 1) / GT_BM) * ((a.N + GT_BN - 1) / GT_BN) * a.KS;
  if (tiles > 0x7fffffff) return OMNI_EUNSUPPORTED;
  hipLaunchKernelGGL((gemm_tile_kernel<WF, EPI>), dim3((unsigned)tiles), dim3(256), 0, st, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// Split-K finish of the tiled GEMM's STORE epilogue: out = finish_store(sum of the KS fp32
// slices in slice order, bias), one thread per 4 consecutive columns.
__global__ __launch_bounds__(256) void tile_finish_kernel(GemvArgs a) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nq = a.N >> 2;
  if (i >= (int64_t)a.M * nq) return;
  const int m = (int)(i / nq), n = (int)(i - (int64_t)m * nq) * 4;
  f32x4 v = *(const f32x4*)(a.partial + (int64_t)m * a.N + n);
  for (int s = 1; s < a.KS; ++s) {
    const f32x4 p = *(const f32x4*)(a.partial + ((int64_t)s * a.M + m) * a.N + n);
    v = (f32x4){v[0] + p[0], v[1] + p[1], v[2] + p[2], v[3] + p[3]};
  }
  half4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = finish_store(v[q], a, n + q);
  *(half4_t*)(a.out + (int64_t)m * a.ldo + n) = o;
}

// The tiled GEMM's STORE epilogue over a.KS K slices: fp32 partials into a.partial, then
// the finish launch.
template <int WF>
static int launch_gemm_tile_split(const GemvArgs& a, hipStream_t st) {
  int rc = launch_gemm_tile<WF, EPI_PARTIAL>(a, st);
  if (rc != OMNI_OK) return rc;
  const int64_t nthr = (int64_t)a.M * (a.N / 4);
  hipLaunchKernelGGL(tile_finish_kernel, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, st, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

struct AttnIn {            // x from split decode-attention states (omni_*_gemm_attn)
  const float* part;
  int S, nkv, G;
};

struct NormIn {            // x from an add+RMSNorm of split-K partials (omni_*_gemm_addnorm)
  const float* parts;
  int nparts;
  const void* res;
  const void* gain;
  float eps;
  void* res_out;
};

static int gemv_common(int wf, const void* x, int ldx, const void* w, const void* scales,
                       const void* bias, int bias_after_round, void* out, int ldo,
                       float* partial, int M, int N, int K, int epilogue, int ksplit, int preset,
                       void* stream, const AttnIn* ain = nullptr, const NormIn* nin = nullptr) {
  if (M <= 0 || N <= 0 || K <= 0) return M == 0 ? OMNI_OK : OMNI_EINVAL;
  if (M > 64 && (ain || epilogue == EPI_PARTIAL)) return OMNI_EUNSUPPORTED;
  if (nin) {
    if (M > 16 || (K & 511)) return OMNI_EUNSUPPORTED;   // one row block; whole waves per row
    if (!nin->parts || nin->nparts < 1 || nin->nparts > 64 || !nin->res || !nin->gain ||
        !nin->res_out || ((uintptr_t)nin->parts & 15) || ((uintptr_t)nin->res & 15) ||
        ((uintptr_t)nin->gain & 15) || ((uintptr_t)nin->res_out & 15))
      return OMNI_EINVAL;
    if (nin->res_out == nin->res) return OMNI_EINVAL;      // read by every workgroup
    if (epilogue != EPI_SILU && epilogue != EPI_PARTIAL && epilogue != EPI_STORE) return OMNI_EINVAL;
  }
  if ((N & 15) || (K & 127)) return OMNI_EUNSUPPORTED;
  if (!w || (wf == W_INT4 && !scales)) return OMNI_EINVAL;
  if (ain) {
    if (!ain->part || ain->S < 1 || ain->S > 64 || ain->nkv < 1 || ain->G < 1) return OMNI_EINVAL;
    if (K != ain->nkv * ain->G * 128) return OMNI_EINVAL;
    if (epilogue == EPI_SILU) return OMNI_EINVAL;
  } else if (!nin) {
    if (!x) return OMNI_EINVAL;
    if (ldx < K || (ldx & 7)) return OMNI_EINVAL;
  }
  if (epilogue != EPI_STORE && epilogue != EPI_SILU && epilogue != EPI_PARTIAL) return OMNI_EINVAL;
  if (epilogue == EPI_SILU && (N & 31)) return OMNI_EUNSUPPORTED;   // gate/up tile pairs
  if (preset == 3 && (N & 31)) return OMNI_EUNSUPPORTED;            // 2 tiles per wave
  const int KG = K >> 7;
  if (ksplit < 1 || ksplit > KG) return OMNI_EINVAL;
  // M > 64 with the STORE epilogue may be split along K too: partial is then the fp32
  // workspace of the slices ([slices][M][N]) and a finish launch stores the sums
  const bool tile_split = M > 64 && epilogue == EPI_STORE && ksplit > 1;
  if (epilogue == EPI_PARTIAL) {
    if (!partial) return OMNI_EINVAL;
  } else {
    if (!out || ldo < (epilogue == EPI_SILU ? N / 2 : N)) return OMNI_EINVAL;
    if (ksplit != 1 && !tile_split) return OMNI_EINVAL;   // a split needs partial sums
    if (tile_split && (!partial || ((uintptr_t)partial & 15) || (ldo & 3) || ((uintptr_t)out & 7)))
      return OMNI_EINVAL;
  }
  GemvArgs a = {};
  a.x = (const half_t*)x;
  a.ldx = ldx;
  a.w = w;
  a.scales = (const half_t*)scales;
  a.bias = (const half_t*)bias;
  a.bias_after_round = bias_after_round;
  a.out = (half_t*)out;
  a.ldo = ldo;
  a.partial = partial;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KC = ((KG + ksplit - 1) / ksplit) * 128;
  a.KS = (K + a.KC - 1) / a.KC;
  a.kx = K;
  hipStream_t st = (hipStream_t)stream;
  if (M > 64) {   // many rows (prefill): STORE / SILU epilogues
    // the pipelined GEMM where its shape and alignment rules hold (every K slice at least
    // 3 groups on int4 weights, whose deepest pipeline is 6 steps of 64, 2 on fp16 weights:
    // 4 steps), else the tiled kernel
    const int slices = tile_split ? omni_gemm_slices(K, ksplit) : 1;
    const bool pipe = (N % 128) == 0 && K >= 256 && KG / slices >= (wf == W_INT4 ? 3 : 2) &&
                      ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
                      ((uintptr_t)out & 7) == 0 && (ldo & 3) == 0 &&
                      (!bias || ((uintptr_t)bias & 15) == 0) &&
                      (wf != W_INT4 || ((uintptr_t)scales & 3) == 0);
    if (pipe)
      return omni_packed_gemm_pipe(x, ldx, w, scales, wf == W_INT4 ? 0 : 1, bias, bias_after_round,
                                   out, ldo, M, N, K, epilogue, 0, slices,
                                   tile_split ? partial : nullptr, stream);
    if (tile_split)
      return wf == W_INT4 ? launch_gemm_tile_split<W_INT4>(a, st) : launch_gemm_tile_split<W_FP16>(a, st);
    a.KS = 1;
    a.KC = K;
    if (wf == W_INT4)
      return epilogue == EPI_SILU ? launch_gemm_tile<W_INT4, EPI_SILU>(a, st)
                                  : launch_gemm_tile<W_INT4, EPI_STORE>(a, st);
    return epilogue == EPI_SILU ? launch_gemm_tile<W_FP16, EPI_SILU>(a, st)
                                : launch_gemm_tile<W_FP16, EPI_STORE>(a, st);
  }
  if (nin) {
    a.nparts = nin->parts;
    a.nnp = nin->nparts;
    a.nres = (const half_t*)nin->res;
    a.ngain = (const half_t*)nin->gain;
    a.nres_out = (half_t*)nin->res_out;
    a.neps = nin->eps;
    if (wf == W_INT4) {
      switch (epilogue) {
        case EPI_SILU: return dispatch_preset<W_INT4, EPI_SILU, 2>(a, preset, st);
        case EPI_PARTIAL: return dispatch_preset<W_INT4, EPI_PARTIAL, 2>(a, preset, st);
        default: return dispatch_preset<W_INT4, EPI_STORE, 2>(a, preset, st);
      }
    }
    switch (epilogue) {
      case EPI_SILU: return dispatch_preset<W_FP16, EPI_SILU, 2>(a, preset, st);
      case EPI_PARTIAL: return dispatch_preset<W_FP16, EPI_PARTIAL, 2>(a, preset, st);
      default: return dispatch_preset<W_FP16, EPI_STORE, 2>(a, preset, st);
    }
  }
  if (ain) {
    a.apart = ain->part;
    a.aS = ain->S;
    a.a_nkv = ain->nkv;
    a.aG = ain->G;
    if (wf == W_INT4)
      return epilogue == EPI_PARTIAL ? dispatch_preset<W_INT4, EPI_PARTIAL, 1>(a, preset, st)
                                     : dispatch_preset<W_INT4, EPI_STORE, 1>(a, preset, st);
    return epilogue == EPI_PARTIAL ? dispatch_preset<W_FP16, EPI_PARTIAL, 1>(a, preset, st)
                                   : dispatch_preset<W_FP16, EPI_STORE, 1>(a, preset, st);
  }
  if (wf == W_INT4) {
    switch (epilogue) {
      case EPI_SILU: return dispatch_preset<W_INT4, EPI_SILU>(a, preset, st);
      case EPI_PARTIAL: return dispatch_preset<W_INT4, EPI_PARTIAL>(a, preset, st);
      default: return dispatch_preset<W_INT4, EPI_STORE>(a, preset, st);
    }
  }
  switch (epilogue) {
    case EPI_SILU: return dispatch_preset<W_FP16, EPI_SILU>(a, preset, st);
    case EPI_PARTIAL: return dispatch_preset<W_FP16, EPI_PARTIAL>(a, preset, st);
    default: return dispatch_preset<W_FP16, EPI_STORE>(a, preset, st);
  }
}

// Number of K slices actually used for (K, ksplit) (slices are whole 128-groups).
extern "C" int omni_gemm_slices(int K, int ksplit) {
  const int KG = K >> 7;
  if (KG <= 0 || ksplit < 1) return 0;
  if (ksplit > KG) ksplit = KG;
  const int kc = (KG + ksplit - 1) / ksplit;
  return (KG + kc - 1) / kc;
}

extern "C" int omni_w4a16_gemm(const void* x, int ldx, const void* qweight_packed,
                               const void* scales_packed, const void* bias, int bias_after_round,
                               void* out, int ldo, float* partial, int M, int N, int K,
                               int epilogue, int ksplit, int preset, void* stream) {
  return gemv_common(W_INT4, x, ldx, qweight_packed, scales_packed, bias, bias_after_round, out,
                     ldo, partial, M, N, K, epilogue, ksplit, preset, stream);
}

extern "C" int omni_w4a16_gemm_attn(const float* attn_states, int attn_splits, int n_kv_heads,
                                    int group, const void* qweight_packed,
                                    const void* scales_packed, const void* bias,
                                    int bias_after_round, void* out, int ldo, float* partial, int M,
                                    int N, int K, int epilogue, int ksplit, int preset,
                                    void* stream) {
  const AttnIn ain = {attn_states, attn_splits, n_kv_heads, group};
  return gemv_common(W_INT4, nullptr, 0, qweight_packed, scales_packed, bias, bias_after_round, out,
                     ldo, partial, M, N, K, epilogue, ksplit, preset, stream, &ain);
}

extern "C" int omni_f16_gemm_attn(const float* attn_states, int attn_splits, int n_kv_heads,
                                  int group, const void* weight_packed, const void* bias, void* out,
                                  int ldo, float* partial, int M, int N, int K, int epilogue,
                                  int ksplit, int preset, void* stream) {
  const AttnIn ain = {attn_states, attn_splits, n_kv_heads, group};
  return gemv_common(W_FP16, nullptr, 0, weight_packed, nullptr, bias, 0, out, ldo, partial, M, N,
                     K, epilogue, ksplit, preset, stream, &ain);
}

extern "C" int omni_f16_gemm(const void* x, int ldx, const void* weight_packed, const void* bias,
                             void* out, int ldo, float* partial, int M, int N, int K, int epilogue,
                             int ksplit, int preset, void* stream) {
  return gemv_common(W_FP16, x, ldx, weight_packed, nullptr, bias, 0, out, ldo, partial, M, N, K,
                     epilogue, ksplit, preset, stream);
}

// add_rms_norm followed by the linear it feeds (model/qwen2_llm.py:145-157: input_layernorm
// -> qkv_proj, post_attention_layernorm -> gate_up_proj; kernels/fused_ops.py:60-70), for one
// row block (M <= 16, K % 512 == 0, M K / 8 <= the preset's threads): the norm's input is the
// previous projection's fp32 split-K partials [nparts][M][K] (omni_w4a16_gemm's
// OMNI_EPI_PARTIAL, summed in slice order), the residual and gain as omni_add_rmsnorm_partials
// takes them.  Every workgroup forms the rows' statistics; one writes the new residual to
// residual_out, which must not alias residual (every workgroup reads it).  The linear's
// output, epilogue (OMNI_EPI_STORE / OMNI_EPI_SILU / OMNI_EPI_PARTIAL), ksplit and preset (1;
// SiLU 1 or 4) as omni_w4a16_gemm.  x and y are identical to omni_add_rmsnorm_partials'.
extern "C" int omni_w4a16_gemm_addnorm(const float* partials, int nparts, const void* residual,
                                       const void* weight, float eps, void* residual_out,
                                       const void* qweight_packed, const void* scales_packed,
                                       const void* bias, int bias_after_round, void* out, int ldo,
                                       float* partial, int M, int N, int K, int epilogue,
                                       int ksplit, int preset, void* stream) {
  const NormIn nin = {partials, nparts, residual, weight, eps, residual_out};
  return gemv_common(W_INT4, nullptr, 0, qweight_packed, scales_packed, bias, bias_after_round, out,
                     ldo, partial, M, N, K, epilogue, ksplit, preset, stream, nullptr, &nin);
}

extern "C" int omni_f16_gemm_addnorm(const float* partials, int nparts, const void* residual,
                                     const void* weight, float eps, void* residual_out,
                                     const void* weight_packed, const void* bias, void* out,
                                     int ldo, float* partial, int M, int N, int K, int epilogue,
                                     int ksplit, int preset, void* stream) {
  const NormIn nin = {partials, nparts, residual, weight, eps, residual_out};
  return gemv_common(W_FP16, nullptr, 0, weight_packed, nullptr, bias, 0, out, ldo, partial, M, N,
                     K, epilogue, ksplit, preset, stream, nullptr, &nin);
}

// Tiled fp16 GEMM at any M for the vision tower's linears (model/qwen2_vit.py:41-44, 83,
// 88-89: nn.Linear in fp16, bias added before the single rounding):
//   h = fp16(x[:, :kx] . W^T + bias), then per epilogue
//   OMNI_EPI_STORE: h;  OMNI_EPI_QGELU: quick_gelu(h);  OMNI_EPI_GELU: gelu_erf(h);
//   OMNI_EPI_RESID: fp16(res + h)  (res may alias out: each element is read, then written,
//   by one thread).
// W packed by omni_f16_pack with K a multiple of 128 (columns past kx zero-padded); x has
// kx valid columns (kx % 8 == 0, row stride ldx).
extern "C" int omni_f16_gemm_tiled(const void* x, int ldx, int kx, const void* weight_packed,
                                   const void* bias, const void* res, int ldr, void* out,
                                   int ldo, int M, int N, int K, int epilogue, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return OMNI_EINVAL;
  if (M == 0) return OMNI_OK;
  if ((N & 15) || (K & 127)) return OMNI_EUNSUPPORTED;
  if (kx <= 0 || kx > K || (kx & 7)) return OMNI_EINVAL;
  if (!x || !weight_packed || !out) return OMNI_EINVAL;
  if (ldx < kx || (ldx & 7) || ldo < N) return OMNI_EINVAL;
  if (epilogue == EPI_RESID && (!res || ldr < N)) return OMNI_EINVAL;
  GemvArgs a = {};
  a.x = (const half_t*)x;
  a.ldx = ldx;
  a.kx = kx;
  a.w = weight_packed;
  a.bias = (const half_t*)bias;
  a.bias_after_round = 0;
  a.out = (half_t*)out;
  a.ldo = ldo;
  a.res = (const half_t*)res;
  a.ldr = ldr;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KC = K;
  a.KS = 1;
  hipStream_t st = (hipStream_t)stream;
  switch (epilogue) {
    case EPI_STORE: return launch_gemm_tile<W_FP16, EPI_STORE>(a, st);
    case EPI_QGELU: return launch_gemm_tile<W_FP16, EPI_QGELU>(a, st);
    case EPI_GELU: return launch_gemm_tile<W_FP16, EPI_GELU>(a, st);
    case EPI_RESID: return launch_gemm_tile<W_FP16, EPI_RESID>(a, st);
    default: return OMNI_EINVAL;
  }
}

// ---------------------------------------------------------------------------
// lm_head + greedy argmax: the GEMM writes one (max, index) candidate per
// workgroup and row; omni_argmax_finalize reduces them.
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// lm_head + greedy-argmax candidates, persistent: one workgroup (8 waves) per CU stages
// x [M <= 64, K] in LDS once, then its waves stream their share of the packed fp16 table
// (column tiles t0 + wave, t0 + wave + 8, ... of the workgroup's contiguous tile range)
// as one run of 4-group (512-k) batches, two batches in flight, so the stream does not
// pause between tiles.  Per tile the accumulation order is the skinny kernel's (groups and
// 32-k steps ascending); the logit is fp16(acc), compared as float, lowest index on ties.
// ---------------------------------------------------------------------------
static int num_cus_gemv() {
  static int n = 0;
  if (n <= 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    n = v;
  }
  return n;
}

template <int MB>
__global__ __launch_bounds__(512, 1) void lmhead_kernel(GemvArgs a) {
#pragma clang fp contract(off)
  // all arguments in one batch of scalar loads (a wait for one is a wait for all)
  asm volatile("" ::"s"(a.x), "s"(a.ldx), "s"(a.w), "s"(a.M), "s"(a.N), "s"(a.K),
               "s"(a.cand_val), "s"(a.cand_idx), "s"(gridDim.x));
  extern __shared__ __attribute__((aligned(16))) char smem[];
  half_t* xs = (half_t*)smem;                  // [MB * 16][K + 8]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q16 = lane >> 4, c16 = lane & 15;
  const int K = a.K;
  const int xstride = K + 8;
  // 1. x rows (zero past M) into LDS
  {
    const int cpr = K >> 3;
    for (int i = threadIdx.x; i < MB * 16 * cpr; i += 512) {
      const int r = i / cpr, c = i - r * cpr;
      half8_t v = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
      if (r < a.M) v = *(const half8_t*)(a.x + (int64_t)r * a.ldx + c * 8);
      *(half8_t*)(xs + r * xstride + c * 8) = v;
    }
  }
  __syncthreads();

  // 32-k steps per batch: 4 (two batches = 8 KB in flight per wave; 16 / 32 KB measured
  // 1-3 % slower: 78.4 / 82.0 / 80.6 us at 32 rows, 74.3 / 74.9 / 76.5 at one row); 8 at 64
  // rows, as measured when that form was sized for its registers
  constexpr int NBU = MB >= 4 ? 8 : 4;
  const int NT = a.N >> 4;
  const int KS32 = K >> 5;                     // 32-k steps per tile
  const int BPT = K / (32 * NBU);              // batches per tile (K % 512 == 0)
  const int G = gridDim.x;
  const int blk = xcd_logical_block(blockIdx.x, G);
  const int t0 = (int)((int64_t)blk * NT / G), t1 = (int)((int64_t)(blk + 1) * NT / G);
  const int ntw = t1 - t0 > wave ? (t1 - t0 - wave + 7) / 8 : 0;   // this wave's tiles
  const int nb = ntw * BPT;
  const half8_t* wp = (const half8_t*)a.w + lane;
  auto load_batch = [&](half8_t (&buf)[NBU], int b) {
    const int bc = min(b, max(nb - 1, 0));        // past the end: re-read the last batch
    const int tile = min(t0 + wave + 8 * (bc / BPT), NT - 1);
    const int s0 = (bc % BPT) * NBU;              // first 32-k step of the batch
#pragma unroll
    for (int u = 0; u < NBU; ++u)
      buf[u] = __builtin_nontemporal_load(wp + ((int64_t)tile * KS32 + s0 + u) * 64);
  };

  float bv[MB][4];
  int bi[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bv[mb][i] = -INFINITY;
      bi[mb][i] = 0x7fffffff;
    }
  f32x4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto use_batch = [&](const half8_t (&buf)[NBU], int b) {
    const int kb = (b % BPT) * (32 * NBU);
#pragma unroll
    for (int u = 0; u < NBU; ++u) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const half8_t af = *(const half8_t*)(xs + (16 * mb + c16) * xstride + kb + 32 * u + 8 * q16);
        acc[mb] = mfma16x16x32(af, buf[u], acc[mb]);
      }
    }
    if (b % BPT == BPT - 1) {                   // tile done: fp16 logits, running argmax
      const int n = (t0 + wave + 8 * (b / BPT)) * 16 + c16;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 16 * mb + 4 * q16 + i;
          const half_t h = (half_t)acc[mb][i];
          if (a.out && m < a.M) a.out[(int64_t)m * a.ldo + n] = h;
          const float v = (float)h;
          if (v > bv[mb][i]) {                  // columns ascend per lane: first max wins
            bv[mb][i] = v;
            bi[mb][i] = n;
          }
        }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
  };

  // 2. the stream: batches b (A) and b + 1 (B) in flight
  half8_t ba[NBU], bb[NBU];
  load_batch(ba, 0);
  load_batch(bb, 1);
  for (int b = 0; b < nb; b += 2) {
    use_batch(ba, b);
    load_batch(ba, b + 2);
    if (b + 1 < nb) use_batch(bb, b + 1);
    load_batch(bb, b + 3);
  }

  // 3. reduce: over the 16 columns of a lane group, then over the waves (LDS)
  __shared__ float red_v[8][64];
  __shared__ int red_i[8][64];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = bv[mb][i];
      int ix = bi[mb][i];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(ix, o, 64);
        if (ov > v || (ov == v && oi < ix)) { v = ov; ix = oi; }
      }
      if (c16 == 0) {
        red_v[wave][16 * mb + 4 * q16 + i] = v;
        red_i[wave][16 * mb + 4 * q16 + i] = ix;
      }
    }
  __syncthreads();
  if ((int)threadIdx.x < a.M) {
    const int m = threadIdx.x;
    float v = red_v[0][m];
    int ix = red_i[0][m];
#pragma unroll
    for (int w = 1; w < 8; ++w) {
      const float ov = red_v[w][m];
      const int oi = red_i[w][m];
      if (ov > v || (ov == v && oi < ix)) { v = ov; ix = oi; }
    }
    a.cand_val[(int64_t)blockIdx.x * a.M + m] = v;
    a.cand_idx[(int64_t)blockIdx.x * a.M + m] = ix;
  }
}

// Rows one omni_lmhead_candidates call takes for hidden size K: x is staged in LDS as
// whole 16-row blocks of K + 8 halves, at most 64 rows (48 at K = 1536 in 160 KiB).
extern "C" int omni_lmhead_max_rows(int K) {
  if (K <= 0) return 0;
  const size_t per16 = (size_t)16 * (K + 8) * sizeof(half_t);
  const int blocks = (int)(max_dynamic_lds() / per16);
  return (blocks > 4 ? 4 : blocks) * 16;
}

// Candidate slots per row written by omni_lmhead_candidates (= its grid size).
extern "C" int omni_lmhead_argmax_grid(int N) {
  const int NT = N >> 4;
  const int cus = num_cus_gemv();
  return NT < cus ? NT : cus;
}

extern "C" int omni_lmhead_candidates(const void* x, int ldx, const void* weight_packed, int M,
                                      int N, int K, void* logits_out, float* cand_val,
                                      int* cand_idx, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return M == 0 ? OMNI_OK : OMNI_EINVAL;
  if (M > 64) return OMNI_EUNSUPPORTED;
  if ((N & 31) || (K & 127)) return OMNI_EUNSUPPORTED;
  if (!x || !weight_packed || !cand_val || !cand_idx) return OMNI_EINVAL;
  if (ldx < K || (ldx & 7)) return OMNI_EINVAL;
  GemvArgs a = {};
  a.x = (const half_t*)x;
  a.ldx = ldx;
  a.w = weight_packed;
  a.out = (half_t*)logits_out;
  a.ldo = N;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KS = 1;
  a.KC = K;
  a.cand_val = cand_val;
  a.cand_idx = cand_idx;
  if (K & 511) return OMNI_EUNSUPPORTED;          // 512-k batches
  const size_t lds = (size_t)((M + 15) / 16) * 16 * (K + 8) * sizeof(half_t);
  if (lds > max_dynamic_lds()) return OMNI_EUNSUPPORTED;
  const int grid = omni_lmhead_argmax_grid(N);
  hipStream_t st = (hipStream_t)stream;
  switch ((M + 15) / 16) {
#define OMNI_LMHEAD_CASE(MBV)                                                                   \
    case MBV: {                                                                                  \
      static bool attr = false;                                                                  \
      if (!attr) {                                                                               \
        (void)hipFuncSetAttribute((const void*)lmhead_kernel<MBV>,                               \
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_dynamic_lds()); \
        attr = true;                                                                             \
      }                                                                                          \
      hipLaunchKernelGGL(lmhead_kernel<MBV>, dim3(grid), dim3(512), lds, st, a);                 \
      break;                                                                                     \
    }
    OMNI_LMHEAD_CASE(1)
    OMNI_LMHEAD_CASE(2)
    OMNI_LMHEAD_CASE(3)
    OMNI_LMHEAD_CASE(4)
#undef OMNI_LMHEAD_CASE
    default: return OMNI_EUNSUPPORTED;
  }
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// ids_out[m] = index of the max candidate (lowest index on ties).  Decode-step
// bookkeeping folded in: next_ids[m] = ids_out[m] and lengths[m] += 1 when given.
__global__ __launch_bounds__(256) void argmax_finalize_kernel(
    const float* __restrict__ cv, const int* __restrict__ ci, int nblk, int M,
    int64_t* __restrict__ ids_out, int64_t* __restrict__ next_ids, int64_t* __restrict__ lengths) {
  const int m = blockIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int b = threadIdx.x; b < nblk; b += 256) {
    const float ov = cv[(int64_t)b * M + m];
    const int oi = ci[(int64_t)b * M + m];
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  __shared__ float sv[4];
  __shared__ int si[4];
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) { bv = sv[w]; bi = si[w]; }
    ids_out[m] = bi;
    if (next_ids) next_ids[m] = bi;
    if (lengths) lengths[m] += 1;
  }
}

extern "C" int omni_argmax_finalize(const float* cand_val, const int* cand_idx, int nblk, int M,
                                    int64_t* ids_out, int64_t* next_ids, int64_t* lengths,
                                    void* stream) {
  if (M < 0 || nblk <= 0) return OMNI_EINVAL;
  if (M == 0) return OMNI_OK;
  if (!cand_val || !cand_idx || !ids_out) return OMNI_EINVAL;
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3(M), dim3(256), 0, (hipStream_t)stream, cand_val,
                     cand_idx, nblk, M, ids_out, next_ids, lengths);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free lm_head + greedy argmax, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops).  The per-workgroup candidates live
// in `scratch`, a file-scope device array every GPU holds once for the whole process:
// NOALLOC_SLOTS (grid x rows) fp32 values, then as many int32 indices (256 KiB).  Every slot
// a call reads, the same call's candidates launch wrote first, so nothing is cleared.
// Calls that overlap on one GPU (two streams) share the array and race.
// ---------------------------------------------------------------------------
#define NOALLOC_SLOTS (512 * 64)
#define NOALLOC_MAX_DEVICES 64

static __device__ __align__(256) unsigned char scratch[NOALLOC_SLOTS * 8];

// This GPU's address of `scratch` (host code passes that, never the array's name), looked
// up once per device with the device current; NULL if the lookup fails.
static void* noalloc_scratch(int dev) {
  static std::mutex mu;
  static void* ptrs[NOALLOC_MAX_DEVICES] = {};
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

extern "C" int omni_lmhead_argmax_noalloc(const void* x, int ldx, const void* weight_packed,
                                          int M, int N, int K, void* logits_out, int64_t* ids_out,
                                          int64_t* next_ids, int64_t* lengths, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return OMNI_EINVAL;
  if (M == 0) return OMNI_OK;
  if (!x || !weight_packed || !ids_out) return OMNI_EINVAL;
  if (M > 64 || (N & 31)) return OMNI_EUNSUPPORTED;
  const int grid = omni_lmhead_argmax_grid(N);
  // beyond the array: only on a part with more than 512 CUs (one workgroup per CU)
  if ((int64_t)grid * M > NOALLOC_SLOTS) return OMNI_EUNSUPPORTED;
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  unsigned char* base = (unsigned char*)noalloc_scratch(dev);
  if (!base) return OMNI_EUNSUPPORTED;
  float* cand_val = (float*)base;
  int* cand_idx = (int*)(base + (size_t)NOALLOC_SLOTS * sizeof(float));
  const int rc = omni_lmhead_candidates(x, ldx, weight_packed, M, N, K, logits_out, cand_val,
                                        cand_idx, stream);
  if (rc != OMNI_OK) return rc;
  return omni_argmax_finalize(cand_val, cand_idx, grid, M, ids_out, next_ids, lengths, stream);
}

// ---------------------------------------------------------------------------
// Load-time repacking.
// ---------------------------------------------------------------------------
// AutoGPTQ qweight [K/8, N] int32 (8 consecutive k per word, k%8 at bits 4*(k%8))
// + scales [K/128, N] fp16  ->  packed layout above.  With interleave_halves the
// column tiles of the two halves of N are interleaved (tile t of the first half
// -> 2t, of the second half -> 2t+1): the fused gate|up layout the SiLU epilogue
// consumes (marlin_linear.py:130-139 concatenates gate|up along N).
__device__ __forceinline__ int dst_tile(int t, int NT, int interleave) {
  if (!interleave) return t;
  const int h = NT >> 1;
  return t < h ? 2 * t : 2 * (t - h) + 1;
}

__global__ void gptq_repack_kernel(const uint32_t* __restrict__ qw, const half_t* __restrict__ sc,
                                   uint32_t* __restrict__ qp, half_t* __restrict__ sp, int K, int N,
                                   int interleave) {
  const int NT = N >> 4, KG = K >> 7;
  const int64_t total = (int64_t)NT * KG * 64 * 4;
  for (int64_t idx = blockIdx.x * 256LL + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int j = (int)(idx & 3);
    const int lane = (int)((idx >> 2) & 63);
    const int64_t blk = idx >> 8;
    const int kg = (int)(blk % KG);
    const int st = (int)(blk / KG);   // source tile
    const int n = st * 16 + (lane & 15);
    const int kbase = kg * 128 + 32 * j + 8 * (lane >> 4);
    const uint32_t src = qw[(int64_t)(kbase >> 3) * N + n];
    uint32_t dst = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t code = (src >> (4 * e)) & 0xFu;
      const int bit = (e & 1) ? 16 + 2 * (e - 1) : 2 * e;
      dst |= code << bit;
    }
    const int dt = dst_tile(st, NT, interleave);
    qp[(((int64_t)dt * KG + kg) * 64 + lane) * 4 + j] = dst;
    if (j == 0 && lane < 16) sp[((int64_t)dt * KG + kg) * 16 + lane] = sc[(int64_t)kg * N + n];
  }
}

extern "C" int omni_gptq_repack(const int32_t* qweight, const void* scales, int32_t* qweight_packed,
                                void* scales_packed, int K, int N, int interleave_halves,
                                void* stream) {
  if (K <= 0 || N <= 0) return OMNI_EINVAL;
  if ((K & 127) || (N & 15)) return OMNI_EUNSUPPORTED;
  if (interleave_halves && (N & 31)) return OMNI_EUNSUPPORTED;
  if (!qweight || !scales || !qweight_packed || !scales_packed) return OMNI_EINVAL;
  const int64_t total = (int64_t)(N >> 4) * (K >> 7) * 256;
  int grid = (int)((total + 255) / 256);
  if (grid > 16384) grid = 16384;
  hipLaunchKernelGGL(gptq_repack_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)qweight, (const half_t*)scales, (uint32_t*)qweight_packed,
                     (half_t*)scales_packed, K, N, interleave_halves);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// fp16 weight [N, K] (nn.Linear layout) -> packed [N/16][K/32][64][8].
__global__ void f16_pack_kernel(const half_t* __restrict__ w, half_t* __restrict__ wp, int K, int N,
                                int interleave) {
  const int NT = N >> 4, KS = K >> 5;
  const int64_t total = (int64_t)NT * KS * 64;   // one 16-byte chunk per item
  for (int64_t idx = blockIdx.x * 256LL + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int lane = (int)(idx & 63);
    const int64_t blk = idx >> 6;
    const int ks = (int)(blk % KS);
    const int st = (int)(blk / KS);
    const int n = st * 16 + (lane & 15);
    const int k = ks * 32 + 8 * (lane >> 4);
    const half8_t v = *(const half8_t*)(w + (int64_t)n * K + k);
    const int dt = dst_tile(st, NT, interleave);
    *(half8_t*)(wp + (((int64_t)dt * KS + ks) * 64 + lane) * 8) = v;
  }
}

extern "C" int omni_f16_pack(const void* weight, void* weight_packed, int K, int N,
                             int interleave_halves, void* stream) {
  if (K <= 0 || N <= 0) return OMNI_EINVAL;
  if ((K & 31) || (N & 15)) return OMNI_EUNSUPPORTED;
  if (interleave_halves && (N & 31)) return OMNI_EUNSUPPORTED;
  if (!weight || !weight_packed) return OMNI_EINVAL;
  const int64_t total = (int64_t)(N >> 4) * (K >> 5) * 64;
  int grid = (int)((total + 255) / 256);
  if (grid > 16384) grid = 16384;
  hipLaunchKernelGGL(f16_pack_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const half_t*)weight, (half_t*)weight_packed, K, N, interleave_halves);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// Packed int4 -> dense fp16 W^T [K, N] (the reference's dequantised weight,
// W[k, n] = fp16((q - 8) * s)).  Load-time/verification helper.
__global__ void w4_dequant_kernel(const uint32_t* __restrict__ qp, const half_t* __restrict__ sp,
                                  half_t* __restrict__ w, int K, int N) {
  const int NT = N >> 4, KG = K >> 7;
  const int64_t total = (int64_t)NT * KG * 64 * 4;
  for (int64_t idx = blockIdx.x * 256LL + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int j = (int)(idx & 3);
    const int lane = (int)((idx >> 2) & 63);
    const int64_t blk = idx >> 8;
    const int kg = (int)(blk % KG);
    const int nt = (int)(blk / KG);
    const uint32_t word = qp[idx];
    const half_t s = sp[blk * 16 + (lane & 15)];
    const half2_t s2 = {s, s};
    const half8_t v = dequant8(word, s2);
    const int n = nt * 16 + (lane & 15);
    const int kb = kg * 128 + 32 * j + 8 * (lane >> 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) w[(int64_t)(kb + e) * N + n] = v[e];
  }
}

// Packed int4 -> the packed fp16 layout of omni_f16_pack (same tile order, so a gate|up
// interleave carries over): word j of (tile, group, lane) becomes the lane's 8 halfs of
// 32-k block 4 group + j, fp16((q - 8) s) as every int4 kernel dequantises it.  For the
// prefill linears at many rows, where the fp16 GEMM outruns the in-loop dequantisation.
__global__ __launch_bounds__(256) void w4_unpack_f16_kernel(const u32x4* __restrict__ qp,
                                                            const half_t* __restrict__ sp,
                                                            half8_t* __restrict__ w, int K, int N) {
  // thread = (tile, group, lane): its 16 bytes of codes become 4 x 16 bytes, one in each of
  // the group's four 32-k blocks (a wave reads 1 KB and writes four 1 KB runs)
  const int64_t total = (int64_t)(N >> 4) * (K >> 7) * 64;
  for (int64_t idx = blockIdx.x * 256LL + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int lane = (int)(idx & 63);
    const int64_t blk = idx >> 6;                 // nt * KG + kg
    const u32x4 q = __builtin_nontemporal_load(qp + idx);
    const half_t s = sp[blk * 16 + (lane & 15)];
    const half2_t s2 = {s, s};
#pragma unroll
    for (int j = 0; j < 4; ++j) w[(blk * 4 + j) * 64 + lane] = dequant8(q[j], s2);
  }
}

extern "C" int omni_w4_unpack_f16(const int32_t* qweight_packed, const void* scales_packed,
                                  void* weight_packed, int K, int N, void* stream) {
  if (K <= 0 || N <= 0) return OMNI_EINVAL;
  if ((K & 127) || (N & 15)) return OMNI_EUNSUPPORTED;
  if (!qweight_packed || !scales_packed || !weight_packed || ((uintptr_t)weight_packed & 15) ||
      ((uintptr_t)qweight_packed & 15))
    return OMNI_EINVAL;
  const int64_t total = (int64_t)(N >> 4) * (K >> 7) * 64;
  int grid = (int)((total + 255) / 256);
  if (grid > 16384) grid = 16384;
  hipLaunchKernelGGL(w4_unpack_f16_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4*)qweight_packed, (const half_t*)scales_packed,
                     (half8_t*)weight_packed, K, N);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_w4_dequant(const int32_t* qweight_packed, const void* scales_packed, void* w,
                               int K, int N, void* stream) {
  if (K <= 0 || N <= 0) return OMNI_EINVAL;
  if ((K & 127) || (N & 15)) return OMNI_EUNSUPPORTED;
  if (!qweight_packed || !scales_packed || !w) return OMNI_EINVAL;
  const int64_t total = (int64_t)(N >> 4) * (K >> 7) * 256;
  int grid = (int)((total + 255) / 256);
  if (grid > 16384) grid = 16384;
  hipLaunchKernelGGL(w4_dequant_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)qweight_packed, (const half_t*)scales_packed, (half_t*)w, K, N);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

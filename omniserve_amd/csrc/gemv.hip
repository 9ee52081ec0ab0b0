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
// In both, one 16-byte load per lane is exactly one MFMA 16x16x32 B operand set
// (four of them for int4), a wavefront reads 1 KB contiguous per load, and the
// int4 dequant is the magic-exponent trick on packed fp16 (no LUT, no shuffles).
//
// Work split: a workgroup of NW waves owns NW*CPW column tiles of 16 and one
// K-split; it stages x[:, k-split] in LDS once, each wave streams its tiles'
// weights (prefetch depth PF k-groups) and runs MB*CPW MFMAs per 32-k step.
// Split-K partials go to an fp32 workspace; the last workgroup of a column
// group (device-scope counter it resets itself) sums them in split order, so
// results are deterministic and the kernel is graph-replayable.
#include "common.h"

enum { W_INT4 = 0, W_FP16 = 1 };
enum { EPI_STORE = 0, EPI_SILU = 1, EPI_ARGMAX = 2 };

struct GemvArgs {
  const half_t* x;
  int ldx;
  const void* w;
  const half_t* scales;
  const half_t* bias;
  int bias_after_round;  // 1: fp16(fp16(acc) + b) (GPTQ path); 0: fp16(acc + b)
  half_t* out;
  int ldo;
  int M, N, K;
  int KS, KC;            // k splits, k per split (multiple of 128)
  float* ws;             // [KS][M][N] fp32 partials (KS > 1)
  int* counters;         // [column groups] (KS > 1) or [1] (argmax)
  float* cand_val;       // [grid][M] (argmax)
  int* cand_idx;         // [grid][M]
  int64_t* ids_out;      // [M]
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

template <int WF>
__device__ __forceinline__ void load_frag(WFrag<WF>& f, const GemvArgs& a, int nt, int kg, int lane) {
  if constexpr (WF == W_INT4) {
    const int KG = a.K >> 7;
    const int64_t blk = (int64_t)nt * KG + kg;
    f.q = __builtin_nontemporal_load((const u32x4*)a.w + blk * 64 + lane);
    f.s = a.scales[blk * 16 + (lane & 15)];
  } else {
    const int KS32 = a.K >> 5;
    const half8_t* wp = (const half8_t*)a.w + ((int64_t)nt * KS32 + kg * 4) * 64 + lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) f.h[j] = __builtin_nontemporal_load(wp + j * 64);
  }
}

__device__ __forceinline__ float silu_ref(float g) { return g * (1.0f / (1.0f + __expf(-g))); }

__device__ __forceinline__ half_t finish_store(float v, const GemvArgs& a, int n) {
#pragma clang fp contract(off)
  if (a.bias) {
    const float b = (float)a.bias[n];
    if (a.bias_after_round) return (half_t)((float)(half_t)v + b);
    return (half_t)(v + b);
  }
  return (half_t)v;
}

template <int WF, int MB, int EPI, int CPW, int NW, int PF>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(GemvArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) half_t xs[];
  __shared__ float red_v[NW][MB * 16];
  __shared__ int red_i[NW][MB * 16];
  __shared__ int last_flag;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q16 = lane >> 4;
  const int c16 = lane & 15;
  const int NT = a.N >> 4;
  constexpr int TPW = NW * CPW;  // column tiles per workgroup
  const int ngroups = (NT + TPW - 1) / TPW;
  const int ng = blockIdx.x % ngroups;
  const int ksi = blockIdx.x / ngroups;
  const int k0 = ksi * a.KC;
  const int kc = min(a.KC, a.K - k0);
  const int xstride = a.KC + 8;

  // Stage x[0:M, k0:k0+kc] (rows >= M zero) into LDS.
  {
    const int cpr = kc >> 3;
    const int total = MB * 16 * cpr;
    for (int i = threadIdx.x; i < total; i += NW * 64) {
      const int r = i / cpr;
      const int c = i - r * cpr;
      half8_t v = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
      if (r < a.M) v = *(const half8_t*)(a.x + (int64_t)r * a.ldx + k0 + c * 8);
      *(half8_t*)(xs + r * xstride + c * 8) = v;
    }
  }
  __syncthreads();

  const int tile0 = ng * TPW + wave * CPW;
  const bool active = tile0 < NT;
  f32x4 acc[CPW][MB];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[c][mb] = (f32x4){0.f, 0.f, 0.f, 0.f};

  if (active) {
    const int ngk = kc >> 7;
    const int kg0 = k0 >> 7;
    WFrag<WF> buf[PF][CPW];
#pragma unroll
    for (int p = 0; p < PF; ++p)
      if (p < ngk)
#pragma unroll
        for (int c = 0; c < CPW; ++c) load_frag<WF>(buf[p][c], a, tile0 + c, kg0 + p, lane);

    for (int base = 0; base < ngk; base += PF) {
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        const int i = base + p;
        if (i < ngk) {
          WFrag<WF> cur[CPW];
#pragma unroll
          for (int c = 0; c < CPW; ++c) cur[c] = buf[p][c];
          if (i + PF < ngk)
#pragma unroll
            for (int c = 0; c < CPW; ++c) load_frag<WF>(buf[p][c], a, tile0 + c, kg0 + i + PF, lane);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            half8_t af[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              af[mb] = *(const half8_t*)(xs + (16 * mb + c16) * xstride + i * 128 + 32 * j + 8 * q16);
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
              half8_t bf;
              if constexpr (WF == W_INT4) {
                const half2_t s2 = {cur[c].s, cur[c].s};
                bf = dequant8(cur[c].q[j], s2);
              } else {
                bf = cur[c].h[j];
              }
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) acc[c][mb] = mfma16x16x32(af[mb], bf, acc[c][mb]);
            }
          }
        }
      }
    }
  }

  // ------------------------------------------------------------ epilogues
  if constexpr (EPI == EPI_ARGMAX) {
    // logits = fp16(acc); greedy argmax on the fp16 values, lowest index wins ties
    // (torch.argmax semantics).  Optional logits store.
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
          red_v[wave][m] = bv;
          red_i[wave][m] = bi;
        }
      }
    __syncthreads();
    if (threadIdx.x < a.M) {
      const int m = threadIdx.x;
      float bv = red_v[0][m];
      int bi = red_i[0][m];
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        const float ov = red_v[w][m];
        const int oi = red_i[w][m];
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      a.cand_val[(int64_t)blockIdx.x * a.M + m] = bv;
      a.cand_idx[(int64_t)blockIdx.x * a.M + m] = bi;
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
      const int prev = __hip_atomic_fetch_add(a.counters, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == (int)gridDim.x - 1;
      if (last) __hip_atomic_store(a.counters, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_flag = last;
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    // Final reduction over all workgroups: wave w handles rows w, w+NW, ...
    for (int m = wave; m < a.M; m += NW) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int b = lane; b < (int)gridDim.x; b += 64) {
        const float ov = __builtin_nontemporal_load(a.cand_val + (int64_t)b * a.M + m);
        const int oi = __builtin_nontemporal_load(a.cand_idx + (int64_t)b * a.M + m);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if (lane == 0) a.ids_out[m] = bi;
    }
    return;
  } else {
    if (a.KS == 1) {
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
            a.out[(int64_t)m * a.ldo + j] = (half_t)(silu_ref(g) * u);
          } else {
#pragma unroll
            for (int c = 0; c < CPW; ++c) {
              const int n = (tile0 + c) * 16 + c16;
              a.out[(int64_t)m * a.ldo + n] = finish_store(acc[c][mb][i], a, n);
            }
          }
        }
      return;
    }
    // Split-K: fp32 partials, then the last workgroup of this column group reduces.
    if (active) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 16 * mb + 4 * q16 + i;
          if (m >= a.M) continue;
#pragma unroll
          for (int c = 0; c < CPW; ++c) {
            const int n = (tile0 + c) * 16 + c16;
            a.ws[((int64_t)ksi * a.M + m) * a.N + n] = acc[c][mb][i];
          }
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
      int* ctr = a.counters + ng;
      const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == a.KS - 1;
      if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_flag = last;
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    const int ncol_tiles = min(TPW, NT - ng * TPW);
    if constexpr (EPI == EPI_SILU) {
      const int npairs = ncol_tiles >> 1;
      const int total = a.M * npairs * 16;
      for (int idx = threadIdx.x; idx < total; idx += NW * 64) {
        const int m = idx / (npairs * 16);
        const int r = idx - m * npairs * 16;
        const int pr = (ng * TPW >> 1) + (r >> 4);
        const int cc = r & 15;
        const int ng_ = pr * 32 + cc;       // gate column in packed (interleaved) order
        const int nu_ = ng_ + 16;
        float g = 0.f, u = 0.f;
        for (int s = 0; s < a.KS; ++s) {
          g += __builtin_nontemporal_load(a.ws + ((int64_t)s * a.M + m) * a.N + ng_);
          u += __builtin_nontemporal_load(a.ws + ((int64_t)s * a.M + m) * a.N + nu_);
        }
        g = (float)(half_t)g;
        u = (float)(half_t)u;
        a.out[(int64_t)m * a.ldo + pr * 16 + cc] = (half_t)(silu_ref(g) * u);
      }
    } else {
      const int ncols = ncol_tiles * 16;
      const int total = a.M * ncols;
      for (int idx = threadIdx.x; idx < total; idx += NW * 64) {
        const int m = idx / ncols;
        const int n = ng * TPW * 16 + (idx - m * ncols);
        float v = 0.f;
        for (int s = 0; s < a.KS; ++s) v += __builtin_nontemporal_load(a.ws + ((int64_t)s * a.M + m) * a.N + n);
        a.out[(int64_t)m * a.ldo + n] = finish_store(v, a, n);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------
// Largest dynamic LDS a workgroup may request on the current device, leaving room
// for the kernel's static arrays.
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

template <int WF, int MB, int EPI, int CPW, int NW, int PF>
static int launch_gemv(const GemvArgs& a, int grid, hipStream_t st) {
  auto kern = gemv_kernel<WF, MB, EPI, CPW, NW, PF>;
  const size_t lds = (size_t)MB * 16 * (a.KC + 8) * sizeof(half_t);
  const size_t lim = max_dynamic_lds();
  if (lds > lim) return OMNI_EUNSUPPORTED;
  static bool attr_set = false;
  if (!attr_set) {
    hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lim);
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), lds, st, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

template <int WF, int EPI, int CPW, int NW, int PF>
static int dispatch_mb(const GemvArgs& a, int grid, hipStream_t st) {
  const int mb = (a.M + 15) / 16;
  switch (mb) {
    case 1: return launch_gemv<WF, 1, EPI, CPW, NW, PF>(a, grid, st);
    case 2: return launch_gemv<WF, 2, EPI, CPW, NW, PF>(a, grid, st);
    case 3: return launch_gemv<WF, 3, EPI, CPW, NW, PF>(a, grid, st);
    case 4: return launch_gemv<WF, 4, EPI, CPW, NW, PF>(a, grid, st);
    default: return OMNI_EUNSUPPORTED;
  }
}

// Tuning: (CPW, NW) per weight format / epilogue.
template <int WF, int EPI>
static int dispatch(const GemvArgs& a, int cpw, hipStream_t st) {
  const int NT = a.N >> 4;
  if constexpr (EPI == EPI_SILU) {
    constexpr int NW = 4;
    const int ngroups = (NT + 2 * NW - 1) / (2 * NW);
    const int grid = ngroups * a.KS;
    if constexpr (WF == W_INT4) return dispatch_mb<WF, EPI, 2, NW, 4>(a, grid, st);
    else return dispatch_mb<WF, EPI, 2, NW, 2>(a, grid, st);
  } else {
    constexpr int NW = 4;
    if (cpw == 1) {
      const int grid = ((NT + NW - 1) / NW) * a.KS;
      if constexpr (WF == W_INT4) return dispatch_mb<WF, EPI, 1, NW, 4>(a, grid, st);
      else return dispatch_mb<WF, EPI, 1, NW, 2>(a, grid, st);
    }
    const int grid = ((NT + 2 * NW - 1) / (2 * NW)) * a.KS;
    if constexpr (WF == W_INT4) return dispatch_mb<WF, EPI, 2, NW, 4>(a, grid, st);
    else return dispatch_mb<WF, EPI, 2, NW, 2>(a, grid, st);
  }
}

static int gemv_common(int wf, const void* x, int ldx, const void* w, const void* scales,
                       const void* bias, int bias_after_round, void* out, int ldo, int M, int N,
                       int K, int epilogue, int ksplit, int cpw, float* ws, int* counters,
                       void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return M == 0 ? OMNI_OK : OMNI_EINVAL;
  if (M > 64) return OMNI_EUNSUPPORTED;
  if ((N & 15) || (K & 127)) return OMNI_EUNSUPPORTED;
  if (!x || !w || !out || (wf == W_INT4 && !scales)) return OMNI_EINVAL;
  if (ldx < K || (ldx & 7)) return OMNI_EINVAL;
  if (epilogue != EPI_STORE && epilogue != EPI_SILU) return OMNI_EINVAL;
  if (epilogue == EPI_SILU && (N & 31)) return OMNI_EUNSUPPORTED;
  if (ldo < (epilogue == EPI_SILU ? N / 2 : N)) return OMNI_EINVAL;
  if (cpw != 1 && cpw != 2) return OMNI_EINVAL;
  if (epilogue == EPI_SILU) cpw = 2;
  if (cpw == 2 && (N & 31)) return OMNI_EUNSUPPORTED;  // tiles are taken in pairs
  const int KG = K >> 7;
  if (ksplit < 1 || ksplit > KG) return OMNI_EINVAL;
  if (ksplit > 1 && (!ws || !counters)) return OMNI_EINVAL;
  GemvArgs a = {};
  a.x = (const half_t*)x;
  a.ldx = ldx;
  a.w = w;
  a.scales = (const half_t*)scales;
  a.bias = (const half_t*)bias;
  a.bias_after_round = bias_after_round;
  a.out = (half_t*)out;
  a.ldo = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KS = ksplit;
  a.KC = ((KG + ksplit - 1) / ksplit) * 128;
  a.KS = (K + a.KC - 1) / a.KC;  // effective splits after rounding the chunk
  a.ws = ws;
  a.counters = counters;
  hipStream_t st = (hipStream_t)stream;
  if (wf == W_INT4) {
    return epilogue == EPI_SILU ? dispatch<W_INT4, EPI_SILU>(a, cpw, st)
                                : dispatch<W_INT4, EPI_STORE>(a, cpw, st);
  }
  return epilogue == EPI_SILU ? dispatch<W_FP16, EPI_SILU>(a, cpw, st)
                              : dispatch<W_FP16, EPI_STORE>(a, cpw, st);
}

extern "C" int omni_w4a16_gemm(const void* x, int ldx, const void* qweight_packed,
                               const void* scales_packed, const void* bias, int bias_after_round,
                               void* out, int ldo, int M, int N, int K, int epilogue, int ksplit,
                               int cols_per_wave, float* workspace, int* counters, void* stream) {
  return gemv_common(W_INT4, x, ldx, qweight_packed, scales_packed, bias, bias_after_round, out,
                     ldo, M, N, K, epilogue, ksplit, cols_per_wave, workspace, counters, stream);
}

extern "C" int omni_f16_gemm(const void* x, int ldx, const void* weight_packed, const void* bias,
                             void* out, int ldo, int M, int N, int K, int epilogue, int ksplit,
                             int cols_per_wave, float* workspace, int* counters, void* stream) {
  return gemv_common(W_FP16, x, ldx, weight_packed, nullptr, bias, 0, out, ldo, M, N, K, epilogue,
                     ksplit, cols_per_wave, workspace, counters, stream);
}

// Number of workgroups omni_lmhead_argmax launches (sizes its candidate buffers).
extern "C" int omni_lmhead_argmax_grid(int N) {
  const int NT = N >> 4;
  return (NT + 7) / 8;
}

extern "C" int omni_lmhead_argmax(const void* x, int ldx, const void* weight_packed, int M, int N,
                                  int K, void* logits_out, int64_t* ids_out, float* cand_val,
                                  int* cand_idx, int* counter, void* stream) {
  if (M <= 0 || N <= 0 || K <= 0) return M == 0 ? OMNI_OK : OMNI_EINVAL;
  if (M > 64) return OMNI_EUNSUPPORTED;
  if ((N & 31) || (K & 127)) return OMNI_EUNSUPPORTED;
  if (!x || !weight_packed || !ids_out || !cand_val || !cand_idx || !counter) return OMNI_EINVAL;
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
  a.counters = counter;
  a.cand_val = cand_val;
  a.cand_idx = cand_idx;
  a.ids_out = ids_out;
  const int grid = omni_lmhead_argmax_grid(N);
  return dispatch_mb<W_FP16, EPI_ARGMAX, 2, 4, 2>(a, grid, (hipStream_t)stream);
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

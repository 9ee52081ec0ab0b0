// M-RoPE applied in place on Q/K with a fused KV-pool write.
//
// Follows omniserve/model/qwen2_llm.py:59-72 (apply_mrope / rotate_half) and
// cache/kv_prealloc.py:253-261 (_write_kv: rotated K and raw V go to pool row
// slot*max_len + write_pos before attention runs).
//
// For head_dim 128 the rotary pair (d, d+64) shares frequency j = d and one
// position axis: with doubled sections [s0,s1,s2,s0,s1,s2], dim d (< 64) uses
// axis 0 when d < s0, axis 1 when d < s0+s1, else axis 2.  The rotation is
// done with the reference's fp16 roundings:
//   y[d]    = fp16( fp16(x[d]*c)    + fp16(-x[d+64]*s) )
//   y[d+64] = fp16( fp16(x[d+64]*c) + fp16( x[d]*s)    )
// where c, s are the fp16 cos/sin of pos*inv_freq[d] (fp32 then cast, as in
// qwen2_llm.py:172-177, 181), read from a host-built table [max_pos, 64].
#include "common.h"

#define ROPE_HD 128

// Optional input from the qkv projection's fp32 split-K partials [nparts][T][qkv_stride]:
// the qkv row is then fp16(sum of partials in slice order) (+ bias: fp16(fp16(acc) + b)
// when bias_after_round, the GPTQ path, else fp16(acc + b)), and is written back to
// qkv (rotated q/k, raw v) so the attention reads q from there.
struct QkvParts {
  const float* parts;
  int nparts;
  const half_t* bias;
  int bias_after_round;
};

__device__ __forceinline__ half8_t qkv_chunk(const half_t* row, const QkvParts& qp, int t, int T,
                                             int stride, int col) {
#pragma clang fp contract(off)
  if (!qp.parts) return *(const half8_t*)(row + col);
  float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  sum_slices8(qp.parts + (int64_t)t * stride + col, (int64_t)T * stride, qp.nparts, sum);
  half8_t v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (qp.bias) {
      const float b = (float)qp.bias[col + e];
      v[e] = qp.bias_after_round ? (half_t)((float)(half_t)sum[e] + b) : (half_t)(sum[e] + b);
    } else {
      v[e] = (half_t)sum[e];
    }
  }
  return v;
}

__global__ __launch_bounds__(256) void mrope_kv_kernel(
    half_t* __restrict__ qkv, int qkv_stride, const int64_t* __restrict__ positions,
    const int64_t* __restrict__ base_pos, const int64_t* __restrict__ rope_delta,
    const half_t* __restrict__ cos_tab, const half_t* __restrict__ sin_tab, int max_pos,
    half_t* __restrict__ k_cache, half_t* __restrict__ v_cache, const int64_t* __restrict__ slots,
    const int64_t* __restrict__ write_pos, int pool_rows, int max_len, int T, int nh, int nkv,
    int s0, int s1, QkvParts qp) {
#pragma clang fp contract(off)
  // one workgroup per token: every (head, 8-dim chunk) item has its own thread
  const int lane = threadIdx.x;
  const int t = blockIdx.x;
  if (t >= T) return;

  const int64_t slot = slots ? slots[t] : t;
  int64_t p[3];
  if (positions) {
#pragma unroll
    for (int a = 0; a < 3; ++a) p[a] = positions[(int64_t)a * T + t];
  } else {
    // Decode: every axis is write_pos + rope_delta (models/qwen2_vl.py:108-112).
    // base_pos / rope_delta are indexed by pool row; out-of-range rows read nothing.
    const bool row_ok = slot >= 0 && (!slots || slot < pool_rows);
    const int64_t wp = row_ok ? base_pos[slots ? slot : t] : 0;
    const int64_t d = (row_ok && rope_delta) ? rope_delta[slots ? slot : t] : 0;
    p[0] = p[1] = p[2] = wp + d;
  }
#pragma unroll
  for (int a = 0; a < 3; ++a) p[a] = p[a] < 0 ? 0 : (p[a] >= max_pos ? max_pos - 1 : p[a]);

  // The write position is only read when there is a pool to write into (rotate-only
  // calls pass neither write_pos nor base_pos).
  bool do_write = k_cache != nullptr && slot >= 0 && slot < pool_rows;
  int64_t wpos = 0;
  if (do_write) {
    wpos = write_pos ? write_pos[t] : base_pos[slots ? slot : t];
    do_write = wpos >= 0 && wpos < max_len;
  }

  half_t* row = qkv + (int64_t)t * qkv_stride;
  const int rot_items = (nh + nkv) * 8;  // 8 chunks of 8 dims in the first half of each head
  const int total = rot_items + nkv * 16;
  for (int it = lane; it < total; it += 256) {
    if (it < rot_items) {
      const int head = it >> 3;
      const int d0 = (it & 7) * 8;
      const int axis = d0 < s0 ? 0 : (d0 < s0 + s1 ? 1 : 2);
      const half8_t c = *(const half8_t*)(cos_tab + p[axis] * 64 + d0);
      const half8_t s = *(const half8_t*)(sin_tab + p[axis] * 64 + d0);
      half_t* hp = row + head * ROPE_HD;
      const half8_t x1 = qkv_chunk(row, qp, t, T, qkv_stride, head * ROPE_HD + d0);
      const half8_t x2 = qkv_chunk(row, qp, t, T, qkv_stride, head * ROPE_HD + d0 + 64);
      // IEEE fp16 multiplies and adds (each rounds once, RNE), no contraction:
      // exactly the three fp16 roundings of q*cos + rotate_half(q)*sin.
      const half8_t a1 = x1 * c;
      const half8_t b1 = (-x2) * s;
      const half8_t a2 = x2 * c;
      const half8_t b2 = x1 * s;
      const half8_t y1 = a1 + b1;
      const half8_t y2 = a2 + b2;
      *(half8_t*)(hp + d0) = y1;
      *(half8_t*)(hp + d0 + 64) = y2;
      if (head >= nh && do_write) {
        const int g = head - nh;
        half_t* kp = k_cache + ((slot * max_len + wpos) * nkv + g) * ROPE_HD;
        *(half8_t*)(kp + d0) = y1;
        *(half8_t*)(kp + d0 + 64) = y2;
      }
    } else if (do_write || qp.parts) {
      const int idx = it - rot_items;
      const int g = idx >> 4;
      const int d0 = (idx & 15) * 8;
      const int col = (nh + nkv) * ROPE_HD + g * ROPE_HD + d0;
      const half8_t v = qkv_chunk(row, qp, t, T, qkv_stride, col);
      if (qp.parts) *(half8_t*)(row + col) = v;
      if (do_write) *(half8_t*)(v_cache + ((slot * max_len + wpos) * nkv + g) * ROPE_HD + d0) = v;
    }
  }
}

// positions: int64 [3, T] (t/h/w axes), or NULL to use base_pos[slot] + rope_delta[slot]
// on all three axes (decode).  write_pos: int64 [T], or NULL to use base_pos[slot].
// slots: int64 [T] pool rows, or NULL for row t.  k_cache/v_cache NULL = rotate only.
extern "C" int omni_mrope_kv_write(void* qkv, int qkv_stride, const int64_t* positions,
                                   const int64_t* base_pos, const int64_t* rope_delta,
                                   const void* cos_tab, const void* sin_tab, int max_pos,
                                   void* k_cache, void* v_cache, const int64_t* slots,
                                   const int64_t* write_pos, int pool_rows, int max_len, int T,
                                   int n_heads, int n_kv_heads, int head_dim, int sec0, int sec1,
                                   int sec2, void* stream) {
  if (T < 0 || n_heads <= 0 || n_kv_heads <= 0 || max_pos <= 0) return OMNI_EINVAL;
  if (head_dim != ROPE_HD || sec0 + sec1 + sec2 != ROPE_HD / 2) return OMNI_EUNSUPPORTED;
  if ((sec0 & 7) || (sec1 & 7) || (sec2 & 7)) return OMNI_EUNSUPPORTED;
  if (qkv_stride < (n_heads + 2 * n_kv_heads) * ROPE_HD || (qkv_stride & 7)) return OMNI_EINVAL;
  if (T == 0) return OMNI_OK;
  if (!qkv || !cos_tab || !sin_tab) return OMNI_EINVAL;
  if (!positions && !base_pos) return OMNI_EINVAL;
  if (!write_pos && !base_pos && k_cache) return OMNI_EINVAL;
  if ((k_cache == nullptr) != (v_cache == nullptr)) return OMNI_EINVAL;
  if (k_cache && (pool_rows <= 0 || max_len <= 0)) return OMNI_EINVAL;
  QkvParts qp = {nullptr, 0, nullptr, 0};
  hipLaunchKernelGGL(mrope_kv_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream,
                     (half_t*)qkv, qkv_stride, positions, base_pos, rope_delta,
                     (const half_t*)cos_tab, (const half_t*)sin_tab, max_pos, (half_t*)k_cache,
                     (half_t*)v_cache, slots, write_pos, pool_rows, max_len, T, n_heads, n_kv_heads,
                     sec0, sec1, qp);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// As omni_mrope_kv_write, with the qkv rows taken from the qkv projection's fp32
// split-K partials [nparts][T][qkv_stride] (+ bias) and written to qkv.
extern "C" int omni_mrope_kv_write_partials(
    void* qkv, int qkv_stride, const float* partials, int nparts, const void* bias,
    int bias_after_round, const int64_t* positions, const int64_t* base_pos,
    const int64_t* rope_delta, const void* cos_tab, const void* sin_tab, int max_pos,
    void* k_cache, void* v_cache, const int64_t* slots, const int64_t* write_pos, int pool_rows,
    int max_len, int T, int n_heads, int n_kv_heads, int head_dim, int sec0, int sec1, int sec2,
    void* stream) {
  if (T < 0 || n_heads <= 0 || n_kv_heads <= 0 || max_pos <= 0 || nparts <= 0) return OMNI_EINVAL;
  if (head_dim != ROPE_HD || sec0 + sec1 + sec2 != ROPE_HD / 2) return OMNI_EUNSUPPORTED;
  if ((sec0 & 7) || (sec1 & 7) || (sec2 & 7)) return OMNI_EUNSUPPORTED;
  if (qkv_stride != (n_heads + 2 * n_kv_heads) * ROPE_HD) return OMNI_EINVAL;
  if (T == 0) return OMNI_OK;
  if (!qkv || !partials || !cos_tab || !sin_tab) return OMNI_EINVAL;
  if (!positions && !base_pos) return OMNI_EINVAL;
  if (!write_pos && !base_pos && k_cache) return OMNI_EINVAL;
  if ((k_cache == nullptr) != (v_cache == nullptr)) return OMNI_EINVAL;
  if (k_cache && (pool_rows <= 0 || max_len <= 0)) return OMNI_EINVAL;
  QkvParts qp = {partials, nparts, (const half_t*)bias, bias_after_round};
  hipLaunchKernelGGL(mrope_kv_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream,
                     (half_t*)qkv, qkv_stride, positions, base_pos, rope_delta,
                     (const half_t*)cos_tab, (const half_t*)sin_tab, max_pos, (half_t*)k_cache,
                     (half_t*)v_cache, slots, write_pos, pool_rows, max_len, T, n_heads, n_kv_heads,
                     sec0, sec1, qp);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// GQA decode attention over the preallocated KV pool.
//
// Replaces the paged flash-decode call in omniserve/cache/kv_prealloc.py:272-290:
// for every query token t (pool row slot[t]) and query head h the output is
//   softmax(scale * q[t,h] . K[slot, 0:L, h div G]^T) . V[slot, 0:L, h div G]
// with L = kv_len (keys [0, L), inclusive of the token written this step),
// G = n_heads / n_kv_heads query heads per KV head (6 for Qwen2-VL-2B).
//
// Pool layout (kept from the reference): K, V = [pool_rows, max_len, n_kv, 128] fp16.
//
// Work split: one workgroup per (token, kv head); its NWA waves (4, 8 or 16) each
// stream a contiguous 32-token-aligned range of the context, so each K/V row of a
// KV head is read from HBM exactly once for all G query heads sharing it, and the
// waves' partial softmax states are merged in LDS.  Nothing crosses workgroups (no
// device-scope fences).  Per 32-token block a wave does
//   S^T[16 tok x 16 heads] = K[16 x 128] . Q^T     (4 MFMA 16x16x32 per 16 tokens,
//                                                   K fed straight from global)
//   online softmax in fp32 (exp2, running max/sum per head)
//   O[16 heads x 128] += P[16 x 32] . V[32 x 128]  (8 MFMAs, V transposed via LDS)
// while the next block's K and V loads are already in flight (streamed with
// non-temporal loads: each pool row is read once per step).
#include "common.h"

#define ATT_HD 128
#define ATT_BLK 32
#define ATT_VSTRIDE 144   // LDS row stride (halfs) of the V tile: rows 8 banks apart, so the
                          // 4 rows x 32 bytes of one 16-lane transpose read hit 32 distinct banks
#define ATT_MAXG 16       // query heads per KV head supported (MFMA N = 16)
#define ATT_FUSED_MAXG 8  // ... by the fused decode prologue
#define ATT_WAVES 4       // waves per workgroup of the prefill kernel

struct AttnArgs {
  const half_t* q;
  int q_stride;          // elements between tokens
  const half_t* k_cache;
  const half_t* v_cache;
  int pool_rows, max_len, nkv, G;
  const int64_t* slots;  // [T] or NULL (row t)
  const int64_t* kv_len; // [T] (or indexed by slot when kv_by_slot)
  int kv_by_slot;
  int kv_add;            // kv = kv_len[...] + kv_add
  half_t* out;           // [T, nkv*G, 128]
  float* part;           // parts_out: [T][nkv][S][G][ATT_REC] fp32 split states
  int S;                 // workgroups per (token, kv head)
  int parts_out;         // 1: states to part (S > 1, or left for the consumer); 0: fp16 out
  float scale_log2;
  int T;
  // Fused decode prologue (qparts != NULL): q, and the new token's k / v, are formed
  // from the qkv projection's fp32 split-K partials [nq][T][(nh + 2 nkv) * 128] (+ bias),
  // M-RoPE'd at position kv_len[slot] + rope_delta[slot] (the token is written at
  // kv_len[slot], kv_add must be 1), and the new K/V row is written to the pool.
  const float* qparts;
  int nq;
  const half_t* qbias;
  int bias_after_round;
  const half_t* cos_tab;
  const half_t* sin_tab;
  int max_pos;
  const int64_t* rope_delta;
  int s0, s1;
  // Precomputed rotary rows [T][128] fp16: cos | sin of p * inv_freq at each token's
  // position p (the same for every layer of a decode step, so written once per step).
  const half_t* rope_rows;
};

#define ATT_MAXPARTS 8   // qkv partial slices the fused prologue sums (one batch of loads)

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// FUSED: q and the new token's k / v come from the qkv partials (a.qparts != NULL), with
// the rotary row looked up in the cos/sin tables at the token's position (FUSED = 1) or
// read from precomputed rows (FUSED = 2, requested with the partials, so that it is not a
// second round trip behind the context length, queued behind the grid's K/V stream).  The
// forms are separate instantiations so that none carries another's wait states.
template <int NWA, int FUSED>
__global__ __launch_bounds__(NWA * 64, NWA <= 8 ? 8 / NWA : 1) void decode_attn_kernel(AttnArgs a) {
  constexpr int NT = NWA * 64;
  // The V tiles (block loop), the fused prologue's pre-rotation rows (before it) and
  // the per-wave partial outputs (after it) share one LDS buffer.
  constexpr int kVsBytes = NWA * ATT_BLK * ATT_VSTRIDE * 2;
  constexpr int kOBytes = NWA * ATT_MAXG * ATT_HD * 4;
  constexpr int kRawBytes = (ATT_FUSED_MAXG + 2) * ATT_HD * 2;
  constexpr int kSmem = kVsBytes > kOBytes ? (kVsBytes > kRawBytes ? kVsBytes : kRawBytes)
                                           : (kOBytes > kRawBytes ? kOBytes : kRawBytes);
  __shared__ __attribute__((aligned(16))) char smem[kSmem];
  __shared__ float ml_lds[NWA][ATT_MAXG][2];
  __shared__ __attribute__((aligned(16))) half_t q_lds[ATT_FUSED_MAXG][ATT_HD];   // fused prologue
  __shared__ __attribute__((aligned(16))) half_t kv_new[2][ATT_HD];
  __shared__ __attribute__((aligned(16))) half_t cs_lds[2][ATT_HD / 2];
  half_t (*vs_lds)[ATT_BLK * ATT_VSTRIDE] = (half_t (*)[ATT_BLK * ATT_VSTRIDE])smem;
  // per-wave partial outputs for the merge: [wave][head][c16][dt] = O[head][16 dt + c16]
  float (*o_lds)[ATT_MAXG][16][8] = (float (*)[ATT_MAXG][16][8])smem;
  half_t* raw = (half_t*)smem;   // fused: [G + 2][128] q heads | k | v before M-RoPE

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q16 = lane >> 4;     // lane group 0..3
  const int c16 = lane & 15;     // column within MFMA tile
  // Every argument the prologue's addresses need is read into registers in one batch
  // first: scalar loads complete out of order, so a wait for any one of them waits for all,
  // and an argument fetched after the context length would hold the prologue's global
  // loads behind the length's round trip (each such chain is a memory round trip).
  asm volatile("" ::"s"(a.S), "s"(a.nkv), "s"(a.G), "s"(a.T), "s"(a.nq), "s"(a.max_len),
               "s"(a.pool_rows), "s"(a.kv_by_slot), "s"(a.kv_add), "s"(a.max_pos),
               "s"(a.qparts), "s"(a.qbias), "s"(a.kv_len), "s"(a.slots), "s"(a.rope_delta),
               "s"(a.cos_tab), "s"(a.sin_tab), "s"(a.k_cache), "s"(a.v_cache), "s"(gridDim.x),
               "s"(a.bias_after_round), "s"(a.out), "s"(a.part), "s"(a.parts_out),
               "s"(a.scale_log2), "s"(a.q), "s"(a.q_stride), "s"(a.s0), "s"(a.s1),
               "s"(a.rope_rows));
  const int S = a.S;
  // The S workgroups of one (token, kv head) are neighbours in XCD-aware order, so they
  // share an L2 and the token's qkv partials are fetched from HBM once, not S times.
  const int blk = xcd_logical_block(blockIdx.x, gridDim.x);
  const int sp = blk % S;
  const int g = (blk / S) % a.nkv;
  const int t = blk / (S * a.nkv);
  const int G = a.G;
  const int nh = a.nkv * G;
  constexpr bool fused = FUSED != 0;

  // 1. Loads that do not depend on the context length, all issued before any is used (a
  //    load placed after a store or a use would cost the prologue another memory round
  //    trip): for the fused prologue, q heads g*G .. g*G+G-1 and k, v of kv head g as fp32
  //    split-K partials (at most ATT_MAXPARTS slices, all in flight at once) and their
  //    bias, then the context length and rope delta of this token's pool row.  Optional
  //    operands are read through a valid stand-in address and replaced by zero, so no
  //    load sits behind a branch.
  // The context length first, as scalar loads: they are counted apart from the vector
  // loads below, so the first K/V block can go out once the length is in, without waiting
  // for the partials.
  // (Read through the constant address space: this launch never writes them, and the
  // compiler would otherwise use vector loads, as the kernel stores to global memory.)
  typedef __attribute__((address_space(4))) const int64_t c_i64;
  const int64_t slot = a.slots ? ((const c_i64*)a.slots)[t] : t;
  const bool slot_ok = slot >= 0 && slot < a.pool_rows;
  const int64_t srow = slot_ok ? slot : 0;
  const int64_t kv_raw = ((const c_i64*)a.kv_len)[a.kv_by_slot ? srow : t];
  const int64_t* dptr = a.rope_delta ? a.rope_delta : a.kv_len;
  const int64_t delta_raw = FUSED == 1 ? ((const c_i64*)dptr)[srow] : 0;
  constexpr int PI = ((ATT_FUSED_MAXG + 2) * ATT_HD / 2 + NT - 1) / NT;
  float2 pv[PI][8];
  half2_t bias2[PI];
  const int nel2 = (G + 2) * (ATT_HD / 2);
  const int W = (nh + 2 * a.nkv) * ATT_HD;
  const int64_t ps = (int64_t)a.T * W;
  auto gathered_col = [&](int e) {       // element e of the gathered row -> qkv column
    const int hh = e / ATT_HD;
    const int d = e % ATT_HD;
    const int head = hh < G ? g * G + hh : (hh == G ? nh + g : nh + a.nkv + g);
    return head * ATT_HD + d;
  };
  if (fused) {
    const float* rowp = a.qparts + (int64_t)t * W;
    const half_t* bptr = a.qbias ? a.qbias : (const half_t*)a.qparts;
#pragma unroll
    for (int j = 0; j < PI; ++j) {
      // an element past the gathered row re-reads this thread's first one and is not used;
      // a slot past nq re-reads the last slice and is not added
      const int i = threadIdx.x + j * NT;
      const int col = gathered_col(2 * (i < nel2 ? i : (int)threadIdx.x % nel2));
      const float* src = rowp + col;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int uu = u < a.nq ? u : a.nq - 1;
        pv[j][u] = *(const float2*)(src + uu * ps);
      }
      bias2[j] = *(const half2_t*)(bptr + col);
    }
  }
  // cos (threads 0-7) / sin (8-15) chunk of the token's rotary row.  Every thread issues
  // the load (threads past 15 re-read a chunk and drop it): a load behind a thread-index
  // branch leaves the compiler unsure whether it is outstanding, and it then waits for it
  // (vmcnt(0)) before using any load issued earlier.
  half8_t csv = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
  if constexpr (FUSED == 2)
    csv = *(const half8_t*)(a.rope_rows + (int64_t)t * ATT_HD + (threadIdx.x & 15) * 8);

  // 2. Context length, this workgroup's key range, the rotary row.
  const int64_t L_raw = slot_ok ? kv_raw + a.kv_add : 0;
  const int64_t L = clamp64(L_raw, 0, a.max_len);
  // fused decode: the token written this step sits at index L - 1 (= kv_len[slot]); a row
  // already at capacity (kv_len >= max_len) writes nothing and attends to the pool as is.
  const int newtok = fused && L_raw == L ? (int)L - 1 : -1;

  // The context's 32-token blocks are dealt out evenly to the S*NWA waves of the
  // (token, kv head): wave w gets blocks [w*nblk/nw, (w+1)*nblk/nw).
  const int nblk = (int)((L + ATT_BLK - 1) / ATT_BLK);
  const int nw = S * NWA;
  const int wsplit = sp * NWA + wave;
  const int beg = (int)min((int64_t)((int64_t)wsplit * nblk / nw) * ATT_BLK, L);
  const int end = (int)min((int64_t)((int64_t)(wsplit + 1) * nblk / nw) * ATT_BLK, L);
  const int wg_b0 = (int)((int64_t)sp * NWA * nblk / nw);
  const int wg_b1 = (int)((int64_t)(sp + 1) * NWA * nblk / nw);

  // FUSED = 1: the rotary row from the tables at the token's position (a load that waits
  // for the context length).
  if constexpr (FUSED == 1) {
    int64_t pos = slot_ok ? kv_raw + (a.rope_delta ? delta_raw : 0) : 0;
    pos = clamp64(pos, 0, a.max_pos - 1);
    const half_t* tab = (threadIdx.x & 15) < 8 ? a.cos_tab : a.sin_tab;
    csv = *(const half8_t*)(tab + pos * (ATT_HD / 2) + (threadIdx.x & 7) * 8);
  }

  // 3. The K/V blocks of this wave (the first is issued below).
  const int64_t row_base = (slot_ok ? slot : 0) * (int64_t)a.max_len;
  const int tok_hi = end > 0 ? end - 1 : 0;    // loads past the range re-read this row
  const half_t* kbase = a.k_cache + g * ATT_HD;
  const half_t* vbase = a.v_cache + g * ATT_HD;
  const int64_t tok_stride = (int64_t)a.nkv * ATT_HD;
  half_t* vs = vs_lds[wave];

  auto load_block = [&](half8_t (&kf)[2][4], half8_t (&vr)[8], int tb) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int tok = tb + 16 * j + c16;
      tok = tok < tok_hi ? tok : tok_hi;
      const half_t* kp = kbase + (row_base + tok) * tok_stride + q16 * 8;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kf[j][ks] = __builtin_nontemporal_load((const half8_t*)(kp + ks * 32));
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int c = lane + 64 * r;          // 512 chunks of 8 halfs = 32 tokens x 128 dims
      int tok = tb + (c >> 4);
      tok = tok < tok_hi ? tok : tok_hi;
      vr[r] = __builtin_nontemporal_load((const half8_t*)(vbase + (row_base + tok) * tok_stride + (c & 15) * 8));
    }
  };
  // One 32-token block (16 KB of K and V) in flight per wave: the next block is requested
  // once the current one's K and V have been consumed (V staged in LDS, scores done).
  // Measured on a plain 67 MB stream, 8 waves per CU each keeping 8 / 16 / 32 KB in flight
  // take 11.9 / 13.0 / 15.7 us: more requests outstanding per CU only lengthen the queues.
  // The first block goes out as soon as the context length is in (after the prologue's own
  // loads, which a load issued behind the grid's K/V requests would wait for); the wave's
  // issue of it stalls while the CU has many requests outstanding, so nothing of the
  // prologue waits behind a second block.  (A wave without blocks re-reads its clamped
  // last row, from cache: with a branch around the load the compiler's wait counts would
  // no longer be exact.)
  half8_t kf0[2][4], vr0[8];
  load_block(kf0, vr0, beg);

  if (fused) {
    // 4. Partial sums (slice order, as the unfused path) + bias -> fp16 rows in LDS.
#pragma clang fp contract(off)
    const float* rowp = a.qparts + (int64_t)t * W;
#pragma unroll
    for (int j = 0; j < PI; ++j) {
      const int i = threadIdx.x + j * NT;
      if (i < nel2) {
        const int col = gathered_col(2 * i);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bool on = u < a.nq;
          s0 += on ? pv[j][u].x : 0.f;
          s1 += on ? pv[j][u].y : 0.f;
        }
        half_t h0 = (half_t)s0, h1 = (half_t)s1;
        if (a.qbias) {
          const float b0 = (float)bias2[j][0], b1 = (float)bias2[j][1];
          h0 = a.bias_after_round ? (half_t)((float)h0 + b0) : (half_t)(s0 + b0);
          h1 = a.bias_after_round ? (half_t)((float)h1 + b1) : (half_t)(s1 + b1);
        }
        raw[2 * i] = h0;
        raw[2 * i + 1] = h1;
      }
    }
    if (threadIdx.x < 16) *(half8_t*)(&cs_lds[threadIdx.x >> 3][(threadIdx.x & 7) * 8]) = csv;
    lds_barrier();
    // 5. M-RoPE (decode: one position on all three axes) in fp16 ops, one rounding
    //    each and no contraction: y1 = x1*c + (-x2)*s, y2 = x2*c + x1*s.
    for (int i = threadIdx.x; i < (G + 1) * 64 + 64; i += NT) {
      if (i < (G + 1) * 64) {
        const int hh = i >> 6;
        const int d = i & 63;
        const half_t x1 = raw[hh * ATT_HD + d];
        const half_t x2 = raw[hh * ATT_HD + d + 64];
        const half_t c = cs_lds[0][d];
        const half_t s = cs_lds[1][d];
        const half_t y1 = x1 * c + (-x2) * s;
        const half_t y2 = x2 * c + x1 * s;
        half_t* dst = hh < G ? q_lds[hh] : kv_new[0];
        dst[d] = y1;
        dst[d + 64] = y2;
      } else {
        const int j = i - (G + 1) * 64;
        kv_new[1][2 * j] = raw[(G + 1) * ATT_HD + 2 * j];
        kv_new[1][2 * j + 1] = raw[(G + 1) * ATT_HD + 2 * j + 1];
      }
    }
    lds_barrier();
    // 6. The workgroup whose blocks hold the new token stores its K/V row in the pool.
    const int nb = newtok >> 5;
    if (newtok >= 0 && nb >= wg_b0 && nb < wg_b1 && threadIdx.x < 32) {
      const int kvsel = threadIdx.x >> 4;
      const int c = threadIdx.x & 15;
      half_t* dst = const_cast<half_t*>(kvsel ? a.v_cache : a.k_cache) +
                    (row_base + newtok) * tok_stride + g * ATT_HD + c * 8;
      *(half8_t*)dst = *(const half8_t*)(kv_new[kvsel] + c * 8);
    }
  }

  // Q fragments: B operand of S^T = K Q^T.  Lane holds head c16, dims 32ks + 8*q16 + e.
  half8_t qf[4];
  {
    const bool hv = c16 < G;
    const half_t* qp = fused ? q_lds[hv ? c16 : 0]
                             : a.q + (int64_t)t * a.q_stride + (int64_t)(g * G + (hv ? c16 : 0)) * ATT_HD;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      half8_t v = *(const half8_t*)(qp + ks * 32 + q16 * 8);
      if (!hv) v = (half8_t){0, 0, 0, 0, 0, 0, 0, 0};
      qf[ks] = v;
    }
  }

  float m_run = -INFINITY;   // per head c16 (identical across q16 groups)
  float l_run = 0.f;         // lane-partial sum, reduced at the end
  f32x4 o_acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o_acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // One 32-token block: its K/V sit in (kf, vr); once they are consumed the same
  // registers are refilled with the next block.
  auto process = [&](half8_t (&kf)[2][4], half8_t (&vr)[8], int tb) {
    // The new token's K/V come from the prologue, not from the pool row being written.
    // Rows past the range were loaded from row end - 1 (= newtok in the last range), so
    // they are compared by that clamped index: masked rows never carry stale pool data.
    if (newtok >= tb && newtok < tb + ATT_BLK) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (min(tb + 16 * j + c16, end - 1) == newtok)
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) kf[j][ks] = *(const half8_t*)(kv_new[0] + ks * 32 + q16 * 8);
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int c = lane + 64 * r;
        if (min(tb + (c >> 4), end - 1) == newtok) vr[r] = *(const half8_t*)(kv_new[1] + (c & 15) * 8);
      }
    }
    // Stage this block's V into LDS (row-major, padded).
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int c = lane + 64 * r;
      *(half8_t*)(vs + (c >> 4) * ATT_VSTRIDE + (c & 15) * 8) = vr[r];
    }
    // Scores: acc[j][i] = token tb + 16j + 4*q16 + i, head c16.
    f32x4 sacc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(kf[j][ks], qf[ks], acc);
      sacc[j] = acc;
    }
    if (tb + ATT_BLK < end) load_block(kf, vr, tb + ATT_BLK);   // the next block

    float sc[8];
    float mblk = -INFINITY;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = tb + 16 * j + 4 * q16 + i;
        const float s = tok < end ? sacc[j][i] * a.scale_log2 : -INFINITY;
        sc[4 * j + i] = s;
        mblk = fmaxf(mblk, s);
      }
    mblk = fmaxf(mblk, __shfl_xor(mblk, 16, 64));
    mblk = fmaxf(mblk, __shfl_xor(mblk, 32, 64));
    const float m_new = fmaxf(m_run, mblk);
    const float alpha = exp2f(m_run - m_new);   // m_run = -inf -> 0
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

    // Rescale O rows (heads 4*q16 + i) by their head's alpha.
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * q16 + i, 64);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o_acc[dt][i] *= al[i];

    // P (A operand: head c16, slot s8 <-> token 16*(s8/4) + 4*q16 + s8%4) times V.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const half8_t vb = lds_read_b_tr16(vs + dt * 16, ATT_VSTRIDE, q16, c16);
      o_acc[dt] = mfma16x16x32(pa, vb, o_acc[dt]);
    }
    __builtin_amdgcn_wave_barrier();
  };

  for (int tb = beg; tb < end; tb += ATT_BLK) process(kf0, vr0, tb);

  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  __syncthreads();   // every wave is done with its V tile before o_lds reuses the space

  // Merge the waves' softmax states.  Lane (q16, c16) holds O[head 4 q16 + i][16 dt + c16];
  // it stores them as 32 contiguous bytes per head, so that thread (h, c) of the merge
  // reads the 8 dims 16 dt + c of every wave with two 16-byte LDS reads.
  if (lane < G) {
    ml_lds[wave][lane][0] = m_run;
    ml_lds[wave][lane][1] = l_run;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * q16 + i;
    if (h < G) {
      f32x4 lo = {o_acc[0][i], o_acc[1][i], o_acc[2][i], o_acc[3][i]};
      f32x4 hi = {o_acc[4][i], o_acc[5][i], o_acc[6][i], o_acc[7][i]};
      *(f32x4*)&o_lds[wave][h][c16][0] = lo;
      *(f32x4*)&o_lds[wave][h][c16][4] = hi;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < G * 16) {
    const int h = threadIdx.x >> 4;
    const int c = threadIdx.x & 15;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWA; ++w) M = fmaxf(M, ml_lds[w][h][0]);
    float lsum = 0.f;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NWA; ++w) {
        const float f = exp2f(ml_lds[w][h][0] - M);
        lsum += f * ml_lds[w][h][1];
        const f32x4 lo = *(const f32x4*)&o_lds[w][h][c][0];
        const f32x4 hi = *(const f32x4*)&o_lds[w][h][c][4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] += f * lo[e];
          o[4 + e] += f * hi[e];
        }
      }
    }
    if (!a.parts_out) {
      half_t* op = a.out + ((int64_t)t * nh + g * G + h) * ATT_HD + c;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) op[16 * dt] = (half_t)(lsum > 0.f ? o[dt] / lsum : 0.f);
    } else {
      float* pp = a.part + ((((int64_t)t * a.nkv + g) * S + sp) * G + h) * ATT_REC;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) pp[16 * dt + c] = o[dt];
      if (c == 0) {
        pp[ATT_HD] = M;
        pp[ATT_HD + 1] = lsum;
      }
    }
  }
}

// Merge of the S partial softmax states of each (token, kv head) written by
// decode_attn_kernel (a separate launch: ordering comes from the kernel boundary).
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ part,
                                                           half_t* __restrict__ out, int nkv,
                                                           int G, int S) {
  const int g = blockIdx.x % nkv;
  const int t = blockIdx.x / nkv;
  const int nh = nkv * G;
  const float* base = part + ((int64_t)t * nkv + g) * S * G * ATT_REC;
  for (int idx = threadIdx.x; idx < G * (ATT_HD / 8); idx += blockDim.x) {
    const int h = idx / (ATT_HD / 8);
    const int d0 = (idx % (ATT_HD / 8)) * 8;
    *(half8_t*)(out + ((int64_t)t * nh + g * G + h) * ATT_HD + d0) =
        attn_merge8(base + (int64_t)h * ATT_REC, (int64_t)G * ATT_REC, S, d0);
  }
}

static int launch_decode_attn(AttnArgs a, int n_kv_heads, int T, int G, int waves, int splits,
                              int merge, float* workspace, hipStream_t st);

// Decode / append attention over the pool.
//   q          fp16, token t head h at q + t*q_stride + h*128
//   k/v_cache  fp16 [pool_rows, max_len, n_kv, 128]
//   slots      int64 [T] pool rows (NULL = row t)
//   kv_len     int64; keys visible to token t = kv_len[kv_by_slot ? slot : t] + kv_add
//   out        fp16 [T, n_heads, 128]
//   waves      waves per workgroup: 4 or 8
//   splits     workgroups per (token, kv head); > 1 writes partial states to
//              workspace (fp32, workspace_floats >= T * n_kv * splits * G * 132, else
//              the call is rejected) merged by a second launch
// fp32 workspace of the split states: [T][n_kv][splits][G][132].
static int64_t attn_workspace_floats(int T, int n_kv, int splits, int G) {
  return (int64_t)T * n_kv * splits * G * ATT_REC;
}

extern "C" int omni_decode_attention(const void* q, int q_stride, const void* k_cache,
                                     const void* v_cache, int pool_rows, int max_len,
                                     const int64_t* slots, const int64_t* kv_len, int kv_by_slot,
                                     int kv_add, void* out, int T, int n_heads, int n_kv_heads,
                                     int head_dim, float scale, int waves, int splits,
                                     float* workspace, int64_t workspace_floats, void* stream) {
  if (T < 0 || n_heads <= 0 || n_kv_heads <= 0 || pool_rows <= 0 || max_len <= 0) return OMNI_EINVAL;
  if (head_dim != ATT_HD || n_heads % n_kv_heads) return OMNI_EUNSUPPORTED;
  const int G = n_heads / n_kv_heads;
  if (G > ATT_MAXG) return OMNI_EUNSUPPORTED;
  if (waves != 4 && waves != 8) return OMNI_EINVAL;
  if (splits < 1 || splits > 64) return OMNI_EINVAL;
  if (q_stride < n_heads * ATT_HD || (q_stride & 7)) return OMNI_EINVAL;
  if (T == 0) return OMNI_OK;
  if (!q || !k_cache || !v_cache || !kv_len || !out) return OMNI_EINVAL;
  if (splits > 1 && (!workspace || workspace_floats < attn_workspace_floats(T, n_kv_heads, splits, G)))
    return OMNI_EINVAL;
  AttnArgs a;
  a.q = (const half_t*)q;
  a.q_stride = q_stride;
  a.k_cache = (const half_t*)k_cache;
  a.v_cache = (const half_t*)v_cache;
  a.pool_rows = pool_rows;
  a.max_len = max_len;
  a.nkv = n_kv_heads;
  a.G = G;
  a.slots = slots;
  a.kv_len = kv_len;
  a.kv_by_slot = kv_by_slot;
  a.kv_add = kv_add;
  a.out = (half_t*)out;
  a.part = workspace;
  a.S = splits;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.T = T;
  a.qparts = nullptr;
  a.nq = 0;
  a.qbias = nullptr;
  a.bias_after_round = 0;
  a.cos_tab = a.sin_tab = nullptr;
  a.max_pos = 0;
  a.rope_delta = nullptr;
  a.s0 = a.s1 = 0;
  a.rope_rows = nullptr;
  return launch_decode_attn(a, n_kv_heads, T, G, waves, splits, 1, workspace, (hipStream_t)stream);
}

static int launch_decode_attn(AttnArgs a, int n_kv_heads, int T, int G, int waves, int splits,
                              int merge, float* workspace, hipStream_t st) {
  a.parts_out = splits > 1 || !merge;
  const int64_t nblocks = (int64_t)n_kv_heads * T * splits;
  if (nblocks > 0x7fffffff) return OMNI_EUNSUPPORTED;
  const int form = a.qparts == nullptr ? 0 : (a.rope_rows ? 2 : 1);
  const dim3 grid((unsigned)nblocks);
  switch (waves * 4 + form) {
    case 16: hipLaunchKernelGGL((decode_attn_kernel<4, 0>), grid, dim3(256), 0, st, a); break;
    case 17: hipLaunchKernelGGL((decode_attn_kernel<4, 1>), grid, dim3(256), 0, st, a); break;
    case 18: hipLaunchKernelGGL((decode_attn_kernel<4, 2>), grid, dim3(256), 0, st, a); break;
    case 32: hipLaunchKernelGGL((decode_attn_kernel<8, 0>), grid, dim3(512), 0, st, a); break;
    case 33: hipLaunchKernelGGL((decode_attn_kernel<8, 1>), grid, dim3(512), 0, st, a); break;
    case 34: hipLaunchKernelGGL((decode_attn_kernel<8, 2>), grid, dim3(512), 0, st, a); break;
    default: return OMNI_EINVAL;
  }
  OMNI_CHECK_LAUNCH();
  if (splits > 1 && merge) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3(n_kv_heads * T), dim3(G * ATT_HD / 8 > 128 ? 256 : 128),
                       0, st, workspace, a.out, n_kv_heads, G, splits);
    OMNI_CHECK_LAUNCH();
  }
  return OMNI_OK;
}

// Decode step attention fused with its producer's epilogue: q and the new token's k / v
// are formed from the qkv projection's fp32 split-K partials [nparts][T][(nh+2nkv)*128]
// plus bias (bias_after_round: GPTQ rounding order), M-RoPE'd at position
// lengths[slot] + rope_delta[slot] with the fp16 cos/sin tables - or, when rope_rows is
// given, with that token's precomputed row rope_rows[t] = cos | sin at its position
// (omni_rope_rows / omni_embed_rmsnorm_rope) - the new K/V row is stored at
// pool[slot, lengths[slot]], and token t attends to keys [0, lengths[slot]].
// Replaces omni_mrope_kv_write + omni_decode_attention for a decode step (lengths are
// not advanced).  merge = 0 leaves the split states in workspace (out unused) for the
// o_proj GEMM that merges them while staging its input (omni_*_gemm_attn).
extern "C" int omni_decode_attention_fused(
    const float* qkv_partials, int nparts, const void* qkv_bias, int bias_after_round,
    const void* cos_tab, const void* sin_tab, int max_pos, const int64_t* rope_delta, int sec0,
    int sec1, int sec2, void* k_cache, void* v_cache, int pool_rows, int max_len,
    const int64_t* slots, const int64_t* lengths, void* out, int T, int n_heads, int n_kv_heads,
    int head_dim, float scale, int waves, int splits, float* workspace, int64_t workspace_floats,
    int merge, const void* rope_rows, void* stream) {
  if (T < 0 || n_heads <= 0 || n_kv_heads <= 0 || pool_rows <= 0 || max_len <= 0) return OMNI_EINVAL;
  if (!rope_rows && max_pos <= 0) return OMNI_EINVAL;
  if (head_dim != ATT_HD || n_heads % n_kv_heads) return OMNI_EUNSUPPORTED;
  if (sec0 + sec1 + sec2 != ATT_HD / 2 || (sec0 & 7) || (sec1 & 7) || (sec2 & 7)) return OMNI_EUNSUPPORTED;
  const int G = n_heads / n_kv_heads;
  if (G > ATT_FUSED_MAXG) return OMNI_EUNSUPPORTED;
  if (nparts < 1 || nparts > ATT_MAXPARTS) return OMNI_EUNSUPPORTED;
  if (waves != 4 && waves != 8) return OMNI_EINVAL;
  if (splits < 1 || splits > 64) return OMNI_EINVAL;
  if (T == 0) return OMNI_OK;
  if (!qkv_partials || !k_cache || !v_cache || !lengths) return OMNI_EINVAL;
  if (!rope_rows && (!cos_tab || !sin_tab)) return OMNI_EINVAL;
  if (merge ? !out : false) return OMNI_EINVAL;
  if ((splits > 1 || !merge) &&
      (!workspace || workspace_floats < attn_workspace_floats(T, n_kv_heads, splits, G)))
    return OMNI_EINVAL;
  AttnArgs a;
  a.q = nullptr;
  a.q_stride = 0;
  a.k_cache = (const half_t*)k_cache;
  a.v_cache = (const half_t*)v_cache;
  a.pool_rows = pool_rows;
  a.max_len = max_len;
  a.nkv = n_kv_heads;
  a.G = G;
  a.slots = slots;
  a.kv_len = lengths;
  a.kv_by_slot = 1;
  a.kv_add = 1;
  a.out = (half_t*)out;
  a.part = workspace;
  a.S = splits;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.T = T;
  a.qparts = qkv_partials;
  a.nq = nparts;
  a.qbias = (const half_t*)qkv_bias;
  a.bias_after_round = bias_after_round;
  a.cos_tab = (const half_t*)cos_tab;
  a.sin_tab = (const half_t*)sin_tab;
  a.max_pos = max_pos;
  a.rope_delta = rope_delta;
  a.s0 = sec0;
  a.s1 = sec1;
  a.rope_rows = (const half_t*)rope_rows;
  return launch_decode_attn(a, n_kv_heads, T, G, waves, splits, merge, workspace,
                            (hipStream_t)stream);
}

// ===========================================================================
// Packed (varlen) causal prefill / append attention over the pool.
//
// Replaces the varlen flash call of cache/kv_prealloc.py:181-203 (and, with
// kv_len = start + i + 1, the append form of :149-174): each query token t of
// a packed batch attends to keys [0, kv_len[t]) of its own pool row slot[t].
// One wave owns a query block of up to 16 consecutive tokens of one segment
// (same slot, increasing positions) for one query head; the MFMA structure is
// the decode kernel's with "rows" = query tokens instead of query heads:
//   S^T[16 keys x 16 queries] = K . Q^T;  O[16 queries x 128] += P . V.
// Query rows past the block end replicate its last row (never all-masked).
// ===========================================================================
struct PrefillArgs {
  const half_t* q;
  int q_stride;
  const half_t* k_cache;
  const half_t* v_cache;
  int pool_rows, max_len, nkv, G, nh;
  const int64_t* slots;    // [T]
  const int64_t* kv_len;   // [T]
  const int* qblocks;      // [nqb][2] = (first token, count <= 16)
  int nqb;
  half_t* out;
  int out_stride;
  float scale_log2;
};

// One wave's part of a (query block, head) item: the online softmax over the 32-key tiles
// [tlo, thi) of the block's key range [0, end) (tile t = keys 32 t .. 32 t + 31), for the
// 16 query rows whose Q fragments qf hold (lane (q16, c16): row c16, dims 32 ks + 8 q16 ..
// +7; lim = keys visible to row c16).  K fragments go global -> registers, the next tile's
// loads in flight during the current tile's MFMAs; V goes through the wave's LDS tile vs
// for the transposed B-operand reads.  On return: m_run = running max of row c16's scores
// (log2 units; -inf while none of its keys has been seen), l_run = this lane's part of that
// row's sum (keys 4 q16 .. +3 of every 16), o_acc = unnormalised output (row 4 q16 + i,
// column 16 dt + c16).
__device__ __forceinline__ void prefill_wave_tiles(const PrefillArgs& a, int64_t slot, int g,
                                                   int end, int lim, int tlo, int thi,
                                                   const half8_t (&qf)[4], half_t* vs,
                                                   float& m_run, float& l_run,
                                                   f32x4 (&o_acc)[8]) {
  const int lane = threadIdx.x & 63;
  const int q16 = lane >> 4;
  const int c16 = lane & 15;
  const int64_t row_base = slot * (int64_t)a.max_len;
  const half_t* kbase = a.k_cache + g * ATT_HD;
  const half_t* vbase = a.v_cache + g * ATT_HD;
  const int64_t tok_stride = (int64_t)a.nkv * ATT_HD;

  half8_t kf[2][4];
  half8_t vr[8];
  auto load_block = [&](int tb) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int tok = tb + 16 * j + c16;
      tok = tok < end ? tok : end - 1;
      const half_t* kp = kbase + (row_base + tok) * tok_stride + q16 * 8;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kf[j][ks] = *(const half8_t*)(kp + ks * 32);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int c = lane + 64 * r;
      int tok = tb + (c >> 4);
      tok = tok < end ? tok : end - 1;
      vr[r] = *(const half8_t*)(vbase + (row_base + tok) * tok_stride + (c & 15) * 8);
    }
  };

  if (tlo >= thi) return;
  load_block(tlo * ATT_BLK);
  for (int t = tlo; t < thi; ++t) {
    const int tb = t * ATT_BLK;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int c = lane + 64 * r;
      *(half8_t*)(vs + (c >> 4) * ATT_VSTRIDE + (c & 15) * 8) = vr[r];
    }
    half8_t kc[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kc[j][ks] = kf[j][ks];
    if (t + 1 < thi) load_block(tb + ATT_BLK);

    f32x4 sacc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(kc[j][ks], qf[ks], acc);
      sacc[j] = acc;
    }
    float sc[8];
    float mblk = -INFINITY;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = tb + 16 * j + 4 * q16 + i;
        const float s = key < lim ? sacc[j][i] * a.scale_log2 : -INFINITY;
        sc[4 * j + i] = s;
        mblk = fmaxf(mblk, s);
      }
    mblk = fmaxf(mblk, __shfl_xor(mblk, 16, 64));
    mblk = fmaxf(mblk, __shfl_xor(mblk, 32, 64));
    const float m_new = fmaxf(m_run, mblk);
    // -inf only for a row none of whose keys this wave has seen yet (a tile range that
    // starts past the row's last key); exp2(-inf - -inf) would be NaN.  From tile 0 on,
    // key 0 is visible to every row, so a range that starts there never needs it.
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_ref);
    m_run = m_new;
    half8_t pa;
    float psum = 0.f;
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      const float p = exp2f(sc[s8] - m_ref);
      psum += p;
      pa[s8] = (half_t)p;
    }
    l_run = l_run * alpha + psum;
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * q16 + i, 64);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o_acc[dt][i] *= al[i];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const half8_t vb = lds_read_b_tr16(vs + dt * 16, ATT_VSTRIDE, q16, c16);
      o_acc[dt] = mfma16x16x32(pa, vb, o_acc[dt]);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// The Q fragments of a wave's 16 query rows (row c16 of the lane; rows past the block's n
// tokens replicate its last one).
__device__ __forceinline__ void prefill_load_q(const PrefillArgs& a, int t0, int row, int h,
                                               half8_t (&qf)[4]) {
  const int q16 = (threadIdx.x & 63) >> 4;
  const half_t* qp = a.q + (int64_t)(t0 + row) * a.q_stride + (int64_t)h * ATT_HD;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) qf[ks] = *(const half8_t*)(qp + ks * 32 + q16 * 8);
}

__global__ __launch_bounds__(256, 2) void prefill_attn_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) half_t vs_lds[ATT_WAVES][ATT_BLK * ATT_VSTRIDE];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q16 = lane >> 4;
  const int c16 = lane & 15;
  const int item = blockIdx.x * ATT_WAVES + wave;
  if (item >= a.nqb * a.nh) return;   // no workgroup barriers below
  const int qb = item / a.nh;
  const int h = item % a.nh;
  const int g = h / a.G;
  const int t0 = a.qblocks[2 * qb];
  const int n = a.qblocks[2 * qb + 1];
  const int64_t slot = a.slots[t0];
  if (slot < 0 || slot >= a.pool_rows || n <= 0) return;

  const int my_row = c16 < n ? c16 : n - 1;
  const int lim = (int)clamp64(a.kv_len[t0 + my_row], 1, a.max_len);   // keys row c16 sees
  const int end = (int)clamp64(a.kv_len[t0 + n - 1], 1, a.max_len);     // the block's keys

  half8_t qf[4];
  prefill_load_q(a, t0, my_row, h, qf);
  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x4 o_acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o_acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
  prefill_wave_tiles(a, slot, g, end, lim, 0, ceil_div(end, ATT_BLK), qf, vs_lds[wave], m_run,
                     l_run, o_acc);

  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  float li[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) li[i] = __shfl(l_run, 4 * q16 + i, 64);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * q16 + i;
    if (r < n) {
      half_t* op = a.out + (int64_t)(t0 + r) * a.out_stride + (int64_t)h * ATT_HD;
      const float inv = 1.0f / li[i];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) op[dt * 16 + c16] = (half_t)(o_acc[dt][i] * inv);
    }
  }
}

// The same attention with each (query block, head) item spread over the four waves of one
// workgroup: wave w takes the w-th quarter of the item's key tiles (prefill_wave_tiles) and
// the four softmax states are merged through LDS, each wave's sums and outputs scaled by
// 2^(m_w - max_w m_w) and added in wave order.  For prompts of a few hundred tokens, where
// one wave per item leaves most CUs idle and walks the longest block's tiles one after
// another.  The scores are prefill_attn_kernel's; P is rounded to fp16 against a wave's own
// running max, so the outputs agree with it to fp16 rounding, not bit for bit.
__global__ __launch_bounds__(256, 2) void prefill_attn_split_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) half_t vs_lds[ATT_WAVES][ATT_BLK * ATT_VSTRIDE];
  // row stride ATT_HD + 4 floats: the 16-lane column runs of rows 4 apart fall on
  // different banks (row r at bank offset 16 r mod 64)
  __shared__ __attribute__((aligned(16))) float o_lds[ATT_WAVES][16][ATT_HD + 4];
  __shared__ float m_lds[ATT_WAVES][16], l_lds[ATT_WAVES][16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q16 = lane >> 4;
  const int c16 = lane & 15;
  // the query heads of one KV head in one XCD's range: they read the same K/V rows
  const int item = xcd_logical_block(blockIdx.x, gridDim.x);
  const int qb = item / a.nh;
  const int h = item % a.nh;
  const int g = h / a.G;
  const int t0 = a.qblocks[2 * qb];
  const int n = a.qblocks[2 * qb + 1];
  const int64_t slot = a.slots[t0];
  if (slot < 0 || slot >= a.pool_rows || n <= 0) return;   // the whole workgroup

  const int my_row = c16 < n ? c16 : n - 1;
  const int lim = (int)clamp64(a.kv_len[t0 + my_row], 1, a.max_len);
  const int end = (int)clamp64(a.kv_len[t0 + n - 1], 1, a.max_len);
  const int ntiles = ceil_div(end, ATT_BLK);
  // the waves' ranges partition [0, ntiles): the one holding tile 0 (key 0, visible to
  // every row) gives every row a finite maximum
  const int tlo = wave * ntiles / ATT_WAVES;
  const int thi = (wave + 1) * ntiles / ATT_WAVES;

  half8_t qf[4];
  prefill_load_q(a, t0, my_row, h, qf);
  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x4 o_acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o_acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
  prefill_wave_tiles(a, slot, g, end, lim, tlo, thi, qf, vs_lds[wave], m_run, l_run, o_acc);

  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (q16 == 0) {
    m_lds[wave][c16] = m_run;
    l_lds[wave][c16] = l_run;
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) o_lds[wave][4 * q16 + i][dt * 16 + c16] = o_acc[dt][i];
  __syncthreads();

  // wave w writes columns 32 w .. 32 w + 31 of the 16 rows: lane -> row lane / 4, 8 columns
  const int r = lane >> 2;
  const int col = 32 * wave + 8 * (lane & 3);
  if (r >= n) return;
  float mx = m_lds[0][r];
#pragma unroll
  for (int w = 1; w < ATT_WAVES; ++w) mx = fmaxf(mx, m_lds[w][r]);
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float l = 0.f;
#pragma unroll
  for (int w = 0; w < ATT_WAVES; ++w) {
    const float sw = exp2f(m_lds[w][r] - mx);   // 0 for a wave that saw none of the row's keys
    l += l_lds[w][r] * sw;
    const float4 lo = *(const float4*)&o_lds[w][r][col];
    const float4 hi = *(const float4*)&o_lds[w][r][col + 4];
    o[0] += lo.x * sw;
    o[1] += lo.y * sw;
    o[2] += lo.z * sw;
    o[3] += lo.w * sw;
    o[4] += hi.x * sw;
    o[5] += hi.y * sw;
    o[6] += hi.z * sw;
    o[7] += hi.w * sw;
  }
  const float inv = 1.0f / l;
  half8_t ov;
#pragma unroll
  for (int e = 0; e < 8; ++e) ov[e] = (half_t)(o[e] * inv);
  *(half8_t*)(a.out + (int64_t)(t0 + r) * a.out_stride + (int64_t)h * ATT_HD + col) = ov;
}

// The same attention for long segments: one workgroup (4 waves) per (block of up to 32
// query tokens of one segment, KV head).  The block's keys go global -> registers -> LDS
// one 32-key tile at a time (the next two tiles' loads in flight during the current tile's
// MFMAs), and every wave reads them from LDS for its 16 query rows (wave & 1) and half of
// the group's query heads (wave >> 1): each K/V byte crosses the L2 once per 32 queries and
// G heads instead of once per 16 queries and head.  Per (query, head) the arithmetic is
// prefill_attn_kernel's, tile for tile (a tile past a row's last key adds exactly nothing),
// so the two kernels agree bit for bit.  K tiles are stored with their 16-byte chunks
// XOR-swizzled by row (the A-operand reads of 16 rows then spread over the banks); V tiles
// as the decode kernel stages them, for the transposed B-operand reads.
// HALVES = 2: the block's key tiles are split between two groups of 4 waves (tiles
// [0, ceil(n/2)) and the rest), each with its own LDS tiles, so the longest blocks' tile
// loop is half as long and two waves share each SIMD; the second group hands its
// normalised output (fp16) and softmax state through LDS to the first, which merges.
// Tile 0 (key 0, visible to every row) is always in the first group.
template <int HPW, int HALVES>
__global__ __launch_bounds__(256 * HALVES, 1) void prefill_attn_gqa_kernel(PrefillArgs a) {
  constexpr int KS_BYTES = HALVES * 2 * ATT_BLK * ATT_HD * 2;
  constexpr int VS_BYTES = HALVES * 2 * ATT_BLK * ATT_VSTRIDE * 2;
  __shared__ __attribute__((aligned(16))) char smem[KS_BYTES + VS_BYTES];
  half_t (*ks_lds)[2][ATT_BLK * ATT_HD] = (half_t (*)[2][ATT_BLK * ATT_HD])smem;
  half_t (*vs_lds)[2][ATT_BLK * ATT_VSTRIDE] = (half_t (*)[2][ATT_BLK * ATT_VSTRIDE])(smem + KS_BYTES);
  const int tid = threadIdx.x;
  const int hf = HALVES > 1 ? tid >> 8 : 0;     // key-range group
  const int ltid = tid & 255;                    // thread within the group
  const int lane = tid & 63;
  const int wave = ltid >> 6;                    // wave within the group
  const int q16 = lane >> 4;
  const int c16 = lane & 15;
  // longest blocks first: a segment's later blocks see more keys
  const int item = (int)gridDim.x - 1 - (int)blockIdx.x;
  const int qb = item / a.nkv;
  const int g = item - qb * a.nkv;
  const int t0 = a.qblocks[2 * qb];
  const int n = a.qblocks[2 * qb + 1];
  const int64_t slot = a.slots[t0];
  if (slot < 0 || slot >= a.pool_rows || n <= 0) return;   // the whole workgroup
  const int sub = wave & 1;                     // query rows 16 sub .. +15 of the block
  const int h0 = (wave >> 1) * HPW;             // first of this wave's heads in the group
  const bool rows_here = 16 * sub < n;
  const int my_row = min(16 * sub + c16, n - 1);
  const int lim = (int)clamp64(a.kv_len[t0 + my_row], 1, a.max_len);
  const int end = (int)clamp64(a.kv_len[t0 + n - 1], 1, a.max_len);
  const int ntiles = (end + ATT_BLK - 1) / ATT_BLK;
  // this group's tiles [tbeg, tbeg + nt); both groups run `steps` loop steps (the same
  // barriers), computing only their own tiles
  const int steps = HALVES > 1 ? (ntiles + 1) / 2 : ntiles;
  const int tbeg = hf == 0 ? 0 : steps;
  const int nt = hf == 0 ? steps : ntiles - steps;

  half8_t qf[HPW][4];
#pragma unroll
  for (int u = 0; u < HPW; ++u) {
    const int h = g * a.G + min(h0 + u, a.G - 1);
    const half_t* qp = a.q + (int64_t)(t0 + my_row) * a.q_stride + (int64_t)h * ATT_HD;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[u][ks] = *(const half8_t*)(qp + ks * 32 + q16 * 8);
  }
  float m_run[HPW], l_run[HPW];
  f32x4 o_acc[HPW][8];
#pragma unroll
  for (int u = 0; u < HPW; ++u) {
    m_run[u] = -INFINITY;
    l_run[u] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o_acc[u][i] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }

  const int64_t row_base = slot * (int64_t)a.max_len;
  const int64_t tok_stride = (int64_t)a.nkv * ATT_HD;
  const half_t* kbase = a.k_cache + g * ATT_HD;
  const half_t* vbase = a.v_cache + g * ATT_HD;
  // thread ltid moves 16-byte chunks c = ltid and ltid + 256 of the tile's K and of its V:
  // row c / 16, chunk c % 16.  Two register sets hold the next two tiles' loads.
  struct TileRegs {
    half8_t k[2], v[2];
  };
  auto load_tile = [&](int tb, TileRegs& t) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = ltid + 256 * u;
      const int tok = min(tb + (c >> 4), end - 1);
      const int64_t off = (row_base + tok) * tok_stride + (c & 15) * 8;
      t.k[u] = *(const half8_t*)(kbase + off);
      t.v[u] = *(const half8_t*)(vbase + off);
    }
  };
  auto store_tile = [&](int buf, const TileRegs& t) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = ltid + 256 * u;
      const int r = c >> 4, ch = c & 15;
      *(half8_t*)(&ks_lds[hf][buf][r * ATT_HD + ((ch ^ (r & 15)) << 3)]) = t.k[u];
      *(half8_t*)(&vs_lds[hf][buf][r * ATT_VSTRIDE + ch * 8]) = t.v[u];
    }
  };
  // One head's scores (S^T, keys along the lane quads) turned into fp16 probabilities
  // (pa) and the factors that rescale its running output rows (al), with m_run / l_run
  // updated.
  auto softmax_tile = [&](int u, int tb, const f32x4 (&sacc)[2], half8_t& pa, float (&al)[4]) {
    float sc[8];
    float mblk = -INFINITY;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = tb + 16 * j + 4 * q16 + i;
        const float sv = key < lim ? sacc[j][i] * a.scale_log2 : -INFINITY;
        sc[4 * j + i] = sv;
        mblk = fmaxf(mblk, sv);
      }
    mblk = fmaxf(mblk, __shfl_xor(mblk, 16, 64));
    mblk = fmaxf(mblk, __shfl_xor(mblk, 32, 64));
    const float m_new = fmaxf(m_run[u], mblk);
    // -inf only in the second key group, for a row none of whose keys it has seen yet
    // (exp2(-inf - -inf) would be NaN); the first group starts at key 0
    const float m_ref = HALVES > 1 && m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run[u] - m_ref);
    m_run[u] = m_new;
    float psum = 0.f;
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      const float p = exp2f(sc[s8] - m_ref);
      psum += p;
      pa[s8] = (half_t)p;
    }
    l_run[u] = l_run[u] * alpha + psum;
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * q16 + i, 64);
  };
  auto compute_tile = [&](int buf, int tb) {
    if (!rows_here) return;
    if constexpr (HALVES > 1) {
      // Two waves share each SIMD here, so registers are tighter: every head's scores are
      // formed one 16-key chunk of K fragments at a time, then V is read one 16-column
      // strip at a time (the same arithmetic per element as below, in another order).
      f32x4 sacc[HPW][2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        half8_t kc[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          kc[ks] = *(const half8_t*)(&ks_lds[hf][buf][(16 * j + c16) * ATT_HD + (((4 * ks + q16) ^ c16) << 3)]);
#pragma unroll
        for (int u = 0; u < HPW; ++u) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(kc[ks], qf[u][ks], acc);
          sacc[u][j] = acc;
        }
      }
      half8_t pa[HPW];
      float al[HPW][4];
#pragma unroll
      for (int u = 0; u < HPW; ++u)
        if (h0 + u < a.G) softmax_tile(u, tb, sacc[u], pa[u], al[u]);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const half8_t vb = lds_read_b_tr16(&vs_lds[hf][buf][dt * 16], ATT_VSTRIDE, q16, c16);
#pragma unroll
        for (int u = 0; u < HPW; ++u) {
          if (h0 + u >= a.G) continue;
#pragma unroll
          for (int i = 0; i < 4; ++i) o_acc[u][dt][i] *= al[u][i];
          o_acc[u][dt] = mfma16x16x32(pa[u], vb, o_acc[u][dt]);
        }
      }
      return;
    }
    {
      // K fragments (A operand of S^T = K Q^T): key 16 j + c16, dims 32 ks + 8 q16 .. +7
      half8_t kc[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          kc[j][ks] = *(const half8_t*)(&ks_lds[hf][buf][(16 * j + c16) * ATT_HD + (((4 * ks + q16) ^ c16) << 3)]);
      half8_t vb[8];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) vb[dt] = lds_read_b_tr16(&vs_lds[hf][buf][dt * 16], ATT_VSTRIDE, q16, c16);
#pragma unroll
      for (int u = 0; u < HPW; ++u) {
        if (h0 + u >= a.G) continue;
        f32x4 sacc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(kc[j][ks], qf[u][ks], acc);
          sacc[j] = acc;
        }
        half8_t pa;
        float al[4];
        softmax_tile(u, tb, sacc, pa, al);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) o_acc[u][dt][i] *= al[i];
          o_acc[u][dt] = mfma16x16x32(pa, vb[dt], o_acc[u][dt]);
        }
      }
    }
  };

  // Tile i of the group sits in LDS buffer i % 2 while it is computed; during step i the
  // registers hold tiles i + 1 (landed by now, stored into the other buffer after the
  // step's MFMAs) and i + 2 (in flight), and the freed set takes tile i + 3's loads.  Steps
  // go in pairs so that the two register sets keep fixed roles.
  TileRegs ra, rb;
  if (nt > 0) {
    load_tile(tbeg * ATT_BLK, ra);
    store_tile(0, ra);
  }
  __syncthreads();
  if (nt > 1) load_tile((tbeg + 1) * ATT_BLK, rb);
  if (nt > 2) load_tile((tbeg + 2) * ATT_BLK, ra);
  for (int it = 0; it < steps; it += 2) {
    if (it < nt) compute_tile(0, (tbeg + it) * ATT_BLK);
    if (it + 1 < nt) {
      store_tile(1, rb);                      // tile it + 1; buffer 1's last reader is done
      if (it + 3 < nt) load_tile((tbeg + it + 3) * ATT_BLK, rb);
    }
    lds_barrier();   // the stores are visible and every wave is done with this tile
    if (it + 1 >= steps) break;
    if (it + 1 < nt) compute_tile(1, (tbeg + it + 1) * ATT_BLK);
    if (it + 2 < nt) {
      store_tile(0, ra);                      // tile it + 2
      if (it + 4 < nt) load_tile((tbeg + it + 4) * ATT_BLK, ra);
    }
    lds_barrier();
  }

  // The row sums (each lane holds keys 4 q16 .. +3 of every 16) reduced to row c16.
  float lrow[HPW];
#pragma unroll
  for (int u = 0; u < HPW; ++u) {
    float l = l_run[u];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    lrow[u] = l;
  }
  // HALVES = 2: the second group's normalised output (fp16) and (max, sum) per row go
  // through LDS (the tile buffers, free after the loop) to the first group's same wave.
  float w1[HPW][4];      // second group's weight l1 2^(m1 - M) per output row (0: none)
  float wd[HPW][4];      // the merged denominator per output row
  float w0[HPW][4];      // first group's 2^(m0 - M)
  half_t (*o1)[HPW][8][64][4] = (half_t (*)[HPW][8][64][4])smem;
  float (*ml1)[HPW][16][2] = (float (*)[HPW][16][2])(smem + 4 * HPW * 8 * 64 * 4 * 2);
  if constexpr (HALVES > 1) {
    static_assert(4 * HPW * 8 * 64 * 4 * 2 + 4 * HPW * 16 * 2 * 4 <= KS_BYTES + VS_BYTES,
                  "merge buffers exceed the tile buffers");
    __syncthreads();                           // every tile read is done: the LDS is free
    if (hf == 1 && rows_here) {
#pragma unroll
      for (int u = 0; u < HPW; ++u) {
        float li[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) li[i] = __shfl(lrow[u], 4 * q16 + i, 64);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          half4_t hv;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            hv[i] = (half_t)(li[i] > 0.f ? o_acc[u][dt][i] / li[i] : 0.f);
          *(half4_t*)&o1[wave][u][dt][lane][0] = hv;
        }
        if (q16 == 0) {
          ml1[wave][u][c16][0] = m_run[u];
          ml1[wave][u][c16][1] = lrow[u];
        }
      }
    }
    __syncthreads();
    if (hf == 1) return;                       // no barrier follows
#pragma unroll
    for (int u = 0; u < HPW; ++u) {
      const float m1 = ml1[wave][u][c16][0], l1 = ml1[wave][u][c16][1];
      const float M = fmaxf(m_run[u], m1);     // finite: key 0 is in the first group
      const float a0 = exp2f(m_run[u] - M);
      const float b1 = l1 > 0.f ? l1 * exp2f(m1 - M) : 0.f;
      const float den = lrow[u] * a0 + b1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w0[u][i] = __shfl(a0, 4 * q16 + i, 64);
        w1[u][i] = __shfl(b1, 4 * q16 + i, 64);
        wd[u][i] = __shfl(den, 4 * q16 + i, 64);
      }
    }
  }
  if (!rows_here) return;
#pragma unroll
  for (int u = 0; u < HPW; ++u) {
    if (h0 + u >= a.G) continue;
    const int h = g * a.G + h0 + u;
    float li[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) li[i] = __shfl(lrow[u], 4 * q16 + i, 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * sub + 4 * q16 + i;
      if (r < n) {
        half_t* op = a.out + (int64_t)(t0 + r) * a.out_stride + (int64_t)h * ATT_HD;
        if constexpr (HALVES > 1) {
          const float inv = 1.0f / wd[u][i];
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) {
            const float o1v = (float)o1[wave][u][dt][lane][i];
            op[dt * 16 + c16] = (half_t)((o_acc[u][dt][i] * w0[u][i] + o1v * w1[u][i]) * inv);
          }
        } else {
          const float inv = 1.0f / li[i];
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) op[dt * 16 + c16] = (half_t)(o_acc[u][dt][i] * inv);
        }
      }
    }
  }
}

// The arguments the prefill entry points share, checked: q [T, q_stride] fp16 (heads of
// head_dim = 128), pool K/V [pool_rows, max_len, n_kv_heads, 128] fp16, qblocks int32
// [nqb][2] = (first token, count), out fp16 rows of out_stride elements.
static int prefill_args(PrefillArgs& a, const void* q, int q_stride, const void* k_cache,
                        const void* v_cache, int pool_rows, int max_len, const int64_t* slots,
                        const int64_t* kv_len, const int* qblocks, int nqb, void* out,
                        int out_stride, int n_heads, int n_kv_heads, int head_dim, float scale) {
  if (nqb < 0 || n_heads <= 0 || n_kv_heads <= 0 || pool_rows <= 0 || max_len <= 0) return OMNI_EINVAL;
  if (head_dim != ATT_HD || n_heads % n_kv_heads) return OMNI_EUNSUPPORTED;
  if (q_stride < n_heads * ATT_HD || (q_stride & 7) || out_stride < n_heads * ATT_HD) return OMNI_EINVAL;
  if (nqb > 0 && (!q || !k_cache || !v_cache || !slots || !kv_len || !qblocks || !out))
    return OMNI_EINVAL;
  a.q = (const half_t*)q;
  a.q_stride = q_stride;
  a.k_cache = (const half_t*)k_cache;
  a.v_cache = (const half_t*)v_cache;
  a.pool_rows = pool_rows;
  a.max_len = max_len;
  a.nkv = n_kv_heads;
  a.G = n_heads / n_kv_heads;
  a.nh = n_heads;
  a.slots = slots;
  a.kv_len = kv_len;
  a.qblocks = qblocks;
  a.nqb = nqb;
  a.out = (half_t*)out;
  a.out_stride = out_stride;
  a.scale_log2 = scale * 1.4426950408889634f;
  return OMNI_OK;
}

// Causal varlen attention for packed query tokens over the pool.
//   qblocks int32 [nqb][2]: (first token, count <= 16); the tokens of a block share
//   slots[t] and have increasing kv_len.  out fp16 rows of out_stride elements.
extern "C" int omni_prefill_attention(const void* q, int q_stride, const void* k_cache,
                                      const void* v_cache, int pool_rows, int max_len,
                                      const int64_t* slots, const int64_t* kv_len,
                                      const int* qblocks, int nqb, void* out, int out_stride,
                                      int n_heads, int n_kv_heads, int head_dim, float scale,
                                      void* stream) {
  PrefillArgs a;
  const int rc = prefill_args(a, q, q_stride, k_cache, v_cache, pool_rows, max_len, slots, kv_len,
                              qblocks, nqb, out, out_stride, n_heads, n_kv_heads, head_dim, scale);
  if (rc || nqb == 0) return rc;
  const int64_t items = (int64_t)nqb * n_heads;
  const int64_t grid = (items + ATT_WAVES - 1) / ATT_WAVES;
  if (grid > 0x7fffffff) return OMNI_EUNSUPPORTED;
  hipLaunchKernelGGL(prefill_attn_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// The same attention (qblocks as above, count <= 16) with each (block, head) item's keys
// split over the four waves of a workgroup and the partial softmax states merged in LDS
// (prefill_attn_split_kernel): for few items with many keys each.  Agrees with
// omni_prefill_attention to the fp16 rounding of the probabilities.
extern "C" int omni_prefill_attention_split(const void* q, int q_stride, const void* k_cache,
                                            const void* v_cache, int pool_rows, int max_len,
                                            const int64_t* slots, const int64_t* kv_len,
                                            const int* qblocks, int nqb, void* out,
                                            int out_stride, int n_heads, int n_kv_heads,
                                            int head_dim, float scale, void* stream) {
  PrefillArgs a;
  const int rc = prefill_args(a, q, q_stride, k_cache, v_cache, pool_rows, max_len, slots, kv_len,
                              qblocks, nqb, out, out_stride, n_heads, n_kv_heads, head_dim, scale);
  if (rc || nqb == 0) return rc;
  const int64_t grid = (int64_t)nqb * n_heads;
  if (grid > 0x7fffffff) return OMNI_EUNSUPPORTED;
  hipLaunchKernelGGL(prefill_attn_split_kernel, dim3((unsigned)grid), dim3(256), 0,
                     (hipStream_t)stream, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// The same attention with query blocks of up to 32 tokens (qblocks as above, count <= 32),
// one workgroup per (block, KV head) sharing each K/V tile among the group's query heads
// (prefill_attn_gqa_kernel; at most 8 query heads per KV head).  Outputs equal
// omni_prefill_attention's bit for bit.
extern "C" int omni_prefill_attention_gqa(const void* q, int q_stride, const void* k_cache,
                                          const void* v_cache, int pool_rows, int max_len,
                                          const int64_t* slots, const int64_t* kv_len,
                                          const int* qblocks, int nqb, void* out, int out_stride,
                                          int n_heads, int n_kv_heads, int head_dim, float scale,
                                          void* stream) {
  PrefillArgs a;
  const int rc = prefill_args(a, q, q_stride, k_cache, v_cache, pool_rows, max_len, slots, kv_len,
                              qblocks, nqb, out, out_stride, n_heads, n_kv_heads, head_dim, scale);
  if (rc) return rc;
  if (a.G > 8) return OMNI_EUNSUPPORTED;
  if (nqb == 0) return OMNI_OK;
  const int64_t grid = (int64_t)nqb * n_kv_heads;
  if (grid > 0x7fffffff) return OMNI_EUNSUPPORTED;
  if (a.G <= 6)
    hipLaunchKernelGGL((prefill_attn_gqa_kernel<3, 1>), dim3((unsigned)grid), dim3(256), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((prefill_attn_gqa_kernel<4, 1>), dim3((unsigned)grid), dim3(256), 0,
                       (hipStream_t)stream, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_prefill_attention_gqa_halves(const void* q, int q_stride, const void* k_cache,
                                                 const void* v_cache, int pool_rows, int max_len,
                                                 const int64_t* slots, const int64_t* kv_len,
                                                 const int* qblocks, int nqb, void* out,
                                                 int out_stride, int n_heads, int n_kv_heads,
                                                 int head_dim, float scale, void* stream) {
  PrefillArgs a;
  const int rc = prefill_args(a, q, q_stride, k_cache, v_cache, pool_rows, max_len, slots, kv_len,
                              qblocks, nqb, out, out_stride, n_heads, n_kv_heads, head_dim, scale);
  if (rc) return rc;
  if (a.G > 6) return OMNI_EUNSUPPORTED;
  if (nqb == 0) return OMNI_OK;
  const int64_t grid = (int64_t)nqb * n_kv_heads;
  if (grid > 0x7fffffff) return OMNI_EUNSUPPORTED;
  hipLaunchKernelGGL((prefill_attn_gqa_kernel<3, 2>), dim3((unsigned)grid), dim3(512), 0,
                     (hipStream_t)stream, a);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

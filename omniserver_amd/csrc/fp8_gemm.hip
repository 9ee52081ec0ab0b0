// FP8 (e4m3fn) W8A8 GEMM with row-wise scales on the CDNA4 fp8 matrix cores.
//
// Replaces FP8Linear (omniserve/kernels/fp8_linear.py:66-126) and its activation
// quantiser (:45-63):
//   weights   sw[n] = amax_k |W[n, :]| / 448,  Wq = e4m3(W / sw)          (:83-86)
//   inputs    sa[m] = amax_k |x[m, :]| / 448,  xq = e4m3(x / sa)          (:45-63)
//   product   y[m, n] = bf16((sum_k xq[m,k] * Wq[n,k]) * sa[m] * sw[n])    (:115-118,
//             torch._scaled_mm with fp32 accumulation and a bf16 result), then cast to
//             fp16 by FP8Linear.forward (two roundings), plus bias in fp16.
// and FP8Linear's default per-tensor form (:87-90, 119-125): one weight scale and one
// activation scale (both fp16-rounded: ops on fp16 tensors), the product written as fp16
// directly (_scaled_mm out_dtype fp16), bias added in fp16.  The GEMM takes the scales as
// the same [M] / [N] arrays, filled with the one value.
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

#include <string.h>

#define F8_BT 128          // tile rows (m) and columns (n) per workgroup
#define F8_BK 128          // K per step (one MFMA)
#define F8_STRIDE 144      // LDS bytes per staged row

typedef int i32x8 __attribute__((ext_vector_type(8)));

typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
typedef float f32x2_hw __attribute__((ext_vector_type(2)));

// The integer form of bf16 rounding: round to nearest even, NaNs quieted (sign and upper
// payload kept).
__device__ __forceinline__ uint32_t bf16_bits_int(uint32_t u) {
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) | 0x0040u) : r;
}

// bf16 bits of (a, b), a in the low half: gfx950's v_cvt_pk_bf16_f32, one instruction per
// pair, equal to bf16_bits_int on every one of the 2^32 float inputs
// (omni_bf16_rne_check).
__device__ __forceinline__ uint32_t bf16x2_bits(float a, float b) {
  const f32x2_hw v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_hw));
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return (uint16_t)(bf16x2_bits(f, 0.f) & 0xffffu);
}

// The bf16 value nearest f (RNE, NaN kept quiet), as a float.
__device__ __forceinline__ float bf16_value(float f) {
  return __builtin_bit_cast(float, bf16x2_bits(f, 0.f) << 16);
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
  int out_mode;          // FP8_OUT_*: how the scaled product is stored (+ bias)
  int n_big;             // persistent 256-column tiles: whole tiles below column n_big, 192-column
                         // tiles from there to N; N elsewhere
};

// Output forms of the scaled product v = acc * sa[m] * sw[n]:
enum {
  FP8_OUT_F16_VIA_BF16 = 0,   // fp16(bf16(v)) + fp16 bias (row-wise forward, :115-118)
  FP8_OUT_BF16 = 1,           // bf16(v) + bf16(bias) as a bf16 add (forward_prequant)
  FP8_OUT_F16 = 2,            // fp16(v) + fp16 bias (per-tensor forward, :122-125)
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
        const float v = (acc[i][j][r] * sm) * sv[r];
        const uint16_t b = f32_to_bf16_rne(v);
        if (a.out_mode == FP8_OUT_BF16) {
          // forward_prequant's bias: out + bias.to(bf16), a bf16 add
          bits[r] = a.bias ? f32_to_bf16_rne(__builtin_bit_cast(float, (uint32_t)b << 16) +
                                             bf16_value((float)a.bias[n + r]))
                           : b;
        } else {
          half_t h = a.out_mode == FP8_OUT_F16 ? (half_t)v
                                               : (half_t)__builtin_bit_cast(float, (uint32_t)b << 16);
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

// Pipelined, persistent form of the same GEMM (the default for K >= 4 steps).  A grid of at most one
// workgroup per CU walks its tiles round by round (round r, slot b: logical tile r * grid
// + b, slots XCD-grouped as above, logical tiles in grouped order so the 32 tiles an XCD
// holds at once form a 4 x 8 block), and the K loop runs straight across tile boundaries,
// so the next tile's first operand tiles are in flight while the current one finishes
// and writes its outputs.
// Operand tiles go global -> LDS directly (global_load_lds_dwordx4: lane i of a load
// writes bytes 16 i .. 16 i + 15 past the instruction's LDS base), NS stages deep.
// WM waves along m, two along n, each wave owning a 64 x 64 block of the 64 WM x 128 tile.  LDS rows are
// 128 bytes (one K step of one row); 16-byte chunk c of row r is stored in slot
// c ^ (r & 7), so the 16 rows an operand read touches spread over the banks.  A stage is
// waited for with vmcnt (each thread's own loads: every stage issues at least OPS per
// thread, the operands and, on most waves, a share of the tile's row / column scales or
// the biases, so waiting for all but OPS loads per younger stage covers a stage) plus a
// barrier (everyone's).  A step's operands are read into registers before that
// barrier, so its slot is refilled right after it, while the step's MFMAs run.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

#define F8_GM 4                        // tile rows per group of the tile order (grouped_tile)
#define F8_ROWB 128                    // LDS bytes per staged row
#define F8_TILEB (F8_BT * F8_ROWB)     // one operand tile of one stage

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// bf16 bits of f, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return bf16x2_bits(f, 0.f) & 0xffffu; }

// One tile's load sources: per-lane x row pointers (rows clamped below M) for the four
// row groups, the w row pointer of group 0 (groups u are 32 u rows further), the lane's
// scale pointer and (wave 0) bias pointer.
struct F8TileSrc {
  const uint8_t* x[4];
  const uint8_t* w;
  const void* s;
  const void* b;
};

template <int WM, int NS>
__global__ __launch_bounds__(128 * WM, 1) void fp8_gemm_pipe_kernel(Fp8GemmArgs a) {
#pragma clang fp contract(off)
  constexpr int BM = 64 * WM;                 // tile rows (tokens); 128 columns (channels)
  constexpr int NWV = 2 * WM;                 // waves
  constexpr int XLD = 4;                      // x loads per wave and stage
  constexpr int WLD = 8 / WM;                 // w loads per wave and stage
  constexpr int SCW = WM + 2;                 // waves loading scales (BM + 128 of them)
  // fewest loads any thread issues per stage (the vmcnt unit of one stage)
  constexpr int OPS = XLD + WLD + (SCW >= NWV ? 1 : 0);
  __shared__ __attribute__((aligned(1024))) uint8_t xl[NS][BM * F8_ROWB];      // [stage] x tile
  __shared__ __attribute__((aligned(1024))) uint8_t wl[NS][F8_BT * F8_ROWB];   // [stage] w tile
  __shared__ __attribute__((aligned(16))) float scl[NS][BM + F8_BT];           // [stage][sa|sw]
  __shared__ __attribute__((aligned(16))) half_t bsl[NS][512];                 // [stage][bias]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1;
  const int wm = wave >> 1;
  const int l16 = lane & 15;
  const int g4 = lane >> 4;

  const int tiles_n = a.N / F8_BT;
  const int tiles_m = (a.M + BM - 1) / BM;
  const int tiles = tiles_m * tiles_n;
  const int G = gridDim.x;
  const int slot = xcd_logical_block(blockIdx.x, G);
  const int my_tiles = (tiles - slot + G - 1) / G;          // grid <= tiles: >= 1
  const int nk = a.K / F8_BK;                               // >= NS (host check)

  // Load u of this wave fills tile rows 8 NWV u + 8 wave .. +7: lane i -> row
  // 8 NWV u + 8 wave + i/8, LDS slot i%8, which holds chunk (i%8) ^ (row & 7).  One more
  // 4-byte-per-lane load brings 64 of the tile's scales: waves 0 .. WM-1 the token scales
  // sa[m0 + 64 wave + lane], waves WM, WM+1 the channel scales sw[n0 + 64 (wave - WM) + lane].
  const int lrow = 8 * wave + (lane >> 3);          // + 8 NWV u
  const int lchunk = (lane & 7) ^ (lrow & 7);       // (8 NWV u + lrow) & 7 == lrow & 7
  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const bool has_bias = a.bias != nullptr;
  auto tile_src = [&](int r, int& m0, int& n0) {     // past the last tile: the last one again
    int tm, tn;
    grouped_tile(min(r, my_tiles - 1) * G + slot, tiles_m, tiles_n, F8_GM, tm, tn);
    m0 = tm * BM;
    n0 = tn * F8_BT;
    F8TileSrc t;
#pragma unroll
    for (int u = 0; u < XLD; ++u)
      t.x[u] = a.xq + (int64_t)min(m0 + 8 * NWV * u + lrow, a.M - 1) * a.K + lchunk * 16;
    t.w = a.wq + (int64_t)(n0 + lrow) * a.K + lchunk * 16;
    t.s = wave < WM ? (const void*)(a.sa + min(m0 + 64 * wave + lane, a.M - 1))
                    : (const void*)(a.sw + n0 + 64 * min(wave - WM, 1) + lane);
    t.b = has_bias ? (const void*)(a.bias + n0 + 8 * min(lane, 15)) : t.s;
    return t;
  };
  const int64_t wstep = (int64_t)8 * NWV * a.K;    // bytes between w row groups
  auto issue = [&](const F8TileSrc& t, int ks, int st) {
    const int k0 = ks * F8_BK;
#pragma unroll
    for (int u = 0; u < XLD; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(t.x[u] + k0),
                                       (lds_void*)((lds_u8*)&xl[st][(8 * NWV * u + 8 * wave) * F8_ROWB]), 16, 0, 0);
#pragma unroll
    for (int u = 0; u < WLD; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(t.w + u * wstep + k0),
                                       (lds_void*)((lds_u8*)&wl[st][(8 * NWV * u + 8 * wave) * F8_ROWB]), 16, 0, 0);
    if (wave < SCW)
      __builtin_amdgcn_global_load_lds(t.s, (lds_void*)((lds_u8*)&scl[st][64 * wave]), 4, 0, 0);
    if (wave == 0 && has_bias)        // the tile's 128 fp16 biases (lanes 0-15; a sixth load,
      __builtin_amdgcn_global_load_lds(t.b, (lds_void*)((lds_u8*)&bsl[st][0]), 16, 0, 0);   // wave 0 only)
  };
  // LDS reads of the staged tiles are inline asm with their own lgkmcnt wait: written as
  // plain loads, the compiler makes each of them wait for every outstanding
  // global->LDS load (vmcnt(0)), which are the later stages in flight; the stage read is
  // complete by the vmcnt wait and barrier before it.
  // Addresses of the 32 operand bytes (k = 32 g4 .. +31) of tile rows base + 16 i + l16.
  auto operand_addrs = [&](int st, int o, int base, uint32_t (&ad)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = base + 16 * i + l16;
      const uint32_t row = (uint32_t)(uintptr_t)(lds_u8*)(o ? &wl[st][r * F8_ROWB] : &xl[st][r * F8_ROWB]);
      ad[2 * i] = row + (((2 * g4) ^ (r & 7)) << 4);
      ad[2 * i + 1] = row + (((2 * g4 + 1) ^ (r & 7)) << 4);
    }
  };
  // Issue the 16 reads of stage st (w rows of this wave's n half, then x rows of its m
  // half) without waiting for them.
  auto read_issue = [&](int st, u32x4 (&v)[16]) {
    uint32_t aw[8], ax[8];
    operand_addrs(st, 1, 64 * wn, aw);
    operand_addrs(st, 0, 64 * wm, ax);
    asm volatile(
        "ds_read_b128 %0, %16\n\tds_read_b128 %1, %17\n\tds_read_b128 %2, %18\n\t"
        "ds_read_b128 %3, %19\n\tds_read_b128 %4, %20\n\tds_read_b128 %5, %21\n\t"
        "ds_read_b128 %6, %22\n\tds_read_b128 %7, %23\n\tds_read_b128 %8, %24\n\t"
        "ds_read_b128 %9, %25\n\tds_read_b128 %10, %26\n\tds_read_b128 %11, %27\n\t"
        "ds_read_b128 %12, %28\n\tds_read_b128 %13, %29\n\tds_read_b128 %14, %30\n\t"
        "ds_read_b128 %15, %31"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
          "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
          "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
        : "v"(aw[0]), "v"(aw[1]), "v"(aw[2]), "v"(aw[3]), "v"(aw[4]), "v"(aw[5]), "v"(aw[6]),
          "v"(aw[7]), "v"(ax[0]), "v"(ax[1]), "v"(ax[2]), "v"(ax[3]), "v"(ax[4]), "v"(ax[5]),
          "v"(ax[6]), "v"(ax[7])
        : "memory");
  };
  // Wait for reads issued by read_issue; the registers pass through the asm so that no
  // use of them is scheduled before the wait.
  auto read_wait = [&](u32x4 (&v)[16]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]),
                   "+v"(v[12]), "+v"(v[13]), "+v"(v[14]), "+v"(v[15])
                 :
                 : "memory");
  };
  auto frag = [](const u32x4& lo, const u32x4& hi) {
    return (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  };

  // Tile scales and biases of a stage slot into registers (read before the slot is
  // refilled).
  float smv[4];
  f32x4 snv[4];
  u32x2 bv[4] = {};                  // 4 fp16 biases per n sub-tile (2 per word)
  auto read_scales = [&](int st) {
    typedef __attribute__((address_space(3))) float lds_f32;
    typedef __attribute__((address_space(3))) half_t lds_f16;
    uint32_t am[4], an[4], ab[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      am[j] = (uint32_t)(uintptr_t)(lds_f32*)&scl[st][64 * wm + 16 * j + l16];
      an[j] = (uint32_t)(uintptr_t)(lds_f32*)&scl[st][BM + 64 * wn + 16 * j + 4 * g4];
      ab[j] = (uint32_t)(uintptr_t)(lds_f16*)&bsl[st][64 * wn + 16 * j + 4 * g4];
    }
    asm volatile(
        "ds_read_b32 %0, %12\n\tds_read_b32 %1, %13\n\tds_read_b32 %2, %14\n\tds_read_b32 %3, %15\n\t"
        "ds_read_b128 %4, %16\n\tds_read_b128 %5, %17\n\tds_read_b128 %6, %18\n\t"
        "ds_read_b128 %7, %19\n\tds_read_b64 %8, %20\n\tds_read_b64 %9, %21\n\t"
        "ds_read_b64 %10, %22\n\tds_read_b64 %11, %23\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(smv[0]), "=&v"(smv[1]), "=&v"(smv[2]), "=&v"(smv[3]), "=&v"(snv[0]),
          "=&v"(snv[1]), "=&v"(snv[2]), "=&v"(snv[3]), "=&v"(bv[0]), "=&v"(bv[1]), "=&v"(bv[2]),
          "=&v"(bv[3])
        : "v"(am[0]), "v"(am[1]), "v"(am[2]), "v"(am[3]), "v"(an[0]), "v"(an[1]), "v"(an[2]),
          "v"(an[3]), "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3])
        : "memory");
  };

  // Steps sidx = 0, 1, ... walk the tiles' K steps back to back; step s sits in slot
  // s % NS.  NS steps are in flight ahead of the one being read: after step s's operands
  // are in registers and step s + 1 has landed everywhere (vmcnt + barrier), step s + NS
  // is loaded into slot s % NS.
  int m0c, n0c, m0n, n0n;
  F8TileSrc cur = tile_src(0, m0c, n0c);
  F8TileSrc nxt = tile_src(1, m0n, n0n);
#pragma unroll
  for (int s = 0; s < NS; ++s) issue(cur, s, s);
  wait_vmcnt<OPS * (NS - 1)>();
  barrier_only();
  int sidx = 0;
  for (int r = 0; r < my_tiles; ++r) {
    f32x4 acc[4][4];   // [n sub-tile][m sub-tile]
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < nk; ++ks, ++sidx) {
      const int st = sidx % NS;
      // step sidx's slot, landed everywhere (vmcnt + barrier at the end of the last step)
      u32x4 ops[16];
      read_issue(st, ops);
      read_wait(ops);
      if (ks == nk - 1) read_scales(st);
      i32x8 wf[4], xf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wf[i] = frag(ops[2 * i], ops[2 * i + 1]);
        xf[i] = frag(ops[8 + 2 * i], ops[8 + 2 * i + 1]);
      }
      // step sidx + 1 has landed for this thread, then for everyone; every wave has also
      // read step sidx's slot, which is refilled with step sidx + NS
      wait_vmcnt<OPS * (NS - 2)>();
      barrier_only();
      {
        const int iks = ks + NS;
        if (iks < nk) issue(cur, iks, st);
        else issue(nxt, iks - nk, st);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[i], xf[j], acc[i][j], 0, 0,
                                                                        0, 127, 0, 127);
    }
    // Epilogue: lane holds n = n0 + 64wn + 16i + 4g4 + q of m = m0 + 64wm + 16j + l16.
    const int m0 = m0c, n0 = n0c;
    const uint32_t bias_mask = has_bias ? 0xffffffffu : 0u;
    const bool direct = a.out_mode == FP8_OUT_F16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + 64 * wm + 16 * j + l16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = n0 + 64 * wn + 16 * i + 4 * g4;
        uint32_t bits[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float v = (acc[i][j][q] * smv[j]) * snv[i][q];
          const uint32_t b = f32_to_bf16_bits(v);
          // fp16 output: the product (FP8_OUT_F16) or its bf16 value rounded to fp16, plus
          // the bias (an fp16 add)
          const half_t hb = (half_t)(direct ? v : __builtin_bit_cast(float, b << 16));
          const uint32_t bw = bv[i][q >> 1] & bias_mask;
          const half_t bb = __builtin_bit_cast(half_t, (uint16_t)((q & 1) ? (bw >> 16) : (bw & 0xffffu)));
          const half_t h = has_bias ? (half_t)((float)hb + (float)bb) : hb;
          // bf16 output (forward_prequant): + bias.to(bf16) as a bf16 add
          const uint32_t bo =
              has_bias ? f32_to_bf16_bits(__builtin_bit_cast(float, b << 16) + bf16_value((float)bb))
                       : b;
          bits[q] = a.out_mode == FP8_OUT_BF16 ? bo : (uint32_t)__builtin_bit_cast(uint16_t, h);
        }
        if (m < a.M) {
          uint2 pk;
          pk.x = bits[0] | (bits[1] << 16);
          pk.y = bits[2] | (bits[3] << 16);
          *(uint2*)((uint16_t*)a.out + (int64_t)m * a.ldo + n) = pk;
        }
      }
    }
    // the next tile becomes current; its successor's sources are computed now
    cur = nxt;
    m0c = m0n;
    n0c = n0n;
    nxt = tile_src(r + 2, m0n, n0n);
  }
  wait_vmcnt<0>();                     // drain the clamped tail loads before exit
}

// Large-tile form: 256 x 256 output tiles, 8 waves (two per SIMD: 2 along m x 4 along n)
// each owning a 128 (m) x 64 (n) block, so every operand byte staged through LDS feeds twice
// the MFMA work it feeds in the 256 x 128 tiles above (those re-read their operand rows from
// L2 for every 128 columns; this one for every 256).  Per K step a wave issues 24 operand
// reads (32 bytes per lane of 4 w and 8 x row groups) and 32 MFMAs; two stages of 64 KB each
// are in LDS (the next step's operands land while this step's MFMAs run), and the second
// wave on each SIMD keeps its matrix core busy while the first waits (on MI355X 6-11 %
// faster than four waves of 128 x 128, outputs bit-equal).  Same staging (direct
// global->LDS loads, XOR-swizzled 128-byte rows) and XCD-grouped tile order as the kernel
// above.  NI = 6 narrows the tile to 256 x 192 (each wave 128 x 48): N = 1536 then makes 8
// column tiles, so M = 8192 gives 256 tiles, one per CU, where the 256-column tiles leave a
// quarter of the CUs idle.
#define F8B_T 256

// Output bits of one product value v = acc * sa * sw: bf16(v), then either that bf16 plus
// bf16(bias) as a bf16 add (FP8_OUT_BF16: forward_prequant, out + bias.to(bf16)) or the
// bf16 rounded to fp16 plus the fp16 bias as an fp16 add (FP8_OUT_F16_VIA_BF16: the
// row-wise forward).  A zero bias is the identity in both (x + 0 rounds to x).  The
// per-tensor form (FP8_OUT_F16) does not run here (omni_fp8_gemm sends it to the 256 x 128
// kernel, which has all three forms).
template <bool OUT_BF16>
__device__ __forceinline__ uint32_t fp8_out_bits(float v, half_t bias) {
  const uint32_t b = f32_to_bf16_bits(v);
  const float bf = __builtin_bit_cast(float, b << 16);
  if (OUT_BF16) return f32_to_bf16_bits(bf + bf16_value((float)bias));
  return (uint32_t)__builtin_bit_cast(uint16_t, (half_t)((float)(half_t)bf + (float)bias));
}

// fp8_out_bits of two adjacent outputs, packed (v0 low): one bf16 conversion per pair.
template <bool OUT_BF16>
__device__ __forceinline__ uint32_t fp8_out_bits2(float v0, float v1, half_t b0, half_t b1) {
  const uint32_t p = bf16x2_bits(v0, v1);
  const float f0 = __builtin_bit_cast(float, p << 16), f1 = __builtin_bit_cast(float, p & 0xffff0000u);
  if (OUT_BF16) return bf16x2_bits(f0 + bf16_value((float)b0), f1 + bf16_value((float)b1));
  const half_t h0 = (half_t)((float)(half_t)f0 + (float)b0);
  const half_t h1 = (half_t)((float)(half_t)f1 + (float)b1);
  return (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
}

// Persistent form of the big tiles: a grid of at most one workgroup per CU walks its tiles
// (round r, slot b: logical tile r * grid + b, in the same XCD-grouped order), and the K
// loop runs straight across tile boundaries: the next tile's first two stages are loaded
// during the current tile's last two steps, so no tile waits for its first operands.  The
// tile's row / column scales and biases ride with its first stage into an LDS slot of their
// own (two, by tile parity), which the epilogue reads with its own lgkmcnt wait: an epilogue
// that read them from global memory would wait (vmcnt) for the next tile's stages in flight.
// TAIL (256 columns): the columns past a.n_big run as 256 x 192 tiles after every whole tile
// (fp8_tail_cols); such a tile loads 3 of the 4 row groups of w, reads its wave's 3 n
// sub-tiles from 48 wn plus a fourth fragment from the slot's next 16 rows (unused), and
// stores 3 of its 4 n sub-tiles, so both kinds share the loop's code and registers.
template <bool OUT_BF16, int NIW, typename ReadCol>
__device__ __forceinline__ void fp8_bigp_epilogue(const f32x4 (&acc)[NIW][8], uint16_t* ob, int ldo,
                                                  const float (&sm)[8], ReadCol read_col,
                                                  bool has_bias, int ni) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < NIW; ++i) {
    if (i >= ni) continue;      // (wave-uniform) a 192-column tail tile stores 3 of 4
    f32x4 snv;
    u32x2 bw;
    read_col(i, snv, bw);       // column scales and biases of n sub-tile i
    const f32x4 sn_i = snv;
    half4_t bb = (half4_t){0, 0, 0, 0};
    if (has_bias) bb = __builtin_bit_cast(half4_t, bw);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (acc[i][j][q] * sm[j]) * sn_i[q];
      uint2 pk;
      pk.x = fp8_out_bits2<OUT_BF16>(v[0], v[1], bb[0], bb[1]);
      pk.y = fp8_out_bits2<OUT_BF16>(v[2], v[3], bb[2], bb[3]);
      *(uint2*)(ob + (16 * j * ldo + 16 * i)) = pk;
    }
  }
}

template <int NI, bool TAIL = false>
__global__ __launch_bounds__(512, 1) void fp8_gemm_bigp_kernel(Fp8GemmArgs a) {
#pragma clang fp contract(off)
  constexpr int NS = 2;                       // stages (64 KB + 16 NI * 2 KB each)
  constexpr int BN = 32 * NI;                 // tile columns: four waves of 8 NI
  constexpr int XLD = 4;                      // x loads per wave and stage (256 rows / 8 / 8)
  constexpr int WLD = NI / 2;                 // w loads per wave and stage (BN rows / 8 / 8)
  constexpr int NIW = NI / 2;                 // n sub-tiles per wave (4 waves along n)
  constexpr int OPS = XLD + WLD;              // operand loads every thread issues per stage
  static_assert(NI == 6 || NI == 8, "tile widths 192 and 256");
  static_assert(!TAIL || NI == 8, "192-column tail tiles after 256-column ones");
  __shared__ __attribute__((aligned(1024))) uint8_t xl[NS][F8B_T * F8_ROWB];
  __shared__ __attribute__((aligned(1024))) uint8_t wl[NS][BN * F8_ROWB];
  __shared__ __attribute__((aligned(16))) float scl[2][F8B_T + BN];    // [tile parity][sa | sw]
  __shared__ __attribute__((aligned(16))) half_t bsl[2][512];          // [tile parity][bias]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 3;
  const int wm = wave >> 2;
  const int l16 = lane & 15;
  const int g4 = lane >> 4;

  const int tiles_n = a.n_big / BN;
  const int tiles_m = a.M / F8B_T;
  const int tiles = tiles_m * tiles_n;
  // 256-column tiles: the columns past n_big as 256 x 192 tiles after every whole tile (a
  // grid whose whole tiles fill R rounds exactly then ends with at most one such tile per CU)
  const int tiles_tn = TAIL ? (a.N - a.n_big) / 192 : 0;
  const int items = tiles + tiles_m * tiles_tn;
  const int G = gridDim.x;
  const int slot = xcd_logical_block(blockIdx.x, G);
  const int my_tiles = (items - slot + G - 1) / G;          // grid <= items: >= 1
  const int nk = a.K / F8_BK;                               // >= NS (host check)
  auto tile_at = [&](int r, int& m0, int& n0, int& tl) {    // past the last tile: the last one
    const int it = min(r, my_tiles - 1) * G + slot;
    int tm, tn;
    if (!TAIL || it < tiles) {
      grouped_tile(it, tiles_m, tiles_n, F8_GM, tm, tn);
      n0 = tn * BN;
      tl = 0;
    } else {
      grouped_tile(it - tiles, tiles_m, tiles_tn, F8_GM, tm, tn);
      n0 = a.n_big + tn * 192;
      tl = 1;
    }
    m0 = tm * F8B_T;
  };

  const int lrow = 8 * wave + (lane >> 3);
  const int lchunk = (lane & 7) ^ (lrow & 7);
  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const bool has_bias = a.bias != nullptr;
  const uint32_t loff = (uint32_t)lrow * (uint32_t)a.K + (uint32_t)lchunk * 16u;
  const uint32_t rstep = 64u * (uint32_t)a.K;
  auto issue = [&](int m0, int n0, int ks, int st, int tl) {
    const uint8_t* const xs = a.xq + (int64_t)m0 * a.K;
    const uint8_t* const ws = a.wq + (int64_t)n0 * a.K;
    const uint32_t k0 = loff + (uint32_t)ks * F8_BK;
#pragma unroll
    for (int u = 0; u < XLD; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(xs + (k0 + u * rstep)),
                                       (lds_void*)((lds_u8*)&xl[st][(64 * u + 8 * wave) * F8_ROWB]), 16, 0, 0);
#pragma unroll
    for (int u = 0; u < WLD; ++u) {
      if (TAIL && tl && u >= 3) break;  // a 192-column tile's 3 row groups of w
      __builtin_amdgcn_global_load_lds((const void*)(ws + (k0 + u * rstep)),
                                       (lds_void*)((lds_u8*)&wl[st][(64 * u + 8 * wave) * F8_ROWB]), 16, 0, 0);
    }
  };
  // the tile's 256 row scales (one per thread), BN column scales (waves < BN / 64) and BN
  // biases (wave 0, 16 bytes a lane; lanes past BN / 8 repeat the last chunk)
  // (wave-uniform bases plus 32-bit lane offsets from a lane index passed through an empty
  // asm, so that the compiler cannot hoist 64-bit lane addresses out of the loops and keep
  // them live beside the accumulators)
  auto issue_scales = [&](int m0, int n0, int p, int tl) {
    uint32_t ln = (uint32_t)lane;
    asm volatile("" : "+v"(ln));
    const int bn = TAIL && tl ? 192 : BN;   // the tile's columns
    if (wave < 4) {
      const uint8_t* const sab = (const uint8_t*)(a.sa + m0 + 64 * wave);
      __builtin_amdgcn_global_load_lds((const void*)(sab + 4u * ln),
                                       (lds_void*)((lds_u8*)&scl[p][64 * wave]), 4, 0, 0);
    }
    if (wave < bn / 64) {
      const uint8_t* const swb = (const uint8_t*)(a.sw + n0 + 64 * wave);
      __builtin_amdgcn_global_load_lds((const void*)(swb + 4u * ln),
                                       (lds_void*)((lds_u8*)&scl[p][F8B_T + 64 * wave]), 4, 0, 0);
    }
    if (wave == 0 && has_bias) {
      const uint8_t* const bb = (const uint8_t*)(a.bias + n0);
      __builtin_amdgcn_global_load_lds((const void*)(bb + 16u * min(ln, (uint32_t)(bn / 8 - 1))),
                                       (lds_void*)((lds_u8*)&bsl[p][0]), 16, 0, 0);
    }
  };
  auto addrs = [&](int st, int o, int base, uint32_t& a0, uint32_t& a1) {
    const int r = base + l16;
    const uint32_t row = (uint32_t)(uintptr_t)(lds_u8*)(o ? &wl[st][r * F8_ROWB] : &xl[st][r * F8_ROWB]);
    a0 = row + (((2 * g4) ^ (l16 & 7)) << 4);
    a1 = row + (((2 * g4 + 1) ^ (l16 & 7)) << 4);
  };
  auto read16 = [&](uint32_t a0, uint32_t a1, u32x4* v) {
    asm volatile(
        "ds_read_b128 %0, %16\n\tds_read_b128 %1, %17\n\t"
        "ds_read_b128 %2, %16 offset:2048\n\tds_read_b128 %3, %17 offset:2048\n\t"
        "ds_read_b128 %4, %16 offset:4096\n\tds_read_b128 %5, %17 offset:4096\n\t"
        "ds_read_b128 %6, %16 offset:6144\n\tds_read_b128 %7, %17 offset:6144\n\t"
        "ds_read_b128 %8, %16 offset:8192\n\tds_read_b128 %9, %17 offset:8192\n\t"
        "ds_read_b128 %10, %16 offset:10240\n\tds_read_b128 %11, %17 offset:10240\n\t"
        "ds_read_b128 %12, %16 offset:12288\n\tds_read_b128 %13, %17 offset:12288\n\t"
        "ds_read_b128 %14, %16 offset:14336\n\tds_read_b128 %15, %17 offset:14336"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
          "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
          "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
        : "v"(a0), "v"(a1)
        : "memory");
  };
  auto wait16 = [&](u32x4* v) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]),
                   "+v"(v[12]), "+v"(v[13]), "+v"(v[14]), "+v"(v[15])
                 :
                 : "memory");
  };
  auto read8 = [&](uint32_t a0, uint32_t a1, u32x4* v) {
    asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %9\n\t"
        "ds_read_b128 %2, %8 offset:2048\n\tds_read_b128 %3, %9 offset:2048\n\t"
        "ds_read_b128 %4, %8 offset:4096\n\tds_read_b128 %5, %9 offset:4096\n\t"
        "ds_read_b128 %6, %8 offset:6144\n\tds_read_b128 %7, %9 offset:6144"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
          "=&v"(v[6]), "=&v"(v[7])
        : "v"(a0), "v"(a1)
        : "memory");
  };
  auto read6 = [&](uint32_t a0, uint32_t a1, u32x4* v) {
    asm volatile(
        "ds_read_b128 %0, %6\n\tds_read_b128 %1, %7\n\t"
        "ds_read_b128 %2, %6 offset:2048\n\tds_read_b128 %3, %7 offset:2048\n\t"
        "ds_read_b128 %4, %6 offset:4096\n\tds_read_b128 %5, %7 offset:4096"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5])
        : "v"(a0), "v"(a1)
        : "memory");
  };
  auto wait8 = [&](u32x4* v) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7])
                 :
                 : "memory");
  };
  auto wait6 = [&](u32x4* v) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5])
                 :
                 : "memory");
  };
  auto frag = [](const u32x4& lo, const u32x4& hi) {
    return (i32x8){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  };
  // The epilogue's scales and biases of tile parity p, each read with its own lgkmcnt
  // wait: row scales of rows 128 wm + 16 j + l16 (64 bytes apart), then per n sub-tile i the
  // column scales and biases of columns 16 NI wn + 16 i + 4 g4 .. +3.
  typedef __attribute__((address_space(3))) float lds_f32;
  typedef __attribute__((address_space(3))) half_t lds_f16;
  auto read_row_scales = [&](int p, float (&sm)[8]) {
    uint32_t ln = (uint32_t)lane;             // (not hoisted: see issue_scales)
    asm volatile("" : "+v"(ln));
    const uint32_t am = (uint32_t)(uintptr_t)(lds_f32*)&scl[p][128 * wm + (ln & 15u)];
    asm volatile(
        "ds_read_b32 %0, %8\n\tds_read_b32 %1, %8 offset:64\n\tds_read_b32 %2, %8 offset:128\n\t"
        "ds_read_b32 %3, %8 offset:192\n\tds_read_b32 %4, %8 offset:256\n\tds_read_b32 %5, %8 offset:320\n\t"
        "ds_read_b32 %6, %8 offset:384\n\tds_read_b32 %7, %8 offset:448\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(sm[0]), "=&v"(sm[1]), "=&v"(sm[2]), "=&v"(sm[3]), "=&v"(sm[4]), "=&v"(sm[5]),
          "=&v"(sm[6]), "=&v"(sm[7])
        : "v"(am)
        : "memory");
  };
  auto read_col = [&](int p, int cw, int i, f32x4& sn, u32x2& bw) {
    uint32_t ln = (uint32_t)lane;             // (not hoisted: see issue_scales)
    asm volatile("" : "+v"(ln));
    const uint32_t c4 = 4u * (ln >> 4);
    const uint32_t an = (uint32_t)(uintptr_t)(lds_f32*)&scl[p][F8B_T + cw + 16 * i + c4];
    const uint32_t ab = (uint32_t)(uintptr_t)(lds_f16*)&bsl[p][cw + 16 * i + c4];
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b64 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(sn), "=&v"(bw)
                 : "v"(an), "v"(ab)
                 : "memory");
  };

  // Steps sidx = 0, 1, ... walk the tiles' K steps back to back in slots sidx % 2; after
  // step s's operands are in registers and step s + 1 has landed everywhere (vmcnt 0 +
  // barrier: with two stages nothing younger is in flight), step s + 2 goes into slot s % 2.
  int m0c, n0c, m0n, n0n, tlc, tln;
  tile_at(0, m0c, n0c, tlc);
  tile_at(1, m0n, n0n, tln);
  issue_scales(m0c, n0c, 0, tlc);
  issue(m0c, n0c, 0, 0, tlc);
  issue(m0c, n0c, 1, 1, tlc);
  wait_vmcnt<OPS>();                          // the scales and stage 0 (issued first)
  barrier_only();
  int sidx = 0;
  for (int r = 0; r < my_tiles; ++r) {
    f32x4 acc[NIW][8];   // [n sub-tile][m sub-tile]
#pragma unroll
    for (int i = 0; i < NIW; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < nk; ++ks, ++sidx) {
      const int st = sidx & 1;
      u32x4 wo[2 * NIW], xo[16];
      {
        uint32_t aw0, aw1, ax0, ax1;
        // a 192-column tile (tlc): the wave's 3 n sub-tiles start at 48 wn; its fourth
        // fragment reads the slot's next 16 rows (the next wave's, or rows 192-255 that this
        // tile leaves unloaded) into accumulators the epilogue does not store
        addrs(st, 1, (TAIL && tlc ? 48 : 16 * NIW) * wn, aw0, aw1);
        addrs(st, 0, 128 * wm, ax0, ax1);
        if constexpr (NIW == 4) read8(aw0, aw1, wo);
        else read6(aw0, aw1, wo);
        read16(ax0, ax1, xo);
        if constexpr (NIW == 4) wait8(wo);
        else wait6(wo);
        wait16(xo);
      }
      wait_vmcnt<0>();
      barrier_only();
      {
        const int iks = ks + NS;
        if (iks < nk) {
          issue(m0c, n0c, iks, st, tlc);
        } else {
          if (iks == nk) issue_scales(m0n, n0n, (r + 1) & 1, tln);
          issue(m0n, n0n, iks - nk, st, tln);
        }
      }
#pragma unroll
      for (int i = 0; i < NIW; ++i) {
        const i32x8 wf = frag(wo[2 * i], wo[2 * i + 1]);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              wf, frag(xo[2 * j], xo[2 * j + 1]), acc[i][j], 0, 0, 0, 127, 0, 127);
      }
    }
    // Epilogue: lane holds n = n0 + 16 NI wn + 16 i + 4 g4 + q of m = m0 + 128 wm + 16 j + l16.
    {
      float sm[8];
      read_row_scales(r & 1, sm);
      uint32_t ln = (uint32_t)lane;           // (not hoisted: see issue_scales)
      asm volatile("" : "+v"(ln));
      const int cw = (TAIL && tlc ? 48 : 16 * NIW) * wn;   // the wave's first column in the tile
      uint16_t* const ob = (uint16_t*)a.out + (int64_t)(m0c + 128 * wm) * a.ldo + n0c + cw +
                           ((ln & 15u) * (uint32_t)a.ldo + 4u * (ln >> 4));
      auto rc = [&](int i, f32x4& sn, u32x2& bw) { read_col(r & 1, cw, i, sn, bw); };
      const int ni = TAIL && tlc ? 3 : NIW;           // n sub-tiles stored
      if (a.out_mode) fp8_bigp_epilogue<true, NIW>(acc, ob, a.ldo, sm, rc, has_bias, ni);
      else fp8_bigp_epilogue<false, NIW>(acc, ob, a.ldo, sm, rc, has_bias, ni);
    }
    m0c = m0n;
    n0c = n0n;
    tlc = tln;
    tile_at(r + 2, m0n, n0n, tln);
  }
  wait_vmcnt<0>();                             // drain the clamped tail loads before exit
}

static int num_cus() {
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

// Row-wise e4m3 quantisation: s[r] = amax_k |x[r, k]| / 448 (clamped below at clamp_min
// when clamp_min > 0; rounded to fp16 when S16: FP8Linear's row-wise weight scale, an op on
// the fp16 weight), q[r, k] = e4m3(x[r, k] / s[r]) (one rounding: fp32 division).  One
// workgroup per row.
template <bool BF16, bool S16 = false>
__global__ __launch_bounds__(256) void fp8_quant_rows_kernel(const unsigned short* __restrict__ x,
                                                             int ldx, uint8_t* __restrict__ q,
                                                             float* __restrict__ s, int K,
                                                             float clamp_min) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const unsigned short* xr = x + (int64_t)row * ldx;
  float amax = 0.f;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    const u16x8 v = *(const u16x8*)(xr + k);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(ld16f<BF16>(v[e])));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sc = amax / 448.0f;
  if (S16) sc = (float)(half_t)sc;
  if (clamp_min > 0.f) sc = fmaxf(sc, clamp_min);
  if (threadIdx.x == 0) s[row] = sc;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    const u16x8 v = *(const u16x8*)(xr + k);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) lo |= (uint32_t)f32_to_e4m3fn(ld16f<BF16>(v[e]) / sc) << (8 * e);
#pragma unroll
    for (int e = 0; e < 4; ++e) hi |= (uint32_t)f32_to_e4m3fn(ld16f<BF16>(v[4 + e]) / sc) << (8 * e);
    *(uint2*)(q + (int64_t)row * K + k) = make_uint2(lo, hi);
  }
}

static int fp8_quant_rows_launch(const void* x, int ldx, void* xq, float* scale, int rows, int K,
                                 float clamp_min, bool bf16, void* stream, bool s16 = false) {
  if (rows < 0 || K <= 0) return OMNI_EINVAL;
  if ((K & 7) || ldx < K || (ldx & 7)) return OMNI_EUNSUPPORTED;
  if (rows == 0) return OMNI_OK;
  if (!x || !xq || !scale) return OMNI_EINVAL;
  auto kern = s16 ? fp8_quant_rows_kernel<false, true>
                  : bf16 ? fp8_quant_rows_kernel<true> : fp8_quant_rows_kernel<false>;
  hipLaunchKernelGGL(kern, dim3(rows), dim3(256), 0, (hipStream_t)stream,
                     (const unsigned short*)x, ldx, (uint8_t*)xq, scale, K, clamp_min);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

extern "C" int omni_fp8_quant_rows(const void* x, int ldx, void* xq, float* scale, int rows, int K,
                                   float clamp_min, void* stream) {
  return fp8_quant_rows_launch(x, ldx, xq, scale, rows, K, clamp_min, false, stream);
}

extern "C" int omni_fp8_quant_rows_bf16(const void* x, int ldx, void* xq, float* scale, int rows,
                                        int K, float clamp_min, void* stream) {
  return fp8_quant_rows_launch(x, ldx, xq, scale, rows, K, clamp_min, true, stream);
}

extern "C" int omni_fp8_quant_weight_rows(const void* w, int ldw, void* wq, float* scale, int N,
                                          int K, void* stream) {
  return fp8_quant_rows_launch(w, ldw, wq, scale, N, K, 0.f, false, stream, true);
}

// Per-tensor e4m3 quantisation (FP8Linear's default form): s = R(amax |x| / 448) and
// q = e4m3(R(x / s)), R the input's own rounding (fp16, or bf16 for bf16 input): the
// reference forms both with ops on the fp16 / bf16 tensor (fp8_linear.py:40-41, 87-89).
// Two launches, no atomics: fp8_amax_kernel writes one partial maximum per workgroup
// (rows b, b + grid, ...), fp8_quant_tensor_kernel reduces the grid's partials in every
// workgroup and quantises the same rows, writing s into scale[r] for each of them.
#define FP8_AMAX_GRID 256

template <bool BF16>
__global__ __launch_bounds__(256) void fp8_amax_kernel(const unsigned short* __restrict__ x,
                                                       int ldx, int rows, int K,
                                                       float* __restrict__ part) {
  __shared__ float red[4];
  float amax = 0.f;
  for (int r = blockIdx.x; r < rows; r += gridDim.x) {
    const unsigned short* xr = x + (int64_t)r * ldx;
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
      const u16x8 v = *(const u16x8*)(xr + k);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(ld16f<BF16>(v[e])));
    }
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <bool BF16>
__device__ __forceinline__ float round_in(float v) {
  return BF16 ? bf16_value(v) : (float)(half_t)v;
}

template <bool BF16>
__global__ __launch_bounds__(256) void fp8_quant_tensor_kernel(const unsigned short* __restrict__ x,
                                                               int ldx, int rows, int K,
                                                               const float* __restrict__ part,
                                                               uint8_t* __restrict__ q,
                                                               float* __restrict__ s) {
#pragma clang fp contract(off)
  __shared__ float red[4];
  float amax = 0.f;
  for (int i = threadIdx.x; i < (int)gridDim.x; i += 256) amax = fmaxf(amax, part[i]);
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = round_in<BF16>(amax / 448.0f);
  for (int r = blockIdx.x; r < rows; r += gridDim.x) {
    const unsigned short* xr = x + (int64_t)r * ldx;
    if (threadIdx.x == 0) s[r] = sc;
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
      const u16x8 v = *(const u16x8*)(xr + k);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        lo |= (uint32_t)f32_to_e4m3fn(round_in<BF16>(ld16f<BF16>(v[e]) / sc)) << (8 * e);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        hi |= (uint32_t)f32_to_e4m3fn(round_in<BF16>(ld16f<BF16>(v[4 + e]) / sc)) << (8 * e);
      *(uint2*)(q + (int64_t)r * K + k) = make_uint2(lo, hi);
    }
  }
}

extern "C" int omni_fp8_quant_tensor_work(int rows) {
  return rows <= 0 ? 0 : (rows < FP8_AMAX_GRID ? rows : FP8_AMAX_GRID);
}

extern "C" int omni_fp8_quant_tensor(const void* x, int ldx, void* q, float* scale, float* work,
                                     int rows, int K, int bf16, void* stream) {
  if (rows < 0 || K <= 0) return OMNI_EINVAL;
  if ((K & 7) || ldx < K || (ldx & 7)) return OMNI_EUNSUPPORTED;
  if (rows == 0) return OMNI_OK;
  if (!x || !q || !scale || !work) return OMNI_EINVAL;
  const int grid = omni_fp8_quant_tensor_work(rows);
  if (bf16) {
    hipLaunchKernelGGL(fp8_amax_kernel<true>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       (const unsigned short*)x, ldx, rows, K, work);
    OMNI_CHECK_LAUNCH();
    hipLaunchKernelGGL(fp8_quant_tensor_kernel<true>, dim3(grid), dim3(256), 0,
                       (hipStream_t)stream, (const unsigned short*)x, ldx, rows, K, work,
                       (uint8_t*)q, scale);
  } else {
    hipLaunchKernelGGL(fp8_amax_kernel<false>, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                       (const unsigned short*)x, ldx, rows, K, work);
    OMNI_CHECK_LAUNCH();
    hipLaunchKernelGGL(fp8_quant_tensor_kernel<false>, dim3(grid), dim3(256), 0,
                       (hipStream_t)stream, (const unsigned short*)x, ldx, rows, K, work,
                       (uint8_t*)q, scale);
  }
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// Kernel choice by shape: the persistent big tiles (256 x 256 or 256 x 192) where a cost
// model of rounds of the grid (one tile per CU per round) times a tile's work puts them
// ahead of the 8-wave pipelined 256 x 128 tiles: a big tile costs 0.85 x its size in
// 256 x 128 tiles (fitted on MI355X: the big tiles' operand bytes per MFMA are lower); the
// pipelined form every other shape with at least 4 K steps; the double-buffered
// one-tile-per-workgroup kernel the rest (K < 512).  MI355X, us (pipelined / persistent
// 256 x 192 / persistent 256 x 256, outputs bit-equal), M = 8192: K 1536 -> N 17920 344.4 /
// - / 302.3; 1536 -> 2048 45.1 / - / 35.6; 1536 -> 1536 43.0 / 28.0 / 33.7; 8960 -> 1536
// 156.7 / 100.3 / 121.4; M = 4096: 1536 -> 17920 172.9 / - / 146.8; 8960 -> 1536 78.8 /
// 95.6 / 119.0 (hipBLASLt's row-wise _scaled_mm on the same shapes 245.9, 29.9, 27.0,
// 93.3, 113.3, 60.8).  Returns the big tile's width (0: not big).
// The persistent 256 x 256 tiles' column split: where whole tiles would leave the last round
// partly idle, the columns past the returned one run as 256 x 192 tiles after R full rounds
// of whole tiles, at most one per CU (config 4's gate_up at M = 8192: 2240 tiles = 8 rounds
// and 192 more, so 2048 whole tiles over columns [0, 16384) and 256 tiles of 192 columns over
// the last 1536: every CU runs 8.75 tiles' work where 192 of them ran 9); N where no such
// split exists.
static int fp8_tail_cols(int M, int N) {
  const int64_t cus = num_cus();
  const int64_t tm = M / F8B_T, tn = N / 256;
  const int64_t tiles = tm * tn;
  const int64_t R = tiles / cus;
  if (R == 0 || tiles % cus == 0 || (R * cus) % tm) return N;
  const int64_t nb = R * cus / tm;                    // whole column tiles
  const int64_t rest = (int64_t)N - nb * 256;
  if (rest % 192 || tm * (rest / 192) > cus) return N;
  return (int)(nb * 256);
}

static int fp8_big_cols(int M, int N, int K, int out_mode = FP8_OUT_F16_VIA_BF16) {
  if (K < 1024 || (M % F8B_T) || out_mode == FP8_OUT_F16) return 0;
  const int64_t cus = num_cus();
  auto rounds = [&](int64_t t) { return (t + cus - 1) / cus; };
  double best = (double)rounds((int64_t)(M / 256) * (N / F8_BT));   // pipelined tiles
  int cols = 0;
  for (int bn : {256, 192}) {
    if (N % bn) continue;
    const int64_t t = (int64_t)(M / F8B_T) * (N / bn);
    // with a 192-column tail (fp8_tail_cols) the last round is 0.75 of a whole one
    const double r = bn == 256 && fp8_tail_cols(M, N) < N ? (double)(t / cus) + 0.75 : (double)rounds(t);
    const double c = r * (bn / 128.0) * 0.85;
    if (c < best) best = c, cols = bn;
  }
  return cols;
}

// Items of the persistent big kernel (whole tiles plus the 192-column tail tiles).
static int64_t fp8_big_items(int M, int N, int bc) {
  if (bc != 256) return (int64_t)(M / F8B_T) * (N / bc);
  const int nb = fp8_tail_cols(M, N);
  return (int64_t)(M / F8B_T) * (nb / 256 + (N - nb) / 192);
}

// Which kernel omni_fp8_gemm runs for a shape: 0 one tile per workgroup, 1 the pipelined
// 256 x 128 tiles, 2 the 256 x 256 tiles, 3 the 256 x 192 tiles; and the grid it launches.
extern "C" int omni_fp8_gemm_plan(int M, int N, int K, int* grid) {
  if (M <= 0 || N <= 0 || K <= 0 || (N % F8_BT) || (K % F8_BK)) return OMNI_EINVAL;
  int kind, g;
  const int bc = fp8_big_cols(M, N, K);
  if (bc) {
    const int64_t t = fp8_big_items(M, N, bc);
    kind = bc == 256 ? 2 : 3, g = (int)(t < num_cus() ? t : num_cus());
  } else if (K / F8_BK >= 4) {
    const int64_t t8 = (int64_t)ceil_div(M, 256) * (N / F8_BT);
    kind = 1, g = (int)(t8 < num_cus() ? t8 : num_cus());
  } else {
    kind = 0, g = ceil_div(M, F8_BT) * (N / F8_BT);
  }
  if (grid) *grid = g;
  return kind;
}

extern "C" int omni_fp8_gemm(const void* xq, const float* sa, const void* wq, const float* sw,
                             const void* bias, void* out, int ldo, int M, int N, int K,
                             int out_mode, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return OMNI_EINVAL;
  if ((N % F8_BT) || (K % F8_BK)) return OMNI_EUNSUPPORTED;
  if (ldo < N || (ldo & 3)) return OMNI_EINVAL;
  if (out_mode < FP8_OUT_F16_VIA_BF16 || out_mode > FP8_OUT_F16) return OMNI_EINVAL;
  if (M == 0) return OMNI_OK;
  if (!xq || !sa || !wq || !sw || !out) return OMNI_EINVAL;
  // the kernels stage operand rows and biases with 16-byte global->LDS loads, scales with
  // 4-byte ones, and store 8 bytes at a time
  if (((uintptr_t)xq & 15) || ((uintptr_t)wq & 15) || ((uintptr_t)bias & 15) ||
      ((uintptr_t)sa & 3) || ((uintptr_t)sw & 3) || ((uintptr_t)out & 7))
    return OMNI_EINVAL;
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
  a.out_mode = out_mode;
  a.n_big = N;
  const int bc = fp8_big_cols(M, N, K, out_mode);
  if (bc) {                                       // persistent 256 x bc tiles
    if (bc == 256) a.n_big = fp8_tail_cols(M, N);
    const int64_t bt = fp8_big_items(M, N, bc);
    const int grid = (int)(bt < num_cus() ? bt : num_cus());
    if (bc == 256 && a.n_big < N)
      hipLaunchKernelGGL((fp8_gemm_bigp_kernel<8, true>), dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream, a);
    else if (bc == 256)
      hipLaunchKernelGGL((fp8_gemm_bigp_kernel<8>), dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL((fp8_gemm_bigp_kernel<6>), dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream, a);
  } else if (K / F8_BK >= 4) {                    // 8 waves, 256 x 128 tiles, 3 stages
    const int64_t t8 = (int64_t)ceil_div(M, 256) * (N / F8_BT);
    const int grid = (int)(t8 < num_cus() ? t8 : num_cus());
    hipLaunchKernelGGL((fp8_gemm_pipe_kernel<4, 3>), dim3((unsigned)grid), dim3(512), 0,
                       (hipStream_t)stream, a);
  } else {
    hipLaunchKernelGGL(fp8_gemm_kernel, dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream, a);
  }
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// Exhaustive device check of the bf16 rounding the FP8 epilogues use: every one of the 2^32
// float bit patterns through bf16x2_bits (the hardware conversion) and bf16_bits_int (the
// integer rounding); mismatches[0] counts non-NaN inputs that differ, mismatches[1] NaNs.
__global__ __launch_bounds__(256) void bf16_rne_check_kernel(unsigned long long* mismatches) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;      // 2^24 threads, 256 patterns each
  uint32_t bad = 0, badnan = 0;
  for (uint32_t k = 0; k < 256; k += 2) {
    const uint32_t u0 = (i << 8) | k, u1 = u0 | 1u;
    const uint32_t hw = bf16x2_bits(__builtin_bit_cast(float, u0), __builtin_bit_cast(float, u1));
    const bool n0 = (u0 & 0x7fffffffu) > 0x7f800000u, n1 = (u1 & 0x7fffffffu) > 0x7f800000u;
    if ((hw & 0xffffu) != bf16_bits_int(u0)) ++(n0 ? badnan : bad);
    if ((hw >> 16) != bf16_bits_int(u1)) ++(n1 ? badnan : bad);
  }
  if (bad) atomicAdd(&mismatches[0], (unsigned long long)bad);
  if (badnan) atomicAdd(&mismatches[1], (unsigned long long)badnan);
}

extern "C" int omni_bf16_rne_check(unsigned long long* mismatches, void* stream) {
  if (!mismatches || ((uintptr_t)mismatches & 7)) return OMNI_EINVAL;
  hipLaunchKernelGGL(bf16_rne_check_kernel, dim3(1u << 16), dim3(256), 0, (hipStream_t)stream,
                     mismatches);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

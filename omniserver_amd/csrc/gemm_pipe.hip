// fp16 GEMM with a multi-stage global -> LDS pipeline, for the vision tower's linears and
// the decoder's prefill linears:
//   out[m, n] = epi(fp16(sum_k x[m, k] w[n, k] + bias[n]))
// x fp16 [M, K] (row stride ldx); w one of
//   GW_ROWS  fp16 [N, K] (nn.Linear layout, row stride K),
//   GW_F16   this library's packed fp16 layout [N/16][K/32][64][8] (omni_f16_pack),
//   GW_INT4  the packed int4 layout [N/16][K/128][64][4] + scales [N/16][K/128][16]
//            (omni_gptq_repack), dequantised as fp16((q - 8) s);
// fp32 accumulation on v_mfma_f32_16x16x32_f16.  Epilogues: STORE (bias added before or,
// GPTQ order, after the fp16 rounding), QGELU (x sigmoid(1.702 x)), GELU (erf), RESID
// (fp16(res + h)), SILU (packed weights with gate|up tiles interleaved: silu(g) * u).
//
// The packed layouts are MFMA operand blocks: 1 KB per (16 columns, 32 k) for fp16, per
// (16 columns, 128 k) for int4 (lane l: column l % 16, k = 8 (l / 16) + e, one 4-byte
// word per 32-k step), so a block is staged to LDS as one contiguous load and read back
// by each lane at 16 l (fp16) or 4 l (int4: the step's two words land as two 256-byte
// planes): no swizzle is needed for them.
//
// Persistent grid (one workgroup per CU at most) walking 64 WM x 128 output tiles in
// grouped, XCD-aware order.  2 WM waves, each owning a 64 (m) x 64 (n) sub-tile: per K
// step of 64 (128 bytes of every operand row) it issues 16 LDS operand reads and 32
// MFMAs.  Operand rows go global -> LDS with global_load_lds (16 bytes per lane), NS
// steps ahead, across tile boundaries (the last steps of a tile load the next tile's
// first ones); the 16-byte chunks of a row are XOR-swizzled by row so that the 16 rows an
// operand read touches spread over the banks.  A step's slot is read once an exact
// per-thread vmcnt and a barrier say it landed everywhere, and refilled after the next
// barrier; the LDS reads of step s + 1 are issued before the MFMAs of step s (two register
// sets), so the read latency hides behind the MFMAs instead of following the barrier that
// every wave of the workgroup passes together.  K slices are whole 128-k groups.
#include "common.h"

#define GP_BN 128        // tile columns (n)
#define GP_BKH 64        // K (halfs) per pipeline step
#define GP_ROWB 128      // LDS bytes per staged operand row (one step)
#define GP_GM 4          // tile rows per group of the tile order

enum { GP_STORE = 0, GP_SILU = 1, GP_PARTIAL = 2, GP_QGELU = 4, GP_GELU = 5, GP_RESID = 6 };
enum { GW_ROWS = 0, GW_F16 = 1, GW_INT4 = 2 };

struct GemmPipeArgs {
  const half_t* x;
  int ldx;
  const half_t* w;       // GW_ROWS / GW_F16
  int ldw;
  const uint32_t* wq;    // GW_INT4 codes
  const half_t* wsc;     // GW_INT4 scales
  int bias_after_round;  // 1: fp16(fp16(acc) + b) (GPTQ); 0: fp16(acc + b)
  const half_t* bias;    // [N] or NULL
  const half_t* res;     // GP_RESID: [M, ldr]
  int ldr;
  half_t* out;
  int ldo;
  int M, N, K;
  int KS;                // K slices; > 1: fp32 partial sums to part, finished by a second kernel
  float* part;           // [KS][M][N]
  int n_big;             // persistent 256-column tiles: whole tiles below column n_big, 128-column
                         // half tiles from there to N (one K slice); N elsewhere
};

template <int N>
__device__ __forceinline__ void gp_wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void gp_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ half_t gp_quick_gelu(half_t h) {
#pragma clang fp contract(off)
  const float t = (float)(half_t)((float)h * 1.702f);
  const float sg = (float)(half_t)(1.0f / (1.0f + expf(-t)));
  return (half_t)((float)h * sg);
}

// fp16 of acc + bias in the linear's order (bias_after_round: added to the fp16 rounding)
__device__ __forceinline__ half_t gp_bias(float acc, half_t b, bool has_bias, int bar) {
#pragma clang fp contract(off)
  if (!has_bias) return (half_t)acc;
  return bar ? (half_t)((float)(half_t)acc + (float)b) : (half_t)(acc + (float)b);
}

__device__ __forceinline__ half_t gp_gelu(half_t h) {
#pragma clang fp contract(off)
  const float x = (float)h;
  return (half_t)(0.5f * x * (1.0f + erff(x * 0.70710678118654752f)));
}

// One work item (output tile x K slice): per-lane operand row pointers (at the slice's
// first k; rows clamped below M) for the four x row groups and w row group 0, the bias
// pointer, and the slice's K steps.
struct GpTileSrc {
  const half_t* x[4];
  const half_t* w;       // GW_ROWS: the lane's row
  const void* wp[6];     // GW_F16 / GW_INT4: the lane's block of each w load (step 0 / group 0)
  const half_t* sp;      // GW_INT4: the lane's scale pair (group 0)
  const half_t* b;
  int kb;                // the slice's first K step
  int kc;
};

// NI: n sub-tiles of 16 per wave (tile columns BN = 32 NI: 128, or 192 for the packed fp16
// weights with the STORE / PARTIAL epilogues).
template <int WF, int WM, int NS, int EPI, int NI = 4>
__global__ __launch_bounds__(128 * WM, 1) void gemm_pipe_kernel(GemmPipeArgs a) {
#pragma clang fp contract(off)
  static_assert(NI == 4 || (NI == 6 && WF == GW_F16 && (EPI == GP_STORE || EPI == GP_PARTIAL)),
                "192-column tiles: packed fp16 weights, STORE / PARTIAL epilogues");
  constexpr int BM = 64 * WM;
  constexpr int BN = 32 * NI;
  constexpr int NWV = 2 * WM;
  constexpr int NV = 2 * NI + 8;        // operand fragments per step: w 2 NI, then x 8
  constexpr int XLD = 4;                // x loads per wave and step (BM rows / 8 / NWV)
  constexpr int WLD = 2 * NI / WM;      // w loads per wave and step (4 NI per step / NWV)
  constexpr int OPS = XLD + WLD;        // loads every thread issues per step (waves 0, 1: + 1)
  constexpr int WB = WF == GW_INT4 ? 16 * 256 : BN * GP_ROWB;      // w bytes per stage
  __shared__ __attribute__((aligned(1024))) uint8_t xl[NS][BM * GP_ROWB];
  __shared__ __attribute__((aligned(1024))) uint8_t wl[NS][WB];
  // bias slot: 64 lanes x 16 bytes land per load (lanes 16-63 repeat lane 15's chunk)
  __shared__ __attribute__((aligned(16))) half_t bsl[NS][512];
  // GW_INT4 scale slot: the 8 tiles' 16 scales of the step's group
  __shared__ __attribute__((aligned(16))) half_t ssl[NS][WF == GW_INT4 ? 128 : 2];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1;
  const int wm = wave >> 1;
  const int l16 = lane & 15;
  const int g4 = lane >> 4;

  const int tiles_n = a.N / BN;
  const int tiles_m = (a.M + BM - 1) / BM;
  const int tiles = tiles_m * tiles_n;
  const int items = tiles * a.KS;                        // slice-major: item = s tiles + tile
  const int G = gridDim.x;
  const int slot = xcd_logical_block(blockIdx.x, G);
  const int my_items = (items - slot + G - 1) / G;       // grid <= items: >= 1
  const int nk = a.K / GP_BKH;                           // every slice has >= NS steps (host check)

  // Load u of this wave fills tile rows 8 NWV u + 8 wave + lane / 8; lane i writes LDS
  // slot i % 8 of its row, which holds the row's chunk (i % 8) ^ (row & 7).
  const int lrow = 8 * wave + (lane >> 3);
  const int lchunk = (lane & 7) ^ (lrow & 7);
  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const bool has_bias = a.bias != nullptr;
  auto tile_src = [&](int r, int& m0, int& n0, int& sl) {   // past the last item: the last one again
    const int it = min(r, my_items - 1) * G + slot;
    sl = it / tiles;
    int tm, tn;
    grouped_tile(it - sl * tiles, tiles_m, tiles_n, GP_GM, tm, tn);
    m0 = tm * BM;
    n0 = tn * BN;
    // slices are whole 128-k groups (pairs of steps): the main loop takes two steps at a
    // time, and an int4 step's scales are its group's
    const int kb = 2 * (sl * (nk / 2) / a.KS);
    const int ke = 2 * ((sl + 1) * (nk / 2) / a.KS);
    GpTileSrc t;
    t.kb = kb;
    t.kc = ke - kb;
#pragma unroll
    for (int u = 0; u < XLD; ++u)
      t.x[u] = a.x + (int64_t)min(m0 + 8 * NWV * u + lrow, a.M - 1) * a.ldx + kb * GP_BKH + lchunk * 8;
    if constexpr (WF == GW_ROWS) {
      t.w = a.w + (int64_t)(n0 + lrow) * a.ldw + kb * GP_BKH + lchunk * 8;
    } else if constexpr (WF == GW_F16) {
      // load u of this wave moves block b = NWV u + wave: column tile b / 2, 32-k block b % 2
#pragma unroll
      for (int u = 0; u < WLD; ++u) {
        const int b = NWV * u + wave;
        t.wp[u] = a.w + (((int64_t)(n0 / 16 + b / 2) * (a.K / 32) + 2 * kb + (b & 1)) * 64 + lane) * 8;
      }
    } else {
      // load u moves word (step parity) b % 2 of column tile b / 2's block, 4 bytes a lane
#pragma unroll
      for (int u = 0; u < WLD; ++u) {
        const int b = NWV * u + wave;
        t.wp[u] = a.wq + ((int64_t)(n0 / 16 + b / 2) * (a.K / 128) * 64 + lane) * 4 + (b & 1);
      }
      // lane i: scales 2 (i % 8), +1 of column tile i / 8
      t.sp = a.wsc + (int64_t)(n0 / 16 + lane / 8) * (a.K / 128) * 16 + 2 * (lane & 7);
    }
    t.b = has_bias ? a.bias + n0 + 8 * min(lane, BN / 8 - 1) : a.x;
    return t;
  };
  const int64_t wstep = (int64_t)8 * NWV * a.ldw;       // halfs between w row groups
  auto issue = [&](const GpTileSrc& t, int ks, int st) {
    const int k0 = ks * GP_BKH;
#pragma unroll
    for (int u = 0; u < XLD; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(t.x[u] + k0),
                                       (lds_void*)((lds_u8*)&xl[st][(8 * NWV * u + 8 * wave) * GP_ROWB]), 16, 0, 0);
    if constexpr (WF == GW_ROWS) {
#pragma unroll
      for (int u = 0; u < WLD; ++u)
        __builtin_amdgcn_global_load_lds((const void*)(t.w + u * wstep + k0),
                                         (lds_void*)((lds_u8*)&wl[st][(8 * NWV * u + 8 * wave) * GP_ROWB]), 16, 0, 0);
    } else if constexpr (WF == GW_F16) {
#pragma unroll
      for (int u = 0; u < WLD; ++u)     // two 1 KB blocks per tile and step
        __builtin_amdgcn_global_load_lds((const void*)((const half_t*)t.wp[u] + ks * 1024),
                                         (lds_void*)((lds_u8*)&wl[st][(NWV * u + wave) * 1024]), 16, 0, 0);
    } else {
      const int S = t.kb + ks;          // absolute step: group S / 2, words 2 (S % 2) + 0/1
      const int64_t woff = (int64_t)(S >> 1) * 256 + 2 * (S & 1);
#pragma unroll
      for (int u = 0; u < WLD; ++u)
        __builtin_amdgcn_global_load_lds((const void*)((const uint32_t*)t.wp[u] + woff),
                                         (lds_void*)((lds_u8*)&wl[st][(NWV * u + wave) * 256]), 4, 0, 0);
      if (wave == 1)                    // the 8 tiles' scales of the group
        __builtin_amdgcn_global_load_lds((const void*)(t.sp + (int64_t)(S >> 1) * 16),
                                         (lds_void*)((lds_u8*)&ssl[st][0]), 4, 0, 0);
    }
    if (wave == 0 && has_bias)        // the tile's 128 biases (lanes 0-15 carry them)
      __builtin_amdgcn_global_load_lds((const void*)t.b, (lds_void*)((lds_u8*)&bsl[st][0]), 16, 0, 0);
  };
  // Operand reads are inline asm with their own lgkmcnt wait: as plain loads the compiler
  // would make each wait for every outstanding global->LDS load (vmcnt(0)).  A step's
  // slot is complete by the vmcnt wait and barrier before it is read.
  // LDS byte addresses of the lane's operand fragments, as bases plus the immediate
  // offsets of the reads.  Row-major tiles (x, and GW_ROWS w): fragment (i, t) holds k =
  // 32 t + 8 g4 .. +7 of tile row base + 16 i + l16, at chunk (4 t + g4) ^ (row & 7) of the
  // row; 16 i leaves row & 7 = l16 & 7, so sub-tiles i sit 16 rows = 2 KB apart from one
  // base per t.  Packed w: block (tile 4 wn + i, half t) at (2 (4 wn + i) + t) 1 KB (fp16)
  // or 256 B (int4 planes), the lane's bytes at 16 lane or 4 lane.
  auto row_bases = [&](const uint8_t* tile, int base, uint32_t (&b)[2]) {
    const int r = base + l16;
    const uint32_t row = (uint32_t)(uintptr_t)(lds_u8*)(tile + r * GP_ROWB);
    b[0] = row + ((g4 ^ (r & 7)) << 4);
    b[1] = row + (((4 + g4) ^ (r & 7)) << 4);
  };
  auto packed_base = [&](int st) -> uint32_t {
    return (uint32_t)(uintptr_t)(lds_u8*)&wl[st][0] + (uint32_t)(2 * NI * wn) * (WF == GW_INT4 ? 256u : 1024u) +
           (uint32_t)lane * (WF == GW_INT4 ? 4u : 16u);
  };
  auto read_issue = [&](int st, u32x4 (&v)[NV]) {
    uint32_t bx[2];
    row_bases(&xl[st][0], 64 * wm, bx);
    if constexpr (WF == GW_ROWS) {
      uint32_t bw[2];
      row_bases(&wl[st][0], 64 * wn, bw);
      asm volatile(
        "ds_read_b128 %0, %16 offset:0\n\t"
        "ds_read_b128 %1, %17 offset:0\n\t"
        "ds_read_b128 %2, %16 offset:2048\n\t"
        "ds_read_b128 %3, %17 offset:2048\n\t"
        "ds_read_b128 %4, %16 offset:4096\n\t"
        "ds_read_b128 %5, %17 offset:4096\n\t"
        "ds_read_b128 %6, %16 offset:6144\n\t"
        "ds_read_b128 %7, %17 offset:6144\n\t"
        "ds_read_b128 %8, %18 offset:0\n\t"
        "ds_read_b128 %9, %19 offset:0\n\t"
        "ds_read_b128 %10, %18 offset:2048\n\t"
        "ds_read_b128 %11, %19 offset:2048\n\t"
        "ds_read_b128 %12, %18 offset:4096\n\t"
        "ds_read_b128 %13, %19 offset:4096\n\t"
        "ds_read_b128 %14, %18 offset:6144\n\t"
        "ds_read_b128 %15, %19 offset:6144"
          : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
          : "v"(bw[0]), "v"(bw[1]), "v"(bx[0]), "v"(bx[1])
          : "memory");
    } else if constexpr (NI == 4) {
      const uint32_t bw = packed_base(st);
      asm volatile(
        "ds_read_b128 %0, %16 offset:0\n\t"
        "ds_read_b128 %1, %16 offset:1024\n\t"
        "ds_read_b128 %2, %16 offset:2048\n\t"
        "ds_read_b128 %3, %16 offset:3072\n\t"
        "ds_read_b128 %4, %16 offset:4096\n\t"
        "ds_read_b128 %5, %16 offset:5120\n\t"
        "ds_read_b128 %6, %16 offset:6144\n\t"
        "ds_read_b128 %7, %16 offset:7168\n\t"
        "ds_read_b128 %8, %17 offset:0\n\t"
        "ds_read_b128 %9, %18 offset:0\n\t"
        "ds_read_b128 %10, %17 offset:2048\n\t"
        "ds_read_b128 %11, %18 offset:2048\n\t"
        "ds_read_b128 %12, %17 offset:4096\n\t"
        "ds_read_b128 %13, %18 offset:4096\n\t"
        "ds_read_b128 %14, %17 offset:6144\n\t"
        "ds_read_b128 %15, %18 offset:6144"
          : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
          : "v"(bw), "v"(bx[0]), "v"(bx[1])
          : "memory");
    } else {
      // 192-column tiles: the wave's 6 column tiles x 2 halves, then x
      const uint32_t bw = packed_base(st);
      asm volatile(
        "ds_read_b128 %0, %20 offset:0\n\t"
        "ds_read_b128 %1, %20 offset:1024\n\t"
        "ds_read_b128 %2, %20 offset:2048\n\t"
        "ds_read_b128 %3, %20 offset:3072\n\t"
        "ds_read_b128 %4, %20 offset:4096\n\t"
        "ds_read_b128 %5, %20 offset:5120\n\t"
        "ds_read_b128 %6, %20 offset:6144\n\t"
        "ds_read_b128 %7, %20 offset:7168\n\t"
        "ds_read_b128 %8, %20 offset:8192\n\t"
        "ds_read_b128 %9, %20 offset:9216\n\t"
        "ds_read_b128 %10, %20 offset:10240\n\t"
        "ds_read_b128 %11, %20 offset:11264\n\t"
        "ds_read_b128 %12, %21 offset:0\n\t"
        "ds_read_b128 %13, %22 offset:0\n\t"
        "ds_read_b128 %14, %21 offset:2048\n\t"
        "ds_read_b128 %15, %22 offset:2048\n\t"
        "ds_read_b128 %16, %21 offset:4096\n\t"
        "ds_read_b128 %17, %22 offset:4096\n\t"
        "ds_read_b128 %18, %21 offset:6144\n\t"
        "ds_read_b128 %19, %22 offset:6144"
          : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15]), "=&v"(v[16]), "=&v"(v[17]), "=&v"(v[18]), "=&v"(v[19])
          : "v"(bw), "v"(bx[0]), "v"(bx[1])
          : "memory");
    }
  };
  // GW_INT4: the 8 x fragments (b128), the 8 step words of the wave's 4 tiles (b32) and
  // their 4 column scales (u16)
  auto read_issue_q = [&](int st, u32x4 (&v)[NV], uint32_t (&wd)[8], uint32_t (&sc)[4]) {
    uint32_t bx[2];
    row_bases(&xl[st][0], 64 * wm, bx);
    const uint32_t bw = packed_base(st);
    typedef __attribute__((address_space(3))) half_t lds_f16;
    const uint32_t bs = (uint32_t)(uintptr_t)(lds_f16*)&ssl[st][64 * wn + l16];
    asm volatile(
        "ds_read_b128 %0, %8 offset:0\n\t"
        "ds_read_b128 %1, %9 offset:0\n\t"
        "ds_read_b128 %2, %8 offset:2048\n\t"
        "ds_read_b128 %3, %9 offset:2048\n\t"
        "ds_read_b128 %4, %8 offset:4096\n\t"
        "ds_read_b128 %5, %9 offset:4096\n\t"
        "ds_read_b128 %6, %8 offset:6144\n\t"
        "ds_read_b128 %7, %9 offset:6144"
        : "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
        : "v"(bx[0]), "v"(bx[1])
        : "memory");
    asm volatile(
        "ds_read_b32 %0, %8 offset:0\n\t"
        "ds_read_b32 %1, %8 offset:256\n\t"
        "ds_read_b32 %2, %8 offset:512\n\t"
        "ds_read_b32 %3, %8 offset:768\n\t"
        "ds_read_b32 %4, %8 offset:1024\n\t"
        "ds_read_b32 %5, %8 offset:1280\n\t"
        "ds_read_b32 %6, %8 offset:1536\n\t"
        "ds_read_b32 %7, %8 offset:1792"
        : "=&v"(wd[0]), "=&v"(wd[1]), "=&v"(wd[2]), "=&v"(wd[3]), "=&v"(wd[4]), "=&v"(wd[5]), "=&v"(wd[6]), "=&v"(wd[7])
        : "v"(bw)
        : "memory");
    asm volatile(
        "ds_read_u16 %0, %4 offset:0\n\t"
        "ds_read_u16 %1, %4 offset:32\n\t"
        "ds_read_u16 %2, %4 offset:64\n\t"
        "ds_read_u16 %3, %4 offset:96"
        : "=&v"(sc[0]), "=&v"(sc[1]), "=&v"(sc[2]), "=&v"(sc[3])
        : "v"(bs)
        : "memory");
  };
  auto read_wait_q = [&](u32x4 (&v)[NV], uint32_t (&wd)[8], uint32_t (&sc)[4]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]), "+v"(v[12]), "+v"(v[13]),
                   "+v"(v[14]), "+v"(v[15]), "+v"(wd[0]), "+v"(wd[1]), "+v"(wd[2]), "+v"(wd[3]),
                   "+v"(wd[4]), "+v"(wd[5]), "+v"(wd[6]), "+v"(wd[7]), "+v"(sc[0]), "+v"(sc[1]),
                   "+v"(sc[2]), "+v"(sc[3])
                 :
                 : "memory");
  };
  auto read_wait = [&](u32x4 (&v)[NV]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]),
                   "+v"(v[12]), "+v"(v[13]), "+v"(v[14]), "+v"(v[15])
                 :
                 : "memory");
    if constexpr (NV > 16) asm volatile("" : "+v"(v[16]), "+v"(v[17]), "+v"(v[18]), "+v"(v[19]));
  };
  // the tile's biases of this lane's columns (4 per n sub-tile), read at the tile's last step
  uint2 bv[NI] = {};
  auto read_bias = [&](int st) {
    typedef __attribute__((address_space(3))) half_t lds_f16;
    uint32_t ab[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) ab[i] = (uint32_t)(uintptr_t)(lds_f16*)&bsl[st][16 * NI * wn + 16 * i + 4 * g4];
    if constexpr (NI == 4) {
      asm volatile(
          "ds_read_b64 %0, %4\n\tds_read_b64 %1, %5\n\tds_read_b64 %2, %6\n\tds_read_b64 %3, %7\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(bv[0]), "=&v"(bv[1]), "=&v"(bv[2]), "=&v"(bv[3])
          : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3])
          : "memory");
    } else {
      asm volatile(
          "ds_read_b64 %0, %6\n\tds_read_b64 %1, %7\n\tds_read_b64 %2, %8\n\t"
          "ds_read_b64 %3, %9\n\tds_read_b64 %4, %10\n\tds_read_b64 %5, %11\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(bv[0]), "=&v"(bv[1]), "=&v"(bv[2]), "=&v"(bv[3]), "=&v"(bv[4]), "=&v"(bv[5])
          : "v"(ab[0]), "v"(ab[1]), "v"(ab[2]), "v"(ab[3]), "v"(ab[4]), "v"(ab[5])
          : "memory");
    }
  };

  int m0c, n0c, m0n, n0n, slc, sln;
  GpTileSrc cur = tile_src(0, m0c, n0c, slc);
  GpTileSrc nxt = tile_src(1, m0n, n0n, sln);
#pragma unroll
  for (int s = 0; s < NS; ++s) issue(cur, s, s);
  gp_wait_vmcnt<OPS * (NS - 1)>();
  gp_barrier();
  // A step's operands: NV fragments (w 0 .. 2 NI - 1, then x) and, GW_INT4, the raw words
  // and scales
  struct Ops {
    u32x4 v[NV];
    uint32_t wd[8], sc[4];
  };
  auto rd_issue = [&](int st, Ops& o) {
    if constexpr (WF == GW_INT4) read_issue_q(st, o.v, o.wd, o.sc);
    else read_issue(st, o.v);
  };
  auto rd_wait = [&](Ops& o) {
    if constexpr (WF == GW_INT4) {
      read_wait_q(o.v, o.wd, o.sc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half_t sv = __builtin_bit_cast(half_t, (uint16_t)o.sc[i]);
        const half2_t s2 = {sv, sv};
#pragma unroll
        for (int t = 0; t < 2; ++t) o.v[2 * i + t] = __builtin_bit_cast(u32x4, dequant8(o.wd[2 * i + t], s2));
      }
    } else {
      read_wait(o.v);
    }
  };
  auto mfmas = [&](const Ops& o, f32x4 (&acc)[NI][4]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const half8_t wf = __builtin_bit_cast(half8_t, o.v[2 * i + t]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const half8_t xf = __builtin_bit_cast(half8_t, o.v[2 * NI + 2 * j + t]);
          acc[i][j] = mfma16x16x32(wf, xf, acc[i][j]);
        }
      }
  };
  // One step: its operands (read into `now`) are complete; once step sidx + 1 has landed
  // for this thread and then (barrier) for everyone - every wave has also finished reading
  // this step's slot - the slot is refilled with step sidx + NS and the next step's operand
  // reads go out into `later`, in flight while this step's MFMAs run.  Two register sets
  // alternate over the steps: every K slice is an even number of steps, so the sets' roles
  // are fixed at compile time within a two-step iteration, and the next tile's first step
  // (read ahead during the last MFMAs of a tile) is always in set A.
  auto step = [&](Ops& now, Ops& later, f32x4 (&acc)[NI][4], int ks, int kc, int sidx, bool last) {
    const int st = sidx % NS;
    rd_wait(now);
    if (last && has_bias) read_bias(st);
    gp_wait_vmcnt<OPS * (NS - 2)>();
    gp_barrier();
    const int iks = ks + NS;
    if (iks < kc) issue(cur, iks, st);
    else issue(nxt, iks - kc, st);
    rd_issue((sidx + 1) % NS, later);
    // the MFMAs' operands pass through an (empty) volatile asm after the reads: volatile
    // asm keeps its order, so the compiler cannot sink the reads below the MFMAs
    asm volatile(""
                 : "+v"(now.v[0]), "+v"(now.v[1]), "+v"(now.v[2]), "+v"(now.v[3]), "+v"(now.v[4]),
                   "+v"(now.v[5]), "+v"(now.v[6]), "+v"(now.v[7]), "+v"(now.v[8]), "+v"(now.v[9]),
                   "+v"(now.v[10]), "+v"(now.v[11]), "+v"(now.v[12]), "+v"(now.v[13]),
                   "+v"(now.v[14]), "+v"(now.v[15]));
    if constexpr (NV > 16)
      asm volatile("" : "+v"(now.v[16]), "+v"(now.v[17]), "+v"(now.v[18]), "+v"(now.v[19]));
    mfmas(now, acc);
  };
  Ops A, B;
  rd_issue(0, A);
  int sidx = 0;
  for (int r = 0; r < my_items; ++r) {
    const int kc = cur.kc;
    f32x4 acc[NI][4];   // [n sub-tile][m sub-tile]
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < kc; ks += 2, sidx += 2) {
      step(A, B, acc, ks, kc, sidx, false);
      step(B, A, acc, ks + 1, kc, sidx + 1, ks + 2 == kc);
    }
    // Epilogue: lane holds n = n0 + 16 NI wn + 16 i + 4 g4 + q of m = m0 + 64 wm + 16 j + l16.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0c + 64 * wm + 16 * j + l16;
      if (m >= a.M) continue;
      if (a.KS > 1 || EPI == GP_PARTIAL) {   // the slice's fp32 partial sums
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int n = n0c + 16 * NI * wn + 16 * i + 4 * g4;
          *(f32x4*)(a.part + ((int64_t)slc * a.M + m) * a.N + n) = acc[i][j];
        }
        continue;
      }
      if constexpr (EPI == GP_SILU) {
        // tiles (4 wn + i, 4 wn + i + 1), i even, are (gate, up) of intermediate columns
        // 16 ((n0 + 64 wn) / 32 + i / 2) + 4 g4 + q
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const int n = (n0c + 64 * wn + 16 * i) / 2 + 4 * g4;
          half4_t o;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            o[q] = (half_t)silu_mul_f32((float)(half_t)acc[i][j][q], (float)(half_t)acc[i + 1][j][q]);
          *(half4_t*)(a.out + (int64_t)m * a.ldo + n) = o;
        }
        continue;
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int n = n0c + 16 * NI * wn + 16 * i + 4 * g4;
        const half4_t bb = __builtin_bit_cast(half4_t, bv[i]);
        half4_t rr = (half4_t){0, 0, 0, 0};
        if constexpr (EPI == GP_RESID) rr = *(const half4_t*)(a.res + (int64_t)m * a.ldr + n);
        half4_t o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          half_t h = gp_bias(acc[i][j][q], bb[q], has_bias, a.bias_after_round);
          if constexpr (EPI == GP_QGELU) h = gp_quick_gelu(h);
          if constexpr (EPI == GP_GELU) h = gp_gelu(h);
          if constexpr (EPI == GP_RESID) h = (half_t)((float)rr[q] + (float)h);
          o[q] = h;
        }
        *(half4_t*)(a.out + (int64_t)m * a.ldo + n) = o;
      }
    }
    cur = nxt;
    m0c = m0n;
    n0c = n0n;
    slc = sln;
    nxt = tile_src(r + 2, m0n, n0n, sln);
  }
  gp_wait_vmcnt<0>();                  // drain the clamped tail loads before exit
}

// Persistent 256 x 256 or 256 x 192 tiles for the packed fp16 weights (STORE without a
// bias, SILU (256 columns) and PARTIAL epilogues, M a multiple of 256, N of the tile width):
// 8 waves (two per SIMD: 2 along m x 4 along n), each owning a 128 (m) x 16 NIW (n) block,
// so every operand byte staged through LDS feeds twice the MFMA work it feeds in the
// 256 x 128 tiles above; two stages of 32 KB of x and 8 NIW KB of w (x rows XOR-swizzled as
// above, w as the packed 1 KB blocks, one global_load_lds per lane); a grid of at most one
// workgroup per CU walks its items (tile x K slice, slice-major, tiles in the XCD-grouped
// order) with the K loop running across item boundaries (the next item's first two stages
// load during the current one's last two steps).  Per 64-k step a wave issues 16 + 2 NIW
// operand reads and 16 NIW MFMAs.  At 256 columns the columns past a.n_big run as 256 x 128
// half tiles after every whole tile (gp_big_tail_cols: the last round of whole tiles would
// leave CUs idle), read and stored by the same code for NIW / 2 column tiles per wave.
// PARTIAL writes each K slice's fp32 sums to part[slice][M][N] for the consumer to add in
// slice order (config 5's down projection at M = 4096: 128 tiles of 256 x 192 in two
// slices fill the 256 CUs once).  (Biased
// linears, e.g. qkv, stay on the kernel above: with the bias staging beside the
// accumulators a four-wave form of this kernel spilled.)  Same k order per output as the
// kernel above within a slice: one-slice results equal its bit for bit.  MI355X, us
// (256 x 128 or 128 x 192 / this, interleaved, median of 7): M = 4096 gate_up + SiLU
// 240.1 / 222.6; M = 8192 gate_up 469.7 / 397.5, down 238.6 / 200.2 (four waves of 128 x 128:
// 440.0 and 216.5).
// The wave's lane index computed afresh (v_mbcnt in an asm block, which the compiler can
// neither hoist nor merge with an earlier value): for addresses needed once per tile, so
// that neither they nor the lane index stay live beside 256 accumulators.
__device__ __forceinline__ uint32_t gp_lane_now() {
  uint32_t l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

template <int EPI, int NIW>
__global__ __launch_bounds__(512, 1) void gemm_bigp_f16_kernel(GemmPipeArgs a) {
#pragma clang fp contract(off)
  static_assert(((EPI == GP_STORE || EPI == GP_PARTIAL) && (NIW == 3 || NIW == 4)) ||
                    (EPI == GP_SILU && NIW == 4),
                "STORE / PARTIAL at 192 or 256 columns, SILU at 256");
  constexpr int NS = 2;
  constexpr int BM = 256;               // tile rows
  constexpr int BN = 64 * NIW;          // tile columns
  constexpr int XLD = 4;                // x loads per wave and stage (256 rows / 8 / 8)
  constexpr int WLD = NIW;              // w loads per wave and stage (8 NIW blocks / 8)
  constexpr int NV = 2 * NIW + 16;      // operand fragments per step: w 2 NIW, then x 16
  __shared__ __attribute__((aligned(1024))) uint8_t xl[NS][BM * GP_ROWB];
  __shared__ __attribute__((aligned(1024))) uint8_t wl[NS][BN * GP_ROWB];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 3;              // 4 waves along n (16 NIW columns each), 2 along m
  const int wm = wave >> 2;
  const int l16 = lane & 15;
  const int g4 = lane >> 4;

  const int tiles_n = a.n_big / BN;
  const int tiles_m = a.M / BM;
  const int tiles = tiles_m * tiles_n;
  const int items_big = tiles * a.KS;                       // slice-major: item = s tiles + tile
  // the columns past n_big in 256 x (BN / 2) half tiles, after every whole tile: a grid whose
  // whole tiles fill R rounds exactly then ends with at most half a tile per workgroup
  const int tiles_hn = NIW == 4 ? (a.N - a.n_big) / (BN / 2) : 0;
  const int items = items_big + tiles_m * tiles_hn;
  const int G = gridDim.x;
  const int slot = xcd_logical_block(blockIdx.x, G);
  const int my_items = (items - slot + G - 1) / G;          // grid <= items: >= 1
  const int nk = a.K / GP_BKH;                              // every slice >= NS steps (host check)
  struct Item {
    int m0, n0, sl, kb, kc;            // tile origin, K slice, its first step and step count
    int half;                          // a 256 x (BN / 2) tile past n_big
  };
  auto item_at = [&](int r) {                               // past the last item: the last one
    Item t;
    const int it = min(r, my_items - 1) * G + slot;
    int tm, tn;
    if (it < items_big) {
      t.sl = it / tiles;
      grouped_tile(it - t.sl * tiles, tiles_m, tiles_n, GP_GM, tm, tn);
      t.n0 = tn * BN;
      t.half = 0;
    } else {
      t.sl = 0;
      grouped_tile(it - items_big, tiles_m, tiles_hn, GP_GM, tm, tn);
      t.n0 = a.n_big + tn * (BN / 2);
      t.half = 1;
    }
    t.m0 = tm * BM;
    // slices are whole 128-k groups (pairs of steps), as in the kernel above
    t.kb = 2 * (t.sl * (nk / 2) / a.KS);
    t.kc = 2 * ((t.sl + 1) * (nk / 2) / a.KS) - t.kb;
    return t;
  };

  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  // Lane byte offsets from wave-uniform bases, recomputed at every issue from the lane index
  // (hoisted, the loads' lane offsets would stay live through the loops): x row 64 u + lrow
  // of the tile (lrow = 8 wave + lane / 8), its 16-byte chunk (lane % 8) ^ (lrow % 8) in LDS
  // slot lane % 8; w block b = 8 u + wave of the step (column tile b / 2, 32-k half b % 2),
  // 1 KB blocks, (K / 32) of them per column tile.  ks: the absolute K step.
  const uint32_t xstep = 64u * (uint32_t)a.ldx * 2u;
  const uint32_t kblk = (uint32_t)(a.K / 32) * 1024u;       // bytes per packed column tile
  auto issue = [&](int m0, int n0, int ks, int st, int half) {
    const uint8_t* const xs = (const uint8_t*)(a.x + (int64_t)m0 * a.ldx) + (uint32_t)ks * 128u;
    const uint8_t* const ws = (const uint8_t*)(a.w + (int64_t)(n0 / 16) * (a.K / 32) * 512) +
                              (uint32_t)ks * 2048u;
    const uint32_t ln = gp_lane_now();
    const uint32_t lrow = 8u * (uint32_t)wave + (ln >> 3);
    const uint32_t xoff = lrow * (uint32_t)a.ldx * 2u + (((ln & 7u) ^ (lrow & 7u)) << 4);
    const uint32_t lw = ln * 16u;
#pragma unroll
    for (int u = 0; u < XLD; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(xs + (xoff + u * xstep)),
                                       (lds_void*)((lds_u8*)&xl[st][(64 * u + 8 * wave) * GP_ROWB]), 16, 0, 0);
#pragma unroll
    for (int u = 0; u < WLD; ++u) {
      if (half && 2 * u >= WLD) break;   // a half tile's 4 NIW blocks
      const int b = 8 * u + wave;
      __builtin_amdgcn_global_load_lds(
          (const void*)(ws + ((uint32_t)(b >> 1) * kblk + (uint32_t)(b & 1) * 1024u + lw)),
          (lds_void*)((lds_u8*)&wl[st][b * 1024]), 16, 0, 0);
    }
  };
  // Operand reads: x fragment (j, t) = k 32 t + 8 g4 .. +7 of row 128 wm + 16 j + l16, at
  // chunk (4 t + g4) ^ (l16 & 7) of the row (16 j keeps row & 7 = l16 & 7): two bases (t)
  // plus 2 KB per j; w fragment (i, t) = the lane's 16 bytes of block 2 (NIW wn + i) + t.
  auto read_ops = [&](int st, u32x4 (&v)[NV], int half) {
    const int r = 128 * wm + l16;
    const uint32_t row = (uint32_t)(uintptr_t)(lds_u8*)&xl[st][r * GP_ROWB];
    const uint32_t bx0 = row + ((g4 ^ (l16 & 7)) << 4);
    const uint32_t bx1 = row + (((4 + g4) ^ (l16 & 7)) << 4);
    const uint32_t bw = (uint32_t)(uintptr_t)(lds_u8*)&wl[st][2 * NIW * wn * 1024] + (uint32_t)lane * 16u;
    if (NIW == 4 && half) {
      // a half tile: the wave's 2 column tiles (blocks 4 wn .. 4 wn + 3) into v[0..3]; x as below
      const uint32_t bh = (uint32_t)(uintptr_t)(lds_u8*)&wl[st][4 * wn * 1024] + (uint32_t)lane * 16u;
      asm volatile(
          "ds_read_b128 %0, %20\n\tds_read_b128 %1, %20 offset:1024\n\t"
          "ds_read_b128 %2, %20 offset:2048\n\tds_read_b128 %3, %20 offset:3072\n\t"
          "ds_read_b128 %4, %21\n\tds_read_b128 %5, %22\n\t"
          "ds_read_b128 %6, %21 offset:2048\n\tds_read_b128 %7, %22 offset:2048\n\t"
          "ds_read_b128 %8, %21 offset:4096\n\tds_read_b128 %9, %22 offset:4096\n\t"
          "ds_read_b128 %10, %21 offset:6144\n\tds_read_b128 %11, %22 offset:6144\n\t"
          "ds_read_b128 %12, %21 offset:8192\n\tds_read_b128 %13, %22 offset:8192\n\t"
          "ds_read_b128 %14, %21 offset:10240\n\tds_read_b128 %15, %22 offset:10240\n\t"
          "ds_read_b128 %16, %21 offset:12288\n\tds_read_b128 %17, %22 offset:12288\n\t"
          "ds_read_b128 %18, %21 offset:14336\n\tds_read_b128 %19, %22 offset:14336\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[2 * NIW]),
            "=&v"(v[2 * NIW + 1]), "=&v"(v[2 * NIW + 2]), "=&v"(v[2 * NIW + 3]), "=&v"(v[2 * NIW + 4]),
            "=&v"(v[2 * NIW + 5]), "=&v"(v[2 * NIW + 6]), "=&v"(v[2 * NIW + 7]), "=&v"(v[2 * NIW + 8]),
            "=&v"(v[2 * NIW + 9]), "=&v"(v[2 * NIW + 10]), "=&v"(v[2 * NIW + 11]),
            "=&v"(v[2 * NIW + 12]), "=&v"(v[2 * NIW + 13]), "=&v"(v[2 * NIW + 14]),
            "=&v"(v[2 * NIW + 15])
          : "v"(bh), "v"(bx0), "v"(bx1)
          : "memory");
      return;
    }
    if constexpr (NIW == 4) asm volatile(
        "ds_read_b128 %0, %24\n\tds_read_b128 %1, %24 offset:1024\n\t"
        "ds_read_b128 %2, %24 offset:2048\n\tds_read_b128 %3, %24 offset:3072\n\t"
        "ds_read_b128 %4, %24 offset:4096\n\tds_read_b128 %5, %24 offset:5120\n\t"
        "ds_read_b128 %6, %24 offset:6144\n\tds_read_b128 %7, %24 offset:7168\n\t"
        "ds_read_b128 %8, %25\n\tds_read_b128 %9, %26\n\t"
        "ds_read_b128 %10, %25 offset:2048\n\tds_read_b128 %11, %26 offset:2048\n\t"
        "ds_read_b128 %12, %25 offset:4096\n\tds_read_b128 %13, %26 offset:4096\n\t"
        "ds_read_b128 %14, %25 offset:6144\n\tds_read_b128 %15, %26 offset:6144\n\t"
        "ds_read_b128 %16, %25 offset:8192\n\tds_read_b128 %17, %26 offset:8192\n\t"
        "ds_read_b128 %18, %25 offset:10240\n\tds_read_b128 %19, %26 offset:10240\n\t"
        "ds_read_b128 %20, %25 offset:12288\n\tds_read_b128 %21, %26 offset:12288\n\t"
        "ds_read_b128 %22, %25 offset:14336\n\tds_read_b128 %23, %26 offset:14336\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
          "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
          "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15]), "=&v"(v[16]), "=&v"(v[17]),
          "=&v"(v[18]), "=&v"(v[19]), "=&v"(v[20]), "=&v"(v[21]), "=&v"(v[22]), "=&v"(v[23])
        : "v"(bw), "v"(bx0), "v"(bx1)
        : "memory");
    else asm volatile(
        "ds_read_b128 %0, %22\n\tds_read_b128 %1, %22 offset:1024\n\t"
        "ds_read_b128 %2, %22 offset:2048\n\tds_read_b128 %3, %22 offset:3072\n\t"
        "ds_read_b128 %4, %22 offset:4096\n\tds_read_b128 %5, %22 offset:5120\n\t"
        "ds_read_b128 %6, %23\n\tds_read_b128 %7, %24\n\t"
        "ds_read_b128 %8, %23 offset:2048\n\tds_read_b128 %9, %24 offset:2048\n\t"
        "ds_read_b128 %10, %23 offset:4096\n\tds_read_b128 %11, %24 offset:4096\n\t"
        "ds_read_b128 %12, %23 offset:6144\n\tds_read_b128 %13, %24 offset:6144\n\t"
        "ds_read_b128 %14, %23 offset:8192\n\tds_read_b128 %15, %24 offset:8192\n\t"
        "ds_read_b128 %16, %23 offset:10240\n\tds_read_b128 %17, %24 offset:10240\n\t"
        "ds_read_b128 %18, %23 offset:12288\n\tds_read_b128 %19, %24 offset:12288\n\t"
        "ds_read_b128 %20, %23 offset:14336\n\tds_read_b128 %21, %24 offset:14336\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
          "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
          "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15]), "=&v"(v[16]), "=&v"(v[17]),
          "=&v"(v[18]), "=&v"(v[19]), "=&v"(v[20]), "=&v"(v[21])
        : "v"(bw), "v"(bx0), "v"(bx1)
        : "memory");
  };
  Item cur = item_at(0), nxt = item_at(1);
  issue(cur.m0, cur.n0, cur.kb, 0, cur.half);
  issue(cur.m0, cur.n0, cur.kb + 1, 1, cur.half);
  gp_wait_vmcnt<XLD + WLD>();           // stage 0
  gp_barrier();
  int sidx = 0;
  for (int r = 0; r < my_items; ++r) {
    f32x4 acc[NIW][8];   // [n sub-tile][m sub-tile]
#pragma unroll
    for (int i = 0; i < NIW; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < cur.kc; ++ks, ++sidx) {
      const int st = sidx & 1;
      u32x4 v[NV];
      read_ops(st, v, cur.half);
      // step sidx + 1 has landed (nothing younger is in flight with two stages) for this
      // thread, then for everyone; every wave has read this slot, refilled with sidx + 2
      gp_wait_vmcnt<0>();
      gp_barrier();
      {
        const int iks = ks + NS;
        if (iks < cur.kc) issue(cur.m0, cur.n0, cur.kb + iks, st, cur.half);
        else issue(nxt.m0, nxt.n0, nxt.kb + iks - cur.kc, st, nxt.half);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < NIW; ++i) {
          if (cur.half && 2 * i >= NIW) break;   // a half tile's NIW / 2 column tiles
          const half8_t wf = __builtin_bit_cast(half8_t, v[2 * i + t]);
#pragma unroll
          for (int j = 0; j < 8; ++j)
            acc[i][j] = mfma16x16x32(wf, __builtin_bit_cast(half8_t, v[2 * NIW + 2 * j + t]), acc[i][j]);
        }
    }
    // Epilogue: lane holds n = n0 + 16 NIW wn + 16 i + 4 g4 + q of m = m0 + 128 wm + 16 j + l16.
    {
      const uint32_t ln = gp_lane_now();
      // the wave's first column: 16 NIW wn of a whole tile, 8 NIW wn of a half tile
      const int wc = cur.n0 + (cur.half ? 8 : 16) * NIW * wn;
      const int ni = cur.half ? NIW / 2 : NIW;
      if constexpr (EPI == GP_PARTIAL) {
        const uint32_t lp = (ln & 15u) * (uint32_t)a.N + 4u * (ln >> 4);
        float* const pb = a.part + ((int64_t)cur.sl * a.M + cur.m0 + 128 * wm) * a.N + wc + lp;
#pragma unroll
        for (int i = 0; i < NIW; ++i) {
          if (i >= ni) break;
#pragma unroll
          for (int j = 0; j < 8; ++j) *(f32x4*)(pb + ((int64_t)16 * j * a.N + 16 * i)) = acc[i][j];
        }
      }
      const int64_t mrow = (int64_t)(cur.m0 + 128 * wm) * a.ldo;
      const uint32_t lo = (ln & 15u) * (uint32_t)a.ldo + 4u * (ln >> 4);
      if constexpr (EPI == GP_SILU) {
        // column tiles (i, i + 1), i even, are (gate, up) of intermediate columns
        // (wc + 16 i) / 2 + 4 g4 + q
        half_t* const ob = a.out + mrow + wc / 2 + lo;
        auto pair = [&](f32x4 (&g)[8], f32x4 (&u)[8], int c) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            half4_t o;
#pragma unroll
            for (int q = 0; q < 4; ++q)
              o[q] = (half_t)silu_mul_f32((float)(half_t)g[j][q], (float)(half_t)u[j][q]);
            *(half4_t*)(ob + (16 * j * a.ldo + c)) = o;
          }
        };
        pair(acc[0], acc[1], 0);
        if (!cur.half) pair(acc[2], acc[3], 16);
      } else if constexpr (EPI == GP_STORE) {
        half_t* const ob = a.out + mrow + wc + lo;
#pragma unroll
        for (int i = 0; i < NIW; ++i) {
          if (i >= ni) break;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            half4_t o;
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = (half_t)acc[i][j][q];
            *(half4_t*)(ob + (16 * j * a.ldo + 16 * i)) = o;
          }
        }
      }
    }
    cur = nxt;
    nxt = item_at(r + 2);
  }
  gp_wait_vmcnt<0>();                   // drain the clamped tail loads before exit
}

// 128 x 160 tiles on the packed fp16 weights, one tile per workgroup, where they fill the
// CUs in one round and the 128- / 256-row x 128 tiles would not: the SiLU-fused gate_up at
// 129-256 rows (five gate|up column pairs; config 1's 256-token prompt, N = 17920: 224 tiles
// where 256 x 128 tiles fill 140 CUs and 128 x 128 ones take two rounds) and the STORE /
// QGELU / GELU / RESID epilogues with a bias (the vision tower's fc1, 1024 x 1280 -> 5120:
// 256 tiles where 256 x 128 ones fill 160 CUs).  A step stages 16 KB of x and 20 KB of w (36
// KB per CU against 48 KB for a 256 x 128 tile; at these sizes a step's time follows the
// bytes it stages).  8 waves, two per SIMD: 4 along m (32 rows each) x 2 along n - for SILU
// the first n group holds pairs 0-2 (column tiles 0-5) and the second pairs 3-4 (tiles 6-9),
// otherwise five column tiles each - so that every SIMD holds one wave of each group.  Per
// 64-k step a wave reads 4 x fragments and 8-12 w fragments and issues 16-24 MFMAs; the K
// order of every output is the 128-column tiles' (steps ascending, each step's two 32-k
// halves in order) and the epilogues are theirs, so the outputs equal theirs bit for bit.  w
// blocks: 20 per step, three loads each for waves 0-3 and two for waves 4-7.
template <int NS, int EPI>
__global__ __launch_bounds__(512, 1) void gemm_n160_kernel(GemmPipeArgs a) {
#pragma clang fp contract(off)
  constexpr int BM = 128, BN = 160;
  constexpr int NCT = BN / 16;          // column tiles
  constexpr int XLD = 2;                // x loads per wave and step (128 rows / 8 / 8)
  constexpr bool SILU = EPI == GP_SILU;
  __shared__ __attribute__((aligned(1024))) uint8_t xl[NS][BM * GP_ROWB];
  __shared__ __attribute__((aligned(1024))) uint8_t wl[NS][2 * NCT * 1024];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 3;
  const int wn = wave >> 2;
  const int ct0 = SILU ? 6 * wn : 5 * wn;       // the wave's first column tile
  const int ncw = SILU ? (wn ? 4 : 6) : 5;      // and its column tiles
  const int l16 = lane & 15;
  const int g4 = lane >> 4;
  const int tiles_m = (a.M + BM - 1) / BM;
  // tiles sharing a column range (the same weights) sit on the same XCD
  const int t = xcd_logical_block(blockIdx.x, gridDim.x);
  const int m0 = (t % tiles_m) * BM;
  const int n0 = (t / tiles_m) * BN;
  const int nk = a.K / GP_BKH;          // >= NS (host check)

  typedef __attribute__((address_space(3))) void lds_void;
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  const int lrow = 8 * wave + (lane >> 3);
  const int lchunk = (lane & 7) ^ (lrow & 7);
  const half_t* xs[XLD];
#pragma unroll
  for (int u = 0; u < XLD; ++u)
    xs[u] = a.x + (int64_t)min(m0 + 64 * u + lrow, a.M - 1) * a.ldx + lchunk * 8;
  // w block b = 8 u + wave (u < 3 for waves 0-3, u < 2 for 4-7): column tile b / 2, 32-k half b % 2
  const half_t* ws[3];
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int b = min(8 * u + wave, 2 * NCT - 1);
    ws[u] = a.w + (((int64_t)(n0 / 16 + b / 2) * (a.K / 32) + (b & 1)) * 64 + lane) * 8;
  }
  auto issue = [&](int ks, int st) {
#pragma unroll
    for (int u = 0; u < XLD; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(xs[u] + ks * GP_BKH),
                                       (lds_void*)((lds_u8*)&xl[st][(64 * u + 8 * wave) * GP_ROWB]), 16, 0, 0);
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      if (u == 2 && wave >= 4) break;
      __builtin_amdgcn_global_load_lds((const void*)(ws[u] + ks * 1024),
                                       (lds_void*)((lds_u8*)&wl[st][(8 * u + wave) * 1024]), 16, 0, 0);
    }
  };
  // operands: w fragments (column tile c of the wave, half t) in v[2 c + t], x (row
  // sub-tile j, half t) in v[12 + 2 j + t]
  auto read_ops = [&](int st, u32x4 (&v)[16]) {
    const int r = 32 * wm + l16;
    const uint32_t row = (uint32_t)(uintptr_t)(lds_u8*)&xl[st][r * GP_ROWB];
    const uint32_t bx0 = row + ((g4 ^ (l16 & 7)) << 4);
    const uint32_t bx1 = row + (((4 + g4) ^ (l16 & 7)) << 4);
    const uint32_t bw = (uint32_t)(uintptr_t)(lds_u8*)&wl[st][2 * ct0 * 1024] + (uint32_t)lane * 16u;
    if (ncw == 6)
      asm volatile(
          "ds_read_b128 %0, %16\n\tds_read_b128 %1, %16 offset:1024\n\t"
          "ds_read_b128 %2, %16 offset:2048\n\tds_read_b128 %3, %16 offset:3072\n\t"
          "ds_read_b128 %4, %16 offset:4096\n\tds_read_b128 %5, %16 offset:5120\n\t"
          "ds_read_b128 %6, %16 offset:6144\n\tds_read_b128 %7, %16 offset:7168\n\t"
          "ds_read_b128 %8, %16 offset:8192\n\tds_read_b128 %9, %16 offset:9216\n\t"
          "ds_read_b128 %10, %16 offset:10240\n\tds_read_b128 %11, %16 offset:11264\n\t"
          "ds_read_b128 %12, %17\n\tds_read_b128 %13, %18\n\t"
          "ds_read_b128 %14, %17 offset:2048\n\tds_read_b128 %15, %18 offset:2048\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
            "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
            "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
          : "v"(bw), "v"(bx0), "v"(bx1)
          : "memory");
    else if (ncw == 5)
      asm volatile(
          "ds_read_b128 %0, %14\n\tds_read_b128 %1, %14 offset:1024\n\t"
          "ds_read_b128 %2, %14 offset:2048\n\tds_read_b128 %3, %14 offset:3072\n\t"
          "ds_read_b128 %4, %14 offset:4096\n\tds_read_b128 %5, %14 offset:5120\n\t"
          "ds_read_b128 %6, %14 offset:6144\n\tds_read_b128 %7, %14 offset:7168\n\t"
          "ds_read_b128 %8, %14 offset:8192\n\tds_read_b128 %9, %14 offset:9216\n\t"
          "ds_read_b128 %10, %15\n\tds_read_b128 %11, %16\n\t"
          "ds_read_b128 %12, %15 offset:2048\n\tds_read_b128 %13, %16 offset:2048\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
            "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[12]), "=&v"(v[13]),
            "=&v"(v[14]), "=&v"(v[15])
          : "v"(bw), "v"(bx0), "v"(bx1)
          : "memory");
    else
      asm volatile(
          "ds_read_b128 %0, %12\n\tds_read_b128 %1, %12 offset:1024\n\t"
          "ds_read_b128 %2, %12 offset:2048\n\tds_read_b128 %3, %12 offset:3072\n\t"
          "ds_read_b128 %4, %12 offset:4096\n\tds_read_b128 %5, %12 offset:5120\n\t"
          "ds_read_b128 %6, %12 offset:6144\n\tds_read_b128 %7, %12 offset:7168\n\t"
          "ds_read_b128 %8, %13\n\tds_read_b128 %9, %14\n\t"
          "ds_read_b128 %10, %13 offset:2048\n\tds_read_b128 %11, %14 offset:2048\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
            "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
          : "v"(bw), "v"(bx0), "v"(bx1)
          : "memory");
  };
  f32x4 acc[6][2];
#pragma unroll
  for (int c = 0; c < 6; ++c)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[c][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NS; ++s) issue(s, s);
  // a thread's loads per stage: 5 for waves 0-3, 4 for waves 4-7; stage 0 landed
  if (wave < 4) gp_wait_vmcnt<5 * (NS - 1)>();
  else gp_wait_vmcnt<4 * (NS - 1)>();
  gp_barrier();
  for (int ks = 0; ks < nk; ++ks) {
    const int st = ks % NS;
    u32x4 v[16];
    read_ops(st, v);
    // step ks + 1 has landed for this thread, then for everyone; every wave has read this
    // slot, refilled with step ks + NS (past the end: the last step again, never read)
    if (wave < 4) gp_wait_vmcnt<5 * (NS - 2)>();
    else gp_wait_vmcnt<4 * (NS - 2)>();
    gp_barrier();
    issue(min(ks + NS, nk - 1), st);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int c = 0; c < 6; ++c) {
        if (c >= ncw) break;
        const half8_t wf = __builtin_bit_cast(half8_t, v[2 * c + h]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[c][j] = mfma16x16x32(wf, __builtin_bit_cast(half8_t, v[12 + 2 * j + h]), acc[c][j]);
      }
  }
  gp_wait_vmcnt<0>();                   // drain the clamped tail loads
  // lane holds columns 16 (ct0 + c) + 4 g4 + q of the tile, rows m0 + 32 wm + 16 j + l16
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = m0 + 32 * wm + 16 * j + l16;
    if (m >= a.M) continue;
    if constexpr (SILU) {
      // pair p of the wave (column tiles 2 p, 2 p + 1) is intermediate pair n0 / 32 + 3 wn + p
      half_t* const ob = a.out + (int64_t)m * a.ldo + n0 / 2 + 48 * wn + 4 * g4;
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        if (2 * p >= ncw) break;
        half4_t o;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          o[q] = (half_t)silu_mul_f32((float)(half_t)acc[2 * p][j][q], (float)(half_t)acc[2 * p + 1][j][q]);
        *(half4_t*)(ob + 16 * p) = o;
      }
    } else {
#pragma unroll
      for (int c = 0; c < 5; ++c) {
        const int n = n0 + 16 * (ct0 + c) + 4 * g4;
        half4_t bb = (half4_t){0, 0, 0, 0};
        if (a.bias) bb = *(const half4_t*)(a.bias + n);
        half4_t rr = (half4_t){0, 0, 0, 0};
        if constexpr (EPI == GP_RESID) rr = *(const half4_t*)(a.res + (int64_t)m * a.ldr + n);
        half4_t o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          half_t hv = gp_bias(acc[c][j][q], bb[q], a.bias != nullptr, a.bias_after_round);
          if constexpr (EPI == GP_QGELU) hv = gp_quick_gelu(hv);
          if constexpr (EPI == GP_GELU) hv = gp_gelu(hv);
          if constexpr (EPI == GP_RESID) hv = (half_t)((float)rr[q] + (float)hv);
          o[q] = hv;
        }
        *(half4_t*)(a.out + (int64_t)m * a.ldo + n) = o;
      }
    }
  }
}

static int gp_num_cus() {
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

// Split-K finish: out = epi(fp16(sum_s part[s] + bias)), slices summed in order; one
// thread per 4 consecutive columns.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_pipe_finish_kernel(GemmPipeArgs a) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nq = a.N >> 2;
  if (i >= (int64_t)a.M * nq) return;
  const int m = (int)(i / nq), n = (int)(i - (int64_t)m * nq) * 4;
  f32x4 v = *(const f32x4*)(a.part + (int64_t)m * a.N + n);
  for (int s = 1; s < a.KS; ++s) {
    const f32x4 p = *(const f32x4*)(a.part + ((int64_t)s * a.M + m) * a.N + n);
    v = (f32x4){v[0] + p[0], v[1] + p[1], v[2] + p[2], v[3] + p[3]};
  }
  half4_t bb = (half4_t){0, 0, 0, 0};
  if (a.bias) bb = *(const half4_t*)(a.bias + n);
  half4_t rr = (half4_t){0, 0, 0, 0};
  if constexpr (EPI == GP_RESID) rr = *(const half4_t*)(a.res + (int64_t)m * a.ldr + n);
  half4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    half_t h = gp_bias(v[q], bb[q], a.bias != nullptr, a.bias_after_round);
    if constexpr (EPI == GP_QGELU) h = gp_quick_gelu(h);
    if constexpr (EPI == GP_GELU) h = gp_gelu(h);
    if constexpr (EPI == GP_RESID) h = (half_t)((float)rr[q] + (float)h);
    o[q] = h;
  }
  *(half4_t*)(a.out + (int64_t)m * a.ldo + n) = o;
}

template <int WF, int WM, int NS, int NI = 4>
static int gp_launch(const GemmPipeArgs& a, int epilogue, hipStream_t st) {
  const int64_t items = (int64_t)ceil_div(a.M, 64 * WM) * (a.N / (32 * NI)) * a.KS;
  if (items > 0x7fffffff) return OMNI_EUNSUPPORTED;
  const int grid = (int)(items < gp_num_cus() ? items : gp_num_cus());
  const dim3 blk(128 * WM);
  if (epilogue == GP_PARTIAL) {      // the slices' partial sums only, for a consumer to add
    if constexpr (WF == GW_ROWS) return OMNI_EINVAL;
    else hipLaunchKernelGGL((gemm_pipe_kernel<WF, WM, NS, GP_PARTIAL, NI>), dim3(grid), blk, 0, st, a);
    OMNI_CHECK_LAUNCH();
    return OMNI_OK;
  }
  if (a.KS > 1) {                    // partial sums, then the finish kernel's epilogue
    if (epilogue == GP_SILU) return OMNI_EINVAL;
    hipLaunchKernelGGL((gemm_pipe_kernel<WF, WM, NS, GP_STORE, NI>), dim3(grid), blk, 0, st, a);
    OMNI_CHECK_LAUNCH();
    const int64_t nthr = (int64_t)a.M * (a.N / 4);
    const dim3 fg((unsigned)((nthr + 255) / 256));
    switch (epilogue) {
      case GP_STORE: hipLaunchKernelGGL((gemm_pipe_finish_kernel<GP_STORE>), fg, dim3(256), 0, st, a); break;
      case GP_QGELU: hipLaunchKernelGGL((gemm_pipe_finish_kernel<GP_QGELU>), fg, dim3(256), 0, st, a); break;
      case GP_GELU: hipLaunchKernelGGL((gemm_pipe_finish_kernel<GP_GELU>), fg, dim3(256), 0, st, a); break;
      case GP_RESID: hipLaunchKernelGGL((gemm_pipe_finish_kernel<GP_RESID>), fg, dim3(256), 0, st, a); break;
      default: return OMNI_EINVAL;
    }
    OMNI_CHECK_LAUNCH();
    return OMNI_OK;
  }
  if constexpr (NI != 4) {            // the wide tiles store only
    if (epilogue != GP_STORE) return OMNI_EINVAL;
    hipLaunchKernelGGL((gemm_pipe_kernel<WF, WM, NS, GP_STORE, NI>), dim3(grid), blk, 0, st, a);
    OMNI_CHECK_LAUNCH();
    return OMNI_OK;
  }
  switch (epilogue) {
    case GP_STORE: hipLaunchKernelGGL((gemm_pipe_kernel<WF, WM, NS, GP_STORE>), dim3(grid), blk, 0, st, a); break;
    case GP_SILU:
      if constexpr (WF == GW_ROWS) return OMNI_EINVAL;
      else hipLaunchKernelGGL((gemm_pipe_kernel<WF, WM, NS, GP_SILU>), dim3(grid), blk, 0, st, a);
      break;
    case GP_QGELU: hipLaunchKernelGGL((gemm_pipe_kernel<WF, WM, NS, GP_QGELU>), dim3(grid), blk, 0, st, a); break;
    case GP_GELU: hipLaunchKernelGGL((gemm_pipe_kernel<WF, WM, NS, GP_GELU>), dim3(grid), blk, 0, st, a); break;
    case GP_RESID: hipLaunchKernelGGL((gemm_pipe_kernel<WF, WM, NS, GP_RESID>), dim3(grid), blk, 0, st, a); break;
    default: return OMNI_EINVAL;
  }
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

// The persistent 256 x 256 tiles' column split (one K slice): where the whole tiles would
// leave a last round partly idle, the columns past the returned one run as 256 x 128 half
// tiles after R full rounds of whole tiles, at most one half tile per CU (config 5's gate_up
// at M = 4096: 1120 tiles = 4 rounds of 256 + 96, so 1024 whole tiles over columns
// [0, 16384) and 192 half tiles over the last 1536); N where no such split exists.
static int gp_big_tail_cols(int M, int N) {
  const int64_t cus = gp_num_cus();
  const int64_t tm = M / 256, tn = N / 256;
  const int64_t tiles = tm * tn;
  const int64_t R = tiles / cus;
  if (R == 0 || tiles % cus == 0 || (R * cus) % tm) return N;
  const int64_t nb = R * cus / tm;                    // whole column tiles
  if (2 * tm * (tn - nb) > cus) return N;
  return (int)(nb * 256);
}

// Relative costs of the packed fp16 weights' tile forms per 128 x 128 outputs (fitted on
// MI355X with grid rounds x tile size): the 8-wave 256 x 128 / 4-wave 128 x 128 tiles 1, the
// 4-wave 128 x 192 tiles 1.3 (config 5's down at M = 4096: 125.1 us for 256 of them against
// 128.6 us for 192 of 256 x 128), the persistent 8-wave 256 x 256 tiles 0.85.
#define GP_WIDE_COST 1.3
#define GP_BIG_COST 0.85
#define GP_PART_ELEMS 400000.0   // fp32 partial sums written and read back per step of cost
#define GP_TAIL_COST 0.65        // a round of 256 x 128 tail tiles, in rounds of 256 x 256 tiles

// Whether the packed fp16 weights take 128 x 192 tiles (4 waves, 64 x 96 each, 3 stages)
// instead of the tiles of tile_rows x 128: when the grid's rounds times a tile's cost come
// out smaller (config 5's N = 1536 projections at M = 4096: 256 tiles in one round against
// 192 of 256 x 128, which leave a quarter of the CUs idle).
static bool gp_wide_tiles(int M, int N, int tile_rows) {
  if (N % 192) return false;
  const int64_t cus = gp_num_cus();
  const int64_t tn = (int64_t)ceil_div(M, tile_rows) * (N / GP_BN);
  const int64_t tw = (int64_t)ceil_div(M, 128) * (N / 192);
  return (double)((tw + cus - 1) / cus) * 1.5 * GP_WIDE_COST <
         (double)((tn + cus - 1) / cus) * (tile_rows / 128);
}

static int gp_tile_rows(int M, int N) {
  // 256-row tiles (8 waves) when they take fewer rounds of the persistent grid than 128-row
  // tiles (e.g. M = 1024, N = 5120: 160 tiles in one round against 320 in two, 31 against
  // 41 us); at equal rounds the 128-row tiles spread the work over more CUs
  const int64_t cus = gp_num_cus();
  const int64_t t128 = (int64_t)ceil_div(M, 128) * (N / GP_BN);
  const int64_t t256 = (int64_t)ceil_div(M, 256) * (N / GP_BN);
  return (t256 + cus - 1) / cus < (t128 + cus - 1) / cus ? 256 : 128;
}

// K slices for (M, N, K) at the given tile height (0: chosen): the count (1-4, each slice
// >= 8 K steps) that minimises rounds of the persistent grid x K steps per slice, with the
// finish launch and the partial sums' traffic charged to a split (ties: fewer slices); none
// when the tiles alone fill the grid.  Measured on MI355X
// at the vision tower's shapes: fc2 (80 tiles, 80 steps) 56 -> 31 us with 3 slices; fc1 at
// 256-row tiles stays whole (2 slices would take two rounds).
extern "C" int omni_f16_gemm_pipe_splits(int M, int N, int K, int tile_rows) {
  if (M <= 0 || N <= 0 || K <= 0 || (N % GP_BN) || (K % 128)) return 1;
  if (tile_rows == 0) tile_rows = gp_tile_rows(M, N);
  const int64_t cus = gp_num_cus();
  const int64_t tiles = (int64_t)ceil_div(M, tile_rows) * (N / GP_BN);
  const int nk = K / GP_BKH;
  int best = 1;
  int64_t best_cost = ((tiles + cus - 1) / cus) * nk;
  if (tiles >= cus) return 1;        // the grid is full: slices would only add partial traffic
  for (int ks = 2; ks <= 4 && nk / ks >= 8; ++ks) {
    // a split is charged two steps for its finish launch plus its fp32 partial traffic
    // (ks M N floats written and read back: one step per 400 K elements, fitted to the
    // 2B decoder's down projection at M = 4096, where 4 slices took 146 us against 140)
    const int64_t cost = ((tiles * ks + cus - 1) / cus) * ((nk + ks - 1) / ks) + 2 +
                         (int64_t)ks * M * N / 400000;
    if (cost < best_cost) {
      best = ks;
      best_cost = cost;
    }
  }
  return best;
}

// out = epi(fp16(x . w^T + bias)) with w fp16 [N, K] in nn.Linear layout (row stride K).
// N % 128 == 0, K % 128 == 0 and K >= 256; x, w 16-byte aligned with ldx % 8 == 0;
// ldo, ldr % 4 == 0.  tile_rows 128 or 256 (0: chosen from the shape).  ksplit K slices
// (0: omni_f16_gemm_pipe_splits; each slice >= 2 groups of 128); ksplit > 1 needs an fp32
// workspace of ksplit * M * N floats (16-byte aligned).
extern "C" int omni_f16_gemm_pipe(const void* x, int ldx, const void* w, const void* bias,
                                  const void* res, int ldr, void* out, int ldo, int M, int N,
                                  int K, int epilogue, int tile_rows, int ksplit,
                                  float* workspace, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || ksplit < 0) return OMNI_EINVAL;
  if ((N % GP_BN) || (K % 128) || K < 4 * GP_BKH) return OMNI_EUNSUPPORTED;
  if (M == 0) return OMNI_OK;
  if (!x || !w || !out) return OMNI_EINVAL;
  if (ldx < K || (ldx & 7) || ldo < N || (ldo & 3)) return OMNI_EINVAL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)out & 7)) return OMNI_EINVAL;
  if (epilogue == GP_RESID && (!res || ldr < N || (ldr & 3) || ((uintptr_t)res & 7))) return OMNI_EINVAL;
  if (epilogue != GP_STORE && epilogue != GP_QGELU && epilogue != GP_GELU && epilogue != GP_RESID)
    return OMNI_EINVAL;
  if (bias && ((uintptr_t)bias & 15)) return OMNI_EINVAL;
  if (tile_rows != 0 && tile_rows != 128 && tile_rows != 256) return OMNI_EINVAL;
  if (tile_rows == 0) tile_rows = gp_tile_rows(M, N);
  if (ksplit == 0) ksplit = omni_f16_gemm_pipe_splits(M, N, K, tile_rows);
  if (2 * (K / 128 / ksplit) < 4) return OMNI_EUNSUPPORTED;    // every slice >= NS steps
  if (ksplit > 1 && (!workspace || ((uintptr_t)workspace & 15))) return OMNI_EINVAL;
  GemmPipeArgs a;
  a.x = (const half_t*)x;
  a.ldx = ldx;
  a.w = (const half_t*)w;
  a.ldw = K;
  a.bias = (const half_t*)bias;
  a.res = (const half_t*)res;
  a.ldr = ldr;
  a.out = (half_t*)out;
  a.ldo = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KS = ksplit;
  a.part = workspace;
  a.n_big = N;
  a.wq = nullptr;
  a.wsc = nullptr;
  a.bias_after_round = 0;
  hipStream_t st = (hipStream_t)stream;
  return tile_rows == 256 ? gp_launch<GW_ROWS, 4, 3>(a, epilogue, st)
                          : gp_launch<GW_ROWS, 2, 4>(a, epilogue, st);
}

// omni_packed_gemm_pipe's tiling for a shape: tile rows and columns and K slices, from the
// caller's tile_rows / ksplit (0: chosen).  128 x 192 and persistent 256 x 256 tiles only
// where both were chosen; the 256 x 256 ones (fp16 weights, STORE without a bias / SILU, M
// and N multiples of 256) where rounds of the grid times the tile's cost (per 128 x 128
// outputs: GP_BIG_COST, against 1 or GP_WIDE_COST) come out below the other plan's.
static void gp_packed_plan(int M, int N, int K, int fmt, int epilogue, bool has_bias, int tile_rows,
                           int ksplit, int& rows, int& cols, int& ks) {
  rows = tile_rows ? tile_rows : gp_tile_rows(M, N);
  ks = ksplit ? ksplit : (epilogue == GP_SILU ? 1 : omni_f16_gemm_pipe_splits(M, N, K, rows));
  cols = GP_BN;
  const bool free_split = ksplit == 0;
  if (fmt != 1 || tile_rows != 0 || ks != 1) return;
  if (epilogue == GP_SILU && M > 128 && M <= 256 && N % 160 == 0 &&
      2 * (int64_t)(N / 160) <= gp_num_cus()) {
    // gemm_n160_kernel: one round of 128 x 160 tiles where the 256 x 128 tiles (also one
    // round) stage a third more bytes per step per CU
    rows = 128;
    cols = 160;
    return;
  }
  if ((epilogue == GP_STORE || epilogue == GP_QGELU || epilogue == GP_GELU || epilogue == GP_RESID) &&
      N % 160 == 0) {
    // one round of 128 x 160 tiles where the 128-column tiles of the chosen height take one
    // round too but on fewer CUs (the vision tower's fc1: 256 against 160 tiles)
    const int64_t cus = gp_num_cus();
    const int64_t t160 = (int64_t)ceil_div(M, 128) * (N / 160);
    const int64_t tcur = (int64_t)ceil_div(M, rows) * (N / GP_BN);
    if (t160 <= cus && tcur <= cus && t160 > tcur && !(cols == 192)) {
      rows = 128;
      cols = 160;
      return;
    }
  }
  if ((epilogue == GP_STORE || epilogue == GP_PARTIAL) && gp_wide_tiles(M, N, rows)) {
    rows = 128;
    cols = 192;
  }
  if (epilogue == GP_PARTIAL && free_split && M % 256 == 0) {
    // fp32 slices are the output anyway: the persistent 256-row tiles (256 or 192 columns)
    // in 1-4 K slices, where rounds of the grid x a slice's steps x the tile's cost per step
    // (128 x 128 outputs: 1, or GP_WIDE_COST for 128 x 192, GP_BIG_COST for the persistent
    // tiles) plus each extra slice's partial traffic (one step per GP_PART_ELEMS floats)
    // come out below the plan above
    const int64_t cus = gp_num_cus();
    const int nk = K / GP_BKH;
    auto rounds = [&](int64_t t) { return (double)((t + cus - 1) / cus); };
    double best = rounds((int64_t)ceil_div(M, rows) * (N / cols)) * nk * (rows * cols) / 16384.0 *
                  (cols == 192 ? GP_WIDE_COST : 1.0);
    for (int c = 256; c >= 192; c -= 64) {
      if (N % c) continue;
      for (int k = 1; k <= 4 && K / 128 >= 2 * k; ++k) {
        const double cost = rounds((int64_t)(M / 256) * (N / c) * k) * (2 * ((nk / 2 + k - 1) / k)) *
                                (c / 64) * GP_BIG_COST +
                            (double)(k - 1) * M * N / GP_PART_ELEMS;
        if (cost < best) {
          best = cost;
          rows = 256;
          cols = c;
          ks = k;
        }
      }
    }
    return;
  }
  if (((epilogue == GP_STORE && !has_bias) || epilogue == GP_SILU) && M % 256 == 0 && N % 256 == 0) {
    const int64_t cus = gp_num_cus();
    auto rounds = [&](int64_t t) { return (double)((t + cus - 1) / cus); };
    const double cur = rounds((int64_t)ceil_div(M, rows) * (N / cols)) * (rows * cols) / 16384.0 *
                       (cols == 192 ? GP_WIDE_COST : 1.0);
    // a half-tile tail round (gp_big_tail_cols) measured at 0.65 of a whole one: M = 4096
    // gate_up + SiLU 204.9 against 221.1 us with whole tiles only
    const int64_t tb = (int64_t)(M / 256) * (N / 256);
    const double big = (gp_big_tail_cols(M, N) < N ? (double)(tb / cus) + GP_TAIL_COST : rounds(tb)) *
                       4.0 * GP_BIG_COST;
    if (big < cur) {
      rows = 256;
      cols = 256;
    }
  }
}

// The tiling omni_packed_gemm_pipe runs for a shape (no reference counterpart: it tells a
// caller or a test which tile form covers the shape).
extern "C" int omni_packed_gemm_pipe_plan(int M, int N, int K, int fmt, int epilogue,
                                          int has_bias, int tile_rows, int ksplit, int* rows,
                                          int* cols, int* ks) {
  if (M <= 0 || N <= 0 || K <= 0 || (N % GP_BN) || (K % 128) || (fmt != 0 && fmt != 1)) return OMNI_EINVAL;
  if (tile_rows != 0 && tile_rows != 128 && tile_rows != 256) return OMNI_EINVAL;
  int r, c, k;
  gp_packed_plan(M, N, K, fmt, epilogue, has_bias != 0, tile_rows, ksplit, r, c, k);
  if (rows) *rows = r;
  if (cols) *cols = c;
  if (ks) *ks = k;
  return OMNI_OK;
}

static int gp_packed_f16_launch(GemmPipeArgs& a, int epilogue, int tile_rows, int cols,
                                hipStream_t st);

// The decoder's prefill linears on the same pipeline with this library's packed weights
// (fmt 0: int4 from omni_gptq_repack with its scales, 1: fp16 from omni_f16_pack); see the
// header for the arguments.  Stages per tile height: int4 6 (128 rows) / 4 (256 rows),
// fp16 4 / 3 (the int4 operand tile is a quarter of the fp16 one).
extern "C" int omni_packed_gemm_pipe(const void* x, int ldx, const void* w_packed,
                                     const void* scales_packed, int fmt, const void* bias,
                                     int bias_after_round, void* out, int ldo, int M, int N, int K,
                                     int epilogue, int tile_rows, int ksplit, float* workspace,
                                     void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || ksplit < 0) return OMNI_EINVAL;
  if (fmt != 0 && fmt != 1) return OMNI_EINVAL;
  if ((N % GP_BN) || (K % 128) || K < 4 * GP_BKH) return OMNI_EUNSUPPORTED;
  if (M == 0) return OMNI_OK;
  if (epilogue != GP_STORE && epilogue != GP_SILU && epilogue != GP_PARTIAL) return OMNI_EINVAL;
  const bool part = epilogue == GP_PARTIAL;     // fp32 slices to workspace, no out, no bias
  if (!x || !w_packed || (!part && !out) || (fmt == 0 && !scales_packed)) return OMNI_EINVAL;
  const int n_out = epilogue == GP_SILU ? N / 2 : N;
  if (ldx < K || (ldx & 7) || (!part && (ldo < n_out || (ldo & 3)))) return OMNI_EINVAL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_packed & 15) || ((uintptr_t)out & 7)) return OMNI_EINVAL;
  if (bias && ((uintptr_t)bias & 15)) return OMNI_EINVAL;
  if ((epilogue == GP_SILU || part) && bias) return OMNI_EINVAL;
  if (tile_rows != 0 && tile_rows != 128 && tile_rows != 256) return OMNI_EINVAL;
  if (fmt == 0 && ((uintptr_t)scales_packed & 3)) return OMNI_EINVAL;
  int cols;
  gp_packed_plan(M, N, K, fmt, epilogue, bias != nullptr, tile_rows, ksplit, tile_rows, cols, ksplit);
  if (epilogue == GP_SILU && ksplit != 1) return OMNI_EINVAL;
  // every slice covers at least NS pipeline steps (slices are whole 128-groups of 2 steps)
  const int ns = fmt == 0 ? (tile_rows == 256 ? 4 : 6) : tile_rows == 256 ? (cols == GP_BN ? 3 : 2) : 4;
  if (2 * (K / 128 / ksplit) < ns) return OMNI_EUNSUPPORTED;
  if ((ksplit > 1 || part) && (!workspace || ((uintptr_t)workspace & 15))) return OMNI_EINVAL;
  GemmPipeArgs a;
  a.x = (const half_t*)x;
  a.ldx = ldx;
  a.w = fmt == 1 ? (const half_t*)w_packed : nullptr;
  a.ldw = K;
  a.wq = fmt == 0 ? (const uint32_t*)w_packed : nullptr;
  a.wsc = (const half_t*)scales_packed;
  a.bias_after_round = bias_after_round;
  a.bias = (const half_t*)bias;
  a.res = nullptr;
  a.ldr = 0;
  a.out = (half_t*)out;
  a.ldo = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KS = ksplit;
  a.part = workspace;
  a.n_big = N;
  hipStream_t st = (hipStream_t)stream;
  if (fmt == 0)
    return tile_rows == 256 ? gp_launch<GW_INT4, 4, 4>(a, epilogue, st)
                            : gp_launch<GW_INT4, 2, 6>(a, epilogue, st);
  return gp_packed_f16_launch(a, epilogue, tile_rows, cols, st);
}

// The packed fp16 weights' launch for a planned tiling (gp_packed_plan): a's fields set,
// a.KS the plan's slices.
static int gp_packed_f16_launch(GemmPipeArgs& a, int epilogue, int tile_rows, int cols,
                                hipStream_t st) {
  const int M = a.M, N = a.N;
  const int ksplit = a.KS;
  const bool bias = a.bias != nullptr;
  if (tile_rows == 256 && cols != GP_BN) {     // persistent 8-wave tiles of 256 x cols
    if (M % 256 || N % cols || (cols == 192 && epilogue == GP_SILU) || (epilogue == GP_STORE && bias) ||
        (epilogue != GP_SILU && epilogue != GP_PARTIAL && epilogue != GP_STORE))
      return OMNI_EINVAL;                      // (the plan picks them only where they hold)
    int64_t t = (int64_t)(M / 256) * (N / cols) * ksplit;
    if (cols == 256 && ksplit == 1) {
      a.n_big = gp_big_tail_cols(M, N);
      t = (int64_t)(M / 256) * (a.n_big / 256 + (N - a.n_big) / 128);
    }
    const int grid = (int)(t < gp_num_cus() ? t : gp_num_cus());
    const dim3 blk(512);
    if (epilogue == GP_SILU)
      hipLaunchKernelGGL((gemm_bigp_f16_kernel<GP_SILU, 4>), dim3(grid), blk, 0, st, a);
    else if (epilogue == GP_PARTIAL && cols == 256)
      hipLaunchKernelGGL((gemm_bigp_f16_kernel<GP_PARTIAL, 4>), dim3(grid), blk, 0, st, a);
    else if (epilogue == GP_PARTIAL)
      hipLaunchKernelGGL((gemm_bigp_f16_kernel<GP_PARTIAL, 3>), dim3(grid), blk, 0, st, a);
    else if (cols == 256)
      hipLaunchKernelGGL((gemm_bigp_f16_kernel<GP_STORE, 4>), dim3(grid), blk, 0, st, a);
    else
      hipLaunchKernelGGL((gemm_bigp_f16_kernel<GP_STORE, 3>), dim3(grid), blk, 0, st, a);
    OMNI_CHECK_LAUNCH();
    return OMNI_OK;
  }
  if (cols == 160) {                         // 128 x 160 tiles, one per workgroup
    if (N % 160 || ksplit != 1 || (epilogue == GP_SILU && M > 256)) return OMNI_EINVAL;
    const int grid = ceil_div(M, 128) * (N / 160);
    switch (epilogue) {
      case GP_SILU: hipLaunchKernelGGL((gemm_n160_kernel<4, GP_SILU>), dim3(grid), dim3(512), 0, st, a); break;
      case GP_STORE: hipLaunchKernelGGL((gemm_n160_kernel<4, GP_STORE>), dim3(grid), dim3(512), 0, st, a); break;
      case GP_QGELU: hipLaunchKernelGGL((gemm_n160_kernel<4, GP_QGELU>), dim3(grid), dim3(512), 0, st, a); break;
      case GP_GELU: hipLaunchKernelGGL((gemm_n160_kernel<4, GP_GELU>), dim3(grid), dim3(512), 0, st, a); break;
      case GP_RESID: hipLaunchKernelGGL((gemm_n160_kernel<4, GP_RESID>), dim3(grid), dim3(512), 0, st, a); break;
      default: return OMNI_EINVAL;
    }
    OMNI_CHECK_LAUNCH();
    return OMNI_OK;
  }
  if (cols == 192) return gp_launch<GW_F16, 2, 3, 6>(a, epilogue, st);
  return tile_rows == 256 ? gp_launch<GW_F16, 4, 3>(a, epilogue, st)
                          : gp_launch<GW_F16, 2, 4>(a, epilogue, st);
}

// omni_f16_gemm_pipe on this library's packed fp16 weights (omni_f16_pack): every epilogue
// of that entry (STORE, QGELU, GELU, RESID, each with the bias added before the rounding)
// and OMNI_EPI_PARTIAL (the K slices' fp32 sums into workspace, no bias, no out); the tiling
// as omni_packed_gemm_pipe plans it (omni_packed_gemm_pipe_plan with fmt 1).  For the vision
// tower's linears (model/qwen2_vit.py:41-44, 83, 88-89, 123-129).
extern "C" int omni_f16_gemm_pipe_packed(const void* x, int ldx, const void* w_packed,
                                         const void* bias, const void* res, int ldr, void* out,
                                         int ldo, int M, int N, int K, int epilogue, int tile_rows,
                                         int ksplit, float* workspace, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || ksplit < 0) return OMNI_EINVAL;
  if ((N % GP_BN) || (K % 128) || K < 4 * GP_BKH) return OMNI_EUNSUPPORTED;
  if (M == 0) return OMNI_OK;
  if (epilogue != GP_STORE && epilogue != GP_QGELU && epilogue != GP_GELU && epilogue != GP_RESID &&
      epilogue != GP_PARTIAL)
    return OMNI_EINVAL;
  const bool part = epilogue == GP_PARTIAL;
  if (!x || !w_packed || (!part && !out)) return OMNI_EINVAL;
  if (ldx < K || (ldx & 7) || (!part && (ldo < N || (ldo & 3)))) return OMNI_EINVAL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_packed & 15) || ((uintptr_t)out & 7)) return OMNI_EINVAL;
  if (bias && (part || ((uintptr_t)bias & 15))) return OMNI_EINVAL;
  if (epilogue == GP_RESID && (!res || ldr < N || (ldr & 3) || ((uintptr_t)res & 7))) return OMNI_EINVAL;
  if (tile_rows != 0 && tile_rows != 128 && tile_rows != 256) return OMNI_EINVAL;
  int cols;
  gp_packed_plan(M, N, K, 1, epilogue, bias != nullptr, tile_rows, ksplit, tile_rows, cols, ksplit);
  const int ns = tile_rows == 256 ? (cols == GP_BN ? 3 : 2) : 4;
  if (2 * (K / 128 / ksplit) < ns) return OMNI_EUNSUPPORTED;
  if ((ksplit > 1 || part) && (!workspace || ((uintptr_t)workspace & 15))) return OMNI_EINVAL;
  GemmPipeArgs a;
  a.x = (const half_t*)x;
  a.ldx = ldx;
  a.w = (const half_t*)w_packed;
  a.ldw = K;
  a.wq = nullptr;
  a.wsc = nullptr;
  a.bias_after_round = 0;
  a.bias = (const half_t*)bias;
  a.res = (const half_t*)res;
  a.ldr = ldr;
  a.out = (half_t*)out;
  a.ldo = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  a.KS = ksplit;
  a.part = workspace;
  a.n_big = N;
  return gp_packed_f16_launch(a, epilogue, tile_rows, cols, (hipStream_t)stream);
}

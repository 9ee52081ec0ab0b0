// KV-pool slot copies: one sequence's cached K/V prefix from pool row src to row dst,
// across every layer, in one launch.
//
// Replaces the per-layer torch copies of omniserve/cache/kv_prealloc.py:51-57
// (move_slot: the whole row of every layer, on pool compaction after a free) and
// :79-84 (copy_slot_kv: the first `length` tokens).  Only the valid prefix is copied
// (tokens past the length are never read before they are written again), and when the
// length lives on the device (lengths[src]) it is read there, so compaction needs no
// host synchronisation.
//
// Pool layout: [n_layers][2 (K, V)][pool_rows][max_len][row_halfs] fp16, row_halfs =
// n_kv * head_dim.  The grid covers n_layers * 2 segments x the capacity in chunks of
// 64 tokens; a workgroup whose chunk starts past the valid length returns at once.
#include "common.h"

#define SLOT_CHUNK 64   // tokens per workgroup

__global__ __launch_bounds__(256) void kv_copy_slot_kernel(half_t* __restrict__ pool, int64_t seg_stride,
                                                           int64_t row_stride, int row_halfs,
                                                           int src, int dst, int64_t length,
                                                           int64_t* __restrict__ lengths,
                                                           int max_len, int nseg) {
  int64_t len = lengths && length < 0 ? lengths[src] : length;
  len = len < 0 ? 0 : (len > max_len ? max_len : len);
  const int seg = blockIdx.x % nseg;                 // (layer, K/V)
  const int64_t t0 = (int64_t)(blockIdx.x / nseg) * SLOT_CHUNK;
  if (src != dst && t0 < len) {
    const int64_t t1 = min(t0 + SLOT_CHUNK, len);
    const int cpr = row_halfs >> 3;                   // 16-byte chunks per token row
    const int64_t total = (t1 - t0) * cpr;
    const half_t* s = pool + seg * seg_stride + (int64_t)src * row_stride + t0 * row_halfs;
    half_t* d = pool + seg * seg_stride + (int64_t)dst * row_stride + t0 * row_halfs;
    for (int64_t i = threadIdx.x; i < total; i += 256)
      ((half8_t*)d)[i] = __builtin_nontemporal_load((const half8_t*)s + i);
  }
  // the destination's length, by one thread (dst != src when anything is copied, so this
  // never changes the length the other workgroups read)
  if (lengths && blockIdx.x == 0 && threadIdx.x == 0) lengths[dst] = len;
}

// Copy tokens [0, length) of pool row src to row dst in every layer's K and V (length < 0:
// lengths[src], read on the device) and set lengths[dst] to that length.  pool fp16
// [n_layers][2][pool_rows][max_len][row_halfs]; lengths int64 [pool_rows] (may be NULL when
// length >= 0: then no length is written).
extern "C" int omni_kv_copy_slot(void* pool, int n_layers, int pool_rows, int max_len,
                                 int row_halfs, int src, int dst, int64_t length,
                                 int64_t* lengths, void* stream) {
  if (n_layers <= 0 || pool_rows <= 0 || max_len <= 0 || row_halfs <= 0) return OMNI_EINVAL;
  if (src < 0 || src >= pool_rows || dst < 0 || dst >= pool_rows) return OMNI_EINVAL;
  if (row_halfs & 7) return OMNI_EUNSUPPORTED;
  if (length < 0 && !lengths) return OMNI_EINVAL;
  if (!pool) return OMNI_EINVAL;
  if (src == dst || length == 0) {
    if (lengths && length >= 0) {
      // nothing to copy; the destination's length is still set (one workgroup)
      hipLaunchKernelGGL(kv_copy_slot_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                         (half_t*)pool, (int64_t)0, (int64_t)0, row_halfs, dst, dst, length,
                         lengths, max_len, 1);
      OMNI_CHECK_LAUNCH();
    }
    return OMNI_OK;
  }
  const int nseg = 2 * n_layers;
  const int64_t cap = length < 0 ? max_len : (length < max_len ? length : max_len);
  const int64_t chunks = (cap + SLOT_CHUNK - 1) / SLOT_CHUNK;
  const int64_t grid = chunks * nseg;
  if (grid > 0x7fffffff) return OMNI_EUNSUPPORTED;
  const int64_t row_stride = (int64_t)max_len * row_halfs;
  const int64_t seg_stride = row_stride * pool_rows;
  hipLaunchKernelGGL(kv_copy_slot_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (half_t*)pool, seg_stride, row_stride, row_halfs, src, dst, length, lengths,
                     max_len, nseg);
  OMNI_CHECK_LAUNCH();
  return OMNI_OK;
}

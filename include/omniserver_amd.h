/*
 * omniserver_amd: C ABI of the MI355X (gfx950) kernels behind the Qwen2-VL text-decoder
 * token loop.  Every entry point takes device pointers, sizes and a hipStream_t (as
 * void*), allocates nothing, never synchronises, and returns
 *     0   success
 *    -1   invalid argument (OMNI_EINVAL)
 *    -2   shape outside what the kernel supports (OMNI_EUNSUPPORTED)
 *   >0    hipError_t of the launch.
 * All calls are capturable in a HIP graph.  Calls on one stream that share a
 * workspace must not overlap (they are stream-ordered when issued on one stream).
 *
 * Reference paths below are relative to the omniserve repository.
 */
#ifndef OMNISERVER_AMD_H
#define OMNISERVER_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- norms / elementwise */

/* rms_norm (kernels/fused_ops.py:32-39): y = fp16(x * rsqrt(mean(x^2) + eps) * w).
 * x, y: fp16 [rows, hidden]; weight fp16 [hidden]; hidden % 8 == 0, <= 8192. */
int omni_rmsnorm(const void* x, const void* weight, void* y, int rows, int hidden, float eps,
                 void* stream);

/* add_rms_norm (kernels/fused_ops.py:60-70): residual_out = fp16(residual + x),
 * y = rms_norm(residual_out).  residual_out may alias residual, y may alias x. */
int omni_add_rmsnorm(const void* x, const void* residual, const void* weight, void* y,
                     void* residual_out, int rows, int hidden, float eps, void* stream);

/* add_rms_norm with x = fp16(sum over nparts of fp32 partials [nparts][rows][hidden],
 * added in slice order): consumes the split-K output of omni_w4a16_gemm/omni_f16_gemm
 * (EPI_PARTIAL) of the reference's o_proj / down_proj (model/qwen2_llm.py:99, 134)
 * followed by the next add_rms_norm (qwen2_llm.py:151, 153, 186). */
int omni_add_rmsnorm_partials(const float* partials, int nparts, const void* residual,
                              const void* weight, void* y, void* residual_out, int rows,
                              int hidden, float eps, void* stream);

/* add_rms_norm_fp8 (kernels/fused_ops.py:94-107): as add_rmsnorm, the normed row
 * quantised to e4m3fn with s = max(amax/448, 1e-12): y_fp8 = e4m3(y32 / s), scale[row] = s. */
int omni_add_rmsnorm_fp8(const void* x, const void* residual, const void* weight, void* y_fp8,
                         float* scale, void* residual_out, int rows, int hidden, float eps,
                         void* stream);

/* Layer-0 input of a decode step (models/qwen2_vl.py:93-94 + qwen2_llm.py:148-150):
 * residual_out = table[ids], y = rms_norm(residual_out).  table fp16 [vocab, hidden], or
 * the packed lm_head layout when table_packed (see omni_f16_pack). */
int omni_embed_rmsnorm(const int64_t* ids, const void* table, int table_packed, int64_t vocab,
                       const void* weight, void* y, void* residual_out, int rows, int hidden,
                       float eps, void* stream);

/* omni_embed_rmsnorm that also writes the decode step's rotary rows (omni_rope_rows for
 * rows 0..rows-1) in the same launch. */
int omni_embed_rmsnorm_rope(const int64_t* ids, const void* table, int table_packed,
                            int64_t vocab, const void* weight, void* y, void* residual_out,
                            int rows, int hidden, float eps, const int64_t* lengths,
                            const int64_t* rope_delta, const void* cos_tab, const void* sin_tab,
                            int max_pos, void* rope_rows, void* stream);

/* Rotary rows of T decode tokens (model/qwen2_llm.py:169-177, 181 at one position on all
 * three M-RoPE axes): rope_rows fp16 [T][128] = cos | sin (fp16 tables [max_pos][64]) at
 * p = lengths[r] + rope_delta[r] (clamped to the tables), r = slots[t] (NULL: t).  A decode
 * step computes them once for all of its layers' omni_decode_attention_fused calls. */
int omni_rope_rows(const int64_t* slots, const int64_t* lengths, const int64_t* rope_delta,
                   const void* cos_tab, const void* sin_tab, int max_pos, int pool_rows, int T,
                   void* rope_rows, void* stream);

/* embed_tokens (models/qwen2_vl.py:93-94): out[t] = table[ids[t]] (ids clamped to range). */
int omni_embedding(const int64_t* ids, const void* table, int table_packed, int64_t vocab,
                   void* out, int rows, int hidden, void* stream);

/* silu_mul (kernels/fused_ops.py:122-130): gate_up fp16 [rows, 2n] (gate first) ->
 * out fp16 [rows, n] = silu(g) * u in fp32. */
int omni_silu_mul(const void* gate_up, void* out, int rows, int n, void* stream);

/* silu_mul on bf16 gate_up (the reference's FP8 MLP route: gate_up.forward_prequant returns
 * bf16, model/qwen2_llm.py:127-131): out bf16 [rows, n], fp32 math, bf16 stores (RNE). */
int omni_silu_mul_bf16(const void* gate_up, void* out, int rows, int n, void* stream);

/* ---------------------------------------------------------------- rope + KV pool */

/* apply_mrope (model/qwen2_llm.py:59-72) in place on the q and k heads of qkv rows
 * [T, qkv_stride] fp16 (q | k | v), fused with _CacheView._write_kv
 * (cache/kv_prealloc.py:253-261): rotated K and raw V of token t go to
 * k/v_cache[slot, wpos] ([pool_rows, max_len, n_kv, 128] fp16).
 *   positions  int64 [3, T] (t/h/w), or NULL: base_pos[slot] + rope_delta[slot] on all
 *              axes (decode, models/qwen2_vl.py:108-112)
 *   write_pos  int64 [T], or NULL: base_pos[slot];  slots int64 [T] or NULL (= t)
 *   cos/sin    fp16 [max_pos, 64] of p * inv_freq (qwen2_llm.py:169-177, 181)
 *   k_cache/v_cache NULL: rotate only.  Sections (sec0, sec1, sec2) = [16, 24, 24]. */
int omni_mrope_kv_write(void* qkv, int qkv_stride, const int64_t* positions,
                        const int64_t* base_pos, const int64_t* rope_delta, const void* cos_tab,
                        const void* sin_tab, int max_pos, void* k_cache, void* v_cache,
                        const int64_t* slots, const int64_t* write_pos, int pool_rows, int max_len,
                        int T, int n_heads, int n_kv_heads, int head_dim, int sec0, int sec1,
                        int sec2, void* stream);

/* omni_mrope_kv_write with the qkv rows formed from the qkv projection's fp32 split-K
 * partials [nparts][T][qkv_stride] plus bias (qwen2_llm.py:88: qkv_proj with bias;
 * bias_after_round = 1 adds it after the fp16 rounding as the GPTQ path does,
 * kernels/marlin_linear.py:59-62); the rows are written to qkv. */
int omni_mrope_kv_write_partials(void* qkv, int qkv_stride, const float* partials, int nparts,
                                 const void* bias, int bias_after_round, const int64_t* positions,
                                 const int64_t* base_pos, const int64_t* rope_delta,
                                 const void* cos_tab, const void* sin_tab, int max_pos,
                                 void* k_cache, void* v_cache, const int64_t* slots,
                                 const int64_t* write_pos, int pool_rows, int max_len, int T,
                                 int n_heads, int n_kv_heads, int head_dim, int sec0, int sec1,
                                 int sec2, void* stream);

/* ---------------------------------------------------------------- KV-pool slots */

/* PreallocatedKVCache.move_slot / copy_slot_kv (cache/kv_prealloc.py:51-57, 79-84): tokens
 * [0, length) of pool row src copied to row dst in every layer's K and V in one launch,
 * lengths[dst] = that length.  length < 0: lengths[src], read on the device (no host
 * synchronisation; only the valid prefix is copied).  pool fp16 [n_layers][2][pool_rows]
 * [max_len][row_halfs] (row_halfs = n_kv * head_dim, a multiple of 8); lengths int64
 * [pool_rows], may be NULL when length >= 0. */
int omni_kv_copy_slot(void* pool, int n_layers, int pool_rows, int max_len, int row_halfs,
                      int src, int dst, int64_t length, int64_t* lengths, void* stream);

/* ---------------------------------------------------------------- attention */

/* _CacheView.flash_decode (cache/kv_prealloc.py:272-290): GQA decode attention over the
 * pool.  Token t (pool row slots[t], or t) attends to keys [0, L), L = kv_len[kv_by_slot ?
 * slot : t] + kv_add; out fp16 [T, n_heads, 128].  waves in {4, 8} per workgroup;
 * splits workgroups per (token, kv head) (1..64): splits > 1 writes partial softmax
 * states to workspace (fp32, workspace_floats of capacity; a call that needs more than
 * T * n_kv * splits * (n_heads/n_kv) * 132 is rejected with -1) and merges them in a
 * second launch. */
int omni_decode_attention(const void* q, int q_stride, const void* k_cache, const void* v_cache,
                          int pool_rows, int max_len, const int64_t* slots, const int64_t* kv_len,
                          int kv_by_slot, int kv_add, void* out, int T, int n_heads,
                          int n_kv_heads, int head_dim, float scale, int waves, int splits,
                          float* workspace, int64_t workspace_floats, void* stream);

/* The decode step's attention fused with its producer (model/qwen2_llm.py:88-99 for one
 * decode token): q and the new k / v are formed from the qkv projection's fp32 split-K
 * partials [nparts <= 16][T][(n_heads + 2 n_kv) * 128] plus qkv_bias (bias_after_round:
 * GPTQ order), M-RoPE'd at lengths[slot] + rope_delta[slot], the new K/V row is stored at
 * pool[slot, lengths[slot]] (cache/kv_prealloc.py:253-261) and token t attends to keys
 * [0, lengths[slot]] (:272-290).  slots NULL = row t.  lengths are not advanced.
 * n_heads / n_kv_heads <= 8.  merge = 1: out fp16 [T, n_heads, 128] (a merge launch
 * follows when splits > 1); merge = 0: the split states stay in workspace (T * n_kv *
 * splits * G * 132 fp32, within workspace_floats or the call is rejected) for
 * omni_*_gemm_attn and out is not written.  waves in {4, 8}.  rope_rows (may be
 * NULL): token t's rotary row from omni_rope_rows instead of a cos/sin table lookup at its
 * position (cos_tab, sin_tab, max_pos, rope_delta are then unused). */
int omni_decode_attention_fused(const float* qkv_partials, int nparts, const void* qkv_bias,
                                int bias_after_round, const void* cos_tab, const void* sin_tab,
                                int max_pos, const int64_t* rope_delta, int sec0, int sec1,
                                int sec2, void* k_cache, void* v_cache, int pool_rows, int max_len,
                                const int64_t* slots, const int64_t* lengths, void* out, int T,
                                int n_heads, int n_kv_heads, int head_dim, float scale, int waves,
                                int splits, float* workspace, int64_t workspace_floats, int merge,
                                const void* rope_rows, void* stream);

/* _PackedPrefillWriter.flash_prefill (cache/kv_prealloc.py:181-203) and the append form
 * of :149-174: token t attends causally to keys [0, kv_len[t]) of pool row slots[t].
 * qblocks int32 [nqb][2] = (first token, count <= 16) of consecutive tokens of one
 * segment.  out fp16 rows of out_stride elements. */
int omni_prefill_attention(const void* q, int q_stride, const void* k_cache, const void* v_cache,
                           int pool_rows, int max_len, const int64_t* slots, const int64_t* kv_len,
                           const int* qblocks, int nqb, void* out, int out_stride, int n_heads,
                           int n_kv_heads, int head_dim, float scale, void* stream);

/* The same attention (qblocks counts <= 16) with each (block, head) item's key tiles split
 * over the four waves of a workgroup and the partial softmax states merged in LDS: for few
 * items with many keys each (a prompt of a few hundred tokens, an appended chunk).  Agrees
 * with omni_prefill_attention to the fp16 rounding of the probabilities (replaces the same
 * cache/kv_prealloc.py:181-203 call). */
int omni_prefill_attention_split(const void* q, int q_stride, const void* k_cache,
                                 const void* v_cache, int pool_rows, int max_len,
                                 const int64_t* slots, const int64_t* kv_len, const int* qblocks,
                                 int nqb, void* out, int out_stride, int n_heads, int n_kv_heads,
                                 int head_dim, float scale, void* stream);

/* The same attention with query blocks of up to 32 tokens (qblocks counts <= 32): one
 * workgroup per (block, KV head) loads each 32-key K/V tile once into LDS for all the
 * group's query heads (n_heads / n_kv_heads <= 8); outputs equal omni_prefill_attention's
 * bit for bit.  For long segments. */
int omni_prefill_attention_gqa(const void* q, int q_stride, const void* k_cache,
                               const void* v_cache, int pool_rows, int max_len,
                               const int64_t* slots, const int64_t* kv_len, const int* qblocks,
                               int nqb, void* out, int out_stride, int n_heads, int n_kv_heads,
                               int head_dim, float scale, void* stream);

/* The omni_prefill_attention_gqa attention (qblocks counts <= 32, n_heads / n_kv_heads
 * <= 6) with each workgroup's key tiles split between two groups of four waves, the second
 * group's normalised output (rounded to fp16) and softmax state merged into the first's in
 * LDS: the longest (last) blocks of a segment take half as many tile steps.  Agrees with
 * omni_prefill_attention to that fp16 rounding (replaces the same
 * cache/kv_prealloc.py:181-203 call); -2 for n_heads / n_kv_heads > 6. */
int omni_prefill_attention_gqa_halves(const void* q, int q_stride, const void* k_cache,
                                      const void* v_cache, int pool_rows, int max_len,
                                      const int64_t* slots, const int64_t* kv_len,
                                      const int* qblocks, int nqb, void* out, int out_stride,
                                      int n_heads, int n_kv_heads, int head_dim, float scale,
                                      void* stream);

/* ---------------------------------------------------------------- linears */

/* Epilogues of the skinny GEMMs. */
#define OMNI_EPI_STORE 0   /* fp16 out (+ bias) */
#define OMNI_EPI_SILU 1    /* gate_up: fp16 silu(gate) * up, out [M, N/2] (interleave_halves pack) */
#define OMNI_EPI_PARTIAL 2 /* fp32 split-K partial sums [slices][M][N], no bias */

/* GPTQMarlinLinear.forward (kernels/marlin_linear.py:54-62, 83-96): y = fp16(x . W), W =
 * fp16((q - 8) * s), bias added after the fp16 rounding when bias_after_round.  x fp16
 * [M, K] (row stride ldx); weights from omni_gptq_repack.  M <= 64 runs the skinny
 * weight-streaming kernel: ksplit > 1 only with OMNI_EPI_PARTIAL (slices =
 * omni_gemm_slices(K, ksplit)), preset selects the workgroup shape (0..3; SiLU 0..9).
 * M > 64 (prefill) runs an MFMA GEMM (omni_packed_gemm_pipe's pipeline where its shape and
 * alignment rules hold, else a tiled kernel): OMNI_EPI_STORE / OMNI_EPI_SILU, preset ignored;
 * with OMNI_EPI_STORE, ksplit > 1 splits K over omni_gemm_slices(K, ksplit) slices whose
 * fp32 sums go to partial ([slices][M][N], 16-byte aligned) before a second launch adds
 * them in order and stores out (+ bias). */
int omni_w4a16_gemm(const void* x, int ldx, const void* qweight_packed, const void* scales_packed,
                    const void* bias, int bias_after_round, void* out, int ldo, float* partial,
                    int M, int N, int K, int epilogue, int ksplit, int preset, void* stream);

/* fp16 nn.Linear (model/qwen2_llm.py:82-83, 120-121): y = fp16(x . W^T + b), weights from
 * omni_f16_pack.  Same epilogues / split rules as omni_w4a16_gemm. */
int omni_f16_gemm(const void* x, int ldx, const void* weight_packed, const void* bias, void* out,
                  int ldo, float* partial, int M, int N, int K, int epilogue, int ksplit,
                  int preset, void* stream);

/* o_proj fed by the decode attention (model/qwen2_llm.py:98-99: o_proj(attn_out)) without
 * the attention's merge launch: x[m, h*128 + d] is the merge of the attn_splits split
 * states [M][n_kv_heads][attn_splits][group][132] fp32 that omni_decode_attention_fused
 * left in its workspace (merge = 0), computed while x is staged (bit-identical to merging
 * first).  K = n_kv_heads * group * 128; epilogue OMNI_EPI_STORE or OMNI_EPI_PARTIAL. */
int omni_w4a16_gemm_attn(const float* attn_states, int attn_splits, int n_kv_heads, int group,
                         const void* qweight_packed, const void* scales_packed, const void* bias,
                         int bias_after_round, void* out, int ldo, float* partial, int M, int N,
                         int K, int epilogue, int ksplit, int preset, void* stream);
int omni_f16_gemm_attn(const float* attn_states, int attn_splits, int n_kv_heads, int group,
                       const void* weight_packed, const void* bias, void* out, int ldo,
                       float* partial, int M, int N, int K, int epilogue, int ksplit, int preset,
                       void* stream);

/* DecoderLayer's add_rms_norm followed by the linear it feeds (model/qwen2_llm.py:145-157:
 * input_layernorm -> qkv_proj, post_attention_layernorm -> gate_up_proj; the norm of
 * kernels/fused_ops.py:60-70), for decode steps of a row or two: x = RMSNorm(h) * weight with
 * h = fp16(fp16(sum of the fp32 split-K partials [nparts][M][K] in slice order) + residual),
 * the previous projection's OMNI_EPI_PARTIAL output, formed by every workgroup in its input
 * staging (x and h bit-identical to omni_add_rmsnorm_partials'), so that no norm launch sits
 * between the two projections.  One workgroup writes h to residual_out, which must not
 * alias residual.  M <= 16, K % 512 == 0, M * K / 8 <= the preset's threads (preset 1: 512;
 * OMNI_EPI_SILU preset 1 or 4: 512 / 768); 16-byte aligned pointers.  The linear as
 * omni_w4a16_gemm / omni_f16_gemm (OMNI_EPI_STORE, OMNI_EPI_SILU or OMNI_EPI_PARTIAL). */
int omni_w4a16_gemm_addnorm(const float* partials, int nparts, const void* residual,
                            const void* weight, float eps, void* residual_out,
                            const void* qweight_packed, const void* scales_packed, const void* bias,
                            int bias_after_round, void* out, int ldo, float* partial, int M, int N,
                            int K, int epilogue, int ksplit, int preset, void* stream);
int omni_f16_gemm_addnorm(const float* partials, int nparts, const void* residual,
                          const void* weight, float eps, void* residual_out,
                          const void* weight_packed, const void* bias, void* out, int ldo,
                          float* partial, int M, int N, int K, int epilogue, int ksplit, int preset,
                          void* stream);

/* Number of K slices (whole 128-groups) a split of ksplit gives for K. */
int omni_gemm_slices(int K, int ksplit);

/* load_gptq_llm / gptq_marlin_repack (kernels/marlin_linear.py:94-95, 114-143): AutoGPTQ
 * qweight int32 [K/8, N] + scales fp16 [K/128, N] -> this library's packed int4 layout
 * (qweight_packed int32 [N/16][K/128][64][4], scales_packed fp16 [N/16][K/128][16]).
 * interleave_halves: column tiles of the two halves of N interleaved (fused gate|up,
 * marlin_linear.py:130-139) for OMNI_EPI_SILU. */
int omni_gptq_repack(const int32_t* qweight, const void* scales, int32_t* qweight_packed,
                     void* scales_packed, int K, int N, int interleave_halves, void* stream);

/* fp16 weight [N, K] (nn.Linear layout) -> packed [N/16][K/32][64][8]. */
int omni_f16_pack(const void* weight, void* weight_packed, int K, int N, int interleave_halves,
                  void* stream);

/* Packed int4 -> dense W^T [K, N] fp16 with W = fp16((q - 8) * s): the reference's
 * dequantised weight (verification / load-time use). */
int omni_w4_dequant(const int32_t* qweight_packed, const void* scales_packed, void* w, int K,
                    int N, void* stream);

/* Packed int4 -> packed fp16 (omni_f16_pack's layout, tile order kept, so gate|up stays
 * interleaved), W = fp16((q - 8) * s) as the int4 kernels dequantise it: the GPTQ prefill
 * linears at many rows (kernels/marlin_linear.py:54-62) then run the fp16 GEMM on the same
 * values.  qweight_packed and weight_packed 16-byte aligned; weight_packed holds N * K halfs. */
int omni_w4_unpack_f16(const int32_t* qweight_packed, const void* scales_packed,
                       void* weight_packed, int K, int N, void* stream);

/* ---------------------------------------------------------------- vision tower */

/* Epilogues of omni_f16_gemm_tiled beyond OMNI_EPI_STORE (h = fp16(x . W^T + bias)). */
#define OMNI_EPI_QGELU 4   /* quick_gelu(h) = h * sigmoid(1.702 h), three fp16 roundings */
#define OMNI_EPI_GELU 5    /* exact (erf) GELU of h */
#define OMNI_EPI_RESID 6   /* fp16(res + h); res may alias out */

/* The vision tower's nn.Linear layers at any M (model/qwen2_vit.py:41-44, 83, 88-89, and
 * their use at :55, 64, 68, 121, 128): tiled MFMA GEMM over weights from omni_f16_pack with
 * K a multiple of 128 (zero-padded past kx); x fp16 [M, kx] (row stride ldx, kx % 8 == 0);
 * bias optional. */
int omni_f16_gemm_tiled(const void* x, int ldx, int kx, const void* weight_packed,
                        const void* bias, const void* res, int ldr, void* out, int ldo, int M,
                        int N, int K, int epilogue, void* stream);

/* The same linears on a multi-stage global -> LDS pipeline GEMM (persistent grid, 128- or
 * 256-row x 128-column tiles): w fp16 [N, K] in nn.Linear layout (row stride K, no
 * packing).  N % 128 == 0, K % 128 == 0, K >= 256; x, w 16-byte aligned, ldx % 8 == 0,
 * ldo / ldr % 4 == 0.  Epilogues as omni_f16_gemm_tiled; tile_rows 128, 256 or 0 (chosen
 * from the shape).  ksplit K slices (0: omni_f16_gemm_pipe_splits), each >= 256 of K;
 * ksplit > 1 writes fp32 partial sums to workspace (ksplit * M * N floats, 16-byte
 * aligned) and finishes the epilogue in a second launch (slices summed in order). */
int omni_f16_gemm_pipe(const void* x, int ldx, const void* w, const void* bias, const void* res,
                       int ldr, void* out, int ldo, int M, int N, int K, int epilogue,
                       int tile_rows, int ksplit, float* workspace, void* stream);

/* The K slices omni_f16_gemm_pipe uses for ksplit = 0 (tile_rows as there). */
int omni_f16_gemm_pipe_splits(int M, int N, int K, int tile_rows);

/* The decoder's linears at prefill sizes (GPTQMarlinLinear.forward,
 * kernels/marlin_linear.py:54-62, 83-96, and the fp16 nn.Linear of model/qwen2.py's
 * attention and MLP) on the pipeline of omni_f16_gemm_pipe, with this library's packed
 * weights: fmt 0 int4 + scales from omni_gptq_repack (W = fp16((q - 8) s)), fmt 1 fp16
 * from omni_f16_pack (scales_packed unused).  out = fp16(x . W^T) (+ bias, after the fp16
 * rounding when bias_after_round); OMNI_EPI_SILU: gate|up packed with interleave_halves,
 * out [M, N/2] = fp16(silu(g) u) of the fp16 g, u (no bias, ksplit 1).  N % 128 == 0,
 * K % 128 == 0, K >= 256; x, w 16-byte and scales 4-byte aligned, ldx % 8 == 0,
 * ldo % 4 == 0, out 8-byte aligned.  tile_rows 128, 256 or 0 (from the shape); ksplit K
 * slices of whole 128-groups (0: omni_f16_gemm_pipe_splits; each slice >= 3 groups for
 * int4 at 128 rows, else >= 2), ksplit > 1 with fp32 workspace (ksplit * M * N floats,
 * 16-byte aligned) summed in order by a second launch.  OMNI_EPI_PARTIAL: the ksplit fp32
 * slices [ksplit][M][N] only, into workspace (out and bias unused, NULL), for a consumer
 * that sums them in order (omni_add_rmsnorm_partials, omni_mrope_kv_write_partials).
 * With tile_rows and ksplit both 0 and fp16 weights, shapes whose 128 x 192 tiles (STORE /
 * PARTIAL, N % 192 == 0) or persistent 256 x 256 tiles (STORE without a bias / SILU, M and
 * N % 256 == 0) take fewer grid rounds x tile work run those, and 128 x 160 tiles (N % 160
 * == 0: the SILU epilogue at 129-256 rows as five gate|up pairs, STORE with a bias where one
 * round of them covers more CUs than one round of 128-column tiles) where they fill the CUs
 * in one round (omni_packed_gemm_pipe_plan; same k order per output: results equal the
 * 128 x 128 tiles' bit for bit). */
int omni_packed_gemm_pipe(const void* x, int ldx, const void* w_packed, const void* scales_packed,
                          int fmt, const void* bias, int bias_after_round, void* out, int ldo,
                          int M, int N, int K, int epilogue, int tile_rows, int ksplit,
                          float* workspace, void* stream);

/* The tiling omni_packed_gemm_pipe runs for a shape (no reference counterpart: it tells a
 * caller or a test which form covers the shape): *rows x *cols tiles (128 / 256 x 128,
 * 128 x 192, 128 x 160, or the persistent 256 x 256) and *ks K slices for the given epilogue, bias
 * (has_bias != 0) and tile_rows / ksplit (0: chosen); any output may be NULL.  -1 for a
 * shape it rejects. */
int omni_packed_gemm_pipe_plan(int M, int N, int K, int fmt, int epilogue, int has_bias,
                               int tile_rows, int ksplit, int* rows, int* cols, int* ks);

/* omni_f16_gemm_pipe on this library's packed fp16 weights (omni_f16_pack with no gate|up
 * interleave): the same epilogues (OMNI_EPI_STORE / QGELU / GELU / RESID, the bias added
 * before the fp16 rounding) plus OMNI_EPI_PARTIAL (each K slice's fp32 sums to
 * workspace[slice][M][N]; no bias, out unused; omni_layernorm_partials adds them).  Tiling
 * and K slices as omni_packed_gemm_pipe plans them (omni_packed_gemm_pipe_plan, fmt 1;
 * ksplit > 0 fixes the slices).  The vision tower's linears (model/qwen2_vit.py:41-44, 83,
 * 88-89, 123-129). */
int omni_f16_gemm_pipe_packed(const void* x, int ldx, const void* w_packed, const void* bias,
                              const void* res, int ldr, void* out, int ldo, int M, int N, int K,
                              int epilogue, int tile_rows, int ksplit, float* workspace,
                              void* stream);

/* nn.LayerNorm(N, eps) of M fp16 rows (model/qwen2_vit.py:39-40, 87): fp32 mean and biased
 * variance, y = (x - mean) rsqrt(var + eps) w + b.  N % 8 == 0, N <= 2048; out may alias x. */
int omni_layernorm(const void* x, int ldx, const void* weight, const void* bias, int M, int N,
                   float eps, void* out, int ldo, void* stream);

/* A split-K linear's residual add followed by a LayerNorm (model/qwen2_vit.py:66-69: x = x +
 * attn(...) then norm2(x); x = x + mlp(...) then the next norm1 or the merger's ln_q):
 * residual_out = fp16(residual + fp16(sum of the fp32 slices [nparts][M][N] in slice order +
 * lin_bias)) - what omni_f16_gemm_pipe's finish launch writes with OMNI_EPI_RESID - and
 * out = LayerNorm(residual_out; weight, bias, eps) as omni_layernorm.  1 <= nparts <= 16;
 * lin_bias may be NULL; residual_out may alias residual; pointers 16-byte aligned. */
int omni_layernorm_partials(const float* partials, int nparts, const void* lin_bias,
                            const void* residual, int ldr, void* residual_out, int ldro,
                            const void* weight, const void* bias, int M, int N, float eps,
                            void* out, int ldo, void* stream);

/* vision_rope (kernels/vision_rope.py:39-47, with the angles of model/qwen2_vit.py:96-116):
 * in place on q heads [0, n_heads) and k heads [n_heads, 2 n_heads) of S qkv rows (row
 * stride ld, head_dim % 16 == 0).  pos_hw int32 [S][2] patch (h, w); inv_freq fp32
 * [head_dim / 4]; pair (d, d + head_dim/2) turns by pos_h inv_freq[d] (d < head_dim/4) or
 * pos_w inv_freq[d - head_dim/4], fp32 math, fp16 out. */
int omni_vision_rope(void* qkv, int ld, int S, int n_heads, int head_dim, const int* pos_hw,
                     const float* inv_freq, void* stream);

/* VisionBlock.attn's flash_attn_varlen_func(causal=False) (model/qwen2_vit.py:58-63):
 * softmax(q k^T scale) v within each segment [cu[s], cu[s+1]) of the rotated qkv rows
 * (q | k | v heads, head_dim 80).  tiles int32 [ntiles][2] = (first query, segment) in
 * steps of 64 queries; out fp16 [S][ldo], head h at column 80 h. */
int omni_vit_attention(const void* qkv, int ld, int S, int n_heads, int head_dim,
                       const int* cu_seqlens, const int* tiles, int ntiles, void* out, int ldo,
                       float scale, void* stream);

/* ---------------------------------------------------------------- fp8 (W8A8) */

/* Row-wise e4m3fn quantisation: scale[r] = amax_k |x[r, k]| / 448 (max(., clamp_min) when
 * clamp_min > 0), q[r, k] = e4m3(x[r, k] / scale[r]).  Activations: quant_fp8
 * (kernels/fp8_linear.py:45-63, no clamp); weights at load: FP8Linear's sw / Wq
 * (fp8_linear.py:83-86).  x fp16 [rows, K] (row stride ldx), q [rows, K] bytes. */
int omni_fp8_quant_rows(const void* x, int ldx, void* q, float* scale, int rows, int K,
                        float clamp_min, void* stream);

/* omni_fp8_quant_rows on bf16 rows: quant_fp8 of the bf16 silu_mul output that an FP8
 * down_proj takes directly (model/qwen2_llm.py:132-134, kernels/fp8_linear.py:45-63). */
int omni_fp8_quant_rows_bf16(const void* x, int ldx, void* q, float* scale, int rows, int K,
                             float clamp_min, void* stream);

/* FP8Linear's row-wise weight quantisation (kernels/fp8_linear.py:83-86) on the fp16 weight
 * [N, K] (row stride ldw): scale[n] = fp16(amax_k |w[n, k]| / 448) (the reference divides
 * the fp16 amax by 448 in fp16), wq[n, k] = e4m3(w[n, k] / scale[n]) (fp32 division, the
 * [N, 1] scale promotes it). */
int omni_fp8_quant_weight_rows(const void* w, int ldw, void* wq, float* scale, int N, int K,
                               void* stream);

/* Per-tensor e4m3 quantisation, FP8Linear's default form: _quant_fp8_pertensor's eager
 * branch (kernels/fp8_linear.py:40-41) for activations and the weight quantisation of
 * :87-89, both ops on the fp16 (bf16 = 1: bf16) tensor: s = R(amax |x| / 448),
 * q = e4m3(R(x / s)), R the input's rounding.  s is written to scale[r] for every row (the
 * [M] / [N] scale array omni_fp8_gemm takes).  work: omni_fp8_quant_tensor_work(rows)
 * floats of scratch (one partial maximum per workgroup).  Two launches. */
int omni_fp8_quant_tensor(const void* x, int ldx, void* q, float* scale, float* work,
                          int rows, int K, int bf16, void* stream);
int omni_fp8_quant_tensor_work(int rows);

/* FP8Linear.forward / forward_prequant (kernels/fp8_linear.py:99-126): the product
 * v[m, n] = (sum_k xq[m,k] wq[n,k]) * sa[m] * sw[n] (fp32 accumulation, as
 * torch._scaled_mm) stored by out_mode:
 *   0  bf16(v) cast to fp16, + fp16 bias in fp16 (row-wise forward, :115-118, 124-125);
 *   1  bf16(v) + bf16(bias) added in bf16 (forward_prequant, :99-108);
 *   2  fp16(v), + fp16 bias in fp16 (per-tensor forward: out_dtype fp16, :119-125; sa and
 *      sw hold one value each, repeated).  This form runs the 256 x 128 kernel where
 *      omni_fp8_gemm_plan names a 256-row big-tile one (their epilogue has no room for it).
 * xq [M, K], wq [N, K] e4m3fn; out [M, ldo]; N % 128 == 0, K % 128 == 0; xq, wq and bias
 * 16-byte aligned, sa / sw 4-byte, out 8-byte (else -1). */
int omni_fp8_gemm(const void* xq, const float* sa, const void* wq, const float* sw,
                  const void* bias, void* out, int ldo, int M, int N, int K, int out_mode,
                  void* stream);

/* Self-check of the bf16 rounding the FP8 GEMM epilogues use (no reference counterpart: a
 * test of this library's arithmetic): every one of the 2^32 float bit patterns through the
 * device's packed bf16 conversion and through the integer round-to-nearest-even with quieted
 * NaNs that the reference's bf16 outputs follow; adds the non-NaN mismatches to
 * mismatches[0] and the NaN ones to mismatches[1] (device memory, zeroed by the caller). */
int omni_bf16_rne_check(unsigned long long* mismatches, void* stream);

/* The kernel omni_fp8_gemm runs for a shape (no reference counterpart: it tells a caller
 * or a test which form covers the shape): 0 one 128 x 128 tile per workgroup (K < 512),
 * 1 the pipelined persistent 256 x 128 tiles, 2 the persistent 256 x 256 tiles (where whole
 * tiles would leave the grid's last round partly idle, the columns past whole rounds as
 * 256 x 192 tiles after them, at most one per CU: config 4's gate_up at M = 8192), 3 the
 * persistent 256 x 192 tiles (2 and 3: K >= 1024, M a multiple of 256, N of the width,
 * where rounds of the grid times the tile's work come out below the 256 x 128 tiles', a big
 * tile counted at 0.85 of its size: e.g. every config-4 shape at M = 8192, not N = 1536 at
 * M = 4096); *grid (may be NULL) = its workgroups.  Returns -1 for a shape omni_fp8_gemm
 * rejects. */
int omni_fp8_gemm_plan(int M, int N, int K, int* grid);

/* ---------------------------------------------------------------- lm_head + greedy */

/* Workgroups (= candidate rows per token) of omni_lmhead_candidates for vocab N. */
int omni_lmhead_argmax_grid(int N);

/* Rows M one omni_lmhead_candidates call takes at hidden size K (x is staged in LDS:
 * 48 at K = 1536); callers split larger batches (helper, no reference counterpart). */
int omni_lmhead_max_rows(int K);

/* Tied lm_head (model/qwen2_llm.py:167-168, 190) with the greedy argmax of
 * runners/multimodal.py:306-310: per workgroup and row the max fp16 logit and its lowest
 * index go to cand_val/cand_idx ([grid][M]); logits_out fp16 [M, N] optional. */
int omni_lmhead_candidates(const void* x, int ldx, const void* weight_packed, int M, int N, int K,
                           void* logits_out, float* cand_val, int* cand_idx, void* stream);

/* ids_out[m] = argmax over the candidates (lowest index on ties, torch.argmax semantics);
 * optionally next_ids[m] = ids_out[m] and lengths[m] += 1 (the decode step's
 * bookkeeping, runners/multimodal.py:355-356). */
int omni_argmax_finalize(const float* cand_val, const int* cand_idx, int nblk, int M,
                         int64_t* ids_out, int64_t* next_ids, int64_t* lengths, void* stream);

/* ---------------------------------------------------------------- allocation-free */

/* No counterpart in the reference: omni_lmhead_candidates followed by omni_argmax_finalize
 * in one call that allocates nothing and takes no workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid it).  The candidates live in a device array the library holds once per GPU
 * for the whole process (256 KiB: up to 32768 workgroup x row slots); shapes that would
 * need more return OMNI_EUNSUPPORTED, as do M > omni_lmhead_max_rows(K) and N % 32 != 0.  Nothing has to start
 * at zero; calls that overlap on one GPU (different streams) share the array and race.
 * ids_out / logits_out / next_ids / lengths as in the two calls it stands for. */
int omni_lmhead_argmax_noalloc(const void* x, int ldx, const void* weight_packed, int M, int N,
                               int K, void* logits_out, int64_t* ids_out, int64_t* next_ids,
                               int64_t* lengths, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OMNISERVER_AMD_H */

/*
 * skv.h -- C ABI of the MI355X (gfx950) KV-cache hot path.
 *
 * Every pointer argument is a device pointer (HBM) unless marked "host".
 * The library never allocates device memory in these entry points: the
 * caller owns the cache, the inputs, the outputs and the split-K workspace.
 * Every entry point only enqueues work on `stream` (a hipStream_t passed as an
 * opaque pointer; NULL = the legacy default stream) and returns without
 * synchronising.
 *
 * Return value: 0 on success, a negative SKV_E* code otherwise. The message
 * for the most recent failure on the calling thread is skv_last_error().
 *
 * Cache layout (contiguous), from the reference's cache indexing
 * (simple-llm/src/gpu/gpu_kernels.py:2791-2793, 2858-2859):
 *   element (b, t, h, d) of a [B, T_cap, H_kv, D] cache sits at
 *   ((b * T_cap + t) * H_kv + h) * D + d.
 * Paged layout (extension; no reference counterpart): a pool of
 *   [n_blocks][block_size][H_kv][D] rows, and token t of sequence b lives in
 *   block block_table[b * max_blocks + t / block_size], row t % block_size.
 *
 * Lengths: lens[b] is the number of filled positions of sequence b. The
 * single-token append writes at position lens[b] and then increments
 * lens[b]; decode attention of sequence b attends positions [0, lens[b]).
 * The reference keeps one scalar for the whole batch
 * (simple-llm/src/gpu/gpu_types.py:443); equal lens[b] reproduce it.
 */
#ifndef SKV_H_
#define SKV_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* skv_stream_t; /* a hipStream_t */

enum skv_dtype { SKV_F32 = 0, SKV_BF16 = 1 };

enum skv_status {
  SKV_OK = 0,
  SKV_E_INVALID = -22,     /* bad argument (shape, dtype, null pointer)   */
  SKV_E_UNSUPPORTED = -95, /* valid request this build has no kernel for   */
  SKV_E_WORKSPACE = -28,   /* workspace smaller than required              */
  SKV_E_HIP = -5           /* a HIP runtime call failed                    */
};

/* Thread-local message describing the last failure ("" if none). */
const char* skv_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int skv_version(void);

/*
 * Append one token per sequence into a contiguous cache.
 * Replaces kv_cache_update (simple-llm/src/gpu/gpu_kv_cache.py:113-186) and
 * its WGSL kernel create_kv_cache_update_kernel
 * (simple-llm/src/gpu/gpu_kernels.py:2725-2798):
 *   k_cache[b, lens[b], :, :] = k_new[b, :, :]   (same for v), then lens[b]++.
 * A sequence with lens[b] >= T_cap is full: nothing is written and lens[b]
 * is left unchanged (the host checks capacity first, as the reference does
 * at gpu_kv_cache.py:148-152).
 * k_new, v_new: [B, H_kv, D] of in_dt. k_cache, v_cache: [B, T_cap, H_kv, D]
 * of cache_dt (fp32 copy is exact; bf16 storage rounds to nearest even).
 * Any D > 0 (16-byte vectors when H_kv * D is a multiple of 8 and the
 * pointers are 16-byte aligned, element copies otherwise).
 */
int skv_append(void* k_cache, void* v_cache, const void* k_new, const void* v_new,
               int32_t* lens, int B, int H_kv, int D, int T_cap, int cache_dt,
               int in_dt, skv_stream_t stream);

/* Paged variant of skv_append (extension; same semantics, paged layout). */
int skv_append_paged(void* k_pool, void* v_pool, const void* k_new,
                     const void* v_new, int32_t* lens, const int32_t* block_table,
                     int max_blocks, int block_size, int B, int H_kv, int D,
                     int cache_dt, int in_dt, skv_stream_t stream);

/*
 * Append a chunk of up to C tokens per sequence without advancing lens.
 * Row i < n_new[b] of k_new[b] goes to position lens[b] + i. Rows that would
 * land at or beyond T_cap are not written (the host rejects such calls).
 * n_new may be NULL, meaning C for every sequence.
 * k_new, v_new: [B, C, H_kv, D] of in_dt.
 * The reference appends one token per call only (gpu_kv_cache.py:157-159);
 * this is the chunked-prefill extension.
 */
int skv_append_chunk(void* k_cache, void* v_cache, const void* k_new,
                     const void* v_new, const int32_t* lens, const int32_t* n_new,
                     int B, int C, int H_kv, int D, int T_cap, int cache_dt,
                     int in_dt, skv_stream_t stream);

/* lens[b] = min(lens[b] + (n_new ? n_new[b] : n_const), T_cap). */
int skv_advance(int32_t* lens, const int32_t* n_new, int n_const, int B, int T_cap,
                skv_stream_t stream);

/*
 * Split-K sizing for decode attention (host-only, no device work).
 * Given the longest sequence the call may see (max_len) and the filled
 * tokens of the whole batch (total_len; <= 0 means B * max_len), picks
 * chunk_tokens (tokens of the flat token stream -- every sequence's filled
 * tokens end to end -- per workgroup) for the pass-1 kernel a call with
 * this head_dim and cache_dtype runs: grouped queries (H_q / H_kv in
 * {2, 4, 8}) over a bf16 cache with head_dim 64 or 128 run on the matrix
 * cores, one busy workgroup per CU for 7/8 of the CUs (HBM streams faster
 * with fewer streams than CUs); the other kernels get about two busy
 * workgroups per CU (512), or one per CU (256) when H_q == H_kv and that
 * still gives chunks of at least 256 tokens. n_chunks_max =
 * ceil(max_len / chunk_tokens) + 1 partial slots per sequence: B *
 * (n_chunks_max - 1) workgroups cover B * max_len tokens, and the spare slot
 * holds the piece of a sequence that starts inside a workgroup's range.
 * H_q must be a multiple of H_kv. chunk_hint > 0 forces that chunk size
 * (rounded up to a multiple of 16). Any plan is valid for any call with
 * these B, H_q and max_len; head_dim and cache_dtype only tune it.
 */
int skv_decode_plan(int B, int H_q, int H_kv, int head_dim, int cache_dtype, int max_len,
                    long long total_len, int chunk_hint, int* chunk_tokens /* host */,
                    int* n_chunks_max /* host */);

/* Bytes of workspace skv_decode_attn needs for this plan: fp32 partials
 * (o[D], m, l) per (query head, slot), then B + 1 int64 prefix sums. */
size_t skv_decode_workspace_bytes(int B, int H_q, int D, int n_chunks_max);

/*
 * Single-query attention over the cache (decode step).
 * Replaces attention_with_kv_cache (simple-llm/src/gpu/gpu_kv_cache.py:194-289)
 * and create_attention_with_kv_cache_kernel
 * (simple-llm/src/gpu/gpu_kernels.py:2801-2938):
 *   out[b, h, :] = softmax(scale * q[b, h, :] . K[b, 0:lens[b], h/G, :]^T)
 *                  . V[b, 0:lens[b], h/G, :],           G = H_q / H_kv.
 * No length cap (the reference caps lens at 256). lens[b] == 0 gives zeros.
 * q, out: [B, H_q, D] of q_dt / out_dt. G in {1, 2, 4, 8}. D: any head dim
 * (the reference takes any, gpu_kernels.py:2846) up to 2048 for G <= 2,
 * 1024 for G = 4 and 512 for G = 8; 64 and 128 run kernels tuned per shape,
 * others the same kernels at the head dim padded to a power of two from 32
 * (rows of 16 lanes up to 256, 128 with G = 8; rows of a whole wavefront
 * past that). Larger head dims return SKV_E_UNSUPPORTED.
 * Split-K: pass 1 writes per-piece (max, sum, unnormalised o) partials into
 * ws; pass 2 merges them. n_chunks_max >= 2. A sequence whose tokens lie
 * past the first B * (n_chunks_max - 1) * chunk_tokens tokens of the flat
 * stream (possible only when some lens[b] > max_len of the plan) gets NaN
 * outputs, never out-of-bounds reads.
 */
int skv_decode_attn(void* out, const void* q, const void* k_cache,
                    const void* v_cache, const int32_t* lens, int B, int H_q,
                    int H_kv, int D, int T_cap, float scale, int chunk_tokens,
                    int n_chunks_max, void* ws, size_t ws_bytes, int cache_dt,
                    int q_dt, int out_dt, skv_stream_t stream);

/*
 * skv_decode_attn without a workspace argument: an entry point that
 * allocates nothing, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It has no counterpart in the reference. The split-K partials
 * live in a file-scope device array of SKV_DECODE_NOALLOC_MAX_BYTES (64 MiB)
 * that each GPU the library runs on holds until the process ends; a plan
 * whose skv_decode_workspace_bytes exceeds it is rejected with
 * SKV_E_WORKSPACE. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams, or threads) race and must not be
 * issued. Arguments and results are those of skv_decode_attn (same kernels:
 * results are bitwise equal for the same plan).
 */
#define SKV_DECODE_NOALLOC_MAX_BYTES ((size_t)64 << 20)
int skv_decode_attn_noalloc(void* out, const void* q, const void* k_cache,
                            const void* v_cache, const int32_t* lens, int B, int H_q,
                            int H_kv, int D, int T_cap, float scale, int chunk_tokens,
                            int n_chunks_max, int cache_dt, int q_dt, int out_dt,
                            skv_stream_t stream);

/* Paged variant of skv_decode_attn (extension; block_size a power of two). */
int skv_decode_attn_paged(void* out, const void* q, const void* k_pool,
                          const void* v_pool, const int32_t* lens,
                          const int32_t* block_table, int max_blocks,
                          int block_size, int B, int H_q, int H_kv, int D,
                          float scale, int chunk_tokens, int n_chunks_max,
                          void* ws, size_t ws_bytes, int cache_dt, int q_dt,
                          int out_dt, skv_stream_t stream);

/*
 * One decode step of one layer in one call: exactly skv_append followed by
 * skv_decode_attn (kv_cache_update then attention_with_kv_cache,
 * simple-llm/src/gpu/gpu_kv_cache.py:113-186, 194-289), without the
 * separate append launch. new_k, new_v: [B, H_kv, D] of in_dt. Sequence b
 * with 0 <= lens[b] < capacity writes its token at lens[b] (rounded to the
 * cache dtype) and attends [0, lens[b]]; others attend their clamped fill
 * unchanged. lens[b] is advanced on the device after the attention. The plan
 * (skv_decode_plan) must cover the lengths after the append.
 */
int skv_append_decode_attn(void* out, const void* q, void* k_cache, void* v_cache,
                           const void* new_k, const void* new_v, int32_t* lens, int B, int H_q,
                           int H_kv, int D, int T_cap, float scale, int chunk_tokens,
                           int n_chunks_max, void* ws, size_t ws_bytes, int cache_dt, int in_dt,
                           int q_dt, int out_dt, skv_stream_t stream);

/* Paged variant of skv_append_decode_attn. */
int skv_append_decode_attn_paged(void* out, const void* q, void* k_pool, void* v_pool,
                                 const void* new_k, const void* new_v, int32_t* lens,
                                 const int32_t* block_table, int max_blocks, int block_size,
                                 int B, int H_q, int H_kv, int D, float scale, int chunk_tokens,
                                 int n_chunks_max, void* ws, size_t ws_bytes, int cache_dt,
                                 int in_dt, int q_dt, int out_dt, skv_stream_t stream);

/*
 * Split count for skv_prefill_attn (host-only): about one workgroup per CU.
 * max_kv_end = the largest start[b] + n_new[b] of the call.
 */
int skv_prefill_plan(int B, int C, int H_q, int H_kv, int max_kv_end, int* n_splits /* host */);

/* Bytes of workspace skv_prefill_attn and skv_append_prefill_attn need (0
 * when n_splits == 1): the split partials, then B int32 (16-byte padded) that
 * skv_append_prefill_attn keeps the fills in. */
size_t skv_prefill_workspace_bytes(int B, int C, int H_q, int D, int n_splits);

/*
 * Causal attention of a chunk of queries over the cache (chunked prefill).
 * The reference's prefill analogue is flash_attention
 * (simple-llm/src/gpu/gpu_pass_forward.py:497-588, kernel
 * create_flash_attention_kernel simple-llm/src/gpu/gpu_kernels.py:499-770),
 * causal over a sequence with no cache prefix; this adds the prefix offset:
 *   out[b, i, h, :] = softmax(scale * q[b, i, h, :] . K[b, 0:start[b]+i+1, h/G, :]^T)
 *                     . V[b, 0:start[b]+i+1, h/G, :]     for i < n_new[b],
 * and zeros for i >= n_new[b]. The chunk's own K/V must already be in the
 * cache at positions start[b] .. start[b]+n_new[b]-1 (skv_append_chunk).
 * q, out: [B, C, H_q, D] of q_dt / out_dt; n_new may be NULL (C for all).
 * Requires start[b] + n_new[b] <= T_cap.
 * bf16 cache: Q, K, V and the probabilities enter v_mfma_f32_32x32x16_bf16
 * as bf16, accumulation and softmax are fp32; D from 1 to 256 (64, 128 and
 * 256 as they are, others padded to 32, 64, 128 or 256 with zeros; the
 * reference's largest flash_attn_max_head_dim is 256, gpu_device.py:468-471);
 * G = H_q / H_kv in {1, 2, 4, 8}; split over the prefix by n_splits; out, q,
 * the caches and ws 16-byte aligned.
 * fp32 cache: q and out fp32, every product in fp32 (v_mfma_f32_32x32x2_f32,
 * the kernel of skv_flash_fwd); D from 1 to 256, any G; n_splits and the
 * workspace are not used.
 */
int skv_prefill_attn(void* out, const void* q, const void* k_cache, const void* v_cache,
                     const int32_t* start, const int32_t* n_new, int B, int C, int H_q,
                     int H_kv, int D, int T_cap, float scale, int n_splits, void* ws,
                     size_t ws_bytes, int cache_dt, int q_dt, int out_dt, skv_stream_t stream);

/*
 * One chunked-prefill call of a layer: skv_append_chunk (the chunk's K/V
 * rows k_new, v_new [B, C, H_kv, D] of in_dt into the cache at lens[b]),
 * then skv_prefill_attn over the cache with start = lens, then the fills
 * advanced as skv_advance(lens, n_new, C, ...) does: the same outputs, cache
 * rows and fills as those three calls in a row. On the split bf16 path
 * (n_splits > 1) the attention keeps the fills in the workspace's tail and
 * its merge pass advances them, so there is no separate advance launch. All
 * of skv_prefill_attn's checks run before anything is launched, so a
 * rejected call changes nothing. The reference's kv_cache_update
 * (simple-llm/src/gpu/gpu_kv_cache.py:113-186) for a chunk of tokens
 * followed by its flash_attention (gpu_pass_forward.py:497-588) with the
 * cache prefix.
 */
int skv_append_prefill_attn(void* out, const void* q, void* k_cache, void* v_cache,
                            const void* k_new, const void* v_new, int32_t* lens,
                            const int32_t* n_new, int B, int C, int H_q, int H_kv, int D,
                            int T_cap, float scale, int n_splits, void* ws, size_t ws_bytes,
                            int cache_dt, int in_dt, int q_dt, int out_dt, skv_stream_t stream);

/* ------------------------------------------------------------------------
 * Decode-step ops of the model around the cache (fp32). They replace the
 * JAX model's per-token work (simple-llm/src/jax_backend.py:78-148) and the
 * greedy pick of generate_text (simple-llm/src/generate.py:29-69,
 * jax_backend.py:466-469), so a whole decode step runs on the GPU.
 * ------------------------------------------------------------------------ */

/* x[m, :] = embedding[ids[m], :] + pos_table[pos[m], :]
 * (jax_backend.py:144). ids and pos are clamped into the tables. */
int skv_embed(float* x, const int32_t* ids, const int32_t* pos, const float* embedding,
              const float* pos_table, int M, int d, int vocab, int ctx, skv_stream_t stream);

/* y[m, :] = (x[m, :] - mean) / sqrt(var + eps) * gamma + beta, population
 * variance (jax_backend.py:78-82). d <= 4096; y may equal x. */
int skv_layernorm(float* y, const float* x, const float* gamma, const float* beta, int M, int d,
                  float eps, skv_stream_t stream);

/* y = act(LN(x) . w_t^T + bias) + residual, x [M, K], w_t [N, K] (the
 * transpose of the reference's [K, N] weight), y [M, N]. activation 0 =
 * none, 1 = GELU, tanh form (jax.nn.gelu's default, jax_backend.py:127).
 * LN is the row LayerNorm with ln_gamma, ln_beta, ln_eps (both NULL: x as
 * is), folded into the reads of x (jax_backend.py:135, 138 put a LayerNorm
 * in front of the attention and MLP projections).
 * bias and residual may be NULL; residual may equal y, x may not.
 * split_cols > 0 writes column n to segment n / split_cols of a
 * [N / split_cols][M][split_cols] output (q, k, v of a fused projection as
 * three contiguous [M, d] blocks). K must be a multiple of 4. Sums run in a
 * fixed order, so results are reproducible run to run.
 * M <= 64 (a decode step's rows): a weight-streaming kernel. ws (may be
 * NULL) of skv_linear_workspace_bytes(M, N, K) bytes lets a narrow
 * projection (few 16-column tiles) split K over more workgroups; the split
 * sums in a different fixed order, so its bits differ from the unsplit
 * result within fp32 rounding. Without LayerNorm and with M <= 16 the last
 * workgroup of each tile to finish sums the split (arrival counters kept in
 * ws): ws must be zero-filled before its first use, and every call leaves
 * the counters at zero again; with LayerNorm a second kernel sums it.
 * M > 64 (a prompt's prefill): a tiled MFMA GEMM (128 x 128 tiles of
 * v_mfma_f32_32x32x2_f32); with LayerNorm, ws of
 * skv_linear_workspace_bytes(M, N, K) bytes holds the row statistics,
 * computed once (without it every column tile computes its rows' own).
 * Calls that share ws must be stream ordered. */
int skv_linear(float* y, const float* x, const float* w_t, const float* bias,
               const float* residual, const float* ln_gamma, const float* ln_beta, float ln_eps,
               int M, int N, int K, int activation, int split_cols, void* ws, size_t ws_bytes,
               skv_stream_t stream);

/* LayerNorm folded into a projection's weights for skv_linear_folded:
 * w_fold[n, k] = ln_gamma[k] * w_t[n, k], c1[n] = sum_k w_fold[n, k],
 * c2[n] = sum_k ln_beta[k] * w_t[n, k] + bias[n] (bias may be NULL), the
 * sums in double. w_fold [N, K] may not alias w_t; c1, c2 [N]. Run once per
 * weight set (no counterpart in the reference, which normalizes x and then
 * multiplies: jax_backend.py:135, 138). */
int skv_linear_fold_ln(float* w_fold, float* c1, float* c2, const float* w_t,
                       const float* ln_gamma, const float* ln_beta, const float* bias, int N,
                       int K, skv_stream_t stream);

/* y = act(LN(x) . w_t^T + bias) + residual, as skv_linear with LayerNorm,
 * from the folded weights of skv_linear_fold_ln:
 *   LN(x)[m] . w_t[n] + bias[n] = rstd_m (sum_k (x[m, k] - c_m) w_fold[n, k]
 *                                 - (mean_m - c_m) c1[n]) + c2[n],
 * c_m = x[m, 0], so the products start before the row statistics are known.
 * M <= 16 rows; K = 16 * s * w for some s in {3, 4, 6, 8, 12} and 4 <= w <=
 * 16 (768, 1024, 3072, ...); otherwise SKV_E_UNSUPPORTED. residual may
 * equal y, x may not; split_cols as for skv_linear. The rounding differs
 * from skv_linear's within fp32 accuracy; sums run in a fixed order. */
int skv_linear_folded(float* y, const float* x, const float* w_fold, const float* c1,
                      const float* c2, const float* residual, float ln_eps, int M, int N, int K,
                      int activation, int split_cols, skv_stream_t stream);

/* Bytes of skv_linear_pack's copy of a [N, K] weight matrix (0 if K is not
 * a multiple of 16): N rounded up to 16 rows. */
size_t skv_linear_packed_bytes(int N, int K);

/* Copies w_t [N, K] into the matrix-core lane order skv_linear_packed reads:
 * 16-column tiles, then 16-k steps, then 64 lanes of 4 floats (lane l holds
 * w_t[16 t + l % 16, 16 s + 4 (l / 16) .. + 3]), rows past N zero. Run once
 * per weight set (no counterpart in the reference, whose weights are used in
 * place). */
int skv_linear_pack(float* w_packed, const float* w_t, int N, int K, skv_stream_t stream);

/* y = act(x . w^T + bias) + residual from skv_linear_pack's copy of w, for
 * one row tile over many columns (the tied logits projection): M <= 16,
 * K in {512, 768, 1024}, 16384 <= N <= 65536; otherwise SKV_E_UNSUPPORTED.
 * Every 16-k step of a tile is 1 KB of consecutive bytes, streamed by 16
 * wavefronts per CU; sums run in a fixed order (its own, so the bits may
 * differ from skv_linear's within fp32 rounding). argmax_cand (may be NULL;
 * skv_linear_packed_cand_bytes(M) bytes): each of the 256 workgroups also
 * writes, per row, the first maximum of y over its columns (value, column),
 * the first step of the argmax that skv_next_embed finishes. */
int skv_linear_packed(float* y, const float* x, const float* w_packed, const float* bias,
                      const float* residual, int M, int N, int K, int activation,
                      float* argmax_cand, skv_stream_t stream);

/* Workspace skv_linear can use for these sizes: the split-K partials (and
 * arrival counters) of a narrow projection of at most 64 rows (0: it never
 * splits them), or, for more than 64 rows, M * 2 floats of LayerNorm row
 * statistics. Zero-fill it once before the first call. */
size_t skv_linear_workspace_bytes(int M, int N, int K);

/* y[m, :] = x[rows[m], :] for m < M, x [n_rows, d] (rows clamped into
 * [0, n_rows)); y and x must not overlap. The prefill's last prompt row of
 * each sequence goes to the logits projection this way (the reference's
 * generate_text takes logits[0, -1], generate.py:52). */
int skv_gather_rows(float* y, const float* x, const int32_t* rows, int M, int d, int n_rows,
                    skv_stream_t stream);

/* Workspace of skv_argmax: per-slice candidates, 0 bytes when N <= 2048
 * (ws may then be NULL); calls that share it must be stream ordered. */
size_t skv_argmax_workspace_bytes(int M, int N);

/* out[m] = index of the largest x[m, :], the first on ties
 * (jnp.argmax, jax_backend.py:469). */
int skv_argmax(int32_t* out, const float* x, int M, int N, void* ws, size_t ws_bytes,
               skv_stream_t stream);

/*
 * Next token of each row drawn from its logits, as sample_token
 * (simple-llm/src/jax_backend.py:413-515) filters them:
 *  - repetition_penalty divides, once per distinct token, the logits of the
 *    tokens in seq[m, max(0, L - repetition_window) : L], L = lens[m];
 *  - temperature == 0: out[m] = first index of the maximum (greedy);
 *  - else p = softmax(logits / temperature); then, when enabled, min_p
 *    (p < min_p * max p -> 0), top_k (the top_k largest; of equal
 *    probabilities the larger index ranks higher) and top_p (the longest
 *    prefix of the descending order whose sum stays <= top_p, at least one
 *    entry), renormalising after each filter;
 *  - out[m] = the first index, in index order, where the running sum of p
 *    exceeds u * sum(p), u = splitmix64(seed, m, L) in [0, 1). The
 *    reference's jax.random stream is not reproduced; a call is bitwise
 *    reproducible for the same inputs.
 * logits [M, V] fp32 (not modified), V <= 65536; seq [M, seq_stride] int32;
 * probs_out (may be NULL): [M, V] fp32, the filtered distribution the draw
 * used (one-hot for greedy). Disabled filters: top_k = 0, top_p >= 1,
 * min_p = 0, repetition_penalty = 1.
 * ws (may be NULL; 8-byte aligned) of skv_sample_workspace_bytes(M, V)
 * bytes: an unfiltered draw (temperature > 0, no min-p, top-k or top-p, no
 * probs_out; the penalty allowed) from rows of 8192 entries or more then
 * runs split over 2048-entry slices (two launches, many workgroups per row)
 * instead of one workgroup per row; its running sums are grouped by slice,
 * so a u * sum within float rounding of a step may draw the neighbouring
 * token: the same seed and logits can therefore give a different token with
 * ws than without it (only at such rounding boundaries; both draw from the
 * same filtered distribution). Calls that share ws must be stream ordered.
 */
int skv_sample(int32_t* out, float* probs_out, const float* logits, const int32_t* seq,
               int seq_stride, const int32_t* lens, int M, int V, float temperature, int top_k,
               float top_p, float min_p, float repetition_penalty, int repetition_window,
               unsigned long long seed, void* ws, size_t ws_bytes, skv_stream_t stream);

/* Workspace of skv_sample's split path: M * ceil(V / 2048) * 8 bytes for
 * 8192 <= V <= 65536, else 0 (the one-workgroup-per-row kernel). */
size_t skv_sample_workspace_bytes(int M, int V);

/* Next input token of each sequence (generate.py:29-69 with a cache):
 * ids[b] = prompt[b, pos[b]] while pos[b] < prompt_len[b], else
 * argmax_prev[b]; the token is also stored at seq[b, pos[b]] when
 * 0 <= pos[b] < seq_cap. pos is the sequence's current fill (layer 0's
 * lens). stop (may be NULL; then lens_all and n_layers are unused): per
 * row, the length it is generated to. Once the token at position
 * stop[b] - 1 is recorded, the row retires: lens_all[l * B + b] = -1 for
 * every layer l < n_layers (lens_all: the n_layers per-layer fill arrays,
 * contiguous, pos being the first). The decode kernels treat a negative
 * fill as an empty row (no append, no advance, zero output), and the
 * next-token calls record nothing for it, so a batch whose rows end at
 * different lengths stops reading the cache of the rows that are done.
 * adv (may be NULL; int32 [B], zero after a prefill): the deferred fill
 * advance of skv_append_decode_attn_direct. Where adv[b] is set, every
 * layer's fill of row b first moves one past the previous step's token
 * (up to seq_cap, none for a negative fill), and pos[b] is that fill; adv[b]
 * is then set for this step's append. */
int skv_next_tokens(int32_t* ids, int32_t* seq, const int32_t* argmax_prev,
                    const int32_t* prompt, const int32_t* prompt_len, const int32_t* pos, int B,
                    int max_prompt, int seq_cap, const int32_t* stop, int32_t* lens_all,
                    int n_layers, int32_t* adv, skv_stream_t stream);

/* skv_append_decode_attn for one query head per kv head (MHA), a
 * contiguous cache (16-byte aligned for fp32, 8-byte for bf16; otherwise
 * SKV_E_UNSUPPORTED) and head_dim 64 or 128, WITHOUT the fill advance: each
 * (sequence, head) gets n_split workgroups (1, 2 or 4) that read its filled
 * row in n_split equal parts, fold in the new token (stored at lens[b] when
 * lens[b] in [0, T_cap)) and write the output; no merge pass. With n_split >
 * 1 the last workgroup of a (sequence, head) to finish merges the parts'
 * partials, in part order (the bits do not depend on which one finishes
 * last), from ws: skv_decode_direct_workspace_bytes(B, H, D, n_split) bytes,
 * zero-filled before its first use; every call leaves its arrival counters
 * at zero again, and calls that share ws must be stream ordered (ws may be
 * NULL for n_split = 1). lens is left as it was: the caller advances it
 * before the next step (skv_next_embed with advance set does, for every
 * layer). A negative fill is an empty row (output 0, nothing stored). The
 * reference's attention_with_kv_cache (gpu_kv_cache.py:194-289) with its
 * kv_cache_update (:113-186), for the decode step's one token per sequence;
 * sums run in another order than the split kernels', so the bits may differ
 * within fp32 rounding. */
int skv_append_decode_attn_direct(void* out, const void* q, void* k_cache, void* v_cache,
                                  const void* new_k, const void* new_v, const int32_t* lens,
                                  int B, int H, int D, int T_cap, float scale, int cache_dtype,
                                  int in_dtype, int q_dtype, int out_dtype, int n_split, void* ws,
                                  size_t ws_bytes, skv_stream_t stream);

/* Workspace of skv_append_decode_attn_direct with n_split parts: a fixed
 * 256 KiB block of arrival counters (B * H <= 65536), then B * H * n_split
 * partials (o[D], m, l); 0 for n_split <= 1. The fixed block lets calls of
 * any shape share one zero-filled workspace. */
size_t skv_decode_direct_workspace_bytes(int B, int H, int D, int n_split);

/* Bytes of skv_linear_packed's argmax candidates for M rows: [M][256]
 * float values, then [M][256] int32 columns (one per workgroup). */
size_t skv_linear_packed_cand_bytes(int M);

/* y = x . w_t^T + bias (bias may be NULL) for M <= 16 rows, as skv_linear
 * computes it, with each row's argmax candidates in argmax_cand
 * (skv_linear_cand_bytes(M, N, K) bytes): for every 16-column tile j of N,
 * [M][ceil(N / 16)] float values (the first maximum of row m over columns
 * [16 j, 16 j + 16); larger value, or equal value and smaller column; NaN
 * never wins), then [M][ceil(N / 16)] int32 columns, for skv_next_embed with
 * n_cand = ceil(N / 16). K must be 16 s w with s in {3, 4, 6, 8, 12} and
 * 4 <= w <= 16 (48..3072), else SKV_E_UNSUPPORTED. ws (may be NULL) of
 * skv_linear_workspace_bytes(M, N, K) bytes lets a narrow projection split
 * K, as for skv_linear (zero-filled before its first use, stream ordered).
 * The tied logits
 * projection (jax_backend.py:147) for vocabularies skv_linear_packed does
 * not take, and the first step of the greedy pick (jnp.argmax,
 * jax_backend.py:469) that skv_next_embed finishes. */
int skv_linear_cand(float* y, const float* x, const float* w_t, const float* bias, int M, int N,
                    int K, float* argmax_cand, void* ws, size_t ws_bytes, skv_stream_t stream);

/* Bytes of skv_linear_cand's candidates: M * ceil(N / 16) * 8, or 0 when
 * skv_linear_cand does not take M and K. */
size_t skv_linear_cand_bytes(int M, int N, int K);

/* skv_next_tokens and skv_embed in one launch, ending the argmax: with
 * n_cand > 0 the previous token of row b is the first maximum over its
 * n_cand candidates (cand: [B][n_cand] float values, then [B][n_cand] int32
 * columns, as skv_linear_packed and skv_linear_cand write them; a row of
 * NaN only gives token 0), else argmax_prev[b]. Then ids[b] and seq as skv_next_tokens, and, when
 * embedding is not NULL, x[b, :] = embedding[ids[b], :] + pos_table[pos[b], :]
 * as skv_embed (ids and positions clamped into the tables); stop, lens_all,
 * n_layers and adv retire finished rows and advance the fills as in
 * skv_next_tokens. No counterpart
 * in the reference, whose generate loop picks and embeds on the host side
 * (generate.py:29-69, jax_backend.py:144, 466-469). */
int skv_next_embed(float* x, int32_t* ids, int32_t* seq, const int32_t* argmax_prev,
                   const float* cand, int n_cand, const int32_t* prompt,
                   const int32_t* prompt_len, const int32_t* pos, int B, int max_prompt,
                   int seq_cap, const float* embedding, const float* pos_table, int d, int vocab,
                   int ctx, const int32_t* stop, int32_t* lens_all, int n_layers, int32_t* adv,
                   skv_stream_t stream);

/* ------------------------------------------------------------------------
 * Training-side attention in fp32: causal FlashAttention forward and backward.
 * ------------------------------------------------------------------------ */

/*
 * Causal attention with the softmax statistics, replacing flash_attention
 * (simple-llm/src/gpu/gpu_pass_forward.py:497-588, kernel
 * create_flash_attention_kernel simple-llm/src/gpu/gpu_kernels.py:499-770):
 * per batch b and head h, with S = scale * Q K^T over keys <= query,
 *   M = row max of S, L = sum exp(S - M), out = softmax(S) V.
 * q, k, v, out: [B, N, H, D] fp32 (the reference's [B*N, H*D] buffers),
 * 16-byte aligned; L, M: [B, N, H] fp32, or NULL to skip them.
 * D from 1 to 256 (the reference's flash_attn_max_head_dim is 128 by
 * default, gpu_types.py:93, and at most 256, gpu_device.py:468-471): the
 * kernel runs at D padded to a multiple of 16 up to 128, to 192 or 256
 * past it, with zeros past D. Products on v_mfma_f32_32x32x2_f32 (fp32).
 */
int skv_flash_fwd(float* out, float* L, float* M, const float* q, const float* k, const float* v,
                  int B, int N, int H, int D, float scale, skv_stream_t stream);

/* Bytes of workspace skv_flash_bwd needs: the row deltas, B*N*H floats. */
size_t skv_flash_bwd_workspace_bytes(int B, int N, int H);

/* Bytes of workspace that let skv_flash_bwd run its five-product form: for
 * D <= 64, the row deltas (a 256-byte aligned block) and then dS in 32 x 32
 * tiles, B*H*ceil(N/32)^2*1024 floats; otherwise
 * skv_flash_bwd_workspace_bytes. No reference
 * counterpart: the reference's own grad_K_workspace, num_q_blocks full copies
 * of dK (gpu_pass_backward.py:522-530), is usually this size or more (head_dim
 * at least its block rows and N a multiple of 32); skv_flash_bwd takes the
 * five-product form whenever ws_bytes is this size. */
size_t skv_flash_bwd_fast_workspace_bytes(int B, int N, int H, int D);

/*
 * Gradients of causal attention, replacing flash_attention_backward and its
 * reduce pass (simple-llm/src/gpu/gpu_pass_backward.py:445-580, kernels
 * create_flash_attention_backward_kernel and _reduce_kernel,
 * simple-llm/src/gpu/gpu_kernels.py:2038-2455). Per batch b and head h, with
 * S = scale * Q K^T over keys <= query:
 *   P = exp(S - M) / L, Dl = rowsum(dO * O), dS = P * (dO V^T - Dl),
 *   dq = scale * dS K, dk = scale * dS^T Q, dv = P^T dO.
 * q, k, v, o, dout, dq, dk, dv: [B, N, H, D] fp32 (the reference's
 * [B*N, H*D] buffers), 16-byte aligned; L, M: [B, N, H] fp32, the forward's
 * softmax sums and row maxima of the scaled scores (the reference's L and M
 * buffers). The outputs must not overlap the inputs. D from 1 to 256. Past
 * 128 the head dim is padded to 192 or 256 and the kernels, which keep two
 * 32-row operands and an accumulator of the head dim per wavefront, spill
 * part of them to scratch: correct, but far below the narrow shapes' rate.
 * Products run on v_mfma_f32_32x32x2_f32 (fp32); no atomics, so results are
 * bitwise reproducible. Two forms, by the workspace: with
 * skv_flash_bwd_workspace_bytes, dQ recomputes S and dP (seven products);
 * with skv_flash_bwd_fast_workspace_bytes (D <= 64), the dK/dV
 * kernel writes dS and dQ is formed from it (five products, dS written and
 * read once). Both give the same bits.
 */
int skv_flash_bwd(float* dq, float* dk, float* dv, const float* q, const float* k, const float* v,
                  const float* o, const float* L, const float* M, const float* dout, int B, int N,
                  int H, int D, float scale, void* ws, size_t ws_bytes, skv_stream_t stream);

/* ------------------------------------------------------------------------
 * Byte-level BPE tokenizer (host code, no device work), replacing the
 * reference's C tokenizer (simple-llm/src/common/bpe_tokenizer.c) that
 * common/bpe_tokenizer.py runs as a subprocess.
 * ------------------------------------------------------------------------ */

/* Training (bpe_tokenizer.c:155-243): merges of the corpus bytes, as
 * (p1, p2, new_id) triples in order, new_id = 256 + i; at most
 * min(vocab_size, 50000) - 256 merges, fewer if the pairs run out. Ties take
 * the first pair of the reference's hash-table order. merges holds
 * max_merges triples (>= vocab_size - 256). */
int skv_bpe_train(const uint8_t* corpus, size_t n, int vocab_size, int32_t* merges,
                  int max_merges, int* n_merges);

/* Encoding (bpe_tokenizer.c:246-355): one pass; a pair of raw bytes that is
 * a merge becomes the first such merge's id, any other byte stays. ids holds
 * n entries; *n_ids gets the count. */
int skv_bpe_encode(const uint8_t* text, size_t n, const int32_t* merges, int n_merges,
                   int32_t* ids, size_t* n_ids);

#ifdef __cplusplus
}
#endif

#endif /* SKV_H_ */

/*
 * dsa_amd.h -- C ABI of the MI355X (gfx950) DeepSeek-sparse-attention decode path.
 *
 * Library: nanoengine_amd/libdsa_amd.so (hipcc, --offload-arch=gfx950).
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers; sizes and strides are in ELEMENTS of the
 *     pointed-to type unless the name ends in `_bytes`.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Kernels are launched asynchronously on it; nothing synchronises the
 *     host, nothing allocates, so every call is capturable in a HIP graph.
 *   - The caller owns and allocates every output and workspace.
 *   - Return value: 0 on success, otherwise a dsa status code
 *     (1 invalid argument, 2 unsupported shape, 3 launch failure,
 *     4 workspace too small); dsa_last_error() then describes the failure.
 *
 * Citations name the reference interface (nano-infra/NanoEngine, package
 * dlengine) that each entry point replaces.
 */
#ifndef DSA_AMD_H_
#define DSA_AMD_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define DSA_API __attribute__((visibility("default")))
#else
#define DSA_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Library version (major*10000 + minor*100 + patch). */
DSA_API int dsa_version(void);

/* Message for the last non-zero status returned on this thread. */
DSA_API const char* dsa_last_error(void);

/* Compute units of `device`.
 * Replaces deep_gemm.get_num_sms() (called at
 * dlengine/runtime/layers/backends/dsa/indexer/lightning.py:633). */
DSA_API int dsa_num_cus(int device);

/* Largest score-row length the top-k kernels accept (positions per row). */
DSA_API int dsa_topk_max_len(void);

/* Indexer work schedule. Writes `batch + 1` int32 values to
 * `schedule_out`: the exclusive prefix sum of per-sequence page counts
 * ceil(max_j context_lens[b, j] / page_size). The logits kernel does not need
 * it (its grid covers every page with early exit), but the call exists so the
 * caller's once-per-forward schedule step stays in place.
 * Replaces deep_gemm.get_paged_mqa_logits_metadata(context_lens, page_size,
 * num_sms) (lightning.py:668-676; built once per forward at
 * dlengine/runtime/models/deepseek_v2/deepseek_v2.py:807-840). */
DSA_API int dsa_indexer_schedule(const int32_t* context_lens, int batch, int next_n,
                         int page_size, int32_t* schedule_out, void* stream);

/* fp8 lightning-indexer logits over the paged indexer cache.
 *   q_fp8        [batch, next_n, num_heads=64, head_dim=128] e4m3fn bytes, contiguous
 *   kv_cache     [num_pages, page_size*132] bytes; page = [page_size x 128 fp8][page_size x f32 scale]
 *   weights      [batch*next_n, num_heads] f32 (q scale and softmax scale folded in)
 *   context_lens [batch, next_n] int32 (per-query causal length)
 *   block_tables [batch, >= ceil(max_ctx/page_size)] int32, row stride `block_table_stride`
 *   logits       [batch*next_n, max_context_len] f32, row stride `logits_stride`
 * logits[b*n+j, t] = sum_h weights[b*n+j, h] * relu(q[b,j,h,:] . k[t,:]) * scale[t]
 * for t < context_lens[b, j]; positions past the context inside the last page
 * are written as -inf, later positions are not written.
 * next_n in {1, 2}; page_size == 64; num_heads == 64; head_dim == 128.
 * Replaces deep_gemm.fp8_paged_mqa_logits(q_fp8, kv_cache, weights,
 * context_lens, block_tables, schedule_meta, max_context_len,
 * clean_logits=False) (lightning.py:1395-1406). */
DSA_API int dsa_indexer_logits(const uint8_t* q_fp8, const uint8_t* kv_cache,
                       const float* weights, const int32_t* context_lens,
                       const int32_t* block_tables, int64_t block_table_stride,
                       int batch, int next_n, int num_heads, int head_dim,
                       int page_size, int64_t max_context_len,
                       float* logits, int64_t logits_stride, void* stream);

/* Workspace bytes dsa_indexer_topk needs for this shape. */
DSA_API size_t dsa_indexer_topk_workspace_bytes(int batch, int next_n, int64_t max_context_len);

/* Fused decode indexer + exact top-k + page translation, without materialising
 * the logits. Inputs as dsa_indexer_logits; outputs as dsa_topk_transform:
 *   out_physical [batch*next_n, top_k] int32 cache slots
 *                block_tables[row / next_n, pos / 64] * 64 + pos % 64, -1 padded
 *   out_logical  [batch*next_n, top_k] int32 token positions (may be NULL)
 * The translation goes through the indexer's own block_tables at the indexer's
 * page size (page_size == 64): a caller whose MLA cache uses another block size
 * must translate with dsa_topk_to_physical instead.
 * Selection, order (ascending position), ties (lowest positions) and padding are
 * those of dsa_topk_transform over dsa_indexer_logits' logits, exactly.
 * Launch sequence on `stream`: logits of 16 sampled pages per row -> per-row
 * score threshold -> all pages, keeping only (key, position) of tokens at or
 * above the threshold in per-row lists -> exact top-k of each list; a row whose
 * list is unusable (fewer than top_k or more than the list capacity) is redone
 * inside that last launch, by the row's workgroup, from the row's full logits.
 * phase_events: NULL, or five hipEvent_t (entries may be NULL) recorded on
 * `stream` before the first launch and after the sample, filter and select
 * phases (the last two entries both after the select), for timing.
 * top_k in {512, 2048}; rows of at most dsa_topk_max_len() positions. The
 * workspace (dsa_indexer_topk_workspace_bytes) should be zero-filled before its
 * first use; a stale one gives the same results, its first call more slowly.
 * Replaces the kernel sequence of Indexer.forward(..., translate_topk=True)
 * (deep_gemm.fp8_paged_mqa_logits then topk_transform, lightning.py:1395-1466;
 * chosen by _can_use_fused_indexer_topk, deepseek_v2.py:78-81, 1917-1935). */
DSA_API int dsa_indexer_topk(const uint8_t* q_fp8, const uint8_t* kv_cache, const float* weights,
                             const int32_t* context_lens, const int32_t* block_tables,
                             int64_t block_table_stride, int batch, int next_n, int num_heads,
                             int head_dim, int page_size, int64_t max_context_len, int top_k,
                             int32_t* out_physical, int32_t* out_logical, void* workspace,
                             size_t workspace_bytes, void* stream, void* const* phase_events);

/* Workspace bytes the top-k entry points use for `batch` rows (per-row
 * threshold, counter, flag and a 6144-entry (key, position) candidate list:
 * 48 KB + 16 B a row). */
DSA_API size_t dsa_topk_workspace_bytes(int batch);

/* Exact top-k selection with page-table translation.
 *   scores          [batch, >= seq_lens[b]] f32, row stride `score_stride`
 *   seq_lens        [batch] int32
 *   page_table      [batch, ...] int32, row stride `page_table_stride`, or NULL:
 *                   then out_page receives the raw positions (no translation)
 *   out_page        [batch, top_k] int32, contiguous
 *   out_raw         [batch, top_k] int32 or NULL
 *   workspace       >= dsa_topk_workspace_bytes(batch) bytes, 16-byte aligned,
 *                   or NULL (then every row takes the slower multi-pass path;
 *                   the result is the same)
 * Row b selects the top_k largest scores among positions [0, seq_lens[b])
 * (ties: lowest positions; NaN ranks as -inf), writes them in ascending
 * position order as raw positions and as slots
 * (page_table[p >> log2(page_size)] << log2(page_size)) | (p & (page_size-1)),
 * then pads with -1. seq_lens[b] <= top_k emits 0..seq_lens[b]-1.
 * top_k in {512, 2048}; page_size a power of two;
 * row length <= dsa_topk_max_len(); `max_len` bounds seq_lens (the score width).
 * Calls that share a workspace must be ordered (same stream).
 * Replaces topk_transform(scores, seq_lens, page_tables, out_page_indices,
 * page_size, top_k, out_raw_indices)
 * (dlengine/runtime/kernel/jit/sgl/deepseek_v4.py:324-367,
 *  kernel csrc/deepseek_v4/topk.cuh:249-287, host TopKKernel::transform :336-394). */
DSA_API int dsa_topk_transform(const float* scores, int64_t score_stride,
                               const int32_t* seq_lens, const int32_t* page_table,
                               int64_t page_table_stride, int32_t* out_page,
                               int32_t* out_raw, int batch, int64_t max_len,
                               int page_size, int top_k, void* workspace,
                               size_t workspace_bytes, void* stream);

/* dsa_topk_transform without a workspace argument and without any allocation:
 * the per-row state lives in a fixed device array of the library (12.6 MB per
 * GPU, held until the process ends), for at most 256 rows (more: status
 * kUnsupported). Results are those of dsa_topk_transform. Calls on one GPU
 * share that array: calls that overlap in time on one device (different
 * streams, or different host threads without ordering) race and must not be
 * made. The kernels reset the state they use, so no clearing is needed
 * between calls.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (HIP graph capture, allocation-free serving loops). */
DSA_API int dsa_topk_transform_noalloc(const float* scores, int64_t score_stride,
                                       const int32_t* seq_lens, const int32_t* page_table,
                                       int64_t page_table_stride, int32_t* out_page,
                                       int32_t* out_raw, int batch, int64_t max_len,
                                       int page_size, int top_k, void* stream);

/* The portable selection tail of the decode indexer (no page translation):
 * row r selects the top_k largest logits among positions [0, context_lens[r]),
 * where a logit that is not finite or has |x| >= 1e30 ranks as -inf; writes
 * the positions in ascending order, then pads with -1. Ties (including the
 * -inf ones) go to the lowest positions. top_k in {512, 2048}; workspace as
 * for dsa_topk_transform.
 * Replaces the non-translating branch of Indexer.forward: masked_fill of
 * t >= ctx, torch.where(isfinite & |x| < 1e30), torch.topk, indices >= ctx
 * -> -1 and the -1 padding
 * (dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1468-1492). */
DSA_API int dsa_indexer_select(const float* logits, int64_t logits_stride,
                               const int32_t* context_lens, int32_t* out, int rows,
                               int64_t max_len, int top_k, void* workspace,
                               size_t workspace_bytes, void* stream);

/* Ragged exact top-k: row b selects among scores[b, row_starts[b] +
 * [0, seq_lens[b])] and writes position + offsets[b], ascending, padded -1.
 * top_k == 2048. Exact (the reference's bounded candidate buffer allows a few
 * differences; this kernel has none). Workspace as for dsa_topk_transform.
 * Replaces topk_transform_ragged(scores, seq_lens, row_starts, offsets,
 * out_indices, top_k) (deepseek_v4.py:370-388, topk.cuh:289-316). */
DSA_API int dsa_topk_transform_ragged(const float* scores, int64_t score_stride,
                                      const int32_t* seq_lens, const int32_t* row_starts,
                                      const int32_t* offsets, int32_t* out,
                                      int batch, int64_t max_len, int top_k,
                                      void* workspace, size_t workspace_bytes, void* stream);

/* Logical token positions -> physical cache slots.
 *   topk_indices [rows, topk] int32, row stride `topk_stride` (-1 = padding)
 *   block_table  [rows / rows_per_table, table_width] int32, row stride `bt_stride`
 *   out          [rows, topk] int32, contiguous
 * out = block_table[r / rows_per_table, i / block_size] * block_size + i % block_size,
 * -1 kept; a position whose page lies beyond table_width also maps to -1.
 * rows_per_table = next_n expresses block_tables.repeat_interleave(next_n)
 * (deepseek_v2.py:1940-1946) without materialising it.
 * Replaces topk_indices_to_physical(topk_indices, block_table, block_size)
 * (dlengine/runtime/layers/backends/attention/mla_utils.py:237-272). */
DSA_API int dsa_topk_to_physical(const int32_t* topk_indices, int64_t topk_stride,
                         const int32_t* block_table, int64_t bt_stride,
                         int table_width, int rows, int topk, int rows_per_table,
                         int block_size, int32_t* out, void* stream);

/* Split count the sparse MLA decode uses for this shape (1 = no workspace). */
DSA_API int dsa_sparse_mla_num_splits(int num_tokens, int num_heads, int topk, int num_cus);

/* Workspace bytes dsa_sparse_mla_decode needs for `num_splits`. */
DSA_API size_t dsa_sparse_mla_workspace_bytes(int num_tokens, int num_heads, int num_splits);

/* Sparse MLA decode over the packed fp8 MLA cache.
 *   q        [num_tokens, num_heads, 576] bf16, row stride q_token_stride,
 *            head stride q_head_stride (elements; last dim contiguous)
 *   kv_cache block b row r at kv_cache + b*kv_block_stride_bytes + r*656:
 *            [512 e4m3fn][4 x f32 tile scale][64 x bf16 rope]; the tile
 *            scales are powers of two, as the reference's writer produces
 *            (2^ceil(log2(amax/448)), fp8_utils.py:32-108) and the kernel
 *            reads them as E8M0 exponents
 *   kv_num_blocks  blocks in the cache: a slot whose block is >= this (or a
 *            negative slot) is skipped like -1, so a stale index never reads
 *            outside the cache
 *   indices  [num_tokens, topk] int32 physical slots (block*kv_block_size+row),
 *            row stride idx_stride, -1 = skip
 *   out      [num_tokens, num_heads, 512] bf16, contiguous
 *   lse      [num_tokens, num_heads] f32 natural-log LSE, contiguous (may be NULL)
 * o = softmax(sm_scale * q . kv) @ kv[:, :512] over valid indices; a token with
 * no valid index yields o = 0 and lse = -inf.
 * num_heads % 16 == 0; topk % 64 == 0; num_splits in [1, topk/64] with
 * workspace >= dsa_sparse_mla_workspace_bytes(...) when num_splits > 1
 * (num_splits <= 0 picks dsa_sparse_mla_num_splits for this device).
 * Replaces flash_mla.flash_mla_with_kvcache(q, k_cache, None, None,
 * head_dim_v=512, sched_meta, None, softmax_scale, causal=False,
 * is_fp8_kvcache=True, indices=...) as called by FlashMlaAttention.forward
 * (dlengine/runtime/layers/backends/mla/flash_mla.py:76-99). */
DSA_API int dsa_sparse_mla_decode(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                          const uint8_t* kv_cache, int64_t kv_block_stride_bytes,
                          int kv_block_size, int64_t kv_num_blocks,
                          const int32_t* indices, int64_t idx_stride,
                          int num_tokens, int num_heads, int topk, float sm_scale,
                          void* out, float* lse, int num_splits,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Quantise and store MLA KV rows into the packed fp8 cache.
 *   kv          [num_tokens, 576] bf16 (row stride kv_row_stride elements, 16-byte aligned rows)
 *   slots       [num_tokens] physical slots (int32, or int64 when slot_is_64), < 0 skipped
 *   kv_cache    block b row r at kv_cache + b*kv_block_stride_bytes + r*656
 * Row: e4m3fn(nope / s_t) for the four 128-dim tiles, s_t = 2^ceil(log2(max(amax_t/448,
 * 1e-12))) as f32, then the 64 rope values as bf16.
 * Replaces store_kcache_fp8(k, k_cache, slot_mapping)
 * (dlengine/runtime/kernel/triton/hopper/fp8_utils.py:202-305, called at
 *  dlengine/runtime/layers/backends/mla/flash_mla.py:42). */
DSA_API int dsa_mla_kv_store(const void* kv, int64_t kv_row_stride, const void* slots,
                             int slot_is_64, int num_tokens, uint8_t* kv_cache,
                             int64_t kv_block_stride_bytes, int kv_block_size, void* stream);

/* Quantise and store indexer keys into the split page layout.
 *   k           [num_tokens, 128] bf16 (row stride k_row_stride elements)
 *   slots       [num_tokens] flat slots (int32, or int64 when slot_is_64), < 0 skipped
 *   cache       [pages, page_size*132] bytes
 * code = e4m3fn(x / sf), sf = 2^ceil(log2(max(amax, 1e-4) / 448)); fp8 at
 * page*page_size*132 + off*128, f32 scale at page*page_size*132 + page_size*128 + off*4.
 * Replaces IndexerCache.store_key_fp8 / store_indexer_key_fp8_fused
 * (dlengine/runtime/layers/backends/dsa/indexer/lightning.py:449-535,
 *  dlengine/runtime/kernel/triton/generic/fp8_ue8m0_quant.py:369-440). */
DSA_API int dsa_indexer_k_store(const void* k, int64_t k_row_stride, const void* slots,
                                int slot_is_64, int num_tokens, uint8_t* cache, int page_size,
                                void* stream);

/* Indexer query prologue: RoPE -> Hadamard-128 -> UE8M0 fp8 quant -> gate scaling.
 *   q            [num_tokens, num_heads, 128] bf16, contiguous, 16-byte aligned
 *   gate         [num_tokens, num_heads] bf16, token stride gate_token_stride elements
 *   cos_sin_cache [cache_positions, 64] f32 = [cos 0..31 | sin 0..31] per position
 *   positions    [num_tokens] (int32, or int64 when pos_is_64), clamped to the cache
 *   q_fp8        [num_tokens, num_heads, 128] e4m3fn codes (out)
 *   weights_out  [num_tokens, num_heads] f32 = gate * weight_scale * sf (out)
 * Dims 0..63 are interleaved (re, im) pairs when rope_interleaved (reordered to
 * the half layout first), else already in the half layout. RoPE output and the
 * Hadamard output (times 128^-0.5) are rounded to bf16; then per row
 * sf = 2^ceil(log2(max(amax, 1e-4) / 448)), code = e4m3fn(x / sf).
 * Replaces indexer_q_rope_hadamard_quant(query, gate_weight, weight_scale,
 * cos_sin_cache, positions) (dlengine/runtime/kernel/jit/sgl/deepseek_v4.py:290-322,
 * kernel jit/sgl/csrc/deepseek_v4/indexer_q.cuh:57-225; called at
 * dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1316-1325). */
DSA_API int dsa_indexer_q_prologue(const void* q, const void* gate, int64_t gate_token_stride,
                                   float weight_scale, const float* cos_sin_cache,
                                   int64_t cache_positions, const void* positions, int pos_is_64,
                                   int num_tokens, int num_heads, int rope_interleaved,
                                   uint8_t* q_fp8, float* weights_out, void* stream);

/* Indexer key transform + cache store: LayerNorm -> RoPE -> Hadamard-128 -> UE8M0
 * fp8 quant -> split-page store.
 *   key          [num_tokens, 128] bf16 (row stride key_row_stride elements, 16-byte aligned rows)
 *   ln_weight, ln_bias [128] f32; eps the LayerNorm epsilon
 *   cos_sin_cache, positions as for dsa_indexer_q_prologue; dims 0..63 of the
 *                LayerNorm output are interleaved (re, im) pairs
 *   slots        [num_tokens] flat slots (int32, or int64 when slot_is_64), < 0 skipped
 *   cache        [pages, page_size*132] bytes, layout as for dsa_indexer_k_store
 * The LayerNorm output and the RoPE output are rounded to bf16; the Hadamard
 * output (times 128^-0.5) stays f32 for the quantisation.
 * Replaces indexer_k_transform_store_fp8(key, weight, bias, eps, positions,
 * cos_sin_cache, cache, slot_mapping, page_size)
 * (dlengine/runtime/kernel/triton/generic/indexer_transform.py:156-288, called at
 *  dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1339-1350). */
DSA_API int dsa_indexer_k_transform_store(const void* key, int64_t key_row_stride,
                                          const float* ln_weight, const float* ln_bias, float eps,
                                          const float* cos_sin_cache, int64_t cache_positions,
                                          const void* positions, int pos_is_64, const void* slots,
                                          int slot_is_64, int num_tokens, uint8_t* cache,
                                          int page_size, void* stream);

/* Ragged fp8 MQA logits (prefill indexer).
 *   q        [num_rows, 64, 128] e4m3fn, contiguous, 16-byte aligned
 *   kv       [num_keys, 128] e4m3fn, contiguous, 16-byte aligned; kv_scale [num_keys] f32
 *   weights  [num_rows, 64] f32 (row stride weights_stride)
 *   ks, ke   [num_rows] int32: row i scores keys [ks[i], ke[i]) (0 <= ks, ke <= num_keys)
 *   logits   [num_rows, logits_stride] f32 (out), columns [0, num_cols), num_cols >= num_keys
 * logits[i, j] = sum_h w[i,h] * relu(q[i,h,:] . kv[j,:]) * kv_scale[j] inside the
 * window; with clean_logits every other column < num_cols is -inf, otherwise it
 * is not written. num_heads must be 64.
 * Replaces deep_gemm.fp8_mqa_logits(q, (kv, kv_scale), weights, ks, ke, clean_logits)
 * (third-party DeepGEMM, called at dlengine/runtime/layers/backends/dsa/indexer/
 *  lightning.py:1212-1219). */
DSA_API int dsa_mqa_logits(const uint8_t* q, const uint8_t* kv, const float* kv_scale,
                           const float* weights, int64_t weights_stride, const int32_t* ks,
                           const int32_t* ke, int num_rows, int64_t num_keys, int num_heads,
                           float* logits, int64_t logits_stride, int64_t num_cols,
                           int clean_logits, void* stream);

/* Ragged fp8 MQA logits fused with the exact ragged top-2048 (prefill
 * indexer): the result of dsa_mqa_logits followed by dsa_topk_transform_ragged
 * (row_starts = offsets = ks, seq_lens = ke - ks clamped to [0, max_len]),
 * bit for bit, without storing the logits.
 *   q, kv, kv_scale, weights, ks, ke as for dsa_mqa_logits (num_heads 64)
 *   max_len    >= every ke[i] - ks[i] that should count, <= dsa_topk_max_len()
 *   out        [num_rows, 2048] int32: global key indices ks[i] + position, -1 padded
 *   workspace  dsa_mqa_topk_workspace_bytes(num_rows, num_keys, 2048) bytes, 256-byte aligned
 * Rows whose sampled threshold misses are redone from full logits in a second
 * phase; the call reads one 4-byte counter back to the host (a stream sync).
 * Replaces deep_gemm.fp8_mqa_logits + top_k_per_row_prefill at
 * dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1212-1246. */
DSA_API size_t dsa_mqa_topk_workspace_bytes(int num_rows, int64_t num_keys, int top_k);
DSA_API int dsa_mqa_topk(const uint8_t* q, const uint8_t* kv, const float* kv_scale, const float* weights,
                         int64_t weights_stride, const int32_t* ks, const int32_t* ke, int num_rows,
                         int64_t num_keys, int num_heads, int64_t max_len, int top_k, int32_t* out,
                         void* workspace, size_t workspace_bytes, void* stream);


/* Paged indexer cache -> contiguous ragged keys and scales (prefill indexer).
 *   cache        [pages, page_bytes] uint8, page = [page_size x 128 fp8][page_size x f32]
 *   block_table  [num_seqs, *] int32, row stride bt_stride
 *   cu_seqlens_k [num_seqs + 1] int32 (int64 when cu_is_64), cu[0] = 0, cu[num_seqs] = total_k
 *   key_out      [total_k, 128] uint8;  scale_out [total_k, 4] uint8 (the f32 scale bytes)
 * Ragged token cu[b] + i is token i of sequence b: page block_table[b, i / page_size],
 * row i % page_size. head_dim must be 128.
 * Replaces gather_indexer_cache(cache, block_table, cu_seqlens_k, page_size=, head_dim=,
 * total_k=, max_seqlen_k=) (dlengine/runtime/kernel/triton/generic/indexer_cache_gather.py:60-114,
 * called at dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1180-1188). */
DSA_API int dsa_gather_indexer_cache(const uint8_t* cache, int64_t page_bytes, int page_size,
                                     int head_dim, const int32_t* block_table, int64_t bt_stride,
                                     const void* cu_seqlens_k, int cu_is_64, int num_seqs,
                                     int64_t total_k, uint8_t* key_out, uint8_t* scale_out,
                                     void* stream);


/* Sparse MLA prefill straight from the paged fp8 MLA cache: the keys a token
 * selects from its sequence's cached prefix are read as 656-byte rows through
 * the block table and dequantised exactly in registers (the decode kernel);
 * only the keys it selects among the chunk's fresh rows are read as bf16, in
 * the same kernel pass and under the same softmax.
 *   q, indices, num_tokens, num_heads, topk, sm_scale, out, max_logits, lse:
 *              as dsa_sparse_mla_prefill, with indices into the ragged key
 *              order of total_k = cu_k[-1] keys (sequence b's keys at cu_k[b] ..)
 *   kv_cache   [blocks, kv_block_size, 656] bytes (block stride, block count)
 *   block_table [num_seqs, bt_width] int32 (row stride bt_stride); a cached
 *              key whose column is past bt_width, or whose block is negative
 *              or >= kv_num_blocks, is skipped like an index of -1
 *   cu_seqlens_q/_k [num_seqs + 1] int32
 *              (cu_is_64 = 0) or int64: key i of sequence b is cached row i
 *              while i < k_len - q_len, else fresh row cu_q[b] + i - (k_len - q_len)
 *   fresh      [total_q, 576] bf16 (row stride fresh_row_stride elements)
 *   workspace  dsa_sparse_mla_prefill_paged_workspace_bytes(num_tokens, topk)
 * Same result as assembling the keys (dsa_mla_prefill_kv) and calling
 * dsa_sparse_mla_prefill, up to the summation order: one kernel runs each
 * token's cached keys (fp8 rows, dequantised exactly in registers) and then its
 * fresh bf16 rows under one softmax.
 * Replaces, at dlengine/runtime/models/deepseek_v2/deepseek_v2.py:1573-1650, the
 * key assembly (_gather_cache_cached_only, restore_mla_fp8_cache_rows,
 * _interleave_cached_fresh: layers/backends/attention/mla_utils.py:118-236)
 * followed by flash_mla_sparse_fwd. */
DSA_API size_t dsa_sparse_mla_prefill_paged_workspace_bytes(int num_tokens, int topk);
DSA_API int dsa_sparse_mla_prefill_paged(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                         const uint8_t* kv_cache, int64_t kv_block_stride_bytes,
                                         int kv_block_size, int64_t kv_num_blocks,
                                         const int32_t* block_table, int64_t bt_stride, int bt_width,
                                         const void* cu_seqlens_q, const void* cu_seqlens_k, int cu_is_64,
                                         int num_seqs, int64_t total_k, const void* fresh,
                                         int64_t fresh_row_stride, int64_t total_q, const int32_t* indices,
                                         int64_t idx_stride, int num_tokens, int num_heads, int topk,
                                         float sm_scale, void* out, float* max_logits, float* lse,
                                         void* workspace, size_t workspace_bytes, void* stream);


/* Per-query key windows of a ragged prefill batch, computed on the device.
 *   cu_seqlens_q/_k [num_seqs + 1] int32 (cu_is_64 = 0) or int64: sequence b's
 *              fresh queries are the last q_len of its k_len keys
 *   ks, ke     [num_queries] int32 out: query i of sequence b scores keys
 *              [cu_k[b], i + 1 + cu_k[b+1] - cu_q[b+1])
 *   status     [4] int64 out: {fault bits, total keys, longest k length, most
 *              pages (of page_size) in one sequence}; fault bit 0: cu_q or cu_k
 *              does not start at 0, bit 1: cu_q does not end at num_queries,
 *              bit 2: a q length < 0 or a k length < its q length (then ks/ke
 *              are meaningless)
 * Replaces the host-side window build of Indexer.compute_prefill_topk_paged
 * (dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1138-1206: the
 * cu_seqlens checks and the ks/ke construction). */
DSA_API int dsa_prefill_windows(const void* cu_seqlens_q, const void* cu_seqlens_k, int cu_is_64,
                                int num_seqs, int num_queries, int page_size, int32_t* ks,
                                int32_t* ke, int64_t* status, void* stream);


/* The sparse prefill's ragged bf16 keys [total_k, 576] from the paged fp8
 * MLA cache (656-byte rows) and the chunk's fresh rows.
 *   kv_cache   [kv_num_blocks, block_size, 656] bytes, block stride kv_block_stride_bytes
 *   block_table [num_seqs, bt_width] int32 (row stride bt_stride); a cached row
 *              whose column is past bt_width, or whose block is negative or
 *              >= kv_num_blocks, is written as zeros
 *   cu_seqlens_q/_k [num_seqs + 1] int32 (cu_is_64 = 0) or int64; sequence b's
 *              fresh queries are the last q_len of its k_len keys
 *   fresh      [cu_q[-1], 576] bf16 rows (row stride fresh_row_stride elements)
 *   out        [total_k = cu_k[-1], 576] bf16 (row stride out_row_stride)
 * Key i of sequence b is its cached row i, dequantised (nope = e4m3 x tile
 * scale, exact in bf16; rope copied), while i < k_len - q_len, else fresh row
 * cu_q[b] + i - (k_len - q_len).
 * Replaces _gather_cache_cached_only + restore_mla_fp8_cache_rows +
 * _interleave_cached_fresh (dlengine/runtime/layers/backends/attention/
 * mla_utils.py:118-236, kernel/triton/hopper/fp8_utils.py:153-196) as called at
 * dlengine/runtime/models/deepseek_v2/deepseek_v2.py:1573-1604. */
DSA_API int dsa_mla_prefill_kv(const uint8_t* kv_cache, int64_t kv_block_stride_bytes,
                               int kv_block_size, int64_t kv_num_blocks, const int32_t* block_table,
                               int64_t bt_stride, int bt_width,
                               const void* cu_seqlens_q, const void* cu_seqlens_k, int cu_is_64,
                               int num_seqs, int64_t total_k, const void* fresh,
                               int64_t fresh_row_stride, void* out, int64_t out_row_stride,
                               void* stream);


/* Sparse MLA prefill over ragged bf16 KV rows.
 *   q          [num_tokens, num_heads, 576] bf16 (row stride q_token_stride, head
 *              stride q_head_stride elements, last dim contiguous)
 *   kv         [s_kv, 576] bf16, row stride kv_row_stride elements (>= 576)
 *   indices    [num_tokens, topk] int32 into kv (row stride idx_stride); entries
 *              < 0 or >= s_kv are skipped
 *   out        [num_tokens, num_heads, 512] bf16, contiguous
 *   max_logits [num_tokens, num_heads] f32 (may be NULL): max_i s_i
 *   lse        [num_tokens, num_heads] f32 natural-log LSE (may be NULL)
 * s_i = sm_scale * q . kv[idx_i]; o = softmax(s) @ kv[idx, :512]. A token with no
 * valid index yields o = 0 and lse = max_logits = -inf.
 * num_heads % 16 == 0; topk % 32 == 0.
 * Replaces flash_mla.flash_mla_sparse_fwd(q, kv, indices, sm_scale, d_v=512)
 * (third-party FlashMLA, called at dlengine/runtime/models/deepseek_v2/
 *  deepseek_v2.py:1644-1650). */
DSA_API int dsa_sparse_mla_prefill(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                   const void* kv, int64_t kv_row_stride, int64_t s_kv,
                                   const int32_t* indices, int64_t idx_stride, int num_tokens,
                                   int num_heads, int topk, float sm_scale, void* out,
                                   float* max_logits, float* lse, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* DSA_AMD_H_ */

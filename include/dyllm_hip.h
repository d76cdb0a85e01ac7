/*
 * dyllm_hip.h -- C ABI of the MI355X (gfx950) DyLLM saliency hot path.
 *
 * Every entry point takes raw device pointers, element counts and a hipStream_t (passed as
 * void*), enqueues its kernels on that stream without any host synchronisation, and
 * returns 0 on success or a non-zero status with a message available from
 * dyllm_last_error() (thread-local). No entry point allocates device memory: temporaries
 * come from a caller-provided workspace whose size the matching *_workspace_bytes()
 * reports. bf16 tensors are passed as uint16_t bit patterns, row-major and contiguous
 * ([tokens, heads, head_dim] == [tokens, heads*head_dim]).
 *
 * Reference interfaces replaced (paths relative to the DyLLM source tree):
 *   dyllm_attention_sparse_varlen  <- attention_sparse_varlen_cuda, dyllm/csrc/attention/attention.cpp:64-179
 *                                     (pybind name "attention_sparse_varlen", attention.cpp:198-203)
 *   dyllm_fused_offset_launch      <- dyllm_launch_fused_offset, attention_aux_kernels.cu:173-200
 *                                     (pybind name "fused_offset_launch", attention.cpp:204)
 *   dyllm_get_seqs / get_block / reset_full / reset_block / scatter_update
 *                                  <- get_seqs_cuda, get_block_cuda, reset_full_cuda, reset_block_cuda,
 *                                     scatter_update_cuda (dyllm/csrc/cache/cache.cpp:19-25,
 *                                     cache_kernels.cu:66-460)
 *   dyllm_flash_attn_varlen        <- flash_attn_varlen_func (third-party flash-attn 2.8.3) as called at
 *                                     dyllm/model_executor/layers/attention.py:41-52 and :76-87
 *   dyllm_cosine_mask              <- tensor_parallel_cosine_mask, dyllm/distributed/parallel_state.py:52-66
 *   dyllm_salient_compact          <- torch.nonzero + torch.searchsorted + fused_offset at attention.py:147-166
 *   dyllm_gather_rows              <- gather_rows_2D, dyllm/utils/util.py:19-36
 *   dyllm_swiglu_ffn               <- LLaDAMLP.forward, dyllm/model_executor/models/llada.py:38-43
 *                                     (+ MLPcache.scatter_update, mlp_cache_manage.py:24-40)
 *   dyllm_silu_and_mul             <- SiluAndMul.forward, dyllm/model_executor/layers/activations.py:11-14
 *   dyllm_moe_gate                 <- moe_gate, dyllm/model_executor/layers/fused_moe.py:375-408
 *   dyllm_moe_align_block_size     <- moe_align_block_size, fused_moe.py:37-85
 *   dyllm_fused_experts            <- fused_experts, fused_moe.py:269-335
 *   dyllm_unmask_step              <- Scheduler.postprocess + ModelRunner.prepare_sparse / prepare_sample
 *                                     (dyllm/engine/scheduler.py:89-145, model_runner.py:186-372) between sparse steps
 *   dyllm_sparse_attention_step, dyllm_attention_colsparse_cached, dyllm_v_delta_update, dyllm_seq_row_starts
 *                                  <- the sparse branch of Attention.forward, attention.py:64-178, with the
 *                                     K/V/context cache gathers and the full-size dV fused away
 *   dyllm_saliency_stats           <- the statistics epilogue of attention_ops_kernels_sm80.cu:436-481
 *                                     as a standalone pass over two bf16 row sets
 */
#ifndef DYLLM_HIP_H_
#define DYLLM_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Last error message of the calling thread ("" when none). */
const char* dyllm_last_error(void);
/* ABI version of this library. */
int dyllm_abi_version(void);

/* Unmasking bookkeeping between two sparse steps of one running batch, on the device (the host
 * work of Scheduler.postprocess + ModelRunner.prepare_sparse / prepare_sample,
 * dyllm/engine/scheduler.py:89-145, dyllm/engine/model_runner.py:186-372). One launch:
 *   commit   tokens[cu_k[b] + p] = tok for the previous sampler output (sampled_pos / sampled_tok,
 *            [batch][ld_sampled], sampled_counts[b] entries); positions that held mask_id and now hold
 *            another token are added to generated[b];
 *   salient  the kept positions p >= answer_start[b], in sampler order, as the next step's lists:
 *            idx_q (p - prompt_len[b] + cu_q[b] when q_pruned, else p + cu_q[b]), idx_k = idx_upd =
 *            p + cu_k[b], positions_k = p, cu_salientlens [batch+1] (capacity: batch * ld_sampled);
 *   inputs   q_pruned and input_ids != NULL: input_ids[cu_q[b] + i] = tokens[cu_k[b] + answer_start[b] + i];
 *   candidates  the first `width` positions p in [offset, limit) holding mask_id, offset = answer_start
 *            (q_pruned) or 0, limit = min(L, block_size * (block_idx + 1) + prompt_len) with
 *            block_idx = generated / block_size: cand_rel[b][j] = p - offset, cand_n[b] = count. */
int dyllm_unmask_step(int64_t* tokens, const int32_t* cu_seqlens_k, int batch, const int64_t* sampled_pos,
                      const int64_t* sampled_tok, const int32_t* sampled_counts, int64_t ld_sampled,
                      int32_t* generated, const int32_t* prompt_len, const int32_t* answer_start,
                      const int32_t* block_size, int64_t mask_id, int q_pruned, const int32_t* cu_seqlens_q,
                      int64_t* idx_q, int32_t* idx_q32, int64_t* idx_k, int32_t* idx_k32, int32_t* idx_upd,
                      int64_t* positions_k, int32_t* cu_salientlens, int64_t* input_ids, int64_t* cand_rel,
                      int32_t* cand_n, int width, void* stream);

/* Launch resources of the fused attention kernel (attention_kernel_info, pybind op of
 * dyllm/csrc/attention/attention.cpp:205-208): out[10] = [registers, local (scratch) bytes per lane,
 * static LDS bytes, dynamic LDS bytes, threads per block, max active blocks per CU, query rows per
 * block, keys per block, d_split, ok (1 when dim == 128)]. mask_v_rows is accepted for the
 * reference's signature; this build has one kernel for both. */
int dyllm_attention_kernel_info(int dim, int mask_v_rows, int64_t* out);

/* Timing of the fused attention kernel inside dyllm_sparse_attention_step (no counterpart in
 * the reference; for benchmarks that need that kernel's own duration): while enabled (per host
 * thread), every step call records a library-owned HIP event pair around the attention launch on
 * its stream. _read synchronises on the recorded events, returns their summed duration and count
 * and forgets them. */
int dyllm_attention_timer(int enable);
int dyllm_attention_timer_read(float* total_ms, int* launches);

/* Issue-rate probe of one SIMD (no counterpart in the reference; for benchmarks): `workgroups`
 * 256-thread workgroups each run `iters` iterations of a loop chosen by mode -- 0: 4 MFMA
 * 32x32x16 bf16, 1: 64 v_fma_f32, 2: 64 v_exp_f32 + 64 v_mul_f32, 3: 0 and 1 in one wavefront,
 * 4: the same pinned as 1 MFMA / 16 VALU groups, 5: 0 and 2, 6: 5 pinned. cycles[w] receives the
 * s_memtime cycles of workgroup w's loop; sink (workgroups * 256 floats) keeps the results live. */
int dyllm_issue_probe(int mode, int workgroups, int iters, void* sink, void* cycles, void* stream);

/* ---- attention ------------------------------------------------------------------------ */

/* Workspace for dyllm_attention_sparse_varlen. */
size_t dyllm_attention_sparse_workspace_bytes(int batch, int num_heads, int64_t total_q, int max_seqlen_k);

/* Column-sparse attention + saliency statistics + tau test (attention.cpp:64-179).
 * q, c, o: [total_q, H, D]; k, v_delta: [total_k, H_kv, D]; o_sal: [num_salient, H, D].
 * idx_salient_q (int32, Q space) lists the rows whose output is o_sal; idx_salient_k (int32,
 * K space) the key rows where v_delta may be non-zero (NULL: same as idx_salient_q).
 * cosine_stats [total_q, 3] fp32 is overwritten (no zero-initialisation needed);
 * cosine_out [total_q] bytes: 1 where cos < threshold. head_dim must be 128. */
int dyllm_attention_sparse_varlen(const void* q, const void* k, const void* v_delta, const void* c,
                                  const void* o_sal, void* o, int batch, int num_heads, int num_kv_heads,
                                  int head_dim, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int max_seqlen_q, int max_seqlen_k, int64_t total_q, int num_salient,
                                  const int32_t* cu_salientlens, const int32_t* idx_salient_q,
                                  const int32_t* idx_salient_k, float* cosine_stats, uint8_t* cosine_out,
                                  float threshold, void* workspace, size_t workspace_bytes, void* stream);

/* Non-causal varlen softmax attention, scale = softmax_scale (head_dim must be 128).
 * q_rows == NULL: rows are q[cu_seqlens_q[b] .. cu_seqlens_q[b+1]) -> o rows at the same index.
 * q_rows != NULL: cu_seqlens_q is the prefix of a compact row list (cu_salientlens); compact
 * row j reads q[q_rows[j]] and writes o[j] (the row-sparse call at attention.py:76-87).
 * max_seqlen_q bounds the rows of one sequence. */
int dyllm_flash_attn_varlen(const void* q, const void* k, const void* v, void* o, int batch, int num_heads,
                            int num_kv_heads, int head_dim, const int32_t* cu_seqlens_q,
                            const int32_t* cu_seqlens_k, const int64_t* kv_start, int max_seqlen_q,
                            int max_seqlen_k, float softmax_scale, const int32_t* q_rows, void* stream);

/* Column-sparse attention straight out of the per-layer caches (no reference counterpart:
 * it fuses the cache gathers and the full-size dV of attention.py:67-139 into the kernel):
 * K rows of sequence b start at k_cache row kv_start[b] (NULL: cu_seqlens_k[b]); dV is compact,
 * row j belonging to key idx_salient_k[j] (packed K space); C rows of sequence b start at
 * c_cache row c_start[b] (NULL: cu_seqlens_q[b]) and, with c_inplace, the new rows are also
 * written back there (the context-cache reset_block). Same outputs as
 * dyllm_attention_sparse_varlen otherwise. */
size_t dyllm_attention_colsparse_workspace_bytes(int batch, int num_heads, int64_t total_q, int64_t total_k,
                                                 int max_seqlen_k);
int dyllm_attention_colsparse_cached(const void* q, const void* k_cache, const int64_t* kv_start,
                                     const void* dv_compact, void* c_cache, const int64_t* c_start,
                                     int c_inplace, const void* o_sal, void* o, int batch, int num_heads,
                                     int num_kv_heads, int head_dim, const int32_t* cu_seqlens_q,
                                     const int32_t* cu_seqlens_k, int max_seqlen_q, int max_seqlen_k,
                                     int64_t total_q, int64_t total_k, int num_salient,
                                     const int32_t* idx_salient_q, const int32_t* idx_salient_k,
                                     float* cosine_stats, uint8_t* cosine_out, float threshold, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* The whole sparse branch of Attention.forward (attention.py:64-178) in one call (four
 * launches that leave the host back to back): dV + V-cache update of the salient keys
 * (v_new rows follow the idx_k32 list), row-sparse attention of the salient queries against the cached
 * K/V, column-sparse attention with statistics and the tau test (context cache updated in place,
 * new rows also written to `out` [total_q, H, D]), and compaction of the next salient set into
 * next_* (capacity total_q; next_count[0] = its size, left on the device). K is packed
 * (k_start == NULL) or read from a cache through per-sequence first rows k_start[b]; the V and
 * context caches are addressed through their seq_start tables (indexed by seq_ids[b]).
 * cu_promptlens != NULL selects a Q-pruned step (Q rows are the response rows; the next set is
 * also produced in K space); otherwise Q space == K space and idx_k* = idx_q*.
 * The salient rows of sequence b are list entries [cu_salientlens[b], cu_salientlens[b+1]), in any
 * order, each key at most once per sequence; an entry whose K row lies outside its sequence is
 * ignored.
 * next_dest_rows (optional, capacity total_q) receives, for every row of the next salient set, its row in
 * another per-layer cache whose sequence starts are dest_seq_starts (indexed by seq_ids[b]): the
 * scatter_update address of its K-space row, i.e. where the layer's FFN writes that row's output
 * (mlp_cache_manage.py:24-40), so no separate address pass is needed.
 * host_meta (optional, pinned host memory of batch + 2 int32 from hipHostMalloc) receives
 * [next_count, next_cu_salientlens...] directly from the compaction kernel, so the host can read
 * the salient count without a device->host copy: each entry is stored once, by the workgroup
 * that owns it, and fenced to system scope before the kernel ends. A host that fills the buffer
 * with -1 before the call can poll it until no entry is negative (no event needed). */
size_t dyllm_sparse_step_workspace_bytes(int batch, int num_heads, int num_kv_heads, int head_dim, int64_t total_q,
                                         int64_t total_k, int max_seqlen_k, int64_t num_salient);
int dyllm_sparse_attention_step(const void* q, const void* k, const int64_t* k_start, void* v_cache,
                                const int64_t* v_seq_starts, const void* v_new, void* c_cache,
                                const int64_t* c_seq_starts, const int64_t* seq_ids, int batch, int num_heads,
                                int num_kv_heads, int head_dim, const int32_t* cu_seqlens_q,
                                const int32_t* cu_seqlens_k, const int32_t* cu_promptlens, int max_seqlen_q,
                                int max_seqlen_k, int64_t total_q, int64_t total_k, int num_salient,
                                int max_salientlen, const int32_t* cu_salientlens, const int32_t* idx_q32,
                                const int64_t* idx_k64, const int32_t* idx_k32, float softmax_scale, float threshold,
                                void* out, float* cosine_stats, uint8_t* cosine_out, int64_t* next_idx64,
                                int32_t* next_idx32, int64_t* next_idx_k64, int32_t* next_idx_k32,
                                int32_t* next_cu_salientlens, int32_t* next_count, const int64_t* dest_seq_starts,
                                int64_t* next_dest_rows, int32_t* host_meta, void* workspace, size_t workspace_bytes,
                                void* stream);

/* Salient-row K/V epilogue carried into dyllm_sparse_attention_step_kv: the reference's K/V
 * projection tail (llada.py:103-146, dream.py:99-141, lladamoe.py:204-239: optional k_norm,
 * rotary_embedding.py:40-54 neox RoPE, CacheManager.scatter_update of k, cache_kernels.cu:388-426)
 * and the v rows Attention.forward receives. Row j of the salient list reads kv row
 * kv_rows[j] (NULL: j) = [k | v] (2 * num_kv_heads * 128 bf16 values, ld_kv apart) and position
 * positions[pos_idx[j]] (pos_idx NULL: positions[j]), clamped to [0, max_position). The rotated k
 * goes to K-cache row k_seq_starts[seq_ids[b]] + (K row - cu_seqlens_k[b]). */
typedef struct dyllm_kv_epilogue {
  const void* kv;
  int64_t ld_kv;
  const int32_t* kv_rows;
  const int64_t* positions;
  const int32_t* pos_idx;
  const float* cos_table;      /* fp32 [max_position, 64] */
  const float* sin_table;
  int max_position;
  const void* k_norm_weight;   /* optional bf16 [128] */
  float eps;
  void* k_cache;               /* bf16 rows of num_kv_heads * 128 */
  const int64_t* k_seq_starts;
} dyllm_kv_epilogue;

/* dyllm_sparse_attention_step with the K/V epilogue fused into its first launch (the reference's
 * scatter_kv + Attention.forward, llada.py:136-147 + attention.py:64-178): k, k_start and v_new
 * must be NULL; K is read from kv_epilogue->k_cache through k_seq_starts (after the salient rows
 * were rotated into it) and v from the kv rows. Same outputs otherwise. */
int dyllm_sparse_attention_step_kv(const dyllm_kv_epilogue* kv_epilogue, const void* q, const void* k,
                                   const int64_t* k_start, void* v_cache, const int64_t* v_seq_starts,
                                   const void* v_new, void* c_cache, const int64_t* c_seq_starts,
                                   const int64_t* seq_ids, int batch, int num_heads, int num_kv_heads, int head_dim,
                                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                   const int32_t* cu_promptlens, int max_seqlen_q, int max_seqlen_k, int64_t total_q,
                                   int64_t total_k, int num_salient, int max_salientlen,
                                   const int32_t* cu_salientlens, const int32_t* idx_q32, const int64_t* idx_k64,
                                   const int32_t* idx_k32, float softmax_scale, float threshold, void* out,
                                   float* cosine_stats, uint8_t* cosine_out, int64_t* next_idx64, int32_t* next_idx32,
                                   int64_t* next_idx_k64, int32_t* next_idx_k32, int32_t* next_cu_salientlens,
                                   int32_t* next_count, const int64_t* dest_seq_starts, int64_t* next_dest_rows,
                                   int32_t* host_meta, void* workspace, size_t workspace_bytes, void* stream);

/* The same step as dyllm_sparse_attention_step without the workspace arguments: no counterpart
 * in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): the workspace is a library-owned device
 * array of dyllm_sparse_step_scratch_bytes() (64 MiB) per GPU, held until the process ends.
 * Calls whose dyllm_sparse_step_workspace_bytes(...) exceeds it fail with an error (config 1,
 * 920 salient rows, needs about 10 MiB). The array keeps the last call's contents; every call on
 * one GPU shares it, so calls that overlap on one GPU (concurrent streams or threads) race.
 * Allocates nothing: no hipMalloc / hipFree, no library allocation. */
size_t dyllm_sparse_step_scratch_bytes(void);
int dyllm_sparse_attention_step_noalloc(const void* q, const void* k, const int64_t* k_start, void* v_cache,
                                        const int64_t* v_seq_starts, const void* v_new, void* c_cache,
                                        const int64_t* c_seq_starts, const int64_t* seq_ids, int batch,
                                        int num_heads, int num_kv_heads, int head_dim,
                                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                        const int32_t* cu_promptlens, int max_seqlen_q, int max_seqlen_k,
                                        int64_t total_q, int64_t total_k, int num_salient, int max_salientlen,
                                        const int32_t* cu_salientlens, const int32_t* idx_q32,
                                        const int64_t* idx_k64, const int32_t* idx_k32, float softmax_scale,
                                        float threshold, void* out, float* cosine_stats, uint8_t* cosine_out,
                                        int64_t* next_idx64, int32_t* next_idx32, int64_t* next_idx_k64,
                                        int32_t* next_idx_k32, int32_t* next_cu_salientlens, int32_t* next_count,
                                        const int64_t* dest_seq_starts, int64_t* next_dest_rows, int32_t* host_meta,
                                        void* stream);

/* dV and V-cache update of attention.py:67-74 (dv = v_new - v_cache[row]; v_cache[row] = v_new)
 * for compact rows; dest_rows are cache rows (dyllm_scatter_dest_rows). */
int dyllm_v_delta_update(void* v_cache, const void* v_new, const int64_t* dest_rows, int64_t rows,
                         int64_t row_elems, void* dv_out, void* stream);

/* out[b] = seq_starts[seq_ids[b]] (+ Lk_b - Lq_b when cu_seqlens_q != NULL: the first cached
 * row of the queried tail block, cache_kernels.cu:224). */
int dyllm_seq_row_starts(const int64_t* seq_starts, const int64_t* seq_ids, const int32_t* cu_seqlens_k,
                         const int32_t* cu_seqlens_q, int batch, int64_t* out, void* stream);

/* ---- saliency and compaction ----------------------------------------------------------- */

/* mask[t] = cos(stats[t]) < threshold (parallel_state.py:62-66). */
int dyllm_cosine_mask(const float* stats, int64_t rows, float threshold, uint8_t* mask, void* stream);

/* Standalone saliency pass: stats[t] = {sum new*old, sum new^2, sum old^2} of bf16 rows of
 * width dim, then the tau test. */
int dyllm_saliency_stats(const void* c_new, const void* c_old, int64_t rows, int64_t dim, float threshold,
                         float* stats, uint8_t* mask, void* stream);

/* Stream compaction of a byte mask over rows [0, rows): ascending salient indices
 * (idx64, and idx32 when non-NULL), cu_salientlens[b] = #indices < cu_seqlens_q[b]
 * for b in [0, batch], count[0] = number of indices, and, when idx_k != NULL,
 * idx_k[t] = idx64[t] + cu_promptlens[seg(t)+1] (fused_offset). idx buffers need
 * capacity `rows`. Runs on the device; the caller reads count[0] when it needs it. */
int dyllm_salient_compact(const uint8_t* mask, int64_t rows, const int32_t* cu_seqlens_q, int batch,
                          const int32_t* cu_promptlens, int64_t* idx64, int32_t* idx32, int64_t* idx_k,
                          int32_t* cu_salientlens, int32_t* count, void* stream);

/* fused_offset_launch (attention_aux_kernels.cu:173-200): out[t] = idxs[t] +
 * cu_promptlens[seg(t)+1] for t < min(*num_idxs, max_threads); num_groups = batch. */
int dyllm_fused_offset_launch(const int32_t* idxs, const int32_t* num_idxs, const int32_t* cu_promptlens,
                              const int32_t* cu_salientlens, int num_groups, int64_t* out, int64_t max_threads,
                              void* stream);

/* ---- packed row caches (row_bytes: bytes per row, multiple of 16) ---------------------- */
int dyllm_get_seqs(const void* cache, void* out, int64_t row_bytes, const int64_t* seq_starts,
                   const int32_t* cu_seqlens, const int64_t* seq_ids, int batch, int64_t total_rows, void* stream);
int dyllm_get_block(const void* cache, void* out, int64_t row_bytes, const int64_t* seq_starts,
                    const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q, const int64_t* seq_ids, int batch,
                    int64_t total_rows, void* stream);
int dyllm_reset_full(void* cache, const void* in, int64_t row_bytes, const int64_t* seq_starts,
                     const int32_t* cu_seqlens, const int64_t* seq_ids, int batch, int64_t total_rows, void* stream);
int dyllm_reset_block(void* cache, const void* in, int64_t row_bytes, const int64_t* seq_starts,
                      const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q, const int64_t* seq_ids, int batch,
                      int64_t total_rows, void* stream);
int dyllm_scatter_update(void* cache, const void* new_vals, int64_t row_bytes, const int64_t* row_idx, int64_t rows,
                         const int32_t* cu_seqlens, const int64_t* seq_starts, const int64_t* seq_ids, int batch,
                         void* stream);
/* Destination cache row of each packed row index (the address part of scatter_update); rows
 * beyond *rows_dev (when given) are skipped. */
int dyllm_scatter_dest_rows(const int64_t* row_idx, int64_t rows, const int32_t* rows_dev,
                            const int32_t* cu_seqlens, const int64_t* seq_starts, const int64_t* seq_ids, int batch,
                            int64_t* dest, void* stream);
/* out[m] = x[idx[m]] for the x_rows rows of x; an index outside [0, x_rows) yields a zero row
 * (the device never reads past x). */
int dyllm_gather_rows(const void* x, int64_t x_rows, void* out, int64_t row_bytes, const int64_t* idx, int64_t rows,
                      void* stream);

/* ---- FFN ------------------------------------------------------------------------------- */
/* Every GEMM operand (the input rows x, h, the weights; one expert's block of a stacked expert
 * weight) must span less than 4 GiB: the kernels address them with 32-bit byte offsets. The
 * weights and ungathered inputs are checked (-> error); a gathered x's extent is not known to
 * the library and is the caller's to keep. */

/* Workspace of dyllm_swiglu_ffn: dyllm_swiglu_ffn_workspace_bytes (the [rows, intermediate]
 * bf16 activations) + dyllm_ffn_down_workspace_bytes (split-K partials of the down GEMM). */
size_t dyllm_swiglu_ffn_workspace_bytes(int64_t rows, int intermediate);
size_t dyllm_ffn_down_workspace_bytes(int64_t rows, int64_t rows_hint, int hidden, int intermediate);

/* Gathered SwiGLU FFN: for m < rows, a = x[rows_idx ? rows_idx[m] : m] (row stride ld_x),
 * h = silu(a W_g^T) * (a W_u^T), y = h W_d^T written to out[out_rows ? out_rows[m] : m]
 * (row stride hidden). w_gate_up: [2*intermediate, hidden] (gate rows first);
 * w_down: [hidden, intermediate]. */
int dyllm_swiglu_ffn(const void* x, int64_t ld_x, const int32_t* rows_idx, int64_t rows, const void* w_gate_up,
                     const void* w_down, int hidden, int intermediate, void* workspace, size_t workspace_bytes,
                     void* out, const int64_t* out_rows, void* stream);

/* SiLU-and-mul of a merged gate_up product (SiluAndMul, activations.py:11-14): for m < rows,
 * out[m][j] = bf16(silu(g) * u) in fp32 with g = gate_up[m][j], u = gate_up[m][intermediate + j]
 * (bf16; row strides ld_in >= 2*intermediate and ld_out >= intermediate, multiples of 8; both
 * buffers 16-byte aligned; out must not overlap gate_up). The same arithmetic as the SwiGLU
 * epilogue of dyllm_ffn_gate_up, for a gate_up product computed by another GEMM (the dense full
 * step runs the library GEMM). */
int dyllm_silu_and_mul(const void* gate_up, int64_t ld_in, int64_t rows, int intermediate, void* out, int64_t ld_out,
                       void* stream);

/* The two stages of dyllm_swiglu_ffn: h_out [rows, intermediate] = silu(a W_g^T) * (a W_u^T)
 * with a = x[rows_idx[m] or m]; then out[out_rows[m] or m] = h[m] W_d^T. `rows` is the capacity
 * (buffers are sized for it); when rows_dev != NULL the row count is read from device memory
 * (e.g. the count written by dyllm_salient_compact), so no host synchronisation is needed.
 * rows_hint (0: rows) is the expected count used to choose the tile shape. */
int dyllm_ffn_gate_up(const void* x, int64_t ld_x, const int32_t* rows_idx, int64_t rows, const int32_t* rows_dev,
                      int64_t rows_hint, const void* w_gate_up, int hidden, int intermediate, void* h_out,
                      void* stream);
int dyllm_ffn_down(const void* h, int64_t rows, const int32_t* rows_dev, int64_t rows_hint, const void* w_down,
                   int hidden, int intermediate, void* out, const int64_t* out_rows, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Tile height (128/192/256) the FFN GEMMs use for `rows` rows, output width n and depth k. */
int dyllm_ffn_tile_rows(int64_t rows, int n, int k, int swiglu);

/* ---- salient-row K/V projection (the step before the sparse attention) ------------------ */

/* Gathered linear: out[m] = x[rows_idx ? rows_idx[m] : m] . w^T (+ bias), out [rows,
 * out_features] bf16, fp32 accumulation rounded once (F.linear, linear.py). Replaces
 * kv_proj(hidden_states[idx_salient_row]) of llada.py:108, dream.py:103, lladamoe.py:204.
 * w: [out_features, in_features]; bias: optional bf16 [out_features]. rows / rows_dev /
 * rows_hint as for dyllm_ffn_gate_up; the workspace holds split-K partials. */
size_t dyllm_linear_workspace_bytes(int64_t rows, int64_t rows_hint, int out_features, int in_features);
int dyllm_linear(const void* x, int64_t ld_x, const int32_t* rows_idx, int64_t rows, const int32_t* rows_dev,
                 int64_t rows_hint, const void* w, int out_features, int in_features, const void* bias, void* out,
                 void* workspace, size_t workspace_bytes, void* stream);

/* K/V epilogue of that projection for the salient rows j < rows (or < *rows_dev): kv row j holds
 * k then v ([num_kv_heads * 128] each, row stride ld_kv). k: optional per-head RMSNorm with
 * k_norm_weight (bf16 [128], lladamoe.py:206-207 / layernorm.py:15-24), then the neox rotary
 * embedding at positions[pos_idx ? pos_idx[j] : j] clamped to max_position - 1
 * (rotary_embedding.py:8-16, 40-54; cos/sin tables fp32 [max_position, 64]), written to the
 * K-cache row of packed K-space row k_rows[j] (the addressing of dyllm_scatter_update,
 * llada.py:136-143). v: copied to v_out [rows, num_kv_heads * 128]. Replaces the zero-filled
 * k_temp, the rotary over all rows and the scatter of llada.py:108-143. */
/* The same epilogue in place for the queries: rows j < rows of x ([rows, num_heads * 128], row
 * stride ld_x): optional per-head RMSNorm (q_norm, lladamoe.py:194-195), then RoPE at
 * positions[j] (rotary_embedding.py:47-54), written back to x. */
int dyllm_rope(void* x, int64_t ld_x, int64_t rows, int num_heads, int head_dim, const int64_t* positions,
               const float* cos_table, const float* sin_table, int max_position, const void* norm_weight, float eps,
               void* stream);
int dyllm_kv_rope_scatter(const void* kv, int64_t ld_kv, int64_t rows, const int32_t* rows_dev, const int32_t* pos_idx,
                          const int64_t* positions, const float* cos_table, const float* sin_table,
                          int max_position, int num_kv_heads, int head_dim, const void* k_norm_weight, float eps,
                          void* k_cache, const int64_t* k_rows, const int32_t* cu_seqlens_k,
                          const int64_t* seq_starts, const int64_t* seq_ids, int batch, void* v_out, void* stream);

/* ---- decoder-layer RMSNorm (the steps either side of the path) ------------------------------ */

/* RMSNorm.rms_forward / add_rms_forward (layernorm.py:15-37) in one pass per row: with a
 * residual, s = x + residual in fp32 and residual_out = bf16(s); without, s = x; then
 * out = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * weight). weight: bf16 [hidden]; hidden a
 * multiple of 8, at most 8192; out may alias x and residual_out may alias residual. Replaces the
 * post-attention (and input) layernorm of llada.py:174-186 / dream.py / lladamoe.py on all rows. */
int dyllm_rms_norm(const void* x, int64_t ld_x, const void* residual, int64_t ld_residual, const void* weight,
                   int64_t rows, int hidden, float eps, void* out, int64_t ld_out, void* residual_out,
                   int64_t ld_residual_out, void* stream);

/* The same norm with x read from a per-layer row cache (no reference counterpart: it removes
 * the packed copy of the cached FFN rows, mlp_cache_manage.py:33-38, that the reference hands to
 * the next layer's norm). Packed row r, of sequence b (cu_seqlens_q[b] <= r < cu_seqlens_q[b+1]),
 * reads cache row seq_starts[seq_ids[b]] + (Lk_b - Lq_b) + (r - cu_seqlens_q[b]), the tail-block
 * addressing of dyllm_get_block (Lq == Lk: the whole sequence, dyllm_get_seqs). */
int dyllm_rms_norm_cache_rows(const void* cache, int64_t ld_cache, const int64_t* seq_starts, const int64_t* seq_ids,
                              const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q, int batch,
                              const void* residual, int64_t ld_residual, const void* weight, int64_t rows, int hidden,
                              float eps, void* out, int64_t ld_out, void* residual_out, int64_t ld_residual_out,
                              void* stream);

/* ---- MoE ------------------------------------------------------------------------------- */

/* Router: topk_weights (bf16) / topk_ids (int32) [tokens, top_k] from fp32 softmax of
 * x[rows_idx[t] or t] . router_w^T; router_w: [num_experts, hidden] bf16; num_experts <= 64,
 * hidden a multiple of 16. */
int dyllm_moe_gate(const void* x, const int32_t* rows_idx, int64_t tokens, int hidden, const void* router_w,
                   int num_experts, int top_k, int renormalize, void* topk_weights, int32_t* topk_ids, void* stream);

/* moe_align_block_size on the device. capacity >= tokens*top_k + E*(block-1), multiple of block.
 * Expert ids outside [0, num_experts) are clamped into that range on the device (the ids are
 * device data: validating them on the host would need a synchronisation). */
int dyllm_moe_align_block_size(const int32_t* topk_ids, int64_t slots, int num_experts, int block,
                               int32_t* sorted_token_ids, int64_t capacity, int32_t* tile_expert,
                               int32_t* num_post_pad, void* stream);

size_t dyllm_fused_experts_workspace_bytes(int64_t tokens, int top_k, int num_experts, int hidden,
                                           int intermediate);

/* fused_experts with SiLU gating: w1 [E, 2*I, hidden], w2 [E, hidden, I]; routing from
 * dyllm_moe_gate. out[out_rows ? out_rows[t] : t] = sum_k w_k * FFN_{e_k}(x_t), bf16, where token t
 * is x row rows_idx[t] (rows_idx NULL: row t; the gather of the salient rows, util.py:19-36,
 * happens inside the first grouped GEMM). */
int dyllm_fused_experts(const void* x, const int32_t* rows_idx, int64_t tokens, int hidden, const void* w1,
                        const void* w2, int num_experts, int intermediate, const void* topk_weights,
                        const int32_t* topk_ids, int top_k, void* out, const int64_t* out_rows, void* workspace,
                        size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DYLLM_HIP_H_ */

// Kernel-side argument structs and launchers shared between the kernel translation units
// and the C-ABI layer (capi.hip).
#pragma once
#include "dyllm_common.h"

namespace dyllm {

enum class RowMap : int { GetSeqs = 0, GetBlock = 1, ResetFull = 2, ResetBlock = 3, Scatter = 4, Gather = 5 };
struct RowMapArgs {
  const char* src;
  char* dst;
  int64_t row_bytes;
  int64_t n_rows;
  const int64_t* seq_starts;
  const int32_t* cu;
  const int32_t* cu_q;
  const int64_t* seq_ids;
  const int64_t* row_idx;
  int B;
  int64_t src_rows;   // Gather: rows of src (indices outside [0, src_rows) give zero rows)
};
int launch_row_map(RowMap mode, const RowMapArgs& a, hipStream_t stream);
// RMSNorm with the optional fused residual add (norm.hip).
struct NormArgs {
  const uint16_t* x;         // [rows, ld_x]
  int64_t ld_x;
  const uint16_t* residual;  // optional [rows, ld_r]
  int64_t ld_r;
  const uint16_t* weight;    // [hidden]
  int64_t rows;
  int hidden;
  float eps;
  uint16_t* out;             // [rows, ld_out] (may alias x)
  int64_t ld_out;
  uint16_t* residual_out;    // with residual: [rows, ld_ro] = bf16(x + residual) (may alias residual)
  int64_t ld_ro;
  // optional: x rows read from a per-layer row cache instead (x = the cache slab, rows ld_x apart):
  // packed row r of sequence b = segment of cu_q holding r reads cache row
  // seq_starts[seq_ids[b]] + (Lk_b - Lq_b) + (r - cu_q[b])  (the tail block, get_block)
  const int64_t* x_seq_starts;
  const int64_t* x_seq_ids;
  const int32_t* x_cu_k;
  const int32_t* x_cu_q;
  int x_batch;
};
int launch_add_rms_norm(const NormArgs& a, hipStream_t s);
// Salient-row K/V epilogue: k -> (k_norm) -> rotary -> K-cache row, v -> v_out (rope.hip).
struct KvRopeArgs {
  const uint16_t* kv;            // [rows, ld_kv]: k (kv_size) then v (kv_size)
  int64_t ld_kv;
  int64_t rows;                  // capacity
  const int32_t* rows_dev;       // optional device row count (<= rows)
  int64_t kv_size;               // Hkv * 128
  int Hkv;
  const int32_t* pos_idx;        // optional [rows]: index into positions (else row j)
  const int64_t* positions;
  const float* cos;              // [max_position, 64]
  const float* sin;
  int64_t max_position;
  const uint16_t* k_norm;        // optional [128] bf16
  float eps;
  uint16_t* k_cache;             // rows of ld_cache elements (in-place mode: the output rows)
  int64_t ld_cache;
  const int64_t* k_rows;         // [rows] packed K-space row of each salient row; NULL: row j
  const int32_t* cu_k;           // [B+1]
  const int64_t* seq_starts;
  const int64_t* seq_ids;        // [B]
  int B;
  uint16_t* v_out;               // [rows, kv_size]; NULL: no v part
};
int launch_kv_rope_scatter(const KvRopeArgs& a, hipStream_t s);
int launch_scatter_dest_rows(const int64_t* row_idx, int64_t M, const int32_t* m_dev, const int32_t* cu,
                             const int64_t* seq_starts, const int64_t* seq_ids, int B, int64_t* dest, hipStream_t s);
int launch_cosine_mask(const float* stats, uint8_t* mask, int64_t T, float tau, hipStream_t s);
int launch_saliency_rows(const uint16_t* c_new, const uint16_t* c_old, float* stats, uint8_t* mask, int64_t T,
                         int64_t D, float tau, hipStream_t s);
int launch_saliency_reduce(const float* part, float* stats, uint8_t* mask, int64_t T, int H, float tau,
                           hipStream_t s);
int launch_compact(const uint8_t* mask, int64_t T, const int32_t* cu_q, int B, const int32_t* cu_prompt,
                   int64_t* idx64, int32_t* idx32, int64_t* idx_k, int32_t* idx_k32, int32_t* cu_sal, int32_t* count,
                   hipStream_t s, int32_t* host_meta = nullptr);
// dest (optional): the row of every salient row in a per-layer cache addressed by dest_starts
// (scatter_update addressing of its K-space row; cu_k = the batch's key prefix)
struct CompactDest {
  const int64_t* dest_starts;
  const int64_t* seq_ids;
  const int32_t* cu_k;
  int64_t* dest;
};
// statistics reduction + tau test + compaction of the native step in one launch (look-back over
// per-workgroup counts). flags: reduce_compact_blocks(T) int32 words, zero before the launch.
constexpr int32_t kCompactLookbackFailed = -2;
int launch_reduce_compact(const float* part, float* stats, uint8_t* mask, int64_t T, int H, float tau,
                          int32_t* flags, const int32_t* cu_q, int B, const int32_t* cu_prompt, int64_t* idx64,
                          int32_t* idx32, int64_t* idx_k, int32_t* idx_k32, int32_t* cu_sal, int32_t* count,
                          int32_t* host_meta, hipStream_t s, const CompactDest& dest);
int64_t reduce_compact_blocks(int64_t T);
int launch_fused_offset(const int32_t* idxs, const int32_t* num_idxs, const int32_t* cu_prompt,
                        const int32_t* cu_sal, int groups, int64_t* out, int64_t cap, hipStream_t s);

enum class AttnMode : int { Dense = 0, RowSparse = 1, ColSparse = 2 };
struct AttnArgs {
  const uint16_t* Q;        // [Tq_all, H, 128]
  const uint16_t* K;        // [*, Hkv, 128]
  const uint16_t* V;        // [*, Hkv, 128]; ColSparse: dV (full, or compact when kslot != NULL)
  const uint16_t* C;        // ColSparse: cached context rows
  const uint16_t* o_sal;    // ColSparse: [n_sal, H, 128]
  uint16_t* O;              // [rows, H, 128]
  const int32_t* cu_rows;   // [B+1] prefix of the rows this launch produces
  const int32_t* cu_k;      // [B+1]
  const int64_t* kv_start;  // optional [B]: first K (and V) row of sequence b (else cu_k[b])
  const int64_t* v_start;   // optional [B]: first V row of sequence b (else as K)
  const int64_t* c_start;   // optional [B]: first C row of sequence b (else cu_rows[b])
  int c_inplace;            // ColSparse: also write the new rows back to C
  const int32_t* q_rows;    // RowSparse: Q row of compact row j
  const int32_t* cu_q;      // RowSparse, fused step: [B+1] Q-space prefix; the tile then writes the
                            // final output row, the context cache row and the statistics itself
  int skip_salient;         // ColSparse, fused step: rows with a slot are left to the row-sparse tiles
  const int32_t* sal_slot;  // ColSparse: [Tq] index into o_sal or -1
  const int32_t* kslot;     // ColSparse, optional: [Tk] row of compact dV or -1
  const uint64_t* kmask;    // ColSparse: [B][nblk] salient-key bits per 64-key block
  float* part;              // ColSparse: [H][3][Tq] per-head partial statistics
  int B, H, Hkv;
  int tiles_per_seq;        // cdiv(max rows per sequence, 128)
  int nblk;                 // kmask row stride
  int64_t Tq;               // ColSparse: rows of part
  float scale_log2;
  // fused step: cache rows through the per-sequence-id start tables (instead of kv_start /
  // v_start / c_start). K row of key k of batch entry b: k_seq_starts[seq_ids[b]] + k; V row
  // likewise; context row of Q row r: c_seq_starts[seq_ids[b]] + (Lk_b - Lq_b) + (r - first Q row).
  const int64_t* seq_ids;       // [B]
  const int64_t* k_seq_starts;  // optional
  const int64_t* v_seq_starts;  // optional
  const int64_t* c_seq_starts;  // optional
  // ColSparse, fused step: the salient maps are built in LDS by each workgroup from the compact
  // lists (no global maps): sal_q / sal_k entries of sequence b are [cu_sal[b], cu_sal[b+1]).
  // dV row of a salient key = cu_sal[b] + its rank among the sequence's salient keys.
  const int32_t* cu_sal;        // [B+1]
  const int32_t* sal_q;         // Q-space rows
  const int32_t* sal_k;         // K-space rows (packed by cu_k)
};
int launch_attention(AttnMode mode, const AttnArgs& a, int max_rows_per_seq, hipStream_t s);
// Row-sparse tiles (fused output) and column-sparse tiles in one launch (4-wave workgroups).
int launch_attention_step(const AttnArgs& rs, int max_rows_rs, const AttnArgs& cs, int max_rows_cs, hipStream_t s);
// device-side unmasking bookkeeping between two sparse steps (unmask.hip)
struct UnmaskArgs {
  int64_t* tok;                 // token rows of the batch, packed by cu_k
  const int32_t* cu_k;          // [B+1]
  const int64_t* pos;           // previous sampler output [B][ld_sampled]: absolute positions
  const int64_t* val;           // ... and tokens
  const int32_t* cnt;           // [B] entries per sequence
  int64_t ld_sampled;
  int32_t* generated;           // [B] generated-token counters (updated)
  const int32_t* prompt_len;    // [B]
  const int32_t* answer_start;  // [B]
  const int32_t* block_size;    // [B]
  int64_t mask_id;
  int pruned;                   // next step queries only the answer rows
  const int32_t* cu_q;          // [B+1] next step's query rows
  int64_t* idx_q;
  int32_t* idx_q32;
  int64_t* idx_k;
  int32_t* idx_k32;
  int32_t* idx_upd;
  int64_t* positions_k;
  int32_t* cu_s;                // [B+1]
  int64_t* input_ids;           // next step's Q-pruned input ids (NULL: not produced)
  int64_t* cand_rel;            // [B][width] candidate offsets from the first queried row
  int32_t* cand_n;              // [B]
  int width;
};
int launch_unmask_step(const UnmaskArgs& a, int batch, hipStream_t s);
// launch resources of the fused step kernel: [regs, local_bytes, static_lds, dynamic_lds, threads,
// max_active_blocks_per_cu, block_q, block_k, d_split, ok]
int attention_kernel_info(int dim, int64_t* out);
int launch_colsparse_prep(const int32_t* idx_q, const int32_t* idx_k, int n_sal, const int32_t* cu_k, int B,
                          int nblk, int32_t* slot, int64_t Tq, uint64_t* kmask, int32_t* kslot, int64_t Tk,
                          hipStream_t s);
// Native sparse step, per salient row (one launch, rope.hip): the optional K/V epilogue (k ->
// k_norm -> RoPE -> K-cache row), dV = bf16(v_new - v_cache[row]) stored at row cu_sal[b] + the
// key's rank among the salient keys of its sequence (the order the column-sparse tiles visit
// them in), and the V-cache row = v_new. Workgroup 0 also zeroes `zero[0..nzero)`.
struct StepRowsArgs {
  int n;                        // salient rows (list entries)
  int B;
  const int32_t* cu_sal;        // [B+1]
  const int32_t* idx_k32;       // [n] K-space rows (packed by cu_k)
  const int32_t* cu_k;          // [B+1]
  const int64_t* seq_ids;       // [B]
  uint16_t* v_cache;            // rows of kv_size elements
  const int64_t* v_seq_starts;
  int64_t kv_size;              // Hkv * 128
  int Hkv;
  const uint16_t* v_new;        // [n, kv_size] in list order; NULL: v is the second half of the kv rows
  const uint16_t* kv;           // optional [*, ld_kv] = [k | v] of the projection (K/V epilogue)
  int64_t ld_kv;
  const int32_t* kv_rows;       // optional: kv row of list entry j (else j)
  const int64_t* positions;
  const int32_t* pos_idx;       // optional: index into positions of entry j (else j)
  const float* cos;             // [max_position, 64]
  const float* sin;
  int64_t max_position;
  const uint16_t* k_norm;       // optional [128]
  float eps;
  uint16_t* k_cache;            // rows of kv_size elements
  const int64_t* k_seq_starts;
  uint16_t* dv;                 // [n, kv_size] out
  int32_t* zero;                // optional words zeroed by workgroup 0
  int nzero;
};
int launch_step_rows(const StepRowsArgs& a, hipStream_t s);
int launch_v_delta_update(uint16_t* v_cache, const uint16_t* v_new, const int64_t* dest_rows, int64_t n,
                          int64_t row_elems, uint16_t* dv, hipStream_t s);
int launch_seq_row_starts(const int64_t* seq_starts, const int64_t* seq_ids, const int32_t* cu_k,
                          const int32_t* cu_q, int B, int64_t* out, hipStream_t s);

enum class GemmEpi : int { Store = 0, SwiGLU = 1 };
struct GemmArgs {
  const uint16_t* A;
  int64_t lda;
  int64_t a_rows;             // rows A holds, when known (0: unknown); A spans < 4 GiB either way
  const int32_t* a_ids;
  int a_div;
  const int32_t* a_map;       // optional: A row of id = a_map[id / a_div] (else id / a_div)
  int64_t id_limit;
  const uint16_t* W;
  int64_t ldw;
  int64_t w_expert_stride;
  const int32_t* tile_expert;
  const int32_t* num_m_dev;
  uint16_t* Cout;
  int64_t ldc;
  const int64_t* c_rows;
  int c_by_id;
  const float* row_scale_f32;
  const uint16_t* row_scale_bf16;
  const uint16_t* bias;       // Store epilogue, optional: bf16 [N] added in fp32 before rounding
  int64_t M;
  int N, K;
  int half_n;
  float* partial;             // split-K: fp32 partial tiles [ksplit][m_pad][N] (Store epilogue only)
  int ksplit;                 // number of K slices (1: no split)
  int64_t m_pad;              // rows of one partial slice (m tiles launched * BM)
};
// tile_m: 128 / 192 / 256, or 0 to choose from M and the grid size. ksplit > 1 needs
// g.partial with gemm_partial_bytes() bytes and is followed by the reduction kernel.
int launch_gemm(GemmEpi epi, const GemmArgs& g, int64_t m_bound, int tile_m, int ksplit, hipStream_t s);
// out[r] = bf16(silu(g) * u) for gu rows [g (inter) | u (inter)] (act.hip)
int launch_silu_and_mul(const uint16_t* gu, int64_t ld_in, int64_t rows, int inter, uint16_t* out, int64_t ld_out,
                        hipStream_t s);
size_t gemm_partial_bytes(int64_t m_bound, int N, int tile_m, int ksplit);
struct GemmPlan {
  int tile_m;   // 128 / 192 / 256
  int ksplit;   // 1 unless the Store epilogue is split along K
};
// tile height and split-K factor for an M x N x K product (measured cost model)
GemmPlan gemm_plan(int64_t M, int N, int K, GemmEpi epi);

int launch_moe_router(const uint16_t* x, const int32_t* rows, const uint16_t* wr, int64_t T, int Hd, int E, int top_k,
                      int renorm, uint16_t* topk_w, int32_t* topk_ids, hipStream_t s);
int launch_moe_align(const int32_t* ids, int64_t S, int E, int bm, int32_t* sorted_ids, int64_t cap,
                     int32_t* tile_expert, int32_t* num_post_pad, hipStream_t s);
int launch_moe_combine(const uint16_t* y, int64_t T, int Hd, int top_k, uint16_t* out, const int64_t* dst_rows,
                       hipStream_t s);

// issue-rate probe (probe.hip): per-wavefront cycles of MFMA / VALU loops alone and together
int launch_issue_probe(int mode, int wgs, int iters, float* sink, unsigned long long* cyc, hipStream_t s);

}  // namespace dyllm

// extern "C" entry points of libdyllm_hip.so: argument validation, workspace carving and
// kernel launches. No host synchronisation and no device allocation happens here.
#include "../../include/dyllm_hip.h"
#include "kernels.h"

#include <cstdint>
#include <initializer_list>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace dyllm {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
int fail(const std::string& msg) {
  g_last_error = msg;
  return 1;
}
int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  return fail(std::string(what) + ": " + hipGetErrorString(e));
}

static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Optional timing of the fused attention kernel of dyllm_sparse_attention_step (for the
// benchmark's live roofline): while enabled, each call records a library-owned event pair around
// that one launch on the caller's stream.
struct AttnTimer {
  bool enabled = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
  size_t used = 0;
};
static thread_local AttnTimer g_attn_timer;
// true when every non-null pointer is a multiple of `bytes` (vector loads / stores of that width)
static inline bool aligned_to(size_t bytes, std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (p && reinterpret_cast<uintptr_t>(p) % bytes != 0) return false;
  return true;
}
static const float kLog2e = 1.4426950408889634f;

// Workspace of dyllm_sparse_attention_step_noalloc: one library-owned device array per GPU,
// resolved to its device address once per device with hipGetSymbolAddress (the host-side name
// is not a device address). Every call on a GPU shares that GPU's array; calls that overlap on
// one GPU race. Nothing in it has to start at zero: the step's first launch resets its maps.
constexpr size_t kStepScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kStepScratchBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kMaxDevices] = {};

static int step_scratch_ptr(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return fail("no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return 0;
}
// Expert bucket height (= grouped GEMM tile height): 192-row tiles once the mean expert load
// reaches 256 slots (config 3, 461 slots per expert: grouped gate_up 346 -> 302 us, down 227 ->
// 207 us against 128-row tiles; 256-row tiles 328 / 219 us), 128-row tiles below that, where the
// padding of each bucket to the tile height weighs more.
static int moe_block(int64_t slots, int E) { return slots >= int64_t(256) * E ? 192 : 128; }

}  // namespace dyllm

using namespace dyllm;

#define DYLLM_STREAM(s) reinterpret_cast<hipStream_t>(s)
#define DYLLM_NONNULL(p) DYLLM_REQUIRE((p) != nullptr, #p " must not be NULL")

extern "C" {

const char* dyllm_last_error(void) { return g_last_error.c_str(); }

int dyllm_attention_timer(int enable) {
  g_attn_timer.enabled = enable != 0;
  return 0;
}

int dyllm_attention_timer_read(float* total_ms, int* launches) {
  DYLLM_NONNULL(total_ms);
  DYLLM_NONNULL(launches);
  AttnTimer& tm = g_attn_timer;
  float sum = 0.f;
  for (size_t i = 0; i < tm.used; ++i) {
    float ms = 0.f;
    if (hipEventSynchronize(tm.ev[i].second) != hipSuccess ||
        hipEventElapsedTime(&ms, tm.ev[i].first, tm.ev[i].second) != hipSuccess)
      return fail("attention timer: event query failed");
    sum += ms;
  }
  *total_ms = sum;
  *launches = int(tm.used);
  tm.used = 0;
  return 0;
}
int dyllm_abi_version(void) { return 5; }

int dyllm_issue_probe(int mode, int workgroups, int iters, void* sink, void* cycles, void* stream) {
  DYLLM_NONNULL(sink);
  DYLLM_NONNULL(cycles);
  DYLLM_REQUIRE(workgroups >= 1 && iters >= 1, "workgroups and iters must be positive");
  return launch_issue_probe(mode, workgroups, iters, static_cast<float*>(sink),
                            static_cast<unsigned long long*>(cycles), DYLLM_STREAM(stream));
}

// ---------------------------------------------------------------------------------------
size_t dyllm_attention_sparse_workspace_bytes(int batch, int num_heads, int64_t total_q, int max_seqlen_k) {
  const int64_t nblk = cdiv(max_seqlen_k > 0 ? max_seqlen_k : 1, 64);
  return align256(size_t(total_q) * 4) + align256(size_t(batch) * nblk * 8) +
         align256(size_t(num_heads) * 3 * size_t(total_q) * 4);
}

size_t dyllm_attention_colsparse_workspace_bytes(int batch, int num_heads, int64_t total_q, int64_t total_k,
                                                 int max_seqlen_k) {
  return dyllm_attention_sparse_workspace_bytes(batch, num_heads, total_q, max_seqlen_k) + align256(size_t(total_k) * 4);
}

// Shared body of the two column-sparse entry points. kslot_bytes > 0 selects a compact dV.
// workspace layout of the column-sparse attention: slot map [Tq], salient-key bits [B][nblk],
// per-head statistics [H][3][Tq], dV slot map [Tk] (compact dV only)
struct ColsWs {
  int32_t* slot;
  uint64_t* kmask;
  float* part;
  int32_t* kslot;
};
static ColsWs cols_ws(void* workspace, int batch, int num_heads, int64_t total_q, int nblk, bool compact_dv) {
  char* ws = static_cast<char*>(workspace);
  ColsWs w{};
  w.slot = reinterpret_cast<int32_t*>(ws);
  ws += align256(size_t(total_q) * 4);
  w.kmask = reinterpret_cast<uint64_t*>(ws);
  ws += align256(size_t(batch) * nblk * 8);
  w.part = reinterpret_cast<float*>(ws);
  ws += align256(size_t(num_heads) * 3 * size_t(total_q) * 4);
  w.kslot = compact_dv ? reinterpret_cast<int32_t*>(ws) : nullptr;
  return w;
}

static int colsparse_impl(const void* q, const void* k, const int64_t* kv_start, const void* v_delta,
                          const void* c, const int64_t* c_start, int c_inplace, const void* o_sal, void* o, int batch,
                          int num_heads, int num_kv_heads, int head_dim, const int32_t* cu_seqlens_q,
                          const int32_t* cu_seqlens_k, int max_seqlen_q, int max_seqlen_k, int64_t total_q,
                          int64_t total_k, int num_salient, const int32_t* idx_salient_q,
                          const int32_t* idx_salient_k, float* cosine_stats, uint8_t* cosine_out, float threshold,
                          void* workspace, size_t workspace_bytes, bool compact_dv, void* stream,
                          bool maps_ready = false, bool reduce = true) {
  DYLLM_NONNULL(q);
  DYLLM_NONNULL(k);
  DYLLM_NONNULL(c);
  DYLLM_NONNULL(o);
  DYLLM_NONNULL(cu_seqlens_q);
  DYLLM_NONNULL(cu_seqlens_k);
  DYLLM_NONNULL(cosine_stats);
  DYLLM_NONNULL(cosine_out);
  DYLLM_REQUIRE(head_dim == 128, "supported head dimension is 128, got " + std::to_string(head_dim));
  DYLLM_REQUIRE(batch >= 1, "batch must be >= 1");
  DYLLM_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
                "query heads must be a positive multiple of KV heads; got " + std::to_string(num_heads) + " and " +
                    std::to_string(num_kv_heads));
  DYLLM_REQUIRE(total_q > 0, "Q and K/V token dimensions must be non-empty");
  DYLLM_REQUIRE(max_seqlen_q > 0 && max_seqlen_q <= total_q && max_seqlen_k > 0,
                "maximum sequence lengths must be positive and fit their packed token dimensions");
  DYLLM_REQUIRE(num_salient >= 0 && num_salient <= total_q, "salient Q index count cannot exceed Q.size(0)");
  DYLLM_REQUIRE(num_salient == 0 || (o_sal && idx_salient_q), "o_sal and idx_salient_q are required");
  DYLLM_REQUIRE(v_delta != nullptr || (compact_dv && num_salient == 0), "v_delta must not be NULL");
  const size_t need = compact_dv
                          ? dyllm_attention_colsparse_workspace_bytes(batch, num_heads, total_q, total_k, max_seqlen_k)
                          : dyllm_attention_sparse_workspace_bytes(batch, num_heads, total_q, max_seqlen_k);
  DYLLM_REQUIRE(workspace && workspace_bytes >= need,
                "workspace too small: need " + std::to_string(need) + " bytes");
  const hipStream_t s = DYLLM_STREAM(stream);
  const int nblk = int(cdiv(max_seqlen_k, 64));
  const ColsWs cw = cols_ws(workspace, batch, num_heads, total_q, nblk, compact_dv);
  int32_t* slot = cw.slot;
  uint64_t* kmask = cw.kmask;
  float* part = cw.part;
  int32_t* kslot = cw.kslot;
  if (!maps_ready) {
    if (int rc = launch_colsparse_prep(idx_salient_q, idx_salient_k ? idx_salient_k : idx_salient_q, num_salient,
                                       cu_seqlens_k, batch, nblk, slot, total_q, kmask, kslot, total_k, s))
      return rc;
  }
  AttnArgs a{};
  a.Q = static_cast<const uint16_t*>(q);
  a.K = static_cast<const uint16_t*>(k);
  a.V = static_cast<const uint16_t*>(v_delta);
  a.C = static_cast<const uint16_t*>(c);
  a.o_sal = static_cast<const uint16_t*>(o_sal);
  a.O = static_cast<uint16_t*>(o);
  a.cu_rows = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.kv_start = kv_start;
  a.c_start = c_start;
  a.c_inplace = c_inplace;
  a.sal_slot = slot;
  a.kslot = kslot;
  a.kmask = kmask;
  a.part = part;
  a.B = batch;
  a.H = num_heads;
  a.Hkv = num_kv_heads;
  a.nblk = nblk;
  a.Tq = total_q;
  // the reference uses rsqrt(head_dim) here, not the layer's scale (sm80.cu:166-168)
  a.scale_log2 = (1.0f / sqrtf(float(head_dim))) * kLog2e;
  if (int rc = launch_attention(AttnMode::ColSparse, a, max_seqlen_q, s)) return rc;
  if (!reduce) return 0;
  return launch_saliency_reduce(part, cosine_stats, cosine_out, total_q, num_heads, threshold, s);
}

int dyllm_attention_sparse_varlen(const void* q, const void* k, const void* v_delta, const void* c,
                                  const void* o_sal, void* o, int batch, int num_heads, int num_kv_heads,
                                  int head_dim, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int max_seqlen_q, int max_seqlen_k, int64_t total_q, int num_salient,
                                  const int32_t* cu_salientlens, const int32_t* idx_salient_q,
                                  const int32_t* idx_salient_k, float* cosine_stats, uint8_t* cosine_out,
                                  float threshold, void* workspace, size_t workspace_bytes, void* stream) {
  (void)cu_salientlens;  // per-sequence salient ranges are implied by the sorted index lists
  return colsparse_impl(q, k, nullptr, v_delta, c, nullptr, 0, o_sal, o, batch, num_heads, num_kv_heads, head_dim,
                        cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, total_q, 0, num_salient,
                        idx_salient_q, idx_salient_k, cosine_stats, cosine_out, threshold, workspace,
                        workspace_bytes, false, stream);
}

int dyllm_attention_colsparse_cached(const void* q, const void* k_cache, const int64_t* kv_start,
                                     const void* dv_compact, void* c_cache, const int64_t* c_start,
                                     int c_inplace, const void* o_sal, void* o, int batch, int num_heads,
                                     int num_kv_heads, int head_dim, const int32_t* cu_seqlens_q,
                                     const int32_t* cu_seqlens_k, int max_seqlen_q, int max_seqlen_k,
                                     int64_t total_q, int64_t total_k, int num_salient,
                                     const int32_t* idx_salient_q, const int32_t* idx_salient_k,
                                     float* cosine_stats, uint8_t* cosine_out, float threshold, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  DYLLM_REQUIRE(total_k > 0, "total_k must be positive");
  return colsparse_impl(q, k_cache, kv_start, dv_compact, c_cache, c_start, c_inplace, o_sal, o, batch, num_heads,
                        num_kv_heads, head_dim, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, total_q,
                        total_k, num_salient, idx_salient_q, idx_salient_k, cosine_stats, cosine_out, threshold,
                        workspace, workspace_bytes, true, stream);
}

size_t dyllm_sparse_step_workspace_bytes(int batch, int num_heads, int num_kv_heads, int head_dim, int64_t total_q,
                                         int64_t total_k, int max_seqlen_k, int64_t num_salient) {
  (void)batch;
  (void)total_k;
  (void)max_seqlen_k;
  const size_t n = size_t(num_salient > 0 ? num_salient : 0);
  return align256(n * num_kv_heads * head_dim * 2) + align256(size_t(cdiv(total_q > 0 ? total_q : 1, 256)) * 4) +
         align256(size_t(num_heads) * 3 * size_t(total_q > 0 ? total_q : 0) * 4);
}

// the fused attention launch, bracketed by the attention timer's events when it is enabled
static int timed_attention_step(const AttnArgs& rs, int rs_rows, const AttnArgs& cs, int cs_rows, hipStream_t s) {
  AttnTimer& tm = g_attn_timer;
  hipEvent_t e1 = nullptr;
  if (tm.enabled) {
    if (tm.used == tm.ev.size()) {
      hipEvent_t a0 = nullptr, a1 = nullptr;
      if (hipEventCreate(&a0) != hipSuccess || hipEventCreate(&a1) != hipSuccess)
        return fail("hipEventCreate failed (attention timer)");
      tm.ev.emplace_back(a0, a1);
    }
    if (hipEventRecord(tm.ev[tm.used].first, s) != hipSuccess) return fail("hipEventRecord failed (attention timer)");
    e1 = tm.ev[tm.used].second;
    ++tm.used;
  }
  if (int rc = launch_attention_step(rs, rs_rows, cs, cs_rows, s)) return rc;
  if (e1 && hipEventRecord(e1, s) != hipSuccess) return fail("hipEventRecord failed (attention timer)");
  return 0;
}

// Body of dyllm_sparse_attention_step(_kv): three launches.
//   1. step_rows_kernel: per salient row, [K/V epilogue], dV (at the key's rank within its
//      sequence) and the V-cache update;
//   2. attention_step_kernel: row-sparse tiles of the salient queries + column-sparse tiles of
//      the others (their salient maps built in LDS from the lists);
//   3. reduce_compact_kernel: head sums, tau test and the next salient set in one pass.
static int sparse_step(const dyllm_kv_epilogue* epi, const void* q, const void* k, const int64_t* k_start,
                       void* v_cache, const int64_t* v_seq_starts, const void* v_new, void* c_cache,
                       const int64_t* c_seq_starts, const int64_t* seq_ids, int batch, int num_heads, int num_kv_heads,
                       int head_dim, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                       const int32_t* cu_promptlens, int max_seqlen_q, int max_seqlen_k, int64_t total_q,
                       int64_t total_k, int num_salient, int max_salientlen, const int32_t* cu_salientlens,
                       const int32_t* idx_q32, const int64_t* idx_k64, const int32_t* idx_k32, float softmax_scale,
                       float threshold, void* out, float* cosine_stats, uint8_t* cosine_out, int64_t* next_idx64,
                       int32_t* next_idx32, int64_t* next_idx_k64, int32_t* next_idx_k32,
                       int32_t* next_cu_salientlens, int32_t* next_count, const int64_t* dest_seq_starts,
                       int64_t* next_dest_rows, int32_t* host_meta, void* workspace, size_t workspace_bytes,
                       void* stream) {
  (void)idx_k64;
  DYLLM_NONNULL(q);
  DYLLM_NONNULL(v_cache);
  DYLLM_NONNULL(v_seq_starts);
  DYLLM_NONNULL(c_cache);
  DYLLM_NONNULL(c_seq_starts);
  DYLLM_NONNULL(seq_ids);
  DYLLM_NONNULL(out);
  DYLLM_NONNULL(cu_seqlens_q);
  DYLLM_NONNULL(cu_seqlens_k);
  DYLLM_NONNULL(cu_salientlens);
  DYLLM_NONNULL(cosine_stats);
  DYLLM_NONNULL(cosine_out);
  DYLLM_NONNULL(next_idx64);
  DYLLM_NONNULL(next_cu_salientlens);
  DYLLM_NONNULL(next_count);
  DYLLM_REQUIRE(head_dim == 128, "supported head dimension is 128, got " + std::to_string(head_dim));
  DYLLM_REQUIRE(batch >= 1, "batch must be >= 1");
  DYLLM_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
                "query heads must be a positive multiple of KV heads");
  DYLLM_REQUIRE(total_q > 0 && total_k > 0 && total_q < (int64_t(1) << 31) && total_k < (int64_t(1) << 31),
                "token counts out of range");
  DYLLM_REQUIRE(max_seqlen_q > 0 && max_seqlen_q <= total_q && max_seqlen_k > 0, "bad maximum sequence lengths");
  DYLLM_REQUIRE(num_salient >= 0 && num_salient <= total_q, "num_salient out of range");
  DYLLM_REQUIRE(num_salient == 0 || (idx_q32 && idx_k32), "salient rows need the int32 Q and K index lists");
  DYLLM_REQUIRE(cu_promptlens == nullptr || next_idx_k64 != nullptr, "Q-pruned steps need next_idx_k64");
  if (epi) {
    DYLLM_REQUIRE(k == nullptr && k_start == nullptr && v_new == nullptr,
                  "with a K/V epilogue, K comes from its cache and v from its rows (k, k_start, v_new must be NULL)");
    DYLLM_REQUIRE(epi->k_cache && epi->k_seq_starts && epi->positions && epi->cos_table && epi->sin_table,
                  "the K/V epilogue needs k_cache, k_seq_starts, positions and the cos / sin tables");
    DYLLM_REQUIRE(num_salient == 0 || epi->kv, "the K/V epilogue needs the kv rows");
    DYLLM_REQUIRE(epi->max_position >= 1, "max_position must be positive");
    DYLLM_REQUIRE(epi->ld_kv >= int64_t(2) * num_kv_heads * head_dim && epi->ld_kv % 8 == 0,
                  "kv row stride must be >= 2 * num_kv_heads * 128 and a multiple of 8");
    DYLLM_REQUIRE(aligned_to(16, {epi->kv, epi->cos_table, epi->sin_table, epi->k_norm_weight, epi->k_cache}),
                  "kv, the cos / sin tables, k_norm_weight and k_cache must be 16-byte aligned");
  } else {
    DYLLM_NONNULL(k);
    DYLLM_REQUIRE(num_salient == 0 || v_new, "salient rows need v_new");
  }
  const size_t need = dyllm_sparse_step_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, total_q, total_k,
                                                        max_seqlen_k, num_salient);
  DYLLM_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need " + std::to_string(need) + " bytes");
  const hipStream_t s = DYLLM_STREAM(stream);
  int32_t* host_meta_dev = nullptr;
  if (host_meta) {
    void* p = nullptr;
    DYLLM_REQUIRE(hipHostGetDevicePointer(&p, host_meta, 0) == hipSuccess && p != nullptr,
                  "host_meta must be pinned host memory (hipHostMalloc)");
    host_meta_dev = static_cast<int32_t*>(p);
  }
  DYLLM_REQUIRE(next_dest_rows == nullptr || dest_seq_starts != nullptr, "next_dest_rows needs dest_seq_starts");
  const int64_t kv_size = int64_t(num_kv_heads) * head_dim;
  const size_t n = size_t(num_salient);
  char* ws = static_cast<char*>(workspace);
  uint16_t* dv = reinterpret_cast<uint16_t*>(ws);
  ws += align256(n * kv_size * 2);
  int32_t* flags = reinterpret_cast<int32_t*>(ws);  // compaction look-back: salient rows + 1 per 256-row block
  const int nflags = int(reduce_compact_blocks(total_q));
  ws += align256(size_t(nflags) * 4);
  float* part = reinterpret_cast<float*>(ws);
  const bool q_pruned = cu_promptlens != nullptr;
  const int nblk = int(cdiv(max_seqlen_k, 64));

  // 1. per salient row: [K/V epilogue], dV, V-cache update (attention.py:67-74, 89-96; llada.py:103-146);
  // workgroup 0 also clears the compaction's look-back flags
  {
    StepRowsArgs ra{};
    ra.n = num_salient;
    ra.B = batch;
    ra.cu_sal = cu_salientlens;
    ra.idx_k32 = idx_k32;
    ra.cu_k = cu_seqlens_k;
    ra.seq_ids = seq_ids;
    ra.v_cache = static_cast<uint16_t*>(v_cache);
    ra.v_seq_starts = v_seq_starts;
    ra.kv_size = kv_size;
    ra.Hkv = num_kv_heads;
    ra.v_new = static_cast<const uint16_t*>(v_new);
    if (epi) {
      ra.kv = static_cast<const uint16_t*>(epi->kv);
      ra.ld_kv = epi->ld_kv;
      ra.kv_rows = epi->kv_rows;
      ra.positions = epi->positions;
      ra.pos_idx = epi->pos_idx;
      ra.cos = epi->cos_table;
      ra.sin = epi->sin_table;
      ra.max_position = epi->max_position;
      ra.k_norm = static_cast<const uint16_t*>(epi->k_norm_weight);
      ra.eps = epi->eps;
      ra.k_cache = static_cast<uint16_t*>(epi->k_cache);
      ra.k_seq_starts = epi->k_seq_starts;
    }
    ra.dv = dv;
    ra.zero = flags;
    ra.nzero = nflags;
    if (int rc = launch_step_rows(ra, s)) return rc;
  }
  // 2. row-sparse attention of the salient queries vs the full cached K/V (attention.py:76-87),
  // launched together with the column-sparse attention of the other rows (statistics + tau
  // inputs, context cache updated in place); each salient row's tile writes its final output,
  // context row and statistics itself (attention_aux_kernels.cu:22-72)
  AttnArgs rs{};
  rs.Q = static_cast<const uint16_t*>(q);
  rs.K = static_cast<const uint16_t*>(epi ? epi->k_cache : k);
  rs.V = static_cast<const uint16_t*>(v_cache);
  rs.C = static_cast<const uint16_t*>(c_cache);
  rs.O = static_cast<uint16_t*>(out);
  rs.cu_rows = cu_salientlens;
  rs.cu_k = cu_seqlens_k;
  rs.cu_q = cu_seqlens_q;
  rs.kv_start = k_start;
  rs.seq_ids = seq_ids;
  rs.k_seq_starts = epi ? epi->k_seq_starts : nullptr;
  rs.v_seq_starts = v_seq_starts;
  rs.c_seq_starts = c_seq_starts;
  rs.c_inplace = 1;
  rs.q_rows = idx_q32;
  rs.part = part;
  rs.Tq = total_q;
  rs.B = batch;
  rs.H = num_heads;
  rs.Hkv = num_kv_heads;
  rs.scale_log2 = softmax_scale * kLog2e;
  AttnArgs cs = rs;
  cs.V = dv;
  cs.cu_rows = cu_seqlens_q;
  cs.cu_q = nullptr;
  cs.q_rows = nullptr;
  cs.v_seq_starts = nullptr;
  cs.skip_salient = 1;
  cs.nblk = nblk;
  cs.cu_sal = cu_salientlens;
  cs.sal_q = num_salient > 0 ? idx_q32 : nullptr;
  cs.sal_k = num_salient > 0 ? idx_k32 : nullptr;
  // the reference's column-sparse kernel uses rsqrt(head_dim), not the layer's scale (sm80.cu:166-168)
  cs.scale_log2 = (1.0f / sqrtf(float(head_dim))) * kLog2e;
  const int rs_rows = num_salient > 0 ? (max_salientlen > 0 ? max_salientlen : max_seqlen_q) : 0;
  if (num_salient == 0) {
    // no salient key: every column-sparse row is C_old + 0 (an empty list drives the same LDS path)
    cs.sal_q = idx_q32 ? idx_q32 : reinterpret_cast<const int32_t*>(cu_salientlens);
    cs.sal_k = idx_k32 ? idx_k32 : reinterpret_cast<const int32_t*>(cu_salientlens);
  }
  if (int rc = timed_attention_step(rs, rs_rows, cs, max_seqlen_q, s)) return rc;
  // 3. statistics reduction, tau test and compaction of the next salient set (attention.py:141-173)
  CompactDest dd{};
  if (next_dest_rows) dd = CompactDest{dest_seq_starts, seq_ids, cu_seqlens_k, next_dest_rows};
  return launch_reduce_compact(part, cosine_stats, cosine_out, total_q, num_heads, threshold, flags, cu_seqlens_q, batch,
                               cu_promptlens, next_idx64, next_idx32, q_pruned ? next_idx_k64 : nullptr,
                               q_pruned ? next_idx_k32 : nullptr, next_cu_salientlens, next_count, host_meta_dev, s,
                               dd);
}

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
                                void* stream) {
  return sparse_step(nullptr, q, k, k_start, v_cache, v_seq_starts, v_new, c_cache, c_seq_starts, seq_ids, batch,
                     num_heads, num_kv_heads, head_dim, cu_seqlens_q, cu_seqlens_k, cu_promptlens, max_seqlen_q,
                     max_seqlen_k, total_q, total_k, num_salient, max_salientlen, cu_salientlens, idx_q32, idx_k64,
                     idx_k32, softmax_scale, threshold, out, cosine_stats, cosine_out, next_idx64, next_idx32,
                     next_idx_k64, next_idx_k32, next_cu_salientlens, next_count, dest_seq_starts, next_dest_rows,
                     host_meta, workspace, workspace_bytes, stream);
}

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
                                   int32_t* host_meta, void* workspace, size_t workspace_bytes, void* stream) {
  DYLLM_NONNULL(kv_epilogue);
  return sparse_step(kv_epilogue, q, k, k_start, v_cache, v_seq_starts, v_new, c_cache, c_seq_starts, seq_ids, batch,
                     num_heads, num_kv_heads, head_dim, cu_seqlens_q, cu_seqlens_k, cu_promptlens, max_seqlen_q,
                     max_seqlen_k, total_q, total_k, num_salient, max_salientlen, cu_salientlens, idx_q32, idx_k64,
                     idx_k32, softmax_scale, threshold, out, cosine_stats, cosine_out, next_idx64, next_idx32,
                     next_idx_k64, next_idx_k32, next_cu_salientlens, next_count, dest_seq_starts, next_dest_rows,
                     host_meta, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------------------
// dyllm_sparse_attention_step_noalloc: the same step with its workspace carved from a
// library-owned device array instead of a caller buffer, for callers that cannot allocate.
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
                                        void* stream) {
  DYLLM_REQUIRE(num_salient >= 0 && batch >= 1 && total_q >= 0 && total_k >= 0, "bad sizes");
  const size_t need = dyllm_sparse_step_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, total_q, total_k,
                                                        max_seqlen_k, num_salient);
  DYLLM_REQUIRE(need <= kStepScratchBytes, "step needs " + std::to_string(need) +
                                               " bytes of scratch; the no-allocation entry point holds " +
                                               std::to_string(kStepScratchBytes) + " (use dyllm_sparse_attention_step)");
  void* ws = nullptr;
  if (int rc = step_scratch_ptr(&ws)) return rc;
  return dyllm_sparse_attention_step(q, k, k_start, v_cache, v_seq_starts, v_new, c_cache, c_seq_starts, seq_ids,
                                     batch, num_heads, num_kv_heads, head_dim, cu_seqlens_q, cu_seqlens_k,
                                     cu_promptlens, max_seqlen_q, max_seqlen_k, total_q, total_k, num_salient,
                                     max_salientlen, cu_salientlens, idx_q32, idx_k64, idx_k32, softmax_scale,
                                     threshold, out, cosine_stats, cosine_out, next_idx64, next_idx32, next_idx_k64,
                                     next_idx_k32, next_cu_salientlens, next_count, dest_seq_starts, next_dest_rows,
                                     host_meta, ws, kStepScratchBytes, stream);
}

size_t dyllm_sparse_step_scratch_bytes(void) { return kStepScratchBytes; }

int dyllm_unmask_step(int64_t* tokens, const int32_t* cu_seqlens_k, int batch, const int64_t* sampled_pos,
                      const int64_t* sampled_tok, const int32_t* sampled_counts, int64_t ld_sampled,
                      int32_t* generated, const int32_t* prompt_len, const int32_t* answer_start,
                      const int32_t* block_size, int64_t mask_id, int q_pruned, const int32_t* cu_seqlens_q,
                      int64_t* idx_q, int32_t* idx_q32, int64_t* idx_k, int32_t* idx_k32, int32_t* idx_upd,
                      int64_t* positions_k, int32_t* cu_salientlens, int64_t* input_ids, int64_t* cand_rel,
                      int32_t* cand_n, int width, void* stream) {
  for (const void* p : {(const void*)tokens, (const void*)cu_seqlens_k, (const void*)sampled_pos,
                        (const void*)sampled_tok, (const void*)sampled_counts, (const void*)generated,
                        (const void*)prompt_len, (const void*)answer_start, (const void*)block_size,
                        (const void*)cu_seqlens_q, (const void*)idx_q, (const void*)idx_q32, (const void*)idx_k,
                        (const void*)idx_k32, (const void*)idx_upd, (const void*)positions_k,
                        (const void*)cu_salientlens, (const void*)cand_rel, (const void*)cand_n})
    DYLLM_REQUIRE(p != nullptr, "null pointer argument");
  UnmaskArgs a{};
  a.tok = tokens;
  a.cu_k = cu_seqlens_k;
  a.pos = sampled_pos;
  a.val = sampled_tok;
  a.cnt = sampled_counts;
  a.ld_sampled = ld_sampled;
  a.generated = generated;
  a.prompt_len = prompt_len;
  a.answer_start = answer_start;
  a.block_size = block_size;
  a.mask_id = mask_id;
  a.pruned = q_pruned ? 1 : 0;
  a.cu_q = cu_seqlens_q;
  a.idx_q = idx_q;
  a.idx_q32 = idx_q32;
  a.idx_k = idx_k;
  a.idx_k32 = idx_k32;
  a.idx_upd = idx_upd;
  a.positions_k = positions_k;
  a.cu_s = cu_salientlens;
  a.input_ids = input_ids;
  a.cand_rel = cand_rel;
  a.cand_n = cand_n;
  a.width = width;
  return launch_unmask_step(a, batch, DYLLM_STREAM(stream));
}

int dyllm_attention_kernel_info(int dim, int mask_v_rows, int64_t* out) {
  DYLLM_NONNULL(out);
  (void)mask_v_rows;   // one kernel: the column-sparse tiles always skip PV on key groups without salient rows
  return attention_kernel_info(dim, out);
}

int dyllm_v_delta_update(void* v_cache, const void* v_new, const int64_t* dest_rows, int64_t rows,
                         int64_t row_elems, void* dv_out, void* stream) {
  DYLLM_REQUIRE(rows == 0 || (v_cache && v_new && dest_rows && dv_out), "null pointer argument");
  return launch_v_delta_update(static_cast<uint16_t*>(v_cache), static_cast<const uint16_t*>(v_new), dest_rows, rows,
                               row_elems, static_cast<uint16_t*>(dv_out), DYLLM_STREAM(stream));
}

int dyllm_seq_row_starts(const int64_t* seq_starts, const int64_t* seq_ids, const int32_t* cu_seqlens_k,
                         const int32_t* cu_seqlens_q, int batch, int64_t* out, void* stream) {
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(seq_ids);
  DYLLM_NONNULL(out);
  DYLLM_REQUIRE(cu_seqlens_q == nullptr || cu_seqlens_k != nullptr, "cu_seqlens_k is required with cu_seqlens_q");
  return launch_seq_row_starts(seq_starts, seq_ids, cu_seqlens_k, cu_seqlens_q, batch, out, DYLLM_STREAM(stream));
}

int dyllm_flash_attn_varlen(const void* q, const void* k, const void* v, void* o, int batch, int num_heads,
                            int num_kv_heads, int head_dim, const int32_t* cu_seqlens_q,
                            const int32_t* cu_seqlens_k, const int64_t* kv_start, int max_seqlen_q, int max_seqlen_k,
                            float softmax_scale, const int32_t* q_rows, void* stream) {
  DYLLM_NONNULL(q);
  DYLLM_NONNULL(k);
  DYLLM_NONNULL(v);
  DYLLM_NONNULL(o);
  DYLLM_NONNULL(cu_seqlens_q);
  DYLLM_NONNULL(cu_seqlens_k);
  DYLLM_REQUIRE(head_dim == 128, "supported head dimension is 128, got " + std::to_string(head_dim));
  DYLLM_REQUIRE(batch >= 1, "batch must be >= 1");
  DYLLM_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0, "bad head counts");
  DYLLM_REQUIRE(max_seqlen_q >= 0 && max_seqlen_k > 0, "bad maximum sequence lengths");
  AttnArgs a{};
  a.Q = static_cast<const uint16_t*>(q);
  a.K = static_cast<const uint16_t*>(k);
  a.V = static_cast<const uint16_t*>(v);
  a.O = static_cast<uint16_t*>(o);
  a.cu_rows = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.kv_start = kv_start;
  a.q_rows = q_rows;
  a.B = batch;
  a.H = num_heads;
  a.Hkv = num_kv_heads;
  a.scale_log2 = softmax_scale * kLog2e;
  return launch_attention(q_rows ? AttnMode::RowSparse : AttnMode::Dense, a, max_seqlen_q, DYLLM_STREAM(stream));
}

// ---------------------------------------------------------------------------------------
int dyllm_cosine_mask(const float* stats, int64_t rows, float threshold, uint8_t* mask, void* stream) {
  DYLLM_NONNULL(stats);
  DYLLM_NONNULL(mask);
  return launch_cosine_mask(stats, mask, rows, threshold, DYLLM_STREAM(stream));
}

int dyllm_saliency_stats(const void* c_new, const void* c_old, int64_t rows, int64_t dim, float threshold,
                         float* stats, uint8_t* mask, void* stream) {
  DYLLM_NONNULL(c_new);
  DYLLM_NONNULL(c_old);
  DYLLM_NONNULL(stats);
  DYLLM_NONNULL(mask);
  return launch_saliency_rows(static_cast<const uint16_t*>(c_new), static_cast<const uint16_t*>(c_old), stats, mask,
                              rows, dim, threshold, DYLLM_STREAM(stream));
}

int dyllm_salient_compact(const uint8_t* mask, int64_t rows, const int32_t* cu_seqlens_q, int batch,
                          const int32_t* cu_promptlens, int64_t* idx64, int32_t* idx32, int64_t* idx_k,
                          int32_t* cu_salientlens, int32_t* count, void* stream) {
  DYLLM_REQUIRE(rows == 0 || mask != nullptr, "mask must not be NULL");
  DYLLM_NONNULL(cu_seqlens_q);
  DYLLM_NONNULL(idx64);
  DYLLM_NONNULL(cu_salientlens);
  DYLLM_NONNULL(count);
  return launch_compact(mask, rows, cu_seqlens_q, batch, cu_promptlens, idx64, idx32, idx_k, nullptr, cu_salientlens,
                        count, DYLLM_STREAM(stream));
}

int dyllm_fused_offset_launch(const int32_t* idxs, const int32_t* num_idxs, const int32_t* cu_promptlens,
                              const int32_t* cu_salientlens, int num_groups, int64_t* out, int64_t max_threads,
                              void* stream) {
  DYLLM_NONNULL(idxs);
  DYLLM_NONNULL(num_idxs);
  DYLLM_NONNULL(cu_promptlens);
  DYLLM_NONNULL(cu_salientlens);
  DYLLM_NONNULL(out);
  DYLLM_REQUIRE(max_threads >= 0, "max_threads must be non-negative");
  return launch_fused_offset(idxs, num_idxs, cu_promptlens, cu_salientlens, num_groups, out, max_threads,
                             DYLLM_STREAM(stream));
}

// ---------------------------------------------------------------------------------------
static int row_map(RowMap mode, const void* src, void* dst, int64_t row_bytes, int64_t n_rows,
                   const int64_t* seq_starts, const int32_t* cu, const int32_t* cu_q, const int64_t* seq_ids,
                   const int64_t* row_idx, int batch, void* stream, int64_t src_rows = 0) {
  DYLLM_NONNULL(src);
  DYLLM_NONNULL(dst);
  DYLLM_REQUIRE(batch >= 0, "batch must be non-negative");
  if (n_rows <= 0 || (batch == 0 && mode != RowMap::Gather)) return 0;
  RowMapArgs a{};
  a.src = static_cast<const char*>(src);
  a.dst = static_cast<char*>(dst);
  a.row_bytes = row_bytes;
  a.n_rows = n_rows;
  a.seq_starts = seq_starts;
  a.cu = cu;
  a.cu_q = cu_q;
  a.seq_ids = seq_ids;
  a.row_idx = row_idx;
  a.B = batch;
  a.src_rows = src_rows;
  return launch_row_map(mode, a, DYLLM_STREAM(stream));
}

int dyllm_get_seqs(const void* cache, void* out, int64_t row_bytes, const int64_t* seq_starts,
                   const int32_t* cu_seqlens, const int64_t* seq_ids, int batch, int64_t total_rows, void* stream) {
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(cu_seqlens);
  DYLLM_NONNULL(seq_ids);
  return row_map(RowMap::GetSeqs, cache, out, row_bytes, total_rows, seq_starts, cu_seqlens, nullptr, seq_ids,
                 nullptr, batch, stream);
}
int dyllm_get_block(const void* cache, void* out, int64_t row_bytes, const int64_t* seq_starts,
                    const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q, const int64_t* seq_ids, int batch,
                    int64_t total_rows, void* stream) {
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(cu_seqlens_k);
  DYLLM_NONNULL(cu_seqlens_q);
  DYLLM_NONNULL(seq_ids);
  return row_map(RowMap::GetBlock, cache, out, row_bytes, total_rows, seq_starts, cu_seqlens_k, cu_seqlens_q,
                 seq_ids, nullptr, batch, stream);
}
int dyllm_reset_full(void* cache, const void* in, int64_t row_bytes, const int64_t* seq_starts,
                     const int32_t* cu_seqlens, const int64_t* seq_ids, int batch, int64_t total_rows, void* stream) {
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(cu_seqlens);
  DYLLM_NONNULL(seq_ids);
  return row_map(RowMap::ResetFull, in, cache, row_bytes, total_rows, seq_starts, cu_seqlens, nullptr, seq_ids,
                 nullptr, batch, stream);
}
int dyllm_reset_block(void* cache, const void* in, int64_t row_bytes, const int64_t* seq_starts,
                      const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q, const int64_t* seq_ids, int batch,
                      int64_t total_rows, void* stream) {
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(cu_seqlens_k);
  DYLLM_NONNULL(cu_seqlens_q);
  DYLLM_NONNULL(seq_ids);
  return row_map(RowMap::ResetBlock, in, cache, row_bytes, total_rows, seq_starts, cu_seqlens_k, cu_seqlens_q,
                 seq_ids, nullptr, batch, stream);
}
int dyllm_scatter_update(void* cache, const void* new_vals, int64_t row_bytes, const int64_t* row_idx, int64_t rows,
                         const int32_t* cu_seqlens, const int64_t* seq_starts, const int64_t* seq_ids, int batch,
                         void* stream) {
  DYLLM_NONNULL(row_idx);
  DYLLM_NONNULL(cu_seqlens);
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(seq_ids);
  return row_map(RowMap::Scatter, new_vals, cache, row_bytes, rows, seq_starts, cu_seqlens, nullptr, seq_ids, row_idx,
                 batch, stream);
}
int dyllm_scatter_dest_rows(const int64_t* row_idx, int64_t rows, const int32_t* rows_dev,
                            const int32_t* cu_seqlens, const int64_t* seq_starts, const int64_t* seq_ids, int batch,
                            int64_t* dest, void* stream) {
  DYLLM_NONNULL(row_idx);
  DYLLM_NONNULL(cu_seqlens);
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(seq_ids);
  DYLLM_NONNULL(dest);
  DYLLM_REQUIRE(batch >= 1, "batch must be >= 1");
  return launch_scatter_dest_rows(row_idx, rows, rows_dev, cu_seqlens, seq_starts, seq_ids, batch, dest,
                                  DYLLM_STREAM(stream));
}
int dyllm_gather_rows(const void* x, int64_t x_rows, void* out, int64_t row_bytes, const int64_t* idx, int64_t rows,
                      void* stream) {
  DYLLM_NONNULL(idx);
  DYLLM_REQUIRE(x_rows >= 0, "x_rows must be non-negative");
  return row_map(RowMap::Gather, x, out, row_bytes, rows, nullptr, nullptr, nullptr, nullptr, idx, 0, stream, x_rows);
}

// ---------------------------------------------------------------------------------------
static int64_t hint_or(int64_t hint, int64_t rows) { return (hint > 0 && hint < rows) ? hint : rows; }

size_t dyllm_ffn_down_workspace_bytes(int64_t rows, int64_t rows_hint, int hidden, int intermediate) {
  if (rows <= 0) return 0;
  const int64_t h = hint_or(rows_hint, rows);
  const GemmPlan pl = gemm_plan(h, hidden, intermediate, GemmEpi::Store);
  return align256(gemm_partial_bytes(rows, hidden, pl.tile_m, pl.ksplit));
}

size_t dyllm_swiglu_ffn_workspace_bytes(int64_t rows, int intermediate) {
  return align256(size_t(rows > 0 ? rows : 0) * size_t(intermediate) * 2);
}

int dyllm_ffn_tile_rows(int64_t rows, int n, int k, int swiglu) {
  if (rows <= 0 || n <= 0 || k <= 0) return 0;
  return gemm_plan(rows, n, k, swiglu ? GemmEpi::SwiGLU : GemmEpi::Store).tile_m;
}

int dyllm_ffn_gate_up(const void* x, int64_t ld_x, const int32_t* rows_idx, int64_t rows, const int32_t* rows_dev,
                      int64_t rows_hint, const void* w_gate_up, int hidden, int intermediate, void* h_out,
                      void* stream) {
  DYLLM_NONNULL(x);
  DYLLM_NONNULL(w_gate_up);
  DYLLM_NONNULL(h_out);
  DYLLM_REQUIRE(hidden > 0 && hidden % 64 == 0, "hidden size must be a positive multiple of 64");
  DYLLM_REQUIRE(intermediate > 0 && intermediate % 64 == 0, "intermediate size must be a positive multiple of 64");
  if (rows <= 0) return 0;
  GemmArgs g{};
  g.A = static_cast<const uint16_t*>(x);
  g.lda = ld_x;
  g.a_ids = rows_idx;
  g.a_div = 1;
  g.id_limit = INT64_MAX;
  g.W = static_cast<const uint16_t*>(w_gate_up);
  g.ldw = hidden;
  g.Cout = static_cast<uint16_t*>(h_out);
  g.ldc = intermediate;
  g.M = rows;
  g.num_m_dev = rows_dev;
  g.N = 2 * intermediate;
  g.K = hidden;
  g.half_n = intermediate;
  const int tm = gemm_plan(hint_or(rows_hint, rows), g.N, g.K, GemmEpi::SwiGLU).tile_m;
  return launch_gemm(GemmEpi::SwiGLU, g, rows, tm, 1, DYLLM_STREAM(stream));
}

// Store-epilogue GEMM out[out_rows[m] or m] = a(m) . W^T (+ bias), a(m) = A[rows_idx[m] or m],
// with the tile / split-K plan of the expected row count.
static int store_gemm(const void* a, int64_t lda, const int32_t* rows_idx, int64_t rows, const int32_t* rows_dev,
                      int64_t rows_hint, const void* w, int n, int k, const void* bias, void* out, int64_t ldc,
                      const int64_t* out_rows, void* workspace, size_t workspace_bytes, const char* ws_fn,
                      hipStream_t s) {
  GemmArgs d{};
  d.A = static_cast<const uint16_t*>(a);
  d.lda = lda;
  d.a_rows = rows_idx ? 0 : rows;   // a gathered source's row count is not known here
  d.a_ids = rows_idx;
  d.a_div = 1;
  d.id_limit = INT64_MAX;
  d.W = static_cast<const uint16_t*>(w);
  d.ldw = k;
  d.Cout = static_cast<uint16_t*>(out);
  d.ldc = ldc;
  d.c_rows = out_rows;
  d.bias = static_cast<const uint16_t*>(bias);
  d.M = rows;
  d.num_m_dev = rows_dev;
  d.N = n;
  d.K = k;
  const GemmPlan pl = gemm_plan(hint_or(rows_hint, rows), n, k, GemmEpi::Store);
  if (pl.ksplit > 1) {
    const size_t need = gemm_partial_bytes(rows, n, pl.tile_m, pl.ksplit);
    DYLLM_REQUIRE(workspace && workspace_bytes >= need,
                  "workspace too small: need " + std::to_string(need) + " bytes (" + ws_fn + ")");
    d.partial = static_cast<float*>(workspace);
  }
  return launch_gemm(GemmEpi::Store, d, rows, pl.tile_m, pl.ksplit, s);
}

int dyllm_ffn_down(const void* h, int64_t rows, const int32_t* rows_dev, int64_t rows_hint, const void* w_down,
                   int hidden, int intermediate, void* out, const int64_t* out_rows, void* workspace,
                   size_t workspace_bytes, void* stream) {
  DYLLM_NONNULL(h);
  DYLLM_NONNULL(w_down);
  DYLLM_NONNULL(out);
  DYLLM_REQUIRE(hidden > 0 && hidden % 64 == 0, "hidden size must be a positive multiple of 64");
  DYLLM_REQUIRE(intermediate > 0 && intermediate % 64 == 0, "intermediate size must be a positive multiple of 64");
  if (rows <= 0) return 0;
  return store_gemm(h, intermediate, nullptr, rows, rows_dev, rows_hint, w_down, hidden, intermediate, nullptr, out,
                    hidden, out_rows, workspace, workspace_bytes, "dyllm_ffn_down_workspace_bytes",
                    DYLLM_STREAM(stream));
}

int dyllm_rope(void* x, int64_t ld_x, int64_t rows, int num_heads, int head_dim, const int64_t* positions,
               const float* cos_table, const float* sin_table, int max_position, const void* norm_weight, float eps,
               void* stream) {
  DYLLM_REQUIRE(head_dim == 128, "supported head dimension is 128");
  DYLLM_REQUIRE(num_heads >= 1 && max_position >= 1, "num_heads and max_position must be positive");
  if (rows <= 0) return 0;
  DYLLM_NONNULL(x);
  DYLLM_NONNULL(positions);
  DYLLM_NONNULL(cos_table);
  DYLLM_NONNULL(sin_table);
  DYLLM_REQUIRE(ld_x >= int64_t(num_heads) * head_dim && ld_x % 8 == 0, "row stride must be >= heads * 128, a multiple of 8");
  DYLLM_REQUIRE(aligned_to(16, {x, cos_table, sin_table, norm_weight}),
                "x, the cos / sin tables and norm_weight must be 16-byte aligned");
  KvRopeArgs a{};
  a.kv = static_cast<const uint16_t*>(x);
  a.ld_kv = ld_x;
  a.rows = rows;
  a.kv_size = int64_t(num_heads) * head_dim;
  a.Hkv = num_heads;
  a.positions = positions;
  a.cos = cos_table;
  a.sin = sin_table;
  a.max_position = max_position;
  a.k_norm = static_cast<const uint16_t*>(norm_weight);
  a.eps = eps;
  a.k_cache = static_cast<uint16_t*>(x);
  a.ld_cache = ld_x;
  return launch_kv_rope_scatter(a, DYLLM_STREAM(stream));
}

int dyllm_kv_rope_scatter(const void* kv, int64_t ld_kv, int64_t rows, const int32_t* rows_dev, const int32_t* pos_idx,
                          const int64_t* positions, const float* cos_table, const float* sin_table,
                          int max_position, int num_kv_heads, int head_dim, const void* k_norm_weight, float eps,
                          void* k_cache, const int64_t* k_rows, const int32_t* cu_seqlens_k,
                          const int64_t* seq_starts, const int64_t* seq_ids, int batch, void* v_out, void* stream) {
  DYLLM_REQUIRE(head_dim == 128, "supported head dimension is 128");
  DYLLM_REQUIRE(num_kv_heads >= 1, "num_kv_heads must be positive");
  DYLLM_REQUIRE(max_position >= 1, "max_position must be positive");
  DYLLM_REQUIRE(batch >= 1, "batch must be positive");
  if (rows <= 0) return 0;
  DYLLM_NONNULL(kv);
  DYLLM_NONNULL(positions);
  DYLLM_NONNULL(cos_table);
  DYLLM_NONNULL(sin_table);
  DYLLM_NONNULL(k_cache);
  DYLLM_NONNULL(k_rows);
  DYLLM_NONNULL(cu_seqlens_k);
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(seq_ids);
  DYLLM_NONNULL(v_out);
  const int64_t kv_size = int64_t(num_kv_heads) * head_dim;
  DYLLM_REQUIRE(ld_kv >= 2 * kv_size && ld_kv % 8 == 0, "kv row stride must be >= 2 * kv_size and a multiple of 8");
  DYLLM_REQUIRE(aligned_to(16, {kv, cos_table, sin_table, k_norm_weight, k_cache, v_out}),
                "kv, the cos / sin tables, k_norm_weight, k_cache and v_out must be 16-byte aligned");
  KvRopeArgs a{};
  a.kv = static_cast<const uint16_t*>(kv);
  a.ld_kv = ld_kv;
  a.rows = rows;
  a.rows_dev = rows_dev;
  a.kv_size = kv_size;
  a.Hkv = num_kv_heads;
  a.pos_idx = pos_idx;
  a.positions = positions;
  a.cos = cos_table;
  a.sin = sin_table;
  a.max_position = max_position;
  a.k_norm = static_cast<const uint16_t*>(k_norm_weight);
  a.eps = eps;
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.ld_cache = kv_size;
  a.k_rows = k_rows;
  a.cu_k = cu_seqlens_k;
  a.seq_starts = seq_starts;
  a.seq_ids = seq_ids;
  a.B = batch;
  a.v_out = static_cast<uint16_t*>(v_out);
  return launch_kv_rope_scatter(a, DYLLM_STREAM(stream));
}

int dyllm_rms_norm(const void* x, int64_t ld_x, const void* residual, int64_t ld_residual, const void* weight,
                   int64_t rows, int hidden, float eps, void* out, int64_t ld_out, void* residual_out,
                   int64_t ld_residual_out, void* stream) {
  DYLLM_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= 8192, "hidden size must be a positive multiple of 8, at most 8192");
  if (rows <= 0) return 0;
  DYLLM_NONNULL(x);
  DYLLM_NONNULL(weight);
  DYLLM_NONNULL(out);
  DYLLM_REQUIRE(residual == nullptr || residual_out != nullptr, "residual_out must be given with a residual");
  DYLLM_REQUIRE(aligned_to(16, {x, residual, weight, out, residual_out}), "all row buffers and the weight must be 16-byte aligned");
  DYLLM_REQUIRE(ld_x >= hidden && ld_x % 8 == 0 && ld_out >= hidden && ld_out % 8 == 0,
                "row strides must be >= hidden and multiples of 8");
  DYLLM_REQUIRE(residual == nullptr || (ld_residual >= hidden && ld_residual % 8 == 0 && ld_residual_out >= hidden &&
                                        ld_residual_out % 8 == 0),
                "residual row strides must be >= hidden and multiples of 8");
  NormArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ld_x = ld_x;
  a.residual = static_cast<const uint16_t*>(residual);
  a.ld_r = ld_residual;
  a.weight = static_cast<const uint16_t*>(weight);
  a.rows = rows;
  a.hidden = hidden;
  a.eps = eps;
  a.out = static_cast<uint16_t*>(out);
  a.ld_out = ld_out;
  a.residual_out = static_cast<uint16_t*>(residual_out);
  a.ld_ro = ld_residual_out;
  return launch_add_rms_norm(a, DYLLM_STREAM(stream));
}

int dyllm_rms_norm_cache_rows(const void* cache, int64_t ld_cache, const int64_t* seq_starts, const int64_t* seq_ids,
                              const int32_t* cu_seqlens_k, const int32_t* cu_seqlens_q, int batch,
                              const void* residual, int64_t ld_residual, const void* weight, int64_t rows, int hidden,
                              float eps, void* out, int64_t ld_out, void* residual_out, int64_t ld_residual_out,
                              void* stream) {
  DYLLM_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= 8192, "hidden size must be a positive multiple of 8, at most 8192");
  if (rows <= 0) return 0;
  DYLLM_NONNULL(cache);
  DYLLM_NONNULL(seq_starts);
  DYLLM_NONNULL(seq_ids);
  DYLLM_NONNULL(cu_seqlens_k);
  DYLLM_NONNULL(cu_seqlens_q);
  DYLLM_NONNULL(weight);
  DYLLM_NONNULL(out);
  DYLLM_REQUIRE(batch >= 1, "batch must be >= 1");
  DYLLM_REQUIRE(residual == nullptr || residual_out != nullptr, "residual_out must be given with a residual");
  DYLLM_REQUIRE(aligned_to(16, {cache, residual, weight, out, residual_out}), "all row buffers and the weight must be 16-byte aligned");
  DYLLM_REQUIRE(ld_cache >= hidden && ld_cache % 8 == 0 && ld_out >= hidden && ld_out % 8 == 0,
                "row strides must be >= hidden and multiples of 8");
  DYLLM_REQUIRE(residual == nullptr || (ld_residual >= hidden && ld_residual % 8 == 0 && ld_residual_out >= hidden &&
                                        ld_residual_out % 8 == 0),
                "residual row strides must be >= hidden and multiples of 8");
  NormArgs a{};
  a.x = static_cast<const uint16_t*>(cache);
  a.ld_x = ld_cache;
  a.x_seq_starts = seq_starts;
  a.x_seq_ids = seq_ids;
  a.x_cu_k = cu_seqlens_k;
  a.x_cu_q = cu_seqlens_q;
  a.x_batch = batch;
  a.residual = static_cast<const uint16_t*>(residual);
  a.ld_r = ld_residual;
  a.weight = static_cast<const uint16_t*>(weight);
  a.rows = rows;
  a.hidden = hidden;
  a.eps = eps;
  a.out = static_cast<uint16_t*>(out);
  a.ld_out = ld_out;
  a.residual_out = static_cast<uint16_t*>(residual_out);
  a.ld_ro = ld_residual_out;
  return launch_add_rms_norm(a, DYLLM_STREAM(stream));
}

size_t dyllm_linear_workspace_bytes(int64_t rows, int64_t rows_hint, int out_features, int in_features) {
  return dyllm_ffn_down_workspace_bytes(rows, rows_hint, out_features, in_features);
}

int dyllm_linear(const void* x, int64_t ld_x, const int32_t* rows_idx, int64_t rows, const int32_t* rows_dev,
                 int64_t rows_hint, const void* w, int out_features, int in_features, const void* bias, void* out,
                 void* workspace, size_t workspace_bytes, void* stream) {
  DYLLM_NONNULL(x);
  DYLLM_NONNULL(w);
  DYLLM_NONNULL(out);
  DYLLM_REQUIRE(in_features > 0 && in_features % 64 == 0, "in_features must be a positive multiple of 64");
  DYLLM_REQUIRE(out_features > 0 && out_features % 8 == 0, "out_features must be a positive multiple of 8");
  DYLLM_REQUIRE(ld_x >= in_features && ld_x % 8 == 0, "x row stride must be >= in_features and a multiple of 8");
  DYLLM_REQUIRE(aligned_to(16, {x, w}) && aligned_to(8, {bias, out}), "x and w must be 16-byte aligned, bias and out 8-byte aligned");
  if (rows <= 0) return 0;
  return store_gemm(x, ld_x, rows_idx, rows, rows_dev, rows_hint, w, out_features, in_features, bias, out,
                    out_features, nullptr, workspace, workspace_bytes, "dyllm_linear_workspace_bytes",
                    DYLLM_STREAM(stream));
}

int dyllm_swiglu_ffn(const void* x, int64_t ld_x, const int32_t* rows_idx, int64_t rows, const void* w_gate_up,
                     const void* w_down, int hidden, int intermediate, void* workspace, size_t workspace_bytes,
                     void* out, const int64_t* out_rows, void* stream) {
  if (rows <= 0) return 0;
  const size_t hb = dyllm_swiglu_ffn_workspace_bytes(rows, intermediate);
  const size_t db = dyllm_ffn_down_workspace_bytes(rows, 0, hidden, intermediate);
  DYLLM_REQUIRE(workspace && workspace_bytes >= hb + db,
                "workspace too small: need " + std::to_string(hb + db) + " bytes");
  if (int rc = dyllm_ffn_gate_up(x, ld_x, rows_idx, rows, nullptr, 0, w_gate_up, hidden, intermediate, workspace,
                                 stream))
    return rc;
  return dyllm_ffn_down(workspace, rows, nullptr, 0, w_down, hidden, intermediate, out, out_rows,
                        static_cast<char*>(workspace) + hb, db, stream);
}

int dyllm_silu_and_mul(const void* gate_up, int64_t ld_in, int64_t rows, int intermediate, void* out, int64_t ld_out,
                       void* stream) {
  if (rows <= 0) return 0;
  DYLLM_NONNULL(gate_up);
  DYLLM_NONNULL(out);
  return launch_silu_and_mul(static_cast<const uint16_t*>(gate_up), ld_in, rows, intermediate,
                             static_cast<uint16_t*>(out), ld_out, DYLLM_STREAM(stream));
}

// ---------------------------------------------------------------------------------------
int dyllm_moe_gate(const void* x, const int32_t* rows_idx, int64_t tokens, int hidden, const void* router_w,
                   int num_experts, int top_k, int renormalize, void* topk_weights, int32_t* topk_ids, void* stream) {
  DYLLM_NONNULL(x);
  DYLLM_NONNULL(router_w);
  DYLLM_NONNULL(topk_weights);
  DYLLM_NONNULL(topk_ids);
  return launch_moe_router(static_cast<const uint16_t*>(x), rows_idx, static_cast<const uint16_t*>(router_w), tokens,
                           hidden, num_experts, top_k, renormalize, static_cast<uint16_t*>(topk_weights), topk_ids,
                           DYLLM_STREAM(stream));
}

int dyllm_moe_align_block_size(const int32_t* topk_ids, int64_t slots, int num_experts, int block,
                               int32_t* sorted_token_ids, int64_t capacity, int32_t* tile_expert,
                               int32_t* num_post_pad, void* stream) {
  if (slots > 0) DYLLM_NONNULL(topk_ids);   // no slots: only the sentinels and the count are written
  DYLLM_NONNULL(sorted_token_ids);
  DYLLM_NONNULL(tile_expert);
  DYLLM_NONNULL(num_post_pad);
  return launch_moe_align(topk_ids, slots, num_experts, block, sorted_token_ids, capacity, tile_expert, num_post_pad,
                          DYLLM_STREAM(stream));
}

static int64_t moe_capacity(int64_t slots, int E) {
  const int bm = moe_block(slots, E);
  return cdiv(slots + int64_t(E) * (bm - 1), bm) * bm;
}

size_t dyllm_fused_experts_workspace_bytes(int64_t tokens, int top_k, int num_experts, int hidden, int intermediate) {
  const int64_t S = tokens * top_k;
  const int64_t cap = moe_capacity(S, num_experts);
  return align256(size_t(cap) * 4) + align256(size_t(cap / moe_block(S, num_experts)) * 4) + align256(4) +
         align256(size_t(S) * intermediate * 2) + align256(size_t(S) * hidden * 2);
}

int dyllm_fused_experts(const void* x, const int32_t* rows_idx, int64_t tokens, int hidden, const void* w1,
                        const void* w2, int num_experts, int intermediate, const void* topk_weights,
                        const int32_t* topk_ids, int top_k, void* out, const int64_t* out_rows, void* workspace,
                        size_t workspace_bytes, void* stream) {
  DYLLM_NONNULL(x);
  DYLLM_NONNULL(w1);
  DYLLM_NONNULL(w2);
  DYLLM_NONNULL(topk_weights);
  DYLLM_NONNULL(topk_ids);
  DYLLM_NONNULL(out);
  DYLLM_REQUIRE(hidden % 64 == 0 && intermediate % 64 == 0, "hidden and intermediate must be multiples of 64");
  if (tokens <= 0) return 0;
  const size_t need = dyllm_fused_experts_workspace_bytes(tokens, top_k, num_experts, hidden, intermediate);
  DYLLM_REQUIRE(workspace && workspace_bytes >= need, "workspace too small: need " + std::to_string(need) + " bytes");
  const hipStream_t s = DYLLM_STREAM(stream);
  const int64_t S = tokens * top_k;
  const int64_t cap = moe_capacity(S, num_experts);
  const int bm = moe_block(S, num_experts);
  char* ws = static_cast<char*>(workspace);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws);
  ws += align256(size_t(cap) * 4);
  int32_t* tile_e = reinterpret_cast<int32_t*>(ws);
  ws += align256(size_t(cap / bm) * 4);
  int32_t* npp = reinterpret_cast<int32_t*>(ws);
  ws += align256(4);
  uint16_t* inter = reinterpret_cast<uint16_t*>(ws);
  ws += align256(size_t(S) * intermediate * 2);
  uint16_t* y = reinterpret_cast<uint16_t*>(ws);
  if (int rc = launch_moe_align(topk_ids, S, num_experts, bm, sorted, cap, tile_e, npp, s)) return rc;
  // GEMM 1: inter[slot] = silu(x[slot/top_k] W1g^T) * (x W1u^T)
  GemmArgs g{};
  g.A = static_cast<const uint16_t*>(x);
  g.lda = hidden;
  g.a_rows = rows_idx ? 0 : tokens;   // a gathered source's row count is not known here
  g.a_ids = sorted;
  g.a_div = top_k;
  g.a_map = rows_idx;                 // token t reads x row rows_idx[t]
  g.id_limit = S;
  g.W = static_cast<const uint16_t*>(w1);
  g.ldw = hidden;
  g.w_expert_stride = int64_t(2) * intermediate * hidden;
  g.tile_expert = tile_e;
  g.num_m_dev = npp;
  g.Cout = inter;
  g.ldc = intermediate;
  g.c_by_id = 1;
  g.M = cap;
  g.N = 2 * intermediate;
  g.K = hidden;
  g.half_n = intermediate;
  if (int rc = launch_gemm(GemmEpi::SwiGLU, g, cap, bm, 1, s)) return rc;
  // GEMM 2: y[slot] = (inter[slot] W2^T) * w[slot]
  GemmArgs d{};
  d.A = inter;
  d.lda = intermediate;
  d.a_rows = S;
  d.a_ids = sorted;
  d.a_div = 1;
  d.id_limit = S;
  d.W = static_cast<const uint16_t*>(w2);
  d.ldw = intermediate;
  d.w_expert_stride = int64_t(hidden) * intermediate;
  d.tile_expert = tile_e;
  d.num_m_dev = npp;
  d.Cout = y;
  d.ldc = hidden;
  d.c_by_id = 1;
  d.row_scale_bf16 = static_cast<const uint16_t*>(topk_weights);
  d.M = cap;
  d.N = hidden;
  d.K = intermediate;
  if (int rc = launch_gemm(GemmEpi::Store, d, cap, bm, 1, s)) return rc;
  return launch_moe_combine(y, tokens, hidden, top_k, static_cast<uint16_t*>(out), out_rows, s);
}

}  // extern "C"

// Device-side unmasking bookkeeping between two sparse denoise steps of one running batch
// (the host work of Scheduler.postprocess -> ModelRunner.prepare_sparse / prepare_sample in
// dyllm/engine/scheduler.py:89-145 and dyllm/engine/model_runner.py:186-372), so the next step is
// built from the previous step's sampler output without a round trip through host lists:
//
//   1. commit   -- the sampled tokens go into the batch's token rows (packed by cu_seqlens_k);
//                  a position that held the mask id and now holds another token counts as
//                  generated (Sequence.update_token), the per-sequence count feeds the block index;
//   2. salient  -- the kept positions of the sampled set (p >= answer start, in sampler order) become
//                  the next step's first-layer salient lists: Q-space rows (p - prompt + cu_q[b] in a
//                  Q-pruned step, p + cu_q[b] otherwise), K-space rows p + cu_k[b], the updated-row
//                  list, their positions and cu_salientlens (model_runner.py:203-231);
//   3. inputs   -- the next step's input ids: the answer rows of every sequence (Q-pruned) or
//                  nothing (the caller reads the token rows themselves);
//   4. candidates -- the first W masked positions p in [offset, limit) of every sequence, with
//                  limit = min(L, block_size * (block_idx + 1) + prompt) and block_idx =
//                  generated // block_size (Sequence.update_block_idx), as offsets from the step's
//                  first queried row (prepare_sample: the ragged candidate lists, already dense).
//
// One 256-thread workgroup per sequence; the ordered compactions use wave ballots and a
// four-wave prefix in LDS. Every write stays inside the caller's capacities (checked on the host).
#include "kernels.h"

namespace dyllm {

constexpr int kUnmaskThreads = 256;

// ordered compaction helper: rank of this thread's flag among the flagged threads of the
// workgroup (and the workgroup total), for one 256-element chunk
__device__ __forceinline__ int block_rank(bool flag, int* wsum, int& total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const unsigned long long bal = __ballot(flag);
  const int before = __popcll(bal & ((1ull << lane) - 1));
  __syncthreads();
  if (lane == 0) wsum[w] = __popcll(bal);
  __syncthreads();
  int off = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < kUnmaskThreads / 64; ++i) {
    off += (i < w) ? wsum[i] : 0;
    total += wsum[i];
  }
  return off + before;
}

__global__ __launch_bounds__(kUnmaskThreads) void unmask_step_kernel(UnmaskArgs a) {
  __shared__ int wsum[kUnmaskThreads / 64];
  __shared__ int red;
  const int b = blockIdx.x, tid = threadIdx.x;
  const int64_t k0 = a.cu_k[b];
  const int L = a.cu_k[b + 1] - a.cu_k[b];
  const int A = a.answer_start[b], P = a.prompt_len[b];
  const int n_prev = a.cnt[b];

  // 1. commit
  if (tid == 0) red = 0;
  __syncthreads();
  int gen = 0;
  for (int j = tid; j < n_prev; j += kUnmaskThreads) {
    const int64_t p = a.pos[int64_t(b) * a.ld_sampled + j];
    const int64_t t = a.val[int64_t(b) * a.ld_sampled + j];
    if (p < 0 || p >= L) continue;
    int64_t* slot = a.tok + k0 + p;
    if (*slot == a.mask_id && t != a.mask_id) ++gen;
    *slot = t;
  }
  if (gen) atomicAdd(&red, gen);
  __syncthreads();
  if (tid == 0 && red) a.generated[b] += red;
  __syncthreads();   // the committed rows and the count are read below by the same workgroup

  // 2. salient lists: kept positions of the earlier sequences give this sequence's base
  int base = 0;
  for (int s = 0; s < b; ++s) {
    int c = 0;
    for (int j = tid; j < a.cnt[s]; j += kUnmaskThreads)
      c += a.pos[int64_t(s) * a.ld_sampled + j] >= a.answer_start[s] ? 1 : 0;
    base += c;
  }
  if (tid == 0) red = 0;
  __syncthreads();
  if (base) atomicAdd(&red, base);
  __syncthreads();
  base = red;
  int kept = 0;
  for (int j0 = 0; j0 < n_prev; j0 += kUnmaskThreads) {
    const int j = j0 + tid;
    int64_t p = -1;
    if (j < n_prev) p = a.pos[int64_t(b) * a.ld_sampled + j];
    const bool keep = j < n_prev && p >= A;
    int total;
    const int r = block_rank(keep, wsum, total);
    if (keep) {
      const int64_t o = base + kept + r;
      const int64_t qrow = a.pruned ? p - P + a.cu_q[b] : p + a.cu_q[b];
      a.idx_q[o] = qrow;
      a.idx_q32[o] = int32_t(qrow);
      a.idx_k[o] = p + k0;
      a.idx_k32[o] = int32_t(p + k0);
      a.idx_upd[o] = int32_t(p + k0);
      a.positions_k[o] = p;
    }
    kept += total;
  }
  if (tid == 0) {
    a.cu_s[b + 1] = base + kept;
    if (b == 0) a.cu_s[0] = 0;
  }

  // 3. input ids of the Q-pruned rows (the answer block of every sequence)
  if (a.input_ids) {
    const int64_t q0 = a.cu_q[b];
    for (int i = tid; i < L - A; i += kUnmaskThreads) a.input_ids[q0 + i] = a.tok[k0 + A + i];
  }

  // 4. sampler candidates
  const int bs = a.block_size[b];
  const int g = a.generated[b];
  const int bidx = (g > 0 && bs > 0) ? g / bs : 0;
  int limit = bs * (bidx + 1) + P;
  if (limit > L) limit = L;
  const int off = a.pruned ? A : 0;
  int found = 0;
  for (int p0 = off; p0 < limit && found < a.width; p0 += kUnmaskThreads) {
    const int p = p0 + tid;
    const bool m = p < limit && a.tok[k0 + p] == a.mask_id;
    int total;
    const int r = block_rank(m, wsum, total);
    if (m && found + r < a.width) a.cand_rel[int64_t(b) * a.width + found + r] = p - off;
    found += total;
  }
  if (tid == 0) a.cand_n[b] = found < a.width ? found : a.width;
}

int launch_unmask_step(const UnmaskArgs& a, int batch, hipStream_t s) {
  DYLLM_REQUIRE(batch >= 1, "batch must be >= 1");
  DYLLM_REQUIRE(a.width >= 1 && a.ld_sampled >= 1, "candidate width and sampler row stride must be positive");
  unmask_step_kernel<<<unsigned(batch), kUnmaskThreads, 0, s>>>(a);
  return check_launch("unmask_step_kernel");
}

}  // namespace dyllm

// Mixture-of-experts pieces around the grouped GEMM (gemm.hip):
//
//   router   -- fp32 logits x . Wr^T, softmax, top-k in descending order, optional
//               renormalisation; weights emitted in bf16 and ids int32
//               (moe_gate, dyllm/model_executor/layers/fused_moe.py:375-408).
//   align    -- stable grouping of the flattened (token, k) slots by expert, each expert
//               bucket padded to the GEMM tile height with the sentinel T*top_k, plus the
//               expert of every tile (moe_align_block_size, fused_moe.py:37-85). Runs on the
//               device: no .item() host sync.
//   combine  -- sum over the top-k slots of each token (fused_moe.py:335), written in bf16,
//               optionally straight into the cached FFN rows (MLPcache scatter).
#include "kernels.h"

#include <float.h>

namespace dyllm {

// ---- router: 16 tokens per workgroup on the matrix cores ----------------------------------
// E <= 64 experts, hidden a multiple of 16. logits[16 tokens][64 experts] = X W^T with
// v_mfma_f32_32x32x16_bf16 (rows 16-31 of the 32-row tile zero: 16 tokens per workgroup put
// 231 workgroups on the 256 CUs at config 3, where 32 left half of them idle and ran the softmax
// and top-k of twice as many tokens per CU: 27.6 -> 20.5 us) (exact bf16 products, fp32 sums): wavefront w takes the experts
// [32 (w & 1), +32) over one eighth of the hidden dimension (w >> 1), straight from global
// memory (each lane a 16-byte piece of its token row and of its expert row per 16-wide step, the
// next four steps loaded while the current four are multiplied); the eighths are added through
// LDS in a fixed order. (Config 3, 3686 tokens: 169 us for the former wavefront-per-token kernel,
// 70 / 46 / 35 us with the hidden dimension split in 2 / 4 / 8.) Then one wavefront per token: lane e holds expert e's logit for the softmax
// and the top-k (each lane counts the experts ranked before its own: no dependent shuffle chain). (The logits' fp32 sums run in the matrix cores' order, not element by element:
// rounding-level differences, which move the top-k only at near-ties.)
constexpr int kRouterTok = 16;   // tokens per workgroup (rows 16-31 of the 32-row MFMA tile are zero)
constexpr int kRouterU = 4;
constexpr int kRouterKS = 8;                       // hidden-dimension slices
constexpr int kRouterThreads = 128 * kRouterKS;    // 2 expert halves x kRouterKS slices
union RouterPack {
  bf16x8_t v;
  uint4 q;
};

__global__ __launch_bounds__(kRouterThreads) void moe_router_kernel(const uint16_t* __restrict__ x,
                                                                    const int32_t* __restrict__ rows,
                                                         const uint16_t* __restrict__ wr, int64_t T, int Hd, int E,
                                                         int top_k, int renorm, uint16_t* __restrict__ topk_w,
                                                         int32_t* __restrict__ topk_ids) {
  __shared__ float part[kRouterKS][kRouterTok][65];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ql = lane & 31, half = lane >> 5;
  const int eh = w & 1, kh = w >> 1;
  const int64_t t0 = int64_t(blockIdx.x) * kRouterTok;
  const int64_t ta = t0 + ql;
  const bool a_ok = ql < kRouterTok && ta < T;
  const int64_t xr = a_ok ? (rows ? int64_t(rows[ta]) : ta) : 0;
  const int eb = 32 * eh + ql;
  const bool b_ok = eb < E;
  const int nk = Hd / 16;   // 16-wide steps, split evenly over the slices
  const int k_beg = kh * nk / kRouterKS, k_end = (kh + 1) * nk / kRouterKS;
  const uint16_t* ap = x + xr * Hd + half * 8;
  const uint16_t* bp = wr + int64_t(b_ok ? eb : 0) * Hd + half * 8;
  f32x16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  RouterPack a0[kRouterU], b0[kRouterU], a1[kRouterU], b1[kRouterU];
  auto load = [&](RouterPack (&af)[kRouterU], RouterPack (&bf)[kRouterU], int k) {
#pragma unroll
    for (int u = 0; u < kRouterU; ++u) {
      const bool in = k + u < k_end;
      af[u].q = (in && a_ok) ? *reinterpret_cast<const uint4*>(ap + int64_t(k + u) * 16) : make_uint4(0, 0, 0, 0);
      bf[u].q = (in && b_ok) ? *reinterpret_cast<const uint4*>(bp + int64_t(k + u) * 16) : make_uint4(0, 0, 0, 0);
    }
  };
  auto mma = [&](RouterPack (&af)[kRouterU], RouterPack (&bf)[kRouterU], int k) {
#pragma unroll
    for (int u = 0; u < kRouterU; ++u)
      if (k + u < k_end) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[u].v, bf[u].v, acc, 0, 0, 0);
  };
  // two register sets: the next kRouterU steps load while the current ones are multiplied
  if (k_beg < k_end) load(a0, b0, k_beg);
  for (int k = k_beg; k < k_end; k += 2 * kRouterU) {
    if (k + kRouterU < k_end) load(a1, b1, k + kRouterU);
    mma(a0, b0, k);
    if (k + kRouterU >= k_end) break;
    if (k + 2 * kRouterU < k_end) load(a0, b0, k + 2 * kRouterU);
    mma(a1, b1, k + kRouterU);
  }
  // C layout: lane (ql, half) holds expert column ql, token rows (r / 4) * 8 + half * 4 + r % 4
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int tr = (r >> 2) * 8 + half * 4 + (r & 3);
    if (tr < kRouterTok) part[kh][tr][32 * eh + ql] = acc[r];
  }
  __syncthreads();
  for (int r = w; r < kRouterTok; r += kRouterThreads / 64) {
    const int64_t t = t0 + r;
    if (t >= T) break;
    float logit = -FLT_MAX;
    if (lane < E) {
      logit = part[0][r][lane];
#pragma unroll
      for (int q = 1; q < kRouterKS; ++q) logit += part[q][r][lane];
    }
    const float mx = wave_max(logit);
    const float e = (lane < E) ? expf(logit - mx) : 0.f;
    const float sum = wave_sum(e);
    const float p = (lane < E) ? e / sum : -1.0f;
    // top-k in descending probability, lowest expert index first among exact ties (torch.topk
    // order is unspecified for exact ties): each lane counts the experts ranked before its own
    // from wave-uniform reads of every lane's probability (no dependent shuffle chain); the
    // k best then sum in rank order, as an iterative argmax would add them
    const float pv = p;
    int rank = 0;
    for (int j = 0; j < E; ++j) {
      const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), j));
      rank += (pj > pv || (pj == pv && j < lane)) ? 1 : 0;
    }
    const int my_rank = (lane < E && rank < top_k) ? rank : -1;
    const float my_w = pv;
    float picked_sum = 0.f;
    for (int k = 0; k < top_k; ++k) {
      const unsigned long long who = __ballot(my_rank == k);
      const int src = __builtin_ctzll(who);
      picked_sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), src));
    }
    if (my_rank >= 0) {
      const float wv = renorm ? my_w / picked_sum : my_w;
      topk_w[t * top_k + my_rank] = f32_to_bf16(wv);
      topk_ids[t * top_k + my_rank] = lane;
    }
  }
}

int launch_moe_router(const uint16_t* x, const int32_t* rows, const uint16_t* wr, int64_t T, int Hd, int E, int top_k,
                      int renorm, uint16_t* topk_w, int32_t* topk_ids, hipStream_t s) {
  DYLLM_REQUIRE(E >= 1 && E <= 64, "router supports 1..64 experts");
  DYLLM_REQUIRE(top_k >= 1 && top_k <= E, "top_k must be in [1, num_experts]");
  DYLLM_REQUIRE(Hd % 16 == 0, "hidden size must be a multiple of 16");
  if (T <= 0) return 0;
  moe_router_kernel<<<unsigned(cdiv(T, kRouterTok)), kRouterThreads, 0, s>>>(x, rows, wr, T, Hd, E, top_k, renorm,
                                                                             topk_w, topk_ids);
  return check_launch("moe_router_kernel");
}

// ---- align: G workgroups of 1024 threads, no communication between them ----------------
// Workgroup g owns the contiguous slot chunk [g0, g1). Every workgroup first builds, with LDS
// atomics over a coalesced read of all slot ids (L2-resident, a few hundred KB at most), the
// per-expert totals and the per-expert counts of the slots before its chunk; all workgroups
// derive the same padded bucket starts from the same integers, so the chunks' bases follow
// without any inter-workgroup exchange. Inside a chunk: 16 contiguous per-wavefront ranges;
// pass 1 counts per (wavefront, expert) with six ballots that group the lanes sharing an expert
// (the group's first lane adds the group size: distinct experts per leader, no conflicts);
// pass 2 writes each slot at its base + its rank among the lanes of its group. Slots keep
// ascending order inside a bucket (chunks, ranges, rounds and lanes in order). The bucket
// padding and tile experts of expert e are written by workgroup e % G, the tail past the last
// bucket striped over all workgroups.
constexpr int kAlignThreads = 1024;
constexpr int kAlignMaxGroups = 64;
constexpr int kAlignMinChunk = 512;

__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(const int32_t* __restrict__ ids, int64_t S, int E,
                                                                  int bm, int32_t* __restrict__ sorted_ids,
                                                                  int64_t cap, int32_t* __restrict__ tile_expert,
                                                                  int32_t* __restrict__ num_post_pad) {
  constexpr int NWV = kAlignThreads / 64;
  __shared__ int wcnt[NWV][64];
  __shared__ int wbase[NWV][64];
  __shared__ int start[65];
  __shared__ int tot[64];
  __shared__ int pre[64];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int G = gridDim.x, g = blockIdx.x;
  for (int x = tid; x < NWV * 64; x += kAlignThreads) (&wcnt[0][0])[x] = 0;
  if (tid < 64) {
    tot[tid] = 0;
    pre[tid] = 0;
  }
  __syncthreads();
  // expert ids are clamped to [0, E): an out-of-range id from a caller can never index past the
  // 64-entry LDS tables (its slot is then routed to the nearest valid expert)
  auto expert_of = [&](int64_t i) { return min(max(int(ids[i]), 0), E - 1); };
  const int64_t per_g = (S + G - 1) / G;
  const int64_t g0 = min(S, int64_t(g) * per_g), g1 = min(S, g0 + per_g);
  // totals and the counts before this chunk; the ids of kBatch rounds are loaded together
  constexpr int kBatch = 8;
  // (each workgroup starts its scan at its own chunk: concurrent workgroups read different lines
  // instead of all requesting the same ones from one L2 channel)
  for (int64_t r0 = 0; r0 < S; r0 += int64_t(kAlignThreads) * kBatch) {
    int ev[kBatch];
    bool before[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t i = r0 + int64_t(kAlignThreads) * u + tid;
      int64_t j = i + g0;
      if (j >= S) j -= S;
      ev[u] = i < S ? expert_of(j) : -1;
      before[u] = j < g0;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (ev[u] < 0) continue;
      atomicAdd(&tot[ev[u]], 1);
      if (before[u]) atomicAdd(&pre[ev[u]], 1);
    }
  }
  const int64_t per = (g1 - g0 + NWV - 1) / NWV;
  const int64_t c0 = min(g1, g0 + int64_t(wid) * per), c1 = min(g1, c0 + per);
  // lanes of this round that share the expert e (ok lanes only)
  auto group = [&](bool ok, int e) -> unsigned long long {
    unsigned long long same = __ballot(ok);
#pragma unroll
    for (int bit = 0; bit < 6; ++bit) {
      const unsigned long long bb = __ballot(ok && ((e >> bit) & 1));
      same &= ((e >> bit) & 1) ? bb : ~bb;
    }
    return same;
  };
  const unsigned long long lt = (1ull << lane) - 1;
  for (int64_t r0 = c0; r0 < c1; r0 += 64 * kBatch) {
    int ev[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t i = r0 + 64 * u + lane;
      ev[u] = i < c1 ? expert_of(i) : -1;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const bool ok = ev[u] >= 0;
      const int e = ok ? ev[u] : 0;
      const unsigned long long same = group(ok, e);
      if (ok && (same & lt) == 0) wcnt[wid][e] += __popcll(same);
    }
  }
  __syncthreads();
  if (tid < 64) {   // padded bucket starts: an exclusive scan over the experts in wavefront 0
    const int pad = tid < E ? (tot[tid] + bm - 1) / bm * bm : 0;
    int inc = pad;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(inc, o, 64);
      if (tid >= o) inc += v;
    }
    if (tid < E) start[tid] = inc - pad;
    if (tid == 63) {
      start[E] = inc;
      if (g == 0) num_post_pad[0] = inc;
    }
  }
  __syncthreads();
  if (tid < E) {
    int bse = start[tid] + pre[tid];
    for (int w = 0; w < NWV; ++w) {
      wbase[w][tid] = bse;
      bse += wcnt[w][tid];
    }
  }
  const int total = start[E];
  // sentinels in the padding of this workgroup's experts' buckets (disjoint from every slot
  // written below) and their tiles' expert; the tail past the last bucket
  for (int e = g; e < E; e += G) {
    const int p0 = start[e] + tot[e], p1 = start[e + 1];
    for (int x = p0 + tid; x < p1; x += kAlignThreads) sorted_ids[x] = int32_t(S);
    const int nt = (p1 - start[e]) / bm;
    for (int t = tid; t < nt; t += kAlignThreads) tile_expert[start[e] / bm + t] = e;
  }
  const int64_t stride = int64_t(G) * kAlignThreads;
  for (int64_t x = total + int64_t(g) * kAlignThreads + tid; x < cap; x += stride) sorted_ids[x] = int32_t(S);
  for (int64_t t = total / bm + int64_t(g) * kAlignThreads + tid; t < cap / bm; t += stride) tile_expert[t] = 0;
  __syncthreads();
  for (int64_t r0 = c0; r0 < c1; r0 += 64 * kBatch) {
    int ev[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t i = r0 + 64 * u + lane;
      ev[u] = i < c1 ? expert_of(i) : -1;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const bool ok = ev[u] >= 0;
      const int e = ok ? ev[u] : 0;
      const unsigned long long same = group(ok, e);
      if (ok) sorted_ids[wbase[wid][e] + __popcll(same & lt)] = int32_t(r0 + 64 * u + lane);
      if (ok && (same & lt) == 0) wbase[wid][e] += __popcll(same);
    }
  }
}

int launch_moe_align(const int32_t* ids, int64_t S, int E, int bm, int32_t* sorted_ids, int64_t cap,
                     int32_t* tile_expert, int32_t* num_post_pad, hipStream_t s) {
  DYLLM_REQUIRE(E >= 1 && E <= 64, "align supports 1..64 experts");
  DYLLM_REQUIRE(S >= 0 && S < (int64_t(1) << 31), "slot count out of range");
  DYLLM_REQUIRE(bm > 0 && cap % bm == 0 && cap >= S + int64_t(E) * (bm - 1), "sorted-id capacity too small");
  DYLLM_REQUIRE(cap < (int64_t(1) << 31), "sorted-id capacity out of range");
  const int G = int(std::min<int64_t>(kAlignMaxGroups, std::max<int64_t>(1, cdiv(S, kAlignMinChunk))));
  moe_align_kernel<<<G, kAlignThreads, 0, s>>>(ids, S, E, bm, sorted_ids, cap, tile_expert, num_post_pad);
  return check_launch("moe_align_kernel");
}

// ---- combine: out[dst(t)] = bf16( sum_k y[t*top_k + k] ) ---------------------------------
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ y, int64_t T, int Hd, int top_k,
                                                          uint16_t* __restrict__ out, const int64_t* __restrict__ dst_rows) {
  const int64_t t = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= T) return;
  const int64_t d = dst_rows ? dst_rows[t] : t;
  // the slots' pieces are loaded kBatch at a time before they are summed (in slot order): one
  // memory round trip per batch instead of one per slot
  constexpr int kBatch = 8;
  for (int c = lane; c < Hd / 8; c += 64) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k0 = 0; k0 < top_k; k0 += kBatch) {
      uint4 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        v[u] = (k0 + u < top_k) ? reinterpret_cast<const uint4*>(y + (t * top_k + k0 + u) * Hd)[c] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (k0 + u >= top_k) break;
        const uint32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[2 * j] += __uint_as_float(vv[j] << 16);
          acc[2 * j + 1] += __uint_as_float(vv[j] & 0xffff0000u);
        }
      }
    }
    uint4 o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    o.z = pack_bf16x2(acc[4], acc[5]);
    o.w = pack_bf16x2(acc[6], acc[7]);
    reinterpret_cast<uint4*>(out + d * Hd)[c] = o;
  }
}

int launch_moe_combine(const uint16_t* y, int64_t T, int Hd, int top_k, uint16_t* out, const int64_t* dst_rows,
                       hipStream_t s) {
  DYLLM_REQUIRE(Hd % 8 == 0, "hidden size must be a multiple of 8");
  if (T <= 0) return 0;
  moe_combine_kernel<<<unsigned(cdiv(T, 4)), 256, 0, s>>>(y, T, Hd, top_k, out, dst_rows);
  return check_launch("moe_combine_kernel");
}

}  // namespace dyllm

// Saliency: per-row cosine statistics, the tau test and stream compaction of the
// salient mask into index lists.
//
// Reference semantics:
//   * tau test  -- dyllm/distributed/parallel_state.py:62-66 (the decisive writer,
//                  attention.py:145) and its CUDA twin attention_aux_kernels.cu:10-20:
//                  cos = dot * rsqrt(max(n1,1e-8)) * rsqrt(max(n2,1e-8)); salient = cos < tau.
//   * stats     -- {sum new*old, sum new^2, sum old^2} in fp32 (sm80.cu:436-443, aux:37-42).
//   * compaction-- torch.nonzero (ascending) + searchsorted(idxs, cu_seqlens_q) +
//                  fused_offset (attention.py:147-166, attention_aux_kernels.cu:112-128).
//
// MI355X design: the stats of the column-sparse attention epilogue are written per (head, row)
// without atomics and reduced here in a fixed order, so the salient set is run-to-run
// deterministic. The sparse step reduces, tests and compacts in one multi-workgroup launch
// (reduce_compact_kernel, a look-back over per-workgroup counts); the standalone compaction is one
// workgroup of 16 wavefronts that scans the byte mask with ballot / popcount prefix sums. Neither
// returns to the host.
#include "kernels.h"

namespace dyllm {

// rsqrt as used by the tau test, computed as 1/sqrt with IEEE sqrt and division so the
// decision is reproducible on the host to the last ulp.
__device__ __forceinline__ float tau_cos(float dot, float n1, float n2) {
  const float r1 = 1.0f / __fsqrt_rn(fmaxf(n1, 1e-8f));
  const float r2 = 1.0f / __fsqrt_rn(fmaxf(n2, 1e-8f));
  return __fmul_rn(__fmul_rn(dot, r1), r2);
}

// ---- tau test from stats [T,3] -------------------------------------------------------
__global__ __launch_bounds__(256) void cosine_mask_kernel(const float* __restrict__ stats, uint8_t* __restrict__ mask,
                                                          int64_t T, float tau) {
  const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= T) return;
  mask[t] = tau_cos(stats[3 * t], stats[3 * t + 1], stats[3 * t + 2]) < tau;
}

int launch_cosine_mask(const float* stats, uint8_t* mask, int64_t T, float tau, hipStream_t s) {
  if (T <= 0) return 0;
  cosine_mask_kernel<<<unsigned(cdiv(T, 256)), 256, 0, s>>>(stats, mask, T, tau);
  return check_launch("cosine_mask_kernel");
}

// ---- standalone saliency pass: bf16 rows new/old -> stats + mask ----------------------
// One wavefront per row, 16-byte loads (8 bf16 per lane per pass), fp32 accumulation and
// a butterfly reduction across the 64 lanes.
__global__ __launch_bounds__(256) void saliency_rows_kernel(const uint16_t* __restrict__ c_new,
                                                            const uint16_t* __restrict__ c_old, float* __restrict__ stats,
                                                            uint8_t* __restrict__ mask, int64_t T, int64_t D, float tau) {
  const int64_t t = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= T) return;
  const uint4* pn = reinterpret_cast<const uint4*>(c_new + t * D);
  const uint4* po = reinterpret_cast<const uint4*>(c_old + t * D);
  float dot = 0.f, nn = 0.f, oo = 0.f;
  const int64_t n16 = D >> 3;
  int64_t i0 = lane;
  // 4 passes' loads in flight per lane before the (unchanged, ascending) accumulation
  for (; i0 + 3 * 64 < n16; i0 += 4 * 64) {
    uint4 an[4], bo[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      an[u] = pn[i0 + u * 64];
      bo[u] = po[i0 + u * 64];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t av[4] = {an[u].x, an[u].y, an[u].z, an[u].w}, bv[4] = {bo[u].x, bo[u].y, bo[u].z, bo[u].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float n0 = __uint_as_float(av[j] << 16), n1 = __uint_as_float(av[j] & 0xffff0000u);
        const float o0 = __uint_as_float(bv[j] << 16), o1 = __uint_as_float(bv[j] & 0xffff0000u);
        dot += n0 * o0 + n1 * o1;
        nn += n0 * n0 + n1 * n1;
        oo += o0 * o0 + o1 * o1;
      }
    }
  }
  for (int64_t i = i0; i < n16; i += 64) {
    const uint4 a = pn[i], b = po[i];
    const uint32_t av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float n0 = __uint_as_float(av[j] << 16), n1 = __uint_as_float(av[j] & 0xffff0000u);
      const float o0 = __uint_as_float(bv[j] << 16), o1 = __uint_as_float(bv[j] & 0xffff0000u);
      dot += n0 * o0 + n1 * o1;
      nn += n0 * n0 + n1 * n1;
      oo += o0 * o0 + o1 * o1;
    }
  }
  dot = wave_sum(dot);
  nn = wave_sum(nn);
  oo = wave_sum(oo);
  if (lane == 0) {
    stats[3 * t] = dot;
    stats[3 * t + 1] = nn;
    stats[3 * t + 2] = oo;
    mask[t] = tau_cos(dot, nn, oo) < tau;
  }
}

int launch_saliency_rows(const uint16_t* c_new, const uint16_t* c_old, float* stats, uint8_t* mask, int64_t T,
                         int64_t D, float tau, hipStream_t s) {
  DYLLM_REQUIRE(D > 0 && D % 8 == 0, "row width must be a positive multiple of 8");
  if (T <= 0) return 0;
  saliency_rows_kernel<<<unsigned(cdiv(T, 4)), 256, 0, s>>>(c_new, c_old, stats, mask, T, D, tau);
  return check_launch("saliency_rows_kernel");
}

// ---- reduce per-head partial stats [H][3][T] -> stats [T,3] + mask ---------------------
// Heads are summed in ascending order (deterministic); coalesced along T.
__global__ __launch_bounds__(256) void saliency_reduce_kernel(const float* __restrict__ part, float* __restrict__ stats,
                                                              uint8_t* __restrict__ mask, int64_t T, int H, float tau) {
  const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= T) return;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll 8
  for (int h = 0; h < H; ++h) {
    s0 += part[(int64_t(h) * 3 + 0) * T + t];
    s1 += part[(int64_t(h) * 3 + 1) * T + t];
    s2 += part[(int64_t(h) * 3 + 2) * T + t];
  }
  stats[3 * t] = s0;
  stats[3 * t + 1] = s1;
  stats[3 * t + 2] = s2;
  mask[t] = tau_cos(s0, s1, s2) < tau;
}

int launch_saliency_reduce(const float* part, float* stats, uint8_t* mask, int64_t T, int H, float tau,
                           hipStream_t s) {
  if (T <= 0) return 0;
  saliency_reduce_kernel<<<unsigned(cdiv(T, 256)), 256, 0, s>>>(part, stats, mask, T, H, tau);
  return check_launch("saliency_reduce_kernel");
}

// ---- stream compaction ----------------------------------------------------------------
// One workgroup of 1024 threads (16 wavefronts). Each pass covers 1024*16 mask bytes:
// thread t owns 16 consecutive bytes (one 16-byte load), counts its set bytes, and the
// workgroup forms an exclusive prefix with a wave-level shuffle scan plus a 16-entry LDS
// scan. Indices are emitted in ascending order, as torch.nonzero does.
constexpr int kCompactThreads = 1024;
constexpr int kCompactItems = 16;

__device__ __forceinline__ void compact_block(
    const uint8_t* __restrict__ mask, int64_t T, const int32_t* __restrict__ cu_q, int B,
    const int32_t* __restrict__ cu_prompt, int64_t* __restrict__ idx64, int32_t* __restrict__ idx32,
    int64_t* __restrict__ idx_k, int32_t* __restrict__ idx_k32, int32_t* __restrict__ cu_sal,
    int32_t* __restrict__ count) {
  __shared__ int wave_tot[16];
  __shared__ int base_sh;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) base_sh = 0;
  __syncthreads();
  constexpr int64_t kPass = int64_t(kCompactThreads) * kCompactItems;
  for (int64_t p0 = 0; p0 < T; p0 += kPass) {
    const int64_t r0 = p0 + int64_t(tid) * kCompactItems;
    uint8_t v[kCompactItems];
    if (r0 + kCompactItems <= T && (reinterpret_cast<uintptr_t>(mask + r0) & 15) == 0) {
      const uint4 q = *reinterpret_cast<const uint4*>(mask + r0);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = (w[j >> 2] >> (8 * (j & 3))) & 0xff;
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = (r0 + j < T) ? mask[r0 + j] : 0;
    }
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) cnt += v[j] != 0;
    // inclusive scan within the wave
    int inc = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(inc, o, 64);
      if (lane >= o) inc += y;
    }
    if (lane == 63) wave_tot[wid] = inc;
    __syncthreads();
    int wbase = 0, pass_total = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const int x = wave_tot[w];
      wbase += (w < wid) ? x : 0;
      pass_total += x;
    }
    int pos = base_sh + wbase + inc - cnt;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (v[j]) {
        idx64[pos] = r0 + j;
        if (idx32) idx32[pos] = int32_t(r0 + j);
        ++pos;
      }
    }
    __syncthreads();
    if (tid == 0) base_sh += pass_total;
    __syncthreads();
  }
  const int n = base_sh;
  __threadfence_block();
  __syncthreads();
  // cu_salientlens[b] = #salient rows < cu_q[b]  (searchsorted, side=left)
  __shared__ int32_t cu_sh[1025];
  for (int b = tid; b <= B; b += kCompactThreads) {
    const int64_t key = cu_q[b];
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (idx64[mid] < key)
        lo = mid + 1;
      else
        hi = mid;
    }
    cu_sal[b] = lo;
    if (b <= 1024) cu_sh[b] = lo;
  }
  if (tid == 0) count[0] = n;
  if (idx_k == nullptr) return;
  __syncthreads();
  // K-space rows: idx + cu_promptlens[seg+1] (attention_aux_kernels.cu:118-127)
  for (int t = tid; t < n; t += kCompactThreads) {
    int lo = 0, hi = B;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      const int32_t c = (B <= 1024) ? cu_sh[mid + 1] : cu_sal[mid + 1];
      if (c <= t)
        lo = mid + 1;
      else
        hi = mid;
    }
    const int64_t kk = idx64[t] + cu_prompt[lo + 1];
    idx_k[t] = kk;
    if (idx_k32) idx_k32[t] = int32_t(kk);
  }
}

// [count, cu_salientlens...] straight into pinned host memory (when given): the host reads the
// salient count once the kernel has completed, with no device->host copy behind it
__device__ __forceinline__ void write_host_meta(int32_t* host_meta, const int32_t* cu_sal, const int32_t* count,
                                                int B) {
  if (!host_meta) return;
  __syncthreads();
  for (int b = threadIdx.x; b <= B; b += kCompactThreads) host_meta[1 + b] = cu_sal[b];
  if (threadIdx.x == 0) host_meta[0] = count[0];
  __threadfence_system();
}

__global__ __launch_bounds__(kCompactThreads) void compact_kernel(
    const uint8_t* __restrict__ mask, int64_t T, const int32_t* __restrict__ cu_q, int B,
    const int32_t* __restrict__ cu_prompt, int64_t* __restrict__ idx64, int32_t* __restrict__ idx32,
    int64_t* __restrict__ idx_k, int32_t* __restrict__ idx_k32, int32_t* __restrict__ cu_sal,
    int32_t* __restrict__ count, int32_t* __restrict__ host_meta) {
  compact_block(mask, T, cu_q, B, cu_prompt, idx64, idx32, idx_k, idx_k32, cu_sal, count);
  write_host_meta(host_meta, cu_sal, count, B);
}

// ---- statistics reduction + tau test + compaction in one launch (native step) ---------------
// Workgroup w reduces the per-head partial statistics of rows [256w, 256w+256): its four
// 256-thread quarters sum contiguous quarters of the heads (ascending) and the quarter sums are
// added in quarter order (a fixed order: deterministic, where the reference's atomicAdd across head
// blocks is not); it writes the statistics and the tau decision, publishes its salient count (count + 1 in flags[w]; 0 = not yet) with a device-scope atomic
// store, then looks back: wavefront 0 reads flags[0..w) (one lane per workgroup, device-scope
// atomic loads, each lane polling until its flag is set) and sums them into the workgroup's base;
// then it places its own rows in ascending order (cu_salientlens[b] by the workgroup that owns row
// cu_q[b], the count by the last workgroup; the same values go to pinned host memory when given).
// Only counts cross workgroups, inside
// the atomics themselves, so no fence orders any other data. Workgroups are dispatched in index
// order, so every flag a workgroup waits for belongs to a workgroup that is running or done; the
// poll is still bounded (kLookbackPolls per flag): a workgroup that exhausts it writes nothing, and
// the last one then reports kCompactLookbackFailed as the count.
constexpr int kReduceRows = kCompactThreads / 4;
constexpr int kLookbackPolls = 1 << 20;

__global__ __launch_bounds__(kCompactThreads) void reduce_compact_kernel(
    const float* __restrict__ part, float* __restrict__ stats, uint8_t* __restrict__ mask, int64_t T, int H,
    float tau, int32_t* __restrict__ flags, const int32_t* __restrict__ cu_q, int B,
    const int32_t* __restrict__ cu_prompt, int64_t* __restrict__ idx64, int32_t* __restrict__ idx32,
    int64_t* __restrict__ idx_k, int32_t* __restrict__ idx_k32, int32_t* __restrict__ cu_sal,
    int32_t* __restrict__ count, int32_t* __restrict__ host_meta, CompactDest dd) {
  constexpr int NWV = kReduceRows / 64;
  __shared__ float red[4][3][kReduceRows];
  __shared__ int wtot[NWV];
  __shared__ int pre[kReduceRows + 1];
  __shared__ int base_sh, fail_sh;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int tl = tid % kReduceRows, hq = tid / kReduceRows;
  const int nblk = gridDim.x, blk = blockIdx.x;
  const int64_t t = int64_t(blk) * kReduceRows + tl;
  // 1. statistics of the block's rows: four quarters of the heads, summed in quarter order
  const int hpq = (H + 3) / 4;
  const int h0 = hq * hpq, h1 = (h0 + hpq < H) ? h0 + hpq : H;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f;
  if (t < T) {
#pragma unroll 4
    for (int h = h0; h < h1; ++h) {
      s0 += part[(int64_t(h) * 3 + 0) * T + t];
      s1 += part[(int64_t(h) * 3 + 1) * T + t];
      s2 += part[(int64_t(h) * 3 + 2) * T + t];
    }
  }
  red[hq][0][tl] = s0;
  red[hq][1][tl] = s1;
  red[hq][2][tl] = s2;
  __syncthreads();
  bool sal = false;
  if (hq == 0 && t < T) {
    s0 = ((red[0][0][tl] + red[1][0][tl]) + red[2][0][tl]) + red[3][0][tl];
    s1 = ((red[0][1][tl] + red[1][1][tl]) + red[2][1][tl]) + red[3][1][tl];
    s2 = ((red[0][2][tl] + red[1][2][tl]) + red[2][2][tl]) + red[3][2][tl];
    stats[3 * t] = s0;
    stats[3 * t + 1] = s1;
    stats[3 * t + 2] = s2;
    sal = tau_cos(s0, s1, s2) < tau;
    mask[t] = sal;
  }
  const unsigned long long bal = __ballot(sal);
  const int before = __popcll(bal & ((1ull << lane) - 1));
  if (hq == 0 && lane == 0) wtot[wid] = __popcll(bal);
  __syncthreads();
  int woff = 0, total = 0;
#pragma unroll
  for (int w = 0; w < NWV; ++w) {
    woff += (w < wid) ? wtot[w] : 0;
    total += wtot[w];
  }
  // 2. publish, 3. look back
  if (tid == 0) __hip_atomic_store(&flags[blk], total + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (wid == 0) {
    int base = 0;
    bool ok = true;
    for (int i0 = 0; i0 < blk; i0 += 64) {
      const int i = i0 + lane;
      int v = 1;   // lanes past the last earlier workgroup add 0
      if (i < blk) {
        v = __hip_atomic_load(&flags[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int p = 0; v == 0 && p < kLookbackPolls; ++p) {
          __builtin_amdgcn_s_sleep(2);
          v = __hip_atomic_load(&flags[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      ok = ok && __ballot(v == 0) == 0;
      int c = v > 0 ? v - 1 : 0;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
      base += c;
    }
    if (lane == 0) {
      base_sh = base;
      fail_sh = ok ? 0 : 1;
    }
  }
  if (hq == 0) pre[tl] = woff + before;
  if (tid == 0) pre[kReduceRows] = total;
  __syncthreads();
  const int base = base_sh;
  if (fail_sh) {
    if (blk == nblk - 1 && tid == 0) {
      count[0] = kCompactLookbackFailed;
      if (host_meta) {
        host_meta[0] = kCompactLookbackFailed;
        __threadfence_system();
      }
    }
    return;
  }
  // 4. placement of the block's salient rows
  if (sal) {
    const int pos = base + woff + before;
    idx64[pos] = t;
    if (idx32) idx32[pos] = int32_t(t);
    if (idx_k || dd.dest) {
      const int seg = find_segment(cu_q, B + 1, t);
      const int64_t kk = idx_k ? t + cu_prompt[seg + 1] : t;   // K-space row (refresh: Q space == K space)
      if (idx_k) {
        idx_k[pos] = kk;
        if (idx_k32) idx_k32[pos] = int32_t(kk);
      }
      if (dd.dest) dd.dest[pos] = dd.dest_starts[dd.seq_ids[seg]] + (kk - dd.cu_k[seg]);
    }
  }
  bool wrote = false;
  const int64_t lo = int64_t(blk) * kReduceRows;
  for (int b = tid; b <= B; b += kCompactThreads) {
    const int64_t p = cu_q[b];
    const int owner = (p >= T) ? nblk - 1 : int(p / kReduceRows);
    if (owner != blk) continue;
    const int64_t local = p - lo;
    const int v = base + (local >= kReduceRows ? total : pre[local]);
    cu_sal[b] = v;
    if (host_meta) host_meta[1 + b] = v;
    wrote = true;
  }
  if (blk == nblk - 1 && tid == 0) {
    count[0] = base + total;
    if (host_meta) host_meta[0] = base + total;
    wrote = true;
  }
  if (host_meta && wrote) __threadfence_system();
}

int launch_reduce_compact(const float* part, float* stats, uint8_t* mask, int64_t T, int H, float tau,
                          int32_t* flags, const int32_t* cu_q, int B, const int32_t* cu_prompt, int64_t* idx64,
                          int32_t* idx32, int64_t* idx_k, int32_t* idx_k32, int32_t* cu_sal, int32_t* count,
                          int32_t* host_meta, hipStream_t s, const CompactDest& dest) {
  DYLLM_REQUIRE(B >= 1, "batch must hold at least one sequence");
  DYLLM_REQUIRE(T >= 1 && T < (int64_t(1) << 31), "row count out of range");
  DYLLM_REQUIRE(idx_k == nullptr || cu_prompt != nullptr, "cu_promptlens is required for K-space indices");
  DYLLM_REQUIRE(dest.dest == nullptr || (dest.dest_starts && dest.seq_ids && dest.cu_k),
                "cache rows need the cache's sequence starts, the sequence ids and cu_seqlens_k");
  reduce_compact_kernel<<<unsigned(cdiv(T, kReduceRows)), kCompactThreads, 0, s>>>(
      part, stats, mask, T, H, tau, flags, cu_q, B, cu_prompt, idx64, idx32, idx_k, idx_k32, cu_sal, count, host_meta,
      dest);
  return check_launch("reduce_compact_kernel");
}

int64_t reduce_compact_blocks(int64_t T) { return cdiv(T, kReduceRows); }

int launch_compact(const uint8_t* mask, int64_t T, const int32_t* cu_q, int B, const int32_t* cu_prompt,
                   int64_t* idx64, int32_t* idx32, int64_t* idx_k, int32_t* idx_k32, int32_t* cu_sal, int32_t* count,
                   hipStream_t s, int32_t* host_meta) {
  DYLLM_REQUIRE(B >= 1, "batch must hold at least one sequence");
  DYLLM_REQUIRE(T >= 0 && T < (int64_t(1) << 31), "row count out of range");
  DYLLM_REQUIRE(idx_k == nullptr || cu_prompt != nullptr, "cu_promptlens is required for K-space indices");
  compact_kernel<<<1, kCompactThreads, 0, s>>>(mask, T, cu_q, B, cu_prompt, idx64, idx32, idx_k, idx_k32, cu_sal,
                                                count, host_meta);
  return check_launch("compact_kernel");
}

// ---- fused_offset_launch (standalone, attention_aux_kernels.cu:112-128) ---------------
__global__ __launch_bounds__(256) void fused_offset_kernel(const int32_t* __restrict__ idxs,
                                                           const int32_t* __restrict__ num_idxs,
                                                           const int32_t* __restrict__ cu_prompt,
                                                           const int32_t* __restrict__ cu_sal, int groups,
                                                           int64_t* __restrict__ out, int64_t cap) {
  const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= cap || t >= num_idxs[0]) return;
  int lo = 0, hi = groups;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (cu_sal[mid + 1] <= t)
      lo = mid + 1;
    else
      hi = mid;
  }
  out[t] = int64_t(idxs[t]) + cu_prompt[lo + 1];
}

int launch_fused_offset(const int32_t* idxs, const int32_t* num_idxs, const int32_t* cu_prompt,
                        const int32_t* cu_sal, int groups, int64_t* out, int64_t cap, hipStream_t s) {
  DYLLM_REQUIRE(groups >= 1, "need at least one sequence");
  if (cap <= 0) return 0;
  fused_offset_kernel<<<unsigned(cdiv(cap, 256)), 256, 0, s>>>(idxs, num_idxs, cu_prompt, cu_sal, groups, out, cap);
  return check_launch("fused_offset_kernel");
}

}  // namespace dyllm

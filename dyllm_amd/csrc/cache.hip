// Packed row-cache copies: the per-sequence caches of context, K, V and FFN output rows
// (`[sum(L), D]`, one contiguous region per sequence starting at seq_starts[seq_id]).
//
// Semantics follow dyllm/csrc/cache/cache_kernels.cu (get_seqs :18-64, reset_full
// :110-156, get_block :200-247, reset_block :296-343, scatter_update :388-426) and the
// row gather of dyllm/utils/util.py:19-36. The design is MI355X-first: one wavefront
// copies one row with 16-byte lanes (a 4096-wide bf16 row = 512 x 16 B = 8 passes of the
// wave), the grid is sized to the exact number of rows (the sequence of a row is found
// by a binary search over the cu_seqlens prefix, not by launching one grid slice per
// sequence), so every launched wave moves bytes.
#include "kernels.h"

namespace dyllm {

template <RowMap M>
__device__ __forceinline__ bool map_row(const RowMapArgs& a, int64_t r, int64_t& src_row, int64_t& dst_row) {
  if constexpr (M == RowMap::Gather) {
    src_row = a.row_idx[r];
    dst_row = r;
    return src_row >= 0 && src_row < a.src_rows;
  } else if constexpr (M == RowMap::Scatter) {
    const int64_t k = a.row_idx[r];
    const int b = find_segment_wave(a.cu, a.B + 1, k);
    if (b >= a.B || k < a.cu[b] || k >= a.cu[b + 1]) return false;
    src_row = r;
    dst_row = a.seq_starts[a.seq_ids[b]] + (k - a.cu[b]);
    return true;
  } else if constexpr (M == RowMap::GetSeqs || M == RowMap::ResetFull) {
    const int b = find_segment_wave(a.cu, a.B + 1, r);
    if (b >= a.B || r >= a.cu[b + 1]) return false;
    const int64_t cache_row = a.seq_starts[a.seq_ids[b]] + (r - a.cu[b]);
    if constexpr (M == RowMap::GetSeqs) {
      src_row = cache_row;
      dst_row = r;
    } else {
      src_row = r;
      dst_row = cache_row;
    }
    return true;
  } else {  // GetBlock / ResetBlock: the tail Lq rows of each cached sequence
    const int b = find_segment_wave(a.cu_q, a.B + 1, r);
    if (b >= a.B || r >= a.cu_q[b + 1]) return false;
    const int64_t Lq = a.cu_q[b + 1] - a.cu_q[b];
    const int64_t Lk = a.cu[b + 1] - a.cu[b];
    const int64_t cache_row = a.seq_starts[a.seq_ids[b]] + Lk - Lq + (r - a.cu_q[b]);
    if constexpr (M == RowMap::GetBlock) {
      src_row = cache_row;
      dst_row = r;
    } else {
      src_row = r;
      dst_row = cache_row;
    }
    return true;
  }
}

// 256 threads = 4 waves; wave w of block x copies row 4x+w.
template <RowMap M>
__global__ __launch_bounds__(256) void row_map_copy_kernel(RowMapArgs a) {
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= a.n_rows) return;
  int64_t s, d;
  if (!map_row<M>(a, r, s, d)) {
    if constexpr (M == RowMap::Gather) {   // out-of-range index: a zero row, no read
      uint4* dst = reinterpret_cast<uint4*>(a.dst + r * a.row_bytes);
      for (int64_t i = lane; i < (a.row_bytes >> 4); i += 64) dst[i] = make_uint4(0, 0, 0, 0);
    }
    return;
  }
  const uint4* src = reinterpret_cast<const uint4*>(a.src + s * a.row_bytes);
  uint4* dst = reinterpret_cast<uint4*>(a.dst + d * a.row_bytes);
  const int64_t n16 = a.row_bytes >> 4;
  int64_t i = lane;
  // 4 independent 16-byte loads in flight per lane before the stores.
  for (; i + 3 * 64 < n16; i += 4 * 64) {
    uint4 v0 = src[i], v1 = src[i + 64], v2 = src[i + 128], v3 = src[i + 192];
    dst[i] = v0;
    dst[i + 64] = v1;
    dst[i + 128] = v2;
    dst[i + 192] = v3;
  }
  for (; i < n16; i += 64) dst[i] = src[i];
}

int launch_row_map(RowMap mode, const RowMapArgs& a, hipStream_t stream) {
  DYLLM_REQUIRE(a.row_bytes > 0 && a.row_bytes % 16 == 0, "row size in bytes must be a positive multiple of 16");
  DYLLM_REQUIRE((reinterpret_cast<uintptr_t>(a.src) | reinterpret_cast<uintptr_t>(a.dst)) % 16 == 0,
                "row buffers must be 16-byte aligned");
  if (a.n_rows <= 0) return 0;
  const dim3 grid(unsigned(cdiv(a.n_rows, 4))), block(256);
  switch (mode) {
    case RowMap::GetSeqs: row_map_copy_kernel<RowMap::GetSeqs><<<grid, block, 0, stream>>>(a); break;
    case RowMap::GetBlock: row_map_copy_kernel<RowMap::GetBlock><<<grid, block, 0, stream>>>(a); break;
    case RowMap::ResetFull: row_map_copy_kernel<RowMap::ResetFull><<<grid, block, 0, stream>>>(a); break;
    case RowMap::ResetBlock: row_map_copy_kernel<RowMap::ResetBlock><<<grid, block, 0, stream>>>(a); break;
    case RowMap::Scatter: row_map_copy_kernel<RowMap::Scatter><<<grid, block, 0, stream>>>(a); break;
    case RowMap::Gather: row_map_copy_kernel<RowMap::Gather><<<grid, block, 0, stream>>>(a); break;
  }
  return check_launch("row_map_copy_kernel");
}

// Destination cache row of each packed row index (the address computation of
// scatter_update, cache_kernels.cu:397-419), so a GEMM epilogue can scatter in place.
__global__ __launch_bounds__(256) void scatter_dest_rows_kernel(const int64_t* __restrict__ row_idx, int64_t M,
                                                                const int32_t* __restrict__ m_dev,
                                                                const int32_t* __restrict__ cu,
                                                                const int64_t* __restrict__ seq_starts,
                                                                const int64_t* __restrict__ seq_ids, int B,
                                                                int64_t* __restrict__ dest) {
  const int64_t m = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (m >= M || (m_dev && m >= m_dev[0])) return;
  const int64_t k = row_idx[m];
  const int b = find_segment(cu, B + 1, k);
  dest[m] = seq_starts[seq_ids[b]] + (k - cu[b]);
}

int launch_scatter_dest_rows(const int64_t* row_idx, int64_t M, const int32_t* m_dev, const int32_t* cu,
                             const int64_t* seq_starts, const int64_t* seq_ids, int B, int64_t* dest, hipStream_t s) {
  if (M <= 0) return 0;
  scatter_dest_rows_kernel<<<unsigned(cdiv(M, 256)), 256, 0, s>>>(row_idx, M, m_dev, cu, seq_starts, seq_ids, B, dest);
  return check_launch("scatter_dest_rows_kernel");
}

}  // namespace dyllm

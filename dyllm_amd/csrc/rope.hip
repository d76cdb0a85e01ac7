// K/V epilogue of the sparse step's salient-row K/V projection (llada.py:103-146,
// dream.py:99-141, lladamoe.py:205-239). For every salient row j of kv = [k | v] (the kv_proj
// output of the gathered salient rows):
//   * k, per kv head: optional RMSNorm over the head (the k_norm of LLaDA-MoE,
//     layernorm.py:15-24: fp32 mean of squares, rsqrt, bf16, times the bf16 weight), then the
//     neox rotary embedding at the row's position (rotary_embedding.py:8-16, 40-54: fp32
//     y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin, rounded to bf16), written straight into the
//     row's K-cache row (CacheManager.scatter_update, cache_kernels.cu:388-426);
//   * v: copied out as the compact v_new the sparse attention step consumes.
// Without a cache mapping (k_rows == NULL) the rotated rows go to row j of the output and there
// is no v: the same pass serves the queries (q_norm + RoPE of all queried rows, in place).
// This replaces the reference's zero-filled [T, kv] temporary, the rotary over all T rows and the
// separate scatter with one pass over the n salient rows.
//
// One 256-thread workgroup per salient row: the row's index chain (position, sequence, cache
// row) is uniform across the workgroup and read once with scalar loads. Thread t works on kv head
// t / 8 (heads beyond 32 loop) and, inside it, on the 8 rotation pairs (d, d + 64) for
// d = 8 (t % 8) ... 8 (t % 8) + 7: 16-byte loads of k, cos and sin, the head's RMS reduced over
// its 8 threads.
#include "kernels.h"

namespace dyllm {

__device__ __forceinline__ void unpack8(const uint4 v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack8(const float* f) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}
__device__ __forceinline__ float bf16_round(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// one head's rotation pairs (d, d + 64) for d = d0 .. d0 + 7 of k (x1 = k[d], x2 = k[d + 64]) ->
// optional per-head RMSNorm (the head's sum of squares reduced over its 8 threads) -> neox
// rotation -> 16-byte stores at crow[d0] and crow[d0 + 64]
__device__ __forceinline__ void rope_k_values(float (&x1)[8], float (&x2)[8], const float (&c)[8], const float (&s)[8],
                                              const uint16_t* __restrict__ k_norm, float eps, int d0,
                                              uint16_t* __restrict__ crow) {
  constexpr int D = 128, HALF = 64;
  if (k_norm) {
    float w1[8], w2[8];
    unpack8(*reinterpret_cast<const uint4*>(k_norm + d0), w1);
    unpack8(*reinterpret_cast<const uint4*>(k_norm + d0 + HALF), w2);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    ss += __shfl_xor(ss, 4, 64);
    const float r = rsqrtf(ss / float(D) + eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x1[i] = bf16_round(__fmul_rn(bf16_round(x1[i] * r), w1[i]));
      x2[i] = bf16_round(__fmul_rn(bf16_round(x2[i] * r), w2[i]));
    }
  }
  float y1[8], y2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // rounded products, then the sum (no contraction): the eager fp32 formula
    y1[i] = mul_sub_mul_rn(x1[i], c[i], x2[i], s[i]);
    y2[i] = mul_add_mul_rn(x2[i], c[i], x1[i], s[i]);
  }
  *reinterpret_cast<uint4*>(crow + d0) = pack8(y1);
  *reinterpret_cast<uint4*>(crow + d0 + HALF) = pack8(y2);
}

// k of one row (Hkv heads of 128) -> optional per-head RMSNorm -> neox rotation at pos -> crow.
// Thread t of the 256-thread workgroup takes head t / 8 (heads beyond 32 loop) and the rotation
// pairs (d, d + 64), d = 8 (t % 8) .. 8 (t % 8) + 7.
__device__ __forceinline__ void rope_k_row(const uint16_t* __restrict__ krow, uint16_t* __restrict__ crow, int Hkv,
                                           int64_t pos, const float* __restrict__ cos_t,
                                           const float* __restrict__ sin_t, const uint16_t* __restrict__ k_norm,
                                           float eps) {
  constexpr int D = 128, HALF = 64;
  const int t = threadIdx.x;
  const int d0 = (t & 7) * 8;
  float c[8], s[8];
  *reinterpret_cast<float4*>(c) = *reinterpret_cast<const float4*>(cos_t + pos * HALF + d0);
  *reinterpret_cast<float4*>(c + 4) = *reinterpret_cast<const float4*>(cos_t + pos * HALF + d0 + 4);
  *reinterpret_cast<float4*>(s) = *reinterpret_cast<const float4*>(sin_t + pos * HALF + d0);
  *reinterpret_cast<float4*>(s + 4) = *reinterpret_cast<const float4*>(sin_t + pos * HALF + d0 + 4);
  for (int h = t >> 3; h < Hkv; h += 32) {
    float x1[8], x2[8];
    unpack8(*reinterpret_cast<const uint4*>(krow + h * D + d0), x1);
    unpack8(*reinterpret_cast<const uint4*>(krow + h * D + d0 + HALF), x2);
    rope_k_values(x1, x2, c, s, k_norm, eps, d0, crow + h * D);
  }
}

// positions are clamped to the table, as the reference does before its table lookup
// (rotary_embedding.py:45-48); the engine refuses sequences longer than the table
__device__ __forceinline__ int64_t clamp_pos(int64_t pos, int64_t max_position) {
  return pos < 0 ? 0 : (pos >= max_position ? max_position - 1 : pos);
}

__global__ __launch_bounds__(256) void kv_rope_scatter_kernel(KvRopeArgs a) {
  const int64_t j = blockIdx.x;
  const int64_t n = a.rows_dev ? int64_t(a.rows_dev[0]) : a.rows;
  if (j >= n) return;
  const int t = threadIdx.x;
  // row-uniform chain
  const int64_t pos = clamp_pos(a.positions[a.pos_idx ? int64_t(a.pos_idx[j]) : j], a.max_position);
  int64_t dest = j;   // in-place mode (no cache mapping): row j of the output
  if (a.k_rows) {
    const int64_t kk = a.k_rows[j];
    const int b = find_segment_wave(a.cu_k, a.B + 1, kk);
    dest = a.seq_starts[a.seq_ids[b]] + (kk - a.cu_k[b]);
  }
  const uint16_t* krow = a.kv + j * a.ld_kv;
  rope_k_row(krow, a.k_cache + dest * a.ld_cache, a.Hkv, pos, a.cos, a.sin, a.k_norm, a.eps);
  // v: kv_size values -> v_out row j (16 bytes per thread per pass)
  if (!a.v_out) return;
  const uint4* vr = reinterpret_cast<const uint4*>(krow + a.kv_size);
  uint4* vo = reinterpret_cast<uint4*>(a.v_out + j * a.kv_size);
  for (int64_t i = t; i < a.kv_size / 8; i += 256) vo[i] = vr[i];
}

// One 256-thread workgroup per salient list entry j (StepRowsArgs). Every wavefront derives the
// entry's sequence and its key's rank among the sequence's salient keys itself (ballot counts over
// the sequence's list segment, a few hundred entries at most), so no workgroup waits on another.
// The loads that depend on j alone (the new v row, the k row, its position and rotary table rows)
// are issued before that index chain, so its round trips overlap them.
__global__ __launch_bounds__(256) void step_rows_kernel(StepRowsArgs a) {
  constexpr int D = 128, HALF = 64;
  const int j = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63;
  if (j == 0)
    for (int i = t; i < a.nzero; i += 256) a.zero[i] = 0;
  if (j >= a.n) return;
  const uint16_t* src = a.kv ? a.kv + (a.kv_rows ? int64_t(a.kv_rows[j]) : int64_t(j)) * a.ld_kv : nullptr;
  const uint4* nr = reinterpret_cast<const uint4*>(src ? src + a.kv_size : a.v_new + int64_t(j) * a.kv_size);
  const int64_t n16 = a.kv_size / 8;
  // the first two 16-byte pieces of this thread's part of the new v row (the rest, if any, later)
  uint4 nv0 = make_uint4(0, 0, 0, 0), nv1 = make_uint4(0, 0, 0, 0);
  if (t < n16) nv0 = nr[t];
  if (t + 256 < n16) nv1 = nr[t + 256];
  // k of head t / 8 (one head per thread group when Hkv <= 32, the common case)
  const bool k_fast = src && a.Hkv <= 32;
  const int h = t >> 3, d0 = (t & 7) * 8;
  float x1[8], x2[8], c[8], sn[8];
  if (k_fast && h < a.Hkv) {
    const int64_t pos = clamp_pos(a.positions[a.pos_idx ? int64_t(a.pos_idx[j]) : int64_t(j)], a.max_position);
    unpack8(*reinterpret_cast<const uint4*>(src + h * D + d0), x1);
    unpack8(*reinterpret_cast<const uint4*>(src + h * D + d0 + HALF), x2);
    *reinterpret_cast<float4*>(c) = *reinterpret_cast<const float4*>(a.cos + pos * HALF + d0);
    *reinterpret_cast<float4*>(c + 4) = *reinterpret_cast<const float4*>(a.cos + pos * HALF + d0 + 4);
    *reinterpret_cast<float4*>(sn) = *reinterpret_cast<const float4*>(a.sin + pos * HALF + d0);
    *reinterpret_cast<float4*>(sn + 4) = *reinterpret_cast<const float4*>(a.sin + pos * HALF + d0 + 4);
  }
  // the sequence of entry j, its key, and the key's rank among the sequence's salient keys
  const int b = find_segment_wave(a.cu_sal, a.B + 1, j);
  const int64_t s0 = a.cu_sal[b], s1 = a.cu_sal[b + 1];
  const int64_t kbeg = a.cu_k[b], Lk = a.cu_k[b + 1] - kbeg;
  const int64_t off = int64_t(a.idx_k32[j]) - kbeg;
  // an entry outside its sequence's keys updates nothing (the attention tiles ignore it as well)
  if (off < 0 || off >= Lk) return;
  int rank = 0;
  for (int64_t base = s0; base < s1; base += 64) {
    const int64_t i = base + lane;
    bool lt = false;
    if (i < s1) {
      const int64_t kk = int64_t(a.idx_k32[i]) - kbeg;
      lt = kk >= 0 && kk < off;
    }
    rank += __popcll(__ballot(lt));
  }
  const int64_t sid = a.seq_ids[b];
  uint4* cr = reinterpret_cast<uint4*>(a.v_cache + (a.v_seq_starts[sid] + off) * a.kv_size);
  uint4* dr = reinterpret_cast<uint4*>(a.dv + (s0 + rank) * a.kv_size);
  {
    const uint4 o0 = t < n16 ? cr[t] : make_uint4(0, 0, 0, 0);
    const uint4 o1 = t + 256 < n16 ? cr[t + 256] : make_uint4(0, 0, 0, 0);
    if (t < n16) {
      dr[t] = bf16x8_sub(nv0, o0);
      cr[t] = nv0;
    }
    if (t + 256 < n16) {
      dr[t + 256] = bf16x8_sub(nv1, o1);
      cr[t + 256] = nv1;
    }
  }
  for (int64_t i = t + 512; i < n16; i += 256) {   // v rows past 512 pieces (more than 32 kv heads)
    const uint4 o = cr[i], nw = nr[i];
    dr[i] = bf16x8_sub(nw, o);
    cr[i] = nw;
  }
  if (!src) return;
  uint16_t* crow = a.k_cache + (a.k_seq_starts[sid] + off) * a.kv_size;
  if (!k_fast) {
    const int64_t pos = clamp_pos(a.positions[a.pos_idx ? int64_t(a.pos_idx[j]) : int64_t(j)], a.max_position);
    rope_k_row(src, crow, a.Hkv, pos, a.cos, a.sin, a.k_norm, a.eps);
    return;
  }
  if (h >= a.Hkv) return;
  rope_k_values(x1, x2, c, sn, a.k_norm, a.eps, d0, crow + h * D);
}

int launch_step_rows(const StepRowsArgs& a, hipStream_t s) {
  const int grid = a.n > 1 ? a.n : 1;
  if (a.n <= 0 && a.nzero <= 0) return 0;
  step_rows_kernel<<<unsigned(grid), 256, 0, s>>>(a);
  return check_launch("step_rows_kernel");
}

int launch_kv_rope_scatter(const KvRopeArgs& a, hipStream_t s) {
  if (a.rows <= 0) return 0;
  kv_rope_scatter_kernel<<<unsigned(a.rows), 256, 0, s>>>(a);
  return check_launch("kv_rope_scatter_kernel");
}

}  // namespace dyllm

// K/V epilogue of the sparse step's salient-row K/V projection (llada.py:103-146,
// dream.py:99-141, lladamoe.py:205-239). For every salient row j of kv = [k | v] (the kv_proj
// output of the gathered salient rows):
//   * k, per kv head: optional RMSNorm over the head (the k_norm of LLaDA-MoE,
//     layernorm.py:15-24: fp32 mean of squares, rsqrt, bf16, times the bf16 weight), then the
//     neox rotary embedding at the row's position (rotary_embedding.py:8-16, 40-54: fp32
//     y1 = x1 cos - x2 sin, y2 = x2 cos + x1 sin, rounded to bf16), written straight into the
//     row's K-cache row (CacheManager.scatter_update, cache_kernels.cu:388-426);
//   * v: copied out as the compact v_new the sparse attention step consumes.
// This replaces the reference's zero-filled [T, kv] temporary, the rotary over all T rows and the
// separate scatter with one pass over the n salient rows.
//
// One wavefront per (row, kv head): lane i holds the rotation pair (d = i, d = i + 64) of the
// 128-wide head, so the rotation and the head RMS reduction stay inside the wavefront.
#include "kernels.h"

namespace dyllm {

__global__ __launch_bounds__(256) void kv_rope_scatter_kernel(KvRopeArgs a) {
  const int64_t wid = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t n = a.rows_dev ? int64_t(a.rows_dev[0]) : a.rows;
  const int64_t j = wid / a.Hkv;
  const int h = int(wid - j * a.Hkv);
  if (j >= n || j >= a.rows) return;
  constexpr int D = 128, HALF = 64;

  const uint16_t* kr = a.kv + j * a.ld_kv + int64_t(h) * D;
  float x1 = bf16_to_f32(kr[lane]);
  float x2 = bf16_to_f32(kr[lane + HALF]);
  if (a.k_norm) {
    float ss = x1 * x1 + x2 * x2;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float r = rsqrtf(ss / float(D) + a.eps);
    x1 = __fmul_rn(bf16_to_f32(f32_to_bf16(x1 * r)), bf16_to_f32(a.k_norm[lane]));
    x2 = __fmul_rn(bf16_to_f32(f32_to_bf16(x2 * r)), bf16_to_f32(a.k_norm[lane + HALF]));
    x1 = bf16_to_f32(f32_to_bf16(x1));
    x2 = bf16_to_f32(f32_to_bf16(x2));
  }
  int64_t pos = a.positions[a.pos_idx ? int64_t(a.pos_idx[j]) : j];
  pos = pos < 0 ? 0 : (pos >= a.max_position ? a.max_position - 1 : pos);
  const float c = a.cos[pos * HALF + lane], s = a.sin[pos * HALF + lane];
  // rounded products and sums in this order (no contraction): the eager fp32 formula
  const float y1 = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
  const float y2 = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));

  const int64_t kk = a.k_rows[j];
  const int b = find_segment(a.cu_k, a.B + 1, kk);
  const int64_t dest = a.seq_starts[a.seq_ids[b]] + (kk - a.cu_k[b]);
  uint16_t* kc = a.k_cache + dest * a.ld_cache + int64_t(h) * D;
  kc[lane] = f32_to_bf16(y1);
  kc[lane + HALF] = f32_to_bf16(y2);

  if (lane < D / 8) {
    const uint4* vr = reinterpret_cast<const uint4*>(a.kv + j * a.ld_kv + a.kv_size + int64_t(h) * D);
    reinterpret_cast<uint4*>(a.v_out + j * a.kv_size + int64_t(h) * D)[lane] = vr[lane];
  }
}

int launch_kv_rope_scatter(const KvRopeArgs& a, hipStream_t s) {
  if (a.rows <= 0) return 0;
  const int64_t waves = a.rows * a.Hkv;
  kv_rope_scatter_kernel<<<unsigned(cdiv(waves, 4)), 256, 0, s>>>(a);
  return check_launch("kv_rope_scatter_kernel");
}

}  // namespace dyllm

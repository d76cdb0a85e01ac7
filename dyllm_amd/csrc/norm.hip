// RMSNorm with the optional fused residual add of the decoder layers (layernorm.py:15-37:
// rms_forward / add_rms_forward): per row
//   s = x (+ residual)                         fp32
//   residual_out = bf16(s)                      (only with a residual)
//   y = bf16( bf16(s * rsqrt(mean(s^2) + eps)) * weight )
// in one pass over the row (the reference's torch ops read and write the [T, hidden] tensors
// several times). One 256-thread workgroup per row, 16-byte loads, up to 4 chunks of 8 values
// per thread (hidden <= 8192), the sum of squares reduced over the workgroup in a fixed order.
// x may also be read straight from a per-layer row cache through the tail-block addressing of
// get_block (the FFN-output cache of a sparse step), so the packed copy of those rows that the
// reference hands to the next layer's norm (mlp_cache_manage.py:33-38) is never made.
#include "kernels.h"

namespace dyllm {

constexpr int kNormThreads = 256;
constexpr int kNormMaxChunks = 4;

__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(NormArgs a) {
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const int nch = a.hidden / 8;
  int64_t xrow = row;
  if (a.x_seq_starts) {   // the row lives in a cache slab (uniform across the workgroup)
    const int b = find_segment_wave(a.x_cu_q, a.x_batch + 1, row);
    xrow = a.x_seq_starts[a.x_seq_ids[b]] + (a.x_cu_k[b + 1] - a.x_cu_k[b]) - (a.x_cu_q[b + 1] - a.x_cu_q[b]) +
           (row - a.x_cu_q[b]);
  }
  const uint4* xr = reinterpret_cast<const uint4*>(a.x + xrow * a.ld_x);
  const uint4* rr = a.residual ? reinterpret_cast<const uint4*>(a.residual + row * a.ld_r) : nullptr;
  float v[kNormMaxChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNormMaxChunks; ++c) {
    const int i = t + c * kNormThreads;
    if (i >= nch) break;
    const uint4 xv = xr[i];
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[c][2 * e] = __uint_as_float(xw[e] << 16);
      v[c][2 * e + 1] = __uint_as_float(xw[e] & 0xffff0000u);
    }
    if (rr) {
      const uint4 rv = rr[i];
      const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[c][2 * e] = __fadd_rn(v[c][2 * e], __uint_as_float(rw[e] << 16));
        v[c][2 * e + 1] = __fadd_rn(v[c][2 * e + 1], __uint_as_float(rw[e] & 0xffff0000u));
      }
      uint4 o;
      o.x = pack_bf16x2(v[c][0], v[c][1]);
      o.y = pack_bf16x2(v[c][2], v[c][3]);
      o.z = pack_bf16x2(v[c][4], v[c][5]);
      o.w = pack_bf16x2(v[c][6], v[c][7]);
      reinterpret_cast<uint4*>(a.residual_out + row * a.ld_ro)[i] = o;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[c][e] * v[c][e];
  }
  // workgroup sum of squares: wavefront butterfly, then the 4 partials in order
  __shared__ float part[kNormThreads / 64];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((t & 63) == 0) part[t >> 6] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float r = rsqrtf(tot / float(a.hidden) + a.eps);
  const uint4* wr = reinterpret_cast<const uint4*>(a.weight);
  uint4* yr = reinterpret_cast<uint4*>(a.out + row * a.ld_out);
#pragma unroll
  for (int c = 0; c < kNormMaxChunks; ++c) {
    const int i = t + c * kNormThreads;
    if (i >= nch) break;
    const uint4 wv = wr[i];
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
    float y[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float n0 = bf16_to_f32(f32_to_bf16(__fmul_rn(v[c][2 * e], r)));
      const float n1 = bf16_to_f32(f32_to_bf16(__fmul_rn(v[c][2 * e + 1], r)));
      y[2 * e] = __fmul_rn(n0, __uint_as_float(ww[e] << 16));
      y[2 * e + 1] = __fmul_rn(n1, __uint_as_float(ww[e] & 0xffff0000u));
    }
    uint4 o;
    o.x = pack_bf16x2(y[0], y[1]);
    o.y = pack_bf16x2(y[2], y[3]);
    o.z = pack_bf16x2(y[4], y[5]);
    o.w = pack_bf16x2(y[6], y[7]);
    yr[i] = o;
  }
}

int launch_add_rms_norm(const NormArgs& a, hipStream_t s) {
  DYLLM_REQUIRE(a.hidden > 0 && a.hidden % 8 == 0 && a.hidden <= 8 * kNormThreads * kNormMaxChunks,
                "hidden size must be a positive multiple of 8, at most 8192");
  if (a.rows <= 0) return 0;
  add_rms_norm_kernel<<<unsigned(a.rows), kNormThreads, 0, s>>>(a);
  return check_launch("add_rms_norm_kernel");
}

}  // namespace dyllm

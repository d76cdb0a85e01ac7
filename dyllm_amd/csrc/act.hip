// SiLU-and-mul of a merged gate_up product (SiluAndMul, activations.py:11-14): for gu rows
// [g (I) | u (I)] in bf16, h = bf16(silu(g) * u) computed in fp32 with one rounding, the same
// arithmetic (and bits) as the SwiGLU epilogue of the fused GEMM. Used after a library GEMM for the
// dense full-step FFN, where the vendor GEMM is faster than the fused one at thousands of rows.
// HBM-bound: 6 I bytes per row; each thread moves 8 elements per iteration with 16-byte accesses.
#include "kernels.h"

namespace dyllm {

__global__ __launch_bounds__(256) void silu_and_mul_kernel(const uint16_t* __restrict__ gu, int64_t ld_in,
                                                           int64_t rows, int inter, uint16_t* __restrict__ out,
                                                           int64_t ld_out) {
  const int64_t per_row = inter / 8;
  const int64_t total = rows * per_row;
  for (int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x; t < total; t += int64_t(gridDim.x) * 256) {
    const int64_t r = t / per_row;
    const int64_t c = (t - r * per_row) * 8;
    const uint4 g = *reinterpret_cast<const uint4*>(gu + r * ld_in + c);
    const uint4 u = *reinterpret_cast<const uint4*>(gu + r * ld_in + inter + c);
    const uint32_t gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = silu_f(__uint_as_float(gv[e] << 16)) * __uint_as_float(uv[e] << 16);
      const float hi = silu_f(__uint_as_float(gv[e] & 0xffff0000u)) * __uint_as_float(uv[e] & 0xffff0000u);
      h[e] = pack_bf16x2(lo, hi);
    }
    *reinterpret_cast<uint4*>(out + r * ld_out + c) = make_uint4(h[0], h[1], h[2], h[3]);
  }
}

int launch_silu_and_mul(const uint16_t* gu, int64_t ld_in, int64_t rows, int inter, uint16_t* out, int64_t ld_out,
                        hipStream_t s) {
  DYLLM_REQUIRE(inter > 0 && inter % 8 == 0, "intermediate size must be a positive multiple of 8");
  DYLLM_REQUIRE(ld_in % 8 == 0 && ld_out % 8 == 0 && ld_in >= 2 * int64_t(inter) && ld_out >= inter,
                "row strides must be multiples of 8 elements covering the rows");
  DYLLM_REQUIRE(reinterpret_cast<uintptr_t>(gu) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
                "gate_up and output must be 16-byte aligned");
  if (rows <= 0) return 0;
  const int64_t chunks = rows * (inter / 8);
  const int64_t blocks = cdiv(chunks, 256) < 8192 ? cdiv(chunks, 256) : 8192;
  silu_and_mul_kernel<<<unsigned(blocks), 256, 0, s>>>(gu, ld_in, rows, inter, out, ld_out);
  return check_launch("silu_and_mul_kernel");
}

}  // namespace dyllm

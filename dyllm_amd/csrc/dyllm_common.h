// Shared helpers for the gfx950 (CDNA4) kernels of the DyLLM saliency hot path.
// Wave64 only; bf16 values are carried as raw uint16_t bits on the host side and as
// clang __bf16 vectors where they feed MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace dyllm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }

// Products rounded before the sum, never fused into an FMA. HIP's __fmul_rn / __fadd_rn are
// plain operators here and would be contracted by the default -ffp-contract; these helpers keep
// the reference's separately rounded forms.
__device__ __forceinline__ float add_mul_rn(float c, float a, float b) {  // c + a*b
#pragma clang fp contract(off)
  return c + a * b;
}
__device__ __forceinline__ float mul_sub_mul_rn(float a, float b, float c, float d) {  // a*b - c*d
#pragma clang fp contract(off)
  return a * b - c * d;
}
__device__ __forceinline__ float mul_add_mul_rn(float a, float b, float c, float d) {  // a*b + c*d
#pragma clang fp contract(off)
  return a * b + c * d;
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

// fp32 -> bf16 with the gfx950 hardware conversion (v_cvt_pk_bf16_f32, round to nearest
// even under the default rounding mode).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2_t r;
  r[0] = (__bf16)a;
  r[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return uint16_t(pack_bf16x2(f, 0.0f) & 0xffffu); }

// x[l] op x[l ^ 32] in every lane through v_permlane32_swap (a register swap between the two
// wave halves, no LDS round trip as __shfl_xor takes); op is commutative, so both halves get the
// same bits.
__device__ __forceinline__ float half_swap_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Index of the segment of a sorted prefix array cu[0..n] (cu[0]=0) that holds row r:
// the largest b in [0, n) with cu[b] <= r.
template <typename T>
__device__ __forceinline__ int find_segment(const T* cu, int n, int64_t r) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (int64_t(cu[mid]) <= r)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

// find_segment for a row index that is the same in every lane of the (fully active) wavefront:
// each lane compares one prefix entry, one coalesced load per 64 entries, and the ballot count
// replaces the binary search's chain of dependent loads. Same result as find_segment (0 when
// r < cu[0]).
template <typename T>
__device__ __forceinline__ int find_segment_wave(const T* cu, int n, int64_t r) {
  const int lane = threadIdx.x & 63;
  int cnt = 0;
  for (int base = 0; base < n - 1; base += 64) {
    const int i = base + lane;
    const bool le = i < n - 1 && int64_t(cu[i]) <= r;
    cnt += __popcll(__ballot(le));
  }
  return cnt > 0 ? cnt - 1 : 0;
}

// bf16 x 8 difference new - old, each element rounded once (the dV of attention.py:67-74)
__device__ __forceinline__ uint4 bf16x8_sub(uint4 nw, uint4 o) {
  const uint32_t ov[4] = {o.x, o.y, o.z, o.w}, nv[4] = {nw.x, nw.y, nw.z, nw.w};
  uint32_t d[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = __fsub_rn(__uint_as_float(nv[e] << 16), __uint_as_float(ov[e] << 16));
    const float hi = __fsub_rn(__uint_as_float(nv[e] & 0xffff0000u), __uint_as_float(ov[e] & 0xffff0000u));
    d[e] = pack_bf16x2(lo, hi);
  }
  return make_uint4(d[0], d[1], d[2], d[3]);
}

// x * sigmoid(x) with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of an IEEE division:
// within 2-3 ulp of fp32 x / (1 + exp(-x)) before the bf16 rounding of the product. v_rcp_f32
// flushes a denormal result, which 1 / (1 + exp(-x)) is for x in (-88.7, -87.3) while
// x / (1 + exp(-x)) is still a normal number there; the reciprocal is therefore taken of the
// denominator scaled by 2^-64 and the product scaled back (both scalings are exact), which leaves
// every other value unchanged and saturates to -0 / x at the tails like the division. Shared by
// the SwiGLU GEMM epilogue and the standalone SiLU-and-mul kernel, so both give the same bits.
__device__ __forceinline__ float silu_f(float x) {
  const float r = __builtin_amdgcn_rcpf((1.0f + __expf(-x)) * 0x1p-64f);
  return (x * r) * 0x1p-64f;
}

__host__ __device__ constexpr inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- host-side error plumbing -------------------------------------------------------
void set_error(const std::string& msg);
int fail(const std::string& msg);            // sets the message, returns a non-zero status
int check_launch(const char* what);          // hipGetLastError -> status
}  // namespace dyllm

#define DYLLM_REQUIRE(cond, msg)                 \
  do {                                           \
    if (!(cond)) return ::dyllm::fail(msg);      \
  } while (0)

// Issue-rate probe of one gfx950 SIMD (no counterpart in the reference; for bench.py
// --probe-issue): how long a wavefront takes per loop iteration of
//   MFMA  -- 4 independent v_mfma_f32_32x32x16_bf16 (accumulators in AGPRs),
//   FMA   -- 64 independent-chain v_fma_f32 (16 chains, 4 deep),
//   EXP   -- 64 v_exp_f32 + 64 v_mul_f32 on the same 16 chains,
// alone and together in one wavefront, the compiler interleaving them (and, for the pinned
// variants, sched_group_barrier forcing 1 MFMA then 16 VALU), at one wavefront per SIMD (one
// 256-thread workgroup per CU). If MFMA and VALU work of one wavefront overlapped, MFMA+FMA would
// take max(MFMA, FMA) cycles; if they serialise, MFMA + FMA. Cycles come from s_memtime.
#include "kernels.h"

namespace dyllm {

template <int MODE, bool PIN>
__global__ __launch_bounds__(256) void issue_probe_kernel(float* __restrict__ sink, unsigned long long* __restrict__ cyc,
                                                          int iters) {
  const int t = threadIdx.x;
  bf16x8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(float((t + i) & 7) * 0.01f);
    b[i] = (__bf16)(float((t * 3 + i) & 7) * 0.01f);
  }
  f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  float v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = float(t + j) * 1e-3f;
  const float x = 0.999f, y = 1e-4f;
  const unsigned long long t0 = __builtin_readcyclecounter();
  for (int it = 0; it < iters; ++it) {
    if constexpr (MODE & 1) {
      c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
    }
    if constexpr ((MODE & 6) != 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          if constexpr ((MODE & 4) != 0)
            v[j] = __builtin_amdgcn_exp2f(v[j]) * x;
          else
            v[j] = fmaf(v[j], x, y);
        }
    }
    if constexpr (PIN) {
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);   // then 16 VALU
      }
    }
  }
  const unsigned long long t1 = __builtin_readcyclecounter();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
#pragma unroll
  for (int j = 0; j < 16; ++j) s += v[j];
  sink[int64_t(blockIdx.x) * blockDim.x + t] = s;
  if (t == 0) cyc[blockIdx.x] = t1 - t0;
}

template <int MODE, bool PIN>
static int run_issue_probe(int wgs, int iters, float* sink, unsigned long long* cyc, hipStream_t s) {
  issue_probe_kernel<MODE, PIN><<<unsigned(wgs), 256, 0, s>>>(sink, cyc, iters);
  return check_launch("issue_probe_kernel");
}

// mode: 0 MFMA, 1 FMA, 2 EXP, 3 MFMA+FMA, 4 MFMA+FMA pinned, 5 MFMA+EXP, 6 MFMA+EXP pinned
int launch_issue_probe(int mode, int wgs, int iters, float* sink, unsigned long long* cyc, hipStream_t s) {
  switch (mode) {
    case 0: return run_issue_probe<1, false>(wgs, iters, sink, cyc, s);
    case 1: return run_issue_probe<2, false>(wgs, iters, sink, cyc, s);
    case 2: return run_issue_probe<4, false>(wgs, iters, sink, cyc, s);
    case 3: return run_issue_probe<3, false>(wgs, iters, sink, cyc, s);
    case 4: return run_issue_probe<3, true>(wgs, iters, sink, cyc, s);
    case 5: return run_issue_probe<5, false>(wgs, iters, sink, cyc, s);
    case 6: return run_issue_probe<5, true>(wgs, iters, sink, cyc, s);
    default: return fail("issue probe: mode must be 0..6");
  }
}

}  // namespace dyllm

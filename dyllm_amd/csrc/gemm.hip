// Gathered bf16 GEMM on gfx950 MFMA: C[row(m)][n] = sum_k A[arow(m)][k] * W[n][k]
// (both operands K-contiguous, the nn.Linear [out, in] weight layout), with
//
//   * an indexed A prologue  -- rows of the compacted tile are read straight from the
//                               packed activations through an index list (gather_rows_2D,
//                               dyllm/utils/util.py:19-36; MoE: token = sorted_id / top_k,
//                               fused_moe.py:144-146);
//   * a SwiGLU epilogue      -- gate and up halves of the merged gate_up weight are
//                               multiplied in the same workgroup, and silu(g) * u is written
//                               (MergedColumnParallelLinear + SiluAndMul, linear.py:76-93,
//                               activations.py:11-14; g and u are rounded to bf16 first, as
//                               the reference's bf16 GEMM output is);
//   * a store epilogue       -- optional per-row routing weight (fused_moe.py:160-162) and a
//                               row remap that scatters straight into the cached FFN output
//                               (MLPcache.scatter_update, mlp_cache_manage.py:24-40).
//
// Tiling: workgroup tile BM x BN x 64, 4 wavefronts in a 2 x 2 grid, each wavefront a
// (BM/2) x (BN/2) block of v_mfma_f32_32x32x16_bf16 tiles. Operands are staged through LDS
// in two buffers (rows padded to 144 B so the 16-byte fragment reads are conflict free),
// with the next K slice prefetched into registers while the current one is multiplied.
// The MFMA is issued as D = W_tile * A_tile^T so that each lane owns one output row and
// four consecutive output columns per register group: 8-byte stores and one row lookup
// per lane for the scatter. Workgroups are ordered M-fastest and remapped XCD-major so the
// M tiles sharing a weight slice run on one XCD and read that slice from HBM once.
#include "kernels.h"

namespace dyllm {

constexpr int kGemmBK = 64;
constexpr int kGemmLds = kGemmBK + 8;  // 72 elements = 144 B per staged row

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }
__device__ __forceinline__ float bf16_rt(float x) { return __uint_as_float(uint32_t(f32_to_bf16(x)) << 16); }

template <int BM, int BN, GemmEpi EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t gsm[];
  constexpr int WM = BM / 2, WN = BN / 2;     // wave tile (rows of A, rows of W)
  constexpr int TM = WM / 32, TN = WN / 32;   // 32x32 MFMA tiles per wave
  constexpr int CA = BM / 32, CW = BN / 32;   // 16-byte chunks per thread per K slice
  constexpr int BUF = (BM + BN) * kGemmLds;

  const int64_t M = g.num_m_dev ? int64_t(g.num_m_dev[0]) : g.M;
  const int n_tiles = (EPI == GemmEpi::SwiGLU) ? (g.half_n / (BN / 2)) : int(cdiv(g.N, BN));
  const int nwg = gridDim.x;
  int wg = blockIdx.x;
  if ((nwg & 7) == 0) wg = (wg & 7) * (nwg >> 3) + (wg >> 3);
  const int m_tiles_launched = nwg / n_tiles;
  const int mt = wg % m_tiles_launched, nt = wg / m_tiles_launched;
  const int64_t m0 = int64_t(mt) * BM;
  if (m0 >= M) return;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1;
  const int l32 = lane & 31, half = lane >> 5;

  const uint16_t* Wb = g.W;
  if (g.tile_expert) Wb += int64_t(g.tile_expert[mt]) * g.w_expert_stride;

  // rows this thread stages: A row r = tid/8 + 32*i, W row likewise; k chunk = tid%8
  const int kc = tid & 7;
  const uint16_t* a_src[CA];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int64_t m = m0 + (tid >> 3) + 32 * i;
    a_src[i] = nullptr;
    if (m < M) {
      int64_t row = m;
      if (g.a_ids) {
        const int64_t id = g.a_ids[m];
        row = (id < g.id_limit) ? id / g.a_div : -1;
      }
      if (row >= 0) a_src[i] = g.A + row * g.lda + kc * 8;
    }
  }
  const uint16_t* w_src[CW];
#pragma unroll
  for (int i = 0; i < CW; ++i) {
    const int r = (tid >> 3) + 32 * i;
    int64_t wrow;
    if constexpr (EPI == GemmEpi::SwiGLU)
      wrow = (r < BN / 2) ? int64_t(nt) * (BN / 2) + r : int64_t(g.half_n) + int64_t(nt) * (BN / 2) + (r - BN / 2);
    else
      wrow = int64_t(nt) * BN + r;
    w_src[i] = (wrow < g.N) ? Wb + wrow * g.ldw + kc * 8 : nullptr;
  }

  uint4 ra[CA], rw[CW];
  auto gload = [&](int kt) {
    const int64_t ko = int64_t(kt) * kGemmBK;
#pragma unroll
    for (int i = 0; i < CA; ++i) ra[i] = a_src[i] ? *reinterpret_cast<const uint4*>(a_src[i] + ko) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < CW; ++i) rw[i] = w_src[i] ? *reinterpret_cast<const uint4*>(w_src[i] + ko) : make_uint4(0, 0, 0, 0);
  };
  auto lstore = [&](int buf) {
    uint16_t* As = gsm + buf * BUF;
    uint16_t* Ws = As + BM * kGemmLds;
#pragma unroll
    for (int i = 0; i < CA; ++i) *reinterpret_cast<uint4*>(&As[((tid >> 3) + 32 * i) * kGemmLds + kc * 8]) = ra[i];
#pragma unroll
    for (int i = 0; i < CW; ++i) *reinterpret_cast<uint4*>(&Ws[((tid >> 3) + 32 * i) * kGemmLds + kc * 8]) = rw[i];
  };

  // W-tile row base of the wave's n-subtile i
  auto wrow_base = [&](int i) -> int {
    if constexpr (EPI == GemmEpi::SwiGLU)
      return (i < TN / 2) ? wn * (BN / 4) + 32 * i : BN / 2 + wn * (BN / 4) + 32 * (i - TN / 2);
    else
      return wn * WN + 32 * i;
  };

  f32x16_t acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = g.K / kGemmBK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const uint16_t* As = gsm + cur * BUF;
    const uint16_t* Ws = As + BM * kGemmLds;
#pragma unroll
    for (int ks = 0; ks < kGemmBK / 16; ++ks) {
      bf16x8_t wf[TN], af[TM];
#pragma unroll
      for (int i = 0; i < TN; ++i)
        wf[i] = *reinterpret_cast<const bf16x8_t*>(&Ws[(wrow_base(i) + l32) * kGemmLds + ks * 16 + half * 8]);
#pragma unroll
      for (int j = 0; j < TM; ++j)
        af[j] = *reinterpret_cast<const bf16x8_t*>(&As[(wm * WM + 32 * j + l32) * kGemmLds + ks * 16 + half * 8]);
#pragma unroll
      for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], af[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane owns row m = m0 + wm*WM + 32j + l32 -------------------------------
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int64_t m = m0 + wm * WM + 32 * j + l32;
    if (m >= M) continue;
    int64_t drow = m;
    int64_t id = m;
    if (g.a_ids) {
      id = g.a_ids[m];
      if (id >= g.id_limit) continue;
      if (g.c_by_id) drow = id;
    }
    if (g.c_rows) drow = g.c_rows[m];
    float scale = 1.0f;
    if (g.row_scale_f32) scale = g.row_scale_f32[id];
    if (g.row_scale_bf16) scale = bf16_to_f32(g.row_scale_bf16[id]);
    uint16_t* crow = g.Cout + drow * g.ldc;
    if constexpr (EPI == GemmEpi::SwiGLU) {
#pragma unroll
      for (int i = 0; i < TN / 2; ++i) {
        const int hc0 = nt * (BN / 2) + wn * (BN / 4) + 32 * i + half * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gv = bf16_rt(acc[i][j][4 * q + e]);
            const float uv = bf16_rt(acc[i + TN / 2][j][4 * q + e]);
            h[e] = silu_f(gv) * uv;
          }
          uint2 st;
          st.x = pack_bf16x2(h[0], h[1]);
          st.y = pack_bf16x2(h[2], h[3]);
          *reinterpret_cast<uint2*>(crow + hc0 + q * 8) = st;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TN; ++i) {
        const int n0 = nt * BN + wn * WN + 32 * i + half * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + q * 8;
          if (n >= g.N) continue;
          uint2 st;
          st.x = pack_bf16x2(acc[i][j][4 * q] * scale, acc[i][j][4 * q + 1] * scale);
          st.y = pack_bf16x2(acc[i][j][4 * q + 2] * scale, acc[i][j][4 * q + 3] * scale);
          *reinterpret_cast<uint2*>(crow + n) = st;
        }
      }
    }
  }
}

template <int BM, int BN, GemmEpi EPI>
static int launch_gemm_cfg(const GemmArgs& g, int64_t m_tiles, hipStream_t s) {
  const int n_tiles = (EPI == GemmEpi::SwiGLU) ? (g.half_n / (BN / 2)) : int(cdiv(g.N, BN));
  const int64_t nwg = m_tiles * n_tiles;
  if (nwg == 0) return 0;
  DYLLM_REQUIRE(nwg < (int64_t(1) << 31), "GEMM grid too large");
  const size_t lds = size_t(2) * (BM + BN) * kGemmLds * sizeof(uint16_t);
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<BM, BN, EPI>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) != hipSuccess)
      return fail("hipFuncSetAttribute(max dynamic LDS) failed for the GEMM kernel");
    attr_set = true;
  }
  gemm_kernel<BM, BN, EPI><<<unsigned(nwg), 256, lds, s>>>(g);
  return check_launch("gemm_kernel");
}

// m_bound: host-side upper bound of M (number of BM tiles launched = cdiv(m_bound, BM)).
int launch_gemm(GemmEpi epi, const GemmArgs& g, int64_t m_bound, int tile_m, hipStream_t s) {
  DYLLM_REQUIRE(g.K > 0 && g.K % kGemmBK == 0, "GEMM K must be a positive multiple of 64");
  DYLLM_REQUIRE(g.N > 0, "GEMM N must be positive");
  DYLLM_REQUIRE(g.lda % 8 == 0 && g.ldw % 8 == 0 && g.ldc % 4 == 0, "GEMM leading dimensions must keep 16-byte rows");
  if (m_bound <= 0) return 0;
  if (epi == GemmEpi::SwiGLU) {
    DYLLM_REQUIRE(g.N == 2 * g.half_n, "SwiGLU weight must hold gate rows then up rows (N = 2 * intermediate)");
    if (tile_m == 256) {
      DYLLM_REQUIRE(g.half_n % 128 == 0, "SwiGLU intermediate size must be a multiple of 128");
      return launch_gemm_cfg<256, 256, GemmEpi::SwiGLU>(g, cdiv(m_bound, 256), s);
    }
    DYLLM_REQUIRE(g.half_n % 64 == 0, "SwiGLU intermediate size must be a multiple of 64");
    return launch_gemm_cfg<128, 128, GemmEpi::SwiGLU>(g, cdiv(m_bound, 128), s);
  }
  if (tile_m == 256) return launch_gemm_cfg<256, 256, GemmEpi::Store>(g, cdiv(m_bound, 256), s);
  return launch_gemm_cfg<128, 128, GemmEpi::Store>(g, cdiv(m_bound, 128), s);
}

}  // namespace dyllm

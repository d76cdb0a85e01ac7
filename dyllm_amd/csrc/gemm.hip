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
//                               (MLPcache.scatter_update, mlp_cache_manage.py:24-40);
//   * split-K                -- for short-M, wide-K products (the down projection of a few
//                               hundred salient rows) the K range is cut into slices whose fp32
//                               partial tiles are summed in slice order by a reduction kernel
//                               that applies the store epilogue (deterministic).
//
// Tiling: workgroup tile BM x 256 x 64, 8 wavefronts (2 per SIMD) in a 2 (M) x 4 (N) grid
// (WGN = 4; a 2 x 2 grid of 1-wave-per-SIMD tiles, and two 4-wave BM x 128 workgroups per CU,
// both measured slower), each wavefront (BM/2) x 64
// of v_mfma_f32_32x32x16_bf16 tiles. Operands move global -> LDS with the gfx950 direct
// LDS-load (buffer_load_dwordx4 ... lds: per-lane row offsets fixed for the tile, the K
// position a scalar offset), no register staging. Operands are staged through
// LDS in unpadded 128-byte rows whose 16-byte chunks are XOR-swizzled by row
// (chunk ^ (row & 7)), so the fragment reads are spread over the banks. A slices (the gathered
// rows, L2-resident) are double-buffered and loaded one slice ahead; W slices (streamed from
// HBM) are triple-buffered and loaded two slices ahead (2*BM*64 + 3*256*64 elements: 144 KB at
// BM = 192, the full 160 KB at 256). One wait + barrier per K slice: vmcnt(4) leaves only the
// newest W loads in flight (32-wide K stages with 4-5 buffers of both operands measured slower). Within a slice the fragment reads of the next 16-wide K
// substep are interleaved one per MFMA with the current substep, pinned with
// sched_group_barrier (the compiler's own schedule clusters the reads and stalls on them;
// 4-8 % with warm caches). The last substep's MFMAs are issued after the slice's barrier, over the first
// fragment reads of the next slice (8-15 % fewer cycles per tile). The MFMA is issued as D = W_tile * A_tile^T
// so that each lane owns one output row and four consecutive output columns per register
// group: 8-byte stores and one row lookup per lane for the scatter. Workgroups are ordered
// M-fastest and remapped XCD-major so the M tiles sharing a weight slice run on one XCD and
// read that slice from HBM once. BM is 128, 192 or 256, picked so the number of tiles
// quantises well onto the 256 CUs.
#include "kernels.h"

#include <cmath>

namespace dyllm {

constexpr int kGemmBK = 64;
constexpr int kGemmBN = 256;

__device__ __forceinline__ float bf16_rt(float x) { return __uint_as_float(uint32_t(f32_to_bf16(x)) << 16); }
__device__ __forceinline__ void bf16x4_to_f32(uint2 v, float* f) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xffff0000u);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8),
// issued through the builtin rather than inline asm so that the compiler's own wait insertion sees
// them (it does not parse inline asm, and would otherwise re-wait on LDS reads already complete)
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int waitcnt_lgkm0() { return 15 | (3 << 14) | (7 << 4); }

// element offset of (row, 16-byte chunk) in a swizzled 64-element-wide tile. gfx950 serves a
// 16-byte LDS read for 16 lanes at a time over 64 banks (two 128-byte rows): the 16 rows a
// fragment read touches must land on distinct (row parity, chunk) pairs, so the chunk is
// XOR-ed with bits 1..3 of the row (measured: zero SQ_LDS_BANK_CONFLICT).
__device__ __forceinline__ int swz_chunk(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * kGemmBK + (swz_chunk(row, chunk) << 3); }

// Source rows of the A blocks a lane loads for M tile mt: the gathered row of each tile row; rows
// past M, padding and out-of-range ids read row 0, whose products are never stored.
template <int BM, int WGN>
__device__ __forceinline__ void gemm_tile_rows(const GemmArgs& g, int64_t M, int mt, int w, int lrow,
                                               int64_t (&rows)[BM / (16 * WGN)]) {
  constexpr int NW = 2 * WGN, CA = BM / (8 * NW);
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int64_t m = int64_t(mt) * BM + (w + NW * i) * 8 + lrow;
    int64_t row = 0;
    if (m < M) {
      row = m;
      if (g.a_ids) {
        const int64_t id = g.a_ids[m];
        row = (id >= 0 && id < g.id_limit) ? id / g.a_div : 0;
        if (g.a_map) row = g.a_map[row];
      }
    }
    rows[i] = row;
  }
}

// One BM x BN output tile (K slice kz of ksplit). The SwiGLU instantiation takes the tile's source
// rows from its caller (rows) and looks up the next tile's (mt_next >= 0, into rows_next) during
// its K loop, so a tile boundary does not wait on the row lookups; the Store instantiation looks
// its rows up itself.
template <int BM, int BN, int WGN, GemmEpi EPI>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, int64_t M, int mt, int nt, int kz,
                                          const int64_t (&rows)[BM / (16 * WGN)], int mt_next,
                                          int64_t (&rows_next)[BM / (16 * WGN)]) {
  extern __shared__ __attribute__((aligned(16))) uint16_t gsm[];
  constexpr int NW = 2 * WGN;                 // wavefronts: 2 along M x WGN along N
  constexpr int WM = BM / 2, WN = BN / WGN;   // wave tile (rows of A, rows of W)
  constexpr int TM = WM / 32, TN = WN / 32;   // 32x32 MFMA tiles per wave
  const int64_t m0 = int64_t(mt) * BM;

  const int tid = threadIdx.x, lane = tid & 63;
  // the wave index in a scalar register: the LDS destinations of the loads are scalar arithmetic
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w & 1, wn = w >> 1;
  constexpr int GW = BN / (2 * WGN);          // SwiGLU: gate (and up) rows per wavefront
  const int l32 = lane & 31, half = lane >> 5;

  const uint16_t* Wb = g.W;
  if (g.tile_expert) Wb += int64_t(g.tile_expert[mt]) * g.w_expert_stride;

  const int nk_total = g.K / kGemmBK;
  const int nk = nk_total / g.ksplit;
  const int k_begin = kz * nk;

  // Direct global->LDS staging: each wavefront fills 1 KB blocks of 8 swizzled rows; lane L
  // of a block lands at byte 16*L, i.e. row L/8, physical chunk L%8, which holds logical
  // chunk swz_chunk(row, L%8) (the XOR is its own inverse). Rows outside the problem
  // (m >= M, padding ids, n >= N) are clamped to a valid row: their products are never stored.
  constexpr int CA = BM / (8 * NW), CW = BN / (8 * NW);  // 1 KB blocks per wavefront per K slice
  const int lrow = lane >> 3;
  // (w + NW * i) * 8 + lrow == lrow (mod 8): the swizzled chunk of a lane is the same in every block
  const int lane_chunk = swz_chunk(w * 8 + lrow, lane & 7) * 8;
  // The loads are buffer loads (buffer_load_dwordx4 ... lds): a scalar resource holds the operand's
  // base at this split-K slice's first column, each lane a fixed 32-bit byte offset of its row and
  // chunk, and the K position of the slice is the scalar offset, so a K slice costs no vector
  // address arithmetic. Offsets are 32-bit: every operand spans less than 4 GiB (checked on the
  // host where the extent is known).
  uint32_t a_vo[CA];
  if (EPI == GemmEpi::SwiGLU || g.tile_expert) {   // rows looked up by the caller (during the previous tile)
#pragma unroll
    for (int i = 0; i < CA; ++i) a_vo[i] = uint32_t((rows[i] * g.lda + lane_chunk) * 2);
  } else {
    int64_t own[CA];
    gemm_tile_rows<BM, WGN>(g, M, mt, w, lrow, own);
#pragma unroll
    for (int i = 0; i < CA; ++i) a_vo[i] = uint32_t((own[i] * g.lda + lane_chunk) * 2);
  }
  uint32_t w_vo[CW];
#pragma unroll
  for (int i = 0; i < CW; ++i) {
    const int r = (w + NW * i) * 8 + lrow;
    int64_t wrow;
    if constexpr (EPI == GemmEpi::SwiGLU)
      wrow = (r < BN / 2) ? int64_t(nt) * (BN / 2) + r : int64_t(g.half_n) + int64_t(nt) * (BN / 2) + (r - BN / 2);
    else
      wrow = int64_t(nt) * BN + r;
    if (wrow >= g.N) wrow = 0;
    w_vo[i] = uint32_t((wrow * g.ldw + lane_chunk) * 2);
  }
  // the resource base must be wave-uniform (a scalar register): the pointer is read from lane 0
  auto uniform_ptr = [](const uint16_t* p) -> void* {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo32 = __builtin_amdgcn_readfirstlane(uint32_t(v)), hi32 = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
    return reinterpret_cast<void*>((uint64_t(hi32) << 32) | lo32);
  };
  // raw buffer (stride 0), range check disabled (num_records = 0xffffffff), gfx9 data format word
  constexpr int kRsrcWord3 = 0x00020000;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(g.A + int64_t(k_begin) * kGemmBK), 0, -1, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(Wb + int64_t(k_begin) * kGemmBK), 0, -1, kRsrcWord3);
  typedef __attribute__((address_space(3))) void lds_void;
  // LDS: A slices double-buffered, W slices (streamed from HBM) triple-buffered so their loads
  // are issued two slices ahead: [A0 | A1 | W0 | W1 | W2]
  uint16_t* const a_lds = gsm;
  uint16_t* const w_lds = gsm + 2 * BM * kGemmBK;
  auto stage_a = [&](int kt, int buf) {
    uint16_t* As = a_lds + buf * (BM * kGemmBK);
#pragma unroll
    for (int i = 0; i < CA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(As + (w + NW * i) * 8 * kGemmBK), 16, int(a_vo[i]),
                                               kt * (kGemmBK * 2), 0, 0);
  };
  auto stage_w = [&](int kt, int buf) {
    uint16_t* Ws = w_lds + buf * (BN * kGemmBK);
#pragma unroll
    for (int i = 0; i < CW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void*)(Ws + (w + NW * i) * 8 * kGemmBK), 16, int(w_vo[i]),
                                               kt * (kGemmBK * 2), 0, 0);
  };

  // W-tile row base of the wave's n-subtile i
  auto wrow_base = [&](int i) -> int {
    if constexpr (EPI == GemmEpi::SwiGLU)
      return (i < TN / 2) ? wn * GW + 32 * i : BN / 2 + wn * GW + 32 * (i - TN / 2);
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

  // Fragments are double-buffered in registers (two named sets so every index stays static):
  // the LDS reads of K-substep ks+1 are issued one by one between the MFMAs of ks. Fragment rows
  // are multiples of 32 plus l32, so the swizzle depends on l32 only: one lane offset per substep
  // (lo), the row base of each fragment an immediate.
  bf16x8_t wf0[TN], af0[TM], wf1[TN], af1[TM];
  int lo[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) lo[ks] = swz(l32, 2 * ks + half);
  auto fload = [&](const uint16_t* As, const uint16_t* Ws, int ks, bf16x8_t* wf, bf16x8_t* af) {
    const uint16_t* wp = Ws + lo[ks];
    const uint16_t* ap = As + wm * WM * kGemmBK + lo[ks];
#pragma unroll
    for (int i = 0; i < TN; ++i) wf[i] = *reinterpret_cast<const bf16x8_t*>(wp + wrow_base(i) * kGemmBK);
#pragma unroll
    for (int j = 0; j < TM; ++j) af[j] = *reinterpret_cast<const bf16x8_t*>(ap + 32 * j * kGemmBK);
  };
  auto mma = [&](const bf16x8_t* wf, const bf16x8_t* af) {
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], af[j], acc[i][j], 0, 0, 0);
  };
  // the TN+TM LDS reads of the next substep spread evenly over this substep's TN*TM MFMAs
  // (one read after every RS MFMAs), then the remaining MFMAs
  constexpr int RS = (TN * TM) / (TN + TM) > 0 ? (TN * TM) / (TN + TM) : 1;
  auto interleave = [&]() {
#pragma unroll
    for (int r = 0; r < TN + TM; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, RS, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int r = (TN + TM) * RS; r < TN * TM; ++r) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  };

  // The per-slice synchronisation is an s_barrier preceded by explicit waits, not
  // __syncthreads(): before it each wave waits for its own LDS reads of the current buffer
  // (lgkmcnt, so no wave refills a buffer still being read) and for its own direct-to-LDS loads of
  // the next slice (vmcnt, so the slice is complete for every wave after the barrier). That is all
  // the LDS ping-pong needs; the workgroup-scope fences of __syncthreads() cost 2-4 % of the step.
  // Loads complete in issue order, so vmcnt(CW) at the end of slice kt leaves only the W loads
  // of slice kt+2 (issued last) in flight: A and W of slice kt+1 have landed.
  static_assert(CW == 4 || CW == 6 || CW == 8, "vmcnt immediates below cover 4, 6 or 8 W blocks per wavefront");
  auto wait_w_in_flight = [&]() {   // vmcnt(CW): only the newest CW loads (W of slice kt+2) in flight
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(CW));
  };
  stage_a(0, 0);
  stage_w(0, 0);
  if (nk > 1) {
    stage_w(1, 1);
    wait_w_in_flight();
  } else {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
  __builtin_amdgcn_s_barrier();
  // the next tile's source rows: issued before every load of the K loop, so the loop's vmcnt
  // waits complete them as well
  if (mt_next >= 0) gemm_tile_rows<BM, WGN>(g, M, mt_next, w, lrow, rows_next);
  int wcur = 0;   // kt % 3
  // The last K substep of each slice is carried across the slice's barrier: its fragments are
  // read before the barrier and its MFMAs issued after it, while the first fragment reads of the
  // next slice are in flight, so the MFMA pipe does not idle through the barrier and the reads.
  fload(a_lds, w_lds, 0, wf0, af0);
  for (int kt = 0; kt < nk; ++kt) {
    const uint16_t* As = a_lds + (kt & 1) * (BM * kGemmBK);
    const uint16_t* Ws = w_lds + wcur * (BN * kGemmBK);
    const int wnext2 = wcur == 0 ? 2 : wcur - 1;   // (kt + 2) % 3
    // raised wave priority over the slice's MFMA stretch: the SIMD's arbiter then favours a
    // wave issuing MFMAs over its partner wave issuing loads
    __builtin_amdgcn_s_setprio(1);
    if (kt > 0) mma(wf1, af1);   // substep 3 of slice kt-1
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < nk) stage_a(kt + 1, (kt & 1) ^ 1);
    __builtin_amdgcn_sched_barrier(0);
    fload(As, Ws, 1, wf1, af1);
    mma(wf0, af0);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    // the weight loads after the first substep's MFMAs (issued last: the vmcnt wait below
    // leaves exactly them in flight)
    if (kt + 2 < nk) stage_w(kt + 2, wnext2);
    __builtin_amdgcn_sched_barrier(0);
    fload(As, Ws, 2, wf0, af0);
    mma(wf1, af1);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    fload(As, Ws, 3, wf1, af1);
    mma(wf0, af0);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    // this wave's LDS reads of the slice (substep 3 included) are done before any wave
    // refills its buffers
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm0());
    if (kt + 2 < nk) {
      wait_w_in_flight();
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
    __builtin_amdgcn_s_barrier();
    wcur = wcur == 2 ? 0 : wcur + 1;
    if (kt + 1 < nk) fload(a_lds + ((kt + 1) & 1) * (BM * kGemmBK), w_lds + wcur * (BN * kGemmBK), 0, wf0, af0);
    __builtin_amdgcn_sched_barrier(0);
  }
  mma(wf1, af1);

  // ---- epilogue: lane owns row m = m0 + wm*WM + 32j + l32 -------------------------------
  if constexpr (EPI == GemmEpi::Store) {
    if (g.partial) {  // split-K slice: raw fp32 partial tile
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const int64_t m = m0 + wm * WM + 32 * j + l32;
        float* prow = g.partial + (int64_t(kz) * g.m_pad + m) * g.N;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = nt * BN + wn * WN + 32 * i + half * 4 + q * 8;
            if (n >= g.N) continue;
            *reinterpret_cast<float4*>(prow + n) =
                make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          }
      }
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int64_t m = m0 + wm * WM + 32 * j + l32;
    if (m >= M) continue;
    int64_t drow = m;
    int64_t id = m;
    if (g.a_ids) {
      id = g.a_ids[m];
      if (id < 0 || id >= g.id_limit) continue;
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
        const int hc0 = nt * (BN / 2) + wn * GW + 32 * i + half * 4;
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
          float bv[4] = {0.f, 0.f, 0.f, 0.f};
          if (g.bias) bf16x4_to_f32(*reinterpret_cast<const uint2*>(g.bias + n), bv);
          uint2 st;
          st.x = pack_bf16x2(acc[i][j][4 * q] * scale + bv[0], acc[i][j][4 * q + 1] * scale + bv[1]);
          st.y = pack_bf16x2(acc[i][j][4 * q + 2] * scale + bv[2], acc[i][j][4 * q + 3] * scale + bv[3]);
          *reinterpret_cast<uint2*>(crow + n) = st;
        }
      }
    }
  }
}

// Persistent launch: one workgroup per CU loops over the output tiles. The number of tiles can
// come from device memory (num_m_dev: the salient count written by the compaction kernel), so
// the GEMM is enqueued without the host knowing M. Workgroup b runs on XCD b % 8; the columns
// (split-K slice, N tile) are split into 8 contiguous ranges, one per XCD, and the M tiles that
// share a weight slice run together on one XCD, so they read it from HBM once:
//   * grouped (SwiGLU GEMM, when the M tiles of one column fit the XCD's workgroups and this
//     takes no more rounds): the XCD's workgroups form groups of as many as there are M tiles; member i of a
//     group always computes M tile i, and a group walks its share of the XCD's columns. The M
//     tiles of a column start together and stream its weight slice in step (one HBM read of it,
//     the others hitting L2), and a workgroup's gathered A rows never change;
//   * M-split (the expert-grouped GEMMs always; the dense ones when it leaves the busiest XCD
//     fewer tiles): each XCD takes a contiguous eighth of the M tiles with all their columns,
//     columns fastest;
//   * otherwise the XCD's tiles in order (M fastest, then N tile, then split-K slice), one per
//     workgroup per round.
struct TileWalk {
  bool grouped, msplit;
  int mtr, n_tiles;
  int64_t t, t_end, stride;   // linear walk: tiles t, t + stride, ... < t_end
  int member;                 // grouped walk: fixed M tile, columns t, t + stride, ... < t_end
  int64_t m_lo, ncols;        // M-split walk: the XCD's M tiles from m_lo, columns fastest
  __device__ __forceinline__ bool valid() const { return t < t_end; }
  __device__ __forceinline__ int mt(int64_t u) const {
    return msplit ? int(m_lo + u / ncols) : (grouped ? member : int(u % mtr));
  }
  __device__ __forceinline__ int64_t col(int64_t u) const { return msplit ? u % ncols : (grouped ? u : u / mtr); }
};

// Expert-grouped GEMMs: each XCD takes a contiguous eighth of the M tiles (consecutive experts'
// buckets) with all their columns, columns fastest, so an M tile's gathered rows are read into
// that XCD's L2 once for all its N tiles and each expert's weights are read by one or two XCDs.
__device__ __forceinline__ TileWalk tile_walk_msplit(int64_t mtr, int n_tiles, int ksplit, int P) {
  TileWalk w{};
  w.msplit = true;
  w.mtr = int(mtr);
  w.n_tiles = n_tiles;
  w.ncols = int64_t(n_tiles) * ksplit;
  const int x = blockIdx.x & 7, local = blockIdx.x >> 3, nloc = P >> 3;
  w.m_lo = mtr * x / 8;
  w.t = local;
  w.t_end = (mtr * (x + 1) / 8 - w.m_lo) * w.ncols;
  w.stride = nloc;
  return w;
}

__device__ __forceinline__ TileWalk tile_walk(int64_t mtr, int n_tiles, int ksplit, int P, bool allow_grouped) {
  TileWalk w{};
  w.mtr = int(mtr);
  w.n_tiles = n_tiles;
  const int64_t ncols = int64_t(n_tiles) * ksplit;
  const int64_t total = mtr * ncols;
  if ((P & 7) != 0) {
    w.t = blockIdx.x;
    w.t_end = total;
    w.stride = P;
    return w;
  }
  const int x = blockIdx.x & 7, local = blockIdx.x >> 3, nloc = P >> 3;
  const int64_t c_lo = ncols * x / 8, c_hi = ncols * (x + 1) / 8;
  const int64_t groups = mtr > 0 ? nloc / mtr : 0;
  // rounds of the XCD's busiest range either way
  const int64_t cols_max = cdiv(ncols, 8);
  if (allow_grouped && groups > 0 && cdiv(cols_max, groups) <= cdiv(cols_max * mtr, nloc)) {
    w.grouped = true;
    const int64_t grp = local / mtr;
    w.member = int(local % mtr);
    w.t = grp < groups ? c_lo + grp : c_hi;
    w.t_end = c_hi;
    w.stride = groups;
  } else {
    w.t = c_lo * mtr + local;
    w.t_end = c_hi * mtr;
    w.stride = nloc;
  }
  return w;
}

template <int BM, int BN, int WGN, GemmEpi EPI>
__global__ __launch_bounds__(128 * WGN) __attribute__((amdgpu_waves_per_eu(WGN == 2 ? 1 : 2, WGN == 2 ? 1 : 2)))
void gemm_kernel(GemmArgs g) {
  const int64_t M = g.num_m_dev ? min(int64_t(g.num_m_dev[0]), g.M) : g.M;   // never past the host capacity
  const int n_tiles = (EPI == GemmEpi::SwiGLU) ? (g.half_n / (BN / 2)) : int(cdiv(g.N, BN));
  // grouped walks for the SwiGLU GEMM only: measured on the Store GEMMs (down projection with
  // split-K, K/V projection) they were 1-3 % slower, while the gate_up GEMM keeps its time and
  // fetches 5 % less from HBM
  // the dense GEMMs take the M-split walk too when it leaves the busiest XCD fewer tiles than
  // the column ranges do (e.g. 14 columns over 8 XCDs: ranges of 2 columns x all M tiles
  // overflow 28 workgroups per XCD into a second round, eighths of the M tiles do not)
  const int64_t m_tiles = cdiv(M, BM), cols = int64_t(n_tiles) * g.ksplit;
  const bool msplit = (gridDim.x & 7) == 0 &&
                      (g.tile_expert != nullptr ||
                       (cdiv(m_tiles, 8) * cols < cdiv(cols, 8) * m_tiles));
  const TileWalk tw = msplit
                          ? tile_walk_msplit(m_tiles, n_tiles, g.ksplit, gridDim.x)
                          : tile_walk(m_tiles, n_tiles, g.ksplit, gridDim.x, EPI == GemmEpi::SwiGLU);
  constexpr int CA = BM / (16 * WGN);
  int64_t rows[CA], rows_next[CA];
  // the SwiGLU and the expert-grouped GEMMs look each tile's source rows up during the previous
  // tile's K loop (the dense Store GEMMs measured 2-5 % slower with it and look them up per tile)
  const bool row_ahead = EPI == GemmEpi::SwiGLU || g.tile_expert != nullptr;
  if (row_ahead) {
    if (tw.valid())
      gemm_tile_rows<BM, WGN>(g, M, tw.mt(tw.t), __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6),
                              (threadIdx.x & 63) >> 3, rows);
  }
  for (int64_t u = tw.t; u < tw.t_end; u += tw.stride) {
    const int mt = tw.mt(u);
    const int64_t c = tw.col(u);
    const int nt = int(c % n_tiles);
    const int kz = int(c / n_tiles);
    // the SwiGLU tile looks the next tile's source rows up during its K loop (grouped walks keep
    // one M tile, whose rows are already in place)
    const int mt_next = (row_ahead && !tw.grouped && u + tw.stride < tw.t_end) ? tw.mt(u + tw.stride) : -1;
    gemm_tile<BM, BN, WGN, EPI>(g, M, mt, nt, kz, rows, mt_next, rows_next);
    if (mt_next >= 0) {
#pragma unroll
      for (int i = 0; i < CA; ++i) rows[i] = rows_next[i];
    }
  }
}

// Sum of the split-K slices in slice order, then the store epilogue (row remap, row scale,
// bf16). One thread per 4 output columns.
__global__ __launch_bounds__(256) void gemm_partial_reduce_kernel(GemmArgs g) {
  const int64_t M = g.num_m_dev ? min(int64_t(g.num_m_dev[0]), g.M) : g.M;
  const int nq = g.N / 4;
  for (int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x; t < M * nq; t += int64_t(gridDim.x) * 256) {
    const int64_t m = t / nq;
    const int n = int(t - m * nq) * 4;
    int64_t drow = m, id = m;
    if (g.a_ids) {
      id = g.a_ids[m];
      if (id < 0 || id >= g.id_limit) continue;
      if (g.c_by_id) drow = id;
    }
    if (g.c_rows) drow = g.c_rows[m];
    float scale = 1.0f;
    if (g.row_scale_f32) scale = g.row_scale_f32[id];
    if (g.row_scale_bf16) scale = bf16_to_f32(g.row_scale_bf16[id]);
    float4 s = *reinterpret_cast<const float4*>(g.partial + m * g.N + n);
    for (int z = 1; z < g.ksplit; ++z) {
      const float4 v = *reinterpret_cast<const float4*>(g.partial + (int64_t(z) * g.m_pad + m) * g.N + n);
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (g.bias) bf16x4_to_f32(*reinterpret_cast<const uint2*>(g.bias + n), bv);
    uint2 st;
    st.x = pack_bf16x2(s.x * scale + bv[0], s.y * scale + bv[1]);
    st.y = pack_bf16x2(s.z * scale + bv[2], s.w * scale + bv[3]);
    *reinterpret_cast<uint2*>(g.Cout + drow * g.ldc + n) = st;
  }
}

static int num_cus() {
  static int n = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    return v;
  }();
  return n;
}

static constexpr size_t lds_bytes(int bm, int bn) { return size_t(2 * bm + 3 * bn) * kGemmBK * sizeof(uint16_t); }

template <int BM, int BN, int WGN, GemmEpi EPI>
static int launch_gemm_cfg(const GemmArgs& g0, int64_t m_tiles, int ksplit, hipStream_t s) {
  GemmArgs g = g0;
  g.ksplit = ksplit;
  g.m_pad = m_tiles * BM;
  const int n_tiles = (EPI == GemmEpi::SwiGLU) ? (g.half_n / (BN / 2)) : int(cdiv(g.N, BN));
  const int64_t tiles = m_tiles * n_tiles * ksplit;
  if (tiles == 0) return 0;
  // a multiple of 8 workgroups (one range per XCD), rounded up: with fewer tiles than CUs every
  // workgroup then takes at most one tile (rounding down would push the last few tiles into a
  // second round), the workgroups past a range's end exit at once
  int64_t nwg = tiles < num_cus() ? tiles : num_cus();
  if (nwg >= 8) nwg = std::min<int64_t>(cdiv(nwg, 8) * 8, std::max(8, num_cus() & ~7));
  const size_t lds = lds_bytes(BM, BN);
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<BM, BN, WGN, EPI>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) != hipSuccess)
      return fail("hipFuncSetAttribute(max dynamic LDS) failed for the GEMM kernel");
    attr_set = true;
  }
  gemm_kernel<BM, BN, WGN, EPI><<<unsigned(nwg), 128 * WGN, lds, s>>>(g);
  if (int rc = check_launch("gemm_kernel")) return rc;
  if (ksplit > 1) {
    const int64_t threads = m_tiles * BM * (g.N / 4);
    const int64_t blocks = cdiv(threads, 256) < 4 * num_cus() ? cdiv(threads, 256) : 4 * num_cus();
    gemm_partial_reduce_kernel<<<unsigned(blocks), 256, 0, s>>>(g);
    return check_launch("gemm_partial_reduce_kernel");
  }
  return 0;
}

// Tile height and split-K choice from a cost model fitted to MI355X measurements of both
// projections (cold caches; hidden 3584 / 4096, intermediate 12288 / 18944, M = 128 ... 6144):
//   rounds  = ceil(tiles / CUs), work = tile_m * (K / ksplit) / 1e6 (per tile, K-elements x rows)
//   Store:  t = 125.5 rounds*work + 38.9 rounds*work*[tile_m == 128] + 1.8 rounds
//               + 1706 ksplit*M*N / 1e9   (split-K partial traffic + reduction, only if ksplit > 1)
//   SwiGLU: t = 71.0 rounds*work + 40.4 rounds
// (microseconds). Over the measured grid the model's pick is within 4 % of the best measured
// configuration in total.
static double plan_cost(int64_t M, int N, int K, GemmEpi epi, int bm, int ks) {
  const double cus = double(num_cus());
  const int64_t n_tiles = (epi == GemmEpi::SwiGLU) ? cdiv(N / 2, kGemmBN / 2) : cdiv(N, kGemmBN);
  const double tiles = double(cdiv(M, bm) * n_tiles * ks);
  const double rounds = std::ceil(tiles / cus);
  const double work = double(bm) * (double(K) / ks) / 1e6;
  if (epi == GemmEpi::SwiGLU) return 71.0 * rounds * work + 40.4 * rounds;
  double t = 125.5 * rounds * work + (bm == 128 ? 38.9 * rounds * work : 0.0) + 1.8 * rounds;
  if (ks > 1) t += 1706.0 * double(ks) * double(M) * double(N) / 1e9;
  return t;
}

GemmPlan gemm_plan(int64_t M, int N, int K, GemmEpi epi) {
  GemmPlan best{256, 1};
  double best_cost = 1e300;
  const int nk = K / kGemmBK;
  for (int bm : {256, 192, 128}) {
    for (int ks : {1, 2, 3, 4, 6, 8}) {
      if (ks > 1 && (epi != GemmEpi::Store || nk % ks != 0 || nk / ks < 4)) continue;
      const double c = plan_cost(M < 1 ? 1 : M, N, K, epi, bm, ks);
      if (c < best_cost - 1e-9) {
        best_cost = c;
        best = GemmPlan{bm, ks};
      }
    }
  }
  return best;
}

size_t gemm_partial_bytes(int64_t m_bound, int N, int tile_m, int ksplit) {
  if (ksplit <= 1) return 0;
  return size_t(ksplit) * size_t(cdiv(m_bound, tile_m) * tile_m) * size_t(N) * sizeof(float);
}

// m_bound: host-side upper bound of M (number of BM tiles launched = cdiv(m_bound, BM)).
int launch_gemm(GemmEpi epi, const GemmArgs& g, int64_t m_bound, int tile_m, int ksplit, hipStream_t s) {
  DYLLM_REQUIRE(g.K > 0 && g.K % kGemmBK == 0, "GEMM K must be a positive multiple of 64");
  DYLLM_REQUIRE(g.N > 0 && g.N % 8 == 0, "GEMM N must be a positive multiple of 8");
  DYLLM_REQUIRE(g.lda % 8 == 0 && g.ldw % 8 == 0 && g.ldc % 4 == 0, "GEMM leading dimensions must keep 16-byte rows");
  // 32-bit byte offsets inside one operand (the buffer loads of the tile): the weight (one expert's
  // block for the grouped GEMM) always, A when the caller states its row count
  DYLLM_REQUIRE(int64_t(g.N) * g.ldw * 2 <= (int64_t(1) << 32), "GEMM weight must span less than 4 GiB");
  DYLLM_REQUIRE(g.a_rows <= 0 || g.a_rows * g.lda * 2 <= (int64_t(1) << 32), "GEMM input rows must span less than 4 GiB");
  DYLLM_REQUIRE(reinterpret_cast<uintptr_t>(g.A) % 16 == 0 && reinterpret_cast<uintptr_t>(g.W) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(g.Cout) % 8 == 0 && reinterpret_cast<uintptr_t>(g.bias) % 8 == 0,
                "GEMM operands must be 16-byte aligned (output and bias 8-byte)");
  if (m_bound <= 0) return 0;
  if (tile_m == 0) tile_m = gemm_plan(m_bound, g.N, g.K, epi).tile_m;
  DYLLM_REQUIRE(tile_m == 128 || tile_m == 192 || tile_m == 256, "tile height must be 128, 192 or 256");
  if (ksplit < 1) ksplit = 1;
  DYLLM_REQUIRE((g.K / kGemmBK) % ksplit == 0, "split-K must divide the number of 64-wide K slices");
  DYLLM_REQUIRE(ksplit == 1 || (epi == GemmEpi::Store && g.partial != nullptr), "split-K needs a partial buffer");
  const int64_t mt = cdiv(m_bound, tile_m);
  if (epi == GemmEpi::SwiGLU) {
    DYLLM_REQUIRE(g.N == 2 * g.half_n, "SwiGLU weight must hold gate rows then up rows (N = 2 * intermediate)");
    DYLLM_REQUIRE(g.half_n % (kGemmBN / 2) == 0, "SwiGLU intermediate size must be a multiple of 128");
    if (tile_m == 256) return launch_gemm_cfg<256, 256, 4, GemmEpi::SwiGLU>(g, mt, 1, s);
    if (tile_m == 192) return launch_gemm_cfg<192, 256, 4, GemmEpi::SwiGLU>(g, mt, 1, s);
    return launch_gemm_cfg<128, 256, 4, GemmEpi::SwiGLU>(g, mt, 1, s);
  }
  if (tile_m == 256) return launch_gemm_cfg<256, 256, 4, GemmEpi::Store>(g, mt, ksplit, s);
  if (tile_m == 192) return launch_gemm_cfg<192, 256, 4, GemmEpi::Store>(g, mt, ksplit, s);
  return launch_gemm_cfg<128, 256, 4, GemmEpi::Store>(g, mt, ksplit, s);
}

}  // namespace dyllm

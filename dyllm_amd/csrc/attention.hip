// Varlen non-causal attention for head_dim 128 on gfx950 MFMA, in three modes:
//
//   Dense      -- softmax(Q K^T * scale) V for every query row (the full / refresh step,
//                 the flash_attn_varlen_func call at attention.py:41-52).
//   RowSparse  -- the same for a compact list of salient query rows (q_rows) against the
//                 full cached K/V; output is compact (attention.py:76-87).
//   ColSparse  -- O = C + softmax(Q K^T / sqrt(D)) dV with PV only on key groups that hold
//                 salient rows, plus the saliency statistics of every row; salient rows take
//                 o_sal instead (attention_ops_kernels_sm80.cu:44-483 together with
//                 attention_aux_kernels.cu:22-72).
//
// Numerics follow the reference: log2-domain online softmax over 64-key blocks, running max
// initialised to -FLT_MAX, P rounded to bf16 (round to nearest even) relative to the running
// max before the PV product while the row sum stays fp32, 1/rowsum as a correctly rounded
// division, new = C + (acc * inv) without contraction, statistics from the unrounded fp32 new
// values (bf16 o_sal for salient rows).
//
// MI355X layout: a workgroup is NW wavefronts x 32 query rows of one (sequence, head). The
// score tile is computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16 so that lane
// l holds query row l%32: row max / row sum / rescale are lane-local (plus one swap with the
// other half-wave), and the P^T accumulator feeds the PV MFMA (O^T = V^T P^T) as its B
// operand with no data movement. K is staged row-major and V transposed in LDS (rows padded so
// that the fragment reads are bank-conflict free); the next 64-key tile is fetched into
// registers while the current one is multiplied. Workgroups are remapped so that all query
// tiles of one (sequence, kv-head) land on the same XCD and share its L2.
#include "kernels.h"

#include <float.h>

namespace dyllm {

constexpr int kD = 128;
constexpr int kBK = 64;              // keys per block (reference block width)
constexpr int kKStride = kD + 8;     // K tile row stride (elements): 272 B, conflict-free b128 reads
constexpr int kVStride = kBK + 12;   // V^T tile row stride (elements): 152 B, conflict-free b64 reads

// Two-pass column-sparse path (keys in chunks of kMaxBlk2 blocks): LDS it needs beyond
// the K / V^T tiles.
constexpr int kMaxBlk2 = 64;
struct ColSparseLds {
  float* m;          // [NW][kMaxBlk2][32] running max of each query row after each key block
  int16_t* keys;     // [kMaxBlk2 * kBK] salient keys in groups of kGroupSlots<CHUNKED>, -1 = padding
  uint8_t* gblk;     // [8 * kMaxBlk2] key block of each group
  int* ngrp;         // number of groups
  float* xch;        // [NW][96] pass-1 partials exchanged between the waves of a pair (64 sums, 32 maxima)
  // maps built from the compact salient lists (AttnArgs::sal_k):
  unsigned long long* kbits;  // [kMaxBlk2] salient-key bits of the chunk's blocks
  int* sblk;                  // [kMaxBlk2] dV row of group slot sl in block kb = cu_sal[b] + sblk[kb] + sl
  uint32_t* rowflag;          // [NW] salient bits of the tile's query rows (32 per wavefront)
};

// Key slots per pass-2 group: 16 (v_mfma_f32_32x32x16_bf16 for PV) for rows that fit the LDS max
// table, 8 (v_mfma_f32_32x32x8_bf16, half the keys per product) for the chunked long rows, whose
// sparse blocks hold a few salient keys each (config 4: about 3 per 64-key block), so half-size
// groups halve pass 2's padding: its score recomputation, staging and exponentials.
template <bool CHUNKED>
constexpr int kGroupSlots = CHUNKED ? 8 : 16;

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4_t;

union Pack8 {
  bf16x8_t v;
  uint32_t u[4];
  uint4 q;
};
union Pack4 {
  bf16x4_t v;
  uint32_t u[2];
  uint2 d;
};

__device__ __forceinline__ int xcd_remap(int wg, int nwg) {
  return ((nwg & 7) == 0) ? (wg & 7) * (nwg >> 3) + (wg >> 3) : wg;
}

// One (sequence, head, query tile) of NW*32 rows. wg is the tile index after the XCD remap
// (all query tiles of one (sequence, kv-head) land on the same XCD and share its L2).
template <AttnMode MODE, int NW, bool CHUNKED = false, bool LISTS = false>
__device__ __forceinline__ void attention_tile(const AttnArgs& a, int wg, uint16_t* __restrict__ k_lds,
                                               uint16_t* __restrict__ vt_lds, const ColSparseLds& sp) {
  constexpr int NT = NW * 64;              // threads
  constexpr int BQ = NW * 32;              // query rows per workgroup
  static_assert(MODE != AttnMode::ColSparse || NW % 2 == 0, "the paired pass 1 needs an even number of wavefronts");
  constexpr int KCH = kBK * kD / 8 / NT;   // 16-byte K chunks per thread per tile
  constexpr int VIT = (kBK / 4) * (kD / 8) / NT;  // (4 keys x 8 d) V items per thread per tile

  // ---- tile -> (seq, head, query tile) ----------------------------------------------
  const int tile = wg % a.tiles_per_seq;
  const int head = (wg / a.tiles_per_seq) % a.H;
  const int b = wg / (a.tiles_per_seq * a.H);
  const int kvh = head / (a.H / a.Hkv);

  const int row_beg = a.cu_rows[b], row_end = a.cu_rows[b + 1];
  if (row_beg + tile * BQ >= row_end) return;
  const int k_beg = a.cu_k[b], Lk = a.cu_k[b + 1] - k_beg;
  const int64_t sid = a.seq_ids ? a.seq_ids[b] : 0;
  const int64_t kv0 = a.k_seq_starts ? a.k_seq_starts[sid] : (a.kv_start ? a.kv_start[b] : int64_t(k_beg));
  // salient lists of this sequence (fused step: the column-sparse maps are built from them)
  constexpr bool lists = MODE == AttnMode::ColSparse && LISTS;
  constexpr int GS = kGroupSlots<CHUNKED>;   // pass-2 key slots per group
  const int s_beg = lists ? a.cu_sal[b] : 0, s_end = lists ? a.cu_sal[b + 1] : 0;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ql = lane & 31, half = lane >> 5;
  const int row = row_beg + tile * BQ + w * 32 + ql;  // compact row of this lane
  const bool row_ok = row < row_end;
  // Waves whose 32 rows all lie past the sequence's last row (the tail tile of a sequence) take
  // part in the tile's staging and barriers only: their scores and accumulators would be discarded
  // by the row-guarded epilogue, so skipping them frees the SIMD for the co-resident workgroup.
  const bool wave_live = __builtin_amdgcn_readfirstlane(int(row_beg + tile * BQ + w * 32 < row_end)) != 0;
  int64_t qrow = row;
  if constexpr (MODE == AttnMode::RowSparse) qrow = row_ok ? a.q_rows[row] : 0;

  const int ldq = a.H * kD, ldkv = a.Hkv * kD;

  // ---- Q fragments (B operand of S^T = K Q^T), held for the whole key loop ----------
  bf16x8_t qf[8];
  {
    const uint16_t* qp = a.Q + qrow * ldq + head * kD + half * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      Pack8 p;
      p.q = row_ok ? *reinterpret_cast<const uint4*>(qp + 16 * s) : make_uint4(0, 0, 0, 0);
      qf[s] = p.v;
    }
  }

  f32x16_t o_acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.f;
  float m_run = -FLT_MAX, l_run = 0.f;
  const float c2 = a.scale_log2;

  const uint16_t* Kb = a.K + kv0 * ldkv + kvh * kD;
  const int64_t v0 = (a.kslot || lists) ? 0 : (a.v_seq_starts ? a.v_seq_starts[sid] : (a.v_start ? a.v_start[b] : kv0));
  const uint16_t* Vb = a.V + v0 * ldkv + kvh * kD;
  const int32_t* ks_b = a.kslot ? a.kslot + k_beg : nullptr;
  const int nkb = (Lk + kBK - 1) / kBK;

  // register stage of one K/V tile. The per-block metadata (salient-key bits, compact dV slot
  // of each key) is loaded one block before the tile it addresses (into the registers the
  // previous fetch has just consumed), so the dependent V loads are issued without waiting.
  uint4 kreg[KCH];
  uint4 vreg[VIT][4];
  uint64_t mask_next = ~0ull;
  uint64_t meta_bm = ~0ull;
  int meta_slot[VIT][4];
  auto load_meta = [&](int kb) {
    if constexpr (MODE != AttnMode::ColSparse) return;
    if (kb >= nkb) return;
    const int key0 = kb * kBK;
    if constexpr (MODE == AttnMode::ColSparse) meta_bm = a.kmask[int64_t(b) * a.nblk + kb];
#pragma unroll
    for (int it = 0; it < VIT; ++it) {
      const int kq = (tid + NT * it) & 15;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = key0 + 4 * kq + j;
        meta_slot[it][j] = (r >= Lk) ? -1 : (ks_b ? ks_b[r] : r);
      }
    }
  };
  auto fetch = [&](int kb) {
    const int key0 = kb * kBK;
    const uint64_t bm = meta_bm;
    mask_next = bm;
    if (MODE != AttnMode::ColSparse && key0 + kBK <= Lk) {
      // dense V and a full block (block-uniform branch): no per-row guards or zero fills
      // (dense -4 %, row-sparse -10 %; the column-sparse tiles keep one path, which measured
      // faster there)
#pragma unroll
      for (int it = 0; it < KCH; ++it) {
        const int c = tid + NT * it;
        const int key = c >> 4, dc = c & 15;
        kreg[it] = *reinterpret_cast<const uint4*>(Kb + int64_t(key0 + key) * ldkv + dc * 8);
      }
      if (bm != 0) {
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
          const int c = tid + NT * it;
          const int dc = c >> 4;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t r = key0 + 4 * ((tid + NT * it) & 15) + j;
            vreg[it][j] = *reinterpret_cast<const uint4*>(Vb + r * ldkv + dc * 8);
          }
        }
      }
      return;
    }
#pragma unroll
    for (int it = 0; it < KCH; ++it) {
      const int c = tid + NT * it;
      const int key = c >> 4, dc = c & 15;
      kreg[it] = (key0 + key < Lk) ? *reinterpret_cast<const uint4*>(Kb + int64_t(key0 + key) * ldkv + dc * 8)
                                   : make_uint4(0, 0, 0, 0);
    }
    if (bm != 0) {
#pragma unroll
      for (int it = 0; it < VIT; ++it) {
        const int c = tid + NT * it;
        const int dc = c >> 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          int64_t r;
          if constexpr (MODE == AttnMode::ColSparse) {
            r = meta_slot[it][j];
          } else {
            r = key0 + 4 * ((tid + NT * it) & 15) + j;
            if (r >= Lk) r = -1;
          }
          vreg[it][j] = (r >= 0) ? *reinterpret_cast<const uint4*>(Vb + r * ldkv + dc * 8) : make_uint4(0, 0, 0, 0);
        }
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int it = 0; it < KCH; ++it) {
      const int c = tid + NT * it;
      const int key = c >> 4, dc = c & 15;
      *reinterpret_cast<uint4*>(&k_lds[key * kKStride + dc * 8]) = kreg[it];
    }
    if (mask_next != 0) {
#pragma unroll
      for (int it = 0; it < VIT; ++it) {
        const int c = tid + NT * it;
        const int kq = c & 15, dc = c >> 4;
        const uint32_t x[4][4] = {{vreg[it][0].x, vreg[it][0].y, vreg[it][0].z, vreg[it][0].w},
                                  {vreg[it][1].x, vreg[it][1].y, vreg[it][1].z, vreg[it][1].w},
                                  {vreg[it][2].x, vreg[it][2].y, vreg[it][2].z, vreg[it][2].w},
                                  {vreg[it][3].x, vreg[it][3].y, vreg[it][3].z, vreg[it][3].w}};
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
          // d = dc*8 + 2*wd (low halves) and +1 (high halves) for the 4 keys
          uint2 lo, hi;
          lo.x = __builtin_amdgcn_perm(x[1][wd], x[0][wd], 0x05040100u);
          lo.y = __builtin_amdgcn_perm(x[3][wd], x[2][wd], 0x05040100u);
          hi.x = __builtin_amdgcn_perm(x[1][wd], x[0][wd], 0x07060302u);
          hi.y = __builtin_amdgcn_perm(x[3][wd], x[2][wd], 0x07060302u);
          *reinterpret_cast<uint2*>(&vt_lds[(dc * 8 + 2 * wd) * kVStride + 4 * kq]) = lo;
          *reinterpret_cast<uint2*>(&vt_lds[(dc * 8 + 2 * wd + 1) * kVStride + 4 * kq]) = hi;
        }
      }
    }
  };

  bool two_pass = false;
  if constexpr (MODE == AttnMode::ColSparse) two_pass = sp.m != nullptr && (CHUNKED || nkb <= kMaxBlk2);
  if (two_pass) {
    // Two passes instead of PV on every 16-key group that holds a salient key.
    // Pass 1: S = Q K^T over all keys for the running max and row sum only (the same fp32
    // arithmetic as the single-pass loop), recording each block's running max m_kb.
    // Pass 2: only the salient keys, grouped 16 per key block: S recomputed with the same MFMA
    // sequence, P = bf16(exp2(S*c2 - m_kb*c2)) -- the identical bf16 values the single pass
    // feeds its PV -- and O += P dV with the accumulator rescaled from the previous group's
    // block max to this one's (the product of the per-block rescales in one factor).
    // The LDS max table holds kMaxBlk2 blocks (4096 keys); longer sequences are taken in chunks of
    // that many blocks, pass 1 and pass 2 of a chunk before the next chunk's pass 1, with the
    // running maxima, the row sums and pass 2's accumulator (and its rescale chain) carried from
    // chunk to chunk: the same P values and the same accumulation as one chunk would give.
    float* m_tab = sp.m + w * (kMaxBlk2 * 32) + ql;
    auto qk = [&](f32x16_t (&sa)[2], const uint16_t* kt) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sa[t][r] = 0.f;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(&kt[(t * 32 + ql) * kKStride + 16 * s + half * 8]);
          sa[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], sa[t], 0, 0, 0);
        }
      }
    };
    // K rows of one 64-key block into registers: a full block (block-uniform branch) loads without
    // per-row guards or zero fills, the ragged last block guards each row
    auto load_k_block = [&](uint4 (&dst)[KCH], int kb) {
      const int key0 = kb * kBK;
      if (key0 + kBK <= Lk) {
        const uint16_t* kp = Kb + int64_t(key0) * ldkv;
#pragma unroll
        for (int it = 0; it < KCH; ++it) {
          const int c = tid + NT * it;
          dst[it] = *reinterpret_cast<const uint4*>(kp + int64_t(c >> 4) * ldkv + (c & 15) * 8);
        }
        return;
      }
#pragma unroll
      for (int it = 0; it < KCH; ++it) {
        const int c = tid + NT * it;
        const int key = c >> 4, dc = c & 15;
        dst[it] = (key0 + key < Lk) ? *reinterpret_cast<const uint4*>(Kb + int64_t(key0 + key) * ldkv + dc * 8)
                                    : make_uint4(0, 0, 0, 0);
      }
    };
    auto fetch_k = [&](int kb) { load_k_block(kreg, kb); };
    auto stage_k = [&](uint16_t* kt) {
#pragma unroll
      for (int it = 0; it < KCH; ++it) {
        const int c = tid + NT * it;
        const int key = c >> 4, dc = c & 15;
        *reinterpret_cast<uint4*>(&kt[key * kKStride + dc * 8]) = kreg[it];
      }
    };

    // ---- pass 1 ----
    // K double-buffered (the V^T tile, idle in this pass, holds the odd blocks): block kb+1 is
    // staged while block kb is scored, one barrier per block
    static_assert(kBK * kKStride <= kD * kVStride, "V^T tile too small for a K tile");
    if (nkb > 0) fetch_k(0);   // in flight while the group list is built
    // salient-key groups of blocks kb0 .. kb0+nkc-1 from the per-block key bits (wave 0; keys and
    // blocks relative to kb0)
    auto build_groups = [&](int kb0, int nkc) {
      if (w != 0) return;
      int keys_before = 0;   // lists: salient keys of the sequence before this chunk
      if constexpr (lists) {
        // the chunk's salient-key bits (and, for the first chunk, the tile's salient query rows)
        // from the sequence's list segment, in LDS; one wavefront, so no barrier is needed
        if (lane < nkc) sp.kbits[lane] = 0;
        if (kb0 == 0 && lane < NW) sp.rowflag[lane] = 0;
        __threadfence_block();
        const int key_lo = kb0 * kBK, key_hi = min(Lk, (kb0 + nkc) * kBK);
        const int r0 = row_beg + tile * BQ;
        for (int i0 = s_beg; i0 < s_end; i0 += 64) {
          const int i = i0 + lane;
          bool bef = false;
          if (i < s_end) {
            const int key = a.sal_k[i] - k_beg;
            if (key >= key_lo && key < key_hi) atomicOr(&sp.kbits[(key - key_lo) >> 6], 1ull << (key & 63));
            bef = key >= 0 && key < key_lo;
            if (kb0 == 0) {
              const int r = a.sal_q[i] - r0;
              if (r >= 0 && r < BQ) atomicOr(&sp.rowflag[r >> 5], 1u << (r & 31));
            }
          }
          keys_before += __popcll(__ballot(bef));
        }
        __threadfence_block();
      }
      uint64_t word = 0;
      int grp = 0;
      if (lane < nkc) {
        word = lists ? sp.kbits[lane] : a.kmask[int64_t(b) * a.nblk + kb0 + lane];
        if (kb0 + lane == nkb - 1 && (Lk & (kBK - 1))) word &= (1ull << (Lk & (kBK - 1))) - 1;   // keys < Lk only
        grp = (__popcll(word) + GS - 1) / GS;
      }
      int inc = grp;
      int pinc = __popcll(word);
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(inc, o, 64);
        const int pv = __shfl_up(pinc, o, 64);
        if (lane >= o) {
          inc += v;
          pinc += pv;
        }
      }
      const int g0 = inc - grp;
      if (lane == 63) *sp.ngrp = inc;
      // dV row of group slot sl of this block: the key's rank among the sequence's salient keys
      if (lists && lane < nkc) sp.sblk[lane] = keys_before + (pinc - __popcll(word)) - GS * g0;
      int n = 0;
      while (word) {
        sp.keys[g0 * GS + n] = int16_t(lane * kBK + __builtin_ctzll(word));
        word &= word - 1;
        ++n;
      }
      for (; n < grp * GS; ++n) sp.keys[g0 * GS + n] = -1;
      for (int j = 0; j < grp; ++j) sp.gblk[g0 + j] = uint8_t(lane);
    };
    // pass 2's accumulator state, carried from chunk to chunk
    float m_prev = -FLT_MAX;
    int blk_prev = -1;
    auto pass2 = [&](int kb0, int ngrp) {
      // ---- pass 2 ---- over the groups of blocks kb0 .. (ngrp groups, read before the barrier
      // that precedes this call)
      constexpr int GPB = kBK / GS;   // groups per 64-slot pass block
      const int npb = (ngrp + GPB - 1) / GPB;
      // slots past the last group (the tail of the last 64-slot block) were never written
      auto slot_key = [&](int sl) -> int {
        const int kr = sl < ngrp * GS ? int(sp.keys[sl]) : -1;
        return kr < 0 ? -1 : kb0 * kBK + kr;
      };
      auto load_meta2 = [&](int pb) {
        if (pb >= npb) return;
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
          const int kq = (tid + NT * it) & 15;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int sl = pb * kBK + 4 * kq + j;
            const int key = slot_key(sl);
            meta_slot[it][j] = key < 0 ? -1 : (lists ? s_beg + sp.sblk[sp.gblk[sl / GS]] + sl : (ks_b ? ks_b[key] : key));
          }
        }
      };
      auto fetch2 = [&](int pb) {
#pragma unroll
        for (int it = 0; it < KCH; ++it) {
          const int c = tid + NT * it;
          const int key = slot_key(pb * kBK + (c >> 4)), dc = c & 15;
          kreg[it] = key >= 0 ? *reinterpret_cast<const uint4*>(Kb + int64_t(key) * ldkv + dc * 8) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int it = 0; it < VIT; ++it) {
          const int dc = (tid + NT * it) >> 4;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t r = meta_slot[it][j];
            vreg[it][j] = (r >= 0) ? *reinterpret_cast<const uint4*>(Vb + r * ldkv + dc * 8) : make_uint4(0, 0, 0, 0);
          }
        }
      };
      mask_next = ~0ull;
      load_meta2(0);
      if (npb > 0) fetch2(0);
      load_meta2(1);
      for (int pb = 0; pb < npb; ++pb) {
        stage();
        __syncthreads();
        if (pb + 1 < npb) fetch2(pb + 1);
        load_meta2(pb + 2);
        if (wave_live) {
        f32x16_t sa[2];
        qk(sa, k_lds);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < 32 / GS; ++u) {
            const int g = pb * GPB + t * (32 / GS) + u;
            if (g >= ngrp) continue;
            const int blkl = __builtin_amdgcn_readfirstlane(int(sp.gblk[g]));
            const int blk = kb0 + blkl;
            const float m_g = m_tab[blkl * 32];
            if (blk != blk_prev) {
              const float f = __builtin_amdgcn_exp2f((m_prev - m_g) * c2);
              // skipped when no row's running maximum moved since the previous group's block (f is
              // exactly 1 on every lane) or nothing is accumulated yet: the same values either way
              if (blk_prev >= 0 && __ballot(f != 1.0f) != 0) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                  for (int r = 0; r < 16; ++r) o_acc[i][r] *= f;
              }
              m_prev = m_g;
              blk_prev = blk;
            }
            const float m2 = m_g * c2;
            if constexpr (GS == 8) {
              // the group's 8 keys are rows 8u .. 8u+7 of the 32-key score half: this lane holds
              // keys 8u + 4*half + 0..3 in registers 4u .. 4u+3, the layout of the 32x32x8 B operand
              Pack4 p;
#pragma unroll
              for (int j = 0; j < 2; ++j) {
                const float e0 = __builtin_amdgcn_exp2f(fmaf(sa[t][4 * u + 2 * j], c2, -m2));
                const float e1 = __builtin_amdgcn_exp2f(fmaf(sa[t][4 * u + 2 * j + 1], c2, -m2));
                p.u[j] = pack_bf16x2(e0, e1);
              }
              const int kofs8 = t * 32 + u * 8 + half * 4;
#pragma unroll
              for (int dt = 0; dt < 4; ++dt) {
                Pack4 va;
                va.d = *reinterpret_cast<const uint2*>(&vt_lds[(dt * 32 + ql) * kVStride + kofs8]);
                o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(s16x4_t, va.d),
                                                                      __builtin_bit_cast(s16x4_t, p.d), o_acc[dt], 0, 0, 0);
              }
              continue;
            } else {
            Pack8 p;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float e0 = __builtin_amdgcn_exp2f(fmaf(sa[t][8 * u + 2 * j], c2, -m2));
              const float e1 = __builtin_amdgcn_exp2f(fmaf(sa[t][8 * u + 2 * j + 1], c2, -m2));
              p.u[j] = pack_bf16x2(e0, e1);
            }
            const int kofs = t * 32 + u * 16 + half * 4;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
              const uint16_t* vr = &vt_lds[(dt * 32 + ql) * kVStride + kofs];
              Pack4 lo, hi;
              lo.d = *reinterpret_cast<const uint2*>(vr);
              hi.d = *reinterpret_cast<const uint2*>(vr + 8);
              Pack8 va;
              va.u[0] = lo.u[0];
              va.u[1] = lo.u[1];
              va.u[2] = hi.u[0];
              va.u[3] = hi.u[1];
              o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va.v, p.v, o_acc[dt], 0, 0, 0);
            }
            }
          }
        }
        __syncthreads();
      }
    };
    if (!CHUNKED || nkb <= kMaxBlk2) {
      if (nkb > 0) fetch_k(0);   // in flight while the group list is built
      build_groups(0, nkb);
      // Wavefronts pair up (w, w^1) over the pair's two 32-row groups, and wave w scores the key
      // blocks of parity w & 1 for both groups: every K fragment read from LDS feeds two MFMAs (half
      // the LDS reads per row, four independent accumulation chains). Each wave keeps a partial
      // (max, sum) per group over its blocks and records each block's own maximum; afterwards the
      // partner's partial is merged through LDS (fp32-rounding-level difference from the
      // sequential sum) and the block maxima are turned into the exact running maxima pass 2 needs.
      // K: blocks 2j and 2j+1 are staged together (K tile and the idle V^T tile), one barrier each.
      const int pg = w ^ 1, par = w & 1;
      // the pair scores both of its groups: it is idle only when both lie past the last row
      const bool pair_live = __builtin_amdgcn_readfirstlane(int(row_beg + tile * BQ + (w & ~1) * 32 < row_end)) != 0;
      bf16x8_t qf2[8];   // the partner group's Q fragments
      {
        const int prow = row_beg + tile * BQ + pg * 32 + ql;
        const uint16_t* qp = a.Q + int64_t(prow) * ldq + head * kD + half * 8;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          Pack8 p;
          p.q = prow < row_end ? *reinterpret_cast<const uint4*>(qp + 16 * s) : make_uint4(0, 0, 0, 0);
          qf2[s] = p.v;
        }
      }
      float* const mt_par = sp.m + pg * (kMaxBlk2 * 32) + ql;
      float pm[2] = {-FLT_MAX, -FLT_MAX}, pl[2] = {0.f, 0.f};   // [own group, partner group]
      uint4 kreg1[KCH];
      auto fetch_k1 = [&](int kb) { load_k_block(kreg1, kb); };
      auto stage_k1 = [&]() {
#pragma unroll
        for (int it = 0; it < KCH; ++it) {
          const int c = tid + NT * it;
          const int key = c >> 4, dc = c & 15;
          *reinterpret_cast<uint4*>(&vt_lds[key * kKStride + dc * 8]) = kreg1[it];
        }
      };
      if (nkb > 1) fetch_k1(1);
      for (int j = 0; 2 * j < nkb; ++j) {
        stage_k(k_lds);
        if (2 * j + 1 < nkb) stage_k1();
        __syncthreads();
        if (2 * j + 2 < nkb) fetch_k(2 * j + 2);
        if (2 * j + 3 < nkb) fetch_k1(2 * j + 3);
        const int kb = 2 * j + par;
        if (kb < nkb && pair_live) {
          const uint16_t* kt = par ? vt_lds : k_lds;
          f32x16_t sa[2][2];   // [group][32-key half]
#pragma unroll
          for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) sa[0][t][r] = sa[1][t][r] = 0.f;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
              const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(&kt[(t * 32 + ql) * kKStride + 16 * s + half * 8]);
              sa[0][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], sa[0][t], 0, 0, 0);
              sa[1][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf2[s], sa[1][t], 0, 0, 0);
            }
          }
          const int key0 = kb * kBK;
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            if (key0 + kBK > Lk) {  // ragged last block only
#pragma unroll
              for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                  const int key = key0 + t * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
                  if (key >= Lk) sa[g][t][r] = -FLT_MAX;
                }
            }
            float bm = sa[g][0][0];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int r = 0; r < 16; ++r) bm = fmaxf(bm, sa[g][t][r]);
            bm = half_swap_max(bm);
            const float m_new = fmaxf(pm[g], bm);
            const float rescale = __builtin_amdgcn_exp2f((pm[g] - m_new) * c2);
            const float m2 = m_new * c2;
            pm[g] = m_new;
            float psum = 0.f;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int r = 0; r < 16; r += 2) {
                const float e0 = __builtin_amdgcn_exp2f(fmaf(sa[g][t][r], c2, -m2));
                const float e1 = __builtin_amdgcn_exp2f(fmaf(sa[g][t][r + 1], c2, -m2));
                psum += e0 + e1;
              }
            pl[g] = pl[g] * rescale + psum;
            if (half == 0) (g == 0 ? m_tab : mt_par)[kb * 32] = bm;   // the block's own maximum
          }
        }
        __syncthreads();
      }
      // merge the partner's partial for this wave's group; running maxima of the group's blocks
      // (the maximum is shared by both half-waves, the sum is per lane: each half holds other keys)
      sp.xch[pg * 96 + lane] = pl[1];
      if (half == 0) sp.xch[pg * 96 + 64 + ql] = pm[1];
      __syncthreads();
      {
        const float mb = sp.xch[w * 96 + 64 + ql], lb = sp.xch[w * 96 + lane];
        m_run = fmaxf(pm[0], mb);
        l_run = pl[0] * __builtin_amdgcn_exp2f((pm[0] - m_run) * c2) + lb * __builtin_amdgcn_exp2f((mb - m_run) * c2);
        if (half == 0) {
          float run = -FLT_MAX;
          for (int kb = 0; kb < nkb; ++kb) {
            run = fmaxf(run, m_tab[kb * 32]);
            m_tab[kb * 32] = run;
          }
        }
      }
      const int ngrp = *sp.ngrp;
      __syncthreads();
      // (the last barrier also ends pass 1's reads of both tiles before pass 2 restages them)
      pass2(0, ngrp);

    } else if constexpr (CHUNKED) {
        // chunked: pass 1 scores one 32-row group per wavefront (no pairing: pass 2's accumulator
        // stays live through the next chunk's pass 1, which leaves no registers for a second group)
        float m_carry = -FLT_MAX;   // running maximum after the previous chunk (half 0 lanes)
        float pm1 = -FLT_MAX, pl1 = 0.f;
        for (int kb0 = 0; kb0 < nkb; kb0 += kMaxBlk2) {
          const int nkc = min(kMaxBlk2, nkb - kb0);
          fetch_k(kb0);
          build_groups(kb0, nkc);
          for (int kbl = 0; kbl < nkc; ++kbl) {
            stage_k(k_lds);
            __syncthreads();
            if (kbl + 1 < nkc) fetch_k(kb0 + kbl + 1);
            if (wave_live) {
            f32x16_t sa[2];
            qk(sa, k_lds);
            const int key0 = (kb0 + kbl) * kBK;
            if (key0 + kBK > Lk) {  // ragged last block only
#pragma unroll
              for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                  const int key = key0 + t * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
                  if (key >= Lk) sa[t][r] = -FLT_MAX;
                }
            }
            float bm = sa[0][0];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int r = 0; r < 16; ++r) bm = fmaxf(bm, sa[t][r]);
            bm = half_swap_max(bm);
            const float m_new = fmaxf(pm1, bm);
            const float rescale = __builtin_amdgcn_exp2f((pm1 - m_new) * c2);
            const float m2 = m_new * c2;
            pm1 = m_new;
            float psum = 0.f;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
              for (int r = 0; r < 16; r += 2) {
                const float e0 = __builtin_amdgcn_exp2f(fmaf(sa[t][r], c2, -m2));
                const float e1 = __builtin_amdgcn_exp2f(fmaf(sa[t][r + 1], c2, -m2));
                psum += e0 + e1;
              }
            pl1 = pl1 * rescale + psum;
            if (half == 0) m_tab[kbl * 32] = bm;   // the block's own maximum
            }
            __syncthreads();
          }
          // the chunk's group count, read before the barrier below (wave 0 rewrites it for the next
          // chunk only after that barrier)
          const int ngrp = *sp.ngrp;
          // running maxima of the chunk's blocks, continuing from the previous chunk
          if (half == 0) {
            float run = m_carry;
            for (int kbl = 0; kbl < nkc; ++kbl) {
              run = fmaxf(run, m_tab[kbl * 32]);
              m_tab[kbl * 32] = run;
            }
            m_carry = run;
          }
          __syncthreads();
          pass2(kb0, ngrp);
        }
        m_run = pm1;
        l_run = pl1;
    }
    // the blocks after the last salient one rescale the accumulator to the final max
    {
      const float f = __builtin_amdgcn_exp2f((m_prev - m_run) * c2);
      if (blk_prev >= 0 && __ballot(f != 1.0f) != 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) o_acc[i][r] *= f;
      }
    }
  }
  if (!two_pass) {
  load_meta(0);
  if (nkb > 0) fetch(0);
  load_meta(1);
  for (int kb = 0; kb < nkb; ++kb) {
    const int key0 = kb * kBK;
    const uint64_t bmask = mask_next;
    stage();
    __syncthreads();
    if (kb + 1 < nkb) fetch(kb + 1);
    load_meta(kb + 2);
    if (wave_live) {

    // ---- S^T = K Q^T for two 32-key tiles --------------------------------------------
    f32x16_t s_acc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s_acc[t][r] = 0.f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(&k_lds[(t * 32 + ql) * kKStride + 16 * s + half * 8]);
        s_acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], s_acc[t], 0, 0, 0);
      }
    }

    // ---- online softmax (lane = query row) ----------------------------------------------
    if (key0 + kBK > Lk) {  // ragged last block only
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + t * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
          if (key >= Lk) s_acc[t][r] = -FLT_MAX;
        }
    }
    float bm = s_acc[0][0];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) bm = fmaxf(bm, s_acc[t][r]);
    bm = half_swap_max(bm);
    const float m_new = fmaxf(m_run, bm);
    const float rescale = __builtin_amdgcn_exp2f((m_run - m_new) * c2);
    const float m2 = m_new * c2;
    m_run = m_new;
    float psum = 0.f;
    bf16x8_t pf[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        Pack8 p;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e0 = __builtin_amdgcn_exp2f(fmaf(s_acc[t][8 * u + 2 * j], c2, -m2));
          const float e1 = __builtin_amdgcn_exp2f(fmaf(s_acc[t][8 * u + 2 * j + 1], c2, -m2));
          psum += e0 + e1;
          p.u[j] = pack_bf16x2(e0, e1);
        }
        pf[t][u] = p.v;
      }
    l_run = l_run * rescale + psum;
    // the accumulator rescale is skipped when no row's maximum moved in this block (rescale is
    // exactly 1 on every lane) and before the first block's products (all zero): the same values
    if (kb > 0 && __ballot(rescale != 1.0f) != 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[i][r] *= rescale;
    }

    // ---- O^T += V^T P^T on the 16-key groups that carry salient rows -----------------
    if (bmask != 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if (((bmask >> (t * 32 + u * 16)) & 0xffffull) == 0) continue;
          const int kofs = t * 32 + u * 16 + half * 4;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) {
            const uint16_t* vr = &vt_lds[(dt * 32 + ql) * kVStride + kofs];
            Pack4 lo, hi;
            lo.d = *reinterpret_cast<const uint2*>(vr);
            hi.d = *reinterpret_cast<const uint2*>(vr + 8);
            Pack8 va;
            va.u[0] = lo.u[0];
            va.u[1] = lo.u[1];
            va.u[2] = hi.u[0];
            va.u[3] = hi.u[1];
            o_acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va.v, pf[t][u], o_acc[dt], 0, 0, 0);
          }
        }
    }
    }
    __syncthreads();
  }
  }

  // ---- epilogue ---------------------------------------------------------------------------
  const float l_tot = half_swap_sum(l_run);
  const float inv = 1.0f / l_tot;
  if constexpr (MODE == AttnMode::RowSparse) {
    if (a.cu_q) {
      // fused step: the salient row's final output. O[qrow] = bf16(o), the context cache row
      // rewritten, statistics from the bf16 output vs the cached row (attention_aux_kernels.cu:22-72)
      float dot = 0.f, nn = 0.f, oo = 0.f;
      if (row_ok) {
        const int64_t crow = (a.c_seq_starts ? a.c_seq_starts[sid] + (Lk - (a.cu_q[b + 1] - a.cu_q[b])) : a.c_start[b]) +
                             (qrow - a.cu_q[b]);
        uint16_t* cp = const_cast<uint16_t*>(a.C) + crow * ldq + head * kD + half * 4;
        uint16_t* op = a.O + qrow * ldq + head * kD + half * 4;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int off = dt * 32 + g * 8;
            const uint2 cv = *reinterpret_cast<const uint2*>(cp + off);
            const float old[4] = {__uint_as_float(cv.x << 16), __uint_as_float(cv.x & 0xffff0000u),
                                  __uint_as_float(cv.y << 16), __uint_as_float(cv.y & 0xffff0000u)};
            uint2 st;
            st.x = pack_bf16x2(o_acc[dt][4 * g] * inv, o_acc[dt][4 * g + 1] * inv);
            st.y = pack_bf16x2(o_acc[dt][4 * g + 2] * inv, o_acc[dt][4 * g + 3] * inv);
            const float nw[4] = {__uint_as_float(st.x << 16), __uint_as_float(st.x & 0xffff0000u),
                                 __uint_as_float(st.y << 16), __uint_as_float(st.y & 0xffff0000u)};
            *reinterpret_cast<uint2*>(op + off) = st;
            if (a.c_inplace) *reinterpret_cast<uint2*>(cp + off) = st;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              dot += nw[j] * old[j];
              nn += nw[j] * nw[j];
              oo += old[j] * old[j];
            }
          }
      }
      dot = half_swap_sum(dot);
      nn = half_swap_sum(nn);
      oo = half_swap_sum(oo);
      if (row_ok && half == 0) {
        a.part[(int64_t(head) * 3 + 0) * a.Tq + qrow] = dot;
        a.part[(int64_t(head) * 3 + 1) * a.Tq + qrow] = nn;
        a.part[(int64_t(head) * 3 + 2) * a.Tq + qrow] = oo;
      }
      return;
    }
  }
  if constexpr (MODE != AttnMode::ColSparse) {
    if (!row_ok) return;
    uint16_t* op = a.O + int64_t(row) * ldq + head * kD + half * 4;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 st;
        st.x = pack_bf16x2(o_acc[dt][4 * g] * inv, o_acc[dt][4 * g + 1] * inv);
        st.y = pack_bf16x2(o_acc[dt][4 * g + 2] * inv, o_acc[dt][4 * g + 3] * inv);
        *reinterpret_cast<uint2*>(op + dt * 32 + g * 8) = st;
      }
  } else {
    float dot = 0.f, nn = 0.f, oo = 0.f;
    int slot;
    if constexpr (lists)   // fused step: only whether the row is salient matters (its row-sparse tile finishes it)
      slot = (row_ok && ((sp.rowflag[w] >> ql) & 1u)) ? 0 : -1;
    else
      slot = row_ok ? a.sal_slot[row] : -1;
    // salient rows are finished by the row-sparse tiles of the fused step (every lane stays for
    // the half-wave reductions below)
    const bool own = row_ok && !(a.skip_salient && slot >= 0);
    if (own) {
      const int64_t crow = a.c_seq_starts ? a.c_seq_starts[sid] + (Lk - (row_end - row_beg)) + (row - row_beg)
                                          : (a.c_start ? a.c_start[b] + (row - row_beg) : int64_t(row));
      uint16_t* cp = const_cast<uint16_t*>(a.C) + crow * ldq + head * kD + half * 4;
      uint16_t* op = a.O + int64_t(row) * ldq + head * kD + half * 4;
      const uint16_t* sp = slot >= 0 ? a.o_sal + int64_t(slot) * ldq + head * kD + half * 4 : nullptr;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int off = dt * 32 + g * 8;
          const uint2 cv = *reinterpret_cast<const uint2*>(cp + off);
          const float old[4] = {__uint_as_float(cv.x << 16), __uint_as_float(cv.x & 0xffff0000u),
                                __uint_as_float(cv.y << 16), __uint_as_float(cv.y & 0xffff0000u)};
          float nw[4];
          uint2 st;
          if (sp) {
            st = *reinterpret_cast<const uint2*>(sp + off);
            nw[0] = __uint_as_float(st.x << 16);
            nw[1] = __uint_as_float(st.x & 0xffff0000u);
            nw[2] = __uint_as_float(st.y << 16);
            nw[3] = __uint_as_float(st.y & 0xffff0000u);
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) nw[j] = add_mul_rn(old[j], o_acc[dt][4 * g + j], inv);
            st.x = pack_bf16x2(nw[0], nw[1]);
            st.y = pack_bf16x2(nw[2], nw[3]);
          }
          *reinterpret_cast<uint2*>(op + off) = st;
          if (a.c_inplace) *reinterpret_cast<uint2*>(cp + off) = st;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dot += nw[j] * old[j];
            nn += nw[j] * nw[j];
            oo += old[j] * old[j];
          }
        }
    }
    dot = half_swap_sum(dot);
    nn = half_swap_sum(nn);
    oo = half_swap_sum(oo);
    if (own && half == 0) {
      a.part[(int64_t(head) * 3 + 0) * a.Tq + row] = dot;
      a.part[(int64_t(head) * 3 + 1) * a.Tq + row] = nn;
      a.part[(int64_t(head) * 3 + 2) * a.Tq + row] = oo;
    }
  }
}

template <AttnMode MODE, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kBK * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[kD * kVStride];
  if constexpr (MODE == AttnMode::ColSparse) {
    __shared__ float m_lds[NW * kMaxBlk2 * 32];
    __shared__ int16_t key_lds[kMaxBlk2 * kBK];
    __shared__ uint8_t gblk_lds[8 * kMaxBlk2];
    __shared__ int ngrp_lds;
    __shared__ float xch_lds[NW * 96];
    attention_tile<MODE, NW>(a, xcd_remap(blockIdx.x, gridDim.x), k_lds, vt_lds,
                             ColSparseLds{m_lds, key_lds, gblk_lds, &ngrp_lds, xch_lds});
  } else {
    attention_tile<MODE, NW>(a, xcd_remap(blockIdx.x, gridDim.x), k_lds, vt_lds, ColSparseLds{});
  }
}

// Fused sparse step: the row-sparse tiles of the salient queries (finishing their rows) and the
// column-sparse tiles of all other queries in one launch, so the two run concurrently. The
// row-sparse tiles come first (n_rs_pad of them, a multiple of 8, the excess returning at once),
// each range remapped XCD-major on its own.
template <int NW, bool CHUNKED>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_step_kernel(
    AttnArgs rs, AttnArgs cs, int n_rs, int n_rs_pad) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kBK * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[kD * kVStride];
  __shared__ float m_lds[NW * kMaxBlk2 * 32];
  __shared__ int16_t key_lds[kMaxBlk2 * kBK];
  __shared__ uint8_t gblk_lds[8 * kMaxBlk2];
  __shared__ int ngrp_lds;
  __shared__ float xch_lds[NW * 96];
  __shared__ unsigned long long kbits_lds[kMaxBlk2];
  __shared__ int sblk_lds[kMaxBlk2];
  __shared__ uint32_t rowflag_lds[NW];
  const int wg = blockIdx.x;
  if (wg < n_rs_pad) {
    const int t = xcd_remap(wg, n_rs_pad);
    if (t < n_rs) attention_tile<AttnMode::RowSparse, NW>(rs, t, k_lds, vt_lds, ColSparseLds{});
  } else {
    attention_tile<AttnMode::ColSparse, NW, CHUNKED, true>(cs, xcd_remap(wg - n_rs_pad, int(gridDim.x) - n_rs_pad), k_lds,
                                                     vt_lds,
                                                     ColSparseLds{m_lds, key_lds, gblk_lds, &ngrp_lds, xch_lds, kbits_lds,
                                                                  sblk_lds, rowflag_lds});
  }
}

// ---- column-sparse preparation: slot maps + per-block salient key bits -----------------
__global__ __launch_bounds__(256) void colsparse_fill_kernel(int32_t* __restrict__ slot, int64_t Tq,
                                                             uint64_t* __restrict__ kmask, int64_t nmask,
                                                             int32_t* __restrict__ kslot, int64_t Tk) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < Tq) slot[i] = -1;
  if (i < nmask) kmask[i] = 0;
  if (kslot && i < Tk) kslot[i] = -1;
}

__global__ __launch_bounds__(256) void colsparse_scatter_kernel(const int32_t* __restrict__ idx_q,
                                                                const int32_t* __restrict__ idx_k, int n_sal,
                                                                const int32_t* __restrict__ cu_k, int B, int nblk,
                                                                int32_t* __restrict__ slot,
                                                                unsigned long long* __restrict__ kmask,
                                                                int32_t* __restrict__ kslot) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n_sal) return;
  slot[idx_q[j]] = j;
  const int64_t k = idx_k[j];
  if (kslot) kslot[k] = j;
  const int b = find_segment(cu_k, B + 1, k);
  if (b >= B || k >= cu_k[b + 1]) return;
  const int off = int(k - cu_k[b]);
  atomicOr(&kmask[int64_t(b) * nblk + off / kBK], 1ull << (off % kBK));
}


// dV = bf16(v_new - v_cache[row]) then v_cache[row] = v_new (attention.py:67-74, 89-96),
// one wavefront per salient row, 16-byte lanes.
__global__ __launch_bounds__(256) void v_delta_update_kernel(uint16_t* __restrict__ v_cache,
                                                             const uint16_t* __restrict__ v_new,
                                                             const int64_t* __restrict__ dest_rows, int64_t n,
                                                             int64_t row_elems, uint16_t* __restrict__ dv) {
  const int64_t j = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (j >= n) return;
  uint4* cr = reinterpret_cast<uint4*>(v_cache + dest_rows[j] * row_elems);
  const uint4* nr = reinterpret_cast<const uint4*>(v_new + j * row_elems);
  uint4* dr = reinterpret_cast<uint4*>(dv + j * row_elems);
  for (int64_t i = lane; i < row_elems / 8; i += 64) {
    const uint4 o = cr[i], nw = nr[i];
    dr[i] = bf16x8_sub(nw, o);
    cr[i] = nw;
  }
}

int launch_v_delta_update(uint16_t* v_cache, const uint16_t* v_new, const int64_t* dest_rows, int64_t n,
                          int64_t row_elems, uint16_t* dv, hipStream_t s) {
  DYLLM_REQUIRE(row_elems % 8 == 0, "V row width must be a multiple of 8");
  if (n <= 0) return 0;
  v_delta_update_kernel<<<unsigned(cdiv(n, 4)), 256, 0, s>>>(v_cache, v_new, dest_rows, n, row_elems, dv);
  return check_launch("v_delta_update_kernel");
}

// out[b] = seq_starts[seq_ids[b]] (+ Lk_b - Lq_b when cu_q is given: the first cached row of
// the queried tail block, cache_kernels.cu:224).
__global__ void seq_row_starts_kernel(const int64_t* __restrict__ seq_starts, const int64_t* __restrict__ seq_ids,
                                      const int32_t* __restrict__ cu_k, const int32_t* __restrict__ cu_q, int B,
                                      int64_t* __restrict__ out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  int64_t v = seq_starts[seq_ids[b]];
  if (cu_q) v += int64_t(cu_k[b + 1] - cu_k[b]) - int64_t(cu_q[b + 1] - cu_q[b]);
  out[b] = v;
}

int launch_seq_row_starts(const int64_t* seq_starts, const int64_t* seq_ids, const int32_t* cu_k,
                          const int32_t* cu_q, int B, int64_t* out, hipStream_t s) {
  if (B <= 0) return 0;
  seq_row_starts_kernel<<<unsigned(cdiv(B, 256)), 256, 0, s>>>(seq_starts, seq_ids, cu_k, cu_q, B, out);
  return check_launch("seq_row_starts_kernel");
}

template <AttnMode MODE, int NW>
static void launch_mode(const AttnArgs& a, int max_rows_per_seq, hipStream_t s) {
  AttnArgs g = a;
  g.tiles_per_seq = int(cdiv(max_rows_per_seq, NW * 32));
  const int64_t nwg = int64_t(g.tiles_per_seq) * a.H * a.B;
  attention_kernel<MODE, NW><<<unsigned(nwg), NW * 64, 0, s>>>(g);
}

// Q, K, V and the context rows are moved with 16-byte loads / 8-byte stores
static bool attn_aligned(const AttnArgs& a) {
  const uintptr_t m = reinterpret_cast<uintptr_t>(a.Q) | reinterpret_cast<uintptr_t>(a.K) |
                      reinterpret_cast<uintptr_t>(a.V) | reinterpret_cast<uintptr_t>(a.C) |
                      reinterpret_cast<uintptr_t>(a.o_sal);
  return (m % 16) == 0 && reinterpret_cast<uintptr_t>(a.O) % 8 == 0;
}

int attention_kernel_info(int dim, int64_t* out) {
  hipFuncAttributes fa{};
  const void* fn = reinterpret_cast<const void*>(&attention_step_kernel<4, false>);
  if (hipFuncGetAttributes(&fa, fn) != hipSuccess) return fail("hipFuncGetAttributes failed for attention_step_kernel");
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, 256, 0) != hipSuccess)
    return fail("hipOccupancyMaxActiveBlocksPerMultiprocessor failed for attention_step_kernel");
  const int64_t v[10] = {fa.numRegs, int64_t(fa.localSizeBytes), int64_t(fa.sharedSizeBytes), 0, 256, blocks,
                         4 * 32, kBK, 1, dim == kD ? 1 : 0};
  for (int i = 0; i < 10; ++i) out[i] = v[i];
  return 0;
}

int launch_attention(AttnMode mode, const AttnArgs& a, int max_rows_per_seq, hipStream_t s) {
  DYLLM_REQUIRE(a.B >= 1 && a.H >= 1 && a.Hkv >= 1 && a.H % a.Hkv == 0, "bad head counts");
  DYLLM_REQUIRE(attn_aligned(a), "Q, K, V and context buffers must be 16-byte aligned (output 8-byte)");
  DYLLM_REQUIRE(max_rows_per_seq >= 0, "bad row bound");
  if (max_rows_per_seq == 0) return 0;
  DYLLM_REQUIRE(cdiv(max_rows_per_seq, 128) * a.H * a.B < (int64_t(1) << 31), "grid too large");
  // 4-wave workgroups (128 rows) at every grid size: 2-wave workgroups on small grids (twice the
  // workgroups, each staging every K/V block for half the rows, and spilling at 256 VGPRs) measured
  // slower in every case tried, from 16 to 384 rows per sequence
  switch (mode) {
    case AttnMode::Dense:
      launch_mode<AttnMode::Dense, 4>(a, max_rows_per_seq, s);
      break;
    case AttnMode::RowSparse:
      launch_mode<AttnMode::RowSparse, 4>(a, max_rows_per_seq, s);
      break;
    case AttnMode::ColSparse:
      launch_mode<AttnMode::ColSparse, 4>(a, max_rows_per_seq, s);
      break;
  }
  return check_launch("attention_kernel");
}

int launch_attention_step(const AttnArgs& rs0, int max_rows_rs, const AttnArgs& cs0, int max_rows_cs,
                          hipStream_t s) {
  DYLLM_REQUIRE(cs0.B >= 1 && cs0.H >= 1 && cs0.Hkv >= 1 && cs0.H % cs0.Hkv == 0, "bad head counts");
  DYLLM_REQUIRE(attn_aligned(rs0) && attn_aligned(cs0), "Q, K, V and context buffers must be 16-byte aligned (output 8-byte)");
  AttnArgs rs = rs0, cs = cs0;
  rs.tiles_per_seq = int(cdiv(max_rows_rs > 0 ? max_rows_rs : 1, 128));
  cs.tiles_per_seq = int(cdiv(max_rows_cs, 128));
  const int64_t n_rs = max_rows_rs > 0 ? int64_t(rs.tiles_per_seq) * rs.H * rs.B : 0;
  const int64_t n_rs_pad = cdiv(n_rs, 8) * 8;
  const int64_t n_cs = int64_t(cs.tiles_per_seq) * cs.H * cs.B;
  DYLLM_REQUIRE(n_rs_pad + n_cs < (int64_t(1) << 31), "grid too large");
  if (n_rs_pad + n_cs == 0) return 0;
  // sequences longer than the LDS max table (kMaxBlk2 key blocks) take the chunked two-pass
  // instantiation; the other one keeps its registers for the paired pass 1
  if (cs.nblk > kMaxBlk2)
    attention_step_kernel<4, true><<<unsigned(n_rs_pad + n_cs), 256, 0, s>>>(rs, cs, int(n_rs), int(n_rs_pad));
  else
    attention_step_kernel<4, false><<<unsigned(n_rs_pad + n_cs), 256, 0, s>>>(rs, cs, int(n_rs), int(n_rs_pad));
  return check_launch("attention_step_kernel");
}

int launch_colsparse_prep(const int32_t* idx_q, const int32_t* idx_k, int n_sal, const int32_t* cu_k, int B,
                          int nblk, int32_t* slot, int64_t Tq, uint64_t* kmask, int32_t* kslot, int64_t Tk,
                          hipStream_t s) {
  const int64_t nmask = int64_t(B) * nblk;
  int64_t n = Tq > nmask ? Tq : nmask;
  if (kslot && Tk > n) n = Tk;
  if (n > 0) {
    colsparse_fill_kernel<<<unsigned(cdiv(n, 256)), 256, 0, s>>>(slot, Tq, kmask, nmask, kslot, Tk);
    if (int rc = check_launch("colsparse_fill_kernel")) return rc;
  }
  if (n_sal > 0) {
    colsparse_scatter_kernel<<<unsigned(cdiv(n_sal, 256)), 256, 0, s>>>(
        idx_q, idx_k, n_sal, cu_k, B, nblk, slot, reinterpret_cast<unsigned long long*>(kmask), kslot);
    return check_launch("colsparse_scatter_kernel");
  }
  return 0;
}

}  // namespace dyllm

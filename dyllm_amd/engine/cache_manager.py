"""Per-layer packed row cache (context, K, V and FFN-output rows).

Interface and semantics of dyllm/engine/cache_manager.py:11-181: rows of one sequence are
contiguous, ``seq_start_gpu[seq_id]`` holds its first row, and the copy ops run on the HIP
row kernels (get_seqs / get_block / reset_full / reset_block / scatter_update).

MI355X-first differences (same results):
  * the rows live in a preallocated slab that grows geometrically, instead of a tensor
    re-built with ``torch.cat`` on every new sequence (cache_manager.py:69-137);
  * ``get_seqs`` returns a zero-copy view when the running sequences sit in the slab in
    batch order (the common case: they were allocated in that order by ``reset_full``),
    instead of re-gathering the whole [T, D] cache every layer;
  * ``row_starts`` / ``dest_rows`` expose the cache addressing so that kernels read and
    write the cache in place (attention on cached K/V/context, FFN scatter epilogue).
"""
from __future__ import annotations

from typing import List, Optional

import torch

from .. import ops
from ..utils.context import get_context


class CacheManager:

    def __init__(self, hidden_dim: int, max_num_seqs: int = 16384, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device = torch.device("cuda"), initial_rows: int = 0):
        self._seq_to_start: dict[int, int] = {}
        self._seq_to_len: dict[int, int] = {}
        self.hidden_dim = hidden_dim
        self.dtype = dtype
        self.max_num_seqs = max_num_seqs
        self.device = device
        self._slab = torch.empty((max(initial_rows, 0), hidden_dim), dtype=dtype, device=device)
        self._used = 0
        self.seq_start_gpu = torch.full((max_num_seqs,), -1, dtype=torch.long, device=device)
        self.seq_len_gpu = torch.zeros((max_num_seqs,), dtype=torch.long, device=device)

    # -- storage --------------------------------------------------------------------
    @property
    def cache(self) -> torch.Tensor:
        """The used rows, ``[sum(L), D]`` (a view of the slab)."""
        return self._slab[: self._used]

    @property
    def num_total_seqs(self) -> int:
        return len(self._seq_to_start)

    def _reserve(self, rows: int):
        if rows <= self._slab.shape[0]:
            return
        cap = max(rows, 2 * self._slab.shape[0], 1024)
        slab = torch.empty((cap, self.hidden_dim), dtype=self.dtype, device=self.device)
        if self._used:
            slab[: self._used].copy_(self._slab[: self._used])
        self._slab = slab

    def select_seq_range(self, seq_id: int):
        start = self._seq_to_start[seq_id]
        return start, start + self._seq_to_len[seq_id]

    def get_start_indices(self, seq_ids: List[int]) -> torch.Tensor:
        return torch.tensor([self._seq_to_start[s] for s in seq_ids], dtype=torch.long)

    def _contiguous_view(self, seq_ids_list: Optional[List[int]], cu_k_cpu: Optional[List[int]]):
        """The slab rows of the running batch when they are stored back to back in batch
        order (so the packed layout equals the cache layout), else None."""
        if not seq_ids_list or cu_k_cpu is None or len(cu_k_cpu) != len(seq_ids_list) + 1:
            return None
        s0 = self._seq_to_start.get(seq_ids_list[0])
        if s0 is None:
            return None
        for b, sid in enumerate(seq_ids_list):
            if self._seq_to_start.get(sid) != s0 + cu_k_cpu[b] or self._seq_to_len.get(sid) != cu_k_cpu[b + 1] - cu_k_cpu[b]:
                return None
        return self._slab[s0: s0 + cu_k_cpu[-1]]

    # -- reads ------------------------------------------------------------------------
    def get_seqs(self, seq_ids: torch.Tensor, seq_ids_list: Optional[List[int]] = None) -> torch.Tensor:
        """Packed rows of the running sequences (cache_manager.py:39-43)."""
        ctx = get_context()
        view = self._contiguous_view(seq_ids_list, ctx.cu_seqlens_k_cpu)
        if view is not None and ctx.total_seqlen <= ctx.total_seqlen_k:
            return view
        return ops.get_seqs_cuda(self._slab, self.seq_start_gpu, ctx.cu_seqlens_k, seq_ids,
                                 max(ctx.total_seqlen, ctx.total_seqlen_k))

    def get_seqs_block(self, seq_ids: torch.Tensor) -> torch.Tensor:
        """Tail ``Lq`` rows of every running sequence (cache_manager.py:45-49)."""
        ctx = get_context()
        return ops.get_block_cuda(self._slab, self.seq_start_gpu, ctx.cu_seqlens_k, ctx.cu_seqlens_q, seq_ids,
                                  ctx.total_seqlen)

    def row_starts(self, seq_ids: torch.Tensor, block: bool = False) -> torch.Tensor:
        """First cache row of each running sequence ([B] int64, device); with ``block`` the
        first row of its queried tail block."""
        ctx = get_context()
        return ops.seq_row_starts(self.seq_start_gpu, seq_ids, ctx.cu_seqlens_k,
                                  ctx.cu_seqlens_q if block else None)

    def dest_rows(self, seq_ids: torch.Tensor, row_idx: torch.Tensor, count=None) -> torch.Tensor:
        """Cache rows of packed K-space row indices (the addressing of scatter_update); with a
        device ``count`` only its first count[0] entries are mapped."""
        ctx = get_context()
        return ops.scatter_dest_rows(row_idx, ctx.cu_seqlens_k, self.seq_start_gpu, seq_ids, count)

    # -- allocation ---------------------------------------------------------------------
    def reset_seq(self, c: torch.Tensor, seq_id):
        if seq_id in self._seq_to_start:
            start, end = self.select_seq_range(seq_id)
            if end - start == c.size(0):
                self._slab[start:end] = c
                return
            self.remove_seq(seq_id)
        self.add_seq(c, seq_id)

    def add_seq(self, c: torch.Tensor, seq_id: int):
        start = self._used
        self._reserve(start + c.size(0))
        self._slab[start: start + c.size(0)] = c
        self._used += c.size(0)
        self._seq_to_start[seq_id] = start
        self._seq_to_len[seq_id] = c.size(0)
        self.seq_start_gpu[seq_id] = start
        self.seq_len_gpu[seq_id] = c.size(0)

    def remove_seq(self, seq_id: int):
        if seq_id not in self._seq_to_start:
            return
        start, end = self.select_seq_range(seq_id)
        length = end - start
        if end < self._used:
            self._slab[start: self._used - length] = self._slab[end: self._used].clone()
        self._used -= length
        moved = [o for o, s in self._seq_to_start.items() if o != seq_id and s > start]
        for o in moved:
            self._seq_to_start[o] -= length
        if moved:
            ids = torch.tensor(moved, device=self.device, dtype=torch.long)
            self.seq_start_gpu[ids] -= length
        del self._seq_to_start[seq_id]
        del self._seq_to_len[seq_id]
        self.seq_start_gpu[seq_id] = -1
        self.seq_len_gpu[seq_id] = 0

    def _vectorized_allocate_new_seqs(self, new_ids: List[int], new_lengths: List[int]):
        total_new = sum(new_lengths)
        if total_new == 0:
            return
        base = self._used
        self._reserve(base + total_new)
        starts = []
        acc = base
        for sid, L in zip(new_ids, new_lengths):
            self._seq_to_start[sid] = acc
            self._seq_to_len[sid] = L
            starts.append(acc)
            acc += L
        self._used = acc
        ids = torch.tensor(new_ids, device=self.device, dtype=torch.long)
        self.seq_start_gpu[ids] = torch.tensor(starts, device=self.device, dtype=torch.long)
        self.seq_len_gpu[ids] = torch.tensor(new_lengths, device=self.device, dtype=torch.long)

    # -- writes -------------------------------------------------------------------------
    def reset_full(self, c: torch.Tensor, seq_ids: torch.Tensor, seq_ids_list: Optional[List[int]] = None):
        """Write all rows of the running sequences, allocating new ones (cache_manager.py:139-159)."""
        ctx = get_context()
        c = c.flatten(1).contiguous()
        if seq_ids_list is None:
            seq_ids_list = seq_ids.cpu().tolist()
        lens = ctx.context_lens_cpu
        new_ids, new_lens = [], []
        for i, sid in enumerate(seq_ids_list):
            if sid not in self._seq_to_start:
                new_ids.append(sid)
                new_lens.append(lens[i])
        if new_ids:
            self._vectorized_allocate_new_seqs(new_ids, new_lens)
        ops.reset_full_cuda(self._slab, c, self.seq_start_gpu, ctx.cu_seqlens_q, seq_ids, ctx.total_seqlen)

    def reset_block(self, c: torch.Tensor, seq_ids: torch.Tensor):
        """Write the tail ``Lq`` rows of every running sequence (cache_manager.py:161-167)."""
        ctx = get_context()
        c = c.flatten(1).contiguous()
        ops.reset_block_cuda(self._slab, c, self.seq_start_gpu, ctx.cu_seqlens_k, ctx.cu_seqlens_q, seq_ids,
                             ctx.total_seqlen)

    def scatter_update(self, seq_ids: torch.Tensor, row_idx: torch.Tensor, new: torch.Tensor):
        """cache[row of packed K index row_idx[m]] = new[m] (cache_manager.py:172-174)."""
        ctx = get_context()
        ops.scatter_update_cuda(self._slab, new, row_idx, ctx.cu_seqlens_k, self.seq_start_gpu, seq_ids)

    def scatter_kv_rope(self, seq_ids: torch.Tensor, row_idx: torch.Tensor, kv: torch.Tensor, num_kv_heads: int,
                        positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos_idx: torch.Tensor,
                        k_norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6) -> torch.Tensor:
        """scatter_update of the salient rows' rotated keys, fused with their k_norm / RoPE
        (llada.py:108-143): kv = [k | v] rows of the salient-row projection; returns v."""
        ctx = get_context()
        return ops.kv_rope_scatter(kv, num_kv_heads, positions, cos, sin, self._slab, row_idx, ctx.cu_seqlens_k,
                                   self.seq_start_gpu, seq_ids, pos_idx=pos_idx, k_norm_weight=k_norm_weight,
                                   eps=eps)

    def kv_rows(self, kv: torch.Tensor, num_kv_heads: int, positions: torch.Tensor, cos: torch.Tensor,
                sin: torch.Tensor, pos_idx: torch.Tensor, kv_rows: Optional[torch.Tensor] = None,
                k_norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6) -> "ops.KvRows":
        """The salient rows' [k | v] projection output as the sparse step's ``v`` (ops.KvRows): the
        step itself writes their rotated keys into this cache (scatter_update fused with k_norm /
        RoPE, llada.py:108-143) before its attention reads them."""
        return ops.KvRows(kv, num_kv_heads, positions, cos, sin, self._slab, self.seq_start_gpu, kv_rows=kv_rows,
                          pos_idx=pos_idx, k_norm_weight=k_norm_weight, eps=eps)

    def finish(self, finished_seq_ids: List[int]):
        if len(finished_seq_ids) == 0:
            return False
        for seq_id in sorted(finished_seq_ids, key=lambda x: self._seq_to_start.get(x, -1), reverse=True):
            self.remove_seq(seq_id)
        return True

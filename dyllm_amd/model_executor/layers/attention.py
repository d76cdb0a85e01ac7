"""Attention layer of the sparse diffusion step (dyllm/model_executor/layers/attention.py:13-178).

Same constructor, ``forward(q, k, v)`` contract and context mutation as the reference:

* full step  -- dense varlen attention; the context and V caches are rewritten
                (attention.py:39-62);
* sparse step -- ``v`` holds the new V rows of the salient keys. dV and the V-cache update,
                row-sparse attention of the salient queries against the full cached K/V,
                column-sparse attention ``C_old + softmax(QK^T/sqrt(D)) dV`` with the saliency
                statistics and tau test, compaction of the new salient set, context-cache
                update, and the next layer's ``ctx.idx_salient_row`` / ``cu_salientlens`` /
                ``idx_salient_row_k`` (attention.py:64-178).

Differences in *how*, not *what*: dV stays compact ([n_sal] rows addressed through a key->slot
map inside the kernel) instead of a zero-filled [T_k] tensor; the column-sparse kernel reads the
cached context rows in place and writes the new rows straight back (the reference's
get_seqs_block + reset_block round trip); compaction runs on the device and returns the
per-sequence counts without torch.nonzero/searchsorted. One host read of the salient count per
layer remains, as in the reference (torch.nonzero).
"""
from __future__ import annotations

import torch
from torch import nn

from ... import ops
from ...engine.cache_manager import CacheManager
from ...utils.context import get_context
from ...utils.metadata import get_metadata


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale, num_kv_heads, threshold: float = 0.99,
                 device: torch.device | str = "cuda"):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.threshold = threshold
        self.context_cache = CacheManager(self.num_heads * self.head_dim, device=torch.device(device))
        self.v_cache = CacheManager(self.num_kv_heads * self.head_dim, device=torch.device(device))

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        ctx = get_context()
        md = get_metadata()
        q = q.contiguous()
        k = k.contiguous()
        v = v.contiguous()

        if ctx.is_full:
            o = ops.flash_attn_varlen_func(q, k, v, ctx.cu_seqlens_q, ctx.cu_seqlens_k, ctx.max_seqlen_q,
                                           ctx.max_seqlen_k, softmax_scale=self.scale)
            self.context_cache.reset_full(o.reshape(o.shape[0], -1), md.running_seqs_tensor,
                                          seq_ids_list=md.running_seqs)
            self.v_cache.reset_full(v.reshape(v.shape[0], -1), md.running_seqs_tensor, seq_ids_list=md.running_seqs)
            self.context_cache.finish(md.finished_seqs)
            self.v_cache.finish(md.finished_seqs)
            return o

        seq_ids = md.running_seqs_tensor
        q_pruned = ctx.idx_salient_row_k is not None
        idx_q = ctx.idx_salient_row
        idx_k = ctx.idx_salient_row_k if q_pruned else ctx.idx_salient_row
        idx_q32 = ctx.idx_salient_row_i32 if ctx.idx_salient_row_i32 is not None else idx_q.to(torch.int32)
        idx_k32 = idx_k.to(torch.int32) if q_pruned else idx_q32

        # dV of the salient keys and the V-cache update (attention.py:67-74, 89-96)
        dv = ops.v_delta_update(self.v_cache._slab, v, self.v_cache.dest_rows(seq_ids, idx_k))
        v_full = self.v_cache.get_seqs(seq_ids, md.running_seqs).view(-1, self.num_kv_heads, self.head_dim)

        # row-sparse attention of the salient queries vs the full cached K/V (attention.py:76-87)
        max_sal = ctx.max_salientlen if ctx.max_salientlen > 0 else ctx.max_seqlen_q
        o_sal = ops.flash_attn_varlen_func(q, k, v_full, ctx.cu_salientlens, ctx.cu_seqlens_k, max_sal,
                                           ctx.max_seqlen_k, softmax_scale=self.scale, q_rows=idx_q32)

        # column-sparse attention + stats + tau test, context cache updated in place
        # (attention.py:107-145 and the reset_block/reset_full of :153,168)
        c_start = self.context_cache.row_starts(seq_ids, block=q_pruned)
        new_c, _, mask = ops.attention_colsparse_cached(
            q, k, None, dv.view(-1, self.num_kv_heads, self.head_dim), self.context_cache._slab, c_start, o_sal,
            ctx.cu_seqlens_q, ctx.cu_seqlens_k, ctx.max_seqlen_q, ctx.max_seqlen_k, k.shape[0], idx_q32, idx_k32,
            self.threshold, c_inplace=True)

        # compaction of the next salient set (attention.py:147-173)
        comp = ops.salient_compact(mask, ctx.cu_seqlens_q, ctx.cu_promptlens if q_pruned else None)
        n, cu_host = comp.host()
        ctx.max_salientlen = max(cu_host[i + 1] - cu_host[i] for i in range(len(cu_host) - 1))
        ctx.idx_salient_row = comp.idx64[:n]
        ctx.idx_salient_row_i32 = comp.idx32[:n]
        ctx.cu_salientlens = comp.cu_salientlens
        if q_pruned:
            ctx.idx_salient_row_k = comp.idx_k[:n]

        self.v_cache.finish(md.finished_seqs)
        self.context_cache.finish(md.finished_seqs)
        return new_c.view(-1, self.num_heads, self.head_dim)

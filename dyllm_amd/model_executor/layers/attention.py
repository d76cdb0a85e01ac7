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
per-sequence counts without torch.nonzero/searchsorted. The one host read of the salient count
per layer (the reference's torch.nonzero sync) is deferred until the next layer needs it, so the
FFN of this layer is already enqueued when the host waits.
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
        self._bufs = None  # reusable outputs / workspace of the sparse step (ops.StepBuffers)
        # optional: the FFN-output cache of this layer; the step's compaction then also produces
        # the rows of the next salient set in it (the FFN's scatter targets)
        self.ffn_cache = None

    def forward(self, q: torch.Tensor, k, v) -> torch.Tensor:
        """``k``, ``v`` as the reference's (the V rows of the salient keys on a sparse step); or,
        on a sparse step, ``k = None`` and ``v`` an ``ops.KvRows``: the salient-row projection
        output whose K/V epilogue the step's first launch applies (K then read from its cache)."""
        ctx = get_context()
        md = get_metadata()
        q = q.contiguous()
        kv_rows = isinstance(v, ops.KvRows)
        if kv_rows and ctx.is_full:
            raise RuntimeError("KvRows is for sparse steps; a full step takes the dense k and v")
        if not kv_rows:
            k = k.contiguous()
            v = v.contiguous()

        if ctx.is_full:
            o = ops.flash_attn_varlen_func(q, k, v, ctx.cu_seqlens_q, ctx.cu_seqlens_k, ctx.max_seqlen_q,
                                           ctx.max_seqlen_k, softmax_scale=self.scale)
            self.context_cache.reset_full(o.flatten(1), md.running_seqs_tensor,
                                          seq_ids_list=md.running_seqs)
            self.v_cache.reset_full(v.flatten(1), md.running_seqs_tensor, seq_ids_list=md.running_seqs)
            self.context_cache.finish(md.finished_seqs)
            self.v_cache.finish(md.finished_seqs)
            return o

        seq_ids = md.running_seqs_tensor
        q_pruned = ctx.q_pruned
        idx_q = ctx.idx_salient_row            # resolves the previous layer's set (host read)
        n = idx_q.numel()
        idx_q32 = ctx.idx_salient_row_i32
        if q_pruned:
            idx_k64, idx_k32 = ctx.idx_salient_row_k, ctx.idx_salient_row_k_i32
        else:
            idx_k64, idx_k32 = idx_q, idx_q32
        Tq, B = q.shape[0], seq_ids.numel()
        Tk = int(ctx.total_seqlen_k or ctx.cu_seqlens_k_cpu[-1]) if kv_rows else k.shape[0]
        key = (Tq, Tk, B, q_pruned, ctx.max_seqlen_k)
        bufs = self._bufs
        if bufs is None or bufs.key != key:
            bufs = self._bufs = ops.StepBuffers(key, q.device, Tq, Tk, B, self.num_heads, self.num_kv_heads,
                                                self.head_dim, ctx.max_seqlen_k, q_pruned)
        # one native call: dV + V-cache update, row-sparse attention (attention.py:67-87),
        # column-sparse attention + stats + tau test with the context cache updated in place
        # (:107-145, :153/:168), and compaction of the next salient set (:147-173)
        ops.sparse_attention_step(
            bufs, q, k, self.v_cache._slab, self.v_cache.seq_start_gpu,
            v if kv_rows else v.view(n, self.num_kv_heads, self.head_dim),
            self.context_cache._slab, self.context_cache.seq_start_gpu, seq_ids, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
            ctx.cu_promptlens if q_pruned else None, ctx.max_seqlen_q, ctx.max_seqlen_k, Tk, n, ctx.max_salientlen,
            ctx.cu_salientlens, idx_q32, idx_k64, idx_k32, self.scale, self.threshold,
            dest_seq_starts=self.ffn_cache.seq_start_gpu if self.ffn_cache is not None else None)
        # the next layer's salient set stays on the device until it is needed (Context.resolve_salient)
        ctx.set_pending(bufs.compacted())
        new_c = bufs.out

        self.v_cache.finish(md.finished_seqs)
        self.context_cache.finish(md.finished_seqs)
        return new_c.view(-1, self.num_heads, self.head_dim)

"""FFN-output cache (dyllm/model_executor/layers/mlp_cache_manage.py:11-40): on a full step
all rows are written; on a sparse step the salient rows are scattered in and all queried rows
are returned (stale rows from the cache, fresh rows just computed)."""
import torch
from torch import nn

from ... import ops
from ...engine.cache_manager import CacheManager
from ...utils.context import get_context
from ...utils.metadata import get_metadata


class MLPcache(nn.Module):

    def __init__(self, hidden_dim: int = 0, device="cuda"):
        super().__init__()
        self.cache_manager = CacheManager(hidden_dim=hidden_dim, device=torch.device(device))

    def salient_rows(self):
        """K-space salient indices of this step (the rows the FFN recomputes)."""
        ctx = get_context()
        return ctx.idx_salient_row_k if ctx.idx_salient_row_k is not None else ctx.idx_salient_row

    def dest_rows(self):
        """Cache rows the salient FFN outputs go to (for an in-place scatter epilogue)."""
        md = get_metadata()
        return self.cache_manager.dest_rows(md.running_seqs_tensor, self.salient_rows())

    def gather_all(self, lazy: bool = False):
        """All queried rows, packed (mlp_cache_manage.py:33/38). With ``lazy``, a Q-pruned step
        returns them as ``ops.CacheRows`` (read in place by the next layer's norm, no copy)."""
        ctx = get_context()
        md = get_metadata()
        if ctx.q_pruned:
            if lazy:
                cm = self.cache_manager
                return ops.CacheRows(cm._slab, cm.seq_start_gpu, md.running_seqs_tensor, ctx.cu_seqlens_k,
                                     ctx.cu_seqlens_q, ctx.total_seqlen)
            return self.cache_manager.get_seqs_block(md.running_seqs_tensor)
        return self.cache_manager.get_seqs(md.running_seqs_tensor, md.running_seqs)

    def forward(self, x: torch.Tensor):
        ctx = get_context()
        md = get_metadata()
        if ctx.is_full:
            self.cache_manager.reset_full(x, md.running_seqs_tensor, seq_ids_list=md.running_seqs)
            self.cache_manager.finish(md.finished_seqs)
            return self.cache_manager.get_seqs(md.running_seqs_tensor, md.running_seqs)
        self.cache_manager.scatter_update(md.running_seqs_tensor, self.salient_rows(), x)
        self.cache_manager.finish(md.finished_seqs)
        return self.gather_all()

"""LLaDA-MoE decoder (dyllm/model_executor/models/lladamoe.py:56-352): per-head RMSNorm of q and
k, and a sparse mixture-of-experts FFN (fp32 softmax router, top-k of E experts, SwiGLU experts)
in place of the dense MLP. On sparse steps only the salient rows are routed; their outputs are
scattered into the FFN cache by the combine kernel (no separate scatter pass)."""
from __future__ import annotations

import torch
from torch import nn

from ... import ops
from ...utils.context import get_context
from ...utils.metadata import get_metadata
from ..layers.mlp_cache_manage import MLPcache
from .llada import LLaDADecoderLayer, LLaDAForDLM, _param


class LLaDAMoESparseBlock(nn.Module):
    """Router + stacked experts (lladamoe.py:56-105): ``gate`` [E, H], ``gate_up_proj``
    [E, 2I, H] (gate rows then up rows), ``down_proj`` [E, H, I]."""

    def __init__(self, cfg, device="cuda", gen=None):
        super().__init__()
        E, H, I = cfg.num_experts, cfg.hidden_size, cfg.expert_intermediate_size
        self.num_experts, self.top_k = E, cfg.num_experts_per_tok
        self.renormalize = bool(cfg.norm_topk_prob)
        self.gate = _param(E, H, device=device, gen=gen)
        self.gate_up_proj = _param(E, 2 * I, H, device=device, gen=gen)
        self.down_proj = _param(E, H, I, device=device, gen=gen)
        self.cache_update = MLPcache(H, device=device)

    def experts(self, x, out=None, out_rows=None, rows_idx=None):
        w, ids = ops.moe_gate(x, self.gate, self.top_k, renormalize=self.renormalize, rows_idx=rows_idx)
        return ops.fused_experts(x, self.gate_up_proj, self.down_proj, w, ids, out=out, out_rows=out_rows,
                                 rows_idx=rows_idx)

    def forward(self, x):
        """Reference interface: x = gathered salient rows (sparse) or all rows (full)."""
        return self.cache_update(self.experts(x.contiguous()))

    def forward_salient(self, h_all, timing=None, lazy=False):
        """Sparse step: route the salient rows of ``h_all`` (read in place by the router and the
        first grouped GEMM, util.py:19-36's gather fused away) and write the expert outputs
        straight into the FFN cache rows."""
        ctx = get_context()
        md = get_metadata()
        cm = self.cache_update.cache_manager
        dest = self.cache_update.dest_rows()
        self.experts(h_all.contiguous(), out=cm._slab, out_rows=dest, rows_idx=ctx.idx_salient_row_i32)
        cm.finish(md.finished_seqs)
        return self.cache_update.gather_all(lazy)


class LLaDAMoEDecoderLayer(LLaDADecoderLayer):
    def _make_mlp(self, cfg, device, gen):
        return LLaDAMoESparseBlock(cfg, device=device, gen=gen)


class LLaDAMoEForDLM(LLaDAForDLM):
    packed_modules_mapping = {"kv_proj": ["k_proj", "v_proj"]}
    layer_cls = LLaDAMoEDecoderLayer

    def normalize_weight_name(self, name: str) -> str:
        return name.replace(".mlp.gate.weight", ".mlp.gate")

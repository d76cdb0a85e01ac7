"""LLaDA bidirectional decoder wired to the sparse hot path
(dyllm/model_executor/models/llada.py:26-260), random-initialised from shape fields only.

The hot path (attention saliency / compaction / gathered SwiGLU + scatter) runs on the HIP
kernels, as do the salient-row K/V projection with its RoPE / K-cache epilogue, the query RoPE
and the decoder-layer RMSNorms; the remaining dense ops on either side of the path (embeddings,
the Q and O projections, the LM head) use PyTorch-ROCm. MLP and Dream/MoE variants share this
structure.
"""
from __future__ import annotations

import re

import torch
import torch.nn.functional as F
from torch import nn

from ... import ops
from ...engine.cache_manager import CacheManager
from ...utils.context import get_context
from ...utils.metadata import get_metadata
from ..layers.attention import Attention
from ..layers.mlp_cache_manage import MLPcache


def _param(*shape, std=0.02, device="cuda", dtype=torch.bfloat16, gen=None):
    w = torch.empty(*shape, dtype=torch.float32, device=device)
    w.normal_(0.0, std, generator=gen)
    return nn.Parameter(w.to(dtype), requires_grad=False)


class RMSNorm(nn.Module):
    """RMSNorm / fused residual-add RMSNorm (layernorm.py:5-51)."""

    def __init__(self, hidden, eps=1e-6, device="cuda"):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden, dtype=torch.bfloat16, device=device), requires_grad=False)

    def forward(self, x, residual=None):
        hidden = x.shape[-1]
        if isinstance(x, ops.CacheRows):   # rows read in place from a layer's FFN cache
            if residual is None:
                return ops.rms_norm(x, self.weight, self.eps)
            return ops.rms_norm(x, self.weight, self.eps, residual=residual.reshape(-1, hidden).contiguous())
        if x.is_cuda and x.dtype == torch.bfloat16 and 1024 <= hidden <= 8192 and hidden % 8 == 0:
            # decoder-layer norms over the hidden size: one native pass per row (dyllm_rms_norm)
            x2 = x.reshape(-1, hidden).contiguous()
            if residual is None:
                return ops.rms_norm(x2, self.weight, self.eps).view(x.shape)
            y, r = ops.rms_norm(x2, self.weight, self.eps, residual=residual.reshape(-1, hidden).contiguous())
            return y.view(x.shape), r.view(residual.shape)
        if residual is not None:
            xf = x.float() + residual.float()
            residual = xf.to(x.dtype)
        else:
            xf = x.float()
        y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight
        return y if residual is None else (y, residual)


class RotaryEmbedding(nn.Module):
    """Neox-style rotary embedding tables (rotary_embedding.py:19-38): fp32 cos / sin
    [max_position, head_dim / 2]; the rotation itself runs in dyllm_rope / dyllm_kv_rope_scatter."""

    def __init__(self, head_dim, max_position, base, device="cuda"):
        super().__init__()
        inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
        t = torch.arange(max_position, dtype=torch.float32, device=device)
        f = torch.outer(t, inv)
        self.register_buffer("cos", f.cos(), persistent=False)
        self.register_buffer("sin", f.sin(), persistent=False)



class LLaDAMLP(nn.Module):
    """SwiGLU FFN + FFN-output cache (llada.py:26-43). On sparse steps the salient rows are
    gathered inside the gate_up GEMM and the down GEMM scatters straight into the cache."""

    def __init__(self, hidden, inter, device="cuda", gen=None):
        super().__init__()
        self.gate_up_proj = _param(2 * inter, hidden, device=device, gen=gen)  # gate rows, then up rows
        self.down_proj = _param(hidden, inter, device=device, gen=gen)
        self.cache_update = MLPcache(hidden, device=device)

    def forward(self, x):
        """Reference interface: x = gathered salient rows (sparse) or all rows (full)."""
        y = ops.swiglu_ffn(x.contiguous(), self.gate_up_proj, self.down_proj)
        return self.cache_update(y)

    def forward_salient(self, h_all, timing=None, lazy=False):
        """Sparse step, fused: h_all = all queried rows after post_attention_layernorm. The
        salient rows are gathered inside the gate_up GEMM and the down GEMM scatters into the FFN
        cache. When the salient set is still on the device (Context.salient_pending), the GEMMs
        read its size from device memory: no host synchronisation.
        ``timing`` (optional): {"gate_up": (start, end), "down": (start, end)} HIP events that
        bracket the gathered gate_up GEMM and the down GEMM (with its split-K reduction).
        ``lazy``: return the queried rows of a Q-pruned step as ``ops.CacheRows`` (no copy)."""
        ctx = get_context()
        md = get_metadata()
        cm = self.cache_update.cache_manager
        comp = ctx.salient_pending
        if comp is not None:
            rows, count, hint = comp.idx32, comp.count, ctx.salient_hint
            kidx = comp.idx_k if comp.idx_k is not None else comp.idx64
        else:
            rows, count, hint = ctx.idx_salient_row_i32, None, 0
            kidx = ctx.idx_salient_row_k if ctx.idx_salient_row_k is not None else ctx.idx_salient_row
        h_all = h_all.contiguous()
        tg = timing.get("gate_up") if timing else None
        td = timing.get("down") if timing else None
        if tg is not None:
            tg[0].record()
        h = ops.ffn_gate_up(h_all, self.gate_up_proj, rows_idx=rows, count=count, hint=hint)
        if tg is not None:
            tg[1].record()
        if comp is not None and comp.dest_rows is not None and comp.dest_starts is cm.seq_start_gpu:
            dest = comp.dest_rows        # produced by the attention step's compaction
        else:
            dest = cm.dest_rows(md.running_seqs_tensor, kidx, count)
        if td is not None:
            td[0].record()
        ops.ffn_down(h, self.down_proj, out=cm._slab, out_rows=dest, count=count, hint=hint)
        if td is not None:
            td[1].record()
        cm.finish(md.finished_seqs)
        return self.cache_update.gather_all(lazy)


class LLaDAAttention(nn.Module):
    """Projections + RoPE + K cache around ``Attention`` (llada.py:46-149)."""

    def __init__(self, hidden, num_heads, num_kv_heads, head_dim, max_position, rope_theta, threshold,
                 qkv_bias=False, qk_layernorm=False, rms_norm_eps=1e-6, device="cuda", gen=None):
        super().__init__()
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.q_size, self.kv_size = num_heads * head_dim, num_kv_heads * head_dim
        self.q_proj = _param(self.q_size, hidden, device=device, gen=gen)
        self.kv_proj = _param(2 * self.kv_size, hidden, device=device, gen=gen)
        self.q_bias = nn.Parameter(torch.zeros(self.q_size, dtype=torch.bfloat16, device=device),
                                   requires_grad=False) if qkv_bias else None
        self.kv_bias = nn.Parameter(torch.zeros(2 * self.kv_size, dtype=torch.bfloat16, device=device),
                                    requires_grad=False) if qkv_bias else None
        self.o_proj = _param(hidden, self.q_size, device=device, gen=gen)
        # per-head RMSNorm of q and k before RoPE (LLaDA-MoE, lladamoe.py:194-199,227-236)
        self.q_norm = RMSNorm(head_dim, rms_norm_eps, device=device) if qk_layernorm else None
        self.k_norm = RMSNorm(head_dim, rms_norm_eps, device=device) if qk_layernorm else None
        self.k_cache = CacheManager(self.kv_size, device=torch.device(device))
        self.rotary = RotaryEmbedding(head_dim, max_position, rope_theta, device=device)
        self.attn = Attention(num_heads, head_dim, head_dim ** -0.5, num_kv_heads, threshold, device=device)

    def forward(self, positions, hidden):
        ctx = get_context()
        md = get_metadata()
        # q_norm + RoPE of every queried row in place, one native pass (dyllm_rope)
        q = F.linear(hidden, self.q_proj, self.q_bias)
        qn, kn = self.q_norm, self.k_norm
        ops.rope_(q, self.num_heads, positions, self.rotary.cos, self.rotary.sin,
                  None if qn is None else qn.weight, 1e-6 if qn is None else qn.eps)
        q = q.view(-1, self.num_heads, self.head_dim)
        if ctx.is_full:
            kv = F.linear(hidden, self.kv_proj, self.kv_bias)
            k, v = kv.split([self.kv_size, self.kv_size], dim=-1)
            ops.rope_(k, self.num_kv_heads, positions, self.rotary.cos, self.rotary.sin,
                      None if kn is None else kn.weight, 1e-6 if kn is None else kn.eps)
            k = k.reshape(-1, self.num_kv_heads, self.head_dim)
            v = v.reshape(-1, self.num_kv_heads, self.head_dim)
            self.k_cache.reset_full(k.flatten(1), md.running_seqs_tensor, seq_ids_list=md.running_seqs)
            o = self.attn(q, k, v)
        else:
            # salient-row K/V projection as one gathered GEMM; its epilogue (k_norm, RoPE, the
            # K-cache row write, llada.py:108-146) runs in the sparse step's first launch, which
            # also takes the v rows from it, and attention reads K from the cache in place
            idx = ctx.idx_salient_row_i32
            kv = ops.linear(hidden, self.kv_proj, self.kv_bias, rows_idx=idx)
            v = self.k_cache.kv_rows(kv, self.num_kv_heads, positions, self.rotary.cos, self.rotary.sin, idx,
                                     k_norm_weight=None if kn is None else kn.weight,
                                     eps=1e-6 if kn is None else kn.eps)
            o = self.attn(q, None, v)
        out = F.linear(o.flatten(1), self.o_proj)
        self.k_cache.finish(md.finished_seqs)
        return out


class LLaDADecoderLayer(nn.Module):
    """llada.py:152-187."""

    def __init__(self, cfg, threshold, device="cuda", gen=None):
        super().__init__()
        self.self_attn = LLaDAAttention(cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads,
                                        cfg.head_dim, cfg.max_position_embeddings, cfg.rope_theta, threshold,
                                        qkv_bias=cfg.qkv_bias, qk_layernorm=cfg.qk_layernorm,
                                        rms_norm_eps=cfg.rms_norm_eps, device=device, gen=gen)
        self.mlp = self._make_mlp(cfg, device, gen)
        if isinstance(self.mlp, LLaDAMLP):   # the attention step computes the FFN's scatter rows
            self.self_attn.attn.ffn_cache = self.mlp.cache_update.cache_manager
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device=device)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device=device)

    def _make_mlp(self, cfg, device, gen):
        return LLaDAMLP(cfg.hidden_size, cfg.intermediate_size, device=device, gen=gen)

    def forward(self, positions, hidden, residual=None):
        if residual is None:
            hidden, residual = self.input_layernorm(hidden), hidden
        else:
            hidden, residual = self.input_layernorm(hidden, residual)
        hidden = self.self_attn(positions, hidden)
        hidden, residual = self.post_attention_layernorm(hidden, residual)
        if get_context().is_full:
            hidden = self.mlp(hidden)
        else:
            # the FFN rows stay in the FFN cache: the next norm reads them in place
            hidden = self.mlp.forward_salient(hidden, lazy=True)
        return hidden, residual


class LLaDAModel(nn.Module):
    def __init__(self, cfg, threshold, device="cuda", gen=None, layer_cls=LLaDADecoderLayer):
        super().__init__()
        self.embed_tokens = _param(cfg.vocab_size, cfg.hidden_size, device=device, gen=gen)
        self.layers = nn.ModuleList([layer_cls(cfg, threshold, device=device, gen=gen)
                                     for _ in range(cfg.num_hidden_layers)])
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device=device)

    def forward(self, input_ids, positions):
        hidden = F.embedding(input_ids, self.embed_tokens)
        residual = None
        for layer in self.layers:
            hidden, residual = layer(positions, hidden, residual)
        hidden, _ = self.norm(hidden, residual)
        return hidden


# LLaDA checkpoint names -> module names (llada.py:223-245): ordered (pattern, replacement)
_LLADA_RENAMES = [
    (r"transformer\.blocks\.", "layers."),
    (r"transformer\.", ""),
    (r"\bwte\b", "embed_tokens"),
    (r"\bln_f\b", "norm"),
    (r"^model\.ff_out\b", "lm_head"),
    (r"\.(q_proj|k_proj|v_proj)\.", r".self_attn.\1."),
    (r"\.attn_out\.", ".self_attn.o_proj."),
    (r"\.ff_out\.", ".mlp.down_proj."),
    (r"\.ff_proj\.", ".mlp.gate_proj."),
    (r"\.up_proj\.", ".mlp.up_proj."),
    (r"\battn_norm\b", "input_layernorm"),
    (r"\bff_norm\b", "post_attention_layernorm"),
]


class LLaDAForDLM(nn.Module):
    packed_modules_mapping = {"kv_proj": ["k_proj", "v_proj"], "gate_up_proj": ["gate_proj", "up_proj"]}
    layer_cls = LLaDADecoderLayer

    def __init__(self, cfg, threshold, device="cuda", seed=0):
        super().__init__()
        gen = torch.Generator(device=device).manual_seed(seed)
        self.config = cfg
        self.model = LLaDAModel(cfg, threshold, device=device, gen=gen, layer_cls=self.layer_cls)
        self.lm_head = _param(cfg.vocab_size, cfg.hidden_size, device=device, gen=gen)
        if cfg.tie_word_embeddings:
            self.lm_head.data.copy_(self.model.embed_tokens.data)

    def forward(self, input_ids, positions):
        return self.model(input_ids, positions)

    def normalize_weight_name(self, name: str) -> str:
        if "transformer." not in name:
            return name
        for pat, rep in _LLADA_RENAMES:
            name = re.sub(pat, rep, name)
        return name

    def load_weights(self, weights):
        from ...utils.weight_loader import load_weights

        return load_weights(self, weights)

    def compute_logits(self, hidden):
        return F.linear(hidden, self.lm_head)

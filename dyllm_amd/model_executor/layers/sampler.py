"""Unmasking sampler (dyllm/model_executor/layers/sampler.py:176-357).

For every running sequence: take the logits of its still-masked positions in the current block,
apply temperature / top-k / top-p, score every candidate (confidence, margin, random, or
Dream's negative entropy), order the candidates by score and unmask the first
``num_transfer`` of them plus every candidate whose score reaches the sequence's confidence
threshold. Returns ``(positions [B, W], tokens [B, W], counts [B])`` with the kept candidates
first in each row (W = block width). The work runs as a handful of torch ops on the device; the
ragged->dense packing and the keep/count filter are index arithmetic on [B, W] tensors.

Tie order: candidates with equal scores keep ascending position order (a stable sort); the
reference uses an unstable descending sort there (sampler.py:300).
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch
import torch.nn.functional as F
from torch import nn


def top_p_logits(logits: torch.Tensor, top_p: Union[float, torch.Tensor, None] = None) -> torch.Tensor:
    """Nucleus filter per row (sampler.py:183-199)."""
    if top_p is None:
        return logits
    p = top_p if torch.is_tensor(top_p) else torch.full((logits.size(0),), float(top_p), device=logits.device)
    sorted_logits, sorted_idx = torch.sort(logits, descending=True)
    cum = torch.cumsum(F.softmax(sorted_logits, dim=-1), dim=-1)
    drop = cum > p.view(-1, 1).to(cum.dtype)
    drop[..., 1:] = drop[..., :-1].clone()
    drop[..., 0] = False
    mask = torch.zeros_like(logits, dtype=torch.bool).scatter_(-1, sorted_idx, drop)
    return logits.masked_fill(mask, torch.finfo(logits.dtype).min)


def top_k_logits(logits: torch.Tensor, top_k: Union[int, torch.Tensor, None] = None) -> torch.Tensor:
    """Keep the k largest logits per row (sampler.py:202-211)."""
    if top_k is None:
        return logits
    k = top_k if torch.is_tensor(top_k) else torch.full((logits.size(0),), int(top_k), device=logits.device)
    kmax = min(int(k.max().item()), logits.size(-1))
    vals, _ = torch.topk(logits, kmax, dim=-1)
    thr = vals.gather(1, (k.long() - 1).clamp(0, kmax - 1).unsqueeze(-1))
    return logits.masked_fill(logits < thr, torch.finfo(logits.dtype).min)


class RowLogits:
    """Logits computed only for the rows the sampler asks for: ``index_select(0, rows)`` runs the LM
    head on those hidden rows. The reference computes the LM head over every queried row
    (model_runner.py:375-388) and then keeps the candidate rows (sampler.py:264-266); each logits
    row depends only on its own hidden row, so the selected rows are the same values. ``shift``
    (Dream) reads row r from hidden row max(r - shift, 0), the one-row shift of sampler.py:322-326."""

    def __init__(self, hidden: torch.Tensor, compute, shift: int = 0):
        self.hidden, self.compute, self.shift = hidden, compute, shift
        self.device = hidden.device

    def size(self, dim: int = 0) -> int:
        return self.hidden.size(dim) if dim == 0 else self.compute(self.hidden[:1]).size(dim)

    def shifted(self, k: int) -> "RowLogits":
        return RowLogits(self.hidden, self.compute, self.shift + k)

    def index_select(self, dim: int, rows: torch.Tensor) -> torch.Tensor:
        assert dim == 0
        if self.shift:
            rows = (rows - self.shift).clamp_min(0)
        return self.compute(self.hidden.index_select(0, rows))


class DenseCandidates:
    """Candidate rows already laid out [B, W] on the device (dyllm_unmask_step): rel[b, j] is the
    offset of candidate j from sequence b's first queried row, valid for j < count[b], in ascending
    position order; offsets[b] turns an offset into the absolute position."""

    def __init__(self, rel: torch.Tensor, count: torch.Tensor, offsets: torch.Tensor, n_valid: Optional[int] = None):
        self.rel, self.count, self.offsets = rel, count, offsets
        # total of count[] when the host knows it (its token mirrors): the sampler then runs the
        # LM head, softmax and sampling on the valid candidates only, in the host path's order
        self.n_valid = n_valid


class BaseSampler(nn.Module):

    def __init__(self, algorithm: str = "confidence"):
        super().__init__()
        self.algorithm = algorithm

    def adjust_logits(self, logits: torch.Tensor) -> torch.Tensor:
        return logits

    def sample_token(self, probs, top_tokens, temperatures):
        return top_tokens

    def compute_scores(self, probs: torch.Tensor, top_probs: torch.Tensor) -> torch.Tensor:
        if self.algorithm == "confidence":
            return top_probs
        if self.algorithm == "margin_confidence":
            top2, _ = probs.topk(k=2, dim=-1)
            return top2[:, 0] - top2[:, 1]
        if self.algorithm == "random":
            return torch.rand_like(top_probs)
        raise ValueError(f"Unsupported algorithm for LLaDA: {self.algorithm}")

    def forward(self, input_logits: torch.Tensor, ctx, input_indices: Tuple[torch.Tensor, torch.Tensor, torch.Tensor],
                temperatures: Optional[torch.Tensor] = None, num_transfer: Optional[torch.Tensor] = None,
                top_k: Optional[torch.Tensor] = None, top_p: Optional[torch.Tensor] = None, block_size: int = 32,
                confidence_thresholds: Optional[torch.Tensor] = None):
        logits = self.adjust_logits(input_logits)
        dev = logits.device
        if isinstance(input_indices, DenseCandidates):
            return self._forward_dense(logits, ctx, input_indices, temperatures, num_transfer, top_k, top_p,
                                       confidence_thresholds)
        rel, offsets, cu = input_indices
        B = cu.numel() - 1
        n = rel.numel()
        counts = cu[1:] - cu[:-1]
        group = torch.repeat_interleave(torch.arange(B, device=dev), counts.long(), output_size=n)
        rows = ctx.cu_seqlens_q[:-1].long().index_select(0, group) + rel
        cand = logits.index_select(0, rows)
        if temperatures is not None:
            cand = cand / temperatures.unsqueeze(-1)
        cand = top_k_logits(cand, top_k)
        cand = top_p_logits(cand, top_p)
        probs = F.softmax(cand, dim=-1)
        top_probs, top_tokens = probs.max(dim=-1)
        scores = self.compute_scores(probs, top_probs)
        tokens = self.sample_token(probs, top_tokens, temperatures)
        pos = rel + offsets.index_select(0, group)

        # ragged -> dense [B, W] (sampler.py:114-175), W = block width
        W = int(block_size)
        slot = torch.arange(n, device=dev) - cu[:-1].long().index_select(0, group)
        inside = slot < W
        d_scores = torch.full((B, W), float("-inf"), dtype=scores.dtype, device=dev)
        d_tokens = torch.zeros((B, W), dtype=tokens.dtype, device=dev)
        d_pos = torch.zeros((B, W), dtype=pos.dtype, device=dev)
        g, s = group[inside], slot[inside]
        d_scores[g, s] = scores[inside]
        d_tokens[g, s] = tokens[inside]
        d_pos[g, s] = pos[inside]

        return self._select(d_scores, d_tokens, d_pos, num_transfer, confidence_thresholds)

    def _forward_dense(self, logits, ctx, cands: DenseCandidates, temperatures, num_transfer, top_k, top_p,
                       confidence_thresholds):
        """The same selection from candidates laid out [B, W] on the device: per-sequence knobs
        ([B] tensors) apply to every candidate of the sequence; empty slots score -inf."""
        dev = cands.rel.device
        B, W = cands.rel.shape
        valid = torch.arange(W, device=dev).unsqueeze(0) < cands.count.long().unsqueeze(1)
        rows = (ctx.cu_seqlens_q[:-1].long().unsqueeze(1) + cands.rel).masked_fill(~valid, 0).reshape(-1)
        rep = lambda t: t.reshape(-1).repeat_interleave(W, output_size=B * W)
        # the valid slots first (ascending (b, j): the host path's candidate order), sized by the
        # host's count so nothing waits on the device; a padding slot (-1) lands in a spare slot
        # B * W that is dropped. Without the host count every slot runs (empty ones masked).
        if cands.n_valid is not None:
            sel = torch.nonzero_static(valid.reshape(-1), size=int(cands.n_valid), fill_value=-1).reshape(-1)
            dst = torch.where(sel >= 0, sel, torch.full_like(sel, B * W))
            pick = lambda t: t.index_select(0, sel.clamp_min(0))
        else:
            dst = None
            pick = lambda t: t
        cand = logits.index_select(0, pick(rows))
        if temperatures is not None:
            cand = cand / pick(rep(temperatures)).unsqueeze(-1)
        cand = top_k_logits(cand, pick(rep(top_k)) if top_k is not None else None)
        cand = top_p_logits(cand, pick(rep(top_p)) if top_p is not None else None)
        probs = F.softmax(cand, dim=-1)
        top_probs, top_tokens = probs.max(dim=-1)
        scores = self.compute_scores(probs, top_probs)
        tokens = self.sample_token(probs, top_tokens, pick(rep(temperatures)) if temperatures is not None else None)
        if dst is not None:
            full_s = torch.full((B * W + 1,), float("-inf"), dtype=scores.dtype, device=dev)
            full_t = torch.zeros((B * W + 1,), dtype=tokens.dtype, device=dev)
            scores = full_s.index_copy_(0, dst, scores)[: B * W]
            tokens = full_t.index_copy_(0, dst, tokens)[: B * W]
        d_scores = scores.view(B, W).masked_fill(~valid, float("-inf"))
        d_tokens = tokens.view(B, W).masked_fill(~valid, 0)
        d_pos = (cands.rel + cands.offsets.long().unsqueeze(1)).masked_fill(~valid, 0)
        return self._select(d_scores, d_tokens, d_pos, num_transfer, confidence_thresholds)

    def _select(self, d_scores, d_tokens, d_pos, num_transfer, confidence_thresholds):
        """Order every sequence's candidates by score (stable: ties keep position order) and keep
        the first num_transfer plus every one whose score reaches the threshold (sampler.py:44-86)."""
        dev = d_scores.device
        B, W = d_scores.shape
        s_scores, order = torch.sort(d_scores, dim=1, descending=True, stable=True)
        s_tokens = d_tokens.gather(1, order)
        s_pos = d_pos.gather(1, order)
        if num_transfer is None:
            nt = torch.zeros(B, dtype=torch.long, device=dev)
        else:
            nt = num_transfer.reshape(-1).long().clamp_min(0).to(dev)
        if confidence_thresholds is None:
            thr = torch.full((B,), float("inf"), dtype=s_scores.dtype, device=dev)
        else:
            thr = confidence_thresholds.to(device=dev, dtype=s_scores.dtype)
        # keep = top num_transfer, or score >= threshold, and a real candidate (sampler.py:44-86)
        j = torch.arange(W, device=dev).unsqueeze(0)
        keep = ((j < nt.unsqueeze(1)) | (s_scores >= thr.unsqueeze(1))) & (s_scores > float("-inf"))
        out_tokens = torch.where(keep, s_tokens, torch.full_like(s_tokens, -1))
        out_pos = torch.where(keep, s_pos, torch.zeros_like(s_pos))
        out_counts = keep.sum(dim=1, dtype=torch.int32)
        return out_pos, out_tokens, out_counts


class LLaDASampler(BaseSampler):
    pass


class DreamSampler(BaseSampler):
    """Dream predicts token t from position t-1: the logits are shifted by one row over the
    packed batch (sampler.py:322-326); sampling is categorical when a temperature is set."""

    def adjust_logits(self, logits):
        if isinstance(logits, RowLogits):
            return logits.shifted(1)
        if logits.size(0) <= 1:
            return logits
        return torch.cat([logits[:1], logits[:-1]], dim=0)

    def sample_token(self, probs, top_tokens, temperatures):
        if temperatures is not None and bool(torch.any(temperatures > 0)):
            return torch.multinomial(probs.float(), 1).squeeze(-1)
        return top_tokens

    def compute_scores(self, probs, top_probs):
        if self.algorithm == "entropy":
            return torch.sum(probs * torch.log(probs + 1e-10), dim=-1)
        if self.algorithm == "origin":
            return torch.rand_like(top_probs)
        raise ValueError(f"Unsupported algorithm for Dream: {self.algorithm}")

"""Per-step context shared by all layers (dyllm/utils/context.py:6-109, the fields the
mask-based models use). Layers read it and the attention layer mutates the salient index
lists for the next layer, as in the reference (attention.py:166,172-173)."""
from dataclasses import dataclass
from typing import List, Optional

import torch


@dataclass
class Context:
    is_full: bool = False
    cu_seqlens_q: Optional[torch.Tensor] = None      # int32 [B+1] (device)
    cu_seqlens_q_cpu: Optional[List[int]] = None
    cu_seqlens_k: Optional[torch.Tensor] = None      # int32 [B+1] (device)
    cu_seqlens_k_cpu: Optional[List[int]] = None
    cu_promptlens: Optional[torch.Tensor] = None     # int32 [B+1] (device)
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    context_lens: Optional[torch.Tensor] = None
    context_lens_cpu: Optional[List[int]] = None
    cu_updatedlens: Optional[torch.Tensor] = None
    cu_salientlens: Optional[torch.Tensor] = None    # int32 [B+1]
    idx_salient_row: Optional[torch.Tensor] = None   # int64 [n] (Q space)
    idx_salient_row_k: Optional[torch.Tensor] = None  # int64 [n] (K space) when Q-pruned, else None
    idx_salient_row_i32: Optional[torch.Tensor] = None  # int32 copy of idx_salient_row (kernel operand)
    max_salientlen: int = 0                          # max salient rows of one sequence (0: unknown)
    idx_updated_row: Optional[torch.Tensor] = None
    total_seqlen_k: int = 0
    total_seqlen: int = 0
    positions_k: Optional[torch.Tensor] = None


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_full, **kwargs) -> Context:
    global _CONTEXT
    _CONTEXT = Context(is_full=is_full, **kwargs)
    return _CONTEXT


def reset_context():
    global _CONTEXT
    _CONTEXT = Context()

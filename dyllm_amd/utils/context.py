"""Per-step context shared by all layers (dyllm/utils/context.py:6-109, the fields the
mask-based models use). Layers read it and the attention layer mutates the salient index
lists for the next layer, as in the reference (attention.py:166,172-173).

The salient set produced by a layer's compaction stays on the device until something needs its
size on the host: the attention layer stores the device result in ``salient_pending`` and the
first read of ``idx_salient_row`` / ``idx_salient_row_i32`` / ``idx_salient_row_k`` /
``max_salientlen`` performs the one device->host read (the reference's torch.nonzero sync).
The fused FFN of the same layer consumes the pending device buffers directly, so it is
enqueued before that read and the GPU stays busy while the host catches up.
"""
from typing import List, Optional

import torch

_FIELDS = dict(
    is_full=False,
    cu_seqlens_q=None,        # int32 [B+1] (device)
    cu_seqlens_q_cpu=None,
    cu_seqlens_k=None,        # int32 [B+1] (device)
    cu_seqlens_k_cpu=None,
    cu_promptlens=None,       # int32 [B+1] (device)
    max_seqlen_q=0,
    max_seqlen_k=0,
    context_lens=None,
    context_lens_cpu=None,
    cu_updatedlens=None,
    cu_salientlens=None,      # int32 [B+1]
    idx_updated_row=None,
    total_seqlen_k=0,
    total_seqlen=0,
    positions_k=None,
    salient_pending=None,     # device result of the last compaction, not yet read by the host
    salient_hint=0,           # salient count of the previous layer (tile-shape hint)
    salient_n=-1,             # host copy of len(idx_salient_row) once resolved
)


class Context:
    """Step context. ``idx_salient_row`` is int64 [n] (Q space), ``idx_salient_row_k`` int64
    [n] (K space) in Q-pruned steps and None otherwise, ``idx_salient_row_i32`` an int32 copy."""

    def __init__(self, is_full=False, idx_salient_row=None, idx_salient_row_k=None, idx_salient_row_i32=None,
                 max_salientlen=0, **kwargs):
        for k, v in _FIELDS.items():
            setattr(self, k, v)
        unknown = set(kwargs) - set(_FIELDS)
        if unknown:
            raise TypeError(f"unknown context fields {sorted(unknown)}")
        for k, v in kwargs.items():
            setattr(self, k, v)
        self.is_full = is_full
        self._idx_salient_row = idx_salient_row
        self._idx_salient_row_k = idx_salient_row_k
        self._idx_salient_row_i32 = idx_salient_row_i32
        self._idx_salient_row_k_i32 = None
        self._max_salientlen = max_salientlen
        if idx_salient_row is not None and not self.salient_hint:
            self.salient_hint = int(idx_salient_row.numel())

    # -- salient set (resolved lazily) ---------------------------------------------------
    def resolve_salient(self):
        comp = self.salient_pending
        if comp is None:
            return
        n, cu = comp.host()
        self.salient_pending = None
        self._idx_salient_row = comp.idx64[:n]
        self._idx_salient_row_i32 = comp.idx32[:n]
        self._idx_salient_row_k = comp.idx_k[:n] if comp.idx_k is not None else None
        self._idx_salient_row_k_i32 = comp.idx_k32[:n] if comp.idx_k32 is not None else None
        self.cu_salientlens = comp.cu_salientlens
        self._max_salientlen = max(cu[i + 1] - cu[i] for i in range(len(cu) - 1))
        self.salient_hint = n
        self.salient_n = n

    def set_pending(self, comp):
        """Install a compaction result as the next layer's salient set (device only)."""
        self.salient_pending = comp
        self.cu_salientlens = comp.cu_salientlens

    @property
    def q_pruned(self) -> bool:
        if self.salient_pending is not None:
            return self.salient_pending.idx_k is not None
        return self._idx_salient_row_k is not None

    @property
    def idx_salient_row(self) -> Optional[torch.Tensor]:
        self.resolve_salient()
        return self._idx_salient_row

    @idx_salient_row.setter
    def idx_salient_row(self, v):
        self.salient_pending = None
        self._idx_salient_row = v
        self._idx_salient_row_i32 = None

    @property
    def idx_salient_row_i32(self) -> Optional[torch.Tensor]:
        self.resolve_salient()
        if self._idx_salient_row_i32 is None and self._idx_salient_row is not None:
            self._idx_salient_row_i32 = self._idx_salient_row.to(torch.int32)
        return self._idx_salient_row_i32

    @idx_salient_row_i32.setter
    def idx_salient_row_i32(self, v):
        self._idx_salient_row_i32 = v

    @property
    def idx_salient_row_k(self) -> Optional[torch.Tensor]:
        self.resolve_salient()
        return self._idx_salient_row_k

    @idx_salient_row_k.setter
    def idx_salient_row_k(self, v):
        self._idx_salient_row_k = v
        self._idx_salient_row_k_i32 = None

    @property
    def idx_salient_row_k_i32(self) -> Optional[torch.Tensor]:
        self.resolve_salient()
        if self._idx_salient_row_k_i32 is None and self._idx_salient_row_k is not None:
            self._idx_salient_row_k_i32 = self._idx_salient_row_k.to(torch.int32)
        return self._idx_salient_row_k_i32

    @property
    def max_salientlen(self) -> int:
        self.resolve_salient()
        return self._max_salientlen

    @max_salientlen.setter
    def max_salientlen(self, v):
        self._max_salientlen = v


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

"""Step scheduler (dyllm/engine/scheduler.py:11-145).

A new sequence first runs ``num_full_steps`` full (dense) steps, then sparse steps until it is
finished. Full work is scheduled before sparse work; one step runs either kind, never a mix.
Sparse sequences are re-queued at the front in their order, so the same batch keeps running.
"""
from __future__ import annotations

from collections import deque
from typing import Deque, List, Tuple

import numpy as np
import torch

from ..config import Config
from ..utils.metadata import get_metadata
from .sequence import Sequence, SequenceStatus


class Scheduler:

    def __init__(self, config: Config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.eos = config.eos
        self.mask = config.mask_id
        self.full: Deque[Sequence] = deque()
        self.sparse: Deque[Sequence] = deque()
        self.finished: List[int] = []
        self._host_buf = None   # host staging of the sampler output (postprocess)
        self._host_dev = None

    def is_finished(self) -> bool:
        return not self.full and not self.sparse

    def add(self, seq: Sequence):
        self.full.append(seq)

    def schedule(self) -> Tuple[List[Sequence], bool]:
        """(sequences of this step, is_full) -- scheduler.py:29-77."""
        batch: List[Sequence] = []
        ids = set()
        tokens = 0
        while self.full and len(batch) < self.max_num_seqs:
            seq = self.full[0]
            if tokens + len(seq) > self.max_num_batched_tokens or seq.seq_id in ids:
                break
            self.full.popleft()
            seq.processed_steps += 1
            tokens += len(seq)
            batch.append(seq)
            ids.add(seq.seq_id)
            if seq.processed_steps < seq.num_full_steps:
                seq.status = SequenceStatus.FULL
                self.full.append(seq)
            else:
                seq.status = SequenceStatus.SPARSE
                self.sparse.append(seq)
        if batch:
            return batch, True

        while self.sparse and len(batch) < self.max_num_seqs:
            if tokens > self.max_num_batched_tokens:
                break
            seq = self.sparse[0]
            if seq.seq_id in ids:
                break
            self.sparse.popleft()
            tokens += len(seq)
            batch.append(seq)
            seq.processed_steps += 1
            ids.add(seq.seq_id)
        if not batch:
            raise RuntimeError("schedule() called with no runnable sequence")
        self.sparse.extendleft(reversed(batch))
        return batch, False

    def preempt(self, seq: Sequence):
        seq.status = SequenceStatus.FULL
        self.full.appendleft(seq)

    def eos_and_done(self, seq: Sequence, pos: int) -> bool:
        """True when no mask token precedes ``pos`` (scheduler.py:83-87)."""
        return not bool((seq.token_arr[:pos] == self.mask).any())

    def _finish(self, seq: Sequence, finished: List[int]):
        seq.status = SequenceStatus.FINISHED
        finished.append(seq.seq_id)
        queue = self.full if seq.processed_steps < seq.num_full_steps else self.sparse
        if seq in queue:
            queue.remove(seq)

    def _to_host(self, counts: torch.Tensor, tokens: torch.Tensor, positions: torch.Tensor):
        """The sampler's [B] counts and [B, W] tokens / positions as numpy arrays, through one
        reusable host staging buffer: three asynchronous copies into it, then a single wait
        (pinned when the inputs live on the GPU)."""
        B = counts.numel()
        W = tokens.shape[-1] if tokens.dim() == 2 else 0
        need = B * (1 + 2 * W)
        dev = tokens.device
        buf = self._host_buf
        if buf is None or buf.numel() < need or self._host_dev != dev:
            buf = torch.empty(max(need, 64), dtype=torch.int64, pin_memory=dev.type == "cuda")
            self._host_buf, self._host_dev = buf, dev
        views = (buf[:B], buf[B: B + B * W].view(B, W), buf[B + B * W: need].view(B, W))
        for dst, src in zip(views, (counts.reshape(B), tokens.reshape(B, W), positions.reshape(B, W))):
            dst.copy_(src, non_blocking=True)
        if dev.type == "cuda":
            torch.cuda.current_stream(dev).synchronize()
        return tuple(v.numpy() for v in views)

    def _spent(self, seq: Sequence) -> bool:
        """Step budget used up (fixed-count unmasking) or every answer token generated."""
        if seq.confidence_threshold is None and seq.processed_steps == seq.num_steps:
            return True
        return seq.num_completion_tokens >= seq.max_new_tokens

    def postprocess(self, seqs: List[Sequence], selected_positions: torch.Tensor, selected_tokens: torch.Tensor,
                    selected_counts: torch.Tensor) -> List[int]:
        """Commit one step's sampled tokens and retire finished sequences (the contract of
        scheduler.py:89-145). A sequence finishes when it samples EOS with no mask token before
        it (unless it ignores EOS), when its step budget is spent, or when its answer is complete.
        With device-built sparse steps the same tokens are also committed on the device
        (unmask_step_kernel); this host copy keeps the mirrors that finish detection and the next
        step's launch sizes read."""
        counts, toks, poss = self._to_host(selected_counts, selected_tokens, selected_positions)
        finished: List[int] = []
        for seq, n, tok_row, pos_row in zip(seqs, counts.tolist(), toks, poss):
            if n > 0:
                tok, pos = tok_row[:n], pos_row[:n]
                seq.update_token(pos, tok)
                seq.update_block_idx()
                eos_at = np.flatnonzero(tok == self.eos)
                if eos_at.size and not seq.ignore_eos and self.eos_and_done(seq, int(pos[eos_at[0]])):
                    self._finish(seq, finished)
                    continue
            if self._spent(seq):
                self._finish(seq, finished)
        get_metadata().finished_seqs = finished
        self.finished.extend(finished)
        return finished

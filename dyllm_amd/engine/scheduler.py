"""Step scheduler (dyllm/engine/scheduler.py:11-145).

A new sequence first runs ``num_full_steps`` full (dense) steps, then sparse steps until it is
finished. Full work is scheduled before sparse work; one step runs either kind, never a mix.
Sparse sequences are re-queued at the front in their order, so the same batch keeps running.
"""
from __future__ import annotations

from collections import deque
from typing import Deque, List, Tuple

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

    def postprocess(self, seqs: List[Sequence], selected_positions: torch.Tensor, selected_tokens: torch.Tensor,
                    selected_counts: torch.Tensor) -> List[int]:
        """Write the sampled tokens back and retire finished sequences (scheduler.py:89-145).
        One device->host copy carries counts, tokens and positions."""
        finished: List[int] = []
        B = selected_counts.size(0)
        L = selected_tokens.size(1) if selected_tokens.dim() == 2 else 0
        packed = torch.cat([selected_counts.reshape(-1).long(), selected_tokens.reshape(-1).long(),
                            selected_positions.reshape(-1).long()]).cpu().tolist()
        counts = packed[:B]
        toks = packed[B: B + B * L]
        poss = packed[B + B * L:]
        for b, seq in enumerate(seqs):
            n = counts[b]
            if n > 0:
                tok = toks[b * L: b * L + n]
                pos = poss[b * L: b * L + n]
                seq.update_token(pos, tok)
                seq.update_block_idx()
                if self.eos in tok:
                    eos_pos = pos[tok.index(self.eos)]
                    if self.eos_and_done(seq, eos_pos) and not seq.ignore_eos:
                        self._finish(seq, finished)
                        continue
            steps_done = seq.confidence_threshold is None and seq.processed_steps == seq.num_steps
            if steps_done or seq.num_completion_tokens >= seq.max_new_tokens:
                self._finish(seq, finished)
        get_metadata().finished_seqs = finished
        self.finished.extend(finished)
        return finished

"""One generation request: the prompt followed by ``max_new_tokens`` mask tokens, unmasked block
by block over the denoising steps (the request record of dyllm/engine/sequence.py:8-82).

The tokens live in one int64 numpy array, the form the step builder slices and compares
(model_runner.py reads whole rows of it per step); the list view ``token_ids`` is produced on
demand for API results. Per-request decoding knobs are read through from the request's own
``SamplingParams`` instead of being copied field by field.
"""
from __future__ import annotations

from enum import Enum, auto
from itertools import count
from typing import List, Sequence as Seq

import numpy as np

from ..sampling_params import SamplingParams


class SequenceStatus(Enum):
    """Scheduler queue a request is in (scheduler.py:29-77)."""
    FULL = auto()
    SPARSE = auto()
    FINISHED = auto()


def _knob(name: str):
    return property(lambda self: getattr(self.params, name), doc=f"SamplingParams.{name} of the request")


class Sequence:
    _next_id = count()

    temperature = _knob("temperature")
    max_new_tokens = _knob("max_new_tokens")
    ignore_eos = _knob("ignore_eos")
    top_p = _knob("top_p")
    top_k = _knob("top_k")
    confidence_threshold = _knob("confidence_threshold")
    block_size = _knob("block_size")
    num_full_steps = _knob("num_full_steps")
    num_steps = _knob("steps")
    mask_id = _knob("mask_id")

    def __init__(self, token_ids: Seq[int], sampling_params: SamplingParams = SamplingParams()):
        self.params = sampling_params
        self.seq_id = next(Sequence._next_id)
        self.status = SequenceStatus.FULL
        self.token_arr = np.array(token_ids, dtype=np.int64).reshape(-1)
        mask = self.mask_id
        n_masked = 0 if mask is None else int(np.count_nonzero(self.token_arr == mask))
        self.num_prompt_tokens = self.token_arr.size - n_masked
        self.num_tokens = self.num_prompt_tokens          # prompt + unmasked answer tokens
        self.processed_steps = 0
        self.block_idx = 0
        # what the previous step wrote: the first layer's salient rows of the next sparse step
        # (model_runner.py:207-214); before any step, position 0 stands in
        self.last_token_pos: List[int] = [0]
        self.last_tokens: List[int] = [int(self.token_arr[-1])] if self.token_arr.size else []

    # -- token views ----------------------------------------------------------------------
    def __len__(self) -> int:
        return self.token_arr.size

    def __getitem__(self, key):
        v = self.token_arr[key]
        return v.tolist() if isinstance(v, np.ndarray) else int(v)

    @property
    def token_ids(self) -> List[int]:
        return self.token_arr.tolist()

    @property
    def prompt_token_ids(self) -> List[int]:
        return self.token_arr[: self.num_prompt_tokens].tolist()

    @property
    def completion_token_ids(self) -> List[int]:
        return self.token_arr[self.num_prompt_tokens:].tolist()

    # -- progress -------------------------------------------------------------------------
    @property
    def is_finished(self) -> bool:
        return self.status is SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self) -> int:
        return self.num_tokens - self.num_prompt_tokens

    @property
    def answer_start(self) -> int:
        """First row of the answer region (the Q rows of a Q-pruned step)."""
        return self.token_arr.size - self.max_new_tokens

    @property
    def output_length(self) -> int:
        return self.max_new_tokens

    @property
    def num_transfer_tokens(self) -> int:
        """Answer tokens unmasked per step when no confidence threshold is set: the answer
        length spread evenly over the steps (sequence.py:68-71 requires it to divide)."""
        q, r = divmod(self.max_new_tokens, self.num_steps)
        if r:
            raise ValueError(f"max_new_tokens ({self.max_new_tokens}) must be a multiple of steps ({self.num_steps})")
        return q

    def update_token(self, pos: Seq[int], token_id: Seq[int]) -> None:
        """Write one step's sampled tokens (distinct positions). Positions that held the mask
        and now hold a real token count as generated."""
        p = np.asarray(pos, dtype=np.int64).reshape(-1)
        t = np.asarray(token_id, dtype=np.int64).reshape(-1)
        if p.size:
            if self.mask_id is not None:
                newly = (self.token_arr[p] == self.mask_id) & (t != self.mask_id)
                self.num_tokens += int(np.count_nonzero(newly))
            self.token_arr[p] = t
        self.last_token_pos = p.tolist()
        self.last_tokens = t.tolist()

    def update_block_idx(self) -> None:
        """The block the next unmasking works in: completed answer tokens // block size."""
        bs = self.block_size
        done = self.num_completion_tokens
        if done > 0 and bs:
            self.block_idx = done // bs
